"""Loss-side hologram reconstruction on the GPU.

Mirrors ``propagator`` of the reference's ``utils/propagator.py`` (:172-636)
for the configuration its training uses (train.py:867-885):
``propagation_type='Bandlimited Angular Spectrum'``,
``propagator_type='forward'``, ``laser_channel_power=eye(3)``, a circular
Fourier-plane aperture of ``aperture_size``.  ``reconstruct(hologram_phases,
amplitude, no_grad, get_complex)`` returns the (frames, depths, channels,
m, n) intensities (or complex fields) as ``_reconstruct_impl`` does, and is
differentiable with ``no_grad=False`` (train.py:282).

The pipeline is four HIP steps: the hologram fields w a e^{i s phi} of the
(frame, channel) pairs with nonzero laser power (``hrf_recon_fields``), the
band-limited ASM to every depth (each field transformed once for all
depths, through the multi-plane propagation kernels run with negated
distances: the fused LDS-FFT passes where the grid size has a plan), the
intensity (``hrf_recon_intensity``), and the mirror-image backward.  The transfer function is the reference's own band-limited ASM
kernel (cuda_prop, the one the rasterizer's hologram uses); the reference's
reconstruction takes it from odak's ``get_propagation_kernel``, which is not
available here, so agreement with odak's kernel is not checked.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib, propagation


# fields per propagation call (the ASM entry points' channel limit)
_BATCH = 3


def _fan_out(fields, wavelengths, pitch, distances, S, aperture):
    """(K,S,S) hologram fields -> (D,K,S,S): each field propagated to every
    depth.  This is the multi-plane adjoint's data flow (one spectrum per
    channel, one inverse transform per plane) with the distances negated:
    conj(T(-d)) = T(d), the band limit depending on d^2 only, so the fused
    LDS-FFT kernels serve it where the grid size has a plan."""
    return propagation.multiplane_adjoint(fields, (S, S), wavelengths, pitch,
                                          [-d for d in distances], S, aperture)


def _fan_in(grads, wavelengths, pitch, distances, S, aperture):
    """Adjoint of _fan_out: (D,K,S,S) -> (K,S,S), summed over the depths
    (the multi-plane forward with the distances negated)."""
    return propagation.multiplane(grads, wavelengths, pitch, [-d for d in distances], S,
                                  aperture)


def _pairs(laser_powers: torch.Tensor, F: int, C: int):
    lp = laser_powers.detach().to("cpu", torch.float32).reshape(F, C)
    pairs = [(f, c, float(lp[f, c])) for f in range(F) for c in range(C) if float(lp[f, c]) != 0]
    return pairs


def _arrays(pairs, scales):
    K = len(pairs)
    fr = (ctypes.c_int32 * K)(*[p[0] for p in pairs])
    ch = (ctypes.c_int32 * K)(*[p[1] for p in pairs])
    pw = (ctypes.c_float * K)(*[p[2] for p in pairs])
    sc = (ctypes.c_float * K)(*[float(scales[p[1]]) for p in pairs])
    return fr, ch, pw, sc


class _Reconstruct(torch.autograd.Function):
    @staticmethod
    def forward(ctx, phases, amplitude, pairs, scales, wavelengths, pitch, distances, aperture,
                get_complex):
        F, S = phases.shape[0], phases.shape[-1]
        C = amplitude.shape[0]
        D = len(distances)
        hw = S * S
        dev = phases.device
        out_dtype = torch.complex64 if get_complex else torch.float32
        out = torch.zeros((F, D, C, S, S), dtype=out_dtype, device=dev)
        ctx.meta = (pairs, scales, wavelengths, pitch, distances, aperture, get_complex, F, C)
        if not pairs:
            ctx.save_for_backward(phases, amplitude, None)
            return out
        K = len(pairs)
        fr, ch, pw, sc = _arrays(pairs, scales)
        lib = _lib.load()
        fields = torch.empty((K, S, S), dtype=torch.complex64, device=dev)
        with torch.cuda.device(dev):
            stream = _lib.stream_ptr(dev)
            _lib.check(lib.hrf_recon_fields(amplitude.data_ptr(), phases.data_ptr(), F, C, hw,
                                            fr, ch, pw, sc, K, fields.data_ptr(), stream))
        wl = [wavelengths[c] for _, c, _ in pairs]
        u = torch.cat([_fan_out(fields[k0:k0 + _BATCH], wl[k0:k0 + _BATCH], pitch, distances,
                                S, aperture)
                       for k0 in range(0, K, _BATCH)], dim=1)  # (D,K,S,S)
        if get_complex:
            res = u
        else:
            res = torch.empty((D, K, S, S), dtype=torch.float32, device=dev)
            with torch.cuda.device(dev):
                _lib.check(lib.hrf_recon_intensity(u.data_ptr(), u.numel(), res.data_ptr(),
                                                   _lib.stream_ptr(dev)))
        for k, (f, c, _) in enumerate(pairs):
            out[f, :, c] = res[:, k]
        ctx.save_for_backward(phases, amplitude, u)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        phases, amplitude, u = ctx.saved_tensors
        pairs, scales, wavelengths, pitch, distances, aperture, get_complex, F, C = ctx.meta
        S = phases.shape[-1]
        if not pairs:
            return (torch.zeros_like(phases), torch.zeros_like(amplitude), None, None, None,
                    None, None, None, None)
        dev = phases.device
        K, hw = len(pairs), S * S
        lib = _lib.load()
        g = torch.stack([grad_out[f, :, c] for f, c, _ in pairs], dim=1).contiguous()
        if get_complex:
            gu = g.to(torch.complex64).contiguous()
        else:
            g = g.to(torch.float32).contiguous()
            gu = torch.empty_like(u)
            with torch.cuda.device(dev):
                _lib.check(lib.hrf_recon_intensity_backward(u.data_ptr(), g.data_ptr(), u.numel(),
                                                            gu.data_ptr(), _lib.stream_ptr(dev)))
        wl = [wavelengths[c] for _, c, _ in pairs]
        gfields = torch.cat([_fan_in(gu[:, k0:k0 + _BATCH].contiguous(), wl[k0:k0 + _BATCH],
                                     pitch, distances, S, aperture)
                             for k0 in range(0, K, _BATCH)], dim=0)
        fr, ch, pw, sc = _arrays(pairs, scales)
        g_amp = torch.empty_like(amplitude)
        g_phase = torch.empty_like(phases)
        with torch.cuda.device(dev):
            _lib.check(lib.hrf_recon_fields_backward(
                amplitude.data_ptr(), phases.data_ptr(), F, C, hw, fr, ch, pw, sc, K,
                gfields.data_ptr(), g_amp.data_ptr(), g_phase.data_ptr(), _lib.stream_ptr(dev)))
        return g_phase, g_amp, None, None, None, None, None, None, None


class Propagator:
    """The reference's ``propagator`` (utils/propagator.py:172-636) for the
    band-limited angular spectrum, ``forward`` propagator type.  Arguments as
    the reference's; configurations this build does not provide raise."""

    def __init__(self, resolution=(1920, 1080), wavelengths=(515e-9,), pixel_pitch=8e-6,
                 resolution_factor=1, number_of_frames=1, number_of_depth_layers=1,
                 volume_depth=1e-2, image_location_offset=5e-3,
                 propagation_type='Bandlimited Angular Spectrum', propagator_type='back and forth',
                 back_and_forth_distance=0.3, laser_channel_power=None, aperture=None,
                 aperture_size=None, distances=None, aperture_samples=(20, 20, 5, 5),
                 method='conventional', device=torch.device('cuda')):
        if propagation_type != 'Bandlimited Angular Spectrum':
            raise NotImplementedError(f"propagation_type {propagation_type!r}: only the "
                                      "band-limited angular spectrum is provided")
        if propagator_type != 'forward':
            raise NotImplementedError(f"propagator_type {propagator_type!r}: only 'forward' "
                                      "(the reference's training configuration) is provided")
        if aperture is not None:
            raise NotImplementedError("a custom aperture tensor is not provided; use "
                                      "aperture_size (circular)")
        if int(resolution[0]) != int(resolution[1]):
            raise NotImplementedError("the ASM kernels take square holograms")
        if method not in ('conventional', 'multi-color'):
            raise ValueError(f"method {method!r}")
        self.device = torch.device(device)
        self.resolution = [int(resolution[0]), int(resolution[1])]
        self.wavelengths = [float(w) for w in wavelengths]
        self.pixel_pitch = float(pixel_pitch)
        self.resolution_factor = 1  # only used by Impulse Response Fresnel in the reference
        self.number_of_frames = int(number_of_frames)
        self.number_of_channels = len(self.wavelengths)
        self.volume_depth = volume_depth
        self.image_location_offset = image_location_offset
        self.propagation_type = propagation_type
        self.propagator_type = propagator_type
        self.method = method
        if distances is None:
            self.distances = (torch.linspace(-volume_depth / 2., volume_depth / 2.,
                                             number_of_depth_layers) + image_location_offset)
        else:
            self.distances = torch.as_tensor(distances)
        self.number_of_depth_layers = int(self.distances.numel())
        self.channel_power = (torch.eye(self.number_of_frames, self.number_of_channels)
                              if laser_channel_power is None else
                              torch.as_tensor(laser_channel_power))
        self.phase_scale = [1.0] * self.number_of_channels  # propagator.py:315-328
        # circular Fourier-plane aperture; the reference's default radius is
        # the longer edge of the hologram
        self.aperture_size = float(max(self.resolution) if aperture_size is None
                                   else aperture_size)

    def get_laser_powers(self) -> torch.Tensor:
        if self.method == 'multi-color':
            return torch.abs(torch.cos(self.channel_power))
        return self.channel_power

    def set_laser_powers(self, laser_power):
        self.channel_power = laser_power

    def reconstruct(self, hologram_phases, amplitude=None, no_grad=True, get_complex=False):
        """(frames, m, n) phases (+ (channels, m, n) amplitudes, default
        ones) -> (frames, depths, channels, m, n) intensities (complex
        fields with get_complex)."""
        if hologram_phases.dim() > 3:
            hologram_phases = hologram_phases.squeeze(0)
        S = self.resolution[0]
        F, C = self.number_of_frames, self.number_of_channels
        if tuple(hologram_phases.shape) != (F, S, S):
            raise RuntimeError(f"hologram_phases must be ({F}, {S}, {S}); "
                               f"got {tuple(hologram_phases.shape)}")
        if not hologram_phases.is_cuda:
            raise RuntimeError("the HIP reconstruction needs GPU tensors")
        if amplitude is None:
            amplitude = torch.ones((C, S, S), device=hologram_phases.device)
        if tuple(amplitude.shape) != (C, S, S):
            raise RuntimeError(f"amplitude must be ({C}, {S}, {S}); got {tuple(amplitude.shape)}")
        phases = hologram_phases.to(torch.float32).contiguous()
        amplitude = amplitude.to(torch.float32).contiguous()
        pairs = _pairs(self.get_laser_powers(), F, C)
        args = (pairs, self.phase_scale, self.wavelengths, self.pixel_pitch,
                [float(d) for d in self.distances], self.aperture_size, bool(get_complex))
        if no_grad:
            with torch.no_grad():
                return _Reconstruct.apply(phases, amplitude, *args)
        return _Reconstruct.apply(phases, amplitude, *args)
