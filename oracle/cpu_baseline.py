"""The reference's CPU PyTorch path, restated — TEST INFRASTRUCTURE / BASELINE ONLY.

Used only by bench.py's cpu_baseline leg (and tests).  It restates, with
torch ops on the CPU, the path a user of the reference gets without the CUDA
extension:

* ``Scene.splat(render_using_python=True)`` (model.py:1194-1228): 64x64
  tiles, per tile the Gaussians whose 3-sigma diagonal box (clamped to the
  image) overlaps it (``calculate_gaussian_bounds``, model.py:553-592);
* ``splat_tile_python`` (model.py:1276-1363) with the geometry fallbacks
  ``compute_means_2D`` / ``compute_cov_2D`` / ``_compute_jacobian`` /
  ``compute_cov_3D`` / ``invert_cov_2D`` (model.py:406-551), the cumprod
  transmittance (model.py:1090-1103), and the CUDA-only helper ops
  (batch_matrix_mult_cuda.cu:48-49, sum_last_dim_cuda.cu:39,
  element_wise_mult_cuda.cu:34-35) replaced by the equivalent torch ops;
* the pure-torch band-limited ASM (python_function.py:35-78) per (plane,
  wavelength) with ``distance = -distances[p]``, summed over planes.

Backward is torch autograd through the same graph.  pytorch3d's
quaternion_to_matrix and odak's pad/crop/circular mask are restated from
their published definitions (centred pad/crop; a disc of radius r about the
grid centre).  Semantics differ slightly from the CUDA rasterizer (no 0.99
alpha clamp, 3-sigma boxes, float32 kz) — this path is for timing, parity is
measured against hrf_oracle.c.
"""
from __future__ import annotations

import math
import time

import torch


def quaternion_to_matrix(q):
    r, i, j, k = torch.unbind(q, -1)
    two_s = 2.0 / (q * q).sum(-1)
    o = torch.stack((
        1 - two_s * (j * j + k * k), two_s * (i * j - k * r), two_s * (i * k + j * r),
        two_s * (i * j + k * r), 1 - two_s * (i * i + k * k), two_s * (j * k - i * r),
        two_s * (i * k - j * r), two_s * (j * k + i * r), 1 - two_s * (i * i + j * j)), -1)
    return o.reshape(q.shape[:-1] + (3, 3))


def means_2d(cam, fx, fy, px, py, near=1.0, far=1000.0):
    mask = (cam[:, 2] > near) & (cam[:, 2] < far)
    inv_z = 1.0 / cam[:, 2].unsqueeze(1)
    xy = -cam[:, :2] * inv_z
    m = torch.stack([fx * xy[:, 0] + px, fy * xy[:, 1] + py], 1)
    return torch.where(mask[:, None], m, torch.full_like(m, 1e6))


def jacobian(cam, fx, fy, W, H, near=1.0, far=1000.0):
    lim_x = 1.3 * (0.5 * W / fx)
    lim_y = 1.3 * (0.5 * H / fy)
    tx, ty, tz = cam[:, 0], cam[:, 1], cam[:, 2]
    mask = ((tz > near) & (tz < far)).float()
    tx = torch.clamp(tx / tz, -lim_x, lim_x) * tz
    ty = torch.clamp(ty / tz, -lim_y, lim_y) * tz
    z = torch.zeros_like(tz)
    J = torch.stack([fx / tz, z, -(fx * tx) / (tz * tz), z, fy / tz, -(fy * ty) / (tz * tz)], 1)
    return J.reshape(-1, 2, 3) * mask[:, None, None]


def cov_2d(cam, quats, scales, fx, fy, R, W, H):
    J = jacobian(cam, fx, fy, W, H)
    n = J.shape[0]
    Wm = R.expand(n, 3, 3)
    S = torch.diag_embed(scales)
    rots = quaternion_to_matrix(quats)
    cov3 = rots @ S @ S.transpose(1, 2) @ rots.transpose(1, 2)
    c = J @ Wm @ cov3 @ Wm.transpose(1, 2) @ J.transpose(1, 2)
    return c + 0.3 * torch.eye(2)


def invert_cov_2d(c):
    det = (c[:, 0, 0] * c[:, 1, 1] - c[:, 1, 0] * c[:, 0, 1])[:, None, None]
    inv = torch.stack([c[:, 1, 1], -c[:, 0, 1], -c[:, 1, 0], c[:, 0, 0]], 1).reshape(-1, 2, 2)
    return inv / det


def gaussian_bounds(m, c, W, H, conf=3.0):
    rx = conf * torch.sqrt(c[:, 0, 0])
    ry = conf * torch.sqrt(c[:, 1, 1])
    return torch.stack([torch.clamp(m[:, 0] - rx, 0, W - 1), torch.clamp(m[:, 1] - ry, 0, H - 1),
                        torch.clamp(m[:, 0] + rx, 0, W - 1), torch.clamp(m[:, 1] + ry, 0, H - 1)], 1)


def splat_tile(params, idx, x0, y0, tw, th, fx, fy, px, py, R, W, H, nplanes, nch):
    cam, quats, scales, colours, phase, opac, pprobs = params
    if idx.numel() == 0:
        return torch.zeros((nplanes, nch, th, tw), dtype=torch.complex64)
    xs, ys = torch.meshgrid(torch.arange(x0, x0 + tw), torch.arange(y0, y0 + th), indexing="xy")
    pts = torch.stack([xs.flatten(), ys.flatten()], 1).float()
    tc = cam[idx]
    valid = (tc[:, 2] > 1.0) & (tc[:, 2] < 1000.0)
    idx = idx[valid]
    tc = tc[valid]
    tm = means_2d(tc, fx, fy, px, py).unsqueeze(1)
    diff = pts.unsqueeze(0) - tm
    c2 = cov_2d(tc, quats[idx], scales[idx], fx, fy, R, W, H)
    ci = invert_cov_2d(c2)
    term = torch.matmul(diff, ci)                 # compute_bmm_cuda
    term = (term * diff)                          # element_wise_multiplication_cuda
    term = term[..., 0] + term[..., 1]            # sum_last_dim_cuda
    term = term.view(-1, th, tw)
    gexp = torch.exp(-0.5 * term)
    base = opac[idx].view(-1, 1, 1) * gexp
    tp = pprobs[idx]
    out = []
    for p in range(nplanes):
        a = base * tp[:, p].view(-1, 1, 1)
        one = torch.ones((1, th, tw))
        T = torch.cumprod(torch.cat((one, 1.0 - a), 0), 0)[:-1]
        T = torch.where(T < 1e-4, torch.zeros_like(T), T)
        chans = []
        for c in range(nch):
            col = colours[idx, c].view(-1, 1, 1)
            ph = phase[idx, c].view(-1, 1, 1)
            chans.append(torch.sum(col * a * T * torch.exp(1j * ph), 0))
        out.append(torch.stack(chans, 0))
    return torch.stack(out, 0)


def asm_torch(field, wavelength, pitch, distance, S, aperture):
    M = 2 * S
    H, W = field.shape
    pad = torch.zeros((M, M), dtype=torch.complex64)
    r0, c0 = M // 2 - H // 2, M // 2 - W // 2
    pad = pad.index_put((torch.arange(r0, r0 + H)[:, None], torch.arange(c0, c0 + W)[None, :]),
                        field)
    yy, xx = torch.meshgrid(torch.arange(M), torch.arange(M), indexing="ij")
    ap = (((xx - M / 2) ** 2 + (yy - M / 2) ** 2) < aperture ** 2).float()
    ff = torch.fft.fftshift(torch.fft.fft2(pad))
    fx = torch.fft.fftshift(torch.fft.fftfreq(M, d=pitch))
    FX, FY = torch.meshgrid(fx, fx, indexing="ij")
    L = torch.tensor(pitch * M)
    d = torch.tensor(distance)
    lam = torch.tensor(wavelength)
    fxmax = 1 / torch.sqrt((2 * d * (1 / L)) ** 2 + 1) / lam
    mask = (torch.abs(FX) < fxmax) & (torch.abs(FY) < fxmax)
    k = 2 * torch.pi / lam
    kz = torch.sqrt(k ** 2 - (2 * torch.pi * FX) ** 2 - (2 * torch.pi * FY) ** 2)
    kz = torch.where(torch.isnan(kz), torch.zeros_like(kz), kz)
    Hf = torch.exp(1j * d * kz) * mask
    out = torch.fft.ifft2(torch.fft.ifftshift(ff * Hf * ap))
    s0 = M // 2 - S // 2
    return out[s0:s0 + S, s0:s0 + S]


def asm_torch_adjoint(grad, wavelength, pitch, distance, S, aperture, H, W):
    """The exact adjoint of ``asm_torch`` (a linear map of the field): the
    pure-torch ASM's autograd backward written out (python_function.py:35-78
    differentiated): pad the (S, S) gradient into the M x M grid, forward
    FFT, shift, multiply by the conjugate transfer function and aperture,
    unshift, inverse FFT, crop to (H, W).  Same FFT and elementwise work as
    a forward propagation."""
    M = 2 * S
    pad = torch.zeros((M, M), dtype=torch.complex64)
    s0 = M // 2 - S // 2
    pad = pad.index_put((torch.arange(s0, s0 + S)[:, None], torch.arange(s0, s0 + S)[None, :]),
                        grad)
    yy, xx = torch.meshgrid(torch.arange(M), torch.arange(M), indexing="ij")
    ap = (((xx - M / 2) ** 2 + (yy - M / 2) ** 2) < aperture ** 2).float()
    gf = torch.fft.fftshift(torch.fft.fft2(pad))
    fx = torch.fft.fftshift(torch.fft.fftfreq(M, d=pitch))
    FX, FY = torch.meshgrid(fx, fx, indexing="ij")
    L = torch.tensor(pitch * M)
    d = torch.tensor(distance)
    lam = torch.tensor(wavelength)
    fxmax = 1 / torch.sqrt((2 * d * (1 / L)) ** 2 + 1) / lam
    mask = (torch.abs(FX) < fxmax) & (torch.abs(FY) < fxmax)
    k = 2 * torch.pi / lam
    kz = torch.sqrt(k ** 2 - (2 * torch.pi * FX) ** 2 - (2 * torch.pi * FY) ** 2)
    kz = torch.where(torch.isnan(kz), torch.zeros_like(kz), kz)
    Hc = torch.exp(-1j * d * kz) * mask
    out = torch.fft.ifft2(torch.fft.ifftshift(gf * Hc * ap))
    r0, c0 = M // 2 - H // 2, M // 2 - W // 2
    return out[r0:r0 + H, c0:c0 + W]


def _cpu_params(sc, grad: bool):
    t = lambda a: torch.from_numpy(a.copy()).requires_grad_(grad)  # noqa: E731
    return [t(sc.cam_means), t(sc.quats), t(sc.scales), t(sc.colours), t(sc.phase), t(sc.opac),
            t(sc.pprobs)]


def run_frame(sc, backward: bool = True, cap_s: float = 600.0):
    """The whole CPU frame of scene ``sc``, not sampled: every 64x64 tile of
    the Python splat, every (plane, wavelength) pure-torch propagation and
    the sum over planes (Scene.splat, model.py:1194-1272), then (backward)
    autograd of Re<hologram, g> with the scene's upstream gradient g.
    Stops once ``cap_s`` seconds of wall time have passed (the protocol's
    did-not-finish cap).  Returns dict(finished, fwd_ms, bwd_ms, elapsed_s,
    tiles_done, tiles)."""
    spec = sc.spec
    W, H, P, C, S = spec.width, spec.height, spec.planes, len(spec.wavelengths), spec.size
    params = _cpu_params(sc, backward)
    R = torch.from_numpy(sc.view.copy())
    fx, fy, px, py = sc.fx, sc.fy, sc.px, sc.py
    tile = 64
    xt, yt = math.ceil(W / tile), math.ceil(H / tile)
    t0 = time.perf_counter()
    res = dict(finished=False, fwd_ms=None, bwd_ms=None, tiles=xt * yt, tiles_done=0)
    with torch.set_grad_enabled(backward):
        with torch.no_grad():
            m = means_2d(params[0], fx, fy, px, py)
            c2 = cov_2d(params[0], params[1], params[2], fx, fy, R, W, H)
            bounds = gaussian_bounds(m, c2, W, H)
        rows = []
        for yi in range(yt):
            row = []
            for xi in range(xt):
                x, y = xi * tile, yi * tile
                tw, th = min(tile, W - x), min(tile, H - y)
                sel = ((bounds[:, 0] <= x + tw - 1) & (bounds[:, 2] >= x) &
                       (bounds[:, 1] <= y + th - 1) & (bounds[:, 3] >= y))
                row.append(splat_tile(params, torch.where(sel)[0], x, y, tw, th, fx, fy, px, py,
                                      R, W, H, P, C))
                res["tiles_done"] += 1
                if time.perf_counter() - t0 > cap_s:
                    res["elapsed_s"] = time.perf_counter() - t0
                    return res
            rows.append(torch.cat(row, dim=3))
        field = torch.cat(rows, dim=2)  # (P, C, H, W)
        holo = []
        for c in range(C):
            acc = None
            for p in range(P):
                o = asm_torch(field[p, c], spec.wavelengths[c], 3.74e-6, -spec.distances[p], S,
                              float(S))
                acc = o if acc is None else acc + o
            holo.append(acc)
            if time.perf_counter() - t0 > cap_s:
                res["elapsed_s"] = time.perf_counter() - t0
                return res
        holo = torch.stack(holo, 0)
    t1 = time.perf_counter()
    res["fwd_ms"] = (t1 - t0) * 1e3
    if backward:
        g = torch.from_numpy(sc.grad_holo.copy())
        (holo.real * g.real + holo.imag * g.imag).sum().backward()
        res["bwd_ms"] = (time.perf_counter() - t1) * 1e3
        res["grads"] = [q.grad for q in params]
    res["elapsed_s"] = time.perf_counter() - t0
    res["finished"] = res["elapsed_s"] <= cap_s
    res["hologram"] = holo.detach()
    return res


def run_frame_tiled(sc, cap_s: float = 600.0, progress=None):
    """The whole CPU frame of scene ``sc``, forward and backward, with the
    backward run tile by tile so that it fits in host memory (the whole
    graph of every 64x64 tile's per-(Gaussian, pixel) tensors would hold
    ~1e2 GB at 3e5 Gaussians).  The frame's loss Re<hologram, g> is linear
    in the plane fields, so their gradient is the propagation's adjoint of g
    whatever the fields are: it is formed first (asm_torch_adjoint per
    (plane, wavelength), summed into the plane field gradients), then each
    tile runs its forward with autograd and its backward with its slice of
    that gradient, and frees its graph; the propagation forward of the
    assembled fields gives the hologram.  The same operations as run_frame's
    forward + backward, in a different order.  Forward time: the tiles'
    forwards + the propagations; backward time: the adjoints + the tiles'
    backwards.  Stops at ``cap_s`` seconds of wall time (did not finish).
    ``progress`` (optional) is called with (tiles done, tiles) after each
    row of tiles.  Returns dict(finished, fwd_ms, bwd_ms, elapsed_s,
    tiles_done, tiles, grads (the 7 parameter gradients), hologram)."""
    spec = sc.spec
    W, H, P, C, S = spec.width, spec.height, spec.planes, len(spec.wavelengths), spec.size
    params = _cpu_params(sc, True)
    R = torch.from_numpy(sc.view.copy())
    fx, fy, px, py = sc.fx, sc.fy, sc.px, sc.py
    tile = 64
    xt, yt = math.ceil(W / tile), math.ceil(H / tile)
    res = dict(finished=False, fwd_ms=None, bwd_ms=None, tiles=xt * yt, tiles_done=0)
    t_start = time.perf_counter()
    fwd = bwd = 0.0
    g = torch.from_numpy(sc.grad_holo.copy())
    t0 = time.perf_counter()
    with torch.no_grad():
        gfield = torch.zeros((P, C, H, W), dtype=torch.complex64)
        for p in range(P):
            for c in range(C):
                gfield[p, c] = asm_torch_adjoint(g[c], spec.wavelengths[c], 3.74e-6,
                                                 -spec.distances[p], S, float(S), H, W)
    bwd += time.perf_counter() - t0
    with torch.no_grad():
        m = means_2d(params[0], fx, fy, px, py)
        c2 = cov_2d(params[0], params[1], params[2], fx, fy, R, W, H)
        bounds = gaussian_bounds(m, c2, W, H)
    field = torch.zeros((P, C, H, W), dtype=torch.complex64)
    for yi in range(yt):
        for xi in range(xt):
            x, y = xi * tile, yi * tile
            tw, th = min(tile, W - x), min(tile, H - y)
            t0 = time.perf_counter()
            sel = ((bounds[:, 0] <= x + tw - 1) & (bounds[:, 2] >= x) &
                   (bounds[:, 1] <= y + th - 1) & (bounds[:, 3] >= y))
            out = splat_tile(params, torch.where(sel)[0], x, y, tw, th, fx, fy, px, py, R, W, H,
                             P, C)
            t1 = time.perf_counter()
            if out.requires_grad:
                gt = gfield[:, :, y:y + th, x:x + tw]
                (out.real * gt.real + out.imag * gt.imag).sum().backward()
            t2 = time.perf_counter()
            fwd += t1 - t0
            bwd += t2 - t1
            field[:, :, y:y + th, x:x + tw] = out.detach()
            del out
            res["tiles_done"] += 1
            if time.perf_counter() - t_start > cap_s:
                res["elapsed_s"] = time.perf_counter() - t_start
                return res
        if progress:
            progress(res["tiles_done"], res["tiles"])
    t0 = time.perf_counter()
    with torch.no_grad():
        holo = []
        for c in range(C):
            acc = None
            for p in range(P):
                o = asm_torch(field[p, c], spec.wavelengths[c], 3.74e-6, -spec.distances[p], S,
                              float(S))
                acc = o if acc is None else acc + o
            holo.append(acc)
        holo = torch.stack(holo, 0)
    fwd += time.perf_counter() - t0
    res["fwd_ms"] = fwd * 1e3
    res["bwd_ms"] = bwd * 1e3
    res["elapsed_s"] = time.perf_counter() - t_start
    res["finished"] = res["elapsed_s"] <= cap_s
    res["grads"] = [q.grad for q in params]
    res["hologram"] = holo
    return res


def time_propagations(jobs, S, aperture, pitch=3.74e-6, seed=0):
    """Every pure-torch propagation of ``jobs`` (a list of (field (H, W)
    complex64, wavelength, distance)) forward, then its backward by autograd
    with a seeded CN(0,1) upstream gradient, one after another (not
    sampled).  Returns (forward ms, backward ms) summed over the jobs."""
    gen = torch.Generator().manual_seed(seed)
    fwd = bwd = 0.0
    for field, wl, d in jobs:
        f = field.detach().clone().requires_grad_(True)
        t0 = time.perf_counter()
        o = asm_torch(f, wl, pitch, d, S, aperture)
        t1 = time.perf_counter()
        g = torch.complex(torch.randn(o.shape, generator=gen), torch.randn(o.shape, generator=gen))
        (o.real * g.real + o.imag * g.imag).sum().backward()
        t2 = time.perf_counter()
        fwd += (t1 - t0) * 1e3
        bwd += (t2 - t1) * 1e3
    return fwd, bwd


def time_frame(sc, budget_s: float = 12.0, seed: int = 0):
    """ESTIMATE of the CPU path's time for one frame of scene ``sc`` from a
    bounded sample (for frames far beyond the did-not-finish cap): random
    64x64 tiles forward+backward until the budget is spent, scaled by the
    ratio of all tiles' selected-Gaussian counts to the sampled tiles'
    counts (the tile cost grows with the Gaussians it evaluates), plus the
    per-frame projection setup and one propagation forward+backward scaled
    by P*C.  Returns (ms_per_frame_estimate, sample description)."""
    torch.manual_seed(seed)
    spec = sc.spec
    W, H, P, C = spec.width, spec.height, spec.planes, len(spec.wavelengths)
    t = lambda a: torch.from_numpy(a.copy())  # noqa: E731
    params = [t(sc.cam_means).requires_grad_(True), t(sc.quats).requires_grad_(True),
              t(sc.scales).requires_grad_(True), t(sc.colours).requires_grad_(True),
              t(sc.phase).requires_grad_(True), t(sc.opac).requires_grad_(True),
              t(sc.pprobs).requires_grad_(True)]
    R = t(sc.view)
    fx, fy, px, py = sc.fx, sc.fy, sc.px, sc.py
    tile = 64
    xt, yt = math.ceil(W / tile), math.ceil(H / tile)
    order = torch.randperm(xt * yt).tolist()
    # Per-frame setup the reference runs once: means/cov/bounds for all Gaussians.
    t0 = time.perf_counter()
    with torch.no_grad():
        m = means_2d(params[0], fx, fy, px, py)
        c2 = cov_2d(params[0], params[1], params[2], fx, fy, R, W, H)
        bounds = gaussian_bounds(m, c2, W, H)
    setup_s = time.perf_counter() - t0
    # Gaussians each tile evaluates (tile pixels x selected Gaussians)
    work = []
    for ti in range(xt * yt):
        yi, xi = divmod(ti, xt)
        x, y = xi * tile, yi * tile
        tw, th = min(tile, W - x), min(tile, H - y)
        sel = ((bounds[:, 0] <= x + tw - 1) & (bounds[:, 2] >= x) & (bounds[:, 1] <= y + th - 1) &
               (bounds[:, 3] >= y))
        work.append(float(sel.sum()) * tw * th)
    done = 0
    raster_s = 0.0
    work_done = 0.0
    for ti in order:
        yi, xi = divmod(ti, xt)
        x, y = xi * tile, yi * tile
        tw, th = min(tile, W - x), min(tile, H - y)
        sel = ((bounds[:, 0] <= x + tw - 1) & (bounds[:, 2] >= x) & (bounds[:, 1] <= y + th - 1) &
               (bounds[:, 3] >= y))
        idx = torch.where(sel)[0]
        work_done += work[ti]
        t1 = time.perf_counter()
        out = splat_tile(params, idx, x, y, tw, th, fx, fy, px, py, R, W, H, P, C)
        if out.requires_grad:
            g = torch.randn(out.shape, dtype=torch.complex64)
            (out.real * g.real + out.imag * g.imag).sum().backward()
        raster_s += time.perf_counter() - t1
        done += 1
        if raster_s > budget_s * 0.7:
            break
    raster_frame_s = raster_s * (sum(work) / work_done if work_done > 0 else (xt * yt) / done)
    # ASM: one (plane, wavelength) propagation forward+backward, times P*C.
    f = torch.randn((H, W), dtype=torch.complex64).requires_grad_(True)
    S = spec.size
    t2 = time.perf_counter()
    o = asm_torch(f, spec.wavelengths[0], 3.74e-6, -spec.distances[0], S, float(S))
    g = torch.randn(o.shape, dtype=torch.complex64)
    (o.real * g.real + o.imag * g.imag).sum().backward()
    asm_one_s = time.perf_counter() - t2
    total_s = setup_s + raster_frame_s + asm_one_s * P * C
    desc = (f"ESTIMATE from a sample: reference CPU PyTorch path restated "
            f"(oracle/cpu_baseline.py), {done} of {xt * yt} random 64x64 tiles fwd+bwd scaled "
            f"by the tiles' selected-Gaussian work ({work_done / max(sum(work), 1):.1%} of the "
            f"frame's), 1 of {P * C} ASM fwd+bwd scaled by P*C, projection setup; "
            f"{spec.name} N={sc.cam_means.shape[0]}")
    return total_s * 1000.0, desc


# ------------------------------------------------- render preprocess (glue)
class _STE(torch.autograd.Function):
    """STEFunction (model.py:41-56): one-hot forward, softmax(x/0.001) backward."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return torch.nn.functional.one_hot(torch.argmax(x, dim=1), num_classes=x.size(1)).float()

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        return g * torch.nn.functional.softmax(x / 0.001, dim=1)


def preprocess_torch(means, pq, ps, col, ph, po, pp, R, T, near=1.0, far=1000.0):
    """Scene.render's steps before splat, as the reference runs them
    (model.py:1377-1402, 1105-1125, 594-608; the transform of Scene.splat,
    model.py:1161-1162), on CPU torch.  Returns the rasterizer inputs."""
    import torch.nn.functional as F

    z_all = (means @ R + T)[:, -1]
    valid = torch.where((z_all > near) & (z_all < far))[0]
    srt, ind = torch.sort(z_all[valid].detach())
    idxs = valid[torch.masked_select(ind, srt >= 0)]
    m = means[idxs]
    cam = m @ R + T
    return (cam, (m @ R + T)[:, -1], F.normalize(pq[idxs]), torch.exp(ps[idxs]), col[idxs],
            ph[idxs] % (2.0 * math.pi), torch.sigmoid(po[idxs]), _STE.apply(pp[idxs]), idxs)


def time_preprocess(params: dict, reps: int = 2):
    """Forward + backward (sum of the outputs as the loss) of preprocess_torch
    over the given numpy parameters; returns (fwd_ms, bwd_ms)."""
    leaves = [torch.from_numpy(params[k].copy()).requires_grad_(True) for k in
              ("means", "pre_quats", "pre_scales", "colours", "pre_phase", "pre_opac",
               "pre_plane")]
    R, T = torch.from_numpy(params["R"]), torch.from_numpy(params["T"])
    fwd, bwd = [], []
    for _ in range(reps):
        for x in leaves:
            x.grad = None
        t0 = time.perf_counter()
        out = preprocess_torch(*leaves, R, T)
        t1 = time.perf_counter()
        sum(o.sum() for o in out[:-1]).backward()
        t2 = time.perf_counter()
        fwd.append((t1 - t0) * 1e3)
        bwd.append((t2 - t1) * 1e3)
    return min(fwd), min(bwd)


# ------------------------------------------------------- optimizer step
def adan_foreach_torch(params, grads, states, lrs, step, betas=(0.98, 0.92, 0.99), eps=1e-8):
    """The reference's clip + Adan step on CPU torch: clip_grad_norm_
    (train.py:319) then the foreach sequence of _multi_tensor_adan
    (utils/optimizer.py:538-589), one parameter group per tensor."""
    b1, b2, b3 = betas
    for p, g in zip(params, grads):
        p.grad = g
    torch.nn.utils.clip_grad_norm_(params, 1.0)
    for i, p in enumerate(params):
        m, n, d, q = states[i]
        g = [p.grad]
        if step == 1:
            q.copy_(p.grad).mul_(-1.0)
        bc1, bc2, bc3 = 1 - b1 ** step, 1 - b2 ** step, 1 - b3 ** step
        torch._foreach_mul_(g, 1.0)
        torch._foreach_add_([q], g)
        torch._foreach_mul_([m], b1)
        torch._foreach_add_([m], g, alpha=1 - b1)
        torch._foreach_mul_([d], b2)
        torch._foreach_add_([d], [q], alpha=1 - b2)
        torch._foreach_mul_([q], b2)
        torch._foreach_add_([q], g)
        torch._foreach_mul_([n], b3)
        torch._foreach_addcmul_([n], [q], [q], value=1 - b3)
        denom = torch._foreach_sqrt([n])
        torch._foreach_div_(denom, math.sqrt(bc3))
        torch._foreach_add_(denom, eps)
        torch._foreach_addcdiv_([p.data], [m], denom, value=-lrs[i] / bc1)
        torch._foreach_addcdiv_([p.data], [d], denom, value=-lrs[i] * b2 / bc2)
        torch._foreach_div_([p.data], 1.0)
        torch._foreach_zero_([q])
        torch._foreach_add_([q], g, alpha=-1.0)


def time_adan(shapes, lrs, reps: int = 3):
    """Best-of-reps time (ms) of one clip + Adan step over
    parameter tensors of the given shapes on CPU torch."""
    gen = torch.Generator().manual_seed(0)
    params = [torch.randn(s, generator=gen) for s in shapes]
    states = [[torch.zeros(s) for _ in range(4)] for s in shapes]
    best = float("inf")
    for k in range(1, reps + 1):
        grads = [torch.randn(s, generator=gen) * 0.1 for s in shapes]
        t0 = time.perf_counter()
        adan_foreach_torch(params, grads, states, lrs, k)
        best = min(best, (time.perf_counter() - t0) * 1e3)
    return best
