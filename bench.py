#!/usr/bin/env python3
"""Benchmark: fwd+bwd ms/frame of the holographic hot path on one MI355X.

A step (frame) = rasterizer forward (projection, binning, complex tile
render) + multi-plane band-limited ASM to the (C,S,S) hologram, then the ASM
adjoint of a CN(0,1) hologram gradient + rasterizer backward to the 8
Gaussian gradients.  Default workload: the BASELINE.json headline, 1M
Gaussians at 800x800, 3 planes, 3 wavelengths, synthetic seeded scene.

Prints ONE JSON line (see the repository contract).  Per-stage times are
measured live with hipEvents recorded by the library on the stream each
stage runs on (hrf_trace_*), over the same timed steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

METRIC = "fwd+bwd ms/frame, 1M Gaussians @800x800, 3 planes; % HBM roofline"
HBM_PEAK_GBS = 8000.0
STAGES = ["project", "depth_sort", "scan", "emit", "tile_sort", "ranges", "render_fwd",
          "render_bwd", "geom_bwd", "asm_rows_in", "asm_col_fwd", "asm_col_adj",
          "asm_rows_out", "asm_pad", "asm_fft", "asm_mac_fwd", "asm_mac_adj", "asm_crop"]


# Stage -> kernel name in the rocprofv3 summaries under profiles/.
STAGE_KERNEL = {"render_bwd": "k_render_bwd<{C}, true>", "render_fwd": "k_render_fwd<{C}>",
                "project": "k_project", "geom_bwd": "k_geom_backward",
                # the headline's variants: zero-padded inputs at most half the grid
                "asm_col_fwd": "k_col_fwd<{M}, true>", "asm_col_adj": "k_col_adj<{M}, true>",
                "asm_rows_in": "k_rows_in<{M}, true>", "asm_rows_out": "k_rows_out<{M}>",
                "emit": "k_emit_packed<false, false>", "ranges": "k_tile_diff"}


def profiled_traffic(config, stage, C, M):
    """HBM bytes per dispatch of `stage`'s kernel from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary of this workload (calibrated
    against a copy kernel of known size), or None."""
    path = os.path.join(REPO, "profiles", f"hbm_traffic_{config}.txt")
    name = STAGE_KERNEL.get(stage, "").format(C=C, M=M)
    if not name or not os.path.exists(path):
        return None, None
    with open(path) as f:
        for line in f:
            # "traffic <kernel name, may hold spaces> <bytes>"
            if not line.startswith("traffic "):
                continue
            head, _, val = line.rstrip().rpartition(" ")
            if head[len("traffic "):] == name:
                return int(val), os.path.relpath(path, REPO)
    return None, None


def profiled_valu(config, stage, C, M):
    """VALU issue model of `stage`'s kernel from the committed rocprofv3
    summary of this workload, or None: a dict with the wave-instruction and
    transcendental counts per dispatch, the issue peak (the published FP32
    vector peak in wave64 instructions/s), the extra issue slots a
    transcendental takes, and the measured rate of the forward's own member
    loop (a calibration kernel with no memory traffic or barriers; its rate
    per shader cycle at the forward kernel's clock in the same counter
    run)."""
    path = os.path.join(REPO, "profiles", f"valu_{config}.txt")
    name = STAGE_KERNEL.get(stage, "").format(C=C, M=M)
    if not name or not os.path.exists(path):
        return None
    row, keys = None, {}
    with open(path) as f:
        for line in f:
            parts = line.split()
            if len(parts) == 2 and parts[0] in ("valu_peak", "trans_extra_slots", "fwdloop_rate"):
                keys[parts[0]] = float(parts[1])
            elif not line.startswith("#") and line.startswith(name + " "):
                # columns after the name: n, waves, valu, trans, salu, lds, ...
                rest = line[len(name):].split()
                if len(rest) >= 4:
                    row = (int(float(rest[2])), int(float(rest[3])))
    if row is None or len(keys) < 3:
        return None
    return {"valu": row[0], "trans": row[1], **keys}


def algorithmic_bytes(N, K, P, C, W, H, S, T):
    """Compulsory-dataflow byte model per frame and per stage launch.

    Frame model (the metric's definition): each tensor crosses HBM once per
    producer and once per consumer; index maps (shift, pad, crop) are free; a
    2-D FFT is one read + one write of its M x M complex64 grid.  g_in =
    48+4P+8C bytes of Gaussian inputs, g_rec = 32+4P+8C bytes of per-Gaussian
    render record.

    The propagation kernels here move fewer bytes than that frame model
    counts: an M x M grid (20 MB at M = 1600) does not fit on chip, so a 2-D
    transform needs one intermediate written and read once, and only the H
    nonzero rows of a padded field (the S kept rows of an output) exist.  The
    rows pass writes (P*C, H, M) row spectra; the column pass (FFT, transfer
    multiply summed over planes, inverse FFT, row crop) writes (C, S, M); the
    inverse rows pass writes (C, S, S); the adjoint mirrors it.  The
    per-launch figures of the asm_* kernels and `fused` use this dataflow.
    """
    M = 2 * S
    g_in = 48 + 4 * P + 8 * C
    g_rec = 32 + 4 * P + 8 * C
    RF = N * g_in + 64 * N + 48 * K + N * g_rec + 8 * P * C * W * H + 8 * P * W * H
    RB = (8 * P * C * W * H + 8 * P * W * H + 4 * K + N * g_rec + N * (28 + 4 * P + 8 * C) +
          104 * N)
    AF = P * C * (8 * W * H + 32 * M * M) + C * (16 * M * M + 8 * S * S)
    AB = C * (8 * S * S + 16 * M * M) + P * C * (32 * M * M + 8 * W * H)
    pcx = 8 * P * C * H * M      # row spectra of the P*C fields
    csz = 8 * C * S * M          # column-pass output / adjoint row spectra
    AF_fused = 8 * P * C * W * H + 2 * pcx + 2 * csz + 8 * C * S * S
    AB_fused = 8 * C * S * S + 2 * csz + 2 * pcx + 8 * P * C * W * H
    per_launch = {
        # the render kernels' terms of RF and RB exactly: the forward reads
        # the point list (4K) and the records and writes the fields, final_T
        # and n_contrib; the backward reads the upstream fields, final_T,
        # n_contrib, the point list and the records and writes the
        # per-Gaussian render gradients.  (This build's forward also writes
        # per-plane member lists that its backward reads instead of the point
        # list; the model does not count them.)
        "render_fwd": 4 * K + N * g_rec + 8 * P * C * W * H + 8 * P * W * H,
        "render_bwd": (8 * P * C * W * H + 8 * P * W * H + 4 * K + N * g_rec +
                       N * (28 + 4 * P + 8 * C)),
        "project": N * g_in + N * (g_rec + 24),
        "geom_bwd": N * g_in + N * (20 + 4 * P + 8 * C) + N * (40 + 4 * P + 8 * C),
        # row launches alternate forward (P*C fields) and adjoint (C holograms):
        "asm_rows_in": (8 * P * C * W * H + pcx + 8 * C * S * S + csz) / 2,
        "asm_rows_out": (csz + 8 * C * S * S + pcx + 8 * P * C * W * H) / 2,
        "asm_col_fwd": pcx + csz,
        "asm_col_adj": csz + pcx,
        "tile_sort": 2 * 16 * K,
        "depth_sort": 4 * 16 * N,
    }
    return dict(RF=RF, RB=RB, AF=AF, AB=AB, total=RF + RB + AF + AB,
                fused_fwd=RF + AF_fused, fused_total=RF + RB + AF_fused + AB_fused,
                per_launch=per_launch)


def measure_preprocess(spec, dev, no_cpu):
    """The fused Scene.render glue (hrf_preprocess_*) on the same scene as
    model parameters: forward (selection + gathers + activations) and
    backward, timed with hipEvents; not part of the frame (the metric starts
    at the rasterizer's inputs).  Compulsory bytes: forward reads the means
    (12 B per Gaussian) and the selected rows' parameters and writes the
    rasterizer inputs; backward reads the output gradients and the selected
    parameters and writes the N parameter-gradient rows."""
    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import preprocess, scenes

    p = scenes.generate_params(spec)
    keys = ("means", "pre_quats", "pre_scales", "colours", "pre_phase", "pre_opac", "pre_plane")
    t = {k: torch.from_numpy(np.ascontiguousarray(p[k])).to(dev) for k in keys + ("R", "T")}
    args = [t[k] for k in keys]
    N, C, P = p["means"].shape[0], p["colours"].shape[1], p["pre_plane"].shape[1]

    def fwd():
        return preprocess.forward(*args, t["R"], t["T"], scenes.NEAR, scenes.FAR)

    out = fwd()
    M = int(out[-1].numel())
    grads = [torch.ones_like(o) for o in out[:-1]]

    def bwd(o):
        return preprocess.backward(grads, *args, t["R"], o[-1])

    for _ in range(3):
        bwd(fwd())
    torch.cuda.synchronize()
    reps = 20
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
    f_ms, b_ms = [], []
    for _ in range(reps):
        ev[0].record()
        o = fwd()
        ev[1].record()
        bwd(o)
        ev[2].record()
        torch.cuda.synchronize()
        f_ms.append(ev[0].elapsed_time(ev[1]))
        b_ms.append(ev[1].elapsed_time(ev[2]))
    f_ms, b_ms = float(np.median(f_ms)), float(np.median(b_ms))
    row_in = 16 + 12 + 8 * C + 4 + 4 * P + 12        # selected parameter row read
    row_out = 12 + 4 + 16 + 12 + 8 * C + 4 + 4 * P + 8  # rasterizer inputs + idx written
    fwd_b = 12 * N + M * (row_in + row_out)
    bwd_b = M * (row_out + 16 + 12 + 4 + 4 * P) + N * (12 + 16 + 12 + 8 * C + 4 + 4 * P)
    ach = (fwd_b + bwd_b) / ((f_ms + b_ms) * 1e-3) / 1e9
    res = {"workload": f"{spec.name} parameters: {N} Gaussians, {M} selected",
           "fwd_ms": round(f_ms, 4), "bwd_ms": round(b_ms, 4),
           "timing": f"median of {reps} (forward includes its count read-back)",
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                        "alg_bytes": int(fwd_b + bwd_b)},
           "cpu_torch": None}
    if not no_cpu:
        try:
            from oracle import cpu_baseline

            cf, cb = cpu_baseline.time_preprocess(p)
            res["cpu_torch"] = {"fwd_ms": round(cf, 1), "bwd_ms": round(cb, 1),
                                "cores": torch.get_num_threads(),
                                "kind": "reference op sequence on CPU torch "
                                        "(oracle/cpu_baseline.py), full N, best of 2"}
        except Exception as e:  # reported, never fatal to the GPU measurement
            res["cpu_torch"] = {"failed": repr(e)}
    return res


def measure_optimizer(spec, dev, no_cpu):
    """The training step's optimizer side (train.py:319-324): gradient-norm
    clip + Adan over the seven parameter tensors of the headline scene
    (utils/optimizer.py:46-54 learning rates), as two HIP passes (norm, then
    the update with the clip coefficient applied inside it), timed with
    hipEvents.  Compulsory bytes: the norm reads every gradient (4 B per
    element); the update reads and writes param, grad and the four state
    tensors (48 B per element)."""
    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import optim

    N, C, P = spec.n, len(spec.wavelengths), spec.planes
    groups = [("scales", 0.005, 3), ("phase", 0.0025, C), ("colours", 0.0025, C),
              ("means", 1e-3, 3), ("opacity", 0.025, 1), ("plane assignment", 1e-3, P),
              ("rot", 0.001, 4)]
    gen = torch.Generator(device=dev).manual_seed(0)
    ps = [torch.randn((N, k), generator=gen, device=dev).requires_grad_() for _, _, k in groups]
    for p in ps:
        p.grad = torch.randn(p.shape, generator=gen, device=dev) * 0.1
    opt = optim.Adan([{"params": [p], "lr": lr, "name": nm} for p, (nm, lr, _) in zip(ps, groups)],
                     lr=0, eps=1e-8)
    for _ in range(3):
        optim.training_step_update(opt, ps, 1.0)
    torch.cuda.synchronize()
    reps = 20
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ms = []
    for _ in range(reps):
        ev[0].record()
        optim.training_step_update(opt, ps, 1.0)
        ev[1].record()
        torch.cuda.synchronize()
        ms.append(ev[0].elapsed_time(ev[1]))
    ms = float(np.median(ms))
    E = sum(p.numel() for p in ps)
    alg = 4 * E + 48 * E
    ach = alg / (ms * 1e-3) / 1e9
    res = {"workload": f"{spec.name} parameters: 7 tensors, {E} elements (N={N})",
           "ms": round(ms, 4), "timing": f"median of {reps}, clip + Adan step",
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "alg_bytes": alg},
           "cpu_torch": None}
    if not no_cpu:
        try:
            from oracle import cpu_baseline

            cms = cpu_baseline.time_adan([(N, k) for _, _, k in groups],
                                         [lr for _, lr, _ in groups])
            res["cpu_torch"] = {"ms": round(cms, 1), "cores": torch.get_num_threads(),
                                "kind": "reference clip_grad_norm_ + _multi_tensor_adan on "
                                        "CPU torch (oracle/cpu_baseline.py), full N, best of 3"}
        except Exception as e:  # reported, never fatal to the GPU measurement
            res["cpu_torch"] = {"failed": repr(e)}
    return res


def measure_reconstruction(spec, dev, no_cpu):
    """The loss side right after the hologram (train.py:272-282): the
    training propagator (3 frames, laser powers eye(3), one depth per plane
    distance, band-limited ASM) reconstructs the (3, S, S) phase and
    amplitude maps and backpropagates a synthetic intensity gradient.
    Byte model: config 3's (every M x M transform one read + one write),
    with K = 3 lit (frame, channel) pairs and D depths, plus the elementwise
    passes (fields, intensities and their backward)."""
    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import scenes
    from complex_valued_holographic_radiance_fields_amd.reconstruction import Propagator

    S, M = spec.size, 2 * spec.size
    dist = [float(d) for d in spec.distances]  # args_prop.distances (train.py:859-866)
    K, D = 3, len(dist)
    prop = Propagator(resolution=[S, S], wavelengths=spec.wavelengths, pixel_pitch=scenes.PITCH,
                      number_of_frames=3, propagator_type="forward", distances=dist,
                      aperture_size=float(S))
    gen = torch.Generator(device=dev).manual_seed(3)
    ph = (torch.rand((3, S, S), generator=gen, device=dev) * 6.28 - 3.14).requires_grad_(True)
    am = torch.rand((3, S, S), generator=gen, device=dev).requires_grad_(True)
    g = torch.randn((3, D, 3, S, S), generator=gen, device=dev)

    def step():
        out = prop.reconstruct(ph, am, no_grad=False)
        torch.autograd.backward(out, g)

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    reps = 10
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    ev[0].record()
    for _ in range(reps):
        step()
    ev[1].record()
    torch.cuda.synchronize()
    ms = ev[0].elapsed_time(ev[1]) / reps
    fwd_b = K * (8 * S * S + 16 * M * M) + D * K * (32 * M * M + 8 * S * S)
    adj_b = D * K * (8 * S * S + 32 * M * M) + K * (16 * M * M + 8 * S * S)
    elem = K * S * S * (8 + 8) + D * K * S * S * (8 + 4) + D * K * S * S * (8 + 4 + 8) \
        + K * S * S * (8 + 8 + 8)
    alg = fwd_b + adj_b + elem
    ach = alg / (ms * 1e-3) / 1e9
    res = {"workload": f"{spec.name}: 3 frames x 3 channels (eye powers), {D} depths, "
                       f"{S}x{S} on the {M} grid, fwd+bwd",
           "ms": round(ms, 4), "timing": f"mean of {reps} (hipEvents)",
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "alg_bytes": alg},
           "transfer_function": "the reference's band-limited ASM (odak's kernel unavailable)",
           "cpu_torch": None}
    if not no_cpu:
        try:
            from oracle import cpu_baseline

            torch.set_num_threads(len(os.sched_getaffinity(0)))
            gen_c = torch.Generator().manual_seed(3)
            jobs = [(torch.complex(torch.rand((S, S), generator=gen_c),
                                   torch.rand((S, S), generator=gen_c)), spec.wavelengths[k],
                     d) for k in range(K) for d in dist]
            cf, cb = cpu_baseline.time_propagations(jobs, S, float(S), scenes.PITCH)
            res["cpu_torch"] = {"ms": round(cf + cb, 1), "fwd_ms": round(cf, 1),
                                "bwd_ms": round(cb, 1), "cores": torch.get_num_threads(),
                                "kind": f"all {D * K} pure-torch ASM propagations "
                                        "(oracle/cpu_baseline.py) forward + autograd backward, "
                                        "not sampled"}
        except Exception as e:  # reported, never fatal to the GPU measurement
            res["cpu_torch"] = {"failed": repr(e)}
    return res


CPU_CAP_S = 600.0


def cpu_baseline_leg(spec, sc, budget_s):
    """The reference's CPU PyTorch path (oracle/cpu_baseline.py) on this
    host's cores: config 0 (forward only) run in full, median of 3, and, for
    a larger workload, an ESTIMATE of its frame from a bounded sample, kept
    under its own key (never `value`): the whole frame would take minutes
    of host time, more than the bench's budget."""
    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import scenes

    try:
        from oracle import cpu_baseline

        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        sc0 = sc if spec.name == "cfg0" else scenes.generate(scenes.config("cfg0"))
        runs = [cpu_baseline.run_frame(sc0, backward=False, cap_s=CPU_CAP_S) for _ in range(3)]
        ok = all(r["finished"] for r in runs)
        cfg0 = {"fwd_ms": round(float(np.median([r["fwd_ms"] for r in runs])), 1) if ok else None,
                "finished": ok, "cores": cores,
                "run": "config 0 in full (10k Gaussians, 256x256, P=C=1, forward only: every "
                       "64x64 tile of the Python splat and the propagation), median of 3"}
        if spec.name == "cfg0":
            return {"value": cfg0["fwd_ms"], "unit": "ms/frame", "cores": cores, "kind": "port",
                    "sample": "the whole frame (not sampled): " + cfg0["run"], "config0": cfg0}
        est_ms, desc = cpu_baseline.time_frame(sc, budget_s=budget_s)
        out = {"value": None, "unit": "ms/frame", "cores": cores, "kind": "port",
               "sample": f"the {spec.name} frame on the reference's CPU PyTorch path "
                         "(oracle/cpu_baseline.py) is not run whole by the bench (about "
                         f"{est_ms / 60e3:.0f} min of host time by the estimate below, "
                         "against a bench budget of minutes); config 0 is run whole",
               "estimate_ms_per_frame": round(est_ms, 1), "estimate_from": desc,
               "config0": cfg0}
        whole = committed_cpu_frame(spec.name)
        if whole:
            out["whole_frame"] = whole
        return out
    except Exception as e:  # reported, never fatal to the GPU measurement
        return {"value": None, "unit": "ms/frame", "cores": None, "kind": "port",
                "sample": f"failed: {e!r}"}


def committed_cpu_frame(name):
    """The whole-frame CPU measurement of this workload committed under
    profiles/ (`bench.py --cpu-frame NAME` on a GPU box's host), or None."""
    path = os.path.join(REPO, "profiles", f"cpu_baseline_{name}.txt")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        rows = [l for l in f if l.startswith("{")]
    if not rows:
        return None
    d = json.loads(rows[-1])
    return {"value": d.get("value"), "unit": d.get("unit"), "cores": d.get("cores"),
            "did_not_finish": d.get("did_not_finish"), "kind": d.get("kind"),
            "source": os.path.relpath(path, REPO),
            "command": f"python bench.py --cpu-frame {name}"}


def cpu_whole_frame(name):
    """One whole frame of a BASELINE configuration on the reference's CPU
    PyTorch path (oracle/cpu_baseline.py) on all of this host's cores, under
    the protocol's 600 s did-not-finish cap; never sampled or extrapolated.
    Configurations with a backward run it tile by tile (run_frame_tiled: the
    whole graph would not fit in host memory); config 3 runs its 24
    propagations (3 wavelengths x 8 distances, 2048^2 fields on the 4096 grid)
    forward + backward one after another."""
    import torch

    from complex_valued_holographic_radiance_fields_amd import scenes
    from oracle import cpu_baseline

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t0 = time.perf_counter()
    if name in ("cfg3", "3"):
        field, wl, dist = scenes.cfg3_fields()
        C, S = field.shape[0], field.shape[1]
        fwd = bwd = 0.0
        done = 0
        finished = True
        for d in dist:
            for c in range(C):
                f, b = cpu_baseline.time_propagations(
                    [(torch.from_numpy(field[c]), wl[c], d)], S, float(S), pitch=scenes.PITCH,
                    seed=done)
                fwd += f
                bwd += b
                done += 1
                print(f"[cpu cfg3] propagation {done}/{len(dist) * C}: {f + b:.0f} ms",
                      file=sys.stderr, flush=True)
                if time.perf_counter() - t0 > CPU_CAP_S:
                    finished = False
                    break
            if not finished:
                break
        res = dict(finished=finished, fwd_ms=fwd if finished else None,
                   bwd_ms=bwd if finished else None, propagations_done=done,
                   propagations=len(dist) * C)
        run = ("config 3 whole: 24 pure-torch propagations (python_function.py:35-78) of "
               "(2048, 2048) fields on the 4096 grid, forward + autograd backward each")
    else:
        spec = scenes.config(name)
        sc = scenes.generate(spec)
        res = cpu_baseline.run_frame_tiled(
            sc, cap_s=CPU_CAP_S,
            progress=lambda d, n: print(f"[cpu {name}] {d}/{n} tiles, "
                                        f"{time.perf_counter() - t0:.0f} s", file=sys.stderr,
                                        flush=True))
        res.pop("grads", None)
        res.pop("hologram", None)
        run = (f"{spec.name} whole: every 64x64 tile of the Python splat forward + backward "
               "(backward tile by tile, its upstream field gradient the propagation adjoint of "
               "the scene's hologram gradient) and every (plane, wavelength) propagation")
    total = (res["fwd_ms"] + res["bwd_ms"]) if res["finished"] else None
    return {"cpu_frame": name, "value": round(total, 1) if total else None, "unit": "ms/frame",
            "did_not_finish": not res["finished"], "cap_s": CPU_CAP_S, "cores": cores,
            "kind": "port", "run": run,
            "detail": {k: (round(v, 1) if isinstance(v, float) else v) for k, v in res.items()},
            "wall_s": round(time.perf_counter() - t0, 1)}


def bench_cfg3(args, dev):
    """Config 3, the propagation-only microbench: a (3, 2048, 2048) field to
    8 distances on the 4096 grid, forward (D*C outputs) + adjoint (sum over
    distances back to the field) per step, through the multi-distance entry
    points.  Byte model: every 2-D transform is one read and one write of
    its M x M complex64 grid, plus the S x S inputs and outputs (the same
    compulsory-dataflow model as the headline frame)."""
    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import _lib, propagation, scenes

    field, wl, dist = scenes.cfg3_fields()
    C, S = field.shape[0], field.shape[1]
    D, M = len(dist), 2 * S
    x = torch.from_numpy(field).to(dev)
    gen = torch.Generator(device=dev).manual_seed(7)
    y = torch.randn((D, C, S, S), dtype=torch.complex64, device=dev, generator=gen)

    def step():
        propagation.multidistance(x, wl, scenes.PITCH, dist, (S, S), float(S))
        propagation.multidistance_adjoint(y, (S, S), wl, scenes.PITCH, dist, (S, S), float(S))

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(args.steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    fwd_b = C * (8 * S * S + 16 * M * M) + D * C * (32 * M * M + 8 * S * S)
    adj_b = D * C * (8 * S * S + 32 * M * M) + C * (16 * M * M + 8 * S * S)
    ach = (fwd_b + adj_b) / (ms * 1e-3) / 1e9
    # What the fused passes move (the multi-distance workspace holds the
    # column results of G = 2 distances at a time): forward = field in, row
    # spectra (C,S,M) out once and in once per group, (D,C,S,M) column results
    # out and in, (D,C,S,S) out; the adjoint mirrors it with the (C,S,M)
    # column sum written per group and read back by the next group and by the
    # inverse rows pass.
    groups = (D + 1) // 2
    row_b, col_b = 8 * C * S * M, 8 * D * C * S * M
    fused_b = (8 * C * S * S + row_b * (1 + groups) + 2 * col_b + 8 * D * C * S * S +
               8 * D * C * S * S + 2 * col_b + row_b * 2 * groups + 8 * C * S * S)
    fused_gbs = fused_b / (ms * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_baseline

        torch.set_num_threads(len(os.sched_getaffinity(0)))
        jobs = [(torch.from_numpy(field[c]), wl[c], dist[d]) for d in range(D) for c in range(C)]
        cf, cb = cpu_baseline.time_propagations(jobs, S, float(S), scenes.PITCH)
        cpu = {"value": round(cf + cb, 1), "unit": "ms/step", "cores": torch.get_num_threads(),
               "kind": "port", "fwd_ms": round(cf, 1), "bwd_ms": round(cb, 1),
               "sample": f"the whole step (not sampled): all {D * C} 2048x2048 propagations of "
                         "the pure-torch ASM (oracle/cpu_baseline.py, python_function.py:35-78) "
                         "forward, each with its autograd backward"}
    out = {"metric": "config 3 propagation microbench: (3,2048,2048) field to 8 distances, "
                     "fwd+adjoint, ms/step", "value": round(ms, 3), "unit": "ms/step",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
           "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
           "data": "synthetic",
           "config": {"workload": f"cfg3: ({C},{S},{S}) c64 to {D} distances, grid {M}, "
                                  "fwd+adjoint", "channels": C, "size": S, "distances": D,
                      "fft_grid": M, "parallelism": "single-gpu"},
           "roofline": {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4),
                        "traffic": None,
                        "kernel": "whole step (fused LDS-FFT row and column passes)",
                        "bytes_per_step": int(fwd_b + adj_b)},
           "fused_dataflow_bytes": int(fused_b),
           "fused_dataflow_frac": round(fused_gbs / HBM_PEAK_GBS, 4),
           "cpu_baseline": cpu}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="headline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--cpu-frame", default=None, metavar="CONFIG",
                    help="run only the CPU baseline, one whole frame of CONFIG (cfg1, headline: "
                         "forward + backward, the backward tile by tile; cfg3: the 24 "
                         "propagations forward + backward), under the 600 s did-not-finish cap, "
                         "and print one JSON line (no GPU is used)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run 3 elementwise copies of 256 MiB (x*2 -> y), a kernel of "
                         "known HBM traffic for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; --gpus/WORLD_SIZE above 1 is not "
              "supported (the hot path has no multi-GPU leg in this build).", file=sys.stderr)
        sys.exit(2)

    if args.cpu_frame:
        print(json.dumps(cpu_whole_frame(args.cpu_frame)), flush=True)
        return

    import numpy as np
    import torch

    from complex_valued_holographic_radiance_fields_amd import _lib, scenes
    from complex_valued_holographic_radiance_fields_amd.frame import Frame

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device=dev)
        for _ in range(3):
            dst = src * 2.0
        torch.cuda.synchronize()
        del src, dst
    if args.config in ("cfg3", "3"):
        bench_cfg3(args, dev)
        return
    spec = scenes.config(args.config)
    t_gen = time.perf_counter()
    sc = scenes.generate(spec)
    print(f"[bench] generated {spec.name}: N={sc.cam_means.shape[0]} in "
          f"{time.perf_counter() - t_gen:.1f}s", file=sys.stderr, flush=True)
    t = scenes.to_torch(sc, dev)
    fr = Frame(t, spec, sc.fx, sc.fy, sc.px, sc.py)
    grad = t["grad_holo"]

    def step():
        fr.forward()
        if spec.backward:
            fr.backward(grad)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    # Stage breakdown: a short pass with every stage traced.  Each traced
    # stage adds two event records to the stream (queue time), so this pass
    # only attributes time; it is not the measurement.
    prof_steps = max(1, min(3, args.steps))
    _lib.trace_reset()
    _lib.trace_only(None)
    _lib.trace_enable(True)
    torch.cuda.synchronize()
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    _lib.trace_enable(False)
    stages = {}
    for s in STAGES:
        n, ms = _lib.trace_read(s)
        if n:
            stages[s] = {"launches": n, "ms_per_frame": ms / prof_steps,
                         "avg_launch_ms": ms / n}
    _lib.trace_reset()

    N = int(sc.cam_means.shape[0])
    K = fr.num_pairs
    P, C, W, H, S = spec.planes, len(spec.wavelengths), spec.width, spec.height, spec.size
    T = ((W + 15) // 16) * ((H + 15) // 16)
    B = algorithmic_bytes(N, K, P, C, W, H, S, T)
    dom = max((s for s in stages if s in B["per_launch"]),
              key=lambda s: stages[s]["ms_per_frame"], default=None)

    # Timed region: exactly `steps` frames; only the dominant stage is traced
    # (its launches are bracketed by hipEvents on the stream they run on).
    # An event at every frame boundary and between each frame's forward and
    # backward gives the per-frame times whose median is `value` and the
    # forward/backward split.
    _lib.trace_only(dom)
    _lib.trace_enable(dom is not None)
    marks = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(args.steps)]
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for k in range(args.steps):
        marks[k][0].record()
        fr.forward()
        marks[k][1].record()
        if spec.backward:
            fr.backward(grad)
    end.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - wall0
    _lib.trace_enable(False)
    _lib.trace_only(None)
    total_ms = marks[0][0].elapsed_time(end)
    ms_mean = total_ms / args.steps
    starts = [m[0] for m in marks] + [end]
    frame_ms = [starts[k].elapsed_time(starts[k + 1]) for k in range(args.steps)]
    fwd_frames = [marks[k][0].elapsed_time(marks[k][1]) for k in range(args.steps)]
    bwd_frames = [marks[k][1].elapsed_time(starts[k + 1]) for k in range(args.steps)]
    ms_per_step = float(np.median(frame_ms))
    dom_live = None
    if dom is not None:
        n_l, ms_l = _lib.trace_read(dom)
        if n_l:
            dom_live = ms_l / n_l
    _lib.trace_reset()

    frame_bytes = B["total"] if spec.backward else B["RF"] + B["AF"]
    frame_gbs = frame_bytes / (ms_per_step * 1e-3) / 1e9
    fused_bytes = B["fused_total"] if spec.backward else B["fused_fwd"]
    fused_gbs = fused_bytes / (ms_per_step * 1e-3) / 1e9

    # Dominant kernel stage and its roofline (launch time measured live in
    # the timed region).
    roof = None
    if dom is not None and dom_live:
        ach = B["per_launch"][dom] / (dom_live * 1e-3) / 1e9
        traffic, src = profiled_traffic(spec.name, dom, C, 2 * S)
        roof = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": traffic, "kernel": dom,
                "avg_launch_ms": round(dom_live, 4),
                "bytes_per_launch": int(B["per_launch"][dom]), "traffic_source": src}

    # Diagnostic: the render kernels are VALU-bound, so their issue time at
    # the FP32 vector peak (instruction counts from the committed profile)
    # against the measured launch time is the fraction that matters there.
    valu = {}
    for st in ("render_fwd", "render_bwd"):
        prof = profiled_valu(spec.name, st, C, 2 * S)
        t_ms = dom_live if (st == dom and dom_live) else stages.get(st, {}).get("avg_launch_ms")
        if prof and t_ms:
            slots = prof["valu"] + prof["trans_extra_slots"] * prof["trans"]
            issue_ms = slots / prof["valu_peak"] * 1e3
            valu[st] = {"wave_instructions": prof["valu"], "transcendental": prof["trans"],
                        "issue_ms_at_peak": round(issue_ms, 4),
                        "peak_wave_instr_per_s": prof["valu_peak"],
                        "measured_ms": round(t_ms, 4), "frac": round(issue_ms / t_ms, 3)}
            if st == "render_fwd":
                # the same instructions at the rate the forward's member
                # loop reaches on its own (calibration kernel)
                loop_ms = prof["valu"] / prof["fwdloop_rate"] * 1e3
                valu[st].update({"member_loop_rate": prof["fwdloop_rate"],
                                 "ms_at_member_loop_rate": round(loop_ms, 4),
                                 "frac_of_member_loop_rate": round(loop_ms / t_ms, 3)})
    if valu:
        valu["source"] = f"profiles/valu_{spec.name}.txt"

    # The training-loop rows around the frame are measured on the headline
    # scene only (their own workloads, reported beside the frame).
    pre = opt_step = recon = None
    if spec.name == "headline":
        pre = measure_preprocess(spec, dev, args.no_cpu_baseline)
        opt_step = measure_optimizer(spec, dev, args.no_cpu_baseline)
        recon = measure_reconstruction(spec, dev, args.no_cpu_baseline)

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_leg(spec, sc, args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(ms_per_step, 4),
        "unit": "ms/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"{spec.name}: {N} Gaussians @{W}x{H}, P={P}, C={C}, "
                               f"{'fwd+bwd' if spec.backward else 'fwd'}",
                   "gaussians": N, "width": W, "height": H, "planes": P, "channels": C,
                   "pairs_K": K, "fft_grid": 2 * S, "parallelism": "single-gpu"},
        "timing": f"median of {args.steps} frames, each bracketed by hipEvents on the stream "
                  f"(ms_per_step_mean: the whole timed region / steps)",
        "ms_per_step_mean": round(ms_mean, 4),
        "fwd_ms": round(float(np.median(fwd_frames)), 4),
        "bwd_ms": round(float(np.median(bwd_frames)), 4) if spec.backward else None,
        "fwd_bwd_split_from": "median per-frame hipEvents of the timed region (untraced but for "
                              "the dominant kernel's two events)",
        "gaussians_per_s": round(N / (ms_per_step * 1e-3), 1),
        "frame_alg_bytes": int(frame_bytes),
        "frame_achieved_GBs": round(frame_gbs, 1),
        "frame_hbm_frac": round(frame_gbs / HBM_PEAK_GBS, 4),
        "frame_fused_dataflow_bytes": int(fused_bytes),
        "frame_fused_dataflow_frac": round(fused_gbs / HBM_PEAK_GBS, 4),
        "wall_s": round(wall_s, 3),
        "stages_ms_per_frame": {s: round(v["ms_per_frame"], 4) for s, v in stages.items()},
        "stages_from": f"stage-traced pass of {prof_steps} frames",
        "roofline": roof,
        "valu": valu or None,
        "cpu_baseline": cpu,
        "preprocess": pre,
        "optimizer": opt_step,
        "reconstruction": recon,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
