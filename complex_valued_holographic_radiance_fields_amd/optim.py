"""Fused optimizer step on the GPU: global-norm gradient clipping and Adan.

Mirrors the optimizer side of the reference's training step (train.py:319-324):
``torch.nn.utils.clip_grad_norm_(parameters, 1.0)`` and ``Adan.step()``
(utils/optimizer.py:288-466; the reference runs its foreach path
``_multi_tensor_adan``, :538-589, with betas (0.98, 0.92, 0.99), eps 1e-8,
no weight decay, seven parameter groups with their own learning rates).

``Adan`` keeps the reference's constructor, defaults, parameter-group keys
and per-parameter state (``exp_avg``, ``exp_avg_sq``, ``exp_avg_diff``,
``neg_pre_grad``; ``group['step']``), so its state dict and the reference's
``setup_optimizer`` / scheduler code work unchanged; every step is one HIP
launch over all tensors (``hrf_adan_step``).  ``clip_grad_norm_`` is one
norm pass plus one rescaling pass; ``grad_norm_clip_coef`` skips the
rescaling and hands the device-side coefficient to ``Adan.step(grad_scale=)``,
which applies it inside the update.
"""
from __future__ import annotations

import ctypes
from typing import Iterable

import torch
from torch.optim.optimizer import Optimizer

from . import _lib


def _grads_of(parameters) -> list[torch.Tensor]:
    if isinstance(parameters, torch.Tensor):
        parameters = [parameters]
    grads = [p.grad for p in parameters if p.grad is not None]
    for g in grads:
        if not g.is_cuda or g.dtype != torch.float32 or not g.is_contiguous():
            raise RuntimeError("gradients must be contiguous float32 GPU tensors (the HIP "
                               "optimizer has no CPU path)")
    return grads


def _ptr_array(ts: list[torch.Tensor]):
    arr = (ctypes.c_void_p * max(len(ts), 1))(*[t.data_ptr() for t in ts])
    nums = (ctypes.c_int64 * max(len(ts), 1))(*[t.numel() for t in ts])
    return arr, nums


def grad_norm_clip_coef(parameters, max_norm: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(total_norm, clip_coef) as device float tensors: the 2-norm of all
    gradients and min(max_norm / (total_norm + 1e-6), 1) (NaN propagates),
    as torch.nn.utils.clip_grad_norm_ forms them; the gradients are left
    untouched."""
    grads = _grads_of(parameters)
    if not grads:
        z = torch.zeros((), dtype=torch.float32)
        return z, torch.ones((), dtype=torch.float32)
    dev = grads[0].device
    lib = _lib.load()
    out = torch.empty(2, dtype=torch.float32, device=dev)
    arr, nums = _ptr_array(grads)
    with torch.cuda.device(dev):
        stream = _lib.stream_ptr(dev)
        wbytes = lib.hrf_grad_norm_workspace_size(nums, len(grads))
        ws = _lib.workspace("grad_norm", dev, stream, wbytes)
        _lib.check(lib.hrf_grad_norm(arr, nums, len(grads), float(max_norm), out.data_ptr(),
                                     out.data_ptr() + 4, _lib.ptr(ws), wbytes, stream))
    return out[0], out[1]


def clip_grad_norm_(parameters, max_norm: float, norm_type: float = 2.0,
                    error_if_nonfinite: bool = False, foreach=None) -> torch.Tensor:
    """Drop-in for torch.nn.utils.clip_grad_norm_ with the 2-norm (the
    reference's call, train.py:319): returns the total norm and multiplies
    every gradient by the clip coefficient."""
    if float(norm_type) != 2.0:
        raise RuntimeError("only the 2-norm is implemented (the reference's clip)")
    grads = _grads_of(parameters)
    total, coef = grad_norm_clip_coef(parameters, max_norm)
    if not grads:
        return total
    if error_if_nonfinite and not bool(torch.isfinite(total)):
        raise RuntimeError(f"The total norm of order {float(norm_type)} for gradients from "
                           "`parameters` is non-finite, so it cannot be clipped.")
    dev = grads[0].device
    lib = _lib.load()
    arr, nums = _ptr_array(grads)
    with torch.cuda.device(dev):
        _lib.check(lib.hrf_scale_grads(arr, nums, len(grads), coef.data_ptr(),
                                       _lib.stream_ptr(dev)))
    return total


def _cfg_key(group) -> tuple:
    b1, b2, b3 = group["betas"]
    return (float(b1), float(b2), float(b3), float(group["eps"]), float(group["weight_decay"]),
            bool(group["no_prox"]))


class Adan(Optimizer):
    """Adan (utils/optimizer.py:288-466) with every step fused into one HIP
    launch.  Arguments as the reference's; ``foreach`` and ``fused`` are
    accepted and kept in the defaults (the update is always the fused HIP
    kernel)."""

    def __init__(self, params, lr=1e-3, betas=(0.98, 0.92, 0.99), eps=1e-8, weight_decay=0.0,
                 max_grad_norm=0.0, no_prox=False, foreach: bool = True, fused: bool = False):
        if not 0.0 <= max_grad_norm:
            raise ValueError('Invalid Max grad norm: {}'.format(max_grad_norm))
        if not 0.0 <= lr:
            raise ValueError('Invalid learning rate: {}'.format(lr))
        if not 0.0 <= eps:
            raise ValueError('Invalid epsilon value: {}'.format(eps))
        for i in range(3):
            if not 0.0 <= betas[i] < 1.0:
                raise ValueError('Invalid beta parameter at index {}: {}'.format(i, betas[i]))
        defaults = dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay,
                        max_grad_norm=max_grad_norm, no_prox=no_prox, foreach=foreach,
                        fused=fused)
        super().__init__(params, defaults)

    def __setstate__(self, state):
        super().__setstate__(state)
        for group in self.param_groups:
            group.setdefault('no_prox', False)

    @torch.no_grad()
    def restart_opt(self):
        for group in self.param_groups:
            group['step'] = 0
            for p in group['params']:
                if p.requires_grad:
                    state = self.state[p]
                    state['exp_avg'] = torch.zeros_like(p)
                    state['exp_avg_sq'] = torch.zeros_like(p)
                    state['exp_avg_diff'] = torch.zeros_like(p)

    def _own_clip(self, grad_scale: torch.Tensor | None) -> float:
        """Adan's max_grad_norm clip (optimizer.py:391-409): a host float,
        formed in float32 on the device and read back as the reference's
        .item() does; the eps is the last group's (the reference's loop
        variable).  The norm is of the gradients after grad_scale."""
        params = [p for g in self.param_groups for p in g['params']]
        total, _ = grad_norm_clip_coef(params, 1.0)
        if grad_scale is not None:
            total = total * grad_scale.to(total.device).reshape(())
        eps = self.param_groups[-1]['eps']
        mx = torch.tensor(self.defaults['max_grad_norm'], device=total.device)
        return torch.clamp(mx / (total + eps), max=1.0).item()

    @torch.no_grad()
    def step(self, closure=None, grad_scale: torch.Tensor | None = None):
        """One step.  grad_scale: optional device float scalar (for example
        grad_norm_clip_coef's coefficient) that multiplies every gradient
        first; the gradients are left holding the scaled values, as after
        clip_grad_norm_."""
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        clip = self._own_clip(grad_scale) if self.defaults['max_grad_norm'] > 0 else 1.0

        batches: dict[tuple, list] = {}
        keep = []  # tensors the ctypes structs point into
        for group in self.param_groups:
            group['step'] = group['step'] + 1 if 'step' in group else 1
            for p in group['params']:
                if p.grad is None:
                    continue
                for name, t in (("param", p), ("grad", p.grad)):
                    if not t.is_cuda or t.dtype != torch.float32 or not t.is_contiguous():
                        raise RuntimeError(f"Adan: {name} must be a contiguous float32 GPU "
                                           "tensor (the HIP optimizer has no CPU path)")
                state = self.state[p]
                if len(state) == 0:
                    state['exp_avg'] = torch.zeros_like(p)
                    state['exp_avg_sq'] = torch.zeros_like(p)
                    state['exp_avg_diff'] = torch.zeros_like(p)
                init = 'neg_pre_grad' not in state or group['step'] == 1
                if 'neg_pre_grad' not in state:
                    state['neg_pre_grad'] = torch.empty_like(p)
                ts = [p, p.grad, state['exp_avg'], state['exp_avg_sq'], state['exp_avg_diff'],
                      state['neg_pre_grad']]
                for t in ts[2:]:
                    if t.shape != p.shape or not t.is_contiguous() or t.dtype != torch.float32:
                        raise RuntimeError("Adan: optimizer state must match its parameter "
                                           "(contiguous float32)")
                keep.extend(ts)
                batches.setdefault((p.device, _cfg_key(group)), []).append(
                    _lib.HrfAdanTensor(*[t.data_ptr() for t in ts], p.numel(),
                                       float(group['lr']), int(group['step']), int(init)))
        if not batches:
            return loss
        if grad_scale is not None:
            if not grad_scale.is_cuda or grad_scale.dtype != torch.float32 \
                    or grad_scale.numel() != 1:
                raise RuntimeError("grad_scale must be a one-element float32 GPU tensor")
        lib = _lib.load()
        for (dev, key), items in batches.items():
            b1, b2, b3, eps, wd, no_prox = key
            cfg = _lib.HrfAdanConfig(b1, b2, b3, eps, wd, clip, int(no_prox))
            arr = (_lib.HrfAdanTensor * len(items))(*items)
            gs = grad_scale.to(dev) if grad_scale is not None else None
            with torch.cuda.device(dev):
                _lib.check(lib.hrf_adan_step(arr, len(items), ctypes.byref(cfg), _lib.ptr(gs),
                                             _lib.stream_ptr(dev)))
        del keep
        return loss


def training_step_update(optimizer: Adan, parameters: Iterable[torch.Tensor],
                         max_norm: float = 1.0) -> torch.Tensor:
    """train.py:319-324 in two passes: the gradient norm, then the Adan
    update with the clip coefficient applied inside it (no separate
    rescaling pass).  Returns the total norm (device tensor)."""
    params = list(parameters)
    total, coef = grad_norm_clip_coef(params, max_norm)
    optimizer.step(grad_scale=coef if coef.is_cuda else None)
    return total


def sparse_adam_update(param: torch.Tensor, grad: torch.Tensor, exp_avg: torch.Tensor,
                       exp_avg_sq: torch.Tensor, visible_chunk: torch.Tensor, lr: float,
                       b1: float, b2: float, eps: float) -> None:
    """Adam step of the visible rows, in place (spadam.cu:8-55 behind
    python_import.py:457-460): param, exp_avg, exp_avg_sq (B, N, D); grad
    (B, V, D) the visible rows' gradients; visible_chunk (V) int64 row
    indices.  No bias correction; the scalars are used in float32, as the
    reference's kernel arguments.  Rows outside [0, N) are skipped."""
    ts = {"param": param, "exp_avg": exp_avg, "exp_avg_sq": exp_avg_sq, "grad": grad}
    for name, t in ts.items():
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{name} must be a CUDA tensor (the HIP optimizer has no CPU path)")
        if t.dtype != torch.float32 or t.dim() != 3 or not t.is_contiguous():
            raise RuntimeError(f"{name} must be a contiguous 3-D float32 tensor; got "
                               f"{t.dtype} {tuple(t.shape)}")
    if exp_avg.shape != param.shape or exp_avg_sq.shape != param.shape:
        raise RuntimeError("exp_avg and exp_avg_sq must have the shape of param")
    if not isinstance(visible_chunk, torch.Tensor) or not visible_chunk.is_cuda or \
            visible_chunk.dtype != torch.int64 or visible_chunk.dim() != 1:
        raise RuntimeError("visible_chunk must be a 1-D int64 CUDA tensor")
    B, N, D = param.shape
    V = visible_chunk.shape[0]
    if tuple(grad.shape) != (B, V, D):
        raise RuntimeError(f"grad must have shape ({B}, {V}, {D}); got {tuple(grad.shape)}")
    vis = visible_chunk.contiguous()
    _lib.check(_lib.load().hrf_sparse_adam_update(
        param.data_ptr(), grad.data_ptr(), exp_avg.data_ptr(), exp_avg_sq.data_ptr(),
        vis.data_ptr(), B, N, D, V, float(lr), float(b1), float(b2), float(eps),
        _lib.stream_ptr(param.device)))
