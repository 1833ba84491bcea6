"""Gaussian checkpoints in the reference's file format.

``Gaussians.save_gaussians`` (model.py:610-624) writes ``torch.save`` of a
dict of the seven pre-activation parameter tensors (CPU); ``_load_gaussians``
(model.py:120-136) reads a ``.pth`` back as contiguous float32.  The same
dict layout and key names are written and read here, so checkpoints move
between the reference and this package both ways.  Loading always uses
``torch.load(..., weights_only=True)``: a checkpoint is tensors only, and a
file that needs anything else to unpickle is refused rather than executed
(the reference loads with weights_only=False).
"""
from __future__ import annotations

import os

import torch

# model.py:612-621, in the reference's order
KEYS = ("pre_act_quats", "means", "pre_act_scales", "colours", "pre_act_phase",
        "pre_act_opacities", "pre_act_plane_assignment")

# column counts: None = any (colours / phase: C; plane logits: P)
_COLS = {"pre_act_quats": 4, "means": 3, "pre_act_scales": 3, "colours": None,
         "pre_act_phase": None, "pre_act_opacities": 1, "pre_act_plane_assignment": None}


def save_gaussians(params: dict, save_path: str) -> None:
    """Writes params[k] for the seven keys (any device) as the reference
    does: a dict of CPU tensors through torch.save."""
    missing = [k for k in KEYS if k not in params]
    if missing:
        raise KeyError(f"save_gaussians: missing parameters {missing}")
    torch.save({k: params[k].detach().cpu() for k in KEYS}, save_path)


def load_gaussians(path: str, device: str | torch.device = "cuda") -> dict:
    """Reads a reference checkpoint: dict of the seven tensors as contiguous
    float32 on `device`, with the reference's shape conventions checked
    (N rows each; quats (N,4), means and log-scales (N,3), opacities (N,1)
    or (N), colours and phase (N,C), plane logits (N,P))."""
    if not path.endswith(".pth"):
        raise ValueError(f"load_gaussians: expected a .pth checkpoint, got {path!r}")
    if not os.path.exists(path):
        raise FileNotFoundError(path)
    try:
        ckpt = torch.load(path, map_location="cpu", weights_only=True)
    except Exception as e:  # the safe loader refuses anything but tensors/containers
        raise RuntimeError(f"load_gaussians: {path} is not a tensors-only checkpoint ({e})") \
            from e
    if not isinstance(ckpt, dict):
        raise RuntimeError(f"load_gaussians: {path} does not hold a dict")
    missing = [k for k in KEYS if k not in ckpt]
    if missing:
        raise KeyError(f"load_gaussians: {path} lacks {missing}")
    data = {k: ckpt[k].clone().detach().to(torch.float32).contiguous() for k in KEYS}
    n = data["means"].shape[0]
    for k, t in data.items():
        cols = _COLS[k]
        if t.shape[0] != n:
            raise ValueError(f"load_gaussians: {k} has {t.shape[0]} rows, means has {n}")
        if k == "pre_act_opacities":
            if not (t.dim() == 1 or (t.dim() == 2 and t.shape[1] == 1)):
                raise ValueError(f"load_gaussians: {k} must be (N) or (N,1), got {tuple(t.shape)}")
        elif t.dim() != 2 or (cols is not None and t.shape[1] != cols):
            raise ValueError(f"load_gaussians: {k} has shape {tuple(t.shape)}")
    if data["colours"].shape[1] != data["pre_act_phase"].shape[1]:
        raise ValueError("load_gaussians: colours and pre_act_phase disagree on C")
    return {k: t.to(device) for k, t in data.items()}
