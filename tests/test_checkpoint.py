"""Checkpoint format (model.py:610-624 save, :120-136 load): the reference's
dict of seven pre-activation tensors round-trips, converts to contiguous
float32, and is read with the tensors-only loader (CPU; no GPU needed)."""
import numpy as np
import pytest
import torch

from complex_valued_holographic_radiance_fields_amd import checkpoint as ck


def _params(n=50, C=3, P=3, dtype=torch.float32):
    g = torch.Generator().manual_seed(1)
    shapes = {"pre_act_quats": (n, 4), "means": (n, 3), "pre_act_scales": (n, 3),
              "colours": (n, C), "pre_act_phase": (n, C), "pre_act_opacities": (n, 1),
              "pre_act_plane_assignment": (n, P)}
    return {k: torch.randn(s, generator=g).to(dtype) for k, s in shapes.items()}


def test_round_trip(tmp_path):
    p = _params()
    path = str(tmp_path / "g.pth")
    ck.save_gaussians(p, path)
    raw = torch.load(path, map_location="cpu", weights_only=True)
    assert list(raw.keys()) == list(ck.KEYS)          # the reference's key order
    got = ck.load_gaussians(path, device="cpu")
    for k in ck.KEYS:
        assert got[k].dtype == torch.float32 and got[k].is_contiguous()
        torch.testing.assert_close(got[k], p[k], rtol=0, atol=0)


def test_reference_layout_other_dtypes(tmp_path):
    """A file written the way save_gaussians writes it, in float64 and with
    non-contiguous tensors, loads as contiguous float32 (model.py:124-131)."""
    p = _params(dtype=torch.float64)
    p["means"] = p["means"].t().contiguous().t()        # non-contiguous
    path = str(tmp_path / "ref.pth")
    torch.save({k: p[k] for k in ck.KEYS}, path)
    got = ck.load_gaussians(path, device="cpu")
    for k in ck.KEYS:
        np.testing.assert_array_equal(got[k].numpy(), p[k].to(torch.float32).numpy())


def test_refusals(tmp_path):
    p = _params()
    with pytest.raises(ValueError):
        ck.load_gaussians(str(tmp_path / "g.ply"), device="cpu")
    bad = dict(p)
    del bad["colours"]
    path = str(tmp_path / "missing.pth")
    torch.save(bad, path)
    with pytest.raises(KeyError):
        ck.load_gaussians(path, device="cpu")
    p2 = dict(p)
    p2["pre_act_quats"] = p2["pre_act_quats"][:, :3]
    path = str(tmp_path / "shape.pth")
    torch.save(p2, path)
    with pytest.raises(ValueError):
        ck.load_gaussians(path, device="cpu")


class _NotATensor:
    pass


def test_code_objects_are_refused(tmp_path):
    """Anything beyond tensors and containers is refused by the safe
    loader instead of being unpickled."""
    p = _params()
    p["extra"] = _NotATensor()
    path = str(tmp_path / "obj.pth")
    torch.save(p, path)
    with pytest.raises(RuntimeError):
        ck.load_gaussians(path, device="cpu")
