"""The torch-CPU restatement (oracle/torch_tower.py, the timed CPU baseline) agrees with the numpy
oracle: fp32 within rel-L2 1e-5 (accumulation order only), bf16 within 1e-2 (rounding-point
placement is shared; bf16 values differ only where fp32 accumulation order flips a rounding)."""
import numpy as np
import pytest

from oracle import torch_tower as tt
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("precision,tol", [("fp32", 1e-5), ("bf16", 1e-2)])
def test_torch_tower_matches_numpy_oracle(precision, tol):
    spec = vt.VisionSpec(hidden_size=256, out_hidden_size=192, depth=3, num_heads=4, intermediate_size=512,
                         deepstack_visual_indexes=(0, 2))
    params = vt.init_params(spec, seed=3, bias_std=0.05, ln_noise=0.05)
    grids = [(1, 8, 12), (2, 4, 6)]
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(4).standard_normal((n, spec.patch_volume)).astype(np.float32)
    ref = vt.encode_vision(params, px, grids, spec, precision)
    tok, ds = tt.TorchTower(params, spec, precision)(px, grids)
    assert len(ds) == 2
    errs = []
    for got, want in zip([tok, *ds], [ref.tokens, *ref.deepstack]):
        assert got.shape == want.shape
        errs.append(rel_l2(got.float().numpy(), want))
        assert errs[-1] <= tol
    if precision == "fp32":
        # a planted mistake in the restatement (rotate_half without the sign) lands far outside
        bad = tt.TorchTower(params, spec, precision)
        bad._rotate_half = lambda x: torch.cat(x.chunk(2, dim=-1)[::-1], dim=-1)
        assert rel_l2(bad(px, grids)[0].float().numpy(), ref.tokens) > 100 * tol


def test_torch_tower_without_pos_table():
    spec = vt.VisionSpec(hidden_size=128, out_hidden_size=64, depth=1, num_heads=2, intermediate_size=256,
                         deepstack_visual_indexes=(), num_position_embeddings=None)
    params = vt.init_params(spec, seed=5)
    px = np.random.default_rng(6).standard_normal((16, spec.patch_volume)).astype(np.float32)
    ref = vt.encode_vision(params, px, [(1, 4, 4)], spec, "fp32")
    tok, _ = tt.TorchTower(params, spec, "fp32")(px, [(1, 4, 4)])
    assert rel_l2(tok.numpy(), ref.tokens) <= 1e-5
