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


@pytest.mark.parametrize("precision,tol_layer", [("fp32", 1e-6), ("bf16", 4e-3)])
def test_torch_tower_layer_taps_match_numpy_oracle(precision, tol_layer):
    """The per-layer taps the full-depth GPU tests compare against (TorchTower.run(keep_layers=True):
    x after the patch embed + pos-embed and after every block): the embed equals the numpy oracle's,
    and each block of the torch restatement (TorchTower.block, what run() chains) fed the numpy
    oracle's input matches the numpy block's output (fp32 within 1e-6, bf16 within 4e-3: the two
    restatements round at the same points and differ only where an fp32 accumulation order flips a
    rounding). Checkpoint-like parameters (non-zero biases, noisy LayerNorm affines) and a video grid
    (the jnp.repeat quirk)."""
    from oracle import indices as ix
    spec = vt.VisionSpec(hidden_size=256, out_hidden_size=192, depth=4, num_heads=4, intermediate_size=512,
                         deepstack_visual_indexes=(1, 3))
    params = vt.init_params(spec, seed=8, bias_std=0.02, ln_noise=0.1)
    grids = np.asarray([(1, 8, 12), (3, 4, 6)])
    n = int((grids[:, 0] * grids[:, 1] * grids[:, 2]).sum())
    px = np.random.default_rng(9).standard_normal((n, spec.patch_volume)).astype(np.float32)
    ref = vt.encode_vision(params, px, grids, spec, precision, keep_layers=True)
    tower = tt.TorchTower(params, spec, precision)
    out = tower.run(px, grids, keep_layers=True)
    assert len(out["layers"]) == spec.depth
    assert rel_l2(out["embed"].float().numpy(), ref.embed) <= tol_layer
    cos, sin = vt.rotary_cos_sin(grids, spec, vt._P(precision))
    c = torch.from_numpy(cos).to(tower.dt)[:, None, :]
    s = torch.from_numpy(sin).to(tower.dt)[:, None, :]
    cu = ix.cu_seqlens_ref(grids)
    for i in range(spec.depth):
        xin = ref.embed if i == 0 else ref.layers[i - 1]
        with torch.inference_mode():
            x = tower.block(i, torch.from_numpy(np.ascontiguousarray(xin, np.float32)).to(tower.dt), c, s, cu)
        assert rel_l2(x.float().numpy(), ref.layers[i]) <= tol_layer, i
