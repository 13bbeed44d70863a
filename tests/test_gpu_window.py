"""GPU parity of the window-attention path (specs whose fullatt_block_indexes miss blocks,
model.py:808-850) through the fused tower entry, and of the row-gather kernel it uses."""
import dataclasses

import numpy as np
import pytest

from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def to_np(t):
    return t.float().cpu().numpy()


def window_specs(pkg, depth=4, fullatt=(1, 3), ds=(0, 2), window=64, shape="2b", npos=2304):
    s = pkg.spec_2b() if shape == "2b" else pkg.spec_8b()
    s = dataclasses.replace(s, depth=depth, deepstack_visual_indexes=tuple(ds), fullatt_block_indexes=tuple(fullatt),
                            window_size=window, num_position_embeddings=npos)
    o = vt.VisionSpec(hidden_size=s.hidden_size, out_hidden_size=s.out_hidden_size, depth=depth,
                      num_heads=s.num_heads, intermediate_size=s.intermediate_size, deepstack_visual_indexes=tuple(ds),
                      window_size=window, fullatt_block_indexes=tuple(fullatt), num_position_embeddings=npos)
    return s, o


@pytest.mark.parametrize("grids,window", [([(1, 8, 12), (2, 4, 4)], 64), ([(1, 32, 48)], 112), ([(2, 16, 20)], 64)])
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_window_tower_vs_oracle(pkg, grids, window, dtype):
    spec, ospec = window_specs(pkg, window=window)
    assert spec.use_window and ospec.use_window
    params = pkg.random_params(spec, seed=31)
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(5).standard_normal((n, 1536), dtype=np.float32)
    tower = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(params)
    tok, ds = tower(px, np.array(grids, np.int32))
    ref64 = vt.encode_vision(params, px, grids, ospec, "fp64")
    pairs = [(to_np(tok), ref64.tokens)] + [(to_np(a), b) for a, b in zip(ds, ref64.deepstack)]
    assert len(pairs) == 3
    if dtype == "float32":
        for got, r in pairs:
            assert rel_l2(got, r) <= 1e-4
    else:
        refb = vt.encode_vision(params, px, grids, ospec, "bf16")
        for (got, r), rb in zip(pairs, [refb.tokens, *refb.deepstack]):
            assert rel_l2(got, rb) <= 1e-2
            assert rel_l2(got, r) <= max(1.1 * rel_l2(rb, r), 1e-2)
    # window blocks do restrict attention: the all-full spec gives a different answer
    full = pkg.Qwen3VisionTransformer(dataclasses.replace(spec, fullatt_block_indexes=None), dtype=dtype).bind(params)
    tf, _ = full(px, np.array(grids, np.int32))
    assert rel_l2(to_np(tf), to_np(tok)) > 1e-3


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_window_tower_head_dim72_vs_oracle(pkg, dtype):
    """Window attention on the 8B shape (head_dim 72: the general attention kernel over the window
    work list, the rotary relayout for the windowed order): tokens and deepstack features against
    the fp64 oracle (fp32: 1e-4) and the bf16 oracle (bf16: 1e-2)."""
    grids = [(1, 8, 12), (2, 4, 4)]
    spec, ospec = window_specs(pkg, depth=2, fullatt=(1,), ds=(0,), shape="8b")
    assert spec.use_window and spec.head_dim == 72
    params = pkg.random_params(spec, seed=33)
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(6).standard_normal((n, 1536), dtype=np.float32)
    tower = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(params)
    tok, ds = tower(px, np.array(grids, np.int32))
    ref = vt.encode_vision(params, px, grids, ospec, "fp64" if dtype == "float32" else "bf16")
    tol = 1e-4 if dtype == "float32" else 1e-2
    for got, r in [(to_np(tok), ref.tokens)] + [(to_np(a), b) for a, b in zip(ds, ref.deepstack)]:
        assert rel_l2(got, r) <= tol


@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_window_tower_without_pos_embed(pkg, dtype):
    """A Qwen2.5-style spec: window attention and no learned pos-embed table
    (num_position_embeddings None, model.py:676-680 / 803-806): the tower runs the patch embed
    alone and matches the oracle (fp32 <= 1e-4 of fp64, bf16 <= 1e-2 of the bf16 oracle)."""
    spec, ospec = window_specs(pkg, window=64, npos=None)
    params = pkg.random_params(spec, seed=32)
    assert "pos_embed" not in params["visual"]
    grids = [(1, 8, 12), (2, 4, 4)]
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(6).standard_normal((n, 1536), dtype=np.float32)
    tower = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(params)
    tok, ds = tower(px, np.array(grids, np.int32))
    if dtype == "float32":
        ref = vt.encode_vision(params, px, grids, ospec, "fp64")
        bound = 1e-4
    else:
        ref = vt.encode_vision(params, px, grids, ospec, "bf16")
        bound = 1e-2
    for got, r in zip([tok, *ds], [ref.tokens, *ref.deepstack]):
        assert rel_l2(to_np(got), r) <= bound


@pytest.mark.parametrize("sdt,ddt", [("float32", "bfloat16"), ("float32", "float32"), ("bfloat16", "bfloat16"),
                                     ("bfloat16", "float32")])
@pytest.mark.parametrize("group,width", [(4, 1536), (1, 2048), (4, 6), (1, 37)])
def test_gather_rows_bit_exact(pkg, sdt, ddt, group, width):
    rng = np.random.default_rng(group * 1000 + width)
    groups = 50
    src = rng.standard_normal((groups * group, width)).astype(np.float32)
    if sdt == "bfloat16":
        src = vt.bf16_round(src)
    idx = rng.permutation(groups).astype(np.int32)
    s = torch.from_numpy(src).cuda().to(getattr(torch, sdt))
    d = torch.empty((groups * group, width), dtype=getattr(torch, ddt), device="cuda")
    ti = torch.from_numpy(idx).cuda()
    cp = pkg.capi
    dt = {"float32": cp.QVL_DTYPE_F32, "bfloat16": cp.QVL_DTYPE_BF16}
    lib = cp.load()
    assert lib.qvl_gather_rows(None, dt[sdt], s.data_ptr(), width, dt[ddt], d.data_ptr(), width, ti.data_ptr(),
                               groups * group, group, width) == 0
    rows = (idx[:, None] * group + np.arange(group)[None, :]).reshape(-1)
    want = src[rows]
    if ddt == "bfloat16":
        want = vt.bf16_round(want)
    got = to_np(d)
    assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(want, np.float32).view(np.uint32))
