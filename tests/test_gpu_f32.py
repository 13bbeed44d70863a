"""fp32 path (the reference's default dtype) on the GPU, through the C ABI,
against the oracle's fp32 / fp64 restatement and torch fp64.

Bar (north star): relative L2 <= 1e-4 in fp32, per layer and at the final tokens / deepstack.
The kernels accumulate in fp32 in a different order from numpy's BLAS, so the references are
fp64 (what fp32 rounding is measured against) with the oracle's fp32 mode alongside."""
import ctypes as C

import numpy as np
import pytest

from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
TOL = 1e-4


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV)


def to_np(t):
    return t.double().cpu().numpy()


def pack32(lib, cp, kernel):
    kin, nout = kernel.shape
    src = dev32(kernel)
    out = torch.empty((-(-nout // 64) * 64, -(-kin // 64) * 64), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_pack_dense_weight(stream(), cp.QVL_DTYPE_F32, src.data_ptr(), kin, nout, out.data_ptr()))
    return out


def test_pack_weight_f32_is_exact_transpose(pkg, lib):
    k = np.random.default_rng(0).standard_normal((100, 70)).astype(np.float32)
    out = pack32(lib, pkg.capi, k).cpu().numpy()
    assert out.shape == (128, 128)
    np.testing.assert_array_equal(out[:70, :100], k.T)
    assert not out[70:].any() and not out[:, 100:].any()


@pytest.mark.parametrize("ws", [False, True])
@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", [(300, 192, 128), (784, 3072, 1024), (196, 2048, 4096), (257, 4352, 1152),
                                   (784, 1024, 4096), (784, 1024, 1024)])
def test_dense_f32_vs_fp64(pkg, lib, epi, m, n, k, ws):
    """fp32 GEMM + epilogue vs float64 on the same fp32 operands: rel-L2 <= 2e-6 and every
    element within 1e-5 of sum_k |x w| (the fp32 accumulation bound). With a workspace
    (qvl_dense_ws) the shapes whose 128 x 128 tiles leave most workgroup slots idle split K into
    fp32 partials summed in order by a second kernel (config 0's fc2 and proj: 56 tiles, 8 parts;
    its qkv: 3 parts; 300 x 192 x 128 has too few k-steps to split): same bounds; the residual
    epilogue runs in place (y is the residual)."""
    cp = pkg.capi
    rng = np.random.default_rng(m + n + k + epi)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((k, n)) * 0.05).astype(np.float32)
    b = (rng.standard_normal(n) * 0.1).astype(np.float32)
    r = rng.standard_normal((m, n)).astype(np.float32)
    xt, wp, bt = dev32(x), pack32(lib, cp, w), dev32(b)
    y = dev32(r) if epi == 2 else torch.empty((m, n), dtype=torch.float32, device=DEV)
    if ws:
        nb = C.c_size_t()
        cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
        wsb = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
        cp.check(lib.qvl_dense_ws(stream(), cp.QVL_DTYPE_F32, epi, xt.data_ptr(), k, wp.data_ptr(), bt.data_ptr(),
                                  y.data_ptr() if epi == 2 else None, n, y.data_ptr(), n, m, n, k, wsb.data_ptr(),
                                  nb.value))
    else:
        cp.check(lib.qvl_dense(stream(), cp.QVL_DTYPE_F32, epi, xt.data_ptr(), k, wp.data_ptr(), bt.data_ptr(),
                               y.data_ptr() if epi == 2 else None, n, y.data_ptr(), n, m, n, k))
    ref = x.astype(np.float64) @ w.astype(np.float64) + b
    if epi == 1:
        ref = 0.5 * ref * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (ref + 0.044715 * ref ** 3)))
    if epi == 2:
        ref = ref + r
    got = to_np(y)
    assert rel_l2(got, ref) <= 2e-6
    bound = np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64) + np.abs(b) + (np.abs(r) if epi == 2 else 0)
    assert np.all(np.abs(got - ref) <= 1e-5 * bound + 1e-6)


@pytest.mark.parametrize("cols", [1024, 1152, 4096, 4608])
def test_layer_norm_f32_vs_fp64(pkg, lib, cols):
    cp = pkg.capi
    rng = np.random.default_rng(cols)
    rows = 259
    x = (rng.standard_normal((rows, cols)) * 3 + 1.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    xt, gt, bt = dev32(x), dev32(g), dev32(b)
    y = torch.empty_like(xt)
    cp.check(lib.qvl_layer_norm(stream(), cp.QVL_DTYPE_F32, xt.data_ptr(), cols, gt.data_ptr(), bt.data_ptr(),
                                y.data_ptr(), cols, rows, cols, 1e-6))
    ref = vt.layer_norm(x, g, b, 1e-6, vt._P("fp64"))
    assert rel_l2(to_np(y), ref) <= 1e-6


@pytest.mark.parametrize("grids", [[(1, 28, 28)], [(2, 16, 12), (1, 8, 8)]])
def test_pos_embed_f32_bit_exact_vs_oracle(pkg, lib, grids):
    """fp32 products and sums in the reference's order: bit-identical to the oracle's fp32 mode."""
    cp = pkg.capi
    spec = vt.VisionSpec()
    tab = (np.random.default_rng(5).standard_normal((spec.num_position_embeddings, spec.hidden_size)) * 0.02
           ).astype(np.float32)
    m = pkg.grid_metadata(grids, dtype=cp.QVL_DTYPE_F32)
    N, D = m.n_tokens, spec.hidden_size
    tt, it, wt = dev32(tab), torch.from_numpy(m.tap_idx).to(DEV), dev32(m.tap_w)
    y = torch.empty((N, D), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_pos_embed(stream(), cp.QVL_DTYPE_F32, tt.data_ptr(), it.data_ptr(), wt.data_ptr(), y.data_ptr(),
                               N, D))
    ref = vt.pos_embed(tab, np.array(grids), spec, vt._P("fp32"))
    np.testing.assert_array_equal(y.cpu().numpy(), ref)


def _attention_f32(pkg, lib, grids, H, hd, seed):
    cp = pkg.capi
    m = pkg.grid_metadata(grids, dtype=cp.QVL_DTYPE_F32, num_heads=H)
    N, D = m.n_tokens, H * hd
    qkv = np.random.default_rng(seed).standard_normal((N, 3 * D)).astype(np.float32)
    qkv_t = dev32(qkv)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, hd // 2, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_F32, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    items = torch.from_numpy(m.tiles if len(m.tiles) else np.zeros((1, 4), np.int32)).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_vision_attention_workspace_size(cp.QVL_DTYPE_F32, N, H, hd, C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    out = torch.full((N, D), float("nan"), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_vision_attention(stream(), cp.QVL_DTYPE_F32, qkv_t.data_ptr(), qkv_t.data_ptr() + 4 * D,
                                      qkv_t.data_ptr() + 8 * D, 3 * D, cs.data_ptr(), items.data_ptr(), len(m.tiles),
                                      out.data_ptr(), D, N, H, hd, ws.data_ptr(), nb.value))
    torch.cuda.synchronize()
    spec = vt.VisionSpec(hidden_size=D, num_heads=H)
    p = vt._P("fp64")
    cos, sin = vt.rotary_cos_sin(grids, spec, p)
    q = vt.apply_rotary(qkv[:, :D].reshape(N, H, hd), cos, sin, p)
    k = vt.apply_rotary(qkv[:, D:2 * D].reshape(N, H, hd), cos, sin, p)
    v = qkv[:, 2 * D:].reshape(N, H, hd)
    ref = vt.attention_varlen(q, k, v, m.cu_seqlens, p).reshape(N, D)
    return to_np(out), ref, m


def test_attention_f32_config1_vs_fp64(pkg, lib):
    """BASELINE config 1's packing (4 images, 4544 tokens, 16 x 64) in fp32: rel-L2 <= 1e-5."""
    got, ref, _ = _attention_f32(pkg, lib, [(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48)], 16, 64, 0)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-5


@pytest.mark.parametrize("hd", [64, 72, 80])
def test_attention_f32_ragged_vs_fp64(pkg, lib, hd):
    """Ragged segments (4..130 tokens) at head_dim 64, 72 and 80: per-segment rel-L2 <= 1e-5."""
    got, ref, m = _attention_f32(pkg, lib, [(1, 2, 2), (1, 4, 2), (3, 2, 6), (1, 10, 14), (1, 64, 2)], 3, hd, 4)
    assert np.isfinite(got).all()
    cu = m.cu_seqlens
    for i in range(len(cu) - 1):
        assert rel_l2(got[cu[i]:cu[i + 1]], ref[cu[i]:cu[i + 1]]) <= 1e-5, i


@pytest.mark.parametrize("hd,H,grids", [(64, 16, [(1, 28, 28)]), (72, 16, [(1, 28, 28)]), (80, 16, [(1, 16, 16), (1, 10, 30)]),
                                        (64, 4, [(1, 2, 2), (1, 4, 2), (3, 2, 6), (1, 10, 14), (1, 32, 32)])])
def test_attention_f32_split_list(pkg, lib, hd, H, grids):
    """fp32 attention on a qvl_attention_worklist_split list (config 0's 784-token image: 112 items for
    256 CUs, each split into key parts whose partials attn_combine_kernel sums; ragged segments)
    against the plain list (rel-L2 <= 1e-6: the same online softmax in another order) and fp64
    (<= 1e-5), every output written; on head-major operands in qvl_attention_headmajor's fp32 layout.
    (The ragged list runs 4 heads: with 16 its 208 items fill more than half the CUs, which the list
    builder leaves whole.)"""
    cp = pkg.capi
    m = pkg.grid_metadata(grids, dtype=cp.QVL_DTYPE_F32, num_heads=H)
    N = m.n_tokens
    Np = -(-N // 64) * 64
    vrows = -(-hd // 32) * 32
    rng = np.random.default_rng(hd + N)
    q = np.zeros((H, Np, hd), np.float32); k = np.zeros((H, Np, hd), np.float32); v = np.zeros((H, vrows, Np), np.float32)
    q[:, :N] = rng.standard_normal((H, N, hd)) * 0.25
    k[:, :N] = rng.standard_normal((H, N, hd))
    v[:, :hd, :N] = rng.standard_normal((H, hd, N))
    qt, kt, vt_ = dev32(q), dev32(k), dev32(v)
    n_cus = torch.cuda.get_device_properties(0).multi_processor_count
    split, n_whole = pkg.attention_worklist_split(m.cu_seqlens, H, hd, n_cus)
    plain = torch.from_numpy(m.tiles).to(DEV)
    st = torch.from_numpy(split).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_attention_split_workspace_size(hd, len(split), n_whole, C.byref(nb)))
    ws = torch.empty(max(nb.value, 256), dtype=torch.uint8, device=DEV)
    outs = []
    for lst in ("plain", "split"):
        out = torch.full((N, H * hd), float("nan"), dtype=torch.float32, device=DEV)
        if lst == "plain":
            cp.check(lib.qvl_attention_headmajor(stream(), cp.QVL_DTYPE_F32, qt.data_ptr(), kt.data_ptr(), vt_.data_ptr(),
                                                 plain.data_ptr(), len(m.tiles), N, H, hd, out.data_ptr(), H * hd))
        else:
            cp.check(lib.qvl_attention_headmajor_split(stream(), cp.QVL_DTYPE_F32, qt.data_ptr(), kt.data_ptr(),
                                                       vt_.data_ptr(), st.data_ptr(), len(split), n_whole, N, H, hd,
                                                       out.data_ptr(), H * hd, ws.data_ptr(), nb.value))
        torch.cuda.synchronize()
        outs.append(to_np(out))
    assert len(split) > n_whole, "the list should have parts"
    ref = np.zeros((N, H * hd))
    cu = m.cu_seqlens
    for i in range(len(cu) - 1):
        a, b = cu[i], cu[i + 1]
        for h in range(H):
            sc = q[h, a:b].astype(np.float64) @ k[h, a:b].astype(np.float64).T
            w = np.exp2(sc - sc.max(-1, keepdims=True))
            ref[a:b, h * hd:(h + 1) * hd] = (w @ v[h, :hd, a:b].astype(np.float64).T) / w.sum(-1, keepdims=True)
    for got in outs:
        assert np.isfinite(got).all()
        assert rel_l2(got, ref) <= 1e-5
    assert rel_l2(outs[1], outs[0]) <= 1e-6


@pytest.fixture(scope="module")
def params2b(pkg):
    return pkg.random_params(pkg.spec_2b(), seed=21)


def _ospec(s):
    return vt.VisionSpec(hidden_size=s.hidden_size, out_hidden_size=s.out_hidden_size, depth=s.depth,
                         num_heads=s.num_heads, intermediate_size=s.intermediate_size,
                         deepstack_visual_indexes=tuple(s.deepstack_visual_indexes))


def test_config0_fp32_tower_per_layer_and_final(pkg, params2b):
    """one 448x448 image with the frame duplicated (grid 1x28x28 = 784
    patches), the 2B tower in fp32, all 24 blocks and the deepstack taps. Every block (fed the
    fp64 oracle's input) and the whole tower (fused entry, and the staged per-op entries with
    per-layer taps) within rel-L2 1e-4 of the fp64 oracle, for tokens and every deepstack
    feature; the oracle's own fp32 mode is within the same bar."""
    spec = pkg.spec_2b()
    ospec = _ospec(spec)
    img = np.random.default_rng(7).standard_normal((3, 448, 448)).astype(np.float32)
    px, g = vt.patchify(np.stack([img, img]), patch=16, tpatch=2, merge=2)
    assert g.tolist() == [[1, 28, 28]] and px.shape == (784, 1536)
    ref = vt.encode_vision(params2b, px, g, ospec, "fp64", keep_layers=True)
    r32 = vt.encode_vision(params2b, px, g, ospec, "fp32")
    model = pkg.Qwen3VLModel(pkg.Qwen3VLSpec(text=None, vision=spec))   # float32 tower, as the reference builds it
    assert model.visual.dtype == "float32"
    emb = model.apply({"params": params2b}, px, g)
    assert emb.tokens.dtype == torch.float32 and emb.tokens.shape == (196, 2048)
    outs = [(to_np(emb.tokens), ref.tokens, r32.tokens)] + [
        (to_np(a), b, c) for a, b, c in zip(emb.deepstack, ref.deepstack, r32.deepstack)]
    assert len(outs) == 4
    for got, r64, rf in outs:
        assert rel_l2(rf, r64) <= TOL
        assert rel_l2(got, r64) <= TOL
    tower = model.visual
    ctx = tower._staged_ctx(g)
    x0 = tower.embed_staged(px, ctx)
    assert rel_l2(to_np(x0), ref.embed) <= TOL
    for i in range(spec.depth):
        xin = ref.embed if i == 0 else ref.layers[i - 1]
        x = dev32(xin)
        tower.block_staged(i, x, ctx)
        assert rel_l2(to_np(x), ref.layers[i]) <= TOL, f"block {i}"
    tok, ds, layers = tower.forward_staged(px, g, keep_layers=True)
    assert rel_l2(to_np(tok), ref.tokens) <= TOL
    for a, b in zip(ds, ref.deepstack):
        assert rel_l2(to_np(a), b) <= TOL
    for i, (a, b) in enumerate(zip(layers, ref.layers)):
        assert rel_l2(to_np(a), b) <= TOL, f"layer {i}"


def test_fp32_8b_shape_reduced_depth(pkg):
    """8B shape in fp32 (head_dim 72, I 4304 padded to 4352): first 3 blocks + deepstack after
    block 1 + the merger on two images, within rel-L2 1e-4 of the fp64 oracle."""
    spec = pkg.spec_8b()
    spec.depth = 3
    spec.deepstack_visual_indexes = (1,)
    params = pkg.random_params(spec, seed=22)
    grids = [(1, 16, 16), (1, 8, 12)]
    px = np.random.default_rng(8).standard_normal((352, 1536)).astype(np.float32)
    ref = vt.encode_vision(params, px, grids, _ospec(spec), "fp64")
    tower = pkg.Qwen3VisionTransformer(spec, dtype="float32").bind(params)
    tok, ds = tower(px, np.array(grids, np.int32))
    assert rel_l2(to_np(tok), ref.tokens) <= TOL
    assert rel_l2(to_np(ds[0]), ref.deepstack[0]) <= TOL


@pytest.mark.parametrize("shape", ["2b", "8b"])
def test_fp32_random_small_grids_vs_fp64(pkg, shape):
    """Seeded random small batches (1-3 images or short videos, even h and w up to 40, at most 2000
    patches) through the fp32 tower: the split-K GEMM plans and the split attention lists at
    varied sizes. The first 2 blocks + a deepstack tap after block 1 + the merger: tokens and
    deepstack within rel-L2 1e-4 of the fp64 oracle, every value finite."""
    spec = pkg.spec_2b() if shape == "2b" else pkg.spec_8b()
    spec.depth = 2
    spec.deepstack_visual_indexes = (1,)
    params = pkg.random_params(spec, seed=23 if shape == "2b" else 24)
    tower = pkg.Qwen3VisionTransformer(spec, dtype="float32").bind(params)
    rng = np.random.default_rng(2029 if shape == "2b" else 2030)
    for case in range(4):
        while True:
            grids = [(int(rng.choice([1, 1, 1, 2])), 2 * int(rng.integers(1, 21)), 2 * int(rng.integers(1, 21)))
                     for _ in range(int(rng.integers(1, 4)))]
            if sum(t * h * w for t, h, w in grids) <= 2000:
                break
        n = sum(t * h * w for t, h, w in grids)
        px = np.random.default_rng(200 + case).standard_normal((n, 1536)).astype(np.float32)
        ref = vt.encode_vision(params, px, grids, _ospec(spec), "fp64")
        tok, ds = tower(px, np.array(grids, np.int32))
        tok, ds0 = to_np(tok), to_np(ds[0])
        assert np.isfinite(tok).all() and np.isfinite(ds0).all(), grids
        assert rel_l2(tok, ref.tokens) <= TOL, (grids, rel_l2(tok, ref.tokens))
        assert rel_l2(ds0, ref.deepstack[0]) <= TOL, (grids, rel_l2(ds0, ref.deepstack[0]))
