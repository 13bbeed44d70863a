"""Kernel-level parity on the GPU, through the C ABI (libqvl.so), against the CPU oracle / a torch
fp32 reference of the same op. Tolerances are stated per test."""
import ctypes as C

import numpy as np
import pytest

from oracle import indices as ix
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def stream():
    return torch.cuda.current_stream().cuda_stream


def to_np(t):
    return t.float().cpu().numpy()


def bf(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def pack(lib, cp, kernel):
    kin, nout = kernel.shape
    src = torch.from_numpy(np.ascontiguousarray(kernel, np.float32)).to(DEV)
    kp, npad = -(-kin // 64) * 64, -(-nout // 64) * 64
    out = torch.empty((npad, kp), dtype=torch.bfloat16, device=DEV)
    cp.check(lib.qvl_pack_dense_weight(stream(), cp.QVL_DTYPE_BF16, src.data_ptr(), kin, nout, out.data_ptr()))
    return out


def ref_dense(x, w, bias, res, epi, n, k):
    """torch fp32 GEMM with the reference's bf16 cast points (flax Dense in bf16):
    y = bf16(bf16(x.W) + b); GELU: bf16(gelu(y)); residual: bf16(res + y)."""
    r = lambda t: t.to(torch.bfloat16).float()
    y = r(r(x.float() @ w[:n, :k].float().T) + bias)
    if epi == 1:
        y = r(torch.nn.functional.gelu(y, approximate="tanh"))
    if epi == 2:
        y = r(y + res.float())
    return y


def test_pack_weight_is_transpose_cast_pad(pkg, lib):
    rng = np.random.default_rng(0)
    k = rng.standard_normal((100, 70)).astype(np.float32)
    out = to_np(pack(lib, pkg.capi, k))
    assert out.shape == (128, 128)
    np.testing.assert_array_equal(out[:70, :100], vt.bf16_round(k.T))
    assert not out[70:].any() and not out[:, 100:].any()


@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", [(300, 192, 128), (1024, 3072, 1024), (257, 4096, 64), (4608, 2048, 4096)])
def test_dense_epilogues_vs_torch_fp32(pkg, lib, epi, m, n, k):
    """bf16 GEMM + epilogue vs torch fp32 on the same bf16 operands with the same bf16 cast
    points: rel-L2 <= 4e-3, every element within one bf16 ulp of the output and of the
    pre-residual product, + 1e-2 absolute."""
    cp = pkg.capi
    g = torch.Generator(device="cpu").manual_seed(m * 7 + n + k + epi)
    x = torch.randn((m, k), generator=g).to(DEV).to(torch.bfloat16)
    wk = (torch.randn((k, n), generator=g) * 0.05).numpy()
    w = pack(lib, cp, wk)
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).float().to(DEV)
    res = torch.randn((m, n), generator=g).to(DEV).to(torch.bfloat16)
    y = res.clone() if epi == 2 else torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    r_ptr = y.data_ptr() if epi == 2 else 0      # residual aliases the output (in-place x += ...)
    cp.check(lib.qvl_dense(stream(), cp.QVL_DTYPE_BF16, epi, x.data_ptr(), k, w.data_ptr(), bias.data_ptr(),
                           r_ptr, n, y.data_ptr(), n, m, n, k))
    ref = ref_dense(x, w, bias, res, epi, n, k)
    torch.cuda.synchronize()
    got, ref = to_np(y), ref.cpu().numpy()
    assert rel_l2(got, ref) <= 4e-3
    # one bf16 ulp of the output and of the pre-residual product (an fp32 summation-order
    # difference can move that product's rounding by one ulp before the residual add)
    pre = np.abs(ref - to_np(res)) if epi == 2 else np.abs(ref)
    assert np.all(np.abs(got - ref) <= 2 ** -7 * (np.abs(ref) + pre) + 1e-2)


@pytest.mark.parametrize("cols", [1024, 1152, 4096, 4608])
def test_layer_norm_vs_oracle(pkg, lib, cols):
    """bf16 LayerNorm vs the oracle's bf16 LayerNorm: rel-L2 <= 4e-3, max 2 bf16 ulps."""
    cp = pkg.capi
    rng = np.random.default_rng(cols)
    rows = 517
    x = vt.bf16_round(rng.standard_normal((rows, cols)) * 3 + 1.5)
    gm = vt.bf16_round(1 + 0.1 * rng.standard_normal(cols)); bt = vt.bf16_round(0.1 * rng.standard_normal(cols))
    xt, yt = bf(x), torch.empty((rows, cols), dtype=torch.bfloat16, device=DEV)
    gt, btt = torch.from_numpy(gm).to(DEV), torch.from_numpy(bt).to(DEV)
    cp.check(lib.qvl_layer_norm(stream(), cp.QVL_DTYPE_BF16, xt.data_ptr(), cols, gt.data_ptr(), btt.data_ptr(),
                                yt.data_ptr(), cols, rows, cols, 1e-6))
    ref = vt.layer_norm(x, gm, bt, 1e-6, vt._P("bf16"))
    got = to_np(yt)
    assert rel_l2(got, ref) <= 4e-3
    assert np.all(np.abs(got - ref) <= 2 * 2 ** -8 * np.abs(ref) + 1e-6)


@pytest.mark.parametrize("grids", [[(8, 32, 32)], [(2, 48, 48)], [(1, 84, 84), (3, 10, 6)]])
def test_pos_embed_vs_oracle(pkg, lib, grids):
    """4-tap gather in the reference's bf16 arithmetic (each tap product and each partial sum
    rounded, left to right, model.py:751-752): bit-identical to the oracle's bf16 pos-embed, on
    config 3's video grid (repeat quirk), config 4's grid and a ragged batch. On a 48 x 48 grid
    (the table's own side) every token has one tap of weight 1 and three of weight 0, which the
    kernel skips: the output is exactly that table row."""
    cp = pkg.capi
    spec = vt.VisionSpec()
    table = np.random.default_rng(0).standard_normal((2304, 1024)).astype(np.float32) * 0.02
    m = pkg.grid_metadata(grids)
    idx, w = torch.from_numpy(m.tap_idx).to(DEV), torch.from_numpy(m.tap_w).to(DEV)
    tt = bf(table)
    out = torch.empty((m.n_tokens, 1024), dtype=torch.bfloat16, device=DEV)
    cp.check(lib.qvl_pos_embed(stream(), cp.QVL_DTYPE_BF16, tt.data_ptr(), idx.data_ptr(), w.data_ptr(),
                               out.data_ptr(), m.n_tokens, 1024))
    ref = vt.pos_embed(table, grids, spec, vt._P("bf16"))
    np.testing.assert_array_equal(to_np(out), ref)
    if grids[0][1] == 48:
        wn = m.tap_w.reshape(4, -1)
        assert np.all(np.sort(wn, axis=0)[-1] == 1.0) and np.all(np.sort(wn, axis=0)[:-1] == 0.0)
        row = m.tap_idx.reshape(4, -1)[np.argmax(wn, axis=0), np.arange(m.n_tokens)]
        np.testing.assert_array_equal(to_np(out), vt.bf16_round(table)[row])


@pytest.mark.parametrize("grids,k,parts", [([(1, 48, 48), (1, 48, 48)], 1536, True), ([(1, 84, 84), (3, 10, 6)], 1536, True),
                                           ([(8, 32, 32)], 1216, False), ([(1, 20, 36)], 64, True),
                                           ([(1, 48, 48)], 1536, True), ([(1, 28, 28)], 1536, True)])
def test_dense_pos_embed_equals_pos_embed_then_residual(pkg, lib, grids, k, parts):
    """qvl_dense_pos_embed_ws (the patch embed with the pos-embed gathered in its epilogue, the
    tower's bf16 path) against qvl_pos_embed followed by the residual Dense (qvl_dense_rowstats_ws,
    or qvl_dense_ws with the split-K tail off): the output and the row partials bit for bit, on
    config 2's two-image grid (48 x 48: single-tap rows), config 4's grid with a ragged image
    (four live taps per row), config 3's video (the jnp.repeat frame quirk), a short K and one
    768 x 768 image (2304 rows: 128 x 128 tiles by the small-grid rule) and a 448 x 448 one (784 rows:
    64 x 128 tiles)."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    N, D = m.n_tokens, 1024
    rng = np.random.default_rng(N + k)
    table = bf(rng.standard_normal((2304, D)).astype(np.float32) * 0.02)
    x = bf(rng.standard_normal((N, k)).astype(np.float32))
    w = pack(lib, cp, (rng.standard_normal((k, D)) * 0.03).astype(np.float32))
    bias = torch.from_numpy(vt.bf16_round((rng.standard_normal(D) * 0.02).astype(np.float32))).to(DEV)
    idx, tw = torch.from_numpy(m.tap_idx).to(DEV), torch.from_numpy(m.tap_w).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    pos = torch.empty((N, D), dtype=torch.bfloat16, device=DEV)
    cp.check(lib.qvl_pos_embed(stream(), cp.QVL_DTYPE_BF16, table.data_ptr(), idx.data_ptr(), tw.data_ptr(),
                               pos.data_ptr(), N, D))
    y_ref = torch.empty((N, D), dtype=torch.bfloat16, device=DEV)
    y = torch.full((N, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    p_ref = torch.zeros((N, D // 128, 2), dtype=torch.float32, device=DEV)
    p_got = torch.full((N, D // 128, 2), float("nan"), dtype=torch.float32, device=DEV)
    try:
        cp.check(lib.qvl_set_gemm_plan(0, -1, 0))
        if parts:
            cp.check(lib.qvl_dense_rowstats_ws(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), k, w.data_ptr(),
                                               bias.data_ptr(), pos.data_ptr(), D, y_ref.data_ptr(), D, N, D, k,
                                               p_ref.data_ptr(), ws.data_ptr(), nb.value))
        else:
            cp.check(lib.qvl_dense_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_RESIDUAL, x.data_ptr(), k,
                                      w.data_ptr(), bias.data_ptr(), pos.data_ptr(), D, y_ref.data_ptr(), D, N, D, k,
                                      ws.data_ptr(), nb.value))
    finally:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
    cp.check(lib.qvl_dense_pos_embed_ws(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), k, w.data_ptr(), bias.data_ptr(),
                                        table.data_ptr(), idx.data_ptr(), tw.data_ptr(), y.data_ptr(), D, N, D, k,
                                        p_got.data_ptr() if parts else None, ws.data_ptr(), nb.value))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(y), to_np(y_ref))
    if parts:
        np.testing.assert_array_equal(p_got.cpu().numpy(), p_ref.cpu().numpy())
    # and against the oracle's bf16 pos-embed + Dense arithmetic within the GEMM tolerance
    ref = ref_dense(x, w, bias, torch.from_numpy(vt.pos_embed(to_np(table), grids, vt.VisionSpec(), vt._P("bf16"))).to(DEV),
                    2, D, k)
    assert rel_l2(to_np(y), ref.cpu().numpy()) <= 4e-3


def test_rotary_table_vs_oracle(pkg, lib):
    """cos/sin table in bf16 mode: the oracle's bf16 cos/sin, up to one bf16 ulp where device and
    numpy float32 cos/sin round a value near a bf16 rounding boundary differently."""
    cp = pkg.capi
    grids = [(1, 84, 84), (2, 8, 4)]
    m = pkg.grid_metadata(grids)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    for hd in (64, 72):
        cs = torch.empty((m.n_tokens, hd // 2, 2), dtype=torch.float32, device=DEV)
        cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), m.n_tokens, hd, 10000.0,
                                      cs.data_ptr()))
        spec = vt.VisionSpec(hidden_size=16 * hd, num_heads=16)
        cref, sref = vt.rotary_cos_sin(grids, spec, vt._P("bf16"))
        got = cs.cpu().numpy()
        for k, ref in ((0, cref[:, : hd // 2]), (1, sref[:, : hd // 2])):
            g = got[..., k]
            ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref), 1e-30))) - 7)
            assert np.all(np.abs(g - ref) <= ulp + 1e-30)          # at most one bf16 ulp
            assert np.mean(g == ref) >= 0.99                        # and almost always equal


def _attention_case(pkg, lib, grids, H=16, hd=64, seed=0, perturb=None):
    cp = pkg.capi
    m = pkg.grid_metadata(grids, num_heads=H)
    N, D = m.n_tokens, H * hd
    rng = np.random.default_rng(seed)
    qkv = vt.bf16_round(rng.standard_normal((N, 3 * D)).astype(np.float32))
    if perturb is not None:
        perturb(qkv, m)
    qkv_t = bf(qkv)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, hd // 2, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    tiles = torch.from_numpy(m.tiles if len(m.tiles) else np.zeros((1, 4), np.int32)).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_vision_attention_workspace_size(cp.QVL_DTYPE_BF16, N, H, hd, C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    out = torch.full((N, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    cp.check(lib.qvl_vision_attention(stream(), cp.QVL_DTYPE_BF16, qkv_t.data_ptr(), qkv_t.data_ptr() + 2 * D,
                                      qkv_t.data_ptr() + 4 * D, 3 * D, cs.data_ptr(), tiles.data_ptr(), len(m.tiles),
                                      out.data_ptr(), D, N, H, hd, ws.data_ptr(), nb.value))
    torch.cuda.synchronize()
    # oracle: reference rotary (bf16 arithmetic) + fp32 segment softmax
    spec = vt.VisionSpec(hidden_size=D, num_heads=H)
    p = vt._P("bf16")
    cos, sin = vt.rotary_cos_sin(grids, spec, p)
    q = vt.apply_rotary(qkv[:, :D].reshape(N, H, hd), cos, sin, p)
    k = vt.apply_rotary(qkv[:, D:2 * D].reshape(N, H, hd), cos, sin, p)
    v = qkv[:, 2 * D:].reshape(N, H, hd)
    ref = vt.attention_varlen(q, k, v, m.cu_seqlens, vt._P("fp32")).reshape(N, D)
    return to_np(out), ref, m


def test_attention_config1_vs_oracle(pkg, lib):
    """BASELINE config 1 (4 images packed, 4544 tokens, 16x64): rel-L2 <= 1e-2 vs the oracle (bf16
    P and one bf16 rounding of scaled q; the reference rounds rotary per op)."""
    got, ref, _ = _attention_case(pkg, lib, [(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48)])
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-2


@pytest.mark.parametrize("grids", [[(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48)], [(1, 10, 14), (2, 6, 8)]])
def test_attention_relayout_paths_bit_exact(pkg, lib, grids):
    """qvl_vision_attention (head_dim 64) takes the 16-byte relayout kernel for aligned q/k/v and a
    row stride that is a multiple of 8 elements, and the element-wise one otherwise: the same
    q/k/v stored with row stride 3D (aligned) and 3D + 4 give bit-identical outputs."""
    cp = pkg.capi
    H, hd = 16, 64
    m = pkg.grid_metadata(grids, num_heads=H)
    N, D = m.n_tokens, H * hd
    rng = np.random.default_rng(11)
    qkv = vt.bf16_round(rng.standard_normal((N, 3 * D)).astype(np.float32))
    wide = np.zeros((N, 3 * D + 4), np.float32)
    wide[:, :3 * D] = qkv
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, hd // 2, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    tiles = torch.from_numpy(m.tiles).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_vision_attention_workspace_size(cp.QVL_DTYPE_BF16, N, H, hd, C.byref(nb)))
    outs = []
    for arr in (qkv, wide):
        t = bf(arr)
        ld = arr.shape[1]
        ws = torch.full((nb.value // 2,), float("nan"), dtype=torch.bfloat16, device=DEV)
        out = torch.full((N, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        cp.check(lib.qvl_vision_attention(stream(), cp.QVL_DTYPE_BF16, t.data_ptr(), t.data_ptr() + 2 * D,
                                          t.data_ptr() + 4 * D, ld, cs.data_ptr(), tiles.data_ptr(), len(m.tiles),
                                          out.data_ptr(), D, N, H, hd, ws.data_ptr(), nb.value))
        torch.cuda.synchronize()
        outs.append((to_np(out), ws.view(torch.int16).cpu().numpy()))
    assert np.isfinite(outs[0][0]).all()
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])      # the staged Q | K | V^T, padding rows included


@pytest.mark.parametrize("grids", [[(1, 2, 2)], [(1, 2, 2), (1, 4, 2), (3, 2, 6)], [(1, 10, 14), (2, 6, 8)],
                                   [(1, 64, 2)]])
def test_attention_ragged_segments(pkg, lib, grids):
    """Tiny and ragged segments (lengths 4..130, not multiples of the 64-key tile): every row
    finite, rel-L2 <= 1e-2 per segment, and rows never see keys of another segment."""
    got, ref, m = _attention_case(pkg, lib, grids, H=2, seed=3)
    assert np.isfinite(got).all()
    cu = m.cu_seqlens
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        assert rel_l2(got[s:e], ref[s:e]) <= 1e-2, (i, s, e)


def test_attention_segment_isolation_exact(pkg, lib):
    """Changing the last segment's q/k/v leaves the other segments' outputs bit-identical."""
    grids = [(1, 8, 8), (1, 4, 4), (1, 6, 6)]
    a, _, m = _attention_case(pkg, lib, grids, H=4, seed=5)

    def bump(qkv, m):
        qkv[m.cu_seqlens[2]:] += 3.0

    b, _, _ = _attention_case(pkg, lib, grids, H=4, seed=5, perturb=bump)
    e = m.cu_seqlens[2]
    np.testing.assert_array_equal(a[:e], b[:e])
    assert not np.array_equal(a[e:], b[e:])


def test_attention_config4_hd72_vs_oracle(pkg, lib):
    """BASELINE config 4's attention: one 7056-token segment (grid 1x84x84), 16 heads x head_dim 72
    (Q/K rows of 88 dims, V^T of 72 rows inside the library): rel-L2 <= 1e-2 vs the oracle."""
    got, ref, _ = _attention_case(pkg, lib, [(1, 84, 84)], H=16, hd=72, seed=9)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-2


@pytest.mark.parametrize("hd", [72, 80])
@pytest.mark.parametrize("grids", [[(1, 2, 2), (1, 4, 2), (3, 2, 6)], [(1, 10, 14), (2, 6, 8)]])
def test_attention_hd72_ragged(pkg, lib, grids, hd):
    """The 88-element-row kernel (head_dim 72 and 80) on tiny and ragged segments: per-segment
    rel-L2 <= 1e-2 against the oracle, every row finite."""
    got, ref, m = _attention_case(pkg, lib, grids, H=2, hd=hd, seed=4)
    assert np.isfinite(got).all()
    cu = m.cu_seqlens
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        assert rel_l2(got[s:e], ref[s:e]) <= 1e-2, (i, s, e)


def test_attention_hd80_vs_oracle(pkg, lib):
    """head_dim 80 (a 1280-wide, 16-head tower's heads; here 4 heads) on one 2304-token segment: the
    88-element-row kernel with the ones row at 80 for the row sums, rel-L2 <= 1e-2 vs the oracle."""
    got, ref, _ = _attention_case(pkg, lib, [(1, 48, 48)], H=4, hd=80, seed=10)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 1e-2


def _headmajor_operands(H, hd, cu, seed):
    """Random head-major attention operands in qvl_attention_headmajor's bf16 layout: q (already
    scaled by head_dim^-0.5 * log2 e) and k as [H][Np][hdp], v^T as [H][vrows][Np] with the keys
    at their vt_pos positions (hdp, vrows = 64, 64 or 88, hd), padding zero."""
    N = int(cu[-1])
    Np = (max(N, 1) + 63) // 64 * 64
    hdp = 64 if hd == 64 else 88
    g = torch.Generator().manual_seed(seed)
    q = torch.zeros((H, Np, hdp)); k = torch.zeros((H, Np, hdp)); vt = torch.zeros((H, hd, Np))
    q[:, :N, :hd] = torch.randn((H, N, hd), generator=g) * (hd ** -0.5 * 1.4426950408889634)
    k[:, :N, :hd] = torch.randn((H, N, hd), generator=g)
    vt[:, :, :N] = torch.randn((H, hd, N), generator=g)
    q, k, vt = (t.to(torch.bfloat16) for t in (q, k, vt))
    # V^T stores key n at position vt_pos(n): the middle two groups of 4 in every 16 swap
    n = np.arange(Np)
    quad = (n >> 2) & 3
    pos = (n & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (n & 3)
    vt_mem = torch.empty_like(vt)
    vt_mem[:, :, torch.from_numpy(pos)] = vt
    # fp32 reference on the CPU: per segment softmax_2(q k^T) v
    ref = torch.zeros((N, H * hd))
    for s, e in zip(cu[:-1], cu[1:]):
        if e <= s:
            continue
        sc = torch.einsum("hqd,hkd->hqk", q[:, s:e, :hd].float(), k[:, s:e, :hd].float())
        p = torch.softmax(sc * 0.6931471805599453, dim=-1)
        o = torch.einsum("hqk,hdk->hqd", p, vt[:, :, s:e].float())
        ref[s:e] = o.permute(1, 0, 2).reshape(e - s, H * hd)
    return q.to(DEV), k.to(DEV), vt_mem.to(DEV), ref.numpy()


@pytest.mark.parametrize("hd,cu,H,n_cus", [(64, [0, 4096, 8192, 18432], 16, 280),     # config 2's segments, 8 parts
                                           (72, [0, 7056], 16, 256),                   # config 4, 6 parts
                                           (64, [0, 1000, 1003, 5099, 5100], 4, 20),  # ragged, 1-key segments
                                           (72, [0, 130, 4226], 2, 22),
                                           (80, [0, 130, 4226], 2, 22)])
def test_attention_split_items_match_whole(pkg, lib, hd, cu, H, n_cus):
    """qvl_attention_headmajor_split on a split list agrees with qvl_attention_headmajor on the
    whole list (rel-L2 <= 5e-3: only the bf16 rounding of P against the parts' running maxima
    differs) and with an fp32 reference (rel-L2 <= 1e-2)."""
    cp = pkg.capi
    cu = np.array(cu, np.int32)
    N = int(cu[-1])
    q, k, vt, ref = _headmajor_operands(H, hd, cu, seed=hd + N)
    base = pkg.vision._worklist(lib, cu, H)
    split, n_whole = pkg.attention_worklist_split(cu, H, hd, n_cus)
    assert len(split) > n_whole                                   # the case does split
    outs = []
    for items, nw in ((base, None), (split, n_whole)):
        t = torch.from_numpy(np.ascontiguousarray(items)).to(DEV)
        out = torch.full((N, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
        if nw is None:
            cp.check(lib.qvl_attention_headmajor(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(), vt.data_ptr(),
                                                 t.data_ptr(), len(items), N, H, hd, out.data_ptr(), H * hd))
        else:
            nb = C.c_size_t()
            cp.check(lib.qvl_attention_split_workspace_size(hd, len(items), nw, C.byref(nb)))
            ws = torch.full((max(nb.value, 16) // 4,), float("nan"), dtype=torch.float32, device=DEV)
            for _ in range(2):                                     # stale workspace contents do not leak
                cp.check(lib.qvl_attention_headmajor_split(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(),
                                                           vt.data_ptr(), t.data_ptr(), len(items), nw, N, H, hd,
                                                           out.data_ptr(), H * hd, ws.data_ptr(), nb.value))
        torch.cuda.synchronize()
        outs.append(to_np(out))
    whole, parts = outs
    assert np.isfinite(parts).all()
    assert rel_l2(parts, whole) <= 5e-3
    assert rel_l2(parts, ref) <= 1e-2
    for s, e in zip(cu[:-1], cu[1:]):
        if e > s:
            assert rel_l2(parts[s:e], ref[s:e]) <= 1e-2, (s, e)


@pytest.mark.parametrize("hd", [64, 72, 80])
@pytest.mark.parametrize("spike", [40.0, 100.0])
def test_attention_late_score_spike(pkg, lib, hd, spike):
    """Scores far above the rest of their row, late in the key range. The kernels take p = 2^s
    unshifted (s in log2 units) and check each wave's rows after the key loop: a row sum outside
    [2^-64, 2^96] or an accumulator above 2^120 (inf / NaN included) sends the wave to its exact
    recompute (row max first, then p = 2^(s - max)). A spike of 40 stays inside the fast path's
    range; a spike of 100 overflows the row sum and takes the recompute. Keys in a middle tile and
    in the segment's last (masked) tile spike for some query rows of every head, on the whole and
    the split work lists: rel-L2 <= 1e-2 against an fp32 reference per segment, every row finite."""
    cp = pkg.capi
    H = 4
    cu = np.array([0, 100, 2600, 2700, 7000], np.int32)
    N = int(cu[-1])
    q, k, vt, _ = _headmajor_operands(H, hd, cu, seed=11 + hd)
    q, k, vt = q.cpu(), k.cpu(), vt.cpu()
    # rows r of segment [s, e) get q[r, 0] = 8 and spiking keys j get k[j, 0] = (spike + 8) / 8 * 8 / 8;
    # the other keys' dimension 0 is cleared so the spike stands out by ~spike
    rows_keys = [(range(110, 400, 7), 1000), (range(2620, 2700, 3), 2690), (range(4000, 7000, 11), 6990),
                 (range(2610, 2640), 2650), (range(3000, 3010), 6500)]
    kval = spike / 8.0
    for rows, key in rows_keys:
        for r in rows:
            q[:, r, 0] = 8.0
        k[:, key, 0] = kval
    for h in range(H):
        for s, e in zip(cu[:-1], cu[1:]):
            others = [j for j in range(s, e) if j not in {key for _, key in rows_keys}]
            k[h, others, 0] = 0.0
    ref = torch.zeros((N, H * hd))
    vt_keys = torch.empty_like(vt)
    n = np.arange(vt.shape[2])
    quad = (n >> 2) & 3
    pos = (n & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (n & 3)
    vt_keys[:, :, :] = vt[:, :, torch.from_numpy(pos)]
    for s, e in zip(cu[:-1], cu[1:]):
        sc = torch.einsum("hqd,hkd->hqk", q[:, s:e, :hd].float(), k[:, s:e, :hd].float())
        p = torch.softmax(sc * 0.6931471805599453, dim=-1)
        ref[s:e] = torch.einsum("hqk,hdk->hqd", p, vt_keys[:, :, s:e].float()).permute(1, 0, 2).reshape(e - s, H * hd)
    ref = ref.numpy()
    q, k, vt = q.to(DEV), k.to(DEV), vt.to(DEV)
    lists = [(pkg.vision._worklist(lib, cu, H), None)]
    split, n_whole = pkg.attention_worklist_split(cu, H, hd, 40)
    if len(split) > n_whole:
        lists.append((split, n_whole))
    for items, nw in lists:
        t = torch.from_numpy(np.ascontiguousarray(items)).to(DEV)
        out = torch.full((N, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
        if nw is None:
            cp.check(lib.qvl_attention_headmajor(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(), vt.data_ptr(),
                                                 t.data_ptr(), len(items), N, H, hd, out.data_ptr(), H * hd))
        else:
            nb = C.c_size_t()
            cp.check(lib.qvl_attention_split_workspace_size(hd, len(items), nw, C.byref(nb)))
            ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=DEV)
            cp.check(lib.qvl_attention_headmajor_split(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(),
                                                       vt.data_ptr(), t.data_ptr(), len(items), nw, N, H, hd,
                                                       out.data_ptr(), H * hd, ws.data_ptr(), nb.value))
        torch.cuda.synchronize()
        got = to_np(out)
        assert np.isfinite(got).all(), nw
        for s, e in zip(cu[:-1], cu[1:]):
            assert rel_l2(got[s:e], ref[s:e]) <= 1e-2, (nw, s, e, rel_l2(got[s:e], ref[s:e]))
        for rows, key in rows_keys:             # the spiking rows follow their key's value row
            r = np.array(list(rows))
            assert rel_l2(got[r], ref[r]) <= 1e-2, (nw, key)


def _run_attention_lists(pkg, lib, q, k, vt, cu, H, hd):
    """qvl_attention_headmajor on the plain work list and qvl_attention_headmajor_split on the
    split list of 40 CUs (when it splits), head_dim 64 under both key-group plans (one group of 4
    waves per item; two, each taking half of the item's key tiles): [(label, bf16 output as fp32
    numpy)]."""
    cp = pkg.capi
    N = int(cu[-1])
    lists = [(pkg.vision._worklist(lib, cu, H), None)]
    split, n_whole = pkg.attention_worklist_split(cu, H, hd, 40)
    if len(split) > n_whole:
        lists.append((split, n_whole))
    outs = []
    for groups in ((1, 2) if hd == 64 else (0,)):
        for items, nw in lists:
            t = torch.from_numpy(np.ascontiguousarray(items)).to(DEV)
            out = torch.full((N, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
            try:
                cp.check(lib.qvl_set_attention_plan(groups))
                if nw is None:
                    cp.check(lib.qvl_attention_headmajor(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(),
                                                         vt.data_ptr(), t.data_ptr(), len(items), N, H, hd,
                                                         out.data_ptr(), H * hd))
                else:
                    nb = C.c_size_t()
                    cp.check(lib.qvl_attention_split_workspace_size(hd, len(items), nw, C.byref(nb)))
                    ws = torch.empty(max(nb.value, 16), dtype=torch.uint8, device=DEV)
                    cp.check(lib.qvl_attention_headmajor_split(stream(), cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(),
                                                               vt.data_ptr(), t.data_ptr(), len(items), nw, N, H, hd,
                                                               out.data_ptr(), H * hd, ws.data_ptr(), nb.value))
            finally:
                cp.check(lib.qvl_set_attention_plan(0))
            torch.cuda.synchronize()
            outs.append((("whole" if nw is None else "split") + f"/groups{groups}", to_np(out)))
    return outs


@pytest.mark.parametrize("cu,H", [([0, 784], 16),                                   # one 448x448 image
                                  ([0, 1024, 1984, 2240, 4544], 16),                # config 1's segments
                                  ([0, 1, 65, 129, 130, 300, 1000], 4),              # 1 / 1 / 2 / 1 / 3 / 11 key tiles
                                  ([0, 4096, 8192, 18432], 2)])
def test_attention_key_groups_match(pkg, lib, cu, H):
    """Head_dim-64 attention with two key groups per work item (8 waves: group 1 takes the second
    half of the item's key tiles and hands its O, shift and row sums to group 0 through LDS; a
    1-tile item leaves group 1 empty) against one group, on the plain and the split work lists:
    every row finite, rel-L2 <= 3e-3 against one group (the bf16 rounding of the output and the
    fp32 order of the two halves' sums differ) and <= 1e-2 against an fp32 reference per
    segment. The default rule takes two groups where the items number at most 2x the CUs."""
    cu = np.array(cu, np.int32)
    N = int(cu[-1])
    q, k, vt, ref = _headmajor_operands(H, 64, cu, seed=N + H)
    outs = dict(_run_attention_lists(pkg, lib, q, k, vt, cu, H, 64))
    for label, got in outs.items():
        assert np.isfinite(got).all(), label
        for s, e in zip(cu[:-1], cu[1:]):
            assert rel_l2(got[s:e], ref[s:e]) <= 1e-2, (label, s, e)
    for lst in ("whole", "split"):
        if f"{lst}/groups1" in outs:
            assert rel_l2(outs[f"{lst}/groups2"], outs[f"{lst}/groups1"]) <= 3e-3, lst


@pytest.mark.parametrize("hd", [64, 72])
@pytest.mark.parametrize("case", ["sum_below_2^-64", "sum_zero", "accumulator_above_2^120"])
def test_attention_exact_recompute_triggers(pkg, lib, hd, case):
    """The other two triggers of the exact recompute (see test_attention_late_score_spike for the
    row-sum overflow). "sum_below_2^-64": every score of some rows is about -80 (log2 units), so
    their unshifted row sums (~L * 2^-80) fall under 2^-64; "sum_zero": about -200, so every
    2^s underflows fp32 and the unshifted sums are 0 (0/0 without the recompute);
    "accumulator_above_2^120": scores about +30 (row sums ~L * 2^30, inside the range) against V
    rows of magnitude ~2^100, so the unnormalised accumulator passes 2^120 (overflows fp32) while
    the row sums do not. Rows in a short segment, a long one and the last (masked) key tiles, on
    the whole and the split work lists: rel-L2 <= 1e-2 against an fp32 softmax reference per
    segment, every row finite."""
    H = 4
    cu = np.array([0, 100, 2600, 2700, 7000], np.int32)
    N = int(cu[-1])
    q, k, vt, _ = _headmajor_operands(H, hd, cu, seed=31 + hd)
    q, k, vt = q.cpu(), k.cpu(), vt.cpu()
    n = np.arange(vt.shape[2])
    quad = (n >> 2) & 3
    pos = torch.from_numpy((n & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (n & 3))
    v_keys = vt[:, :, pos].float()                         # V^T in key order
    shift = {"sum_below_2^-64": -80.0, "sum_zero": -200.0, "accumulator_above_2^120": 30.0}[case]
    rows = list(range(10, 60, 3)) + list(range(2610, 2700, 2)) + list(range(2700, 7000, 13))
    for r in rows:
        q[:, r, 0] = 8.0
    k[:, :N, 0] = shift / 8.0                             # every key: the shifted rows score ~shift
    if case == "accumulator_above_2^120":
        v_keys[:, :, :N] *= 2.0 ** 100
    vt[:, :, pos] = v_keys.to(torch.bfloat16)
    v_keys = vt[:, :, pos].float()
    ref = torch.zeros((N, H * hd))
    for s, e in zip(cu[:-1], cu[1:]):
        sc = torch.einsum("hqd,hkd->hqk", q[:, s:e, :hd].float(), k[:, s:e, :hd].float())
        p = torch.softmax(sc * 0.6931471805599453, dim=-1)
        ref[s:e] = torch.einsum("hqk,hdk->hqd", p, v_keys[:, :, s:e]).permute(1, 0, 2).reshape(e - s, H * hd)
    ref = ref.numpy()
    for label, got in _run_attention_lists(pkg, lib, q.to(DEV), k.to(DEV), vt.to(DEV), cu, H, hd):
        assert np.isfinite(got).all(), label
        for s, e in zip(cu[:-1], cu[1:]):
            assert rel_l2(got[s:e], ref[s:e]) <= 1e-2, (label, s, e, rel_l2(got[s:e], ref[s:e]))
        r = np.array(rows)
        assert rel_l2(got[r], ref[r]) <= 1e-2, label


_TILES = {"288x256": 1, "256x256": 2, "256x128": 3, "288x128": 4, "rowsplit": 5, "128x128": 6, "64x192": 7,
          "64x128": 8}


def set_plan(lib, cp, plan):
    """Pin the calling thread's GEMM tile plan ("<tile>:split|:nosplit"); None restores the cost model."""
    if plan is None:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0), "qvl_set_gemm_plan")
        return
    tile, mode = plan.split(":")
    cp.check(lib.qvl_set_gemm_plan(_TILES[tile], 1 if mode == "split" else -1, 0), "qvl_set_gemm_plan")


PLANS = ["288x256:nosplit", "256x256:nosplit", "256x128:nosplit", "288x128:nosplit", "rowsplit:nosplit",
         "128x128:nosplit", "64x128:nosplit", "288x256:split", "256x256:split", "256x128:split", "288x128:split",
         "128x128:split", "64x128:split"]


def dense_ws(lib, cp, epi, x, w, bias, res, m, n, k, ws):
    y = res.clone() if epi == 2 else torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    r_ptr = y.data_ptr() if epi == 2 else 0
    cp.check(lib.qvl_dense_ws(stream(), cp.QVL_DTYPE_BF16, epi, x.data_ptr(), k, w.data_ptr(), bias.data_ptr(),
                              r_ptr, n, y.data_ptr(), n, m, n, k, ws.data_ptr(), ws.numel()))
    return to_np(y)


@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("m,n,k", [(18432, 1024, 1024), (4600, 2048, 4096), (2304, 4096, 1024), (300, 192, 128),
                                   (18000, 1152, 4352), (300, 192, 64), (1000, 640, 192), (8192, 3072, 1024),
                                   (784, 4096, 1024)])
def test_dense_tile_plans_agree(pkg, lib, epi, m, n, k):
    """Every tile shape (288x256 / 256x256 / 256x128 / 288x128 / 128x128 / 64x128, 128x128 the
    default at 784 x 4096 x 1024) and the row split (whole rounds of
    288x256 tiles, the remaining rows as 256x128 tiles in a second launch: taken at 18000 and 8192
    rows, elsewhere it falls back to 288x256) gives bit-identical results without the tail split
    (same K order per output); with the split (fp32 partials summed by the reduce kernel) within
    rel-L2 2e-3 of them; all within rel-L2 4e-3 of torch fp32 on the same bf16 operands. Shapes
    include M not a multiple of any tile height and N not a multiple of 256, and K of 1, 2 and 3
    k-steps (the three-stage ring of the 128-column tiles with fewer k-steps than stages; split
    units of one k-step)."""
    cp = pkg.capi
    g = torch.Generator(device="cpu").manual_seed(m + n + k + epi)
    x = torch.randn((m, k), generator=g).to(DEV).to(torch.bfloat16)
    w = pack(lib, cp, (torch.randn((k, n), generator=g) * 0.05).numpy())
    bias = (torch.randn(n, generator=g) * 0.1).to(torch.bfloat16).float().to(DEV)
    res = torch.randn((m, n), generator=g).to(DEV).to(torch.bfloat16)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    outs = {}
    try:
        for plan in PLANS:
            set_plan(lib, cp, plan)
            outs[plan] = dense_ws(lib, cp, epi, x, w, bias, res, m, n, k, ws)
    finally:
        set_plan(lib, cp, None)
    outs["auto"] = dense_ws(lib, cp, epi, x, w, bias, res, m, n, k, ws)
    ref = ref_dense(x, w, bias, res, epi, n, k).cpu().numpy()
    base = outs["256x256:nosplit"]
    for plan, got in outs.items():
        if plan.endswith(":nosplit"):
            np.testing.assert_array_equal(got, base, err_msg=plan)
        else:
            assert rel_l2(got, base) <= 2e-3, plan
        assert rel_l2(got, ref) <= 4e-3, plan


@pytest.mark.parametrize("grids", [[(1, 48, 48)] * 8, [(1, 16, 16), (2, 10, 14), (1, 6, 8)], [(8, 32, 32)],
                                   [(1, 28, 28)]])
def test_qkv_rotary_tile_plans_agree(pkg, lib, grids):
    """The fused qkv+rotary GEMM writes bit-identical head-major Q/K/V^T (including the zeroed
    padding rows [N, Np)) with 288x256, 256x256, 256x128, 128x128 and 64x192 tiles (the last three
    with the three-stage operand ring and one head per wave; 64x192 tiles straddle the q | k
    boundary at D = 1024 and are the default for one 784-token image and the mixed small grid)
    and the row split (config 3's 8192 tokens: 252 tiles of 288x256, then 216 of 256x128); with
    the tail split within rel-L2 2e-3."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    N, D, H = m.n_tokens, 1024, 16
    g = torch.Generator(device="cpu").manual_seed(3)
    x = torch.randn((N, D), generator=g).to(DEV).to(torch.bfloat16)
    w = pack(lib, cp, (torch.randn((D, 3 * D), generator=g) * 0.03).numpy())
    bias = (torch.randn(3 * D, generator=g) * 0.1).to(torch.bfloat16).float().to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, 32, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, 64, 10000.0, cs.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    Np = -(-N // 64) * 64
    outs = {}
    for plan in ["256x256:nosplit", "288x256:nosplit", "256x128:nosplit", "rowsplit:nosplit", "128x128:nosplit",
                 "64x192:nosplit", "64x128:nosplit", "256x256:split", "288x256:split", "256x128:split", "128x128:split",
                 "64x128:split", None]:
        set_plan(lib, cp, plan)
        q = torch.full((H, Np, 64), 7.0, dtype=torch.bfloat16, device=DEV)      # padding must be overwritten
        k, vt = q.clone(), q.clone()
        cp.check(lib.qvl_dense_qkv_rotary(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(), bias.data_ptr(),
                                          cs.data_ptr(), q.data_ptr(), k.data_ptr(), vt.data_ptr(), N, D, H,
                                          ws.data_ptr(), nb.value))
        outs[plan] = [to_np(t) for t in (q, k, vt)]
    set_plan(lib, cp, None)
    base = outs["256x256:nosplit"]
    for plan, got in outs.items():
        for a, b in zip(got, base):
            if plan and plan.endswith(":nosplit"):
                np.testing.assert_array_equal(a, b, err_msg=plan)
            else:
                assert rel_l2(a, b) <= 2e-3, plan
        q, k, vt = got
        assert not q[:, N:].any() and not k[:, N:].any(), plan


def vt_positions(n):
    """vt_pos of key index n: the middle two 4-key quads of each 16-key group swap."""
    n = np.asarray(n)
    quad = (n >> 2) & 3
    return (n & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (n & 3)


@pytest.mark.parametrize("fold", [False, True])
@pytest.mark.parametrize("grids", [[(1, 84, 84)], [(1, 50, 110)], [(1, 28, 26)], [(1, 16, 16), (2, 10, 14), (1, 6, 8)]])
def test_qkv_rotary72_row_split(pkg, lib, grids, fold):
    """The head_dim-72 qkv + rotary GEMM's row split (whole rounds of 256 x 288 tiles, the remaining
    rows as 128 x 288 tiles in a second launch: the cost rule's choice at config 4's 7056 tokens
    and at 5500, forced by plan 2 elsewhere, where the 128-row launch may run alone; or as 64 x 288
    tiles: the rule's choice at 728 tokens, forced by plan 3 elsewhere) against one launch of
    256 x 288 tiles (plan 1): Q, K and V^T bit-identical (the k order is the same), every
    element written (the buffers start as NaN), padding rows and dims 72..87 zero; plain and with
    norm1 folded from row partials (the tower's path)."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    H, hd = 16, 72
    N, D = m.n_tokens, H * hd
    Np = -(-N // 64) * 64
    rng = np.random.default_rng(N + 720)
    x_h = vt.bf16_round((rng.standard_normal((N, D)) + 0.3).astype(np.float32))
    w_h = (rng.standard_normal((D, 3 * D)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(3 * D) * 0.1).astype(np.float32))
    x, w, bias = bf(x_h), pack(lib, cp, w_h), torch.from_numpy(b_h).to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    tab = torch.empty((m.n_positions, hd // 4), dtype=torch.int32, device=DEV)
    cp.check(lib.qvl_rotary_pos_table(stream(), hd, 10000.0, m.n_positions, tab.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    if fold:
        g = vt.bf16_round((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
        b = vt.bf16_round((0.1 * rng.standard_normal(D)).astype(np.float32))
        wf = torch.empty_like(w)
        cd = torch.empty((w.shape[0], 2), dtype=torch.float32, device=DEV)
        cp.check(lib.qvl_fold_ln_weight(stream(), cp.QVL_DTYPE_BF16, w.data_ptr(), D, w.shape[0],
                                        torch.from_numpy(g).to(DEV).data_ptr(), torch.from_numpy(b).to(DEV).data_ptr(),
                                        wf.data_ptr(), cd.data_ptr()))
        xg = x_h.astype(np.float64).reshape(N, D // 128, 128)
        sg = xg.sum(-1)
        parts = torch.from_numpy(np.stack([sg, ((xg - sg[..., None] / 128) ** 2).sum(-1)], -1).astype(np.float32)).to(DEV)
    outs = {}
    for tile in (1, 0, 2, 3):
        q = torch.full((H, Np, 88), float("nan"), dtype=torch.bfloat16, device=DEV)
        k = q.clone()
        vtm = torch.full((H, hd, Np), float("nan"), dtype=torch.bfloat16, device=DEV)
        try:
            cp.check(lib.qvl_set_gemm_plan(tile, -1, 0))
            if fold:
                cp.check(lib.qvl_dense_qkv_rotary_ln_parts(
                    stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, wf.data_ptr(), cd.data_ptr(), parts.data_ptr(),
                    D // 128, 1e-6, bias.data_ptr(), None, pos.data_ptr(), tab.data_ptr(), m.n_positions, q.data_ptr(),
                    k.data_ptr(), vtm.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            else:
                cp.check(lib.qvl_dense_qkv_rotary_pos(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(),
                                                      bias.data_ptr(), pos.data_ptr(), tab.data_ptr(), m.n_positions,
                                                      q.data_ptr(), k.data_ptr(), vtm.data_ptr(), N, D, H,
                                                      ws.data_ptr(), nb.value))
        finally:
            cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
        torch.cuda.synchronize()
        outs[tile] = (to_np(q), to_np(k), to_np(vtm))
    for tile in (0, 2, 3):
        for name, a, b_ in zip("qkv", outs[tile], outs[1]):
            assert np.isfinite(a).all(), (tile, name)
            np.testing.assert_array_equal(a, b_, err_msg=f"plan {tile} {name}")
    q, k, vtm = outs[2]
    assert not q[:, N:].any() and not k[:, N:].any() and not q[:, :, hd:].any() and not k[:, :, hd:].any()
    pad = np.arange(N, Np)
    assert not vtm[:, :, pad[vt_positions(pad) >= N]].any()   # positions holding no token


@pytest.mark.parametrize("fold", [False, True])
@pytest.mark.parametrize("grids", [[(1, 84, 84)], [(1, 16, 16), (2, 10, 14), (1, 6, 8)]])
def test_qkv_rotary72_split_tail(pkg, lib, grids, fold):
    """The head_dim-72 qkv + rotary GEMM with its last partial round of 256 x 288 tiles split along K
    (fp32 partials + gemm_splitk_reduce_rope72_kernel; the cost model's choice at config 4's 336
    tiles) against the same entry without the split: Q, K and V^T within rel-L2 2e-3 (fp32 sums in
    another order), every element written (the buffers start as NaN), padding rows and dims 72..87
    zero; plain (qvl_dense_qkv_rotary) and with norm1 folded from row partials
    (qvl_dense_qkv_rotary_ln_parts, the tower's path)."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    H, hd = 16, 72
    N, D = m.n_tokens, H * hd
    Np = -(-N // 64) * 64
    rng = np.random.default_rng(N + 72)
    x_h = vt.bf16_round((rng.standard_normal((N, D)) + 0.3).astype(np.float32))
    w_h = (rng.standard_normal((D, 3 * D)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(3 * D) * 0.1).astype(np.float32))
    x, w, bias = bf(x_h), pack(lib, cp, w_h), torch.from_numpy(b_h).to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, hd // 2, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    if fold:
        g = vt.bf16_round((1 + 0.2 * rng.standard_normal(D)).astype(np.float32))
        b = vt.bf16_round((0.1 * rng.standard_normal(D)).astype(np.float32))
        wf = torch.empty_like(w)
        cd = torch.empty((w.shape[0], 2), dtype=torch.float32, device=DEV)
        cp.check(lib.qvl_fold_ln_weight(stream(), cp.QVL_DTYPE_BF16, w.data_ptr(), D, w.shape[0],
                                        torch.from_numpy(g).to(DEV).data_ptr(), torch.from_numpy(b).to(DEV).data_ptr(),
                                        wf.data_ptr(), cd.data_ptr()))
        xg = x_h.astype(np.float64).reshape(N, D // 128, 128)
        sg = xg.sum(-1)
        parts = torch.from_numpy(np.stack([sg, ((xg - sg[..., None] / 128) ** 2).sum(-1)], -1).astype(np.float32)).to(DEV)
    outs = []
    for split in (-1, 1):
        q = torch.full((H, Np, 88), float("nan"), dtype=torch.bfloat16, device=DEV)
        k = q.clone()
        vtm = torch.full((H, hd, Np), float("nan"), dtype=torch.bfloat16, device=DEV)
        try:
            cp.check(lib.qvl_set_gemm_plan(0, split, 0))
            if fold:
                cp.check(lib.qvl_dense_qkv_rotary_ln_parts(
                    stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, wf.data_ptr(), cd.data_ptr(), parts.data_ptr(),
                    D // 128, 1e-6, bias.data_ptr(), cs.data_ptr(), None, None, 0, q.data_ptr(), k.data_ptr(),
                    vtm.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            else:
                cp.check(lib.qvl_dense_qkv_rotary(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(),
                                                  bias.data_ptr(), cs.data_ptr(), q.data_ptr(), k.data_ptr(),
                                                  vtm.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
        finally:
            cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
        torch.cuda.synchronize()
        outs.append((to_np(q), to_np(k), to_np(vtm)))
    for name, a, b_ in zip("qkv", outs[0], outs[1]):
        assert np.isfinite(a).all() and np.isfinite(b_).all(), name
        assert rel_l2(b_, a) <= 2e-3, (name, rel_l2(b_, a))
    q, k, vtm = outs[1]
    assert not q[:, N:].any() and not k[:, N:].any() and not q[:, :, hd:].any() and not k[:, :, hd:].any()
    cols = np.arange(Np)
    quad = (cols >> 2) & 3
    vpos = (cols & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (cols & 3)
    assert not vtm[:, :, vpos[N:]].any()


@pytest.mark.parametrize("hd,grids", [(64, [(1, 48, 48)]), (64, [(1, 16, 16), (2, 10, 14), (1, 6, 8)]),
                                      (72, [(1, 84, 84)]), (72, [(1, 16, 16), (2, 10, 14), (1, 6, 8)])])
def test_qkv_rotary_matches_oracle_rotary(pkg, lib, hd, grids):
    """The fused qkv Dense + rotary epilogue (qvl_dense_qkv_rotary, the entry the tower runs)
    against the oracle's bf16 apply_rotary (model.py:579-582: each product and the sum rounded to
    bf16) applied to the GPU's own qkv Dense output and cos/sin table: bit-exact once the layout is
    undone (Q = bf16(q_rot * head_dim^-0.5 * log2 e) as [H][Np][hdp], K = k_rot, V^T[h][d][vt_pos(n)]
    = v[n][h][d]), padding rows zero; head_dim 64 (hdp 64) and head_dim 72 (the 8B tower: hdp 88,
    dims 72..87 zero). The Dense output itself is within one bf16 ulp of the oracle's Dense on the
    same operands for every element (equal for >= 99 %)."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    H = 16
    N, D = m.n_tokens, H * hd
    hdp, half = (64 if hd == 64 else 88), hd // 2
    Np = -(-N // 64) * 64
    rng = np.random.default_rng(N)
    x_h = vt.bf16_round(rng.standard_normal((N, D)).astype(np.float32))
    w_h = (rng.standard_normal((D, 3 * D)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(3 * D) * 0.1).astype(np.float32))
    x = bf(x_h)
    w = pack(lib, cp, w_h)
    bias = torch.from_numpy(b_h).to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, half, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    qkv = torch.empty((N, 3 * D), dtype=torch.bfloat16, device=DEV)
    q = torch.full((H, Np, hdp), 3.0, dtype=torch.bfloat16, device=DEV)   # every element must be written
    k = q.clone()
    vtm = torch.full((H, hd, Np), 3.0, dtype=torch.bfloat16, device=DEV)
    try:
        cp.check(lib.qvl_set_gemm_plan(0, -1, 0))          # no tail split: one K order for both entries
        cp.check(lib.qvl_dense(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS, x.data_ptr(), D, w.data_ptr(),
                               bias.data_ptr(), None, 0, qkv.data_ptr(), 3 * D, N, 3 * D, D))
        cp.check(lib.qvl_dense_qkv_rotary(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(), bias.data_ptr(),
                                          cs.data_ptr(), q.data_ptr(), k.data_ptr(), vtm.data_ptr(), N, D, H,
                                          ws.data_ptr(), nb.value))
    finally:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
    torch.cuda.synchronize()
    qkv_h = to_np(qkv)
    # the Dense against the oracle's (fp32 accumulation in another order: bf16(x.W) may differ by
    # one ulp of the product, which the bias add carries over, plus one ulp of the output)
    ref_qkv = vt.dense(x_h, w_h, b_h, vt._P("bf16"))
    prod = vt.bf16_round(x_h @ vt.bf16_round(w_h))
    ulp = lambda a: np.exp2(np.floor(np.log2(np.maximum(np.abs(a), 1e-30))) - 7)
    assert np.all(np.abs(qkv_h - ref_qkv) <= ulp(prod) + ulp(ref_qkv) + 1e-30)
    assert np.mean(qkv_h == ref_qkv) >= 0.99
    # rotary, oracle arithmetic on the GPU's qkv and table
    c_h = cs.cpu().numpy()
    cos = np.concatenate([c_h[..., 0], c_h[..., 0]], axis=1)
    sin = np.concatenate([c_h[..., 1], c_h[..., 1]], axis=1)
    P = vt._P("bf16")
    qr = vt.apply_rotary(qkv_h[:, :D].reshape(N, H, hd), cos, sin, P)
    kr = vt.apply_rotary(qkv_h[:, D:2 * D].reshape(N, H, hd), cos, sin, P)
    vv = qkv_h[:, 2 * D:].reshape(N, H, hd)
    qscale = np.float32(np.float32(1.0) / np.sqrt(np.float32(hd))) * np.float32(1.4426950408889634)
    want_q = vt.bf16_round(qr * qscale).transpose(1, 0, 2)
    got_q, got_k, got_vt = to_np(q), to_np(k), to_np(vtm)
    np.testing.assert_array_equal(got_q[:, :N, :hd], want_q)
    np.testing.assert_array_equal(got_k[:, :N, :hd], kr.transpose(1, 0, 2))
    np.testing.assert_array_equal(got_vt[:, :, vt_positions(np.arange(N))], vv.transpose(1, 2, 0))
    assert not got_q[:, N:].any() and not got_k[:, N:].any()
    assert not got_q[:, :, hd:].any() and not got_k[:, :, hd:].any()
    assert not got_vt[:, :, vt_positions(np.arange(N, Np))].any()
    # and equal to the oracle's rotary on its own Dense wherever the Dense values agree
    qr_ref = vt.apply_rotary(ref_qkv[:, :D].reshape(N, H, hd), cos, sin, P).transpose(1, 0, 2)
    same = (qkv_h[:, :D] == ref_qkv[:, :D]).reshape(N, H, hd).transpose(1, 0, 2)
    same &= same[..., list(range(half, hd)) + list(range(half))]    # the rotary pair as well
    np.testing.assert_array_equal(got_q[:, :N, :hd][same], vt.bf16_round(qr_ref * qscale)[same])


@pytest.mark.parametrize("hd,grids,plan", [(64, [(1, 48, 48)] * 8, None), (64, [(1, 16, 16), (2, 10, 14), (1, 6, 8)], None),
                                           (64, [(1, 48, 48)] * 3, "288x256:split"), (72, [(1, 84, 84)], None),
                                           (72, [(1, 16, 16), (2, 10, 14)], None)])
def test_qkv_rotary_position_table_bit_identical(pkg, lib, hd, grids, plan):
    """qvl_dense_qkv_rotary_pos (cos, sin looked up per rotary position from an LDS table, the
    tower's path) writes Q, K, V^T bit-identical to qvl_dense_qkv_rotary (per-token table), with the
    tail split's reduce kernel reading the position table from memory; and qvl_rotary_pos_table's
    entries equal the per-token table's at every token's (h, w) ids."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    H = 16
    N, D = m.n_tokens, H * hd
    Np, hdp, half, q4 = -(-N // 64) * 64, (64 if hd == 64 else 88), hd // 2, hd // 4
    g = torch.Generator(device="cpu").manual_seed(N + hd)
    x = torch.randn((N, D), generator=g).to(DEV).to(torch.bfloat16)
    w = pack(lib, cp, (torch.randn((D, 3 * D), generator=g) * 0.03).numpy())
    bias = (torch.randn(3 * D, generator=g) * 0.1).to(torch.bfloat16).float().to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, half, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    P = m.n_positions
    tab = torch.empty((P, q4), dtype=torch.int32, device=DEV)
    cp.check(lib.qvl_rotary_pos_table(stream(), hd, 10000.0, P, tab.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    outs = []
    try:
        set_plan(lib, cp, plan)
        for use_tab in (False, True):
            q = torch.full((H, Np, hdp), 5.0, dtype=torch.bfloat16, device=DEV)
            k = q.clone()
            vt = torch.full((H, hd, Np), 5.0, dtype=torch.bfloat16, device=DEV)
            if use_tab:
                cp.check(lib.qvl_dense_qkv_rotary_pos(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(),
                                                      bias.data_ptr(), pos.data_ptr(), tab.data_ptr(), P, q.data_ptr(),
                                                      k.data_ptr(), vt.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            else:
                cp.check(lib.qvl_dense_qkv_rotary(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), D, w.data_ptr(),
                                                  bias.data_ptr(), cs.data_ptr(), q.data_ptr(), k.data_ptr(),
                                                  vt.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            torch.cuda.synchronize()
            outs.append([t.cpu() for t in (q, k, vt)])
    finally:
        set_plan(lib, cp, None)
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    # the table's entries are the per-token table's values at the token's ids
    t = tab.cpu().numpy().view(np.uint32)
    c, s_ = (t & 0xFFFF).astype(np.uint32) << 16, t & 0xFFFF0000
    cos_t, sin_t = c.view(np.float32), s_.astype(np.uint32).view(np.float32)
    c_h = cs.cpu().numpy()
    ph, pw = m.pos_hw[:, 0], m.pos_hw[:, 1]
    np.testing.assert_array_equal(c_h[:, :q4, 0], cos_t[ph]); np.testing.assert_array_equal(c_h[:, :q4, 1], sin_t[ph])
    np.testing.assert_array_equal(c_h[:, q4:, 0], cos_t[pw]); np.testing.assert_array_equal(c_h[:, q4:, 1], sin_t[pw])


def test_qkv_rotary_position_table_limits(pkg, lib):
    """Tables past the epilogue's LDS room are refused before any launch."""
    cp = pkg.capi
    buf = torch.zeros(1 << 16, dtype=torch.bfloat16, device=DEV)
    p = buf.data_ptr()
    rc = lib.qvl_dense_qkv_rotary_pos(stream(), cp.QVL_DTYPE_BF16, p, 1024, p, p, p, p, 257, p, p, p, 64, 1024, 16,
                                      None, 0)
    assert rc == -2 and "positions" in lib.qvl_last_error().decode()
    assert lib.qvl_dense_qkv_rotary_pos(stream(), cp.QVL_DTYPE_BF16, p, 1024, p, p, None, p, 8, p, p, p, 64, 1024, 16,
                                        None, 0) == -1
