"""LayerNorm folded into the Dense after it (qvl_row_stats, qvl_fold_ln_weight, qvl_dense_ln_ws,
qvl_dense_qkv_rotary_ln), through the C ABI, against fp64 / torch fp32 references of the
reference's LayerNorm + Dense (model.py:375-388 feeding 556 / 570-582 / 611 / 651-655).

The fold computes LN(x) . W as rstd * (x . W') - rstd * mean * c + d with W' = bf16(gamma W): the
reference's rounding of the LayerNorm output to bf16 is replaced by the rounding of W'. The bar:
within rel-L2 6e-3 of the reference's bf16 arithmetic (LN output rounded, then the bf16 Dense), and
at least as close to the exact fp64 result as that bf16 arithmetic is (x1.25 + 5e-4)."""
import ctypes as C

import numpy as np
import pytest

from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"
EPS = 1e-6


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def stream():
    return torch.cuda.current_stream().cuda_stream


def to_np(t):
    return t.float().cpu().numpy()


def pack(lib, cp, kernel):
    kin, nout = kernel.shape
    src = torch.from_numpy(np.ascontiguousarray(kernel, np.float32)).to(DEV)
    out = torch.empty((-(-nout // 64) * 64, -(-kin // 64) * 64), dtype=torch.bfloat16, device=DEV)
    cp.check(lib.qvl_pack_dense_weight(stream(), cp.QVL_DTYPE_BF16, src.data_ptr(), kin, nout, out.data_ptr()))
    return out


def rows(rng, m, k):
    """bf16 rows with per-row offsets and scales (some rows far off zero)."""
    off = rng.standard_normal((m, 1)) * 2 + np.where(rng.random((m, 1)) < 0.1, 40.0, 0.0)
    return vt.bf16_round((rng.standard_normal((m, k)) * rng.uniform(0.3, 3.0, (m, 1)) + off).astype(np.float32))


def ln_params(rng, k):
    return (vt.bf16_round((1 + 0.2 * rng.standard_normal(k)).astype(np.float32)),
            vt.bf16_round((0.1 * rng.standard_normal(k)).astype(np.float32)))


def ln64(x, g, b):
    x = x.astype(np.float64)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + EPS) * g + b


def gelu64(y):
    return 0.5 * y * (1 + np.tanh(np.sqrt(2 / np.pi) * (y + 0.044715 * y ** 3)))


def fold(lib, cp, w, g, b):
    n_pad, k = w.shape
    out = torch.empty_like(w)
    cd = torch.empty((n_pad, 2), dtype=torch.float32, device=DEV)
    gt, bt = torch.from_numpy(g).to(DEV), torch.from_numpy(b).to(DEV)
    cp.check(lib.qvl_fold_ln_weight(stream(), cp.QVL_DTYPE_BF16, w.data_ptr(), k, n_pad, gt.data_ptr(), bt.data_ptr(),
                                    out.data_ptr(), cd.data_ptr()))
    return out, cd


def stats(lib, cp, x, cols):
    m = x.shape[0]
    st = torch.empty((m, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_row_stats(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), x.shape[1], m, cols, EPS, st.data_ptr()))
    return st


def host_parts(x):
    """Per-128-column (sum, sum of squared deviations from the group mean) of bf16-valued rows, fp64."""
    m, k = x.shape
    g = np.asarray(x, np.float64).reshape(m, k // 128, 128)
    s = g.sum(-1)
    return np.stack([s, ((g - s[..., None] / 128) ** 2).sum(-1)], -1).astype(np.float32)


def combine_parts(parts):
    """(mean, var) of each row from its partials, fp64 (Chan et al.'s pairwise update)."""
    p = np.asarray(parts, np.float64)
    n = 128 * p.shape[1]
    mean = p[..., 0].sum(-1) / n
    m2 = (p[..., 1] + (p[..., 0] - 128 * mean[:, None]) ** 2 / 128).sum(-1)
    return mean, m2 / n


@pytest.mark.parametrize("cols", [1024, 1152, 4096])
def test_row_stats_vs_fp64(pkg, lib, cols):
    """(mean, rstd) per row: within 1e-6 (mean, relative to |mean| + std) and 2e-6 (rstd, relative)
    of a two-pass fp64 computation, rows with offsets up to 40 standard deviations included."""
    cp = pkg.capi
    rng = np.random.default_rng(cols)
    x = rows(rng, 517, cols)
    st = to_np(stats(lib, cp, torch.from_numpy(x).to(DEV).to(torch.bfloat16), cols))
    x64 = x.astype(np.float64)
    mu = x64.mean(-1)
    sd = np.sqrt(((x64 - mu[:, None]) ** 2).mean(-1))
    assert np.all(np.abs(st[:, 0] - mu) <= 1e-6 * (np.abs(mu) + sd))
    assert np.all(np.abs(st[:, 1] * np.sqrt(sd ** 2 + EPS) - 1) <= 2e-6)


def test_fold_ln_weight_exact(pkg, lib):
    """W' = bf16(gamma W) bit for bit (a bf16 x bf16 product is exact in fp32, so one rounding),
    c = sum_k W' and d = sum_k beta W within fp32 summation error of fp64, padding rows zero."""
    cp = pkg.capi
    rng = np.random.default_rng(3)
    k, n = 1152, 4304                                   # the 8B fc1: 4304 outputs packed to 4352
    w = pack(lib, cp, (rng.standard_normal((k, n)) * 0.03).astype(np.float32))
    g, b = ln_params(rng, k)
    wf, cd = fold(lib, cp, w, g, b)
    torch.cuda.synchronize()
    w_h, wf_h, cd_h = to_np(w), to_np(wf), cd.cpu().numpy()
    np.testing.assert_array_equal(wf_h, vt.bf16_round(w_h * g[None, :]))
    c64 = wf_h.astype(np.float64).sum(1)
    d64 = (w_h.astype(np.float64) * b[None, :].astype(np.float64)).sum(1)
    assert np.all(np.abs(cd_h[:, 0] - c64) <= 1e-5 * np.abs(wf_h).sum(1) + 1e-30)
    assert np.all(np.abs(cd_h[:, 1] - d64) <= 1e-5 * np.abs(w_h * b[None, :]).sum(1) + 1e-30)
    assert not wf_h[n:].any() and not cd_h[n:].any()


def ref_bf16_dense(xn, w_h, b_h, epi):
    """The reference's arithmetic after a bf16 LayerNorm output xn: bf16(bf16(xn.W) + b), GELU."""
    r = vt.bf16_round
    y = r(r(xn.astype(np.float32) @ r(w_h)) + b_h)
    return r(gelu64(y.astype(np.float64)).astype(np.float32)) if epi == 1 else y


@pytest.mark.parametrize("epi,m,n,k,plan", [(0, 1000, 3072, 1024, 0), (1, 700, 4096, 1024, 0),
                                            (1, 300, 4096, 4096, 0), (1, 257, 4304, 1152, 0),
                                            (1, 700, 4096, 1024, 1), (0, 1000, 3072, 1024, 1)])
def test_dense_ln_vs_reference(pkg, lib, epi, m, n, k, plan):
    """qvl_row_stats + qvl_fold_ln_weight + qvl_dense_ln_ws (bias / bias+GELU) against the
    reference's LayerNorm (bf16 output) + bf16 Dense, and against exact fp64; plan 1 forces the
    288x256 tiles with a tail split (the split-K reduce applies the fold); at 700 x 4096 x 1024 and
    1000 x 3072 x 1024 the cost model takes 128x128 tiles."""
    cp = pkg.capi
    rng = np.random.default_rng(m + n + k + epi)
    x = rows(rng, m, k)
    g, b = ln_params(rng, k)
    w_h = (rng.standard_normal((k, n)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(n) * 0.1).astype(np.float32))
    w = pack(lib, cp, w_h)
    wf, cd = fold(lib, cp, w, g, b)
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    st = stats(lib, cp, xt, k)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    bias = torch.zeros(-(-n // 64) * 64, dtype=torch.float32, device=DEV)
    bias[:n] = torch.from_numpy(b_h).to(DEV)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    try:
        if plan:
            cp.check(lib.qvl_set_gemm_plan(1, 1, 0))
        cp.check(lib.qvl_dense_ln_ws(stream(), cp.QVL_DTYPE_BF16, epi, xt.data_ptr(), k, wf.data_ptr(), cd.data_ptr(),
                                     st.data_ptr(), bias.data_ptr(), y.data_ptr(), n, m, n, k, ws.data_ptr(), nb.value))
    finally:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
    torch.cuda.synchronize()
    got = to_np(y)
    xn64 = ln64(x, g, b)
    exact = xn64 @ vt.bf16_round(w_h).astype(np.float64) + b_h
    if epi == 1:
        exact = gelu64(exact)
    ref = ref_bf16_dense(vt.bf16_round(xn64.astype(np.float32)), w_h, b_h, epi)
    assert np.isfinite(got).all()
    assert rel_l2(got, ref) <= 6e-3
    assert rel_l2(got, exact) <= 1.25 * rel_l2(ref, exact) + 5e-4


def vt_positions(n):
    n = np.asarray(n)
    quad = (n >> 2) & 3
    return (n & ~15) | (np.choose(quad, [0, 2, 1, 3]) << 2) | (n & 3)


@pytest.mark.parametrize("hd,grids,plan", [(64, [(1, 48, 48)], None), (64, [(1, 16, 16), (2, 10, 14)], (1, 1)),
                                           (64, [(8, 32, 32)], (3, -1)), (64, [(1, 16, 16), (2, 10, 14)], (3, 1)),
                                           (72, [(1, 32, 40)], None)])
def test_qkv_rotary_ln_vs_reference(pkg, lib, hd, grids, plan):
    """qvl_dense_qkv_rotary_ln (norm1 folded into the fused qkv + rotary GEMM, the tower's path)
    against (a) the unfolded entries (qvl_layer_norm + qvl_dense_qkv_rotary) and (b) exact fp64
    LayerNorm + Dense + rotary + pre-scale, layouts undone; the per-position-table form equals the
    per-token form bit for bit. plan (tile, split mode) pins a tile plan for every entry: (1, 1) a
    288x256 tail split, (3, -1) / (3, 1) 256x128 tiles (three-stage ring, the position table in LDS
    beside it; config 3's grid) without / with the split."""
    cp = pkg.capi
    m = pkg.grid_metadata(grids)
    H = 16
    N, D = m.n_tokens, H * hd
    Np, hdp, half, q4 = -(-N // 64) * 64, (64 if hd == 64 else 88), hd // 2, hd // 4
    rng = np.random.default_rng(N + hd)
    x = rows(rng, N, D)
    g, b = ln_params(rng, D)
    w_h = (rng.standard_normal((D, 3 * D)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(3 * D) * 0.1).astype(np.float32))
    w = pack(lib, cp, w_h)
    wf, cd = fold(lib, cp, w, g, b)
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    st = stats(lib, cp, xt, D)
    gt, bt = torch.from_numpy(g).to(DEV), torch.from_numpy(b).to(DEV)
    xn = torch.empty_like(xt)
    cp.check(lib.qvl_layer_norm(stream(), cp.QVL_DTYPE_BF16, xt.data_ptr(), D, gt.data_ptr(), bt.data_ptr(),
                                xn.data_ptr(), D, N, D, EPS))
    bias = torch.from_numpy(b_h).to(DEV)
    pos = torch.from_numpy(m.pos_hw).to(DEV)
    cs = torch.empty((N, half, 2), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_rotary_table(stream(), cp.QVL_DTYPE_BF16, pos.data_ptr(), N, hd, 10000.0, cs.data_ptr()))
    P = m.n_positions
    tab = torch.empty((P, q4), dtype=torch.int32, device=DEV)
    cp.check(lib.qvl_rotary_pos_table(stream(), hd, 10000.0, P, tab.data_ptr()))
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    outs = {}
    try:
        if plan:
            cp.check(lib.qvl_set_gemm_plan(plan[0], plan[1], 0))
        parts = torch.from_numpy(host_parts(x)).to(DEV)
        for mode in ("unfolded", "folded", "folded_tab", "folded_parts"):
            if mode == "folded_tab" and hd != 64:
                continue
            q = torch.full((H, Np, hdp), 5.0, dtype=torch.bfloat16, device=DEV)
            k = q.clone()
            vtm = torch.full((H, hd, Np), 5.0, dtype=torch.bfloat16, device=DEV)
            if mode == "unfolded":
                cp.check(lib.qvl_dense_qkv_rotary(stream(), cp.QVL_DTYPE_BF16, xn.data_ptr(), D, w.data_ptr(),
                                                  bias.data_ptr(), cs.data_ptr(), q.data_ptr(), k.data_ptr(),
                                                  vtm.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            elif mode == "folded_parts":
                tb = hd == 64
                cp.check(lib.qvl_dense_qkv_rotary_ln_parts(
                    stream(), cp.QVL_DTYPE_BF16, xt.data_ptr(), D, wf.data_ptr(), cd.data_ptr(), parts.data_ptr(),
                    D // 128, EPS, bias.data_ptr(), None if tb else cs.data_ptr(), pos.data_ptr() if tb else None,
                    tab.data_ptr() if tb else None, P if tb else 0, q.data_ptr(), k.data_ptr(), vtm.data_ptr(), N, D,
                    H, ws.data_ptr(), nb.value))
            else:
                tb = mode == "folded_tab"
                cp.check(lib.qvl_dense_qkv_rotary_ln(stream(), cp.QVL_DTYPE_BF16, xt.data_ptr(), D, wf.data_ptr(),
                                                     cd.data_ptr(), st.data_ptr(), bias.data_ptr(),
                                                     None if tb else cs.data_ptr(), pos.data_ptr() if tb else None,
                                                     tab.data_ptr() if tb else None, P if tb else 0, q.data_ptr(),
                                                     k.data_ptr(), vtm.data_ptr(), N, D, H, ws.data_ptr(), nb.value))
            torch.cuda.synchronize()
            outs[mode] = (to_np(q), to_np(k), to_np(vtm))
    finally:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
    if "folded_tab" in outs:
        for a, c in zip(outs["folded"], outs["folded_tab"]):
            np.testing.assert_array_equal(a, c)
    # exact fp64: LN, Dense on the bf16 kernel, rotary with the table's (bf16) cos / sin, pre-scale
    qkv = ln64(x, g, b) @ vt.bf16_round(w_h).astype(np.float64) + b_h
    c_h = cs.cpu().numpy().astype(np.float64)
    cos = np.concatenate([c_h[..., 0], c_h[..., 0]], axis=1)[:, None, :]
    sin = np.concatenate([c_h[..., 1], c_h[..., 1]], axis=1)[:, None, :]
    rot = lambda t: t * cos + np.concatenate([-t[..., half:], t[..., :half]], axis=-1) * sin
    qscale = 1.4426950408889634 / np.sqrt(hd)
    exact = (rot(qkv[:, :D].reshape(N, H, hd)).transpose(1, 0, 2) * qscale,
             rot(qkv[:, D:2 * D].reshape(N, H, hd)).transpose(1, 0, 2),
             qkv[:, 2 * D:].reshape(N, H, hd).transpose(1, 2, 0))
    cols = vt_positions(np.arange(N))
    view = lambda o: (o[0][:, :N, :hd], o[1][:, :N, :hd], o[2][:, :, cols])
    for name, got, unf, ex in zip("qkv", view(outs["folded"]), view(outs["unfolded"]), exact):
        assert np.isfinite(got).all(), name
        assert rel_l2(got, unf) <= 6e-3, name
        assert rel_l2(got, ex) <= 1.25 * rel_l2(unf, ex) + 5e-4, name
    # the statistics as 128-column partials: the same fold up to fp32 rounding of mean and rstd
    for name, got, st_form, ex in zip("qkv", view(outs["folded_parts"]), view(outs["folded"]), exact):
        assert rel_l2(got, st_form) <= 2e-3, name
        assert rel_l2(got, ex) <= 1.25 * rel_l2(st_form, ex) + 5e-4, name
    q, k, _ = outs["folded"]
    assert not q[:, N:].any() and not k[:, N:].any() and not q[:, :, hd:].any()


def rowstats_dense(lib, cp, x, w, bias, res, n, k, ws, nb):
    m = x.shape[0]
    y = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    parts = torch.full((m, n // 128, 2), float("nan"), dtype=torch.float32, device=DEV)
    cp.check(lib.qvl_dense_rowstats_ws(stream(), cp.QVL_DTYPE_BF16, x.data_ptr(), k, w.data_ptr(), bias.data_ptr(),
                                       res.data_ptr(), n, y.data_ptr(), n, m, n, k, parts.data_ptr(), ws.data_ptr(), nb))
    return y, parts


@pytest.mark.parametrize("split", [-1, 1])
@pytest.mark.parametrize("m,n,k,plan", [(1000, 1024, 4096, 0), (517, 1152, 1152, 0), (600, 1024, 1024, 1),
                                        (300, 1280, 1024, 3), (784, 1024, 4096, 0), (784, 1024, 1024, 6),
                                        (784, 1024, 1024, 0), (784, 1024, 1024, 8)])
def test_dense_rowstats(pkg, lib, m, n, k, plan, split):
    """qvl_dense_rowstats_ws: the residual Dense's output bit for bit as qvl_dense_ws gives it under the
    same pinned plan (tile 288x256 for plan 1, 256x128 for plan 3, 128x128 for plan 6, 64x128 for
    plan 8, the default for 0; split -1
    forbids the tail split-K, 1 forces it: then the tail tiles' rows come from the split-K reduction,
    which writes their partials too), and per 128-column group of each row the sum and the sum of
    squared deviations of those bf16 outputs within fp32 summation error of fp64 (rows with offsets
    up to 40 standard deviations)."""
    cp = pkg.capi
    rng = np.random.default_rng(m + n + k)
    x = torch.from_numpy(rows(rng, m, k)).to(DEV).to(torch.bfloat16)
    res = torch.from_numpy(rows(rng, m, n)).to(DEV).to(torch.bfloat16)
    w = pack(lib, cp, (rng.standard_normal((k, n)) * 0.03).astype(np.float32))
    bias = torch.from_numpy(vt.bf16_round((rng.standard_normal(n) * 0.1).astype(np.float32))).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    y_ws = torch.empty((m, n), dtype=torch.bfloat16, device=DEV)
    try:
        cp.check(lib.qvl_set_gemm_plan(plan, split, 0))
        y, parts = rowstats_dense(lib, cp, x, w, bias, res, n, k, ws, nb.value)
        cp.check(lib.qvl_dense_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_RESIDUAL, x.data_ptr(), k, w.data_ptr(),
                                  bias.data_ptr(), res.data_ptr(), n, y_ws.data_ptr(), n, m, n, k, ws.data_ptr(),
                                  nb.value))
    finally:
        cp.check(lib.qvl_set_gemm_plan(0, 0, 0))
    torch.cuda.synchronize()
    yh = to_np(y)
    np.testing.assert_array_equal(yh, to_np(y_ws))
    got = parts.cpu().numpy()
    want = host_parts(yh).astype(np.float64)
    g = np.abs(yh.astype(np.float64)).reshape(m, n // 128, 128)
    assert np.isfinite(got).all()
    assert np.all(np.abs(got[..., 0] - want[..., 0]) <= 1e-6 * g.sum(-1) + 1e-30)
    assert np.all(np.abs(got[..., 1] - want[..., 1]) <= 1e-5 * want[..., 1] + 1e-11 * g.sum(-1) ** 2)
    mean, var = combine_parts(got)
    y64 = yh.astype(np.float64)
    mu = y64.mean(-1)
    v64 = ((y64 - mu[:, None]) ** 2).mean(-1)
    assert np.all(np.abs(mean - mu) <= 1e-6 * (np.abs(mu) + np.sqrt(v64)))
    assert np.all(np.abs(var / v64 - 1) <= 1e-5)


@pytest.mark.parametrize("shape", ["fc1", "merger"])
def test_rowstats_feed_folded_dense(pkg, lib, shape):
    """The tower's chain without a LayerNorm launch: a residual Dense writes x and its partials,
    qvl_dense_ln_parts_ws (bias+GELU) consumes them, as fc1 after proj or a deepstack merger's fc1
    after fc2 (the [N/4, 4D] view: 4 token rows = 32 groups). Against qvl_row_stats +
    qvl_dense_ln_ws on the same x (the same fold, statistics by the other route: within 2e-3),
    against the reference's bf16 LayerNorm + Dense (6e-3) and no further from exact fp64 than it."""
    cp = pkg.capi
    D, m = 1024, 1000
    rng = np.random.default_rng(11 if shape == "fc1" else 12)
    x0 = torch.from_numpy(rows(rng, m, D)).to(DEV).to(torch.bfloat16)
    r0 = torch.from_numpy(rows(rng, m, D)).to(DEV).to(torch.bfloat16)
    wp = pack(lib, cp, (rng.standard_normal((D, D)) * 0.03).astype(np.float32))
    bp = torch.from_numpy(vt.bf16_round((rng.standard_normal(D) * 0.1).astype(np.float32))).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    x, parts = rowstats_dense(lib, cp, x0, wp, bp, r0, D, D, ws, nb.value)
    rows_n, k = (m, D) if shape == "fc1" else (m // 4, 4 * D)
    n = 4096
    g, b = ln_params(rng, k)
    w_h = (rng.standard_normal((k, n)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(n) * 0.1).astype(np.float32))
    wf, cd = fold(lib, cp, pack(lib, cp, w_h), g, b)
    bias = torch.from_numpy(b_h).to(DEV)
    y_parts = torch.empty((rows_n, n), dtype=torch.bfloat16, device=DEV)
    y_stats = torch.empty_like(y_parts)
    cp.check(lib.qvl_dense_ln_parts_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_GELU, x.data_ptr(), k,
                                       wf.data_ptr(), cd.data_ptr(), parts.data_ptr(), k // 128, EPS, bias.data_ptr(),
                                       y_parts.data_ptr(), n, rows_n, n, k, ws.data_ptr(), nb.value))
    st = stats(lib, cp, x.view(rows_n, k), k)
    cp.check(lib.qvl_dense_ln_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_GELU, x.data_ptr(), k, wf.data_ptr(),
                                 cd.data_ptr(), st.data_ptr(), bias.data_ptr(), y_stats.data_ptr(), n, rows_n, n, k,
                                 ws.data_ptr(), nb.value))
    torch.cuda.synchronize()
    got, alt = to_np(y_parts), to_np(y_stats)
    xh = to_np(x).reshape(rows_n, k)
    xn64 = ln64(xh, g, b)
    exact = gelu64(xn64 @ vt.bf16_round(w_h).astype(np.float64) + b_h)
    ref = ref_bf16_dense(vt.bf16_round(xn64.astype(np.float32)), w_h, b_h, 1)
    assert np.isfinite(got).all()
    assert rel_l2(got, alt) <= 2e-3
    assert rel_l2(got, ref) <= 6e-3
    assert rel_l2(got, exact) <= 1.25 * rel_l2(ref, exact) + 5e-4


@pytest.mark.parametrize("ratio", [100, 1000])
def test_folded_dense_badly_conditioned_rows(pkg, lib, ratio):
    """Rows whose mean is `ratio` standard deviations off zero (measured on the bf16 rows: median
    |mean| / std within a factor 2 of `ratio`). The fold computes rstd * (x . W') - rstd * mean * c,
    two terms of size ~|mean| / std that cancel, so its fp32 rounding grows with that ratio; the
    reference subtracts the mean before the Dense. Folded (statistics from qvl_row_stats and from
    128-column partials) and unfolded (qvl_layer_norm + qvl_dense_ws) bias+GELU Dense against the
    reference's bf16 LayerNorm + Dense (6e-3) and no further from exact fp64 than it (x1.25 + 5e-4).
    The measured errors are printed. (A row of identical values has std 0 and rstd = eps^-1/2: the
    fold then amplifies the rounding of x . W' - mean * c by 1000, which is why ln_fold=False
    remains available; the tower's rows are never constant.)"""
    cp = pkg.capi
    m, k, n = 512, 1024, 4096
    rng = np.random.default_rng(ratio)
    sign = np.where(rng.random((m, 1)) < 0.5, -1.0, 1.0)
    # a bf16 row mean mu (binade [2^e, 2^(e+1)), spacing 2^(e-7)) plus whole bf16 steps, so that the
    # deviations survive rounding: N(0, s) steps with s = |mu| / spacing / ratio when that is >= 1
    # (ratio 100); otherwise +-1 steps on c of the k columns, std = spacing * sqrt(c / k)
    e = rng.integers(-1, 3, (m, 1)).astype(np.float64)
    mu = sign * 2.0 ** e * rng.uniform(1.0, 1.9, (m, 1))
    spacing = 2.0 ** (e - 7)
    s = np.abs(mu) / spacing / ratio
    steps = np.rint(rng.standard_normal((m, k)) * s)
    if ratio > 200:
        c = np.clip(np.rint((np.abs(mu) / spacing / ratio) ** 2 * k), 2, k // 4).astype(int)
        steps = np.zeros((m, k))
        for i in range(m):
            cols = rng.choice(k, size=c[i, 0], replace=False)
            steps[i, cols] = rng.choice([-1.0, 1.0], size=c[i, 0])
    x = (vt.bf16_round(mu.astype(np.float32)) + steps * spacing).astype(np.float32)
    assert np.array_equal(vt.bf16_round(x), x)
    x64 = x.astype(np.float64)
    sd = x64.std(-1)
    assert np.all(sd > 0)
    cond = np.median(np.abs(x64.mean(-1)) / sd)
    assert 0.5 * ratio <= cond <= 2 * ratio, cond
    g, b = ln_params(rng, k)
    w_h = (rng.standard_normal((k, n)) * 0.03).astype(np.float32)
    b_h = vt.bf16_round((rng.standard_normal(n) * 0.1).astype(np.float32))
    w = pack(lib, cp, w_h)
    wf, cd = fold(lib, cp, w, g, b)
    xt = torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    st = stats(lib, cp, xt, k)
    parts = torch.from_numpy(host_parts(x)).to(DEV)
    nb = C.c_size_t()
    cp.check(lib.qvl_dense_workspace_size(C.byref(nb)))
    ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
    bias = torch.from_numpy(b_h).to(DEV)
    outs = {name: torch.empty((m, n), dtype=torch.bfloat16, device=DEV) for name in ("stats", "parts", "unfolded")}
    cp.check(lib.qvl_dense_ln_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_GELU, xt.data_ptr(), k, wf.data_ptr(),
                                 cd.data_ptr(), st.data_ptr(), bias.data_ptr(), outs["stats"].data_ptr(), n, m, n, k,
                                 ws.data_ptr(), nb.value))
    cp.check(lib.qvl_dense_ln_parts_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_GELU, xt.data_ptr(), k,
                                       wf.data_ptr(), cd.data_ptr(), parts.data_ptr(), k // 128, EPS, bias.data_ptr(),
                                       outs["parts"].data_ptr(), n, m, n, k, ws.data_ptr(), nb.value))
    gt, bt = torch.from_numpy(g).to(DEV), torch.from_numpy(b).to(DEV)
    xn = torch.empty_like(xt)
    cp.check(lib.qvl_layer_norm(stream(), cp.QVL_DTYPE_BF16, xt.data_ptr(), k, gt.data_ptr(), bt.data_ptr(),
                                xn.data_ptr(), k, m, k, EPS))
    cp.check(lib.qvl_dense_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_GELU, xn.data_ptr(), k, w.data_ptr(),
                              bias.data_ptr(), None, 0, outs["unfolded"].data_ptr(), n, m, n, k, ws.data_ptr(),
                              nb.value))
    torch.cuda.synchronize()
    xn64 = ln64(x, g, b)
    exact = gelu64(xn64 @ vt.bf16_round(w_h).astype(np.float64) + b_h)
    ref = ref_bf16_dense(vt.bf16_round(xn64.astype(np.float32)), w_h, b_h, 1)
    e_ref = rel_l2(ref, exact)
    msg = []
    for name, y in outs.items():
        got = to_np(y)
        assert np.isfinite(got).all(), name
        a, e = rel_l2(got, ref), rel_l2(got, exact)
        msg.append(f"{name}: vs reference arithmetic {a:.2e}, vs fp64 {e:.2e}")
        assert a <= 6e-3, name
        assert e <= 1.25 * e_ref + 5e-4, name
    print(f"\n[|mean|/std ~ {cond:.0f}] reference arithmetic vs fp64 {e_ref:.2e}; " + "; ".join(msg), flush=True)


def test_rowstats_rejects_bad_shapes(pkg, lib):
    """Row statistics need 128-column groups and 8-element row strides; the folded entries need
    groups * 128 == the LayerNorm width and a positive eps (checked on the host, no launch)."""
    cp = pkg.capi
    bad = []
    p = torch.empty(1 << 16, dtype=torch.uint8, device=DEV)
    a = p.data_ptr()
    bad.append(lib.qvl_dense_rowstats_ws(stream(), cp.QVL_DTYPE_BF16, a, 64, a, a, a, 192, a, 192, 8, 192, 64, a, a, 4096))
    bad.append(lib.qvl_dense_rowstats_ws(stream(), cp.QVL_DTYPE_BF16, a, 64, a, a, a, 132, a, 132, 8, 128, 64, a, a, 4096))
    bad.append(lib.qvl_dense_ln_parts_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS, a, 256, a, a, a, 1, EPS, a, a,
                                         128, 8, 128, 256, a, 4096))
    bad.append(lib.qvl_dense_ln_parts_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS, a, 256, a, a, a, 2, 0.0, a, a,
                                         128, 8, 128, 256, a, 4096))
    bad.append(lib.qvl_dense_ln_parts_ws(stream(), cp.QVL_DTYPE_BF16, cp.QVL_EPI_BIAS_RESIDUAL, a, 256, a, a, a, 2, EPS,
                                         a, a, 128, 8, 128, 256, a, 4096))
    assert all(rc != cp.QVL_OK for rc in bad), bad
