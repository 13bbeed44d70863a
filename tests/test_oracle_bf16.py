"""Pins the oracle's bf16 mode (where it rounds) against torch-CPU bf16 computations written op by op
the way the reference writes them in eager JAX: torch's bf16 elementwise ops compute in fp32 and
round each result to bf16, as XLA does for each eager jnp op. Each check also plants the likely
mistake (one rounding instead of several) and shows the comparison would catch it."""
import numpy as np
import pytest

from oracle import indices as ix
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")

P = vt._P("bf16")


def tb(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16)


def rotate_half_t(t):
    x1, x2 = torch.chunk(t, 2, dim=-1)
    return torch.cat((-x2, x1), dim=-1)


@pytest.mark.parametrize("hd", [64, 72])
def test_apply_rotary_rounds_like_eager_bf16(hd):
    """model.py:579-582, q * cos + rotate_half(q) * sin in bf16: three roundings per element."""
    rng = np.random.default_rng(hd)
    n, h = 300, 4
    q = vt.bf16_round(rng.standard_normal((n, h, hd)).astype(np.float32))
    ang = rng.uniform(0, 40, (n, hd // 2)).astype(np.float32)
    ang = np.concatenate([ang, ang], axis=1)
    cos, sin = vt.bf16_round(np.cos(ang)), vt.bf16_round(np.sin(ang))
    tq, tc, ts = tb(q), tb(cos)[:, None, :], tb(sin)[:, None, :]
    want = (tq * tc + rotate_half_t(tq) * ts).float().numpy()
    got = vt.apply_rotary(q, cos, sin, P)
    np.testing.assert_array_equal(got, want)
    # planted mistake: one rounding of the fp32 expression differs from the reference's arithmetic
    once = vt.bf16_round(q * cos[:, None] + vt.rotate_half(q) * sin[:, None])
    assert np.mean(once != want) > 0.01


@pytest.mark.parametrize("grids", [[(1, 28, 28)], [(3, 10, 6), (1, 16, 20)]])
def test_pos_embed_rounds_like_eager_bf16(grids):
    """model.py:749-752: Embed(idx) * weight (bf16) per tap, then p0 + p1 + p2 + p3 left to right in
    bf16, on the reference's taps (incl. the repeat quirk for t > 1)."""
    spec = vt.VisionSpec()
    table = (np.random.default_rng(1).standard_normal((2304, 1024)) * 0.02).astype(np.float32)
    idx, wts = ix.pos_embed_taps_ref(np.array(grids), 2304, 2)
    t, w = tb(table), tb(wts)
    terms = [t[torch.from_numpy(np.asarray(idx[j], np.int64))] * w[j][:, None] for j in range(4)]
    want = (terms[0] + terms[1] + terms[2] + terms[3]).float().numpy()
    got = vt.pos_embed(table, grids, spec, P)
    np.testing.assert_array_equal(got, want)
    # planted mistake: the 4-tap sum accumulated in fp32 with one rounding
    tab, ww = vt.bf16_round(table), vt.bf16_round(wts)
    once = vt.bf16_round(sum(tab[idx[j]] * ww[j][:, None] for j in range(4)))
    assert np.mean(once != want) > 0.01


def test_dense_rounds_like_bf16_dense():
    """flax Dense in bf16 (model.py:570 etc.): bf16(bf16(x . W) + b), the product accumulated in fp32
    (torch's bf16 CPU matmul does the same; accumulation order differs, so one ulp of the product
    at most). Planted mistake: the bias added before the product is rounded."""
    rng = np.random.default_rng(2)
    x = vt.bf16_round(rng.standard_normal((256, 512)).astype(np.float32))
    k = vt.bf16_round((rng.standard_normal((512, 384)) * 0.05).astype(np.float32))
    b = vt.bf16_round((rng.standard_normal(384) * 0.3).astype(np.float32))
    want = ((tb(x) @ tb(k)) + tb(b)).float().numpy()
    got = vt.dense(x, k, b, P)
    prod = vt.bf16_round(x @ k)
    ulp = lambda a: np.exp2(np.floor(np.log2(np.maximum(np.abs(a), 1e-30))) - 7)
    assert np.all(np.abs(got - want) <= ulp(prod) + ulp(want) + 1e-30)
    assert np.mean(got == want) >= 0.99
    once = vt.bf16_round(x @ k + b)
    assert np.mean(once == want) < 0.99


def test_residual_and_merger_reshape_in_bf16():
    """x + attn(...) in bf16 (model.py:628-629) rounds once per add; the 2x2 merge is a reshape."""
    rng = np.random.default_rng(3)
    x = vt.bf16_round(rng.standard_normal((64, 32)).astype(np.float32))
    a = vt.bf16_round(rng.standard_normal((64, 32)).astype(np.float32) * 1e-2)
    np.testing.assert_array_equal(P.r(x + a), (tb(x) + tb(a)).float().numpy())
    np.testing.assert_array_equal(x.reshape(-1, 4 * 32), tb(x).reshape(-1, 128).float().numpy())
