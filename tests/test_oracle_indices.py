"""Pins the oracle's integer metadata (CPU): reference reshape chains vs closed forms vs
transformers' independent `vision_utils` helpers."""
import itertools

import numpy as np
import pytest

from oracle import indices as ix

SMALL_GRIDS = [(t, h, w) for t in (1, 2, 3) for h in (2, 4, 6, 8) for w in (2, 4, 6, 8)]


@pytest.mark.parametrize("g", SMALL_GRIDS)
def test_rot_ids_ref_equals_closed(g):
    assert np.array_equal(ix.rot_pos_ids_ref([g]), ix.rot_pos_ids_closed([g]))


@pytest.mark.parametrize("g", SMALL_GRIDS)
def test_pos_embed_rows_ref_equals_closed(g):
    t, h, w = g
    assert np.array_equal(ix.pos_embed_rows_ref(t, h, w), ix.pos_embed_rows_closed(t, h, w))


def test_cu_seqlens_ref_equals_closed():
    rng = np.random.default_rng(0)
    for _ in range(50):
        n = rng.integers(1, 6)
        g = [(int(rng.integers(1, 4)), 2 * int(rng.integers(1, 9)), 2 * int(rng.integers(1, 9))) for _ in range(n)]
        assert np.array_equal(ix.cu_seqlens_ref(g), ix.cu_seqlens_closed(g))
    assert list(ix.cu_seqlens_ref([(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48)])) == [0, 1024, 1984, 2240, 4544]
    assert list(ix.cu_seqlens_ref([(8, 32, 32)])) == [1024 * i for i in range(9)]


def test_merge_rows_are_2x2_blocks():
    """Merged row G gathers tokens 4G..4G+3, which are exactly one 2x2 patch block of one frame."""
    grids = [(1, 4, 6), (2, 8, 4), (1, 2, 2)]
    G = ix.merged_row_closed(grids)
    n = sum(t * h * w for t, h, w in grids)
    assert np.array_equal(G, np.arange(n) // 4)
    f, r, c = ix.token_coords_closed(grids)
    src = ix.merge_source_rows(n)
    for g in range(n // 4):
        rows = src[g]
        assert len(set(f[rows])) == 1
        assert sorted(zip(r[rows] % 2, c[rows] % 2)) == [(0, 0), (0, 1), (1, 0), (1, 1)]
        assert len(set(r[rows] // 2)) == 1 and len(set(c[rows] // 2)) == 1


def test_against_transformers_vision_utils():
    torch = pytest.importorskip("torch")
    vu = pytest.importorskip("transformers.vision_utils")
    grids = [(1, 4, 6), (1, 8, 8), (3, 4, 4), (2, 6, 2), (1, 48, 48), (1, 84, 84), (1, 24, 40)]
    gt = torch.tensor(grids, dtype=torch.int64)
    assert np.array_equal(vu.get_vision_cu_seqlens(gt).numpy(), ix.cu_seqlens_ref(grids))
    assert np.array_equal(vu.get_vision_position_ids(gt, 2).numpy(), ix.rot_pos_ids_ref(grids))
    # pos-embed taps: transformers tiles frames; the reference repeats rows in place (t>1 quirk),
    # so compare on t=1 grids only (taps equal exactly, weights to f32 rounding).
    g1 = [g for g in grids if g[0] == 1]
    idx, wts = vu.get_vision_interpolation_indices_and_weights(
        torch.tensor(g1), num_grid_per_side=48, mode="bilinear", align_corners=True, spatial_merge_size=2)
    ridx, rw = ix.pos_embed_taps_ref(g1, 2304)
    assert np.array_equal(idx.numpy().T, ridx)
    np.testing.assert_allclose(wts.numpy().T, rw, rtol=0, atol=2e-6)


def test_pos_embed_quirk_differs_from_tiling():
    """For t>1 the reference expands frames with repeat-in-place, not tiling: rows E[i] = P[i//t]."""
    t, h, w = 2, 4, 4
    rows = ix.pos_embed_rows_ref(t, h, w)
    tiled = np.tile(ix.pos_embed_rows_ref(1, h, w), t)
    assert not np.array_equal(rows, tiled)
    # first frame of the quirk takes raster rows 0..7 (each twice) in merge-block order
    assert sorted(set(rows[: h * w].tolist())) == list(range(h * w // t))


def test_rotary_half_table():
    """angles[n] = [pos_h * inv_freq, pos_w * inv_freq], inv_freq_j = theta^(-2j/(hd/2))."""
    g = [(1, 6, 8), (2, 4, 4)]
    for hd in (64, 72, 32):
        tab = ix.rotary_half_ref(g, hd)
        pos = ix.rot_pos_ids_closed(g)
        j = np.arange(hd // 4)
        inv = 10000.0 ** (-2.0 * j / (hd // 2))
        exp = np.concatenate([pos[:, :1] * inv, pos[:, 1:] * inv], axis=1)
        np.testing.assert_allclose(tab, exp, rtol=2e-6, atol=0)


@pytest.mark.parametrize("heads", [1, 3, 16])
def test_attention_tiles_cover_every_query_once(heads):
    """Schedule invariants: every query row of every segment in exactly one item per head; a
    (segment, head) group never spans two queues; each queue is longest-segment-first; padding
    items are empty; queue work is balanced within one group's work (the greedy bound)."""
    cu = ix.cu_seqlens_ref([(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48), (1, 2, 2)])
    for bm in (64, 128, 256):
        items = ix.attention_tiles(cu, bm, heads)
        assert len(items) % 8 == 0
        seen = np.zeros((heads, cu[-1]), np.int32)
        queue_of = {}
        load = np.zeros(8, np.int64)
        for k, (s, e, q0, h) in enumerate(items):
            if e <= s:
                assert (s, e, q0, h) == (0, 0, 0, 0)
                continue
            assert s <= q0 < e and 0 <= h < heads
            seen[h, q0:min(q0 + bm, e)] += 1
            assert queue_of.setdefault((s, h), k % 8) == k % 8
            load[k % 8] += e - s
        assert (seen == 1).all()
        for q in range(8):
            lens = [e - s for (s, e, _, _) in items[q::8] if e > s]
            assert all(a >= b for a, b in zip(lens, lens[1:]))
        seg_len = np.diff(cu)
        biggest = max(-(-L // bm) * L for L in seg_len)
        assert load.max() - load.min() <= biggest


# ---------------------------------------------------------------------------------------------
# window attention metadata (model.py:769-799, 828-830)
# ---------------------------------------------------------------------------------------------
WINDOW_GRIDS = [[(1, 8, 12)], [(1, 8, 12), (2, 4, 4)], [(3, 10, 6)], [(1, 2, 2)], [(2, 14, 18), (1, 6, 4)],
                [(1, 16, 16)], [(4, 6, 10)]]


@pytest.mark.parametrize("grids", WINDOW_GRIDS)
@pytest.mark.parametrize("merge,patch,window", [(2, 14, 112), (2, 16, 64), (2, 16, 32), (2, 14, 56)])
def test_window_index_ref_vs_closed_and_transformers(grids, merge, patch, window):
    torch = pytest.importorskip("torch")
    a, ca = ix.window_index_ref(grids, merge, patch, window)
    b, cb = ix.window_index_closed(grids, merge, patch, window)
    assert np.array_equal(a, b) and np.array_equal(ca, cb)
    assert sorted(a.tolist()) == list(range(len(a)))                  # a permutation of merge groups
    try:
        from transformers.vision_utils import get_vision_window_index
    except ImportError:
        pytest.skip("transformers.vision_utils not available")
    hi, hc = get_vision_window_index(torch.tensor(grids), spatial_merge_size=merge, window_size=window,
                                     patch_size=patch)
    assert np.array_equal(a, hi.numpy()) and np.array_equal(ca, np.asarray(hc))


@pytest.mark.parametrize("grids", WINDOW_GRIDS)
def test_cu_full_window_matches_slice_semantics(grids):
    """The reference's q[start:end] over [0, N) with the unclamped merge^2-scaled bounds."""
    g = np.asarray(grids)
    n = int((g[:, 0] * g[:, 1] * g[:, 2]).sum())
    raw = np.concatenate([[0], np.cumsum(g[:, 0] * g[:, 1] * g[:, 2] * 4)])
    cu = ix.cu_full_window_ref(grids, 2)
    tokens = list(range(n))
    for i in range(len(raw) - 1):
        assert tokens[raw[i]:raw[i + 1]] == tokens[cu[i]:cu[i + 1]]
    assert cu[-1] == n


@pytest.mark.parametrize("grids", WINDOW_GRIDS)
@pytest.mark.parametrize("patch,window", [(14, 112), (16, 64)])
def test_window_metadata_host_bit_exact(pkg, grids, patch, window):
    widx, cuw, cuf = pkg.vision.window_metadata(grids, 2, patch, window)
    a, ca = ix.window_index_ref(grids, 2, patch, window)
    assert np.array_equal(widx, a) and np.array_equal(cuw, ca)
    assert np.array_equal(cuf, ix.cu_full_window_ref(grids, 2))
