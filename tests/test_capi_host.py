"""C-ABI host checks (no GPU): every declared symbol is exported, host metadata is bit-exact with
the oracle's restatement of the reference, and the argument checks reject bad input."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from oracle import indices as ix

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"^\s*(?:const\s+)?[a-z_][a-z0-9_]*\s*\**\s*(qvl_[a-z0-9_]+)\s*\(", text, re.M))
    return sorted(names)


def test_header_declares_entries():
    syms = declared_symbols()
    for must in ("qvl_encode_vision", "qvl_vision_attention", "qvl_dense", "qvl_layer_norm", "qvl_vision_metadata"):
        assert must in syms


def test_library_exports_every_declared_symbol(pkg):
    lib = pkg.capi.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    # and the ctypes prototypes cover the header exactly
    assert sorted(pkg.capi.SIGNATURES) == declared_symbols()


GRIDS = [
    [(1, 28, 28)],                                            # config 0
    [(1, 32, 32), (1, 24, 40), (1, 16, 16), (1, 48, 48)],     # config 1
    [(1, 48, 48)] * 8,                                        # config 2
    [(8, 32, 32)],                                            # config 3 (t > 1: the repeat quirk)
    [(1, 84, 84)],                                            # config 4
    [(3, 4, 6), (2, 2, 2), (1, 6, 2)],
]


@pytest.mark.parametrize("grids", GRIDS)
def test_metadata_bit_exact_vs_oracle(pkg, grids):
    m = pkg.grid_metadata(grids, dtype=pkg.capi.QVL_DTYPE_F32)
    assert np.array_equal(m.cu_seqlens, ix.cu_seqlens_ref(grids))
    assert np.array_equal(m.pos_hw, ix.rot_pos_ids_ref(grids))
    idx, w = ix.pos_embed_taps_ref(grids, 2304)
    assert np.array_equal(m.tap_idx, idx)
    assert np.array_equal(m.tap_w.view(np.uint32), w.view(np.uint32))   # bit-exact f32 weights
    # bf16 mode rounds the weights exactly like the oracle's bf16 cast
    from oracle.vision_tower import bf16_round
    mb = pkg.grid_metadata(grids, dtype=pkg.capi.QVL_DTYPE_BF16)
    assert np.array_equal(mb.tap_w.view(np.uint32), bf16_round(w).view(np.uint32))


@pytest.mark.parametrize("grids", GRIDS)
def test_worklist_covers_every_query_once(pkg, grids):
    for heads in (1, 16):
        m = pkg.grid_metadata(grids, num_heads=heads)
        ref = ix.attention_tiles(m.cu_seqlens, 128, heads)
        assert np.array_equal(m.tiles, ref)


def test_inv_freq_matches_oracle(pkg):
    lib = pkg.capi.load()
    for hd in (64, 72, 128):
        out = np.zeros(hd // 4, np.float32)
        pkg.capi.check(lib.qvl_rotary_inv_freq(hd, 10000.0, out.ctypes.data_as(C.POINTER(C.c_float))))
        ref = ix.rotary_inv_freq(hd)
        ulps = np.abs(out.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
        assert ulps.max() <= 1, ulps       # numpy's f32 pow vs a correctly rounded one
        j = np.arange(hd // 4)
        np.testing.assert_allclose(out, 10000.0 ** (-2.0 * j / (hd // 2)), rtol=2e-6)   # f32 exponent


def test_rejects_bad_grids(pkg):
    with pytest.raises(pkg.capi.QVLError, match="not divisible"):
        pkg.grid_metadata([(1, 5, 4)])
    with pytest.raises(pkg.capi.QVLError, match="non-positive"):
        pkg.grid_metadata([(0, 4, 4)])
    lib = pkg.capi.load()
    cu = np.array([0, 8, 4], np.int32)
    n = C.c_int64()
    rc = lib.qvl_attention_worklist(cu.ctypes.data_as(C.POINTER(C.c_int32)), 2, 1, None, 0, C.byref(n))
    assert rc == -1 and b"monotone" in lib.qvl_last_error()
    rc = lib.qvl_attention_worklist(np.array([0, 4], np.int32).ctypes.data_as(C.POINTER(C.c_int32)), 1, 0, None, 0,
                                    C.byref(n))
    assert rc == -1 and b"num_heads" in lib.qvl_last_error()


def test_empty_segments_are_skipped(pkg):
    lib = pkg.capi.load()
    cu = np.array([0, 0, 130, 130, 131], np.int32)
    n = C.c_int64()
    assert lib.qvl_attention_worklist(cu.ctypes.data_as(C.POINTER(C.c_int32)), 4, 1, None, 0, C.byref(n)) == 0
    assert n.value == 16  # 130 -> 2 tiles of 128 in one queue, 1 -> 1 tile in another; 8 queues of 2 slots
    items = np.zeros((n.value, 4), np.int32)
    assert lib.qvl_attention_worklist(cu.ctypes.data_as(C.POINTER(C.c_int32)), 4, 1,
                                      items.ctypes.data_as(C.POINTER(C.c_int32)), n.value, C.byref(n)) == 0
    live = items[items[:, 1] > items[:, 0]]
    assert sorted(map(tuple, live.tolist())) == [(0, 130, 0, 0), (0, 130, 128, 0), (130, 131, 130, 0)]


def test_dense_argument_checks(pkg):
    lib = pkg.capi.load()
    cp = pkg.capi
    fake = 1 << 20   # never dereferenced: validation fails first
    # K not a multiple of 64
    assert lib.qvl_dense(None, cp.QVL_DTYPE_BF16, 0, fake, 100, fake, fake, None, 0, fake, 64, 8, 64, 100) == -1
    # misaligned x
    assert lib.qvl_dense(None, cp.QVL_DTYPE_BF16, 0, fake + 2, 64, fake, fake, None, 0, fake, 64, 8, 64, 64) == -3
    # residual epilogue without residual
    assert lib.qvl_dense(None, cp.QVL_DTYPE_BF16, 2, fake, 64, fake, fake, None, 64, fake, 64, 8, 64, 64) == -1
    # unsupported dtype
    assert lib.qvl_dense(None, 7, 0, fake, 64, fake, fake, None, 0, fake, 64, 8, 64, 64) == -2
    # fp32: rows must be 16-byte aligned (lda % 4)
    assert lib.qvl_dense(None, cp.QVL_DTYPE_F32, 0, fake, 66, fake, fake, None, 0, fake, 64, 8, 64, 64) == -3
    assert lib.qvl_layer_norm(None, cp.QVL_DTYPE_BF16, fake, 100, fake, fake, fake, 100, 4, 100, 1e-6) == -1
    assert lib.qvl_layer_norm(None, cp.QVL_DTYPE_F32, fake + 4, 64, fake, fake, fake, 64, 4, 64, 1e-6) == -3
    # the fp32 tower runs qvl_dense + qvl_vision_attention; the fused qkv+rotary entry is bf16 only
    assert lib.qvl_dense_qkv_rotary(None, cp.QVL_DTYPE_F32, fake, 1024, fake, fake, fake, fake, fake, fake, 64, 1024,
                                    16, None, 0) == -2


def test_workspace_sizes(pkg):
    lib = pkg.capi.load()
    spec = pkg.spec_2b()
    tower = pkg.Qwen3VisionTransformer.__new__(pkg.Qwen3VisionTransformer)
    cfg = pkg.capi.VisionConfig(hidden_size=1024, out_hidden_size=2048, depth=24, num_heads=16,
                                intermediate_size=4096, patch_volume=1536, spatial_merge_size=2,
                                num_position_embeddings=2304, n_deepstack=3, ln_eps=1e-6, rope_theta=1e4,
                                dtype=pkg.capi.QVL_DTYPE_BF16)
    nb = C.c_size_t()
    assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == 0
    assert 200e6 < nb.value < 600e6
    assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18430, C.byref(nb)) == -1   # not a multiple of 4
    bf16_bytes = nb.value
    cfg.dtype = pkg.capi.QVL_DTYPE_F32        # fp32 activations
    assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == 0
    assert 1.5 * bf16_bytes < nb.value < 2.5 * bf16_bytes
    cfg.dtype = 5
    assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == -2
    cfg.dtype = pkg.capi.QVL_DTYPE_BF16
    cfg.spatial_merge_size = 3
    assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == -2
    cfg.spatial_merge_size = 2
    # head_dim 64, 72 and 80 (1280 / 16) are taken, 96 is not; patch volumes that are multiples of 4
    # (patch 14: 1176) are taken (their rows are staged zero-padded to 1216), others are not
    for dt in (pkg.capi.QVL_DTYPE_BF16, pkg.capi.QVL_DTYPE_F32):
        cfg.dtype = dt
        for hidden, heads, rc in ((1280, 16, 0), (1152, 16, 0), (1536, 16, -2)):
            cfg.hidden_size, cfg.num_heads = hidden, heads
            assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == rc, (dt, hidden)
        cfg.hidden_size, cfg.num_heads = 1024, 16
        for pv, rc in ((1176, 0), (1350, -2), (768, 0)):
            cfg.patch_volume = pv
            assert lib.qvl_encode_vision_workspace_size(C.byref(cfg), 18432, C.byref(nb)) == rc, (dt, pv)
        cfg.patch_volume = 1536
    for dt, hd, want in ((pkg.capi.QVL_DTYPE_BF16, 72, 16 * 64 * (88 + 88 + 72) * 2),
                         (pkg.capi.QVL_DTYPE_BF16, 80, 16 * 64 * (88 + 88 + 80) * 2),
                         (pkg.capi.QVL_DTYPE_F32, 72, 16 * 64 * (72 + 72 + 96) * 4),
                         (pkg.capi.QVL_DTYPE_F32, 64, 16 * 64 * (64 + 64 + 64) * 4)):
        assert lib.qvl_vision_attention_workspace_size(dt, 10, 16, hd, C.byref(nb)) == 0
        assert nb.value == want


def test_io_entry_argument_checks(pkg):
    """patchify / positions / scatter reject bad arguments before any launch."""
    lib = pkg.capi.load()
    cp = pkg.capi
    fake = 1 << 20   # never dereferenced: validation fails first
    BF, F32 = cp.QVL_DTYPE_BF16, cp.QVL_DTYPE_F32
    # height not divisible by patch, grid not divisible by merge, bad channels / dtype / ld_out
    assert lib.qvl_patchify(None, F32, fake, 1, 40, 64, 3, 16, 2, 2, fake, 1536) == -1
    assert b"divisible" in lib.qvl_last_error()
    assert lib.qvl_patchify(None, F32, fake, 1, 48, 64, 3, 16, 2, 2, fake, 1536) == -1
    assert lib.qvl_patchify(None, F32, fake, 1, 32, 32, 2, 16, 2, 2, fake, 1536) == -1
    assert lib.qvl_patchify(None, 9, fake, 1, 32, 32, 3, 16, 2, 2, fake, 1536) == -2
    assert lib.qvl_patchify(None, BF, fake, 1, 32, 32, 3, 16, 2, 2, fake, 1535) == -1
    assert lib.qvl_patchify(None, BF, fake, 0, 32, 32, 3, 16, 2, 2, fake, 1536) == -1
    assert lib.qvl_patchify(None, BF, None, 1, 32, 32, 3, 16, 2, 2, fake, 1536) == -1
    # positions: empty batch is a no-op; negative sizes / NULL rejected
    assert lib.qvl_vision_positions(None, fake, 0, 10, 5, 4, fake, fake) == 0
    assert lib.qvl_vision_positions(None, fake, 1, -1, 5, 4, fake, fake) == -1
    assert lib.qvl_vision_positions(None, fake, 1, 10, 5, 4, fake, None) == -1
    # scatter: bad mode, dtype, sizes; empty work is a no-op
    assert lib.qvl_scatter_vision_rows(None, 2, BF, fake, 1, 8, 4, BF, fake, 0, 2, fake, fake) == -1
    assert lib.qvl_scatter_vision_rows(None, cp.QVL_SCATTER_SET, 3, fake, 1, 8, 4, BF, fake, 0, 2, fake, fake) == -2
    assert lib.qvl_scatter_vision_rows(None, cp.QVL_SCATTER_ADD, BF, fake, 1, 8, 4, F32, fake, -1, 2, fake, fake) == -1
    assert lib.qvl_scatter_vision_rows(None, cp.QVL_SCATTER_ADD, BF, fake, 1, 8, 4, F32, fake, 0, 0, fake, fake) == 0
    assert lib.qvl_scatter_vision_rows(None, cp.QVL_SCATTER_SET, BF, fake, 1, 8, 4, F32, None, 0, 2, fake, fake) == -1


def test_window_entry_argument_checks(pkg):
    lib = pkg.capi.load()
    cp = pkg.capi
    g = np.array([[1, 8, 12]], np.int32)
    n = C.c_int64()
    gp = g.ctypes.data_as(C.POINTER(C.c_int32))
    # window smaller than one merge group, odd grid, missing count pointer
    assert lib.qvl_window_metadata(gp, 1, 2, 16, 16, None, None, 0, C.byref(n), None) == -1
    bad = np.array([[1, 7, 12]], np.int32)
    assert lib.qvl_window_metadata(bad.ctypes.data_as(C.POINTER(C.c_int32)), 1, 2, 16, 64, None, None, 0,
                                   C.byref(n), None) == -1
    assert lib.qvl_window_metadata(gp, 1, 2, 16, 64, None, None, 0, None, None) == -1
    # capacity too small
    assert lib.qvl_window_metadata(gp, 1, 2, 16, 64, None, None, 0, C.byref(n), None) == 0
    cu = np.zeros(n.value, np.int32)
    assert lib.qvl_window_metadata(gp, 1, 2, 16, 64, None, cu.ctypes.data_as(C.POINTER(C.c_int32)), n.value - 1,
                                   C.byref(n), None) == -1
    fake = 1 << 20
    assert lib.qvl_gather_rows(None, cp.QVL_DTYPE_F32, fake, 8, 5, fake, 8, fake, 8, 4, 8) == -2
    assert lib.qvl_gather_rows(None, cp.QVL_DTYPE_F32, fake, 8, cp.QVL_DTYPE_F32, fake, 8, fake, 6, 4, 8) == -1
    assert lib.qvl_gather_rows(None, cp.QVL_DTYPE_F32, fake, 4, cp.QVL_DTYPE_F32, fake, 8, fake, 8, 4, 8) == -1
    assert lib.qvl_gather_rows(None, cp.QVL_DTYPE_F32, fake, 8, cp.QVL_DTYPE_F32, fake, 8, fake, 0, 4, 8) == 0


def _split_list(pkg, cu, heads, hd, n_cus):
    items, n_whole = pkg.attention_worklist_split(np.asarray(cu, np.int32), heads, hd, n_cus)
    base = pkg.vision._worklist(pkg.capi.load(), np.asarray(cu, np.int32), heads)
    return items, n_whole, base


@pytest.mark.parametrize("cu,heads,hd,n_cus", [([0, 4096, 8192, 18432], 16, 64, 256),   # no split
                                               ([0, 4096, 8192, 18432], 16, 64, 280),   # 64-item tail, 8 parts
                                               ([0] + [2304 * i for i in range(1, 9)], 16, 64, 256),   # config 2
                                               ([0, 1024, 1984, 2240, 4544], 16, 64, 256),   # config 1
                                               ([0] + [1024 * i for i in range(1, 9)], 16, 64, 256),   # config 3
                                               ([0, 7056], 16, 72, 256),                # config 4: 6 parts
                                               ([0, 1024, 2048, 6144], 16, 72, 256),    # 768 items, 768 slots
                                               ([0, 4096, 4100], 16, 72, 58),   # 1-tile items stay whole
                                               ([0, 130, 4226], 2, 80, 22),     # head_dim 80: 3 per CU
                                               ([0, 200], 2, 64, 8)])
def test_attention_worklist_split(pkg, cu, heads, hd, n_cus):
    """The split list keeps the whole items in place, empties those of the last partial round of
    workgroup slots, and appends parts whose key tiles cover each such item's keys exactly once."""
    items, n_whole, base = _split_list(pkg, cu, heads, hd, n_cus)
    assert n_whole == len(base)
    whole, parts = items[:n_whole], items[n_whole:]
    real = lambda a: a[a[:, 1] > a[:, 0]]
    slots = n_cus * (4 if hd == 64 else 3)
    nb = len(real(base))
    tail = nb % slots if nb >= slots else nb
    gone = [k for k in range(n_whole) if base[k, 1] > base[k, 0] and whole[k, 1] == whole[k, 0]]
    kept = np.ones(n_whole, bool)
    kept[gone] = False
    assert (whole[kept] == base[kept]).all() and (whole[~kept] == 0).all()
    assert len(gone) <= tail
    if tail == 0 or 2 * tail > n_cus:      # split only when the last round leaves half the CUs idle
        assert len(parts) == 0 and not gone
    head = parts[:, 3] & 0xFFF
    part_i = (parts[:, 3] >> 12) & 0xFF
    n_parts = parts[:, 3] >> 20
    assert len(parts) <= slots and (n_parts >= 2).all() and (n_parts <= 8).all()
    covered = {}
    for it, h, p, npart in zip(parts, head, part_i, n_parts):
        key = (it[0], it[1], it[2], h)
        covered.setdefault(key, []).append((p, npart))
    assert sorted(covered) == sorted(tuple(base[k]) for k in gone)
    for key, ps in covered.items():
        npart = ps[0][1]
        assert sorted(p for p, _ in ps) == list(range(npart)) and all(n == npart for _, n in ps)
        # the kernel's key-tile ranges t0 = n_kt * p / parts tile [0, n_kt) and none is below 2 tiles
        n_kt = (key[1] - (key[0] & ~63) + 63) // 64
        bounds = [n_kt * p // npart for p in range(npart + 1)]
        assert bounds[0] == 0 and bounds[-1] == n_kt and min(np.diff(bounds)) >= 2
    # every query row of every (segment, head) exactly once: a whole item's 128 rows, or those of a
    # split item through its parts
    count = {}
    for it in list(real(whole)) + list(covered):
        s0, s1, q0, h = (int(v) for v in it[:4])
        for r in range(q0, min(s1, q0 + 128)):
            count[(s0, s1, h & 0xFFF, r)] = count.get((s0, s1, h & 0xFFF, r), 0) + 1
    want = {(s0, s1, h, r) for s0, s1 in zip(cu[:-1], cu[1:]) for h in range(heads) for r in range(s0, s1)}
    assert set(count) == want and set(count.values()) == {1}


def test_attention_worklist_split_checks(pkg):
    lib = pkg.capi.load()
    cu = np.array([0, 256], np.int32)
    n, nw = C.c_int64(), C.c_int64()
    p = cu.ctypes.data_as(C.POINTER(C.c_int32))
    assert lib.qvl_attention_worklist_split(p, 1, 16, 96, 256, None, 0, C.byref(n), C.byref(nw)) == -2
    assert lib.qvl_attention_worklist_split(p, 1, 16, 64, 0, None, 0, C.byref(n), C.byref(nw)) == -1
    assert lib.qvl_attention_worklist_split(p, 1, 16, 64, 256, None, 0, C.byref(n), C.byref(nw)) == 0
    small = np.zeros((1, 4), np.int32)
    assert lib.qvl_attention_worklist_split(p, 1, 16, 64, 256, small.ctypes.data_as(C.POINTER(C.c_int32)), 1,
                                            C.byref(n), C.byref(nw)) == -1
    nb = C.c_size_t()
    assert lib.qvl_attention_split_workspace_size(64, 10, 4, C.byref(nb)) == 0 and nb.value == 6 * 128 * 66 * 4
    assert lib.qvl_attention_split_workspace_size(72, 10, 11, C.byref(nb)) == -1


def test_metadata_packed_into_one_transfer(pkg):
    """The per-grid device metadata goes to the device in one copy (_to_device_packed): every array
    comes back with its shape, dtype and bits, at a 256-byte-aligned offset of one allocation
    (run on the CPU device here; the tower passes its GPU)."""
    import torch
    m = pkg.grid_metadata([(1, 48, 48), (2, 10, 14)])
    host = {"cu_seqlens": m.cu_seqlens, "pos_hw": m.pos_hw, "tap_idx": m.tap_idx, "tap_w": m.tap_w, "tiles": m.tiles}
    out = pkg.vision._to_device_packed(host, "cpu")
    base = out["cu_seqlens"].data_ptr()
    for name, a in host.items():
        t = out[name]
        assert tuple(t.shape) == a.shape, name
        assert t.dtype == (torch.float32 if a.dtype == np.float32 else torch.int32), name
        np.testing.assert_array_equal(t.numpy(), a)
        assert (t.data_ptr() - base) % 256 == 0, name
    with pytest.raises(TypeError):
        pkg.vision._to_device_packed({"x": np.zeros(3, np.int64)}, "cpu")
