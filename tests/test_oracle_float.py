"""Pins the oracle's floating-point ops (CPU) against torch library routines, attention invariants
and transformers' independent Qwen3VLVisionModel (float64)."""
import numpy as np
import pytest

from oracle import indices as ix
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
F = torch.nn.functional
P64 = vt._P("fp64")


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def test_bf16_round_matches_torch():
    x = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1e3
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(vt.bf16_round(x), ref)
    assert np.isnan(vt.bf16_round(np.array([np.nan], np.float32)))[0]


def test_layer_norm_vs_torch():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 96)) * 3 + 5
    w = rng.standard_normal(96); b = rng.standard_normal(96)
    ref = F.layer_norm(torch.from_numpy(x), (96,), torch.from_numpy(w), torch.from_numpy(b), 1e-6).numpy()
    np.testing.assert_allclose(vt.layer_norm(x, w, b, 1e-6, P64), ref, rtol=1e-12, atol=1e-12)


def test_gelu_tanh_vs_torch():
    x = np.linspace(-8, 8, 4001)
    ref = F.gelu(torch.from_numpy(x), approximate="tanh").numpy()
    np.testing.assert_allclose(vt.gelu_tanh(x, P64), ref, rtol=1e-12, atol=1e-14)
    # and it is not the exact-erf GELU
    assert np.abs(vt.gelu_tanh(x, P64) - F.gelu(torch.from_numpy(x)).numpy()).max() > 1e-5


def test_rotary_vs_complex_rotation():
    """neox rotate-half == complex multiply of (x_d + i x_{d+hd/2}) by e^{i theta_d}."""
    rng = np.random.default_rng(2)
    n, h, hd = 11, 3, 64
    x = rng.standard_normal((n, h, hd))
    ang = rng.standard_normal((n, hd // 2))
    emb = np.concatenate([ang, ang], -1)
    out = vt.apply_rotary(x, np.cos(emb), np.sin(emb), P64)
    z = (x[..., : hd // 2] + 1j * x[..., hd // 2:]) * np.exp(1j * ang)[:, None, :]
    np.testing.assert_allclose(out, np.concatenate([z.real, z.imag], -1), rtol=1e-12, atol=1e-12)


def _qkv(rng, n, h, hd):
    return [rng.standard_normal((n, h, hd)) for _ in range(3)]


def test_attention_vs_sdpa_and_invariants():
    rng = np.random.default_rng(3)
    cu = np.array([0, 5, 5, 37, 38, 100], np.int32)   # includes an empty and a length-1 segment
    n, h, hd = 100, 4, 32
    q, k, v = _qkv(rng, n, h, hd)
    out = vt.attention_varlen(q, k, v, cu, P64)
    for i in range(len(cu) - 1):
        s, e = cu[i], cu[i + 1]
        if s == e:
            continue
        t = lambda a: torch.from_numpy(a[s:e].transpose(1, 0, 2)).unsqueeze(0)
        ref = F.scaled_dot_product_attention(t(q), t(k), t(v))[0].numpy().transpose(1, 0, 2)
        np.testing.assert_allclose(out[s:e], ref, rtol=1e-10, atol=1e-12)
    # length-1 segment returns v
    np.testing.assert_allclose(out[37], v[37], rtol=1e-12)
    # permuting keys/values inside a segment leaves outputs unchanged
    perm = np.arange(n); perm[5:37] = 5 + rng.permutation(32)
    out2 = vt.attention_varlen(q, k[perm], v[perm], cu, P64)
    np.testing.assert_allclose(out2, out, rtol=1e-10, atol=1e-12)
    # no cross-segment leakage: changing segment 4's k/v leaves segment 2 alone
    k3 = k.copy(); k3[38:] += 10
    out3 = vt.attention_varlen(q, k3, v, cu, P64)
    np.testing.assert_array_equal(out3[:38], out[:38])


TINY = vt.VisionSpec(hidden_size=64, out_hidden_size=48, depth=3, num_heads=2, intermediate_size=96,
                     patch_size=4, temporal_patch_size=2, spatial_merge_size=2, in_channels=3,
                     num_position_embeddings=64, deepstack_visual_indexes=(0, 2))


@pytest.mark.parametrize("grids", [[(1, 4, 6)], [(1, 8, 8), (1, 2, 4)], [(3, 4, 4)], [(2, 6, 2), (1, 4, 4)]])
def test_tower_fp64_vs_transformers(grids):
    from tests.hf_pin import hf_vision_model, hf_encode
    params = vt.init_params(TINY, seed=7, bias_std=0.02, ln_noise=0.1)
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(8).standard_normal((n, TINY.patch_volume))
    ours = vt.encode_vision(params, px, grids, TINY, "fp64")
    model = hf_vision_model(params, TINY)
    taps = ix.pos_embed_taps_ref(grids, TINY.num_position_embeddings)   # the reference's t>1 quirk
    tok, ds = hf_encode(model, px, grids, taps=taps)
    assert rel_l2(ours.tokens, tok) < 1e-7
    assert len(ds) == len(ours.deepstack)
    for a, b in zip(ours.deepstack, ds):
        assert rel_l2(a, b) < 1e-7


def test_tower_bf16_and_fp32_close_to_fp64():
    grids = [(1, 8, 8), (2, 4, 4)]
    params = vt.init_params(TINY, seed=3)
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(4).standard_normal((n, TINY.patch_volume)).astype(np.float32)
    ref = vt.encode_vision(params, px, grids, TINY, "fp64")
    f32 = vt.encode_vision(params, px, grids, TINY, "fp32")
    b16 = vt.encode_vision(params, px, grids, TINY, "bf16")
    assert rel_l2(f32.tokens, ref.tokens) < 1e-5
    assert 1e-4 < rel_l2(b16.tokens, ref.tokens) < 2e-2


def test_patchify_layout():
    """sample.py:112-121: rows in merge-block order, each (C, Tp, P, P)."""
    rng = np.random.default_rng(5)
    frames = rng.standard_normal((1, 3, 8, 12)).astype(np.float32)
    px, g = vt.patchify(frames, patch=2, tpatch=2, merge=2)
    assert g.tolist() == [[1, 4, 6]]
    f, r, c = ix.token_coords_closed(g)
    dup = np.concatenate([frames, frames], 0)       # temporal pad duplicates the frame
    for n in range(px.shape[0]):
        blk = dup[:, :, 2 * r[n]:2 * r[n] + 2, 2 * c[n]:2 * c[n] + 2]       # (Tp, C, P, P)
        np.testing.assert_array_equal(px[n], blk.transpose(1, 0, 2, 3).reshape(-1))


# ---------------------------------------------------------------------------------------------
# window-attention path (model.py:808-850): permutation formulation vs a dense mask in token order
# ---------------------------------------------------------------------------------------------
def _masked_window_tower(params, px, grid, spec):
    """The window path without any shuffle: every block attends through an explicit token x token
    mask in the original order (same window / same full-attention range of the window order)."""
    p = P64
    prm = params["visual"]
    x = vt.dense(px, prm["patch_embed"]["proj"]["kernel"], prm["patch_embed"]["proj"]["bias"], p)
    x = x + vt.pos_embed(prm["pos_embed"]["embedding"], grid, spec, p)
    cos, sin = vt.rotary_cos_sin(grid, spec, p)
    n, D, H, hd = x.shape[0], spec.hidden_size, spec.num_heads, spec.head_dim
    widx, cuw = ix.window_index_closed(grid, spec.spatial_merge_size, spec.patch_size, spec.window_size)
    wpos = np.empty(n, np.int64)                           # window-order position of each token
    for r, g in enumerate(widx):
        wpos[4 * g:4 * g + 4] = 4 * r + np.arange(4)
    win = np.searchsorted(cuw, wpos, side="right")
    full = np.searchsorted(ix.cu_full_window_ref(grid, 2), wpos, side="right")
    masks = {True: full[:, None] == full[None, :], False: win[:, None] == win[None, :]}
    feats = []
    for i in range(spec.depth):
        b = prm[f"blocks_{i}"]
        h = vt.layer_norm(x, b["norm1"]["weight"], b["norm1"]["bias"], 1e-6, p)
        qkv = vt.dense(h, b["attn"]["qkv"]["kernel"], b["attn"]["qkv"]["bias"], p)
        q = vt.apply_rotary(qkv[:, :D].reshape(n, H, hd), cos, sin, p)
        k = vt.apply_rotary(qkv[:, D:2 * D].reshape(n, H, hd), cos, sin, p)
        v = qkv[:, 2 * D:].reshape(n, H, hd)
        m = masks[i in set(spec.fullatt_block_indexes)]
        o = np.zeros((n, H, hd))
        for hh in range(H):
            sc = (q[:, hh] @ k[:, hh].T) * hd ** -0.5
            sc = np.where(m, sc, -np.inf)
            sc = np.exp(sc - sc.max(axis=1, keepdims=True))
            o[:, hh] = (sc / sc.sum(axis=1, keepdims=True)) @ v[:, hh]
        x = x + vt.dense(o.reshape(n, D), b["attn"]["proj"]["kernel"], b["attn"]["proj"]["bias"], p)
        h = vt.layer_norm(x, b["norm2"]["weight"], b["norm2"]["bias"], 1e-6, p)
        x = x + vt.vision_mlp(h, b["mlp"], p)
        if i in set(spec.deepstack_visual_indexes):
            feats.append(vt.patch_merger(x, prm[f"deepstack_mergers_{len(feats)}"], spec, True, p))
    return vt.patch_merger(x, prm["merger"], spec, False, p), feats


WSPEC = vt.VisionSpec(hidden_size=32, out_hidden_size=24, depth=4, num_heads=2, intermediate_size=48,
                      patch_size=4, temporal_patch_size=2, spatial_merge_size=2, in_channels=3,
                      num_position_embeddings=64, deepstack_visual_indexes=(0, 2), window_size=16,
                      fullatt_block_indexes=(1, 3))


@pytest.mark.parametrize("grids", [[(1, 8, 12)], [(1, 8, 12), (2, 4, 4)], [(2, 6, 10)], [(1, 12, 4), (1, 4, 8)]])
def test_window_path_vs_dense_mask(grids):
    params = vt.init_params(WSPEC, seed=6, bias_std=0.1, ln_noise=0.1)
    n = sum(t * h * w for t, h, w in grids)
    px = np.random.default_rng(1).standard_normal((n, WSPEC.patch_volume))
    out = vt.encode_vision(params, px, grids, WSPEC, "fp64")
    tok, feats = _masked_window_tower(params, px, np.asarray(grids), WSPEC)
    np.testing.assert_allclose(out.tokens, tok, rtol=1e-10, atol=1e-10)
    for a, b in zip(out.deepstack, feats):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-10)
    # and the windows really restrict attention: the full-attention-only tower differs
    import dataclasses
    full = vt.encode_vision(params, px, grids, dataclasses.replace(WSPEC, fullatt_block_indexes=None), "fp64")
    assert rel_l2(full.tokens, out.tokens) > 1e-3


def test_window_covering_whole_frames_equals_full_path():
    """One window per frame (window_size >= frame) and no full blocks: window order is the identity
    and cu_window the per-frame cu_seqlens, so the window path equals the standard path."""
    import dataclasses
    spec = dataclasses.replace(WSPEC, window_size=64, fullatt_block_indexes=())
    params = vt.init_params(spec, seed=2)
    grids = [(1, 8, 8), (2, 4, 8)]
    px = np.random.default_rng(3).standard_normal((sum(t * h * w for t, h, w in grids), spec.patch_volume))
    a = vt.encode_vision(params, px, grids, spec, "fp64")
    b = vt.encode_vision(params, px, grids, dataclasses.replace(spec, fullatt_block_indexes=None), "fp64")
    np.testing.assert_allclose(a.tokens, b.tokens, rtol=1e-12, atol=1e-12)
