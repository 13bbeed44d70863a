"""CPU pins for the steps either side of the tower: the preprocessing oracle, the injection /
deepstack oracle, the host-side `smart_resize` and the HF-checkpoint key mapping."""
import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import indices as ix
from oracle import preprocess as opp
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")


# ---------------------------------------------------------------------------------------------
# normalisation: exact rational arithmetic, rounded to float32 at each of the reference's ops
# ---------------------------------------------------------------------------------------------
def _round_f32(q: Fraction) -> np.float32:
    """Nearest float32 to the rational q, ties to even (exact comparisons)."""
    c = np.float32(float(q))
    cands = {c, np.nextafter(c, np.float32(np.inf)), np.nextafter(c, np.float32(-np.inf))}
    best = min(cands, key=lambda v: (abs(Fraction(float(v)) - q),
                                     int(np.array(v, np.float32).view(np.uint32)) & 1))
    return np.float32(best)


def test_normalize_matches_exact_rounding():
    u = np.arange(256, dtype=np.uint8)
    got = opp.normalize_u8_ref(np.stack([u, u, u], -1))[:, 0]
    for k in range(256):
        t = _round_f32(Fraction(k, 255))
        s = _round_f32(Fraction(float(t)) - Fraction(1, 2))
        v = _round_f32(Fraction(float(s)) / Fraction(1, 2))
        assert got[k].view(np.uint32) == v.view(np.uint32), k
    # the mathematics: (2u - 255) / 255 within one float32 rounding of each op
    np.testing.assert_allclose(got, (2 * u.astype(np.float64) - 255) / 255, rtol=0, atol=2e-7)
    assert got[0] == -1.0 and got[255] == 1.0


# ---------------------------------------------------------------------------------------------
# patch layout: transformers' Qwen2-VL image processor (independent) + per-pixel closed form
# ---------------------------------------------------------------------------------------------
def test_preprocess_layout_vs_transformers():
    mod = pytest.importorskip("transformers.models.qwen2_vl.image_processing_pil_qwen2_vl")
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, size=(64, 96, 3), dtype=np.uint8)
    px, g = opp.preprocess_frames_ref(img, patch=16, tpatch=2, merge=2)
    assert g.tolist() == [[1, 4, 6]]
    chw = np.transpose(opp.normalize_u8_ref(img), (2, 0, 1))
    ref, gh, gw = mod.Qwen2VLImageProcessorPil().patchify(chw, patch_size=16, merge_size=2, temporal_patch_size=2)
    assert (gh, gw) == (4, 6)
    assert np.array_equal(px, np.asarray(ref, np.float32))


@pytest.mark.parametrize("F,cin", [(1, 3), (1, 4), (3, 3), (4, 4)])
def test_preprocess_closed_form(F, cin):
    """pixel_values[n, (c, tp, ph, pw)] = norm(frame[min(t*Tp + tp, F-1)][2*r+.. rows][..][c])."""
    rng = np.random.default_rng(F * 10 + cin)
    P, Tp, m, H, W = 4, 2, 2, 16, 24
    frames = rng.integers(0, 256, size=(F, H, W, cin), dtype=np.uint8)
    px, g = opp.preprocess_frames_ref(frames, patch=P, tpatch=Tp, merge=m)
    gt = -(-F // Tp)
    assert g.tolist() == [[gt, H // P, W // P]]
    f_idx, r_idx, c_idx = ix.token_coords_closed(g)
    lut = opp.normalize_u8_ref(np.stack([np.arange(256, dtype=np.uint8)] * 3, -1))[:, 0]
    for n in range(px.shape[0]):
        for c in range(3):
            for tp in range(Tp):
                fr = min(f_idx[n] * Tp + tp, F - 1)
                blk = frames[fr, P * r_idx[n]:P * r_idx[n] + P, P * c_idx[n]:P * c_idx[n] + P, c]
                got = px[n, (c * Tp + tp) * P * P:(c * Tp + tp + 1) * P * P].reshape(P, P)
                assert np.array_equal(got, lut[blk])


# ---------------------------------------------------------------------------------------------
# smart_resize (product host code) vs transformers' copy of the same rule
# ---------------------------------------------------------------------------------------------
def test_smart_resize_vs_transformers(pkg):
    mod = pytest.importorskip("transformers.models.qwen2_vl.image_processing_pil_qwen2_vl")
    sr = pkg.preprocess.smart_resize
    f, lo, hi = 32, 56 * 56, 12845056
    checked = 0
    for h in list(range(20, 400, 7)) + [768, 1000, 3000, 5000]:
        for w in list(range(20, 400, 11)) + [768, 1344, 4000]:
            if max(h, w) / min(h, w) > 200:
                continue
            if round(h / f) < 1 or round(w / f) < 1:
                continue      # the reference clamps to `factor` first (max(factor, ...)); HF does not
            got = sr(h, w, f, lo, hi)
            ref = mod.smart_resize(h, w, factor=f, min_pixels=lo, max_pixels=hi)
            if min(ref) < f:
                continue
            assert got == tuple(ref), (h, w)
            checked += 1
    assert checked > 500
    # clamp cases worked by hand: h rounds to 0 blocks -> factor; area then within bounds
    assert sr(10, 500, 32, lo, hi) == (32, 512)
    assert sr(768, 768, 32, lo, hi) == (768, 768)
    with pytest.raises(ValueError):
        sr(1, 500, 32, lo, hi)
    with pytest.raises(ValueError):
        sr(0, 5, 32, lo, hi)


# ---------------------------------------------------------------------------------------------
# injection / deepstack: element-by-element loops applying the reference's updates in order
# ---------------------------------------------------------------------------------------------
def _positions_loop(tokens_row, match, n):
    out = []
    for s, t in enumerate(tokens_row):
        if t == match and len(out) < n:
            out.append(s)
    return out + [-1] * (n - len(out)), sum(1 for t in tokens_row if t == match)


def _cast(x, bf16):
    return float(vt.bf16_round(np.array([x], np.float32))[0]) if bf16 else float(np.float32(x))


def _inject_loop(hidden, tokens, vis, pad, bf16):
    h = np.array(hidden, np.float32, copy=True)
    B, S, D = h.shape
    for b in range(B):
        vb = vis[0] if vis.shape[0] == 1 else vis[b]
        V = vb.shape[0]
        pos, _ = _positions_loop(list(tokens[b]), pad, V)
        old0 = h[b, 0].copy()
        for j in range(V):           # .at[pos].set(updates), one update at a time
            if pos[j] >= 0:
                for d in range(D):
                    h[b, pos[j], d] = _cast(vb[j, d], bf16)
            else:
                h[b, 0] = old0       # the unfilled update carries the row gathered before the scatter
    return h


def _deepstack_loop(hidden, mask, feat, bf16):
    h = np.array(hidden, np.float32, copy=True)
    B, S, D = h.shape
    for b in range(B):
        fb = feat[0] if feat.shape[0] == 1 else feat[b]
        pos, _ = _positions_loop(list(mask[b].astype(int)), 1, fb.shape[0])
        for j in range(fb.shape[0]):
            row = pos[j] if pos[j] >= 0 else 0
            for d in range(D):
                u = _cast(fb[j, d], bf16) if pos[j] >= 0 else 0.0
                h[b, row, d] = _cast(np.float32(h[b, row, d]) + np.float32(u), bf16)
    return h


CASES = {
    # name: (tokens, V)
    "exact": ([[5, 9, 9, 1, 9, 2, 9]], 4),
    "fewer_pads": ([[9, 3, 9, 4]], 4),              # 2 pads, 4 rows; a pad at position 0
    "fewer_pads_no0": ([[3, 9, 4, 9]], 3),
    "more_pads": ([[9, 9, 9, 9, 9]], 2),
    "no_pads": ([[1, 2, 3]], 2),
    "batch": ([[9, 1, 9, 2], [3, 9, 9, 9]], 2),
}


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", sorted(CASES))
def test_inject_and_deepstack_vs_loops(case, bf16):
    toks, V = CASES[case]
    tokens = np.array(toks, np.int64)
    B, S, D = tokens.shape[0], tokens.shape[1], 5
    rng = np.random.default_rng(len(case))
    hidden = rng.standard_normal((B, S, D)).astype(np.float32) * 3
    hidden[:, 0, 0] = -0.0                           # signed zero: an ADD of +0 makes it +0
    if bf16:
        hidden = vt.bf16_round(hidden)
    vis = rng.standard_normal((B, V, D)).astype(np.float32)
    feat = rng.standard_normal((1, V, D)).astype(np.float32)      # broadcast over the batch
    pos, cnt = opp.vision_positions_ref(tokens == 9, V)
    for b in range(B):
        lp, lc = _positions_loop(list(tokens[b]), 9, V)
        assert pos[b].tolist() == lp and cnt[b] == lc
    assert np.array_equal(opp.inject_ref(hidden, tokens, vis, 9, bf16), _inject_loop(hidden, tokens, vis, 9, bf16))
    mask = tokens == 9
    a = opp.deepstack_add_ref(hidden, mask, feat, bf16)
    b_ = _deepstack_loop(hidden, mask, feat, bf16)
    assert np.array_equal(a.view(np.uint32), b_.view(np.uint32))   # bitwise: signed zeros included


def test_inject_ambiguous_row0_keeps_old_value():
    """pad at position 0 with fewer pads than rows: the trailing unfilled updates restore row 0."""
    tokens = np.array([[9, 1, 9]])
    hidden = np.arange(15, dtype=np.float32).reshape(1, 3, 5)
    vis = -np.ones((1, 4, 5), np.float32)
    out = opp.inject_ref(hidden, tokens, vis, 9, False)
    assert np.array_equal(out[0, 0], hidden[0, 0]) and np.array_equal(out[0, 2], vis[0, 1])


# ---------------------------------------------------------------------------------------------
# HF checkpoint -> Flax tree: round trip through transformers' own parameter names
# ---------------------------------------------------------------------------------------------
def test_hf_checkpoint_loader_round_trip(pkg, tmp_path):
    pytest.importorskip("transformers")
    from safetensors.torch import save_file
    from tests.hf_pin import hf_vision_model

    spec = vt.VisionSpec(hidden_size=64, out_hidden_size=48, depth=2, num_heads=2, intermediate_size=96,
                         patch_size=4, temporal_patch_size=2, spatial_merge_size=2, in_channels=3,
                         num_position_embeddings=64, deepstack_visual_indexes=(0,))
    params = vt.init_params(spec, seed=4, bias_std=0.1, ln_noise=0.1)
    model = hf_vision_model(params, spec, dtype="float32")
    sd = {"model.visual." + k: v.contiguous() for k, v in model.state_dict().items() if "inv_freq" not in k}
    sd["model.language_model.layers.0.mlp.up_proj.weight"] = torch.zeros(2, 2)     # ignored (text)
    save_file(sd, str(tmp_path / "model-00001.safetensors"))
    got = pkg.weights.load_hf_vision_params(str(tmp_path))

    def flat(d, pre=""):
        for k, v in d.items():
            if isinstance(v, dict):
                yield from flat(v, pre + k + "/")
            else:
                yield pre + k, v

    ref = dict(flat(params))
    out = dict(flat(got))
    assert sorted(ref) == sorted(out)
    for k in ref:
        assert out[k].shape == ref[k].shape and np.array_equal(out[k], ref[k]), k
    assert pkg.weights.torch_key_to_flax("visual.blocks.3.mlp.linear_fc1.weight") == "visual/blocks_3/mlp/linear_fc1/kernel"
    assert pkg.weights.torch_key_to_flax("model.visual.merger.norm.weight") == "visual/merger/norm/weight"
    assert pkg.weights.torch_key_to_flax("model.language_model.norm.weight") is None
