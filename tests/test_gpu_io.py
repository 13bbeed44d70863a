"""GPU parity for the steps either side of the tower, through the C ABI: on-device patchify
(bit-exact against the preprocessing oracle), vision-token injection and deepstack adds
(bit-exact against the scatter oracle), and the pre-packed weight file (bit-identical tower)."""
import numpy as np
import pytest

from oracle import preprocess as opp
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(np.asarray(a, np.float32)).view(np.uint32)


# ---------------------------------------------------------------------------------------------
# patchify
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("F,H,W,cin,P,Tp", [
    (1, 64, 96, 3, 16, 2),      # one image, frame duplicated (config 0 style)
    (1, 32, 32, 4, 16, 2),      # RGBA: alpha dropped
    (3, 64, 64, 3, 16, 2),      # 3 frames -> padded to 4 (2 temporal patches)
    (16, 64, 32, 3, 16, 2),     # video, t = 8
    (1, 56, 84, 3, 14, 2),      # patch 14: the element-wise path
    (2, 48, 48, 3, 12, 1),      # temporal patch 1
])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_patchify_bit_exact(pkg, F, H, W, cin, P, Tp, dtype):
    rng = np.random.default_rng(F * 100 + H + W + cin + P)
    frames = rng.integers(0, 256, size=(F, H, W, cin), dtype=np.uint8)
    frames[0, 0, 0, :3] = [0, 255, 128]
    px, g = pkg.preprocess.patchify_frames(frames, P, 2, Tp, dtype=dtype)
    ref, gref = opp.preprocess_frames_ref(frames, patch=P, tpatch=Tp, merge=2)
    assert g.tolist() == gref.tolist()
    got = px.float().cpu().numpy()
    want = ref if dtype == "float32" else vt.bf16_round(ref)
    assert got.shape == want.shape
    assert np.array_equal(bits(got), bits(want))


def test_patchify_errors(pkg):
    f = np.zeros((1, 40, 64, 3), np.uint8)
    with pytest.raises(ValueError):
        pkg.preprocess.patchify_frames(f, 16, 2, 2)          # 40 not divisible by 16
    f = np.zeros((1, 48, 64, 3), np.uint8)
    with pytest.raises(ValueError):
        pkg.preprocess.patchify_frames(f, 16, 2, 2)          # grid 3 x 4: 3 not divisible by merge 2
    lib = pkg.capi.load()
    buf = torch.empty(16, dtype=torch.uint8, device="cuda")
    assert lib.qvl_patchify(None, 1, buf.data_ptr(), 1, 32, 48, 3, 16, 2, 2, buf.data_ptr(), 1536) == -1
    assert lib.qvl_patchify(None, 1, buf.data_ptr(), 1, 32, 32, 5, 16, 2, 2, buf.data_ptr(), 1536) == -1
    assert lib.qvl_patchify(None, 7, buf.data_ptr(), 1, 32, 32, 3, 16, 2, 2, buf.data_ptr(), 1536) == -2


def test_preprocess_image_into_tower(pkg):
    """preprocess_image (PIL resize on the host, patchify on the GPU) feeds the tower the same
    pixel values as the reference's numpy preprocessing, so the tower outputs are bit-identical."""
    from PIL import Image
    rng = np.random.default_rng(7)
    img = Image.fromarray(rng.integers(0, 256, size=(70, 101, 3), dtype=np.uint8))
    px, g = pkg.preprocess.preprocess_image(img, 16, 2, 2)
    new_h, new_w = pkg.preprocess.smart_resize(70, 101, 32, pkg.preprocess.DEFAULT_MIN_PIXELS,
                                               pkg.preprocess.DEFAULT_MAX_PIXELS)
    assert g.tolist() == [[1, new_h // 16, new_w // 16]]
    host = np.asarray(img.resize((new_w, new_h), Image.Resampling.BICUBIC), np.uint8)
    ref, _ = opp.preprocess_frames_ref(host, patch=16, tpatch=2, merge=2)
    assert np.array_equal(bits(px.cpu().numpy()), bits(ref))
    spec = pkg.spec_2b()
    spec.depth, spec.deepstack_visual_indexes = 2, (0,)
    tower = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(pkg.random_params(spec, seed=3))
    a = tower(px, g)
    b = tower(torch.from_numpy(ref).cuda(), g)
    assert torch.equal(a[0], b[0]) and all(torch.equal(x, y) for x, y in zip(a[1], b[1]))


# ---------------------------------------------------------------------------------------------
# injection / deepstack
# ---------------------------------------------------------------------------------------------
def _case(seed, B, S, D, V, pad, n_pad, pad_at0=False):
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, 50, size=(B, S)).astype(np.int32)
    tokens[tokens == pad] = pad + 1
    for b in range(B):
        idx = rng.choice(S, size=min(n_pad, S), replace=False)
        if pad_at0:
            idx[0] = 0
        tokens[b, idx] = pad
    hidden = (rng.standard_normal((B, S, D)) * 2).astype(np.float32)
    hidden[:, 0, :3] = -0.0
    vis = rng.standard_normal((B, V, D)).astype(np.float32)
    return tokens, hidden, vis


@pytest.mark.parametrize("hdt,rdt", [("bfloat16", "bfloat16"), ("bfloat16", "float32"), ("float32", "float32"),
                                     ("float32", "bfloat16")])
@pytest.mark.parametrize("B,S,D,V,n_pad,pad_at0", [
    (2, 300, 64, 40, 40, False),       # exact count
    (1, 3000, 128, 64, 20, True),      # fewer pads than rows, a pad at position 0
    (3, 2100, 96, 30, 20, False),      # fewer pads, none at 0: the trailing +0 on row 0
    (2, 500, 64, 10, 50, False),       # more pads than rows
    (1, 100, 32, 8, 0, False),         # no pads
    (2, 400, 36, 20, 10, True),        # rows not a multiple of 8 elements: the element-wise kernel
])
def test_inject_and_deepstack_bit_exact(pkg, hdt, rdt, B, S, D, V, n_pad, pad_at0):
    io = pkg.decoder_io
    pad = 77
    tokens, hidden, vis = _case(B * S + V, B, S, D, V, pad, n_pad, pad_at0)
    hb = hdt == "bfloat16"
    h0 = vt.bf16_round(hidden) if hb else hidden
    th, tr = getattr(torch, hdt), getattr(torch, rdt)
    vis_in = vt.bf16_round(vis) if rdt == "bfloat16" else vis
    h = torch.from_numpy(h0).cuda().to(th)
    tk = torch.from_numpy(tokens).cuda()
    out, mask, _ = io.inject_vision(h, tk, torch.from_numpy(vis_in).cuda().to(tr), pad)
    ref = opp.inject_ref(h0, tokens, vis_in, pad, hb)
    assert np.array_equal(bits(out.float().cpu().numpy()), bits(ref))
    assert torch.equal(mask.cpu(), torch.from_numpy(tokens == pad))
    # positions kernel alone
    pos, cnt = io.vision_positions(tk, V, match=pad)
    rp, rc = opp.vision_positions_ref(tokens == pad, V)
    assert np.array_equal(pos.cpu().numpy()[:, :V], rp) and np.array_equal(cnt.cpu().numpy(), rc)
    # two deepstack layers on top (features broadcast over the batch)
    rng = np.random.default_rng(5)
    ref_h = ref
    for layer in range(2):
        feat = rng.standard_normal((1, V, D)).astype(np.float32)
        feat_in = vt.bf16_round(feat) if rdt == "bfloat16" else feat
        out = io.apply_deepstack(out, mask, torch.from_numpy(feat_in).cuda().to(tr))
        ref_h = opp.deepstack_add_ref(ref_h, tokens == pad, feat_in, hb)
        assert np.array_equal(bits(out.float().cpu().numpy()), bits(ref_h)), layer


def test_inject_vision_embeddings_pack(pkg):
    """A VisionEmbeddings from the tower (tokens + deepstack) through the forward_vlm steps."""
    io = pkg.decoder_io
    spec = pkg.spec_2b()
    spec.depth, spec.deepstack_visual_indexes = 3, (0, 2)
    tower = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(pkg.random_params(spec, seed=9))
    grid = np.array([[1, 8, 8]], np.int32)
    px = torch.from_numpy(np.random.default_rng(2).standard_normal((64, 1536), dtype=np.float32)).cuda()
    tokens_v, ds = tower(px, grid)
    ve = pkg.VisionEmbeddings(tokens=tokens_v, deepstack=tuple(ds))
    S, D, pad = 40, spec.out_hidden_size, 5
    toks = np.zeros((2, S), np.int32)
    toks[:, 3:19] = pad                      # 16 = 64 / 4 vision tokens per row
    hidden = torch.randn((2, S, D), device="cuda").to(torch.bfloat16)
    h0 = hidden.float().cpu().numpy()
    out, mask, dsf = io.inject_vision(hidden, torch.from_numpy(toks).cuda(), ve, pad)
    ref = opp.inject_ref(h0, toks, tokens_v.float().cpu().numpy()[None], pad, True)
    assert np.array_equal(bits(out.float().cpu().numpy()), bits(ref))
    assert len(dsf) == 2 and dsf[0].shape == (2, 16, D)
    out = io.apply_deepstack(out, mask, dsf[1])
    ref = opp.deepstack_add_ref(ref, toks == pad, ds[1].float().cpu().numpy()[None], True)
    assert np.array_equal(bits(out.float().cpu().numpy()), bits(ref))


# ---------------------------------------------------------------------------------------------
# pre-packed weight file
# ---------------------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", ["bfloat16", "float32"])
def test_packed_weights_round_trip(pkg, tmp_path, dtype):
    spec = pkg.spec_2b()
    spec.depth, spec.deepstack_visual_indexes = 2, (1,)
    tower = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(pkg.random_params(spec, seed=21))
    path = str(tmp_path / "vision.packed.safetensors")
    pkg.weights.save_packed(tower, path)
    meta = pkg.weights.read_packed_metadata(path)
    assert meta["dtype"] == dtype
    t2 = pkg.weights.load_packed(path)
    assert t2.spec.deepstack_visual_indexes == (1,) and t2.dtype == dtype
    for k, v in tower.packed_state().items():
        assert torch.equal(v, t2.packed_state()[k]), k
    grid = np.array([[1, 8, 12]], np.int32)
    px = torch.from_numpy(np.random.default_rng(1).standard_normal((96, 1536), dtype=np.float32)).cuda()
    a, b = tower(px, grid), t2(px, grid)
    assert torch.equal(a[0], b[0]) and all(torch.equal(x, y) for x, y in zip(a[1], b[1]))
    st = t2.packed_state()
    st["blocks.0.fc1.w"] = st["blocks.0.fc1.w"][:, :64].contiguous()
    with pytest.raises(ValueError):
        pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind_packed(st)


def test_hf_checkpoint_into_tower(pkg, tmp_path):
    """HF safetensors -> load_hf_vision_params -> tower equals the tower bound to the same params."""
    pytest.importorskip("transformers")
    from safetensors.torch import save_file
    from tests.hf_pin import hf_vision_model

    spec = pkg.spec_2b()
    spec.depth, spec.deepstack_visual_indexes = 2, (0,)
    ospec = vt.VisionSpec(depth=2, deepstack_visual_indexes=(0,))
    params = vt.init_params(ospec, seed=8, bias_std=0.05, ln_noise=0.05)
    sd = {"model.visual." + k: v.contiguous() for k, v in hf_vision_model(params, ospec, "float32").state_dict().items()
          if "inv_freq" not in k}
    save_file(sd, str(tmp_path / "m.safetensors"))
    loaded = pkg.weights.load_hf_vision_params(str(tmp_path))
    t1 = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(loaded)
    t2 = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(params)
    grid = np.array([[1, 8, 8]], np.int32)
    px = torch.from_numpy(np.random.default_rng(4).standard_normal((64, 1536), dtype=np.float32)).cuda()
    a, b = t1(px, grid), t2(px, grid)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1][0], b[1][0])


@pytest.mark.parametrize("D", [64, 36])
def test_scatter_drops_out_of_range_positions(pkg, D):
    """Caller-supplied positions past the row (>= seq_len) are dropped, as XLA drops out-of-bounds
    scatter updates; the in-range ones apply as usual (SET and ADD, vector and element kernels)."""
    cp = pkg.capi
    lib = cp.load()
    B, S, V = 2, 50, 6
    rng = np.random.default_rng(9)
    hidden = rng.standard_normal((B, S, D)).astype(np.float32)
    rows = rng.standard_normal((B, V, D)).astype(np.float32)
    pos = np.array([[3, S, 7, S + 5, 49, 10], [S + 100, 0, 1, 2, S, 4]], np.int32)
    cnt = np.full(B, V, np.int32)          # every row "filled": no row-0 bookkeeping
    st = torch.cuda.current_stream().cuda_stream
    for mode in (cp.QVL_SCATTER_SET, cp.QVL_SCATTER_ADD):
        h = torch.from_numpy(hidden).cuda()
        r = torch.from_numpy(rows).cuda()
        p, c = torch.from_numpy(pos).cuda(), torch.from_numpy(cnt).cuda()
        cp.check(lib.qvl_scatter_vision_rows(st, mode, cp.QVL_DTYPE_F32, h.data_ptr(), B, S, D, cp.QVL_DTYPE_F32,
                                             r.data_ptr(), V * D, V, p.data_ptr(), c.data_ptr()), "scatter")
        ref = hidden.copy()
        for b in range(B):
            for j in range(V):
                if 0 <= pos[b, j] < S:
                    ref[b, pos[b, j]] = rows[b, j] if mode == cp.QVL_SCATTER_SET else ref[b, pos[b, j]] + rows[b, j]
        assert np.array_equal(bits(h.cpu().numpy()), bits(ref)), mode
