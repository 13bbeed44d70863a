"""Tower parity at full depth: checkpoint-like parameters, and BASELINE configs 3 and 4 end to end.

Checkpoint-like parameters (`ckpt_params`): Dense kernels and the pos-embed table N(0, 0.02), Dense
biases N(0, 0.02), LayerNorm gamma 1 + N(0, 0.1) and beta N(0, 0.1), every value rounded to bf16 as
an HF checkpoint stores it. With them the folded LayerNorm is not the identity (W' = bf16(gamma W)
differs from W, and d = sum_k beta_k W_k is not zero) and every bias epilogue adds a non-zero bias,
which the BASELINE recipe (biases 0, gamma 1, beta 0) leaves unexercised.

Checkers: the numpy oracle (oracle/vision_tower.py) on the small grids, the torch-CPU restatement
(oracle/torch_tower.py, the same rounding points; pinned against the numpy oracle by
tests/test_oracle_torch.py) on the large ones, in bf16 (the reference's bf16 mode, model.py:549-656
with Qwen3VisionTransformer(spec, dtype=jnp.bfloat16)) and in fp32 / fp64.

Bars:
  per block in isolation (the block fed the oracle's input): rel-L2 <= 1e-2 (north star);
  end to end, bf16: the reference's own bf16 mode drifts ~1.4e-2 from its fp32 mode over 24 blocks,
  so no bf16 implementation that is not bit-identical to it can sit within 1e-2 of it there. The
  GPU tower must be about as close to the fp32 reference as the reference's bf16 mode is (within
  x E2E_DRIFT of it), and within x E2E_BF16_REL of that noise floor and E2E_BF16 absolutely of the bf16
  reference, for the tokens and every deepstack feature;
  fp32: within 1e-4 of the fp64 oracle, per block and end to end.
The measured values are printed."""
import numpy as np
import pytest

from oracle import torch_tower as tt
from oracle import vision_tower as vt

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL = 1e-2
# End-to-end bars, from the values measured on MI355X with a few percent of margin: the GPU tower's
# distance to the fp32 reference over the reference bf16 mode's own (measured <= 1.008 over the
# tests below), its distance to the bf16 reference over that same noise floor (<= 1.091) and
# absolutely (<= 1.61e-2, the 8B shape with checkpoint-like parameters).
E2E_DRIFT = 1.03
E2E_BF16_REL = 1.12
E2E_BF16 = 1.75e-2


def rel_l2(a, b):
    a = np.asarray(a, np.float64); b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def to_np(t):
    return t.float().cpu().numpy()


def dev_bf16(a):
    if isinstance(a, torch.Tensor):
        return a.to("cuda:0").to(torch.bfloat16).contiguous()
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to("cuda:0").to(torch.bfloat16)


def ckpt_params(ospec, seed):
    """init_params with non-zero biases and noisy LayerNorm affines, every leaf rounded to bf16."""
    p = vt.init_params(ospec, seed=seed, std=0.02, bias_std=0.02, ln_noise=0.1)

    def rnd(d):
        return {k: rnd(v) if isinstance(v, dict) else vt.bf16_round(v) for k, v in d.items()}
    return rnd(p)


def specs(pkg, shape, depth=None, ds=None):
    s = pkg.spec_2b() if shape == "2b" else pkg.spec_8b()
    if depth is not None:
        s.depth = depth
        s.fullatt_block_indexes = tuple(range(depth))
    if ds is not None:
        s.deepstack_visual_indexes = tuple(ds)
    o = vt.VisionSpec(hidden_size=s.hidden_size, out_hidden_size=s.out_hidden_size, depth=s.depth,
                      num_heads=s.num_heads, intermediate_size=s.intermediate_size,
                      deepstack_visual_indexes=tuple(s.deepstack_visual_indexes))
    return s, o


def pixels(grids, seed):
    n = sum(t * h * w for t, h, w in grids)
    return np.random.default_rng(seed).standard_normal((n, 1536), dtype=np.float32)


def end_to_end(label, got_tok, got_ds, rb, rf):
    """Assert the bf16 end-to-end bars on tokens + deepstack; rb / rf: bf16 / fp32 reference outputs
    (tokens, deepstack). Returns the printed summary."""
    rows = []
    names = ["tokens"] + [f"ds{j}" for j in range(len(got_ds))]
    assert len(got_ds) == len(rb[1]) == len(rf[1])
    for name, got, b, f in zip(names, [got_tok, *got_ds], [rb[0], *rb[1]], [rf[0], *rf[1]]):
        got, b, f = to_np(got), np.asarray(b, np.float32), np.asarray(f, np.float32)
        assert np.isfinite(got).all(), (label, name)
        e_b, e_f, e_ref = rel_l2(got, b), rel_l2(got, f), rel_l2(b, f)
        rows.append(f"{name} {e_b:.3e}/{e_f:.3e}/{e_ref:.3e}")
        assert e_f <= E2E_DRIFT * e_ref, (label, name, e_f, e_ref)
        assert e_b <= min(E2E_BF16_REL * e_ref, E2E_BF16), (label, name, e_b, e_ref)
    return f"{label}: " + ", ".join(rows) + " (vs bf16 ref / vs fp32 ref / bf16 ref vs fp32 ref)"


def per_block(tower, ctx, xin_of, ref_layers, depth, fused=True):
    """Each block fed the oracle's input: worst rel-L2 against the oracle's output."""
    worst = 0.0
    for i in range(depth):
        x = dev_bf16(xin_of(i))
        (tower.block_fused if fused else tower.block_staged)(i, x, ctx)
        r = rel_l2(to_np(x), np.asarray(ref_layers[i], np.float32))
        worst = max(worst, r)
        assert r <= TOL, (i, r)
    return worst


@pytest.mark.parametrize("shape", ["2b", "8b"])
def test_ckpt_params_small_grids_full_depth(pkg, shape):
    """2B (24 blocks, taps 5/11/17) and 8B (27 blocks, taps 8/16/24) towers with checkpoint-like
    parameters, two images (352 tokens), against the numpy oracle.
    bf16: every block in isolation through the staged entries, the fused entries with LayerNorm
    launches and the fused entries with the LayerNorms folded (the tower's default); every
    deepstack merger (folded and not) and the final merger; end to end through the whole-tower
    entry (folded and not) and the staged entries.
    fp32: every block in isolation and the tower end to end within 1e-4 of fp64."""
    spec, ospec = specs(pkg, shape)
    params = ckpt_params(ospec, seed=21 if shape == "2b" else 22)
    grids = [(1, 16, 16), (1, 8, 12)]
    g = np.array(grids, np.int32)
    px = pixels(grids, 23)
    ref = vt.encode_vision(params, px, grids, ospec, "bf16", keep_layers=True)
    f32 = vt.encode_vision(params, px, grids, ospec, "fp32")
    tower = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16", ln_fold=False).bind(params)
    towerf = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(params)
    assert towerf.ln_fold and not tower.ln_fold
    # the folds are not the identity here: W' = bf16(gamma W) != W and d != 0
    wq, (wf, cd) = tower.packed_state()["blocks.0.qkv.w"], towerf._folds["blocks.0.qkv"]
    assert not torch.equal(wq, wf) and float(cd[:, 1].abs().max()) > 0
    ctx, ctxf = tower._staged_ctx(g), towerf._staged_ctx(g)
    assert rel_l2(to_np(tower.embed_staged(px, ctx)), ref.embed) <= TOL
    xin = lambda i: ref.embed if i == 0 else ref.layers[i - 1]
    worst = max(per_block(tower, ctx, xin, ref.layers, spec.depth, fused=False),
                per_block(tower, ctx, xin, ref.layers, spec.depth),
                per_block(towerf, ctxf, xin, ref.layers, spec.depth))
    P = vt._P("bf16")
    xl = dev_bf16(ref.layers[-1])
    r = rel_l2(to_np(tower.merger_staged(xl, ctx)), vt.patch_merger(ref.layers[-1], params["visual"]["merger"],
                                                                    ospec, False, P))
    assert r <= TOL
    worst = max(worst, r)
    for j, li in enumerate(spec.deepstack_visual_indexes):
        xl = dev_bf16(ref.layers[li])
        for r in (rel_l2(to_np(tower.merger_staged(xl, ctx, j)), ref.deepstack[j]),
                  rel_l2(to_np(towerf.merger_fused(xl, ctxf, j)), ref.deepstack[j])):
            assert r <= TOL, (j, r)
            worst = max(worst, r)
    rb, rf = (ref.tokens, ref.deepstack), (f32.tokens, f32.deepstack)
    lines = [end_to_end("folded", *towerf(px, g), rb, rf), end_to_end("unfolded", *tower(px, g), rb, rf)]
    tok2, ds2, _ = tower.forward_staged(px, g)
    lines.append(end_to_end("staged", tok2, ds2, rb, rf))
    # fp32 tower against fp64
    r64 = vt.encode_vision(params, px, grids, ospec, "fp64", keep_layers=True)
    t32 = pkg.Qwen3VisionTransformer(spec, dtype="float32").bind(params)
    c32 = t32._staged_ctx(g)
    worst32 = 0.0
    for i in range(spec.depth):
        x = torch.from_numpy(np.ascontiguousarray(r64.embed if i == 0 else r64.layers[i - 1], np.float32)).to("cuda:0")
        t32.block_staged(i, x, c32)
        worst32 = max(worst32, rel_l2(to_np(x), r64.layers[i]))
    assert worst32 <= 1e-4
    tok32, ds32 = t32(px, g)
    e32 = [rel_l2(to_np(a), b) for a, b in zip([tok32, *ds32], [r64.tokens, *r64.deepstack])]
    assert max(e32) <= 1e-4, e32
    print(f"\n[{shape} ckpt params, 352 tokens] worst block/merger in isolation {worst:.3e}; " + "; ".join(lines)
          + f"; fp32 vs fp64: worst block {worst32:.2e}, end to end {max(e32):.2e}", flush=True)


@pytest.mark.parametrize("ln_fold", [True, False])
def test_ckpt_params_config2_image_full_depth(pkg, ln_fold):
    """One full config-2 image (grid 1x48x48, 2304 patches) on the 2B tower with checkpoint-like
    parameters, all 24 blocks and taps 5/11/17, against the torch-CPU oracle: every block and
    deepstack merger in isolation through the tower's entries, and the whole-tower entry end to
    end, with the LayerNorms folded (the benchmarked path) and with LayerNorm launches."""
    spec, ospec = specs(pkg, "2b")
    params = ckpt_params(ospec, seed=24)
    grids = [(1, 48, 48)]
    g = np.array(grids, np.int32)
    px = pixels(grids, 25)
    ref = tt.TorchTower(params, ospec, "bf16").run(px, grids, keep_layers=True)
    f32 = tt.TorchTower(params, ospec, "fp32").run(px, grids)
    tower = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16", ln_fold=ln_fold).bind(params)
    ctx = tower._staged_ctx(g)
    xin = lambda i: ref["embed"] if i == 0 else ref["layers"][i - 1]
    worst = per_block(tower, ctx, xin, [to_np(t) for t in ref["layers"]], spec.depth)
    for j, li in enumerate(spec.deepstack_visual_indexes):
        r = rel_l2(to_np(tower.merger_fused(dev_bf16(ref["layers"][li]), ctx, j)), to_np(ref["deepstack"][j]))
        assert r <= TOL, (j, r)
        worst = max(worst, r)
    rb = (to_np(ref["tokens"]), [to_np(t) for t in ref["deepstack"]])
    rf = (to_np(f32["tokens"]), [to_np(t) for t in f32["deepstack"]])
    line = end_to_end("fold" if ln_fold else "no fold", *tower(px, g), rb, rf)
    print(f"\n[config-2 image, ckpt params, 24 blocks] worst block/merger in isolation {worst:.3e}; {line}", flush=True)


def _baseline_full_depth(pkg, shape, grids, px, seed):
    spec, ospec = specs(pkg, shape)
    params = pkg.random_params(spec, seed=seed)            # the BASELINE recipe
    g = np.array(grids, np.int32)
    ref = tt.TorchTower(params, ospec, "bf16").run(px, grids, keep_layers=True)
    f32 = tt.TorchTower(params, ospec, "fp32").run(px, grids)
    tower = pkg.Qwen3VisionTransformer(spec, dtype="bfloat16").bind(params)
    ctx = tower._staged_ctx(g)
    xin = lambda i: ref["embed"] if i == 0 else ref["layers"][i - 1]
    worst = per_block(tower, ctx, xin, [to_np(t) for t in ref["layers"]], spec.depth)
    for j, li in enumerate(spec.deepstack_visual_indexes):
        r = rel_l2(to_np(tower.merger_fused(dev_bf16(ref["layers"][li]), ctx, j)), to_np(ref["deepstack"][j]))
        assert r <= TOL, (j, r)
        worst = max(worst, r)
    rb = (to_np(ref["tokens"]), [to_np(t) for t in ref["deepstack"]])
    rf = (to_np(f32["tokens"]), [to_np(t) for t in f32["deepstack"]])
    tok, ds = tower(px, g)
    return worst, end_to_end("whole tower", tok, ds, rb, rf), tok


def test_config3_video_full_depth(pkg):
    """BASELINE config 3 at full depth: 16 correlated 512x512 frames, temporal patch 2, grid
    (8, 32, 32) = 8192 patches in 8 per-frame segments, the 2B tower (BASELINE weights), all 24
    blocks and taps 5/11/17, against the torch-CPU oracle: every block and deepstack merger in
    isolation, and the whole-tower entry end to end."""
    rng = np.random.default_rng(3)
    frames = [rng.standard_normal((3, 512, 512)).astype(np.float32)]
    for _ in range(15):
        frames.append(frames[-1] + 0.1 * rng.standard_normal((3, 512, 512)).astype(np.float32))
    px, g = vt.patchify(np.stack(frames), patch=16, tpatch=2, merge=2)
    assert g.tolist() == [[8, 32, 32]]
    worst, line, tok = _baseline_full_depth(pkg, "2b", g.tolist(), px, seed=31)
    assert tuple(tok.shape) == (2048, 2048)
    print(f"\n[config 3, 24 blocks] worst block/merger in isolation {worst:.3e}; {line}", flush=True)


def test_config4_full_depth(pkg):
    """BASELINE config 4 at full depth: one 1344x1344 image (grid 1x84x84 = 7056 patches, one
    segment) on the 8B tower (head_dim 72, BASELINE weights), all 27 blocks and taps 8/16/24,
    against the torch-CPU oracle: every block and deepstack merger in isolation, and the
    whole-tower entry end to end (its attention runs the split work list on 256 CUs)."""
    grids = [(1, 84, 84)]
    worst, line, tok = _baseline_full_depth(pkg, "8b", grids, pixels(grids, 41), seed=32)
    assert tuple(tok.shape) == (1764, 4096)
    print(f"\n[config 4, 27 blocks] worst block/merger in isolation {worst:.3e}; {line}", flush=True)
