"""Shape robustness of the whole-tower entry: random grid lists (1-4 images or videos, even sides from
2 to 64 merge-block rows, temporal 1-3) through the bf16 tower (LayerNorms folded, the benchmarked
path) and the fp32 tower, on the 2B shape (head_dim 64) and the 8B shape (head_dim 72), three blocks
with checkpoint-like parameters and a deepstack tap, against the torch-CPU oracle. The token counts
land anywhere relative to the GEMM tiles (256 / 288 rows), the attention's 128-query tiles and 64-key
tiles, so every edge path of the tile plans, the three-stage operand ring and the work lists runs.
Bars: bf16 tokens and deepstack features within rel-L2 1e-2 of the oracle's bf16 mode, overall and
per image (measured 6.4e-3 to 7.4e-3 on MI355X); fp32 within 1e-5 of the oracle's fp32 mode, overall
and per image (measured 2.1e-6 to 2.4e-6: fp32 accumulation order only)."""
import numpy as np
import pytest

from oracle import torch_tower as tt
from tests.test_gpu_parity_depth import ckpt_params, pixels, rel_l2, specs, to_np

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def random_grids(seed):
    rng = np.random.default_rng(seed)
    grids = []
    for _ in range(int(rng.integers(1, 5))):
        t = int(rng.choice([1, 1, 2, 3]))
        h, w = (2 * int(v) for v in rng.integers(1, 33, size=2))
        grids.append((t, h, w))
    return grids


def per_image(got, want, grids, rows_per_patch_group):
    """rel-L2 of each image's rows (merged tokens: t*h*w/4 rows per image)."""
    out, r0 = [], 0
    for t, h, w in grids:
        n = t * h * w // rows_per_patch_group
        out.append(rel_l2(got[r0:r0 + n], want[r0:r0 + n]))
        r0 += n
    return out


@pytest.mark.parametrize("shape", ["2b", "8b"])
@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_tower_random_grids(pkg, shape, seed):
    grids = random_grids(100 * seed + (shape == "8b"))
    spec, ospec = specs(pkg, shape, depth=3, ds=(1,))
    params = ckpt_params(ospec, seed=seed)
    g = np.array(grids, np.int32)
    px = pixels(grids, seed)
    n = int(sum(t * h * w for t, h, w in grids))
    print(f"[random grids] {shape} seed {seed}: {grids} ({n} patches)", flush=True)
    for dtype, prec, tol, tol_img in (("bfloat16", "bf16", 1e-2, 1e-2), ("float32", "fp32", 1e-5, 1e-5)):
        ref = tt.TorchTower(params, ospec, prec).run(px, grids)
        tower = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(params)
        tok, ds = tower(px, g)
        want = [to_np(ref["tokens"]), *[to_np(t) for t in ref["deepstack"]]]
        got = [to_np(tok), *[to_np(t) for t in ds]]
        assert len(got) == len(want) == 2
        for name, a, b in zip(("tokens", "ds0"), got, want):
            assert a.shape == b.shape and np.isfinite(a).all(), (dtype, name)
            e = rel_l2(a, b)
            worst_img = max(per_image(a, b, grids, 4))
            print(f"  {dtype} {name}: {e:.3e} (worst image {worst_img:.3e})", flush=True)
            assert e <= tol, (dtype, name, e)
            assert worst_img <= tol_img, (dtype, name, worst_img)


def random_window_grids(seed):
    rng = np.random.default_rng(seed)
    grids = []
    for _ in range(int(rng.integers(1, 4))):
        t = int(rng.choice([1, 1, 2]))
        h, w = (2 * int(v) for v in rng.integers(1, 13, size=2))
        grids.append((t, h, w))
    return grids, int(rng.choice([64, 112]))


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_window_tower_random_grids(pkg, seed):
    """Window attention (blocks 0 and 2 windowed, 1 and 3 full) on random grid lists whose sides need
    not be multiples of the window (the reference's -100 padding of partial windows), bf16 and fp32,
    against the numpy oracle: bf16 within rel-L2 1e-2 of its bf16 mode (measured 5.1e-3 to 7.9e-3 on
    MI355X), fp32 within 1e-5 of fp64 (measured 2.0e-6 to 2.3e-6)."""
    from oracle import vision_tower as vt
    from tests.test_gpu_window import window_specs
    grids, window = random_window_grids(seed)
    spec, ospec = window_specs(pkg, window=window)
    params = pkg.random_params(spec, seed=seed)
    n = int(sum(t * h * w for t, h, w in grids))
    px = np.random.default_rng(seed).standard_normal((n, 1536), dtype=np.float32)
    g = np.array(grids, np.int32)
    print(f"[random window grids] seed {seed}: {grids}, window {window} ({n} patches)", flush=True)
    for dtype, prec, tol in (("bfloat16", "bf16", 1e-2), ("float32", "fp64", 1e-5)):
        ref = vt.encode_vision(params, px, grids, ospec, prec)
        tok, ds = pkg.Qwen3VisionTransformer(spec, dtype=dtype).bind(params)(px, g)
        for name, a, b in zip(("tokens", "ds0", "ds1"), [tok, *ds], [ref.tokens, *ref.deepstack]):
            e = rel_l2(to_np(a), b)
            print(f"  {dtype} {name}: {e:.3e}", flush=True)
            assert np.isfinite(to_np(a)).all() and e <= tol, (dtype, name, e)
