"""The allocation-free split attention entry (qvl_attention_headmajor_split_noalloc): its scratch is
a file-scope device array of the library, so the caller passes only inputs and outputs. Checked
bit-exact against the workspace entry (qvl_attention_headmajor_split) on the same split lists, on
two calls in a row (the second smaller, reusing the scratch the first left behind), and the
size limit is rejected with a clear error before anything launches."""
import ctypes as C

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _noalloc(lib):
    return lib.qvl_attention_headmajor_split_noalloc


def _case(pkg, lib, hd, cu, H, n_cus, seed):
    from tests.test_gpu_kernels import _headmajor_operands
    cu = np.array(cu, np.int32)
    q, k, vt, _ = _headmajor_operands(H, hd, cu, seed)
    split, n_whole = pkg.attention_worklist_split(cu, H, hd, n_cus)
    assert len(split) > n_whole
    return int(cu[-1]), q, k, vt, torch.from_numpy(np.ascontiguousarray(split)).to(DEV), len(split), n_whole


def test_noalloc_split_attention_matches_workspace_entry(pkg):
    cp = pkg.capi
    lib = cp.load()
    fn = _noalloc(lib)
    st = torch.cuda.current_stream().cuda_stream
    assert lib.qvl_noalloc_scratch_bytes() == 40 << 20
    # config 4's 7056-token segment at head_dim 72 (768 parts, 29 MB of scratch), then a smaller
    # ragged head_dim-64 list: the second call finds the first call's partials in the scratch
    cases = [(72, [0, 7056], 16, 256, 1), (64, [0, 1000, 1003, 5099, 5100], 4, 20, 2)]
    for hd, cu, H, n_cus, seed in cases:
        N, q, k, vt, items, n_items, n_whole = _case(pkg, lib, hd, cu, H, n_cus, seed)
        print(f"[no-alloc] hd={hd} N={N} H={H} items={n_items} parts={n_items - n_whole}", flush=True)
        nb = C.c_size_t()
        cp.check(lib.qvl_attention_split_workspace_size(hd, n_items, n_whole, C.byref(nb)))
        assert 0 < nb.value <= lib.qvl_noalloc_scratch_bytes()
        ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
        want = torch.full((N, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
        got = torch.full((N, H * hd), float("nan"), dtype=torch.bfloat16, device=DEV)
        cp.check(lib.qvl_attention_headmajor_split(st, cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(), vt.data_ptr(),
                                                   items.data_ptr(), n_items, n_whole, N, H, hd, want.data_ptr(),
                                                   H * hd, ws.data_ptr(), nb.value), "split")
        cp.check(fn(st, cp.QVL_DTYPE_BF16, q.data_ptr(), k.data_ptr(), vt.data_ptr(), items.data_ptr(), n_items,
                    n_whole, N, H, hd, got.data_ptr(), H * hd), "split_noalloc")
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, want), hd


def test_noalloc_split_attention_fp32_matches_workspace_entry(pkg):
    """The same entry on fp32 operands (qvl_attention_headmajor's fp32 layout: q, k [H][Np][hd],
    v^T [H][32 ceil(hd/32)][Np]): bit-exact against the workspace entry, on two calls in a row, the
    second smaller."""
    cp = pkg.capi
    lib = cp.load()
    fn = _noalloc(lib)
    st = torch.cuda.current_stream().cuda_stream
    cases = [(72, [0, 7056], 16, 256, 3), (64, [0, 1000, 1003, 5099, 5100], 4, 20, 4)]
    for hd, cu, H, n_cus, seed in cases:
        cu = np.array(cu, np.int32)
        N = int(cu[-1])
        Np = -(-N // 64) * 64
        g = torch.Generator(device="cpu").manual_seed(seed)
        q = (torch.randn((H, Np, hd), generator=g) * 0.2).to(DEV)
        k = torch.randn((H, Np, hd), generator=g).to(DEV)
        vt = torch.randn((H, -(-hd // 32) * 32, Np), generator=g).to(DEV)
        split, n_whole = pkg.attention_worklist_split(cu, H, hd, n_cus)
        assert len(split) > n_whole
        items = torch.from_numpy(np.ascontiguousarray(split)).to(DEV)
        n_items = len(split)
        print(f"[no-alloc fp32] hd={hd} N={N} H={H} items={n_items} parts={n_items - n_whole}", flush=True)
        nb = C.c_size_t()
        cp.check(lib.qvl_attention_split_workspace_size(hd, n_items, n_whole, C.byref(nb)))
        assert 0 < nb.value <= lib.qvl_noalloc_scratch_bytes()
        ws = torch.empty(nb.value, dtype=torch.uint8, device=DEV)
        want = torch.full((N, H * hd), float("nan"), dtype=torch.float32, device=DEV)
        got = torch.full((N, H * hd), float("nan"), dtype=torch.float32, device=DEV)
        cp.check(lib.qvl_attention_headmajor_split(st, cp.QVL_DTYPE_F32, q.data_ptr(), k.data_ptr(), vt.data_ptr(),
                                                   items.data_ptr(), n_items, n_whole, N, H, hd, want.data_ptr(),
                                                   H * hd, ws.data_ptr(), nb.value), "split fp32")
        cp.check(fn(st, cp.QVL_DTYPE_F32, q.data_ptr(), k.data_ptr(), vt.data_ptr(), items.data_ptr(), n_items,
                    n_whole, N, H, hd, got.data_ptr(), H * hd), "split_noalloc fp32")
        torch.cuda.synchronize()
        assert torch.isfinite(got).all()
        assert torch.equal(got, want), hd


def test_noalloc_rejects_lists_beyond_the_scratch(pkg):
    """A split list whose parts need more than the scratch holds is refused (QVL_ERR_WORKSPACE,
    naming the limit) before any launch; bad sizes keep the workspace entry's errors."""
    cp = pkg.capi
    lib = cp.load()
    fn = _noalloc(lib)
    st = torch.cuda.current_stream().cuda_stream
    buf = torch.zeros(4096, dtype=torch.bfloat16, device=DEV)
    p = buf.data_ptr()
    n_parts = (lib.qvl_noalloc_scratch_bytes() // (128 * 66 * 4)) + 1      # one part past the limit, head_dim 64
    rc = fn(st, cp.QVL_DTYPE_BF16, p, p, p, p, n_parts + 10, 10, 64, 1, 64, p, 64)
    assert rc == -4
    assert "maximum" in lib.qvl_last_error().decode()
    assert fn(st, cp.QVL_DTYPE_BF16, p, p, p, p, 5, 6, 64, 1, 64, p, 64) == -1      # n_whole > n_tiles
    assert fn(st, 99, p, p, p, p, 5, 5, 64, 1, 64, p, 64) == -2                     # unknown dtype
    torch.cuda.synchronize()
