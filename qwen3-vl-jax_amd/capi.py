"""ctypes binding of libqvl.so (the C ABI declared in include/qvl_vision.h).

Loading fails loudly when the library was not built: there is no CPU or eager fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqvl.so"

QVL_OK = 0
QVL_DTYPE_F32 = 0
QVL_DTYPE_BF16 = 1
QVL_EPI_BIAS = 0
QVL_EPI_BIAS_GELU = 1
QVL_EPI_BIAS_RESIDUAL = 2
QVL_SCATTER_SET = 0
QVL_SCATTER_ADD = 1

_p = C.c_void_p
_i64 = C.c_int64
_i32 = C.c_int32
_f32 = C.c_float
_sz = C.c_size_t
_pi32 = C.POINTER(C.c_int32)
_pf32 = C.POINTER(C.c_float)


class VisionConfig(C.Structure):
    _fields_ = [("hidden_size", _i32), ("out_hidden_size", _i32), ("depth", _i32), ("num_heads", _i32),
                ("intermediate_size", _i32), ("patch_volume", _i32), ("spatial_merge_size", _i32),
                ("num_position_embeddings", _i32), ("n_deepstack", _i32), ("deepstack_indexes", _i32 * 8),
                ("ln_eps", _f32), ("rope_theta", _f32), ("dtype", _i32), ("use_window", _i32),
                ("fullatt_mask", C.c_uint64)]


class LnFold(C.Structure):
    _fields_ = [("w", _p), ("cd", _p)]


class BlockWeights(C.Structure):
    _fields_ = [("norm1_w", _p), ("norm1_b", _p), ("norm2_w", _p), ("norm2_b", _p),
                ("qkv_w", _p), ("qkv_b", _p), ("proj_w", _p), ("proj_b", _p),
                ("fc1_w", _p), ("fc1_b", _p), ("fc2_w", _p), ("fc2_b", _p),
                ("qkv_ln", LnFold), ("fc1_ln", LnFold)]


class MergerWeights(C.Structure):
    _fields_ = [("norm_w", _p), ("norm_b", _p), ("fc1_w", _p), ("fc1_b", _p), ("fc2_w", _p), ("fc2_b", _p),
                ("fc1_ln", LnFold)]


class VisionWeights(C.Structure):
    _fields_ = [("patch_w", _p), ("patch_b", _p), ("pos_table", _p), ("blocks", C.POINTER(BlockWeights)),
                ("merger", MergerWeights), ("deepstack", C.POINTER(MergerWeights))]


class VisionMetadataDev(C.Structure):
    _fields_ = [("n_tokens", _i64), ("n_tiles", _i64), ("pos_hw", _p), ("tap_idx", _p), ("tap_w", _p),
                ("tiles", _p), ("n_window_tiles", _i64), ("window_tiles", _p), ("window_index", _p),
                ("window_reverse", _p), ("n_split_tiles", _i64), ("n_split_whole", _i64), ("split_tiles", _p),
                ("n_positions", _i64)]


# name -> (restype, argtypes); every function in include/qvl_vision.h
SIGNATURES = {
    "qvl_last_error": (C.c_char_p, []),
    "qvl_status_string": (C.c_char_p, [C.c_int]),
    "qvl_version": (C.c_int, []),
    "qvl_grid_counts": (C.c_int, [_pi32, _i64, _i32, C.POINTER(_i64), C.POINTER(_i64)]),
    "qvl_vision_metadata": (C.c_int, [_pi32, _i64, _i32, _i32, _i32, _pi32, _pi32, _pi32, _pf32]),
    "qvl_attention_worklist": (C.c_int, [_pi32, _i64, _i32, _pi32, _i64, C.POINTER(_i64)]),
    "qvl_attention_worklist_split": (C.c_int, [_pi32, _i64, _i32, _i32, _i32, _pi32, _i64, C.POINTER(_i64),
                                               C.POINTER(_i64)]),
    "qvl_rotary_inv_freq": (C.c_int, [_i32, _f32, _pf32]),
    "qvl_pack_dense_weight": (C.c_int, [_p, _i32, _p, _i64, _i64, _p]),
    "qvl_cast": (C.c_int, [_p, _i32, _p, _p, _i64]),
    "qvl_dense": (C.c_int, [_p, _i32, _i32, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64]),
    "qvl_set_gemm_plan": (C.c_int, [_i32, _i32, _i32]),
    "qvl_set_attention_plan": (C.c_int, [_i32]),
    "qvl_dense_workspace_size": (C.c_int, [C.POINTER(_sz)]),
    "qvl_dense_ws": (C.c_int, [_p, _i32, _i32, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _sz]),
    "qvl_layer_norm": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _i64, _i64, _i64, _f32]),
    "qvl_row_stats": (C.c_int, [_p, _i32, _p, _i64, _i64, _i64, _f32, _p]),
    "qvl_fold_ln_weight": (C.c_int, [_p, _i32, _p, _i64, _i64, _p, _p, _p, _p]),
    "qvl_dense_ln_ws": (C.c_int, [_p, _i32, _i32, _p, _i64, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p, _sz]),
    "qvl_dense_qkv_rotary_ln": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i64,
                                          _i64, _i32, _p, _sz]),
    "qvl_dense_rowstats_ws": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _p,
                                        _sz]),
    "qvl_dense_pos_embed_ws": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p,
                                         _p, _sz]),
    "qvl_dense_ln_parts_ws": (C.c_int, [_p, _i32, _i32, _p, _i64, _p, _p, _p, _i32, _f32, _p, _p, _i64, _i64, _i64,
                                        _i64, _p, _sz]),
    "qvl_dense_qkv_rotary_ln_parts": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _i32, _f32, _p, _p, _p, _p, _i32,
                                                _p, _p, _p, _i64, _i64, _i32, _p, _sz]),
    "qvl_pos_embed": (C.c_int, [_p, _i32, _p, _p, _p, _p, _i64, _i64]),
    "qvl_rotary_table": (C.c_int, [_p, _i32, _p, _i64, _i32, _f32, _p]),
    "qvl_vision_attention_workspace_size": (C.c_int, [_i32, _i64, _i32, _i32, C.POINTER(_sz)]),
    "qvl_vision_attention": (C.c_int, [_p, _i32, _p, _p, _p, _i64, _p, _p, _i64, _p, _i64, _i64, _i32, _i32,
                                       _p, _sz]),
    "qvl_dense_qkv_rotary": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _p, _p, _p, _i64, _i64, _i32, _p, _sz]),
    "qvl_rotary_pos_table": (C.c_int, [_p, _i32, _f32, _i32, _p]),
    "qvl_dense_qkv_rotary_pos": (C.c_int, [_p, _i32, _p, _i64, _p, _p, _p, _p, _i32, _p, _p, _p, _i64, _i64, _i32,
                                           _p, _sz]),
    "qvl_attention_headmajor": (C.c_int, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _p, _i64]),
    "qvl_attention_split_workspace_size": (C.c_int, [_i32, _i64, _i64, C.POINTER(_sz)]),
    "qvl_attention_headmajor_split": (C.c_int, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p, _i64,
                                                _p, _sz]),
    "qvl_noalloc_scratch_bytes": (_sz, []),
    "qvl_attention_headmajor_split_noalloc": (C.c_int, [_p, _i32, _p, _p, _p, _p, _i64, _i64, _i64, _i32, _i32, _p,
                                                        _i64]),
    "qvl_encode_vision_workspace_size": (C.c_int, [C.POINTER(VisionConfig), _i64, C.POINTER(_sz)]),
    "qvl_encode_vision": (C.c_int, [_p, C.POINTER(VisionConfig), C.POINTER(VisionWeights),
                                    C.POINTER(VisionMetadataDev), _p, _p, C.POINTER(_p), _p, _sz]),
    "qvl_window_metadata": (C.c_int, [_pi32, _i64, _i32, _i32, _i32, _pi32, _pi32, _i64, C.POINTER(_i64), _pi32]),
    "qvl_gather_rows": (C.c_int, [_p, _i32, _p, _i64, _i32, _p, _i64, _p, _i64, _i32, _i64]),
    "qvl_patchify": (C.c_int, [_p, _i32, _p, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _p, _i64]),
    "qvl_vision_positions": (C.c_int, [_p, _p, _i64, _i64, _i32, _i64, _p, _p]),
    "qvl_scatter_vision_rows": (C.c_int, [_p, _i32, _i32, _p, _i64, _i64, _i64, _i32, _p, _i64, _i64, _p, _p]),
}


class QVLError(RuntimeError):
    pass


_LIB = None


def load(path: Path | str | None = None):
    """Load libqvl.so and attach prototypes. Raises if the library is missing."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise QVLError(f"{p} not found: build it first (python __graft_entry__.py build, or "
                       f"python qwen3-vl-jax_amd/build.py). There is no CPU fallback.")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str = "") -> None:
    if rc != QVL_OK:
        lib = load()
        msg = lib.qvl_last_error().decode(errors="replace")
        raise QVLError(f"{what}: {lib.qvl_status_string(rc).decode()} ({rc}): {msg}")


def call(name: str, *args):
    rc = getattr(load(), name)(*args)
    check(rc, name)
    return rc
