"""Host-side mirror of the reference's vision-tower interface, running on libqvl (HIP, gfx950).

Mirrors /root/reference/model.py:
  VisionEmbeddings              27-64    output pytree (tokens + deepstack), concatenate/cast/with_batch_dim
  VisionBackboneSpec            84-98    shape/config
  Qwen3VisionTransformer        659-851  the tower; `__call__(pixel_values, grid_thw) -> (tokens, deepstack)`
  Qwen3VLModel.encode_vision    940-944  `apply({"params": params}, pixel_values, grid_thw, method="encode_vision")`

Parameters use the reference's Flax tree (`{"visual": {"patch_embed": {"proj": {"kernel", "bias"}}, ...}}`,
kernels [in, out]); they are packed once onto the device ([out, in] in the tower dtype, zero-padded to 64) when
the tower is bound to them. torch supplies device memory and the stream; every computation is a
libqvl kernel launched through the C ABI (no torch math on the product path).
"""
from __future__ import annotations

import ctypes as C
from collections import OrderedDict
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from . import capi


def _torch():
    import torch
    return torch


# ---------------------------------------------------------------------------------------------
# spec (model.py:84-98) and the two BASELINE shapes
# ---------------------------------------------------------------------------------------------
@dataclass
class VisionBackboneSpec:
    hidden_size: int
    out_hidden_size: int
    depth: int
    num_heads: int
    intermediate_size: int
    patch_size: int = 16
    temporal_patch_size: int = 2
    spatial_merge_size: int = 2
    window_size: int = 32
    in_channels: int = 3
    # None = every block (what spec_from_config fixes for qwen3_vl, model.py:1033-1034); a list
    # that misses blocks selects the window-attention path for them (model.py:808-850).
    fullatt_block_indexes: Optional[Sequence[int]] = None
    num_position_embeddings: Optional[int] = 2304
    deepstack_visual_indexes: Sequence[int] = ()

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def use_window(self) -> bool:
        """model.py:809-810: window attention when the full-attention set is smaller than the depth."""
        fa = self.fullatt_block_indexes
        return fa is not None and len(set(fa)) < self.depth

    @property
    def patch_volume(self) -> int:
        return self.in_channels * self.temporal_patch_size * self.patch_size ** 2


@dataclass
class TextBackboneSpec:
    """The reference's text spec (model.py:67-81). The text decoder is outside this build; the spec
    is parsed (with the reference's key lookups and errors) so that `Qwen3VLSpec` and
    `spec_from_config` keep the reference's shape."""
    hidden_size: int
    num_attention_heads: int
    num_hidden_layers: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    rope_theta: float
    rope_section: Sequence[int]
    rope_scaling_type: Optional[str]
    rope_scaling_factor: Optional[float]
    mrope_interleaved: bool
    rms_norm_eps: float
    vocab_size: int


@dataclass
class Qwen3VLSpec:
    """The reference's model spec (model.py:101-107): text spec, optional vision spec, token ids."""
    text: Optional[TextBackboneSpec]
    vision: Optional[VisionBackboneSpec]
    pad_token_id: Optional[int] = None
    bos_token_id: Optional[int] = None
    eos_token_id: Optional[int] = None


def vision_spec_from_config(vision_cfg: Optional[Dict]) -> Optional[VisionBackboneSpec]:
    """The vision branch of spec_from_config (model.py:1027-1043), same keys, fallbacks and
    defaults: patch_size | spatial_patch_size; temporal_patch_size | temporal_patch | 1;
    window_size | patch_size * spatial_merge_size; in_channels | in_chans | 3;
    fullatt_block_indexes | deepstack_visual_indexes | [], forced to every block when the config's
    model_type is exactly "qwen3_vl" (model.py:1033-1034; other model types, e.g. transformers'
    "qwen3_vl_vision", keep the generic rule, as in the reference);
    num_position_embeddings None when absent. An empty or missing config gives None."""
    if not vision_cfg:
        return None
    patch = vision_cfg.get("patch_size", vision_cfg.get("spatial_patch_size"))
    temporal = vision_cfg.get("temporal_patch_size", vision_cfg.get("temporal_patch", 1))
    window = vision_cfg.get("window_size", patch * vision_cfg.get("spatial_merge_size", 1))
    fullatt = vision_cfg.get("fullatt_block_indexes", vision_cfg.get("deepstack_visual_indexes", []))
    if vision_cfg.get("model_type") == "qwen3_vl":
        fullatt = list(range(vision_cfg["depth"]))
    return VisionBackboneSpec(
        hidden_size=vision_cfg["hidden_size"], out_hidden_size=vision_cfg["out_hidden_size"],
        depth=vision_cfg["depth"], num_heads=vision_cfg["num_heads"],
        intermediate_size=vision_cfg["intermediate_size"], patch_size=patch, temporal_patch_size=temporal,
        spatial_merge_size=vision_cfg["spatial_merge_size"], window_size=window,
        in_channels=vision_cfg.get("in_channels", vision_cfg.get("in_chans", 3)),
        fullatt_block_indexes=tuple(fullatt),
        num_position_embeddings=vision_cfg.get("num_position_embeddings"),
        deepstack_visual_indexes=tuple(vision_cfg.get("deepstack_visual_indexes", [])))


def spec_from_config(cfg: Dict) -> Qwen3VLSpec:
    """HF `config.json` dict -> Qwen3VLSpec (model.py:987-1049), with the reference's lookups,
    defaults and errors: head_dim = text head_dim or hidden_size // num_attention_heads; a
    `vision_config` key (even an empty one) without `rope_scaling.mrope_section` is rejected; a
    vision model's section must have 3 entries; unless `mrope_interleaved`, the section must sum
    to head_dim // 2 (model.py:1000-1009); missing text keys raise KeyError as there."""
    text_cfg = cfg.get("text_config", cfg)
    rope_cfg = text_cfg.get("rope_scaling", cfg.get("rope_scaling", {}))
    head_dim = text_cfg.get("head_dim") or text_cfg["hidden_size"] // text_cfg["num_attention_heads"]
    vision_cfg = cfg.get("vision_config")
    is_dict = isinstance(rope_cfg, dict)
    rope_type = rope_cfg.get("type") if is_dict else None
    rope_factor = rope_cfg.get("factor", rope_cfg.get("finetuned_factor")) if is_dict else None
    interleaved = bool(rope_cfg.get("mrope_interleaved", False)) if is_dict else False
    raw_section = rope_cfg.get("mrope_section") if is_dict else None
    if raw_section is None:
        if vision_cfg is not None:
            raise ValueError("Missing rope_scaling.mrope_section for vision model")
        section = [head_dim // 2]
    else:
        section = [int(x) for x in raw_section]
        if vision_cfg and len(section) != 3:
            raise ValueError("mrope_section must have 3 entries for vision models")
        if not interleaved and sum(section) != head_dim // 2:
            raise ValueError(f"mrope_section sum must equal head_dim//2 ({head_dim // 2})")
    text = TextBackboneSpec(
        hidden_size=text_cfg["hidden_size"], num_attention_heads=text_cfg["num_attention_heads"],
        num_hidden_layers=text_cfg["num_hidden_layers"], num_key_value_heads=text_cfg["num_key_value_heads"],
        head_dim=head_dim, intermediate_size=text_cfg["intermediate_size"],
        rope_theta=text_cfg.get("rope_theta", cfg.get("rope_theta", 10000.0)), rope_section=section,
        rope_scaling_type=rope_type, rope_scaling_factor=float(rope_factor) if rope_factor else None,
        mrope_interleaved=interleaved, rms_norm_eps=text_cfg["rms_norm_eps"], vocab_size=text_cfg["vocab_size"])
    return Qwen3VLSpec(text=text, vision=vision_spec_from_config(vision_cfg), pad_token_id=cfg.get("pad_token_id"),
                       bos_token_id=cfg.get("bos_token_id"), eos_token_id=cfg.get("eos_token_id"))


def spec_2b() -> VisionBackboneSpec:
    """Qwen3-VL-2B vision tower shape."""
    return VisionBackboneSpec(hidden_size=1024, out_hidden_size=2048, depth=24, num_heads=16, intermediate_size=4096,
                              fullatt_block_indexes=tuple(range(24)), deepstack_visual_indexes=(5, 11, 17))


def spec_8b() -> VisionBackboneSpec:
    """Qwen3-VL-8B vision tower shape."""
    return VisionBackboneSpec(hidden_size=1152, out_hidden_size=4096, depth=27, num_heads=16, intermediate_size=4304,
                              fullatt_block_indexes=tuple(range(27)), deepstack_visual_indexes=(8, 16, 24))


def random_params(spec: VisionBackboneSpec, seed: int = 0, std: float = 0.02) -> Dict:
    """Random-init Flax-tree params: Dense kernels and the pos-embed table N(0, std), biases 0,
    LayerNorm weight 1 / bias 0 (the BASELINE synthetic-weights recipe)."""
    rng = np.random.default_rng(seed)
    D, I, Do = spec.hidden_size, spec.intermediate_size, spec.out_hidden_size
    M4 = D * spec.spatial_merge_size ** 2

    def dense(i, o):
        return {"kernel": (rng.standard_normal((i, o), dtype=np.float32) * np.float32(std)),
                "bias": np.zeros(o, np.float32)}

    def ln(d):
        return {"weight": np.ones(d, np.float32), "bias": np.zeros(d, np.float32)}

    v = {"patch_embed": {"proj": dense(spec.patch_volume, D)}}
    if spec.num_position_embeddings:
        v["pos_embed"] = {"embedding": rng.standard_normal((spec.num_position_embeddings, D),
                                                           dtype=np.float32) * np.float32(std)}
    for i in range(spec.depth):
        v[f"blocks_{i}"] = {"norm1": ln(D), "norm2": ln(D),
                            "attn": {"qkv": dense(D, 3 * D), "proj": dense(D, D)},
                            "mlp": {"linear_fc1": dense(D, I), "linear_fc2": dense(I, D)}}
    v["merger"] = {"norm": ln(D), "linear_fc1": dense(M4, M4), "linear_fc2": dense(M4, Do)}
    for j in range(len(spec.deepstack_visual_indexes)):
        v[f"deepstack_mergers_{j}"] = {"norm": ln(M4), "linear_fc1": dense(M4, M4), "linear_fc2": dense(M4, Do)}
    return {"visual": v}


# ---------------------------------------------------------------------------------------------
# VisionEmbeddings (model.py:27-64)
# ---------------------------------------------------------------------------------------------
@dataclass
class VisionEmbeddings:
    """Container for vision tower outputs: tokens [N/4, Dout] + deepstack features."""
    tokens: "object"
    deepstack: Tuple = ()

    @classmethod
    def concatenate(cls, embeds: Sequence["VisionEmbeddings"]) -> "VisionEmbeddings":
        torch = _torch()
        if not embeds:
            return cls(tokens=torch.zeros((0, 0), dtype=torch.float32), deepstack=())
        base = len(embeds[0].deepstack)
        for e in embeds[1:]:
            if len(e.deepstack) != base:
                raise ValueError("All VisionEmbeddings must have same deepstack length")
        return cls(tokens=torch.cat([e.tokens for e in embeds], 0),
                   deepstack=tuple(torch.cat([e.deepstack[i] for e in embeds], 0) for i in range(base)))

    def cast(self, dtype) -> "VisionEmbeddings":
        return VisionEmbeddings(tokens=self.tokens.to(dtype), deepstack=tuple(f.to(dtype) for f in self.deepstack))

    def with_batch_dim(self, batch: int) -> "VisionEmbeddings":
        tokens = self.tokens if self.tokens.ndim == 3 else self.tokens[None, ...]
        if tokens.shape[0] == 1 and batch > 1:
            tokens = tokens.repeat(batch, 1, 1)
        ds = []
        for f in self.deepstack:
            f = f if f.ndim == 3 else f[None, ...]
            if f.shape[0] == 1 and batch > 1:
                f = f.repeat(batch, 1, 1)
            ds.append(f)
        return VisionEmbeddings(tokens=tokens, deepstack=tuple(ds))


# ---------------------------------------------------------------------------------------------
# host metadata (C ABI)
# ---------------------------------------------------------------------------------------------
def _i32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int32))


def _f32p(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_float))


@dataclass
class GridMetadata:
    """Host integer metadata of one grid_thw (qvl_vision_metadata + qvl_attention_worklist)."""
    n_tokens: int
    cu_seqlens: np.ndarray
    pos_hw: np.ndarray
    tap_idx: np.ndarray
    tap_w: np.ndarray
    tiles: np.ndarray
    # window mode only (model.py:769-799, 808-830): pos_hw / tap_* above are then in window order
    # and `tiles` is the worklist of cu_full
    window_index: Optional[np.ndarray] = None
    window_reverse: Optional[np.ndarray] = None
    cu_window: Optional[np.ndarray] = None
    cu_full: Optional[np.ndarray] = None
    window_tiles: Optional[np.ndarray] = None
    n_positions: int = 0          # 1 + the largest rotary (h, w) id: max over grids of max(h, w)


def _worklist_capacity(cu: np.ndarray, num_heads: int, extra: int = 0) -> int:
    """An upper bound on a work list's length, so that one call fills it: the padded list holds
    8 queues of at most every (segment, head) group's query tiles each, plus `extra` parts."""
    lens = np.diff(cu.astype(np.int64))
    tiles = int(((np.maximum(lens, 0) + 127) // 128).sum()) * num_heads
    return 8 * max(tiles, 1) + extra


def _worklist(lib, cu: np.ndarray, num_heads: int) -> np.ndarray:
    cu = np.ascontiguousarray(cu, np.int32)
    n = C.c_int64()
    cap = _worklist_capacity(cu, num_heads)
    tiles = np.empty((cap, 4), np.int32)          # the first n items are written
    capi.check(lib.qvl_attention_worklist(_i32p(cu), len(cu) - 1, num_heads, _i32p(tiles), cap, C.byref(n)),
               "qvl_attention_worklist")
    return tiles[: n.value]


def attention_worklist_split(cu: np.ndarray, num_heads: int, head_dim: int, n_cus: int) -> Tuple[np.ndarray, int]:
    """(items, n_whole) of qvl_attention_worklist_split: the work list of `cu` with the items of
    the last, partial round of workgroup slots on `n_cus` compute units split along their keys."""
    lib = capi.load()
    cu = np.ascontiguousarray(cu, np.int32)
    n, nw = C.c_int64(), C.c_int64()
    cap = _worklist_capacity(cu, num_heads, extra=4 * max(int(n_cus), 0))   # parts: at most one per slot
    items = np.empty((cap, 4), np.int32)          # the first n items are written
    capi.check(lib.qvl_attention_worklist_split(_i32p(cu), len(cu) - 1, num_heads, head_dim, n_cus, _i32p(items),
                                                cap, C.byref(n), C.byref(nw)), "qvl_attention_worklist_split")
    return items[: n.value], nw.value


def window_metadata(grid_thw, merge: int = 2, patch_size: int = 16, window_size: int = 32):
    """(window_index [N/merge^2], cu_window, cu_full) of `_get_window_index` and the window path's
    full-attention cu_seqlens (model.py:769-799, 828-830), from qvl_window_metadata."""
    g = np.ascontiguousarray(np.asarray(grid_thw, dtype=np.int32).reshape(-1, 3))
    lib = capi.load()
    nt = C.c_int64()
    capi.check(lib.qvl_grid_counts(_i32p(g), g.shape[0], merge, C.byref(nt), None), "qvl_grid_counts")
    ncu = C.c_int64()
    capi.check(lib.qvl_window_metadata(_i32p(g), g.shape[0], merge, patch_size, window_size, None, None, 0,
                                       C.byref(ncu), None), "qvl_window_metadata")
    widx = np.zeros(max(nt.value // (merge * merge), 1), np.int32)
    cuw = np.zeros(ncu.value, np.int32)
    cuf = np.zeros(g.shape[0] + 1, np.int32)
    capi.check(lib.qvl_window_metadata(_i32p(g), g.shape[0], merge, patch_size, window_size, _i32p(widx), _i32p(cuw),
                                       ncu.value, C.byref(ncu), _i32p(cuf)), "qvl_window_metadata")
    return widx[: nt.value // (merge * merge)], cuw, cuf


def grid_metadata(grid_thw, merge: int = 2, num_position_embeddings: Optional[int] = 2304,
                  dtype: int = capi.QVL_DTYPE_BF16, num_heads: int = 16) -> GridMetadata:
    """Integer metadata of one grid_thw. Without a learned pos-embed table
    (num_position_embeddings None or 0, model.py:676-680) the taps are zeros and unused."""
    g = np.ascontiguousarray(np.asarray(grid_thw, dtype=np.int32).reshape(-1, 3))
    lib = capi.load()
    nt, ns = C.c_int64(), C.c_int64()
    capi.check(lib.qvl_grid_counts(_i32p(g), g.shape[0], merge, C.byref(nt), C.byref(ns)), "qvl_grid_counts")
    N, S = nt.value, ns.value
    npos = int(num_position_embeddings or 0)
    # (qvl_vision_metadata writes every entry of cu and pos, and of the taps when the spec has a
    # pos-embed table; without one they stay zeros, unused)
    cu = np.empty(S + 1, np.int32)
    pos = np.empty((N, 2), np.int32)
    idx = np.empty((4, N), np.int32) if npos else np.zeros((4, N), np.int32)
    w = np.empty((4, N), np.float32) if npos else np.zeros((4, N), np.float32)
    capi.check(lib.qvl_vision_metadata(_i32p(g), g.shape[0], merge, npos, dtype, _i32p(cu), _i32p(pos),
                                       _i32p(idx) if npos else None, _f32p(w) if npos else None),
               "qvl_vision_metadata")
    n_pos = int(g[:, 1:].max()) if len(g) else 0
    return GridMetadata(N, cu, pos, idx, w, _worklist(lib, cu, num_heads), n_positions=n_pos)


def window_grid_metadata(m: GridMetadata, grid_thw, merge: int, patch_size: int, window_size: int,
                         num_heads: int) -> GridMetadata:
    """`m` re-expressed for the window path: per-token metadata in window order (the reference
    shuffles x and the rotary ids by merge groups, model.py:809-812), the worklists of cu_full and
    cu_window, and the unshuffle index argsort(window_index) (model.py:845-848)."""
    lib = capi.load()
    widx, cuw, cuf = window_metadata(grid_thw, merge, patch_size, window_size)
    mm = merge * merge
    perm = (widx.astype(np.int64)[:, None] * mm + np.arange(mm)[None, :]).reshape(-1)
    rev = np.argsort(widx, kind="stable").astype(np.int32)
    return GridMetadata(m.n_tokens, m.cu_seqlens, np.ascontiguousarray(m.pos_hw[perm]),
                        np.ascontiguousarray(m.tap_idx[:, perm]), np.ascontiguousarray(m.tap_w[:, perm]),
                        _worklist(lib, cuf, num_heads), widx, rev, cuw, cuf, _worklist(lib, cuw, num_heads),
                        n_positions=m.n_positions)


# ---------------------------------------------------------------------------------------------
# the tower (model.py:659-851)
# ---------------------------------------------------------------------------------------------
def _ptr(t) -> int:
    return t.data_ptr() if t is not None else 0


def _to_device_packed(arrays: Dict[str, np.ndarray], device) -> Dict[str, object]:
    """Copy 4-byte host arrays (int32 / float32) to the device in one transfer: packed into one
    int32 buffer at 256-byte-aligned offsets, returned as device views of their shapes and dtypes
    (the views share the one device allocation)."""
    torch = _torch()
    offs, total = {}, 0
    for name, a in arrays.items():
        if a.dtype.itemsize != 4:
            raise TypeError(f"{name}: {a.dtype} (4-byte elements expected)")
        offs[name] = total
        total += -(-a.size // 64) * 64
    buf = np.zeros(max(total, 64), np.int32)
    for name, a in arrays.items():
        buf[offs[name]: offs[name] + a.size] = np.ascontiguousarray(a).reshape(-1).view(np.int32)
    dev = torch.from_numpy(buf).to(device)
    out = {}
    for name, a in arrays.items():
        v = dev[offs[name]: offs[name] + a.size].view(a.shape)
        out[name] = v.view(torch.float32) if a.dtype == np.float32 else v
    return out


class Qwen3VisionTransformer:
    """The vision tower on libqvl. Bind params once (`bind`), then call like the reference module:
    `tokens, deepstack = tower(pixel_values, grid_thw)`. `dtype` defaults to float32, as the
    reference module's does (model.py:661); "bfloat16" is the reference's bf16 tower."""

    META_CACHE_SIZE = 16   # grids whose device metadata stays cached (LRU)
    SPLIT_MIN_KEYS_BF16 = 2048   # the bf16 tower runs split attention lists from this segment length

    def __init__(self, spec: VisionBackboneSpec, dtype: str = "float32", device: str = "cuda:0",
                 split_attention: bool = True, ln_fold: bool = True):
        if dtype not in ("bfloat16", "float32"):
            raise NotImplementedError(f"dtype {dtype!r}: the tower runs in bfloat16 or float32")
        if spec.spatial_merge_size != 2:
            raise NotImplementedError("spatial_merge_size must be 2")
        self.spec = spec
        self.dtype = dtype
        self.qdtype = capi.QVL_DTYPE_BF16 if dtype == "bfloat16" else capi.QVL_DTYPE_F32
        self.device = device
        # bf16 full attention runs a qvl_attention_worklist_split list (the last round's items split
        # along keys) when true
        self.split_attention = split_attention
        # ln_fold (bf16, the default): each block's norm1 / norm2 and the deepstack mergers'
        # post-shuffle norms are folded into the Dense after them (qvl_fold_ln_weight at bind time);
        # at run time the residual Dense that writes x also writes its row statistics as 128-column
        # partials and the folded Dense combines them, so no LayerNorm runs between the GEMMs
        # (same-box A/Bs at config 2: 16.31 vs 16.47 and 16.06 vs 16.14 ms per forward). The fold
        # rounds bf16(gamma W) where the reference rounds the LayerNorm output (within the bf16
        # tolerances). ln_fold=False runs the reference's LayerNorm launches.
        self.ln_fold = bool(ln_fold) and self.qdtype == capi.QVL_DTYPE_BF16
        self._folds: Dict[str, tuple] = {}
        self._lib = capi.load()
        self._w = None
        self._keep = []
        self._state: Dict[str, object] = {}
        # per-grid device metadata, least recently used first (at most META_CACHE_SIZE grids)
        self._meta_cache: "OrderedDict[tuple, tuple]" = OrderedDict()
        self._ws = None
        cfg = capi.VisionConfig()
        cfg.hidden_size = spec.hidden_size
        cfg.out_hidden_size = spec.out_hidden_size
        cfg.depth = spec.depth
        cfg.num_heads = spec.num_heads
        cfg.intermediate_size = spec.intermediate_size
        cfg.patch_volume = spec.patch_volume
        cfg.spatial_merge_size = spec.spatial_merge_size
        cfg.num_position_embeddings = spec.num_position_embeddings or 0
        ds = tuple(spec.deepstack_visual_indexes)
        if len(ds) > 8:
            raise ValueError("at most 8 deepstack taps")
        cfg.n_deepstack = len(ds)
        for j, d in enumerate(ds):
            cfg.deepstack_indexes[j] = d
        cfg.ln_eps = 1e-6
        cfg.rope_theta = 10000.0
        cfg.dtype = self.qdtype
        if spec.use_window:
            if spec.depth > 64:
                raise NotImplementedError("window attention with depth > 64")
            cfg.use_window = 1
            cfg.fullatt_mask = sum(1 << i for i in set(spec.fullatt_block_indexes) if 0 <= i < spec.depth)
        self._cfg = cfg

    # -- weights --------------------------------------------------------------------------------
    def _stream(self):
        return _torch().cuda.current_stream().cuda_stream

    def _tdtype(self):
        """torch dtype of the tower's activations, packed weights and outputs."""
        torch = _torch()
        return torch.bfloat16 if self.qdtype == capi.QVL_DTYPE_BF16 else torch.float32

    def _round(self, t):
        """Values as the tower dtype holds them (bf16 rounding in the bf16 mode), kept in fp32."""
        torch = _torch()
        return t.to(torch.bfloat16).to(torch.float32) if self.qdtype == capi.QVL_DTYPE_BF16 else t

    def _pack_dense(self, p):
        """Flax Dense {kernel [in, out], bias [out]} -> (packed [n_pad, k_pad] weight, bias [n_pad])."""
        torch = _torch()
        k = np.ascontiguousarray(np.asarray(p["kernel"], np.float32))
        kin, nout = k.shape
        kp, npad = -(-kin // 64) * 64, -(-nout // 64) * 64
        src = torch.from_numpy(k).to(self.device)
        out = torch.empty((npad, kp), dtype=self._tdtype(), device=self.device)
        capi.check(self._lib.qvl_pack_dense_weight(self._stream(), self.qdtype, src.data_ptr(), kin, nout,
                                                   out.data_ptr()), "qvl_pack_dense_weight")
        b = np.zeros(npad, np.float32)
        b[:nout] = np.asarray(p["bias"], np.float32)
        return out, self._round(torch.from_numpy(b).to(self.device))

    def _fold(self, w, gamma, beta):
        """(W', cd) of a LayerNorm (gamma, beta) folded into the packed Dense kernel w [n_pad, k]:
        W' = bf16(gamma * W) and (c, d) per output feature (qvl_fold_ln_weight)."""
        torch = _torch()
        n_pad, k = w.shape
        out = torch.empty_like(w)
        cd = torch.empty((n_pad, 2), dtype=torch.float32, device=self.device)
        capi.check(self._lib.qvl_fold_ln_weight(self._stream(), self.qdtype, w.data_ptr(), k, n_pad, gamma.data_ptr(),
                                                beta.data_ptr(), out.data_ptr(), cd.data_ptr()), "qvl_fold_ln_weight")
        return out, cd

    def _vec(self, v):
        torch = _torch()
        t = torch.from_numpy(np.ascontiguousarray(np.asarray(v, np.float32))).to(self.device)
        return self._round(t)                             # LayerNorm params live in the tower dtype

    def bind(self, params: Dict) -> "Qwen3VisionTransformer":
        """Pack a Flax-tree param dict onto the device (load-time, model.py:1105-1160 layout)."""
        torch = _torch()
        v = params.get("visual", params)
        s = self.spec
        st: Dict[str, object] = {}

        def dense(name, p):
            st[name + ".w"], st[name + ".b"] = self._pack_dense(p)

        dense("patch_embed", v["patch_embed"]["proj"])
        if s.num_position_embeddings:
            st["pos_table"] = torch.from_numpy(np.ascontiguousarray(v["pos_embed"]["embedding"], np.float32)).to(
                self.device).to(self._tdtype()).contiguous()
        for i in range(s.depth):
            b = v[f"blocks_{i}"]
            for n in ("norm1", "norm2"):
                st[f"blocks.{i}.{n}.w"], st[f"blocks.{i}.{n}.b"] = self._vec(b[n]["weight"]), self._vec(b[n]["bias"])
            for name, key in (("qkv", ("attn", "qkv")), ("proj", ("attn", "proj")),
                              ("fc1", ("mlp", "linear_fc1")), ("fc2", ("mlp", "linear_fc2"))):
                dense(f"blocks.{i}.{name}", b[key[0]][key[1]])
        mergers = [("merger", v["merger"])] + [(f"deepstack.{j}", v[f"deepstack_mergers_{j}"])
                                               for j in range(len(s.deepstack_visual_indexes))]
        for name, m in mergers:
            st[name + ".norm.w"], st[name + ".norm.b"] = self._vec(m["norm"]["weight"]), self._vec(m["norm"]["bias"])
            dense(name + ".fc1", m["linear_fc1"])
            dense(name + ".fc2", m["linear_fc2"])
        torch.cuda.current_stream().synchronize()
        return self._bind_state(st)

    def packed_state(self) -> Dict[str, object]:
        """The bound device buffers by name (packed weights, biases, LayerNorm params, pos table)."""
        if self._w is None:
            raise RuntimeError("tower is not bound")
        return dict(self._state)

    def expected_packed_shapes(self) -> Dict[str, Tuple[Tuple[int, ...], str]]:
        """name -> (shape, "w" for tower-dtype buffers | "f" for fp32 vectors) of a bound tower."""
        s = self.spec
        r64 = lambda x: -(-x // 64) * 64
        D, I, PV, Do = s.hidden_size, s.intermediate_size, s.patch_volume, s.out_hidden_size
        M4 = D * s.spatial_merge_size ** 2
        out = {}

        def dense(name, kin, nout):
            out[name + ".w"] = ((r64(nout), r64(kin)), "w")
            out[name + ".b"] = ((r64(nout),), "f")

        dense("patch_embed", PV, D)
        if s.num_position_embeddings:
            out["pos_table"] = ((s.num_position_embeddings, D), "w")
        for i in range(s.depth):
            for n in ("norm1", "norm2"):
                out[f"blocks.{i}.{n}.w"], out[f"blocks.{i}.{n}.b"] = ((D,), "f"), ((D,), "f")
            dense(f"blocks.{i}.qkv", D, 3 * D)
            dense(f"blocks.{i}.proj", D, D)
            dense(f"blocks.{i}.fc1", D, I)
            dense(f"blocks.{i}.fc2", I, D)
        for j, name in enumerate(["merger"] + [f"deepstack.{k}" for k in range(len(s.deepstack_visual_indexes))]):
            nd = D if j == 0 else M4
            out[name + ".norm.w"], out[name + ".norm.b"] = ((nd,), "f"), ((nd,), "f")
            dense(name + ".fc1", M4, M4)
            dense(name + ".fc2", M4, Do)
        return out

    def bind_packed(self, state: Dict[str, object]) -> "Qwen3VisionTransformer":
        """Bind already-packed device buffers (e.g. `load_packed`), checking every name, shape and
        dtype against this tower's spec and dtype; no packing kernels run."""
        torch = _torch()
        exp = self.expected_packed_shapes()
        missing = sorted(set(exp) - set(state))
        extra = sorted(set(state) - set(exp))
        if missing or extra:
            raise ValueError(f"packed state mismatch: missing {missing[:4]}, unexpected {extra[:4]}")
        st = {}
        for name, (shape, kind) in exp.items():
            t = state[name]
            want = self._tdtype() if kind == "w" else torch.float32
            if tuple(t.shape) != shape or t.dtype != want:
                raise ValueError(f"{name}: {tuple(t.shape)} {t.dtype}, expected {shape} {want}")
            st[name] = t.to(self.device).contiguous()
        return self._bind_state(st)

    def _bind_state(self, st: Dict[str, object]) -> "Qwen3VisionTransformer":
        s = self.spec
        p = lambda name: st[name].data_ptr()
        W = capi.VisionWeights()
        W.patch_w, W.patch_b = p("patch_embed.w"), p("patch_embed.b")
        W.pos_table = p("pos_table") if "pos_table" in st else None
        blocks = (capi.BlockWeights * s.depth)()
        for i in range(s.depth):
            bw = blocks[i]
            bw.norm1_w, bw.norm1_b = p(f"blocks.{i}.norm1.w"), p(f"blocks.{i}.norm1.b")
            bw.norm2_w, bw.norm2_b = p(f"blocks.{i}.norm2.w"), p(f"blocks.{i}.norm2.b")
            for name in ("qkv", "proj", "fc1", "fc2"):
                setattr(bw, name + "_w", p(f"blocks.{i}.{name}.w"))
                setattr(bw, name + "_b", p(f"blocks.{i}.{name}.b"))
        W.blocks = blocks
        folds: Dict[str, tuple] = {}
        if self.ln_fold:
            for i in range(s.depth):
                for name, norm in (("qkv", "norm1"), ("fc1", "norm2")):
                    f = self._fold(st[f"blocks.{i}.{name}.w"], st[f"blocks.{i}.{norm}.w"], st[f"blocks.{i}.{norm}.b"])
                    folds[f"blocks.{i}.{name}"] = f
                    fl = getattr(blocks[i], name + "_ln")
                    fl.w, fl.cd = f[0].data_ptr(), f[1].data_ptr()
            for j in range(len(s.deepstack_visual_indexes)):
                folds[f"deepstack.{j}.fc1"] = self._fold(st[f"deepstack.{j}.fc1.w"], st[f"deepstack.{j}.norm.w"],
                                                         st[f"deepstack.{j}.norm.b"])

        def merger(name):
            mw = capi.MergerWeights()
            mw.norm_w, mw.norm_b = p(name + ".norm.w"), p(name + ".norm.b")
            mw.fc1_w, mw.fc1_b, mw.fc2_w, mw.fc2_b = p(name + ".fc1.w"), p(name + ".fc1.b"), p(name + ".fc2.w"), p(
                name + ".fc2.b")
            if name + ".fc1" in folds:
                mw.fc1_ln.w, mw.fc1_ln.cd = folds[name + ".fc1"][0].data_ptr(), folds[name + ".fc1"][1].data_ptr()
            return mw

        W.merger = merger("merger")
        nds = len(s.deepstack_visual_indexes)
        ds = (capi.MergerWeights * max(nds, 1))()
        for j in range(nds):
            ds[j] = merger(f"deepstack.{j}")
        W.deepstack = ds
        self._state = st
        self._folds = folds
        self._keep = list(st.values()) + [t for f in folds.values() for t in f]
        self._blocks_arr, self._ds_arr = blocks, ds
        self._w = W
        return self

    # -- per-grid metadata ----------------------------------------------------------------------
    def metadata(self, grid_thw):
        """Device copy of the grid's integer metadata, built once per grid and cached."""
        torch = _torch()
        g = np.asarray(grid_thw, dtype=np.int32).reshape(-1, 3)
        key = (tuple(map(tuple, g.tolist())), bool(self.split_attention))
        hit = self._meta_cache.get(key)
        if hit is not None:
            self._meta_cache.move_to_end(key)
            return hit
        s = self.spec
        m = grid_metadata(g, s.spatial_merge_size, s.num_position_embeddings, self.qdtype, s.num_heads)
        if s.use_window:
            m = window_grid_metadata(m, g, s.spatial_merge_size, s.patch_size, s.window_size, s.num_heads)
        nz = lambda a: a if a is not None and len(a) else np.zeros((1, 4), np.int32)
        host = {"cu_seqlens": m.cu_seqlens, "pos_hw": m.pos_hw, "tap_idx": m.tap_idx, "tap_w": m.tap_w,
                "tiles": nz(m.tiles)}
        if s.use_window:
            host["window_tiles"] = nz(m.window_tiles)
            host["window_index"] = m.window_index if len(m.window_index) else np.zeros(1, np.int32)
            host["window_reverse"] = m.window_reverse if len(m.window_reverse) else np.zeros(1, np.int32)
        split = None
        cu_full = m.cu_full if s.use_window else m.cu_seqlens
        longest = int(np.diff(cu_full).max()) if len(cu_full) > 1 else 0
        # The bf16 kernels gain from key parts only on long segments (MI355X, attention alone: a lone
        # 784- or 1024-token segment runs 12.0 / 13.7 us on the plain list against 21.0 / 29.0 us
        # split; config 4's 7056-token one gains); the fp32 kernel, ~4x slower per key tile, gains
        # from them at 784 tokens already.
        if (self.split_attention and s.head_dim in (64, 72, 80) and
                (self.qdtype == capi.QVL_DTYPE_F32 or longest >= self.SPLIT_MIN_KEYS_BF16)):
            n_cus = torch.cuda.get_device_properties(torch.device(self.device)).multi_processor_count
            split, n_whole = attention_worklist_split(cu_full, s.num_heads, s.head_dim, n_cus)
            host["split_tiles"] = nz(split)
        tens = _to_device_packed(host, self.device)
        md = capi.VisionMetadataDev()
        md.n_tokens = m.n_tokens
        md.n_positions = m.n_positions
        md.n_tiles = len(m.tiles)
        md.pos_hw, md.tap_idx, md.tap_w, md.tiles = (tens["pos_hw"].data_ptr(), tens["tap_idx"].data_ptr(),
                                                     tens["tap_w"].data_ptr(), tens["tiles"].data_ptr())
        if s.use_window:
            md.n_window_tiles = len(m.window_tiles)
            md.window_tiles = tens["window_tiles"].data_ptr()
            md.window_index = tens["window_index"].data_ptr()
            md.window_reverse = tens["window_reverse"].data_ptr()
        if split is not None:
            md.n_split_tiles = len(split)
            md.n_split_whole = n_whole
            md.split_tiles = tens["split_tiles"].data_ptr()
        entry = (m, tens, md)
        self._meta_cache[key] = entry
        while len(self._meta_cache) > self.META_CACHE_SIZE:
            self._meta_cache.popitem(last=False)
        return entry

    def clear_metadata_cache(self) -> None:
        """Drop every cached grid's device metadata."""
        self._meta_cache.clear()

    def workspace(self, n_tokens: int):
        torch = _torch()
        nb = C.c_size_t()
        capi.check(self._lib.qvl_encode_vision_workspace_size(C.byref(self._cfg), n_tokens, C.byref(nb)),
                   "qvl_encode_vision_workspace_size")
        if self._ws is None or self._ws.numel() < nb.value:
            self._ws = torch.empty(max(nb.value, 256), dtype=torch.uint8, device=self.device)
        return self._ws, nb.value

    # -- forward (model.py:801-851) ---------------------------------------------------------------
    def __call__(self, pixel_values, grid_thw):
        torch = _torch()
        if self._w is None:
            raise RuntimeError("bind(params) first")
        m, tens, md = self.metadata(grid_thw)
        N = m.n_tokens
        px = pixel_values
        if not isinstance(px, torch.Tensor):
            px = torch.from_numpy(np.ascontiguousarray(np.asarray(px, np.float32)))
        px = px.to(device=self.device, dtype=torch.float32).contiguous()
        if tuple(px.shape) != (N, self.spec.patch_volume):
            raise ValueError(f"pixel_values shape {tuple(px.shape)} != ({N}, {self.spec.patch_volume})")
        s = self.spec
        tokens = torch.empty((N // 4, s.out_hidden_size), dtype=self._tdtype(), device=self.device)
        ds = [torch.empty((N // 4, s.out_hidden_size), dtype=self._tdtype(), device=self.device)
              for _ in s.deepstack_visual_indexes]
        ds_ptrs = (C.c_void_p * max(len(ds), 1))(*[t.data_ptr() for t in ds])
        ws, nbytes = self.workspace(N)
        capi.check(self._lib.qvl_encode_vision(self._stream(), C.byref(self._cfg), C.byref(self._w), C.byref(md),
                                               px.data_ptr(), tokens.data_ptr(), ds_ptrs, ws.data_ptr(), nbytes),
                   "qvl_encode_vision")
        return tokens, tuple(ds)


    # -- staged forward: one C-ABI stage entry per reference op, with per-layer taps -------------
    def _staged_ctx(self, grid_thw):
        torch = _torch()
        if self.spec.use_window:
            raise NotImplementedError("the staged path runs full attention only; window specs run through __call__")
        m, tens, md = self.metadata(grid_thw)
        s = self.spec
        N, D, H, hd = m.n_tokens, s.hidden_size, s.num_heads, s.head_dim
        I = -(-s.intermediate_size // 64) * 64
        dev = dict(device=self.device)
        bf = self._tdtype()
        cs = torch.empty((N, hd // 2, 2), dtype=torch.float32, **dev)
        capi.check(self._lib.qvl_rotary_table(self._stream(), self.qdtype, tens["pos_hw"].data_ptr(), N, hd, 10000.0,
                                              cs.data_ptr()), "qvl_rotary_table")
        nb = C.c_size_t()
        capi.check(self._lib.qvl_vision_attention_workspace_size(self.qdtype, N, H, hd, C.byref(nb)), "attention ws")
        return dict(m=m, tens=tens, md=md, N=N, D=D, H=H, hd=hd, I=I, cs=cs, aws_bytes=nb.value,
                    aws=torch.empty(max(nb.value, 256), dtype=torch.uint8, **dev),
                    xn=torch.empty((N, D), dtype=bf, **dev), qkv=torch.empty((N, 3 * D), dtype=bf, **dev),
                    o=torch.empty((N, D), dtype=bf, **dev), h=torch.empty((N, I), dtype=bf, **dev))

    def block_staged(self, i: int, x, ctx) -> None:
        """VisionBlock i (model.py:627-630) applied in place to the residual stream x [N, D],
        one C-ABI stage entry per reference op (qkv Dense, rotary + varlen attention, proj Dense +
        residual, LayerNorms, fc1 + GELU, fc2 + residual)."""
        lib, st, dt, ck = self._lib, self._stream(), self.qdtype, capi.check
        N, D, H, hd, I = ctx["N"], ctx["D"], ctx["H"], ctx["hd"], ctx["I"]
        xn, qkv, o, h = ctx["xn"], ctx["qkv"], ctx["o"], ctx["h"]
        B = self._blocks_arr[i]
        ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D, B.norm1_w, B.norm1_b, xn.data_ptr(), D, N, D, 1e-6), "ln1")
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS, xn.data_ptr(), D, B.qkv_w, B.qkv_b, None, 0, qkv.data_ptr(),
                         3 * D, N, 3 * D, D), "qkv")
        esz = qkv.element_size()
        ck(lib.qvl_vision_attention(st, dt, qkv.data_ptr(), qkv.data_ptr() + esz * D, qkv.data_ptr() + 2 * esz * D, 3 * D,
                                    ctx["cs"].data_ptr(), ctx["tens"]["tiles"].data_ptr(), ctx["md"].n_tiles,
                                    o.data_ptr(), D, N, H, hd, ctx["aws"].data_ptr(), ctx["aws_bytes"]), "attention")
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS_RESIDUAL, o.data_ptr(), D, B.proj_w, B.proj_b, x.data_ptr(), D,
                         x.data_ptr(), D, N, D, D), "proj")
        ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D, B.norm2_w, B.norm2_b, xn.data_ptr(), D, N, D, 1e-6), "ln2")
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS_GELU, xn.data_ptr(), D, B.fc1_w, B.fc1_b, None, 0, h.data_ptr(),
                         I, N, I, D), "fc1")
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS_RESIDUAL, h.data_ptr(), I, B.fc2_w, B.fc2_b, x.data_ptr(), D,
                         x.data_ptr(), D, N, D, I), "fc2")

    def _fused_ctx(self, ctx):
        """Buffers of block_fused, added to a _staged_ctx: head-major Q/K/V^T, the split-K
        partials of the GEMMs and the split attention's partial outputs."""
        torch = _torch()
        if "qb" in ctx:
            return ctx
        N, H, hd = ctx["N"], ctx["H"], ctx["hd"]
        if self.qdtype != capi.QVL_DTYPE_BF16 or not (hd == 64 or (hd == 72 and H % 4 == 0)):
            raise NotImplementedError("block_fused runs the bf16 fused qkv+rotary entry (head_dim 64, or 72 "
                                      "with num_heads % 4 == 0)")
        Np = -(-N // 64) * 64
        hdp = 64 if hd == 64 else 88            # Q/K row length of the attention kernels
        dev = dict(device=self.device)
        ctx["qb"] = torch.empty((H, Np, hdp), dtype=torch.bfloat16, **dev)
        ctx["kb"] = torch.empty_like(ctx["qb"])
        ctx["vb"] = torch.empty((H, hd, Np), dtype=torch.bfloat16, **dev)
        nb = C.c_size_t()
        capi.check(self._lib.qvl_dense_workspace_size(C.byref(nb)), "qvl_dense_workspace_size")
        ctx["gws"] = torch.empty(max(nb.value, 256), dtype=torch.uint8, **dev)
        ctx["gws_bytes"] = nb.value
        md = ctx["md"]
        ab = C.c_size_t(0)
        if md.split_tiles:
            capi.check(self._lib.qvl_attention_split_workspace_size(hd, md.n_split_tiles, md.n_split_whole,
                                                                    C.byref(ab)), "attention split ws")
        ctx["apart"] = torch.empty(max(ab.value, 256), dtype=torch.uint8, **dev)
        ctx["apart_bytes"] = ab.value
        ctx["stats"] = torch.empty((N, 2), dtype=torch.float32, **dev)     # folded LayerNorms' (mean, rstd)
        # per-128-column row partials written by the residual Dense layers (hidden % 128 == 0)
        ctx["parts"] = torch.empty((N, max(1, self.spec.hidden_size // 128), 2), dtype=torch.float32, **dev)
        # (cos, sin) per rotary position, as the tower looks them up when the grid's positions fit
        n_pos = ctx["m"].n_positions
        cap = (12032 if self.ln_fold else 16384) if hd == 64 else 12288   # the folded kernels' LDS leaves less
        if hd == 64 and 0 < n_pos and n_pos * (hd // 4) * 4 <= cap:
            ctx["rtab"] = torch.empty((n_pos, hd // 4), dtype=torch.int32, **dev)
            capi.check(self._lib.qvl_rotary_pos_table(self._stream(), hd, 10000.0, n_pos, ctx["rtab"].data_ptr()),
                       "qvl_rotary_pos_table")
        return ctx

    def block_fused(self, i: int, x, ctx, x_parts: bool = False, marks: Optional[list] = None) -> None:
        """VisionBlock i (model.py:627-630) in place on x [N, D] through exactly the entries the
        whole-tower call runs for a bf16 tower (head_dim 64 or 72): LayerNorm, the fused qkv Dense +
        rotary (qvl_dense_qkv_rotary, head-major Q/K/V^T), attention on the tower's work list
        (qvl_attention_headmajor_split when the tower builds a split list, else
        qvl_attention_headmajor), proj + residual, LayerNorm, fc1 + GELU, fc2 + residual, the
        GEMMs with the tower's split-K workspace. With ln_fold each LayerNorm is folded into the Dense
        after it, as in the tower: proj and fc2 write x's row partials (qvl_dense_rowstats_ws) and fc1
        reads them (qvl_dense_ln_parts_ws); norm1 reads the partials the previous block's fc2 left in
        ctx when x_parts is true (blocks run in sequence, the tower's exact launches), and otherwise
        (a block run on its own) takes its statistics from qvl_row_stats (the same mean and rstd up
        to fp32 rounding) into qvl_dense_qkv_rotary_ln (hidden % 128 != 0: qvl_row_stats for both
        norms). marks: a list that receives (kernel class, start event, end event) for each of the
        five GEMM / attention launches, recorded on the launch stream."""
        ctx = self._fused_ctx(ctx)
        lib, st, dt, ck = self._lib, self._stream(), self.qdtype, capi.check
        N, D, H, hd, I = ctx["N"], ctx["D"], ctx["H"], ctx["hd"], ctx["I"]
        xn, o, h = ctx["xn"], ctx["o"], ctx["h"]
        qb, kb, vb = ctx["qb"].data_ptr(), ctx["kb"].data_ptr(), ctx["vb"].data_ptr()
        gws, gwn = ctx["gws"].data_ptr(), ctx["gws_bytes"]
        md = ctx["md"]
        B = self._blocks_arr[i]
        fold = self.ln_fold
        G = D // 128 if fold and D % 128 == 0 else 0
        parts = ctx["parts"].data_ptr()
        torch = _torch()
        tstream = torch.cuda.current_stream()

        def timed(name, launch):
            if marks is None:
                launch()
                return
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(tstream)
            launch()
            b.record(tstream)
            marks.append((name, a, b))
        if fold and G and x_parts:
            fq = self._folds[f"blocks.{i}.qkv"]
            ff = self._folds[f"blocks.{i}.fc1"]
            rt = "rtab" in ctx
            timed("qkv", lambda: ck(lib.qvl_dense_qkv_rotary_ln_parts(
                st, dt, x.data_ptr(), D, fq[0].data_ptr(), fq[1].data_ptr(), parts, G, 1e-6, B.qkv_b,
                None if rt else ctx["cs"].data_ptr(), ctx["tens"]["pos_hw"].data_ptr() if rt else None,
                ctx["rtab"].data_ptr() if rt else None, ctx["rtab"].shape[0] if rt else 0, qb, kb, vb, N, D, H, gws,
                gwn), "qkv_rotary_ln_parts"))
        elif fold:
            stats = ctx["stats"].data_ptr()
            fq, ff = self._folds[f"blocks.{i}.qkv"], self._folds[f"blocks.{i}.fc1"]
            ck(lib.qvl_row_stats(st, dt, x.data_ptr(), D, N, D, 1e-6, stats), "ln1 stats")
            rt = "rtab" in ctx
            timed("qkv", lambda: ck(lib.qvl_dense_qkv_rotary_ln(
                st, dt, x.data_ptr(), D, fq[0].data_ptr(), fq[1].data_ptr(), stats, B.qkv_b,
                None if rt else ctx["cs"].data_ptr(), ctx["tens"]["pos_hw"].data_ptr() if rt else None,
                ctx["rtab"].data_ptr() if rt else None, ctx["rtab"].shape[0] if rt else 0, qb, kb, vb, N, D, H, gws,
                gwn), "qkv_rotary_ln"))
        else:
            ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D, B.norm1_w, B.norm1_b, xn.data_ptr(), D, N, D, 1e-6), "ln1")
            if "rtab" in ctx:
                timed("qkv", lambda: ck(lib.qvl_dense_qkv_rotary_pos(
                    st, dt, xn.data_ptr(), D, B.qkv_w, B.qkv_b, ctx["tens"]["pos_hw"].data_ptr(),
                    ctx["rtab"].data_ptr(), ctx["rtab"].shape[0], qb, kb, vb, N, D, H, gws, gwn), "qkv_rotary_pos"))
            else:
                timed("qkv", lambda: ck(lib.qvl_dense_qkv_rotary(
                    st, dt, xn.data_ptr(), D, B.qkv_w, B.qkv_b, ctx["cs"].data_ptr(), qb, kb, vb, N, D, H, gws, gwn),
                    "qkv_rotary"))
        if md.split_tiles:
            timed("attention", lambda: ck(lib.qvl_attention_headmajor_split(
                st, dt, qb, kb, vb, md.split_tiles, md.n_split_tiles, md.n_split_whole, N, H, hd, o.data_ptr(), D,
                ctx["apart"].data_ptr(), ctx["apart_bytes"]), "attention_split"))
        else:
            timed("attention", lambda: ck(lib.qvl_attention_headmajor(
                st, dt, qb, kb, vb, md.tiles, md.n_tiles, N, H, hd, o.data_ptr(), D), "attention"))
        if G:
            timed("proj", lambda: ck(lib.qvl_dense_rowstats_ws(
                st, dt, o.data_ptr(), D, B.proj_w, B.proj_b, x.data_ptr(), D, x.data_ptr(), D, N, D, D, parts, gws,
                gwn), "proj (+ row partials)"))
        else:
            timed("proj", lambda: ck(lib.qvl_dense_ws(
                st, dt, capi.QVL_EPI_BIAS_RESIDUAL, o.data_ptr(), D, B.proj_w, B.proj_b, x.data_ptr(), D, x.data_ptr(),
                D, N, D, D, gws, gwn), "proj"))
        if G:
            timed("fc1", lambda: ck(lib.qvl_dense_ln_parts_ws(
                st, dt, capi.QVL_EPI_BIAS_GELU, x.data_ptr(), D, ff[0].data_ptr(), ff[1].data_ptr(), parts, G, 1e-6,
                B.fc1_b, h.data_ptr(), I, N, I, D, gws, gwn), "fc1 (folded ln2)"))
        elif fold:
            ck(lib.qvl_row_stats(st, dt, x.data_ptr(), D, N, D, 1e-6, stats), "ln2 stats")
            timed("fc1", lambda: ck(lib.qvl_dense_ln_ws(
                st, dt, capi.QVL_EPI_BIAS_GELU, x.data_ptr(), D, ff[0].data_ptr(), ff[1].data_ptr(), stats, B.fc1_b,
                h.data_ptr(), I, N, I, D, gws, gwn), "fc1 (folded ln2)"))
        else:
            ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D, B.norm2_w, B.norm2_b, xn.data_ptr(), D, N, D, 1e-6), "ln2")
            timed("fc1", lambda: ck(lib.qvl_dense_ws(
                st, dt, capi.QVL_EPI_BIAS_GELU, xn.data_ptr(), D, B.fc1_w, B.fc1_b, None, 0, h.data_ptr(), I, N, I, D,
                gws, gwn), "fc1"))
        if G:
            timed("fc2", lambda: ck(lib.qvl_dense_rowstats_ws(
                st, dt, h.data_ptr(), I, B.fc2_w, B.fc2_b, x.data_ptr(), D, x.data_ptr(), D, N, D, I, parts, gws, gwn),
                "fc2 (+ row partials)"))
        else:
            timed("fc2", lambda: ck(lib.qvl_dense_ws(
                st, dt, capi.QVL_EPI_BIAS_RESIDUAL, h.data_ptr(), I, B.fc2_w, B.fc2_b, x.data_ptr(), D, x.data_ptr(), D,
                N, D, I, gws, gwn), "fc2"))

    def merger_fused(self, x, ctx, which: int = -1):
        """The merger as the whole-tower call runs it: a deepstack merger of a tower with ln_fold folds
        its post-shuffle norm into fc1 (qvl_dense_ln_ws on the [N/4, 4D] rows; the tower reads the
        row partials fc2 wrote, here on its own the statistics come from qvl_row_stats); every other
        merger is merger_staged."""
        if which < 0 or not self.ln_fold:
            return self.merger_staged(x, ctx, which)
        torch = _torch()
        ctx = self._fused_ctx(ctx)
        lib, st, dt, ck = self._lib, self._stream(), self.qdtype, capi.check
        N, D, s = ctx["N"], ctx["D"], self.spec
        D4 = 4 * D
        mw = self._ds_arr[which]
        f = self._folds[f"deepstack.{which}.fc1"]
        dev = dict(device=self.device)
        stats = ctx["stats"].data_ptr()
        ck(lib.qvl_row_stats(st, dt, x.data_ptr(), D4, N // 4, D4, 1e-6, stats), "merger ln stats")
        hm = torch.empty((N // 4, D4), dtype=self._tdtype(), **dev)
        ck(lib.qvl_dense_ln_ws(st, dt, capi.QVL_EPI_BIAS_GELU, x.data_ptr(), D4, f[0].data_ptr(), f[1].data_ptr(), stats,
                               mw.fc1_b, hm.data_ptr(), D4, N // 4, D4, D4, ctx["gws"].data_ptr(), ctx["gws_bytes"]),
           "merger fc1 (folded ln)")
        out = torch.empty((N // 4, s.out_hidden_size), dtype=self._tdtype(), **dev)
        ck(lib.qvl_dense_ws(st, dt, capi.QVL_EPI_BIAS, hm.data_ptr(), D4, mw.fc2_w, mw.fc2_b, None, 0, out.data_ptr(),
                            s.out_hidden_size, N // 4, s.out_hidden_size, D4, ctx["gws"].data_ptr(), ctx["gws_bytes"]),
           "merger fc2")
        return out

    def merger_staged(self, x, ctx, which: int = -1):
        """VisionPatchMerger (model.py:648-656) on the residual stream x: main merger (which=-1) or
        deepstack merger `which` (postshuffle LayerNorm over 4D)."""
        torch = _torch()
        lib, st, dt, ck = self._lib, self._stream(), self.qdtype, capi.check
        N, D = ctx["N"], ctx["D"]
        s = self.spec
        D4 = 4 * D
        mw = self._w.merger if which < 0 else self._ds_arr[which]
        dev = dict(device=self.device)
        xm = torch.empty((N // 4, D4), dtype=self._tdtype(), **dev)
        if which >= 0:
            ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D4, mw.norm_w, mw.norm_b, xm.data_ptr(), D4, N // 4, D4,
                                  1e-6), "merger ln")
        else:
            ck(lib.qvl_layer_norm(st, dt, x.data_ptr(), D, mw.norm_w, mw.norm_b, xm.data_ptr(), D, N, D, 1e-6),
               "merger ln")
        hm = torch.empty((N // 4, D4), dtype=self._tdtype(), **dev)
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS_GELU, xm.data_ptr(), D4, mw.fc1_w, mw.fc1_b, None, 0, hm.data_ptr(),
                         D4, N // 4, D4, D4), "merger fc1")
        out = torch.empty((N // 4, s.out_hidden_size), dtype=self._tdtype(), **dev)
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS, hm.data_ptr(), D4, mw.fc2_w, mw.fc2_b, None, 0, out.data_ptr(),
                         s.out_hidden_size, N // 4, s.out_hidden_size, D4), "merger fc2")
        return out

    def embed_staged(self, pixel_values, ctx):
        """Patch embed + learned pos-embed (model.py:802-806) via qvl_cast (bf16) / qvl_pos_embed /
        qvl_dense."""
        torch = _torch()
        lib, st, dt, ck = self._lib, self._stream(), self.qdtype, capi.check
        N, D = ctx["N"], ctx["D"]
        s = self.spec
        px = pixel_values if isinstance(pixel_values, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(np.asarray(pixel_values, np.float32)))
        px = px.to(device=self.device, dtype=torch.float32).contiguous()
        W = self._w
        if self.qdtype == capi.QVL_DTYPE_BF16:
            x16 = torch.empty((N, s.patch_volume), dtype=torch.bfloat16, device=self.device)
            ck(lib.qvl_cast(st, dt, px.data_ptr(), x16.data_ptr(), px.numel()), "qvl_cast")
        else:
            x16 = px
        pos = torch.empty((N, D), dtype=self._tdtype(), device=self.device)
        ck(lib.qvl_pos_embed(st, dt, W.pos_table, ctx["tens"]["tap_idx"].data_ptr(), ctx["tens"]["tap_w"].data_ptr(),
                             pos.data_ptr(), N, D), "qvl_pos_embed")
        x = torch.empty((N, D), dtype=self._tdtype(), device=self.device)
        ck(lib.qvl_dense(st, dt, capi.QVL_EPI_BIAS_RESIDUAL, x16.data_ptr(), s.patch_volume, W.patch_w, W.patch_b,
                         pos.data_ptr(), D, x.data_ptr(), D, N, D, s.patch_volume), "qvl_dense(patch)")
        return x

    def forward_staged(self, pixel_values, grid_thw, keep_layers: bool = False):
        """Same tower, driven stage by stage through the per-op C-ABI entries — the sequence a
        per-stage FFI registration runs. Returns (tokens, deepstack, layers) where `layers[i]` is
        the residual stream after block i when keep_layers (model.py:838-843)."""
        if self._w is None:
            raise RuntimeError("bind(params) first")
        ctx = self._staged_ctx(grid_thw)
        x = self.embed_staged(pixel_values, ctx)
        layers, feats = [], []
        taps = tuple(self.spec.deepstack_visual_indexes)
        for i in range(self.spec.depth):
            self.block_staged(i, x, ctx)
            if keep_layers:
                layers.append(x.clone())
            if i in taps:
                feats.append(self.merger_staged(x, ctx, len(feats)))
        return self.merger_staged(x, ctx), tuple(feats), layers


class Qwen3VLModel:
    """The `encode_vision` entry of the reference model (model.py:858-871, 940-944).

    `spec` is the reference's `Qwen3VLSpec` (as `spec_from_config` returns it); a bare
    `VisionBackboneSpec` is accepted as the vision spec of a model without a text spec. As in the
    reference, the tower is built in float32 unless asked otherwise (model.py:871 builds
    `Qwen3VisionTransformer(spec.vision)`, whose dtype defaults to float32, model.py:661; `dtype`
    is the text backbone's, which this build does not run). `vision_dtype="bfloat16"` selects the
    bf16 tower (the reference's `Qwen3VisionTransformer(spec, dtype=jnp.bfloat16)`)."""

    def __init__(self, spec, dtype: str = "bfloat16", device: str = "cuda:0", vision_dtype: str = "float32"):
        if isinstance(spec, VisionBackboneSpec):
            spec = Qwen3VLSpec(text=None, vision=spec)
        self.spec = spec
        self.dtype = dtype
        vision = spec.vision if spec is not None else None
        self.vision_spec = vision
        self.visual = Qwen3VisionTransformer(vision, vision_dtype, device) if vision else None
        self._bound = None

    def encode_vision(self, pixel_values, grid_thw) -> VisionEmbeddings:
        if self.visual is None:
            raise ValueError("Vision backbone not configured")
        tokens, deepstack = self.visual(pixel_values, grid_thw)
        return VisionEmbeddings(tokens=tokens, deepstack=deepstack)

    def apply(self, variables: Dict, pixel_values, grid_thw, method="encode_vision") -> VisionEmbeddings:
        """`model.apply({"params": params}, pixel_values, grid_thw, method=model.encode_vision)`."""
        if self.visual is None:
            raise ValueError("Vision backbone not configured")
        params = variables["params"]
        if self._bound is not params:
            self.visual.bind(params)
            self._bound = params
        fn = method if callable(method) else getattr(self, method)
        return fn(pixel_values, grid_thw)
