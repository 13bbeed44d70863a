"""numpy restatement of the Qwen3-VL vision tower forward (TEST INFRASTRUCTURE ONLY).

Follows /root/reference/model.py:
  LayerNorm            375-388   fp32 statistics, output cast back to the input dtype
  rotate_half          146-149
  VisionPatchEmbed     549-556   x.astype(dtype) @ kernel[1536, D] + bias
  VisionAttention      559-601   qkv Dense, split q|k|v, rotary in `dtype`, per-segment fp32 softmax
  VisionMLP            604-614   fc1 -> gelu(approximate=True) -> fc2
  VisionBlock          617-630   pre-LN residual block
  VisionPatchMerger    633-656   main (LN then reshape) / deepstack (reshape then LN)
  Qwen3VisionTransformer.__call__ 801-851 (full-attention branch only: every block is full
                       attention for qwen3_vl, model.py:1033-1034)

Precision modes:
  "fp64": every op in float64 (exact maths; what library routines are compared against).
  "fp32": every op in float32 (the reference default: Qwen3VisionTransformer.dtype = float32).
  "bf16": the reference's bf16 mode (`Qwen3VisionTransformer(spec, dtype=jnp.bfloat16)`): each
          Dense rounds its inputs, weights and fp32-accumulated output to bf16 and adds a
          bf16-rounded bias in bf16; rotary runs in bf16 arithmetic (eager jnp ops, one rounding
          per op); LayerNorm statistics and attention softmax stay fp32; residual adds in bf16.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import indices as ix


# ---------------------------------------------------------------------------------------------
# bf16 emulation
# ---------------------------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returned as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    r = (u >> 16) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u                      # uint32 wrap-around only for NaN payloads, restored below
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32(np.nan)
    return out


class _P:
    """Precision helper: array dtype + rounding at the reference's cast points."""

    def __init__(self, mode: str):
        if mode not in ("fp64", "fp32", "bf16"):
            raise ValueError(f"unknown precision {mode!r}")
        self.mode = mode
        self.acc = np.float64 if mode == "fp64" else np.float32

    def r(self, x):
        """Cast to the tower dtype (bf16 rounding in bf16 mode)."""
        x = np.asarray(x, dtype=self.acc)
        return bf16_round(x) if self.mode == "bf16" else x

    def f(self, x):
        """The fp32 'island' dtype (LN stats, softmax); fp64 in fp64 mode."""
        return np.asarray(x, dtype=self.acc)


# ---------------------------------------------------------------------------------------------
# primitive ops
# ---------------------------------------------------------------------------------------------
def dense(x, kernel, bias, p: _P):
    """flax.linen.Dense with dtype=p: promote x, kernel, bias to dtype; dot; add bias (a18)."""
    xk = p.r(x)
    k = p.r(kernel)
    y = p.r(xk @ k)
    return p.r(y + p.r(bias))


def layer_norm(x, weight, bias, eps: float, p: _P):
    """LayerNorm (model.py:384-388): fp32 mean / biased var / rsqrt, affine, cast back."""
    xf = p.f(x)
    mean = xf.mean(axis=-1, keepdims=True)
    var = ((xf - mean) ** 2).mean(axis=-1, keepdims=True)
    normed = (xf - mean) * (1.0 / np.sqrt(var + p.acc(eps)))
    return p.r(normed * p.f(p.r(weight)) + p.f(p.r(bias)))


def gelu_tanh(x, p: _P):
    """jax.nn.gelu(approximate=True): x * 0.5 * (1 + tanh(sqrt(2/pi) * (x + 0.044715 x^3)))."""
    xf = p.f(x)
    c = p.acc(np.sqrt(2.0 / np.pi))
    cdf = 0.5 * (1.0 + np.tanh(c * (xf + p.acc(0.044715) * xf ** 3)))
    return p.r(xf * cdf)


def rotate_half(x):
    """model.py:146-149: concat(-x2, x1) over the last axis halves."""
    h = x.shape[-1] // 2
    return np.concatenate([-x[..., h:], x[..., :h]], axis=-1)


def apply_rotary(x, cos, sin, p: _P):
    """model.py:579-582: x*cos + rotate_half(x)*sin, each op rounded to dtype (eager jnp).

    x: [N, H, hd]; cos/sin: [N, hd] already cast to dtype.
    """
    c = cos[:, None, :]
    s = sin[:, None, :]
    return p.r(p.r(x * c) + p.r(rotate_half(x) * s))


def attention_varlen(q, k, v, cu_seqlens, p: _P):
    """Per-segment full softmax attention (model.py:585-600), non-causal, fp32 softmax.

    q, k, v: [N, H, hd] (already rotated); returns [N, H, hd] in dtype. Empty segments are
    skipped (model.py:589-590); rows outside every segment stay zero.
    """
    n, h, hd = q.shape
    scale = p.acc(hd ** -0.5)
    out = np.zeros((n, h, hd), dtype=p.acc)
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    for i in range(len(cu) - 1):
        s, e = int(cu[i]), int(cu[i + 1])
        if s >= e:
            continue
        qw = np.ascontiguousarray(p.f(q[s:e]).transpose(1, 0, 2))
        kw = np.ascontiguousarray(p.f(k[s:e]).transpose(1, 0, 2))
        vw = np.ascontiguousarray(p.f(v[s:e]).transpose(1, 0, 2))
        for hh in range(h):
            sc = qw[hh] @ kw[hh].T
            sc *= scale
            sc -= sc.max(axis=-1, keepdims=True)
            np.exp(sc, out=sc)                          # softmax (jax.nn.softmax, model.py:596)
            sc /= sc.sum(axis=-1, keepdims=True)
            out[s:e, hh] = sc @ vw[hh]
    return p.r(out)


# ---------------------------------------------------------------------------------------------
# spec + params
# ---------------------------------------------------------------------------------------------
@dataclass
class VisionSpec:
    """The VisionBackboneSpec fields the tower reads (model.py:84-98)."""
    hidden_size: int = 1024
    out_hidden_size: int = 2048
    depth: int = 24
    num_heads: int = 16
    intermediate_size: int = 4096
    patch_size: int = 16
    temporal_patch_size: int = 2
    spatial_merge_size: int = 2
    in_channels: int = 3
    num_position_embeddings: Optional[int] = 2304          # None: no learned pos-embed table
    deepstack_visual_indexes: Tuple[int, ...] = (5, 11, 17)
    window_size: int = 32
    fullatt_block_indexes: Optional[Tuple[int, ...]] = None      # None: every block (qwen3_vl)

    @property
    def use_window(self) -> bool:
        fa = self.fullatt_block_indexes
        return fa is not None and len(set(fa)) < self.depth

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def patch_volume(self) -> int:
        return self.in_channels * self.temporal_patch_size * self.patch_size ** 2


def init_params(spec: VisionSpec, seed: int = 0, std: float = 0.02, bias_std: float = 0.0,
                ln_noise: float = 0.0) -> Dict:
    """Random params in the reference's Flax tree (model.py:663-680, Appendix B naming).

    Dense kernels [in, out] and the pos-embed table ~ N(0, std); biases N(0, bias_std) (0 by
    default, as Flax init); LayerNorm weight 1 + N(0, ln_noise), bias N(0, ln_noise).
    """
    rng = np.random.default_rng(seed)
    D, I, Do = spec.hidden_size, spec.intermediate_size, spec.out_hidden_size
    M4 = D * spec.spatial_merge_size ** 2

    def dense_p(i, o):
        return {"kernel": (rng.standard_normal((i, o)) * std).astype(np.float32),
                "bias": (rng.standard_normal(o) * bias_std).astype(np.float32)}

    def ln_p(d):
        return {"weight": (1.0 + rng.standard_normal(d) * ln_noise).astype(np.float32),
                "bias": (rng.standard_normal(d) * ln_noise).astype(np.float32)}

    params = {"patch_embed": {"proj": dense_p(spec.patch_volume, D)}}
    if spec.num_position_embeddings:
        params["pos_embed"] = {"embedding": (rng.standard_normal((spec.num_position_embeddings, D)) * std).astype(
            np.float32)}
    for i in range(spec.depth):
        params[f"blocks_{i}"] = {
            "norm1": ln_p(D), "norm2": ln_p(D),
            "attn": {"qkv": dense_p(D, 3 * D), "proj": dense_p(D, D)},
            "mlp": {"linear_fc1": dense_p(D, I), "linear_fc2": dense_p(I, D)},
        }
    params["merger"] = {"norm": ln_p(D), "linear_fc1": dense_p(M4, M4), "linear_fc2": dense_p(M4, Do)}
    for j in range(len(spec.deepstack_visual_indexes)):
        params[f"deepstack_mergers_{j}"] = {"norm": ln_p(M4), "linear_fc1": dense_p(M4, M4),
                                            "linear_fc2": dense_p(M4, Do)}
    return {"visual": params}


# ---------------------------------------------------------------------------------------------
# tower pieces
# ---------------------------------------------------------------------------------------------
def pos_embed(table, grid_thw, spec: VisionSpec, p: _P):
    """_fast_pos_embed_interpolate (model.py:700-767): 4 taps, gathered rows weighted in dtype."""
    idx, wts = ix.pos_embed_taps_ref(grid_thw, spec.num_position_embeddings, spec.spatial_merge_size)
    tab = p.r(table)
    w = p.r(wts)
    terms = [p.r(tab[idx[j]] * w[j][:, None]) for j in range(4)]
    acc = terms[0]
    for j in range(1, 4):
        acc = p.r(acc + terms[j])
    return acc


def rotary_cos_sin(grid_thw, spec: VisionSpec, p: _P):
    """model.py:807, 821-823: emb = [rot, rot]; cos/sin in fp32, cast to dtype."""
    rot = ix.rotary_half_ref(grid_thw, spec.head_dim, spec.spatial_merge_size)
    emb = np.concatenate([rot, rot], axis=-1).astype(np.float32)
    return p.r(np.cos(emb.astype(p.acc))), p.r(np.sin(emb.astype(p.acc)))


def vision_attention(x, prm, cos, sin, cu_seqlens, spec: VisionSpec, p: _P):
    """VisionAttention.__call__ (model.py:569-601)."""
    n = x.shape[0]
    D, H, hd = spec.hidden_size, spec.num_heads, spec.head_dim
    qkv = dense(x, prm["qkv"]["kernel"], prm["qkv"]["bias"], p)
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    q = q.reshape(n, H, hd); k = k.reshape(n, H, hd); v = v.reshape(n, H, hd)
    q = apply_rotary(q, cos[:, :hd], sin[:, :hd], p)
    k = apply_rotary(k, cos[:, :hd], sin[:, :hd], p)
    o = attention_varlen(q, k, v, cu_seqlens, p).reshape(n, D)
    return dense(o, prm["proj"]["kernel"], prm["proj"]["bias"], p)


def vision_mlp(x, prm, p: _P):
    """VisionMLP.__call__ (model.py:610-614)."""
    h = dense(x, prm["linear_fc1"]["kernel"], prm["linear_fc1"]["bias"], p)
    h = gelu_tanh(h, p)
    return dense(h, prm["linear_fc2"]["kernel"], prm["linear_fc2"]["bias"], p)


def vision_block(x, prm, cos, sin, cu_seqlens, spec: VisionSpec, p: _P):
    """VisionBlock.__call__ (model.py:627-630)."""
    a = vision_attention(layer_norm(x, prm["norm1"]["weight"], prm["norm1"]["bias"], 1e-6, p),
                         prm["attn"], cos, sin, cu_seqlens, spec, p)
    x = p.r(x + a)
    m = vision_mlp(layer_norm(x, prm["norm2"]["weight"], prm["norm2"]["bias"], 1e-6, p), prm["mlp"], p)
    return p.r(x + m)


def patch_merger(x, prm, spec: VisionSpec, postshuffle: bool, p: _P):
    """VisionPatchMerger.__call__ (model.py:648-656)."""
    unit = spec.spatial_merge_size ** 2
    D = spec.hidden_size
    if postshuffle:
        x = x.reshape(-1, unit * D)
        x = layer_norm(x, prm["norm"]["weight"], prm["norm"]["bias"], 1e-6, p)
    else:
        x = layer_norm(x, prm["norm"]["weight"], prm["norm"]["bias"], 1e-6, p)
        x = x.reshape(-1, unit * D)
    h = gelu_tanh(dense(x, prm["linear_fc1"]["kernel"], prm["linear_fc1"]["bias"], p), p)
    return dense(h, prm["linear_fc2"]["kernel"], prm["linear_fc2"]["bias"], p)


@dataclass
class OracleOutput:
    tokens: np.ndarray
    deepstack: Tuple[np.ndarray, ...]
    layers: List[np.ndarray] = field(default_factory=list)   # x after each block
    embed: Optional[np.ndarray] = None                         # x after patch embed + pos


def encode_vision(params: Dict, pixel_values, grid_thw, spec: VisionSpec, precision: str = "bf16",
                  keep_layers: bool = False, depth: Optional[int] = None) -> OracleOutput:
    """Qwen3VisionTransformer.__call__ (model.py:801-851) + encode_vision (model.py:940-944).

    `params` is the Flax tree ({"visual": {...}} or the inner dict). `depth` truncates the block
    loop (a test convenience); the final merger still runs.
    """
    p = _P(precision)
    prm = params.get("visual", params)
    grid = np.asarray(grid_thw, dtype=np.int64).reshape(-1, 3)
    x = dense(p.r(pixel_values), prm["patch_embed"]["proj"]["kernel"], prm["patch_embed"]["proj"]["bias"], p)
    if spec.num_position_embeddings:      # no table: nothing added (model.py:701-702, 803-806)
        pe = pos_embed(prm["pos_embed"]["embedding"], grid, spec, p)
        if pe.shape[0] == x.shape[0]:
            x = p.r(x + pe)
    embed = x.copy() if keep_layers else None
    cos, sin = rotary_cos_sin(grid, spec, p)
    cu = ix.cu_seqlens_ref(grid)
    window = spec.use_window
    if window:
        # model.py:808-830: shuffle x and the rotary table by merge groups into window order;
        # window blocks use cu_window, full blocks the window path's cu_seqlens
        mm = spec.spatial_merge_size ** 2
        widx, cu_win = ix.window_index_ref(grid, spec.spatial_merge_size, spec.patch_size, spec.window_size)
        n = x.shape[0]
        x = x.reshape(n // mm, mm, -1)[widx].reshape(n, -1)
        cos = cos.reshape(n // mm, mm, -1)[widx].reshape(n, -1)
        sin = sin.reshape(n // mm, mm, -1)[widx].reshape(n, -1)
        cu = ix.cu_full_window_ref(grid, spec.spatial_merge_size)
        fullatt = set(spec.fullatt_block_indexes)
    ds = set(spec.deepstack_visual_indexes)
    feats, layers = [], []
    nblk = spec.depth if depth is None else depth
    for i in range(nblk):
        cu_i = cu if (not window or i in fullatt) else cu_win
        x = vision_block(x, prm[f"blocks_{i}"], cos, sin, cu_i, spec, p)
        if keep_layers:
            layers.append(x.copy())
        if i in ds:
            j = len(feats)
            feats.append(patch_merger(x, prm[f"deepstack_mergers_{j}"], spec, True, p))
    tokens = patch_merger(x, prm["merger"], spec, False, p)
    if window:
        rev = np.argsort(widx, kind="stable")          # model.py:845-848
        tokens = tokens[rev]
        feats = [f[rev] for f in feats]
    return OracleOutput(tokens=tokens, deepstack=tuple(feats), layers=layers, embed=embed)


# ---------------------------------------------------------------------------------------------
# synthetic inputs
# ---------------------------------------------------------------------------------------------
def patchify(frames: np.ndarray, patch: int = 16, tpatch: int = 2, merge: int = 2) -> Tuple[np.ndarray, np.ndarray]:
    """sample.py:86-121 patch layout for frames [T, C, H, W] already normalised.

    Pads T to a multiple of `tpatch` by repeating the last frame, then emits rows in merge-block
    order, each row laid out (C, tpatch, patch, patch).
    """
    f = np.asarray(frames, dtype=np.float32)
    if f.shape[0] % tpatch:
        pad = tpatch - f.shape[0] % tpatch
        f = np.concatenate([f, np.repeat(f[-1:], pad, axis=0)], axis=0)
    T, C, H, W = f.shape
    gt, gh, gw = T // tpatch, H // patch, W // patch
    x = f.reshape(gt, tpatch, C, gh // merge, merge, patch, gw // merge, merge, patch)
    x = x.transpose(0, 3, 6, 4, 7, 2, 1, 5, 8)
    return x.reshape(gt * gh * gw, C * tpatch * patch * patch), np.array([[gt, gh, gw]], np.int32)
