"""Image preprocessing and decoder-side vision-row injection, restated from the reference
(TEST INFRASTRUCTURE ONLY: imported by tests/ as the checker, never by the product).

* `normalize_u8_ref`      sample.py:86-87   float32 numpy ops: x / 255.0, then (x - 0.5) / 0.5
* `preprocess_frames_ref` sample.py:73-76, 86-121  uint8 HWC frames (alpha dropped) -> normalised
                          CHW -> temporal pad by repeating the last frame -> merge-block patch rows
                          (the layout step is `vision_tower.patchify`, the sample.py:112-119 chain)
* `vision_positions_ref`  model.py:880-882, 930-931  `jnp.where(mask, size=n, fill_value=-1)[0]`
* `inject_ref`            model.py:932-935  `_inject`: h.at[pos].set(where(valid, vis, h[pos]))
* `deepstack_add_ref`     model.py:880-886  `_add`: h.at[idx].add(where(valid, feat, 0))

Scatters with repeated indices are applied in update order (XLA's CPU scatter loop): for `set`
the last write wins, for `add` every update accumulates in the operand dtype.

Pins (tests/test_oracle_io.py): normalize_u8_ref against exact rational arithmetic rounded to
float32 for all 256 inputs; preprocess_frames_ref against transformers' Qwen2-VL image-processor
`patchify` (an independent implementation of the layout) and a per-pixel closed form including
the frame padding; the position / scatter functions against element-by-element loops that apply
the reference's updates one at a time, on edge cases (fewer or more <|image_pad|> tokens than
vision rows, a pad at position 0, no pads, signed zeros, bf16 rounding).
"""
from __future__ import annotations

import numpy as np

from .vision_tower import bf16_round, patchify

IMAGE_MEAN = np.array([0.5, 0.5, 0.5], dtype=np.float32)
IMAGE_STD = np.array([0.5, 0.5, 0.5], dtype=np.float32)


def normalize_u8_ref(frames_u8: np.ndarray) -> np.ndarray:
    """sample.py:86-87 on [..., 3] uint8: float32 / 255.0, then (x - mean) / std per channel."""
    x = np.asarray(frames_u8, dtype=np.float32) / 255.0
    return (x - IMAGE_MEAN) / IMAGE_STD


def preprocess_frames_ref(frames_u8: np.ndarray, patch: int, tpatch: int, merge: int):
    """uint8 [F, H, W, C] (C 3 or 4) -> (pixel_values float32 [N, 3*Tp*P*P], grid [[gt, gh, gw]])."""
    f = np.asarray(frames_u8)
    if f.ndim == 3:
        f = f[None]
    f = f[..., :3]                                        # RGBA -> RGB drops alpha (sample.py:74-75)
    x = normalize_u8_ref(f)                               # [F, H, W, 3]
    chw = np.transpose(x, (0, 3, 1, 2))                   # (F, C, H, W) (sample.py:90)
    return patchify(chw, patch=patch, tpatch=tpatch, merge=merge)


def vision_positions_ref(mask: np.ndarray, n: int):
    """Per batch row: the first n indices where mask is true, -1 fill; and the match count."""
    m = np.asarray(mask).astype(bool)
    if m.ndim == 1:
        m = m[None]
    pos = np.full((m.shape[0], n), -1, np.int64)
    count = np.zeros(m.shape[0], np.int64)
    for b in range(m.shape[0]):
        idx = np.flatnonzero(m[b])
        count[b] = idx.size
        k = min(n, idx.size)
        pos[b, :k] = idx[:k]
    return pos, count


def _cast(x: np.ndarray, bf16: bool) -> np.ndarray:
    return bf16_round(x) if bf16 else np.asarray(x, np.float32)


def inject_ref(hidden: np.ndarray, tokens: np.ndarray, vis: np.ndarray, pad_id: int, bf16: bool) -> np.ndarray:
    """`_inject` per batch row (model.py:928-935). hidden [B, S, D] holds values of the hidden dtype
    (bf16 values as float32 when bf16=True); vis [B or 1, V, D] is cast to the hidden dtype."""
    h = np.array(hidden, dtype=np.float32, copy=True)
    v = np.asarray(vis, np.float32)
    if v.ndim == 2:
        v = v[None]
    B, V = h.shape[0], v.shape[1]
    pos, _ = vision_positions_ref(np.asarray(tokens) == pad_id, V)
    for b in range(B):
        vb = _cast(v[0] if v.shape[0] == 1 else v[b], bf16)
        valid = pos[b] >= 0
        p = np.where(valid, pos[b], 0)
        updates = np.where(valid[:, None], vb, h[b][p])       # gathered before the scatter
        for j in range(V):                                     # set, in update order
            h[b, p[j]] = updates[j]
    return h


def deepstack_add_ref(hidden: np.ndarray, mask: np.ndarray, feat: np.ndarray, bf16: bool) -> np.ndarray:
    """`_add` per batch row (model.py:878-886): add in the hidden dtype, in update order."""
    h = np.array(hidden, dtype=np.float32, copy=True)
    f = np.asarray(feat, np.float32)
    if f.ndim == 2:
        f = f[None]
    B, F = h.shape[0], f.shape[1]
    if F == 0:
        return h
    pos, _ = vision_positions_ref(mask, F)
    for b in range(B):
        fb = _cast(f[0] if f.shape[0] == 1 else f[b], bf16)
        valid = pos[b] >= 0
        p = np.where(valid, pos[b], 0)
        updates = np.where(valid[:, None], fb, np.zeros_like(fb))
        for j in range(F):
            h[b, p[j]] = _cast(h[b, p[j]] + updates[j], bf16)
    return h
