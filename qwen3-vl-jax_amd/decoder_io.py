"""The decoder-side consumers of `VisionEmbeddings` on the GPU (model.py:874-886, 909-938).

`forward_vlm` (model.py:909-938) embeds the prompt, then writes the vision tokens over the
hidden rows of the <|image_pad|> positions (`_inject`), and after decoder layer i adds deepstack
feature i at the same rows (`_apply_deepstack`). The decoder itself is outside this library; these
functions do the row movement with `qvl_vision_positions` + `qvl_scatter_vision_rows`, in place on
torch device tensors:

    hidden, visual_mask, deepstack = inject_vision(hidden, tokens, vision, image_pad_id)
    ... decoder layer i ...
    hidden = apply_deepstack(hidden, visual_mask, deepstack[i])
"""
from __future__ import annotations

from typing import Optional

from . import capi
from .vision import VisionEmbeddings


def _torch():
    import torch
    return torch


def _qdtype(t):
    torch = _torch()
    if t.dtype == torch.bfloat16:
        return capi.QVL_DTYPE_BF16
    if t.dtype == torch.float32:
        return capi.QVL_DTYPE_F32
    raise TypeError(f"unsupported dtype {t.dtype} (bfloat16 or float32)")


def vision_positions(mask_or_tokens, n_rows: int, match: int = 1):
    """(pos [B, n_rows] int32, count [B] int32) on the device: the first n_rows indices of each row
    where the input equals `match` (a bool mask counts True), -1 fill — `jnp.where(mask, size=n_rows,
    fill_value=-1)` per batch row (model.py:880-882, 930-931)."""
    torch = _torch()
    t = mask_or_tokens
    if t.dtype == torch.bool:
        t, match = t.to(torch.int32), 1
    elif t.dtype != torch.int32:
        t = t.to(torch.int32)
    t = t.contiguous()
    if t.dim() == 1:
        t = t.unsqueeze(0)
    B, S = int(t.shape[0]), int(t.shape[1])
    pos = torch.empty((B, max(int(n_rows), 1)), dtype=torch.int32, device=t.device)
    count = torch.empty((B,), dtype=torch.int32, device=t.device)
    lib = capi.load()
    st = torch.cuda.current_stream(t.device).cuda_stream
    capi.check(lib.qvl_vision_positions(st, t.data_ptr(), B, S, int(match), int(n_rows), pos.data_ptr(),
                                        count.data_ptr()), "qvl_vision_positions")
    return pos, count


def scatter_rows(hidden, rows, pos, count, mode: int):
    """In place: hidden[b, pos[b, j]] = rows[b, j] (SET) or += (ADD), rows cast to hidden's dtype."""
    torch = _torch()
    if hidden.dim() != 3 or not hidden.is_contiguous():
        raise ValueError("hidden must be a contiguous [B, S, D] tensor")
    B, S, D = (int(s) for s in hidden.shape)
    r = rows if rows.dim() == 3 else rows.unsqueeze(0)
    r = r.contiguous()
    if int(r.shape[-1]) != D:
        raise ValueError(f"row width {int(r.shape[-1])} != hidden width {D}")
    if int(r.shape[0]) not in (1, B):
        raise ValueError(f"rows batch {int(r.shape[0])} vs hidden batch {B}")
    n_rows = int(r.shape[1])
    bstride = 0 if (int(r.shape[0]) == 1 and B > 1) else n_rows * D
    lib = capi.load()
    st = torch.cuda.current_stream(hidden.device).cuda_stream
    capi.check(lib.qvl_scatter_vision_rows(st, int(mode), _qdtype(hidden), hidden.data_ptr(), B, S, D, _qdtype(r),
                                           r.data_ptr(), bstride, n_rows, pos.data_ptr(), count.data_ptr()),
               "qvl_scatter_vision_rows")
    return hidden


def inject_vision(hidden, tokens, vision_embeds, image_pad_id: int):
    """`forward_vlm` up to the decoder (model.py:915-936): normalise the vision input (a
    VisionEmbeddings or a [V, D] / [B, V, D] array) to the hidden dtype and batch, write its tokens
    over the first V <|image_pad|> rows of each batch row (in place), and return (hidden,
    visual_mask, deepstack features)."""
    torch = _torch()
    B = int(hidden.shape[0])
    if isinstance(vision_embeds, VisionEmbeddings):
        pack = vision_embeds.with_batch_dim(B)
        vis, deepstack = pack.tokens, tuple(pack.deepstack)
    else:
        vis = torch.as_tensor(vision_embeds, device=hidden.device)
        if vis.dim() == 2:
            vis = vis.unsqueeze(0)
        deepstack = ()
    tokens = torch.as_tensor(tokens, device=hidden.device)
    if tokens.dim() == 1:
        tokens = tokens.unsqueeze(0)
    visual_mask = tokens == int(image_pad_id)
    pos, count = vision_positions(tokens, int(vis.shape[1]), match=int(image_pad_id))
    scatter_rows(hidden, vis, pos, count, capi.QVL_SCATTER_SET)
    return hidden, visual_mask, deepstack


def apply_deepstack(hidden, visual_mask: Optional[object], features):
    """`_apply_deepstack` (model.py:874-886): hidden[b, mask positions][:F] += features[b] (in the
    hidden dtype), in place. No-op without a mask or with empty features."""
    if visual_mask is None or features.numel() == 0:
        return hidden
    f = features if features.dim() == 3 else features.unsqueeze(0)
    if int(f.shape[1]) == 0:
        return hidden
    pos, count = vision_positions(visual_mask, int(f.shape[1]))
    return scatter_rows(hidden, f, pos, count, capi.QVL_SCATTER_ADD)

