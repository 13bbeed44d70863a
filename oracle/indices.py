"""Integer metadata of the vision tower, restated from the reference (TEST INFRASTRUCTURE ONLY).

Everything here is host-side numpy, exactly as the reference builds it before the device work:

* `cu_seqlens_ref`      model.py:825-834  (full-attention branch: one segment per frame)
* `rot_pos_ids_ref`     model.py:682-698  ((h, w) ids in 2x2 merge-block order, tiled over t)
* `rotary_half_ref`     model.py:540-546, 694-698 (inv_freq table, gather, [h-freqs, w-freqs])
* `pos_embed_taps_ref`  model.py:700-767  (4 bilinear taps per raster patch, then the
                        `jnp.repeat(.., t, axis=0)` frame expansion and the merge-block reshape)
* `window_index_ref`    model.py:769-799  (window order of merge groups, cu_window) and
  `cu_full_window_ref`  model.py:828-830  (the window path's full-attention cu_seqlens)

The `*_closed` functions are the same quantities written as closed forms of the token index; the
tests check each `*_ref` against its closed form on every small grid, so a slip in either
(a transposed reshape, a wrong repeat axis) fails.
"""
from __future__ import annotations

import numpy as np


def _grid(grid_thw):
    g = np.asarray(grid_thw, dtype=np.int64).reshape(-1, 3)
    return g


# ---------------------------------------------------------------------------------------------
# cu_seqlens (model.py:831-834)
# ---------------------------------------------------------------------------------------------
def cu_seqlens_ref(grid_thw) -> np.ndarray:
    """`[0] ++ cumsum(repeat(h*w, t))` as int32 (model.py:831-834)."""
    g = _grid(grid_thw)
    frame_sizes = np.repeat(g[:, 1] * g[:, 2], g[:, 0])
    return np.concatenate([np.zeros(1, np.int32), np.cumsum(frame_sizes, dtype=np.int32)]).astype(np.int32)


def cu_seqlens_closed(grid_thw) -> np.ndarray:
    out = [0]
    for t, h, w in _grid(grid_thw):
        for _ in range(int(t)):
            out.append(out[-1] + int(h) * int(w))
    return np.asarray(out, dtype=np.int32)


# ---------------------------------------------------------------------------------------------
# rotary (h, w) position ids (model.py:682-693)
# ---------------------------------------------------------------------------------------------
def rot_pos_ids_ref(grid_thw, merge: int = 2) -> np.ndarray:
    """[N, 2] int32 (h, w) per token, merge-block order, tiled over frames (model.py:686-693)."""
    chunks = []
    for t, h, w in _grid(grid_thw):
        t, h, w = int(t), int(h), int(w)
        hpos = np.repeat(np.arange(h)[:, None], w, axis=1)
        wpos = np.repeat(np.arange(w)[None, :], h, axis=0)
        hpos = hpos.reshape(h // merge, merge, w // merge, merge).transpose(0, 2, 1, 3).reshape(-1)
        wpos = wpos.reshape(h // merge, merge, w // merge, merge).transpose(0, 2, 1, 3).reshape(-1)
        pos = np.stack([hpos, wpos], axis=-1)
        chunks.append(np.tile(pos, (t, 1)))
    if not chunks:
        return np.zeros((0, 2), np.int32)
    return np.concatenate(chunks, axis=0).astype(np.int32)


def token_coords_closed(grid_thw, merge: int = 2):
    """Per token n: (frame f, row, col) from the merge-block order closed form.

    Local index n in an image of (t,h,w): f = n // (h*w), r = n % (h*w), g = r // m^2,
    hb = g // (w/m), wb = g % (w/m), mi = (r % m^2) // m, mj = r % m; row = m*hb+mi, col = m*wb+mj.
    """
    fs, rows, cols = [], [], []
    mm = merge * merge
    for t, h, w in _grid(grid_thw):
        n = np.arange(int(t) * int(h) * int(w))
        f = n // (h * w)
        r = n % (h * w)
        g = r // mm
        hb = g // (w // merge)
        wb = g % (w // merge)
        mi = (r % mm) // merge
        mj = r % merge
        fs.append(f); rows.append(merge * hb + mi); cols.append(merge * wb + mj)
    if not fs:
        z = np.zeros(0, np.int64)
        return z, z, z
    return np.concatenate(fs), np.concatenate(rows), np.concatenate(cols)


def rot_pos_ids_closed(grid_thw, merge: int = 2) -> np.ndarray:
    _, rows, cols = token_coords_closed(grid_thw, merge)
    return np.stack([rows, cols], axis=-1).astype(np.int32)


def rotary_inv_freq(head_dim: int, theta: float = 10000.0) -> np.ndarray:
    """VisionRotaryEmbedding.inv_freq with dim = head_dim // 2 (model.py:544, 672), float32."""
    dim = head_dim // 2
    return (np.float32(1.0) / (np.float32(theta) ** (np.arange(0, dim, 2, dtype=np.float32) / np.float32(dim)))).astype(np.float32)


def rotary_half_ref(grid_thw, head_dim: int, merge: int = 2, theta: float = 10000.0) -> np.ndarray:
    """[N, head_dim/2] float32 angles: [h-freqs | w-freqs] (model.py:694-698, 545-546)."""
    pos = rot_pos_ids_ref(grid_thw, merge)
    g = _grid(grid_thw)
    if pos.shape[0] == 0:
        return np.zeros((0, head_dim // 2), np.float32)
    max_grid = int(g[:, 1:].max())
    inv = rotary_inv_freq(head_dim, theta)
    table = np.outer(np.arange(max_grid, dtype=np.float32), inv).astype(np.float32)
    return table[pos].reshape(pos.shape[0], -1)


# ---------------------------------------------------------------------------------------------
# learned pos-embed bilinear taps (model.py:700-767)
# ---------------------------------------------------------------------------------------------
def _raster_taps(h: int, w: int, num_grid: int):
    """4 taps/weights over the raster h*w grid of one image (model.py:713-739)."""
    h_idxs = np.linspace(0, num_grid - 1, h, dtype=np.float32)
    w_idxs = np.linspace(0, num_grid - 1, w, dtype=np.float32)
    h_floor = h_idxs.astype(np.int32)
    w_floor = w_idxs.astype(np.int32)
    h_ceil = np.clip(h_floor + 1, 0, num_grid - 1)
    w_ceil = np.clip(w_floor + 1, 0, num_grid - 1)
    dh = h_idxs - h_floor
    dw = w_idxs - w_floor
    base_h = h_floor * num_grid
    base_h_ceil = h_ceil * num_grid
    idx = np.stack([
        (base_h[:, None] + w_floor[None]).reshape(-1),
        (base_h[:, None] + w_ceil[None]).reshape(-1),
        (base_h_ceil[:, None] + w_floor[None]).reshape(-1),
        (base_h_ceil[:, None] + w_ceil[None]).reshape(-1),
    ]).astype(np.int32)
    wts = np.stack([
        ((1.0 - dh)[:, None] * (1.0 - dw)[None]).reshape(-1),
        ((1.0 - dh)[:, None] * dw[None]).reshape(-1),
        (dh[:, None] * (1.0 - dw)[None]).reshape(-1),
        (dh[:, None] * dw[None]).reshape(-1),
    ]).astype(np.float32)
    return idx, wts


def pos_embed_rows_ref(t: int, h: int, w: int, merge: int = 2) -> np.ndarray:
    """Raster row (of the h*w interpolated table) feeding each token of one image/video.

    Applies the reference's exact chain to an arange: `jnp.repeat(pe, t, axis=0)` (the t>1
    quirk: each raster row repeated t times in place), then reshape (t, h/m, m, w/m, m) and
    transpose (0, 1, 3, 2, 4) (model.py:761-764).
    """
    rows = np.arange(h * w)
    if t > 1:
        rows = np.repeat(rows, t, axis=0)
    rows = rows.reshape(t, h // merge, merge, w // merge, merge)
    return rows.transpose(0, 1, 3, 2, 4).reshape(-1)


def pos_embed_taps_ref(grid_thw, num_position_embeddings: int = 2304, merge: int = 2):
    """Per-token taps: (idx [4, N] int32, weights [4, N] float32) after the quirk + merge order."""
    num_grid = int(num_position_embeddings ** 0.5)
    idx_c, w_c = [], []
    for t, h, w in _grid(grid_thw):
        t, h, w = int(t), int(h), int(w)
        idx, wts = _raster_taps(h, w, num_grid)
        rows = pos_embed_rows_ref(t, h, w, merge)
        idx_c.append(idx[:, rows]); w_c.append(wts[:, rows])
    if not idx_c:
        return np.zeros((4, 0), np.int32), np.zeros((4, 0), np.float32)
    return np.concatenate(idx_c, axis=1), np.concatenate(w_c, axis=1)


def pos_embed_rows_closed(t: int, h: int, w: int, merge: int = 2) -> np.ndarray:
    """Closed form of `pos_embed_rows_ref`: E[i] = P[i // t], i = f*h*w + row*w + col."""
    f, rows, cols = token_coords_closed([[t, h, w]], merge)
    i = f * h * w + rows * w + cols
    return (i // t).astype(np.int64)


# ---------------------------------------------------------------------------------------------
# spatial merge (model.py:650, 654): merged row G = concat(x[4G], x[4G+1], x[4G+2], x[4G+3])
# ---------------------------------------------------------------------------------------------
def merge_source_rows(n_tokens: int, merge: int = 2) -> np.ndarray:
    """[N/m^2, m^2] token rows gathered into each merged row: a plain reshape in the reference."""
    mm = merge * merge
    return np.arange(n_tokens).reshape(-1, mm)


def merged_row_closed(grid_thw, merge: int = 2) -> np.ndarray:
    """Merged row index G of each token n (the patch block it falls in), from (f, row, col)."""
    out = []
    off = 0
    for t, h, w in _grid(grid_thw):
        f, rows, cols = token_coords_closed([[t, h, w]], merge)
        G = off // (merge * merge) + (f * (h // merge) + rows // merge) * (w // merge) + cols // merge
        out.append(G)
        off += int(t * h * w)
    return np.concatenate(out) if out else np.zeros(0, np.int64)


def window_index_ref(grid_thw, merge: int, patch: int, window_size: int):
    """`_get_window_index` (model.py:769-799): pad each frame's merge-group grid to whole windows
    with -100, reshape/transpose into windows, drop the padding. Returns (window_index, cu_window)."""
    vw = window_size // merge // patch
    idxs, cu, wid = [], [0], 0
    for t, h, w in _grid(grid_thw):
        gh, gw = h // merge, w // merge
        index = np.arange(t * gh * gw).reshape(t, gh, gw)
        ph, pw = (vw - gh % vw) % vw, (vw - gw % vw) % vw
        nh, nw = (gh + ph) // vw, (gw + pw) // vw
        pad = np.pad(index, ((0, 0), (0, ph), (0, pw)), constant_values=-100)
        pad = pad.reshape(t, nh, vw, nw, vw).transpose(0, 1, 3, 2, 4).reshape(t, nh * nw, vw, vw)
        seqlens = (pad != -100).sum(axis=(2, 3)).reshape(-1)
        flat = pad.reshape(-1)
        idxs.append(flat[flat != -100] + wid)
        cu.extend(list(np.cumsum(seqlens) * merge * merge + cu[-1]))
        wid += int(t * gh * gw)
    cu = np.asarray(cu, np.int64)
    keep = np.concatenate([[True], cu[1:] != cu[:-1]])
    widx = np.concatenate(idxs) if idxs else np.zeros(0, np.int64)
    return widx.astype(np.int64), cu[keep]


def window_index_closed(grid_thw, merge: int, patch: int, window_size: int):
    """Window id and window-order position of every merge group, from its (frame, row, col):
    window = (frame, row // vw, col // vw) numbered frame-major then row-major over the padded
    window grid; inside a window, groups are row-major. Returns (window_index, cu_window)."""
    vw = window_size // merge // patch
    keyed, sizes, wid, win_off = [], [], 0, 0
    for t, h, w in _grid(grid_thw):
        gh, gw = h // merge, w // merge
        nh, nw = -(-gh // vw), -(-gw // vw)
        for f in range(t):
            for r in range(gh):
                for c in range(gw):
                    win = win_off + (f * nh + r // vw) * nw + c // vw
                    keyed.append((win, (r % vw) * vw + c % vw, wid + (f * gh + r) * gw + c))
        for f in range(t):
            for a in range(nh):
                for b in range(nw):
                    sizes.append(min(vw, gh - a * vw) * min(vw, gw - b * vw))
        win_off += t * nh * nw
        wid += t * gh * gw
    keyed.sort()
    cu = np.concatenate([[0], np.cumsum(sizes) * merge * merge])
    keep = np.concatenate([[True], cu[1:] != cu[:-1]])
    return np.asarray([k[2] for k in keyed], np.int64), cu[keep]


def cu_full_window_ref(grid_thw, merge: int) -> np.ndarray:
    """model.py:828-830: [0, cumsum(t*h*w*merge^2)] — in tokens times merge^2 — with each bound
    clamped to n_tokens as the reference's q[start:end] slicing clamps it."""
    g = _grid(grid_thw)
    n = int((g[:, 0] * g[:, 1] * g[:, 2]).sum())
    cu = np.concatenate([[0], np.cumsum(g[:, 0] * g[:, 1] * g[:, 2] * merge * merge)])
    return np.minimum(cu, n)


def attention_tiles(cu_seqlens, block_m: int, num_heads: int = 1, queues: int = 8):
    """Work list of (segment start, segment end, q0, head) items, dealt to `queues` queues.

    Not a reference quantity: the schedule the HIP attention kernel walks. (segment, head)
    groups, longest segment first (stable), each go whole to the queue with the least work so far
    (work = query tiles x keys; ties to the lowest queue); item k is entry k // queues of queue
    k % queues; short queues are padded with (0, 0, 0, 0). Every query row of every non-empty
    segment must appear in exactly one item per head.
    """
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    segs = [(int(cu[i]), int(cu[i + 1])) for i in range(len(cu) - 1) if cu[i + 1] > cu[i]]
    segs.sort(key=lambda s: -(s[1] - s[0]))
    qs = [[] for _ in range(queues)]
    load = [0] * queues
    for s, e in segs:
        ntile = -(-(e - s) // block_m)
        for h in range(num_heads):
            qi = min(range(queues), key=lambda j: (load[j], j))
            load[qi] += ntile * (e - s)
            qs[qi].extend((s, e, q0, h) for q0 in range(s, e, block_m))
    longest = max((len(q) for q in qs), default=0)
    items = [qs[k % queues][k // queues] if k // queues < len(qs[k % queues]) else (0, 0, 0, 0)
             for k in range(longest * queues)]
    return np.asarray(items, dtype=np.int32).reshape(-1, 4)
