"""Image preprocessing on the GPU: the reference's `preprocess_image` (sample.py:51-121).

Host side (as in the reference): load / convert to RGB / `smart_resize` / PIL bicubic resize.
Device side (`qvl_patchify`): normalisation ((x/255 - 0.5) / 0.5 in float32), temporal padding
and the merge-block patch layout, written straight into the pixel_values buffer the tower reads.
"""
from __future__ import annotations

import math
from typing import Any, Tuple, Union

import numpy as np

from . import capi

# sample.py:22-25
IMAGE_MEAN = np.array([0.5, 0.5, 0.5], dtype=np.float32)
IMAGE_STD = np.array([0.5, 0.5, 0.5], dtype=np.float32)
DEFAULT_MIN_PIXELS = 56 * 56
DEFAULT_MAX_PIXELS = 12845056


def smart_resize(height: int, width: int, factor: int, min_pixels: int, max_pixels: int) -> Tuple[int, int]:
    """Target (height, width): multiples of `factor` near the input size with the pixel count in
    [min_pixels, max_pixels] (sample.py:28-48, same integer/float steps and errors)."""
    if height <= 0 or width <= 0:
        raise ValueError("Image dimensions must be positive")
    if min(height, width) == 0 or (max(height, width) / min(height, width)) > 200:
        raise ValueError("Aspect ratio must be < 200")
    h_bar = max(factor, round(height / factor) * factor)
    w_bar = max(factor, round(width / factor) * factor)
    area = h_bar * w_bar
    if area > max_pixels:
        beta = math.sqrt((height * width) / max_pixels)
        h_bar = max(factor, math.floor(height / beta / factor) * factor)
        w_bar = max(factor, math.floor(width / beta / factor) * factor)
    elif area < min_pixels:
        beta = math.sqrt(min_pixels / (height * width))
        h_bar = max(factor, math.ceil(height * beta / factor) * factor)
        w_bar = max(factor, math.ceil(width * beta / factor) * factor)
    return int(h_bar), int(w_bar)


def _torch():
    import torch
    return torch


def patchify_frames(frames, patch_size: int, spatial_merge_size: int, temporal_patch_size: int,
                    dtype: str = "float32", device: str = "cuda:0"):
    """uint8 frames [F, H, W, C] (C = 3 or 4; numpy or a torch tensor) -> (pixel_values [N, 3*Tp*P*P]
    on `device` in `dtype`, grid_thw int32 [[gt, gh, gw]]), the array half of sample.py:86-121.

    F frames are padded to a multiple of Tp by repeating the last one (sample.py:93-98); a single
    image is F = 1. `dtype` "float32" is the reference's pixel_values; "bfloat16" is the same values
    rounded to nearest even (what the tower's patch embed casts them to, model.py:556)."""
    torch = _torch()
    if dtype not in ("float32", "bfloat16"):
        raise ValueError(f"dtype {dtype!r}")
    if isinstance(frames, np.ndarray):
        if frames.dtype != np.uint8:
            raise TypeError("frames must be uint8 (the reference converts through PIL RGB, sample.py:62-76)")
        arr = np.ascontiguousarray(frames)
        if not arr.flags.writeable:        # e.g. np.asarray of a PIL image; torch wants a writable buffer
            arr = arr.copy()
        t = torch.from_numpy(arr).to(device)
    else:
        if frames.dtype != torch.uint8:
            raise TypeError("frames must be uint8")
        t = frames.to(device).contiguous()
    if t.dim() == 3:
        t = t.unsqueeze(0)
    if t.dim() != 4 or t.shape[-1] not in (3, 4):
        raise ValueError("Expected frames [F, H, W, C] with 3 or 4 channels")
    F, H, W, Cin = (int(s) for s in t.shape)
    P, Tp, m = int(patch_size), int(temporal_patch_size), int(spatial_merge_size)
    gt = -(-F // Tp)
    gh, gw = H // P, W // P
    if gh == 0 or gw == 0:
        raise ValueError("Image too small for patch size")
    if gh * P != H or gw * P != W:
        raise ValueError("Dimensions must be divisible by patch_size")
    if gh % m or gw % m:
        raise ValueError("Grid must be divisible by spatial_merge_size")
    K = 3 * Tp * P * P
    out = torch.empty((gt * gh * gw, K), dtype=torch.float32 if dtype == "float32" else torch.bfloat16,
                      device=device)
    lib = capi.load()
    qd = capi.QVL_DTYPE_F32 if dtype == "float32" else capi.QVL_DTYPE_BF16
    st = torch.cuda.current_stream(t.device).cuda_stream
    capi.check(lib.qvl_patchify(st, qd, t.data_ptr(), F, H, W, Cin, P, Tp, m, out.data_ptr(), K), "qvl_patchify")
    return out, np.array([[gt, gh, gw]], dtype=np.int32)


def preprocess_image(image: Union[str, Any], patch_size: int, spatial_merge_size: int, temporal_patch_size: int,
                     min_pixels: int = DEFAULT_MIN_PIXELS, max_pixels: int = DEFAULT_MAX_PIXELS,
                     dtype: str = "float32", device: str = "cuda:0"):
    """Path, PIL image or HWC array -> (pixel_values [N, patch_volume] on `device`, grid_thw [[t, h, w]]),
    like sample.py:51-121: the load, RGB conversion, smart_resize and bicubic resize run on the
    host with PIL (as in the reference), the rest in `qvl_patchify`."""
    import os
    from PIL import Image

    if isinstance(image, str):
        if not os.path.exists(image):
            raise FileNotFoundError(f"Image not found: {image}")
        with Image.open(image) as img:
            pil_img = img.convert("RGB")
    elif hasattr(image, "convert"):
        pil_img = image.convert("RGB")
    else:
        arr = np.asarray(image)
        if arr.ndim != 3 or arr.shape[2] not in (3, 4):
            raise ValueError("Expected HWC array with 3 or 4 channels")
        if arr.shape[2] == 4:
            arr = arr[:, :, :3]
        pil_img = Image.fromarray(arr.astype(np.uint8), mode="RGB")
    width, height = pil_img.size
    factor = patch_size * spatial_merge_size
    new_h, new_w = smart_resize(height, width, factor, min_pixels, max_pixels)
    if (new_w, new_h) != (width, height):
        pil_img = pil_img.resize((new_w, new_h), Image.Resampling.BICUBIC)
    frames = np.asarray(pil_img, dtype=np.uint8)[None]          # [1, H, W, 3]
    return patchify_frames(frames, patch_size, spatial_merge_size, temporal_patch_size, dtype, device)
