"""Load-time weight handling for the vision tower (model.py:1071-1160).

* `torch_key_to_flax` / `load_hf_vision_params`: HuggingFace safetensors (torch names, Linear
  weights [out, in], Conv3d patch embed [D, C, Tp, P, P]) -> the reference's Flax tree under
  "visual" (kernels [in, out]; the patch-embed kernel [C*Tp*P*P, D]), the vision half of
  `create_model_from_hf` (model.py:1105-1160) and its key rules (model.py:1071-1103).
* `load_hf_vision`: config.json + safetensors -> (VisionBackboneSpec, params), through
  `spec_from_config` (model.py:981-1049).
* `save_packed` / `load_packed`: the tower's device-ready buffers (weights packed to [n_out, k_in]
  in the tower dtype, zero-padded to 64; fp32 biases / LayerNorm vectors; the pos-embed table) in
  one safetensors file with a JSON header naming the format, dtype and spec. Loading copies the
  buffers straight to the GPU and binds them: no transposes or packing at load time.
"""
from __future__ import annotations

import dataclasses
import glob
import json
import os
import re
from typing import Dict, Optional, Tuple

import numpy as np

from .vision import Qwen3VisionTransformer, VisionBackboneSpec, spec_from_config

PACKED_FORMAT = "qvl-packed-vision"
PACKED_VERSION = "1"

# The vision key rules of model.py:1071-1089 (torch name regex -> Flax path), same targets.
_VISION_RULES = [
    (r"(model\.)?visual\.blocks\.(\d+)\.(norm1|norm2)\.(weight|bias)", r"visual/blocks_\2/\3/\4"),
    (r"(model\.)?visual\.blocks\.(\d+)\.attn\.(qkv|proj)\.weight", r"visual/blocks_\2/attn/\3/kernel"),
    (r"(model\.)?visual\.blocks\.(\d+)\.attn\.(qkv|proj)\.bias", r"visual/blocks_\2/attn/\3/bias"),
    (r"(model\.)?visual\.blocks\.(\d+)\.mlp\.linear_fc1\.(weight|bias)", r"visual/blocks_\2/mlp/linear_fc1/\3"),
    (r"(model\.)?visual\.blocks\.(\d+)\.mlp\.linear_fc2\.(weight|bias)", r"visual/blocks_\2/mlp/linear_fc2/\3"),
    (r"(model\.)?visual\.blocks\.(\d+)\.mlp\.(gate|up|down)_proj\.weight", r"visual/blocks_\2/mlp/\3_proj/kernel"),
    (r"(model\.)?visual\.blocks\.(\d+)\.mlp\.(gate|up|down)_proj\.bias", r"visual/blocks_\2/mlp/\3_proj/bias"),
    (r"(model\.)?visual\.patch_embed\.proj\.weight", "visual/patch_embed/proj/kernel"),
    (r"(model\.)?visual\.patch_embed\.proj\.bias", "visual/patch_embed/proj/bias"),
    (r"(model\.)?visual\.pos_embed\.weight", "visual/pos_embed/embedding"),
    (r"(model\.)?visual\.merger\.norm\.(weight|bias)", r"visual/merger/norm/\2"),
    (r"(model\.)?visual\.merger\.linear_fc1\.(weight|bias)", r"visual/merger/linear_fc1/\2"),
    (r"(model\.)?visual\.merger\.linear_fc2\.(weight|bias)", r"visual/merger/linear_fc2/\2"),
    (r"(model\.)?visual\.deepstack_merger_list\.(\d+)\.norm\.(weight|bias)", r"visual/deepstack_mergers_\2/norm/\3"),
    (r"(model\.)?visual\.deepstack_merger_list\.(\d+)\.linear_fc1\.(weight|bias)",
     r"visual/deepstack_mergers_\2/linear_fc1/\3"),
    (r"(model\.)?visual\.deepstack_merger_list\.(\d+)\.linear_fc2\.(weight|bias)",
     r"visual/deepstack_mergers_\2/linear_fc2/\3"),
]


def torch_key_to_flax(key: str) -> Optional[str]:
    """Flax path of a HF vision parameter name, or None (model.py:1091-1103: first matching rule;
    a "/weight" leaf outside norms and embeddings becomes "/kernel")."""
    for pattern, target in _VISION_RULES:
        if re.match(pattern, key):
            flax_key = re.sub(pattern, target, key)
            if flax_key.endswith("/weight"):
                parts = flax_key.split("/")
                if not any("norm" in q for q in parts) and not any("embed" in q for q in parts):
                    flax_key = flax_key[: -len("/weight")] + "/kernel"
            return flax_key
    return None


def _safetensor_files(path: str):
    if os.path.isdir(path):
        files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    else:
        files = [path]
    if not files:
        raise FileNotFoundError(f"No safetensors in {path}")
    return files


def load_hf_vision_params(path: str) -> Dict:
    """HF checkpoint (a .safetensors file or a directory of them) -> {"visual": Flax tree} as
    float32 numpy, like the vision part of model.py:1130-1153: the Conv3d patch-embed weight is
    flattened to [D, C*Tp*P*P] and transposed, Linear weights are transposed to [in, out]."""
    from safetensors import safe_open

    params: Dict = {}
    for fname in _safetensor_files(path):
        with safe_open(fname, framework="pt", device="cpu") as f:
            for key in f.keys():
                if "patch_embed.proj.weight" in key:
                    t = f.get_tensor(key).float().numpy()
                    kernel = np.ascontiguousarray(t.reshape(t.shape[0], -1).T)
                    params.setdefault("visual", {}).setdefault("patch_embed", {}).setdefault("proj", {})["kernel"] = kernel
                    continue
                target = torch_key_to_flax(key)
                if target is None:
                    continue
                t = f.get_tensor(key).float().numpy()
                keys = target.split("/")
                d = params
                for k in keys[:-1]:
                    d = d.setdefault(k, {})
                d[keys[-1]] = np.ascontiguousarray(t.T) if "kernel" in keys[-1] else t
    if "visual" not in params:
        raise ValueError(f"no vision parameters in {path}")
    return params


def load_hf_vision(hf_dir: str) -> Tuple[VisionBackboneSpec, Dict]:
    """A HF checkpoint directory (config.json + *.safetensors) -> (vision spec, {"visual": params}):
    the vision half of `create_model_from_hf` (model.py:1105-1160), the spec from config.json
    through spec_from_config (model.py:981-1049). Raises ValueError when the config has no
    vision backbone."""
    with open(os.path.join(hf_dir, "config.json")) as f:
        cfg = json.load(f)
    spec = spec_from_config(cfg).vision
    if spec is None:
        raise ValueError(f"{hf_dir}/config.json has no vision_config")
    return spec, load_hf_vision_params(hf_dir)


def spec_to_json(spec: VisionBackboneSpec) -> str:
    """The spec as the packed file's header stores it (sequences as lists, None kept as null)."""
    d = dataclasses.asdict(spec)
    return json.dumps({k: (list(v) if isinstance(v, (tuple, list)) else v) for k, v in d.items()}, sort_keys=True)


def spec_from_json(text: str) -> VisionBackboneSpec:
    """Inverse of spec_to_json. `fullatt_block_indexes` keeps None ("every block is full
    attention") distinct from an empty list (window attention on every block)."""
    d = json.loads(text)
    fa = d.get("fullatt_block_indexes")
    d["fullatt_block_indexes"] = None if fa is None else tuple(fa)
    d["deepstack_visual_indexes"] = tuple(d.get("deepstack_visual_indexes") or ())
    return VisionBackboneSpec(**d)


def save_packed(tower: Qwen3VisionTransformer, path: str) -> None:
    """Write the bound tower's device buffers to `path` (safetensors + JSON metadata)."""
    from safetensors.torch import save_file

    state = {k: v.detach().contiguous().cpu() for k, v in tower.packed_state().items()}
    meta = {"format": PACKED_FORMAT, "version": PACKED_VERSION, "dtype": tower.dtype,
            "layout": "dense weights [n_out_pad64, k_in_pad64] row-major in dtype; vectors float32",
            "spec": spec_to_json(tower.spec)}
    save_file(state, path, metadata=meta)


def read_packed_metadata(path: str) -> Dict[str, str]:
    from safetensors import safe_open

    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
    if meta.get("format") != PACKED_FORMAT:
        raise ValueError(f"{path}: not a {PACKED_FORMAT} file")
    if meta.get("version") != PACKED_VERSION:
        raise ValueError(f"{path}: packed format version {meta.get('version')} (this build reads {PACKED_VERSION})")
    return meta


def load_packed(path: str, device: str = "cuda:0") -> Qwen3VisionTransformer:
    """A bound tower from a `save_packed` file: spec and dtype from its header, buffers copied to
    `device` as stored."""
    from safetensors.torch import load_file

    meta = read_packed_metadata(path)
    spec = spec_from_json(meta["spec"])
    tower = Qwen3VisionTransformer(spec, dtype=meta["dtype"], device=device)
    state = load_file(path, device=device)
    return tower.bind_packed(state)
