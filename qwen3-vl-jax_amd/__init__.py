"""MI355X (gfx950) drop-in for the Qwen3-VL vision tower (`encode_vision`) of sdan/Qwen3-VL-JAX.

Imported as `qwen3_vl_jax_amd` (the directory name `qwen3-vl-jax_amd` is not a Python identifier;
`__graft_entry__.load_package()` registers it). The HIP kernels and C ABI live in `csrc/` and
build into `libqvl.so` next to this file (`build.py`).
"""
from . import capi
from .vision import (GridMetadata, Qwen3VisionTransformer, Qwen3VLModel, Qwen3VLSpec, VisionBackboneSpec,
                     VisionEmbeddings, attention_worklist_split, grid_metadata, random_params, spec_2b, spec_8b,
                     spec_from_config, vision_spec_from_config)
from . import decoder_io, preprocess, vision, weights

__all__ = ["capi", "GridMetadata", "Qwen3VisionTransformer", "Qwen3VLModel", "Qwen3VLSpec", "VisionBackboneSpec",
           "VisionEmbeddings", "attention_worklist_split", "grid_metadata", "random_params", "spec_2b", "spec_8b",
           "spec_from_config", "vision_spec_from_config", "decoder_io", "preprocess", "weights"]
