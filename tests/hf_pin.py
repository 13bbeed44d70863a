"""Build transformers' Qwen3VLVisionModel with the oracle's weights (an independent implementation
of the same tower, used to pin the oracle). Helper for tests/test_oracle_float.py,
tests/test_oracle_io.py and tests/test_gpu_io.py."""
import numpy as np


def hf_vision_model(params, spec, dtype="float64"):
    import torch
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig
    from transformers.models.qwen3_vl.modeling_qwen3_vl import Qwen3VLVisionModel

    cfg = Qwen3VLVisionConfig(
        depth=spec.depth, hidden_size=spec.hidden_size, hidden_act="gelu_pytorch_tanh",
        intermediate_size=spec.intermediate_size, num_heads=spec.num_heads, in_channels=spec.in_channels,
        patch_size=spec.patch_size, spatial_merge_size=spec.spatial_merge_size,
        temporal_patch_size=spec.temporal_patch_size, out_hidden_size=spec.out_hidden_size,
        num_position_embeddings=spec.num_position_embeddings,
        deepstack_visual_indexes=list(spec.deepstack_visual_indexes))
    cfg._attn_implementation = "sdpa"
    m = Qwen3VLVisionModel(cfg).eval()
    prm = params.get("visual", params)
    D = spec.hidden_size
    sd = {}

    def lin(prefix, p):
        sd[prefix + ".weight"] = np.ascontiguousarray(p["kernel"].T)
        sd[prefix + ".bias"] = p["bias"]

    def ln(prefix, p):
        sd[prefix + ".weight"] = p["weight"]
        sd[prefix + ".bias"] = p["bias"]

    pe = prm["patch_embed"]["proj"]
    sd["patch_embed.proj.weight"] = pe["kernel"].T.reshape(D, spec.in_channels, spec.temporal_patch_size,
                                                           spec.patch_size, spec.patch_size)
    sd["patch_embed.proj.bias"] = pe["bias"]
    sd["pos_embed.weight"] = prm["pos_embed"]["embedding"]
    for i in range(spec.depth):
        b = prm[f"blocks_{i}"]
        ln(f"blocks.{i}.norm1", b["norm1"]); ln(f"blocks.{i}.norm2", b["norm2"])
        lin(f"blocks.{i}.attn.qkv", b["attn"]["qkv"]); lin(f"blocks.{i}.attn.proj", b["attn"]["proj"])
        lin(f"blocks.{i}.mlp.linear_fc1", b["mlp"]["linear_fc1"]); lin(f"blocks.{i}.mlp.linear_fc2", b["mlp"]["linear_fc2"])
    for name, key in [("merger", "merger")] + [(f"deepstack_merger_list.{j}", f"deepstack_mergers_{j}")
                                               for j in range(len(spec.deepstack_visual_indexes))]:
        ln(f"{name}.norm", prm[key]["norm"])
        lin(f"{name}.linear_fc1", prm[key]["linear_fc1"]); lin(f"{name}.linear_fc2", prm[key]["linear_fc2"])
    tdt = getattr(torch, dtype)
    state = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)).to(tdt) for k, v in sd.items()}
    missing, unexpected = m.load_state_dict(state, strict=False)
    missing = [k for k in missing if "inv_freq" not in k]
    assert not missing and not unexpected, (missing, unexpected)
    # jax.nn.gelu defaults to the tanh approximation in every merger (model.py:655); transformers'
    # merger uses exact GELU, so align it to the reference.
    for mod in [m.merger, *m.deepstack_merger_list]:
        mod.act_fn = torch.nn.GELU(approximate="tanh")
    return m.to(tdt)


def hf_encode(model, pixel_values, grid_thw, taps=None, dtype="float64"):
    """Run the HF tower; `taps` = (idx [4,N], w [4,N]) overrides its pos-embed interpolation."""
    import torch
    tdt = getattr(torch, dtype)
    kw = {}
    if taps is not None:
        kw["interp_indices"] = torch.from_numpy(np.ascontiguousarray(taps[0].T).astype(np.int64))
        kw["interp_weights"] = torch.from_numpy(np.ascontiguousarray(taps[1].T)).to(tdt)
    with torch.no_grad():
        out = model(torch.from_numpy(np.asarray(pixel_values, np.float64)).to(tdt),
                    torch.tensor(np.asarray(grid_thw), dtype=torch.int64), **kw)
    return (out.pooler_output.double().numpy(), tuple(f.double().numpy() for f in out.deepstack_features))
