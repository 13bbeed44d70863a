"""CPU tests of the host-side spec handling: spec_from_config (model.py:987-1049, vision branch),
load_hf_vision (config.json + safetensors) and the packed file's spec header round trip."""
import json

import numpy as np
import pytest


def hf_config(vision: dict, mrope=(24, 20, 20)) -> dict:
    """A Qwen3-VL style top-level HF config around `vision`."""
    return {"model_type": "qwen3_vl", "vision_config": vision,
            "text_config": {"hidden_size": 2048, "num_attention_heads": 16, "num_hidden_layers": 28,
                            "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 6144,
                            "rms_norm_eps": 1e-6, "vocab_size": 151936,
                            "rope_scaling": {"mrope_section": list(mrope), "mrope_interleaved": True}},
            "pad_token_id": 151643, "bos_token_id": 151643, "eos_token_id": 151645}


VISION_2B = {"model_type": "qwen3_vl", "depth": 24, "hidden_size": 1024, "intermediate_size": 4096,
             "num_heads": 16, "in_channels": 3, "patch_size": 16, "spatial_merge_size": 2, "temporal_patch_size": 2,
             "out_hidden_size": 2048, "num_position_embeddings": 2304, "deepstack_visual_indexes": [5, 11, 17]}
VISION_8B = dict(VISION_2B, depth=27, hidden_size=1152, intermediate_size=4304, out_hidden_size=4096,
                 deepstack_visual_indexes=[8, 16, 24])
VISION_QWEN25 = {"model_type": "qwen2_5_vl", "depth": 32, "hidden_size": 1280, "intermediate_size": 3420,
                 "num_heads": 16, "in_chans": 3, "spatial_patch_size": 14, "spatial_merge_size": 2,
                 "temporal_patch_size": 2, "window_size": 112, "out_hidden_size": 2048,
                 "fullatt_block_indexes": [7, 15, 23, 31]}


def test_qwen3_vl_2b_and_8b(pkg):
    for vc, ref in ((VISION_2B, pkg.spec_2b()), (VISION_8B, pkg.spec_8b())):
        spec = pkg.spec_from_config(hf_config(vc)).vision
        assert spec == ref                        # the BASELINE shapes, field by field
        # qwen3_vl forces full attention on every block (model.py:1033-1034)
        assert tuple(spec.fullatt_block_indexes) == tuple(range(vc["depth"])) and not spec.use_window
        assert spec.window_size == 32             # patch_size * spatial_merge_size (model.py:1031)
        assert spec.num_position_embeddings == 2304 and spec.in_channels == 3


def test_qwen25_style_window_config(pkg):
    top = hf_config(VISION_QWEN25)
    spec = pkg.spec_from_config(top).vision
    assert spec.patch_size == 14                       # spatial_patch_size fallback
    assert spec.in_channels == 3                       # in_chans fallback
    assert spec.window_size == 112
    assert tuple(spec.fullatt_block_indexes) == (7, 15, 23, 31) and spec.use_window
    assert spec.num_position_embeddings is None        # absent -> no learned table
    assert tuple(spec.deepstack_visual_indexes) == ()
    # defaults when keys are missing: temporal_patch -> 1, window = patch * merge
    vc = {k: v for k, v in VISION_QWEN25.items() if k not in ("temporal_patch_size", "window_size")}
    spec = pkg.vision_spec_from_config(dict(vc, temporal_patch=3))
    assert spec.temporal_patch_size == 3 and spec.window_size == 28
    spec = pkg.vision_spec_from_config(vc)
    assert spec.temporal_patch_size == 1


def test_fullatt_fallback_to_deepstack_indexes(pkg):
    """Outside model_type "qwen3_vl" the reference falls back to fullatt_block_indexes, then to
    deepstack_visual_indexes, then [] (model.py:1032). transformers >= 5 labels its Qwen3-VL
    vision config "qwen3_vl_vision", which takes that generic rule, as it does in the reference."""
    tf = pytest.importorskip("transformers")
    from transformers.models.qwen3_vl.configuration_qwen3_vl import Qwen3VLVisionConfig

    d = Qwen3VLVisionConfig(depth=4, deepstack_visual_indexes=[1, 2]).to_dict()
    spec = pkg.spec_from_config(hf_config(d)).vision
    assert spec.depth == 4 and spec.hidden_size == d["hidden_size"] and spec.num_heads == d["num_heads"]
    assert spec.intermediate_size == d["intermediate_size"] and spec.out_hidden_size == d["out_hidden_size"]
    assert spec.num_position_embeddings == d["num_position_embeddings"]
    if d.get("model_type") == "qwen3_vl":
        assert tuple(spec.fullatt_block_indexes) == (0, 1, 2, 3)
    else:
        assert tuple(spec.fullatt_block_indexes) == (1, 2) and spec.use_window
    assert tuple(spec.deepstack_visual_indexes) == (1, 2)
    no_ds = {k: v for k, v in d.items() if k != "deepstack_visual_indexes"}
    no_ds["model_type"] = "other"
    assert tuple(pkg.vision_spec_from_config(no_ds).fullatt_block_indexes) == ()


def test_config_errors_and_text_only(pkg):
    with pytest.raises(ValueError, match="mrope_section"):
        pkg.spec_from_config({"vision_config": VISION_2B, "text_config": dict(hf_config({})["text_config"],
                                                                               rope_scaling={})})
    with pytest.raises(ValueError, match="3 entries"):
        pkg.spec_from_config(hf_config(VISION_2B, mrope=(64, 64)))
    top = hf_config(VISION_2B)
    del top["vision_config"]
    s = pkg.spec_from_config(top)
    assert s.vision is None and s.eos_token_id == 151645 and s.text.head_dim == 128
    with pytest.raises(KeyError):
        pkg.vision_spec_from_config({k: v for k, v in VISION_2B.items() if k != "depth"})


def test_mrope_section_rules(pkg):
    """model.py:991-1009. A `vision_config` key that is present but empty still demands a section
    (the reference tests `is not None` there); the 3-entry rule applies only to a non-empty vision
    config; unless `mrope_interleaved`, the section must sum to head_dim // 2, with head_dim from
    the text config (`head_dim`, else hidden_size // num_attention_heads)."""
    top = hf_config(VISION_2B)
    top["vision_config"] = {}
    del top["text_config"]["rope_scaling"]
    with pytest.raises(ValueError, match="Missing rope_scaling.mrope_section"):
        pkg.spec_from_config(top)
    top = hf_config({}, mrope=(32, 32))                  # empty vision config: no 3-entry rule
    top["text_config"]["rope_scaling"]["mrope_interleaved"] = False
    s = pkg.spec_from_config(top)
    assert s.vision is None and list(s.text.rope_section) == [32, 32]
    # non-interleaved: the sum must be head_dim // 2 = 64
    top = hf_config(VISION_2B, mrope=(24, 20, 20))
    top["text_config"]["rope_scaling"]["mrope_interleaved"] = False
    assert pkg.spec_from_config(top).vision == pkg.spec_2b()
    top["text_config"]["rope_scaling"]["mrope_section"] = [24, 20, 16]
    with pytest.raises(ValueError, match=r"mrope_section sum must equal head_dim//2 \(64\)"):
        pkg.spec_from_config(top)
    top["text_config"]["rope_scaling"]["mrope_interleaved"] = True     # interleaved: no sum rule
    assert pkg.spec_from_config(top).text.mrope_interleaved
    # head_dim from hidden_size // num_attention_heads when the text config has none
    top = hf_config(VISION_2B, mrope=(16, 24, 24))
    top["text_config"]["rope_scaling"]["mrope_interleaved"] = False
    del top["text_config"]["head_dim"]
    top["text_config"]["hidden_size"] = 2048
    top["text_config"]["num_attention_heads"] = 16
    s = pkg.spec_from_config(top)
    assert s.text.head_dim == 128 and list(s.text.rope_section) == [16, 24, 24]
    # without a section, a text-only model gets [head_dim // 2]
    top = hf_config(VISION_2B)
    del top["vision_config"]
    del top["text_config"]["rope_scaling"]
    assert list(pkg.spec_from_config(top).text.rope_section) == [64]


def test_text_spec_fields_and_missing_keys(pkg):
    """The text half of spec_from_config (model.py:1011-1025): the fields it reads, their
    defaults (rope_theta 10000, scaling type / factor None) and a KeyError for a missing
    required key, as the reference raises."""
    top = hf_config(VISION_2B)
    top["text_config"]["rope_scaling"].update(type="mrope", factor=2)
    t = pkg.spec_from_config(top).text
    assert (t.hidden_size, t.num_attention_heads, t.num_hidden_layers, t.num_key_value_heads) == (2048, 16, 28, 8)
    assert (t.intermediate_size, t.rms_norm_eps, t.vocab_size) == (6144, 1e-6, 151936)
    assert t.rope_theta == 10000.0 and t.rope_scaling_type == "mrope" and t.rope_scaling_factor == 2.0
    top["rope_theta"] = 5e6
    assert pkg.spec_from_config(top).text.rope_theta == 5e6
    for key in ("num_hidden_layers", "vocab_size", "rms_norm_eps"):
        bad = hf_config(VISION_2B)
        del bad["text_config"][key]
        with pytest.raises(KeyError):
            pkg.spec_from_config(bad)


def test_model_construction_like_the_reference(pkg):
    """Qwen3VLModel(spec) takes the Qwen3VLSpec that spec_from_config returns and builds the
    vision tower in float32, as the reference does (model.py:858-871 builds
    Qwen3VisionTransformer(spec.vision), whose dtype defaults to float32, model.py:661);
    vision_dtype selects the bf16 tower; a spec without vision gives no tower; a bare
    VisionBackboneSpec is taken as the vision spec. No GPU work: construction only."""
    spec = pkg.spec_from_config(hf_config(VISION_2B))
    m = pkg.Qwen3VLModel(spec)
    assert m.spec is spec and m.visual is not None and m.visual.dtype == "float32"
    assert m.visual.spec == pkg.spec_2b()
    assert pkg.Qwen3VLModel(spec, vision_dtype="bfloat16").visual.dtype == "bfloat16"
    assert pkg.Qwen3VisionTransformer(pkg.spec_2b()).dtype == "float32"
    assert pkg.Qwen3VLModel(pkg.spec_8b()).visual.spec == pkg.spec_8b()
    top = hf_config(VISION_2B)
    del top["vision_config"]
    assert pkg.Qwen3VLModel(pkg.spec_from_config(top)).visual is None
    with pytest.raises(ValueError, match="Vision backbone"):
        pkg.Qwen3VLModel(pkg.spec_from_config(top)).encode_vision(None, None)


@pytest.mark.parametrize("fullatt", [None, (), (1, 3), tuple(range(24))])
def test_packed_spec_header_round_trip(pkg, fullatt):
    """The packed file's JSON spec header keeps `fullatt_block_indexes` None ("every block is full
    attention") distinct from () (window attention on every block)."""
    w = pkg.weights
    spec = pkg.VisionBackboneSpec(hidden_size=1024, out_hidden_size=2048, depth=24, num_heads=16,
                                  intermediate_size=4096, fullatt_block_indexes=fullatt,
                                  deepstack_visual_indexes=(5, 11, 17), num_position_embeddings=None)
    back = w.spec_from_json(w.spec_to_json(spec))
    assert back == spec or (fullatt is not None and tuple(back.fullatt_block_indexes) == tuple(fullatt))
    assert back.use_window == spec.use_window
    assert (back.fullatt_block_indexes is None) == (fullatt is None)
    assert back.num_position_embeddings is None
    assert json.loads(w.spec_to_json(spec))["fullatt_block_indexes"] == (None if fullatt is None else list(fullatt))


def test_load_hf_vision_directory(pkg, tmp_path):
    """config.json + safetensors -> (spec, params) with the reference's Flax shapes."""
    from safetensors.numpy import save_file

    vc = dict(VISION_2B, depth=2, deepstack_visual_indexes=[0])
    (tmp_path / "config.json").write_text(json.dumps(hf_config(vc)))
    rng = np.random.default_rng(0)
    D, I, P = 1024, 4096, 1536
    sd = {"model.visual.patch_embed.proj.weight": rng.standard_normal((D, 3, 2, 16, 16), dtype=np.float32),
          "model.visual.patch_embed.proj.bias": np.zeros(D, np.float32),
          "model.visual.pos_embed.weight": rng.standard_normal((2304, D), dtype=np.float32)}
    for i in range(2):
        b = f"model.visual.blocks.{i}."
        sd.update({b + "norm1.weight": np.ones(D, np.float32), b + "norm1.bias": np.zeros(D, np.float32),
                   b + "norm2.weight": np.ones(D, np.float32), b + "norm2.bias": np.zeros(D, np.float32),
                   b + "attn.qkv.weight": rng.standard_normal((3 * D, D), dtype=np.float32),
                   b + "attn.qkv.bias": np.zeros(3 * D, np.float32),
                   b + "attn.proj.weight": rng.standard_normal((D, D), dtype=np.float32),
                   b + "attn.proj.bias": np.zeros(D, np.float32),
                   b + "mlp.linear_fc1.weight": rng.standard_normal((I, D), dtype=np.float32),
                   b + "mlp.linear_fc1.bias": np.zeros(I, np.float32),
                   b + "mlp.linear_fc2.weight": rng.standard_normal((D, I), dtype=np.float32),
                   b + "mlp.linear_fc2.bias": np.zeros(D, np.float32)})
    save_file(sd, str(tmp_path / "model.safetensors"))
    spec, params = pkg.weights.load_hf_vision(str(tmp_path))
    assert spec.depth == 2 and tuple(spec.deepstack_visual_indexes) == (0,) and not spec.use_window
    v = params["visual"]
    assert v["patch_embed"]["proj"]["kernel"].shape == (P, D)
    np.testing.assert_array_equal(v["patch_embed"]["proj"]["kernel"],
                                  sd["model.visual.patch_embed.proj.weight"].reshape(D, -1).T)
    assert v["blocks_1"]["attn"]["qkv"]["kernel"].shape == (D, 3 * D)
    np.testing.assert_array_equal(v["blocks_1"]["mlp"]["linear_fc2"]["kernel"],
                                  sd["model.visual.blocks.1.mlp.linear_fc2.weight"].T)
    assert v["pos_embed"]["embedding"].shape == (2304, D)
    (tmp_path / "config.json").write_text(json.dumps({k: v for k, v in hf_config(vc).items() if k != "vision_config"}))
    with pytest.raises(ValueError, match="vision"):
        pkg.weights.load_hf_vision(str(tmp_path))
