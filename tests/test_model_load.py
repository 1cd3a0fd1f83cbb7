"""config.json as the reference runtime reads it (sparkmv_config_load,
tools/vq-runtime/src/config.rs:39-85 Config::load). Host only: no GPU.

The reference ships no config.json, so the files are written here: the
shapes of the Spark checkpoint (hidden 2560, GQA
16/4 heads of 256, FFN 10240, a full layer every fourth), and variations
that exercise each rule of Config::load: required numeric keys and
layer_types, "full_attention" as the only sliding/full switch (other
strings slide; non-strings and layers past the list count as full),
rope_parameters per layer type with the checkpoint's fallbacks, values kept
in f32, keys looked up in their own object, and the last of a repeated key.
"""
import json

import numpy as np
import pytest

SPARK = {
    "hidden_size": 2560, "num_hidden_layers": 8, "num_attention_heads": 16, "num_key_value_heads": 4,
    "head_dim": 256, "intermediate_size": 10240, "vocab_size": 151936, "rms_norm_eps": 1e-06,
    "sliding_window": 512,
    "layer_types": ["sliding_attention", "sliding_attention", "sliding_attention", "full_attention"] * 2,
    "rope_parameters": {"full_attention": {"rope_theta": 5000000.0, "partial_rotary_factor": 0.25,
                                           "rope_type": "default"},
                        "sliding_attention": {"rope_theta": 10000.0, "rope_type": "default"}},
    "architectures": ["SparkForCausalLM"], "torch_dtype": "bfloat16", "tie_word_embeddings": True,
}


def write(tmp_path, obj, name="config.json"):
    p = tmp_path / name
    p.write_text(obj if isinstance(obj, str) else json.dumps(obj, indent=2))
    return p


def test_spark_config(sm, tmp_path):
    cfg, full = sm.config_load(write(tmp_path, SPARK))
    assert (cfg["hidden"], cfg["layers"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"]) == (2560, 8, 16, 4, 256)
    assert (cfg["intermediate"], cfg["vocab"], cfg["sliding_window"]) == (10240, 151936, 512)
    assert cfg["eps"] == float(np.float32(1e-6))
    assert full == [False, False, False, True] * 2
    assert (cfg["rope_full_theta"], cfg["rope_full_partial"]) == (5e6, 0.25)
    # the sliding block gives a theta but no partial factor: the fallback 1.0
    assert (cfg["rope_slide_theta"], cfg["rope_slide_partial"]) == (1e4, 1.0)


def test_rope_fallbacks_and_f32(sm, tmp_path):
    c = dict(SPARK)
    del c["rope_parameters"]
    cfg, _ = sm.config_load(write(tmp_path, c))
    assert (cfg["rope_full_theta"], cfg["rope_full_partial"], cfg["rope_slide_theta"], cfg["rope_slide_partial"]) == \
        (5e6, 0.25, 1e4, 1.0)
    c["rope_parameters"] = {"sliding_attention": {"rope_theta": 0.1, "partial_rotary_factor": 0.3}}
    cfg, _ = sm.config_load(write(tmp_path, c))
    assert cfg["rope_slide_theta"] == float(np.float32(0.1)) and cfg["rope_slide_theta"] != 0.1
    assert cfg["rope_slide_partial"] == float(np.float32(0.3))
    assert (cfg["rope_full_theta"], cfg["rope_full_partial"]) == (5e6, 0.25)


def test_layer_types_rules(sm, tmp_path):
    c = dict(SPARK, num_hidden_layers=6)
    # another string slides; a non-string counts as full; past the list: full
    c["layer_types"] = ["sliding_attention", "chunked_attention", 7, "full_attention"]
    _, full = sm.config_load(write(tmp_path, c))
    assert full == [False, False, True, True, True, True]
    # escapes are decoded before the comparison
    c["layer_types"] = ["full\\u005fattention"]
    p = tmp_path / "esc.json"
    p.write_text(json.dumps(c).replace("full\\\\u005fattention", "full\\u005fattention"))
    _, full = sm.config_load(p)
    assert full[0] is True


@pytest.mark.parametrize("key", ["hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads",
                                 "head_dim", "intermediate_size", "vocab_size", "rms_norm_eps", "sliding_window"])
def test_required_numbers(sm, tmp_path, key):
    c = dict(SPARK)
    del c[key]
    with pytest.raises(sm.SparkmvError, match=f"config.json has no numeric {key}"):
        sm.config_load(write(tmp_path, c))
    c[key] = "2560"   # a string is not a number
    with pytest.raises(sm.SparkmvError, match=f"config.json has no numeric {key}"):
        sm.config_load(write(tmp_path, c))


def test_structure_not_text(sm, tmp_path):
    # head_dim only inside a nested object does not count
    c = dict(SPARK)
    del c["head_dim"]
    c["text_config"] = {"head_dim": 256}
    with pytest.raises(sm.SparkmvError, match="no numeric head_dim"):
        sm.config_load(write(tmp_path, c))
    # a repeated key: the last one counts
    text = json.dumps(SPARK)[:-1] + ', "hidden_size": 1024}'
    cfg, _ = sm.config_load(write(tmp_path, text, "dup.json"))
    assert cfg["hidden"] == 1024


def test_refusals(sm, tmp_path):
    c = dict(SPARK)
    del c["layer_types"]
    with pytest.raises(sm.SparkmvError, match="config.json has no layer_types"):
        sm.config_load(write(tmp_path, c))
    with pytest.raises(sm.SparkmvError, match="expected"):
        sm.config_load(write(tmp_path, '{"hidden_size": 2560,,}', "bad.json"))
    with pytest.raises(sm.SparkmvError, match="trailing"):
        sm.config_load(write(tmp_path, json.dumps(SPARK) + " x", "trail.json"))
    with pytest.raises(sm.SparkmvError, match="nope.json"):
        sm.config_load(tmp_path / "nope.json")
    with pytest.raises(sm.SparkmvError, match="outside"):
        sm.config_load(write(tmp_path, dict(SPARK, head_dim=0), "zero.json"))
    # a layer count past any model is refused before its flags are allocated
    with pytest.raises(sm.SparkmvError, match="1000000000 layers, above 65536"):
        sm.config_load(write(tmp_path, dict(SPARK, num_hidden_layers=10 ** 9), "huge.json"))
