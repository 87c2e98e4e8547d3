"""Gemma 4 package loading through the C ABI (ribn_rocm_gemma_open), CPU only: the
config.json and SafeTensors checks of Gemma4Source::open / Gemma4Config::from_json
(crates/gemma4/src/source.rs:56-160, config.rs:59-380) reject a broken package with
RIBN_ERR_FORMAT and a message naming the field, before any device work."""
import json
import os

import numpy as np
import pytest

import gemma_oracle as g4
import ribn_amd

KINDS = ("S", "F", "S", "F")


def small():
    c = g4.config(vocab=50, hidden=16, intermediate=24, heads=2, kv_heads=1, head_dim=8, global_head_dim=8, ple=4,
                  context=32, window=8, layers=KINDS)
    return c, g4.synth_named(c, seed=1, std=0.3)


def open_err(d):
    with pytest.raises(ribn_amd.RibnError) as e:
        ribn_amd.GemmaRocm(str(d))
    return e.value


def test_missing_files(tmp_path):
    e = open_err(tmp_path)
    assert e.code == -2 and "config.json" in str(e)


@pytest.mark.parametrize("mutate,needle", [
    (lambda cfg: cfg["text_config"].update(layer_types=["sliding_attention"] * 4), "last layer must"),
    (lambda cfg: cfg.update(model_type="llama"), "model_type"),
    (lambda cfg: cfg["text_config"].update(num_key_value_heads=3), "num_key_value_heads"),
    (lambda cfg: cfg["text_config"]["rope_parameters"]["full_attention"].update(partial_rotary_factor=0.5),
     "rope_parameters"),
    (lambda cfg: cfg["text_config"].update(num_kv_shared_layers=4), "num_kv_shared_layers"),
    (lambda cfg: cfg["text_config"].update(hidden_activation="relu"), "hidden_activation"),
])
def test_config_rejections(tmp_path, mutate, needle):
    c, named = small()
    g4.write_package(str(tmp_path), c, named, KINDS)
    cfg = json.load(open(tmp_path / "config.json"))
    mutate(cfg)
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    e = open_err(tmp_path)
    assert e.code == -3 and needle in str(e), str(e)


def test_tensor_rejections(tmp_path):
    c, named = small()
    bad = dict(named)
    del bad[g4.PREFIX + "layers.2.mlp.up_proj.weight"]
    g4.write_package(str(tmp_path / "a"), c, bad, KINDS)
    e = open_err(tmp_path / "a")
    assert e.code == -3 and "layers.2.mlp.up_proj.weight" in str(e)
    bad = dict(named)
    bad[g4.PREFIX + "norm.weight"] = np.zeros(15, np.uint16)
    g4.write_package(str(tmp_path / "b"), c, bad, KINDS)
    e = open_err(tmp_path / "b")
    assert e.code == -3 and "norm.weight" in str(e) and "shape" in str(e)
    g4.write_package(str(tmp_path / "c"), c, named, KINDS)
    raw = open(tmp_path / "c" / "model.safetensors", "rb").read()
    open(tmp_path / "c" / "model.safetensors", "wb").write(raw[:len(raw) // 2])
    e = open_err(tmp_path / "c")
    assert e.code == -3 and "outside the file" in str(e)
