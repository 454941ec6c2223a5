"""Synthetic checkpoints: determinism and the shapes the reference expects."""

import hashlib
import json
import os

import numpy as np

from quicklm_amd import synth

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy.npz")


def _tensor(name, cfg="tiny"):
    c = synth.CONFIGS[cfg]
    spec = {s[0]: s for s in synth.tensor_specs(c)}[name]
    _, shape, dtype, init = spec
    buf = np.empty(int(np.prod(shape)), np.float32 if dtype == "F32" else np.uint16)
    seed = int(synth.lib().qlm_synth_tensor_seed(synth.BASE_SEED + c["index"], name.encode()))
    synth._fill(buf, dtype, seed, init)
    return buf


def test_generator_matches_golden_hashes():
    g = np.load(GOLDEN)
    for name, sha in zip(g["tensor_names"], g["tensor_sha"]):
        assert hashlib.sha256(_tensor(str(name)).tobytes()).hexdigest() == str(sha), name


def test_normal_statistics():
    x = _tensor("model.layers.0.mlp.gate_proj.weight")
    assert abs(float(x.mean())) < 1e-4 and abs(float(x.std()) - 0.02) < 1e-4


def test_micro_checkpoint_layout(tmp_path):
    d = synth.write_model(str(tmp_path), "micro")
    cfg = json.load(open(os.path.join(d, "config.json")))
    assert cfg["layer_types"] == ["linear_attention"] * 3 + ["full_attention"]
    from oracle.oracle import read_safetensors

    t = read_safetensors(os.path.join(d, "model.safetensors"))
    assert t["model.layers.3.self_attn.q_proj.weight"].shape == (2 * 4 * 128, 256)  # gated
    assert t["model.layers.0.linear_attn.conv1d.weight"].shape == (3 * 256, 1, 4)
    assert "lm_head.weight" not in t  # tied
    h1 = hashlib.sha256(open(os.path.join(d, "model.safetensors"), "rb").read()).hexdigest()
    d2 = synth.write_model(str(tmp_path / "again"), "micro")
    h2 = hashlib.sha256(open(os.path.join(d2, "model.safetensors"), "rb").read()).hexdigest()
    assert h1 == h2


def test_prompt_tokens_in_range():
    p = synth.prompt_tokens(2048, seed=1, batch=16)
    assert p.shape == (16, 2048) and p.min() >= 0 and p.max() < 151936
    assert not np.array_equal(p[0], p[1])
