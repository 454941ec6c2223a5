"""Seeded random-init checkpoints of the hybrid family, written as safetensors.

The reference has no test weights and the real checkpoints are not available
offline, so every workload here runs on random-init weights of the target
architecture. Values come from the deterministic counter-based generator in
libqlm_engine.so (qlm_synth_*): tensor `name` of a model with base seed B is
filled from seed qlm_synth_tensor_seed(B, name), so the same bytes are written
on any host and by any number of threads.

Initialisation (stated in every config.json under "synthetic_init"):
  linear weights      N(0, 0.02)            stored F32 (tiny) or BF16 (4B)
  embed_tokens        N(0, 0.02)            F32, tied lm_head
  zero-centred norms  N(0, 0.02)            input/post/final norm, q_norm, k_norm
  linear_attn.norm    1 + N(0, 0.02)        plain gain
  conv1d.weight       N(0, 0.3)
  A_log               log U(1, 16)
  dt_bias             softplus^-1(dt), dt = exp(U(log 1e-3, log 1e-1))
"""

from __future__ import annotations

import ctypes as C
import json
import os
import struct

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
ENGINE_LIB = os.path.join(PKG, "libqlm_engine.so")

BASE_SEED = 0x514C4D00

# Model shapes of the two workload configurations.
TINY = dict(name="tiny", index=0, vocab_size=151936, hidden_size=1024, num_hidden_layers=24,
            intermediate_size=3584, linear_num_heads=8, linear_head_dim=128,
            num_attention_heads=8, num_key_value_heads=2, head_dim=128, rope_theta=1e6,
            partial_rotary_factor=0.25, linear_dtype="F32")
HYBRID_4B = dict(name="4b", index=4, vocab_size=151936, hidden_size=2560, num_hidden_layers=36,
                 intermediate_size=9728, linear_num_heads=16, linear_head_dim=128,
                 num_attention_heads=16, num_key_value_heads=4, head_dim=128, rope_theta=1e6,
                 partial_rotary_factor=0.25, linear_dtype="BF16")
# A few-MB model of the same family (one GQA layer after three DeltaNet
# layers) for smoke runs and quick CPU checks.
MICRO = dict(name="micro", index=9, vocab_size=4096, hidden_size=256, num_hidden_layers=4,
             intermediate_size=512, linear_num_heads=2, linear_head_dim=128,
             num_attention_heads=4, num_key_value_heads=1, head_dim=128, rope_theta=1e6,
             partial_rotary_factor=0.25, linear_dtype="BF16")
CONFIGS = {"tiny": TINY, "4b": HYBRID_4B, "micro": MICRO}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(ENGINE_LIB):
            raise ImportError(f"{ENGINE_LIB} missing: run `python -m quicklm_amd.build`")
        L = C.CDLL(ENGINE_LIB)
        L.qlm_synth_tensor_seed.restype = C.c_uint64
        L.qlm_synth_tensor_seed.argtypes = [C.c_uint64, C.c_char_p]
        for fn in ("qlm_synth_normal_f32", "qlm_synth_normal_bf16"):
            getattr(L, fn).argtypes = [C.c_void_p, C.c_size_t, C.c_uint64, C.c_float, C.c_float]
        L.qlm_synth_uniform_f32.argtypes = [C.c_void_p, C.c_size_t, C.c_uint64, C.c_float,
                                            C.c_float]
        _lib = L
    return _lib


def layer_types(n_layers: int) -> list[str]:
    return ["full_attention" if i % 4 == 3 else "linear_attention" for i in range(n_layers)]


def config_json(c: dict) -> dict:
    return {
        "architectures": ["Qwen3_5ForCausalLM"],
        "model_type": "qwen3_5_text",
        "vocab_size": c["vocab_size"],
        "hidden_size": c["hidden_size"],
        "intermediate_size": c["intermediate_size"],
        "num_hidden_layers": c["num_hidden_layers"],
        "num_attention_heads": c["num_attention_heads"],
        "num_key_value_heads": c["num_key_value_heads"],
        "head_dim": c["head_dim"],
        "linear_num_key_heads": c["linear_num_heads"],
        "linear_num_value_heads": c["linear_num_heads"],
        "linear_key_head_dim": c["linear_head_dim"],
        "linear_value_head_dim": c["linear_head_dim"],
        "linear_conv_kernel_dim": 4,
        "rms_norm_eps": 1e-6,
        "rope_theta": c["rope_theta"],
        "partial_rotary_factor": c["partial_rotary_factor"],
        "attn_output_gate": True,
        "tie_word_embeddings": True,
        "layer_types": layer_types(c["num_hidden_layers"]),
        "synthetic_init": {
            "base_seed": BASE_SEED + c["index"],
            "linear": "N(0,0.02) " + c["linear_dtype"],
            "embed_tokens": "N(0,0.02) F32 (tied lm_head)",
            "zero_centred_norms": "N(0,0.02)",
            "linear_attn.norm": "1+N(0,0.02)",
            "conv1d": "N(0,0.3)",
            "A_log": "log U(1,16)",
            "dt_bias": "softplus^-1(exp(U(log 1e-3, log 1e-1)))",
        },
    }


def tensor_specs(c: dict):
    """(name, shape, dtype, init) for every tensor, in file order."""
    H, F, V = c["hidden_size"], c["intermediate_size"], c["vocab_size"]
    nh, d = c["linear_num_heads"], c["linear_head_dim"]
    nq, nkv, hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
    lin = c["linear_dtype"]
    HD = nh * d
    out = [("model.embed_tokens.weight", [V, H], "F32", ("normal", 0.0, 0.02)),
           ("model.norm.weight", [H], "F32", ("normal", 0.0, 0.02))]
    for i, t in enumerate(layer_types(c["num_hidden_layers"])):
        p = f"model.layers.{i}."
        out += [(p + "input_layernorm.weight", [H], "F32", ("normal", 0.0, 0.02)),
                (p + "post_attention_layernorm.weight", [H], "F32", ("normal", 0.0, 0.02))]
        if t == "linear_attention":
            out += [(p + "linear_attn.in_proj_qkv.weight", [3 * HD, H], lin, ("normal", 0.0, 0.02)),
                    (p + "linear_attn.in_proj_z.weight", [HD, H], lin, ("normal", 0.0, 0.02)),
                    (p + "linear_attn.in_proj_b.weight", [nh, H], lin, ("normal", 0.0, 0.02)),
                    (p + "linear_attn.in_proj_a.weight", [nh, H], lin, ("normal", 0.0, 0.02)),
                    (p + "linear_attn.conv1d.weight", [3 * HD, 1, 4], "F32", ("normal", 0.0, 0.3)),
                    (p + "linear_attn.norm.weight", [d], "F32", ("normal", 1.0, 0.02)),
                    (p + "linear_attn.A_log", [nh], "F32", ("A_log",)),
                    (p + "linear_attn.dt_bias", [nh], "F32", ("dt_bias",)),
                    (p + "linear_attn.out_proj.weight", [H, HD], lin, ("normal", 0.0, 0.02))]
        else:
            out += [(p + "self_attn.q_proj.weight", [2 * nq * hd, H], lin, ("normal", 0.0, 0.02)),
                    (p + "self_attn.k_proj.weight", [nkv * hd, H], lin, ("normal", 0.0, 0.02)),
                    (p + "self_attn.v_proj.weight", [nkv * hd, H], lin, ("normal", 0.0, 0.02)),
                    (p + "self_attn.o_proj.weight", [H, nq * hd], lin, ("normal", 0.0, 0.02)),
                    (p + "self_attn.q_norm.weight", [hd], "F32", ("normal", 0.0, 0.02)),
                    (p + "self_attn.k_norm.weight", [hd], "F32", ("normal", 0.0, 0.02))]
        out += [(p + "mlp.gate_proj.weight", [F, H], lin, ("normal", 0.0, 0.02)),
                (p + "mlp.up_proj.weight", [F, H], lin, ("normal", 0.0, 0.02)),
                (p + "mlp.down_proj.weight", [H, F], lin, ("normal", 0.0, 0.02))]
    return out


def _fill(view: np.ndarray, dtype: str, seed: int, init) -> None:
    L = lib()
    n = view.size
    ptr = view.ctypes.data
    kind = init[0]
    if kind == "normal":
        fn = L.qlm_synth_normal_bf16 if dtype == "BF16" else L.qlm_synth_normal_f32
        if fn(ptr, n, seed, init[1], init[2]) != 0:
            raise RuntimeError("synth fill failed")
        return
    assert dtype == "F32"
    u = np.empty(n, np.float32)
    L.qlm_synth_uniform_f32(u.ctypes.data, n, seed, 0.0, 1.0)
    if kind == "A_log":
        view[:] = np.log(1.0 + 15.0 * u.astype(np.float64)).astype(np.float32)
    elif kind == "dt_bias":
        lo, hi = np.log(1e-3), np.log(1e-1)
        dt = np.exp(lo + (hi - lo) * u.astype(np.float64))
        view[:] = (dt + np.log(-np.expm1(-dt))).astype(np.float32)
    else:
        raise ValueError(kind)


def write_model(out_dir: str, cfg: str | dict = "tiny") -> str:
    """Write config.json + model.safetensors for a named or explicit config."""
    c = CONFIGS[cfg] if isinstance(cfg, str) else cfg
    os.makedirs(out_dir, exist_ok=True)
    base = BASE_SEED + c["index"]
    specs = tensor_specs(c)
    header, off = {}, 0
    for name, shape, dtype, _ in specs:
        nbytes = int(np.prod(shape)) * (4 if dtype == "F32" else 2)
        header[name] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + nbytes]}
        off += nbytes
    header["__metadata__"] = {"format": "pt", "generator": "quicklm_amd.synth",
                              "base_seed": hex(base)}
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    path = os.path.join(out_dir, "model.safetensors")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hj)))
        f.write(hj)
        for name, shape, dtype, init in specs:
            buf = np.empty(int(np.prod(shape)), np.float32 if dtype == "F32" else np.uint16)
            _fill(buf, dtype, int(lib().qlm_synth_tensor_seed(base, name.encode())), init)
            buf.tofile(f)
    with open(os.path.join(out_dir, "config.json"), "w") as f:
        json.dump(config_json(c), f, indent=1)
    return out_dir


def prompt_tokens(n: int, seed: int, vocab: int = 151936, batch: int = 1) -> np.ndarray:
    """Uniform random prompt ids [batch, n] from the same counter generator."""
    u = np.empty(batch * n, np.float32)
    lib().qlm_synth_uniform_f32(u.ctypes.data, u.size, int(lib().qlm_synth_tensor_seed(
        BASE_SEED, f"prompt/{seed}".encode())), 0.0, 1.0)
    ids = np.minimum((u.astype(np.float64) * vocab).astype(np.int64), vocab - 1)
    return ids.astype(np.int32).reshape(batch, n)
