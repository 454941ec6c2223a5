"""CPU oracle bindings (TEST INFRASTRUCTURE ONLY).

Two checkers, both on the CPU:
  - `Oracle`: this repo's C restatement of the reference arithmetic
    (oracle/qlm_oracle.c -> oracle/liboracle.so).
  - `Reference`: the reference QuickLM sources compiled where they lie by
    oracle/Makefile into oracle/_ref/ (IEEE build for bit-level checks, the
    reference's own -O3 -ffast-math flags for the CPU baseline).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REF_DIR = os.path.join(HERE, "_ref")

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(_vp)


def build(ref: bool = False) -> None:
    """Compile the oracle (and, with ref=True, the reference) via oracle/Makefile."""
    targets = ["oracle"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", HERE, *targets], check=True)


class Oracle:
    """ctypes face of liboracle.so (the C restatement)."""

    _lib = None

    def __init__(self) -> None:
        if Oracle._lib is None:
            path = os.path.join(HERE, "liboracle.so")
            if not os.path.exists(path):
                build()
            Oracle._lib = C.CDLL(path)
        self.lib = Oracle._lib
        self.lib.orc_sumsq.restype = _f
        self.lib.orc_argmax.restype = _i

    def set_threads(self, n: int) -> None:
        self.lib.orc_set_threads(_i(n))

    def quantize(self, w: np.ndarray, group: int):
        rows, K = w.shape
        q = np.empty((rows, K), np.int8)
        nb = 1 if group >= K else (K + group - 1) // group
        s = np.empty((rows, nb), np.float32)
        if w.dtype == np.float32:
            self.lib.orc_quantize_rows_f32(_p(w), _i(rows), _i(K), _i(group), _p(q), _p(s))
        elif w.dtype == np.uint16:
            self.lib.orc_quantize_rows_bf16(_p(w), _i(rows), _i(K), _i(group), _p(q), _p(s))
        else:
            raise TypeError(w.dtype)
        return q, s

    def matmul_i8(self, A: np.ndarray, q: np.ndarray, s: np.ndarray, group: int) -> np.ndarray:
        M, K = A.shape
        N = q.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.orc_matmul_i8(_p(A), _i(M), _i(K), _p(q), _p(s), _i(group), _i(N), _p(out), _i(N))
        return out

    def quantize_q4(self, w: np.ndarray):
        """Packed int4 rows [rows, (K+1)//2] (low nibble = even column) and
        scales [rows, ceil(K/32)]."""
        rows, K = w.shape
        q = np.empty((rows, (K + 1) // 2), np.uint8)
        s = np.empty((rows, (K + 31) // 32), np.float32)
        fn = {np.float32: "orc_quantize_rows_q4_f32", np.uint16: "orc_quantize_rows_q4_bf16"}
        getattr(self.lib, fn[w.dtype.type])(_p(w), _i(rows), _i(K), _p(q), _p(s))
        return q, s

    def unpack_q4(self, p: np.ndarray, K: int) -> np.ndarray:
        rows = p.shape[0]
        q = np.empty((rows, K), np.int8)
        self.lib.orc_unpack_q4(_p(np.ascontiguousarray(p)), _i(rows), _i(K), _p(q))
        return q

    def matmul_i4(self, A: np.ndarray, p: np.ndarray, s: np.ndarray) -> np.ndarray:
        M, K = A.shape
        N = p.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.orc_matmul_i4(_p(A), _i(M), _i(K), _p(p), _p(s), _i(N), _p(out), _i(N))
        return out

    def matmul_w(self, A: np.ndarray, W: np.ndarray) -> np.ndarray:
        """Native weights W [N, K]: float32, or uint16 bf16 bits."""
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.orc_matmul_w(_p(A), _i(M), _i(K), _p(np.ascontiguousarray(W)),
                              _i(1 if W.dtype == np.uint16 else 0), _i(N), _p(out), _i(N))
        return out

    def sumsq(self, x: np.ndarray) -> float:
        return float(self.lib.orc_sumsq(_p(x), _i(x.size)))

    def rms_norm(self, x, w, eps):
        rows, n = x.shape
        y = np.empty_like(x)
        self.lib.orc_rms_norm(_p(x), _p(w), _p(y), _i(rows), _i(n), _f(eps))
        return y

    def add_rms_norm(self, res, d, w, eps):
        rows, n = res.shape
        res = res.copy()
        y = np.empty_like(res)
        self.lib.orc_add_rms_norm(_p(res), _p(d), _p(w), _p(y), _i(rows), _i(n), _f(eps))
        return res, y

    def silu_mul(self, a, b):
        a = a.copy()
        self.lib.orc_silu_mul(_p(a), _p(b), _i(a.size))
        return a

    def rope_neox(self, t, pos, theta, rot, head_stride=None):
        t = t.copy()
        nh, hs = t.shape
        self.lib.orc_rope_neox(_p(t), _i(nh), _i(head_stride or hs), _i(pos), _f(theta), _i(rot))
        return t

    def rope_table(self, theta, rot, n_pos):
        half = rot // 2
        c = np.empty((n_pos, half), np.float32)
        s = np.empty((n_pos, half), np.float32)
        self.lib.orc_rope_table(_f(theta), _i(rot), _i(n_pos), _p(c), _p(s))
        return c, s

    def conv1d_tapmajor(self, x, state, oldest, w_t):
        state = state.copy()
        out = np.empty_like(x)
        self.lib.orc_conv1d_tapmajor(_p(x), _p(state), _i(oldest), _p(w_t), _p(out),
                                     _i(x.size), _i(w_t.shape[0]))
        return out, state

    def gated_delta_step(self, q, k, v, decay, beta, state):
        B, H, d = q.shape
        state = state.copy()
        out = np.empty_like(q)
        self.lib.orc_gated_delta_step(_p(q), _p(k), _p(v), _p(decay), _p(beta), _p(state),
                                      _p(out), _i(B), _i(H), _i(d))
        return out, state

    def deltanet_core(self, proj, conv_state, oldest, conv_w_t, A_log, dt_bias, norm_w, state,
                      H, d):
        """Mutates conv_state and state in place; returns the gated output [H*d]."""
        out = np.empty(H * d, np.float32)
        self.lib.orc_deltanet_core(_p(proj), _p(conv_state), _i(oldest), _p(conv_w_t),
                                   _p(A_log), _p(dt_bias), _p(norm_w), _p(state), _p(out),
                                   _i(H), _i(d))
        return out

    def gqa_core(self, qkv, q_norm, k_norm, theta, rot, k_cache, v_cache, pos, n_q, n_kv, hd,
                 gated):
        """Mutates qkv and the caches in place; returns the attention output [n_q*hd]."""
        out = np.empty(n_q * hd, np.float32)
        self.lib.orc_gqa_core(_p(qkv), _p(q_norm), _p(k_norm), _f(theta), _i(rot), _p(k_cache),
                              _p(v_cache), _i(k_cache.shape[0]), _i(pos), _p(out), _i(n_q),
                              _i(n_kv), _i(hd), _i(1 if gated else 0))
        return out

    def attention(self, q, k_cache, v_cache, ctx):
        n_q, hd = q.shape
        n_kv = k_cache.shape[1]
        out = np.empty_like(q)
        self.lib.orc_attention(_p(q), _p(k_cache), _p(v_cache), _i(ctx), _p(out), _i(n_q),
                               _i(n_kv), _i(hd))
        return out

    def argmax(self, x: np.ndarray) -> int:
        return int(self.lib.orc_argmax(_p(x), _i(x.size)))


def ref_available(kind: str = "ieee") -> bool:
    return os.path.exists(os.path.join(REF_DIR, f"libqlm_ref_{kind}.so"))


def _cpu_has_avx512() -> bool:
    try:
        with open("/proc/cpuinfo") as f:
            flags = f.read()
        return all(x in flags for x in ("avx512f", "avx512bw", "avx512vl", "avx512dq", "avx512cd"))
    except OSError:
        return False


class Reference:
    """ctypes face of the reference compiled from its own sources (oracle/_ref)."""

    def __init__(self, kind: str = "ieee") -> None:
        if kind == "fast":
            kind = "v4" if _cpu_has_avx512() and ref_available("v4") else "v3"
        self.kind = kind
        path = os.path.join(REF_DIR, f"libqlm_ref_{kind}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built (make -C oracle ref)")
        self.lib = C.CDLL(path)
        L = self.lib
        L.qref_sumsq.restype = _f
        for fn in ("qref_deltanet_create", "qref_gqa_create", "qref_model_load"):
            getattr(L, fn).restype = _vp
        L.qref_model_vocab.restype = _i
        L.qref_model_sample_greedy.restype = _i
        L.qref_model_generate.restype = _i

    def init_threads(self, n: int) -> None:
        self.lib.qref_init_threads(_i(n))

    def quantize(self, w: np.ndarray):
        rows, K = w.shape
        nb = (K + 31) // 32
        q = np.empty((rows, K), np.int8)
        s = np.empty((rows, nb), np.float32)
        if w.dtype == np.float32:
            self.lib.qref_quantize_rows_f32(_p(w), _i(rows), _i(K), _p(q), _p(s))
        else:
            self.lib.qref_quantize_rows_bf16(_p(w), _i(rows), _i(K), _p(q), _p(s))
        return q, s

    def matmul_i8(self, A, q, s):
        M, K = A.shape
        N = q.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.qref_matmul_i8(_p(A), _i(M), _i(K), _p(q), _p(s), _i(N), _p(out), _i(N))
        return out

    def quantize_q4(self, w: np.ndarray):
        rows, K = w.shape
        q = np.empty((rows, (K + 1) // 2), np.uint8)
        s = np.empty((rows, (K + 31) // 32), np.float32)
        fn = "qref_quantize_rows_f32_int4" if w.dtype == np.float32 else "qref_quantize_rows_bf16_int4"
        getattr(self.lib, fn)(_p(w), _i(rows), _i(K), _p(q), _p(s))
        return q, s

    def matmul_i4(self, A, p, s):
        M, K = A.shape
        N = p.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.qref_matmul_i4(_p(A), _i(M), _i(K), _p(p), _p(s), _i(N), _p(out), _i(N))
        return out

    def matmul_w(self, A, W):
        M, K = A.shape
        N = W.shape[0]
        out = np.empty((M, N), np.float32)
        self.lib.qref_matmul_w(_p(A), _i(M), _i(K), _p(np.ascontiguousarray(W)),
                               _i(1 if W.dtype == np.uint16 else 0), _i(N), _p(out), _i(N))
        return out

    def sumsq(self, x):
        return float(self.lib.qref_sumsq(_p(x), _i(x.size)))

    def rms_norm(self, x, w, eps):
        rows, n = x.shape
        y = np.empty_like(x)
        self.lib.qref_rms_norm(_p(x), _p(w), _p(y), _i(rows), _i(n), _f(eps))
        return y

    def add_rms_norm(self, res, d, w, eps):
        rows, n = res.shape
        res = res.copy()
        y = np.empty_like(res)
        self.lib.qref_add_rms_norm(_p(res), _p(d), _p(w), _p(y), _i(rows), _i(n), _f(eps))
        return res, y

    def silu_mul(self, a, b):
        a = a.copy()
        self.lib.qref_silu_mul(_p(a), _p(b), _i(a.size))
        return a

    def rope_neox(self, t, pos, theta, rot):
        t = t.copy()
        nh, hd = t.shape
        self.lib.qref_rope_neox(_p(t), _i(nh), _i(hd), _i(pos), _f(theta), _i(rot))
        return t

    def conv1d_tapmajor(self, x, state, oldest, w_t):
        state = state.copy()
        out = np.empty_like(x)
        self.lib.qref_conv1d_tapmajor(_p(x), _p(state), _i(oldest), _p(w_t), _p(out),
                                      _i(x.size), _i(w_t.shape[0]))
        return out, state

    # ---- modules ----
    def deltanet(self, w: dict, hidden: int, n_heads: int, head_dim: int):
        L = self.lib
        h = L.qref_deltanet_create(
            _p(w["qkv_q"]), _p(w["qkv_s"]), _p(w["z_q"]), _p(w["z_s"]), _p(w["b_q"]),
            _p(w["b_s"]), _p(w["a_q"]), _p(w["a_s"]), _p(w["conv_w"]), _p(w["norm_w"]),
            _p(w["A_log"]), _p(w["dt_bias"]), _p(w["out_q"]), _p(w["out_s"]), _i(hidden),
            _i(n_heads), _i(head_dim), _i(w["conv_w"].shape[-1]))
        return _RefModule(L, h, "qref_deltanet_forward", "qref_deltanet_destroy", hidden)

    def gqa(self, w: dict, hidden: int, n_q: int, n_kv: int, hd: int, rot: int, theta: float,
            max_seq: int):
        L = self.lib
        h = L.qref_gqa_create(
            _p(w["q_q"]), _p(w["q_s"]), _i(w["q_q"].shape[0]), _p(w["k_q"]), _p(w["k_s"]),
            _p(w["v_q"]), _p(w["v_s"]), _p(w["o_q"]), _p(w["o_s"]), _p(w["q_norm"]),
            _p(w["k_norm"]), _i(hidden), _i(n_q), _i(n_kv), _i(hd), _i(rot), _f(theta),
            _i(max_seq))
        return _RefModule(L, h, "qref_gqa_forward", "qref_gqa_destroy", hidden)

    def load_model(self, model_dir: str, max_seq_len: int = 2048, precision: str = "int8"):
        h = self.lib.qref_model_load(model_dir.encode(), _i(max_seq_len), precision.encode())
        if not h:
            raise RuntimeError(f"reference failed to load {model_dir}")
        return RefModel(self.lib, h)


class _RefModule:
    def __init__(self, lib, h, fwd, dtor, hidden):
        self.lib, self.h, self.fwd, self.dtor, self.hidden = lib, h, fwd, dtor, hidden

    def forward(self, x: np.ndarray, pos: int) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        rows = 1 if x.ndim == 1 else x.shape[0]
        out = np.empty_like(x)
        getattr(self.lib, self.fwd)(_vp(self.h), _p(x), _i(rows), _i(self.hidden), _p(out), _i(pos))
        return out

    def __del__(self):
        if getattr(self, "h", None):
            getattr(self.lib, self.dtor)(_vp(self.h))
            self.h = None


class RefModel:
    def __init__(self, lib, h):
        self.lib, self.h = lib, h
        self.vocab = int(lib.qref_model_vocab(_vp(h)))

    def reset(self):
        self.lib.qref_model_reset(_vp(self.h))

    def forward(self, token: int, pos: int) -> np.ndarray:
        lg = np.empty(self.vocab, np.float32)
        self.lib.qref_model_forward(_vp(self.h), _i(token), _i(pos), _p(lg))
        return lg

    def forward_batch(self, tokens, pos: int) -> np.ndarray:
        t = np.ascontiguousarray(tokens, np.int32)
        lg = np.empty((t.size, self.vocab), np.float32)
        self.lib.qref_model_forward_batch(_vp(self.h), _p(t), _i(t.size), _i(pos), _p(lg))
        return lg

    def generate(self, prompt, n_new: int, keep_logits: bool = False):
        """Greedy loop with the CLI's convention; returns (tokens, prefill_s, decode_s, logits)."""
        p = np.ascontiguousarray(prompt, np.int32)
        out = np.empty(n_new, np.int32)
        pre = C.c_double()
        dec = C.c_double()
        lg = np.empty((n_new, self.vocab), np.float32) if keep_logits else None
        self.lib.qref_model_generate(_vp(self.h), _p(p), _i(p.size), _i(n_new), _p(out),
                                     C.byref(pre), C.byref(dec), _p(lg))
        return out, pre.value, dec.value, lg

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.qref_model_free(_vp(self.h))
            self.h = None


def read_safetensors(path: str) -> dict:
    """name -> array view of a .safetensors file (F32 as float32, BF16 as
    raw uint16 bit patterns, I32/I64 as integers)."""
    import json
    import struct

    kinds = {"F32": np.float32, "BF16": np.uint16, "I32": np.int32, "I64": np.int64,
             "F16": np.float16, "I8": np.int8, "U8": np.uint8}
    with open(path, "rb") as f:
        (hlen,) = struct.unpack("<Q", f.read(8))
        header = json.loads(f.read(hlen))
    base = 8 + hlen
    mm = np.memmap(path, dtype=np.uint8, mode="r")
    out = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        o0, o1 = info["data_offsets"]
        out[name] = mm[base + o0:base + o1].view(kinds[info["dtype"]]).reshape(info["shape"])
    return out


class OracleModel:
    """DecoderModel restated over the C oracle ops (model.cpp:151-274,
    modules.hpp:210-241, attention.cpp; fusion off, speculative off).

    Weights are read with safetensors' numpy loader and quantised by the
    oracle quantiser: group 32 (the reference's Q8_0, the default) or
    group="row" (one scale per output row, G = K)."""

    def __init__(self, model_dir: str, max_seq_len: int = 2048, oracle: Oracle | None = None,
                 group=32):
        import json

        self.o = oracle or Oracle()
        with open(os.path.join(model_dir, "config.json")) as f:
            c = json.load(f)
        c = c.get("text_config", c)
        self.c = c
        t = {}
        for fn in sorted(os.listdir(model_dir)):
            if fn.endswith(".safetensors"):
                t.update(read_safetensors(os.path.join(model_dir, fn)))
        self.t = t
        self.H = c["hidden_size"]
        self.nh, self.d = c["linear_num_key_heads"], c["linear_key_head_dim"]
        self.nq, self.nkv, self.hd = c["num_attention_heads"], c["num_key_value_heads"], c["head_dim"]
        self.rot = int(self.hd * c.get("partial_rotary_factor", 1.0))
        self.theta = float(c["rope_theta"])
        self.eps = float(c.get("rms_norm_eps", 1e-6))
        self.types = c["layer_types"]
        self.max_seq = max_seq_len
        self.row = group == "row"
        if not self.row and group != 32:
            raise ValueError("group is 32 or 'row'")
        self.q = {}
        self.embed = self._f32("model.embed_tokens.weight")
        self.lm = self.o.quantize(self.embed, self._g(self.embed.shape[1]))
        self.reset()

    def _g(self, K):
        return K if self.row else 32

    def _f32(self, name):
        a = self.t[name]
        if a.dtype == np.uint16:  # bf16 bit patterns
            a = (a.astype(np.uint32) << 16).view(np.float32)
        return np.ascontiguousarray(a, np.float32)

    def _w(self, name):
        if name not in self.q:
            w = np.ascontiguousarray(self.t[name])
            self.q[name] = self.o.quantize(w, self._g(w.shape[1]))
        return self.q[name]

    def reset(self):
        HD = self.nh * self.d
        self.conv, self.S, self.kc, self.vc = {}, {}, {}, {}
        for i, ty in enumerate(self.types):
            if ty == "full_attention":
                self.kc[i] = np.zeros((self.max_seq, self.nkv, self.hd), np.float32)
                self.vc[i] = np.zeros_like(self.kc[i])
            else:
                self.conv[i] = np.zeros((3, 3 * HD), np.float32)
                self.S[i] = np.zeros((self.nh, self.d, self.d), np.float32)
        self.ring = 0

    def _mm(self, x, name):
        q, s = self._w(name)
        return self.o.matmul_i8(x[None, :], q, s, self._g(q.shape[1]))[0]

    def forward(self, token: int, pos: int) -> np.ndarray:
        o, H = self.o, self.H
        h = self.embed[token].copy()
        for i, ty in enumerate(self.types):
            p = f"model.layers.{i}."
            n1 = o.rms_norm(h[None, :], self._f32(p + "input_layernorm.weight"), self.eps)[0]
            if ty == "full_attention":
                qkv = np.concatenate([self._mm(n1, p + "self_attn.q_proj.weight"),
                                      self._mm(n1, p + "self_attn.k_proj.weight"),
                                      self._mm(n1, p + "self_attn.v_proj.weight")])
                gated = self.t[p + "self_attn.q_proj.weight"].shape[0] == 2 * self.nq * self.hd
                core = o.gqa_core(qkv, self._f32(p + "self_attn.q_norm.weight"),
                                  self._f32(p + "self_attn.k_norm.weight"), self.theta, self.rot,
                                  self.kc[i], self.vc[i], pos, self.nq, self.nkv, self.hd, gated)
                a = self._mm(core, p + "self_attn.o_proj.weight")
            else:
                proj = np.concatenate([self._mm(n1, p + "linear_attn.in_proj_qkv.weight"),
                                       self._mm(n1, p + "linear_attn.in_proj_z.weight"),
                                       self._mm(n1, p + "linear_attn.in_proj_b.weight"),
                                       self._mm(n1, p + "linear_attn.in_proj_a.weight")])
                cw = self._f32(p + "linear_attn.conv1d.weight")
                wt = np.ascontiguousarray(cw.reshape(cw.shape[0], -1).T)
                core = o.deltanet_core(proj, self.conv[i], self.ring, wt,
                                       self._f32(p + "linear_attn.A_log"),
                                       self._f32(p + "linear_attn.dt_bias"),
                                       self._f32(p + "linear_attn.norm.weight"), self.S[i],
                                       self.nh, self.d)
                a = self._mm(core, p + "linear_attn.out_proj.weight")
            h = (h + a).astype(np.float32)
            n2 = o.rms_norm(h[None, :], self._f32(p + "post_attention_layernorm.weight"),
                            self.eps)[0]
            g = self._mm(n2, p + "mlp.gate_proj.weight")
            u = self._mm(n2, p + "mlp.up_proj.weight")
            m = self._mm(o.silu_mul(g, u), p + "mlp.down_proj.weight")
            h = (h + m).astype(np.float32)
        self.ring = (self.ring + 1) % 3
        hn = o.rms_norm(h[None, :], self._f32("model.norm.weight"), self.eps)[0]
        return self.o.matmul_i8(hn[None, :], self.lm[0], self.lm[1],
                                  self._g(self.H))[0]

    def generate(self, prompt, n_new: int, keep_logits: bool = False):
        """main.cpp:574-690 convention: prefill prompt[:-1], then n_new steps."""
        self.reset()
        for p in range(len(prompt) - 1):
            self.forward(int(prompt[p]), p)
        nxt, pos, out, lgs = int(prompt[-1]), len(prompt) - 1, [], []
        for _ in range(n_new):
            lg = self.forward(nxt, pos)
            pos += 1
            if keep_logits:
                lgs.append(lg)
            nxt = self.o.argmax(lg)
            out.append(nxt)
        return np.array(out, np.int32), (np.stack(lgs) if keep_logits else None)
