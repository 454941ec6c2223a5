"""ctypes binding of the host engine's C ABI (include/qlm_engine.h)."""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import hip as _hip  # noqa: F401  (loads libqlm_hip.so first; raises if missing)

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqlm_engine.so")
_lib = None

_vp, _i = C.c_void_p, C.c_int


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _hip.lib()
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m quicklm_amd.build`")
        L = C.CDLL(LIB_PATH)
        L.qlm_engine_last_error.restype = C.c_char_p
        L.qlm_engine_load.argtypes = [C.c_char_p, _i, _i, C.c_char_p, C.POINTER(_vp)]
        L.qlm_engine_free.argtypes = [_vp]
        L.qlm_engine_info.argtypes = [_vp] + [C.POINTER(_i)] * 6 + [C.POINTER(C.c_size_t)]
        L.qlm_engine_reset.argtypes = [_vp]
        L.qlm_engine_forward.argtypes = [_vp, _i, _i, _vp]
        L.qlm_engine_generate.argtypes = [_vp, _vp, _i, _i, _i, _vp, C.POINTER(C.c_double),
                                          C.POINTER(C.c_double), _i, _i]
        L.qlm_engine_last_logits.argtypes = [_vp, _i, _vp]
        L.qlm_engine_start.argtypes = [_vp, _vp, _i, _i, _i, C.POINTER(C.c_double)]
        L.qlm_engine_steps.argtypes = [_vp, _i, _i, C.POINTER(C.c_double)]
        L.qlm_engine_tokens.argtypes = [_vp, _i, _i, _i, _vp]
        L.qlm_engine_kernels_per_step.argtypes = [_vp]
        L.qlm_engine_snapshot.argtypes = [_vp]
        L.qlm_engine_restore.argtypes = [_vp]
        L.qlm_engine_forward_greedy.argtypes = [_vp, _i, _i, C.POINTER(_i)]
        L.qlm_engine_forward_batch.argtypes = [_vp, _vp, _i, _i, _vp, _vp]
        L.qlm_session_create.argtypes = [_vp, _vp, _i, _i, _i, _i, C.POINTER(_vp)]
        L.qlm_session_free.argtypes = [_vp]
        L.qlm_session_reset.argtypes = [_vp]
        L.qlm_session_turn.argtypes = [_vp, _vp, _i, _i, _vp, _i, C.POINTER(_i), _vp,
                                       C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.qlm_session_cached.argtypes = [_vp, _vp, _i, C.POINTER(_i)]
        _lib = L
    return _lib


class EngineError(RuntimeError):
    pass


def _check(rc: int) -> None:
    if rc != 0:
        raise EngineError(lib().qlm_engine_last_error().decode())


class Engine:
    """DecoderModel on the GPU: load a checkpoint directory, decode greedily."""

    def __init__(self, model_dir: str, max_seq_len: int = 2048, max_batch: int = 1,
                 precision: str = "int8"):
        h = _vp()
        _check(lib().qlm_engine_load(model_dir.encode(), max_seq_len, max_batch,
                                     precision.encode(), C.byref(h)))
        self.h = h.value
        vals = [_i() for _ in range(6)]
        wb = C.c_size_t()
        _check(lib().qlm_engine_info(self.h, *[C.byref(v) for v in vals], C.byref(wb)))
        (self.vocab, self.hidden, self.layers, self.group, self.max_seq,
         self.max_batch) = [v.value for v in vals]
        self.weight_bytes = wb.value

    def reset(self) -> None:
        _check(lib().qlm_engine_reset(self.h))

    def forward(self, token: int, pos: int) -> np.ndarray:
        lg = np.empty(self.vocab, np.float32)
        _check(lib().qlm_engine_forward(self.h, token, pos, lg.ctypes.data))
        return lg

    PREFILL_STEPS, PREFILL_CHUNKED, PREFILL_ROWS = 0, 1, 2

    def generate(self, prompts: np.ndarray, n_new: int, use_graph: bool = True,
                 batched_prefill=True):
        """prompts [B, n] int32 -> (tokens [B, n_new], prefill_s, decode_s).
        batched_prefill: True (or PREFILL_CHUNKED) = batched prefill with the
        chunked DeltaNet form; PREFILL_ROWS = batched with the row-by-row
        recurrence; False = each prompt position forwarded by a decode step."""
        mode = self._mode(batched_prefill)
        p = np.ascontiguousarray(np.atleast_2d(prompts), np.int32)
        B, n = p.shape
        out = np.empty((B, n_new), np.int32)
        pre, dec = C.c_double(), C.c_double()
        _check(lib().qlm_engine_generate(self.h, p.ctypes.data, B, n, n_new, out.ctypes.data,
                                         C.byref(pre), C.byref(dec), 1 if use_graph else 0,
                                         mode))
        return out, pre.value, dec.value

    @staticmethod
    def _mode(batched_prefill) -> int:
        if batched_prefill is True:
            return 1
        if batched_prefill is False:
            return 0
        return int(batched_prefill)

    def start(self, prompts: np.ndarray, batched_prefill=False) -> float:
        """Install prompts; with batched_prefill (as in generate) also prefill
        positions 0..n-2 and return its wall time in seconds (the next step
        forwards n-1)."""
        p = np.ascontiguousarray(np.atleast_2d(prompts), np.int32)
        self._prompts = p
        pre = C.c_double()
        _check(lib().qlm_engine_start(self.h, p.ctypes.data, p.shape[0], p.shape[1],
                                      self._mode(batched_prefill), C.byref(pre)))
        return pre.value

    def steps(self, k: int, use_graph: bool = True) -> float:
        """Run k decode steps; returns their GPU time in ms."""
        ms = C.c_double()
        _check(lib().qlm_engine_steps(self.h, k, 1 if use_graph else 0, C.byref(ms)))
        return ms.value

    def tokens(self, b: int, first: int, count: int) -> np.ndarray:
        out = np.empty(count, np.int32)
        _check(lib().qlm_engine_tokens(self.h, b, first, count, out.ctypes.data))
        return out

    def last_logits(self, b: int = 0) -> np.ndarray:
        lg = np.empty(self.vocab, np.float32)
        _check(lib().qlm_engine_last_logits(self.h, b, lg.ctypes.data))
        return lg

    def snapshot(self) -> None:
        """Snapshot every DeltaNet recurrence and conv ring (one slot)."""
        _check(lib().qlm_engine_snapshot(self.h))

    def restore(self) -> None:
        _check(lib().qlm_engine_restore(self.h))

    def forward_greedy(self, token: int, pos: int) -> int:
        """One decode step of `token` at `pos`; returns the greedy pick."""
        nx = _i()
        _check(lib().qlm_engine_forward_greedy(self.h, token, pos, C.byref(nx)))
        return nx.value

    def forward_batch(self, tokens, pos: int, argmax: bool = True, logits: bool = False):
        """tokens at positions pos.. through every layer at once; returns
        (argmax [n] or None, logits [n, vocab] or None)."""
        t = np.ascontiguousarray(tokens, np.int32).ravel()
        am = np.empty(t.size, np.int32) if argmax else None
        lg = np.empty((t.size, self.vocab), np.float32) if logits else None
        _check(lib().qlm_engine_forward_batch(self.h, t.ctypes.data, t.size, pos,
                                              None if am is None else am.ctypes.data,
                                              None if lg is None else lg.ctypes.data))
        return am, lg

    def kernels_per_step(self) -> int:
        return int(lib().qlm_engine_kernels_per_step(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().qlm_engine_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """The CLI's multi-turn loop over token ids (include/qlm_engine.h,
    qlm_session_*): kv-reuse of the live state, batched prefill of the new
    prompt suffix, then speculative decoding when a draft engine is given
    (K = draft_tokens drafted per round), else plain greedy steps."""

    INFO = ("reused", "recomputed", "rounds", "drafted", "accepted", "emitted", "rejections")

    def __init__(self, target: Engine, draft: Engine | None = None, draft_tokens: int = 4,
                 eos_id: int = -1, im_end_id: int = -1, kv_reuse: bool = True):
        h = _vp()
        _check(lib().qlm_session_create(target.h, None if draft is None else draft.h,
                                        draft_tokens, eos_id, im_end_id, 1 if kv_reuse else 0,
                                        C.byref(h)))
        self.h = h.value
        self._keep = (target, draft)

    def turn(self, ids, max_tokens: int):
        """-> (tokens, info dict with the INFO counters and prefill_s / decode_s)."""
        p = np.ascontiguousarray(ids, np.int32).ravel()
        out = np.empty(max(1, max_tokens), np.int32)
        n_out = _i()
        info = np.zeros(7, np.int32)
        pre, dec = C.c_double(), C.c_double()
        _check(lib().qlm_session_turn(self.h, p.ctypes.data, p.size, max_tokens, out.ctypes.data,
                                      out.size, C.byref(n_out), info.ctypes.data, C.byref(pre),
                                      C.byref(dec)))
        d = dict(zip(self.INFO, (int(v) for v in info)))
        d.update(prefill_s=pre.value, decode_s=dec.value)
        return out[:n_out.value].copy(), d

    def cached(self) -> np.ndarray:
        n = _i()
        _check(lib().qlm_session_cached(self.h, None, 0, C.byref(n)))
        out = np.empty(n.value, np.int32)
        _check(lib().qlm_session_cached(self.h, out.ctypes.data, out.size, C.byref(n)))
        return out

    def reset(self) -> None:
        _check(lib().qlm_session_reset(self.h))

    def close(self) -> None:
        if getattr(self, "h", None):
            lib().qlm_session_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
