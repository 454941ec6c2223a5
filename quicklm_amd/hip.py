"""ctypes binding of the gfx950 kernel library's C ABI (include/qlm_hip.h).

The library is built in-tree (`python -m quicklm_amd.build`). There is no
fallback: importing the binding when libqlm_hip.so is missing raises.
"""

from __future__ import annotations

import ctypes as C
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libqlm_hip.so")

_vp, _i, _f, _sz, _u8 = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint8
_lib = None


class HipError(RuntimeError):
    pass


class L2Plan(C.Structure):
    """qlm_l2_plan: a later kernel's operands by tile (segment s of tile t:
    bytes[s] bytes at base[s] + t * stride[s], for t < tiles[s])."""
    _fields_ = [("base", C.c_void_p * 8), ("stride", C.c_longlong * 8), ("bytes", C.c_int * 8),
                ("tiles", C.c_int * 8), ("nseg", C.c_int)]


# name -> (restype, argtypes)
_SIGS = {
    "qlm_error_string": (C.c_char_p, [_i]),
    "qlm_device_count": (_i, [C.POINTER(_i)]),
    "qlm_set_device": (_i, [_i]),
    "qlm_device_name": (_i, [C.c_char_p, _i]),
    "qlm_mem_info": (_i, [C.POINTER(_sz), C.POINTER(_sz)]),
    "qlm_malloc": (_i, [C.POINTER(_vp), _sz]),
    "qlm_free": (_i, [_vp]),
    "qlm_memcpy_h2d": (_i, [_vp, _vp, _sz, _vp]),
    "qlm_memcpy_d2h": (_i, [_vp, _vp, _sz, _vp]),
    "qlm_memcpy_d2d": (_i, [_vp, _vp, _sz, _vp]),
    "qlm_fill_u8": (_i, [_vp, _u8, _sz, _vp]),
    "qlm_stream_create": (_i, [C.POINTER(_vp)]),
    "qlm_stream_destroy": (_i, [_vp]),
    "qlm_stream_sync": (_i, [_vp]),
    "qlm_device_sync": (_i, []),
    "qlm_event_create": (_i, [C.POINTER(_vp)]),
    "qlm_event_destroy": (_i, [_vp]),
    "qlm_event_record": (_i, [_vp, _vp]),
    "qlm_event_elapsed_ms": (_i, [C.POINTER(_f), _vp, _vp]),
    "qlm_graph_begin": (_i, [_vp]),
    "qlm_graph_end": (_i, [_vp, C.POINTER(_vp)]),
    "qlm_graph_launch": (_i, [_vp, _vp]),
    "qlm_graph_destroy": (_i, [_vp]),
    "qlm_quantize_q8_f32": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "qlm_quantize_q8_bf16": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "qlm_gemv_i8": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "qlm_deltanet_prefill": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _i,
                                  _vp]),
    "qlm_deltanet_chunk_workspace_bytes": (_sz, [_i, _i, _i]),
    "qlm_deltanet_prefill_chunked": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i,
                                          _i, _i, _vp, _sz, _vp]),
    "qlm_gqa_prefill_workspace_bytes": (_sz, [_i, _i, _i]),
    "qlm_gqa_prefill": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _vp, _i, _i,
                             _i, _i, _i, _vp, _vp]),
    "qlm_matmul_i8_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "qlm_matmul_i8": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _sz,
                           _vp]),
    "qlm_matmul_i8_tm": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _sz,
                              _vp]),
    "qlm_gemv_i8_config": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "qlm_gemv_i8_mx_config": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i,
                                   _vp]),
    "qlm_mx_layout_bytes": (_i, [_i, _i, _i, _i, C.POINTER(_sz), C.POINTER(_sz)]),
    "qlm_gemv_i8_mx": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _vp]),
    "qlm_matmul_i8_mx_workspace_bytes": (_sz, [_i, _i]),
    "qlm_matmul_i8_rows64_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "qlm_matmul_i8_rows64": (_i, [_vp, _i, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz,
                                  _vp]),
    "qlm_matmul_i8_t_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "qlm_matmul_i8_t": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _sz,
                             _vp]),
    "qlm_matmul_i8_t_config": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i,
                                    _i, _i, _i, _vp, _sz, _vp]),
    "qlm_matmul_i8_t_whole_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "qlm_matmul_i8_t_whole_config": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i,
                                          _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "qlm_matmul_i8_mx": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _sz,
                              _vp]),
    "qlm_gemv_i8_mx_shape": (_i, [_i, _i, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i)]),
    "qlm_matmul_i8_mx_shape": (_i, [_i, _i, _i, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i),
                                    C.POINTER(_i)]),
    "qlm_mx_swizzle": (_i, [_vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp]),
    "qlm_gemv_i8_rmsnorm": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "qlm_gemv_i8_residual": (_i, [_vp, _i, _vp, _vp, _i, _vp, _i, _i, _i, _i, _vp]),
    "qlm_gemv_i8_swiglu_rmsnorm": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _i,
                                        _vp]),
    "qlm_rms_norm": (_i, [_vp, _vp, _vp, _i, _i, _f, _vp]),
    "qlm_add_rms_norm": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "qlm_silu_mul": (_i, [_vp, _vp, _i, _vp]),
    "qlm_rope_neox": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "qlm_conv1d_update": (_i, [_vp, _vp, _i, _vp, _vp, _i, _i, _vp]),
    "qlm_gated_delta_step": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "qlm_deltanet_decode": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i,
                                 _i, _vp]),
    "qlm_deltanet_decode_cols": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp,
                                      _vp, _i, _i, _i, _vp]),
    "qlm_deltanet_decode_cols_pf": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i,
                                         _vp, _vp, _i, _i, _i, C.POINTER(L2Plan), _vp]),
    "qlm_gemv_mx_l2_plan": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, C.POINTER(L2Plan)]),
    "qlm_gemv_i8_mx_headnorm": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _i, _vp]),
    "qlm_gemv_i4_mx_headnorm": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "qlm_gqa_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "qlm_gqa_decode": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i,
                            _i, _i, _i, _i, _vp, _vp]),
    "qlm_attention_decode": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp]),
    "qlm_attention_decode_noalloc_bytes": (_sz, [_i, _i, _i, _i]),
    "qlm_attention_decode_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp, _i, _i, _i, _i, _vp]),
    "qlm_argmax": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "qlm_argmax_workspace_bytes": (_sz, [_i, _i]),
    "qlm_greedy_advance": (_i, [_vp, _i, _i, _i, _vp, _vp, _i, _vp, _vp, _vp]),
    "qlm_lm_head_greedy_workspace_bytes": (_sz, []),
    "qlm_lm_head_greedy": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _i, _vp, _vp,
                                _vp, _i, _vp, _vp]),
    "qlm_lm_head_greedy_mx": (_i, [_vp, _vp, _f, _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _i, _vp, _vp,
                                _vp, _i, _vp, _vp]),
    "qlm_embed_tokens": (_i, [_vp, _i, _i, _vp, _i, _vp, _vp, _i, _i, _vp]),
    "qlm_matmul_w_workspace_bytes": (_sz, [_i]),
    "qlm_matmul_bf16_workspace_bytes": (_sz, [_i, _i]),
    "qlm_matmul_bf16": (_i, [_vp, _i, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "qlm_matmul_w": (_i, [_vp, _i, _vp, _f, _vp, _i, _vp, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "qlm_gemv_w_config": (_i, [_vp, _vp, _f, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _vp]),
    "qlm_quantize_q4_f32": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "qlm_quantize_q4_bf16": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "qlm_mx4_layout_bytes": (_i, [_i, _i, _i, C.POINTER(_sz), C.POINTER(_sz)]),
    "qlm_mx4_swizzle": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "qlm_gemv_i4_mx_config": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "qlm_gemv_i4_mx": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "qlm_lm_head_greedy_mx4": (_i, [_vp, _vp, _f, _vp, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _vp,
                                    _vp, _i, _vp, _vp]),
}


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m quicklm_amd.build` "
                              "(there is no CPU fallback)")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGS)


def check(rc: int) -> None:
    if rc != 0:
        msg = lib().qlm_error_string(rc)
        raise HipError(f"qlm call failed ({rc}): {msg.decode() if msg else '?'}")


def device_count() -> int:
    n = _i(0)
    rc = lib().qlm_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def device_name() -> str:
    buf = C.create_string_buffer(256)
    check(lib().qlm_device_name(buf, 256))
    return buf.value.decode()


def mem_free() -> int:
    """Free bytes of the current device."""
    f, t = _sz(), _sz()
    check(lib().qlm_mem_info(C.byref(f), C.byref(t)))
    return f.value


def sync() -> None:
    check(lib().qlm_device_sync())


class DeviceBuffer:
    """Owned device allocation (hipMalloc through the C ABI)."""

    def __init__(self, nbytes: int):
        p = _vp()
        check(lib().qlm_malloc(C.byref(p), max(int(nbytes), 1)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        check(lib().qlm_memcpy_h2d(b.ptr, a.ctypes.data, a.nbytes, None))
        sync()
        return b

    def to_numpy(self, shape, dtype) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(lib().qlm_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes, None))
        sync()
        return out

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        check(lib().qlm_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes, None))
        sync()

    def zero(self) -> None:
        check(lib().qlm_fill_u8(self.ptr, 0, self.nbytes, None))

    def free(self) -> None:
        if self.ptr:
            lib().qlm_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = _vp()
        check(lib().qlm_event_create(C.byref(p)))
        self.ptr = p.value

    def record(self, stream=None):
        check(lib().qlm_event_record(self.ptr, stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = _f()
        check(lib().qlm_event_elapsed_ms(C.byref(ms), self.ptr, later.ptr))
        return ms.value

    def __del__(self):
        try:
            lib().qlm_event_destroy(self.ptr)
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _vp()
        check(lib().qlm_stream_create(C.byref(p)))
        self.ptr = p.value

    def sync(self):
        check(lib().qlm_stream_sync(self.ptr))

    def __del__(self):
        try:
            lib().qlm_stream_destroy(self.ptr)
        except Exception:
            pass


def call(name: str, *args) -> None:
    """Invoke a C ABI entry point; DeviceBuffer arguments pass their pointer."""
    conv = [a.ptr if isinstance(a, DeviceBuffer) else a for a in args]
    check(getattr(lib(), name)(*conv))
