"""The C ABI libraries load and export every entry point their headers
declare, and the Python bindings describe exactly those symbols. No GPU call
is made."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header: str) -> list[str]:
    text = open(os.path.join(ROOT, "include", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qlm_\w+)\s*\(", text)))


@pytest.mark.parametrize("header,lib", [("qlm_hip.h", "libqlm_hip.so"),
                                        ("qlm_engine.h", "libqlm_engine.so")])
def test_library_exports_every_declared_symbol(header, lib):
    path = os.path.join(ROOT, "quicklm_amd", lib)
    assert os.path.exists(path), f"{lib} not built"
    L = ctypes.CDLL(path)
    names = declared(header)
    assert len(names) > 10
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_python_binding_covers_kernel_abi():
    from quicklm_amd import hip

    assert sorted(hip.exported_symbols()) == declared("qlm_hip.h")


def test_error_strings_need_no_device():
    from quicklm_amd import hip

    L = hip.lib()
    assert b"unsupported shape" in L.qlm_error_string(-2)
    assert b"invalid argument" in L.qlm_error_string(-1)


def test_shape_checks_run_before_any_launch():
    """Invalid shapes are rejected on the host (no device memory touched)."""
    from quicklm_amd import hip

    L = hip.lib()
    assert L.qlm_gemv_i8(None, 0, None, None, 32, None, 0, 1, 1, 1, None) == -1
    fake = 4096  # never dereferenced: the checks fire first
    assert L.qlm_gemv_i8(fake, 40, fake, fake, 40, fake, 4, 1, 4, 40, None) == -2  # K % 16
    assert L.qlm_gemv_i8(fake, 48, fake, fake, 32, fake, 4, 1, 4, 48, None) == -2  # K % 32
    assert L.qlm_deltanet_decode(fake, 8, fake, fake, fake, fake, fake, fake, None, fake, 8, 1, 1,
                                 64, None) == -2  # d must be 128
    assert L.qlm_gqa_decode(fake, 4096, fake, fake, fake, fake, 32, fake, fake, 64, fake, fake,
                            4096, 1, 3, 2, 128, 1, fake, None) == -2  # 3 q heads over 2 kv heads


def test_noalloc_attention_rejects_oversize_on_host():
    """qlm_attention_decode_noalloc refuses work beyond its static scratch
    (QLM_ERR_SCRATCH) before touching any device memory."""
    from quicklm_amd import hip

    L = hip.lib()
    cap = 32 << 20
    # B * n_q * ceil(ctx / C) * (hd + 4) * 4 bytes: C = 256 positions for 16
    # sequences of 32768 at hd 256 (128 chunks), 64 for one of 300 at hd 128
    # the bf16 layout bounds it here: min(256, 32768 / 32) records a head
    assert L.qlm_attention_decode_noalloc_bytes(16, 16, 256, 32768) == 16 * 16 * 256 * 260 * 4
    assert L.qlm_attention_decode_noalloc_bytes(1, 16, 128, 300) == 16 * 5 * 132 * 4
    assert L.qlm_attention_decode_noalloc_bytes(0, 16, 128, 300) == 0
    assert L.qlm_attention_decode_noalloc_bytes(1, 16, 64, 300) == 0
    assert L.qlm_attention_decode_noalloc_bytes(16, 16, 256, 32768) > cap
    fake = 4096  # never dereferenced: the checks fire first
    # fp32 cache: 16 x 16 heads x 128 records of 260 floats = 34 MB
    assert L.qlm_attention_decode_noalloc(fake, fake, fake, 0, 32768, 32768, fake, 16, 16, 2, 256,
                                          None) == -4
    # bf16 cache: 128 x 16 heads x 32 records (1024 positions each) = 68 MB
    assert L.qlm_attention_decode_noalloc(fake, fake, fake, 1, 32768, 32768, fake, 128, 16, 2,
                                          256, None) == -4
    assert b"static device scratch" in L.qlm_error_string(-4)
    assert L.qlm_attention_decode_noalloc(fake, fake, fake, 1, 100, 200, fake, 1, 16, 2, 256,
                                          None) == -1  # ctx > max_seq
    assert L.qlm_attention_decode_noalloc(fake, fake, fake, 1, 100, 50, fake, 1, 16, 2, 96,
                                          None) == -2  # head dim
