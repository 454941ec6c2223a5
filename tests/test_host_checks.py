"""Argument refusals that the C ABI decides on the host, tested without a
GPU: every case here is rejected before any device call, so the arguments
include addresses that are never dereferenced (4096). Run in the CPU suite
only, where no kernel can launch even if a check regressed (the HIP calls
after the checks would then fail on the missing device, not touch memory).
"""

import ctypes as C

import pytest

from quicklm_amd import hip

FAKE = 4096


@pytest.fixture(scope="module")
def lib():
    L = hip.lib()
    if hip.device_count() > 0:
        pytest.skip("host-only refusal tests run where no GPU is visible")
    return L


def test_noalloc_attention_oversize_refused(lib):
    """Calls whose chunk records exceed the 32 MiB static scratch return
    QLM_ERR_SCRATCH (-4) before any launch; the byte query agrees."""
    cap = 32 << 20
    for kv, B, ctx in ((0, 16, 32768), (1, 128, 32768)):
        assert lib.qlm_attention_decode_noalloc_bytes(B, 16, 256, ctx) > cap
        assert lib.qlm_attention_decode_noalloc(FAKE, FAKE, FAKE, kv, ctx, ctx, FAKE, B, 16, 2,
                                                256, None) == -4
    assert lib.qlm_attention_decode_noalloc_bytes(2, 16, 256, 3000) <= cap


def test_noalloc_attention_bad_arguments(lib):
    assert lib.qlm_attention_decode_noalloc(None, FAKE, FAKE, 0, 64, 64, FAKE, 1, 16, 2, 256,
                                            None) == -1
    assert lib.qlm_attention_decode_noalloc(FAKE, FAKE, FAKE, 0, 64, 65, FAKE, 1, 16, 2, 256,
                                            None) == -1  # ctx > max_seq
    assert lib.qlm_attention_decode_noalloc(FAKE, FAKE, FAKE, 0, 64, 64, FAKE, 1, 12, 8, 256,
                                            None) == -2  # 12 q heads over 8 kv heads
    assert lib.qlm_attention_decode_noalloc(FAKE, FAKE, FAKE, 0, 64, 64, FAKE, 1, 16, 2, 192,
                                            None) == -2  # head dim 192


def test_matmul_i8_rows64_refused(lib):
    """Shapes outside the int8-digit form are refused with QLM_ERR_SHAPE (-2):
    1 or 65 rows, SwiGLU, K not a multiple of 64; the workspace query returns
    0 for them."""
    for M, K, e in ((1, 256, 0), (65, 256, 0), (32, 256, 2), (32, 200, 0)):
        assert lib.qlm_matmul_i8_rows64(FAKE, K, None, C.c_float(0.0), FAKE, FAKE, FAKE, 64, M,
                                        64, K, e, FAKE, C.c_size_t(1 << 30), None) == -2
    assert lib.qlm_matmul_i8_rows64_workspace_bytes(1, 64, 256, 0) == 0
    assert lib.qlm_matmul_i8_rows64_workspace_bytes(33, 64, 256, 2) == 0
