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


def test_l2_plan_of_the_4b_projections():
    """qlm_gemv_mx_l2_plan (host only) lists, per half, the tiles the
    one-row GEMV's workgroups read first: tile t of the tile-major copy at
    t * (K / 64) fragments, the plan of a whole matrix ending exactly where
    the layout's bytes end, and never more tiles than the launch has
    workgroups."""
    from quicklm_amd import hip

    L = hip.lib()
    q, s = 1 << 32, 1 << 36  # never dereferenced: the builder only does arithmetic

    def layout(rows, K, group, halves):
        qb, sb = ctypes.c_size_t(), ctypes.c_size_t()
        assert L.qlm_mx_layout_bytes(rows, K, group, halves, ctypes.byref(qb),
                                     ctypes.byref(sb)) == 0
        return qb.value, sb.value

    def grid(N, K, epi):
        w, r, g = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        assert L.qlm_gemv_i8_mx_shape(N, K, epi, ctypes.byref(w), ctypes.byref(r),
                                      ctypes.byref(g)) == 0
        return g.value

    # out-projection 2560 x 2048, residual epilogue, group-32 scales
    p = hip.L2Plan()
    assert L.qlm_gemv_mx_l2_plan(q, s, 32, 0, 2560, 2048, 1, 1 << 30, ctypes.byref(p)) == 0
    qb, sb = layout(2560, 2048, 32, 1)
    assert p.nseg == 2 and list(p.tiles[:2]) == [160, 160] and grid(2560, 2048, 1) >= 160
    assert (p.base[0], p.base[1]) == (q, s)
    assert p.base[0] + p.tiles[0] * p.stride[0] == q + qb and p.bytes[0] == p.stride[0]
    assert p.base[1] + p.tiles[1] * p.stride[1] == s + sb and p.bytes[1] == p.stride[1]

    # gate/up [2F, K]: both halves, first tiles only (one per workgroup)
    F, H = 9728, 2560
    g = grid(F, H, 2)
    assert L.qlm_gemv_mx_l2_plan(q, s, 32, 0, F, H, 2, 1 << 30, ctypes.byref(p)) == 0
    qb, sb = layout(F, H, 32, 2)
    assert p.nseg == 6 and list(p.tiles[2:6]) == [g] * 4 and g < F // 16
    assert p.base[2] == q and p.base[4] == q + qb // 2  # half 1 starts mid-layout
    assert p.base[3] == s and p.base[5] == s + sb // 2
    assert p.stride[2] == (H // 64) * 1024 and p.stride[3] == (H // 64) * 128

    # no room for four more segments: refused, the plan unchanged
    assert L.qlm_gemv_mx_l2_plan(q, s, 32, 0, F, H, 2, 1 << 30, ctypes.byref(p)) == -2
    assert p.nseg == 6

    # fewer tiles on request; int4 halves the weight bytes; per-row scales
    # add no segment
    p = hip.L2Plan()
    assert L.qlm_gemv_mx_l2_plan(q, s, 32, 1, 2560, 2048, 1, 24, ctypes.byref(p)) == 0
    assert p.nseg == 2 and p.tiles[0] == 24 and p.bytes[0] == 32 * 512
    p = hip.L2Plan()
    assert L.qlm_gemv_mx_l2_plan(q, s, 2048, 0, 2560, 2048, 1, 1 << 30, ctypes.byref(p)) == 0
    assert p.nseg == 1 and p.bytes[0] == 32 * 1024
    assert L.qlm_gemv_mx_l2_plan(q, s, 32, 0, 2560, 2000, 1, 8, ctypes.byref(p)) == -2  # K % 64


def test_mixer_plan_checks_run_before_any_launch():
    """qlm_deltanet_decode_cols_pf rejects a malformed plan (-1) and a plan
    with B > 1 (-2) on the host."""
    from quicklm_amd import hip

    L = hip.lib()
    fake = 4096
    p = hip.L2Plan()
    p.nseg, p.base[0], p.stride[0], p.bytes[0], p.tiles[0] = 1, fake, 1024, 1000, 8  # 1000 % 16
    H, d = 16, 128
    args = (fake, 4 * H * d + 2 * H, fake, fake, fake, fake, fake, fake, fake, fake, H * d, fake,
            fake)
    assert L.qlm_deltanet_decode_cols_pf(*args, 1, H, d, ctypes.byref(p), None) == -1
    p.bytes[0], p.base[0] = 1024, fake + 8  # base not 16-byte aligned
    assert L.qlm_deltanet_decode_cols_pf(*args, 1, H, d, ctypes.byref(p), None) == -1
    p.base[0], p.stride[0] = fake, 1000  # stride not a multiple of 16
    assert L.qlm_deltanet_decode_cols_pf(*args, 1, H, d, ctypes.byref(p), None) == -1
    p.stride[0], p.tiles[0] = 1024, 1 << 27  # more pieces than the kernel counts
    assert L.qlm_deltanet_decode_cols_pf(*args, 1, H, d, ctypes.byref(p), None) == -1
    p.tiles[0] = 8
    assert L.qlm_deltanet_decode_cols_pf(*args, 2, H, d, ctypes.byref(p), None) == -2
