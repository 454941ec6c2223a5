"""int4 (Q4_0) weights on the GPU (reference --precision int4).

Bars: the device quantiser is bit-exact with the oracle (which is bit-exact
with the reference, tests/test_oracle.py), including the int8 expansion of
its values; the int4 tile-major copy holds exactly the documented nibbles;
the one-row GEMV over int4 tiles is bit-identical to the int8 matrix-core
GEMV over the expanded weights (same digits, same exact int32 sums, same
scaling) and within 1e-5 normwise of the oracle's int4 matmul.
"""

import ctypes as C

import numpy as np
import pytest

from tests.util import bf16_bits, rel_err, say

pytestmark = pytest.mark.gpu


def dev(hip, a):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def _q4(hip, w):
    """Device int4 quantisation of fp32 (or bf16 bits) rows: packed, scales, int8 values."""
    rows, K = w.shape
    dq4 = hip.DeviceBuffer(rows * K // 2)
    ds = hip.DeviceBuffer(rows * (K // 32) * 4)
    dq8 = hip.DeviceBuffer(rows * K)
    fn = "qlm_quantize_q4_bf16" if w.dtype == np.uint16 else "qlm_quantize_q4_f32"
    dw = dev(hip, w)
    hip.call(fn, dw, rows, K, dq4, ds, dq8, None)
    return dq4, ds, dq8


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_quantize_q4_bitexact(hip, orc, rng, dtype):
    rows, K = 97, 2560
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    w[3] = 0.0                                     # all-zero row: scale 1, nibbles 8
    w[5, :32] = np.arange(32, dtype=np.float32) * np.float32(0.25) - 4  # exact halves
    w[7, 5] = 1e30                                 # one huge value dominates its group
    src = bf16_bits(w) if dtype == "bf16" else w
    p_ref, s_ref = orc.quantize_q4(src)
    say("quantize_q4", dtype, rows, K)
    dq4, ds, dq8 = _q4(hip, src)
    assert np.array_equal(dq4.to_numpy((rows, K // 2), np.uint8), p_ref)
    assert np.array_equal(ds.to_numpy(s_ref.shape, np.float32).view(np.uint32),
                          s_ref.view(np.uint32))
    assert np.array_equal(dq8.to_numpy((rows, K), np.int8), orc.unpack_q4(p_ref, K))


def test_quantize_q4_rejects_bad_k(hip):
    d = hip.DeviceBuffer(64 * 4)
    with pytest.raises(hip.HipError):
        hip.call("qlm_quantize_q4_f32", d, 1, 48, d, d, None, None)


def _mx4_layout(hip, dq4, ds, rows, K, halves):
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx4_layout_bytes(rows, K, halves, C.byref(qb), C.byref(sb)))
    qz, sz = hip.DeviceBuffer(qb.value), hip.DeviceBuffer(sb.value)
    hip.call("qlm_mx4_swizzle", dq4, ds, rows, K, halves, qz, sz, None)
    return qz, sz


def _mx8_layout(hip, dq8, ds, rows, K, halves):
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx_layout_bytes(rows, K, 32, halves, C.byref(qb), C.byref(sb)))
    qz, sz = hip.DeviceBuffer(qb.value), hip.DeviceBuffer(sb.value)
    hip.call("qlm_mx_swizzle", dq8, ds, 32, rows, K, halves, qz, sz, None)
    return qz, sz


def test_mx4_swizzle_layout(hip, orc, rng):
    """Fragment (tile, block), lane l = 16q + n: 8 bytes for columns
    64b + 16q .. +15 of row 16t + n as nibbles value + 8 -- byte i of the
    first word = columns i (low) and 4 + i (high), of the second word
    8 + i and 12 + i; padded rows hold value 0 (0x88); scales as int8's."""
    rows, K, halves = 37, 192, 2
    w = (rng.standard_normal((halves * rows, K)) * 0.02).astype(np.float32)
    dq4, ds, dq8 = _q4(hip, w)
    vals = dq8.to_numpy((halves * rows, K), np.int8).astype(np.int32) + 8
    s = ds.to_numpy((halves * rows, K // 32), np.float32)
    qz, sz = _mx4_layout(hip, dq4, ds, rows, K, halves)
    tiles, nblk = (rows + 15) // 16, K // 64
    got = qz.to_numpy((halves * tiles, nblk, 64, 2), np.uint32)
    gs = sz.to_numpy((halves * tiles, nblk, 2, 16), np.float32)
    for g in range(halves * tiles):
        half, t = divmod(g, tiles)
        for b in range(nblk):
            for lane in range(64):
                n, qd = lane & 15, lane >> 4
                r = t * 16 + n
                v = vals[half * rows + r, 64 * b + 16 * qd:64 * b + 16 * qd + 16] if r < rows \
                    else np.full(16, 8)
                wa = sum(int(v[i] | (v[4 + i] << 4)) << (8 * i) for i in range(4))
                wb = sum(int(v[8 + i] | (v[12 + i] << 4)) << (8 * i) for i in range(4))
                assert (got[g, b, lane, 0], got[g, b, lane, 1]) == (wa, wb), (g, b, lane)
            for h in range(2):
                for n in range(16):
                    r = t * 16 + n
                    want = s[half * rows + r, 2 * b + h] if r < rows else 0.0
                    assert gs[g, b, h, n] == want


MX4_CASES = [  # (N, K, waves, ring, grid)
    (1000, 2560, 8, 5, 7), (1000, 2560, 4, 10, None), (300, 2048, 16, 2, None),
    (160, 9728, 16, 10, None), (2000, 2048, 8, 4, 5), (129, 512, 4, 2, 4),
]


@pytest.mark.parametrize("epi", ["store", "norm", "resid", "swiglu"])
def test_gemv_i4_mx(hip, orc, rng, epi):
    eps = 1e-6
    code = {"store": 0, "norm": 0, "resid": 1, "swiglu": 2}[epi]
    for N, K, waves, ring, grid in MX4_CASES:
        rows_w = 2 * N if epi == "swiglu" else N
        halves = 2 if epi == "swiglu" else 1
        w = (rng.standard_normal((rows_w, K)) * 0.02).astype(np.float32)
        p, s = orc.quantize_q4(w)
        x = rng.standard_normal((1, K)).astype(np.float32)
        nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
        y0 = rng.standard_normal((1, N)).astype(np.float32)
        if epi == "store":
            ref = orc.matmul_i4(x, p, s)
        elif epi == "resid":
            ref = y0 + orc.matmul_i4(x, p, s)
        else:
            lg = orc.matmul_i4(orc.rms_norm(x, nw, eps), p, s)
            ref = lg if epi == "norm" else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
        say("gemv_i4_mx", epi, N, K, waves, ring, grid)
        dq4, ds, dq8 = _q4(hip, w)
        q4z, s4z = _mx4_layout(hip, dq4, ds, N, K, halves)
        q8z, s8z = _mx8_layout(hip, dq8, ds, N, K, halves)
        dx = dev(hip, x)
        dnw = dev(hip, nw) if epi in ("norm", "swiglu") else None
        g_ = grid or (N + 15) // 16
        y4, y8 = dev(hip, y0), dev(hip, y0)
        hip.call("qlm_gemv_i4_mx_config", dx, dnw, eps, q4z, s4z, y4, N, K, code, waves, ring,
                 g_, None)
        hip.call("qlm_gemv_i8_mx_config", dx, dnw, eps, q8z, s8z, 32, y8, N, K, code, waves,
                 ring, g_, None)
        a4 = y4.to_numpy((1, N), np.float32)
        assert np.array_equal(a4.view(np.uint32), y8.to_numpy((1, N), np.float32).view(np.uint32))
        err = rel_err(a4, ref)
        assert err < 1e-5, (epi, N, K, waves, ring, grid, err)


@pytest.mark.parametrize("N,K,epi", [(9728, 2560, 2), (2560, 9728, 1), (8224, 2560, 0),
                                     (2560, 2048, 1)])
def test_gemv_i4_mx_auto(hip, orc, rng, N, K, epi):
    """Launch shapes picked like the int8 path's (the 4B decode projections)."""
    rows_w = 2 * N if epi == 2 else N
    w = (rng.standard_normal((rows_w, K)) * 0.02).astype(np.float32)
    p, s = orc.quantize_q4(w)
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    y0 = rng.standard_normal((1, N)).astype(np.float32)
    if epi == 1:
        ref = y0 + orc.matmul_i4(x, p, s)
    else:
        lg = orc.matmul_i4(orc.rms_norm(x, nw, 1e-6), p, s)
        ref = lg if epi == 0 else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dq4, ds, _ = _q4(hip, w)
    q4z, s4z = _mx4_layout(hip, dq4, ds, N, K, 2 if epi == 2 else 1)
    dy = dev(hip, y0)
    say("gemv_i4_mx auto", N, K, epi)
    hip.call("qlm_gemv_i4_mx", dev(hip, x), None if epi == 1 else dev(hip, nw), 1e-6, q4z, s4z,
             dy, N, K, epi, None)
    assert rel_err(dy.to_numpy((1, N), np.float32), ref) < 1e-5


def test_lm_head_greedy_mx4(hip, orc, rng):
    """The greedy tail over int4 tiles: logits as the oracle's int4 matmul,
    token, position and next embedding as the int8 form's semantics."""
    V, K, L = 151936, 1024, 16
    w = (rng.standard_normal((V, K)) * 0.02).astype(np.float32)
    p, s = orc.quantize_q4(w)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    table = rng.standard_normal((V, K)).astype(np.float32)
    tokens = np.zeros(L, np.int32)
    tokens[:3] = [11, 22, 33]
    dtok, dpos = dev(hip, tokens), dev(hip, np.array([1], np.int32))
    dplen = dev(hip, np.array([3], np.int32))
    work = hip.DeviceBuffer(hip.lib().qlm_lm_head_greedy_workspace_bytes())
    dq4, ds, _ = _q4(hip, w)
    q4z, s4z = _mx4_layout(hip, dq4, ds, V, K, 1)
    dnw, dtab = dev(hip, nw), dev(hip, table)
    dlg, dh = hip.DeviceBuffer(V * 4), hip.DeviceBuffer(K * 4)
    pp = 1
    for step in range(3):
        x = (rng.standard_normal((1, K)) * 2).astype(np.float32)
        lg_ref = orc.matmul_i4(orc.rms_norm(x, nw, 1e-6), p, s)[0]
        say("lm_head_greedy_mx4 step", step)
        hip.call("qlm_lm_head_greedy_mx4", dev(hip, x), dnw, 1e-6, q4z, s4z, dlg, V, K, work,
                 dtok, L, dpos, dplen, dtab, K, dh, None)
        lg = dlg.to_numpy(V, np.float32)
        assert rel_err(lg, lg_ref) < 1e-5
        want = int(np.argmax(lg))
        t = dtok.to_numpy(L, np.int32)
        if pp + 1 >= 3:
            assert t[pp + 1] == want, step
            tokens[pp + 1] = want
        assert np.array_equal(t, tokens)
        pp += 1
        assert int(dpos.to_numpy(1, np.int32)[0]) == pp
        assert np.array_equal(dh.to_numpy(K, np.float32), table[tokens[pp]])
