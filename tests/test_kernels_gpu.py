"""Operator parity: each HIP kernel (through the C ABI) against the CPU oracle.

Bars: int8 quantisation and argmax bit-exact; fp32-accumulating
ops within a normwise relative error of 1e-3 (FP32_TOL). Where the GPU
evaluates exactly the reference's per-element arithmetic (conv1d tap sums,
RoPE from the reference's own cos/sin table), the bar is bit-exactness.
"""

import ctypes as C

import numpy as np
import pytest

from tests.util import FP32_TOL, bf16_bits, bf16_to_f32, rel_err, say

pytestmark = pytest.mark.gpu


def dev(hip, a):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


# ---------------------------------------------------------------- A2 quantiser
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("group", [32, "K"])
def test_quantize_bitexact(hip, orc, rng, dtype, group):
    rows, K = 97, 2560
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    w[3] = 0.0                                   # all-zero row -> scale 1, q 0
    w[5, :32] = np.arange(32, dtype=np.float32) - 16.0   # exact halves after scaling
    w[7, 5] = 1e30                               # one huge value dominates its group
    g = K if group == "K" else 32
    src = bf16_bits(w) if dtype == "bf16" else w
    q_ref, s_ref = orc.quantize(src, g)
    say("quantize", dtype, g, rows, K)
    dw = dev(hip, src)
    dq = hip.DeviceBuffer(rows * K)
    ds = hip.DeviceBuffer(s_ref.nbytes)
    fn = "qlm_quantize_q8_bf16" if dtype == "bf16" else "qlm_quantize_q8_f32"
    hip.call(fn, dw, rows, K, g, dq, ds, None)
    q = dq.to_numpy((rows, K), np.int8)
    s = ds.to_numpy(s_ref.shape, np.float32)
    assert np.array_equal(s.view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q, q_ref)


def test_quantize_rejects_bad_group(hip):
    d = hip.DeviceBuffer(64 * 4)
    with pytest.raises(hip.HipError):
        hip.call("qlm_quantize_q8_f32", d, 1, 64, 16, d, d, None)


# ---------------------------------------------------------------- A3 GEMV
def _weights(orc, rng, N, K, group):
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    return orc.quantize(w, group)


GEMV_SHAPES = [  # (N, K): model projections and the config-1 matrices
    (4096, 4096), (12288, 4096), (4096, 12288), (151936, 2560),
    (8224, 2560), (2560, 2048), (16, 2560), (77, 1024), (3, 3584),
]


@pytest.mark.parametrize("N,K", GEMV_SHAPES)
@pytest.mark.parametrize("group", [32, "K"])
def test_gemv_parity(hip, orc, rng, N, K, group):
    g = K if group == "K" else 32
    q, s = _weights(orc, rng, N, K, g)
    dq, ds = dev(hip, q), dev(hip, s)
    for M in (1, 4):
        x = rng.standard_normal((M, K)).astype(np.float32)
        ref = orc.matmul_i8(x, q, s, g)
        say("gemv", N, K, g, M)
        dx = dev(hip, x)
        dy = hip.DeviceBuffer(M * N * 4)
        hip.call("qlm_gemv_i8", dx, K, dq, ds, g, dy, N, M, N, K, None)
        y = dy.to_numpy((M, N), np.float32)
        err = rel_err(y, ref)
        assert err <= FP32_TOL, err
        assert err < 1e-5, err  # fp32 accumulation: far inside the bar


@pytest.mark.parametrize("N,K", [(2560, 9728), (1000, 2560), (77, 1024)])
def test_gemv_launch_shapes(hip, orc, rng, N, K):
    """Every lanes-per-row / rows / grid combination of the M = 1 kernel gives
    the oracle's result (grid-stride loop, ragged last block, idle slots)."""
    for g in (32, K):
        q, s = _weights(orc, rng, N, K, g)
        x = rng.standard_normal((1, K)).astype(np.float32)
        ref = orc.matmul_i8(x, q, s, g)
        dq, ds, dx = dev(hip, q), dev(hip, s), dev(hip, x)
        dy = hip.DeviceBuffer(N * 4)
        for lpr in (16, 32, 64, 128, 256):
            if (K // 16 + lpr - 1) // lpr > 6:
                continue
            for rows in (1, 2):
                for grid in (1, 7, 300):
                    dy.zero()
                    hip.call("qlm_gemv_i8_config", dx, None, 0.0, dq, ds, g, dy, N, K, 0, lpr,
                             rows, grid, None)
                    err = rel_err(dy.to_numpy((1, N), np.float32), ref)
                    assert err < 1e-5, (g, lpr, rows, grid, err)


@pytest.mark.parametrize("epi", ["norm", "resid", "swiglu"])
def test_gemv_config_fused(hip, orc, rng, epi):
    """The fused M = 1 forms under explicit launch shapes (ragged last block,
    grids smaller and larger than the row-block count)."""
    N, K, g, eps = 1000, 1536, 32, 1e-6
    rows_w = 2 * N if epi == "swiglu" else N
    q, s = _weights(orc, rng, rows_w, K, g)
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    y0 = rng.standard_normal((1, N)).astype(np.float32)
    if epi == "resid":
        ref = y0 + orc.matmul_i8(x, q, s, g)
    else:
        lg = orc.matmul_i8(orc.rms_norm(x, nw, eps), q, s, g)
        ref = lg if epi == "norm" else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dq, ds, dx, dnw = dev(hip, q), dev(hip, s), dev(hip, x), dev(hip, nw)
    dy = hip.DeviceBuffer(N * 4)
    code = {"norm": 0, "resid": 1, "swiglu": 2}[epi]
    for lpr in (32, 64, 128):
        for rows in (1, 2):
            for grid in (3, 250):
                dy.upload(y0)
                hip.call("qlm_gemv_i8_config", dx, None if epi == "resid" else dnw, eps, dq, ds,
                         g, dy, N, K, code, lpr, rows, grid, None)
                err = rel_err(dy.to_numpy((1, N), np.float32), ref)
                assert err < 1e-5, (epi, lpr, rows, grid, err)


MX_CASES = [  # (N, K, waves, ring, grid): ragged last tile, several tiles per workgroup
    (1000, 2560, 4, 10, None), (1000, 2560, 8, 5, 7), (300, 2048, 16, 2, None),
    (517, 4096, 8, 8, 3), (160, 9728, 16, 10, None), (37, 12288, 16, 12, 1),
    (2000, 2048, 4, 8, 5), (77, 2048, 8, 4, None), (300, 256, 4, 1, None), (129, 512, 4, 2, 4),
    (700, 1024, 4, 4, None),
]


def _mx_layout(hip, q, s, g, rows, K, halves):
    """Weights and scales on the device in the tile-major layout."""
    dq, ds = dev(hip, q), dev(hip, s)
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx_layout_bytes(rows, K, g, halves, C.byref(qb), C.byref(sb)))
    qz = hip.DeviceBuffer(qb.value)
    sz = hip.DeviceBuffer(max(sb.value, 16))
    hip.call("qlm_mx_swizzle", dq, ds, g, rows, K, halves, qz, sz if sb.value else None, None)
    return qz, (sz if sb.value else ds), (dq, ds, qz, sz)


def test_mx_swizzle_layout(hip, orc, rng):
    """Tile-major layout: fragment (tile, block) holds, in lane order l = 16q
    + n, bytes 64b + 16q .. +15 of row 16t + n of its half; rows past the
    half are zero; scales follow as [h][n] = s[row n, group 2b + h]."""
    rows, K, halves = 37, 192, 2
    q, s = _weights(orc, rng, halves * rows, K, 32)
    dq, ds, keep = _mx_layout(hip, q, s, 32, rows, K, halves)
    tiles, nblk = (rows + 15) // 16, K // 64
    qz = dq.to_numpy((halves * tiles, nblk, 64, 16), np.int8)
    sz = ds.to_numpy((halves * tiles, nblk, 2, 16), np.float32)
    for g in range(halves * tiles):
        half, t = divmod(g, tiles)
        for b in range(nblk):
            for lane in range(64):
                n, qd = lane & 15, lane >> 4
                r = t * 16 + n
                want = q[half * rows + r, 64 * b + 16 * qd:64 * b + 16 * qd + 16] if r < rows \
                    else np.zeros(16, np.int8)
                assert np.array_equal(qz[g, b, lane], want), (g, b, lane)
            for h in range(2):
                for n in range(16):
                    r = t * 16 + n
                    want = s[half * rows + r, 2 * b + h] if r < rows else 0.0
                    assert sz[g, b, h, n] == want


@pytest.mark.parametrize("epi", ["store", "norm", "resid", "swiglu"])
@pytest.mark.parametrize("group", [32, "K"])
def test_gemv_mx(hip, orc, rng, epi, group):
    """The matrix-core M = 1 GEMV (int8 digits of x on v_mfma_i32_16x16x64_i8,
    tile-major weights) under every instantiated launch pair: within 1e-5
    normwise of the fp32 oracle (the fp32 GEMV's own bar), fused prologue and
    epilogues included."""
    eps = 1e-6
    code = {"store": 0, "norm": 0, "resid": 1, "swiglu": 2}[epi]
    for N, K, waves, ring, grid in MX_CASES:
        g = K if group == "K" else 32
        rows_w = 2 * N if epi == "swiglu" else N
        q, s = _weights(orc, rng, rows_w, K, g)
        x = rng.standard_normal((1, K)).astype(np.float32)
        nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
        y0 = rng.standard_normal((1, N)).astype(np.float32)
        if epi == "store":
            ref = orc.matmul_i8(x, q, s, g)
        elif epi == "resid":
            ref = y0 + orc.matmul_i8(x, q, s, g)
        else:
            lg = orc.matmul_i8(orc.rms_norm(x, nw, eps), q, s, g)
            ref = lg if epi == "norm" else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
        dy = dev(hip, y0)
        tiles = (N + 15) // 16
        say("gemv_mx", epi, g, N, K, waves, ring, grid)
        dq, ds, keep = _mx_layout(hip, q, s, g, N, K, 2 if epi == "swiglu" else 1)
        hip.call("qlm_gemv_i8_mx_config", dev(hip, x),
                 dev(hip, nw) if epi in ("norm", "swiglu") else None, eps, dq, ds, g, dy, N, K,
                 code, waves, ring, grid or tiles, None)
        err = rel_err(dy.to_numpy((1, N), np.float32), ref)
        assert err < 1e-5, (epi, g, N, K, waves, ring, grid, err)


@pytest.mark.parametrize("N,K,epi", [(9728, 2560, "swiglu"), (2560, 9728, "resid"),
                                     (8224, 2560, "norm"), (2560, 2048, "resid"),
                                     (3584, 1024, "swiglu"), (1024, 3584, "resid"),
                                     (300, 4160, "norm")])
def test_gemv_mx_auto(hip, orc, rng, N, K, epi):
    """qlm_gemv_i8_mx picks its launch shape (tuned table for the 4B decode
    projections, rule elsewhere) and matches the oracle; a K no instantiated
    shape fits (4160 = 65 blocks) is refused with QLM_ERR_SHAPE."""
    g, eps = 32, 1e-6
    code = {"norm": 0, "resid": 1, "swiglu": 2}[epi]
    rows_w = 2 * N if epi == "swiglu" else N
    q, s = _weights(orc, rng, rows_w, K, g)
    x = rng.standard_normal((1, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    y0 = rng.standard_normal((1, N)).astype(np.float32)
    if epi == "resid":
        ref = y0 + orc.matmul_i8(x, q, s, g)
    else:
        lg = orc.matmul_i8(orc.rms_norm(x, nw, eps), q, s, g)
        ref = lg if epi == "norm" else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dq, ds, keep = _mx_layout(hip, q, s, g, N, K, 2 if epi == "swiglu" else 1)
    dy, dx, dnw = dev(hip, y0), dev(hip, x), dev(hip, nw)
    rc = hip.lib().qlm_gemv_i8_mx(dx.ptr, None if epi == "resid" else dnw.ptr, C.c_float(eps),
                                  dq.ptr, ds.ptr, g, dy.ptr, N, K, code, None)
    if K == 4160:
        assert rc == -2
        return
    hip.check(rc)
    assert rel_err(dy.to_numpy((1, N), np.float32), ref) < 1e-5


def test_gemv_mx_dynamic_range(hip, orc, rng):
    """Activations spanning 1e-6 .. 1e3 (one power-of-two scale for all
    digits), a zero activation (exact zeros out) and a one-hot activation."""
    N, K = 500, 2560
    q, s = _weights(orc, rng, N, K, 32)
    dq, ds, keep = _mx_layout(hip, q, s, 32, N, K, 1)
    dy = hip.DeviceBuffer(N * 4)
    mags = 10.0 ** rng.uniform(-6, 3, K)
    cases = {"wide": (rng.standard_normal(K) * mags).astype(np.float32),
             "zero": np.zeros(K, np.float32),
             "onehot": np.eye(1, K, 1234, dtype=np.float32)[0] * 3.0}
    for name, xv in cases.items():
        x = xv[None, :]
        ref = orc.matmul_i8(x, q, s, 32)
        hip.call("qlm_gemv_i8_mx_config", dev(hip, x), None, 0.0, dq, ds, 32, dy, N, K, 0, 4,
                 10, 32, None)
        y = dy.to_numpy((1, N), np.float32)
        if name == "zero":
            assert not y.any()
        else:
            assert rel_err(y, ref) < 1e-5, name


def test_gemv_mx_rejects_bad_shapes(hip, orc, rng):
    """Launch pairs that are not instantiated or do not match K are refused
    before any launch."""
    q, s = _weights(orc, rng, 64, 4096, 32)
    x = dev(hip, rng.standard_normal((1, 4096)).astype(np.float32))
    dq, ds = dev(hip, q), dev(hip, s)
    dy = hip.DeviceBuffer(64 * 4)
    for waves, ring, K in ((4, 5, 2560), (16, 3, 2560), (4, 10, 2560 + 32), (4, 13, 3328)):
        assert hip.lib().qlm_gemv_i8_mx_config(x.ptr, None, 0.0, dq.ptr, ds.ptr, 32, dy.ptr,
                                               64, K, 0, waves, ring, 4, None) != 0


def test_gemv_exact_integers(hip, orc, rng):
    """Integer activations and power-of-two scales make every sum exact in
    fp32, so any accumulation order must agree bit for bit with the oracle."""
    N, K = 1000, 2048
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, (N, K // 32))).astype(np.float32)
    x = rng.integers(-16, 17, (3, K)).astype(np.float32)
    ref = orc.matmul_i8(x, q, s, 32)
    dy = hip.DeviceBuffer(3 * N * 4)
    hip.call("qlm_gemv_i8", dev(hip, x), K, dev(hip, q), dev(hip, s), 32, dy, N, 3, N, K, None)
    assert np.array_equal(dy.to_numpy((3, N), np.float32), ref)


# ------------------------------------------------------------ A4 matrix cores
MM_CASES = [  # (M, N, K): batched decode (M <= 64, K % 128 == 0) and prefill tiles
    (2, 300, 1024), (16, 1000, 2560), (16, 2560, 9728), (33, 517, 1024), (64, 160, 2048),
    (100, 300, 1056), (300, 1000, 1024), (127, 3584, 1024),
]


@pytest.mark.parametrize("M,N,K", MM_CASES)
@pytest.mark.parametrize("group", [32, "K"])
def test_matmul_mfma_parity(hip, orc, rng, M, N, K, group):
    """bf16 hi/lo split activations, exact int8 weights, fp32 group scaling:
    within 1e-5 normwise of the fp32 oracle (ragged M and N tiles)."""
    g = K if group == "K" else 32
    q, s = _weights(orc, rng, N, K, g)
    x = rng.standard_normal((M, K)).astype(np.float32)
    ref = orc.matmul_i8(x, q, s, g)
    ldy = N + 8
    dy = hip.DeviceBuffer(M * ldy * 4)
    say("matmul", M, N, K, g)
    _matmul(hip, dev(hip, x), K, None, 0.0, dev(hip, q), dev(hip, s), g, dy, ldy, M, N, K, 0)
    y = dy.to_numpy((M, ldy), np.float32)[:, :N]
    assert rel_err(y, ref) < 1e-5


def _matmul(hip, x, ldx, nw, eps, q, s, g, y, ldy, M, N, K, epi):
    nbytes = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, epi)
    work = hip.DeviceBuffer(nbytes)
    work.upload(np.full(nbytes, 0xA5, np.uint8))  # no initial contents are required
    hip.call("qlm_matmul_i8", x, ldx, nw, eps, q, s, g, y, ldy, M, N, K, epi, work, nbytes, None)


@pytest.mark.parametrize("M,K", [(16, 2560), (7, 9728), (200, 1024)])
@pytest.mark.parametrize("epi", ["store_norm", "resid", "swiglu_norm"])
def test_matmul_mfma_epilogues(hip, orc, rng, M, K, epi):
    """Residual add, SwiGLU and the fused RMSNorm prologue, on the K-split
    path (M <= 64) and the prefill tiles."""
    N, eps = 700, 1e-6
    rows_w = 2 * N if epi.startswith("swiglu") else N
    q, s = _weights(orc, rng, rows_w, K, 32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    xin = orc.rms_norm(x, nw, eps) if epi.endswith("norm") else x
    lg = orc.matmul_i8(xin, q, s, 32)
    if epi == "resid":
        ref = y0 + lg
    elif epi == "store_norm":
        ref = lg
    else:
        ref = orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dy = dev(hip, y0)
    say("matmul", epi, M, K)
    code = {"store_norm": 0, "resid": 1, "swiglu_norm": 2}[epi]
    _matmul(hip, dev(hip, x), K, dev(hip, nw) if epi.endswith("norm") else None, eps,
            dev(hip, q), dev(hip, s), 32, dy, N, M, N, K, code)
    assert rel_err(dy.to_numpy((M, N), np.float32), ref) < 1e-5


MMX_CASES = [  # (M, N, K): batched decode rows over every K range the tile-major form serves
    (2, 300, 1024), (3, 517, 2560), (5, 1000, 2048), (8, 160, 9728), (16, 2560, 9728),
    (16, 1000, 2560), (16, 77, 3584), (7, 300, 512), (12, 130, 2560),
]


@pytest.mark.parametrize("M,N,K", MMX_CASES)
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid", "swiglu_norm"])
@pytest.mark.parametrize("group", [32, "K"])
def test_matmul_mx(hip, orc, rng, M, N, K, epi, group):
    """Batched decode on the int8 matrix cores over tile-major weights
    (per-row digits, one MFMA per row pair, K inside the workgroup): within
    1e-5 normwise of the fp32 oracle, strided output rows, every epilogue."""
    g, eps = (K if group == "K" else 32), 1e-6
    rows_w = 2 * N if epi.startswith("swiglu") else N
    q, s = _weights(orc, rng, rows_w, K, g)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    ldy = N + 5
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    xin = orc.rms_norm(x, nw, eps) if epi.endswith("norm") else x
    lg = orc.matmul_i8(xin, q, s, g)
    if epi == "resid":
        ref = y0[:, :N] + lg
    elif epi.startswith("store"):
        ref = lg
    else:
        ref = orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dq, ds, keep = _mx_layout(hip, q, s, g, N, K, 2 if epi.startswith("swiglu") else 1)
    nwork = hip.lib().qlm_matmul_i8_mx_workspace_bytes(M, K)
    work = hip.DeviceBuffer(nwork)
    work.upload(np.full(nwork, 0x5A, np.uint8))  # no initial contents are required
    dy = dev(hip, y0)
    code = {"store": 0, "store_norm": 0, "resid": 1, "swiglu_norm": 2}[epi]
    say("matmul_mx", epi, g, M, N, K)
    hip.call("qlm_matmul_i8_mx", dev(hip, x), K, dev(hip, nw) if epi.endswith("norm") else None,
             eps, dq, ds, g, dy, ldy, M, N, K, code, work, nwork, None)
    y = dy.to_numpy((M, ldy), np.float32)
    assert rel_err(y[:, :N], ref) < 1e-5
    assert np.array_equal(y[:, N:], y0[:, N:])  # the stride gap is untouched


def test_matmul_mx_refuses(hip, orc, rng):
    """M > 16 and K outside the served ranges return QLM_ERR_SHAPE before
    any launch."""
    lib = hip.lib()
    q, s = _weights(orc, rng, 64, 4096, 32)
    dq, ds = dev(hip, q), dev(hip, s)
    x = dev(hip, rng.standard_normal((17, 4096)).astype(np.float32))
    y = hip.DeviceBuffer(17 * 64 * 4)
    work = hip.DeviceBuffer(1 << 20)
    for M, K in ((17, 2560), (4, 6144), (4, 8192), (4, 2560 + 32)):
        assert lib.qlm_matmul_i8_mx(x.ptr, K, None, C.c_float(0.0), dq.ptr, ds.ptr, 32, y.ptr, 64,
                                    M, 64, K, 0, work.ptr, C.c_size_t(1 << 20), None) != 0


@pytest.mark.parametrize("M", [16, 130])
def test_matmul_mfma_exact_integers(hip, orc, rng, M):
    """Small-integer activations are exact in bf16 (lo = 0) and every
    product and sum is exact, so the matrix-core path is bit-identical."""
    N, K = 500, 2048
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, (N, K // 32))).astype(np.float32)
    x = rng.integers(-16, 17, (M, K)).astype(np.float32)
    ref = orc.matmul_i8(x, q, s, 32)
    dy = hip.DeviceBuffer(M * N * 4)
    _matmul(hip, dev(hip, x), K, None, 0.0, dev(hip, q), dev(hip, s), 32, dy, N, M, N, K, 0)
    assert np.array_equal(dy.to_numpy((M, N), np.float32), ref)


def test_gemv_batched_m(hip, orc, rng):
    """M > 4 runs in slices of four activation rows; strided output rows."""
    N, K, M = 300, 1024, 11
    q, s = _weights(orc, rng, N, K, 32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    ref = orc.matmul_i8(x, q, s, 32)
    ldy = N + 20
    dy = hip.DeviceBuffer(M * ldy * 4)
    hip.call("qlm_gemv_i8", dev(hip, x), K, dev(hip, q), dev(hip, s), 32, dy, ldy, M, N, K, None)
    y = dy.to_numpy((M, ldy), np.float32)[:, :N]
    assert rel_err(y, ref) < 1e-5


@pytest.mark.parametrize("M", [1, 3])
def test_gemv_rmsnorm_prologue(hip, orc, rng, M):
    N, K, eps = 8224, 2560, 1e-6
    q, s = _weights(orc, rng, N, K, 32)
    x = (rng.standard_normal((M, K)) * 3).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    ref = orc.matmul_i8(orc.rms_norm(x, nw, eps), q, s, 32)
    dy = hip.DeviceBuffer(M * N * 4)
    hip.call("qlm_gemv_i8_rmsnorm", dev(hip, x), K, dev(hip, nw), eps, dev(hip, q), dev(hip, s),
             32, dy, N, M, N, K, None)
    assert rel_err(dy.to_numpy((M, N), np.float32), ref) < 1e-5


def test_gemv_residual_epilogue(hip, orc, rng):
    N, K = 2560, 9728
    q, s = _weights(orc, rng, N, K, 32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    h = rng.standard_normal((1, N)).astype(np.float32)
    ref = h + orc.matmul_i8(x, q, s, 32)
    dh = dev(hip, h)
    hip.call("qlm_gemv_i8_residual", dev(hip, x), K, dev(hip, q), dev(hip, s), 32, dh, N, 1, N, K,
             None)
    assert rel_err(dh.to_numpy((1, N), np.float32), ref) < 1e-5


@pytest.mark.parametrize("M", [1, 2])
def test_gemv_swiglu_epilogue(hip, orc, rng, M):
    F, K, eps = 3584, 1024, 1e-6
    qg, sg = _weights(orc, rng, F, K, 32)
    qu, su = _weights(orc, rng, F, K, 32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    xn = orc.rms_norm(x, nw, eps)
    g = orc.matmul_i8(xn, qg, sg, 32)
    u = orc.matmul_i8(xn, qu, su, 32)
    ref = np.stack([orc.silu_mul(g[m], u[m]) for m in range(M)])
    dq = dev(hip, np.concatenate([qg, qu]))
    ds = dev(hip, np.concatenate([sg, su]))
    dy = hip.DeviceBuffer(M * F * 4)
    hip.call("qlm_gemv_i8_swiglu_rmsnorm", dev(hip, x), K, dev(hip, nw), eps, dq, ds, 32, dy, F, M,
             F, K, None)
    assert rel_err(dy.to_numpy((M, F), np.float32), ref) < 1e-5


def test_gemv_rejects_bad_shapes(hip):
    d = hip.DeviceBuffer(4096)
    with pytest.raises(hip.HipError):  # K not a multiple of 16
        hip.call("qlm_gemv_i8", d, 40, d, d, 40, d, 4, 1, 4, 40, None)
    with pytest.raises(hip.HipError):  # G = 32 needs K % 32 == 0
        hip.call("qlm_gemv_i8", d, 48, d, d, 32, d, 4, 1, 4, 48, None)


# ---------------------------------------------------------------- A5-A7
def test_rms_norm_and_add(hip, orc, rng):
    rows, n, eps = 5, 2560, 1e-6
    x = rng.standard_normal((rows, n)).astype(np.float32)
    d = rng.standard_normal((rows, n)).astype(np.float32)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    dy = hip.DeviceBuffer(x.nbytes)
    hip.call("qlm_rms_norm", dev(hip, x), dev(hip, w), dy, rows, n, eps, None)
    assert rel_err(dy.to_numpy(x.shape, np.float32), orc.rms_norm(x, w, eps)) < 1e-6
    res_ref, y_ref = orc.add_rms_norm(x, d, w, eps)
    dr = dev(hip, x)
    hip.call("qlm_add_rms_norm", dr, dev(hip, d), dev(hip, w), dy, rows, n, eps, None)
    assert np.array_equal(dr.to_numpy(x.shape, np.float32), res_ref)
    assert rel_err(dy.to_numpy(x.shape, np.float32), y_ref) < 1e-6


def test_silu_mul(hip, orc, rng):
    a = (rng.standard_normal(9728) * 4).astype(np.float32)
    b = rng.standard_normal(9728).astype(np.float32)
    da = dev(hip, a)
    hip.call("qlm_silu_mul", da, dev(hip, b), a.size, None)
    assert rel_err(da.to_numpy(a.shape, np.float32), orc.silu_mul(a, b)) < 1e-6


@pytest.mark.parametrize("rot", [32, 128])
def test_rope_bitexact(hip, orc, rng, rot):
    theta, n_pos, heads, hd = 1e6, 2304, 6, 128
    cos_t, sin_t = orc.rope_table(theta, rot, n_pos)
    dc, dsn = dev(hip, cos_t), dev(hip, sin_t)
    t = rng.standard_normal((heads, hd)).astype(np.float32)
    for pos in (0, 1, 1000, n_pos - 1):
        ref = orc.rope_neox(t, pos, theta, rot)
        dt = dev(hip, t)
        hip.call("qlm_rope_neox", dt, heads, hd, rot, dc, dsn, dev(hip, np.array([pos], np.int32)),
                 None)
        assert np.array_equal(dt.to_numpy(t.shape, np.float32), ref), pos


def test_conv1d_bitexact(hip, orc, rng):
    C = 6144
    x = rng.standard_normal(C).astype(np.float32)
    st = rng.standard_normal((3, C)).astype(np.float32)
    wt = rng.standard_normal((4, C)).astype(np.float32)
    for oldest in range(3):
        out_ref, st_ref = orc.conv1d_tapmajor(x, st, oldest, wt)
        dst = dev(hip, st)
        do = hip.DeviceBuffer(C * 4)
        hip.call("qlm_conv1d_update", dev(hip, x), dst, oldest, dev(hip, wt), do, C, 4, None)
        assert np.array_equal(do.to_numpy(C, np.float32), out_ref)
        assert np.array_equal(dst.to_numpy((3, C), np.float32), st_ref)


# ---------------------------------------------------------------- A14 argmax
def test_argmax_first_max_wins(hip, orc, rng):
    B, V = 3, 151936
    lg = rng.standard_normal((B, V)).astype(np.float32)
    lg[0, 100] = 50.0
    lg[0, 90000] = 50.0           # tie: lowest index wins
    lg[1, V - 1] = 60.0           # last element
    lg[2, :] = -np.inf
    lg[2, 7] = 0.0
    work = hip.DeviceBuffer(hip.lib().qlm_argmax_workspace_bytes(B, V))
    di = hip.DeviceBuffer(B * 4)
    hip.call("qlm_argmax", dev(hip, lg), V, V, B, di, work, None)
    got = di.to_numpy(B, np.int32)
    assert list(got) == [orc.argmax(lg[b]) for b in range(B)] == [100, V - 1, 7]


def test_greedy_advance_and_embed(hip, rng):
    B, V, H, L = 2, 5000, 64, 16
    lg = rng.standard_normal((B, V)).astype(np.float32)
    tokens = np.zeros((B, L), np.int32)
    tokens[:, :4] = [[5, 6, 7, 8], [9, 10, 11, 12]]
    pos = np.array([3, 1], np.int32)          # seq 0 generating, seq 1 still in its prompt
    plen = np.array([4, 4], np.int32)
    dt, dp = dev(hip, tokens), dev(hip, pos)
    work = hip.DeviceBuffer(hip.lib().qlm_argmax_workspace_bytes(B, V))
    hip.call("qlm_greedy_advance", dev(hip, lg), V, V, B, work, dt, L, dp, dev(hip, plen), None)
    t2 = dt.to_numpy((B, L), np.int32)
    assert t2[0, 4] == int(np.argmax(lg[0])) and t2[1, 2] == 11
    assert list(dp.to_numpy(B, np.int32)) == [4, 2]
    table = rng.standard_normal((V, H)).astype(np.float32)
    out = hip.DeviceBuffer(B * H * 4)
    hip.call("qlm_embed_tokens", dev(hip, table), V, H, dt, L, dp, out, H, B, None)
    e = out.to_numpy((B, H), np.float32)
    assert np.array_equal(e[0], table[t2[0, 4]]) and np.array_equal(e[1], table[11])


@pytest.mark.parametrize("group", [32, "K"])
@pytest.mark.parametrize("tiles", [False, True])
def test_lm_head_greedy_fused(hip, orc, rng, group, tiles):
    """Final norm + lm_head + argmax + advance + next embedding (two launches),
    three calls in a row (prompt position, then two generated tokens); with
    row-major weights and, on the matrix cores, tile-major ones."""
    V, K, L = 151936, 1024, 16
    g = K if group == "K" else 32
    q, s = _weights(orc, rng, V, K, g)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    table = rng.standard_normal((V, K)).astype(np.float32)
    tokens = np.zeros(L, np.int32)
    tokens[:3] = [11, 22, 33]
    dtok, dpos = dev(hip, tokens), dev(hip, np.array([1], np.int32))
    dplen = dev(hip, np.array([3], np.int32))
    nwork = hip.lib().qlm_lm_head_greedy_workspace_bytes()
    work = hip.DeviceBuffer(nwork)
    work.upload(np.full(nwork, 0xA5, np.uint8))  # no initial contents are required
    if tiles:
        dq, ds, keep = _mx_layout(hip, q, s, g, V, K, 1)
    else:
        dq, ds = dev(hip, q), dev(hip, s)
    dnw, dtab = dev(hip, nw), dev(hip, table)
    dlg, dh = hip.DeviceBuffer(V * 4), hip.DeviceBuffer(K * 4)
    p = 1
    for step in range(3):
        x = (rng.standard_normal((1, K)) * 2).astype(np.float32)
        lg_ref = orc.matmul_i8(orc.rms_norm(x, nw, 1e-6), q, s, g)[0]
        hip.call("qlm_lm_head_greedy_mx" if tiles else "qlm_lm_head_greedy", dev(hip, x), dnw,
                 1e-6, dq, ds, g, dlg, V, K, work, dtok, L, dpos, dplen, dtab, K, dh, None)
        lg = dlg.to_numpy(V, np.float32)
        assert rel_err(lg, lg_ref) < 1e-5
        want = int(np.argmax(lg))  # first maximum of the GPU's own logits
        t = dtok.to_numpy(L, np.int32)
        if p + 1 >= 3:
            assert t[p + 1] == want, step
            tokens[p + 1] = want
        assert np.array_equal(t, tokens)
        p += 1
        assert int(dpos.to_numpy(1, np.int32)[0]) == p
        assert np.array_equal(dh.to_numpy(K, np.float32), table[tokens[p]])


# ---------------------------------------------------------------- A12 DeltaNet
def _l2n(x):
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("B,H", [(1, 32), (4, 32), (8, 32), (3, 5)])
def test_gated_delta_step(hip, orc, rng, B, H):
    """The isolated step over 3 steps: column-split workgroups at B <= 4, one
    workgroup a head above."""
    d = 128
    S = (rng.standard_normal((B, H, d, d)) * 0.01).astype(np.float32)
    dS = dev(hip, S)
    Sref = S.copy()
    for step in range(3):
        q = _l2n(rng.standard_normal((B, H, d)))
        k = _l2n(rng.standard_normal((B, H, d)))
        v = rng.standard_normal((B, H, d)).astype(np.float32)
        a = (1 / (1 + np.exp(-(rng.standard_normal((B, H)) + 2)))).astype(np.float32)
        b = (1 / (1 + np.exp(-rng.standard_normal((B, H))))).astype(np.float32)
        o_ref, Sref = orc.gated_delta_step(q, k, v, a, b, Sref)
        do = hip.DeviceBuffer(q.nbytes)
        say("delta", B, H, step)
        hip.call("qlm_gated_delta_step", dev(hip, q), dev(hip, k), dev(hip, v), dev(hip, a),
                 dev(hip, b), dS, do, B, H, d, None)
        assert rel_err(do.to_numpy(q.shape, np.float32), o_ref) < 1e-5
        assert rel_err(dS.to_numpy(S.shape, np.float32), Sref) < 1e-5


def test_deltanet_decode_fused(hip, orc, rng):
    """Fused mixer core over 5 steps (ring index pos % 3) for 2 sequences."""
    B, H, d = 2, 16, 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    conv = np.zeros((B, 3, 3 * HD), np.float32)
    S = (rng.standard_normal((B, H, d, d)) * 0.01).astype(np.float32)
    dconv, dS = dev(hip, conv), dev(hip, S)
    conv_ref = [conv[b].copy() for b in range(B)]
    S_ref = [S[b].copy() for b in range(B)]
    dwt, dA, ddt, dnw = dev(hip, wt), dev(hip, A_log), dev(hip, dtb), dev(hip, nw)
    for step in range(5):
        proj = (rng.standard_normal((B, ldp)) * 0.6).astype(np.float32)
        pos = np.array([step, step + 7], np.int32)
        ref = np.stack([orc.deltanet_core(proj[b], conv_ref[b], int(pos[b] % 3), wt, A_log, dtb,
                                          nw, S_ref[b], H, d) for b in range(B)])
        do = hip.DeviceBuffer(B * HD * 4)
        say("deltanet_decode", step)
        hip.call("qlm_deltanet_decode", dev(hip, proj), ldp, dconv, dwt, dA, ddt, dnw, dS,
                 dev(hip, pos), do, HD, B, H, d, None)
        assert rel_err(do.to_numpy((B, HD), np.float32), ref) < 1e-4
        assert np.array_equal(dconv.to_numpy(conv.shape, np.float32), np.stack(conv_ref))
        assert rel_err(dS.to_numpy(S.shape, np.float32), np.stack(S_ref)) < 1e-5


@pytest.mark.parametrize("p0,T", [(0, 64), (5, 130)])
def test_deltanet_prefill(hip, orc, rng, p0, T):
    """Prefill over T rows == the oracle's row-by-row recurrence, and
    bit-identical to T single decode steps (outputs, conv ring, state)."""
    H, d = 16, 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((3, 3 * HD)) * (0.5 if p0 else 0.0)).astype(np.float32)
    S = (rng.standard_normal((H, d, d)) * (0.01 if p0 else 0.0)).astype(np.float32)
    proj = (rng.standard_normal((T, ldp)) * 0.6).astype(np.float32)
    conv_ref, S_ref = conv.copy(), S.copy()
    ref = np.stack([orc.deltanet_core(proj[t], conv_ref, (p0 + t) % 3, wt, A_log, dtb, nw, S_ref,
                                      H, d) for t in range(T)])
    dwt, dA, ddt, dnw = dev(hip, wt), dev(hip, A_log), dev(hip, dtb), dev(hip, nw)
    dconv, dS, dproj = dev(hip, conv), dev(hip, S), dev(hip, proj)
    do = hip.DeviceBuffer(T * HD * 4)
    say("deltanet_prefill", p0, T)
    hip.call("qlm_deltanet_prefill", dproj, ldp, T, dconv, dwt, dA, ddt, dnw, dS, p0, do, HD, H, d,
             None)
    out = do.to_numpy((T, HD), np.float32)
    assert rel_err(out, ref) < 1e-4
    assert np.array_equal(dconv.to_numpy(conv.shape, np.float32), conv_ref)
    assert rel_err(dS.to_numpy(S.shape, np.float32), S_ref) < 1e-4
    # the same rows through the decode kernel, one step at a time
    dconv2, dS2 = dev(hip, conv), dev(hip, S)
    do2 = hip.DeviceBuffer(HD * 4)
    steps = []
    for t in range(T):
        hip.call("qlm_deltanet_decode", dev(hip, proj[t:t + 1]), ldp, dconv2, dwt, dA, ddt, dnw,
                 dS2, dev(hip, np.array([p0 + t], np.int32)), do2, HD, 1, H, d, None)
        steps.append(do2.to_numpy(HD, np.float32))
    assert np.array_equal(out, np.stack(steps))
    assert np.array_equal(dS.to_numpy(S.shape, np.float32), dS2.to_numpy(S.shape, np.float32))
    assert np.array_equal(dconv.to_numpy(conv.shape, np.float32),
                          dconv2.to_numpy(conv.shape, np.float32))


@pytest.mark.parametrize("p0,T", [(0, 64), (0, 200), (5, 130), (1, 2), (3, 65), (2, 1),
                                  (0, 1024), (0, 4096), (9, 3001)])
def test_deltanet_prefill_chunked(hip, orc, rng, p0, T):
    """Chunked (WY, matrix-core) prefill == the row-by-row recurrence: outputs
    against the oracle, state and conv ring against the sequential kernel
    (ragged last chunk, a last chunk of one row, continuation from p0 > 0,
    T < 3, one row)."""
    H, d = 16, 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((3, 3 * HD)) * (0.5 if p0 else 0.0)).astype(np.float32)
    S = (rng.standard_normal((H, d, d)) * (0.01 if p0 else 0.0)).astype(np.float32)
    proj = (rng.standard_normal((T, ldp)) * 0.6).astype(np.float32)
    dwt, dA, ddt, dnw, dproj = (dev(hip, a) for a in (wt, A_log, dtb, nw, proj))
    # sequential kernel (bit-identical to decode steps) as the state reference
    dconv1, dS1, do1 = dev(hip, conv), dev(hip, S), hip.DeviceBuffer(T * HD * 4)
    hip.call("qlm_deltanet_prefill", dproj, ldp, T, dconv1, dwt, dA, ddt, dnw, dS1, p0, do1, HD,
             H, d, None)
    nbytes = hip.lib().qlm_deltanet_chunk_workspace_bytes(T, H, d)
    work = hip.DeviceBuffer(nbytes)
    dconv2, dS2, do2 = dev(hip, conv), dev(hip, S), hip.DeviceBuffer(T * HD * 4)
    say("deltanet_prefill_chunked", p0, T)
    hip.call("qlm_deltanet_prefill_chunked", dproj, ldp, T, dconv2, dwt, dA, ddt, dnw, dS2, p0,
             do2, HD, H, d, work, nbytes, None)
    out_seq = do1.to_numpy((T, HD), np.float32)
    out = do2.to_numpy((T, HD), np.float32)
    assert rel_err(out, out_seq) < 1e-4
    assert rel_err(dS2.to_numpy(S.shape, np.float32), dS1.to_numpy(S.shape, np.float32)) < 1e-4
    assert np.array_equal(dconv2.to_numpy(conv.shape, np.float32),
                          dconv1.to_numpy(conv.shape, np.float32))
    if T <= 200:  # and against the oracle's own recurrence
        conv_ref, S_ref = conv.copy(), S.copy()
        ref = np.stack([orc.deltanet_core(proj[t], conv_ref, (p0 + t) % 3, wt, A_log, dtb, nw,
                                          S_ref, H, d) for t in range(T)])
        assert rel_err(out, ref) < 1e-4


@pytest.mark.parametrize("n_q,n_kv,hd,rot,gated,p0,T", [(16, 4, 128, 32, 1, 0, 300),
                                                        (16, 4, 128, 32, 1, 37, 90),
                                                        (16, 2, 256, 64, 0, 10, 40),
                                                        (8, 2, 128, 64, 0, 0, 127),
                                                        (16, 16, 128, 32, 1, 5, 33),
                                                        (16, 8, 128, 128, 0, 250, 17),
                                                        (16, 2, 128, 32, 1, 100, 499)])
def test_gqa_prefill(hip, orc, rng, n_q, n_kv, hd, rot, gated, p0, T):
    """T prompt rows at positions p0.. == the oracle row by row: outputs and
    the cache rows they write. head_dim 128 runs the one-launch tiled form
    (1, 2, 4 and 8 query heads a kv head, ragged last tiles, passes after
    earlier ones); 256 the per-row chunks and their merge (two 256-row
    slices)."""
    max_seq, theta = 600, 1e6
    qs = (2 if gated else 1) * hd
    ld = n_q * qs + 2 * n_kv * hd
    qn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    cos_t, sin_t = orc.rope_table(theta, rot, max_seq)
    kc = np.zeros((max_seq, n_kv, hd), np.float32)
    vc = np.zeros_like(kc)
    kc[:p0] = rng.standard_normal((p0, n_kv, hd))
    vc[:p0] = rng.standard_normal((p0, n_kv, hd))
    dkc, dvc = dev(hip, kc), dev(hip, vc)
    qkv = rng.standard_normal((T, ld)).astype(np.float32)
    kref, vref = kc.copy(), vc.copy()
    ref = np.stack([orc.gqa_core(qkv[t].copy(), qn, kn, theta, rot, kref, vref, p0 + t, n_q, n_kv,
                                 hd, gated) for t in range(T)])
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_prefill_workspace_bytes(n_q, hd, max_seq))
    do = hip.DeviceBuffer(T * n_q * hd * 4)
    say("gqa_prefill", n_q, n_kv, hd, p0, T)
    hip.call("qlm_gqa_prefill", dev(hip, qkv), ld, dev(hip, qn), dev(hip, kn), dev(hip, cos_t),
             dev(hip, sin_t), rot, dkc, dvc, max_seq, p0, T, do, n_q * hd, n_q, n_kv, hd, gated,
             work, None)
    assert rel_err(do.to_numpy((T, n_q * hd), np.float32), ref) < 1e-5
    got_k = dkc.to_numpy(kc.shape, np.float32)
    assert rel_err(got_k[p0:p0 + T], kref[p0:p0 + T]) < 1e-6
    assert np.array_equal(got_k[:p0], kc[:p0])
    assert np.array_equal(dvc.to_numpy(vc.shape, np.float32)[:p0 + T], vref[:p0 + T])


# ---------------------------------------------------------------- A8/A9 GQA
@pytest.mark.parametrize("n_q,n_kv,hd,rot,gated,max_seq,start",
                         [(16, 4, 128, 32, 1, 600, (300, 511)),
                          (8, 2, 128, 128, 1, 600, (300, 511)),
                          (16, 2, 256, 64, 0, 600, (300, 511)),
                          # > 128 chunks of 64: the combine runs two tiles
                          (16, 4, 128, 32, 1, 9000, (8300, 8500))])
def test_gqa_decode_fused(hip, orc, rng, n_q, n_kv, hd, rot, gated, max_seq, start):
    B, theta = 2, 1e6
    qs = (2 if gated else 1) * hd
    ld = n_q * qs + 2 * n_kv * hd
    qn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    cos_t, sin_t = orc.rope_table(theta, rot, max_seq)
    kc = np.zeros((B, max_seq, n_kv, hd), np.float32)
    vc = np.zeros_like(kc)
    dkc, dvc = dev(hip, kc), dev(hip, vc)
    kref = [kc[b].copy() for b in range(B)]
    vref = [vc[b].copy() for b in range(B)]
    # fill a history so the split over chunks is exercised
    for b in range(B):
        kref[b][: start[b] + 40] = rng.standard_normal((start[b] + 40, n_kv, hd))
        vref[b][: start[b] + 40] = rng.standard_normal((start[b] + 40, n_kv, hd))
    dkc.upload(np.stack(kref))
    dvc.upload(np.stack(vref))
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
    dcos, dsin = dev(hip, cos_t), dev(hip, sin_t)
    for step in range(3):
        pos = np.array([start[0] + step, start[1] + step], np.int32)
        qkv = rng.standard_normal((B, ld)).astype(np.float32)
        ref = np.stack([orc.gqa_core(qkv[b].copy(), qn, kn, theta, rot, kref[b], vref[b],
                                     int(pos[b]), n_q, n_kv, hd, gated) for b in range(B)])
        do = hip.DeviceBuffer(B * n_q * hd * 4)
        say("gqa", n_q, n_kv, hd, step)
        hip.call("qlm_gqa_decode", dev(hip, qkv), ld, dev(hip, qn), dev(hip, kn), dcos, dsin, rot,
                 dkc, dvc, max_seq, dev(hip, pos), do, n_q * hd, B, n_q, n_kv, hd, gated, work,
                 None)
        assert rel_err(do.to_numpy((B, n_q * hd), np.float32), ref) < 1e-5
        got_k = dkc.to_numpy(kc.shape, np.float32)
        got_v = dvc.to_numpy(vc.shape, np.float32)
        for b in range(B):
            # K went through QK-norm (sum-of-squares order differs) and RoPE
            assert rel_err(got_k[b, pos[b]], kref[b][pos[b]]) < 1e-6
            assert np.array_equal(got_v[b, pos[b]], vref[b][pos[b]])


@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("ctx", [1, 257, 2048])
def test_attention_decode(hip, orc, rng, kv, ctx):
    B, n_q, n_kv, hd, max_seq = 2, 16, 2, 256, 2048
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    k = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    if kv == "bf16":
        kb, vb = bf16_bits(k), bf16_bits(v)
        k, v = bf16_to_f32(kb), bf16_to_f32(vb)
        dk, dv = dev(hip, kb), dev(hip, vb)
    else:
        dk, dv = dev(hip, k), dev(hip, v)
    ref = np.stack([orc.attention(q[b], k[b], v[b], ctx) for b in range(B)])
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
    work.zero()
    do = hip.DeviceBuffer(q.nbytes)
    hip.call("qlm_attention_decode", dev(hip, q), dk, dv, 0 if kv == "f32" else 1, max_seq, ctx,
             do, B, n_q, n_kv, hd, work, None)
    assert rel_err(do.to_numpy(q.shape, np.float32), ref) < 1e-5
    if ctx == 1:  # one position: the output is V[0] exactly up to rounding
        assert rel_err(do.to_numpy(q.shape, np.float32)[:, :n_q // n_kv],
                       np.broadcast_to(v[:, 0, :1], (B, n_q // n_kv, hd))) < 1e-6


@pytest.mark.parametrize("hd,n_q,n_kv", [(128, 8, 8), (128, 8, 4), (128, 16, 4), (256, 4, 2)])
@pytest.mark.parametrize("ctx", [1, 17, 1000, 3000])
def test_attention_decode_bf16_shapes(hip, orc, rng, hd, n_q, n_kv, ctx):
    """The bf16 matrix-core attention at every group size (1, 2, 4 query
    heads a kv head; 8 is the config-3 shape above), both head dims, and
    contexts that end inside a 16-position step and a chunk, over 3
    sequences of a cache longer than the context (max_seq 3072)."""
    B, max_seq = 3, 3072
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    kb = bf16_bits(rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32))
    vb = bf16_bits(rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32))
    k, v = bf16_to_f32(kb), bf16_to_f32(vb)
    ref = np.stack([orc.attention(q[b], k[b], v[b], ctx) for b in range(B)])
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
    do = hip.DeviceBuffer(q.nbytes)
    hip.call("qlm_attention_decode", dev(hip, q), dev(hip, kb), dev(hip, vb), 1, max_seq, ctx, do,
             B, n_q, n_kv, hd, work, None)
    # q and the probabilities enter the matrix cores as bf16 hi + lo (2^-18
    # of each value); the fp32 sums then differ from the oracle's order only
    assert rel_err(do.to_numpy(q.shape, np.float32), ref) < 1e-5


@pytest.mark.parametrize("B,H", [(1, 16), (2, 8)])
def test_deltanet_decode_cols(hip, orc, rng, B, H):
    """Column-split mixer over 5 steps (ring index pos % 3): u scaled by the
    head norm from the 8 partial sums equals the oracle's mixer output; the
    state and conv ring equal the oracle's; the tickets stay a multiple of 8."""
    d = 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((B, 3, 3 * HD)) * 0.5).astype(np.float32)
    S = (rng.standard_normal((B, H, d, d)) * 0.01).astype(np.float32)
    dconv, dS = dev(hip, conv), dev(hip, S)
    conv_ref = [conv[b].copy() for b in range(B)]
    S_ref = [S[b].copy() for b in range(B)]
    dwt, dA, ddt, dnw = dev(hip, wt), dev(hip, A_log), dev(hip, dtb), dev(hip, nw)
    stride = 32  # QLM_DN_TICKET_STRIDE
    ticket = hip.DeviceBuffer(B * H * stride * 4)
    ticket.zero()
    du, dss = hip.DeviceBuffer(B * HD * 4), hip.DeviceBuffer(B * H * 8 * 4)
    for step in range(5):
        proj = (rng.standard_normal((B, ldp)) * 0.6).astype(np.float32)
        pos = np.array([step + 11 * b for b in range(B)], np.int32)
        ref = np.stack([orc.deltanet_core(proj[b], conv_ref[b], int(pos[b] % 3), wt, A_log, dtb,
                                          nw, S_ref[b], H, d) for b in range(B)])
        say("deltanet_decode_cols", B, H, step)
        hip.call("qlm_deltanet_decode_cols", dev(hip, proj), ldp, dconv, dwt, dA, ddt, dnw, dS,
                 dev(hip, pos), du, HD, dss, ticket, B, H, d, None)
        u = du.to_numpy((B, H, d), np.float32).astype(np.float64)
        ss = dss.to_numpy((B, H, 8), np.float32).astype(np.float64).sum(axis=2)
        out = (u / np.sqrt(ss / d + 1e-6)[:, :, None]).reshape(B, HD)
        assert rel_err(out, ref) < 1e-4
        assert np.array_equal(dconv.to_numpy(conv.shape, np.float32), np.stack(conv_ref))
        assert rel_err(dS.to_numpy(S.shape, np.float32), np.stack(S_ref)) < 1e-5
        tk = ticket.to_numpy(B * H * stride, np.uint32).reshape(B * H, stride)
        assert np.all(tk[:, 0] == 8 * (step + 1)) and not tk[:, 1:].any()


@pytest.mark.parametrize("plan_kind", ["out", "out+gate_up", "few", "row", "int4"])
def test_deltanet_decode_cols_with_l2_plan(hip, rng, plan_kind):
    """The mixer carrying an L2 prefetch plan writes the same bits as without
    one: u, the partial sums, the state, the conv ring and the tickets, over
    3 steps of two copies of the inputs. Plans: the 4B out-projection's tiles
    (as the engine passes them), with the gate/up projection's first tiles,
    3 tiles only (XCDs 3-7 get none), per-row scales (weights only) and int4
    tiles (512-byte fragments)."""
    H, d = 16, 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    Hm, F = 2560, 9728
    cases = {"out": [(Hm, HD, 1, 1, 32, 0, 1 << 30)],
             "out+gate_up": [(Hm, HD, 1, 1, 32, 0, 1 << 30), (F, Hm, 2, 2, 32, 0, 1 << 30)],
             "few": [(Hm, HD, 1, 1, 32, 0, 3)],
             "row": [(Hm, HD, 1, 1, HD, 0, 1 << 30)],
             "int4": [(Hm, HD, 1, 1, 32, 1, 1 << 30)]}[plan_kind]
    plan = hip.L2Plan()
    keep = []
    for N, K, epi, halves, group, int4, max_tiles in cases:
        qb, sb = C.c_size_t(), C.c_size_t()
        if int4:
            hip.check(hip.lib().qlm_mx4_layout_bytes(N, K, halves, C.byref(qb), C.byref(sb)))
        else:
            hip.check(hip.lib().qlm_mx_layout_bytes(N, K, group, halves, C.byref(qb),
                                                    C.byref(sb)))
        qz, sz = hip.DeviceBuffer(qb.value), hip.DeviceBuffer(max(sb.value, 4 * N * halves))
        qz.zero()
        sz.zero()
        keep += [qz, sz]
        hip.call("qlm_gemv_mx_l2_plan", qz, sz, group, int4, N, K, epi, max_tiles,
                 C.byref(plan))
    assert plan.nseg == {"out": 2, "out+gate_up": 6, "few": 2, "row": 1, "int4": 2}[plan_kind]
    if plan_kind == "few":
        assert list(plan.tiles[:2]) == [3, 3]
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    conv = (rng.standard_normal((1, 3, 3 * HD)) * 0.5).astype(np.float32)
    S = (rng.standard_normal((1, H, d, d)) * 0.01).astype(np.float32)
    dwt, dA, ddt, dnw = dev(hip, wt), dev(hip, A_log), dev(hip, dtb), dev(hip, nw)
    runs = []
    for _ in range(2):
        tk = hip.DeviceBuffer(H * 32 * 4)
        tk.zero()
        runs.append(dict(conv=dev(hip, conv), S=dev(hip, S), u=hip.DeviceBuffer(HD * 4),
                         ss=hip.DeviceBuffer(H * 8 * 4), tk=tk))
    for step in range(3):
        proj = dev(hip, (rng.standard_normal((1, ldp)) * 0.6).astype(np.float32))
        pos = dev(hip, np.array([step + 5], np.int32))
        say("deltanet_decode_cols l2 plan", plan_kind, step)
        for r, pl in zip(runs, (None, C.byref(plan))):
            hip.call("qlm_deltanet_decode_cols_pf", proj, ldp, r["conv"], dwt, dA, ddt, dnw,
                     r["S"], pos, r["u"], HD, r["ss"], r["tk"], 1, H, d, pl, None)
        a, b = runs
        assert np.array_equal(a["u"].to_numpy(HD, np.float32), b["u"].to_numpy(HD, np.float32))
        assert np.array_equal(a["ss"].to_numpy(H * 8, np.float32),
                              b["ss"].to_numpy(H * 8, np.float32))
        assert np.array_equal(a["S"].to_numpy(S.size, np.float32),
                              b["S"].to_numpy(S.size, np.float32))
        assert np.array_equal(a["conv"].to_numpy(conv.size, np.float32),
                              b["conv"].to_numpy(conv.size, np.float32))
        assert np.array_equal(a["tk"].to_numpy(H * 32, np.uint32),
                              b["tk"].to_numpy(H * 32, np.uint32))


@pytest.mark.parametrize("group", [32, "K", "int4"])
def test_gemv_mx_headnorm(hip, orc, rng, group):
    """The out-projection over the column-split mixer's output: x = u scaled
    per 128-column head by 1/sqrt(sum of its 8 partials / 128 + eps), then
    y += W x (residual epilogue), against the oracle's matmul of x."""
    N, K, eps = 2560, 2048, 1e-6
    u = rng.standard_normal(K).astype(np.float32)
    ss = rng.uniform(0.5, 40.0, (K // 128, 8)).astype(np.float32)
    sn = (1.0 / np.sqrt(ss.astype(np.float64).sum(axis=1) / 128.0 + eps))
    x = (u.reshape(-1, 128) * sn[:, None]).reshape(1, K).astype(np.float32)
    res = rng.standard_normal(N).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    dy = dev(hip, res)
    say("gemv_mx_headnorm", group)
    if group == "int4":
        p4, s4 = orc.quantize_q4(w)
        ref = res + orc.matmul_i4(x, p4, s4)[0]
        qb, sb = C.c_size_t(), C.c_size_t()
        hip.check(hip.lib().qlm_mx4_layout_bytes(N, K, 1, C.byref(qb), C.byref(sb)))
        qz, sz = hip.DeviceBuffer(qb.value), hip.DeviceBuffer(sb.value)
        hip.call("qlm_mx4_swizzle", dev(hip, p4), dev(hip, s4), N, K, 1, qz, sz, None)
        hip.call("qlm_gemv_i4_mx_headnorm", dev(hip, u), dev(hip, ss), eps, qz, sz, dy, N, K, 1,
                 None)
    else:
        g = K if group == "K" else 32
        q, s = orc.quantize(w, g)
        ref = res + orc.matmul_i8(x, q, s, g)[0]
        qz, sz, keep = _mx_layout(hip, q, s, g, N, K, 1)
        hip.call("qlm_gemv_i8_mx_headnorm", dev(hip, u), dev(hip, ss), eps, qz, sz, g, dy, N, K,
                 1, None)
    assert rel_err(dy.to_numpy(N, np.float32), ref) < 1e-5


def test_gqa_decode_batches_share_workspace(hip, orc, rng):
    """Calls with 2, 1, 2 and 1 sequences on one workspace sized for 2: the
    records of each call are laid out for its own batch and merged by its own
    combine launch, whatever earlier calls left in the workspace."""
    n_q, n_kv, hd, rot, max_seq, theta = 16, 4, 128, 32, 700, 1e6
    ld = n_q * 2 * hd + 2 * n_kv * hd
    qn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    cos_t, sin_t = orc.rope_table(theta, rot, max_seq)
    kref = [rng.standard_normal((max_seq, n_kv, hd)).astype(np.float32) for _ in range(2)]
    vref = [rng.standard_normal((max_seq, n_kv, hd)).astype(np.float32) for _ in range(2)]
    dkc, dvc = dev(hip, np.stack(kref)), dev(hip, np.stack(vref))
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(2, n_q, hd, max_seq))
    work.zero()
    dcos, dsin = dev(hip, cos_t), dev(hip, sin_t)
    for step, B in enumerate((2, 1, 2, 1)):
        pos = np.array([300 + 70 * step, 600 - 50 * step][:B], np.int32)
        qkv = rng.standard_normal((B, ld)).astype(np.float32)
        ref = np.stack([orc.gqa_core(qkv[b].copy(), qn, kn, theta, rot, kref[b], vref[b],
                                     int(pos[b]), n_q, n_kv, hd, True) for b in range(B)])
        do = hip.DeviceBuffer(B * n_q * hd * 4)
        say("gqa shared workspace", step, B)
        hip.call("qlm_gqa_decode", dev(hip, qkv), ld, dev(hip, qn), dev(hip, kn), dcos, dsin, rot,
                 dkc, dvc, max_seq, dev(hip, pos), do, n_q * hd, B, n_q, n_kv, hd, 1, work, None)
        assert rel_err(do.to_numpy((B, n_q * hd), np.float32), ref) < 1e-5
