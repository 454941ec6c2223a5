"""Native (unquantised) weights on the GPU (reference --precision bf16).

qlm_matmul_w against the oracle's fp32 dot products over fp32 or bf16 rows
(orc_matmul_w, itself bit-exact with the reference's dot_avx2 /
dot_avx2_bf16, tests/test_oracle.py). The summation order differs (matrix
cores over 16-row tiles for several rows, per-lane fp32 sums and lane
reductions for one row), so the bar is fp32 rounding: 1e-5 normwise per
call.
"""

import numpy as np
import pytest

from tests.util import bf16_bits, rel_err, say

pytestmark = pytest.mark.gpu

EPI = {"store": 0, "norm": 0, "resid": 1, "swiglu": 2}
TOL = 1e-5      # fp32 products (vector ALUs; fp32 matrix cores)
TOL_HILO = 5e-5  # bf16 rows, M > 16: activation split into bf16 hi + lo (2^-17 of x)


def dev(hip, a):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def _ref(orc, epi, x, w, nw, y0, N, eps):
    if epi == "store":
        return orc.matmul_w(x, w)
    if epi == "resid":
        return y0 + orc.matmul_w(x, w)
    lg = orc.matmul_w(orc.rms_norm(x, nw, eps), w)
    return lg if epi == "norm" else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())


def _run(hip, epi, x, ldx, w, nw, y0, ldy, M, N, K, eps, with_work=False):
    """x [M, ldx] and y [M, ldy] padded rows; returns y's first N columns.
    The workspace goes with the RMSNorm (or always with with_work: bf16 rows
    with M > 16 then split the activation once)."""
    xp = np.zeros((M, ldx), np.float32)
    xp[:, :K] = x
    yp = np.full((M, ldy), 7.0, np.float32)
    yp[:, :N] = y0
    dx, dy, dw = dev(hip, xp), dev(hip, yp), dev(hip, w)
    dnw = dev(hip, nw) if epi in ("norm", "swiglu") else None
    wb = max(hip.lib().qlm_matmul_w_workspace_bytes(K),
             hip.lib().qlm_matmul_bf16_workspace_bytes(M, K))
    work = hip.DeviceBuffer(wb) if dnw is not None or with_work else None
    hip.call("qlm_matmul_w", dx, ldx, dnw, eps, dw, 1 if w.dtype == np.uint16 else 0, dy, ldy,
             M, N, K, EPI[epi], work, wb if work is not None else 0, None)
    got = dy.to_numpy((M, ldy), np.float32)
    assert np.all(got[:, N:] == 7.0), "wrote past N"
    return got[:, :N]


CASES = [  # (M, N, K); bf16 rows with M > 16 take the tiled prefill GEMM
    (1, 100, 256), (3, 37, 48), (16, 513, 1040), (20, 200, 2560), (1, 2560, 9728),
    (5, 16, 16), (17, 1000, 512), (130, 300, 1024), (300, 70, 512),
]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("epi", ["store", "norm", "resid", "swiglu"])
def test_matmul_w(hip, orc, rng, dtype, epi):
    eps = 1e-6
    for M, N, K in CASES:
        rows_w = 2 * N if epi == "swiglu" else N
        w32 = (rng.standard_normal((rows_w, K)) * 0.02).astype(np.float32)
        w = bf16_bits(w32) if dtype == "bf16" else w32
        x = rng.standard_normal((M, K)).astype(np.float32)
        nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
        y0 = rng.standard_normal((M, N)).astype(np.float32)
        ldx, ldy = K + (4 if M > 1 else 0), N + (3 if M > 1 else 0)
        ref = _ref(orc, epi, x, w, nw, y0, N, eps)
        for with_work in ((False, True) if M > 16 else (False,)):
            say("matmul_w", dtype, epi, M, N, K, with_work)
            got = _run(hip, epi, x, ldx, w, nw, y0, ldy, M, N, K, eps, with_work)
            tol = TOL_HILO if dtype == "bf16" and M > 16 and K % 32 == 0 else TOL
            for m in range(M):  # each activation row on its own scale
                err = rel_err(got[m], ref[m])
                assert err < tol, (dtype, epi, M, N, K, m, with_work, err)


def test_matmul_w_4b_shapes(hip, orc, rng):
    """The 4B model's one-row projections with bf16 rows."""
    for N, K, epi in [(9728, 2560, "swiglu"), (2560, 9728, "resid"), (8224, 2560, "norm")]:
        rows_w = 2 * N if epi == "swiglu" else N
        w = bf16_bits((rng.standard_normal((rows_w, K)) * 0.02).astype(np.float32))
        x = rng.standard_normal((1, K)).astype(np.float32)
        nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
        y0 = rng.standard_normal((1, N)).astype(np.float32)
        say("matmul_w 4b", N, K, epi)
        got = _run(hip, epi, x, K, w, nw, y0, N, 1, N, K, 1e-6)
        assert rel_err(got, _ref(orc, epi, x, w, nw, y0, N, 1e-6)) < TOL


def test_matmul_w_rejects_bad_args(hip):
    d = hip.DeviceBuffer(1 << 16)
    wb = hip.lib().qlm_matmul_w_workspace_bytes(64)
    with pytest.raises(hip.HipError):  # K not a multiple of 16
        hip.call("qlm_matmul_w", d, 40, None, 1e-6, d, 0, d, 8, 1, 8, 40, 0, None, 0, None)
    with pytest.raises(hip.HipError):  # SwiGLU needs the fused norm
        hip.call("qlm_matmul_w", d, 64, None, 1e-6, d, 0, d, 8, 1, 8, 64, 2, None, 0, None)
    with pytest.raises(hip.HipError):  # norm without a workspace
        hip.call("qlm_matmul_w", d, 64, d, 1e-6, d, 0, d, 8, 1, 8, 64, 0, None, 0, None)
    with pytest.raises(hip.HipError):  # workspace too small
        hip.call("qlm_matmul_w", d, 64, d, 1e-6, d, 0, d, 8, 1, 8, 64, 0, d, wb - 4, None)


WV_SHAPES = [(4, 1, 1, 4), (8, 1, 1, 4), (4, 2, 1, 3), (8, 2, 1, 3), (4, 4, 1, 2), (8, 2, 4, 3),
             (8, 1, 4, 4), (16, 1, 8, 4)]
WV_CASES = [  # (N, K, grid): ragged K (a part chunk), K under one chunk, N off the tile size
    (100, 1040, 0), (37, 48, 3), (300, 2560, 7), (64, 9728, 0), (1001, 512, 5)]


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("epi", ["store", "norm", "resid", "swiglu"])
def test_gemv_w_shapes(hip, orc, rng, dtype, epi):
    """Every built one-row launch shape against the oracle."""
    eps = 1e-6
    for N, K, grid in WV_CASES:
        rows_w = 2 * N if epi == "swiglu" else N
        w32 = (rng.standard_normal((rows_w, K)) * 0.02).astype(np.float32)
        w = bf16_bits(w32) if dtype == "bf16" else w32
        x = rng.standard_normal((1, K)).astype(np.float32)
        nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
        y0 = rng.standard_normal((1, N)).astype(np.float32)
        ref = _ref(orc, epi, x, w, nw, y0, N, eps)
        dx, dw = dev(hip, x), dev(hip, w)
        dnw = dev(hip, nw) if epi in ("norm", "swiglu") else None
        cw = 64 * (8 if dtype == "bf16" else 4)
        kp4 = ((K + cw - 1) // cw + 1) * (cw // 4)  # staged float4, zero chunk included
        for nwv, rg, ks, ring in WV_SHAPES:
            say("gemv_w_config", dtype, epi, N, K, grid, nwv, rg, ks, ring)
            yp = np.full((1, N + 8), 7.0, np.float32)
            yp[:, :N] = y0
            dy = dev(hip, yp)
            if kp4 > 5 * 64 * nwv:  # more than 20 staged columns per thread: refused
                with pytest.raises(hip.HipError):
                    hip.call("qlm_gemv_w_config", dx, dnw, eps, dw, 1 if dtype == "bf16" else 0,
                             dy, N, K, EPI[epi], nwv, rg, ks, ring, grid, None)
                continue
            hip.call("qlm_gemv_w_config", dx, dnw, eps, dw, 1 if dtype == "bf16" else 0, dy, N,
                     K, EPI[epi], nwv, rg, ks, ring, grid, None)
            got = dy.to_numpy((1, N + 8), np.float32)
            assert np.all(got[:, N:] == 7.0), "wrote past N"
            err = rel_err(got[:, :N], ref)
            assert err < TOL, (dtype, epi, N, K, grid, nwv, rg, ks, ring, err)


def test_gemv_w_config_rejects(hip):
    d = hip.DeviceBuffer(1 << 16)
    with pytest.raises(hip.HipError):  # a shape that is not built
        hip.call("qlm_gemv_w_config", d, None, 1e-6, d, 1, d, 8, 64, 0, 8, 3, 1, 3, 0, None)
    with pytest.raises(hip.HipError):  # K past the staged-x limit
        hip.call("qlm_gemv_w_config", d, None, 1e-6, d, 0, d, 8, 65536, 0, 4, 1, 1, 4, 0, None)
