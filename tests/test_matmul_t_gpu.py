"""Batched decode matmul on the bf16 matrix cores over tile-major weights
(qlm_matmul_i8_t): the weights streamed from registers, regrouped by lane
swaps into their scale groups; activations split into bf16 hi + lo.

Bars: within 1e-5 normwise of the fp32 oracle (orc_matmul_i8, bit-exact with
the reference's int8 matmul) for every epilogue, launch shape and K slicing;
bit-exact on small-integer activations with power-of-two scales, where every
product and sum is exact.
"""

import ctypes as C

import numpy as np
import pytest

from tests.test_kernels_gpu import _mx_layout, _weights, dev
from tests.util import rel_err, say

pytestmark = pytest.mark.gpu

EPI = {"store": 0, "store_norm": 0, "resid": 1, "swiglu_norm": 2}
CASES = [  # (M, N, K)
    (2, 300, 1024), (3, 517, 2560), (16, 2560, 9728), (16, 1000, 2560), (16, 77, 3584),
    (7, 300, 512), (12, 130, 2560), (16, 2560, 2048), (5, 40, 64),
]
SHAPES = [(4, 4, 2), (4, 2, 3), (8, 2, 2), (8, 4, 2), (4, 8, 1), (4, 8, 2), (8, 8, 1)]


def _case(hip, orc, rng, M, N, K, epi, eps=1e-6):
    rows_w = 2 * N if epi.startswith("swiglu") else N
    q, s = _weights(orc, rng, rows_w, K, 32)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    ldy = N + 5
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    lg = orc.matmul_i8(orc.rms_norm(x, nw, eps) if epi.endswith("norm") else x, q, s, 32)
    if epi == "resid":
        ref = y0[:, :N] + lg
    elif epi.startswith("store"):
        ref = lg
    else:
        ref = orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy())
    dq, ds, keep = _mx_layout(hip, q, s, 32, N, K, 2 if epi.startswith("swiglu") else 1)
    return dict(x=dev(hip, x), nw=dev(hip, nw) if epi.endswith("norm") else None, dq=dq, ds=ds,
                keep=keep, y0=y0, ldy=ldy, ref=ref)


def _check(hip, c, M, N):
    y = c["dy"].to_numpy((M, c["ldy"]), np.float32)
    assert np.array_equal(y[:, N:], c["y0"][:, N:])  # the stride gap is untouched
    return rel_err(y[:, :N], c["ref"])


@pytest.mark.parametrize("M,N,K", CASES)
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid", "swiglu_norm"])
def test_matmul_t(hip, orc, rng, M, N, K, epi):
    c = _case(hip, orc, rng, M, N, K, epi)
    nwork = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, EPI[epi])
    work = hip.DeviceBuffer(nwork)
    work.upload(np.full(nwork, 0x5A, np.uint8))  # no initial contents are required
    c["dy"] = dev(hip, c["y0"])
    say("matmul_t", epi, M, N, K)
    hip.call("qlm_matmul_i8_t", c["x"], K, c["nw"], 1e-6, c["dq"], c["ds"], 32, c["dy"],
             c["ldy"], M, N, K, EPI[epi], work, nwork, None)
    err = _check(hip, c, M, N)
    assert err < 1e-5, (epi, M, N, K, err)


@pytest.mark.parametrize("epi", ["store_norm", "resid", "swiglu_norm"])
def test_matmul_t_shapes(hip, orc, rng, epi):
    """Every built launch shape and several K slicings, including slices
    with fewer blocks than waves and a ragged last slice."""
    M, N, K = 16, 200, 2560  # 40 blocks
    c = _case(hip, orc, rng, M, N, K, epi)
    rows_w = 2 * N if epi.startswith("swiglu") else N
    nwork = (K // 64) * M * rows_w * 4  # one block per slice at most
    work = hip.DeviceBuffer(nwork)
    for nw_, nt, p in SHAPES:
        for ks in (3, 4, 7, 13, 40):
            c["dy"] = dev(hip, c["y0"])
            say("matmul_t_config", epi, nw_, nt, p, ks)
            hip.call("qlm_matmul_i8_t_config", c["x"], K, c["nw"], 1e-6, c["dq"], c["ds"], 32,
                     c["dy"], c["ldy"], M, N, K, EPI[epi], nw_, nt, p, ks, work, nwork, None)
            err = _check(hip, c, M, N)
            assert err < 1e-5, (epi, nw_, nt, p, ks, err)


# whole-K form: (waves, tiles per half); grids 1 (one workgroup walks every
# tile group), 3 (a ragged share) and one group per workgroup
WHOLE = [(8, 1), (8, 2), (16, 1), (16, 2)]
WHOLE_CASES = [  # (M, N, K): K of 2, 4, 5 and 7 blocks per wave at 8 waves
    (16, 1000, 2560), (3, 517, 2560), (16, 2560, 2048), (7, 300, 1024), (16, 77, 3584),
    (12, 130, 2560), (2, 40, 1984), (16, 33, 960),
]


def _whole_built(nw, nth, K, norm, swiglu, slices=1):
    nblk = K // 64
    bps = -(-nblk // slices)
    px = -(-bps // nw)
    built = (nw == 8 and px in (2, 4, 5, 7)) or (nw == 16 and px == 2)
    spills = (px >= 7 and norm) or (swiglu and nth == 2 and (nw == 16 or px >= 5))
    return built and not spills and not (norm and K > 4096)


def _run_whole(hip, c, M, N, K, epi, nw_, nth, grid, slices):
    lib = hip.lib()
    nwork = lib.qlm_matmul_i8_t_whole_workspace_bytes(M, N, K, EPI[epi], slices)
    work = hip.DeviceBuffer(max(nwork, 16))
    work.upload(np.full(max(nwork, 16), 0x5A, np.uint8))  # no initial contents are required
    c["dy"] = dev(hip, c["y0"])
    say("matmul_t_whole", epi, M, N, K, nw_, nth, grid, slices)
    return lib.qlm_matmul_i8_t_whole_config(
        c["x"].ptr, K, c["nw"].ptr if c["nw"] else None, C.c_float(1e-6), c["dq"].ptr,
        c["ds"].ptr, 32, c["dy"].ptr, c["ldy"], M, N, K, EPI[epi], nw_, nth, grid, slices,
        work.ptr if nwork else None, C.c_size_t(nwork), None)


@pytest.mark.parametrize("M,N,K", WHOLE_CASES)
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid", "swiglu_norm"])
def test_matmul_t_whole(hip, orc, rng, M, N, K, epi):
    """The whole-K form for every built (waves, tiles) and several grids,
    within the tolerance of the K-sliced form; unbuilt or spilling shapes are
    refused with QLM_ERR_SHAPE before any launch."""
    c = _case(hip, orc, rng, M, N, K, epi)
    tiles_half = -(-N // 16)
    norm, swiglu = epi.endswith("norm"), epi.startswith("swiglu")
    ran = 0
    for nw_, nth in WHOLE:
        ok = _whole_built(nw_, nth, K, norm, swiglu)
        groups = -(-tiles_half // nth)
        for grid in sorted({1, min(3, groups), groups}):
            rc = _run_whole(hip, c, M, N, K, epi, nw_, nth, grid, 1)
            if not ok:
                assert rc == -2, (nw_, nth, K, rc)  # QLM_ERR_SHAPE
                continue
            hip.check(rc)
            err = _check(hip, c, M, N)
            assert err < 1e-5, (epi, M, N, K, nw_, nth, grid, err)
            ran += 1
    # K = 3584 with the RMSNorm gains spills at every built shape
    assert ran > 0 or (K == 3584 and norm)


@pytest.mark.parametrize("M,N,K,slices", [(16, 2560, 9728, 4), (5, 300, 9728, 3), (16, 200, 2560, 2),
                                          (16, 1000, 4096, 2), (7, 130, 3584, 2)])
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid", "swiglu_norm"])
def test_matmul_t_whole_sliced(hip, orc, rng, M, N, K, slices, epi):
    """K cut into slices (raw partial sums, then the ordered reduction with
    the epilogue and the RMSNorm) at every built (waves, tiles), including a
    ragged last slice; RMSNorm past K = 4096 is refused."""
    c = _case(hip, orc, rng, M, N, K, epi)
    norm, swiglu = epi.endswith("norm"), epi.startswith("swiglu")
    ran = 0
    for nw_, nth in WHOLE:
        ok = _whole_built(nw_, nth, K, norm, swiglu, slices)
        rc = _run_whole(hip, c, M, N, K, epi, nw_, nth, 160, slices)
        if not ok:
            assert rc == -2, (nw_, nth, K, slices, rc)
            continue
        hip.check(rc)
        err = _check(hip, c, M, N)
        assert err < 1e-5, (epi, M, N, K, slices, nw_, nth, err)
        ran += 1
    assert ran > 0 or (norm and K > 4096)


@pytest.mark.parametrize("N,K,epi", [(9728, 2560, "swiglu_norm"), (8224, 2560, "store_norm"),
                                     (2560, 2048, "resid"), (151936, 2560, "store_norm")])
def test_matmul_t_4b_projections(hip, orc, rng, N, K, epi):
    """The 4B projections at 16 rows through qlm_matmul_i8_t, which takes the
    whole-K form for them (no workspace)."""
    M = 16
    c = _case(hip, orc, rng, M, N, K, epi)
    nwork = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, EPI[epi])
    assert nwork == 0
    work = hip.DeviceBuffer(nwork) if nwork else None
    c["dy"] = dev(hip, c["y0"])
    say("matmul_t_4b", epi, M, N, K)
    hip.call("qlm_matmul_i8_t", c["x"], K, c["nw"], 1e-6, c["dq"], c["ds"], 32, c["dy"],
             c["ldy"], M, N, K, EPI[epi], work, nwork, None)
    err = _check(hip, c, M, N)
    assert err < 1e-5, (epi, N, K, err)


def test_matmul_t_exact_integers(hip, orc, rng):
    """Small-integer activations are exact in bf16 (lo = 0) and power-of-two
    scales keep every product and sum exact: bit-identical to the oracle."""
    M, N, K = 16, 300, 2048
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-8, -2, (N, K // 32))).astype(np.float32)
    x = rng.integers(-16, 17, (M, K)).astype(np.float32)
    ref = orc.matmul_i8(x, q, s, 32)
    dq, ds, keep = _mx_layout(hip, q, s, 32, N, K, 1)
    nwork = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, 0)
    work = hip.DeviceBuffer(nwork)
    dy = hip.DeviceBuffer(M * N * 4)
    hip.call("qlm_matmul_i8_t", dev(hip, x), K, None, 0.0, dq, ds, 32, dy, N, M, N, K, 0, work,
             nwork, None)
    assert np.array_equal(dy.to_numpy((M, N), np.float32), ref)


def test_matmul_t_refuses(hip, orc, rng):
    """M > 16, K not a multiple of 64, group K, an unbuilt shape and a slice
    longer than 64 blocks return an error before any launch."""
    lib = hip.lib()
    # buffers sized for the largest call below (64 rows, K up to 4160, 17
    # activation rows), so not even a regressed check could read past them
    q, s = _weights(orc, rng, 64, 4160, 32)
    dq, ds = dev(hip, q), dev(hip, s)
    x = dev(hip, rng.standard_normal((17, 4160)).astype(np.float32))
    y = hip.DeviceBuffer(17 * 64 * 4)
    work = hip.DeviceBuffer(1 << 22)
    for M, K, g in ((17, 2560, 32), (4, 2560 + 32, 32), (4, 2560, 2560)):
        assert lib.qlm_matmul_i8_t(x.ptr, K, None, C.c_float(0.0), dq.ptr, ds.ptr, g, y.ptr, 64,
                                   M, 64, K, 0, work.ptr, C.c_size_t(1 << 22), None) != 0
    assert lib.qlm_matmul_i8_t_config(x.ptr, 4096, None, C.c_float(0.0), dq.ptr, ds.ptr, 32,
                                      y.ptr, 64, 4, 64, 4096, 0, 4, 3, 2, 8, work.ptr,
                                      C.c_size_t(1 << 22), None) != 0
    assert lib.qlm_matmul_i8_t_config(x.ptr, 4160, None, C.c_float(0.0), dq.ptr, ds.ptr, 32,
                                      y.ptr, 64, 4, 64, 4160, 0, 4, 4, 2, 1, work.ptr,
                                      C.c_size_t(1 << 22), None) != 0  # 65-block slice


@pytest.mark.parametrize("M,N,K", [(17, 300, 2560), (64, 2560, 9728), (5, 1000, 2048),
                                   (130, 517, 1024), (300, 160, 2560), (1, 77, 3584)])
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid", "swiglu_norm"])
@pytest.mark.parametrize("group", [32, "K"])
def test_matmul_i8_tile_major(hip, orc, rng, M, N, K, epi, group):
    """qlm_matmul_i8_tm (prefill tiles and the K-split path over the
    tile-major weights, with its ragged last tiles) is bit-identical to
    qlm_matmul_i8 over the row-major weights, and within 1e-5 of the oracle."""
    g = K if group == "K" else 32
    rows_w = 2 * N if epi.startswith("swiglu") else N
    q, s = _weights(orc, rng, rows_w, K, g)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    ldy = N + 3
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    lg = orc.matmul_i8(orc.rms_norm(x, nw, 1e-6) if epi.endswith("norm") else x, q, s, g)
    ref = (y0[:, :N] + lg if epi == "resid" else lg if epi.startswith("store")
           else orc.silu_mul(lg[:, :N].copy(), lg[:, N:].copy()))
    dq, ds, keep = _mx_layout(hip, q, s, g, N, K, 2 if epi.startswith("swiglu") else 1)
    dx = dev(hip, x)
    dnw = dev(hip, nw) if epi.endswith("norm") else None
    nbytes = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, EPI[epi])
    work = hip.DeviceBuffer(nbytes)
    outs = []
    for fn, wq, ws in (("qlm_matmul_i8", keep[0], keep[1]), ("qlm_matmul_i8_tm", dq, ds)):
        dy = dev(hip, y0)
        work.upload(np.full(nbytes, 0xA5, np.uint8))
        say(fn, epi, g, M, N, K)
        hip.call(fn, dx, K, dnw, 1e-6, wq, ws, g, dy, ldy, M, N, K, EPI[epi], work, nbytes, None)
        outs.append(dy.to_numpy((M, ldy), np.float32))
    # 2..64 rows with one scale per weight row take the int8-digit form
    # (qlm_matmul_i8_rows64): the same product to ~1e-7, not the same bits
    digits = (group == "K" and 2 <= M <= 64 and not epi.startswith("swiglu")
              and (N >= 8192 or (M > 16 and K > 4096)))
    if not digits:
        assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[1][:, N:], y0[:, N:])
    assert rel_err(outs[1][:, :N], ref) < 1e-5
    assert rel_err(outs[0][:, :N], ref) < 1e-5


@pytest.mark.parametrize("M", [2, 5, 16, 17, 33, 64])
@pytest.mark.parametrize("N,K", [(77, 3584), (1000, 2560), (2560, 9728), (300, 192)])
@pytest.mark.parametrize("epi", ["store", "store_norm", "resid"])
def test_matmul_i8_rows64(hip, orc, rng, M, N, K, epi):
    """2..64 rows, one scale per weight row: the int8-digit form over the
    tile-major weights against the oracle (1e-5 normwise), directly and
    through qlm_matmul_i8_tm (bit-identical where it takes this form), with
    ragged tiles (N = 77), a single K slice (K = 192) and sliced K with the
    ordered reduction; columns past N of y untouched."""
    q, s = _weights(orc, rng, N, K, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    nw = (rng.standard_normal(K) * 0.02).astype(np.float32)
    ldy = N + 5
    y0 = rng.standard_normal((M, ldy)).astype(np.float32)
    lg = orc.matmul_i8(orc.rms_norm(x, nw, 1e-6) if epi == "store_norm" else x, q, s, K)
    ref = y0[:, :N] + lg if epi == "resid" else lg
    dq, ds, keep = _mx_layout(hip, q, s, K, N, K, 1)
    dx = dev(hip, x)
    dnw = dev(hip, nw) if epi == "store_norm" else None
    e = EPI[epi]
    need = hip.lib().qlm_matmul_i8_rows64_workspace_bytes(M, N, K, e)
    assert 0 < need <= hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, e)
    ntm = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, e)
    work = hip.DeviceBuffer(ntm)
    outs = []
    for fn in ("qlm_matmul_i8_rows64", "qlm_matmul_i8_tm"):
        dy = dev(hip, y0)
        work.upload(np.full(ntm, 0xA5, np.uint8))
        say(fn, epi, M, N, K)
        if fn == "qlm_matmul_i8_rows64":
            hip.call(fn, dx, K, dnw, 1e-6, dq, keep[1], dy, ldy, M, N, K, e, work, need, None)
        else:
            hip.call(fn, dx, K, dnw, 1e-6, dq, keep[1], K, dy, ldy, M, N, K, e, work, ntm, None)
        outs.append(dy.to_numpy((M, ldy), np.float32))
    # qlm_matmul_i8_tm takes the digit form from N = 8192, or above 16 rows
    # with K > 4096
    if N >= 8192 or (M > 16 and K > 4096):
        assert np.array_equal(outs[0], outs[1])
    for out in outs:
        assert np.array_equal(out[:, N:], y0[:, N:])
        assert rel_err(out[:, :N], ref) < 1e-5


@pytest.mark.parametrize("M", [4, 33, 64])
@pytest.mark.parametrize("N,K", [(65836, 192), (65536, 128), (66000, 320)])
@pytest.mark.parametrize("epi", ["store", "resid"])
def test_matmul_i8_rows64_rounds(hip, orc, rng, M, N, K, epi):
    """More than 256 tile groups: whole rounds over whole K, and the groups of
    the partial round split over K (65836 and 66000 rows: 2 groups past 256,
    cut into 3 and 5 slices) or none left (65536 rows); against the oracle."""
    q, s = _weights(orc, rng, N, K, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y0 = rng.standard_normal((M, N)).astype(np.float32)
    lg = orc.matmul_i8(x, q, s, K)
    ref = y0 + lg if epi == "resid" else lg
    dq, ds, keep = _mx_layout(hip, q, s, K, N, K, 1)
    dx = dev(hip, x)
    e = EPI[epi]
    need = hip.lib().qlm_matmul_i8_rows64_workspace_bytes(M, N, K, e)
    work = hip.DeviceBuffer(need)
    dy = dev(hip, y0)
    say("qlm_matmul_i8_rows64", epi, M, N, K)
    hip.call("qlm_matmul_i8_rows64", dx, K, None, 0.0, dq, keep[1], dy, N, M, N, K, e, work, need,
             None)
    assert rel_err(dy.to_numpy((M, N), np.float32), ref) < 1e-5


