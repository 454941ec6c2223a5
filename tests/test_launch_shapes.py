"""Launch shapes of the matrix-core GEMV/GEMM (host-side choice, no GPU call):
for every K the kernels accept, each wave's weight-block slots stay inside
the tile, every 64-column block is taken by exactly one (wave, slot), and
every wave owns at least one block. A wave with no block of its own once
computed its "last block" from a negative remainder and read past the tile;
these checks pin the host-side choices that keep that from happening."""

import ctypes as C

import pytest

from quicklm_amd import hip


def _blocks(nblk, nw, slots):
    """Block each (wave, slot) loads, and whether it is a real block: the
    kernels load min(w + nw*u, last block of wave w) and multiply slots
    past K by zero digits."""
    out = {}
    for w in range(nw):
        blast = nblk - 1 - ((nblk - 1 - w) % nw) if w < nblk else nblk - 1
        for u in range(slots):
            b = w + nw * u
            out[(w, u)] = (min(b, blast), b < nblk)
    return out


def _check(nblk, nw, slots):
    seen = []
    loads = _blocks(nblk, nw, slots)
    for (w, u), (b, real) in loads.items():
        assert 0 <= b < nblk, (nblk, nw, slots, w, u, b)
        if real:
            seen.append(b)
    assert sorted(seen) == list(range(nblk))
    assert all(any(real for (w2, _), (_, real) in loads.items() if w2 == w) for w in range(nw))


def test_gemv_mx_shapes():
    lib = hip.lib()
    w, r, g = C.c_int(), C.c_int(), C.c_int()
    served = 0
    for K in range(64, 16385, 64):
        for epi in (0, 1, 2):
            for N in (16, 300, 2560, 151936):
                rc = lib.qlm_gemv_i8_mx_shape(N, K, epi, C.byref(w), C.byref(r), C.byref(g))
                if rc != 0:
                    assert rc == -2
                    continue
                served += 1
                nblk = K // 64
                assert r.value == -(-nblk // w.value)
                assert 1 <= g.value <= max(1, -(-N // 16))
                _check(nblk, w.value, r.value)
    assert served > 100


@pytest.mark.parametrize("M", [2, 3, 4, 8, 16])
def test_matmul_mx_shapes(M):
    lib = hip.lib()
    w, u, r, g = C.c_int(), C.c_int(), C.c_int(), C.c_int()
    served = 0
    for K in range(64, 16385, 64):
        for epi in (0, 1, 2):
            for N in (16, 2560, 9728):
                rc = lib.qlm_matmul_i8_mx_shape(M, N, K, epi, C.byref(w), C.byref(u), C.byref(r),
                                                C.byref(g))
                if rc != 0:
                    assert rc == -2
                    continue
                served += 1
                nblk, nw = K // 64, w.value
                assert u.value >= -(-nblk // nw) and u.value % r.value == 0
                mp = 1 if M <= 2 else 2 if M <= 4 else 4 if M <= 8 else 8
                t = 2 if epi == 2 else 1
                lds = 2 * 2 * mp * 4 * 64 * nw + 2 * nw * t * 2 * mp * 16 * 4
                assert lds <= 96 * 1024
                _check(nblk, nw, u.value)
    assert served > 50
    assert lib.qlm_matmul_i8_mx_shape(17, 2560, 2560, 0, C.byref(w), C.byref(u), C.byref(r),
                                      C.byref(g)) == -2
