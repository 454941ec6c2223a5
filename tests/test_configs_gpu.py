"""Parity at the isolated-kernel workloads' own sizes: the int8 matmul
shapes, the Gated DeltaNet step and chunked prefill at 32 heads, and the GQA
decode attention at long contexts, each against the CPU oracle.

  int8 matmul      N x K in {4096x4096, 12288x4096, 4096x12288, 151936x2560},
                   Wq int8 U{-127..127}, per-row scales U(0.001, 0.01) (and
                   group-32 scales for the tile-major forms), x N(0,1), at
                   M = 1, 4, 16, 64 (math_ops.cpp:820-900), through the
                   row-major entry point and through exactly the kernel
                   bench.py times at each M. The 151936-row case is scored on
                   a sample of rows (every output row is an independent dot
                   product).
  DeltaNet         decode step at B = 32, 32 heads, d = 128: S N(0, 0.01),
                   q, k L2-normalised N(0,1), v N(0,1), decay =
                   sigmoid(N(0,1) + 2), beta = sigmoid(N(0,1))
                   (attention.cpp:498-571); chunked prefill of T = 4096 rows
                   at 32 heads against the oracle's row-by-row recurrence
                   (attention.cpp:600-758), on a sample of heads (the heads
                   are independent) for every row and the final state.
  GQA attention    16 query / 2 KV heads, hd 256, bf16 K/V N(0,1), fp32 q,
                   B in {1, 16}, ctx in {8192, 32768} (attention.cpp:54-82),
                   scored on a sample of sequences at full context; and the
                   fused decode (QK-norm, RoPE, cache write) at ctx 8192 and
                   32768 with an fp32 cache.
Bars as the other kernel tests: 1e-5 normwise for the matmuls and the
attention (fp32 accumulation), 1e-4 for the DeltaNet recurrence over many
rows (reassociated fp32 in the chunked form).
"""

import ctypes as C

import numpy as np
import pytest

from tests.util import bf16_bits, bf16_to_f32, rel_err, say

pytestmark = pytest.mark.gpu

SHAPES = [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 2560)]


def dev(hip, a):
    return hip.DeviceBuffer.from_numpy(np.ascontiguousarray(a))


def cfg1_weights(rng, N, K, group):
    q = rng.integers(-127, 128, (N, K), dtype=np.int8)
    nb = 1 if group == K else K // group
    s = rng.uniform(0.001, 0.01, (N, nb)).astype(np.float32)
    return q, s


def sample_rows(N):
    """Rows scored against the oracle: all of them, or every 37th (plus the
    last) for the 151936-row matrix."""
    return np.arange(N) if N <= 12288 else np.unique(np.r_[np.arange(0, N, 37), N - 1])


def swizzle(hip, dq, ds, group, N, K):
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx_layout_bytes(N, K, group, 1, C.byref(qb), C.byref(sb)))
    qz = hip.DeviceBuffer(qb.value)
    sz = hip.DeviceBuffer(sb.value) if sb.value else ds
    hip.call("qlm_mx_swizzle", dq, ds, group, N, K, 1, qz, sz if sb.value else None, None)
    return qz, sz


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_cfg1_matmul_row_scales(hip, orc, rng, N, K, M):
    """Per-row scales (G = K): M = 1 on the int8 matrix cores over the
    tile-major copy (the decode GEMV), M = 16 and 64 through qlm_matmul_i8."""
    q, s = cfg1_weights(rng, N, K, K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    rows = sample_rows(N)
    ref = orc.matmul_i8(x, np.ascontiguousarray(q[rows]), np.ascontiguousarray(s[rows]), K)
    dq, ds, dx = dev(hip, q), dev(hip, s), dev(hip, x)
    dy = hip.DeviceBuffer(M * N * 4)
    say(f"cfg1 row scales {N}x{K} M={M}")
    if M == 1:
        qz, sz = swizzle(hip, dq, ds, K, N, K)
        hip.call("qlm_gemv_i8_mx", dx, None, 0.0, qz, sz, K, dy, N, K, 0, None)
    else:
        nbytes = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, 0)
        work = hip.DeviceBuffer(nbytes)
        hip.call("qlm_matmul_i8", dx, K, None, 0.0, dq, ds, K, dy, N, M, N, K, 0, work, nbytes,
                 None)
    y = dy.to_numpy((M, N), np.float32)[:, rows]
    assert rel_err(y, ref) < 1e-5


@pytest.mark.parametrize("N,K", SHAPES)
def test_cfg1_matmul_tile_major_m16(hip, orc, rng, N, K):
    """Group-32 scales, M = 16: the batched-decode matmul over the tile-major
    copy (qlm_matmul_i8_t), the form the engine runs for 2-16 rows."""
    q, s = cfg1_weights(rng, N, K, 32)
    M = 16
    x = rng.standard_normal((M, K)).astype(np.float32)
    rows = sample_rows(N)
    ref = orc.matmul_i8(x, np.ascontiguousarray(q[rows]), np.ascontiguousarray(s[rows]), 32)
    qz, sz = swizzle(hip, dev(hip, q), dev(hip, s), 32, N, K)
    nbytes = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, 0)
    work = hip.DeviceBuffer(nbytes)
    dy = hip.DeviceBuffer(M * N * 4)
    say(f"cfg1 tile-major {N}x{K} M=16")
    hip.call("qlm_matmul_i8_t", dev(hip, x), K, None, 0.0, qz, sz, 32, dy, N, M, N, K, 0, work,
             nbytes, None)
    assert rel_err(dy.to_numpy((M, N), np.float32)[:, rows], ref) < 1e-5


@pytest.fixture(scope="module")
def cfg1_cache():
    """One weight draw per (shape, scale group), on the host and on the
    device in the tile-major layout, shared by the M cases below."""
    return {}


@pytest.mark.parametrize("N,K", SHAPES)
@pytest.mark.parametrize("group", ["row", 32])
@pytest.mark.parametrize("M", [4, 16, 64])
def test_cfg1_bench_kernels(hip, orc, cfg1_cache, N, K, group, M):
    """The kernel bench.py times at each M over the tile-major weights, at the
    workload's own shapes: group-32 scales at 4 and 16 rows qlm_matmul_i8_t,
    every other case qlm_matmul_i8_tm (which takes its int8-digit form,
    k_act_digits + k_mm_rows64, for per-row scales at N >= 8192 or more than
    16 rows with K > 4096, and the bf16 matrix-core form elsewhere)."""
    g = K if group == "row" else 32
    key = (N, K, g)
    if key not in cfg1_cache:
        cfg1_cache.clear()  # one shape's weights resident at a time
        wr = np.random.default_rng(N * 31 + K + g)
        q, s = cfg1_weights(wr, N, K, g)
        qz, sz = swizzle(hip, dev(hip, q), dev(hip, s), g, N, K)
        cfg1_cache[key] = (q, s, qz, sz)
    q, s, qz, sz = cfg1_cache[key]
    rng = np.random.default_rng(N + K + M)
    x = rng.standard_normal((M, K)).astype(np.float32)
    rows = sample_rows(N)
    ref = orc.matmul_i8(x, np.ascontiguousarray(q[rows]), np.ascontiguousarray(s[rows]), g)
    dy = hip.DeviceBuffer(M * N * 4)
    if M <= 16 and g == 32:
        kern = "qlm_matmul_i8_t"
        nbytes = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, 0)
    else:
        kern = "qlm_matmul_i8_tm"
        nbytes = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, 0)
    work = hip.DeviceBuffer(nbytes)
    say(f"cfg1 bench kernel {kern} {N}x{K} M={M} group={group}")
    hip.call(kern, dev(hip, x), K, None, 0.0, qz, sz, g, dy, N, M, N, K, 0, work, nbytes, None)
    assert rel_err(dy.to_numpy((M, N), np.float32)[:, rows], ref) < 1e-5


def _l2n(x):
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


def _sig(x):
    return (1 / (1 + np.exp(-x))).astype(np.float32)


@pytest.mark.parametrize("B", [1, 8, 32])
def test_cfg2_delta_step(hip, orc, rng, B):
    """The recurrent step at the workload's batches (1, 8, 32 sequences), 32
    heads, three steps in a row."""
    H, d = 32, 128
    S = (rng.standard_normal((B, H, d, d)) * 0.01).astype(np.float32)
    dS, Sref = dev(hip, S), S.copy()
    for step in range(3):
        q = _l2n(rng.standard_normal((B, H, d)))
        k = _l2n(rng.standard_normal((B, H, d)))
        v = rng.standard_normal((B, H, d)).astype(np.float32)
        a = _sig(rng.standard_normal((B, H)) + 2)
        b = _sig(rng.standard_normal((B, H)))
        o_ref, Sref = orc.gated_delta_step(q, k, v, a, b, Sref)
        do = hip.DeviceBuffer(q.nbytes)
        say(f"cfg2 delta step B={B} H=32 step", step)
        hip.call("qlm_gated_delta_step", dev(hip, q), dev(hip, k), dev(hip, v), dev(hip, a),
                 dev(hip, b), dS, do, B, H, d, None)
        assert rel_err(do.to_numpy(q.shape, np.float32), o_ref) < 1e-5
        assert rel_err(dS.to_numpy(S.shape, np.float32), Sref) < 1e-5


def head_subset(proj, wt, A_log, dtb, heads, H, d):
    """The mixer inputs of a subset of heads as a smaller problem: proj rows
    [q|k|v|z|b|a] and the tap-major conv weights restricted to their channels."""
    HD = H * d
    cols = np.concatenate([np.arange(sec * HD + h * d, sec * HD + (h + 1) * d)
                           for sec in range(4) for h in heads])
    gcols = np.array([4 * HD + h for h in heads] + [4 * HD + H + h for h in heads])
    conv_cols = cols[: 3 * len(heads) * d]
    return (np.ascontiguousarray(proj[..., np.r_[cols, gcols]]),
            np.ascontiguousarray(wt[:, conv_cols]), A_log[heads].copy(), dtb[heads].copy(),
            conv_cols)


def test_cfg2_chunked_prefill_t4096_h32(hip, orc, rng):
    """Chunked (WY) prefill of 4096 rows at 32 heads from a zero state
    against the oracle's row-by-row recurrence on three heads: every output
    row of those heads and their final state and conv ring."""
    T, H, d = 4096, 32, 128
    HD = H * d
    ldp = 4 * HD + 2 * H
    wt = (rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32)
    A_log = np.log(rng.uniform(1, 16, H)).astype(np.float32)
    dtb = (rng.standard_normal(H) * 0.5 - 4).astype(np.float32)
    nw = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    proj = (rng.standard_normal((T, ldp)) * 0.6).astype(np.float32)
    conv = np.zeros((3, 3 * HD), np.float32)
    S = np.zeros((H, d, d), np.float32)
    dconv, dS = dev(hip, conv), dev(hip, S)
    nbytes = hip.lib().qlm_deltanet_chunk_workspace_bytes(T, H, d)
    work = hip.DeviceBuffer(nbytes)
    do = hip.DeviceBuffer(T * HD * 4)
    say("cfg2 chunked prefill T=4096 H=32")
    hip.call("qlm_deltanet_prefill_chunked", dev(hip, proj), ldp, T, dconv, dev(hip, wt),
             dev(hip, A_log), dev(hip, dtb), dev(hip, nw), dS, 0, do, HD, H, d, work, nbytes,
             None)
    out = do.to_numpy((T, HD), np.float32)
    S_gpu = dS.to_numpy(S.shape, np.float32)
    conv_gpu = dconv.to_numpy(conv.shape, np.float32)
    heads = [0, 13, 31]
    hp, hwt, hA, hdt, conv_cols = head_subset(proj, wt, A_log, dtb, heads, H, d)
    h_n = len(heads)
    conv_ref = np.zeros((3, 3 * h_n * d), np.float32)
    S_ref = np.zeros((h_n, d, d), np.float32)
    ref = np.stack([orc.deltanet_core(hp[t], conv_ref, t % 3, hwt, hA, hdt, nw, S_ref, h_n, d)
                    for t in range(T)])
    got = np.concatenate([out[:, h * d:(h + 1) * d] for h in heads], axis=1)
    assert rel_err(got, ref) < 1e-4
    assert rel_err(S_gpu[heads], S_ref) < 1e-4
    # the ring holds the last three rows' inputs at the slots position T reads
    assert np.array_equal(conv_gpu[:, conv_cols], conv_ref)


@pytest.mark.parametrize("B", [1, 16])
@pytest.mark.parametrize("ctx", [8192, 32768])
def test_cfg3_attention_bf16_long(hip, orc, rng, B, ctx):
    n_q, n_kv, hd = 16, 2, 256
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    kb = bf16_bits(rng.standard_normal((B, ctx, n_kv, hd), dtype=np.float32))
    vb = bf16_bits(rng.standard_normal((B, ctx, n_kv, hd), dtype=np.float32))
    dk, dv = dev(hip, kb), dev(hip, vb)
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, ctx))
    do = hip.DeviceBuffer(q.nbytes)
    say(f"cfg3 attention bf16 B={B} ctx={ctx}")
    hip.call("qlm_attention_decode", dev(hip, q), dk, dv, 1, ctx, ctx, do, B, n_q, n_kv, hd, work,
             None)
    out = do.to_numpy(q.shape, np.float32)
    for b in sorted({0, B - 1}):
        ref = orc.attention(q[b], bf16_to_f32(kb[b]), bf16_to_f32(vb[b]), ctx)
        assert rel_err(out[b], ref) < 1e-5, b


@pytest.mark.parametrize("pos", [8191, 32767])
def test_cfg3_gqa_decode_long(hip, orc, rng, pos):
    """Fused decode (QK-norm, RoPE at pos, cache write, attention, no gate)
    with 16 q / 2 kv heads at hd 256 over pos + 1 positions, fp32 cache."""
    n_q, n_kv, hd, rot, theta = 16, 2, 256, 64, 1e6
    max_seq = pos + 1
    ld = n_q * hd + 2 * n_kv * hd
    qn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    kn = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    cos_t, sin_t = orc.rope_table(theta, rot, max_seq)
    kc = rng.standard_normal((max_seq, n_kv, hd), dtype=np.float32)
    vc = rng.standard_normal((max_seq, n_kv, hd), dtype=np.float32)
    dkc, dvc = dev(hip, kc), dev(hip, vc)
    qkv = rng.standard_normal((1, ld)).astype(np.float32)
    ref = orc.gqa_core(qkv[0].copy(), qn, kn, theta, rot, kc, vc, pos, n_q, n_kv, hd, False)
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(1, n_q, hd, max_seq))
    do = hip.DeviceBuffer(n_q * hd * 4)
    say(f"cfg3 gqa decode pos={pos}")
    hip.call("qlm_gqa_decode", dev(hip, qkv), ld, dev(hip, qn), dev(hip, kn), dev(hip, cos_t),
             dev(hip, sin_t), rot, dkc, dvc, max_seq, dev(hip, np.array([pos], np.int32)), do,
             n_q * hd, 1, n_q, n_kv, hd, 0, work, None)
    assert rel_err(do.to_numpy(n_q * hd, np.float32), ref) < 1e-5
    assert np.array_equal(dvc.to_numpy(vc.shape, np.float32)[pos], vc[pos])
