#!/usr/bin/env python3
"""Benchmark: 4B-class int8 hybrid decode on one MI355X, the isolated
kernels of the path at their own workload sizes, and the reference CPU path
timed beside them.

Workload of `value` (one "step" = one greedy decode step of every sequence):
  4B-class hybrid LM, 36 layers (27 Gated DeltaNet + 9 GQA), hidden 2560,
  FFN 9728, vocab 151936, seeded random-init weights quantised to int8 at load
  (Q8_0 group-32 scales, the reference's format), 2048-token uniform random
  prompts (batched prefill of positions 0..2046, untimed), greedy decode; the
  whole step is one replayed hipGraph. `value` = batch-1 decode tokens/s over
  exactly --steps timed steps after --warmup untimed steps; batch 16 beside it.
  `parity` compares greedy streams with the reference's IEEE build on the same
  checkpoint and prompts (tests/golden/4b_greedy.npz, 4b_greedy_seq1.npz:
  sequences 0 and 1 of the batch, 256 steps each), at batch 1 and as rows of
  the batch-16 run, from generate runs of their own outside the timed region.

Isolated kernels (every launch timed with HIP events around graph replays of
back-to-back launches on the launching stream, operands cycled over copies
larger than the 256 MB last-level cache so each launch streams from HBM):
  config1_gemv       int8 matmul, N x K in {4096^2, 12288x4096, 4096x12288,
                     151936x2560}, M in {1, 4, 16, 64}: HBM GB/s, and MFMA
                     utilisation at M = 64
  config2_deltanet   Gated DeltaNet step at batch 1/8/32 x 32 heads (GB/s) and
                     the chunked prefill of 4096 rows (fp32 matrix-core
                     utilisation)
  config3_attention  GQA decode attention, 16 q / 2 kv heads, hd 256, bf16 KV,
                     batch 1/16 x ctx 2048/8192/32768 (GB/s)
  prefill            the 4B 2047-row prefill and its gate/up matmul (bf16
                     matrix-core utilisation)
`roofline` is the dominant decode kernel (the fused RMSNorm + gate/up GEMV +
SwiGLU, 36 launches per step). `cpu_baseline` is the reference's own sources
built with its release flags, one thread per physical core, on a bounded
sample of the same 4B workload.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--kernel-only]
"""

from __future__ import annotations

import argparse
import hashlib
import ctypes as C
import json
import os
import subprocess
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_FLOPS = 2.5e15   # dense bf16 matrix-core peak of MI355X
FP32_MFMA_PEAK_FLOPS = 157.3e12  # dense fp32 matrix-core peak of MI355X
METRIC = "decode tokens/sec at batch 1 and 16 (4B int8); int8 GEMV achieved HBM GB/s"
GOLDEN_4B = os.path.join(ROOT, "tests", "golden", "4b_greedy.npz")
GOLDEN_4B_SEQ1 = os.path.join(ROOT, "tests", "golden", "4b_greedy_seq1.npz")
# the dominant kernel's source: a PMC record is this build's only if it
# carries the same hash
DOM_SOURCES = [os.path.join(ROOT, "quicklm_amd", "csrc", "kernels", f)
               for f in ("gemv.hip", "common.hpp")]
POOL_BYTES = 1 << 30  # operands cycled over at least this many bytes


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def n_copies(nbytes, lo=2, hi=256):
    return int(max(lo, min(hi, -(-POOL_BYTES // max(1, nbytes)))))


def graph_time(hip, st, launch, per, launches=400):
    """Average duration (us) of one launch: `per` launches (launch(i), i <
    per) captured into one graph, replayed until about `launches` have run,
    HIP events recorded on the same stream around the replays."""
    lib = hip.lib()
    for i in range(per):  # warm-up: code objects loaded, copies touched
        launch(i)
    hip.check(lib.qlm_graph_begin(st.ptr))
    for i in range(per):
        launch(i)
    g = C.c_void_p()
    hip.check(lib.qlm_graph_end(st.ptr, C.byref(g)))
    hip.check(lib.qlm_graph_launch(g, st.ptr))
    reps = max(1, launches // per)
    e0, e1 = hip.Event(), hip.Event()
    e0.record(st.ptr)
    for _ in range(reps):
        hip.check(lib.qlm_graph_launch(g, st.ptr))
    e1.record(st.ptr)
    st.sync()
    us = e0.elapsed_ms(e1) * 1000.0 / (reps * per)
    hip.check(lib.qlm_graph_destroy(g))
    return us


def dev_copies(hip, a, n):
    """n device copies of host array a (one upload, then device copies)."""
    first = hip.DeviceBuffer.from_numpy(a)
    out = [first]
    for _ in range(n - 1):
        b = hip.DeviceBuffer(first.nbytes)
        hip.check(hip.lib().qlm_memcpy_d2d(b.ptr, first.ptr, first.nbytes, None))
        out.append(b)
    hip.sync()
    return out


def free_all(bufs):
    for b in bufs:
        b.free()


# ------------------------------------------------------------ config 1
def gemv_bytes(N, K, M, group):
    nb = 1 if group == K else K // group
    return N * K + 4 * N * nb + 4 * M * K + 4 * M * N


def tile_major(hip, dq, ds, group, rows, K, halves=1):
    """Tile-major copies (qlm_mx_swizzle) of each weight copy (halves = 2: a
    [gate; up] matrix of 2 x rows, each half tiled on its own); per-row
    scales keep their layout."""
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx_layout_bytes(rows, K, group, halves, C.byref(qb), C.byref(sb)))
    out = []
    for q_, s_ in zip(dq, ds):
        qz = hip.DeviceBuffer(qb.value)
        sz = hip.DeviceBuffer(sb.value) if sb.value else s_
        hip.call("qlm_mx_swizzle", q_, s_, group, rows, K, halves, qz, sz if sb.value else None,
                 None)
        out.append((qz, sz))
    hip.sync()
    return out


def bench_config1(hip, Ms=(1, 4, 16, 64)):
    """int8 matmul y = x (Wq s)^T: Wq U{-127..127}, s U(0.001, 0.01), x N(0,1).
    Per-row scales (the workload's scheme) with the kernel the engine runs at
    each M over its tile-major weights: M = 1 the matrix-core GEMV; M = 4, 16
    qlm_matmul_i8_tm (bf16 matrix cores), M = 64 its int8-digit form
    (qlm_matmul_i8_rows64). Group-32 scales beside them, where M = 4 and 16
    take the batched-decode form (qlm_matmul_i8_t) and M = 64
    qlm_matmul_i8_tm."""
    rng = np.random.default_rng(0)
    st = hip.Stream()
    out = []
    for (N, K) in [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 2560)]:
        q = rng.integers(-127, 128, (N, K), dtype=np.int8)
        for group in (K, 32):
            nb = 1 if group == K else K // group
            s = rng.uniform(0.001, 0.01, (N, nb)).astype(np.float32)
            ncopy = n_copies(N * K + 4 * N * nb, lo=3, hi=128)
            dq, ds = dev_copies(hip, q, ncopy), dev_copies(hip, s, ncopy)
            dz = tile_major(hip, dq, ds, group, N, K)
            for M in Ms:
                x = hip.DeviceBuffer.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
                y = hip.DeviceBuffer(M * N * 4)
                if M == 1:
                    kern = "qlm_gemv_i8_mx"

                    def launch(i):
                        qz, sz = dz[i % ncopy]
                        hip.call(kern, x, None, 0.0, qz, sz, group, y, N, K, 0, st.ptr)
                    work = None
                elif M <= 16 and group == 32:
                    kern = "qlm_matmul_i8_t"
                    nwork = hip.lib().qlm_matmul_i8_t_workspace_bytes(M, N, K, 0)
                    work = hip.DeviceBuffer(nwork)

                    def launch(i):
                        qz, sz = dz[i % ncopy]
                        hip.call(kern, x, K, None, 0.0, qz, sz, group, y, N, M, N, K, 0, work,
                                 nwork, st.ptr)
                else:
                    # the tile-major copy the engine holds: per-row scales at
                    # 17..64 rows take the int8-digit form inside it
                    kern = "qlm_matmul_i8_tm"
                    nwork = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, 0)
                    work = hip.DeviceBuffer(nwork)

                    def launch(i):
                        qz, sz = dz[i % ncopy]
                        hip.call(kern, x, K, None, 0.0, qz, sz, group, y, N, M, N, K, 0, work,
                                 nwork, st.ptr)
                us = graph_time(hip, st, launch, ncopy, launches=max(100, 2 * ncopy))
                b = gemv_bytes(N, K, M, group)
                r = {"N": N, "K": K, "M": M, "scales": "row" if group == K else "group32",
                     "kernel": kern, "us": round(us, 2), "GBps": round(b / us / 1e3, 1),
                     "bytes": b, "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
                if M == 64:  # algorithmic flops over the dense bf16 matrix-core peak
                    r["mfma_util"] = round(2.0 * M * N * K / (us * 1e-6) / BF16_PEAK_FLOPS, 4)
                out.append(r)
                log(f"config1 {N}x{K} M={M} {r['scales']} {kern}: {us:.2f} us, "
                    f"{r['GBps']:.0f} GB/s" + (f", MFMA util {r['mfma_util']:.3f}"
                                               if M == 64 else ""))
                x.free()
                y.free()
                if work is not None:
                    work.free()
            free_all(dq + ds + [t for pair in dz for t in pair if t not in ds])
    return out


# ------------------------------------------------------------ config 2
def l2n(x):
    return (x / np.linalg.norm(x, axis=-1, keepdims=True)).astype(np.float32)


def sigmoid(x):
    return (1.0 / (1.0 + np.exp(-x))).astype(np.float32)


def bench_config2(hip, H=32, d=128, T=4096):
    """Gated DeltaNet: the recurrent step (attention.cpp:498-571) at batch
    1/8/32 x 32 heads, S N(0, 0.01), q/k L2-normalised N(0,1), v N(0,1),
    decay sigmoid(N(0,1)+2), beta sigmoid(N(0,1)); bytes = B H (2*4 d^2 +
    4*4 d + 8). Then the chunked prefill of T rows (64-row chunks) at batch 1,
    with the chunked form's matrix-core flops per chunk and head, 8 C^2 d +
    6 C d^2 (K K^T, Q K^T, the triangular solve on [bK | bV], W S, Q S, the
    masked intra-chunk product, K^T W), over the fp32 matrix-core peak."""
    rng = np.random.default_rng(2)
    st = hip.Stream()
    res = {"heads": H, "head_dim": d, "decode": []}
    for B in (1, 8, 32):
        sbytes = B * H * d * d * 4
        ncopy = n_copies(sbytes, lo=2, hi=256)
        S = (rng.standard_normal((B, H, d, d)) * 0.01).astype(np.float32)
        dS = dev_copies(hip, S, ncopy)
        q = hip.DeviceBuffer.from_numpy(l2n(rng.standard_normal((B, H, d))))
        k = hip.DeviceBuffer.from_numpy(l2n(rng.standard_normal((B, H, d))))
        v = hip.DeviceBuffer.from_numpy(rng.standard_normal((B, H, d)).astype(np.float32))
        a = hip.DeviceBuffer.from_numpy(sigmoid(rng.standard_normal((B, H)) + 2))
        bt = hip.DeviceBuffer.from_numpy(sigmoid(rng.standard_normal((B, H))))
        o = hip.DeviceBuffer(B * H * d * 4)

        def launch(i):
            hip.call("qlm_gated_delta_step", q, k, v, a, bt, dS[i % ncopy], o, B, H, d, st.ptr)

        us = graph_time(hip, st, launch, ncopy, launches=max(200, ncopy))
        nbytes = B * H * (2 * 4 * d * d + 4 * 4 * d + 8)
        res["decode"].append({"batch": B, "us": round(us, 2), "bytes": nbytes,
                              "GBps": round(nbytes / us / 1e3, 1),
                              "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)})
        log(f"config2 DeltaNet step B={B} H={H}: {us:.2f} us, {nbytes / us / 1e3:.0f} GB/s")
        free_all(dS + [q, k, v, a, bt, o])
    # chunked prefill, batch 1
    HD = H * d
    ldp = 4 * HD + 2 * H
    proj = hip.DeviceBuffer.from_numpy((rng.standard_normal((T, ldp)) * 0.6).astype(np.float32))
    wt = hip.DeviceBuffer.from_numpy((rng.standard_normal((4, 3 * HD)) * 0.3).astype(np.float32))
    A_log = hip.DeviceBuffer.from_numpy(np.log(rng.uniform(1, 16, H)).astype(np.float32))
    dtb = hip.DeviceBuffer.from_numpy((rng.standard_normal(H) * 0.5 - 4).astype(np.float32))
    nw = hip.DeviceBuffer.from_numpy((1 + rng.standard_normal(d) * 0.02).astype(np.float32))
    conv, S1 = hip.DeviceBuffer(3 * 3 * HD * 4), hip.DeviceBuffer(H * d * d * 4)
    out = hip.DeviceBuffer(T * HD * 4)
    nbytes = hip.lib().qlm_deltanet_chunk_workspace_bytes(T, H, d)
    work = hip.DeviceBuffer(nbytes)

    conv.zero()
    S1.zero()
    hip.sync()

    def launch_pf():
        # each run continues from the last one's state (the arithmetic per
        # row is the same); launched directly: four kernels of ~ms each
        hip.call("qlm_deltanet_prefill_chunked", proj, ldp, T, conv, wt, A_log, dtb, nw, S1, 0,
                 out, HD, H, d, work, nbytes, st.ptr)

    launch_pf()
    reps = 5
    e0, e1 = hip.Event(), hip.Event()
    e0.record(st.ptr)
    for _ in range(reps):
        launch_pf()
    e1.record(st.ptr)
    st.sync()
    ms = e0.elapsed_ms(e1) / reps
    C_ = 64
    flops = (T // C_) * H * (8 * C_ * C_ * d + 6 * C_ * d * d)
    res["chunked_prefill"] = {"rows": T, "chunk": C_, "batch": 1, "ms": round(ms, 3),
                              "flops": flops, "TFLOPs": round(flops / ms / 1e9, 2),
                              "mfma_util_fp32": round(flops / (ms * 1e-3) /
                                                      FP32_MFMA_PEAK_FLOPS, 4),
                              "rows_per_s": round(T / (ms * 1e-3), 1)}
    log(f"config2 chunked prefill T={T} H={H}: {ms:.3f} ms, {flops / ms / 1e9:.1f} TFLOP/s")
    free_all([proj, wt, A_log, dtb, nw, conv, S1, out, work])
    return res


# ------------------------------------------------------------ config 3
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (chunked, in place)."""
    out = np.empty(x.shape, np.uint16)
    flat, of = x.reshape(-1), out.reshape(-1)
    step = 1 << 24
    for i in range(0, flat.size, step):
        u = flat[i:i + step].view(np.uint32)
        of[i:i + step] = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return out


def bench_config3(hip, n_q=16, n_kv=2, hd=256, ctx_max=32768, Bmax=16):
    """GQA decode attention over a bf16 KV cache [B, max_seq, n_kv, hd]
    (attention.cpp:54-82; the reference's fp32 cache upcast): K/V N(0,1), q
    fp32 N(0,1) (already rotated), softmax over ctx positions; bytes =
    B * 2 * ctx * n_kv * hd * 2 + 8 * B * n_q * hd. One 16 x 32768-position
    cache is generated; smaller cases read windows of it at distinct
    offsets, so that successive launches stream different bytes."""
    rng = np.random.default_rng(3)
    st = hip.Stream()
    shape = (Bmax, ctx_max, n_kv, hd)
    kv = [hip.DeviceBuffer.from_numpy(bf16_bits(rng.standard_normal(shape, dtype=np.float32)))
          for _ in range(2)]
    row = n_kv * hd * 2  # bytes per cached position
    total_pos = Bmax * ctx_max
    res = []
    for B in (1, Bmax):
        q = hip.DeviceBuffer.from_numpy(rng.standard_normal((B, n_q, hd)).astype(np.float32))
        o = hip.DeviceBuffer(B * n_q * hd * 4)
        for ctx in (2048, 8192, 32768):
            # windows of B sequences (stride ctx_max) starting at distinct offsets
            last = total_pos - ((B - 1) * ctx_max + ctx)
            offs = list(range(0, last + 1, ctx))[:64] or [0]
            work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, ctx_max))

            def launch(i):
                off = offs[i % len(offs)] * row
                hip.check(hip.lib().qlm_attention_decode(q.ptr, kv[0].ptr + off, kv[1].ptr + off,
                                                         1, ctx_max, ctx, o.ptr, B, n_q, n_kv,
                                                         hd, work.ptr, st.ptr))

            per = max(2, len(offs))
            us = graph_time(hip, st, launch, per, launches=max(100, per))
            nbytes = B * 2 * ctx * n_kv * hd * 2 + 8 * B * n_q * hd
            res.append({"batch": B, "ctx": ctx, "us": round(us, 2), "bytes": nbytes,
                        "GBps": round(nbytes / us / 1e3, 1),
                        "frac_hbm": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)})
            log(f"config3 attention B={B} ctx={ctx}: {us:.2f} us, {nbytes / us / 1e3:.0f} GB/s")
            work.free()
        free_all([q, o])
    free_all(kv)
    return {"n_q": n_q, "n_kv": n_kv, "head_dim": hd, "kv_dtype": "bf16", "cases": res}


# ------------------------------------------------------------ prefill matmul
def bench_prefill_matmul(hip, M=2047, F=9728, K=2560):
    """The 4B prefill's largest matmul: RMSNorm + gate/up (2F = 19456 int8
    rows, group-32 scales) + SwiGLU over M prompt rows, bf16 matrix cores, over
    the tile-major weights the engine holds (qlm_matmul_i8_tm); utilisation =
    2 M (2F) K / t over the dense bf16 peak."""
    rng = np.random.default_rng(5)
    st = hip.Stream()
    rows = 2 * F
    q = rng.integers(-127, 128, (rows, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, (rows, K // 32)).astype(np.float32)
    ncopy = n_copies(rows * K, lo=2, hi=16)
    dq, ds = dev_copies(hip, q, ncopy), dev_copies(hip, s, ncopy)
    dz = tile_major(hip, dq, ds, 32, F, K, halves=2)
    free_all(dq + ds)
    x = hip.DeviceBuffer.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
    nw = hip.DeviceBuffer.from_numpy((rng.standard_normal(K) * 0.02).astype(np.float32))
    y = hip.DeviceBuffer(M * F * 4)
    nwork = hip.lib().qlm_matmul_i8_workspace_bytes(M, F, K, 2)
    work = hip.DeviceBuffer(nwork)

    def launch(i):
        qz, sz = dz[i % ncopy]
        hip.call("qlm_matmul_i8_tm", x, K, nw, 1e-6, qz, sz, 32, y, F, M, F, K, 2, work, nwork,
                 st.ptr)

    us = graph_time(hip, st, launch, ncopy, launches=40)
    flops = 2.0 * M * rows * K
    free_all([t for pair in dz for t in pair] + [x, nw, y, work])
    r = {"rows": M, "N": rows, "K": K,
         "kernel": "qlm_matmul_i8_tm (RMSNorm + gate/up + SwiGLU, tile-major weights)",
         "us": round(us, 1), "TFLOPs": round(flops / us / 1e6, 1),
         "mfma_util": round(flops / (us * 1e-6) / BF16_PEAK_FLOPS, 4)}
    log(f"prefill gate/up matmul M={M}: {us:.1f} us, {r['TFLOPs']} TFLOP/s, util "
        f"{r['mfma_util']:.3f}")
    return r


def linear_params_4b():
    """Weights of the 4B hybrid's linear layers (every projection but the
    lm_head): what a prefill row multiplies."""
    H, F, nh, d, nq, nkv, hd = 2560, 9728, 16, 128, 16, 4, 128
    mlp = 2 * F * H + H * F
    dn = (4 * nh * d + 2 * nh) * H + H * nh * d + mlp
    at = (2 * nq * hd + 2 * nkv * hd) * H + H * nq * hd + mlp
    return 27 * dn + 9 * at


# ------------------------------------------------------------ dominant kernel
# The dominant kernel of the batch-1 decode step (about a third of the step):
# the fused RMSNorm + gate/up projection + SwiGLU GEMV of every layer, 4B
# shape (F = 9728 outputs from 2F = 19456 int8 rows of K = 2560, group-32
# scales), on the int8 matrix cores over tile-major weights.
DOM_F, DOM_K = 9728, 2560
DOM_NAME = ("k_gemv_mx<8, 2, 5, false, 1, 2, false> (RMSNorm + gate/up GEMV + SwiGLU on the int8 "
            "matrix cores, 19456x2560 int8 G=32, tile-major)")
PMC_FILE = os.path.join(ROOT, "profiles", "gemv_gate_up_4b_pmc.json")


def dominant_source_sha():
    """sha256 over the dominant kernel's source files, in order."""
    h = hashlib.sha256()
    for path in DOM_SOURCES:
        with open(path, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def dominant_bytes():
    """Algorithmic HBM bytes of one launch: int8 weights, group scales, x and
    the norm gain read once, the F outputs written once."""
    rows = 2 * DOM_F
    return rows * DOM_K + 4 * rows * (DOM_K // 32) + 4 * DOM_K + 4 * DOM_K + 4 * DOM_F


def measure_dominant(hip):
    """Average launch duration of the dominant kernel, HIP events recorded on
    the stream it is launched on (around graph replays of back-to-back
    launches), weights cycled over > 1 GiB of copies."""
    rng = np.random.default_rng(1)
    st = hip.Stream()
    rows, nb = 2 * DOM_F, DOM_K // 32
    q = rng.integers(-127, 128, (rows, DOM_K), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, (rows, nb)).astype(np.float32)
    dq1 = [hip.DeviceBuffer.from_numpy(q)]
    ds1 = [hip.DeviceBuffer.from_numpy(s)]
    qb, sb = C.c_size_t(), C.c_size_t()
    hip.check(hip.lib().qlm_mx_layout_bytes(DOM_F, DOM_K, 32, 2, C.byref(qb), C.byref(sb)))
    qz, sz = hip.DeviceBuffer(qb.value), hip.DeviceBuffer(sb.value)
    hip.call("qlm_mx_swizzle", dq1[0], ds1[0], 32, DOM_F, DOM_K, 2, qz, sz, None)
    hip.sync()
    free_all(dq1 + ds1)
    ncopy = n_copies(qb.value + sb.value, lo=2, hi=64)
    dz = [(qz, sz)] + [(hip.DeviceBuffer(qb.value), hip.DeviceBuffer(sb.value))
                       for _ in range(ncopy - 1)]
    for a, b in dz[1:]:
        hip.check(hip.lib().qlm_memcpy_d2d(a.ptr, qz.ptr, qb.value, None))
        hip.check(hip.lib().qlm_memcpy_d2d(b.ptr, sz.ptr, sb.value, None))
    hip.sync()
    x = hip.DeviceBuffer.from_numpy(rng.standard_normal(DOM_K).astype(np.float32))
    nw = hip.DeviceBuffer.from_numpy((rng.standard_normal(DOM_K) * 0.02).astype(np.float32))
    y = hip.DeviceBuffer(DOM_F * 4)

    def launch(i):
        a, b = dz[i % ncopy]
        hip.call("qlm_gemv_i8_mx", x, nw, 1e-6, a, b, 32, y, DOM_F, DOM_K, 2, st.ptr)

    us = graph_time(hip, st, launch, 4 * ncopy, launches=400)
    free_all([t for pair in dz for t in pair] + [x, nw, y])
    return us


def copy_calibration(hip, nbytes=256 << 20, reps=4):
    """A plain device-to-device copy of known size: the reference point for
    the FETCH_SIZE / WRITE_SIZE counters (profiled with --kernel-only)."""
    a, b = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    a.zero()
    for _ in range(reps):
        hip.check(hip.lib().qlm_memcpy_d2d(b.ptr, a.ptr, nbytes, None))
    hip.sync()
    free_all([a, b])


# ------------------------------------------------------------ decode runs
def run_decode(eng, prompts, warmup, steps, graph=True):
    """Batched prefill of positions 0..n-2, warmup, then exactly `steps` timed
    decode steps (HIP events on the engine stream, device synchronised on
    both sides)."""
    from quicklm_amd import hip

    B, n = prompts.shape
    prefill_s = eng.start(prompts, batched_prefill=True)
    if warmup:
        eng.steps(warmup, graph)
    hip.sync()
    t1 = time.perf_counter()
    gpu_ms = eng.steps(steps, graph)
    hip.sync()
    wall_s = time.perf_counter() - t1
    toks = np.stack([eng.tokens(b, n, warmup + steps) for b in range(B)])
    return {"batch": B, "prefill_s": round(prefill_s, 4), "gpu_ms": gpu_ms, "wall_s": wall_s,
            "ms_per_step": gpu_ms / steps, "tok_s": B * steps / (gpu_ms / 1000.0),
            "tokens": toks}


def ieee_parity(eng, prompts, batch):
    """Greedy streams against the reference's IEEE build on the same
    checkpoint and prompts (committed fixtures: sequences 0 and 1 of the
    batch, 256 steps each), from generate runs of their own outside the timed
    region: each sequence at batch 1, and rows 0 and 1 of a batch-`batch`
    run. Per stream: the length of the prefix equal to the reference's and
    the reference's top-2 margin where it first differs."""
    gold = []
    for k, path in ((0, GOLDEN_4B), (1, GOLDEN_4B_SEQ1)):
        if not os.path.exists(path):
            continue
        g = np.load(path)
        if prompts.shape[1] != len(g["prompt"]) or not np.array_equal(prompts[k], g["prompt"]):
            return {"note": "prompts differ from the fixtures' (non-default --prompt-len)"}
        gold.append((k, g))
    if not gold:
        return None

    def cmp(got, g):
        ref = g["tokens"]
        diff = np.nonzero(got[:len(ref)] != ref)[0]
        first = int(diff[0]) if diff.size else int(len(ref))
        return {"steps_compared": int(len(ref)), "match_prefix": first,
                "margin_at_divergence": float(g["margin"][first]) if first < len(ref) else None,
                "min_margin_in_prefix": float(g["margin"][:first].min()) if first else None}

    res = {"reference": "reference sources built with IEEE flags, same checkpoint and prompts "
                        "(tests/golden/4b_greedy.npz, 4b_greedy_seq1.npz)", "batch1": {},
           "batch" + str(batch): {}}
    n = max(len(g["tokens"]) for _, g in gold)
    for k, g in gold:
        out, _, _ = eng.generate(prompts[k:k + 1], n)
        res["batch1"][f"seq{k}"] = cmp(out[0], g)
    if batch > 1:
        out, _, _ = eng.generate(prompts[:batch], n)
        for k, g in gold:
            res["batch" + str(batch)][f"seq{k}"] = cmp(out[k], g)
    g0 = gold[0][1]
    fd = np.nonzero(g0["tokens_fast"] != g0["tokens"])[0]
    res["reference_fast_math_matches_ieee_prefix"] = int(fd[0]) if fd.size else len(fd)
    return res


def run_spec(target, draft, prompt, n_new, K, name):
    """One session turn: prefill the prompt on both models, then n_new tokens
    by speculative rounds; also the plain greedy stream for comparison."""
    from quicklm_amd.engine import Session

    s = Session(target, draft, draft_tokens=K)
    out, info = s.turn(prompt, n_new)
    s.close()
    p = Session(target)
    plain, pinfo = p.turn(prompt, n_new)
    p.close()
    return {"target": name, "draft": "int4", "draft_tokens": K, "tokens": int(len(out)),
            "tok_s": round(len(out) / info["decode_s"], 2),
            "decode_s": round(info["decode_s"], 4), "rounds": info["rounds"],
            "drafted": info["drafted"], "accepted": info["accepted"],
            "rejections": info["rejections"],
            "plain_session_tok_s": round(len(plain) / pinfo["decode_s"], 2),
            "matches_plain_greedy": bool(np.array_equal(out, plain))}


# ------------------------------------------------------------ CPU baseline
def host_cpus():
    """Physical cores of this process's CPU set (one logical CPU each, SMT
    siblings left out) and what lscpu says about the host."""
    cpus = sorted(os.sched_getaffinity(0))
    seen, phys = set(), []
    for c in cpus:
        base = f"/sys/devices/system/cpu/cpu{c}/topology/"
        try:
            key = (open(base + "physical_package_id").read().strip(),
                   open(base + "core_id").read().strip())
        except OSError:
            key = ("?", str(c))
        if key not in seen:
            seen.add(key)
            phys.append(c)
    info = {"logical_cpus_in_affinity": len(cpus), "physical_cores_in_affinity": len(phys)}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = dict(l.split(":", 1) for l in out.splitlines() if ":" in l)
        kv = {k.strip(): v.strip() for k, v in kv.items()}
        info.update({"model": kv.get("Model name"), "sockets": kv.get("Socket(s)"),
                     "threads_per_core": kv.get("Thread(s) per core"),
                     "numa_nodes": kv.get("NUMA node(s)")})
    except (OSError, subprocess.SubprocessError):
        pass
    tpc = info.get("threads_per_core")
    info["smt"] = "off" if tpc == "1" else f"on ({tpc} threads per core; one per core used)"
    return phys, info


def cpu_baseline(model_dir, prompt, n_prompt, n_decode):
    """The reference QuickLM CPU path (its own sources, -O3 -ffast-math) on the
    same checkpoint: batched prefill of n_prompt-1 ids, then n_decode greedy
    steps; decode tokens/s as the reference CLI reports it (main.cpp:686-690).
    One thread per physical core of this process's CPU set, pinned there."""
    from oracle.oracle import Reference

    phys, info = host_cpus()
    os.sched_setaffinity(0, phys)
    ref = Reference("fast")
    ref.init_threads(len(phys))
    t0 = time.perf_counter()
    m = ref.load_model(model_dir, n_prompt + n_decode + 8, "int8")
    load_s = time.perf_counter() - t0
    toks, pre, dec, _ = m.generate(prompt[:n_prompt], n_decode)
    del m
    numa = info.get("numa_nodes")
    return {"value": round(n_decode / dec, 3), "unit": "tokens/s", "cores": len(phys),
            "kind": "reference", "build": f"reference sources, -O3 -ffast-math -march=x86-64-"
                                           f"{ref.kind}",
            "host": dict(info, numa_binding="single NUMA node: none needed" if numa == "1"
                         else "threads pinned to the affinity set's physical cores"),
            "load_s": round(load_s, 1), "prefill_s": round(pre, 2), "decode_s": round(dec, 2),
            "tokens": toks}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt-len", type=int, default=2048)
    ap.add_argument("--batch", type=int, default=16, help="second batch size (0 to skip)")
    ap.add_argument("--cpu-prompt", type=int, default=2048,
                    help="prompt ids of the CPU baseline (a prefix of the benchmark prompt; its "
                         "first n-1 are prefilled untimed)")
    ap.add_argument("--cpu-decode", type=int, default=64)
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant-kernel timing and the copy of known size (for "
                         "rocprofv3 --pmc passes)")
    ap.add_argument("--section", choices=["config1", "config2", "config3", "prefill"],
                    help="run only this isolated-kernel section and print its results (for "
                         "rocprofv3 kernel traces of one workload)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-kernels", action="store_true",
                    help="skip the isolated-kernel sections (config 1-3, prefill matmul)")
    ap.add_argument("--skip-int4", action="store_true",
                    help="skip the batch-1 decode at --precision int4")
    ap.add_argument("--skip-native", action="store_true",
                    help="skip the batch-1 decode at --precision bf16 (weights as stored)")
    ap.add_argument("--spec", action="store_true",
                    help="also run speculative sessions (int4 draft, K = --draft-tokens)")
    ap.add_argument("--draft-tokens", type=int, default=4)
    ap.add_argument("--skip-parity", action="store_true",
                    help="skip the full-length parity runs against the reference's streams "
                         "(for kernel traces of the timed steps)")
    ap.add_argument("--skip-row", action="store_true",
                    help="skip the batch-1 decode with one scale per output row (int8_row)")
    ap.add_argument("--model-dir", default=None)
    ap.add_argument("--eager", action="store_true",
                    help="launch each step's kernels directly instead of replaying the "
                         "captured hipGraph (for tracers that cannot follow graphs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the decode path is built for a single MI355X)", file=sys.stderr)
        sys.exit(2)

    from quicklm_amd import hip, synth
    from quicklm_amd.engine import Engine

    if hip.device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    hip.check(hip.lib().qlm_set_device(0))
    log("device", hip.device_name())

    if args.section:
        fn = {"config1": bench_config1, "config2": bench_config2, "config3": bench_config3,
              "prefill": bench_prefill_matmul}[args.section]
        print(json.dumps({args.section: fn(hip)}), flush=True)
        return

    if args.kernel_only:
        us = measure_dominant(hip)
        copy_calibration(hip)
        b = dominant_bytes()
        print(json.dumps({"kernel": DOM_NAME, "us_per_launch": round(us, 3), "bytes": b,
                          "GBps": round(b / us / 1e3, 1)}), flush=True)
        return

    result = {"metric": METRIC}
    base = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    own_dir = args.model_dir is None
    mdir = args.model_dir or tempfile.mkdtemp(prefix="qlm_4b_", dir=base)
    spec = []
    try:
        t0 = time.perf_counter()
        if own_dir:
            synth.write_model(mdir, "4b")
        log(f"4B checkpoint written in {time.perf_counter() - t0:.1f}s ({mdir})")
        # room for the parity runs' 256 steps after the prompt too
        max_seq = args.prompt_len + max(args.warmup + args.steps, 256) + 8
        Bmax = max(1, args.batch)
        t0 = time.perf_counter()
        eng = Engine(mdir, max_seq_len=max_seq, max_batch=Bmax, precision="int8")
        log(f"engine load + device quantisation {time.perf_counter() - t0:.1f}s, "
            f"{eng.weight_bytes / 1e9:.3f} GB of int8 weights+scales")
        prompts = synth.prompt_tokens(args.prompt_len, seed=4, batch=max(2, Bmax))
        graph = not args.eager
        r1 = run_decode(eng, prompts[:1], args.warmup, args.steps, graph)
        log(f"batch 1: {r1['tok_s']:.1f} tok/s ({r1['ms_per_step']:.3f} ms/step), prefill "
            f"{r1['prefill_s']:.3f}s, kernels/step {eng.kernels_per_step()}")
        rB = None
        if args.batch > 1:
            rB = run_decode(eng, prompts[:args.batch], args.warmup, args.steps, graph)
            log(f"batch {args.batch}: {rB['tok_s']:.1f} tok/s ({rB['ms_per_step']:.3f} ms/step)")
            a0, b0 = rB["tokens"][0], r1["tokens"][0]
            same = len(a0) if np.array_equal(a0, b0) else int(np.argmax(a0 != b0))
            rB["row0_matches_batch1"] = same
            log(f"batch row 0 matches the batch-1 stream for {same}/{len(a0)} tokens")
        parity = None if args.skip_parity else ieee_parity(eng, prompts, args.batch)
        if parity:
            log(f"IEEE reference parity: {parity}")

        cpu = None
        if not args.skip_cpu:
            cpu = cpu_baseline(mdir, prompts[0], args.cpu_prompt, args.cpu_decode)
            # the same prompt on the GPU: the fast-math build's stream beside it
            g, _, _ = eng.generate(prompts[:1, :args.cpu_prompt], args.cpu_decode)
            match = int(np.argmax(g[0] != cpu["tokens"])) if not np.array_equal(
                g[0], cpu["tokens"]) else args.cpu_decode
            cpu["gpu_tokens_match_prefix_fast_math"] = match
            log(f"cpu baseline {cpu['value']} tok/s on {cpu['cores']} cores "
                f"({cpu['host'].get('model')}); GPU stream matches the fast-math build for "
                f"{match}/{args.cpu_decode} tokens")
            cpu.pop("tokens")
        eng.close()

        rrow = None
        if not args.skip_row:
            erow = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="int8_row")
            rrow = run_decode(erow, prompts[:1], args.warmup, args.steps, graph)
            rrow["weight_bytes"] = erow.weight_bytes
            erow.close()
            log(f"batch 1, per-row scales: {rrow['tok_s']:.1f} tok/s "
                f"({rrow['ms_per_step']:.3f} ms/step), {rrow['weight_bytes'] / 1e9:.3f} GB")

        r4 = e4 = None
        if not args.skip_int4:
            e4 = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="int4")
            r4 = run_decode(e4, prompts[:1], args.warmup, args.steps, graph)
            r4["weight_bytes"] = e4.weight_bytes
            log(f"batch 1, int4 weights: {r4['tok_s']:.1f} tok/s "
                f"({r4['ms_per_step']:.3f} ms/step), {r4['weight_bytes'] / 1e9:.3f} GB")
        rn = en = None
        if not args.skip_native:
            en = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="bf16")
            rn = run_decode(en, prompts[:1], args.warmup, args.steps, graph)
            rn["weight_bytes"] = en.weight_bytes
            log(f"batch 1, native weights: {rn['tok_s']:.1f} tok/s "
                f"({rn['ms_per_step']:.3f} ms/step), {rn['weight_bytes'] / 1e9:.3f} GB, "
                f"prefill {rn['prefill_s']:.3f}s")
        if args.spec and e4 is not None:
            et = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="int8")
            targets = [("int8", et)] + ([("bf16", en)] if en is not None else [])
            for name, t_ in targets:
                spec.append(run_spec(t_, e4, prompts[0], args.steps, args.draft_tokens, name))
                log(f"speculative, target {name} + int4 draft: {spec[-1]['tok_s']:.1f} tok/s, "
                    f"accepted {spec[-1]['accepted']}/{spec[-1]['drafted']}")
            et.close()
        for e_ in (e4, en):
            if e_ is not None:
                e_.close()
    finally:
        if own_dir:
            import shutil

            shutil.rmtree(mdir, ignore_errors=True)

    kern = {}
    if not args.skip_kernels:
        kern["config1_gemv"] = bench_config1(hip)
        kern["config2_deltanet"] = bench_config2(hip)
        kern["config3_attention"] = bench_config3(hip)
        kern["prefill_gate_up"] = bench_prefill_matmul(hip)

    dom_us = measure_dominant(hip)
    dom_b = dominant_bytes()
    log(f"dominant kernel: {dom_us:.2f} us/launch, {dom_b / dom_us / 1e3:.0f} GB/s")
    wbytes = eng.weight_bytes
    step_s = r1["ms_per_step"] / 1000.0
    pf_flops = 2.0 * (args.prompt_len - 1) * linear_params_4b()

    def frac_w(r):
        return round(r["weight_bytes"] / (r["ms_per_step"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4)

    result.update({
        "value": round(r1["tok_s"], 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r1["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 weights, fp32 activations and accumulation",
        "data": "synthetic: seeded random-init weights of the 4B hybrid architecture, "
                "uniform random prompt ids",
        "config": {"workload": "4B-class hybrid int8 decode: 36 layers (27 Gated DeltaNet "
                               "16x128 + 9 GQA 16q/4kv x128), hidden 2560, FFN 9728, vocab "
                               "151936, tied embeddings; 2048-token prompt, greedy decode, "
                               "one hipGraph per step",
                   "batch": 1, "prompt_len": args.prompt_len, "scale_group": 32,
                   "launch": "eager" if args.eager else "hipGraph",
                   "weight_bytes": wbytes, "parallelism": "single GPU"},
        "parity": parity,
        "batch16": None if rB is None else {"tok_s": round(rB["tok_s"], 2),
                                            "ms_per_step": round(rB["ms_per_step"], 4),
                                            "batch": rB["batch"],
                                            "row0_matches_batch1_tokens":
                                                rB["row0_matches_batch1"]},
        "decode_roofline": {"bound": "hbm", "weight_bytes_per_step": wbytes,
                            "achieved": round(wbytes / step_s / 1e9, 1),
                            "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(wbytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
                            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / wbytes, 1)},
        "prefill": {"rows": args.prompt_len - 1, "batch": 1, "s": r1["prefill_s"],
                    "rows_per_s": round((args.prompt_len - 1) / r1["prefill_s"], 1),
                    "linear_flops": pf_flops,
                    "mfma_util_linear": round(pf_flops / r1["prefill_s"] / BF16_PEAK_FLOPS, 4),
                    "gate_up_matmul": kern.get("prefill_gate_up")},
        "per_row_scales": None if rrow is None else {
            "tok_s": round(rrow["tok_s"], 2), "ms_per_step": round(rrow["ms_per_step"], 4),
            "batch": 1, "scale_group": "row", "weight_bytes": rrow["weight_bytes"],
            "frac_of_weight_roofline": frac_w(rrow)},
        "int4": None if r4 is None else {
            "tok_s": round(r4["tok_s"], 2), "ms_per_step": round(r4["ms_per_step"], 4),
            "batch": 1, "precision": "int4 (Q4_0, group 32)", "weight_bytes": r4["weight_bytes"],
            "frac_of_weight_roofline": frac_w(r4),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / r4["weight_bytes"], 1)},
        "native": None if rn is None else {
            "tok_s": round(rn["tok_s"], 2), "ms_per_step": round(rn["ms_per_step"], 4),
            "prefill_s": round(rn["prefill_s"], 4),
            "batch": 1, "precision": "bf16 (weights as stored: bf16 linears, fp32 tied lm_head)",
            "weight_bytes": rn["weight_bytes"], "frac_of_weight_roofline": frac_w(rn),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / rn["weight_bytes"], 1)},
        "speculative": spec or None,
        "config1_gemv": kern.get("config1_gemv"),
        "config2_deltanet": kern.get("config2_deltanet"),
        "config3_attention": kern.get("config3_attention"),
    })
    traffic, traffic_src = None, None
    if os.path.exists(PMC_FILE):
        with open(PMC_FILE) as f:
            pmc = json.load(f)
        if pmc.get("bytes") == dom_b and pmc.get("kernel_source_sha256") == dominant_source_sha():
            traffic, traffic_src = pmc.get("traffic_bytes"), os.path.relpath(PMC_FILE, ROOT)
        else:
            log("PMC record is not of this build's dominant kernel (source hash differs): "
                "traffic left null")
    achieved = dom_b / dom_us / 1e3
    result["roofline"] = {"kernel": DOM_NAME, "bound": "hbm", "achieved": round(achieved, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                          "traffic_source": traffic_src, "bytes_per_launch": dom_b,
                          "us_per_launch": round(dom_us, 3), "launches_per_step": 36}
    if cpu:
        result["cpu_baseline"] = dict(cpu, sample=(
            f"4B checkpoint, batch 1: prefill (untimed) of the first {args.cpu_prompt - 1} ids "
            f"of the same 2048-token prompt, then {args.cpu_decode} greedy decode steps (timed) "
            f"at context {args.cpu_prompt}-{args.cpu_prompt + args.cpu_decode}"))
        if args.batch > 1:
            # the reference decodes one sequence at a time: a batch of B is B
            # sequential runs, B * n tokens in B times one run's decode time
            result["cpu_baseline"]["batch" + str(args.batch)] = {
                "value": cpu["value"], "unit": "tokens/s",
                "derivation": f"{args.batch} sequential single-sequence runs (the reference "
                              f"has no batched decode): {args.batch}x the tokens in "
                              f"{args.batch}x the time of the measured run above"}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
