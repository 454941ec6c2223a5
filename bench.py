#!/usr/bin/env python3
"""Benchmark: 4B-class int8 hybrid decode on one MI355X, plus the isolated
int8 GEMV, with the reference CPU path timed beside it.

Workload (one "step" = one greedy decode step of every sequence in the batch):
  4B-class hybrid LM, 36 layers (27 Gated DeltaNet + 9 GQA), hidden 2560,
  FFN 9728, vocab 151936, seeded random-init weights quantised to int8 at load
  (Q8_0 group-32 scales, the reference's format), 2048-token uniform random
  prompts (batched prefill of positions 0..2046, untimed), greedy decode; the
  whole step is one replayed hipGraph.
  `value` = batch-1 decode tokens/s over exactly --steps timed steps after
  --warmup untimed steps; batch 16 is reported beside it. The GEMV section
  times the config-1 matrices in isolation (M <= 4: GEMV, M > 4: matrix cores).
  `roofline` is the dominant decode kernel (the fused RMSNorm + gate/up GEMV +
  SwiGLU, 36 launches per step) timed with HIP events on its own stream.
  `cpu_baseline` is the reference's own sources built with its release flags
  on this host's cores, on a bounded sample of the same 4B workload.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 8] [--kernel-only]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_FLOPS = 2.5e15  # dense bf16 matrix-core peak of MI355X
METRIC = "decode tokens/sec at batch 1 and 16 (4B int8); int8 GEMV achieved HBM GB/s"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def gemv_bytes(N, K, M, group):
    nb = 1 if group == K else K // group
    return N * K + 4 * N * nb + 4 * M * K + 4 * M * N


def bench_gemv(hip, shapes, Ms, group_kind, iters=100, pool_bytes=2 << 30):
    """Config-1 GEMV: y = x (q s)^T with W int8 U{-127..127}, s U(0.001,0.01),
    x N(0,1). Weights are cycled over copies totalling > 2 GiB so every launch
    streams from HBM (the 256 MB last-level cache cannot hold them)."""
    rng = np.random.default_rng(0)
    st = hip.Stream()
    out = []
    for (N, K) in shapes:
        group = K if group_kind == "row" else 32
        nb = 1 if group == K else K // group
        wb = N * K + 4 * N * nb
        ncopy = int(max(2, min(48, pool_bytes // wb)))
        q = rng.integers(-127, 128, (N, K), dtype=np.int8)
        s = rng.uniform(0.001, 0.01, (N, nb)).astype(np.float32)
        dq = [hip.DeviceBuffer.from_numpy(q) for _ in range(ncopy)]
        ds = [hip.DeviceBuffer.from_numpy(s) for _ in range(ncopy)]
        dz = _tile_major(hip, dq, ds, group, N, K, 1)
        for M in Ms:
            x = hip.DeviceBuffer.from_numpy(rng.standard_normal((M, K)).astype(np.float32))
            y = hip.DeviceBuffer(M * N * 4)
            n_it = iters if M <= 4 else max(10, iters // 4)
            # M <= 4: the GEMV; M > 4: the matrix-core matmul (one weight pass)
            fn = "qlm_gemv_i8" if M <= 4 else "qlm_matmul_i8"
            nwork = hip.lib().qlm_matmul_i8_workspace_bytes(M, N, K, 0)
            work = hip.DeviceBuffer(nwork)

            def launch(i):
                if M <= 4:
                    hip.call(fn, x, K, dq[i % ncopy], ds[i % ncopy], group, y, N, M, N, K, st.ptr)
                else:
                    hip.call(fn, x, K, None, 0.0, dq[i % ncopy], ds[i % ncopy], group, y, N, M,
                             N, K, 0, work, nwork, st.ptr)

            for i in range(ncopy):
                launch(i)
            e0, e1 = hip.Event(), hip.Event()
            e0.record(st.ptr)
            for i in range(n_it):
                launch(i)
            e1.record(st.ptr)
            us = e0.elapsed_ms(e1) * 1000.0 / n_it
            b = gemv_bytes(N, K, M, group)
            r = {"N": N, "K": K, "M": M, "group": group, "kernel": fn, "us": round(us, 2),
                 "GBps": round(b / us / 1e3, 1), "bytes": b,
                 "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
            if M > 4:
                # algorithmic flops over the dense bf16 matrix-core peak
                r["mfma_util"] = round(2.0 * M * N * K / (us * 1e-6) / BF16_PEAK_FLOPS, 5)
            out.append(r)
            log(f"gemv {N}x{K} M={M} G={group}: {us:.1f} us {b / us / 1e3:.0f} GB/s")
            if M == 1 and dz:
                # the same product on the matrix cores over tile-major weights
                def launch_mx(i):
                    qz, sz = dz[i % ncopy]
                    hip.call("qlm_gemv_i8_mx", x, None, 0.0, qz, sz, group, y, N, K, 0, st.ptr)

                for i in range(ncopy):
                    launch_mx(i)
                e0, e1 = hip.Event(), hip.Event()
                e0.record(st.ptr)
                for i in range(n_it):
                    launch_mx(i)
                e1.record(st.ptr)
                us = e0.elapsed_ms(e1) * 1000.0 / n_it
                out.append({"N": N, "K": K, "M": M, "group": group, "kernel": "qlm_gemv_i8_mx",
                            "layout": "tile-major", "us": round(us, 2),
                            "GBps": round(b / us / 1e3, 1), "bytes": b,
                            "frac_hbm": round(b / us / 1e3 / HBM_PEAK_GBS, 4)})
                log(f"gemv_mx {N}x{K} M=1 G={group}: {us:.1f} us {b / us / 1e3:.0f} GB/s")
            x.free()
            y.free()
            work.free()
        for b_ in dq + ds + [t for pair in dz for t in pair if t not in ds]:
            b_.free()
    return out


def _tile_major(hip, dq, ds, group, rows, K, halves):
    """Tile-major copies (qlm_mx_swizzle) of each weight copy; [] when K has
    no matrix-core launch shape. Per-row scales keep their layout."""
    import ctypes as C

    qb, sb = C.c_size_t(), C.c_size_t()
    if hip.lib().qlm_mx_layout_bytes(rows, K, group, halves, C.byref(qb), C.byref(sb)) != 0:
        return []
    out = []
    for q_, s_ in zip(dq, ds):
        qz = hip.DeviceBuffer(qb.value)
        sz = hip.DeviceBuffer(sb.value) if sb.value else s_
        hip.call("qlm_mx_swizzle", q_, s_, group, rows, K, halves, qz,
                 sz if sb.value else None, None)
        out.append((qz, sz))
    hip.sync()
    return out


# The dominant kernel of the batch-1 decode step (about a third of the step):
# the fused RMSNorm + gate/up projection + SwiGLU GEMV of every layer, 4B
# shape (F = 9728 outputs from 2F = 19456 int8 rows of K = 2560, group-32
# scales), on the int8 matrix cores over tile-major weights.
DOM_F, DOM_K = 9728, 2560
DOM_NAME = ("k_gemv_mx<8, 2, 5, false, 1, 2, false> (RMSNorm + gate/up GEMV + SwiGLU on the int8 "
            "matrix cores, 19456x2560 int8 G=32, tile-major)")
PMC_FILE = os.path.join(ROOT, "profiles", "gemv_gate_up_4b_pmc.json")


def dominant_bytes():
    """Algorithmic HBM bytes of one launch: int8 weights, group scales, x and
    the norm gain read once, the F outputs written once."""
    rows = 2 * DOM_F
    return rows * DOM_K + 4 * rows * (DOM_K // 32) + 4 * DOM_K + 4 * DOM_K + 4 * DOM_F


def measure_dominant(hip, launches=400, pool_bytes=2 << 30):
    """Average launch duration of the dominant kernel, HIP events recorded on
    the stream it is launched on (around graph replays of back-to-back
    launches), weights cycled over > 2 GiB of copies so every launch streams
    them from HBM (not the 256 MB last-level cache)."""
    rng = np.random.default_rng(1)
    st = hip.Stream()
    rows, nb = 2 * DOM_F, DOM_K // 32
    wb = rows * DOM_K + 4 * rows * nb
    ncopy = int(max(2, min(64, pool_bytes // wb)))
    q = rng.integers(-127, 128, (rows, DOM_K), dtype=np.int8)
    s = rng.uniform(0.001, 0.01, (rows, nb)).astype(np.float32)
    dq1 = [hip.DeviceBuffer.from_numpy(q)]
    ds1 = [hip.DeviceBuffer.from_numpy(s)]
    z = _tile_major(hip, dq1, ds1, 32, DOM_F, DOM_K, 2)[0]
    dq1[0].free()
    ds1[0].free()
    # ncopy tile-major copies: the first swizzled, the rest device copies of it
    dz = [z] + [(hip.DeviceBuffer(z[0].nbytes), hip.DeviceBuffer(z[1].nbytes))
                for _ in range(ncopy - 1)]
    for qz, sz in dz[1:]:
        hip.check(hip.lib().qlm_memcpy_d2d(qz.ptr, z[0].ptr, z[0].nbytes, None))
        hip.check(hip.lib().qlm_memcpy_d2d(sz.ptr, z[1].ptr, z[1].nbytes, None))
    hip.sync()
    x = hip.DeviceBuffer.from_numpy(rng.standard_normal(DOM_K).astype(np.float32))
    nw = hip.DeviceBuffer.from_numpy((rng.standard_normal(DOM_K) * 0.02).astype(np.float32))
    y = hip.DeviceBuffer(DOM_F * 4)

    def launch(i):
        qz, sz = dz[i % ncopy]
        hip.call("qlm_gemv_i8_mx", x, nw, 1e-6, qz, sz, 32, y, DOM_F, DOM_K, 2, st.ptr)

    # launched as in the decode step: back-to-back kernels replayed from one
    # captured graph (no host launch gaps between them)
    import ctypes as C

    lib = hip.lib()
    for i in range(ncopy):
        launch(i)
    per = 4 * ncopy
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
    us = e0.elapsed_ms(e1) * 1000.0 / (reps * per)
    hip.check(lib.qlm_graph_destroy(g))
    for b_ in [t for pair in dz for t in pair] + [x, nw, y]:
        b_.free()
    return us


def copy_calibration(hip, nbytes=256 << 20, reps=4):
    """A plain device-to-device copy of known size: the reference point for
    the FETCH_SIZE / WRITE_SIZE counters (profiled with --kernel-only)."""
    a, b = hip.DeviceBuffer(nbytes), hip.DeviceBuffer(nbytes)
    a.zero()
    for _ in range(reps):
        hip.check(hip.lib().qlm_memcpy_d2d(b.ptr, a.ptr, nbytes, None))
    hip.sync()
    a.free()
    b.free()


def run_decode(eng, prompts, warmup, steps, graph=True):
    """Batched prefill of positions 0..n-2, warmup, then exactly `steps` timed
    decode steps."""
    B, n = prompts.shape
    prefill_s = eng.start(prompts, batched_prefill=True)
    if warmup:
        eng.steps(warmup, graph)
    from quicklm_amd import hip

    hip.sync()
    t1 = time.perf_counter()
    gpu_ms = eng.steps(steps, graph)
    hip.sync()
    wall_s = time.perf_counter() - t1
    toks = np.stack([eng.tokens(b, n, warmup + steps) for b in range(B)])
    return {"batch": B, "prefill_s": round(prefill_s, 3), "gpu_ms": gpu_ms, "wall_s": wall_s,
            "ms_per_step": gpu_ms / steps, "tok_s": B * steps / (gpu_ms / 1000.0),
            "tokens": toks}


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


def cpu_baseline(model_dir, prompt, n_prompt, n_decode, threads):
    """The reference QuickLM CPU path (its own sources, -O3 -ffast-math) on the
    same checkpoint: batched prefill of n_prompt-1 ids, then n_decode greedy
    steps; decode tokens/s as the reference CLI reports it (main.cpp:686-690)."""
    from oracle.oracle import Reference

    ref = Reference("fast")
    ref.init_threads(threads)
    t0 = time.perf_counter()
    m = ref.load_model(model_dir, n_prompt + n_decode + 8, "int8")
    load_s = time.perf_counter() - t0
    toks, pre, dec, _ = m.generate(prompt[:n_prompt], n_decode)
    del m
    return {"value": round(n_decode / dec, 3), "unit": "tokens/s", "cores": threads,
            "kind": "reference", "build": f"reference sources, -O3 -ffast-math -march=x86-64-"
                                           f"{ref.kind}", "load_s": round(load_s, 1),
            "prefill_s": round(pre, 2), "decode_s": round(dec, 2), "tokens": toks}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt-len", type=int, default=2048)
    ap.add_argument("--batch", type=int, default=16, help="second batch size (0 to skip)")
    ap.add_argument("--cpu-prompt", type=int, default=128)
    ap.add_argument("--cpu-decode", type=int, default=256)
    ap.add_argument("--kernel-only", action="store_true",
                    help="only the dominant-kernel timing and the copy of known size (for "
                         "rocprofv3 --pmc passes)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-gemv", action="store_true")
    ap.add_argument("--skip-int4", action="store_true",
                    help="skip the batch-1 decode at --precision int4")
    ap.add_argument("--skip-native", action="store_true",
                    help="skip the batch-1 decode at --precision bf16 (weights as stored)")
    ap.add_argument("--skip-spec", action="store_true",
                    help="skip the speculative sessions (int4 draft, K = --draft-tokens)")
    ap.add_argument("--draft-tokens", type=int, default=4)
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

    if args.kernel_only:
        us = measure_dominant(hip)
        copy_calibration(hip)
        b = dominant_bytes()
        print(json.dumps({"kernel": DOM_NAME, "us_per_launch": round(us, 3), "bytes": b,
                          "GBps": round(b / us / 1e3, 1)}), flush=True)
        return

    result = {"metric": METRIC}
    gemv = []
    if not args.skip_gemv:
        shapes = [(4096, 4096), (12288, 4096), (4096, 12288), (151936, 2560)]
        gemv = bench_gemv(hip, shapes, [1, 4, 16, 64], "row")
        gemv += bench_gemv(hip, [(151936, 2560)], [1], "g32")

    base = "/dev/shm" if os.path.isdir("/dev/shm") else tempfile.gettempdir()
    own_dir = args.model_dir is None
    mdir = args.model_dir or tempfile.mkdtemp(prefix="qlm_4b_", dir=base)
    try:
        t0 = time.perf_counter()
        if own_dir:
            synth.write_model(mdir, "4b")
        log(f"4B checkpoint written in {time.perf_counter() - t0:.1f}s ({mdir})")
        max_seq = args.prompt_len + args.warmup + args.steps
        Bmax = max(1, args.batch)
        t0 = time.perf_counter()
        eng = Engine(mdir, max_seq_len=max_seq, max_batch=Bmax, precision="int8")
        log(f"engine load + device quantisation {time.perf_counter() - t0:.1f}s, "
            f"{eng.weight_bytes / 1e9:.3f} GB of int8 weights+scales")
        prompts = synth.prompt_tokens(args.prompt_len, seed=4, batch=Bmax)
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
            log(f"batch row 0 matches the batch-1 stream for {same}/{len(a0)} tokens "
                "(matrix-core vs GEMV rounding)")

        cpu = None
        if not args.skip_cpu:
            threads = min(16, os.cpu_count() or 1)
            cpu = cpu_baseline(mdir, prompts[0], args.cpu_prompt, args.cpu_decode, threads)
            # same short prompt on the GPU for a token-stream check at 4B scale
            g, _, _ = eng.generate(prompts[:1, :args.cpu_prompt], args.cpu_decode)
            match = int(np.argmax(g[0] != cpu["tokens"])) if not np.array_equal(
                g[0], cpu["tokens"]) else args.cpu_decode
            cpu["gpu_tokens_match_prefix"] = match
            log(f"cpu baseline {cpu['value']} tok/s on {threads} threads; GPU stream matches "
                f"the reference for {match}/{args.cpu_decode} tokens")
            cpu.pop("tokens")
        eng.close()

        rrow = None
        if not args.skip_row:
            # the same checkpoint quantised with one fp32 scale per output row
            erow = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="int8_row")
            rrow = run_decode(erow, prompts[:1], args.warmup, args.steps, graph)
            rrow["weight_bytes"] = erow.weight_bytes
            erow.close()
            log(f"batch 1, per-row scales: {rrow['tok_s']:.1f} tok/s "
                f"({rrow['ms_per_step']:.3f} ms/step), {rrow['weight_bytes'] / 1e9:.3f} GB")

        r4 = None
        if not args.skip_int4:
            # the same checkpoint at --precision int4 (Q4_0 weights, lm_head included)
            e4 = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="int4")
            r4 = run_decode(e4, prompts[:1], args.warmup, args.steps, graph)
            r4["weight_bytes"] = e4.weight_bytes
            if args.skip_spec:
                e4.close()
            log(f"batch 1, int4 weights: {r4['tok_s']:.1f} tok/s "
                f"({r4['ms_per_step']:.3f} ms/step), {r4['weight_bytes'] / 1e9:.3f} GB")
        rn = None
        if not args.skip_native:
            # the same checkpoint at --precision bf16, the reference's default:
            # linears as stored (bf16), tied lm_head = the fp32 embedding table
            en = Engine(mdir, max_seq_len=max_seq, max_batch=1, precision="bf16")
            rn = run_decode(en, prompts[:1], args.warmup, args.steps, graph)
            rn["weight_bytes"] = en.weight_bytes
            log(f"batch 1, native weights: {rn['tok_s']:.1f} tok/s "
                f"({rn['ms_per_step']:.3f} ms/step), {rn['weight_bytes'] / 1e9:.3f} GB, "
                f"prefill {rn['prefill_s']:.3f}s")

        spec = []
        if not args.skip_spec and not args.skip_int4:
            # the reference's default decode: the same checkpoint at int4 drafts
            # K tokens per round for the target (main.cpp:166-172, :366-394)
            targets = [("int8", Engine(mdir, max_seq_len=max_seq, max_batch=1,
                                       precision="int8"))]
            if rn is not None:
                targets.append(("bf16", en))
            for name, et in targets:
                spec.append(run_spec(et, e4, prompts[0], args.steps, args.draft_tokens, name))
                log(f"speculative, target {name} + int4 draft, K={args.draft_tokens}: "
                    f"{spec[-1]['tok_s']:.1f} tok/s, accepted {spec[-1]['accepted']}/"
                    f"{spec[-1]['drafted']} drafted, stream equals plain greedy: "
                    f"{spec[-1]['matches_plain_greedy']}")
            targets[0][1].close()
        if rn is not None:
            en.close()
        if r4 is not None and not args.skip_spec:
            e4.close()
    finally:
        if own_dir:
            import shutil

            shutil.rmtree(mdir, ignore_errors=True)

    dom_us = measure_dominant(hip)
    dom_b = dominant_bytes()
    log(f"dominant kernel: {dom_us:.2f} us/launch, {dom_b / dom_us / 1e3:.0f} GB/s")
    wbytes = eng.weight_bytes
    step_s = r1["ms_per_step"] / 1000.0
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
        "per_row_scales": None if rrow is None else {
            "tok_s": round(rrow["tok_s"], 2), "ms_per_step": round(rrow["ms_per_step"], 4),
            "batch": 1, "scale_group": "row", "weight_bytes": rrow["weight_bytes"],
            "frac_of_weight_roofline": round(
                rrow["weight_bytes"] / (rrow["ms_per_step"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4)},
        "int4": None if r4 is None else {
            "tok_s": round(r4["tok_s"], 2), "ms_per_step": round(r4["ms_per_step"], 4),
            "batch": 1, "precision": "int4 (Q4_0, group 32)", "weight_bytes": r4["weight_bytes"],
            "frac_of_weight_roofline": round(
                r4["weight_bytes"] / (r4["ms_per_step"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / r4["weight_bytes"], 1)},
        "native": None if rn is None else {
            "tok_s": round(rn["tok_s"], 2), "ms_per_step": round(rn["ms_per_step"], 4),
            "prefill_s": round(rn["prefill_s"], 4),
            "batch": 1, "precision": "bf16 (weights as stored: bf16 linears, fp32 tied lm_head)",
            "weight_bytes": rn["weight_bytes"],
            "frac_of_weight_roofline": round(
                rn["weight_bytes"] / (rn["ms_per_step"] / 1000.0) / 1e9 / HBM_PEAK_GBS, 4),
            "roofline_tok_s": round(HBM_PEAK_GBS * 1e9 / rn["weight_bytes"], 1)},
        "speculative": spec or None,
        "gemv": gemv,
    })
    traffic, traffic_src = None, None
    if os.path.exists(PMC_FILE):
        with open(PMC_FILE) as f:
            pmc = json.load(f)
        if pmc.get("bytes") == dom_b:
            traffic, traffic_src = pmc.get("traffic_bytes"), os.path.relpath(PMC_FILE, ROOT)
    achieved = dom_b / dom_us / 1e3
    result["roofline"] = {"kernel": DOM_NAME, "bound": "hbm", "achieved": round(achieved, 1),
                          "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                          "traffic_source": traffic_src, "bytes_per_launch": dom_b,
                          "us_per_launch": round(dom_us, 3), "launches_per_step": 36}
    if cpu:
        result["cpu_baseline"] = dict(cpu, sample=(
            f"4B checkpoint, batch 1: prefill of {args.cpu_prompt - 1} prompt ids "
            f"(untimed), then {args.cpu_decode} greedy decode steps (timed)"))
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
