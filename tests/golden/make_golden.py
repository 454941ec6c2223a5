"""Write the committed golden fixtures for the model-level parity tests.

Runs in the build container only (it needs the reference compiled from its
own sources into oracle/_ref by `make -C oracle ref`). It writes the tiny
hybrid model (config 0 shapes) with quicklm_amd.synth, runs the reference
DecoderModel on it with the CLI's greedy convention (batched prefill of
prompt[0..126], 64 decode steps, no EOS stop) and stores:
  prompt, tokens                 the 128 prompt ids and 64 greedy tokens
  top_idx/top_val [64, 32]       the 32 largest logits of every decode step
  margin [64]                    top-1 minus top-2 logit per step
  logits0_head/logits63_head     logits[:4096] of the first and last step
  tensor_sha                     sha256 of a few synthetic tensors (pins the
                                 generator across hosts)
plus the same stream from the reference's own -O3 -ffast-math build
(tokens_fast) for the record; and tiny_greedy_int4.npz, the IEEE build's
run of the same prompt at --precision int4 (prompt, tokens, top_idx,
top_val, margin, logits0_head). Usage: python tests/golden/make_golden.py
[--int4 | --native | --4b (those fixtures only)]; tiny_greedy_native.npz and
micro_greedy_native.npz are the --precision bf16 runs (weights in their
checkpoint dtype: fp32 for the tiny model, bf16 for the micro one);
4b_greedy.npz is the 4B-class int8 model (2048-token prompt, 256 greedy
steps: the decode length of the 4B workload) and 4b_greedy_seq1.npz the same
for the second sequence of that workload's batch, written only with --4b (it
takes minutes of CPU); tiny_greedy_rows.npz holds rows 1 and 2 of the tiny
model's 16-sequence prompt batch (row 0 is tiny_greedy.npz's prompt), written
only with --rows.
"""
import hashlib
import os
import sys
import tempfile
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle.oracle import Reference  # noqa: E402
from quicklm_amd import synth  # noqa: E402

SHA_TENSORS = ["model.embed_tokens.weight", "model.layers.0.linear_attn.in_proj_qkv.weight",
               "model.layers.3.self_attn.q_proj.weight", "model.layers.0.linear_attn.A_log",
               "model.layers.0.linear_attn.dt_bias"]


def tensor_sha(model_dir):
    from oracle.oracle import read_safetensors
    t = read_safetensors(os.path.join(model_dir, "model.safetensors"))
    return {n: hashlib.sha256(t[n].tobytes()).hexdigest() for n in SHA_TENSORS}


def int4_stream(d, prompt):
    """The same run at --precision int4 (Q4_0 weights, lm_head included),
    IEEE build only: tiny_greedy_int4.npz."""
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_greedy_int4.npz")
    ref = Reference("ieee")
    ref.init_threads(os.cpu_count() or 1)
    m = ref.load_model(d, 2048, "int4")
    toks, pre, dec, lg = m.generate(prompt, 64, keep_logits=True)
    print(f"int4 ieee: prefill {pre:.2f}s decode {dec:.2f}s tokens {toks[:8]}...", flush=True)
    order = np.argsort(-lg, axis=1, kind="stable")[:, :32]
    top_val = np.take_along_axis(lg, order, axis=1)
    np.savez_compressed(
        out, prompt=prompt.astype(np.int32), tokens=toks.astype(np.int32),
        top_idx=order.astype(np.int32), top_val=top_val.astype(np.float32),
        margin=(top_val[:, 0] - top_val[:, 1]), logits0_head=lg[0, :4096].copy())
    print("wrote", out)


def native_streams():
    """--precision bf16 (the reference's default: weights in their checkpoint
    dtype), IEEE build: the tiny model (F32 linears: fp32 weights) ->
    tiny_greedy_native.npz; the micro model (BF16 linears: bf16 weights) ->
    micro_greedy_native.npz."""
    here = os.path.dirname(os.path.abspath(__file__))
    for cfg, n_prompt, n_new, vocab in (("tiny", 128, 64, None), ("micro", 24, 32, 4096)):
        with tempfile.TemporaryDirectory() as d:
            synth.write_model(d, cfg)
            prompt = (synth.prompt_tokens(n_prompt, seed=0)[0] if vocab is None else
                      synth.prompt_tokens(n_prompt, seed=0, vocab=vocab)[0])
            ref = Reference("ieee")
            ref.init_threads(os.cpu_count() or 1)
            m = ref.load_model(d, 2048, "bf16")
            toks, pre, dec, lg = m.generate(prompt, n_new, keep_logits=True)
            print(f"{cfg} native ieee: prefill {pre:.2f}s decode {dec:.2f}s tokens {toks[:8]}...",
                  flush=True)
            order = np.argsort(-lg, axis=1, kind="stable")[:, :32]
            top_val = np.take_along_axis(lg, order, axis=1)
            out = os.path.join(here, f"{cfg}_greedy_native.npz")
            np.savez_compressed(
                out, prompt=prompt.astype(np.int32), tokens=toks.astype(np.int32),
                top_idx=order.astype(np.int32), top_val=top_val.astype(np.float32),
                margin=(top_val[:, 0] - top_val[:, 1]),
                logits0_head=lg[0, :4096].copy())
            print("wrote", out)
            del m


SHA_TENSORS_4B = ["model.embed_tokens.weight", "model.layers.0.linear_attn.in_proj_qkv.weight",
                  "model.layers.3.self_attn.q_proj.weight", "model.layers.35.mlp.down_proj.weight",
                  "model.layers.0.linear_attn.A_log", "model.layers.0.linear_attn.dt_bias"]
N_4B_PROMPT, N_4B_STEPS, SEED_4B = 2048, 256, 4


def top32(lg):
    """The 32 largest logits of every step (stable order) and the top-2 margin."""
    order = np.argsort(-lg, axis=1, kind="stable")[:, :32]
    top_val = np.take_along_axis(lg, order, axis=1)
    return order.astype(np.int32), top_val.astype(np.float32), top_val[:, 0] - top_val[:, 1]


def fourb_stream():
    """The 4B-class int8 workload (36 layers, hidden 2560), batch 1: the
    2048-token prompts of seed 4 (sequences 0 and 1 of the decode benchmark's
    batch), batched prefill of prompt[0..2046], then N_4B_STEPS greedy steps,
    IEEE build -> 4b_greedy.npz (sequence 0: prompt, tokens, top_idx/top_val
    [steps, 32], margin, logits0_head, tensor SHAs, plus the fast-math
    build's stream, tokens_fast, for the record) and 4b_greedy_seq1.npz
    (sequence 1: prompt, tokens, top_idx/top_val, margin, logits0_head)."""
    here = os.path.dirname(os.path.abspath(__file__))
    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        t0 = time.time()
        synth.write_model(d, "4b")
        print(f"4B checkpoint written in {time.time() - t0:.1f}s", flush=True)
        from oracle.oracle import read_safetensors
        t = read_safetensors(os.path.join(d, "model.safetensors"))
        shas = [hashlib.sha256(t[n].tobytes()).hexdigest() for n in SHA_TENSORS_4B]
        del t
        prompts = synth.prompt_tokens(N_4B_PROMPT, seed=SEED_4B, batch=2)
        res = {}
        for kind in ("ieee", "fast"):
            ref = Reference(kind)
            ref.init_threads(os.cpu_count() or 1)
            m = ref.load_model(d, N_4B_PROMPT + N_4B_STEPS + 8, "int8")
            for row in ((0, 1) if kind == "ieee" else (0,)):
                toks, pre, dec, lg = m.generate(prompts[row], N_4B_STEPS,
                                                keep_logits=(kind == "ieee"))
                print(f"4B {ref.kind} sequence {row}: prefill {pre:.1f}s decode {dec:.1f}s "
                      f"({N_4B_STEPS / dec:.2f} tok/s) tokens {toks[:8]}...", flush=True)
                if lg is not None:
                    res[(kind, row)] = (toks, top32(lg), lg[0, :4096].copy())
                    del lg
                else:
                    res[(kind, row)] = (toks, None, None)
            del m
        toks, (ti, tv, mg), head = res[("ieee", 0)]
        out = os.path.join(here, "4b_greedy.npz")
        np.savez_compressed(
            out, prompt=prompts[0].astype(np.int32), tokens=toks.astype(np.int32),
            tokens_fast=res[("fast", 0)][0].astype(np.int32), top_idx=ti, top_val=tv,
            margin=mg, logits0_head=head, tensor_names=np.array(SHA_TENSORS_4B),
            tensor_sha=np.array(shas))
        same = np.nonzero(res[("fast", 0)][0] != toks)[0]
        print("wrote", out, "fast build splits from ieee at step",
              int(same[0]) if same.size else None, flush=True)
        toks, (ti, tv, mg), head = res[("ieee", 1)]
        out = os.path.join(here, "4b_greedy_seq1.npz")
        np.savez_compressed(out, prompt=prompts[1].astype(np.int32), tokens=toks.astype(np.int32),
                            top_idx=ti, top_val=tv, margin=mg, logits0_head=head)
        print("wrote", out, flush=True)


def tiny_rows(rows=(1, 2)):
    """Rows 1 and 2 of the tiny model's 16-sequence prompt batch (128 ids of
    seed 0 each; row 0 is tiny_greedy.npz's prompt), 64 greedy steps each,
    IEEE build -> tiny_greedy_rows.npz (rows, prompt [2, 128], tokens [2, 64],
    top_idx/top_val [2, 64, 32], margin [2, 64])."""
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_greedy_rows.npz")
    with tempfile.TemporaryDirectory() as d:
        synth.write_model(d, "tiny")
        prompts = synth.prompt_tokens(128, seed=0, batch=16)
        ref = Reference("ieee")
        ref.init_threads(os.cpu_count() or 1)
        m = ref.load_model(d, 2048, "int8")
        got = []
        for r in rows:
            toks, pre, dec, lg = m.generate(prompts[r], 64, keep_logits=True)
            print(f"tiny ieee row {r}: prefill {pre:.2f}s decode {dec:.2f}s tokens {toks[:8]}...",
                  flush=True)
            got.append((toks, top32(lg)))
        del m
        np.savez_compressed(
            out, rows=np.array(rows, np.int32), prompt=prompts[list(rows)].astype(np.int32),
            tokens=np.stack([g[0] for g in got]).astype(np.int32),
            top_idx=np.stack([g[1][0] for g in got]), top_val=np.stack([g[1][1] for g in got]),
            margin=np.stack([g[1][2] for g in got]))
        print("wrote", out)


def main():
    if "--4b" in sys.argv:  # only the 4B fixtures
        fourb_stream()
        return
    if "--rows" in sys.argv:  # only the tiny batch rows
        tiny_rows()
        return
    if "--native" in sys.argv:  # only the native-precision fixtures
        native_streams()
        return
    if "--int4" in sys.argv:  # only the int4 fixture
        with tempfile.TemporaryDirectory() as d:
            synth.write_model(d, "tiny")
            int4_stream(d, synth.prompt_tokens(128, seed=0)[0])
        return
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_greedy.npz")
    with tempfile.TemporaryDirectory() as d:
        synth.write_model(d, "tiny")
        prompt = synth.prompt_tokens(128, seed=0)[0]
        res = {}
        for kind in ("ieee", "fast"):
            ref = Reference(kind)
            ref.init_threads(os.cpu_count() or 1)
            m = ref.load_model(d, 2048, "int8")
            t0 = time.time()
            toks, pre, dec, lg = m.generate(prompt, 64, keep_logits=True)
            print(f"{ref.kind}: prefill {pre:.2f}s decode {dec:.2f}s ({64/dec:.2f} tok/s) "
                  f"tokens {toks[:8]}...", flush=True)
            res[kind] = (toks, lg)
            del m
        toks, lg = res["ieee"]
        order = np.argsort(-lg, axis=1, kind="stable")[:, :32]
        top_val = np.take_along_axis(lg, order, axis=1)
        np.savez_compressed(
            out, prompt=prompt.astype(np.int32), tokens=toks.astype(np.int32),
            tokens_fast=res["fast"][0].astype(np.int32), top_idx=order.astype(np.int32),
            top_val=top_val.astype(np.float32), margin=(top_val[:, 0] - top_val[:, 1]),
            logits0_head=lg[0, :4096].copy(), logits63_head=lg[63, :4096].copy(),
            tensor_names=np.array(SHA_TENSORS), tensor_sha=np.array(
                [tensor_sha(d)[n] for n in SHA_TENSORS]))
        int4_stream(d, prompt)
    native_streams()
    print("wrote", out, "fast==ieee tokens:", bool(np.array_equal(res["fast"][0], toks)))


if __name__ == "__main__":
    main()
