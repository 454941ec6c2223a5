"""Model-level parity: the GPU engine against the reference CPU path.

Golden fixture tests/golden/tiny_greedy.npz was produced by the reference
sources compiled with IEEE flags (tests/golden/make_golden.py) on the tiny
hybrid model (1024 hidden, 24 layers 3:1 DeltaNet/GQA, vocab 151936, seeded
random weights, 128-token prompt, 64 greedy tokens).
"""

import hashlib
import os
import tempfile

import numpy as np
import pytest

from tests.util import say

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


@pytest.fixture(scope="module")
def tiny_dir():
    from quicklm_amd import synth

    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        say("writing tiny model", d)
        synth.write_model(d, "tiny")
        yield d


@pytest.fixture(scope="module")
def engine(hip, tiny_dir):
    from quicklm_amd.engine import Engine

    e = Engine(tiny_dir, max_seq_len=2048, max_batch=2, precision="int8")
    yield e
    e.close()


def test_synthetic_weights_match_golden(tiny_dir, golden):
    from oracle.oracle import read_safetensors

    t = read_safetensors(os.path.join(tiny_dir, "model.safetensors"))
    for name, sha in zip(golden["tensor_names"], golden["tensor_sha"]):
        assert hashlib.sha256(t[str(name)].tobytes()).hexdigest() == str(sha), name


def test_teacher_forced_logits(engine, golden):
    """Feed the reference's own token stream; every step's top-32 logits must
    agree with the reference within 1e-3 (normwise, fp32 accumulation)."""
    prompt, toks = golden["prompt"], golden["tokens"]
    engine.reset()
    for p in range(127):
        engine.forward(int(prompt[p]), p)
    feed = np.concatenate([prompt[-1:], toks[:-1]])
    worst = 0.0
    devs = []
    for i, t in enumerate(feed):
        lg = engine.forward(int(t), 127 + i)
        idx = golden["top_idx"][i]
        ref = golden["top_val"][i]
        dev = float(np.abs(lg[idx] - ref).max())
        devs.append(dev)
        worst = max(worst, dev / float(np.abs(ref).max()))
        if i == 0:
            head = golden["logits0_head"]
            assert float(np.abs(lg[:4096] - head).max() / np.abs(head).max()) < 1e-3
    say("teacher-forced max |dlogit| per 8 steps", np.round(devs[::8], 6), "worst rel", worst)
    assert worst < 1e-3


@pytest.mark.parametrize("batched_prefill", [True, 2, False])
def test_tiny_greedy_matches_reference(engine, golden, batched_prefill):
    """The reference's 64-token greedy stream, with the prompt prefilled by
    the batched prefill (chunked or row-by-row DeltaNet recurrence) or
    forwarded one decode step per token."""
    out, pre, dec = engine.generate(golden["prompt"][None, :], 64,
                                    batched_prefill=batched_prefill)
    toks = golden["tokens"]
    got = out[0]
    diff = np.nonzero(got != toks)[0]
    say(f"prefill {pre:.3f}s decode {dec:.3f}s; first divergence:",
        int(diff[0]) if diff.size else None,
        "margin there:", float(golden["margin"][diff[0]]) if diff.size else None)
    assert diff.size == 0, f"first divergence at step {diff[0]} (reference top-2 margin " \
                           f"{golden['margin'][diff[0]]:.6f})"


def test_graph_replay_equals_eager(engine, golden):
    p = golden["prompt"][None, :40]
    a, _, _ = engine.generate(p, 16, use_graph=True)
    la = engine.last_logits(0)
    b, _, _ = engine.generate(p, 16, use_graph=False)
    lb = engine.last_logits(0)
    assert np.array_equal(a, b)
    assert np.array_equal(la, lb)


def test_l2_plan_changes_no_result(hip, tiny_dir, golden, engine, monkeypatch):
    """The batch-1 mixer's L2 plan (on by default) moves bytes into the
    caches only: an engine loaded with QLM_L2_PREFETCH=0 decodes the same
    tokens with bit-identical last logits."""
    from quicklm_amd.engine import Engine

    p = golden["prompt"][None, :40]
    a, _, _ = engine.generate(p, 16)
    la = engine.last_logits(0)
    monkeypatch.setenv("QLM_L2_PREFETCH", "0")
    e = Engine(tiny_dir, max_seq_len=256, max_batch=1, precision="int8")
    try:
        b, _, _ = e.generate(p, 16)
        lb = e.last_logits(0)
    finally:
        e.close()
    assert np.array_equal(a, b)
    assert np.array_equal(la, lb)


ROWS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy_rows.npz")


def test_tiny_batch16_rows_match_reference(hip, tiny_dir, golden, engine):
    """Config 0 at batch 16 (the batched kernels: bf16 matrix-core matmuls,
    one workgroup a DeltaNet head, 16-sequence attention): the 16 prompts of
    seed 0 decoded together for 64 steps. Rows 0-2 have reference streams
    (tiny_greedy.npz is row 0, tiny_greedy_rows.npz rows 1 and 2, the IEEE
    build) and must equal them; rows 3-15 must equal the batch-1 engine's
    streams of the same prompts."""
    from quicklm_amd import synth
    from quicklm_amd.engine import Engine

    rows = np.load(ROWS)
    prompts = synth.prompt_tokens(128, seed=0, batch=16)
    assert np.array_equal(prompts[0], golden["prompt"])
    ref = {0: golden["tokens"]}
    for i, r in enumerate(rows["rows"]):
        assert np.array_equal(prompts[int(r)], rows["prompt"][i])
        ref[int(r)] = rows["tokens"][i]
    e16 = Engine(tiny_dir, max_seq_len=256, max_batch=16, precision="int8")
    try:
        out16, _, _ = e16.generate(prompts, 64, batched_prefill=True)
    finally:
        e16.close()
    for r, toks in ref.items():
        d = np.nonzero(out16[r] != toks)[0]
        say(f"batch 16 row {r}: first divergence from the reference",
            int(d[0]) if d.size else None)
        assert d.size == 0, (r, int(d[0]))
    for b in range(3, 16):
        one, _, _ = engine.generate(prompts[b][None, :], 64, batched_prefill=True)
        assert np.array_equal(out16[b], one[0]), b


def test_batch_rows_equal_single(engine, golden):
    """Two sequences in one batch give exactly the single-sequence results."""
    p0 = golden["prompt"][:48]
    p1 = golden["prompt"][48:96]
    s0, _, _ = engine.generate(p0[None, :], 12)
    s1, _, _ = engine.generate(p1[None, :], 12)
    both, _, _ = engine.generate(np.stack([p0, p1]), 12)
    assert np.array_equal(both[0], s0[0]) and np.array_equal(both[1], s1[0])


@pytest.mark.parametrize("n", [128, 1300])
@pytest.mark.parametrize("mode", [True, 2])
def test_batched_prefill_equals_stepwise(engine, golden, n, mode):
    """Batched prefill (matrix-core projections, chunked or row-by-row
    DeltaNet, prefill attention) leaves the model where n-1 decode steps
    leave it: same tokens, logits within 1e-4."""
    rng = np.random.default_rng(11)
    p = golden["prompt"][:n] if n <= 128 else rng.integers(0, 151936, n).astype(np.int32)
    a, pre_a, _ = engine.generate(p[None, :], 8, batched_prefill=mode)
    la = engine.last_logits(0)
    b, pre_b, _ = engine.generate(p[None, :], 8, batched_prefill=False)
    lb = engine.last_logits(0)
    say(f"n={n} mode={mode}: batched prefill {pre_a:.3f}s, stepwise {pre_b:.3f}s")
    assert np.array_equal(a, b)
    assert float(np.abs(la - lb).max() / np.abs(lb).max()) < 1e-4


# batched vs stepwise prefill on the same engine: the int8 and int4 forms
# share the int8 arithmetic (1e-4); the native path's fp32 rows run on the
# fp32 matrix cores in the batched form and on the vector ALUs stepwise, held
# to the decode path's per-op tolerance (1e-3)
PASS_TOL = {"int8": 1e-4, "int4": 1e-4, "bf16": 1e-3}


@pytest.mark.parametrize("precision", ["int8", "int4", "bf16"])
@pytest.mark.parametrize("mode", [True, 2])
def test_prefill_across_passes(hip, tiny_dir, mode, precision):
    """A 2300-row prompt goes through the layers in two passes (2048 rows,
    then 251), the second continuing the first's states and caches: same
    tokens as 2299 decode steps, logits within PASS_TOL, at every weight
    precision (the int4 and native forms have their own prefill matmuls)."""
    from quicklm_amd.engine import Engine

    rng = np.random.default_rng(12)
    p = rng.integers(0, 151936, 2300).astype(np.int32)
    e = Engine(tiny_dir, max_seq_len=2600, max_batch=1, precision=precision)
    try:
        a, pre_a, _ = e.generate(p[None, :], 8, batched_prefill=mode)
        la = e.last_logits(0)
        b, pre_b, _ = e.generate(p[None, :], 8, batched_prefill=False)
        lb = e.last_logits(0)
    finally:
        e.close()
    err = float(np.abs(la - lb).max() / np.abs(lb).max())
    say(f"2300 rows {precision} mode={mode}: batched prefill {pre_a:.3f}s, stepwise "
        f"{pre_b:.3f}s, last-step logit rel err {err:.2e}")
    assert np.array_equal(a, b)
    assert err < PASS_TOL[precision]


def test_context_overflow_rejected(engine):
    from quicklm_amd.engine import EngineError

    with pytest.raises(EngineError, match="context length exceeded"):
        engine.generate(np.zeros((1, 2000), np.int32), 100)
    with pytest.raises(EngineError):
        engine.forward(1, 5000)
    for bad in (-1, 151936):
        with pytest.raises(EngineError, match="token id out of range"):
            engine.forward(bad, 5)


def test_micro_per_row_scales_match_oracle(hip, tmp_path):
    """precision "int8_row" (one fp32 scale per output row, G = K, the scheme
    of an isolated per-row int8 matmul): the engine's greedy stream equals the
    oracle model quantised the same way."""
    from oracle.oracle import Oracle, OracleModel
    from quicklm_amd import synth
    from quicklm_amd.engine import Engine

    d = str(tmp_path)
    synth.write_model(d, "micro")
    prompt = synth.prompt_tokens(24, seed=5, vocab=4096)[0]
    eng = Engine(d, max_seq_len=64, max_batch=1, precision="int8_row")
    try:
        got, _, _ = eng.generate(prompt[None, :], 16)
        lg = eng.last_logits(0)
    finally:
        eng.close()
    want, wlg = OracleModel(d, 64, Oracle(), group="row").generate(prompt, 16, keep_logits=True)
    err = float(np.abs(lg - wlg[-1]).max() / np.abs(wlg[-1]).max())
    say("int8_row micro: last-step logit rel err", err)
    assert np.array_equal(got[0], want)
    assert err < 1e-3


@pytest.mark.parametrize("precision", ["int8", "int4"])
def test_one_weight_copy(hip, tiny_dir, precision):
    """Every device matmul reads the tile-major copy of a linear, so the
    engine keeps no row-major one: the device memory a loaded tiny model
    takes stays within the tile-major weights (int8 values + group scales,
    and at int4 the int4 copy beside them) plus the fp32 embedding and the
    state, where the row-major copies would add 0.6 GB (int8) or 0.87 GB
    (int4)."""
    from quicklm_amd.engine import Engine

    hip.sync()
    free0 = hip.mem_free()
    e = Engine(tiny_dir, max_seq_len=256, max_batch=1, precision=precision)
    try:
        hip.sync()
        used = free0 - hip.mem_free()
        wb = e.weight_bytes
    finally:
        e.close()
    nk = wb / (1.125 if precision == "int8" else 0.625)  # int8 weights of the linears
    tiles = nk * (1.125 if precision == "int8" else 1.625)
    embed = 151936 * 1024 * 4
    say(f"{precision}: device bytes {used / 1e9:.3f} GB, tile-major weights {tiles / 1e9:.3f} GB, "
        f"embedding {embed / 1e9:.3f} GB")
    assert used < tiles + embed + 450e6


def test_shapes_without_fast_forms_fall_back(hip, tmp_path):
    """A model whose hidden size has no launch shape of the matrix-core
    one-row GEMV (3072 = 48 blocks of 64: no instantiated (waves, ring) pair)
    and an odd DeltaNet head count (3 heads: the projection row of 4 * 384 +
    6 = 1542 floats is not a multiple of 4, which the column-split mixer
    needs): the decode step takes the general forms instead (the lm_head
    through the matrix-core matmul and the two-pass argmax, the one-workgroup-
    a-head mixer), at batch 1 and 2, and the greedy stream equals the oracle
    model's."""
    from oracle.oracle import Oracle, OracleModel
    from quicklm_amd import synth
    from quicklm_amd.engine import Engine

    cfg = dict(synth.MICRO, name="odd", index=10, hidden_size=3072, linear_num_heads=3,
               intermediate_size=1024)
    d = str(tmp_path)
    synth.write_model(d, cfg)
    prompt = synth.prompt_tokens(20, seed=6, vocab=4096)[0]
    eng = Engine(d, max_seq_len=64, max_batch=2, precision="int8")
    try:
        got, _, _ = eng.generate(prompt[None, :], 12)
        lg = eng.last_logits(0)
        both, _, _ = eng.generate(np.stack([prompt, prompt[::-1].copy()]), 12)
    finally:
        eng.close()
    want, wlg = OracleModel(d, 64, Oracle()).generate(prompt, 12, keep_logits=True)
    err = float(np.abs(lg - wlg[-1]).max() / np.abs(wlg[-1]).max())
    say("odd-shaped micro: last-step logit rel err", err, "tokens", got[0][:6], want[:6])
    assert np.array_equal(got[0], want)
    assert np.array_equal(both[0], got[0])
    assert err < 1e-3
