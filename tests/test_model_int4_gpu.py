"""Model-level parity at --precision int4 (Q4_0 weights, lm_head included).

Golden fixture tests/golden/tiny_greedy_int4.npz: the reference sources
compiled with IEEE flags, run at --precision int4 on the tiny hybrid model
(tests/golden/make_golden.py): 128-token prompt, 64 greedy tokens, top-32
logits per step.
"""

import os
import tempfile

import numpy as np
import pytest

from tests.util import say

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                      "tiny_greedy_int4.npz")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN)


@pytest.fixture(scope="module")
def tiny_dir4():
    from quicklm_amd import synth

    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        say("writing tiny model", d)
        synth.write_model(d, "tiny")
        yield d


@pytest.fixture(scope="module")
def engine4(hip, tiny_dir4):
    from quicklm_amd.engine import Engine

    e = Engine(tiny_dir4, max_seq_len=2048, max_batch=2, precision="int4")
    yield e
    e.close()


def test_int4_weight_bytes(hip, engine4, tiny_dir4):
    """The one-row step streams int4 weights: K/2 bytes plus a 4-byte scale
    per 32 columns per row, 0.625 bytes a weight against int8's 1.125."""
    from quicklm_amd.engine import Engine

    e8 = Engine(tiny_dir4, max_seq_len=64, max_batch=1, precision="int8")
    w8 = e8.weight_bytes
    e8.close()
    say("weight bytes int4", engine4.weight_bytes, "int8", w8)
    assert engine4.weight_bytes * 9 == w8 * 5


def test_int4_teacher_forced_logits(engine4, golden):
    prompt, toks = golden["prompt"], golden["tokens"]
    engine4.reset()
    for p in range(127):
        engine4.forward(int(prompt[p]), p)
    feed = np.concatenate([prompt[-1:], toks[:-1]])
    worst = 0.0
    for i, t in enumerate(feed):
        lg = engine4.forward(int(t), 127 + i)
        idx, ref = golden["top_idx"][i], golden["top_val"][i]
        worst = max(worst, float(np.abs(lg[idx] - ref).max()) / float(np.abs(ref).max()))
        if i == 0:
            head = golden["logits0_head"]
            assert float(np.abs(lg[:4096] - head).max() / np.abs(head).max()) < 1e-3
    say("int4 teacher-forced worst rel", worst)
    assert worst < 1e-3


@pytest.mark.parametrize("batched_prefill", [True, False])
def test_int4_tiny_greedy_matches_reference(engine4, golden, batched_prefill):
    out, pre, dec = engine4.generate(golden["prompt"][None, :], 64,
                                     batched_prefill=batched_prefill)
    diff = np.nonzero(out[0] != golden["tokens"])[0]
    say(f"int4 prefill {pre:.3f}s decode {dec:.3f}s; first divergence:",
        int(diff[0]) if diff.size else None)
    assert diff.size == 0, f"first divergence at step {diff[0]} (reference top-2 margin " \
                           f"{golden['margin'][diff[0]]:.6f})"


def test_int4_batch_rows_equal_single(engine4, golden):
    """Two sequences at once (int8 kernels over the unpacked values) against
    one at a time (int4 one-row GEMV): identical tokens."""
    p = golden["prompt"][None, :48]
    a, _, _ = engine4.generate(p, 12)
    b, _, _ = engine4.generate(np.concatenate([p, p]), 12)
    assert np.array_equal(b[0], a[0]) and np.array_equal(b[1], a[0])
