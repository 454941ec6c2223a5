"""Model-level parity at --precision bf16, the reference's default: every
linear weight kept in its checkpoint dtype (fp32 rows for the tiny model's
F32 tensors, bf16 rows for the micro model's BF16 ones), fp32 dot products.

Golden fixtures tests/golden/{tiny,micro}_greedy_native.npz: the reference
sources compiled with IEEE flags, run at --precision bf16
(tests/golden/make_golden.py --native): tiny -- 128-token prompt, 64 greedy
tokens; micro -- 24-token prompt (vocab 4096), 32 greedy tokens; top-32
logits per step.
"""

import os
import tempfile

import numpy as np
import pytest

from tests.util import say

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _model_dir(cfg):
    from quicklm_amd import synth

    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    d = tempfile.TemporaryDirectory(dir=base)
    say("writing", cfg, "model", d.name)
    synth.write_model(d.name, cfg)
    return d


@pytest.fixture(scope="module")
def tiny_native():
    d = _model_dir("tiny")
    from quicklm_amd.engine import Engine

    e = Engine(d.name, max_seq_len=2048, max_batch=2, precision="bf16")
    yield e, np.load(os.path.join(HERE, "tiny_greedy_native.npz")), d.name
    e.close()
    d.cleanup()


def test_native_weight_bytes(hip, tiny_native):
    """fp32 rows: 4 bytes a weight, against int8's 1 + 4/32."""
    from quicklm_amd.engine import Engine

    e, _, d = tiny_native
    e8 = Engine(d, max_seq_len=64, max_batch=1, precision="int8")
    w8 = e8.weight_bytes
    e8.close()
    say("weight bytes native", e.weight_bytes, "int8", w8)
    assert e.weight_bytes * 9 == w8 * 32


def test_native_teacher_forced_logits(tiny_native):
    e, golden, _ = tiny_native
    prompt, toks = golden["prompt"], golden["tokens"]
    e.reset()
    for p in range(127):
        e.forward(int(prompt[p]), p)
    feed = np.concatenate([prompt[-1:], toks[:-1]])
    worst = 0.0
    for i, t in enumerate(feed):
        lg = e.forward(int(t), 127 + i)
        idx, ref = golden["top_idx"][i], golden["top_val"][i]
        worst = max(worst, float(np.abs(lg[idx] - ref).max()) / float(np.abs(ref).max()))
        if i == 0:
            head = golden["logits0_head"]
            assert float(np.abs(lg[:4096] - head).max() / np.abs(head).max()) < 1e-3
    say("native teacher-forced worst rel", worst)
    assert worst < 1e-3


@pytest.mark.parametrize("batched_prefill", [True, False])
def test_native_tiny_greedy_matches_reference(tiny_native, batched_prefill):
    e, golden, _ = tiny_native
    out, pre, dec = e.generate(golden["prompt"][None, :], 64, batched_prefill=batched_prefill)
    diff = np.nonzero(out[0] != golden["tokens"])[0]
    say(f"native prefill {pre:.3f}s decode {dec:.3f}s; first divergence:",
        int(diff[0]) if diff.size else None)
    assert diff.size == 0, f"first divergence at step {diff[0]} (reference top-2 margin " \
                           f"{golden['margin'][diff[0]]:.6f})"


def test_native_batch_rows_equal_single(tiny_native):
    e, golden, _ = tiny_native
    p = golden["prompt"][None, :48]
    a, _, _ = e.generate(p, 12)
    b, _, _ = e.generate(np.concatenate([p, p]), 12)
    assert np.array_equal(b[0], a[0]) and np.array_equal(b[1], a[0])


def test_native_micro_bf16_weights_match_reference(hip):
    """BF16 checkpoint tensors stay bf16 on the device (2 bytes a weight) and
    the greedy stream equals the reference's."""
    from quicklm_amd.engine import Engine

    golden = np.load(os.path.join(HERE, "micro_greedy_native.npz"))
    d = _model_dir("micro")
    try:
        e = Engine(d.name, max_seq_len=64, max_batch=1, precision="bf16")
        try:
            out, _, _ = e.generate(golden["prompt"][None, :], len(golden["tokens"]))
            lg = e.last_logits(0)
        finally:
            e.close()
    finally:
        d.cleanup()
    ref = golden["top_val"][-1]
    err = float(np.abs(lg[golden["top_idx"][-1]] - ref).max() / np.abs(ref).max())
    say("native micro: last-step top-32 rel err", err)
    diff = np.nonzero(out[0] != golden["tokens"])[0]
    assert diff.size == 0, f"first divergence at step {diff[0]}"
    assert err < 1e-3
