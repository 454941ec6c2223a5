"""Speculative decoding and sessions on the GPU engine (tiny hybrid model).

The reference's greedy speculative decoding is lossless: the committed
stream is the target's plain greedy stream. So the golden streams of the
reference's own greedy runs pin it: tiny_greedy.npz (int8) and
tiny_greedy_native.npz (--precision bf16), each reproduced here by a session
whose draft is the same checkpoint at int4 (the reference's default draft,
main.cpp:166-172, 366-394). The engine primitives under it are checked
directly: a batched forward against single steps, snapshot/restore
round trips.
"""

import os
import tempfile

import numpy as np
import pytest

from tests.util import say

pytestmark = pytest.mark.gpu

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def tiny_dir():
    from quicklm_amd import synth

    base = "/dev/shm" if os.path.isdir("/dev/shm") else None
    with tempfile.TemporaryDirectory(dir=base) as d:
        say("writing tiny model", d)
        synth.write_model(d, "tiny")
        yield d


@pytest.fixture(scope="module")
def engines(hip, tiny_dir):
    from quicklm_amd.engine import Engine

    es = {p: Engine(tiny_dir, max_seq_len=512, max_batch=1, precision=p)
          for p in ("int8", "int4", "bf16")}
    yield es
    for e in es.values():
        e.close()


def test_forward_batch_matches_steps(engines):
    """A batched forward of rows (the verify pass) against the same tokens
    forwarded one step at a time: same greedy picks, logits within 1e-3."""
    g = np.load(os.path.join(HERE, "tiny_greedy.npz"))
    toks = np.r_[g["prompt"], g["tokens"]].astype(np.int32)
    for prec in ("int8", "bf16"):
        e = engines[prec]
        e.reset()
        e.forward_batch(toks[:100], 0, argmax=False)
        say("forward_batch vs steps", prec)
        am, lg = e.forward_batch(toks[100:108], 100, argmax=True, logits=True)
        e.reset()
        e.forward_batch(toks[:100], 0, argmax=False)
        picks, worst = [], 0.0
        for i in range(8):
            picks.append(e.forward_greedy(int(toks[100 + i]), 100 + i))
            ref = e.last_logits(0)
            worst = max(worst, float(np.abs(lg[i] - ref).max() / np.abs(ref).max()))
        say(prec, "picks", am.tolist(), picks, "worst rel", worst)
        assert am.tolist() == picks
        assert worst < 1e-3
        assert [int(np.argmax(r)) for r in lg] == picks


def test_snapshot_restore_round_trip(engines):
    e = engines["int8"]
    g = np.load(os.path.join(HERE, "tiny_greedy.npz"))
    toks = g["prompt"].astype(np.int32)
    e.reset()
    e.forward_batch(toks[:60], 0, argmax=False)
    e.snapshot()
    a = [e.forward_greedy(int(t), 60 + i) for i, t in enumerate(toks[60:70])]
    la = e.last_logits(0)
    e.forward_batch(toks[70:80], 70, argmax=False)  # run further, then go back
    e.restore()
    b = [e.forward_greedy(int(t), 60 + i) for i, t in enumerate(toks[60:70])]
    assert a == b
    assert np.array_equal(e.last_logits(0), la)


@pytest.mark.parametrize("target,golden,K", [("int8", "tiny_greedy.npz", 4),
                                             ("bf16", "tiny_greedy_native.npz", 4),
                                             ("int8", "tiny_greedy.npz", 2)])
def test_speculative_stream_is_the_reference_greedy_stream(engines, target, golden, K):
    from quicklm_amd.engine import Session

    g = np.load(os.path.join(HERE, golden))
    s = Session(engines[target], engines["int4"], draft_tokens=K)
    try:
        out, info = s.turn(g["prompt"], 64)
        cached = s.cached()
    finally:
        s.close()
    say(f"speculative target {target} K={K}:", info)
    diff = np.nonzero(out != g["tokens"])[0]
    assert len(out) == 64
    assert diff.size == 0, f"first divergence at {diff[0]} (margin {g['margin'][diff[0]]:.6f})"
    assert np.array_equal(cached, np.r_[g["prompt"], g["tokens"]])
    assert info["drafted"] >= info["accepted"] >= 0 and info["emitted"] == 64


def test_plain_session_and_terminator(engines):
    from quicklm_amd.engine import Session

    g = np.load(os.path.join(HERE, "tiny_greedy.npz"))
    s = Session(engines["int8"])
    out, info = s.turn(g["prompt"], 64)
    s.close()
    assert np.array_equal(out, g["tokens"]) and info["reused"] == 0
    eos = int(g["tokens"][30])
    j = int(np.argmax(g["tokens"] == eos))
    for draft in (None, engines["int4"]):
        s = Session(engines["int8"], draft, draft_tokens=4, eos_id=eos)
        out, _ = s.turn(g["prompt"], 64)
        cached = s.cached()
        s.close()
        assert np.array_equal(out, g["tokens"][:j])
        assert np.array_equal(cached, np.r_[g["prompt"], g["tokens"][:j]])


def test_kv_reuse_turn_equals_fresh_turn(engines):
    """A second turn that extends the first one's ids reuses its state and
    prefills only the suffix; its tokens equal a fresh session's."""
    from quicklm_amd.engine import Session

    g = np.load(os.path.join(HERE, "tiny_greedy.npz"))
    s = Session(engines["int8"], engines["int4"], draft_tokens=4)
    s.turn(g["prompt"][:64], 16)
    turn2 = np.r_[s.cached(), g["prompt"][64:80]]
    out2, info2 = s.turn(turn2, 16)
    s.close()
    say("kv-reuse turn 2:", info2)
    assert info2["reused"] == 64 + 16 and info2["recomputed"] == 15
    f = Session(engines["int8"], engines["int4"], draft_tokens=4)
    outf, infof = f.turn(turn2, 16)
    f.close()
    assert infof["reused"] == 0
    assert np.array_equal(out2, outf)
