"""Host logic of speculative decoding and the session loop, on the CPU.

quicklm_amd/csrc/host/speculative.cpp (the round loop of the reference's
SpeculativeDecoder, speculative.cpp:1-222, and the turn loop of
main.cpp:455-690) is compiled with g++ together with tests/spec_fake.cpp, a
deterministic stand-in model whose greedy pick is a hash of the tokens it has
consumed. The stand-in refuses any forward that is not at the next position,
so a lost restore or a misplaced replay fails loudly.

What is pinned: greedy speculative decoding is lossless -- its stream equals
the target's plain greedy stream for every K and rejection rate; both models
end the turn holding exactly cached_ids; terminators and the token budget
cut the stream as the reference's loop does; kv-reuse prefills only the new
suffix and gives the same tokens as a fresh session.
"""

import ctypes as C
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST = os.path.join(ROOT, "quicklm_amd", "csrc", "host")


@pytest.fixture(scope="module")
def fake(tmp_path_factory):
    d = tmp_path_factory.mktemp("specfake")
    so = str(d / "libspecfake.so")
    subprocess.run(["g++", "-std=c++17", "-O1", "-shared", "-fPIC", "-Wall", "-I", HOST,
                    os.path.join(ROOT, "tests", "spec_fake.cpp"),
                    os.path.join(HOST, "speculative.cpp"), "-o", so], check=True)
    L = C.CDLL(so)
    L.fake_last_error.restype = C.c_char_p
    return L


V, MAXSEQ = 97, 512


def run(L, turns_ids, max_tokens, K=4, draft_mod=3, eos=-1, im_end=-1, kv_reuse=True,
        max_seq=MAXSEQ):
    ids = np.concatenate([np.asarray(t, np.int32) for t in turns_ids]).astype(np.int32)
    off = np.cumsum([0] + [len(t) for t in turns_ids]).astype(np.int32)
    T = len(turns_ids)
    out = np.zeros(T * max(1, max_tokens), np.int32)
    n_out = np.zeros(T, np.int32)
    info = np.zeros(7 * T, np.int32)
    hist = np.zeros(3 * max_seq, np.int32)
    hlen = np.zeros(3, np.int32)
    calls = np.zeros(8, np.int32)
    rc = L.fake_session(V, max_seq, K, eos, im_end, draft_mod, 1 if kv_reuse else 0, T,
                        ids.ctypes.data_as(C.c_void_p), off.ctypes.data_as(C.c_void_p),
                        max_tokens, out.ctypes.data_as(C.c_void_p),
                        n_out.ctypes.data_as(C.c_void_p), info.ctypes.data_as(C.c_void_p),
                        hist.ctypes.data_as(C.c_void_p), hlen.ctypes.data_as(C.c_void_p),
                        calls.ctypes.data_as(C.c_void_p))
    if rc:
        raise RuntimeError(L.fake_last_error().decode())
    outs, w = [], 0
    for n in n_out:
        outs.append(out[w:w + n].copy())
        w += n
    h = [hist[i * max_seq:i * max_seq + hlen[i]].copy() for i in range(3)]
    return outs, info.reshape(T, 7), h, calls


PROMPT = [5, 17, 3, 88, 41, 9, 60]


@pytest.mark.parametrize("K", [1, 2, 4, 7])
@pytest.mark.parametrize("draft_mod", [0, 2, 3, 11])
def test_speculative_is_lossless(fake, K, draft_mod):
    plain, _, hp, _ = run(fake, [PROMPT], 50, draft_mod=-1)
    spec, info, hs, calls = run(fake, [PROMPT], 50, K=K, draft_mod=draft_mod)
    assert np.array_equal(spec[0], plain[0])
    assert len(spec[0]) == 50
    # plain loop: the last emitted token is never forwarded; speculative
    # commit: every emitted token has been consumed by both models
    assert np.array_equal(hp[0], np.r_[PROMPT, plain[0][:-1]])
    assert np.array_equal(hs[0], np.r_[PROMPT, spec[0]])
    assert np.array_equal(hs[1], hs[0]) and np.array_equal(hs[2], hs[0])
    reused, recomputed, rounds, drafted, accepted, emitted, rejections = info[0]
    assert (reused, recomputed, emitted) == (0, len(PROMPT) - 1, 50)
    assert 0 <= accepted <= drafted and rounds * 1 <= drafted <= rounds * K
    assert calls[2] == rounds and calls[6] == rounds  # one snapshot per round and model
    if draft_mod == 0:  # the draft agrees everywhere: no rejection
        assert rejections == 0 and accepted == drafted
    else:
        assert rejections > 0


@pytest.mark.parametrize("K", [1, 3, 4])
def test_terminator_cuts_the_stream(fake, K):
    plain, _, _, _ = run(fake, [PROMPT], 60, draft_mod=-1)
    s = plain[0]
    for j in (0, 1, 7, 23):
        eos = int(s[j])
        j0 = int(np.argmax(s == eos))  # first occurrence
        for kw in ({"eos": eos}, {"im_end": eos}):
            p2, _, hp, _ = run(fake, [PROMPT], 60, draft_mod=-1, **kw)
            sp, info, hs, _ = run(fake, [PROMPT], 60, K=K, draft_mod=3, **kw)
            assert np.array_equal(p2[0], s[:j0]) and np.array_equal(sp[0], s[:j0])
            # the terminator is consumed by neither loop's state past what it emitted
            assert np.array_equal(hs[0], np.r_[PROMPT, s[:j0]])
            assert np.array_equal(hs[1], hs[0])
            assert np.array_equal(hp[0], np.r_[PROMPT, s[:j0]])
            assert info[0][5] == j0


@pytest.mark.parametrize("budget", [1, 2, 5, 9, 13])
def test_token_budget_trims_a_round(fake, budget):
    plain, _, _, _ = run(fake, [PROMPT], budget, draft_mod=-1)
    for K in (2, 4, 6):
        sp, info, hs, _ = run(fake, [PROMPT], budget, K=K, draft_mod=0)  # full accepts
        assert np.array_equal(sp[0], plain[0])
        assert np.array_equal(hs[0], np.r_[PROMPT, plain[0]])
        assert np.array_equal(hs[1], hs[0])


def test_kv_reuse_prefills_only_the_suffix(fake):
    first, info1, h1, _ = run(fake, [PROMPT], 20, K=4, draft_mod=3)
    cached = h1[2]
    turn2 = np.r_[cached, [7, 8, 9, 10]]
    outs, info, h, _ = run(fake, [PROMPT, turn2], 20, K=4, draft_mod=3)
    assert np.array_equal(outs[0], first[0])
    assert info[1][0] == len(cached) and info[1][1] == 3  # reused, recomputed
    fresh, finfo, _, _ = run(fake, [turn2], 20, K=4, draft_mod=3)
    assert np.array_equal(outs[1], fresh[0])
    assert finfo[0][0] == 0 and finfo[0][1] == len(turn2) - 1
    assert np.array_equal(h[0], h[1]) and np.array_equal(h[0], h[2])
    # without kv-reuse the second turn starts over
    outs_nr, info_nr, _, _ = run(fake, [PROMPT, turn2], 20, K=4, draft_mod=3, kv_reuse=False)
    assert np.array_equal(outs_nr[1], fresh[0]) and info_nr[1][0] == 0
    # ids that do not extend the cache: reset and full prefill
    other = [1, 2, 3]
    outs_o, info_o, _, _ = run(fake, [PROMPT, other], 20, K=4, draft_mod=3)
    fresh_o, _, _, _ = run(fake, [other], 20, K=4, draft_mod=3)
    assert info_o[1][0] == 0 and np.array_equal(outs_o[1], fresh_o[0])


def test_plain_session_reuse(fake):
    first, _, h1, _ = run(fake, [PROMPT], 12, draft_mod=-1)
    turn2 = np.r_[h1[2], first[0][-1:], [4, 4]]
    outs, info, _, _ = run(fake, [PROMPT, turn2], 12, draft_mod=-1)
    fresh, _, _, _ = run(fake, [turn2], 12, draft_mod=-1)
    assert info[1][0] == len(h1[2]) and np.array_equal(outs[1], fresh[0])


def test_errors(fake):
    with pytest.raises(RuntimeError, match="--draft-tokens must be >= 1, got 0"):
        run(fake, [PROMPT], 5, K=0)
    with pytest.raises(RuntimeError, match="Tokenized turn is empty"):
        run(fake, [[]], 5)
    # the context fills up: same error text as the reference
    with pytest.raises(RuntimeError, match=r"context length exceeded max_seq_len \(16\)"):
        run(fake, [PROMPT], 40, K=4, draft_mod=3, max_seq=16)
    with pytest.raises(RuntimeError, match=r"context length exceeded max_seq_len \(16\)"):
        run(fake, [PROMPT], 40, draft_mod=-1, max_seq=16)
    with pytest.raises(RuntimeError, match="out of range"):
        run(fake, [[1, 2, V]], 5)
