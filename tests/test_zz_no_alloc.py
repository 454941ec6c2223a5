"""The no-allocation attention entry point against the one it mirrors.

qlm_attention_decode_noalloc runs qlm_attention_decode's kernels with the
chunk records in the library's static device scratch instead of a caller
workspace. Both are called through the C ABI on the same seeded inputs; the
outputs must be bit-identical (same kernels, same arithmetic per record),
on two calls in a row, the second smaller than the first, and the first is
also checked against the oracle's attention (1e-5 normwise, as the
workspace form's own test). The entry point is for code under graph capture:
it is captured into a hipGraph and replayed, with eager work between the
replays, and, in a fresh process, its first call on the device is made
under capture (qlm_set_device has resolved the scratch address). The
refusal of an oversize call is a host-side check, tested without a GPU in
tests/test_host_checks.py.
"""

import ctypes as C
import os
import subprocess
import sys

import numpy as np
import pytest

from tests.util import bf16_bits, bf16_to_f32, rel_err, say

pytestmark = pytest.mark.gpu


def run_both(hip, rng, B, n_q, n_kv, hd, max_seq, ctx, kv):
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    k = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    if kv == 1:
        kb, vb = bf16_bits(k), bf16_bits(v)
        k, v = bf16_to_f32(kb), bf16_to_f32(vb)
        dk, dv = hip.DeviceBuffer.from_numpy(kb), hip.DeviceBuffer.from_numpy(vb)
    else:
        dk, dv = hip.DeviceBuffer.from_numpy(k), hip.DeviceBuffer.from_numpy(v)
    dq = hip.DeviceBuffer.from_numpy(q)
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
    a, b = hip.DeviceBuffer(q.nbytes), hip.DeviceBuffer(q.nbytes)
    say(f"noalloc attention B={B} n_q={n_q} n_kv={n_kv} hd={hd} ctx={ctx} kv={kv}")
    hip.call("qlm_attention_decode", dq, dk, dv, kv, max_seq, ctx, a, B, n_q, n_kv, hd, work,
             None)
    hip.call("qlm_attention_decode_noalloc", dq, dk, dv, kv, max_seq, ctx, b, B, n_q, n_kv, hd,
             None)
    return q, k, v, a.to_numpy(q.shape, np.float32), b.to_numpy(q.shape, np.float32)


def test_noalloc_attention_equals_workspace_form(hip, orc, rng):
    assert hip.lib().qlm_attention_decode_noalloc_bytes(2, 16, 256, 3000) <= 32 << 20
    # first call: the config-3 head layout (16 q / 2 kv heads, hd 256, bf16 cache)
    q, k, v, a, b = run_both(hip, rng, 2, 16, 2, 256, 4096, 3000, 1)
    assert np.array_equal(a, b)
    ref = np.stack([orc.attention(q[i], k[i], v[i], 3000) for i in range(2)])
    assert rel_err(b, ref) < 1e-5
    # second call, smaller: fewer sequences, a shorter context, hd 128, fp32
    # cache; the scratch still holds the first call's records
    q, k, v, a, b = run_both(hip, rng, 1, 8, 2, 128, 1024, 700, 0)
    assert np.array_equal(a, b)
    ref = orc.attention(q[0], k[0], v[0], 700)[None]
    assert rel_err(b, ref) < 1e-5


def test_noalloc_attention_in_captured_graph(hip, rng):
    """Captured into a graph and replayed three times, with eager calls of the
    workspace form (which reuse nothing of it) between the replays: every
    replay's output equals the workspace form's bit for bit."""
    hip.check(hip.lib().qlm_set_device(0))  # resolves the scratch address outside the capture
    B, n_q, n_kv, hd, max_seq, ctx = 2, 16, 4, 128, 2400, 2100
    q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
    k = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    v = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
    dq, dk, dv = (hip.DeviceBuffer.from_numpy(a) for a in (q, k, v))
    work = hip.DeviceBuffer(hip.lib().qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
    a, b = hip.DeviceBuffer(q.nbytes), hip.DeviceBuffer(q.nbytes)
    hip.call("qlm_attention_decode", dq, dk, dv, 0, max_seq, ctx, a, B, n_q, n_kv, hd, work, None)
    want = a.to_numpy(q.shape, np.float32)
    L = hip.lib()
    st = hip.Stream()
    hip.check(L.qlm_graph_begin(st.ptr))
    rc = L.qlm_attention_decode_noalloc(dq.ptr, dk.ptr, dv.ptr, 0, max_seq, ctx, b.ptr, B, n_q,
                                        n_kv, hd, st.ptr)
    g = C.c_void_p()
    hip.check(L.qlm_graph_end(st.ptr, C.byref(g)))
    hip.check(rc)
    try:
        for rep in range(3):
            b.zero()
            hip.sync()
            hip.check(L.qlm_graph_launch(g, st.ptr))
            st.sync()
            say("noalloc graph replay", rep)
            assert np.array_equal(b.to_numpy(q.shape, np.float32), want), rep
            hip.call("qlm_attention_decode", dq, dk, dv, 0, max_seq, ctx // 2, a, B, n_q, n_kv,
                     hd, work, None)
            hip.sync()
    finally:
        hip.check(L.qlm_graph_destroy(g))


FRESH = """
import ctypes as C, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from quicklm_amd import hip
L = hip.lib()
hip.check(L.qlm_set_device(0))
rng = np.random.default_rng(7)
B, n_q, n_kv, hd, max_seq, ctx = 1, 16, 2, 256, 3000, 2900
q = rng.standard_normal((B, n_q, hd)).astype(np.float32)
k = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
v = rng.standard_normal((B, max_seq, n_kv, hd)).astype(np.float32)
dq, dk, dv = (hip.DeviceBuffer.from_numpy(a) for a in (q, k, v))
a, b = hip.DeviceBuffer(q.nbytes), hip.DeviceBuffer(q.nbytes)
st = hip.Stream()
print("capture: first no-allocation call of the process", flush=True)
hip.check(L.qlm_graph_begin(st.ptr))
rc = L.qlm_attention_decode_noalloc(dq.ptr, dk.ptr, dv.ptr, 0, max_seq, ctx, b.ptr, B, n_q, n_kv,
                                    hd, st.ptr)
g = C.c_void_p()
hip.check(L.qlm_graph_end(st.ptr, C.byref(g)))
hip.check(rc)
hip.check(L.qlm_graph_launch(g, st.ptr))
st.sync()
work = hip.DeviceBuffer(L.qlm_gqa_workspace_bytes(B, n_q, hd, max_seq))
hip.call("qlm_attention_decode", dq, dk, dv, 0, max_seq, ctx, a, B, n_q, n_kv, hd, work, None)
hip.sync()
same = np.array_equal(a.to_numpy(q.shape, np.float32), b.to_numpy(q.shape, np.float32))
hip.check(L.qlm_graph_destroy(g))
print("equal" if same else "DIFFERENT", flush=True)
sys.exit(0 if same else 1)
"""


def test_noalloc_first_call_under_capture_in_fresh_process(hip):
    """A fresh process whose first call of the entry point is made under
    stream capture (after qlm_set_device, which resolves the scratch
    address): the capture succeeds and the replay equals the workspace
    form."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", FRESH, root], capture_output=True, text=True,
                       timeout=300)
    say("fresh process:", r.stdout.strip().replace("\n", " | "), r.stderr[-500:])
    assert r.returncode == 0 and "equal" in r.stdout
