"""The no-allocation attention entry point against the one it mirrors.

qlm_attention_decode_noalloc runs qlm_attention_decode's kernels with the
chunk records in the library's static device scratch instead of a caller
workspace. Both are called through the C ABI on the same seeded inputs; the
outputs must be bit-identical (same kernels, same arithmetic per record),
on two calls in a row, the second smaller than the first, and the first is
also checked against the oracle's attention (1e-5 normwise, as the
workspace form's own test).
"""

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


def test_noalloc_attention_oversize_rejected(hip):
    fake = 4096  # rejected on the host before any launch
    assert hip.lib().qlm_attention_decode_noalloc(fake, fake, fake, 0, 32768, 32768, fake, 16,
                                                  16, 2, 256, None) == -4
    assert hip.lib().qlm_attention_decode_noalloc(fake, fake, fake, 1, 32768, 32768, fake, 128,
                                                  16, 2, 256, None) == -4
