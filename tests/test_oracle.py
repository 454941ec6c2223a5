"""Pinning the CPU oracle (no GPU).

1. Against the reference itself: oracle/_ref/libqlm_ref_ieee.so is the
   reference's own sources compiled with IEEE flags; the oracle must agree
   bit for bit, op by op, module by module and on whole models.
2. Against mathematics that fixes each function independently of both
   (exact integer sums, closed forms, identities, float64 brute force), so a
   mistake shared by oracle and harness would still be caught.
3. Against the committed golden fixture (reference token stream).
"""

import os

import numpy as np
import pytest

from oracle.oracle import Oracle, OracleModel, Reference, ref_available

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny_greedy.npz")
needs_ref = pytest.mark.skipif(not ref_available("ieee"),
                               reason="reference not built (make -C oracle ref)")


@pytest.fixture(scope="module")
def ref():
    r = Reference("ieee")
    r.init_threads(4)
    return r


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


# ------------------------------------------------------------ 1. vs reference
@needs_ref
@pytest.mark.parametrize("K", [1024, 2560, 1000, 40])
def test_quantizer_vs_reference(orc, ref, rng, K):
    w = (rng.standard_normal((33, K)) * 0.02).astype(np.float32)
    w[1] = 0
    w[2, :16] = 1e-30
    for src in (w, (w.view(np.uint32) >> 16).astype(np.uint16)):
        q1, s1 = orc.quantize(src, 32)
        q2, s2 = ref.quantize(src)
        assert np.array_equal(q1, q2) and np.array_equal(bits(s1), bits(s2))


@needs_ref
@pytest.mark.parametrize("M,K", [(1, 2560), (3, 1024), (2, 1000), (1, 3584)])
def test_matmul_vs_reference(orc, ref, rng, M, K):
    A = rng.standard_normal((M, K)).astype(np.float32)
    q, s = ref.quantize((rng.standard_normal((67, K)) * 0.02).astype(np.float32))
    assert np.array_equal(bits(orc.matmul_i8(A, q, s, 32)), bits(ref.matmul_i8(A, q, s)))


@needs_ref
def test_elementwise_vs_reference(orc, ref, rng):
    for n in (1024, 2560, 1000, 7):
        x = rng.standard_normal((3, n)).astype(np.float32)
        d = rng.standard_normal((3, n)).astype(np.float32)
        w = (rng.standard_normal(n) * 0.02).astype(np.float32)
        assert orc.sumsq(x[0]) == ref.sumsq(x[0])
        assert np.array_equal(bits(orc.rms_norm(x, w, 1e-6)), bits(ref.rms_norm(x, w, 1e-6)))
        a, b = orc.add_rms_norm(x, d, w, 1e-6), ref.add_rms_norm(x, d, w, 1e-6)
        assert np.array_equal(bits(a[0]), bits(b[0])) and np.array_equal(bits(a[1]), bits(b[1]))
        assert np.array_equal(bits(orc.silu_mul(x[0], d[0])), bits(ref.silu_mul(x[0], d[0])))


@needs_ref
def test_rope_and_conv_vs_reference(orc, ref, rng):
    t = rng.standard_normal((4, 256)).astype(np.float32)
    for rot in (32, 64, 256):
        for pos in (0, 1, 999, 32767):
            assert np.array_equal(bits(orc.rope_neox(t, pos, 1e6, rot)),
                                  bits(ref.rope_neox(t, pos, 1e6, rot)))
    x = rng.standard_normal(6144).astype(np.float32)
    st = rng.standard_normal((3, 6144)).astype(np.float32)
    wt = rng.standard_normal((4, 6144)).astype(np.float32)
    for old in range(3):
        a, b = orc.conv1d_tapmajor(x, st, old, wt), ref.conv1d_tapmajor(x, st, old, wt)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def _dn_weights(orc, rng, H, nh, d):
    HD = nh * d

    def lin(n, k):
        return orc.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), 32)

    w = {}
    w["qkv_q"], w["qkv_s"] = lin(3 * HD, H)
    w["z_q"], w["z_s"] = lin(HD, H)
    w["b_q"], w["b_s"] = lin(nh, H)
    w["a_q"], w["a_s"] = lin(nh, H)
    w["out_q"], w["out_s"] = lin(H, HD)
    w["conv_w"] = (rng.standard_normal((3 * HD, 1, 4)) * 0.3).astype(np.float32)
    w["norm_w"] = (1 + rng.standard_normal(d) * 0.02).astype(np.float32)
    w["A_log"] = np.log(rng.uniform(1, 16, nh)).astype(np.float32)
    w["dt_bias"] = (rng.standard_normal(nh) - 4).astype(np.float32)
    return w


@needs_ref
def test_deltanet_module_vs_reference(orc, ref, rng):
    """Qwen3_5GatedDeltaNet::forward over 5 steps (ring wraps) vs the oracle
    composition matmul -> deltanet_core -> matmul."""
    H, nh, d = 512, 2, 128
    HD = nh * d
    w = _dn_weights(orc, rng, H, nh, d)
    mod = ref.deltanet(w, H, nh, d)
    conv = np.zeros((3, 3 * HD), np.float32)
    S = np.zeros((nh, d, d), np.float32)
    wt = np.ascontiguousarray(w["conv_w"].reshape(3 * HD, 4).T)
    for step in range(5):
        x = rng.standard_normal(H).astype(np.float32)
        want = mod.forward(x, step)
        proj = np.concatenate([orc.matmul_i8(x[None], w[k + "_q"], w[k + "_s"], 32)[0]
                               for k in ("qkv", "z", "b", "a")])
        core = orc.deltanet_core(proj, conv, step % 3, wt, w["A_log"], w["dt_bias"], w["norm_w"],
                                 S, nh, d)
        got = orc.matmul_i8(core[None], w["out_q"], w["out_s"], 32)[0]
        assert np.array_equal(bits(got), bits(want)), step


@needs_ref
@pytest.mark.parametrize("gated", [True, False])
def test_gqa_module_vs_reference(orc, ref, rng, gated):
    H, nq, nkv, hd, rot, theta, L = 512, 4, 2, 128, 32, 1e6, 64

    def lin(n, k):
        return orc.quantize((rng.standard_normal((n, k)) * 0.02).astype(np.float32), 32)

    w = {}
    qr = (2 if gated else 1) * nq * hd
    w["q_q"], w["q_s"] = lin(qr, H)
    w["k_q"], w["k_s"] = lin(nkv * hd, H)
    w["v_q"], w["v_s"] = lin(nkv * hd, H)
    w["o_q"], w["o_s"] = lin(H, nq * hd)
    w["q_norm"] = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    w["k_norm"] = (rng.standard_normal(hd) * 0.02).astype(np.float32)
    mod = ref.gqa(w, H, nq, nkv, hd, rot, theta, L)
    kc = np.zeros((L, nkv, hd), np.float32)
    vc = np.zeros_like(kc)
    for pos in range(6):
        x = rng.standard_normal(H).astype(np.float32)
        want = mod.forward(x, pos)
        qkv = np.concatenate([orc.matmul_i8(x[None], w[k + "_q"], w[k + "_s"], 32)[0]
                              for k in ("q", "k", "v")])
        core = orc.gqa_core(qkv, w["q_norm"], w["k_norm"], theta, rot, kc, vc, pos, nq, nkv, hd,
                            gated)
        got = orc.matmul_i8(core[None], w["o_q"], w["o_s"], 32)[0]
        assert np.array_equal(bits(got), bits(want)), pos


@needs_ref
def test_micro_model_vs_reference(orc, ref, tmp_path):
    """Whole decode loop on a few-MB model: oracle logits bit-identical to the
    reference DecoderModel, batched prefill included (forward_batch)."""
    from quicklm_amd import synth

    d = str(tmp_path)
    synth.write_model(d, "micro")
    prompt = synth.prompt_tokens(20, seed=3, vocab=4096)[0]
    m = ref.load_model(d, 64, "int8")
    want, _, _, wlg = m.generate(prompt, 10, keep_logits=True)
    got, glg = OracleModel(d, 64, orc).generate(prompt, 10, keep_logits=True)
    assert np.array_equal(got, want)
    assert np.array_equal(bits(glg), bits(wlg))
    # reference self-check (main.cpp:405-449): forward_batch == sequential forward
    m.reset()
    seq = np.stack([m.forward(int(t), p) for p, t in enumerate(prompt[:8])])
    m.reset()
    assert np.array_equal(bits(m.forward_batch(prompt[:8], 0)), bits(seq))


@needs_ref
@pytest.mark.parametrize("K", [1024, 2560, 1000, 40, 33])
def test_q4_quantizer_vs_reference(orc, ref, rng, K):
    """int4 (Q4_0) quantiser, f32 and bf16 rows, including an all-zero row,
    tiny values, ragged block tails and an odd K."""
    w = (rng.standard_normal((33, K)) * 0.02).astype(np.float32)
    w[1] = 0
    w[2, :16] = 1e-30
    w[3, :min(K, 32)] = (np.arange(32, dtype=np.float32) * np.float32(0.125) - 2)[:min(K, 32)]
    for src in (w, (w.view(np.uint32) >> 16).astype(np.uint16)):
        q1, s1 = orc.quantize_q4(src)
        q2, s2 = ref.quantize_q4(src)
        assert q1.shape == (33, (K + 1) // 2)
        assert np.array_equal(q1, q2) and np.array_equal(bits(s1), bits(s2))


@needs_ref
@pytest.mark.parametrize("M,K", [(1, 2560), (3, 1024), (2, 1000), (1, 3584)])
def test_q4_matmul_vs_reference(orc, ref, rng, M, K):
    """The int4 matmul, and the reference's own int4 matmul equals its int8
    matmul over the unpacked values (the identity the device path builds on)."""
    A = rng.standard_normal((M, K)).astype(np.float32)
    p, s = ref.quantize_q4((rng.standard_normal((67, K)) * 0.02).astype(np.float32))
    got = ref.matmul_i4(A, p, s)
    assert np.array_equal(bits(orc.matmul_i4(A, p, s)), bits(got))
    assert np.array_equal(bits(ref.matmul_i8(A, orc.unpack_q4(p, K), s)), bits(got))


@needs_ref
@pytest.mark.parametrize("M,K", [(1, 2560), (3, 1024), (2, 1000), (1, 3584), (2, 45)])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_native_matmul_vs_reference(orc, ref, rng, M, K, dtype):
    """Native (unquantised) weights: fp32 rows (dot_avx2) and bf16 rows
    (dot_avx2_bf16), ragged K included."""
    A = rng.standard_normal((M, K)).astype(np.float32)
    W = (rng.standard_normal((67, K)) * 0.02).astype(np.float32)
    if dtype == "bf16":
        W = (W.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(bits(orc.matmul_w(A, W)), bits(ref.matmul_w(A, W)))


# ------------------------------------------------------------ 2. mathematics
def test_native_matmul_exact_and_close(orc, rng):
    """Integer activations and weights: every partial sum is exact, so fp32
    and bf16 rows give the float64 product exactly; random inputs within
    fp32 accumulation error of float64."""
    K = 1000
    x = rng.integers(-16, 17, (2, K)).astype(np.float32)
    w = rng.integers(-100, 101, (30, K)).astype(np.float32)
    want = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.array_equal(orc.matmul_w(x, w).astype(np.float64), want)
    wb = (w.view(np.uint32) >> 16).astype(np.uint16)  # small integers are exact in bf16
    assert np.array_equal(orc.matmul_w(x, wb).astype(np.float64), want)
    xr = rng.standard_normal((2, K)).astype(np.float32)
    wr = rng.standard_normal((30, K)).astype(np.float32)
    ref = xr.astype(np.float64) @ wr.astype(np.float64).T
    assert np.abs(orc.matmul_w(xr, wr) - ref).max() / np.abs(ref).max() < 1e-5


def test_q4_quantizer_known_answers(orc):
    """Scale = max|x|/8 (1 for an all-zero block); exact multiples of the
    scale map to those integers, the positive maximum (8 scales) clamps to 7;
    exact halves round half to even in the 8-wide part and half away from
    zero in a block's ragged tail; nibble = value + 8, low nibble = even
    column, an odd K's last byte carries value 0 above its last column."""
    s = np.float32(0.01)
    row = np.zeros((1, 64), np.float32)
    row[0, :8] = np.array([8, -8, 3, -3, 7, 0.5, 1.5, -2.5], np.float32) * s
    p, sc = orc.quantize_q4(row)
    assert sc[0, 0] == np.float32(8 * s) / np.float32(8) and sc[0, 1] == 1.0
    v = orc.unpack_q4(p, 64)[0]
    inv = np.float32(1) / sc[0, 0]
    expect = np.clip(np.rint(row[0, :8] * inv), -8, 7).astype(np.int8)
    assert list(expect[[0, 1, 5, 6, 7]]) == [7, -8, 0, 2, -2]
    assert np.array_equal(v[:8], expect) and not v[8:].any()
    assert np.all(p[0, 16:] == 0x88)  # zero block: value 0 in both nibbles
    # ragged tail (K = 36: block 1 holds 4 columns, all past the 8-wide part)
    t = np.zeros((1, 36), np.float32)
    t[0, 32:36] = np.array([8, 0.5, -0.5, 2.5], np.float32)  # scale 1: lround
    pt, st = orc.quantize_q4(t)
    assert st[0, 1] == 1.0 and list(orc.unpack_q4(pt, 36)[0, 32:]) == [7, 1, -1, 3]
    # odd K: the high nibble of the last byte is 8 (value 0)
    po, _ = orc.quantize_q4(np.array([[0.08, -0.08, 0.04]], np.float32))
    assert po.shape == (1, 2) and po[0, 1] >> 4 == 8
    assert list(orc.unpack_q4(po, 3)[0]) == [7, -8, 4]


def test_q4_unpack_layout(orc, rng):
    p = rng.integers(0, 256, (3, 50), dtype=np.uint8)
    q = orc.unpack_q4(p, 99)
    lo = (p & 15).astype(np.int16) - 8
    hi = (p >> 4).astype(np.int16) - 8
    want = np.stack([lo, hi], axis=2).reshape(3, 100)[:, :99]
    assert np.array_equal(q, want.astype(np.int8))


def test_quantizer_known_answers(orc):
    """Scale = max|x|/127; values at exact multiples of the scale map to those
    integers; ties at .5 round half to even; an all-zero group has scale 1."""
    s = np.float32(0.01)
    row = np.zeros((1, 64), np.float32)
    row[0, 0] = 127 * s
    row[0, 1] = -127 * s
    row[0, 2:10] = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 3.0, 126.0, -64.0], np.float32) * s
    q, sc = orc.quantize(row, 32)
    inv = np.float32(1) / sc[0, 0]
    assert sc[0, 0] == np.float32(127 * s) / np.float32(127)
    expect = np.rint(row[0, :32] * inv).astype(np.int32)
    assert np.array_equal(q[0, :32], np.clip(expect, -127, 127))
    assert sc[0, 1] == 1.0 and not q[0, 32:].any()
    # half-to-even on exact halves
    q2, _ = orc.quantize(np.array([[127, 0.5, 1.5, 2.5, -2.5] + [0] * 27], np.float32), 32)
    assert list(q2[0, 1:5]) == [0, 2, 2, -2]


def test_quantizer_per_row_group(orc, rng):
    w = (rng.standard_normal((5, 96)) * 0.02).astype(np.float32)
    q, s = orc.quantize(w, 96)
    assert s.shape == (5, 1)
    assert np.allclose(s[:, 0], np.abs(w).max(1) / 127, rtol=1e-7)
    assert np.abs(q.astype(np.float32) * s - w).max() <= s.max() / 2 * 1.0001


def test_oracle_model_per_row_scales(orc, tmp_path):
    """group="row" quantises every matrix (lm_head included) with one scale
    per output row; its logits stay within quantisation noise of group 32."""
    from quicklm_amd import synth

    d = str(tmp_path)
    synth.write_model(d, "micro")
    prompt = synth.prompt_tokens(20, seed=3, vocab=4096)[0]
    _, la = OracleModel(d, 64, orc).generate(prompt, 4, keep_logits=True)
    m = OracleModel(d, 64, orc, group="row")
    _, lb = m.generate(prompt, 4, keep_logits=True)
    assert all(s.shape == (q.shape[0], 1) for q, s in m.q.values()) and len(m.q) > 10
    assert m.lm[1].shape == (m.embed.shape[0], 1)
    rel = np.abs(la - lb).max(1) / np.abs(la).max(1)
    assert (rel > 0).all() and (rel < 0.1).all()
    with pytest.raises(ValueError):
        OracleModel(d, 64, orc, group=64)


def test_matmul_exact_on_integers(orc, rng):
    """Integer activations, int8 weights, power-of-two scales: every partial
    sum is an exact integer multiple of the scale, so the result equals the
    float64 product exactly, whatever the summation order."""
    K = 1024
    q = rng.integers(-127, 128, (40, K), dtype=np.int8)
    s = (2.0 ** rng.integers(-6, -1, (40, K // 32))).astype(np.float32)
    x = rng.integers(-16, 17, (2, K)).astype(np.float32)
    want = np.einsum("mk,nk->mn", x.astype(np.float64),
                     q.astype(np.float64) * np.repeat(s, 32, axis=1).astype(np.float64))
    assert np.array_equal(orc.matmul_i8(x, q, s, 32).astype(np.float64), want)
    # per-row scale equals group-32 scale when all blocks share it
    s_row = np.ascontiguousarray(s[:, :1])
    s_rep = np.ascontiguousarray(np.repeat(s_row, K // 32, axis=1))
    assert np.array_equal(orc.matmul_i8(x, q, s_rep, 32), orc.matmul_i8(x, q, s_row, K))


def test_rms_norm_closed_form(orc, rng):
    x = rng.standard_normal((4, 2560)).astype(np.float32)
    w = (rng.standard_normal(2560) * 0.02).astype(np.float32)
    y = orc.rms_norm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-6) * (1 + w)
    assert np.abs(y - want).max() < 1e-5
    # scale invariance (eps negligible at this magnitude)
    assert np.abs(orc.rms_norm(x * 8, w, 1e-6) - y).max() < 1e-5


def test_rope_identity_and_rotation(orc, rng):
    t = rng.standard_normal((3, 128)).astype(np.float32)
    assert np.array_equal(orc.rope_neox(t, 0, 1e6, 64), t)  # cos 0 = 1, sin 0 = 0
    r = orc.rope_neox(t, 123, 1e6, 64)
    assert np.array_equal(r[:, 64:], t[:, 64:])  # pass-through dims
    n0 = np.hypot(t[:, :32], t[:, 32:64])
    n1 = np.hypot(r[:, :32], r[:, 32:64])
    assert np.abs(n0 - n1).max() < 1e-5  # a rotation keeps pair norms
    inv = 1.0 / (1e6 ** (np.arange(32) * 2 / 64))
    ang = 123 * inv
    want = t[:, :32] * np.cos(ang) - t[:, 32:64] * np.sin(ang)
    assert np.abs(r[:, :32] - want).max() < 1e-5


def test_attention_closed_forms(orc, rng):
    nq, nkv, hd = 4, 2, 128
    q = rng.standard_normal((nq, hd)).astype(np.float32)
    k = rng.standard_normal((10, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((10, nkv, hd)).astype(np.float32)
    out = orc.attention(q, k, v, 1)  # one position: softmax weight 1
    assert np.array_equal(out[:2], np.broadcast_to(v[0, 0], (2, hd)))
    kk = np.broadcast_to(k[:1], k.shape).copy()  # equal keys: mean of V
    out = orc.attention(q, kk, v, 7)
    assert np.abs(out[2:] - v[:7, 1].mean(0)).max() < 1e-6
    out = orc.attention(q, k, v, 10)
    s = np.einsum("hd,phd->hp", q.astype(np.float64),
                  np.repeat(k, 2, axis=1).astype(np.float64)) / np.sqrt(hd)
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = np.einsum("hp,phd->hd", p, np.repeat(v, 2, axis=1).astype(np.float64))
    assert np.abs(out - want).max() < 1e-5


def test_delta_rule_closed_forms(orc, rng):
    B, H, d = 1, 3, 128
    q = rng.standard_normal((B, H, d)).astype(np.float32)
    k = rng.standard_normal((B, H, d)).astype(np.float32)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    v = rng.standard_normal((B, H, d)).astype(np.float32)
    S = (rng.standard_normal((B, H, d, d)) * 0.1).astype(np.float32)
    one, zero = np.ones((B, H), np.float32), np.zeros((B, H), np.float32)
    # beta = 0, decay = 1: state unchanged, o = q.S / sqrt(d)
    o, S1 = orc.gated_delta_step(q, k, v, one, zero, S)
    assert np.array_equal(S1, S)
    assert np.abs(o - np.einsum("bhi,bhij->bhj", q, S) / np.sqrt(d)).max() < 1e-5
    # decay = 0: S = beta k v^T
    beta = np.full((B, H), 0.7, np.float32)
    _, S2 = orc.gated_delta_step(q, k, v, zero, beta, S)
    assert np.abs(S2 - 0.7 * np.einsum("bhi,bhj->bhij", k, v)).max() < 1e-6
    # general step in float64
    dec = np.full((B, H), 0.9, np.float32)
    o3, S3 = orc.gated_delta_step(q, k, v, dec, beta, S)
    Sd = S.astype(np.float64) * 0.9
    kv = np.einsum("bhi,bhij->bhj", k, Sd)
    Sw = Sd + 0.7 * np.einsum("bhi,bhj->bhij", k, v - kv)
    assert np.abs(S3 - Sw).max() < 1e-5
    assert np.abs(o3 - np.einsum("bhi,bhij->bhj", q, Sw) / np.sqrt(d)).max() < 1e-5


def test_argmax_first_max(orc):
    x = np.array([1, 5, 5, -1, 5], np.float32)
    assert orc.argmax(x) == 1
    assert orc.argmax(np.full(9, -np.inf, np.float32)) == 0


# ------------------------------------------------------------ 3. golden fixture
def test_golden_fixture_is_consistent():
    g = np.load(GOLDEN)
    assert g["prompt"].shape == (128,) and g["tokens"].shape == (64,)
    assert np.array_equal(g["top_idx"][:, 0], g["tokens"])  # greedy = top-1
    assert (g["margin"] >= 0).all()
    assert np.all(np.diff(g["top_val"], axis=1) <= 0)


@pytest.mark.slow
def test_tiny_model_oracle_matches_golden(orc, tmp_path):
    """The oracle model reproduces the reference's 64-token stream and its
    top-32 logits bit for bit on the 24-layer tiny model."""
    from quicklm_amd import synth

    g = np.load(GOLDEN)
    d = str(tmp_path)
    synth.write_model(d, "tiny")
    toks, lg = OracleModel(d, 2048, orc).generate(g["prompt"], 64, keep_logits=True)
    assert np.array_equal(toks, g["tokens"])
    assert np.array_equal(bits(np.take_along_axis(lg, g["top_idx"].astype(np.int64), 1)),
                          bits(g["top_val"]))
