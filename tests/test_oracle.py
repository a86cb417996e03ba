"""Pins the CPU oracle (oracle/q3t_oracle.cpp) before it is trusted as the
parity checker.  Each check is independent of the oracle's own code: numpy
(IEEE float16 conversion, float64 arithmetic), closed forms, brute force on
small inputs, Random123 known-answer vectors, the reference's fixture
(tests/golden/det_prefill_token_types.json) and invariants that a dropped
term, a sign error or a transposed operand would break.
"""
import json
import os

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd.synth import Weights, quantize_q8_0, dequantize_q8_0

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def ulp_diff(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7fffffff), a)
    b = np.where(b < 0, -(b & 0x7fffffff), b)
    return np.abs(a - b)


# ------------------------------------------------------------ fp16 conversion
def test_f16_to_f32_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    r = ref[::7]
    finite = np.isfinite(r)
    assert np.array_equal(got[finite].view(np.uint32), r[finite].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(r)]))


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10,
        rng.standard_normal(2000).astype(np.float32) * 1e-5,     # fp16 subnormals
        np.array([65504, 65519.99, 65520, 1e6, -65520, 6e-8, 3e-8, 2.9e-8, 0.0, -0.0], np.float32),
        # exact ties between two fp16 values: 1 + k*2^-11
        (1.0 + (2 * np.arange(50) + 1) * 2.0 ** -11).astype(np.float32),
    ])
    got = orc.f32_to_f16_bits(x)
    ref = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------------------------- exp
def test_expf_within_2_ulp_of_float64():
    x = np.linspace(-86.9, 88.7, 20001, dtype=np.float32)
    x = np.concatenate([x, np.random.default_rng(1).uniform(-20, 20, 5000).astype(np.float32)])
    got = orc.expf(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(got, ref).max() <= 2


def test_expf_special_values():
    L = orc.lib()
    assert L.orc_expf(0.0) == 1.0
    assert L.orc_expf(float("-inf")) == 0.0
    assert L.orc_expf(-87.5) == 0.0                  # flushed below 2^-126
    assert L.orc_expf(89.0) == float("inf")
    assert np.isnan(L.orc_expf(float("nan")))


# ----------------------------------------------------------------- Q8_0
def test_weight_quantisation_matches_converter_formula():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)
    x[:32] = 0.0                                     # all-zero block: d = 0, q = 0
    x[32:64] = np.arange(32, dtype=np.float32) - 15.5    # ties at .5 after scaling
    got = orc.quantize_weights(x)
    ref = quantize_q8_0(x)                            # numpy restatement of gguf-py
    assert np.array_equal(got, ref)
    b = ref.reshape(-1, 34)
    assert np.all(b[0] == 0)


def test_round_half_away_from_zero_in_weight_quantisation():
    # block with max 127 -> d = 1 exactly, values k + 0.5 round away from zero
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5, -3.5]
    q = orc.quantize_weights(x).reshape(34)[2:].view(np.int8)
    assert list(q[1:9]) == [1, 2, 3, -1, -2, -3, 4, -4]


def test_dequantisation_is_d_times_q_bit_exact():
    x = (np.random.default_rng(3).standard_normal(32 * 100) * 0.05).astype(np.float32)
    blocks = quantize_q8_0(x)
    got = orc.dequantize(blocks, x.size)
    b = blocks.reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), (d * q).reshape(-1).view(np.uint32))
    assert np.array_equal(got, dequantize_q8_0(blocks))
    assert np.abs(got - x).max() <= np.abs(x).max() / 127 / 2 * 1.01


def test_activation_quantisation_properties():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(32 * 200).astype(np.float32)
    blocks = orc.quantize_act(x).reshape(-1, 34)
    q = blocks[:, 2:].view(np.int8).astype(np.int32)
    d = blocks[:, :2].copy().view(np.float16).astype(np.float32).ravel()
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    # ggml-cpu x86: d = amax/127 stored fp16, q = rint(x * (127/amax))
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float16).astype(np.float32))
    idv = (np.float32(127) / amax).astype(np.float32)
    assert np.array_equal(q, np.rint(xb * idv[:, None]).astype(np.int32))
    assert np.all(np.abs(q).max(axis=1) == 127)
    # round-half-to-even: amax 127 -> scale 1, 2.5 -> 2, 3.5 -> 4
    t = np.zeros(32, np.float32)
    t[0], t[1], t[2] = 127.0, 2.5, 3.5
    tq = orc.quantize_act(t).reshape(34)[2:].view(np.int8)
    assert (tq[1], tq[2]) == (2, 4)
    z = orc.quantize_act(np.zeros(32, np.float32)).reshape(34)
    assert np.all(z == 0)


# ------------------------------------------------------------------- GEMV
def _q8_exact(wblocks, rows, k, x):
    """fp64 brute force: quantise x the ggml way, then sum exact block terms."""
    xb = orc.quantize_act(x).reshape(-1, 34)
    wb = wblocks.reshape(rows, k // 32, 34)
    dw = wb[:, :, :2].copy().view(np.float16).astype(np.float64)[..., 0]
    qw = wb[:, :, 2:].view(np.int8).astype(np.int64)
    dx = xb[:, :2].copy().view(np.float16).astype(np.float64)[:, 0]
    qx = xb[:, 2:].view(np.int8).astype(np.int64)
    isum = (qw * qx[None]).sum(axis=2)
    return ((dw * dx[None]) * isum).sum(axis=1)


def test_gemv_q8_matches_exact_block_sum():
    rng = np.random.default_rng(5)
    rows, k = 96, 512
    w = (rng.standard_normal(rows * k) * 0.02).astype(np.float32)
    wb = quantize_q8_0(w)
    x = rng.standard_normal(k).astype(np.float32)
    y = orc.gemv(orc.Q8_0, wb, rows, k, x)[0]
    exact = _q8_exact(wb, rows, k, x)
    assert ulp_diff(y, exact.astype(np.float32)).max() <= 1
    # a transposed weight or a dropped activation scale would not match
    assert np.abs(y - exact).max() < 1e-6 * np.abs(exact).max() + 1e-9


def test_gemv_f16_rounds_activation_and_accumulates_exactly():
    rng = np.random.default_rng(6)
    rows, k = 64, 256
    w = (rng.standard_normal((rows, k)) * 0.02).astype(np.float16)
    x = rng.standard_normal(k).astype(np.float32)
    y = orc.gemv(orc.F16, w, rows, k, x)[0]
    ref = (w.astype(np.float64) @ x.astype(np.float16).astype(np.float64)).astype(np.float32)
    assert ulp_diff(y, ref).max() <= 1
    # widened (ffn_down of the F16 model): activation stays fp32
    yw = orc.gemv(orc.F16, w, rows, k, x, widen=True)[0]
    refw = (w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    assert ulp_diff(yw, refw).max() <= 1
    assert not np.array_equal(y, yw)


def test_gemv_identity_and_linearity():
    k = 256
    eye = np.eye(k, dtype=np.float16)
    x = np.random.default_rng(7).standard_normal(k).astype(np.float32)
    y = orc.gemv(orc.F16, eye, k, k, x)[0]
    assert np.array_equal(y, x.astype(np.float16).astype(np.float32))
    # scaling x by a power of two scales the Q8_0 output exactly (d scales, q unchanged)
    w = quantize_q8_0((np.random.default_rng(8).standard_normal(64 * k) * 0.02).astype(np.float32))
    y1 = orc.gemv(orc.Q8_0, w, 64, k, x)[0]
    y4 = orc.gemv(orc.Q8_0, w, 64, k, x * 4)[0]
    assert np.array_equal(y4, y1 * 4)


# ---------------------------------------------------------------- RMSNorm
def test_rmsnorm_closed_form():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(1024).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    y = orc.rmsnorm(x, w, 1e-6)
    ss = np.sum((x * x).astype(np.float64))
    mean = np.float32(ss / 1024)
    scale = np.float32(1.0) / np.sqrt(mean + np.float32(1e-6), dtype=np.float32)
    assert np.array_equal(y, (x * scale) * w)
    c = np.full(128, 3.0, np.float32)
    yc = orc.rmsnorm(c, None, 1e-6)
    assert np.allclose(yc, 3.0 / np.sqrt(9.0 + 1e-6), rtol=1e-6)


# ------------------------------------------------------------------- RoPE
def test_rope_table_and_rotation():
    cos, sin = orc.rope_table(1e6, 128, 64)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)       # pos 0 is the identity
    theta = 1 * (1e6 ** (-2.0 * np.arange(64) / 128))
    assert np.allclose(cos[1], np.cos(theta), atol=2e-6)
    assert np.allclose(sin[1], np.sin(theta), atol=2e-6)
    x = np.random.default_rng(10).standard_normal(128).astype(np.float32)
    y0 = orc.rope(x, cos[0], sin[0])
    assert np.array_equal(y0, x)
    y = orc.rope(x, cos[37], sin[37])
    n_in = x[:64] ** 2 + x[64:] ** 2
    n_out = y[:64] ** 2 + y[64:] ** 2
    assert np.allclose(n_in, n_out, rtol=1e-5)                    # pairwise norm preserved
    e = np.zeros(128, np.float32)
    e[5] = 1.0                                                     # NEOX pairs (i, i+64)
    ye = orc.rope(e, cos[3], sin[3])
    assert ye[5] == cos[3][5] and ye[69] == sin[3][5]
    assert np.count_nonzero(ye) == 2


# -------------------------------------------------------------- attention
def test_attention_single_position_returns_v():
    rng = np.random.default_rng(11)
    q = rng.standard_normal((4, 128)).astype(np.float32)
    k = rng.standard_normal((2, 8, 128)).astype(np.float16)
    v = rng.standard_normal((2, 8, 128)).astype(np.float16)
    out, p = orc.attention(q, k, v, 1)
    assert np.all(p == 1.0)
    assert np.array_equal(out[0], v[0, 0].astype(np.float32))
    assert np.array_equal(out[3], v[1, 0].astype(np.float32))    # GQA: head 3 -> kv head 1


def test_attention_matches_float64_softmax():
    rng = np.random.default_rng(12)
    nh, nkv, hd, nctx, n = 4, 2, 128, 32, 20
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k = rng.standard_normal((nkv, nctx, hd)).astype(np.float16)
    v = rng.standard_normal((nkv, nctx, hd)).astype(np.float16)
    out, p = orc.attention(q, k, v, n)
    for h in range(nh):
        g = h // 2
        s = (k[g, :n].astype(np.float64) @ q[h].astype(np.float16).astype(np.float64)) / np.sqrt(128.0)
        pe = np.exp(s - s.max())
        pe /= pe.sum()
        assert np.allclose(p[h], pe, rtol=1e-5, atol=1e-7)
        o = pe.astype(np.float16).astype(np.float64) @ v[g, :n].astype(np.float64)
        assert np.allclose(out[h], o, rtol=2e-3, atol=2e-3)
    # one-hot: a key aligned with q dominates -> output is (nearly) that value row
    k2 = k.copy()
    k2[0, 7] = (q[0] * 50).astype(np.float16)
    out2, p2 = orc.attention(q, k2, v, n)
    assert p2[0, 7] > 0.999
    assert np.allclose(out2[0], v[0, 7].astype(np.float32), atol=1e-2)


def np_bf16_bits(x):
    """fp32 -> bfloat16 bits, round to nearest even (numpy restatement)."""
    u = np.asarray(x, np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    return np.where(nan, ((u >> np.uint32(16)) | np.uint32(64)).astype(np.uint16), r)


def bf16_to_f64(b):
    return (np.asarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float64)


def test_bf16_conversions():
    rng = np.random.default_rng(13)
    x = np.concatenate([rng.standard_normal(3000).astype(np.float32) * 10, rng.standard_normal(500).astype(np.float32)
                        * 1e-39, np.array([0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-45], np.float32),
                        # exact ties between two bfloat16 values: 1 + (2k+1) 2^-8
                        (1.0 + (2 * np.arange(40) + 1) * 2.0 ** -8).astype(np.float32)])
    L = orc.lib()
    got = np.array([L.orc_f32_to_bf16(float(v)) for v in x], np.uint16)
    assert np.array_equal(got, np_bf16_bits(x))
    # ties go to the even neighbour: 1 + 2^-8 -> 1.0, 1 + 3*2^-8 -> 1 + 2^-6
    assert L.orc_f32_to_bf16(1.0 + 2.0 ** -8) == 0x3F80 and L.orc_f32_to_bf16(1.0 + 3 * 2.0 ** -8) == 0x3F82
    assert (L.orc_f32_to_bf16(float("nan")) & 0x7FC0) == 0x7FC0
    b = rng.integers(0, 65536, 2000).astype(np.uint16)
    b = b[(b & 0x7F80) != 0x7F80]
    assert np.array_equal(np.array([L.orc_bf16_to_f32(int(v)) for v in b], np.float32), bf16_to_f64(b).astype(np.float32))


def test_attention_bf16_cache_matches_float64():
    """Over a bfloat16 cache q and P are rounded to bfloat16 (not fp16): the
    rows match a float64 evaluation with those rounding points; the fp16 form
    misses."""
    rng = np.random.default_rng(14)
    nh, nkv, hd, nctx, n = 4, 2, 128, 40, 33
    q = rng.standard_normal((nh, hd)).astype(np.float32)
    k = np_bf16_bits(rng.standard_normal((nkv, nctx, hd)).astype(np.float32))
    v = np_bf16_bits(rng.standard_normal((nkv, nctx, hd)).astype(np.float32))
    out, p = orc.attention_bf16(q, k, v, n)
    kf, vf = bf16_to_f64(k), bf16_to_f64(v)
    for h in range(nh):
        g = h // 2
        qb = bf16_to_f64(np_bf16_bits(q[h]))
        s = (kf[g, :n] @ qb).astype(np.float32) * np.float32(1.0 / np.sqrt(128.0))
        pe = np.exp(s.astype(np.float64) - s.max())
        pe /= pe.sum()
        assert np.allclose(p[h], pe, rtol=1e-5, atol=1e-7)
        o = bf16_to_f64(np_bf16_bits(p[h])) @ vf[g, :n]
        assert np.allclose(out[h], o, rtol=1e-5, atol=1e-6)
        o16 = p[h].astype(np.float16).astype(np.float64) @ vf[g, :n]
        assert np.abs(out[h] - o16).max() > 1e-4
    # the same values in an fp16 cache (bfloat16 values are exact in fp16 at
    # these magnitudes) attend with fp16-rounded q and P: a different result
    out16, _ = orc.attention(q, kf.astype(np.float16), vf.astype(np.float16), n)
    assert np.abs(out16 - out).max() > 1e-4


# ---------------------------------------------------------------- sampler
def test_argmax_first_index_on_ties():
    x = np.array([0.1, 0.7, 0.2, 0.7, 0.7], np.float32)
    assert orc.argmax(x) == 1


def test_cb0_suppression_penalty_and_eos_ramp():
    V, eos = 3072, 2150
    logits = np.zeros(V, np.float32)
    logits[2500] = 9.0            # suppressed window [V-1024, V) except EOS
    logits[10] = 2.0
    logits[11] = 1.99
    seen = np.zeros(V, np.uint8)
    seen[10] = 1                  # 2.0 / 1.05 < 1.99 -> token 11 wins
    tok, l = orc.sample_cb0(logits, eos, seen, rep=1.05)
    assert tok == 11 and l[2500] == -np.inf and l[eos] == 0.0
    assert l[10] == np.float32(2.0) / np.float32(1.05)
    neg = np.zeros(V, np.float32)
    neg[3] = -1.0
    s3 = np.zeros(V, np.uint8)
    s3[3] = 1
    _, l3 = orc.sample_cb0(neg, eos, s3, rep=1.05)
    assert l3[3] == np.float32(-1.0) * np.float32(1.05)            # negative logits multiply
    # EOS ramp: +0.1 per frame past target_frames, capped at 6
    base = np.zeros(V, np.float32)
    base[5] = 0.45
    assert orc.sample_cb0(base, eos, None, rep=1.0, target_frames=10, frame=14)[0] == 5   # bias 0.4
    assert orc.sample_cb0(base, eos, None, rep=1.0, target_frames=10, frame=15)[0] == eos  # bias 0.5
    _, l4 = orc.sample_cb0(np.zeros(V, np.float32), eos, None, rep=1.0, target_frames=1, frame=500)
    assert l4[eos] == 6.0


def test_top_k_keeps_ties_and_sampling_is_reproducible():
    l = np.full(64, -5.0, np.float32)
    l[[3, 9]] = 1.0               # two tied maxima, top_k = 1 keeps both
    draws = {orc.sample_cp(l, temp=1.0, top_k=1, seed=s, frame=0, group=1) for s in range(40)}
    assert draws == {3, 9}
    a = [orc.sample_cp(np.random.default_rng(0).standard_normal(2048).astype(np.float32), 0.9, 50, 7, f, 3)
         for f in range(5)]
    b = [orc.sample_cp(np.random.default_rng(0).standard_normal(2048).astype(np.float32), 0.9, 50, 7, f, 3)
         for f in range(5)]
    assert a == b


def test_sampling_distribution_follows_softmax():
    logits = np.log(np.array([0.5, 0.3, 0.2], np.float32))
    counts = np.bincount([orc.sample_cp(logits, 1.0, 0, 99, f, 1) for f in range(6000)], minlength=3)
    assert np.allclose(counts / 6000, [0.5, 0.3, 0.2], atol=0.03)


def test_philox_known_answer_vectors():
    # Random123 kat_vectors, philox4x32_10
    assert list(orc.philox(0, 0, 0, 0, 0)) == [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]
    assert list(orc.philox(0xffffffffffffffff, 0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff)) == \
        [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]
    assert list(orc.philox(0x299f31d0a4093822, 0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344)) == \
        [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]
    u = [orc.uniform(1, f, g) for f in range(50) for g in range(3)]
    assert min(u) >= 0.0 and max(u) < 1.0


# ------------------------------------------------------------ model level
@pytest.fixture(scope="module")
def tiny():
    cfg = qcfg.tiny()
    w = Weights(cfg, "q8_0", seed=11)
    o = orc.Oracle(cfg, w, threads=4)
    return cfg, w, o


def test_prefill_equals_sequential_steps(tiny):
    cfg, w, o = tiny
    e = (np.random.default_rng(13).standard_normal((7, cfg.hidden_size)) * 0.05).astype(np.float32)
    o.kv_reset(32)
    hid, logits = o.prefill(e, 0)
    o.kv_reset(32)
    for i in range(7):
        l2, h2 = o.step(e[i], i)
        assert np.array_equal(h2, hid[i])
    assert np.array_equal(l2, logits)


def test_code_pred_greedy_is_argmax_of_heads(tiny):
    cfg, w, o = tiny
    o.kv_reset(32)
    hid = np.random.default_rng(14).standard_normal(cfg.hidden_size).astype(np.float32)
    codes, logits = o.code_pred(hid, 42)
    assert np.array_equal(codes, logits.argmax(axis=1))
    c2, _ = o.code_pred(hid, 43)
    assert not np.array_equal(codes, c2)      # cb0 enters through codec_embd


def test_prefill_layout_matches_reference_fixture(tiny):
    """det_prefill_token_types.json: 10 positions for a 10-token prompt
    ("Hello." in the chat template) with a speaker embedding."""
    cfg, w, o = tiny
    spec = json.load(open(os.path.join(GOLDEN, "det_prefill_token_types.json")))
    meta = json.load(open(os.path.join(GOLDEN, "det_metadata.json")))
    assert spec["prefill_sequence_length"] == 10
    text = np.array([1, 2, 3, 9, 13, 4, 5, 6, 7, 8], np.int32)     # 10 ids as in the fixture
    spk = np.random.default_rng(15).standard_normal(cfg.hidden_size).astype(np.float32)
    pre, trail, pad = o.build_prefill(text, spk, language_id=cfg.english_language_id)
    assert pre.shape[0] == spec["prefill_sequence_length"] == meta["shapes"]["prefill_embedding"][1]
    assert trail.shape[0] == meta["shapes"]["trailing_text_hidden"][1]
    sp = o.text_proj(np.array([cfg.tts_bos_id, cfg.tts_eos_id, cfg.tts_pad_id], np.int32))
    bos, eos, tpad = sp
    assert np.array_equal(pad, tpad)
    ids = {"codec_think_id": cfg.codec_think_id}
    for ent in spec["positions"]:
        p, kind = ent["position"], ent["type"]
        if kind == "role_token":
            exp = o.text_proj(text[p:p + 1])[0]
        elif kind == "codec_overlay":
            tok = ent["token_id"]
            # fixture ids are the reference's defaults; map onto this config's ids
            tok = {2154: cfg.codec_think_id, 2156: cfg.codec_think_bos_id, 2050: cfg.english_language_id,
                   2157: cfg.codec_think_eos_id, 2148: cfg.codec_pad_id}[tok]
            overlay = bos if "tts_bos" in ent["description"] else tpad
            exp = overlay + o.embed_row("codec", 0, tok)
        elif kind == "speaker_overlay":
            exp = tpad + spk
        else:   # text_plus_codec_bos
            exp = o.text_proj(text[3:4])[0] + o.embed_row("codec", 0, cfg.codec_bos_id)
        assert np.array_equal(pre[p], exp.astype(np.float32)), (p, kind)
    assert np.array_equal(trail[0], o.text_proj(text[4:5])[0])
    assert np.array_equal(trail[-1], eos)
    del ids


def test_generate_edge_cases(tiny):
    cfg, w, o = tiny
    text = np.arange(12, dtype=np.int32)
    c0, _ = o.generate(text, None, max_len=0, temperature=0.0)
    assert c0.shape[0] == 0
    with pytest.raises(RuntimeError):
        o.generate(np.arange(3, dtype=np.int32), None, max_len=4)
    ce, _ = o.generate(text, None, max_len=8, temperature=0.0, eos_bias=1e4)
    assert ce.shape[0] == 0                          # EOS at frame 0: nothing emitted
    g1, _ = o.generate(text, None, max_len=6, temperature=0.0)
    g2, _ = o.generate(text, None, max_len=6, temperature=0.0)
    assert g1.shape == (6, 16) and np.array_equal(g1, g2)
    assert np.all(g1[:, 0] < cfg.codec_vocab - 1024)  # suppressed window never sampled
    assert np.all(g1[:, 1:] < cfg.cp_vocab)


def test_golden_codes_fixture(tiny):
    """Regression pin: greedy codes of the tiny Q8_0 model (seed 11) recorded
    by tests/golden/make_golden.py."""
    cfg, w, o = tiny
    path = os.path.join(GOLDEN, "tiny_q8_greedy.npz")
    g = np.load(path)
    codes, first = o.generate(g["text"], g["speaker"], max_len=int(g["max_len"]), temperature=0.0)
    assert np.array_equal(codes, g["codes"])
    assert np.array_equal(first, g["first_logits"])


class _Tensors:
    def __init__(self, d):
        self.tensors = d

    def items(self):
        return self.tensors.items()


def test_mtp_projection_equals_projected_inputs():
    """The 1.7B layout (code predictor narrower than the talker, inputs through
    code_pred.mtp_proj, src/tts_transformer.cpp:1942-1947, :2096-2101), pinned
    against a model of the code predictor's width without the projection whose
    hidden row and embedding tables are the projected rows, formed here in
    numpy: y = fp32(sum of fp16(x) * w, exact) + bias in fp32 (F16 weights).
    A projection applied to the wrong rows, or skipped on the step inputs,
    changes the codes."""
    import dataclasses
    cfg = qcfg.tiny_mtp()
    w = Weights(cfg, "f16", seed=21)
    o = orc.Oracle(cfg, w, threads=4)
    d, dc = cfg.hidden_size, cfg.cp_hidden
    W = w["code_pred.mtp_proj.weight"][2].astype(np.float64).reshape(dc, d)
    b = w["code_pred.mtp_proj.bias"][2].astype(np.float32)

    def proj(rows):
        x = np.asarray(rows, np.float32).astype(np.float16).astype(np.float64)
        return (x @ W.T).astype(np.float32) + b

    cfg2 = dataclasses.replace(cfg, hidden_size=dc)
    w2 = Weights(cfg2, "f16", seed=22)
    t = dict(w2.items())
    for name, v in w.items():
        if name.startswith("code_pred.") and "codec_embd" not in name and "mtp_proj" not in name:
            t[name] = v
    codec = w["talker.codec_embd.weight"][2].astype(np.float32).reshape(cfg.codec_vocab, d)
    t["talker.codec_embd.weight"] = (0, (dc, cfg.codec_vocab), np.ascontiguousarray(proj(codec)))
    for g in range(cfg.n_codebooks - 1):
        e = w[f"code_pred.codec_embd.{g}.weight"][2].astype(np.float32).reshape(cfg.cp_vocab, d)
        t[f"code_pred.codec_embd.{g}.weight"] = (0, (dc, cfg.cp_vocab), np.ascontiguousarray(proj(e)))
    o2 = orc.Oracle(cfg2, _Tensors(t), threads=4)
    rng = np.random.default_rng(23)
    for cb0 in (3, 1500):
        hid = rng.standard_normal(d).astype(np.float32)
        o.kv_reset(16)
        o2.kv_reset(16)
        c1, l1 = o.code_pred(hid, cb0)
        c2, l2 = o2.code_pred(proj(hid[None])[0], cb0)
        assert np.array_equal(c1, c2) and np.array_equal(l1, l2)
        c1, _ = o.code_pred(hid, cb0, temperature=0.9, top_k=50, seed=4, frame=2)
        c2, _ = o2.code_pred(proj(hid[None])[0], cb0, temperature=0.9, top_k=50, seed=4, frame=2)
        assert np.array_equal(c1, c2)


def test_frames_from_cache_equals_generate_rows(tiny):
    """orc_frames continues from the cache a prefill left: prefill + frames
    gives generate_rows' codes, greedy and sampled."""
    cfg, w, o = tiny
    rng = np.random.default_rng(61)
    d = cfg.hidden_size
    pre = (rng.standard_normal((9, d)) * 0.05).astype(np.float32)
    trail = (rng.standard_normal((4, d)) * 0.05).astype(np.float32)
    pad = (rng.standard_normal(d) * 0.05).astype(np.float32)
    for kw in (dict(temperature=0.0), dict(temperature=0.9, top_k=50, seed=3)):
        ref = o.generate_rows(pre, trail, pad, max_len=10, **kw)
        o.kv_reset(9 + 10 + 8)
        _, lg = o.prefill(pre, 0)
        got = o.frames(lg, 9, trail, pad, 10, **kw)
        assert got.shape[0] > 0 and np.array_equal(got, ref)


def test_kv_write_layout_matches_prefill_rows(tiny):
    """orc_kv_write takes rows [n_pos][n_kv_head][head_dim]: the rows a
    prefill stored, read back and written into a cleared cache, make the next
    step identical; the same rows with two KV heads swapped do not."""
    cfg, w, o = tiny
    rng = np.random.default_rng(62)
    d = cfg.hidden_size
    pre = (rng.standard_normal((9, d)) * 0.05).astype(np.float32)
    e = (rng.standard_normal(d) * 0.05).astype(np.float32)
    o.kv_reset(32)
    o.prefill(pre, 0)
    rows = [o.kv_read(il, 9) for il in range(cfg.n_layers)]
    lo, ho = o.step(e, 9)
    o.kv_reset(32)
    for il, (k, v) in enumerate(rows):
        assert k.shape == (9, cfg.n_kv_head, cfg.head_dim)
        o.kv_write(il, k, v)
    # the step reads only the cache and its own input, not the prefill state
    l2, h2 = o.step(e, 9)
    assert np.array_equal(l2, lo) and np.array_equal(h2, ho)
    o.kv_reset(32)
    for il, (k, v) in enumerate(rows):
        o.kv_write(il, k[:, ::-1].copy(), v)
    l3, _ = o.step(e, 9)
    assert not np.array_equal(l3, lo)
    with pytest.raises(RuntimeError):
        o.kv_write(cfg.n_layers, rows[0][0], rows[0][1])
