"""HIP path vs the CPU oracle, through the device C ABI (include/q3t_dev.h).

The numerics contract makes the two bit-identical (fp64 accumulation of exact
terms, identical rounding points, the same exp and RoPE table), so most
checks are exact; the contractual bounds from the task (logits within 1e-2
max-abs, identical greedy codebook tokens) are asserted as well.
"""
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import driver
from qwen3_tts_amd.device import Device, DeviceError
from qwen3_tts_amd.synth import Weights, dequantize_q8_0

pytestmark = pytest.mark.gpu

LOGIT_TOL = 1e-2   # max-abs logits tolerance (F16 path) from the parity contract


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def make(cfg, wtype, seed=7, n_ctx=256, norm_mode="one"):
    w = Weights(cfg, wtype, seed=seed, norm_mode=norm_mode)
    dev = Device(cfg)
    dev.upload_weights(w)
    dev.kv_reserve(n_ctx)
    o = orc.Oracle(cfg, w, threads=8)
    o.kv_reset(n_ctx)
    return w, dev, o


@pytest.fixture(params=["persistent", "graph"])
def frame_path(request, monkeypatch):
    """Runs a frame-loop test on both implementations: the persistent
    cooperative frame kernel (the default, Q8_0 or F16 layers) and the
    captured multi-kernel graph (Q3T_FRAME_KERNEL=0)."""
    monkeypatch.setenv("Q3T_FRAME_KERNEL", "1" if request.param == "persistent" else "0")
    return request.param


def check_path(dev, wtype, frame_path):
    us, n, path = dev.frames_stats()
    want = (1, 3) if frame_path == "persistent" else (0,)
    assert path in want, (frame_path, wtype, path)


@pytest.fixture(scope="module", params=["q8_0", "f16"])
def tiny_model(request):
    cfg = qcfg.tiny()
    say(f"[gpu] tiny model {request.param}")
    w, dev, o = make(cfg, request.param)
    yield cfg, w, dev, o
    dev.close()


def test_upload_roundtrip_and_dequant(tiny_model):
    cfg, w, dev, o = tiny_model
    for name in ["talker.blk.0.attn_q.weight", "talker.blk.1.ffn_down.weight", "talker.codec_head.weight",
                 "code_pred.blk.0.attn_v.weight", "talker.output_norm.weight"]:
        ttype, ne, arr = w[name]
        back = dev.download(name, arr.nbytes)
        assert np.array_equal(back, arr.view(np.uint8).ravel()), name
        if ttype == 8:
            deq = dev.dequantize(name, ne[0] * ne[1])
            assert np.array_equal(deq.view(np.uint32), dequantize_q8_0(arr).view(np.uint32)), name
            assert np.array_equal(deq.view(np.uint32), orc.dequantize(arr, ne[0] * ne[1]).view(np.uint32))


@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_ranged_upload_equals_whole_upload(wtype):
    """q3t_dev_upload_tensor_rows: every tensor sent in ranges of 7 rows,
    the first range first and the others in reverse order (Q8_0 blocks
    repacked on the device), downloads equal the whole-tensor upload's bytes,
    Q8_0 dequantises bit-exactly, and a prefill plus a code-predictor pass
    equal the oracle's.  A tensor missing a range is reported by name."""
    cfg = qcfg.tiny()
    w = Weights(cfg, wtype, seed=19)
    dev = Device(cfg)
    try:
        dev.upload_weights(w, chunk_rows=7)
        for name in ["talker.blk.0.attn_q.weight", "talker.blk.0.attn_v.weight", "talker.blk.1.ffn_down.weight",
                     "talker.codec_head.weight", "talker.text_embd.weight", "code_pred.lm_head.3.weight",
                     "talker.output_norm.weight"]:
            ttype, ne, arr = w[name]
            assert np.array_equal(dev.download(name, arr.nbytes), arr.view(np.uint8).ravel()), name
            if ttype == 8:
                deq = dev.dequantize(name, ne[0] * ne[1])
                assert np.array_equal(deq.view(np.uint32), dequantize_q8_0(arr).view(np.uint32)), name
        o = orc.Oracle(cfg, w, threads=4)
        dev.kv_reserve(32)
        o.kv_reset(32)
        embd = (np.random.default_rng(20).standard_normal((6, cfg.hidden_size)) * 0.05).astype(np.float32)
        hg, lg = dev.prefill(embd, 0)
        ho, lo = o.prefill(embd, 0)
        assert np.array_equal(hg, ho) and np.array_equal(lg, lo)
        cg, _ = dev.code_pred(ho[-1], 11)
        co, _ = o.code_pred(ho[-1], 11)
        assert np.array_equal(cg, co)
        o.close()
    finally:
        dev.close()
    # one range short: the first compute call names the tensor
    dev = Device(cfg)
    try:
        items = list(w.items())
        for name, (ttype, ne, arr) in items:
            if name == "talker.blk.1.ffn_up.weight":
                flat = np.ascontiguousarray(arr).view(np.uint8).reshape(ne[1], -1)
                dev.upload_rows(name, ttype, ne, 0, flat[: ne[1] - 5])
            else:
                dev.upload(name, ttype, ne, arr)
        dev.kv_reserve(16)
        with pytest.raises(Exception, match="talker.blk.1.ffn_up.weight incomplete"):
            dev.prefill(embd[:2], 0)
    finally:
        dev.close()


@pytest.fixture(params=["gemv", "mfma"])
def prefill_path(request, monkeypatch):
    """Runs a prefill test on the chunked GEMV prefill and on the int8 MFMA
    prefill (Q8_0 models; F16 models always take the GEMV path)."""
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "1" if request.param == "mfma" else "0")
    return request.param


def test_prefill_and_steps_match_oracle(tiny_model, prefill_path):
    cfg, w, dev, o = tiny_model
    rng = np.random.default_rng(1)
    d = cfg.hidden_size
    embd = (rng.standard_normal((10, d)) * 0.05).astype(np.float32)
    say(f"[gpu] prefill 10 rows ({prefill_path})")
    hid_g, log_g = dev.prefill(embd, 0)
    hid_o, log_o = o.prefill(embd, 0)
    assert np.abs(log_g - log_o).max() <= LOGIT_TOL
    assert np.array_equal(hid_g, hid_o)
    assert np.array_equal(log_g, log_o)
    for s in range(6):
        e = (rng.standard_normal(d) * 0.05).astype(np.float32)
        lg, hg = dev.talker_step(e, 10 + s)
        lo, ho = o.step(e, 10 + s)
        assert np.abs(lg - lo).max() <= LOGIT_TOL
        assert np.array_equal(lg, lo), f"step {s}: max diff {np.abs(lg - lo).max()}"
        assert np.array_equal(hg, ho)


@pytest.mark.parametrize("kv", ["f16", "bf16"])
@pytest.mark.parametrize("att", ["mfma", "rows"])
def test_tiled_prefill_attention_paths(wtype_tiny, kv, att, monkeypatch):
    """A 100-row prefill after 37 cached positions on the tiled prefill
    (MFMA attention over 64-row tiles, or Q3T_PF_ATT_MFMA=0 one workgroup per
    row), then 35, 72, 12 and 150 rows more (72, 12 and 150 leave remainders of
    8, 12 and 22 rows past the last full 64-row tile, which the F16 GEMM gives
    to its tail workgroups; 150 rows are three tiles, whose middle tile the
    scores kernel deals out over the pairs' workgroups): hidden rows and
    logits bit for bit the oracle's."""
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "1")
    monkeypatch.setenv("Q3T_PF_ATT_MFMA", "1" if att == "mfma" else "0")
    cfg = qcfg.tiny()
    w, dev, o = make(cfg, wtype_tiny, seed=43, n_ctx=512)
    try:
        if kv == "bf16":
            dev.kv_set_type(30)
            o.kv_set_type(30)
            o.kv_reset(512)
        rng = np.random.default_rng(44)
        d = cfg.hidden_size
        for n_past, n in ((0, 37), (37, 100), (137, 35), (172, 72), (244, 12), (256, 150)):
            rows = (rng.standard_normal((n, d)) * 0.5).astype(np.float32)
            say(f"[gpu] tiled prefill {n} rows at {n_past} ({wtype_tiny}, {kv} KV, {att})")
            hg, lg = dev.prefill(rows, n_past)
            ho, lo = o.prefill(rows, n_past)
            assert np.array_equal(hg, ho) and np.array_equal(lg, lo), (n_past, n)
    finally:
        dev.close()


@pytest.fixture(params=["q8_0", "f16"])
def wtype_tiny(request):
    return request.param


def test_code_pred_greedy_matches_oracle(tiny_model):
    cfg, w, dev, o = tiny_model
    rng = np.random.default_rng(2)
    hid = rng.standard_normal(cfg.hidden_size).astype(np.float32)
    for cb0 in (0, 17, 2047):
        cg, lg = dev.code_pred(hid, cb0)
        co, lo = o.code_pred(hid, cb0)
        assert np.abs(lg - lo).max() <= LOGIT_TOL
        assert np.array_equal(lg, lo)
        assert np.array_equal(cg, co)
        assert np.array_equal(cg, lg.argmax(axis=1))


def test_code_pred_sampled_matches_oracle(tiny_model):
    cfg, w, dev, o = tiny_model
    hid = np.random.default_rng(3).standard_normal(cfg.hidden_size).astype(np.float32)
    for seed in (1, 99):
        cg, _ = dev.code_pred(hid, 5, temperature=0.9, top_k=50, seed=seed, frame=3)
        co, _ = o.code_pred(hid, 5, temperature=0.9, top_k=50, seed=seed, frame=3)
        assert np.array_equal(cg, co)


def test_predict_codes_matches_oracle(tiny_model):
    """q3t_dev_predict_codes, the single-pass code predictor
    (src/tts_transformer.cpp:2531-2581): the 15 heads' logits bit for bit the
    oracle's, with and without the 15 previous codes (including the last id
    of each table); a code outside its table is an error."""
    cfg, w, dev, o = tiny_model
    rng = np.random.default_rng(21)
    for i in range(3):
        hid = (rng.standard_normal(cfg.hidden_size) * 0.5).astype(np.float32)
        prev = rng.integers(0, cfg.cp_vocab, cfg.n_codebooks - 1).astype(np.int32)
        if i == 2:
            prev[:] = cfg.cp_vocab - 1
        for p in (None, prev):
            lg = dev.predict_codes(hid, p)
            lo = o.predict_codes(hid, p)
            assert np.array_equal(lg, lo), (i, p is None, np.abs(lg - lo).max())
    bad = np.zeros(cfg.n_codebooks - 1, np.int32)
    bad[14] = -1
    with pytest.raises(DeviceError, match="out of range"):
        dev.predict_codes(hid, bad)


@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_predict_codes_mtp_layout(wtype):
    """The single-pass predictor in the 1.7B layout: the input row passes
    through code_pred.mtp_proj into the narrower code predictor."""
    cfg = qcfg.tiny_mtp()
    w, dev, o = make(cfg, wtype, seed=23)
    try:
        rng = np.random.default_rng(24)
        for i in range(2):
            hid = (rng.standard_normal(cfg.hidden_size) * 0.5).astype(np.float32)
            prev = rng.integers(0, cfg.cp_vocab, cfg.n_codebooks - 1).astype(np.int32)
            for p in (None, prev):
                assert np.array_equal(dev.predict_codes(hid, p), o.predict_codes(hid, p)), (i, p is None)
    finally:
        dev.close()


def test_predict_codes_between_frame_runs(tiny_model, frame_path):
    """predict_codes between frames_run calls leaves the frame loop alone:
    the codes equal the oracle's uninterrupted run, and each interleaved call
    equals the oracle's."""
    cfg, w, dev, o = tiny_model
    text = np.random.default_rng(25).integers(0, cfg.text_vocab - 8, 16).astype(np.int32)
    hid = (np.random.default_rng(26).standard_normal(cfg.hidden_size) * 0.5).astype(np.float32)
    co, _ = o.generate(text, None, max_len=20, temperature=0.0)
    calls = []

    def between(codes, n_cb, frame):
        if frame % 5 == 4:
            calls.append((codes[1:].copy(), dev.predict_codes(hid, codes[1:])))
        return True

    say(f"[gpu] predict_codes between frame runs ({frame_path})")
    cg = driver.generate(dev, cfg, text, None, max_len=20, temperature=0.0, chunk=5, on_frame=between)
    check_path(dev, w.wtype, frame_path)
    assert np.array_equal(cg, co)
    assert len(calls) == co.shape[0] // 5
    for prev, lg in calls:
        assert np.array_equal(lg, o.predict_codes(hid, prev))


def test_text_proj_and_embeddings(tiny_model):
    cfg, w, dev, o = tiny_model
    toks = np.array([0, 5, cfg.text_vocab - 1, 1234, 77, 3], np.int32)
    assert np.array_equal(dev.text_proj(toks), o.text_proj(toks))
    rows = dev.embed_rows(0, 0, [cfg.codec_bos_id, 3])
    assert np.array_equal(rows[0], o.embed_row("codec", 0, cfg.codec_bos_id))
    rows = dev.embed_rows(1, 14, [2047])
    assert np.array_equal(rows[0], o.embed_row("cp", 14, 2047))


def test_generate_greedy_64_frames(tiny_model, frame_path):
    cfg, w, dev, o = tiny_model
    text = np.random.default_rng(4).integers(0, cfg.text_vocab - 8, 32).astype(np.int32)
    spk = np.random.default_rng(5).standard_normal(cfg.hidden_size).astype(np.float32)
    say("[gpu] generate greedy 64")
    co, _ = o.generate(text, spk, max_len=64, temperature=0.0, top_k=0)
    cg = driver.generate(dev, cfg, text, spk, max_len=64, temperature=0.0, top_k=0, chunk=16)
    check_path(dev, w.wtype, frame_path)
    assert co.shape == cg.shape, (co.shape, cg.shape)
    assert np.array_equal(cg, co)


def test_generate_sampled_matches_oracle(tiny_model, frame_path):
    cfg, w, dev, o = tiny_model
    text = np.random.default_rng(6).integers(0, cfg.text_vocab - 8, 20).astype(np.int32)
    say("[gpu] generate sampled 24")
    co, _ = o.generate(text, None, max_len=24, temperature=0.9, top_k=50, seed=11)
    cg = driver.generate(dev, cfg, text, None, max_len=24, temperature=0.9, top_k=50, seed=11, chunk=5)
    check_path(dev, w.wtype, frame_path)
    assert np.array_equal(cg, co)


def test_generate_eos_bias_stops(tiny_model, frame_path):
    cfg, w, dev, o = tiny_model
    text = np.arange(12, dtype=np.int32)
    cg = driver.generate(dev, cfg, text, None, max_len=8, temperature=0.0, eos_bias=1e4)
    co, _ = o.generate(text, None, max_len=8, temperature=0.0, eos_bias=1e4)
    assert cg.shape[0] == 0 and co.shape[0] == 0


def test_generate_target_frames_ramp(tiny_model, frame_path):
    cfg, w, dev, o = tiny_model
    text = np.arange(3, 20, dtype=np.int32)
    co, _ = o.generate(text, None, max_len=40, temperature=0.0, eos_bias=0.0, target_frames=2)
    cg = driver.generate(dev, cfg, text, None, max_len=40, temperature=0.0, eos_bias=0.0, target_frames=2, chunk=7)
    check_path(dev, w.wtype, frame_path)
    assert np.array_equal(cg, co)


def test_callback_abort(tiny_model, frame_path):
    cfg, w, dev, o = tiny_model
    text = np.arange(10, 30, dtype=np.int32)
    seen = []

    def cb(codes, n, frame):
        seen.append(frame)
        return frame < 4

    cg = driver.generate(dev, cfg, text, None, max_len=30, temperature=0.0, on_frame=cb, chunk=8)
    assert seen == [0, 1, 2, 3, 4]
    assert cg.shape[0] == 5


def test_attention_capture_matches_oracle(tiny_model, frame_path):
    """q3t_dev_set_attn_capture: the post-softmax rows of one talker layer,
    one per talker step (single steps and every frame of the loop but the
    last), bit for bit the oracle's; capture runs the multi-kernel step."""
    cfg, w, dev, o = tiny_model
    rng = np.random.default_rng(12)
    d = cfg.hidden_size
    try:
        dev.set_attn_capture(1)
        o.set_attn_capture(1)
        embd = (rng.standard_normal((6, d)) * 0.05).astype(np.float32)
        dev.prefill(embd, 0)
        o.prefill(embd, 0)
        for s in range(3):
            e = (rng.standard_normal(d) * 0.05).astype(np.float32)
            lg, _ = dev.talker_step(e, 6 + s)
            lo, _ = o.step(e, 6 + s)
            assert np.array_equal(lg, lo)
        rg, ro = dev.attn_rows(), o.attn_rows()
        assert len(rg) == len(ro) == 3
        for a, b in zip(rg, ro):
            assert a.shape == b.shape and np.array_equal(a, b)
        text = rng.integers(0, cfg.text_vocab - 8, 16).astype(np.int32)
        dev.set_attn_capture(0)
        o.set_attn_capture(0)
        say(f"[gpu] attention capture over 12 greedy frames ({frame_path})")
        co, _ = o.generate(text, None, max_len=12, temperature=0.0, top_k=0)
        cg = driver.generate(dev, cfg, text, None, max_len=12, temperature=0.0, top_k=0, chunk=5)
        assert np.array_equal(cg, co)
        assert dev.frames_stats()[2] == 0
        rg, ro = dev.attn_rows(), o.attn_rows()
        assert len(ro) == min(co.shape[0], 11) and len(rg) == len(ro)
        for a, b in zip(rg, ro):
            assert a.shape == b.shape and np.array_equal(a, b)
    finally:
        dev.set_attn_capture(-1)
        o.set_attn_capture(-1)


def test_bf16_kv_prefill_steps_frames(prefill_path, frame_path):
    """A bfloat16 talker cache: prefill (GEMV or MFMA path), single steps and
    a greedy and a sampled frame loop (persistent kernel or multi-kernel),
    each bit for bit the oracle's bfloat16 form; the fp16 cache gives other
    logits on the same inputs."""
    cfg = qcfg.tiny()
    w, dev, o = make(cfg, "q8_0", seed=41)
    try:
        dev.kv_set_type(30)
        o.kv_set_type(30)
        o.kv_reset(256)
        rng = np.random.default_rng(42)
        d = cfg.hidden_size
        embd = (rng.standard_normal((10, d)) * 0.5).astype(np.float32)
        say(f"[gpu] bf16 KV: prefill 10 rows ({prefill_path})")
        hid_g, log_g = dev.prefill(embd, 0)
        hid_o, log_o = o.prefill(embd, 0)
        assert np.array_equal(hid_g, hid_o) and np.array_equal(log_g, log_o)
        for s in range(4):
            e = (rng.standard_normal(d) * 0.5).astype(np.float32)
            lg, hg = dev.talker_step(e, 10 + s)
            lo, ho = o.step(e, 10 + s)
            assert np.array_equal(lg, lo) and np.array_equal(hg, ho)
        o16 = orc.Oracle(cfg, w, threads=8)
        o16.kv_reset(256)
        _, log16 = o16.prefill(embd, 0)
        o16.close()
        assert not np.array_equal(log16, log_o)
        text = rng.integers(0, cfg.text_vocab - 8, 18).astype(np.int32)
        co, _ = o.generate(text, None, max_len=16, temperature=0.0, top_k=0)
        cg = driver.generate(dev, cfg, text, None, max_len=16, temperature=0.0, top_k=0, chunk=8)
        check_path(dev, "q8_0", frame_path)
        assert np.array_equal(cg, co)
        co, _ = o.generate(text, None, max_len=12, temperature=0.9, top_k=50, seed=3)
        cg = driver.generate(dev, cfg, text, None, max_len=12, temperature=0.9, top_k=50, seed=3, chunk=5)
        assert np.array_equal(cg, co)
    finally:
        dev.close()


def test_fp16_tie_rounding_regression(frame_path):
    """Weights and prompt on which one attention probability of the talker
    (frame 13, layer 1) lands exactly on an fp16 tie after fp32 rounding; a
    fused multiply-and-convert (one rounding) picks the other neighbour and
    codebook 3 of frame 14 flips."""
    cfg = qcfg.tiny()
    w, dev, o = make(cfg, "q8_0", seed=31)
    rng = np.random.default_rng(32)
    text = rng.integers(0, cfg.text_vocab - 8, 26).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)
    co, _ = o.generate(text, spk, max_len=20, temperature=0.0)
    cg = driver.generate(dev, cfg, text, spk, max_len=20, temperature=0.0, top_k=0, chunk=8)
    check_path(dev, "q8_0", frame_path)
    dev.close()
    assert np.array_equal(cg, co)


@pytest.mark.slow
def test_full_f16_tiled_prefill_200_rows():
    """Exact F16 VALU-GEMM prefill of 200 rows at the 0.6B shapes (fp16-rounded
    inputs, widened ffn_down): every normed hidden row and the last-row logits
    equal the oracle, and so does a following talker step over the 200 cached
    rows."""
    cfg = qcfg.full_06b()
    say("[gpu] full 0.6B F16 tiled prefill: synth + upload")
    w, dev, o = make(cfg, "f16", seed=8, n_ctx=256)
    rng = np.random.default_rng(14)
    embd = (rng.standard_normal((200, cfg.hidden_size)) * 0.05).astype(np.float32)
    import os
    os.environ["Q3T_PREFILL_MFMA"] = "1"
    try:
        say("[gpu] full F16: device prefill 200")
        hid_g, log_g = dev.prefill(embd, 0)
        e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
        lg, hg = dev.talker_step(e, 200)
    finally:
        del os.environ["Q3T_PREFILL_MFMA"]
    say("[gpu] full F16: oracle prefill 200")
    hid_o, log_o = o.prefill(embd, 0)
    lo, ho = o.step(e, 200)
    dev.close()
    assert np.array_equal(hid_g, hid_o)
    assert np.array_equal(log_g, log_o)
    assert np.array_equal(lg, lo) and np.array_equal(hg, ho)


@pytest.mark.slow
def test_full_q8_mfma_prefill_200_rows():
    """int8 MFMA prefill of 200 rows at the 0.6B shapes: every normed hidden
    row and the last-row logits equal the oracle; a following talker step
    (which reads the 200 cached K/V rows) matches too."""
    cfg = qcfg.full_06b()
    say("[gpu] full 0.6B Q8_0 MFMA prefill: synth + upload")
    w, dev, o = make(cfg, "q8_0", seed=5, n_ctx=256)
    rng = np.random.default_rng(13)
    embd = (rng.standard_normal((200, cfg.hidden_size)) * 0.05).astype(np.float32)
    import os
    os.environ["Q3T_PREFILL_MFMA"] = "1"
    try:
        say("[gpu] full: device prefill 200")
        hid_g, log_g = dev.prefill(embd, 0)
        e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
        lg, hg = dev.talker_step(e, 200)
    finally:
        del os.environ["Q3T_PREFILL_MFMA"]
    say("[gpu] full: oracle prefill 200")
    hid_o, log_o = o.prefill(embd, 0)
    lo, ho = o.step(e, 200)
    dev.close()
    assert np.array_equal(hid_g, hid_o)
    assert np.array_equal(log_g, log_o)
    assert np.array_equal(lg, lo) and np.array_equal(hg, ho)


@pytest.mark.slow
@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_long_context_persistent_matches_graph(wtype, monkeypatch):
    """The persistent kernel's split talker attention at a 2,100-position
    context (32 chunks of 80 positions per KV head: prefetched and in-phase
    cache loads, a partial last chunk) against the multi-kernel frame, whose
    single-workgroup attention is pinned to the oracle at short contexts.
    Both paths must give the same codes frame for frame."""
    cfg = qcfg.full_06b()
    say(f"[gpu] long context {wtype}: synth + upload")
    w = Weights(cfg, wtype, seed=6, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    rng = np.random.default_rng(23)
    rows = (rng.standard_normal((2100, cfg.hidden_size)) * 0.05).astype(np.float32)
    pad = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
    out = {}
    try:
        dev.kv_reserve(2100 + 16)
        # (Q3T_FRAME_KERNEL, Q3T_FRAME_XCD) -> the path frames_stats reports
        variants = [("1", "1", 3), ("1", "0", 1), ("0", "1", 0)]
        for kern, xcd, want in variants:
            monkeypatch.setenv("Q3T_FRAME_KERNEL", kern)
            monkeypatch.setenv("Q3T_FRAME_XCD", xcd)
            say(f"[gpu] long context {wtype}: prefill 2100, 6 frames, Q3T_FRAME_KERNEL={kern} Q3T_FRAME_XCD={xcd}")
            dev.prefill(rows, 0, want_hidden=False)
            dev.frames_begin(pad[None], pad, 2100, 6, repetition_penalty=1.05, temperature=0.0, top_k=0,
                             eos_bias=-1e4)
            codes, eos = dev.frames_run(6)
            us, n, used = dev.frames_stats()
            assert used == want and codes.shape[0] == 6, (kern, xcd, used)
            out[want] = codes
    finally:
        dev.close()
    for k in out:
        assert np.array_equal(out[k], out[0]), k


@pytest.mark.parametrize("wtype", ["f16", "q8_0"])
def test_prefill_2049_rows_tail_forms(wtype, monkeypatch):
    """A 2,049-row tiled prefill at the 0.6B shapes (the long-context
    prompt: 33 row tiles, one row past the last full one).  The F16 GEMM's
    16-row tail workgroups and the scores kernel's dealt-out middle tile
    against the forms they replace (Q3T_PF_F16_TAIL=0, Q3T_PF_ATT_SPREAD=0:
    a partial 64-row tile, a workgroup of its own), which the 200-row and
    tiny tiled-prefill tests pin to the oracle: hidden rows and logits bit for
    bit."""
    cfg = qcfg.full_06b()
    say(f"[gpu] 2049-row prefill {wtype}: synth + upload")
    w = Weights(cfg, wtype, seed=8, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "1")
    rows = (np.random.default_rng(81).standard_normal((2049, cfg.hidden_size)) * 0.05).astype(np.float32)
    out = []
    try:
        dev.kv_reserve(2049 + 16)
        for knob in ("1", "0"):
            monkeypatch.setenv("Q3T_PF_F16_TAIL", knob)
            monkeypatch.setenv("Q3T_PF_ATT_SPREAD", knob)
            say(f"[gpu] 2049-row prefill {wtype}: Q3T_PF_F16_TAIL=Q3T_PF_ATT_SPREAD={knob}")
            out.append(dev.prefill(rows, 0))
    finally:
        dev.close()
    (h1, l1), (h0, l0) = out
    assert h1.shape == (2049, cfg.hidden_size) and np.isfinite(l1).all()
    assert np.array_equal(h1, h0) and np.array_equal(l1, l0)


@pytest.fixture(params=["persistent", "persistent_rows", "graph"])
def step_path(request, monkeypatch):
    """Single talker steps and code-predictor calls on the persistent kernel's
    step modes (the default; XCD-parallel layers for Q8_0 0.6B models), on
    its row-parallel layer program (Q3T_FRAME_XCD=0) and on the multi-kernel
    sequences (Q3T_FRAME_KERNEL=0).  The choice is made when a context first
    runs one, so each test builds its own device."""
    monkeypatch.setenv("Q3T_FRAME_KERNEL", "0" if request.param == "graph" else "1")
    monkeypatch.setenv("Q3T_FRAME_XCD", "0" if request.param == "persistent_rows" else "1")
    return request.param


def _steps_and_code_pred(cfg, wtype, seed, n_prefill, step_path):
    w, dev, o = make(cfg, wtype, seed=seed, n_ctx=n_prefill + 16)
    try:
        rng = np.random.default_rng(seed + 100)
        d = cfg.hidden_size
        embd = (rng.standard_normal((n_prefill, d)) * 0.05).astype(np.float32)
        say(f"[gpu] steps + code_pred {wtype} ({step_path}): prefill {n_prefill}")
        hid_g, log_g = dev.prefill(embd, 0)
        hid_o, log_o = o.prefill(embd, 0)
        assert np.array_equal(log_g, log_o)
        for s in range(3):
            e = (rng.standard_normal(d) * 0.05).astype(np.float32)
            lg, hg = dev.talker_step(e, n_prefill + s)
            lo, ho = o.step(e, n_prefill + s)
            assert np.array_equal(lg, lo), f"step {s}: max diff {np.abs(lg - lo).max()}"
            assert np.array_equal(hg, ho)
            cb0 = int(np.argmax(lg[:cfg.codec_vocab - 1024]))
            cg, lcg = dev.code_pred(hg, cb0, frame=s)
            co, lco = o.code_pred(ho, cb0, frame=s)
            assert np.array_equal(cg, co) and np.array_equal(lcg, lco)
            cg, _ = dev.code_pred(hg, cb0, temperature=0.9, top_k=50, seed=11 + s, frame=s)
            co, _ = o.code_pred(ho, cb0, temperature=0.9, top_k=50, seed=11 + s, frame=s)
            assert np.array_equal(cg, co)
    finally:
        dev.close()


def test_talker_step_optional_outputs(step_path):
    """q3t_dev_talker_step with only the logits or only the hidden row asked
    for (the other output NULL): the steps still advance the cache, and what
    is returned equals the oracle's."""
    cfg = qcfg.tiny()
    w, dev, o = make(cfg, "q8_0", seed=41, n_ctx=40)
    try:
        rng = np.random.default_rng(141)
        d = cfg.hidden_size
        embd = (rng.standard_normal((8, d)) * 0.05).astype(np.float32)
        dev.prefill(embd, 0)
        o.prefill(embd, 0)
        for s, (wl, wh) in enumerate([(True, False), (False, True), (False, False), (True, True)]):
            e = (rng.standard_normal(d) * 0.05).astype(np.float32)
            lg, hg = dev.talker_step(e, 8 + s, want_logits=wl, want_hidden=wh)
            lo, ho = o.step(e, 8 + s)
            assert (lg is not None) == wl and (hg is not None) == wh
            if wl:
                assert np.array_equal(lg, lo)
            if wh:
                assert np.array_equal(hg, ho)
    finally:
        dev.close()


def test_steps_and_code_pred_tiny(step_path):
    """Talker steps then greedy and sampled code-predictor calls, each checked
    against the oracle, at the small shapes for both weight types."""
    cfg = qcfg.tiny()
    for wtype in ("q8_0", "f16"):
        _steps_and_code_pred(cfg, wtype, 31, 12, step_path)


@pytest.mark.slow
def test_steps_and_code_pred_full_q8(step_path):
    """The same at the 0.6B shapes with Q8_0 layers, after a 300-row prefill
    (the talker steps take the split attention of the persistent kernel)."""
    _steps_and_code_pred(qcfg.full_06b(), "q8_0", 32, 300, step_path)


@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_mtp_layout_matches_oracle(wtype, frame_path):
    """The 1.7B layout at small shapes: a code predictor narrower than the
    talker, reached through code_pred.mtp_proj (src/tts_transformer.cpp:
    1942-1947, :2096-2101).  Talker steps, greedy and sampled code-predictor
    calls and whole greedy and sampled frame loops equal the oracle, on the
    persistent frame kernel (its 1.7B-layout variants, Q8_0 and F16, with the
    projection as one more GEMV phase per code-predictor pass) and on the
    multi-kernel frame."""
    cfg = qcfg.tiny_mtp()
    say(f"[gpu] mtp layout {wtype} ({frame_path})")
    w, dev, o = make(cfg, wtype, seed=41, n_ctx=64)
    try:
        rng = np.random.default_rng(42)
        d = cfg.hidden_size
        embd = (rng.standard_normal((10, d)) * 0.05).astype(np.float32)
        hid_g, log_g = dev.prefill(embd, 0)
        hid_o, log_o = o.prefill(embd, 0)
        assert np.array_equal(log_g, log_o)
        for s in range(2):
            e = (rng.standard_normal(d) * 0.05).astype(np.float32)
            lg, hg = dev.talker_step(e, 10 + s)
            lo, ho = o.step(e, 10 + s)
            assert np.array_equal(lg, lo) and np.array_equal(hg, ho)
            cb0 = int(np.argmax(lg[:cfg.codec_vocab - 1024]))
            cg, lcg = dev.code_pred(hg, cb0, frame=s)
            co, lco = o.code_pred(ho, cb0, frame=s)
            assert np.array_equal(cg, co) and np.array_equal(lcg, lco)
            cg, _ = dev.code_pred(hg, cb0, temperature=0.9, top_k=50, seed=7, frame=s)
            co, _ = o.code_pred(ho, cb0, temperature=0.9, top_k=50, seed=7, frame=s)
            assert np.array_equal(cg, co)
        text = rng.integers(0, cfg.text_vocab - 8, 24).astype(np.int32)
        spk = rng.standard_normal(d).astype(np.float32)
        co, _ = o.generate(text, spk, max_len=20, temperature=0.0, top_k=0)
        cg = driver.generate(dev, cfg, text, spk, max_len=20, temperature=0.0, top_k=0, chunk=7)
        assert co.shape == cg.shape and np.array_equal(cg, co)
        co, _ = o.generate(text, None, max_len=16, temperature=0.9, top_k=50, seed=13)
        cg = driver.generate(dev, cfg, text, None, max_len=16, temperature=0.9, top_k=50, seed=13, chunk=5)
        assert np.array_equal(cg, co)
        us, n, path = dev.frames_stats()
        assert path == (1 if frame_path == "persistent" else 0), path
    finally:
        dev.close()
