"""Multi-stream decode (q3t_dev_streams_*) vs the CPU oracle, one utterance at
a time.

Every stream of a batched run must produce exactly the codes the oracle's
generate() produces for that utterance alone (src/tts_transformer.cpp:3007-3309
is the per-utterance loop): the batched GEMMs, the per-stream attention and
the per-stream samplers follow the same numerics contract as the batch-1 path.
Streams differ in prompt length (ragged KV), max_len, sampling controls and
seed, and stop at different frames.  Q8_0 layers run the int8 MFMA decode
GEMMs, F16 layers the f64 MFMA ones; both at the tiny shapes, and four
streams at the full 0.6B shapes.
"""
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import driver
from qwen3_tts_amd.device import Device, DeviceError
from qwen3_tts_amd.synth import Weights

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", params=["q8_0", "f16"])
def tiny_q8(request):
    """The tiny model with Q8_0 layers (int8 MFMA decode GEMMs) or F16 layers
    (f64 MFMA decode GEMMs)."""
    cfg = qcfg.tiny()
    say(f"[gpu] streams: tiny {request.param} model")
    w = Weights(cfg, request.param, seed=17, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    o = orc.Oracle(cfg, w, threads=8)
    yield cfg, w, dev, o
    dev.close()


def _prompt(cfg, seed, n_text, speaker):
    rng = np.random.default_rng(seed)
    text = rng.integers(0, cfg.text_vocab - 8, n_text).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32) if speaker else None
    return text, spk


def _run(cfg, dev, o, specs, chunk):
    streams, want = [], []
    for sp in specs:
        text, spk = _prompt(cfg, sp["seed_prompt"], sp["n_text"], sp.get("speaker", True))
        kw = {k: sp[k] for k in ("max_len", "temperature", "top_k", "seed", "eos_bias", "target_frames",
                                 "repetition_penalty") if k in sp}
        streams.append(dict(prefill_rows=driver.build_prefill(dev, cfg, text, spk), **kw))
        o.kv_reset(512)
        co, _ = o.generate(text, spk, max_len=sp["max_len"], temperature=sp.get("temperature", 0.9),
                           top_k=sp.get("top_k", 50), seed=sp.get("seed", 0), eos_bias=sp.get("eos_bias", 0.0),
                           target_frames=sp.get("target_frames", 0),
                           repetition_penalty=sp.get("repetition_penalty", 1.05))
        want.append(co)
    say(f"[gpu] streams: {len(specs)} streams, chunk {chunk}")
    got = driver.generate_streams(dev, cfg, streams, chunk=chunk)
    us, launches, path = dev.frames_stats()
    assert path == 2, path
    for b, (g, w) in enumerate(zip(got, want)):
        assert g.shape == w.shape, (b, g.shape, w.shape)
        assert np.array_equal(g, w), b
    return got


def test_streams_greedy_ragged(tiny_q8):
    cfg, w, dev, o = tiny_q8
    specs = [
        dict(seed_prompt=1, n_text=32, max_len=24, temperature=0.0, top_k=0),
        dict(seed_prompt=2, n_text=9, max_len=16, temperature=0.0, top_k=0, speaker=False),
        dict(seed_prompt=3, n_text=57, max_len=30, temperature=0.0, top_k=0),
    ]
    _run(cfg, dev, o, specs, chunk=7)


def test_streams_sampled_per_stream_seeds(tiny_q8):
    cfg, w, dev, o = tiny_q8
    specs = [
        dict(seed_prompt=4, n_text=20, max_len=20, temperature=0.9, top_k=50, seed=11),
        dict(seed_prompt=4, n_text=20, max_len=20, temperature=0.9, top_k=50, seed=12),
        dict(seed_prompt=5, n_text=14, max_len=12, temperature=0.7, top_k=10, seed=13, repetition_penalty=1.3),
        dict(seed_prompt=6, n_text=40, max_len=18, temperature=1.2, top_k=0, seed=14),
    ]
    got = _run(cfg, dev, o, specs, chunk=5)
    # same prompt, different seeds: the draws must differ somewhere
    assert not np.array_equal(got[0], got[1])


def test_streams_stop_at_different_frames(tiny_q8):
    """One stream samples EOS at frame 0, one stops on the target-frames EOS
    ramp, one runs to max_len; the stopped ones idle while the rest go on."""
    cfg, w, dev, o = tiny_q8
    specs = [
        dict(seed_prompt=7, n_text=12, max_len=8, temperature=0.0, top_k=0, eos_bias=1e4),
        dict(seed_prompt=8, n_text=17, max_len=40, temperature=0.0, top_k=0, target_frames=2),
        dict(seed_prompt=9, n_text=25, max_len=21, temperature=0.0, top_k=0),
    ]
    got = _run(cfg, dev, o, specs, chunk=6)
    assert got[0].shape[0] == 0


def test_streams_single_stream_and_rerun(tiny_q8):
    """One stream (batch 1 through the batched path), then a second begin on
    the same reservation with different arguments."""
    cfg, w, dev, o = tiny_q8
    _run(cfg, dev, o, [dict(seed_prompt=10, n_text=16, max_len=10, temperature=0.0, top_k=0)], chunk=4)
    _run(cfg, dev, o, [dict(seed_prompt=11, n_text=22, max_len=13, temperature=0.8, top_k=20, seed=5)], chunk=13)


@pytest.mark.parametrize("n_streams", [16, 12])
def test_streams_many_heads_rows(tiny_q8, n_streams):
    """16 streams put all rows of every head GEMV in one launch of the
    1024-thread multi-row kernel; 12 take one launch of 8 rows and one of 4."""
    cfg, w, dev, o = tiny_q8
    specs = []
    for i in range(n_streams):
        sp = dict(seed_prompt=30 + i, n_text=6 + 3 * i, max_len=6 + (i % 5))
        if i % 3 == 0:
            sp.update(temperature=0.0, top_k=0)
        else:
            sp.update(temperature=0.8, top_k=20, seed=100 + i)
        specs.append(sp)
    _run(cfg, dev, o, specs, chunk=5)


def test_streams_reject_mixed_layer_types():
    """F16 layers take the f64 MFMA GEMMs and Q8_0 layers the int8 ones; a
    model mixing the two in its layers is refused."""
    cfg = qcfg.tiny()
    w = Weights(cfg, "f16", seed=17, norm_mode="one")
    wq = Weights(cfg, "q8_0", seed=17, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    name = next(n for n in wq.tensors if n.endswith("ffn_down.weight"))
    dev.upload(name, *wq[name])
    try:
        with pytest.raises(DeviceError, match="all layer weights"):
            dev.streams_reserve(2, 128)
    finally:
        dev.close()


def test_streams_argument_errors(tiny_q8):
    cfg, w, dev, o = tiny_q8
    with pytest.raises(DeviceError):
        dev.streams_reserve(0, 128)
    dev.streams_reserve(2, 64)
    emb = np.zeros((4, cfg.hidden_size), np.float32)
    with pytest.raises(DeviceError, match="out of range"):
        dev.stream_prefill(2, emb)
    with pytest.raises(DeviceError, match="Context length"):
        dev.stream_prefill(0, np.zeros((65, cfg.hidden_size), np.float32))
    with pytest.raises(DeviceError, match="Context length"):
        dev.stream_prefill(0, emb, n_past=61)
    kv = np.zeros((8, cfg.n_kv_head, cfg.head_dim), np.float16)
    with pytest.raises(DeviceError, match="out of range"):
        dev.stream_kv_write(2, 0, kv, kv)
    with pytest.raises(DeviceError, match="out of range"):
        dev.stream_kv_write(0, cfg.n_layers, kv, kv)
    with pytest.raises(DeviceError, match="out of range"):
        big = np.zeros((65, cfg.n_kv_head, cfg.head_dim), np.float16)
        dev.stream_kv_write(1, 0, big, big)
    pad = np.zeros(cfg.hidden_size, np.float32)
    tr = np.zeros((1, cfg.hidden_size), np.float32)
    with pytest.raises(DeviceError, match="Context length"):
        dev.streams_begin([dict(trailing=tr, tts_pad=pad, n_past=10, max_len=60),
                           dict(trailing=tr, tts_pad=pad, n_past=10, max_len=4)])


@pytest.mark.slow
def test_streams_full_f16_4_streams():
    """0.6B shapes, F16 layers on the f64 MFMA decode GEMMs: four streams
    with ragged prompts, greedy, 16 frames."""
    cfg = qcfg.full_06b()
    say("[gpu] streams full 0.6B f16: synth + upload")
    w = Weights(cfg, "f16", seed=5, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    o = orc.Oracle(cfg, w, threads=8)
    try:
        specs = [dict(seed_prompt=40 + i, n_text=n, max_len=16, temperature=0.0, top_k=0)
                 for i, n in enumerate([24, 9, 50, 13])]
        _run(cfg, dev, o, specs, chunk=8)
    finally:
        dev.close()


@pytest.mark.slow
def test_streams_full_f16_fast_gemm_tolerance(monkeypatch):
    """F16 layers on the fp16-MFMA decode GEMMs (fp32 accumulation, as
    ggml's F16 mul_mat; the default form, Q3T_MS_EXACT=1 selects the exact
    f64-MFMA one) at the 0.6B shapes: four greedy streams, frame by frame.
    While a stream's codes agree with the exact form's, its talker logits
    after every frame stay within 1e-2 of the exact form's (largest
    difference over the largest |logit|); the first frame whose codes differ
    is reported, not asserted."""
    cfg = qcfg.full_06b()
    say("[gpu] streams full 0.6B f16 fast form: synth + upload")
    w = Weights(cfg, "f16", seed=5, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    try:
        streams = []
        for i, n in enumerate([24, 9, 50, 13]):
            text, spk = _prompt(cfg, 40 + i, n, True)
            streams.append(dict(prefill_rows=driver.build_prefill(dev, cfg, text, spk), max_len=16, temperature=0.0,
                                top_k=0))
        runs = {}
        for form in ("exact", "fast"):
            monkeypatch.setenv("Q3T_MS_EXACT", "1" if form == "exact" else "0")
            lg = []
            codes = driver.generate_streams(dev, cfg, streams, chunk=1, logits=lg)
            runs[form] = (codes, lg)
        worst = 0.0
        for b in range(len(streams)):
            ce, cf = runs["exact"][0][b], runs["fast"][0][b]
            n = min(len(ce), len(cf))
            diverge = next((f for f in range(n) if not np.array_equal(ce[f], cf[f])), None)
            last = n if diverge is None else diverge
            for f in range(last):
                le, lf = runs["exact"][1][f][b], runs["fast"][1][f][b]
                rel = float(np.abs(le - lf).max() / np.abs(le).max())
                worst = max(worst, rel)
                assert rel <= 1e-2, (b, f, rel)
            say(f"[gpu] stream {b}: {n} frames, first frame whose codes differ: {diverge}")
        say(f"[gpu] fast form: largest logit difference {worst:.2e} of the largest |logit|")
    finally:
        dev.close()


@pytest.mark.slow
def test_streams_full_q8_4_streams():
    """0.6B shapes, Q8_0: four streams with ragged prompts, greedy, 24 frames."""
    cfg = qcfg.full_06b()
    say("[gpu] streams full 0.6B: synth + upload")
    w = Weights(cfg, "q8_0", seed=3, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    o = orc.Oracle(cfg, w, threads=8)
    try:
        specs = [dict(seed_prompt=20 + i, n_text=n, max_len=24, temperature=0.0, top_k=0)
                 for i, n in enumerate([32, 9, 70, 17])]
        _run(cfg, dev, o, specs, chunk=8)
    finally:
        dev.close()
