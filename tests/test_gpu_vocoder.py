"""HIP vocoder (include/q3t_voc.h) vs the CPU restatement
(oracle/q3t_vocoder.cpp), through the C ABI.

The vocoder's products run on fp16 matrix cores with fp32 accumulation (the
reference's ggml F16 arithmetic class), the oracle sums exactly in fp64, so
results agree within tolerances rather than bit for bit:

  - stage by stage: each stage of the GPU, fed the oracle's previous stage
    output, matches the oracle's own stage output within STAGE_TOL_MAX
    (relative to the stage's largest magnitude; an fp16 activation rounding
    on the other side of a tie moves one element by up to |w| 2^-11 |x|) and
    STAGE_TOL_RMS;
  - end to end, where those differences are amplified through ~40 stages of
    random weights: SNR against the oracle's audio of at least SNR_MIN_DB
    (the reference's own note puts streaming against batch decode at ~50 dB,
    src/qwen3_tts.cpp:239-245).

Integer work is exact: output lengths, the window slicing of decode_window,
and identical results whether codes come from host memory or from the frame
loop's device rows.
"""
import ctypes
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import driver
from qwen3_tts_amd import vocoder as V
from qwen3_tts_amd.device import Device
from qwen3_tts_amd.synth import Weights

pytestmark = pytest.mark.gpu

STAGE_TOL_MAX = 1e-3
STAGE_TOL_RMS = 3e-5
SNR_MIN_DB = 30.0


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def stage_names(c):
    v = ["latent", "pre_conv", "input_proj"] + [f"pre_tfm.{l}" for l in range(c.n_layers)]
    v += ["output_proj", "upsample.0", "upsample.1", "dec.0"]
    for b in range(1, 5):
        v += [f"dec.{b}.conv_t"] + [f"dec.{b}.res.{r}" for r in range(2, 5)]
    return v + ["dec.6"]


def rel_err(got, want):
    d = np.abs(got.astype(np.float64) - want) / max(np.abs(want).max(), 1e-6)
    return float(d.max()), float(np.sqrt((d * d).mean()))


def snr_db(got, want):
    return float(10 * np.log10((want.astype(np.float64) ** 2).mean() / max(((got - want) ** 2).mean(), 1e-30)))


def codes_for(n, seed):
    return np.random.default_rng(seed).integers(0, 2048, (n, 16)).astype(np.int32)


@pytest.fixture(scope="module")
def tiny_voc():
    c = V.tiny()
    w = V.VocWeights(c, seed=11)
    say("[gpu] vocoder tiny")
    g = V.VocDevice(c, w)
    yield c, w, g, orc.VocOracle(c, w, threads=8)
    g.close()


@pytest.mark.parametrize("n,pos0", [(5, 0), (7, 40)])
def test_stages_match_oracle(tiny_voc, n, pos0):
    c, w, g, o = tiny_voc
    codes = codes_for(n, 20 + n)
    st = o.stages(codes, pos0)
    names = stage_names(c)
    errs = {"latent": rel_err(g.run_stage("latent", codes), st["latent"])}
    for prev, name in zip(names, names[1:]):
        say(f"[gpu] stage {name} n={n}")
        got = g.run_stage(name, st[prev], pos0)
        assert got.shape == st[name].shape, (name, got.shape, st[name].shape)
        errs[name] = rel_err(got, st[name])
    worst = max(errs, key=lambda k: errs[k][0])
    say(f"[gpu] worst stage max {worst} {errs[worst]}")
    assert errs[worst][0] <= STAGE_TOL_MAX, (worst, errs[worst])
    worst = max(errs, key=lambda k: errs[k][1])
    say(f"[gpu] worst stage rms {worst} {errs[worst]}")
    assert errs[worst][1] <= STAGE_TOL_RMS, (worst, errs[worst])


@pytest.mark.parametrize("n", [73, 239, 240, 400])
def test_pre_transformer_attention_forms(tiny_voc, n):
    """A pre-transformer layer over n rows at position 19: up to 239 rows at
    these widths (head width 32) the attention stages each head's q, K and V
    rows in LDS (four query rows per workgroup), from 240 rows it takes the
    one-wave-per-row kernel; both within the stage tolerances of the oracle."""
    c, w, g, o = tiny_voc
    width = o.stages(codes_for(2, 1), 0)["input_proj"].shape[1]
    x = (np.random.default_rng(n).standard_normal((n, width)) * 0.5).astype(np.float32)
    say(f"[gpu] pre_tfm.0 over {n} rows")
    got = g.run_stage("pre_tfm.0", x, 19)
    want = o.run_stage("pre_tfm.0", x, 19)
    assert got.shape == want.shape
    mx, rms = rel_err(got, want)
    assert mx <= STAGE_TOL_MAX and rms <= STAGE_TOL_RMS, (mx, rms)


def test_decode_window_matches_oracle(tiny_voc):
    c, w, g, o = tiny_voc
    codes = codes_for(12, 3)
    for start, end, ctx in [(0, 12, 48), (5, 12, 3), (9, 12, 0), (0, 1, 4)]:
        say(f"[gpu] decode_window {start}:{end} ctx {ctx}")
        got = g.decode_window(codes, start, end, ctx)
        want = o.decode_window(codes, start, end, ctx)
        assert got.shape == want.shape
        if want.size:
            say(f"[gpu]   snr {snr_db(got, want):.1f} dB")
            assert snr_db(got, want) >= SNR_MIN_DB, (start, end, ctx, snr_db(got, want))
    whole = g.decode(codes)
    assert whole.shape[0] == c.samples_for_frames(12) == g.samples_for_frames(12)
    assert np.array_equal(whole, g.decode_window(codes, 0, 12, 0))


def test_decode_window_prefix_and_slicing_exact(tiny_voc):
    """every GPU stage is causal and row-local in its arithmetic, so the
    decode of n frames is bit-for-bit the prefix of the decode of n + k
    frames, and a window with full context is the slice of the whole"""
    c, w, g, o = tiny_voc
    codes = codes_for(10, 4)
    a = g.decode(codes[:6])
    b = g.decode(codes)
    assert np.array_equal(a, b[:a.size])
    win = g.decode_window(codes, 6, 10, 48)
    assert np.array_equal(win, b[c.samples_for_frames(6):])


class DeviceCodes:
    """codes copied into a plain hipMalloc buffer (the HIP runtime through
    ctypes), standing for any device-resident code rows"""

    def __init__(self, codes):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.hip.hipFree.argtypes = [ctypes.c_void_p]
        self.p = ctypes.c_void_p()
        assert self.hip.hipMalloc(ctypes.byref(self.p), codes.nbytes) == 0
        assert self.hip.hipMemcpy(self.p, codes.ctypes.data_as(ctypes.c_void_p), codes.nbytes, 1) == 0

    def close(self):
        if self.p:
            self.hip.hipFree(self.p)
            self.p = None


def test_code_out_of_range_fails(tiny_voc):
    c, w, g, o = tiny_voc
    codes = codes_for(4, 5)
    codes[2, 7] = 2048
    with pytest.raises(V.VocError, match="out of range"):
        g.decode_window(codes, 0, 4, 0)
    d = DeviceCodes(codes)
    try:
        with pytest.raises(V.VocError, match="out of range"):
            g.decode_window(None, 0, 4, 0, n_frames=4, device_ptr=d.p.value)
    finally:
        d.close()
    codes[2, 7] = 5
    d = DeviceCodes(codes)
    try:
        got = g.decode_window(None, 1, 4, 1, n_frames=4, device_ptr=d.p.value)
    finally:
        d.close()
    assert np.array_equal(got, g.decode_window(codes, 1, 4, 1))
    with pytest.raises(V.VocError, match="invalid frame range"):
        g.decode_window(codes, 3, 3, 0)


def test_streaming_from_device_codes(tiny_voc):
    """the frame loop's device code rows feed decode_window in place every
    chunk_frames frames (with context); the streamed audio equals the oracle's
    windows over the same codes, and the host-codes path gives identical
    samples"""
    c, w, g, o = tiny_voc
    tcfg = qcfg.tiny()
    tw = Weights(tcfg, "q8_0", seed=7)
    dev = Device(tcfg)
    dev.upload_weights(tw)
    try:
        text = np.random.default_rng(8).integers(0, tcfg.text_vocab - 8, 16).astype(np.int32)
        chunks = []
        say("[gpu] streaming 40 frames, chunk 9, context 6")
        codes, audio, n_win = driver.stream_audio(dev, g, tcfg, text, None, max_len=40, chunk_frames=9,
                                                  context_frames=6, on_audio=lambda s: chunks.append(s) or True,
                                                  temperature=0.0, top_k=0, frame_chunk=4)
        n = codes.shape[0]
        assert n >= 10, n
        assert n_win == len(chunks) and np.array_equal(np.concatenate(chunks), audio)
        assert audio.size == c.samples_for_frames(n)
        emitted, want = 0, []
        for end in list(range(9, n + 1, 9)) + ([n] if n % 9 else []):
            host = g.decode_window(codes, emitted, end, 6)
            ref = o.decode_window(codes, emitted, end, 6)
            seg = audio[sum(x.size for x in want):][:host.size]
            assert np.array_equal(seg, host), (emitted, end)
            assert snr_db(host, ref) >= SNR_MIN_DB
            want.append(host)
            emitted = end
        assert sum(x.size for x in want) == audio.size
    finally:
        dev.close()


def test_streaming_abort_stops_generation(tiny_voc):
    c, w, g, o = tiny_voc
    tcfg = qcfg.tiny()
    dev = Device(tcfg)
    dev.upload_weights(Weights(tcfg, "q8_0", seed=7))
    try:
        text = np.arange(5, 30, dtype=np.int32)
        codes, audio, n_win = driver.stream_audio(dev, g, tcfg, text, None, max_len=40, chunk_frames=5,
                                                  context_frames=4, on_audio=lambda s: False, temperature=0.0,
                                                  top_k=0)
        assert n_win == 1 and codes.shape[0] == 5 and audio.size == c.samples_for_frames(5)
    finally:
        dev.close()


@pytest.mark.slow
def test_full_size_stages_and_window():
    """the 12 Hz tokenizer's decoder widths (random weights): every stage of a
    3-frame segment against the oracle, and a 4-frame window end to end"""
    c = V.full()
    w = V.VocWeights(c, seed=3)
    say("[gpu] vocoder full widths")
    g = V.VocDevice(c, w)
    o = orc.VocOracle(c, w, threads=16)
    try:
        codes = codes_for(4, 9)
        st = o.stages(codes[:3], 5)
        names = stage_names(c)
        errs = {"latent": rel_err(g.run_stage("latent", codes[:3]), st["latent"])}
        for prev, name in zip(names, names[1:]):
            say(f"[gpu] full stage {name}")
            got = g.run_stage(name, st[prev], 5)
            assert got.shape == st[name].shape, name
            errs[name] = rel_err(got, st[name])
        worst = max(errs, key=lambda k: errs[k][0])
        assert errs[worst][0] <= STAGE_TOL_MAX, (worst, errs[worst])
        worst = max(errs, key=lambda k: errs[k][1])
        assert errs[worst][1] <= STAGE_TOL_RMS, (worst, errs[worst])
        got = g.decode_window(codes, 2, 4, 2)
        want = o.decode_window(codes, 2, 4, 2)
        assert got.shape == want.shape
        assert snr_db(got, want) >= SNR_MIN_DB, snr_db(got, want)
    finally:
        g.close()
        o.close()


FUSE_SCRIPT = r"""
import sys, numpy as np
from qwen3_tts_amd import vocoder as V
c = V.full()
g = V.VocDevice(c, V.VocWeights(c, seed=3))
codes = np.random.default_rng(12).integers(0, c.codebook_size, (6, c.n_codebooks)).astype(np.int32)
np.save(sys.argv[1], g.decode_window(codes, 3, 6, 3))
g.close()
"""


def test_fused_residual_units_match_two_launches(tmp_path):
    """The 96- and 192-channel residual units run as one launch (k7 conv,
    snake and 1-tap conv with the intermediate tile in LDS); Q3T_VOC_FUSE=0
    runs them as two.  A 6-frame window at the tokenizer's widths (decoder
    blocks 3-4 over 3,840 and 11,520 rows) gives the same audio bit for bit."""
    import os
    import subprocess
    from qwen3_tts_amd.device import PKG_DIR
    out = {}
    for name, env in (("two", {"Q3T_VOC_FUSE": "0"}), ("fused", {})):
        say(f"[gpu] vocoder residual units: {name}")
        path = tmp_path / f"{name}.npy"
        r = subprocess.run([sys.executable, "-c", FUSE_SCRIPT, str(path)], capture_output=True, text=True, timeout=300,
                           env=dict(os.environ, PYTHONPATH=PKG_DIR, **env))
        assert r.returncode == 0, r.stderr[-2000:]
        out[name] = np.load(path)
    assert out["two"].size == 3 * 1920
    assert np.array_equal(out["two"], out["fused"])
