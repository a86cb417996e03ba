"""HIP path vs the CPU oracle at the benchmark workloads' shapes and contexts
(0.6B shapes; through the device C ABI):

  configuration 1  F16 weights, 32-token prompt, 64 greedy frames
  configuration 2  F16 talker step at KV 512 (n_kv = 513: the persistent
                   kernel's attention chunk is 32 positions), cache pre-filled
                   with bfloat16-valued N(0,1) K/V through q3t_dev_kv_write
  configuration 3  Q8_0 weights, 64-token prompt, 256 greedy frames
  configuration 4  F16 long context: a tiled prefill that attends over more
                   than 1,024 positions (the split attention's four-phase
                   form), then sampled frames (T 0.9, top-k 50, repetition
                   penalty 1.05); and decode past 4,096 positions
  configuration 5  16 Q8_0 streams with talker KV lengths uniform in
                   [128, 2048], greedy, batched decode

Long contexts are pre-filled with seeded K/V rows on both sides (the oracle's
orc_kv_write takes the same [n_pos][n_kv_head][head_dim] rows), so the
oracle runs only the rows and frames under test.  Every comparison is bit for
bit (codes, logits, hidden rows); the F16 logits bound of 1e-2 is asserted
too.
"""
import os
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import driver
from qwen3_tts_amd.device import Device
from qwen3_tts_amd.synth import Weights

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

LOGIT_TOL = 1e-2
THREADS = 16

_weights = {}
_oracle_runs = {}


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def weights(wtype, seed):
    """One 0.6B model held at a time (1-2 GB of host memory)."""
    key = (wtype, seed)
    if key not in _weights:
        _weights.clear()
        say(f"[gpu] synthesising 0.6B {wtype} weights (seed {seed})")
        _weights[key] = Weights(qcfg.full_06b(), wtype, seed=seed)
    return _weights[key]


def open_pair(wtype, seed, n_ctx):
    cfg = qcfg.full_06b()
    w = weights(wtype, seed)
    dev = Device(cfg)
    dev.upload_weights(w)
    dev.kv_reserve(n_ctx)
    o = orc.Oracle(cfg, w, threads=THREADS)
    o.kv_reset(n_ctx)
    return cfg, w, dev, o


def bf16_kv(rng, n_pos, cfg):
    """N(0,1) K and V rows [n_pos][n_kv_head][head_dim], rounded to bfloat16
    (nearest even) and held in the fp16 cache.  bfloat16's 8-bit significand
    fits fp16's 11 bits, so every value of magnitude at least 2^-17 is stored
    exactly."""
    x = rng.standard_normal((2, n_pos, cfg.n_kv_head, cfg.head_dim), dtype=np.float32)
    u = x.view(np.uint32)
    u = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)).astype(np.uint32)
    return u.view(np.float32).astype(np.float16)


def prefill_kv(dev, o, cfg, rng, n_pos):
    say(f"[gpu] writing {n_pos} K/V positions x {cfg.n_layers} layers")
    for il in range(cfg.n_layers):
        kv = bf16_kv(rng, n_pos, cfg)
        dev.kv_write(il, kv[0], kv[1])
        o.kv_write(il, kv[0], kv[1])


@pytest.fixture(params=["persistent", "persistent_rows", "graph"])
def path(request, monkeypatch):
    """The persistent frame kernel (default: with the XCD-parallel layer
    program for 0.6B models), the persistent kernel with its
    row-parallel layer program (Q3T_FRAME_XCD=0), or the captured
    multi-kernel sequences (Q3T_FRAME_KERNEL=0); chosen when a context first
    runs."""
    monkeypatch.setenv("Q3T_FRAME_KERNEL", "0" if request.param == "graph" else "1")
    monkeypatch.setenv("Q3T_FRAME_XCD", "0" if request.param == "persistent_rows" else "1")
    return request.param


def check_path(dev, want, wtype="f16"):
    """graph: 0; persistent_rows: the row-parallel program (1); persistent:
    the XCD-parallel program (3), which the 0.6B shapes take with Q8_0 and F16
    layers alike."""
    _, _, used = dev.frames_stats()
    if want == "graph":
        assert used == 0, (want, used)
    elif want == "persistent_rows":
        assert used == 1, (want, wtype, used)
    else:
        assert used == 3, (want, wtype, used)


def test_config2_f16_talker_step_kv512(path):
    cfg, w, dev, o = open_pair("f16", 51, 528)
    try:
        rng = np.random.default_rng(52)
        prefill_kv(dev, o, cfg, rng, 512)
        for s in range(3):
            e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
            say(f"[gpu] config 2 ({path}): step at n_past {512 + s}")
            lg, hg = dev.talker_step(e, 512 + s)
            lo, ho = o.step(e, 512 + s)
            assert np.abs(lg - lo).max() <= LOGIT_TOL
            assert np.array_equal(lg, lo), f"step {s}: max diff {np.abs(lg - lo).max()}"
            assert np.array_equal(hg, ho)
        cg, co = _frames_both(dev, o, cfg, lo, 515, 4, seed=60)
        check_path(dev, path)
        assert cg.shape == (4, 16) and np.array_equal(cg, co)
    finally:
        dev.close()


def test_context_past_12288_f16(path):
    """A 16,400-position cache (the decode attention's scores then need more
    than 64 KiB of LDS): talker steps at position 16,390 on every path, and
    with attention capture of the last layer (the multi-kernel step), against
    the oracle bit for bit."""
    cfg, w, dev, o = open_pair("f16", 57, 16400)
    try:
        rng = np.random.default_rng(58)
        prefill_kv(dev, o, cfg, rng, 16390)
        e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
        say(f"[gpu] step at n_past 16390 ({path})")
        lg, hg = dev.talker_step(e, 16390)
        lo, ho = o.step(e, 16390)
        assert np.array_equal(lg, lo) and np.array_equal(hg, ho)
        dev.set_attn_capture(cfg.n_layers - 1)
        o.set_attn_capture(cfg.n_layers - 1)
        say(f"[gpu] captured step at n_past 16391 ({path})")
        lg, hg = dev.talker_step(e, 16391)
        lo, ho = o.step(e, 16391)
        assert np.array_equal(lg, lo) and np.array_equal(hg, ho)
        (rg,), (ro,) = dev.attn_rows(), o.attn_rows()
        assert rg.shape == (cfg.n_head, 16392) and np.array_equal(rg, ro)
    finally:
        dev.close()


def test_config2_bf16_kv_step(path):
    """Configuration 2 with a bfloat16 talker cache (q3t_dev_kv_set_type):
    N(0,1) bfloat16 K/V at 512 positions, then steps at 512.. on the
    persistent kernel's step mode (either layer program) or the multi-kernel
    step, bit for bit the oracle's bfloat16 form; then 4 sampled frames."""
    cfg, w, dev, o = open_pair("f16", 51, 528)
    try:
        dev.kv_set_type(30)
        o.kv_set_type(30)
        o.kv_reset(528)
        rng = np.random.default_rng(59)
        say("[gpu] writing 512 bfloat16 K/V positions x 28 layers")
        for il in range(cfg.n_layers):
            x = rng.standard_normal((2, 512, cfg.n_kv_head, cfg.head_dim), dtype=np.float32)
            u = x.view(np.uint32)
            bits = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)
            dev.kv_write(il, bits[0], bits[1])
            o.kv_write(il, bits[0], bits[1])
        for s in range(3):
            e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
            say(f"[gpu] config 2 bf16 KV: step at n_past {512 + s}")
            lg, hg = dev.talker_step(e, 512 + s)
            lo, ho = o.step(e, 512 + s)
            assert np.array_equal(lg, lo), f"step {s}: max diff {np.abs(lg - lo).max()}"
            assert np.array_equal(hg, ho)
        cg, co = _frames_both(dev, o, cfg, lo, 515, 4, seed=60)
        check_path(dev, path)
        assert cg.shape == (4, 16) and np.array_equal(cg, co)
    finally:
        dev.close()


def _frames_both(dev, o, cfg, lo, n_past, n_frames, seed):
    rng = np.random.default_rng(seed)
    trail = (rng.standard_normal((5, cfg.hidden_size)) * 0.05).astype(np.float32)
    pad = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
    kw = dict(repetition_penalty=1.05, temperature=0.9, top_k=50, eos_bias=-1e4, seed=seed)
    dev.frames_begin(trail, pad, n_past, n_frames, **kw)
    cg, _ = dev.frames_run(n_frames)
    co = o.frames(lo, n_past, trail, pad, n_frames, **kw)
    return cg, co


def test_config4_long_context_sampled_f16(path, monkeypatch):
    cfg, w, dev, o = open_pair("f16", 53, 4200)
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "1")
    try:
        rng = np.random.default_rng(54)
        # a 64-row tiled prefill after 1,000 cached positions: its causal
        # attention spans up to 1,064 positions
        prefill_kv(dev, o, cfg, rng, 1000)
        rows = (rng.standard_normal((64, cfg.hidden_size)) * 0.05).astype(np.float32)
        say(f"[gpu] config 4 ({path}): tiled prefill of 64 rows at n_past 1000")
        hg, lg = dev.prefill(rows, 1000)
        ho, lo = o.prefill(rows, 1000)
        assert np.abs(lg - lo).max() <= LOGIT_TOL
        assert np.array_equal(hg, ho) and np.array_equal(lg, lo)
        say(f"[gpu] config 4 ({path}): 8 sampled frames from position 1064")
        cg, co = _frames_both(dev, o, cfg, lo, 1064, 8, seed=55)
        check_path(dev, path)
        assert cg.shape == (8, 16) and np.array_equal(cg, co)
        # past 4,096 positions: one step, then 4 sampled frames
        prefill_kv(dev, o, cfg, rng, 4100)
        e = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
        say(f"[gpu] config 4 ({path}): step at n_past 4100, 4 sampled frames")
        lg, hg = dev.talker_step(e, 4100)
        lo, ho = o.step(e, 4100)
        assert np.array_equal(lg, lo) and np.array_equal(hg, ho)
        cg, co = _frames_both(dev, o, cfg, lo, 4101, 4, seed=56)
        check_path(dev, path)
        assert cg.shape == (4, 16) and np.array_equal(cg, co)
    finally:
        dev.close()


def _golden_config4():
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    import make_config4_golden as g4
    return g4, np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config4_f16_2049.npz"))


def test_config4_full_prefill_2049_sampled_f16(path):
    """Configuration 4 at its full size against the oracle's recorded results
    (tests/golden/config4_f16_2049.npz, made by make_config4_golden.py; the
    oracle needs minutes for this prefill): one N(0,1) speaker row plus the
    device text projection of 2,048 ids uniform in [0, 151936), a 2,049-row
    F16 prefill from position 0 on the tiled MFMA path (causal attention over
    up to 2,049 positions, softmax rows of 2,049-2,560 held in registers, the
    ragged last row tile), then 16 sampled frames (T 0.9, top-k 50,
    repetition penalty 1.05).  Projected rows, every hidden row (per-row
    digests) and the last logits are bit-exact; the codes are identical."""
    g4, gold = _golden_config4()
    cfg = qcfg.full_06b()
    ids, spk, trail_ids = g4.inputs(cfg)
    assert np.array_equal(ids, gold["ids"])
    w = weights("f16", g4.WEIGHT_SEED)
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        n = g4.N_IDS + 1
        dev.kv_reserve(n + g4.N_FRAMES + 8)
        say(f"[gpu] config 4 full ({path}): text_proj of {g4.N_IDS} ids")
        tp = dev.text_proj(ids)
        trail = dev.text_proj(trail_ids)
        pad = dev.text_proj(np.array([cfg.tts_pad_id], np.int32))[0]
        assert np.array_equal(g4.digest(tp), gold["text_proj_digest"])
        assert np.array_equal(g4.digest(trail), gold["trail_digest"])
        assert np.array_equal(g4.digest(pad), gold["pad_digest"])
        rows = np.concatenate([spk[None], tp])
        say(f"[gpu] config 4 full ({path}): prefill of {n} rows")
        hid, lg = dev.prefill(rows, 0)
        dg = g4.row_digests(hid)
        bad = np.flatnonzero(np.any(dg != gold["hidden_digests"], axis=1))
        assert bad.size == 0, f"hidden rows differ from the oracle's, first at row {bad[0]} ({bad.size} rows)"
        assert np.abs(lg - gold["logits"]).max() <= LOGIT_TOL
        assert np.array_equal(lg, gold["logits"])
        say(f"[gpu] config 4 full ({path}): {g4.N_FRAMES} sampled frames from position {n}")
        dev.frames_begin(trail, pad, n, g4.N_FRAMES, seed=g4.SAMPLE_SEED, **g4.SAMPLING)
        cg, _ = dev.frames_run(g4.N_FRAMES)
        check_path(dev, path)
        assert cg.shape == gold["codes"].shape and np.array_equal(cg, gold["codes"])
    finally:
        dev.close()


# The fast F16 prefill (fp16 MFMA, fp32 accumulation, the default for F16
# layers) is checked against the exact oracle by tolerance: the last logits
# within 1e-2 max-abs (the F16 bound of the path's contract) and every hidden
# row within FAST_ROW_TOL of its largest element.
FAST_ROW_TOL = 5e-3


def _rows_rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.abs(a - b).max(axis=1) / np.maximum(np.abs(b).max(axis=1), 1e-30)


@pytest.mark.parametrize("wtype", ["f16", "q8_0"])
def test_fast_prefill_200_rows_within_tolerance(monkeypatch, wtype):
    """200 prompt rows through the default tiled prefill against the oracle's
    exact prefill at the 0.6B shapes.  F16 layers (the weights of
    configuration 4) take the fast fp16-MFMA GEMMs and attention: the last
    logits within 1e-2 max-abs and each hidden row within FAST_ROW_TOL, and the
    exact form on the same rows is bit-exact (the control).  Q8_0 layers keep
    the exact forms by default, so their rows equal the oracle's bit for bit
    with or without Q3T_PF_EXACT."""
    g4, _ = _golden_config4()
    cfg = qcfg.full_06b()
    w = weights(wtype, g4.WEIGHT_SEED if wtype == "f16" else 3)
    dev = Device(cfg)
    o = orc.Oracle(cfg, w, threads=THREADS)
    try:
        dev.upload_weights(w)
        dev.kv_reserve(256)
        o.kv_reset(256)
        rows = (np.random.default_rng(71).standard_normal((200, cfg.hidden_size)) * 0.05).astype(np.float32)
        say(f"[gpu] fast prefill ({wtype}): oracle 200 rows")
        ho, lo = o.prefill(rows, 0)
        monkeypatch.setenv("Q3T_PF_EXACT", "0")
        say(f"[gpu] fast prefill ({wtype}): device 200 rows (fp16 MFMA)")
        hf, lf = dev.prefill(rows, 0)
        rel = _rows_rel(hf, ho)
        say(f"[gpu] fast prefill ({wtype}): logits max-abs {np.abs(lf - lo).max():.3e}, hidden rows rel max "
            f"{rel.max():.3e} median {np.median(rel):.3e}")
        if wtype == "q8_0":
            assert np.array_equal(hf, ho) and np.array_equal(lf, lo)
            return
        assert np.abs(lf - lo).max() <= LOGIT_TOL
        assert rel.max() <= FAST_ROW_TOL
        assert not np.array_equal(hf, ho)          # the fast form really ran
        monkeypatch.setenv("Q3T_PF_EXACT", "1")
        he, le = dev.prefill(rows, 0)
        assert np.array_equal(he, ho) and np.array_equal(le, lo)
    finally:
        o.close()
        dev.close()


def test_fast_f16_config4_full_prefill_2049(monkeypatch):
    """Configuration 4 at full size with the fast F16 prefill: the 2,049-row
    prefill's last logits within 1e-2 of the oracle's recorded ones; then the
    16 sampled frames.  Sampling reads the logits through a softmax and a
    uniform draw, so a fast-form logit that moves by ~1e-4 can change a draw;
    the first frame whose codes differ from the exact run's is reported, not
    asserted."""
    g4, gold = _golden_config4()
    cfg = qcfg.full_06b()
    ids, spk, trail_ids = g4.inputs(cfg)
    w = weights("f16", g4.WEIGHT_SEED)
    dev = Device(cfg)
    monkeypatch.setenv("Q3T_PF_EXACT", "0")
    try:
        dev.upload_weights(w)
        n = g4.N_IDS + 1
        dev.kv_reserve(n + g4.N_FRAMES + 8)
        tp = dev.text_proj(ids)
        trail = dev.text_proj(trail_ids)
        pad = dev.text_proj(np.array([cfg.tts_pad_id], np.int32))[0]
        rows = np.concatenate([spk[None], tp])
        say(f"[gpu] fast F16 config 4: prefill of {n} rows")
        _, lg = dev.prefill(rows, 0)
        err = np.abs(lg - gold["logits"]).max()
        say(f"[gpu] fast F16 config 4: last logits max-abs vs oracle {err:.3e}")
        assert err <= LOGIT_TOL
        dev.frames_begin(trail, pad, n, g4.N_FRAMES, seed=g4.SAMPLE_SEED, **g4.SAMPLING)
        cg, _ = dev.frames_run(g4.N_FRAMES)
        diff = [f for f in range(min(len(cg), len(gold["codes"]))) if not np.array_equal(cg[f], gold["codes"][f])]
        say(f"[gpu] fast F16 config 4: first frame differing from the exact run: "
            f"{diff[0] if diff else 'none'} of {len(cg)}")
    finally:
        dev.close()


def test_fast_f16_config1_tiled_prefill_64_greedy(monkeypatch):
    """Configuration 1 (F16, 32-token prompt, 64 greedy frames) with its
    10-row prompt forced through the tiled prefill in the fast form (its
    default is the exact GEMV prefill): the first logits within 1e-2 of the
    oracle's.  The decode that follows is exact, but it runs on K/V rows that
    differ from the oracle's at fp32 rounding level, so a later greedy
    near-tie can resolve differently; the first frame whose codes differ is
    reported, not asserted."""
    cfg = qcfg.full_06b()
    text = np.random.default_rng(18).integers(0, 151936, 32).astype(np.int32)
    spk = np.random.default_rng(19).standard_normal(1024).astype(np.float32)
    co, first_o = _oracle_generate("config1", "f16", 4, text, spk, 64)
    w = weights("f16", 4)
    dev = Device(cfg)
    monkeypatch.setenv("Q3T_PF_EXACT", "0")
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "1")
    try:
        dev.upload_weights(w)
        pre = driver.build_prefill(dev, cfg, text, spk)
        dev.kv_reserve(pre[0].shape[0] + 64 + 8)
        _, first_g = dev.prefill(pre[0], 0, want_hidden=False)
        say(f"[gpu] fast F16 config 1: first logits max-abs vs oracle {np.abs(first_g - first_o).max():.3e}")
        assert np.abs(first_g - first_o).max() <= LOGIT_TOL
        assert not np.array_equal(first_g, first_o)
        cg = driver.generate(dev, cfg, text, spk, max_len=64, temperature=0.0, top_k=0, prefill_rows=pre)
    finally:
        dev.close()
    diff = [f for f in range(min(len(cg), len(co))) if not np.array_equal(cg[f], co[f])]
    say(f"[gpu] fast F16 config 1: first frame differing from the oracle: {diff[0] if diff else 'none'} of {len(co)}")
    assert cg.shape == co.shape


def _oracle_generate(key, wtype, seed, text, spk, max_len):
    if key not in _oracle_runs:
        cfg = qcfg.full_06b()
        o = orc.Oracle(cfg, weights(wtype, seed), threads=THREADS)
        say(f"[gpu] {key}: oracle generate {max_len}")
        _oracle_runs[key] = o.generate(text, spk, max_len=max_len, temperature=0.0, top_k=0)
        o.close()
    return _oracle_runs[key]


def test_config1_f16_frame_loop_64_greedy(path):
    """F16 GEMVs with fp16-rounded inputs and the widened fp32-input
    ffn_down; a 32-token prompt, 64 greedy frames."""
    cfg = qcfg.full_06b()
    text = np.random.default_rng(18).integers(0, 151936, 32).astype(np.int32)
    spk = np.random.default_rng(19).standard_normal(1024).astype(np.float32)
    co, first_o = _oracle_generate("config1", "f16", 4, text, spk, 64)
    w = weights("f16", 4)
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        say(f"[gpu] config 1: device generate 64 ({path})")
        cg = driver.generate(dev, cfg, text, spk, max_len=64, temperature=0.0, top_k=0, chunk=16)
        check_path(dev, path)
    finally:
        dev.close()
    assert cg.shape == co.shape and np.array_equal(cg, co)


def test_config3_q8_frame_loop_256_greedy(path):
    """Q8_0 layers, a 64-token prompt, 256 greedy frames; the prefill rows
    built on the device equal the oracle's, and so do the first logits."""
    cfg = qcfg.full_06b()
    text = np.random.default_rng(8).integers(0, 151936, 64).astype(np.int32)
    spk = np.random.default_rng(9).standard_normal(1024).astype(np.float32)
    co, first_o = _oracle_generate("config3", "q8_0", 3, text, spk, 256)
    w = weights("q8_0", 3)
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        o = orc.Oracle(cfg, w, threads=THREADS)
        pre = driver.build_prefill(dev, cfg, text, spk)
        opre, otr, opad = o.build_prefill(text, spk)
        o.close()
        assert np.array_equal(pre[0], opre) and np.array_equal(pre[1], otr) and np.array_equal(pre[2], opad)
        dev.kv_reserve(pre[0].shape[0] + 256 + 8)
        _, first_g = dev.prefill(pre[0], 0, want_hidden=False)
        assert np.array_equal(first_g, first_o)
        say(f"[gpu] config 3: device generate 256 ({path})")
        cg = driver.generate(dev, cfg, text, spk, max_len=256, temperature=0.0, top_k=0, prefill_rows=pre)
        check_path(dev, path, "q8_0")
    finally:
        dev.close()
    say(f"[gpu] config 3: frames oracle={co.shape[0]} device={cg.shape[0]}")
    assert cg.shape == co.shape and np.array_equal(cg, co)


def test_xcd_reprobe_switches_to_row_program(monkeypatch):
    """A frames_run on the XCD-parallel program whose waits time out
    re-checks the workgroup dealing; if it changed, the batch runs again from
    the state it began with on the row-parallel program.  The re-check's
    result is forced from the host (Q3T_TEST_XCD_REPROBE_FAIL=1: the batch is
    treated as timed out and the dealing as changed; no wait is made to time
    out).  The second of three 8-frame batches takes the switch; the first
    ran on the XCD-parallel program, the last stays on the row-parallel one,
    and the 24 greedy frames equal the oracle's (configuration 3's model and
    prompt), so the restored state (frame state, repetition set, logits,
    hidden row, head candidates) is the one the batch began with."""
    cfg = qcfg.full_06b()
    text = np.random.default_rng(8).integers(0, 151936, 64).astype(np.int32)
    spk = np.random.default_rng(9).standard_normal(1024).astype(np.float32)
    co, _ = _oracle_generate("config3_24", "q8_0", 3, text, spk, 24)
    w = weights("q8_0", 3)
    dev = Device(cfg)
    monkeypatch.setenv("Q3T_FRAME_KERNEL", "1")
    monkeypatch.setenv("Q3T_FRAME_XCD", "1")
    monkeypatch.delenv("Q3T_TEST_XCD_REPROBE_FAIL", raising=False)
    try:
        dev.upload_weights(w)
        pre, trail, pad = driver.build_prefill(dev, cfg, text, spk)
        dev.kv_reserve(pre.shape[0] + 24 + 8)
        dev.prefill(pre, 0, want_hidden=False)
        dev.frames_begin(trail, pad, pre.shape[0], 24, temperature=0.0, top_k=0)
        got = []
        c, _ = dev.frames_run(8)
        got.append(c)
        assert dev.frames_stats()[2] == 3
        monkeypatch.setenv("Q3T_TEST_XCD_REPROBE_FAIL", "1")
        say("[gpu] XCD re-probe forced to fail: batch 2 reruns on the row-parallel program")
        c, _ = dev.frames_run(8)
        got.append(c)
        assert dev.frames_stats()[2] == 1
        monkeypatch.delenv("Q3T_TEST_XCD_REPROBE_FAIL")
        c, _ = dev.frames_run(8)
        got.append(c)
        assert dev.frames_stats()[2] == 1
    finally:
        dev.close()
    cg = np.concatenate(got)
    assert cg.shape == co.shape and np.array_equal(cg, co)


def test_icl_long_reference_q8(path):
    """generate_icl's layout at the 0.6B shapes with a long reference clip:
    200 reference codec frames and 30 reference text ids make a 210-row
    prefill (the tiled int8 MFMA prefill), built on the device
    (q3t_dev_build_prefill_icl) equal to the oracle's rows, then 24 greedy
    frames with repetition-loop detection on (generate_icl's default)."""
    from test_gpu_facade import icl_rows
    cfg = qcfg.full_06b()
    rng = np.random.default_rng(77)
    text = rng.integers(0, 151936, 40).astype(np.int32)
    ref_text = rng.integers(0, 151936, 30).astype(np.int32)
    ref_codes = np.concatenate([rng.integers(0, 2048, (200, 1)), rng.integers(0, 2048, (200, 15))],
                               axis=1).astype(np.int32)
    spk = rng.standard_normal(1024).astype(np.float32)
    key = "icl200"
    w = weights("q8_0", 3)
    if key not in _oracle_runs:
        o = orc.Oracle(cfg, w, threads=THREADS)
        rows = icl_rows(o, cfg, text, ref_text, ref_codes, spk)
        say(f"[gpu] icl: oracle prefill {rows[0].shape[0]} rows + 24 frames")
        codes = o.generate_rows(*rows, max_len=24, temperature=0.0, top_k=0, rep_loop_detect=True)
        _oracle_runs[key] = (rows, codes)
        o.close()
    (pre_o, trail_o, pad_o), co = _oracle_runs[key]
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        pre, trail, pad = dev.build_prefill_icl(text, ref_text, ref_codes, spk)
        assert pre.shape == pre_o.shape and pre.shape[0] >= 200
        assert np.array_equal(pre, pre_o) and np.array_equal(trail, trail_o) and np.array_equal(pad, pad_o)
        say(f"[gpu] icl: device prefill {pre.shape[0]} rows + 24 frames ({path})")
        cg = driver.generate(dev, cfg, None, None, max_len=24, temperature=0.0, top_k=0, rep_loop_detect=True,
                             prefill_rows=(pre, trail, pad))
        check_path(dev, path, "q8_0")
    finally:
        dev.close()
    assert cg.shape == co.shape and np.array_equal(cg, co)


def test_config5_16_streams_ragged_kv_q8():
    """Configuration 5's shape: 16 streams of the Q8_0 0.6B model whose talker
    KV lengths are drawn uniformly from [128, 2048]: each stream's history is
    seeded K/V rows written to both sides (q3t_dev_stream_kv_write /
    orc_kv_write), then its own prompt rows prefilled at that offset
    (q3t_dev_stream_prefill_at), then 32 greedy frames of all streams together
    (EOS biased off).  Each stream's codes equal the oracle's frame loop over
    the same cache."""
    cfg = qcfg.full_06b()
    w = weights("q8_0", 3)
    B, frames = 16, 32
    rng = np.random.default_rng(91)
    kv_len = rng.integers(128, 2049, B)
    n_ctx = int(kv_len.max()) + frames + 8
    dev = Device(cfg)
    o = orc.Oracle(cfg, w, threads=THREADS)
    try:
        dev.upload_weights(w)
        dev.streams_reserve(B, n_ctx)
        args, want = [], []
        for b in range(B):
            text = rng.integers(0, cfg.text_vocab - 8, int(rng.integers(9, 40))).astype(np.int32)
            spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)
            pre, trail, pad = driver.build_prefill(dev, cfg, text, spk)
            hist = int(kv_len[b]) - pre.shape[0]
            say(f"[gpu] config 5: stream {b}: {hist} cached positions + {pre.shape[0]} prompt rows")
            o.kv_reset(n_ctx)
            for il in range(cfg.n_layers):
                kv = bf16_kv(rng, hist, cfg)
                dev.stream_kv_write(b, il, kv[0], kv[1])
                o.kv_write(il, kv[0], kv[1])
            dev.stream_prefill(b, pre, n_past=hist)
            _, lo = o.prefill(pre, hist)
            want.append(o.frames(lo, int(kv_len[b]), trail, pad, frames, temperature=0.0, top_k=0, eos_bias=-1e4))
            args.append(dict(trailing=trail, tts_pad=pad, n_past=int(kv_len[b]), max_len=frames, temperature=0.0,
                             top_k=0, eos_bias=-1e4))
        say(f"[gpu] config 5: {B} streams x {frames} frames")
        dev.streams_begin(args)
        got, eos = dev.streams_run(frames)
        _, _, used = dev.frames_stats()
        assert used == 2, used
        for b in range(B):
            assert got[b].shape == (frames, 16) and want[b].shape == (frames, 16), b
            assert np.array_equal(got[b], want[b]), b
    finally:
        o.close()
        dev.close()


def weights17(wtype, seed):
    key = ("17b", wtype, seed)
    if key not in _weights:
        _weights.clear()
        say(f"[gpu] synthesising 1.7B {wtype} weights (seed {seed})")
        _weights[key] = Weights(qcfg.full_17b(), wtype, seed=seed)
    return _weights[key]


@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_17b_frame_loop_greedy(wtype, path):
    """The 1.7B layout at its full shapes (talker 2048 wide with FFN 6144, code
    predictor 1024 wide behind code_pred.mtp_proj), Q8_0 and F16: a 24-token
    prompt and 16 greedy frames on the persistent kernel's 1.7B variants
    (three gate/up row groups per wave, the projection as a GEMV phase per
    pass) and on the multi-kernel frame, against the oracle."""
    if path == "persistent_rows":
        pytest.skip("the 1.7B layout has one persistent program (row-parallel)")
    cfg = qcfg.full_17b()
    text = np.random.default_rng(28).integers(0, 151936, 24).astype(np.int32)
    spk = np.random.default_rng(29).standard_normal(cfg.hidden_size).astype(np.float32)
    w = weights17(wtype, 5)
    key = "17b_" + wtype
    if key not in _oracle_runs:
        o = orc.Oracle(cfg, w, threads=THREADS)
        say(f"[gpu] 1.7B {wtype}: oracle generate 16")
        _oracle_runs[key] = o.generate(text, spk, max_len=16, temperature=0.0, top_k=0)
        o.close()
    co, first_o = _oracle_runs[key]
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        say(f"[gpu] 1.7B {wtype}: device generate 16 ({path})")
        cg = driver.generate(dev, cfg, text, spk, max_len=16, temperature=0.0, top_k=0, chunk=8)
        _, _, used = dev.frames_stats()
        assert used == (0 if path == "graph" else 1), used
    finally:
        dev.close()
    assert cg.shape == co.shape and np.array_equal(cg, co)
