"""Prefill rows built on the device (q3t_dev_build_prefill /
q3t_dev_build_prefill_icl, q3t_dev_text_proj) against the CPU oracle.

build_prefill_graph (src/tts_transformer.cpp:1030-1186) and
build_prefill_graph_icl (:1188-1472) assemble the talker's prompt rows from
projected text ids (project_text_tokens, :963-1028) and codec embedding rows.
On the device every id of the layout is projected in one batched pass (the
tiled GEMMs from 16 ids on, the GEMV below) and the overlays are summed by
one kernel; every row must equal the oracle's bit for bit.
"""
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd.device import Device, DeviceError
from qwen3_tts_amd.synth import Weights
from test_gpu_facade import icl_rows

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.fixture(scope="module", params=["q8_0", "f16"])
def model(request):
    cfg = qcfg.tiny()
    say(f"[gpu] prefill build: tiny {request.param}")
    w = Weights(cfg, request.param, seed=23, norm_mode="one")
    dev = Device(cfg)
    dev.upload_weights(w)
    o = orc.Oracle(cfg, w, threads=8)
    yield cfg, dev, o
    dev.close()


def _ids(cfg, rng, n):
    return rng.integers(0, cfg.text_vocab - 8, n).astype(np.int32)


@pytest.mark.parametrize("n_text,speaker,language_id,n_instruct", [
    (26, True, 2050, 0),      # 7 + 17 trailing = 24 projected ids: tiled GEMMs
    (4, False, -1, 0),        # shortest text, no-think prefix, no trailing text: 7 ids, GEMV
    (9, True, 2050, 5),       # instruct rows, still no trailing text: 12 ids, GEMV
    (10, False, 2050, 0),     # one trailing id: 8 ids, GEMV
    (60, True, -1, 40),       # 98 projected ids: tiled GEMMs
])
def test_build_prefill_matches_oracle(model, n_text, speaker, language_id, n_instruct):
    cfg, dev, o = model
    rng = np.random.default_rng(n_text * 7 + n_instruct)
    text = _ids(cfg, rng, n_text)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32) if speaker else None
    instr = _ids(cfg, rng, n_instruct) if n_instruct else None
    say(f"[gpu] build_prefill n={n_text} spk={speaker} lang={language_id} instruct={n_instruct}")
    pre, trail, pad = dev.build_prefill(text, spk, language_id, instr)
    pre_o, trail_o, pad_o = o.build_prefill(text, spk, language_id, instr)
    assert pre.shape == pre_o.shape and trail.shape == trail_o.shape
    assert np.array_equal(pre, pre_o)
    assert np.array_equal(trail, trail_o)
    assert np.array_equal(pad, pad_o)


def test_text_proj_tiled_equals_gemv_and_oracle(model, monkeypatch):
    """80 ids take the tiled GEMMs, the same ids in calls of 1-3 the GEMV:
    a row's projection must not depend on how many rows travel with it."""
    cfg, dev, o = model
    ids = _ids(cfg, np.random.default_rng(5), 80)
    say("[gpu] text_proj 80 ids tiled")
    tiled = dev.text_proj(ids)
    small = np.concatenate([dev.text_proj(ids[i:i + 3]) for i in range(0, 80, 3)])
    monkeypatch.setenv("Q3T_PREFILL_MFMA", "0")
    gemv = dev.text_proj(ids)
    assert np.array_equal(tiled, small)
    assert np.array_equal(tiled, gemv)
    assert np.array_equal(tiled, o.text_proj(ids))


@pytest.mark.parametrize("n_ref_text,n_frames,speaker", [
    (10, 6, True),     # text stream longer than the codec stream: trailing text
    (5, 30, True),     # codec stream longer: tts_pad fills, no trailing text
    (12, 1, False),    # one reference frame, no speaker row
])
def test_build_prefill_icl_matches_oracle(model, n_ref_text, n_frames, speaker):
    cfg, dev, o = model
    rng = np.random.default_rng(n_ref_text * 31 + n_frames)
    text = _ids(cfg, rng, 26)
    ref_text = _ids(cfg, rng, n_ref_text)
    ref_codes = np.concatenate([rng.integers(0, cfg.codec_vocab, (n_frames, 1)),
                                rng.integers(0, cfg.cp_vocab, (n_frames, 15))], axis=1).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32) if speaker else None
    say(f"[gpu] build_prefill_icl ref_text={n_ref_text} frames={n_frames} spk={speaker}")
    pre, trail, pad = dev.build_prefill_icl(text, ref_text, ref_codes, spk)
    pre_o, trail_o, pad_o = icl_rows(o, cfg, text, ref_text, ref_codes, spk)
    assert pre.shape == pre_o.shape and trail.shape == trail_o.shape
    assert np.array_equal(pre, pre_o)
    assert np.array_equal(trail, trail_o)
    assert np.array_equal(pad, pad_o)


def test_build_prefill_argument_errors(model):
    cfg, dev, o = model
    text = np.arange(10, dtype=np.int32)
    with pytest.raises(DeviceError, match="at least 4"):
        dev.build_prefill(text[:3])
    bad = text.copy()
    bad[1] = cfg.text_vocab     # a role id (text[5 .. n-5) is never looked up)
    with pytest.raises(DeviceError, match="out of range"):
        dev.build_prefill(bad)
    with pytest.raises(DeviceError, match="out of range"):
        dev.build_prefill(text, language_id=cfg.codec_vocab)
    codes = np.zeros((2, 16), np.int32)
    codes[1, 5] = cfg.cp_vocab
    with pytest.raises(DeviceError, match="out of range"):
        dev.build_prefill_icl(text, text, codes)
    with pytest.raises(DeviceError, match="reference codec frame"):
        dev.build_prefill_icl(text, text, np.zeros((0, 16), np.int32))
    # the context still works after the refused calls
    pre, _, _ = dev.build_prefill(text)
    assert np.array_equal(pre, o.build_prefill(text)[0])


@pytest.mark.slow
def test_text_proj_full_q8_rows():
    """0.6B shapes (2048-wide text embedding, Q8_0 fc1/fc2): a 2048-id
    projection on the tiled GEMMs; every 32nd row against the oracle."""
    cfg = qcfg.full_06b()
    say("[gpu] text_proj full 0.6B q8_0: synth + upload")
    w = Weights(cfg, "q8_0", seed=3, norm_mode="one")
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        o = orc.Oracle(cfg, w, threads=8)
        ids = np.random.default_rng(9).integers(0, cfg.text_vocab, 2048).astype(np.int32)
        rows = dev.text_proj(ids)
        assert np.array_equal(rows[::32], o.text_proj(ids[::32]))
    finally:
        dev.close()
