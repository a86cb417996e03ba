"""q3t_dev_text_proj_noalloc (no device allocation, work buffers in the
library's static device scratch) against q3t_dev_text_proj through the C ABI:
bit-identical rows on two calls in a row, the second with fewer ids (the
scratch keeps the first call's contents), on both forms of the projection
(tiled GEMMs from 16 ids, the GEMV below) and both weight types; more than
64 ids are rejected with an error.  The rows also equal the CPU oracle's.
"""
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd.device import Device, DeviceError
from qwen3_tts_amd.synth import Weights

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_text_proj_noalloc_matches_text_proj(wtype):
    cfg = qcfg.tiny()
    w = Weights(cfg, wtype, seed=71)
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        o = orc.Oracle(cfg, w, threads=4)
        rng = np.random.default_rng(72)
        for n in (40, 5, 64, 1):
            ids = rng.integers(0, cfg.text_vocab, n).astype(np.int32)
            say(f"[gpu] text_proj_noalloc {wtype}: {n} ids")
            got = dev.text_proj_noalloc(ids)
            ref = dev.text_proj(ids)
            assert got.shape == (n, cfg.hidden_size)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), n
            assert np.array_equal(got, o.text_proj(ids)), n
        with pytest.raises(DeviceError, match="at most 64"):
            dev.text_proj_noalloc(np.zeros(65, np.int32))
        with pytest.raises(DeviceError, match="out of range"):
            dev.text_proj_noalloc(np.array([cfg.text_vocab], np.int32))
    finally:
        dev.close()


def test_text_proj_noalloc_full_width_q8():
    """The 0.6B projection widths (2048 -> 2048 -> 1024), 64 then 9 ids."""
    cfg = qcfg.full_06b()
    say("[gpu] text_proj_noalloc 0.6B Q8_0: synth + upload")
    w = Weights(cfg, "q8_0", seed=73)
    dev = Device(cfg)
    try:
        dev.upload_weights(w)
        rng = np.random.default_rng(74)
        for n in (64, 9):
            ids = rng.integers(0, cfg.text_vocab, n).astype(np.int32)
            got = dev.text_proj_noalloc(ids)
            ref = dev.text_proj(ids)
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), n
    finally:
        dev.close()
