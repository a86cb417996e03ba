"""Writes tests/golden/tiny_q8_greedy.npz: greedy codes and the prefill's
first-frame logits of the tiny Q8_0 model (seed 11) from the CPU oracle.

A regression fixture: once the oracle is pinned by tests/test_oracle.py, the
recorded codes catch any later change to its numerics.  Regenerate only on a
deliberate numerics change:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "qwen3-tts.cpp_amd"), os.path.join(ROOT, "oracle")]

import q3t_oracle as orc  # noqa: E402
from qwen3_tts_amd import config  # noqa: E402
from qwen3_tts_amd.synth import Weights  # noqa: E402


def main():
    cfg = config.tiny()
    w = Weights(cfg, "q8_0", seed=11)
    o = orc.Oracle(cfg, w, threads=4)
    text = np.random.default_rng(21).integers(0, cfg.text_vocab - 8, 24).astype(np.int32)
    spk = np.random.default_rng(22).standard_normal(cfg.hidden_size).astype(np.float32)
    max_len = 24
    codes, first = o.generate(text, spk, max_len=max_len, temperature=0.0)
    np.savez(os.path.join(HERE, "tiny_q8_greedy.npz"), text=text, speaker=spk, max_len=np.int32(max_len),
             codes=codes, first_logits=first)
    print("frames", codes.shape)


if __name__ == "__main__":
    main()
