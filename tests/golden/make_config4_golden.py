"""Writes tests/golden/config4_f16_2049.npz: the CPU oracle's results for the
long-context workload at its full size, as digests small enough to commit.

Workload (F16 0.6B shapes, synthetic weights seed 61): prefill rows = one
N(0,1) speaker row followed by text_proj of 2,048 ids uniform in
[0, 151936); a 2,049-row prefill from position 0; then 16 sampled frames
(temperature 0.9, top-k 50, repetition penalty 1.05, sampler seed 65) with 4
trailing rows (text_proj of 4 more ids) and the tts_pad row.

Stored: the seeds, the ids, a blake2b-128 digest of the projected rows, one
digest per hidden row of the prefill (so a mismatch names its first row), the
prefill's last-row logits as they are, and the frames' codes.  The oracle
takes several minutes for the 2,049-row prefill, too long to run inside a
GPU test; the GPU test recomputes the same inputs from the seeds and compares
against these.  Regenerate only on a deliberate numerics change:
    python tests/golden/make_config4_golden.py
"""
import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "qwen3-tts.cpp_amd"), os.path.join(ROOT, "oracle")]

import q3t_oracle as orc  # noqa: E402
from qwen3_tts_amd import config  # noqa: E402
from qwen3_tts_amd.synth import Weights  # noqa: E402

WEIGHT_SEED, IDS_SEED, SPK_SEED, TRAIL_SEED, SAMPLE_SEED = 61, 62, 63, 64, 65
N_IDS, N_FRAMES = 2048, 16
SAMPLING = dict(repetition_penalty=1.05, temperature=0.9, top_k=50)


def digest(a):
    return np.frombuffer(hashlib.blake2b(np.ascontiguousarray(a).tobytes(), digest_size=16).digest(), np.uint8)


def row_digests(rows):
    return np.stack([digest(r) for r in rows])


def inputs(cfg):
    """(ids, speaker row, trailing ids) from the seeds."""
    ids = np.random.default_rng(IDS_SEED).integers(0, cfg.text_vocab, N_IDS).astype(np.int32)
    spk = np.random.default_rng(SPK_SEED).standard_normal(cfg.hidden_size).astype(np.float32)
    trail_ids = np.random.default_rng(TRAIL_SEED).integers(0, cfg.text_vocab, 4).astype(np.int32)
    return ids, spk, trail_ids


def main():
    cfg = config.full_06b()
    w = Weights(cfg, "f16", seed=WEIGHT_SEED)
    threads = int(os.environ.get("ORACLE_THREADS", os.cpu_count() or 4))
    o = orc.Oracle(cfg, w, threads=threads)
    ids, spk, trail_ids = inputs(cfg)
    t0 = time.time()
    tp = o.text_proj(ids)
    trail = o.text_proj(trail_ids)
    pad = o.text_proj(np.array([cfg.tts_pad_id], np.int32))[0]
    rows = np.concatenate([spk[None], tp])
    n = rows.shape[0]
    o.kv_reset(n + N_FRAMES + 8)
    hid, logits = o.prefill(rows, 0)
    print(f"prefill of {n} rows: {time.time() - t0:.1f} s", flush=True)
    codes = o.frames(logits, n, trail, pad, N_FRAMES, seed=SAMPLE_SEED, **SAMPLING)
    print("frames", codes.shape, flush=True)
    np.savez(os.path.join(HERE, "config4_f16_2049.npz"), ids=ids, seeds=np.array(
        [WEIGHT_SEED, IDS_SEED, SPK_SEED, TRAIL_SEED, SAMPLE_SEED], np.int64), text_proj_digest=digest(tp),
        trail_digest=digest(trail), pad_digest=digest(pad), hidden_digests=row_digests(hid), logits=logits,
        codes=codes)


if __name__ == "__main__":
    main()
