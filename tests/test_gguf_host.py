"""The facade's GGUF reading on the CPU (tests/cpp/test_gguf_config.cpp over
qwen3_tts::load_gguf_config; no device): files in the primary-key form and in
the reference converter's metadata form (scripts/convert_tts_to_gguf.py:421-481:
the alias keys qwen3-tts.block_count, qwen3-tts.code_predictor.*, general.*
strings, the int32 rope.mrope_section array, tokenizer string and int32
arrays) give the same hyperparameters; keys the converter does not write
take parse_config's defaults (src/tts_transformer.cpp:228-377: the tts ids,
and the code predictor's rope theta falls back to the talker's); a tensor of
a type this build cannot load is named with its type."""
import dataclasses
import os
import subprocess

import numpy as np
import pytest

from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import gguf
from qwen3_tts_amd.synth import Weights

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "qwen3-tts.cpp_amd", "lib", "test_gguf_config")


def parsed(path):
    assert os.path.exists(BIN), "build() first"
    r = subprocess.run([BIN, str(path)], capture_output=True, text=True, timeout=60)
    if r.returncode == 2:
        return r.stdout.strip()
    assert r.returncode == 0, r.stdout + r.stderr
    return {k: float(v) for k, v in (ln.split() for ln in r.stdout.strip().splitlines())}


WRITTEN = ["hidden_size", "n_layers", "n_head", "n_kv_head", "head_dim", "ffn_size", "codec_vocab", "n_codebooks",
           "cp_layers", "cp_vocab", "cp_hidden", "cp_ffn", "text_vocab", "text_embd_dim", "rope_theta",
           "cp_rope_theta", "codec_pad_id", "codec_bos_id", "codec_eos_id"]


def expect(cfg, key):
    v = {"n_head": cfg.n_head, "n_kv_head": cfg.n_kv_head, "tts_bos_id": cfg.tts_bos_id,
         "tts_eos_id": cfg.tts_eos_id, "tts_pad_id": cfg.tts_pad_id}
    return float(v.get(key, getattr(cfg, key, None)))


@pytest.fixture(scope="module")
def tiny_weights():
    # distinct thetas, so that the alias and the fallback are both visible
    cfg = dataclasses.replace(qcfg.tiny(), rope_theta=2.0e6, cp_rope_theta=5.0e5, n_layers=3, cp_layers=2)
    return cfg, Weights(cfg, "q8_0", seed=3)


def test_primary_and_converter_forms_parse_alike(tmp_path, tiny_weights):
    cfg, w = tiny_weights
    gguf.write(str(tmp_path / "p.gguf"), cfg, w)
    gguf.write_converter(str(tmp_path / "c.gguf"), cfg, w, "q8_0")
    p, c = parsed(tmp_path / "p.gguf"), parsed(tmp_path / "c.gguf")
    for k in WRITTEN:
        assert p[k] == expect(cfg, k), k
        assert c[k] == expect(cfg, k), k
    assert abs(c["rms_eps"] - cfg.rms_eps) < 1e-12
    # the primary form carries the tts ids; the converter's leaves the defaults
    assert (p["tts_bos_id"], p["tts_eos_id"], p["tts_pad_id"]) == (cfg.tts_bos_id, cfg.tts_eos_id, cfg.tts_pad_id)
    assert (c["tts_bos_id"], c["tts_eos_id"], c["tts_pad_id"]) == (151672, 151673, 151671)


def test_converter_form_cp_theta_falls_back_to_talker(tmp_path, tiny_weights):
    cfg, w = tiny_weights
    kv = [e for e in gguf.converter_kv(cfg, "q8_0") if e[0] != "qwen3-tts.code_predictor.rope.freq_base"]
    path = tmp_path / "c.gguf"
    gguf._write_kv(str(path), kv, list(w.items()))
    assert parsed(path)["cp_rope_theta"] == cfg.rope_theta


def test_unsupported_tensor_type_is_named(tmp_path, tiny_weights):
    cfg, w = tiny_weights
    items = list(w.items())
    # the converter's --type q4_k would write Q4_K (ggml type 12) layer matrices
    name, (ttype, ne, arr) = next((n, v) for n, v in items if n == "talker.blk.1.ffn_gate.weight")
    q4k = np.zeros(ne[0] * ne[1] // 256 * 144, np.uint8)
    items = [(n, (12, ne, q4k) if n == name else v) for n, v in items]
    path = tmp_path / "q4k.gguf"
    gguf._write_kv(str(path), gguf.converter_kv(cfg, "q8_0"), items)
    msg = parsed(path)
    assert isinstance(msg, str) and "unsupported tensor type Q4_K for talker.blk.1.ffn_gate.weight" in msg, msg
