"""The drop-in C++ TTSTransformer (qwen3-tts.cpp_amd/csrc/tts_transformer.h)
loads a GGUF and runs generate / generate_icl / predict_codes_autoregressive /
predict_codes on the GPU; its codes must equal the CPU oracle's.  Mirrors the reference's
tests/test_transformer.cpp (load, KV init, generate, frame comparison)."""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd import gguf
from qwen3_tts_amd.device import PKG_DIR
from qwen3_tts_amd.synth import Weights

pytestmark = pytest.mark.gpu
BIN = os.path.join(PKG_DIR, "lib", "test_transformer_dev")


def icl_rows(o, cfg, text, ref_text, ref_codes, spk):
    """build_prefill_graph_icl (src/tts_transformer.cpp:1188-1472) from oracle primitives."""
    d = cfg.hidden_size
    bos, eos, pad = o.text_proj(np.array([cfg.tts_bos_id, cfg.tts_eos_id, cfg.tts_pad_id], np.int32))
    role = o.text_proj(text[:3])
    rows = [o.embed_row("codec", 0, t) for t in (cfg.codec_nothink_id, cfg.codec_think_bos_id, cfg.codec_think_eos_id)]
    rows += ([] if spk is None else [spk]) + [o.embed_row("codec", 0, cfg.codec_pad_id),
                                             o.embed_row("codec", 0, cfg.codec_bos_id)]
    cin = np.stack(rows).astype(np.float32)
    ov = len(rows) - 1
    over = np.stack([bos if t == ov - 1 else pad for t in range(ov)]) + cin[:ov]
    stream = list(ref_text[3:max(3, len(ref_text) - 5)]) + list(text[3:max(3, len(text) - 5)]) + [cfg.tts_eos_id]
    tp = o.text_proj(np.array(stream, np.int32))
    codec = [o.embed_row("codec", 0, cfg.codec_bos_id)]
    for f in range(ref_codes.shape[0]):
        r = o.embed_row("codec", 0, int(ref_codes[f, 0])).copy()
        for cb in range(1, 16):
            r = (r + o.embed_row("cp", cb - 1, int(ref_codes[f, cb]))).astype(np.float32)
        codec.append(r)
    n_codec = len(codec)
    icl = []
    for i in range(n_codec):
        t = tp[i] if i < len(stream) else pad
        icl.append(((np.zeros(d, np.float32) + t) + codec[i]).astype(np.float32))
    prefill = np.concatenate([role, over.astype(np.float32), np.stack(icl)]).astype(np.float32)
    trailing = tp[n_codec:] if len(stream) > n_codec else np.zeros((0, d), np.float32)
    return prefill, trailing, pad


@pytest.mark.parametrize("layout", ["tiny", "tiny_mtp"])
@pytest.mark.parametrize("wtype", ["q8_0", "f16"])
def test_facade_matches_oracle(tmp_path, wtype, layout):
    """tiny_mtp: the 1.7B layout (code_pred.mtp_proj, a narrower code
    predictor) read from the GGUF keys and tensors."""
    cfg = getattr(qcfg, layout)()
    _facade_check(tmp_path, cfg, Weights(cfg, wtype, seed=31), wtype, layout, 20)


@pytest.mark.slow
def test_facade_full_06b_q8(tmp_path):
    """The facade over a full-size Q8_0 0.6B GGUF file (about 1.3 GB: the
    151,936-row text embedding, 28 + 5 layers, 16 heads) written in the
    reference converter's metadata form (its key aliases, general.* strings,
    the mrope_section array and tokenizer arrays): load_model, generate,
    attention dump, predict_codes_autoregressive and generate_icl against the
    oracle."""
    cfg = qcfg.full_06b()
    print("[gpu] facade full 0.6B q8_0: synth", file=sys.stderr, flush=True)
    _facade_check(tmp_path, cfg, Weights(cfg, "q8_0", seed=31), "q8_0", "full_06b", 12, converter=True)


def _facade_check(tmp_path, cfg, w, wtype, layout, max_len, converter=False):
    """converter: the file carries the reference converter's metadata form
    (gguf.write_converter: alias keys, general.* strings, the mrope_section
    array, tokenizer arrays).  load_model streams every tensor to HBM in row
    ranges through the pinned staging buffer (the 622 MB text embedding in
    64 MiB pieces)."""
    assert os.path.exists(BIN), "build() first"
    model = tmp_path / "model.gguf"
    if converter:
        gguf.write_converter(str(model), cfg, w, wtype)
    else:
        gguf.write(str(model), cfg, w)
    rng = np.random.default_rng(32)
    text = rng.integers(0, cfg.text_vocab - 8, 26).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)
    ref_codes = np.concatenate([rng.integers(0, 2048, (6, 1)), rng.integers(0, 2048, (6, 15))], axis=1).astype(np.int32)
    with open(tmp_path / "in.bin", "wb") as f:
        f.write(struct.pack("<i", len(text)) + text.tobytes() + spk.tobytes())
        f.write(struct.pack("<ii", max_len, ref_codes.shape[0]) + ref_codes.tobytes())
    print(f"[gpu] facade {wtype} {layout}", file=sys.stderr, flush=True)
    r = subprocess.run([BIN, str(model), str(tmp_path / "in.bin"), str(tmp_path)], capture_output=True, text=True,
                       timeout=300, env=dict(os.environ, QWEN3_TTS_TIMING="1",
                                             QWEN3_TTS_DUMP_CODES=str(tmp_path / "dump.bin")))
    print(r.stdout, r.stderr, file=sys.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    # QWEN3_TTS_TIMING=1: the timing report after every generate / generate_icl
    # (src/tts_transformer.cpp:3311-3352)
    assert r.stderr.count("=== Detailed Generation Timing") >= 3, r.stderr
    assert "frames/s" in r.stderr and "Frame loop" in r.stderr
    codes = np.fromfile(tmp_path / "codes.bin", np.int32).reshape(-1, 16)
    o = orc.Oracle(cfg, w, threads=16)
    co, _ = o.generate(text, spk, max_len=max_len, temperature=0.0)
    assert np.array_equal(codes, co)
    # the ATTD file of set_attn_dump (src/tts_transformer.cpp:2978-3005):
    # one row per talker step of the frame loop, layer 1
    raw = (tmp_path / "attn.bin").read_bytes()
    magic, version, layer, n_head, n_rows = struct.unpack_from("<Iiiii", raw, 0)
    assert (magic, version, layer, n_head) == (0x41545444, 1, 1, cfg.n_head)
    o.set_attn_capture(1)
    o.generate(text, spk, max_len=max_len, temperature=0.0)
    rows_o = o.attn_rows()
    o.set_attn_capture(-1)
    assert n_rows == len(rows_o) == min(co.shape[0], max_len - 1)
    off = 20
    for ro in rows_o:
        (n_kv,) = struct.unpack_from("<i", raw, off)
        row = np.frombuffer(raw, np.float32, n_head * n_kv, off + 4).reshape(n_head, n_kv)
        off += 4 + 4 * n_head * n_kv
        assert np.array_equal(row, ro)
    assert off == len(raw)
    hid = np.fromfile(tmp_path / "hidden.bin", np.float32)
    cp = np.fromfile(tmp_path / "cp.bin", np.int32)
    cpo, _ = o.code_pred(hid, 5)
    assert np.array_equal(cp, cpo)
    # predict_codes, the single-pass predictor, without and with the last
    # frame's codes 1..15
    pc0 = np.fromfile(tmp_path / "pc0.bin", np.float32).reshape(15, cfg.cp_vocab)
    pc1 = np.fromfile(tmp_path / "pc1.bin", np.float32).reshape(15, cfg.cp_vocab)
    assert np.array_equal(pc0, o.predict_codes(hid))
    assert np.array_equal(pc1, o.predict_codes(hid, codes[-1, 1:]))
    icl = np.fromfile(tmp_path / "icl.bin", np.int32).reshape(-1, 16)
    # QWEN3_TTS_DUMP_CODES: the last call's codes (generate_icl), int32 n then the codes
    dump = np.fromfile(tmp_path / "dump.bin", np.int32)
    assert dump[0] == icl.size and np.array_equal(dump[1:], icl.ravel())
    pre, trail, pad = icl_rows(o, cfg, text, text, ref_codes, spk)
    io = o.generate_rows(pre, trail, pad, max_len=max_len, temperature=0.0)
    assert np.array_equal(icl, io)


def test_vocoder_facade_streams_from_device_codes(tmp_path):
    """The drop-in AudioTokenizerDecoder loads a tokenizer GGUF (decoder
    widths read from the tensor shapes) and streams generate()'s frames the
    way src/qwen3_tts.cpp:271-316 does, from the frame loop's device code rows:
    the windows equal the host-codes windows bit for bit, their audio equals
    the oracle's windows within the vocoder tolerance, and the streamed length
    equals the whole decode's."""
    from qwen3_tts_amd import vocoder as V
    vbin = os.path.join(PKG_DIR, "lib", "test_vocoder_dev")
    assert os.path.exists(vbin), "build() first"
    cfg = qcfg.tiny()
    w = Weights(cfg, "q8_0", seed=33)
    gguf.write(str(tmp_path / "tts.gguf"), cfg, w)
    vc = V.VocConfig(codebook_dim=16, hidden=64, latent=128, n_layers=2, n_heads=2, ffn=128, cnx_ffn=256,
                     decoder_dim=128)          # head_dim 64, as load_model assumes
    vw = V.VocWeights(vc, seed=34)
    gguf.write_vocoder(str(tmp_path / "voc.gguf"), vc, vw)
    text = np.random.default_rng(35).integers(0, cfg.text_vocab - 8, 18).astype(np.int32)
    chunk, context, max_len = 7, 5, 30
    with open(tmp_path / "in.bin", "wb") as f:
        f.write(struct.pack("<i", len(text)) + text.tobytes() + struct.pack("<iii", max_len, chunk, context))
    print("[gpu] vocoder facade", file=sys.stderr, flush=True)
    r = subprocess.run([vbin, str(tmp_path / "tts.gguf"), str(tmp_path / "voc.gguf"), str(tmp_path / "in.bin"),
                        str(tmp_path)], capture_output=True, text=True, timeout=300)
    print(r.stdout[-3000:], r.stderr[-2000:], file=sys.stderr)
    assert r.returncode == 0 and "ALL PASS" in r.stdout
    codes = np.fromfile(tmp_path / "codes.bin", np.int32).reshape(-1, 16)
    stream = np.fromfile(tmp_path / "stream.bin", np.float32)
    bounds = np.fromfile(tmp_path / "bounds.bin", np.int32)
    whole = np.fromfile(tmp_path / "whole.bin", np.float32)
    n = codes.shape[0]
    assert n > chunk and bounds[-1] == n
    assert stream.size == whole.size == vc.samples_for_frames(n)
    o = orc.VocOracle(vc, vw, threads=8)
    at, start = 0, 0
    for end in bounds:
        ref = o.decode_window(codes, start, int(end), context)
        got = stream[at:at + ref.size]
        snr = 10 * np.log10((ref.astype(np.float64) ** 2).mean() / max(((got - ref) ** 2).mean(), 1e-30))
        assert snr >= 30.0, (start, end, snr)
        at += ref.size
        start = int(end)
    assert at == stream.size
