"""Minimal GGUF v3 writer for synthetic models (the `gguf` package is not
installed here).  Writes the metadata keys parse_config reads
(src/tts_transformer.cpp:250-374) and the tensors of a synth.Weights."""
import struct

import numpy as np

ALIGN = 32
T_U32, T_F32, T_STR = 4, 6, 8


def _s(b):
    b = b.encode()
    return struct.pack("<Q", len(b)) + b


def config_kv(cfg):
    u = {
        "qwen3-tts.text.vocab_size": cfg.text_vocab, "qwen3-tts.text.embedding_dim": cfg.text_embd_dim,
        "qwen3-tts.talker.embedding_length": cfg.hidden_size, "qwen3-tts.talker.block_count": cfg.n_layers,
        "qwen3-tts.talker.attention.head_count": cfg.n_head,
        "qwen3-tts.talker.attention.head_count_kv": cfg.n_kv_head,
        "qwen3-tts.talker.feed_forward_length": cfg.ffn_size, "qwen3-tts.talker.attention.key_length": cfg.head_dim,
        "qwen3-tts.talker.codec_vocab_size": cfg.codec_vocab, "qwen3-tts.talker.num_codebooks": cfg.n_codebooks,
        "qwen3-tts.code_pred.layer_count": cfg.cp_layers, "qwen3-tts.code_pred.vocab_size": cfg.cp_vocab,
        "qwen3-tts.code_pred.embedding_length": cfg.cp_hidden, "qwen3-tts.code_pred.feed_forward_length": cfg.cp_ffn,
        "qwen3-tts.codec.pad_id": cfg.codec_pad_id, "qwen3-tts.codec.bos_id": cfg.codec_bos_id,
        "qwen3-tts.codec.eos_id": cfg.codec_eos_id, "qwen3-tts.tts_bos_token_id": cfg.tts_bos_id,
        "qwen3-tts.tts_eos_token_id": cfg.tts_eos_id, "qwen3-tts.tts_pad_token_id": cfg.tts_pad_id,
        "qwen3-tts.codec.think_id": cfg.codec_think_id, "qwen3-tts.codec.nothink_id": cfg.codec_nothink_id,
        "qwen3-tts.codec.think_bos_id": cfg.codec_think_bos_id, "qwen3-tts.codec.think_eos_id": cfg.codec_think_eos_id,
        "qwen3-tts.language.english_id": cfg.english_language_id,
    }
    f = {
        "qwen3-tts.talker.attention.layer_norm_rms_epsilon": cfg.rms_eps,
        "qwen3-tts.talker.rope.freq_base": cfg.rope_theta, "qwen3-tts.code_pred.rope.freq_base": cfg.cp_rope_theta,
    }
    return u, f


def write(path, cfg, weights):
    u, f = config_kv(cfg)
    _write(path, u, f, list(weights.items()))


def write_vocoder(path, vcfg, weights):
    """the tokenizer GGUF's decoder part: the three keys load_model reads
    (src/audio_tokenizer_decoder.cpp:108-110) and the tok_dec.* tensors"""
    u = {"qwen3-tts.tokenizer.sample_rate": 24000, "qwen3-tts.tokenizer.num_codebooks": vcfg.n_codebooks,
         "qwen3-tts.tokenizer.codebook_size": vcfg.codebook_size}
    _write(path, u, {}, list(weights.items()))


def _write(path, u, f, tensors):
    kv = [("general.architecture", T_STR, "qwen3-tts"), ("general.alignment", T_U32, ALIGN)]
    kv += [(k, T_U32, v) for k, v in u.items()] + [(k, T_F32, v) for k, v in f.items()]
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, t, v in kv:
        head += _s(k) + struct.pack("<I", t)
        head += _s(v) if t == T_STR else struct.pack("<I" if t == T_U32 else "<f", v)
    off = 0
    offsets = []
    for name, (ttype, ne, arr) in tensors:
        if len(ne) == 2:
            dims = [ne[0]] if ne[1] == 1 else [ne[0], ne[1]]
        else:
            dims = list(ne)
        head += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ttype, off)
        offsets.append(off)
        off += (arr.nbytes + ALIGN - 1) // ALIGN * ALIGN
    with open(path, "wb") as fh:
        fh.write(head)
        fh.write(b"\0" * ((-len(head)) % ALIGN))
        for (name, (ttype, ne, arr)), o in zip(tensors, offsets):
            b = np.ascontiguousarray(arr).view(np.uint8).tobytes()
            fh.write(b)
            fh.write(b"\0" * ((-len(b)) % ALIGN))
