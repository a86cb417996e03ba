"""Minimal GGUF v3 writer for synthetic models (the `gguf` package is not
installed here).  Two metadata forms over the tensors of a synth.Weights:

  write(...)            the primary keys parse_config reads first
                        (src/tts_transformer.cpp:250-374);
  write_converter(...)  the keys, arrays and strings the reference converter
                        writes (scripts/convert_tts_to_gguf.py:421-481 and its
                        tokenizer section): the secondary alias keys
                        (qwen3-tts.block_count, qwen3-tts.code_predictor.*),
                        general.* strings, the rope.mrope_section array and
                        tokenizer string / int32 arrays, so a reader's alias
                        and array-skipping paths run."""
import struct

import numpy as np

ALIGN = 32
T_U32, T_I32, T_F32, T_STR, T_ARR = 4, 5, 6, 8, 9


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


# general.file_type of the converter's --type choices (gguf LlamaFileType)
FILE_TYPE = {"f32": 0, "f16": 1, "q8_0": 7}


def converter_kv(cfg, wtype, n_tokens=4096):
    """(key, type, value) entries in the converter's order; arrays are
    (T_ARR, (element type, values))."""
    a = "qwen3-tts"
    kv = [
        ("general.architecture", T_STR, a),
        ("general.name", T_STR, "Qwen3-TTS-12Hz-0.6B-Base"),
        ("general.type", T_STR, "model"),
        ("general.file_type", T_U32, FILE_TYPE[wtype]),
        ("general.quantization_version", T_U32, 2),
        (f"{a}.block_count", T_U32, cfg.n_layers),
        (f"{a}.embedding_length", T_U32, cfg.hidden_size),
        (f"{a}.feed_forward_length", T_U32, cfg.ffn_size),
        (f"{a}.attention.head_count", T_U32, cfg.n_head),
        (f"{a}.attention.head_count_kv", T_U32, cfg.n_kv_head),
        (f"{a}.attention.key_length", T_U32, cfg.head_dim),
        (f"{a}.attention.value_length", T_U32, cfg.head_dim),
        (f"{a}.rope.freq_base", T_F32, cfg.rope_theta),
        (f"{a}.attention.layer_norm_rms_epsilon", T_F32, cfg.rms_eps),
        (f"{a}.vocab_size", T_U32, cfg.codec_vocab),
        (f"{a}.text_vocab_size", T_U32, cfg.text_vocab),
        (f"{a}.text_hidden_size", T_U32, cfg.text_embd_dim),
        (f"{a}.num_code_groups", T_U32, cfg.n_codebooks),
        (f"{a}.rope.mrope_section", T_ARR, (T_I32, [24, 20, 20])),
        (f"{a}.code_predictor.layer_count", T_U32, cfg.cp_layers),
        (f"{a}.code_predictor.vocab_size", T_U32, cfg.cp_vocab),
        (f"{a}.code_predictor.embedding_length", T_U32, cfg.cp_hidden),
        (f"{a}.code_predictor.feed_forward_length", T_U32, cfg.cp_ffn),
        (f"{a}.code_predictor.rope.freq_base", T_F32, cfg.cp_rope_theta),
        (f"{a}.speaker_encoder.embedding_length", T_U32, 1024),
        (f"{a}.speaker_encoder.sample_rate", T_U32, 24000),
        (f"{a}.codec.pad_id", T_U32, cfg.codec_pad_id),
        (f"{a}.codec.bos_id", T_U32, cfg.codec_bos_id),
        (f"{a}.codec.eos_id", T_U32, cfg.codec_eos_id),
        ("tokenizer.ggml.model", T_STR, "gpt2"),
        ("tokenizer.ggml.pre", T_STR, "qwen2"),
        # a synthetic byte-level vocabulary and merge list of the converter's
        # array types (the real ones hold the text tokenizer's 151k entries)
        ("tokenizer.ggml.tokens", T_ARR, (T_STR, [f"tok{i}" for i in range(n_tokens)])),
        ("tokenizer.ggml.token_type", T_ARR, (T_I32, [1] * n_tokens)),
        ("tokenizer.ggml.merges", T_ARR, (T_STR, [f"t o{i}" for i in range(n_tokens // 2)])),
        ("tokenizer.ggml.eos_token_id", T_U32, 151643),
        ("tokenizer.ggml.padding_token_id", T_U32, 151643),
        ("tokenizer.chat_template", T_STR, "{% for message in messages %}{{ message['content'] }}{% endfor %}"),
    ]
    return kv


def write_converter(path, cfg, weights, wtype):
    """the converter's metadata form (see the module docstring); its keys
    leave the tts / think / language ids to parse_config's defaults, so use
    it with the full 0.6B config, whose ids are those defaults"""
    _write_kv(path, converter_kv(cfg, wtype), list(weights.items()))


def write_vocoder(path, vcfg, weights):
    """the tokenizer GGUF's decoder part: the three keys load_model reads
    (src/audio_tokenizer_decoder.cpp:108-110) and the tok_dec.* tensors"""
    u = {"qwen3-tts.tokenizer.sample_rate": 24000, "qwen3-tts.tokenizer.num_codebooks": vcfg.n_codebooks,
         "qwen3-tts.tokenizer.codebook_size": vcfg.codebook_size}
    _write(path, u, {}, list(weights.items()))


def _write(path, u, f, tensors):
    kv = [("general.architecture", T_STR, "qwen3-tts"), ("general.alignment", T_U32, ALIGN)]
    kv += [(k, T_U32, v) for k, v in u.items()] + [(k, T_F32, v) for k, v in f.items()]
    _write_kv(path, kv, tensors)


def _value(t, v):
    if t == T_STR:
        return _s(v)
    if t == T_ARR:
        et, vals = v
        body = b"".join(_value(et, x) for x in vals)
        return struct.pack("<IQ", et, len(vals)) + body
    return struct.pack({T_U32: "<I", T_I32: "<i", T_F32: "<f"}[t], v)


def _write_kv(path, kv, tensors):
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for k, t, v in kv:
        head += _s(k) + struct.pack("<I", t) + _value(t, v)
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
