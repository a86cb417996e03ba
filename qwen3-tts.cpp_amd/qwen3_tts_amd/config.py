"""Model hyperparameters of the qwen3-tts talker + code predictor.

Field order matches ``q3t_config`` in include/q3t_dev.h, which mirrors
``tts_transformer_config`` (src/tts_transformer.h:59-103); defaults are the
values parse_config falls back to (src/tts_transformer.cpp:228-377).
"""
import ctypes
import dataclasses

_FIELDS = [
    ("hidden_size", ctypes.c_int32), ("n_layers", ctypes.c_int32), ("n_head", ctypes.c_int32),
    ("n_kv_head", ctypes.c_int32), ("head_dim", ctypes.c_int32), ("ffn_size", ctypes.c_int32),
    ("codec_vocab", ctypes.c_int32), ("n_codebooks", ctypes.c_int32), ("cp_layers", ctypes.c_int32),
    ("cp_vocab", ctypes.c_int32), ("cp_hidden", ctypes.c_int32), ("cp_ffn", ctypes.c_int32),
    ("text_vocab", ctypes.c_int32), ("text_embd_dim", ctypes.c_int32),
    ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("cp_rope_theta", ctypes.c_float),
    ("codec_pad_id", ctypes.c_int32), ("codec_bos_id", ctypes.c_int32), ("codec_eos_id", ctypes.c_int32),
    ("tts_bos_id", ctypes.c_int32), ("tts_eos_id", ctypes.c_int32), ("tts_pad_id", ctypes.c_int32),
    ("codec_think_id", ctypes.c_int32), ("codec_nothink_id", ctypes.c_int32),
    ("codec_think_bos_id", ctypes.c_int32), ("codec_think_eos_id", ctypes.c_int32),
    ("english_language_id", ctypes.c_int32),
]


class CConfig(ctypes.Structure):
    _fields_ = _FIELDS


@dataclasses.dataclass
class Config:
    hidden_size: int = 1024
    n_layers: int = 28
    n_head: int = 16
    n_kv_head: int = 8
    head_dim: int = 128
    ffn_size: int = 3072
    codec_vocab: int = 3072
    n_codebooks: int = 16
    cp_layers: int = 5
    cp_vocab: int = 2048
    cp_hidden: int = 1024
    cp_ffn: int = 3072
    text_vocab: int = 151936
    text_embd_dim: int = 2048
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    cp_rope_theta: float = 1e6
    codec_pad_id: int = 2148
    codec_bos_id: int = 2149
    codec_eos_id: int = 2150
    tts_bos_id: int = 151672
    tts_eos_id: int = 151673
    tts_pad_id: int = 151671
    codec_think_id: int = 2154
    codec_nothink_id: int = 2155
    codec_think_bos_id: int = 2156
    codec_think_eos_id: int = 2157
    english_language_id: int = 2050

    def to_c(self, cls=CConfig):
        c = cls()
        for name, _ in _FIELDS:
            setattr(c, name, getattr(self, name))
        return c


def full_06b():
    """The reference 0.6B shapes (Qwen3-TTS-12Hz-0.6B-Base)."""
    return Config()


def tiny(n_layers=2, cp_layers=2, hidden=256, ffn=512, n_head=4, n_kv_head=2, text_vocab=4096, text_embd=256):
    """Small shapes for fast parity tests: same head_dim, codec and code-predictor
    vocabularies (the sampler's suppression window and special ids depend on
    them), narrow widths and few layers."""
    return Config(hidden_size=hidden, n_layers=n_layers, n_head=n_head, n_kv_head=n_kv_head, ffn_size=ffn,
                  cp_layers=cp_layers, cp_hidden=hidden, cp_ffn=ffn, text_vocab=text_vocab,
                  text_embd_dim=text_embd, tts_bos_id=text_vocab - 3, tts_eos_id=text_vocab - 2,
                  tts_pad_id=text_vocab - 4)


def tiny_mtp(n_layers=2, cp_layers=2, hidden=512, cp_hidden=256, ffn=512, cp_ffn=512, n_head=4, n_kv_head=2,
             text_vocab=4096, text_embd=256):
    """Small shapes of the 1.7B layout: the code predictor is narrower than the
    talker and its inputs pass through code_pred.mtp_proj."""
    return Config(hidden_size=hidden, n_layers=n_layers, n_head=n_head, n_kv_head=n_kv_head, ffn_size=ffn,
                  cp_layers=cp_layers, cp_hidden=cp_hidden, cp_ffn=cp_ffn, text_vocab=text_vocab,
                  text_embd_dim=text_embd, tts_bos_id=text_vocab - 3, tts_eos_id=text_vocab - 2,
                  tts_pad_id=text_vocab - 4)


def full_17b():
    """The 1.7B layout: a 2048-wide talker (FFN 6144) over a 1024-wide code
    predictor reached through code_pred.mtp_proj."""
    return Config(hidden_size=2048, ffn_size=6144, cp_hidden=1024, cp_ffn=3072)
