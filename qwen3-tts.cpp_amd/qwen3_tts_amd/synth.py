"""Seeded synthetic weights with the reference tensor names, shapes and types.

Names and shapes follow create_tensors (src/tts_transformer.cpp:379-668);
which tensors are Q8_0, F16 or F32 follows the converter's policy
(scripts/convert_tts_to_gguf.py:249-324): 1-D tensors are F32; in the Q8_0
model embeddings, ``codec_head`` and ``lm_head`` stay F16 and every other
matrix is Q8_0.

Weights are N(0, std) from numpy's PCG64, one independent stream per tensor
(seeded by hash of (seed, name)), so any tensor can be regenerated alone.
"""
import hashlib

import numpy as np

F32, F16, Q8_0 = 0, 1, 8


def quantize_q8_0(x):
    """gguf-py's Q8_0 quantisation (used by the converter): per 32-block
    d = max|x| / 127 in float32, q = round-half-away-from-zero(x / d), d
    stored as float16.  Returns uint8 blocks of 34 bytes (d, then 32 int8)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, 32)
    d = np.abs(x).max(axis=1, keepdims=True) / np.float32(127)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = x / d
    a = np.abs(r)
    fl = np.floor(a)
    q = np.sign(r) * (fl + np.floor(np.float32(2) * (a - fl)))
    q[np.broadcast_to(d == 0, q.shape)] = 0
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    out[:, :2] = d.astype(np.float16).view(np.uint8)
    out[:, 2:] = q.astype(np.int8).view(np.uint8)
    return out.reshape(-1)


def dequantize_q8_0(blocks):
    b = np.asarray(blocks, dtype=np.uint8).reshape(-1, 34)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    return (d * q).reshape(-1)


def tensor_specs(cfg, wtype="q8_0"):
    """[(name, type, (ne0, ne1))] for every tensor the frame loop reads.  The
    code predictor's blocks, output norm and heads have its own width
    cp_hidden; its embeddings have the talker width, and a model whose widths
    differ (the 1.7B layout) carries code_pred.mtp_proj between the two
    (src/tts_transformer.cpp:496-553)."""
    d, te, dc = cfg.hidden_size, cfg.text_embd_dim, cfg.cp_hidden
    qd, kd = cfg.n_head * cfg.head_dim, cfg.n_kv_head * cfg.head_dim
    mat = Q8_0 if wtype == "q8_0" else F16
    specs = [
        ("talker.text_embd.weight", F16, (te, cfg.text_vocab)),
        ("talker.text_proj.fc1.weight", mat, (te, te)),
        ("talker.text_proj.fc1.bias", F32, (te, 1)),
        ("talker.text_proj.fc2.weight", mat, (te, d)),
        ("talker.text_proj.fc2.bias", F32, (d, 1)),
        ("talker.codec_embd.weight", F16, (d, cfg.codec_vocab)),
        ("talker.codec_head.weight", F16, (d, cfg.codec_vocab)),
        ("talker.output_norm.weight", F32, (d, 1)),
        ("code_pred.output_norm.weight", F32, (dc, 1)),
    ]
    if dc != d:
        specs += [("code_pred.mtp_proj.weight", mat, (d, dc)), ("code_pred.mtp_proj.bias", F32, (dc, 1))]
    for prefix, nl, ffn, d in (("talker", cfg.n_layers, cfg.ffn_size, d), ("code_pred", cfg.cp_layers, cfg.cp_ffn, dc)):
        for i in range(nl):
            p = f"{prefix}.blk.{i}."
            specs += [
                (p + "attn_norm.weight", F32, (d, 1)),
                (p + "attn_q_norm.weight", F32, (cfg.head_dim, 1)),
                (p + "attn_k_norm.weight", F32, (cfg.head_dim, 1)),
                (p + "attn_q.weight", mat, (d, qd)),
                (p + "attn_k.weight", mat, (d, kd)),
                (p + "attn_v.weight", mat, (d, kd)),
                (p + "attn_output.weight", mat, (qd, d)),
                (p + "ffn_norm.weight", F32, (d, 1)),
                (p + "ffn_gate.weight", mat, (d, ffn)),
                (p + "ffn_up.weight", mat, (d, ffn)),
                (p + "ffn_down.weight", mat, (ffn, d)),
            ]
    for g in range(cfg.n_codebooks - 1):
        specs.append((f"code_pred.codec_embd.{g}.weight", F16, (cfg.hidden_size, cfg.cp_vocab)))
        specs.append((f"code_pred.lm_head.{g}.weight", F16, (dc, cfg.cp_vocab)))
    return specs


def _rng(seed, name):
    h = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(h[:8], "little")))


def make_tensor(seed, name, ttype, ne, std=0.02, norm_mode="one"):
    """Raw tensor bytes (numpy array) in ggml layout.

    Norm weights (1-D ``*_norm.weight``) are 1 + N(0, std) when norm_mode is
    "one" (as trained RMSNorm gains sit near 1) or N(0, std) when "normal";
    biases are N(0, std)."""
    ne0, ne1 = ne
    rng = _rng(seed, name)
    x = rng.standard_normal(ne0 * ne1, dtype=np.float32) * np.float32(std)
    if ne1 == 1 and name.endswith("norm.weight") and norm_mode == "one":
        x += np.float32(1.0)
    if ttype == F32:
        return x.astype(np.float32)
    if ttype == F16:
        return x.astype(np.float16)
    return quantize_q8_0(x)


class Weights:
    """name -> (type, (ne0, ne1), ndarray).  Arrays stay alive as long as this
    object does (the CPU oracle borrows their buffers)."""

    def __init__(self, cfg, wtype="q8_0", seed=1234, std=0.02, norm_mode="one"):
        self.cfg, self.wtype, self.seed = cfg, wtype, seed
        self.tensors = {}
        for name, ttype, ne in tensor_specs(cfg, wtype):
            self.tensors[name] = (ttype, ne, make_tensor(seed, name, ttype, ne, std, norm_mode))

    def items(self):
        return self.tensors.items()

    def __getitem__(self, k):
        return self.tensors[k]

    def nbytes(self):
        return sum(a.nbytes for _, _, a in self.tensors.values())
