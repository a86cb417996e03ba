"""Audio-tokenizer decoder (vocoder): configuration, synthetic weights and the
ctypes binding of the HIP vocoder (include/q3t_voc.h).

Widths follow audio_decoder_config (src/audio_tokenizer_decoder.h:15-29) and
the checkpoint's tensor shapes (docs/model_inspection.txt:923-1182); tensor
names are the GGUF's tok_dec.* names (src/audio_tokenizer_decoder.cpp:158-313),
laid out in ggml ne order (ne0 contiguous).
"""
import ctypes
import dataclasses
import hashlib

import numpy as np

from .synth import F16, F32

_FIELDS = [
    ("n_codebooks", ctypes.c_int32), ("codebook_size", ctypes.c_int32), ("codebook_dim", ctypes.c_int32),
    ("hidden", ctypes.c_int32), ("latent", ctypes.c_int32), ("n_layers", ctypes.c_int32),
    ("n_heads", ctypes.c_int32), ("ffn", ctypes.c_int32), ("cnx_ffn", ctypes.c_int32),
    ("up_kernel", ctypes.c_int32), ("decoder_dim", ctypes.c_int32), ("rates", ctypes.c_int32 * 4),
    ("dec_kernel", ctypes.c_int32 * 4), ("rms_eps", ctypes.c_float), ("rope_theta", ctypes.c_float),
]


class CVocConfig(ctypes.Structure):
    """q3t_voc_config (include/q3t_voc.h) == orc_voc_config (oracle)."""
    _fields_ = _FIELDS


@dataclasses.dataclass
class VocConfig:
    n_codebooks: int = 16
    codebook_size: int = 2048
    codebook_dim: int = 256
    hidden: int = 512
    latent: int = 1024
    n_layers: int = 8
    n_heads: int = 16
    ffn: int = 1024
    cnx_ffn: int = 4096
    up_kernel: int = 2
    decoder_dim: int = 1536
    rates: tuple = (8, 5, 4, 3)
    dec_kernel: tuple = (16, 10, 8, 6)
    rms_eps: float = 1e-5
    rope_theta: float = 1e4

    def to_c(self, cls=CVocConfig):
        c = cls()
        for name, _ in _FIELDS:
            v = getattr(self, name)
            if isinstance(v, tuple):
                arr = getattr(c, name)
                for i, e in enumerate(v):
                    arr[i] = e
            else:
                setattr(c, name, v)
        return c

    def channels(self):
        """input width of decoder blocks 1..4, then the final width"""
        ch = [self.decoder_dim]
        for _ in range(4):
            ch.append(ch[-1] // 2)
        return ch

    def samples_for_frames(self, n):
        """output_samples_for_frames (src/audio_tokenizer_decoder.cpp:845-875)"""
        if n <= 0:
            return 0
        for _ in range(2):
            n = (n - 1) * 2 + self.up_kernel
        for s, k in zip(self.rates, self.dec_kernel):
            n = (n - 1) * s + k - 2 * (k - s)
        return max(n, 0)


def full():
    """The 12 Hz tokenizer's decoder (docs/model_inspection.txt:777-810)."""
    return VocConfig()


def tiny():
    """Narrow widths, the same structure, code range and upsampling."""
    return VocConfig(codebook_dim=16, hidden=64, latent=128, n_layers=2, n_heads=4, ffn=128, cnx_ffn=256,
                     decoder_dim=128)


def tensor_specs(c):
    """[(name, type, ne, std, kind)]: ggml ne tuple; kind picks the synthetic
    distribution ("w": N(0, std), "one": 1 + N(0, std), "usage": U[0.5, 2)
    with a few entries below the 1e-5 clamp, "const": std)."""
    s = []
    cd, h, lt = c.codebook_dim, c.hidden, c.latent

    def w(name, ne, fan_in, gain=1.0):
        s.append((name, F16, ne, gain / np.sqrt(fan_in), "w"))

    def v(name, n, std=0.02, kind="w"):
        s.append((name, F32, (n,), std, kind))

    w("tok_dec.vq_first.output_proj.weight", (1, cd, h), cd)
    w("tok_dec.vq_rest.output_proj.weight", (1, cd, h), cd * 4)
    s.append(("tok_dec.vq_first.0.codebook", F16, (cd, c.codebook_size), 1.0, "w"))
    v("tok_dec.vq_first.0.usage", c.codebook_size, kind="usage")
    for i in range(c.n_codebooks - 1):
        s.append((f"tok_dec.vq_rest.{i}.codebook", F16, (cd, c.codebook_size), 1.0, "w"))
        v(f"tok_dec.vq_rest.{i}.usage", c.codebook_size, kind="usage")
    w("tok_dec.pre_conv.weight", (3, h, lt), 3 * h)
    v("tok_dec.pre_conv.bias", lt)
    w("tok_dec.pre_tfm.input_proj.weight", (lt, h), lt)
    v("tok_dec.pre_tfm.input_proj.bias", h)
    for l in range(c.n_layers):
        p = f"tok_dec.pre_tfm.blk.{l}."
        v(p + "attn_norm.weight", h, 0.05, "one")
        w(p + "attn_q.weight", (h, lt), h)
        w(p + "attn_k.weight", (h, lt), h)
        w(p + "attn_v.weight", (h, lt), h)
        w(p + "attn_output.weight", (lt, h), lt)
        v(p + "attn_scale", h, 0.3)
        v(p + "ffn_norm.weight", h, 0.05, "one")
        w(p + "ffn_gate.weight", (h, c.ffn), h)
        w(p + "ffn_up.weight", (h, c.ffn), h)
        w(p + "ffn_down.weight", (c.ffn, h), c.ffn)
        v(p + "ffn_scale", h, 0.3)
    v("tok_dec.pre_tfm.norm.weight", h, 0.05, "one")
    w("tok_dec.pre_tfm.output_proj.weight", (h, lt), h)
    v("tok_dec.pre_tfm.output_proj.bias", lt)
    for i in range(2):
        p = f"tok_dec.upsample.{i}."
        w(p + "conv.weight", (c.up_kernel, lt, lt), lt)
        v(p + "conv.bias", lt)
        w(p + "dwconv.weight", (7, 1, lt), 7)
        v(p + "dwconv.bias", lt)
        v(p + "norm.weight", lt, 0.05, "one")
        v(p + "norm.bias", lt)
        w(p + "pwconv1.weight", (lt, c.cnx_ffn), lt)
        v(p + "pwconv1.bias", c.cnx_ffn)
        w(p + "pwconv2.weight", (c.cnx_ffn, lt), c.cnx_ffn)
        v(p + "pwconv2.bias", lt)
        v(p + "gamma", lt, 0.3)
    w("tok_dec.dec.0.conv.weight", (7, lt, c.decoder_dim), 7 * lt)
    v("tok_dec.dec.0.conv.bias", c.decoder_dim)
    ch = c.decoder_dim
    for b in range(4):
        p = f"tok_dec.dec.{b + 1}."
        co = ch // 2
        v(p + "snake.alpha", ch, 0.3)
        v(p + "snake.beta", ch, 0.3)
        w(p + "conv_t.weight", (c.dec_kernel[b], co, ch), 2 * ch)
        v(p + "conv_t.bias", co)
        for r in range(2, 5):
            q = p + f"res.{r}."
            v(q + "act1.alpha", co, 0.3)
            v(q + "act1.beta", co, 0.3)
            w(q + "conv1.weight", (7, co, co), 7 * co)
            v(q + "conv1.bias", co)
            v(q + "act2.alpha", co, 0.3)
            v(q + "act2.beta", co, 0.3)
            w(q + "conv2.weight", (1, co, co), co, 0.5)
            v(q + "conv2.bias", co)
        ch = co
    v("tok_dec.dec.5.snake.alpha", ch, 0.3)
    v("tok_dec.dec.5.snake.beta", ch, 0.3)
    w("tok_dec.dec.6.conv.weight", (7, ch, 1), 7 * ch, 0.05)
    v("tok_dec.dec.6.conv.bias", 1)
    return s


def _rng(seed, name):
    h = hashlib.sha256(f"voc:{seed}:{name}".encode()).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(h[:8], "little")))


class VocWeights:
    """name -> (type, ne, ndarray), seeded per tensor; arrays stay alive as long
    as this object does (the oracle borrows them)."""

    def __init__(self, cfg, seed=7):
        self.cfg, self.seed = cfg, seed
        self.tensors = {}
        self.clamped = {}          # codebook name -> entries whose usage is below the 1e-5 clamp
        for name, ttype, ne, std, kind in tensor_specs(cfg):
            rng = _rng(seed, name)
            n = int(np.prod(ne))
            if kind == "usage":
                x = rng.uniform(0.5, 2.0, n).astype(np.float32)
                low = rng.choice(n, 3, replace=False)
                x[low] = np.float32(3e-6)
                self.clamped[name.replace(".usage", ".codebook")] = low
            else:
                x = rng.standard_normal(n, dtype=np.float32) * np.float32(std)
                if kind == "one":
                    x += np.float32(1.0)
            self.tensors[name] = (ttype, ne, x.astype(np.float16 if ttype == F16 else np.float32))
        # rows of clamped entries are scaled down so that the normalised row
        # (divided by the clamped 1e-5) stays in fp16 range
        for cb, low in self.clamped.items():
            ttype, ne, a = self.tensors[cb]
            a = a.reshape(ne[1], ne[0]).astype(np.float32)
            a[low] *= np.float32(1e-5)
            self.tensors[cb] = (ttype, ne, a.reshape(-1).astype(np.float16))

    def items(self):
        return self.tensors.items()

    def __getitem__(self, k):
        return self.tensors[k]

    def nbytes(self):
        return sum(a.nbytes for _, _, a in self.tensors.values())
