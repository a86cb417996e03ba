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


# ---------------------------------------------------------------- device
VOC_EXPORTS = [
    "q3t_voc_create", "q3t_voc_destroy", "q3t_voc_last_error", "q3t_voc_set_tensor", "q3t_voc_finalize",
    "q3t_voc_reserve", "q3t_voc_samples_for_frames", "q3t_voc_decode_window", "q3t_voc_decode",
    "q3t_voc_run_stage",
]

_voc_lib = None


def load_voc_library():
    """the device library (lib/libq3t_hip.so) with the vocoder entry points typed"""
    global _voc_lib
    if _voc_lib is None:
        from .device import load_library
        lib = load_library()
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        lib.q3t_voc_create.argtypes = [ctypes.POINTER(CVocConfig), i32, ctypes.POINTER(ctypes.c_char_p)]
        lib.q3t_voc_create.restype = vp
        lib.q3t_voc_destroy.argtypes = [vp]
        lib.q3t_voc_destroy.restype = None
        lib.q3t_voc_last_error.argtypes = [vp]
        lib.q3t_voc_last_error.restype = ctypes.c_char_p
        lib.q3t_voc_set_tensor.argtypes = [vp, ctypes.c_char_p, i32, vp, ctypes.c_size_t]
        lib.q3t_voc_finalize.argtypes = [vp]
        lib.q3t_voc_reserve.argtypes = [vp, i32]
        lib.q3t_voc_samples_for_frames.argtypes = [vp, i32]
        lib.q3t_voc_samples_for_frames.restype = i64
        lib.q3t_voc_decode_window.argtypes = [vp, vp, i32, i32, i32, i32, i32, vp, i64, ctypes.POINTER(i64)]
        lib.q3t_voc_decode.argtypes = [vp, vp, i32, i32, vp, i64, ctypes.POINTER(i64)]
        lib.q3t_voc_run_stage.argtypes = [vp, ctypes.c_char_p, vp, vp, i64, i64, i32, vp, i64,
                                          ctypes.POINTER(i64), ctypes.POINTER(i64)]
        _voc_lib = lib
    return _voc_lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class VocError(RuntimeError):
    pass


class VocDevice:
    """One HIP vocoder context (q3t_voc) on HIP device `device`."""

    def __init__(self, cfg, weights, device=0):
        self.lib = load_voc_library()
        self.cfg = cfg
        self._cc = cfg.to_c()
        err = ctypes.c_char_p()
        self.h = self.lib.q3t_voc_create(ctypes.byref(self._cc), device, ctypes.byref(err))
        if not self.h:
            raise VocError(err.value.decode() if err.value else "q3t_voc_create failed")
        for name, (ttype, ne, arr) in weights.items():
            self._check(self.lib.q3t_voc_set_tensor(self.h, name.encode(), ttype, _p(arr), arr.nbytes), name)
        self._check(self.lib.q3t_voc_finalize(self.h), "finalize")

    def _check(self, rc, what):
        if rc != 0:
            raise VocError(f"{what}: {self.lib.q3t_voc_last_error(self.h).decode()}")

    def close(self):
        if getattr(self, "h", None):
            self.lib.q3t_voc_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def reserve(self, max_frames):
        self._check(self.lib.q3t_voc_reserve(self.h, max_frames), "reserve")

    def samples_for_frames(self, n):
        return int(self.lib.q3t_voc_samples_for_frames(self.h, n))

    def decode_window(self, codes, start, end, context, n_frames=None, device_ptr=None):
        """codes: host [n_frames][16] int32, or device_ptr (int address of
        device code rows, e.g. Device.frame_codes_ptr()) with n_frames."""
        if device_ptr is None:
            codes = np.ascontiguousarray(codes, dtype=np.int32)
            ptr, on_dev, n_frames = _p(codes), 0, codes.shape[0]
        else:
            ptr, on_dev = ctypes.c_void_p(device_ptr), 1
        cap = self.samples_for_frames(end - max(0, start - max(0, context)))
        out = np.zeros(max(cap, 1), np.float32)
        n = ctypes.c_int64(0)
        self._check(self.lib.q3t_voc_decode_window(self.h, ptr, on_dev, n_frames, start, end, context, _p(out), cap,
                                                   ctypes.byref(n)), "decode_window")
        return out[:n.value].copy()

    def decode(self, codes):
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        cap = self.samples_for_frames(codes.shape[0])
        out = np.zeros(max(cap, 1), np.float32)
        n = ctypes.c_int64(0)
        self._check(self.lib.q3t_voc_decode(self.h, _p(codes), 0, codes.shape[0], _p(out), cap, ctypes.byref(n)),
                    "decode")
        return out[:n.value].copy()

    def run_stage(self, name, x, pos0=0):
        """one stage from fp32 rows x [T][C] (codes [T][16] for "latent")"""
        T = x.shape[0]
        if name == "latent":
            codes, xin, C = np.ascontiguousarray(x, dtype=np.int32), None, 16
        else:
            codes, xin = None, np.ascontiguousarray(x, dtype=np.float32)
            C = xin.shape[1]
        c = self.cfg
        cap = max(T, 2) * 8 * max(c.latent, c.cnx_ffn, c.decoder_dim, 16) + 64
        out = np.zeros(cap, np.float32)
        To, Co = ctypes.c_int64(0), ctypes.c_int64(0)
        self._check(self.lib.q3t_voc_run_stage(self.h, name.encode(), _p(xin), _p(codes), T, C, pos0, _p(out), cap,
                                               ctypes.byref(To), ctypes.byref(Co)), f"run_stage {name}")
        return out[:To.value * Co.value].reshape(To.value, Co.value).copy()
