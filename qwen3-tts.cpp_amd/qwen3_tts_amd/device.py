"""ctypes binding of the device C ABI (include/q3t_dev.h).

This is the Python-side equivalent of the binding a host application adds
(see INTEGRATION.md); tests and the benchmark drive the GPU path only through
it.  The shared library is built in-tree (``lib/libq3t_hip.so``); loading it
fails loudly when it is missing: there is no CPU fallback.
"""
import ctypes
import os

import numpy as np

from .config import CConfig

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "lib", "libq3t_hip.so")

EXPORTS = [
    "q3t_dev_create", "q3t_dev_destroy", "q3t_dev_last_error", "q3t_dev_upload_tensor",
    "q3t_dev_upload_tensor_rows", "q3t_dev_staging",
    "q3t_dev_download_tensor", "q3t_dev_dequantize", "q3t_dev_kv_reserve", "q3t_dev_kv_clear",
    "q3t_dev_kv_capacity", "q3t_dev_kv_set_type", "q3t_dev_kv_write", "q3t_dev_set_attn_capture", "q3t_dev_attn_row_count",
    "q3t_dev_attn_row", "q3t_dev_prefill", "q3t_dev_talker_step",
    "q3t_dev_code_pred", "q3t_dev_predict_codes", "q3t_dev_stream_logits", "q3t_dev_text_proj", "q3t_dev_text_proj_noalloc", "q3t_dev_embed_rows",
    "q3t_dev_build_prefill",
    "q3t_dev_build_prefill_icl", "q3t_dev_frames_begin",
    "q3t_dev_frames_run", "q3t_dev_frame_codes", "q3t_dev_frames_stats", "q3t_dev_streams_reserve", "q3t_dev_stream_prefill",
    "q3t_dev_stream_prefill_at", "q3t_dev_stream_kv_write",
    "q3t_dev_streams_begin", "q3t_dev_streams_run", "q3t_dev_sync", "q3t_dev_time_kernel",
]


class CSampling(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("seed", ctypes.c_uint64)]


class CFrameArgs(ctypes.Structure):
    _fields_ = [
        ("trailing", ctypes.c_void_p), ("n_trailing", ctypes.c_int32), ("tts_pad", ctypes.c_void_p),
        ("n_past", ctypes.c_int32), ("max_len", ctypes.c_int32), ("repetition_penalty", ctypes.c_float),
        ("eos_bias", ctypes.c_float), ("target_frames", ctypes.c_int32), ("sampling", CSampling),
    ]


_lib = None


def load_library(path=LIB_PATH):
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise RuntimeError(f"HIP device library not built: {path} (run __graft_entry__.build())")
        lib = ctypes.CDLL(path)
        vp, i32, u32, f32p = ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_void_p
        lib.q3t_dev_create.argtypes = [ctypes.POINTER(CConfig), i32, ctypes.POINTER(vp)]
        lib.q3t_dev_destroy.argtypes = [vp]
        lib.q3t_dev_destroy.restype = None
        lib.q3t_dev_last_error.argtypes = [vp]
        lib.q3t_dev_last_error.restype = ctypes.c_char_p
        lib.q3t_dev_upload_tensor.argtypes = [vp, ctypes.c_char_p, i32, ctypes.POINTER(ctypes.c_int64), vp, ctypes.c_size_t]
        lib.q3t_dev_upload_tensor_rows.argtypes = [vp, ctypes.c_char_p, i32, ctypes.POINTER(ctypes.c_int64),
                                                   ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_size_t]
        lib.q3t_dev_staging.argtypes = [vp, ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)]
        lib.q3t_dev_staging.restype = vp
        lib.q3t_dev_download_tensor.argtypes = [vp, ctypes.c_char_p, vp, ctypes.c_size_t]
        lib.q3t_dev_dequantize.argtypes = [vp, ctypes.c_char_p, f32p, ctypes.c_size_t]
        lib.q3t_dev_kv_reserve.argtypes = [vp, i32]
        lib.q3t_dev_kv_clear.argtypes = [vp]
        lib.q3t_dev_kv_capacity.argtypes = [vp]
        lib.q3t_dev_kv_write.argtypes = [vp, i32, i32, vp, vp]
        lib.q3t_dev_kv_set_type.argtypes = [vp, i32]
        lib.q3t_dev_set_attn_capture.argtypes = [vp, i32]
        lib.q3t_dev_attn_row_count.argtypes = [vp]
        lib.q3t_dev_attn_row.argtypes = [vp, i32, f32p, ctypes.c_int64, ctypes.POINTER(i32)]
        lib.q3t_dev_prefill.argtypes = [vp, f32p, i32, i32, f32p, f32p]
        lib.q3t_dev_talker_step.argtypes = [vp, f32p, i32, f32p, f32p]
        lib.q3t_dev_code_pred.argtypes = [vp, f32p, i32, ctypes.POINTER(CSampling), u32, vp, f32p]
        lib.q3t_dev_predict_codes.argtypes = [vp, f32p, vp, f32p]
        lib.q3t_dev_stream_logits.argtypes = [vp, i32, f32p]
        lib.q3t_dev_text_proj.argtypes = [vp, vp, i32, f32p]
        lib.q3t_dev_text_proj_noalloc.argtypes = [vp, vp, i32, f32p]
        lib.q3t_dev_embed_rows.argtypes = [vp, i32, i32, vp, i32, f32p]
        pi32 = ctypes.POINTER(i32)
        lib.q3t_dev_build_prefill.argtypes = [vp, vp, i32, f32p, i32, vp, i32, f32p, pi32, f32p, pi32, f32p]
        lib.q3t_dev_build_prefill_icl.argtypes = [vp, vp, i32, vp, i32, vp, i32, f32p, f32p, pi32, f32p, pi32, f32p]
        lib.q3t_dev_frames_begin.argtypes = [vp, ctypes.POINTER(CFrameArgs)]
        lib.q3t_dev_frames_run.argtypes = [vp, i32, vp, ctypes.POINTER(i32), ctypes.POINTER(i32)]
        lib.q3t_dev_sync.argtypes = [vp]
        lib.q3t_dev_frame_codes.argtypes = [vp]
        lib.q3t_dev_frame_codes.restype = vp
        lib.q3t_dev_frames_stats.argtypes = [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int64),
                                             ctypes.POINTER(i32)]
        lib.q3t_dev_streams_reserve.argtypes = [vp, i32, i32]
        lib.q3t_dev_stream_prefill.argtypes = [vp, i32, f32p, i32]
        lib.q3t_dev_stream_prefill_at.argtypes = [vp, i32, f32p, i32, i32]
        lib.q3t_dev_stream_kv_write.argtypes = [vp, i32, i32, i32, vp, vp]
        lib.q3t_dev_streams_begin.argtypes = [vp, ctypes.POINTER(CFrameArgs)]
        lib.q3t_dev_streams_run.argtypes = [vp, i32, vp, vp, vp]
        lib.q3t_dev_time_kernel.argtypes = [vp, i32, i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
        _lib = lib
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class DeviceError(RuntimeError):
    pass


class Device:
    """One device context (q3t_dev) on HIP device `device`."""

    def __init__(self, cfg, device=0):
        self.lib = load_library()
        self.cfg = cfg
        self._c_cfg = cfg.to_c()
        h = ctypes.c_void_p()
        rc = self.lib.q3t_dev_create(ctypes.byref(self._c_cfg), device, ctypes.byref(h))
        self.h = h
        if rc != 0:
            msg = self.error() if h else f"q3t_dev_create returned {rc} (no HIP device?)"
            self.close()
            raise DeviceError(msg)
        self._keep = []

    def error(self):
        return self.lib.q3t_dev_last_error(self.h).decode() if self.h else ""

    def _check(self, rc, what):
        if rc != 0:
            raise DeviceError(f"{what}: {self.error()}")

    def close(self):
        if getattr(self, "h", None):
            self.lib.q3t_dev_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    # -- weights
    def upload(self, name, ttype, ne, arr):
        arr = np.ascontiguousarray(arr)
        ne4 = (ctypes.c_int64 * 4)(ne[0], ne[1], 1, 1)
        self._check(self.lib.q3t_dev_upload_tensor(self.h, name.encode(), ttype, ne4, _p(arr), arr.nbytes), f"upload {name}")

    def upload_rows(self, name, ttype, ne, row0, arr):
        """rows [row0, row0 + n) of a tensor (arr: those rows, ggml layout)"""
        arr = np.ascontiguousarray(arr)
        ne4 = (ctypes.c_int64 * 4)(ne[0], ne[1], 1, 1)
        row_bytes = ne[0] * 2 if ttype == 1 else ne[0] * 4 if ttype == 0 else ne[0] // 32 * 34
        n = arr.nbytes // row_bytes
        self._check(self.lib.q3t_dev_upload_tensor_rows(self.h, name.encode(), ttype, ne4, row0, n, _p(arr),
                                                         arr.nbytes), f"upload rows of {name}")

    def upload_weights(self, weights, chunk_rows=0):
        """chunk_rows > 0: every tensor in ranges of that many rows, the last
        range first (q3t_dev_upload_tensor_rows)"""
        for name, (ttype, ne, arr) in weights.items():
            if chunk_rows <= 0 or ne[1] <= 1:
                self.upload(name, ttype, ne, arr)
                continue
            flat = np.ascontiguousarray(arr).view(np.uint8).reshape(ne[1], -1)
            starts = list(range(0, ne[1], chunk_rows))
            # the first range allocates the tensor; the others in reverse order
            for r0 in [0] + starts[1:][::-1]:
                self.upload_rows(name, ttype, ne, r0, flat[r0:r0 + chunk_rows])

    def download(self, name, nbytes):
        out = np.empty(nbytes, dtype=np.uint8)
        self._check(self.lib.q3t_dev_download_tensor(self.h, name.encode(), _p(out), nbytes), f"download {name}")
        return out

    def dequantize(self, name, n):
        out = np.empty(n, dtype=np.float32)
        self._check(self.lib.q3t_dev_dequantize(self.h, name.encode(), _p(out), n), f"dequantize {name}")
        return out

    # -- caches
    def kv_reserve(self, n_ctx):
        self._check(self.lib.q3t_dev_kv_reserve(self.h, n_ctx), "kv_reserve")

    def kv_set_type(self, ttype):
        """Talker cache element type for the next kv_reserve: 1 (F16) or 30 (BF16)."""
        self._check(self.lib.q3t_dev_kv_set_type(self.h, int(ttype)), "kv_set_type")

    def kv_write(self, layer, k, v):
        """fp16 values, or uint16 element bits as stored (bfloat16 for a BF16 cache)."""
        k = np.ascontiguousarray(k, np.uint16 if np.asarray(k).dtype == np.uint16 else np.float16)
        v = np.ascontiguousarray(v, np.uint16 if np.asarray(v).dtype == np.uint16 else np.float16)
        self._check(self.lib.q3t_dev_kv_write(self.h, layer, k.shape[0], _p(k), _p(v)), "kv_write")

    # -- forward passes
    def prefill(self, embd, n_past=0, want_hidden=True):
        embd = np.ascontiguousarray(embd, dtype=np.float32)
        n = embd.shape[0]
        hid = np.empty((n, self.cfg.hidden_size), np.float32) if want_hidden else None
        logits = np.empty(self.cfg.codec_vocab, np.float32)
        self._check(self.lib.q3t_dev_prefill(self.h, _p(embd), n, n_past, _p(hid), _p(logits)), "prefill")
        return hid, logits

    def set_attn_capture(self, layer):
        """Keep the post-softmax attention row of talker `layer` for every
        talker step from now on (-1: off); clears the kept rows."""
        self._check(self.lib.q3t_dev_set_attn_capture(self.h, int(layer)), "set_attn_capture")

    def attn_rows(self):
        """The kept rows, each [n_head, n_kv] float32."""
        rows = []
        for i in range(self.lib.q3t_dev_attn_row_count(self.h)):
            n_kv = ctypes.c_int32(0)
            self._check(self.lib.q3t_dev_attn_row(self.h, i, None, 0, ctypes.byref(n_kv)), "attn_row")
            out = np.empty((self.cfg.n_head, n_kv.value), np.float32)
            self._check(self.lib.q3t_dev_attn_row(self.h, i, _p(out), out.size, ctypes.byref(n_kv)), "attn_row")
            rows.append(out)
        return rows

    def talker_step(self, embd, n_past, want_logits=True, want_hidden=True):
        """(logits, hidden) of one talker step; an output not wanted is None
        (the C call then receives NULL for it)."""
        embd = np.ascontiguousarray(embd, dtype=np.float32)
        logits = np.empty(self.cfg.codec_vocab, np.float32) if want_logits else None
        hid = np.empty(self.cfg.hidden_size, np.float32) if want_hidden else None
        self._check(self.lib.q3t_dev_talker_step(self.h, _p(embd), n_past, _p(logits), _p(hid)), "talker_step")
        return logits, hid

    def code_pred(self, hidden, cb0, temperature=0.0, top_k=0, seed=0, frame=0):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        codes = np.empty(self.cfg.n_codebooks - 1, np.int32)
        logits = np.empty((self.cfg.n_codebooks - 1, self.cfg.cp_vocab), np.float32)
        s = CSampling(temperature, top_k, seed)
        self._check(self.lib.q3t_dev_code_pred(self.h, _p(hidden), int(cb0), ctypes.byref(s), frame, _p(codes), _p(logits)),
                    "code_pred")
        return codes, logits

    def predict_codes(self, hidden, prev_codes=None):
        """single-pass code predictor: logits [15][cp_vocab]"""
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        prev = None if prev_codes is None else np.ascontiguousarray(prev_codes, dtype=np.int32)
        logits = np.empty((self.cfg.n_codebooks - 1, self.cfg.cp_vocab), np.float32)
        self._check(self.lib.q3t_dev_predict_codes(self.h, _p(hidden), _p(prev), _p(logits)), "predict_codes")
        return logits

    def text_proj(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(tokens), self.cfg.hidden_size), np.float32)
        self._check(self.lib.q3t_dev_text_proj(self.h, _p(tokens), len(tokens), _p(out)), "text_proj")
        return out

    def text_proj_noalloc(self, tokens):
        """q3t_dev_text_proj_noalloc: the same projection with no device
        allocation (at most 64 ids; work buffers in the library's static
        device scratch)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((len(tokens), self.cfg.hidden_size), np.float32)
        self._check(self.lib.q3t_dev_text_proj_noalloc(self.h, _p(tokens), len(tokens), _p(out)), "text_proj_noalloc")
        return out

    def embed_rows(self, table, index, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        dim = self.cfg.text_embd_dim if table == 2 else self.cfg.hidden_size
        out = np.empty((len(tokens), dim), np.float32)
        self._check(self.lib.q3t_dev_embed_rows(self.h, table, index, _p(tokens), len(tokens), _p(out)), "embed_rows")
        return out

    def build_prefill(self, text, speaker=None, language_id=2050, instruct=None):
        """q3t_dev_build_prefill: (prefill [n][d], trailing [m][d], tts_pad [d])."""
        text = np.ascontiguousarray(text, dtype=np.int32)
        spk = None if speaker is None else np.ascontiguousarray(speaker, dtype=np.float32).reshape(-1)
        instr = None if instruct is None or len(instruct) == 0 else np.ascontiguousarray(instruct, dtype=np.int32)
        ni = 0 if instr is None else len(instr)
        npre, ntr = ctypes.c_int32(), ctypes.c_int32()
        args = (_p(text), len(text), _p(spk), int(language_id), _p(instr), ni)
        self._check(self.lib.q3t_dev_build_prefill(self.h, *args, None, ctypes.byref(npre), None, ctypes.byref(ntr),
                                                   None), "build_prefill")
        d = self.cfg.hidden_size
        pre = np.empty((npre.value, d), np.float32)
        trail = np.empty((ntr.value, d), np.float32)
        pad = np.empty(d, np.float32)
        self._check(self.lib.q3t_dev_build_prefill(self.h, *args, _p(pre), ctypes.byref(npre), _p(trail),
                                                   ctypes.byref(ntr), _p(pad)), "build_prefill")
        return pre, trail, pad

    def build_prefill_icl(self, text, ref_text, ref_codes, speaker=None):
        """q3t_dev_build_prefill_icl: (prefill, trailing, tts_pad); ref_codes [frames][16]."""
        text = np.ascontiguousarray(text, dtype=np.int32)
        ref_text = np.ascontiguousarray(ref_text, dtype=np.int32)
        ref_codes = np.ascontiguousarray(ref_codes, dtype=np.int32)
        spk = None if speaker is None else np.ascontiguousarray(speaker, dtype=np.float32).reshape(-1)
        npre, ntr = ctypes.c_int32(), ctypes.c_int32()
        args = (_p(text), len(text), _p(ref_text), len(ref_text), _p(ref_codes), ref_codes.shape[0], _p(spk))
        self._check(self.lib.q3t_dev_build_prefill_icl(self.h, *args, None, ctypes.byref(npre), None,
                                                       ctypes.byref(ntr), None), "build_prefill_icl")
        d = self.cfg.hidden_size
        pre = np.empty((npre.value, d), np.float32)
        trail = np.empty((ntr.value, d), np.float32)
        pad = np.empty(d, np.float32)
        self._check(self.lib.q3t_dev_build_prefill_icl(self.h, *args, _p(pre), ctypes.byref(npre), _p(trail),
                                                       ctypes.byref(ntr), _p(pad)), "build_prefill_icl")
        return pre, trail, pad

    # -- frame loop
    def frames_begin(self, trailing, tts_pad, n_past, max_len, repetition_penalty=1.05, temperature=0.0, top_k=0,
                     eos_bias=0.0, target_frames=0, seed=0):
        trailing = np.ascontiguousarray(trailing, dtype=np.float32)
        tts_pad = np.ascontiguousarray(tts_pad, dtype=np.float32)
        self._keep = [trailing, tts_pad]
        a = CFrameArgs(_p(trailing), trailing.shape[0], _p(tts_pad), n_past, max_len, repetition_penalty, eos_bias,
                       target_frames, CSampling(temperature, top_k, seed))
        self._check(self.lib.q3t_dev_frames_begin(self.h, ctypes.byref(a)), "frames_begin")

    def frames_run(self, n_frames):
        out = np.empty((max(n_frames, 1), self.cfg.n_codebooks), np.int32)
        n = ctypes.c_int32()
        eos = ctypes.c_int32()
        self._check(self.lib.q3t_dev_frames_run(self.h, n_frames, _p(out), ctypes.byref(n), ctypes.byref(eos)),
                    "frames_run")
        return out[: n.value].copy(), bool(eos.value)

    def frame_codes_ptr(self):
        """device address of the frame loop's code rows (q3t_dev_frame_codes), or None"""
        return self.lib.q3t_dev_frame_codes(self.h)

    def streams_reserve(self, n_streams, n_ctx):
        self._check(self.lib.q3t_dev_streams_reserve(self.h, n_streams, n_ctx), "streams_reserve")
        self.n_streams = n_streams

    def stream_prefill(self, stream, embd, n_past=0):
        embd = np.ascontiguousarray(embd, dtype=np.float32)
        if n_past:
            self._check(self.lib.q3t_dev_stream_prefill_at(self.h, stream, _p(embd), embd.shape[0], n_past),
                        "stream_prefill_at")
        else:
            self._check(self.lib.q3t_dev_stream_prefill(self.h, stream, _p(embd), embd.shape[0]), "stream_prefill")

    def stream_kv_write(self, stream, layer, k, v):
        """stream's counterpart of kv_write: fp16 rows [n_pos][n_kv_head][head_dim]."""
        k = np.ascontiguousarray(k, np.uint16 if np.asarray(k).dtype == np.uint16 else np.float16)
        v = np.ascontiguousarray(v, np.uint16 if np.asarray(v).dtype == np.uint16 else np.float16)
        self._check(self.lib.q3t_dev_stream_kv_write(self.h, stream, layer, k.shape[0], _p(k), _p(v)),
                    "stream_kv_write")

    def streams_begin(self, streams):
        """streams: one dict per stream with the keyword arguments of
        frames_begin (trailing, tts_pad, n_past, max_len, ...)."""
        args = (CFrameArgs * len(streams))()
        keep = []
        for b, kw in enumerate(streams):
            tr = np.ascontiguousarray(kw["trailing"], dtype=np.float32)
            pad = np.ascontiguousarray(kw["tts_pad"], dtype=np.float32)
            keep += [tr, pad]
            args[b] = CFrameArgs(_p(tr), tr.shape[0], _p(pad), kw["n_past"], kw["max_len"],
                                 kw.get("repetition_penalty", 1.05), kw.get("eos_bias", 0.0),
                                 kw.get("target_frames", 0),
                                 CSampling(kw.get("temperature", 0.0), kw.get("top_k", 0), kw.get("seed", 0)))
        self._keep = keep
        self._check(self.lib.q3t_dev_streams_begin(self.h, args), "streams_begin")

    def streams_run(self, n_frames):
        """Advances every live stream by up to n_frames frames; returns a list
        of per-stream [frames][16] code arrays and a list of EOS flags."""
        B = self.n_streams
        out = np.empty((B, max(n_frames, 1), self.cfg.n_codebooks), np.int32)
        n = np.zeros(B, np.int32)
        eos = np.zeros(B, np.int32)
        self._check(self.lib.q3t_dev_streams_run(self.h, n_frames, _p(out), _p(n), _p(eos)), "streams_run")
        return [out[b, : n[b]].copy() for b in range(B)], [bool(e) for e in eos]

    def stream_logits(self, stream):
        """stream's talker logits [codec_vocab]: the row its next codebook-0 sampler reads"""
        out = np.empty(self.cfg.codec_vocab, np.float32)
        self._check(self.lib.q3t_dev_stream_logits(self.h, int(stream), _p(out)), "stream_logits")
        return out

    def frames_stats(self):
        """(GPU microseconds of frame launches, frame launches, path) since
        frames_begin / streams_begin; path 1 = persistent frame kernel,
        0 = kernel graph, 2 = multi-stream graph."""
        us = ctypes.c_double()
        n = ctypes.c_int64()
        path = ctypes.c_int32()
        self._check(self.lib.q3t_dev_frames_stats(self.h, ctypes.byref(us), ctypes.byref(n), ctypes.byref(path)),
                    "frames_stats")
        return us.value, n.value, path.value

    def sync(self):
        self._check(self.lib.q3t_dev_sync(self.h), "sync")

    def time_kernel(self, which, iters):
        us = ctypes.c_double()
        b = ctypes.c_double()
        self._check(self.lib.q3t_dev_time_kernel(self.h, which, iters, ctypes.byref(us), ctypes.byref(b)), "time_kernel")
        return us.value, b.value
