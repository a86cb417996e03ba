"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker and the timed CPU baseline.
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def host_isa():
    """"v4" when the host CPU has the AVX-512 subsets of x86-64-v4, else "v3"."""
    need = {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("flags"):
                    return "v4" if need <= set(line.split(":", 1)[1].split()) else "v3"
    except OSError:
        pass
    return "v3"


# Q3T_ORACLE_ISA=v4 (the CPU-baseline leg, on a host with AVX-512) loads the
# x86-64-v4 build; results are the same, only the speed differs.
LIB_PATH = os.path.join(HERE, "liboracle_v4.so" if os.environ.get("Q3T_ORACLE_ISA") == "v4" else "liboracle.so")

F32, F16, Q8_0 = 0, 1, 8


class OrcConfig(ctypes.Structure):
    _fields_ = [
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


class OrcGenParams(ctypes.Structure):
    _fields_ = [
        ("max_len", ctypes.c_int32), ("language_id", ctypes.c_int32), ("repetition_penalty", ctypes.c_float),
        ("temperature", ctypes.c_float), ("top_k", ctypes.c_int32), ("eos_bias", ctypes.c_float),
        ("target_frames", ctypes.c_int32), ("rep_loop_detect", ctypes.c_int32), ("seed", ctypes.c_uint64),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle not built: {LIB_PATH} (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, u32, u64, f32 = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32,
                                       ctypes.c_uint64, ctypes.c_float)
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]; L.orc_f16_to_f32.restype = f32
        L.orc_f32_to_f16.argtypes = [f32]; L.orc_f32_to_f16.restype = ctypes.c_uint16
        L.orc_expf.argtypes = [f32]; L.orc_expf.restype = f32
        L.orc_quantize_q8_0_weights.argtypes = [vp, i64, vp]; L.orc_quantize_q8_0_weights.restype = None
        L.orc_quantize_q8_0_act.argtypes = [vp, i64, vp]; L.orc_quantize_q8_0_act.restype = None
        L.orc_dequantize_q8_0.argtypes = [vp, i64, vp]; L.orc_dequantize_q8_0.restype = None
        L.orc_gemv.argtypes = [ctypes.c_int, vp, i64, i64, vp, i64, vp, ctypes.c_int]; L.orc_gemv.restype = None
        L.orc_rmsnorm.argtypes = [vp, vp, i64, f32, vp]; L.orc_rmsnorm.restype = None
        L.orc_rope_neox.argtypes = [vp, i64, vp, vp]; L.orc_rope_neox.restype = None
        L.orc_rope_table.argtypes = [f32, i64, i64, vp, vp]; L.orc_rope_table.restype = None
        L.orc_attention.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp]; L.orc_attention.restype = None
        L.orc_attention_f32.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp]
        L.orc_attention_f32.restype = None
        L.orc_argmax.argtypes = [vp, i32]; L.orc_argmax.restype = i32
        L.orc_sample_cb0.argtypes = [vp, i32, i32, vp, f32, f32, i32, f32, i32, i32, u64]
        L.orc_sample_cb0.restype = i32
        L.orc_sample_cp.argtypes = [vp, i32, f32, i32, u64, u32, u32]; L.orc_sample_cp.restype = i32
        L.orc_philox4x32.argtypes = [u64, u32, u32, u32, u32, vp]; L.orc_philox4x32.restype = None
        L.orc_uniform.argtypes = [u64, u32, u32]; L.orc_uniform.restype = ctypes.c_double
        L.orc_create.argtypes = [ctypes.POINTER(OrcConfig)]; L.orc_create.restype = vp
        L.orc_destroy.argtypes = [vp]; L.orc_destroy.restype = None
        L.orc_set_threads.argtypes = [vp, i32]; L.orc_set_threads.restype = None
        L.orc_set_tensor.argtypes = [vp, ctypes.c_char_p, i32, vp, ctypes.c_size_t]
        L.orc_check_complete.argtypes = [vp]
        L.orc_last_error.argtypes = [vp]; L.orc_last_error.restype = ctypes.c_char_p
        L.orc_kv_reset.argtypes = [vp, i32]
        L.orc_kv_write.argtypes = [vp, i32, i32, vp, vp]
        L.orc_kv_set_type.argtypes = [vp, i32]
        L.orc_attention_typed.argtypes = [vp, vp, vp, i64, i64, i64, i64, i64, vp, vp, i32]
        L.orc_attention_typed.restype = None
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]; L.orc_bf16_to_f32.restype = f32
        L.orc_f32_to_bf16.argtypes = [f32]; L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_kv_read.argtypes = [vp, i32, i32, vp, vp]
        L.orc_prefill.argtypes = [vp, vp, i32, i32, vp, vp]
        L.orc_step.argtypes = [vp, vp, i32, vp, vp]
        L.orc_set_attn_capture.argtypes = [vp, i32]
        L.orc_attn_row_count.argtypes = [vp]; L.orc_attn_row_count.restype = i32
        L.orc_attn_row.argtypes = [vp, i32, vp, i64]; L.orc_attn_row.restype = i32
        L.orc_code_pred.argtypes = [vp, vp, i32, f32, i32, u64, u32, vp, vp]
        L.orc_predict_codes.argtypes = [vp, vp, vp, vp]
        L.orc_text_proj.argtypes = [vp, vp, i32, vp]
        L.orc_embed_row.argtypes = [vp, ctypes.c_char_p, i32, i32, vp]
        L.orc_build_prefill.argtypes = [vp, vp, i32, vp, i32, vp, i32, vp, vp, vp, ctypes.POINTER(i32)]
        L.orc_generate.argtypes = [vp, vp, i32, vp, ctypes.POINTER(OrcGenParams), vp, i32, vp, vp]
        L.orc_generate_rows.argtypes = [vp, vp, i32, vp, i32, vp, ctypes.POINTER(OrcGenParams), vp, vp]
        L.orc_frames.argtypes = [vp, vp, i32, vp, i32, vp, ctypes.POINTER(OrcGenParams), vp, vp]
        L.orc_voc_create.argtypes = [vp]; L.orc_voc_create.restype = vp
        L.orc_voc_destroy.argtypes = [vp]; L.orc_voc_destroy.restype = None
        L.orc_voc_set_threads.argtypes = [vp, i32]; L.orc_voc_set_threads.restype = None
        L.orc_voc_last_error.argtypes = [vp]; L.orc_voc_last_error.restype = ctypes.c_char_p
        L.orc_voc_set_tensor.argtypes = [vp, ctypes.c_char_p, i32, vp, ctypes.c_size_t]
        L.orc_voc_finalize.argtypes = [vp]
        L.orc_voc_samples_for_frames.argtypes = [vp, i32]; L.orc_voc_samples_for_frames.restype = i64
        L.orc_voc_decode_single.argtypes = [vp, vp, i32, i32, vp, vp]
        L.orc_voc_decode_window.argtypes = [vp, vp, i32, i32, i32, i32, vp, i64, ctypes.POINTER(i64)]
        L.orc_voc_set_record.argtypes = [vp, i32]; L.orc_voc_set_record.restype = None
        L.orc_voc_run_stage.argtypes = [vp, ctypes.c_char_p, vp, vp, i64, i64, i32, vp, i64,
                                        ctypes.POINTER(i64), ctypes.POINTER(i64)]
        L.orc_voc_stage_count.argtypes = [vp]; L.orc_voc_stage_count.restype = i32
        L.orc_voc_stage.argtypes = [vp, i32, ctypes.c_char_p, i32, vp, i64, ctypes.POINTER(i64), ctypes.POINTER(i64)]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- kernel-level helpers (numpy in, numpy out)
def f32_to_f16_bits(x):
    L = lib()
    return np.array([L.orc_f32_to_f16(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint16)


def expf(x):
    L = lib()
    return np.array([L.orc_expf(float(v)) for v in np.asarray(x, np.float32).ravel()], np.float32)


def quantize_weights(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0_weights(_p(x), x.size, _p(out))
    return out


def quantize_act(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().orc_quantize_q8_0_act(_p(x), x.size, _p(out))
    return out


def dequantize(blocks, n):
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty(n, np.float32)
    lib().orc_dequantize_q8_0(_p(blocks), n, _p(out))
    return out


def gemv(ttype, w, rows, k, x, widen=False):
    x = np.ascontiguousarray(x, np.float32).reshape(-1, k)
    w = np.ascontiguousarray(w)
    y = np.empty((x.shape[0], rows), np.float32)
    lib().orc_gemv(ttype, _p(w), rows, k, _p(x), x.shape[0], _p(y), 1 if widen else 0)
    return y


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = None if w is None else np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(w), x.size, eps, _p(y))
    return y


def rope_table(theta, head_dim, n_pos):
    c = np.empty((n_pos, head_dim // 2), np.float32)
    s = np.empty_like(c)
    lib().orc_rope_table(theta, head_dim, n_pos, _p(c), _p(s))
    return c, s


def rope(x, cos_row, sin_row):
    x = np.ascontiguousarray(x, np.float32).copy()
    lib().orc_rope_neox(_p(x), x.size, _p(np.ascontiguousarray(cos_row, np.float32)),
                        _p(np.ascontiguousarray(sin_row, np.float32)))
    return x


def attention(q, k, v, n_kv):
    """q [n_head][hd] f32; k, v fp16 [n_kv_head][n_ctx][hd]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float16)
    v = np.ascontiguousarray(v, np.float16)
    nh, hd = q.shape
    nkv, nctx, _ = k.shape
    out = np.empty((nh, hd), np.float32)
    probs = np.empty((nh, n_kv), np.float32)
    lib().orc_attention(_p(q), _p(k), _p(v), nh, nkv, hd, nctx, n_kv, _p(out), _p(probs))
    return out, probs


def attention_bf16(q, k, v, n_kv):
    """attention() over a bfloat16 cache: k, v uint16 bfloat16 bits
    [n_kv_head][n_ctx][hd]."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    nh, hd = q.shape
    nkv, nctx, _ = k.shape
    out = np.empty((nh, hd), np.float32)
    probs = np.empty((nh, n_kv), np.float32)
    lib().orc_attention_typed(_p(q), _p(k), _p(v), nh, nkv, hd, nctx, n_kv, _p(out), _p(probs), 1)
    return out, probs


def attention_f32(q, k, v):
    """The code predictor's prefill attention: q [n_head][hd], k and v
    [n_kv][n_kv_head][hd], all f32; causal, query i sees rows 0..i when q has
    one row per position ([n_kv][n_head][hd]), or all n_kv rows for one query."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    n_kv, nkv, hd = k.shape
    nh = q.shape[-2]
    out = np.empty(q.shape, np.float32)
    if q.ndim == 2:
        lib().orc_attention_f32(_p(q), _p(k), _p(v), nkv * hd, nh, nkv, hd, n_kv, _p(out))
    else:
        for i in range(q.shape[0]):
            qi = np.ascontiguousarray(q[i])
            oi = np.empty_like(qi)
            lib().orc_attention_f32(_p(qi), _p(k), _p(v), nkv * hd, nh, nkv, hd, i + 1, _p(oi))
            out[i] = oi
    return out


def argmax(x):
    x = np.ascontiguousarray(x, np.float32)
    return lib().orc_argmax(_p(x), x.size)


def sample_cb0(logits, eos_id, seen=None, rep=1.05, temp=0.0, top_k=0, eos_bias=0.0, target_frames=0, frame=0, seed=0):
    l = np.ascontiguousarray(logits, np.float32).copy()
    s = None if seen is None else np.ascontiguousarray(seen, np.uint8)
    tok = lib().orc_sample_cb0(_p(l), l.size, eos_id, _p(s), rep, temp, top_k, eos_bias, target_frames, frame, seed)
    return tok, l


def sample_cp(logits, temp=0.0, top_k=0, seed=0, frame=0, group=1):
    l = np.ascontiguousarray(logits, np.float32).copy()
    return lib().orc_sample_cp(_p(l), l.size, temp, top_k, seed, frame, group)


def philox(key, c0, c1, c2, c3):
    out = np.empty(4, np.uint32)
    lib().orc_philox4x32(key, c0, c1, c2, c3, _p(out))
    return out


def uniform(seed, frame, group):
    return lib().orc_uniform(seed, frame, group)


class Oracle:
    """Model-level CPU restatement; borrows the weight arrays of `weights`."""

    def __init__(self, cfg, weights, threads=4):
        self.L = lib()
        self.cfg = cfg
        self._cc = cfg.to_c(OrcConfig)
        self.h = self.L.orc_create(ctypes.byref(self._cc))
        self.weights = weights            # keep the buffers alive
        for name, (ttype, ne, arr) in weights.items():
            self.L.orc_set_tensor(self.h, name.encode(), ttype, _p(arr), arr.nbytes)
        if self.L.orc_check_complete(self.h) != 0:
            raise RuntimeError(self.error())
        self.L.orc_set_threads(self.h, threads)

    def error(self):
        return self.L.orc_last_error(self.h).decode()

    def close(self):
        if getattr(self, "h", None):
            self.L.orc_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def set_threads(self, n):
        self.L.orc_set_threads(self.h, n)

    def _chk(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.error()}")

    def kv_reset(self, n_ctx):
        self._chk(self.L.orc_kv_reset(self.h, n_ctx), "kv_reset")

    def kv_set_type(self, ttype):
        """Talker cache element type: 1 (F16) or 30 (BF16)."""
        self._chk(self.L.orc_kv_set_type(self.h, int(ttype)), "kv_set_type")

    def kv_write(self, layer, k, v):
        """Rows [n_pos][n_kv_head][head_dim] into positions [0, n_pos): fp16
        values, or uint16 element bits as stored (bfloat16 for a BF16 cache)."""
        k = np.ascontiguousarray(k, np.uint16 if np.asarray(k).dtype == np.uint16 else np.float16)
        v = np.ascontiguousarray(v, np.uint16 if np.asarray(v).dtype == np.uint16 else np.float16)
        self._chk(self.L.orc_kv_write(self.h, layer, k.shape[0], _p(k), _p(v)), "kv_write")

    def kv_read(self, layer, n_pos):
        shape = (n_pos, self.cfg.n_kv_head, self.cfg.head_dim)
        k, v = np.empty(shape, np.float16), np.empty(shape, np.float16)
        self._chk(self.L.orc_kv_read(self.h, layer, n_pos, _p(k), _p(v)), "kv_read")
        return k, v

    def prefill(self, embd, n_past=0):
        embd = np.ascontiguousarray(embd, np.float32)
        n = embd.shape[0]
        hid = np.empty((n, self.cfg.hidden_size), np.float32)
        logits = np.empty(self.cfg.codec_vocab, np.float32)
        self._chk(self.L.orc_prefill(self.h, _p(embd), n, n_past, _p(hid), _p(logits)), "prefill")
        return hid, logits

    def set_attn_capture(self, layer):
        self._chk(self.L.orc_set_attn_capture(self.h, int(layer)), "set_attn_capture")

    def attn_rows(self):
        rows = []
        for i in range(self.L.orc_attn_row_count(self.h)):
            n_kv = self.L.orc_attn_row(self.h, i, None, 0)
            out = np.empty((self.cfg.n_head, n_kv), np.float32)
            self.L.orc_attn_row(self.h, i, _p(out), out.size)
            rows.append(out)
        return rows

    def step(self, embd, n_past):
        embd = np.ascontiguousarray(embd, np.float32)
        logits = np.empty(self.cfg.codec_vocab, np.float32)
        hid = np.empty(self.cfg.hidden_size, np.float32)
        self._chk(self.L.orc_step(self.h, _p(embd), n_past, _p(logits), _p(hid)), "step")
        return logits, hid

    def code_pred(self, hidden, cb0, temperature=0.0, top_k=0, seed=0, frame=0):
        hidden = np.ascontiguousarray(hidden, np.float32)
        codes = np.empty(self.cfg.n_codebooks - 1, np.int32)
        logits = np.empty((self.cfg.n_codebooks - 1, self.cfg.cp_vocab), np.float32)
        self._chk(self.L.orc_code_pred(self.h, _p(hidden), int(cb0), temperature, top_k, seed, frame, _p(codes), _p(logits)),
                  "code_pred")
        return codes, logits

    def predict_codes(self, hidden, prev_codes=None):
        """single-pass code predictor: logits [15][cp_vocab]"""
        hidden = np.ascontiguousarray(hidden, np.float32)
        prev = None if prev_codes is None else np.ascontiguousarray(prev_codes, np.int32)
        logits = np.empty((self.cfg.n_codebooks - 1, self.cfg.cp_vocab), np.float32)
        self._chk(self.L.orc_predict_codes(self.h, _p(hidden), None if prev is None else _p(prev), _p(logits)),
                  "predict_codes")
        return logits

    def text_proj(self, tokens):
        tokens = np.ascontiguousarray(tokens, np.int32)
        out = np.empty((len(tokens), self.cfg.hidden_size), np.float32)
        self._chk(self.L.orc_text_proj(self.h, _p(tokens), len(tokens), _p(out)), "text_proj")
        return out

    def embed_row(self, table, index, token):
        dim = self.cfg.text_embd_dim if table == "text" else self.cfg.hidden_size
        out = np.empty(dim, np.float32)
        self._chk(self.L.orc_embed_row(self.h, table.encode(), index, token, _p(out)), "embed_row")
        return out

    def build_prefill(self, text, speaker=None, language_id=2050, instruct=None):
        text = np.ascontiguousarray(text, np.int32)
        ni = 0 if instruct is None else len(instruct)
        instr = None if instruct is None else np.ascontiguousarray(instruct, np.int32)
        d = self.cfg.hidden_size
        pre = np.empty((ni + 10, d), np.float32)
        trail = np.empty((max(0, len(text) - 9) + 1, d), np.float32)
        pad = np.empty(d, np.float32)
        tl = ctypes.c_int32()
        spk = None if speaker is None else np.ascontiguousarray(speaker, np.float32)
        n = self.L.orc_build_prefill(self.h, _p(text), len(text), _p(spk), language_id, _p(instr), ni, _p(pre),
                                     _p(trail), _p(pad), ctypes.byref(tl))
        if n < 0:
            raise RuntimeError(self.error())
        return pre[:n], trail[: tl.value], pad

    def generate(self, text, speaker=None, max_len=64, language_id=2050, repetition_penalty=1.05, temperature=0.0,
                 top_k=0, eos_bias=0.0, target_frames=0, rep_loop_detect=False, seed=0, instruct=None):
        text = np.ascontiguousarray(text, np.int32)
        spk = None if speaker is None else np.ascontiguousarray(speaker, np.float32)
        ni = 0 if instruct is None else len(instruct)
        instr = None if instruct is None else np.ascontiguousarray(instruct, np.int32)
        p = OrcGenParams(max_len, language_id, repetition_penalty, temperature, top_k, eos_bias, target_frames,
                         1 if rep_loop_detect else 0, seed)
        codes = np.empty((max(max_len, 1), self.cfg.n_codebooks), np.int32)
        first = np.empty(self.cfg.codec_vocab, np.float32)
        n = self.L.orc_generate(self.h, _p(text), len(text), _p(spk), ctypes.byref(p), _p(instr), ni, _p(codes), _p(first))
        if n < 0:
            raise RuntimeError(self.error())
        return codes[:n].copy(), first

    def generate_rows(self, prefill, trailing, pad, max_len=64, repetition_penalty=1.05, temperature=0.0, top_k=0,
                      eos_bias=0.0, target_frames=0, rep_loop_detect=False, seed=0):
        prefill = np.ascontiguousarray(prefill, np.float32)
        trailing = np.ascontiguousarray(trailing, np.float32).reshape(-1, self.cfg.hidden_size)
        pad = np.ascontiguousarray(pad, np.float32)
        p = OrcGenParams(max_len, 0, repetition_penalty, temperature, top_k, eos_bias, target_frames,
                         1 if rep_loop_detect else 0, seed)
        codes = np.empty((max(max_len, 1), self.cfg.n_codebooks), np.int32)
        n = self.L.orc_generate_rows(self.h, _p(prefill), prefill.shape[0], _p(trailing), trailing.shape[0], _p(pad),
                                     ctypes.byref(p), _p(codes), None)
        if n < 0:
            raise RuntimeError(self.error())
        return codes[:n].copy()

    def frames(self, first_logits, n_past, trailing, pad, max_len, repetition_penalty=1.05, temperature=0.0,
               top_k=0, eos_bias=0.0, target_frames=0, seed=0, want_logits=False):
        """The frame loop from the current cache (the device's frames_begin +
        frames_run after a prefill or step).  want_logits: also return the
        talker logits each frame's codebook-0 sampler started from
        ([frames sampled][codec_vocab], the frame that drew EOS included)."""
        first_logits = np.ascontiguousarray(first_logits, np.float32)
        trailing = np.ascontiguousarray(trailing, np.float32).reshape(-1, self.cfg.hidden_size)
        pad = np.ascontiguousarray(pad, np.float32)
        p = OrcGenParams(max_len, 0, repetition_penalty, temperature, top_k, eos_bias, target_frames, 0, seed)
        codes = np.empty((max(max_len, 1), self.cfg.n_codebooks), np.int32)
        lg = np.full((max(max_len, 1), self.cfg.codec_vocab), np.nan, np.float32) if want_logits else None
        n = self.L.orc_frames(self.h, _p(first_logits), n_past, _p(trailing), trailing.shape[0], _p(pad),
                              ctypes.byref(p), _p(codes), _p(lg))
        if n < 0:
            raise RuntimeError(self.error())
        if not want_logits:
            return codes[:n].copy()
        n_lg = int(np.sum(~np.isnan(lg[:, 0])))
        return codes[:n].copy(), lg[:n_lg].copy()


class VocOracle:
    """CPU restatement of the audio-tokenizer decoder (q3t_vocoder.cpp);
    borrows the arrays of `weights` (qwen3_tts_amd.vocoder.VocWeights)."""

    def __init__(self, cfg, weights, threads=8):
        self.L = lib()
        self.cfg = cfg
        self._cc = cfg.to_c()
        self.h = self.L.orc_voc_create(ctypes.byref(self._cc))
        self.weights = weights
        for name, (ttype, ne, arr) in weights.items():
            self.L.orc_voc_set_tensor(self.h, name.encode(), ttype, _p(arr), arr.nbytes)
        if self.L.orc_voc_finalize(self.h) != 0:
            raise RuntimeError(self.error())
        self.L.orc_voc_set_threads(self.h, threads)

    def error(self):
        return self.L.orc_voc_last_error(self.h).decode()

    def close(self):
        if self.h:
            self.L.orc_voc_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def samples_for_frames(self, n):
        return int(self.L.orc_voc_samples_for_frames(self.h, n))

    def decode_single(self, codes, pos0=0, want_latent=False):
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        n = codes.shape[0]
        out = np.zeros(self.samples_for_frames(n), np.float32)
        lat = np.zeros((n, self.cfg.hidden), np.float32) if want_latent else None
        if self.L.orc_voc_decode_single(self.h, _p(codes), n, pos0, _p(out), _p(lat)) != 0:
            raise RuntimeError(self.error())
        return (out, lat) if want_latent else out

    def stages(self, codes, pos0=0):
        """{name: [T][C] fp32} of every stage of decode_single(codes, pos0)."""
        self.L.orc_voc_set_record(self.h, 1)
        try:
            self.decode_single(codes, pos0)
            out = {}
            for i in range(self.L.orc_voc_stage_count(self.h)):
                T, C = ctypes.c_int64(0), ctypes.c_int64(0)
                name = ctypes.create_string_buffer(64)
                self.L.orc_voc_stage(self.h, i, name, 64, None, 0, ctypes.byref(T), ctypes.byref(C))
                a = np.zeros((T.value, C.value), np.float32)
                self.L.orc_voc_stage(self.h, i, name, 64, _p(a), a.size, ctypes.byref(T), ctypes.byref(C))
                out[name.value.decode()] = a
            return out
        finally:
            self.L.orc_voc_set_record(self.h, 0)

    def run_stage(self, name, x, pos0=0):
        """one stage from fp32 rows x [T][C] (codes [T][16] for "latent")."""
        T = x.shape[0]
        if name == "latent":
            codes = np.ascontiguousarray(x, dtype=np.int32)
            xin, C = None, 16
        else:
            codes, xin = None, np.ascontiguousarray(x, dtype=np.float32)
            C = xin.shape[1]
        c = self.cfg
        cap = max(T, self.samples_for_frames(1)) * 8 * max(c.latent, c.cnx_ffn, c.decoder_dim, 16) + 64
        out = np.zeros(cap, np.float32)
        To, Co = ctypes.c_int64(0), ctypes.c_int64(0)
        if self.L.orc_voc_run_stage(self.h, name.encode(), _p(xin), _p(codes), T, C, pos0, _p(out), cap,
                                    ctypes.byref(To), ctypes.byref(Co)) != 0:
            raise RuntimeError(self.error())
        return out[:To.value * Co.value].reshape(To.value, Co.value).copy()

    def decode_window(self, codes, start, end, context):
        codes = np.ascontiguousarray(codes, dtype=np.int32)
        cap = self.samples_for_frames(end - max(0, start - max(0, context)))
        out = np.zeros(max(cap, 1), np.float32)
        n = ctypes.c_int64(0)
        if self.L.orc_voc_decode_window(self.h, _p(codes), codes.shape[0], start, end, context, _p(out), cap,
                                        ctypes.byref(n)) != 0:
            raise RuntimeError(self.error())
        return out[:n.value].copy()
