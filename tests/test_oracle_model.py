"""Pins the oracle's model-level composition (orc_step, orc_prefill,
orc_code_pred, orc_text_proj, and the frame loop orc_frames /
orc_generate_rows) against an independent float64 numpy forward written op by
op from the reference graphs:

  build_step_graph               src/tts_transformer.cpp:1652-1751
  build_prefill_forward_graph    src/tts_transformer.cpp:1474-1617
  build_code_pred_prefill_graph  src/tts_transformer.cpp:1929-2044
  build_code_pred_step_graph     src/tts_transformer.cpp:2055-2215
  project_text_tokens            src/tts_transformer.cpp:963-1028
  generate() frame loop          src/tts_transformer.cpp:3108-3309

The numpy forward keeps ggml's type rules only where they round: an F16 src0
in ggml_mul_mat rounds its src1 to fp16, a Q8_0 src0 quantises it per
32-block, the F16 cache holds fp16 K/V rows and attention over it rounds q and
P to fp16.  Everything else (RMSNorm, RoPE from float64 angles, softmax, SiLU,
residuals) is float64.  Agreement is asserted within a tolerance, and each
test also shows that the same forward with one planted mistake (gate and up
swapped, QK-norm after RoPE, a head index off by one, the text-projection bias
after the SiLU, the code predictor's prefill attending over the fp16 cache)
misses the oracle by far more than that tolerance.  Closed forms add what a
tolerance cannot: zeroed output projections make every layer the identity.
"""
import dataclasses

import numpy as np
import pytest

import q3t_oracle as orc
from qwen3_tts_amd import config as qcfg
from qwen3_tts_amd.synth import F16, F32, Q8_0, Weights, dequantize_q8_0


def f16r(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def q8_act(x):
    """ggml-cpu x86 quantize_row_q8_0 restated (d = fp16(amax/127),
    q = rint(x * (127/amax)) in fp32), returned dequantised as d*q."""
    xf = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(xf).max(axis=1, keepdims=True)
    d = (amax / np.float32(127)).astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore"):
        idv = np.where(amax > 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    q = np.rint(xf * idv).astype(np.float64)
    return (d * q).reshape(-1)


class _Tensors:
    def __init__(self, d):
        self.tensors = d

    def items(self):
        return self.tensors.items()

    def __getitem__(self, k):
        return self.tensors[k]


class NpRef:
    """float64 numpy forward of the talker and code predictor.

    mistakes: a set of planted deviations used to show the comparison is
    sensitive: "swap_gate_up", "qknorm_after_rope", "head_off_by_one",
    "bias_after_silu", "cp_prefill_f16"."""

    def __init__(self, cfg, w, mistakes=()):
        self.cfg, self.w, self.mistakes = cfg, w, set(mistakes)
        self.cache = {}
        self.kv = {}
        self.capture = None      # (talker layer prefix, list): post-softmax rows [n_head][n_kv] of single-row calls

    # -- tensors
    def mat(self, name):
        if name not in self.cache:
            ttype, (ne0, ne1), a = self.w[name]
            x = dequantize_q8_0(a).astype(np.float64) if ttype == Q8_0 else a.astype(np.float64)
            self.cache[name] = (ttype, x.reshape(ne1, ne0))
        return self.cache[name]

    def vec(self, name):
        return self.mat(name)[1].reshape(-1)

    def mm(self, name, x, widen=False):
        """ggml_mul_mat(W, x) for one activation row x."""
        ttype, W = self.mat(name)
        x = np.asarray(x, np.float64)
        if ttype == F16 and not widen:
            x = f16r(x)
        elif ttype == Q8_0:
            x = q8_act(x)
        else:
            x = x.astype(np.float32).astype(np.float64)
        return W @ x

    def rms(self, x, w):
        x = np.asarray(x, np.float64)
        return x / np.sqrt(np.mean(x * x) + self.cfg.rms_eps) * w

    def rope(self, x, pos, theta):
        hd = x.shape[-1]
        half = hd // 2
        ang = pos * theta ** (-2.0 * np.arange(half) / hd)
        c, s = np.cos(ang), np.sin(ang)
        x0, x1 = x[..., :half], x[..., half:]
        return np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)

    @staticmethod
    def silu(x):
        return x / (1.0 + np.exp(-x))

    # -- one layer over the rows x [n][d] at positions pos0.. ; `cache`
    # is the layer's list of (k, v) fp16 rows by position
    def layer(self, prefix, x, pos0, cache, theta, f32_prefill):
        c = self.cfg
        nh, nkv, hd = c.n_head, c.n_kv_head, c.head_dim
        n = x.shape[0]
        qn, kn = self.vec(prefix + "attn_q_norm.weight"), self.vec(prefix + "attn_k_norm.weight")
        out = np.empty((n, nh * hd))
        rows = []
        for i in range(n):
            h = self.rms(x[i], self.vec(prefix + "attn_norm.weight"))
            q = self.mm(prefix + "attn_q.weight", h).reshape(nh, hd)
            k = self.mm(prefix + "attn_k.weight", h).reshape(nkv, hd)
            v = self.mm(prefix + "attn_v.weight", h).reshape(nkv, hd)
            pos = pos0 + i
            if "qknorm_after_rope" in self.mistakes:
                q = np.stack([self.rms(r, qn) for r in self.rope(q, pos, theta)])
                k = np.stack([self.rms(r, kn) for r in self.rope(k, pos, theta)])
            else:
                q = self.rope(np.stack([self.rms(r, qn) for r in q]), pos, theta)
                k = self.rope(np.stack([self.rms(r, kn) for r in k]), pos, theta)
            cache[pos] = (f16r(k), f16r(v))
            rows.append((q, k, v))
        for i in range(n):
            q = rows[i][0]
            pos = pos0 + i
            f32 = f32_prefill and "cp_prefill_f16" not in self.mistakes
            if f32:
                K = np.stack([rows[j][1] for j in range(i + 1)])      # [n_kv][nkv][hd] unrounded
                V = np.stack([rows[j][2] for j in range(i + 1)])
            else:
                K = np.stack([cache[j][0] for j in range(pos + 1)])
                V = np.stack([cache[j][1] for j in range(pos + 1)])
            for hh in range(nh):
                g = hh // (nh // nkv)
                qh = q[hh] if f32 else f16r(q[hh])
                s = K[:, g] @ qh / np.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                if self.capture is not None and n == 1 and prefix == self.capture[0]:
                    if hh == 0:
                        self.capture[1].append(np.empty((nh, pos + 1)))
                    self.capture[1][-1][hh] = f16r(p) if "attn_row_f16" in self.mistakes else p
                if not f32:
                    p = f16r(p)
                out[i, hh * hd:(hh + 1) * hd] = p @ V[:, g]
        y = np.empty_like(x)
        for i in range(n):
            a = self.mm(prefix + "attn_output.weight", out[i]) + x[i]
            h = self.rms(a, self.vec(prefix + "ffn_norm.weight"))
            gate = self.mm(prefix + "ffn_gate.weight", h)
            up = self.mm(prefix + "ffn_up.weight", h)
            if "swap_gate_up" in self.mistakes:
                gate, up = up, gate
            f = self.silu(gate) * up
            y[i] = self.mm(prefix + "ffn_down.weight", f, widen=True) + a
        return y

    # -- talker
    def kv_reset(self):
        self.kv = {il: {} for il in range(self.cfg.n_layers)}

    def talker(self, embd, pos0):
        """rows embd [n][d] at positions pos0..: (normed hidden [n][d], last-row logits).
        The last row before the output norm is kept in self.last_x."""
        c = self.cfg
        x = np.asarray(embd, np.float64).reshape(-1, c.hidden_size)
        for il in range(c.n_layers):
            x = self.layer(f"talker.blk.{il}.", x, pos0, self.kv[il], c.rope_theta, False)
        self.last_x = x[-1].copy()
        hid = np.stack([self.rms(r, self.vec("talker.output_norm.weight")) for r in x])
        return hid, self.mm("talker.codec_head.weight", hid[-1])

    # -- the generate() frame loop, greedy (src/tts_transformer.cpp:3108-3309)
    def cb0_greedy(self, logits, seen, frame, rep, eos_bias, target_frames):
        """Codebook-0 choice of one frame (:3109-3145, :3177-3184): the top
        1024 codec ids are suppressed except EOS; every distinct earlier token
        gets the HF penalty (positive logits divided, others multiplied); the
        EOS bias grows by 0.1 per frame past target_frames, capped at 6; the
        first maximum wins."""
        c = self.cfg
        l = np.asarray(logits, np.float64).copy()
        ids = np.arange(c.codec_vocab)
        l[(ids >= c.codec_vocab - 1024) & (ids != c.codec_eos_id)] = -np.inf
        penalised = list(seen)
        if "penalty_per_occurrence" in self.mistakes:
            penalised = self.cb0_history
        eff = eos_bias
        if target_frames > 0 and frame > target_frames:
            slope = 0.2 if "ramp_slope" in self.mistakes else 0.1
            eff = min(eff + slope * (frame - target_frames), 6.0)
        if "penalty_after_bias" in self.mistakes:
            l[c.codec_eos_id] += eff
        for t in penalised:
            if "penalty_sign" in self.mistakes:
                l[t] = l[t] * rep if l[t] > 0 else l[t] / rep
            else:
                l[t] = l[t] / rep if l[t] > 0 else l[t] * rep
        if "penalty_after_bias" not in self.mistakes:
            l[c.codec_eos_id] += eff
        return int(np.argmax(l))

    def generate(self, prefill, trailing, pad, max_len, rep=1.05, eos_bias=0.0, target_frames=0):
        """Greedy frames from prefill rows [n][d], trailing rows [t][d] and
        the tts_pad row: (codes [frames][16], the talker logits each frame's
        sampler started from).  Per frame: codebook 0 from the talker logits;
        the code predictor on the talker's normed hidden row; the next step
        embedding codec_embd[c0] + sum_g code_pred.codec_embd[g-1][c_g] +
        (trailing[frame] if frame < len(trailing) else pad); one talker step."""
        c = self.cfg
        self.kv_reset()
        hid, lg = self.talker(prefill, 0)
        n_past = len(prefill)
        codec = self.mat("talker.codec_embd.weight")[1]
        cpe = [self.mat(f"code_pred.codec_embd.{g}.weight")[1] for g in range(c.n_codebooks - 1)]
        seen, self.cb0_history = set(), []
        codes, logs = [], []
        for frame in range(max_len):
            logs.append(lg)
            tok = self.cb0_greedy(lg, seen, frame, rep, eos_bias, target_frames)
            if tok == c.codec_eos_id:
                break
            seen.add(tok)
            self.cb0_history.append(tok)
            cp_in = self.last_x if "cp_unnormed" in self.mistakes else hid[-1]
            rest, _ = self.code_pred(cp_in, tok)
            fc = [tok] + [int(v) for v in rest]
            codes.append(fc)
            if frame + 1 >= max_len:
                break
            e = codec[fc[0]].copy()
            for g in range(1, c.n_codebooks):
                table = min(g, c.n_codebooks - 2) if "cp_embd_g" in self.mistakes else g - 1
                e = e + cpe[table][fc[g]]
            ti = frame + 1 if "trailing_next" in self.mistakes else frame
            e = e + (trailing[ti] if ti < len(trailing) else pad)
            hid, lg = self.talker(e[None], n_past)
            n_past += 1
        return np.array(codes, np.int32).reshape(-1, c.n_codebooks), np.stack(logs)

    # -- code predictor, greedy
    def code_pred(self, hidden, cb0):
        c = self.cfg
        cache = {il: {} for il in range(c.cp_layers)}
        codec = self.mat("talker.codec_embd.weight")[1]
        x = np.stack([np.asarray(hidden, np.float64), codec[cb0]])
        codes, logits = [], []
        for step in range(c.n_codebooks - 1):
            pos0 = 0 if step == 0 else step + 1
            for il in range(c.cp_layers):
                x = self.layer(f"code_pred.blk.{il}.", x, pos0, cache[il], c.cp_rope_theta, step == 0)
            h = self.rms(x[-1], self.vec("code_pred.output_norm.weight"))
            head = step + 1 if "head_off_by_one" in self.mistakes and step + 1 < c.n_codebooks - 1 else step
            lg = self.mm(f"code_pred.lm_head.{head}.weight", h)
            logits.append(lg)
            codes.append(int(np.argmax(lg)))
            x = self.mat(f"code_pred.codec_embd.{step}.weight")[1][codes[-1]][None] if step + 1 < c.n_codebooks - 1 \
                else None
        return np.array(codes), np.stack(logits)

    # -- the single-pass code predictor (build_code_pred_graph,
    # src/tts_transformer.cpp:1771-1899), written out as the graph does it:
    # Q and K with their norms, a softmax over the one score, P times V
    def predict_codes(self, hidden, prev=None):
        c = self.cfg
        nh, nkv, hd = c.n_head, c.n_kv_head, c.head_dim
        x = np.asarray(hidden, np.float64)
        if prev is not None:
            n = c.n_codebooks - 2 if "single_drop_last" in self.mistakes else c.n_codebooks - 1
            for g in range(n):
                x = x + self.mat(f"code_pred.codec_embd.{g}.weight")[1][prev[g]]
        if c.cp_hidden != c.hidden_size:
            x = self.mm("code_pred.mtp_proj.weight", x) + self.vec("code_pred.mtp_proj.bias")
        for il in range(c.cp_layers):
            p = f"code_pred.blk.{il}."
            h = self.rms(x, self.vec(p + "attn_norm.weight"))
            q = self.mm(p + "attn_q.weight", h).reshape(nh, hd)
            k = self.mm(p + "attn_k.weight", h).reshape(nkv, hd)
            v = self.mm(p + "attn_v.weight", h).reshape(nkv, hd)
            q = np.stack([self.rms(r, self.vec(p + "attn_q_norm.weight")) for r in q])
            k = np.stack([self.rms(r, self.vec(p + "attn_k_norm.weight")) for r in k])
            out = np.empty(nh * hd)
            for hh in range(nh):
                g = hh % nkv if "single_gqa_mod" in self.mistakes else hh // (nh // nkv)
                s = np.array([k[g] @ q[hh] / np.sqrt(hd)])
                pr = np.exp(s - s.max())
                pr /= pr.sum()
                out[hh * hd:(hh + 1) * hd] = pr[0] * v[g]
            a = self.mm(p + "attn_output.weight", out) + x
            h = self.rms(a, self.vec(p + "ffn_norm.weight"))
            f = self.silu(self.mm(p + "ffn_gate.weight", h)) * self.mm(p + "ffn_up.weight", h)
            x = self.mm(p + "ffn_down.weight", f, widen=True) + a
        if "single_out_norm" in self.mistakes:
            x = self.rms(x, self.vec("code_pred.output_norm.weight"))
        return np.stack([self.mm(f"code_pred.lm_head.{g}.weight", x) for g in range(c.n_codebooks - 1)])

    def text_proj(self, tokens):
        te = self.mat("talker.text_embd.weight")[1]
        b1, b2 = self.vec("talker.text_proj.fc1.bias"), self.vec("talker.text_proj.fc2.bias")
        out = []
        for t in tokens:
            h = self.mm("talker.text_proj.fc1.weight", te[t])
            h = self.silu(h) + b1 if "bias_after_silu" in self.mistakes else self.silu(h + b1)
            out.append(self.mm("talker.text_proj.fc2.weight", h) + b2)
        return np.stack(out)


def rel_err(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def small_cfg():
    # one talker layer and one code-predictor layer at the tiny widths keep the
    # float64 forward fast; four query heads over two KV heads keep GQA
    return qcfg.tiny(n_layers=1, cp_layers=1)


# The two forwards differ only by fp32-vs-fp64 rounding (~5e-8 relative),
# except where a value lands within that distance of an fp16 (or Q8_0
# activation) rounding boundary and rounds the other way: then a row moves by
# up to ~5e-4 (F16) or a few 1e-3 (Q8_0).  Such flips are rare, so the median
# error over a run must sit at the fp32 noise level and the worst one within a
# flip; every planted mistake moves the median by 1e-3 or more.
NOISE = 1e-6
FLIP = {"f16": 2e-3, "q8_0": 1e-2}


def assert_agrees(errs, wt):
    errs = np.asarray(errs, np.float64)
    assert np.median(errs) < NOISE and errs.max() < FLIP[wt], errs


def assert_misses(errs):
    errs = np.asarray(errs, np.float64)
    assert np.median(errs) > 100 * NOISE, errs


@pytest.fixture(scope="module", params=["f16", "q8_0"])
def model(request):
    cfg = small_cfg()
    w = Weights(cfg, request.param, seed=31)
    return request.param, cfg, w, orc.Oracle(cfg, w, threads=4)


def _talker_run(ref, o, cfg, embd):
    o.kv_reset(32)
    ref.kv_reset()
    hid_o, lg_o = o.prefill(embd[:5], 0)
    hid_r, lg_r = ref.talker(embd[:5], 0)
    steps = []
    for i in range(5, embd.shape[0]):
        lo, ho = o.step(embd[i], i)
        hr, lr = ref.talker(embd[i:i + 1], i)
        steps.append((lo, ho, lr, hr[0]))
    return (hid_o, lg_o, hid_r, lg_r), steps


def test_talker_prefill_and_steps_match_numpy_forward(model):
    wt, cfg, w, o = model
    embd = (np.random.default_rng(41).standard_normal((8, cfg.hidden_size)) * 0.5).astype(np.float32)
    (hid_o, lg_o, hid_r, lg_r), steps = _talker_run(NpRef(cfg, w), o, cfg, embd)
    assert_agrees([rel_err(hid_o[i], hid_r[i]) for i in range(5)] + [rel_err(lg_o, lg_r)], wt)
    assert_agrees([e for lo, ho, lr, hr in steps for e in (rel_err(ho, hr), rel_err(lo, lr))], wt)
    for mistake in ("swap_gate_up", "qknorm_after_rope"):
        (_, lg_o2, _, lg_m), steps_m = _talker_run(NpRef(cfg, w, {mistake}), o, cfg, embd)
        assert_misses([rel_err(lg_o2, lg_m)] + [rel_err(s[0], s[2]) for s in steps_m])


def test_code_pred_matches_numpy_forward(model):
    """The 2-token prefill over F32 K/V plus 14 steps over the fp16 cache;
    each step's logits come from its own head."""
    wt, cfg, w, o = model
    rng = np.random.default_rng(42)
    errs, miss = [], []
    for cb0 in (5, 1777, 300):
        hid = rng.standard_normal(cfg.hidden_size).astype(np.float32)
        codes_o, lg_o = o.code_pred(hid, cb0)
        codes_r, lg_r = NpRef(cfg, w).code_pred(hid, cb0)
        # the two forwards see the same inputs while their codes agree
        n_same = int(np.argmax(codes_o != codes_r)) if np.any(codes_o != codes_r) else len(codes_o)
        assert n_same >= 1
        errs += [rel_err(lg_o[s], lg_r[s]) for s in range(n_same)]
        _, lg_m = NpRef(cfg, w, {"head_off_by_one"}).code_pred(hid, cb0)
        miss.append(rel_err(lg_o[0], lg_m[0]))
    assert len(errs) >= 30
    assert_agrees(errs, wt)
    assert_misses(miss)


def test_code_pred_prefill_attends_over_f32_rows():
    """The prefill's head-0 logits follow the F32 attention of
    src/tts_transformer.cpp:1999-2012; attending over the fp16 cache with
    fp16 q and P instead (the form this oracle had before) misses them.
    F16 weights, so only the attention's rounding separates the forms; the
    attention's values are scaled up so its rounding matters at the logits."""
    cfg = small_cfg()
    w = Weights(cfg, "f16", seed=33, std=0.2)
    o = orc.Oracle(cfg, w, threads=4)
    rng = np.random.default_rng(43)
    good, bad = [], []
    for cb0 in (7, 100, 901, 2047, 3000, 11, 12, 13):
        hid = rng.standard_normal(cfg.hidden_size).astype(np.float32)
        _, lg_o = o.code_pred(hid, cb0)
        _, lg_r = NpRef(cfg, w).code_pred(hid, cb0)
        _, lg_m = NpRef(cfg, w, {"cp_prefill_f16"}).code_pred(hid, cb0)
        good.append(rel_err(lg_o[0], lg_r[0]))
        bad.append(rel_err(lg_o[0], lg_m[0]))
    assert_agrees(good, "f16")
    assert_misses(bad)


def test_attention_f32_matches_float64_and_not_fp16_form():
    """orc_attention_f32 over 2 positions: within 1e-6 of a float64
    evaluation over the unrounded rows; the fp16-rounded form (fp16 q, K, V
    and P, orc_attention over an fp16 cache) is off by ~1e-3."""
    rng = np.random.default_rng(44)
    nh, nkv, hd = 4, 2, 128
    q = rng.standard_normal((2, nh, hd)).astype(np.float32)
    k = rng.standard_normal((2, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((2, nkv, hd)).astype(np.float32)
    out = orc.attention_f32(q, k, v)
    # position 0 sees itself only: p = 1, the output is its V row exactly
    for h in range(nh):
        assert np.array_equal(out[0, h], v[0, h // 2])
    worst_f32, best_f16 = 0.0, np.inf
    kc = np.ascontiguousarray(k.transpose(1, 0, 2)).astype(np.float16)    # [nkv][n_ctx][hd]
    vc = np.ascontiguousarray(v.transpose(1, 0, 2)).astype(np.float16)
    o16, _ = orc.attention(q[1], kc, vc, 2)
    for h in range(nh):
        g = h // 2
        s = k[:, g].astype(np.float64) @ q[1, h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        ref = p @ v[:, g].astype(np.float64)
        worst_f32 = max(worst_f32, np.abs(out[1, h] - ref).max())
        best_f16 = min(best_f16, np.abs(o16[h] - ref).max())
    assert worst_f32 < 1e-6
    assert best_f16 > 1e-4


def test_zeroed_output_projections_make_layers_identity():
    """attn_output = 0 and ffn_down = 0: every layer passes its input through,
    so hidden = RMSNorm(embd) * output_norm and logits = codec_head . hidden
    (fp16-rounded hidden, F16 head), in closed form; the code predictor's
    head 0 then sees RMSNorm(codec_embd[cb0]) and step g's head sees
    RMSNorm(code_pred_embd[g-1][code])."""
    cfg = small_cfg()
    w = Weights(cfg, "q8_0", seed=34)
    t = dict(w.items())
    for name, (ttype, ne, a) in list(t.items()):
        if name.endswith("attn_output.weight") or name.endswith("ffn_down.weight"):
            t[name] = (ttype, ne, np.zeros_like(a))
    tw = _Tensors(t)
    o = orc.Oracle(cfg, tw, threads=2)
    d = cfg.hidden_size
    x = (np.random.default_rng(45).standard_normal(d) * 0.3).astype(np.float32)
    o.kv_reset(8)
    lg, hid = o.step(x, 0)
    onorm = t["talker.output_norm.weight"][2]
    exp_h = orc.rmsnorm(x, onorm, cfg.rms_eps)
    assert np.array_equal(hid, exp_h)
    head = t["talker.codec_head.weight"][2].astype(np.float64).reshape(cfg.codec_vocab, d)
    exp_l = head @ exp_h.astype(np.float16).astype(np.float64)
    assert np.allclose(lg, exp_l, rtol=1e-6, atol=1e-6)
    codes, lgs = o.code_pred(x, 9)
    cnorm = t["code_pred.output_norm.weight"][2]
    codec = t["talker.codec_embd.weight"][2].astype(np.float32).reshape(cfg.codec_vocab, d)
    rows = [codec[9]] + [t[f"code_pred.codec_embd.{g}.weight"][2].astype(np.float32).reshape(cfg.cp_vocab, d)[codes[g]]
                         for g in range(cfg.n_codebooks - 2)]
    for g in range(cfg.n_codebooks - 1):
        hh = orc.rmsnorm(rows[g], cnorm, cfg.rms_eps)
        lm = t[f"code_pred.lm_head.{g}.weight"][2].astype(np.float64).reshape(cfg.cp_vocab, d)
        assert np.allclose(lgs[g], lm @ hh.astype(np.float16).astype(np.float64), rtol=1e-6, atol=1e-6), g


def test_distinct_heads_are_read_in_step_order():
    """Give lm_head g a single non-zero row, row 100 + g: step g's logits are
    then zero except at 100 + g, so its greedy code is 100 + g whatever the
    input (positive row entries meet a positive-fp16 hidden).  An off-by-one
    head index would put the spike at 101 + g or 99 + g."""
    cfg = small_cfg()
    w = Weights(cfg, "f16", seed=35)
    t = dict(w.items())
    d = cfg.hidden_size
    onorm = np.abs(t["code_pred.output_norm.weight"][2]).astype(np.float32)
    t["code_pred.output_norm.weight"] = (F32, (d, 1), onorm)
    for g in range(cfg.n_codebooks - 1):
        lm = np.zeros((cfg.cp_vocab, d), np.float16)
        lm[100 + g] = 1.0
        t[f"code_pred.lm_head.{g}.weight"] = (F16, (d, cfg.cp_vocab), lm.reshape(-1))
    o = orc.Oracle(cfg, _Tensors(t), threads=2)
    # the sign of each step's normed row varies; the single-row head sums it
    # (logit = sum(fp16(h))), so check the logits' support, not the argmax
    codes, lgs = o.code_pred(np.random.default_rng(46).standard_normal(d).astype(np.float32), 3)
    for g in range(cfg.n_codebooks - 1):
        nz = np.flatnonzero(lgs[g])
        assert list(nz) == [100 + g], (g, nz[:4])


def test_text_proj_matches_numpy_and_zero_fc1_closed_form(model):
    wt, cfg, w, o = model
    toks = np.array([0, 17, cfg.text_vocab - 1, 1234], np.int32)
    got = o.text_proj(toks)
    ref = NpRef(cfg, w).text_proj(toks)
    assert_agrees([rel_err(got[i], ref[i]) for i in range(len(toks))], wt)
    bad = NpRef(cfg, w, {"bias_after_silu"}).text_proj(toks)
    assert_misses([rel_err(got[i], bad[i]) for i in range(len(toks))])
    # fc1 = 0: every row is fc2 . silu(b1) + b2, the same for all tokens
    t = dict(w.items())
    ttype, ne, a = t["talker.text_proj.fc1.weight"]
    t["talker.text_proj.fc1.weight"] = (ttype, ne, np.zeros_like(a))
    o0 = orc.Oracle(cfg, _Tensors(t), threads=2)
    z = o0.text_proj(toks)
    b1 = t["talker.text_proj.fc1.bias"][2].astype(np.float64)
    b2 = t["talker.text_proj.fc2.bias"][2].astype(np.float64)
    r = NpRef(cfg, _Tensors(t))
    exp = r.mm("talker.text_proj.fc2.weight", b1 / (1.0 + np.exp(-b1))) + b2
    assert np.all(z == z[0])
    assert rel_err(z[0], exp) < FLIP[wt]


def test_full_width_layer_matches_numpy_forward():
    """One talker layer and one code-predictor layer at the 0.6B widths
    (d 1024, 16 query / 8 KV heads, FFN 3072), Q8_0."""
    cfg = dataclasses.replace(qcfg.full_06b(), n_layers=1, cp_layers=1, text_vocab=4096, text_embd_dim=256,
                              tts_bos_id=4093, tts_eos_id=4094, tts_pad_id=4092)
    w = Weights(cfg, "q8_0", seed=36)
    o = orc.Oracle(cfg, w, threads=8)
    embd = (np.random.default_rng(47).standard_normal((3, cfg.hidden_size)) * 0.5).astype(np.float32)
    ref = NpRef(cfg, w)
    ref.kv_reset()
    o.kv_reset(8)
    hid_o, lg_o = o.prefill(embd, 0)
    hid_r, lg_r = ref.talker(embd, 0)
    errs = [rel_err(hid_o[i], hid_r[i]) for i in range(3)] + [rel_err(lg_o, lg_r)]
    codes_o, lgs_o = o.code_pred(embd[0], 11)
    codes_r, lgs_r = ref.code_pred(embd[0], 11)
    n_same = int(np.argmax(codes_o != codes_r)) if np.any(codes_o != codes_r) else len(codes_o)
    errs += [rel_err(lgs_o[s], lgs_r[s]) for s in range(max(n_same, 1))]
    assert_agrees(errs, "q8_0")


def test_attention_rows_match_numpy_forward():
    """orc_set_attn_capture keeps layer L's post-softmax row of every
    orc_step (not of the prefill): [n_head][n_kv] with n_kv = position + 1,
    each head's row summing to 1, equal to the float64 forward's softmax
    before the fp16 rounding that feeds P.V.  Capturing the neighbouring layer
    or the fp16-rounded P misses."""
    cfg = qcfg.tiny(n_layers=2, cp_layers=1)
    w = Weights(cfg, "f16", seed=37)
    o = orc.Oracle(cfg, w, threads=4)
    embd = (np.random.default_rng(43).standard_normal((9, cfg.hidden_size)) * 0.5).astype(np.float32)

    def run(layer, mistakes=()):
        ref = NpRef(cfg, w, mistakes)
        ref.capture = (f"talker.blk.{layer}.", [])
        _talker_run(ref, o, cfg, embd)
        return ref.capture[1]

    o.set_attn_capture(1)
    rows_r = run(1)
    rows_o = o.attn_rows()
    assert len(rows_o) == len(rows_r) == 4            # the four steps after a 5-row prefill
    for i, (ro, rr) in enumerate(zip(rows_o, rows_r)):
        assert ro.shape == (cfg.n_head, 5 + i + 1) and rr.shape == ro.shape
        assert np.allclose(ro.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    assert_agrees([rel_err(ro, rr) for ro, rr in zip(rows_o, rows_r)], "f16")
    o.set_attn_capture(1)
    _talker_run(NpRef(cfg, w), o, cfg, embd)
    rows_o = o.attn_rows()
    for mistake, layer in ((("attn_row_f16",), 1), ((), 0)):
        rows_m = run(layer, mistake)
        assert_misses([rel_err(ro, rm) for ro, rm in zip(rows_o, rows_m)])
    o.set_attn_capture(-1)
    _talker_run(NpRef(cfg, w), o, cfg, embd)
    assert o.attn_rows() == []


# ---------------------------------------------------------------- frame loop
def _loop_weights(cfg, wt, seed):
    """Synthetic weights whose talker output-norm gains spread over
    [0.25, 1.75], so the talker's normed hidden row differs from the
    un-normed one in direction, not only in scale (gains near 1 would leave
    the code predictor's own RMSNorm nearly blind to the difference)."""
    t = dict(Weights(cfg, wt, seed=seed).items())
    rng = np.random.default_rng(seed + 1000)
    g = rng.uniform(0.25, 1.75, cfg.hidden_size).astype(np.float32)
    t["talker.output_norm.weight"] = (F32, (cfg.hidden_size, 1), g)
    return _Tensors(t)


def _loop_inputs(cfg, seed, n_pre=10, n_trail=4):
    rng = np.random.default_rng(seed)
    d = cfg.hidden_size
    pre = (rng.standard_normal((n_pre, d)) * 0.5).astype(np.float32)
    trail = (rng.standard_normal((n_trail, d)) * 0.5).astype(np.float32)
    pad = (rng.standard_normal(d) * 0.5).astype(np.float32)
    return pre, trail, pad


def _oracle_loop(o, pre, trail, pad, max_len, rep, eos_bias, target_frames):
    o.kv_reset(len(pre) + max_len + 8)
    _, lg = o.prefill(pre, 0)
    return o.frames(lg, len(pre), trail, pad, max_len, repetition_penalty=rep, eos_bias=eos_bias,
                    target_frames=target_frames, want_logits=True)


# (seed, planted sampler mistakes that change this run's codes)
LOOP_RUNS = {"f16": ((31, ("penalty_per_occurrence", "penalty_sign")), (33, ("penalty_per_occurrence", "penalty_sign"))),
             "q8_0": ((35, ("penalty_per_occurrence", "penalty_sign")), (36, ("penalty_per_occurrence",)))}


@pytest.mark.parametrize("wt", ["f16", "q8_0"])
def test_frame_loop_matches_numpy_generate(wt):
    """orc_frames after orc_prefill (orc_generate_rows' composition) against
    NpRef.generate, the float64 frame loop written from
    src/tts_transformer.cpp:3108-3309: 12 greedy frames of the one-layer tiny
    model from 10 prefill rows, 4 trailing rows (so frames 4.. add tts_pad),
    repetition penalty 1.05 and an EOS bias of -2.  The codes agree exactly
    and every frame's talker logits within the forward tolerance.  Planted
    mistakes in the loop glue each miss: the trailing row of frame + 1, the
    code-predictor embedding table g instead of g - 1, the talker's un-normed
    hidden row into the code predictor (each moves the later frames' logits
    far past the tolerance), the penalty once per earlier occurrence instead
    of once per distinct token, and the inverted penalty sign rule (each
    changes a code).  Applying the penalty after the EOS bias instead of
    before cannot change a result, since the loop stops when EOS is drawn and
    EOS never enters the penalised set; the test shows that too."""
    cfg = small_cfg()
    for seed, sampler_misses in LOOP_RUNS[wt]:
        w = _loop_weights(cfg, wt, seed)
        o = orc.Oracle(cfg, w, threads=4)
        pre, trail, pad = _loop_inputs(cfg, seed)
        kw = dict(rep=1.05, eos_bias=-2.0, target_frames=0)
        co, lgo = _oracle_loop(o, pre, trail, pad, 12, **kw)
        cr, lgr = NpRef(cfg, w).generate(pre, trail, pad, 12, **kw)
        assert co.shape == (12, cfg.n_codebooks) and np.array_equal(co, cr), (seed, co, cr)
        assert lgo.shape == lgr.shape == (12, cfg.codec_vocab)
        assert_agrees([rel_err(lgo[f], lgr[f]) for f in range(12)], wt)
        # a frame's logits are the talker's on the previous frame's step
        # embedding; the code predictor's rows come out of the codes
        for mistake in ("trailing_next", "cp_embd_g", "cp_unnormed"):
            cm, lgm = NpRef(cfg, w, {mistake}).generate(pre, trail, pad, 12, **kw)
            assert_misses([rel_err(lgo[f], lgm[f]) for f in range(1, min(len(lgm), 12))])
        for mistake in sampler_misses:
            cm, _ = NpRef(cfg, w, {mistake}).generate(pre, trail, pad, 12, **kw)
            assert not np.array_equal(cm, co), (seed, mistake)
        cm, _ = NpRef(cfg, w, {"penalty_after_bias"}).generate(pre, trail, pad, 12, **kw)
        assert np.array_equal(cm, co)


@pytest.mark.parametrize("wt", ["f16", "q8_0"])
def test_frame_loop_eos_ramp_matches_numpy_generate(wt):
    """The EOS ramp ends the loop (src/tts_transformer.cpp:3134-3145,
    3186-3188): with target_frames 2 and no base bias, EOS gains 0.1 per
    frame past frame 2 until it is the greedy choice.  The oracle and NpRef
    stop at the same frame with the same codes and logits; a ramp of 0.2 per
    frame stops earlier."""
    cfg = small_cfg()
    w = _loop_weights(cfg, wt, 31)
    o = orc.Oracle(cfg, w, threads=4)
    pre, trail, pad = _loop_inputs(cfg, 31)
    kw = dict(rep=1.05, eos_bias=0.0, target_frames=2)
    co, lgo = _oracle_loop(o, pre, trail, pad, 24, **kw)
    cr, lgr = NpRef(cfg, w).generate(pre, trail, pad, 24, **kw)
    assert 4 <= len(co) < 23, len(co)                 # stopped by EOS, not by max_len
    assert np.array_equal(co, cr)
    assert len(lgo) == len(lgr) == len(co) + 1        # the frame that drew EOS is logged too
    assert_agrees([rel_err(a, b) for a, b in zip(lgo, lgr)], wt)
    cm, _ = NpRef(cfg, w, {"ramp_slope"}).generate(pre, trail, pad, 24, **kw)
    assert len(cm) < len(co)


SINGLE_MISTAKES = ["single_out_norm", "single_gqa_mod", "single_drop_last"]


@pytest.mark.parametrize("layout", ["tiny", "tiny_mtp"])
@pytest.mark.parametrize("wt", ["f16", "q8_0"])
def test_predict_codes_matches_numpy(wt, layout):
    """orc_predict_codes (the single-pass code predictor) against the float64
    graph restatement above, which computes Q, K, their norms and the softmax
    over the one score that the oracle leaves out; with and without the 15
    previous codes, in both layouts (tiny_mtp: the MTP projection).  Dropping
    the last embedding, normalising before the heads or pairing query heads
    with KV heads by h % n_kv instead of h / group all miss."""
    cfg = getattr(qcfg, layout)(n_layers=1, cp_layers=1)
    w = Weights(cfg, wt, seed=37)
    o = orc.Oracle(cfg, w, threads=4)
    rng = np.random.default_rng(38)
    cases = []
    for i in range(3):
        hid = (rng.standard_normal(cfg.hidden_size) * 0.5).astype(np.float32)
        prev = rng.integers(0, cfg.cp_vocab, cfg.n_codebooks - 1).astype(np.int32)
        cases += [(hid, None), (hid, prev)]
    got = [o.predict_codes(h, p) for h, p in cases]
    ref = NpRef(cfg, w)
    assert_agrees([rel_err(g[j], r[j]) for g, (h, p) in zip(got, cases)
                   for r in [ref.predict_codes(h, p)] for j in range(cfg.n_codebooks - 1)], wt)
    for m in SINGLE_MISTAKES:
        bad = NpRef(cfg, w, mistakes=[m])
        sel = [(g, h, p) for g, (h, p) in zip(got, cases) if p is not None or m != "single_drop_last"]
        assert_misses([rel_err(g[j], r[j]) for g, h, p in sel for r in [bad.predict_codes(h, p)]
                       for j in range(cfg.n_codebooks - 1)])
    # a code outside the table is an error, not a read past it
    bad_prev = np.zeros(cfg.n_codebooks - 1, np.int32)
    bad_prev[4] = cfg.cp_vocab
    with pytest.raises(RuntimeError):
        o.predict_codes(cases[0][0], bad_prev)
    o.close()
