"""Pins the oracle's audio-tokenizer decoder (oracle/q3t_vocoder.cpp) against
an independent float64 torch forward written op by op from the reference
graph (src/audio_tokenizer_decoder.cpp:402-843), using torch's own conv1d /
conv_transpose1d / layer_norm / scaled-dot-product attention / GELU(tanh) as
the library routines the graph's ops reduce to.

The torch forward keeps the graph's rounding points only where ggml rounds:
the activation into every F16-weight product (linear layers, im2col
convolutions, depthwise and transposed convolutions) is rounded to fp16.
Everything else is float64.  Agreement is within a stated tolerance, and each
planted mistake (the transposed conv cropped on one side only, RoPE on
interleaved instead of NEOX pairs, the snake's exp(-beta) taken as exp(beta), a
dilation dropped) misses the oracle by far more than that tolerance.  Exact
properties add what a tolerance cannot: windows decoded with all their
context equal the matching slice of the whole decode, a decode of n frames is
a prefix of the decode of n + k frames (every stage is causal), and the output
length follows output_samples_for_frames.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import q3t_oracle as orc
from qwen3_tts_amd import vocoder as V

# per stage, relative to the stage's largest magnitude: the only differences
# are the fp32 rounding of each op (the torch forward stays float64) and,
# through it, an occasional fp16 activation rounding that lands on the other
# side of a tie (one element moves by up to |w| * 2^-11 |x|), hence a loose
# max and a tight rms
STAGE_TOL_MAX = 5e-4
STAGE_TOL_RMS = 2e-5


def f16r(x):
    return x.to(torch.float32).to(torch.float16).to(torch.float64)


class TorchDecoder:
    """float64 restatement with planted-mistake switches."""

    def __init__(self, cfg, w, crop_one_side=False, rope_interleaved=False, beta_sign=False, no_dilation=False):
        self.c, self.w = cfg, w
        self.crop_one_side, self.rope_interleaved = crop_one_side, rope_interleaved
        self.beta_sign, self.no_dilation = beta_sign, no_dilation

    def t(self, name):
        ttype, ne, a = self.w[name]
        x = torch.from_numpy(a.astype(np.float64))
        return x.reshape(tuple(reversed(ne)))            # ggml ne -> torch row-major

    def linear(self, x, name, bias=None):
        W = self.t(name).reshape(self.w[name][1][-1] if len(self.w[name][1]) == 3 else self.w[name][1][1], -1)
        y = f16r(x) @ W.T
        return y if bias is None else y + self.t(bias)

    def conv(self, x, name, bias, dil=1):
        # x [T][C] -> conv1d over [1][C][T], causal left pad (K-1)*dil
        W = self.t(name)                                   # [Co][Ci][K]
        K = W.shape[-1]
        d = 1 if self.no_dilation else dil
        xi = F.pad(f16r(x).T.unsqueeze(0), ((K - 1) * dil, 0))
        y = F.conv1d(xi, W, dilation=d)[0].T
        if self.no_dilation and dil != 1:
            y = y[-x.shape[0]:]
        return y + self.t(bias)

    def conv_t(self, x, name, bias, stride, crop):
        W = self.t(name)                                   # [Ci][Co][K]
        y = F.conv_transpose1d(f16r(x).T.unsqueeze(0), W, stride=stride)[0].T
        if crop:
            y = y[crop:] if self.crop_one_side else y[crop:-crop]
        return y + self.t(bias)

    def snake(self, x, a, b):
        ea = torch.exp(self.t(a))
        eb = torch.exp(self.t(b) if self.beta_sign else -self.t(b))
        return x + torch.sin(x * ea) ** 2 * eb

    def rms(self, x, name):
        return x / torch.sqrt((x * x).mean(-1, keepdim=True) + self.c.rms_eps) * self.t(name)

    def rope(self, x, pos):
        hd = x.shape[-1]
        i = torch.arange(hd // 2, dtype=torch.float64)
        th = pos[:, None].to(torch.float64) * self.c.rope_theta ** (-2.0 * i / hd)
        cs, sn = torch.cos(th)[:, None, :], torch.sin(th)[:, None, :]
        if self.rope_interleaved:                 # GPT-J pairs (2i, 2i+1) instead of NEOX (i, i + hd/2)
            a, b = x[..., 0::2], x[..., 1::2]
            return torch.stack([a * cs - b * sn, a * sn + b * cs], -1).reshape(x.shape)
        a, b = x[..., :hd // 2], x[..., hd // 2:]
        return torch.cat([a * cs - b * sn, a * sn + b * cs], -1)

    def latent(self, codes):
        c = self.c
        emb = []
        for q in range(c.n_codebooks):
            p = "tok_dec.vq_first.0." if q == 0 else f"tok_dec.vq_rest.{q - 1}."
            cb = torch.from_numpy(self.w[p + "codebook"][2].astype(np.float32)).reshape(c.codebook_size, -1)
            u = torch.from_numpy(self.w[p + "usage"][2]).clamp(min=1e-5)
            cbn = (cb * (1.0 / u)[:, None]).to(torch.float16).to(torch.float64)
            wn = "tok_dec.vq_first.output_proj.weight" if q == 0 else "tok_dec.vq_rest.output_proj.weight"
            emb.append(self.linear(cbn[torch.from_numpy(codes[:, q]).long()], wn))
        return emb[0] + sum(emb[1:])

    def stage(self, name, x, pos0=0):
        """the oracle's stage `name` (q3t_vocoder.cpp stage_names) on float64 rows"""
        c = self.c
        if name == "pre_conv":
            return self.conv(x, "tok_dec.pre_conv.weight", "tok_dec.pre_conv.bias")
        if name == "input_proj":
            return self.linear(x, "tok_dec.pre_tfm.input_proj.weight", "tok_dec.pre_tfm.input_proj.bias")
        if name.startswith("pre_tfm."):
            p = f"tok_dec.pre_tfm.blk.{int(name[8:])}."
            n, nh, hd = x.shape[0], c.n_heads, c.latent // c.n_heads
            pos = torch.arange(n) + pos0
            h = self.rms(x, p + "attn_norm.weight")
            q = self.rope(self.linear(h, p + "attn_q.weight").reshape(n, nh, hd), pos)
            k = self.rope(self.linear(h, p + "attn_k.weight").reshape(n, nh, hd), pos)
            v = self.linear(h, p + "attn_v.weight").reshape(n, nh, hd)
            a = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1),
                                               is_causal=True)
            a = a.transpose(0, 1).reshape(n, nh * hd)
            x = x + self.linear(a, p + "attn_output.weight") * self.t(p + "attn_scale")
            h = self.rms(x, p + "ffn_norm.weight")
            g = self.linear(h, p + "ffn_gate.weight")
            u = self.linear(h, p + "ffn_up.weight")
            return x + self.linear(F.silu(g) * u, p + "ffn_down.weight") * self.t(p + "ffn_scale")
        if name == "output_proj":
            x = self.rms(x, "tok_dec.pre_tfm.norm.weight")
            return self.linear(x, "tok_dec.pre_tfm.output_proj.weight", "tok_dec.pre_tfm.output_proj.bias")
        if name.startswith("upsample."):
            p = f"tok_dec.upsample.{int(name[9:])}."
            y = self.conv_t(x, p + "conv.weight", p + "conv.bias", 2, 0)
            W = self.t(p + "dwconv.weight")                # [C][1][7]
            z = F.conv1d(F.pad(f16r(y).T.unsqueeze(0), (6, 0)), W, groups=W.shape[0])[0].T + self.t(p + "dwconv.bias")
            z = F.layer_norm(z, (z.shape[-1],), self.t(p + "norm.weight"), self.t(p + "norm.bias"), eps=1e-6)
            h = F.gelu(self.linear(z, p + "pwconv1.weight", p + "pwconv1.bias"), approximate="tanh")
            return y + self.linear(h, p + "pwconv2.weight", p + "pwconv2.bias") * self.t(p + "gamma")
        if name == "dec.0":
            return self.conv(x, "tok_dec.dec.0.conv.weight", "tok_dec.dec.0.conv.bias")
        if name == "dec.6":
            x = self.snake(x, "tok_dec.dec.5.snake.alpha", "tok_dec.dec.5.snake.beta")
            return self.conv(x, "tok_dec.dec.6.conv.weight", "tok_dec.dec.6.conv.bias")
        b = int(name[4])
        p = f"tok_dec.dec.{b}."
        if name.endswith(".conv_t"):
            s, K = c.rates[b - 1], c.dec_kernel[b - 1]
            x = self.snake(x, p + "snake.alpha", p + "snake.beta")
            return self.conv_t(x, p + "conv_t.weight", p + "conv_t.bias", s, K - s)
        r = int(name[-1])
        q = p + f"res.{r}."
        h = self.snake(x, q + "act1.alpha", q + "act1.beta")
        h = self.conv(h, q + "conv1.weight", q + "conv1.bias", (1, 3, 9)[r - 2])
        h = self.snake(h, q + "act2.alpha", q + "act2.beta")
        return x + self.conv(h, q + "conv2.weight", q + "conv2.bias")

    def forward(self, codes, pos0):
        x = self.latent(codes)
        for name in stage_names(self.c)[1:]:
            x = self.stage(name, x, pos0)
        return torch.tanh(x[:, 0]).numpy()


def stage_names(c):
    v = ["latent", "pre_conv", "input_proj"] + [f"pre_tfm.{l}" for l in range(c.n_layers)]
    v += ["output_proj", "upsample.0", "upsample.1", "dec.0"]
    for b in range(1, 5):
        v += [f"dec.{b}.conv_t"] + [f"dec.{b}.res.{r}" for r in range(2, 5)]
    return v + ["dec.6"]


def stage_err(got, want):
    """(max, rms) of |got - want| relative to the stage's largest magnitude"""
    d = np.abs(got - want) / max(np.abs(want).max(), 1e-6)
    return float(d.max()), float(np.sqrt((d * d).mean()))


@pytest.fixture(scope="module")
def tiny_voc():
    c = V.tiny()
    w = V.VocWeights(c, seed=11)
    return c, w, orc.VocOracle(c, w, threads=8)


def _codes(n, seed, size=2048):
    return np.random.default_rng(seed).integers(0, size, (n, 16)).astype(np.int32)


def test_output_length_formula(tiny_voc):
    c, w, o = tiny_voc
    full = V.full()
    for n in (1, 2, 7, 25, 73, 200):
        assert o.samples_for_frames(n) == c.samples_for_frames(n)
    # the full decoder: 4n rows after the two x2 upsamplers, then each
    # decoder block maps m rows to (m - 1) * rate:
    # 3(4(5(8(4n - 1) - 1) - 1) - 1) = 1920 n - 555 samples at 24 kHz
    for n in (1, 2, 10, 73, 100):
        assert full.samples_for_frames(n) == 1920 * n - 555


def test_codebook_clamp_in_latent(tiny_voc):
    """latent = sum_q proj_q(normalised codebook row); entries whose usage is
    below 1e-5 are divided by the clamped 1e-5."""
    c, w, o = tiny_voc
    cb = "tok_dec.vq_first.0.codebook"
    low = int(w.clamped[cb][0])
    codes = _codes(3, 1)
    codes[1, 0] = low
    _, lat = o.decode_single(codes, want_latent=True)
    ref = TorchDecoder(c, w)
    rows = []
    for q in range(16):
        p = "tok_dec.vq_first.0." if q == 0 else f"tok_dec.vq_rest.{q - 1}."
        cbt = torch.from_numpy(w[p + "codebook"][2].astype(np.float32)).reshape(c.codebook_size, -1)
        u = torch.from_numpy(w[p + "usage"][2]).clamp(min=1e-5)
        cbn = (cbt * (1.0 / u)[:, None]).to(torch.float16).to(torch.float64)
        wn = "tok_dec.vq_first.output_proj.weight" if q == 0 else "tok_dec.vq_rest.output_proj.weight"
        rows.append(ref.linear(cbn[torch.from_numpy(codes[:, q]).long()], wn))
    want = (rows[0] + sum(rows[1:])).numpy()
    assert np.abs(lat - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    # without the clamp (dividing by the raw 3e-6) the first-codebook row would be 3.3x larger
    assert np.abs(want[1]).max() > 0.1


@pytest.mark.parametrize("n,pos0", [(5, 0), (4, 9)])
def test_stages_match_torch(tiny_voc, n, pos0):
    """every stage, run by torch from the oracle's previous stage output,
    matches the oracle's own stage output within STAGE_TOL relative"""
    c, w, o = tiny_voc
    codes = _codes(n, 100 + n)
    st = o.stages(codes, pos0)
    assert list(st) == stage_names(c)
    ref = TorchDecoder(c, w)
    errs = {"latent": stage_err(st["latent"], ref.latent(codes).numpy())}
    names = stage_names(c)
    for prev, name in zip(names, names[1:]):
        want = ref.stage(name, torch.from_numpy(st[prev].astype(np.float64)), pos0).numpy()
        assert st[name].shape == want.shape, name
        errs[name] = stage_err(st[name], want)
    worst = max(errs, key=lambda k: errs[k][0])
    assert errs[worst][0] <= STAGE_TOL_MAX, (worst, errs[worst])
    worst = max(errs, key=lambda k: errs[k][1])
    assert errs[worst][1] <= STAGE_TOL_RMS, (worst, errs[worst])
    # run_stage is the same computation as the recorded chain
    for prev, name in zip(names, names[1:]):
        assert np.array_equal(o.run_stage(name, st[prev], pos0), st[name]), name


def test_end_to_end_snr_vs_torch(tiny_voc):
    """the whole decode against the float64 forward: rounding-cliff noise
    (an fp16 rounding that lands on the other side of a tie) is amplified
    stage by stage, so only a loose bound holds end to end"""
    c, w, o = tiny_voc
    codes = _codes(5, 105)
    got = o.decode_single(codes, 0)
    want = TorchDecoder(c, w).forward(codes, 0)
    snr = 10 * np.log10((want ** 2).mean() / ((got - want) ** 2).mean())
    assert snr >= 25.0, snr
    assert np.abs(want).std() > 0.05          # neither saturated nor silent


@pytest.mark.parametrize("mistake,stage", [("crop_one_side", "dec.2.conv_t"), ("rope_interleaved", "pre_tfm.1"),
                                           ("beta_sign", "dec.3.res.2"), ("no_dilation", "dec.1.res.4")])
def test_planted_mistakes_miss(tiny_voc, mistake, stage):
    c, w, o = tiny_voc
    codes = _codes(4, 104)
    st = o.stages(codes, 9)
    names = stage_names(c)
    prev = names[names.index(stage) - 1]
    bad = TorchDecoder(c, w, **{mistake: True}).stage(stage, torch.from_numpy(st[prev].astype(np.float64)), 9)
    bad = bad.numpy()
    assert bad.shape != st[stage].shape or stage_err(st[stage], bad)[0] > 50 * STAGE_TOL_MAX


def test_window_with_full_context_equals_whole_decode(tiny_voc):
    c, w, o = tiny_voc
    codes = _codes(9, 3)
    whole = o.decode_single(codes)
    win = o.decode_window(codes, 4, 9, 48)          # context reaches frame 0
    drop = o.samples_for_frames(4)
    assert np.array_equal(win, whole[drop:])
    first = o.decode_window(codes, 0, 4, 48)
    assert np.array_equal(first, whole[:o.samples_for_frames(4)])


def test_decode_prefix_is_causal(tiny_voc):
    c, w, o = tiny_voc
    codes = _codes(8, 4)
    a = o.decode_single(codes[:5])
    b = o.decode_single(codes)
    assert np.array_equal(a, b[:len(a)])


def test_window_drops_warmup_at_absolute_positions(tiny_voc):
    """A window whose context does not reach frame 0 decodes frames
    [start - context, end) at their absolute positions and keeps the last
    samples_for_frames(end - ctx_start) - samples_for_frames(context)."""
    c, w, o = tiny_voc
    codes = _codes(10, 5)
    win = o.decode_window(codes, 6, 10, 3)
    seg = o.decode_single(codes[3:10], 3)
    assert np.array_equal(win, seg[o.samples_for_frames(3):])
    with pytest.raises(RuntimeError):
        o.decode_window(codes, 6, 11, 3)
    with pytest.raises(RuntimeError):
        o.decode_window(codes, 5, 5, 3)
