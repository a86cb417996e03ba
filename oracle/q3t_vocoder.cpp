// q3t_vocoder.cpp -- CPU restatement of the qwen3-tts.cpp audio-tokenizer
// decoder (the vocoder that turns 16-codebook frames into 24 kHz PCM).
//
// TEST INFRASTRUCTURE ONLY: the parity checker for the HIP vocoder.  Nothing
// in qwen3-tts.cpp_amd/ links, loads or calls it.
//
// Restated from (reference paths relative to the reference checkout):
//   codebook normalisation     src/audio_tokenizer_decoder.cpp:66-100
//   snake activation           src/audio_tokenizer_decoder.cpp:402-426
//   pre-transformer layer      src/audio_tokenizer_decoder.cpp:436-500
//   upsample (ConvNeXt) block  src/audio_tokenizer_decoder.cpp:502-563
//   residual unit              src/audio_tokenizer_decoder.cpp:565-593
//   decoder block              src/audio_tokenizer_decoder.cpp:595-634
//   whole graph                src/audio_tokenizer_decoder.cpp:636-843
//   output length              src/audio_tokenizer_decoder.cpp:845-875
//   decode / decode_window     src/audio_tokenizer_decoder.cpp:877-960, 1003-1024
//
// Numerics (ggml semantics restated; ggml itself is absent):
//   - activations fp32, time-major [T][C] here (ggml keeps [C][T] for convs;
//     the layout does not change any value);
//   - every F16-weight product (linear layers, 1-D convolutions through
//     im2col, the depthwise conv, the transposed conv) rounds its fp32
//     activation to fp16 first, as ggml's F16 im2col / vec_dot_type does; the
//     fp16 x fp16 products are exact and are summed in fp64, rounded to fp32
//     once (ggml sums in fp32 lanes: tolerance-level difference);
//   - bias, layer scale, gamma and residual adds are separate fp32 ops in the
//     graph's order;
//   - attention in the pre-transformer is all-F32 (Q, K, V are F32 views):
//     no fp16 rounding; scores and P.V summed in fp64, rounded once;
//   - RMSNorm: sum of float squares in double, y = x * (1/sqrtf(mean+eps)),
//     then * w; LayerNorm (ggml_norm): double mean, centred fp32 values,
//     double variance, scale 1/sqrtf(var+eps), then * w + b;
//   - exp, sin, tanh are the C library's expf/sinf/tanhf; GELU is the tanh
//     form 0.5x(1+tanh(sqrt(2/pi) x (1+0.044715x^2))) (ggml_gelu's formula;
//     ggml-cpu's fp16 lookup table for it is not restated); SiLU is
//     x / (1 + expf(-x)).
#include "q3t_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <string>
#include <thread>
#include <vector>

namespace {

inline float h2f(uint16_t h) { return orc_f16_to_f32(h); }
inline float r16(float x) { return orc_f16_to_f32(orc_f32_to_f16(x)); }

template <class F>
void par_for(int threads, int64_t n, F fn) {
    if (threads <= 1 || n < 64) { fn((int64_t) 0, n); return; }
    std::vector<std::thread> th;
    const int nt = (int) std::min<int64_t>(threads, n);
    for (int i = 1; i < nt; ++i) th.emplace_back([&, i] { fn(n * i / nt, n * (i + 1) / nt); });
    fn(0, n / nt);
    for (auto & t : th) t.join();
}

struct Tensor {
    int32_t type = -1;
    const void * data = nullptr;
    size_t nbytes = 0;
};

// fp32 activation [T][C]
struct Act {
    int64_t T = 0, C = 0;
    std::vector<float> v;
    Act() = default;
    Act(int64_t t, int64_t c) : T(t), C(c), v((size_t) (t * c), 0.0f) {}
    float * row(int64_t t) { return v.data() + t * C; }
    const float * row(int64_t t) const { return v.data() + t * C; }
};

}  // namespace

struct orc_voc {
    orc_voc_config cfg;
    int threads = 4;
    std::map<std::string, Tensor> t;
    std::vector<std::vector<uint16_t>> cb;      // normalised codebooks [16][size*dim] fp16
    std::string err;
    bool record = false;                        // keep every stage's output (tests)
    std::vector<std::pair<std::string, Act>> stages;
    void keep(const std::string & name, const Act & a) {
        if (record) stages.emplace_back(name, a);
    }

    const Tensor * get(const std::string & name) const {
        auto it = t.find(name);
        return it == t.end() ? nullptr : &it->second;
    }
    const uint16_t * f16(const std::string & name) const { return (const uint16_t *) get(name)->data; }
    const float * f32(const std::string & name) const {
        const Tensor * x = get(name);
        return x ? (const float *) x->data : nullptr;
    }
};

namespace {

// y[t][o] = sum_{k,i} fp16(x[t + k*dil - pad][i]) * W[o][i][k], W in ggml
// conv layout ne = (K, Ci, Co) fp16; rows outside [0, T) are zero padding.
// Then + bias.  (ggml_pad_ext + ggml_conv_1d + ggml_add.)
Act conv1d(const orc_voc * m, const Act & x, const uint16_t * w, const float * b, int K, int Co, int dil, int pad) {
    const int64_t T = x.T, Ci = x.C;
    Act xh(T, Ci);
    for (size_t i = 0; i < x.v.size(); ++i) xh.v[i] = r16(x.v[i]);
    std::vector<float> wf((size_t) K * Ci * Co);
    for (size_t i = 0; i < wf.size(); ++i) wf[i] = h2f(w[i]);
    Act y(T, Co);
    par_for(m->threads, T, [&](int64_t t0, int64_t t1) {
        for (int64_t t = t0; t < t1; ++t)
            for (int o = 0; o < Co; ++o) {
                double acc = 0.0;
                for (int k = 0; k < K; ++k) {
                    const int64_t src = t + (int64_t) k * dil - pad;
                    if (src < 0 || src >= T) continue;
                    const float * xr = xh.row(src);
                    const float * wr = wf.data() + (size_t) o * Ci * K + k;
                    for (int64_t i = 0; i < Ci; ++i) acc += (double) xr[i] * (double) wr[i * K];
                }
                float v = (float) acc;
                if (b) v = v + b[o];
                y.row(t)[o] = v;
            }
    });
    return y;
}

// ConvTranspose1d (ggml_conv_transpose_1d, p0 = 0, d0 = 1), W ne = (K, Co, Ci):
// full[t][o] = sum_{l,k: l*s + k = t} sum_i fp16(x[l][i]) * W[i][o][k];
// then rows [crop, len - crop) are kept and the bias is added.
Act conv_t1d(const orc_voc * m, const Act & x, const uint16_t * w, const float * b, int K, int Co, int s, int crop) {
    const int64_t L = x.T, Ci = x.C;
    const int64_t full = (L - 1) * s + K, T = full - 2 * crop;
    Act xh(L, Ci);
    for (size_t i = 0; i < x.v.size(); ++i) xh.v[i] = r16(x.v[i]);
    std::vector<float> wf((size_t) K * Ci * Co);
    for (size_t i = 0; i < wf.size(); ++i) wf[i] = h2f(w[i]);
    Act y(std::max<int64_t>(T, 0), Co);
    par_for(m->threads, y.T, [&](int64_t t0, int64_t t1) {
        for (int64_t tt = t0; tt < t1; ++tt) {
            const int64_t t = tt + crop;
            for (int o = 0; o < Co; ++o) {
                double acc = 0.0;
                for (int k = 0; k < K; ++k) {
                    if ((t - k) % s != 0 || t - k < 0) continue;
                    const int64_t l = (t - k) / s;
                    if (l >= L) continue;
                    const float * xr = xh.row(l);
                    for (int64_t i = 0; i < Ci; ++i)
                        acc += (double) xr[i] * (double) wf[((size_t) i * Co + o) * K + k];
                }
                float v = (float) acc;
                if (b) v = v + b[o];
                y.row(tt)[o] = v;
            }
        }
    });
    return y;
}

// y[t][n] = sum_k fp16(x[t][k]) * W[n][k] (W ne = (K, N) fp16), then + bias.
Act linear(const orc_voc * m, const Act & x, const uint16_t * w, const float * b, int N) {
    const int64_t T = x.T, K = x.C;
    std::vector<float> wf((size_t) K * N);
    for (size_t i = 0; i < wf.size(); ++i) wf[i] = h2f(w[i]);
    Act y(T, N);
    par_for(m->threads, T, [&](int64_t t0, int64_t t1) {
        std::vector<float> xh((size_t) K);
        for (int64_t t = t0; t < t1; ++t) {
            for (int64_t k = 0; k < K; ++k) xh[k] = r16(x.row(t)[k]);
            for (int n = 0; n < N; ++n) {
                const float * wr = wf.data() + (size_t) n * K;
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += (double) xh[k] * (double) wr[k];
                float v = (float) acc;
                if (b) v = v + b[n];
                y.row(t)[n] = v;
            }
        }
    });
    return y;
}

void snake(Act & x, const float * alpha, const float * beta) {
    for (int64_t c = 0; c < x.C; ++c) {
        const float ea = std::exp(alpha[c]);
        const float eb = std::exp(beta[c] * -1.0f);
        for (int64_t t = 0; t < x.T; ++t) {
            float & v = x.row(t)[c];
            const float s = std::sin(v * ea);
            const float sq = s * s;
            v = v + sq * eb;
        }
    }
}

void rmsnorm_rows(Act & x, const float * w, float eps) {
    for (int64_t t = 0; t < x.T; ++t) orc_rmsnorm(x.row(t), w, x.C, eps, x.row(t));
}

float gelu(float x) {
    const float c = 0.79788456080286535587989211986876f, a = 0.044715f;
    return 0.5f * x * (1.0f + std::tanh(c * x * (1.0f + a * x * x)));
}

float silu(float x) { return x / (1.0f + std::exp(-x)); }

std::string blk(int i, const char * s) { return "tok_dec.pre_tfm.blk." + std::to_string(i) + "." + s; }

// pre-transformer layer (src/audio_tokenizer_decoder.cpp:436-500), positions
// pos0 .. pos0 + T - 1.
void pre_tfm_layer(const orc_voc * m, Act & x, int l, int64_t pos0) {
    const orc_voc_config & c = m->cfg;
    const int64_t T = x.T, D = x.C;
    const int nh = c.n_heads, hd = c.latent / c.n_heads, qd = c.latent;
    Act h = x;
    rmsnorm_rows(h, m->f32(blk(l, "attn_norm.weight")), c.rms_eps);
    Act q = linear(m, h, m->f16(blk(l, "attn_q.weight")), nullptr, qd);
    Act k = linear(m, h, m->f16(blk(l, "attn_k.weight")), nullptr, qd);
    Act v = linear(m, h, m->f16(blk(l, "attn_v.weight")), nullptr, qd);
    std::vector<float> cs((size_t) (pos0 + T) * hd / 2), sn(cs.size());
    orc_rope_table(c.rope_theta, hd, pos0 + T, cs.data(), sn.data());
    for (int64_t t = 0; t < T; ++t)
        for (int hh = 0; hh < nh; ++hh) {
            const float * cr = cs.data() + (pos0 + t) * hd / 2;
            const float * sr = sn.data() + (pos0 + t) * hd / 2;
            orc_rope_neox(q.row(t) + hh * hd, hd, cr, sr);
            orc_rope_neox(k.row(t) + hh * hd, hd, cr, sr);
        }
    Act att(T, qd);
    const float scale = 1.0f / std::sqrt((float) hd);
    par_for(m->threads, T * nh, [&](int64_t b0, int64_t b1) {
        std::vector<float> p((size_t) T);
        for (int64_t bi = b0; bi < b1; ++bi) {
            const int64_t t = bi / nh;
            const int hh = (int) (bi % nh);
            const float * qr = q.row(t) + hh * hd;
            float mx = -INFINITY;
            for (int64_t j = 0; j <= t; ++j) {
                const float * kr = k.row(j) + hh * hd;
                double s = 0.0;
                for (int d = 0; d < hd; ++d) s += (double) qr[d] * (double) kr[d];
                p[j] = (float) s * scale;
                mx = std::max(mx, p[j]);
            }
            double sum = 0.0;
            for (int64_t j = 0; j <= t; ++j) {
                p[j] = std::exp(p[j] - mx);
                sum += (double) p[j];
            }
            const float inv = (float) (1.0 / sum);
            for (int64_t j = 0; j <= t; ++j) p[j] = p[j] * inv;
            for (int d = 0; d < hd; ++d) {
                double o = 0.0;
                for (int64_t j = 0; j <= t; ++j) o += (double) p[j] * (double) v.row(j)[hh * hd + d];
                att.row(t)[hh * hd + d] = (float) o;
            }
        }
    });
    Act o = linear(m, att, m->f16(blk(l, "attn_output.weight")), nullptr, (int) D);
    const float * as = m->f32(blk(l, "attn_scale"));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t i = 0; i < D; ++i) {
            float y = o.row(t)[i];
            if (as) y = y * as[i];
            x.row(t)[i] = x.row(t)[i] + y;
        }
    h = x;
    rmsnorm_rows(h, m->f32(blk(l, "ffn_norm.weight")), c.rms_eps);
    Act g = linear(m, h, m->f16(blk(l, "ffn_gate.weight")), nullptr, c.ffn);
    Act u = linear(m, h, m->f16(blk(l, "ffn_up.weight")), nullptr, c.ffn);
    for (size_t i = 0; i < g.v.size(); ++i) g.v[i] = silu(g.v[i]) * u.v[i];
    Act dn = linear(m, g, m->f16(blk(l, "ffn_down.weight")), nullptr, (int) D);
    const float * fs = m->f32(blk(l, "ffn_scale"));
    for (int64_t t = 0; t < T; ++t)
        for (int64_t i = 0; i < D; ++i) {
            float y = dn.row(t)[i];
            if (fs) y = y * fs[i];
            x.row(t)[i] = x.row(t)[i] + y;
        }
}

// ConvNeXt upsample block (src/audio_tokenizer_decoder.cpp:502-563).
Act upsample_block(const orc_voc * m, const Act & x, int i) {
    const orc_voc_config & c = m->cfg;
    const std::string p = "tok_dec.upsample." + std::to_string(i) + ".";
    const int C = c.latent;
    Act y = conv_t1d(m, x, m->f16(p + "conv.weight"), m->f32(p + "conv.bias"), c.up_kernel, C, 2, 0);
    const int64_t T = y.T;
    // depthwise k7, causal left pad 6: z[t][c] = sum_k fp16(y[t+k-6][c]) * w[c][k]
    const uint16_t * dw = m->f16(p + "dwconv.weight");
    const float * db = m->f32(p + "dwconv.bias");
    Act z(T, C);
    for (int64_t t = 0; t < T; ++t)
        for (int ch = 0; ch < C; ++ch) {
            double acc = 0.0;
            for (int k = 0; k < 7; ++k) {
                const int64_t s = t + k - 6;
                if (s < 0) continue;
                acc += (double) r16(y.row(s)[ch]) * (double) h2f(dw[(size_t) ch * 7 + k]);
            }
            float v = (float) acc;
            if (db) v = v + db[ch];
            z.row(t)[ch] = v;
        }
    // LayerNorm over channels, eps 1e-6 (ggml_norm), then * w + b
    const float * nw = m->f32(p + "norm.weight");
    const float * nb = m->f32(p + "norm.bias");
    for (int64_t t = 0; t < T; ++t) {
        float * r = z.row(t);
        double sum = 0.0;
        for (int ch = 0; ch < C; ++ch) sum += (double) r[ch];
        const float mean = (float) (sum / C);
        double sum2 = 0.0;
        for (int ch = 0; ch < C; ++ch) {
            const float v = r[ch] - mean;
            r[ch] = v;
            sum2 += (double) (v * v);
        }
        const float var = (float) (sum2 / C);
        const float sc = 1.0f / std::sqrt(var + 1e-6f);
        for (int ch = 0; ch < C; ++ch) {
            float v = r[ch] * sc;
            v = v * nw[ch];
            r[ch] = v + nb[ch];
        }
    }
    Act h = linear(m, z, m->f16(p + "pwconv1.weight"), m->f32(p + "pwconv1.bias"), c.cnx_ffn);
    for (auto & v : h.v) v = gelu(v);
    Act o = linear(m, h, m->f16(p + "pwconv2.weight"), m->f32(p + "pwconv2.bias"), C);
    const float * gm = m->f32(p + "gamma");
    for (int64_t t = 0; t < T; ++t)
        for (int ch = 0; ch < C; ++ch) {
            float v = o.row(t)[ch];
            if (gm) v = v * gm[ch];
            o.row(t)[ch] = y.row(t)[ch] + v;
        }
    return o;
}

int conv_t_kernel(const orc_voc * m, int blk_i) { return m->cfg.dec_kernel[blk_i]; }

}  // namespace

extern "C" {

orc_voc * orc_voc_create(const orc_voc_config * cfg) {
    orc_voc * m = new orc_voc();
    m->cfg = *cfg;
    return m;
}

void orc_voc_destroy(orc_voc * m) { delete m; }

void orc_voc_set_threads(orc_voc * m, int32_t n) { m->threads = std::max(1, (int) n); }

const char * orc_voc_last_error(const orc_voc * m) { return m->err.c_str(); }

int orc_voc_set_tensor(orc_voc * m, const char * name, int32_t type, const void * data, size_t nbytes) {
    if (!m || !name || !data) return -1;
    m->t[name] = Tensor{type, data, nbytes};
    return 0;
}

// Checks presence, types and sizes, and normalises the codebooks
// (src/audio_tokenizer_decoder.cpp:66-100): cb = fp16(fp32(cb) * (1/max(u, 1e-5))).
int orc_voc_finalize(orc_voc * m) {
    const orc_voc_config & c = m->cfg;
    const int hd = c.latent / c.n_heads;
    struct Want { std::string name; int32_t type; size_t n; };
    std::vector<Want> want;
    auto add = [&](const std::string & n, int32_t ty, size_t cnt) { want.push_back({n, ty, cnt}); };
    add("tok_dec.vq_first.output_proj.weight", ORC_TYPE_F16, (size_t) c.codebook_dim * c.hidden);
    add("tok_dec.vq_rest.output_proj.weight", ORC_TYPE_F16, (size_t) c.codebook_dim * c.hidden);
    add("tok_dec.vq_first.0.codebook", ORC_TYPE_F16, (size_t) c.codebook_dim * c.codebook_size);
    add("tok_dec.vq_first.0.usage", ORC_TYPE_F32, (size_t) c.codebook_size);
    for (int i = 0; i < c.n_codebooks - 1; ++i) {
        add("tok_dec.vq_rest." + std::to_string(i) + ".codebook", ORC_TYPE_F16, (size_t) c.codebook_dim * c.codebook_size);
        add("tok_dec.vq_rest." + std::to_string(i) + ".usage", ORC_TYPE_F32, (size_t) c.codebook_size);
    }
    add("tok_dec.pre_conv.weight", ORC_TYPE_F16, (size_t) 3 * c.hidden * c.latent);
    add("tok_dec.pre_conv.bias", ORC_TYPE_F32, (size_t) c.latent);
    add("tok_dec.pre_tfm.input_proj.weight", ORC_TYPE_F16, (size_t) c.latent * c.hidden);
    add("tok_dec.pre_tfm.input_proj.bias", ORC_TYPE_F32, (size_t) c.hidden);
    for (int l = 0; l < c.n_layers; ++l) {
        add(blk(l, "attn_norm.weight"), ORC_TYPE_F32, (size_t) c.hidden);
        add(blk(l, "attn_q.weight"), ORC_TYPE_F16, (size_t) c.hidden * c.latent);
        add(blk(l, "attn_k.weight"), ORC_TYPE_F16, (size_t) c.hidden * c.latent);
        add(blk(l, "attn_v.weight"), ORC_TYPE_F16, (size_t) c.hidden * c.latent);
        add(blk(l, "attn_output.weight"), ORC_TYPE_F16, (size_t) c.latent * c.hidden);
        add(blk(l, "attn_scale"), ORC_TYPE_F32, (size_t) c.hidden);
        add(blk(l, "ffn_norm.weight"), ORC_TYPE_F32, (size_t) c.hidden);
        add(blk(l, "ffn_gate.weight"), ORC_TYPE_F16, (size_t) c.hidden * c.ffn);
        add(blk(l, "ffn_up.weight"), ORC_TYPE_F16, (size_t) c.hidden * c.ffn);
        add(blk(l, "ffn_down.weight"), ORC_TYPE_F16, (size_t) c.ffn * c.hidden);
        add(blk(l, "ffn_scale"), ORC_TYPE_F32, (size_t) c.hidden);
    }
    add("tok_dec.pre_tfm.norm.weight", ORC_TYPE_F32, (size_t) c.hidden);
    add("tok_dec.pre_tfm.output_proj.weight", ORC_TYPE_F16, (size_t) c.hidden * c.latent);
    add("tok_dec.pre_tfm.output_proj.bias", ORC_TYPE_F32, (size_t) c.latent);
    for (int i = 0; i < 2; ++i) {
        const std::string p = "tok_dec.upsample." + std::to_string(i) + ".";
        add(p + "conv.weight", ORC_TYPE_F16, (size_t) c.up_kernel * c.latent * c.latent);
        add(p + "conv.bias", ORC_TYPE_F32, (size_t) c.latent);
        add(p + "dwconv.weight", ORC_TYPE_F16, (size_t) 7 * c.latent);
        add(p + "dwconv.bias", ORC_TYPE_F32, (size_t) c.latent);
        add(p + "norm.weight", ORC_TYPE_F32, (size_t) c.latent);
        add(p + "norm.bias", ORC_TYPE_F32, (size_t) c.latent);
        add(p + "pwconv1.weight", ORC_TYPE_F16, (size_t) c.latent * c.cnx_ffn);
        add(p + "pwconv1.bias", ORC_TYPE_F32, (size_t) c.cnx_ffn);
        add(p + "pwconv2.weight", ORC_TYPE_F16, (size_t) c.cnx_ffn * c.latent);
        add(p + "pwconv2.bias", ORC_TYPE_F32, (size_t) c.latent);
        add(p + "gamma", ORC_TYPE_F32, (size_t) c.latent);
    }
    add("tok_dec.dec.0.conv.weight", ORC_TYPE_F16, (size_t) 7 * c.latent * c.decoder_dim);
    add("tok_dec.dec.0.conv.bias", ORC_TYPE_F32, (size_t) c.decoder_dim);
    int ch = c.decoder_dim;
    for (int b = 0; b < 4; ++b) {
        const std::string p = "tok_dec.dec." + std::to_string(b + 1) + ".";
        const int co = ch / 2;
        add(p + "snake.alpha", ORC_TYPE_F32, (size_t) ch);
        add(p + "snake.beta", ORC_TYPE_F32, (size_t) ch);
        add(p + "conv_t.weight", ORC_TYPE_F16, (size_t) c.dec_kernel[b] * co * ch);
        add(p + "conv_t.bias", ORC_TYPE_F32, (size_t) co);
        for (int r = 2; r <= 4; ++r) {
            const std::string q = p + "res." + std::to_string(r) + ".";
            add(q + "act1.alpha", ORC_TYPE_F32, (size_t) co);
            add(q + "act1.beta", ORC_TYPE_F32, (size_t) co);
            add(q + "conv1.weight", ORC_TYPE_F16, (size_t) 7 * co * co);
            add(q + "conv1.bias", ORC_TYPE_F32, (size_t) co);
            add(q + "act2.alpha", ORC_TYPE_F32, (size_t) co);
            add(q + "act2.beta", ORC_TYPE_F32, (size_t) co);
            add(q + "conv2.weight", ORC_TYPE_F16, (size_t) co * co);
            add(q + "conv2.bias", ORC_TYPE_F32, (size_t) co);
        }
        ch = co;
    }
    add("tok_dec.dec.5.snake.alpha", ORC_TYPE_F32, (size_t) ch);
    add("tok_dec.dec.5.snake.beta", ORC_TYPE_F32, (size_t) ch);
    add("tok_dec.dec.6.conv.weight", ORC_TYPE_F16, (size_t) 7 * ch);
    add("tok_dec.dec.6.conv.bias", ORC_TYPE_F32, (size_t) 1);
    (void) hd;
    for (const Want & w : want) {
        const Tensor * x = m->get(w.name);
        if (!x) { m->err = "missing tensor " + w.name; return -1; }
        const size_t es = w.type == ORC_TYPE_F32 ? 4 : 2;
        if (x->type != w.type || x->nbytes != w.n * es) {
            m->err = "tensor " + w.name + ": unexpected type or size";
            return -1;
        }
    }
    m->cb.assign((size_t) c.n_codebooks, {});
    for (int i = 0; i < c.n_codebooks; ++i) {
        const std::string p = i == 0 ? "tok_dec.vq_first.0." : "tok_dec.vq_rest." + std::to_string(i - 1) + ".";
        const uint16_t * src = m->f16(p + "codebook");
        const float * u = m->f32(p + "usage");
        std::vector<uint16_t> & dst = m->cb[(size_t) i];
        dst.resize((size_t) c.codebook_size * c.codebook_dim);
        for (int e = 0; e < c.codebook_size; ++e) {
            float uu = u[e];
            if (uu < 1e-5f) uu = 1e-5f;
            const float inv = 1.0f / uu;
            for (int d = 0; d < c.codebook_dim; ++d) {
                const size_t at = (size_t) e * c.codebook_dim + d;
                dst[at] = orc_f32_to_f16(h2f(src[at]) * inv);
            }
        }
    }
    return 0;
}

// output_samples_for_frames (src/audio_tokenizer_decoder.cpp:845-875)
int64_t orc_voc_samples_for_frames(const orc_voc * m, int32_t n_frames) {
    if (n_frames <= 0) return 0;
    int64_t n = n_frames;
    for (int i = 0; i < 2; ++i) n = (n - 1) * 2 + m->cfg.up_kernel;
    for (int i = 0; i < 4; ++i) {
        const int64_t s = m->cfg.rates[i], k = m->cfg.dec_kernel[i];
        n = (n - 1) * s + k - 2 * (k - s);
    }
    return n > 0 ? n : 0;
}

// codes: [n_frames][n_codebooks]; positions pos0.. (decode_single's
// position_offset).  out: orc_voc_samples_for_frames(n_frames) floats.
// stage_out (optional): the latent after the VQ sum [n][hidden], for tests.
}  // extern "C"

namespace {

// The graph as a chain of stages, each a function of the previous stage's
// fp32 rows (the first of the codes): latent, pre_conv, input_proj,
// pre_tfm.<l>, output_proj (final RMSNorm + projection), upsample.<i>, dec.0,
// dec.<b>.conv_t (block snake + transposed conv), dec.<b>.res.<r>, dec.6
// (final snake + conv, before tanh).
std::vector<std::string> stage_names(const orc_voc_config & c) {
    std::vector<std::string> v = {"latent", "pre_conv", "input_proj"};
    for (int l = 0; l < c.n_layers; ++l) v.push_back("pre_tfm." + std::to_string(l));
    v.push_back("output_proj");
    v.push_back("upsample.0");
    v.push_back("upsample.1");
    v.push_back("dec.0");
    for (int b = 1; b <= 4; ++b) {
        v.push_back("dec." + std::to_string(b) + ".conv_t");
        for (int r = 2; r <= 4; ++r) v.push_back("dec." + std::to_string(b) + ".res." + std::to_string(r));
    }
    v.push_back("dec.6");
    return v;
}

// VQ: first + ((rest_0 + rest_1) + ... ) (src/audio_tokenizer_decoder.cpp:663-727)
Act stage_latent(const orc_voc * m, const int32_t * codes, int32_t n) {
    const orc_voc_config & c = m->cfg;
    Act lat(n, c.hidden);
    std::vector<Act> proj;
    for (int q = 0; q < c.n_codebooks; ++q) {
        Act e(n, c.codebook_dim);
        for (int f = 0; f < n; ++f) {
            const uint16_t * row = m->cb[(size_t) q].data() + (size_t) codes[(size_t) f * c.n_codebooks + q] * c.codebook_dim;
            for (int d = 0; d < c.codebook_dim; ++d) e.row(f)[d] = h2f(row[d]);
        }
        const char * wn = q == 0 ? "tok_dec.vq_first.output_proj.weight" : "tok_dec.vq_rest.output_proj.weight";
        proj.push_back(linear(m, e, m->f16(wn), nullptr, c.hidden));
    }
    for (int f = 0; f < n; ++f)
        for (int d = 0; d < c.hidden; ++d) {
            float r = proj[1].row(f)[d];
            for (int q = 2; q < c.n_codebooks; ++q) r = r + proj[(size_t) q].row(f)[d];
            lat.row(f)[d] = proj[0].row(f)[d] + r;
        }
    return lat;
}

// one stage after "latent"; returns false on an unknown name
bool run_stage(const orc_voc * m, const std::string & name, Act & x, int32_t pos0) {
    const orc_voc_config & c = m->cfg;
    static const int dil[3] = {1, 3, 9};
    if (name == "pre_conv") {
        x = conv1d(m, x, m->f16("tok_dec.pre_conv.weight"), m->f32("tok_dec.pre_conv.bias"), 3, c.latent, 1, 2);
    } else if (name == "input_proj") {
        x = linear(m, x, m->f16("tok_dec.pre_tfm.input_proj.weight"), m->f32("tok_dec.pre_tfm.input_proj.bias"), c.hidden);
    } else if (name.rfind("pre_tfm.", 0) == 0) {
        pre_tfm_layer(m, x, std::stoi(name.substr(8)), pos0);
    } else if (name == "output_proj") {
        rmsnorm_rows(x, m->f32("tok_dec.pre_tfm.norm.weight"), c.rms_eps);
        x = linear(m, x, m->f16("tok_dec.pre_tfm.output_proj.weight"), m->f32("tok_dec.pre_tfm.output_proj.bias"), c.latent);
    } else if (name.rfind("upsample.", 0) == 0) {
        x = upsample_block(m, x, std::stoi(name.substr(9)));
    } else if (name == "dec.0") {
        x = conv1d(m, x, m->f16("tok_dec.dec.0.conv.weight"), m->f32("tok_dec.dec.0.conv.bias"), 7, c.decoder_dim, 1, 6);
    } else if (name == "dec.6") {
        snake(x, m->f32("tok_dec.dec.5.snake.alpha"), m->f32("tok_dec.dec.5.snake.beta"));
        x = conv1d(m, x, m->f16("tok_dec.dec.6.conv.weight"), m->f32("tok_dec.dec.6.conv.bias"), 7, 1, 1, 6);
    } else if (name.size() > 6 && name.rfind("dec.", 0) == 0) {
        const int b = name[4] - '1';
        if (b < 0 || b > 3) return false;
        const std::string p = "tok_dec.dec." + std::to_string(b + 1) + ".";
        const int co = (int) x.C / 2;
        if (name.compare(5, std::string::npos, ".conv_t") == 0) {
            const int s = c.rates[b], K = conv_t_kernel(m, b);
            snake(x, m->f32(p + "snake.alpha"), m->f32(p + "snake.beta"));
            x = conv_t1d(m, x, m->f16(p + "conv_t.weight"), m->f32(p + "conv_t.bias"), K, co, s, K - s);
        } else if (name.compare(5, 5, ".res.") == 0) {
            const int r = std::stoi(name.substr(10)) - 2;
            if (r < 0 || r > 2) return false;
            const int C = (int) x.C;
            const std::string q = p + "res." + std::to_string(r + 2) + ".";
            Act h = x;
            snake(h, m->f32(q + "act1.alpha"), m->f32(q + "act1.beta"));
            h = conv1d(m, h, m->f16(q + "conv1.weight"), m->f32(q + "conv1.bias"), 7, C, dil[r], 6 * dil[r]);
            snake(h, m->f32(q + "act2.alpha"), m->f32(q + "act2.beta"));
            h = conv1d(m, h, m->f16(q + "conv2.weight"), m->f32(q + "conv2.bias"), 1, C, 1, 0);
            for (size_t i = 0; i < x.v.size(); ++i) x.v[i] = x.v[i] + h.v[i];
        } else {
            return false;
        }
    } else {
        return false;
    }
    return true;
}

bool codes_ok(orc_voc * m, const int32_t * codes, int64_t n) {
    for (int64_t i = 0; i < n * m->cfg.n_codebooks; ++i)
        if (codes[i] < 0 || codes[i] >= m->cfg.codebook_size) { m->err = "code out of range"; return false; }
    return true;
}

}  // namespace

extern "C" {

int orc_voc_decode_single(orc_voc * m, const int32_t * codes, int32_t n, int32_t pos0, float * out,
                          float * stage_out) {
    if (n <= 0) return 0;
    if (!codes_ok(m, codes, n)) return -1;
    m->stages.clear();
    Act x = stage_latent(m, codes, n);
    if (stage_out) std::memcpy(stage_out, x.v.data(), x.v.size() * 4);
    m->keep("latent", x);
    const std::vector<std::string> names = stage_names(m->cfg);
    for (size_t i = 1; i < names.size(); ++i) {
        run_stage(m, names[i], x, pos0);
        m->keep(names[i], x);
    }
    const int64_t ns = orc_voc_samples_for_frames(m, n);
    if (x.T != ns) { m->err = "internal: output length mismatch"; return -1; }
    for (int64_t i = 0; i < ns; ++i) out[i] = std::tanh(x.v[(size_t) i]);
    return 0;
}

// One named stage from given input rows in[T][C] (C is the stage's input
// width); "latent" reads codes instead ([T][n_codebooks] int32).  out gets
// [T_out][C_out] fp32.  Positions (pre_tfm.<l>) start at pos0.
int orc_voc_run_stage(orc_voc * m, const char * name, const float * in, const int32_t * codes, int64_t T,
                      int64_t C, int32_t pos0, float * out, int64_t cap, int64_t * T_out, int64_t * C_out) {
    Act x;
    if (std::string(name) == "latent") {
        if (!codes || !codes_ok(m, codes, T)) return -1;
        x = stage_latent(m, codes, (int32_t) T);
    } else {
        x = Act(T, C);
        std::memcpy(x.v.data(), in, (size_t) (T * C) * 4);
        if (!run_stage(m, name, x, pos0)) { m->err = std::string("unknown stage ") + name; return -1; }
    }
    *T_out = x.T;
    *C_out = x.C;
    if ((int64_t) x.v.size() > cap) { m->err = "run_stage: output buffer too small"; return -1; }
    std::memcpy(out, x.v.data(), x.v.size() * 4);
    return 0;
}

void orc_voc_set_record(orc_voc * m, int32_t on) {
    m->record = on != 0;
    m->stages.clear();
}

int32_t orc_voc_stage_count(const orc_voc * m) { return (int32_t) m->stages.size(); }

// stage `i` of the last decode_single with recording on: its name and [T][C]
// fp32 rows (out may be NULL to query T and C).
int orc_voc_stage(const orc_voc * m, int32_t i, char * name, int32_t name_cap, float * out, int64_t cap,
                  int64_t * T, int64_t * C) {
    if (i < 0 || i >= (int32_t) m->stages.size()) return -1;
    const auto & st = m->stages[(size_t) i];
    if (name && name_cap > 0) {
        std::strncpy(name, st.first.c_str(), (size_t) name_cap - 1);
        name[name_cap - 1] = 0;
    }
    *T = st.second.T;
    *C = st.second.C;
    if (out) {
        if ((int64_t) st.second.v.size() > cap) return -1;
        std::memcpy(out, st.second.v.data(), st.second.v.size() * 4);
    }
    return 0;
}

// decode_window (src/audio_tokenizer_decoder.cpp:946-980): decodes frames
// [max(0, start - context), end) at their absolute positions and returns the
// samples of [start, end).  *n_out = samples written (cap checked).
int orc_voc_decode_window(orc_voc * m, const int32_t * codes, int32_t n_frames, int32_t start, int32_t end,
                          int32_t context, float * out, int64_t cap, int64_t * n_out) {
    if (start < 0 || end <= start || end > n_frames) { m->err = "decode_window: invalid frame range"; return -1; }
    const int32_t ctx_start = std::max(0, start - std::max(0, context));
    const int32_t seg = end - ctx_start;
    std::vector<float> s((size_t) orc_voc_samples_for_frames(m, seg));
    if (orc_voc_decode_single(m, codes + (size_t) ctx_start * m->cfg.n_codebooks, seg, ctx_start, s.data(), nullptr))
        return -1;
    const int64_t drop = std::min<int64_t>(orc_voc_samples_for_frames(m, start - ctx_start), (int64_t) s.size());
    const int64_t keep = (int64_t) s.size() - drop;
    if (keep > cap) { m->err = "decode_window: output buffer too small"; return -1; }
    std::memcpy(out, s.data() + drop, (size_t) keep * 4);
    *n_out = keep;
    return 0;
}

}  // extern "C"
