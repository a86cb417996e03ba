// q3t_voc.hip -- device context and C ABI (include/q3t_voc.h) of the MI355X
// audio-tokenizer decoder.  Host code lays the GGUF tensors out for the
// kernels of q3t_voc_kernels.h, sizes the launches and moves data; every
// arithmetic step of a decode runs on the device.  No CPU fallback: without
// a HIP device q3t_voc_create fails.
//
// Graph (src/audio_tokenizer_decoder.cpp:636-843), as stages:
//   latent       VQ sum of 16 projected codebook rows          k_vq_sum
//   pre_conv     causal conv k3                                  GEMM, 3 taps
//   input_proj   linear                                          GEMM
//   pre_tfm.<l>  RMSNorm, QKV, RoPE, causal F32 attention, Wo * scale + x,
//                RMSNorm, gate/up + SwiGLU, down * scale + x       k_rms_h, GEMMs, k_rope_qk, k_attn_causal
//   output_proj  RMSNorm + linear                                k_rms_h, GEMM
//   upsample.<i> transposed conv (x2), depthwise k7 + LayerNorm, pwconv1 + GELU,
//                pwconv2 * gamma + y                             GEMM (2 phases), k_dwconv_ln, GEMMs
//   dec.0        causal conv k7                                  GEMM, 7 taps
//   dec.<b>      snake + transposed conv (stride s, kernel 2s, cropped), then
//                3 residual units snake/conv k7 (dilation 1,3,9)/snake/conv k1 + x
//                                                                GEMM (s phases x 2 taps), GEMMs
//   dec.6        snake + conv k7 to one channel + tanh            k_out_conv
// A stage's snake (or other input activation) runs in the epilogue of the
// GEMM that produced its input, so the fp16 conv input is written once.

#include "../../include/q3t_voc.h"
#include "q3t_voc_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

using namespace q3t;
using namespace q3t::voc;

namespace {

struct HostTensor {
    int32_t type = -1;
    std::vector<uint8_t> bytes;
};

// One GEMM's weights: [phases][Np][KT][Cp] fp16, zero-padded.
struct GemmW {
    uint16_t * w = nullptr;
    int32_t N = 0, Np = 0, KT = 1, Cp = 0, phases = 1, WM = 4;
};

struct Snake {
    float * ea = nullptr;    // e^alpha per channel
    float * eb = nullptr;    // e^-beta per channel
};

struct PreLayer {
    GemmW qkv, wo, gu, down;
    float * attn_norm = nullptr, * ffn_norm = nullptr, * attn_scale = nullptr, * ffn_scale = nullptr;
};

struct UpBlock {
    GemmW conv_t, pw1, pw2;
    float * conv_b = nullptr, * dw_b = nullptr, * norm_w = nullptr, * norm_b = nullptr, * pw1_b = nullptr,
          * pw2_b = nullptr, * gamma = nullptr;
    uint16_t * dw_w = nullptr;
};

struct ResUnit {
    Snake act1, act2;
    GemmW conv1, conv2;
    float * b1 = nullptr, * b2 = nullptr;
};

struct DecBlock {
    Snake snake;
    GemmW conv_t;
    float * conv_t_b = nullptr;
    ResUnit res[3];
};

int32_t rup(int32_t x, int32_t m) { return (x + m - 1) / m * m; }

// channel tile 32*WM with the least padding (ties: the larger tile)
int32_t pick_wm(int32_t N, bool even) {
    int best = 4;
    int32_t best_pad = rup(N, 128);
    for (int wm = 3; wm >= 1; --wm) {
        if (even && (wm & 1)) continue;
        const int32_t p = rup(N, 32 * wm);
        if (p < best_pad) { best = wm; best_pad = p; }
    }
    return best;
}

}  // namespace

struct q3t_voc {
    int32_t device = 0;
    hipStream_t stream = nullptr;
    q3t_voc_config cfg{};
    std::string err;
    std::map<std::string, HostTensor> host;
    std::vector<void *> allocs;
    bool ready = false;

    // weights
    float * vq_tab = nullptr;                     // [n_codebooks][size][hidden]
    GemmW pre_conv, in_proj, out_proj;
    float * pre_conv_b = nullptr, * in_proj_b = nullptr, * out_proj_b = nullptr, * final_norm = nullptr;
    std::vector<PreLayer> pre;
    UpBlock up[2];
    GemmW dec0;
    float * dec0_b = nullptr;
    DecBlock dec[4];
    Snake snake5;
    uint16_t * out_w = nullptr;                   // [Cp][7] fp16
    float out_b = 0.0f;
    float * rope_cos = nullptr, * rope_sin = nullptr;
    int32_t rope_n = 0;

    // buffers (sized for cap_frames)
    int32_t cap_frames = 0;
    float * xf = nullptr, * qkv = nullptr, * pre_out = nullptr, * audio = nullptr;
    uint16_t * h[2] = {nullptr, nullptr}, * mid = nullptr, * wide = nullptr, * hq = nullptr, * att = nullptr,
             * ffn = nullptr;
    int32_t * codes = nullptr;
    int32_t * bad = nullptr;
    int n_cu = 256;
    size_t xf_n = 0, h_n = 0, mid_n = 0, wide_n = 0, audio_n = 0;
};

namespace {

int fail(q3t_voc * v, const std::string & msg) { v->err = msg; return -1; }

#define HIP_OK(call)                                                                              \
    do {                                                                                          \
        hipError_t e_ = (call);                                                                   \
        if (e_ != hipSuccess) return fail(v, std::string(#call) + ": " + hipGetErrorString(e_)); \
    } while (0)

template <typename T>
int alloc(q3t_voc * v, T ** p, size_t count) {
    void * d = nullptr;
    HIP_OK(hipMalloc(&d, std::max<size_t>(count * sizeof(T), 256)));
    v->allocs.push_back(d);
    *p = (T *) d;
    return 0;
}

void release(q3t_voc * v, void * p) {
    if (!p) return;
    auto it = std::find(v->allocs.begin(), v->allocs.end(), p);
    if (it != v->allocs.end()) v->allocs.erase(it);
    (void) hipFree(p);
}

template <typename T>
int upload(q3t_voc * v, T ** p, const std::vector<T> & h) {
    if (alloc(v, p, h.size())) return -1;
    HIP_OK(hipMemcpy(*p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice));
    return 0;
}

const HostTensor * get(q3t_voc * v, const std::string & name) {
    auto it = v->host.find(name);
    return it == v->host.end() ? nullptr : &it->second;
}
const uint16_t * f16(q3t_voc * v, const std::string & n) { return (const uint16_t *) get(v, n)->bytes.data(); }
const float * f32(q3t_voc * v, const std::string & n) { return (const float *) get(v, n)->bytes.data(); }

int upload_f32(q3t_voc * v, float ** p, const std::string & name) {
    const HostTensor * t = get(v, name);
    std::vector<float> h(t->bytes.size() / 4);
    std::memcpy(h.data(), t->bytes.data(), t->bytes.size());
    return upload(v, p, h);
}

int upload_snake(q3t_voc * v, Snake & s, const std::string & prefix) {
    const HostTensor * a = get(v, prefix + "alpha");
    const size_t n = a->bytes.size() / 4;
    const float * al = f32(v, prefix + "alpha"), * be = f32(v, prefix + "beta");
    std::vector<float> ea(n), eb(n);
    for (size_t i = 0; i < n; ++i) {
        ea[i] = std::exp(al[i]);
        eb[i] = std::exp(be[i] * -1.0f);
    }
    return upload(v, &s.ea, ea) || upload(v, &s.eb, eb) ? -1 : 0;
}

// Builds [phases][Np][KT][Cp] from a fetch(phase, n, tap, c) of the source.
template <typename F>
int build_gemm(q3t_voc * v, GemmW & g, int32_t N, int32_t KT, int32_t C, int32_t phases, bool even, F fetch) {
    g.N = N;
    g.KT = KT;
    g.Cp = rup(C, 32);
    g.phases = phases;
    g.WM = pick_wm(N, even);
    g.Np = rup(N, 32 * g.WM);
    std::vector<uint16_t> h((size_t) phases * g.Np * KT * g.Cp, 0);
    for (int p = 0; p < phases; ++p)
        for (int n = 0; n < N; ++n)
            for (int k = 0; k < KT; ++k) {
                uint16_t * dst = h.data() + (((size_t) p * g.Np + n) * KT + k) * g.Cp;
                for (int c = 0; c < C; ++c) dst[c] = fetch(p, n, k, c);
            }
    return upload(v, &g.w, h);
}

// linear: ggml ne (K, N) = rows [n][k]
int build_linear(q3t_voc * v, GemmW & g, const uint16_t * w, int32_t K, int32_t N) {
    return build_gemm(v, g, N, 1, K, 1, false, [&](int, int n, int, int c) { return w[(size_t) n * K + c]; });
}

// conv1d: ggml ne (K, Ci, Co) = [o][i][k]
int build_conv(q3t_voc * v, GemmW & g, const uint16_t * w, int32_t K, int32_t Ci, int32_t Co) {
    return build_gemm(v, g, Co, K, Ci, 1, false,
                      [&](int, int o, int k, int i) { return w[((size_t) o * Ci + i) * K + k]; });
}

std::vector<std::string> stage_names(const q3t_voc_config & c) {
    std::vector<std::string> s = {"latent", "pre_conv", "input_proj"};
    for (int l = 0; l < c.n_layers; ++l) s.push_back("pre_tfm." + std::to_string(l));
    s.push_back("output_proj");
    s.push_back("upsample.0");
    s.push_back("upsample.1");
    s.push_back("dec.0");
    for (int b = 1; b <= 4; ++b) {
        s.push_back("dec." + std::to_string(b) + ".conv_t");
        for (int r = 2; r <= 4; ++r) s.push_back("dec." + std::to_string(b) + ".res." + std::to_string(r));
    }
    s.push_back("dec.6");
    return s;
}

int64_t samples_for(const q3t_voc_config & c, int64_t n) {
    if (n <= 0) return 0;
    for (int i = 0; i < 2; ++i) n = (n - 1) * 2 + c.up_kernel;
    for (int i = 0; i < 4; ++i) n = (n - 1) * c.rates[i] + c.dec_kernel[i] - 2 * (c.dec_kernel[i] - c.rates[i]);
    return n > 0 ? n : 0;
}

// rows and width of each stage's output for an n-frame segment
struct Shape { int64_t rows; int32_t ch; };

Shape stage_shape(const q3t_voc_config & c, const std::string & name, int64_t n) {
    if (name == "latent" || name == "input_proj" || name.rfind("pre_tfm.", 0) == 0) return {n, c.hidden};
    if (name == "pre_conv" || name == "output_proj") return {n, c.latent};
    if (name == "upsample.0") return {(n - 1) * 2 + c.up_kernel, c.latent};
    int64_t r = (n - 1) * 2 + c.up_kernel;
    r = (r - 1) * 2 + c.up_kernel;
    if (name == "upsample.1") return {r, c.latent};
    if (name == "dec.0") return {r, c.decoder_dim};
    int32_t ch = c.decoder_dim;
    for (int b = 1; b <= 4; ++b) {
        r = (r - 1) * c.rates[b - 1];
        ch /= 2;
        if (name.rfind("dec." + std::to_string(b) + ".", 0) == 0) return {r, ch};
    }
    return {r, 1};                                          // dec.6
}

// ---------------------------------------------------------------- launches
int gemm(q3t_voc * v, const GemmW & W, const uint16_t * x, int32_t xs, int32_t rows_in, int32_t off0, int32_t dil,
         int32_t M, int32_t ostride, const float * bias, const float * scale, const float * res, int32_t rs,
         float * yf, int32_t yfs, uint16_t * yh, int32_t yhs, int32_t act, const Snake * sn) {
    if (M <= 0) return 0;
    if (xs % 8 || xs < W.Cp) return fail(v, "internal: GEMM input stride");
    // the kernels address outputs and residuals with 32-bit element offsets
    // and read inputs and weights through 32-bit buffer ranges
    if ((int64_t) M * ostride * std::max({yfs, yhs, rs, W.N}) >= ((int64_t) 1 << 31) ||
        (int64_t) rows_in * xs * 2 >= ((int64_t) 1 << 31) ||
        (int64_t) W.Np * W.KT * W.Cp * 2 >= ((int64_t) 1 << 31))
        return fail(v, "decode segment too long: a vocoder layer exceeds 2^31 elements");
    ConvArgs a{};
    a.x = x; a.xs = xs; a.rows_in = rows_in;
    a.w = W.w; a.Cp = W.Cp; a.KT = W.KT; a.dil = dil; a.off0 = off0;
    a.M = M; a.N = W.N; a.Np = W.Np; a.ostride = ostride;
    a.bias = bias; a.scale = scale; a.res = res; a.rs = rs;
    a.yf = yf; a.yfs = yfs; a.yh = yh; a.yhs = yhs;
    a.act = act;
    a.ea = sn ? sn->ea : nullptr;
    a.eb = sn ? sn->eb : nullptr;
    // tile: the largest (32 WM channels x 32 WN rows per workgroup, WN at
    // most 2: measured faster than 4 over a streaming window, 3.13 against
    // 3.51 ms) that still gives the launch a workgroup per CU; a smaller WM
    // divides the weights' padded width (SwiGLU pairs need WM even).
    // Q3T_VOC_WN=1/2/4 sets the largest WN.
    static const int wn_max = [] {
        const char * e = std::getenv("Q3T_VOC_WN");
        const int v = e ? std::atoi(e) : 2;
        return v == 1 || v == 4 ? v : 2;
    }();
    int WM = W.WM, WN = wn_max;
    auto wgs = [&](int wm, int wn) {
        return (int64_t) (W.Np / (32 * wm)) * ((M + 32 * wn - 1) / (32 * wn)) * W.phases;
    };
    while (wgs(WM, WN) < v->n_cu) {
        if (WN > 1) WN >>= 1;
        else if (WM == 4) WM = 2;
        else if ((WM == 2 || WM == 3) && act != ACT_SWIGLU) WM = 1;
        else break;
    }
    const dim3 grid((unsigned) (W.Np / (32 * WM)), (unsigned) ((M + 32 * WN - 1) / (32 * WN)), (unsigned) W.phases);
    // a launch that cannot fill the CUs (the 73-row pre-transformer GEMMs)
    // stages 4 K chunks per step: a quarter of the serial load-and-barrier
    // round trips of its K loop
    // (and any launch over at most 128 rows: the pre-transformer's Q/K/V
    // GEMM fills the CUs with 288 workgroups but its 16-step K loop over 73
    // rows is the same chain; 1.891-1.898 -> 1.871-1.877 ms per window)
    const bool ks4 = (wgs(WM, WN) < v->n_cu || M <= 128) && WN == 1 && WM <= 2 && W.KT * (W.Cp / 32) >= 8;
    if (ks4) {
        if (WM == 2) hipLaunchKernelGGL((k_conv_gemm<2, 1, 4>), grid, dim3(kGemmT), 0, v->stream, a);
        else hipLaunchKernelGGL((k_conv_gemm<1, 1, 4>), grid, dim3(kGemmT), 0, v->stream, a);
        HIP_OK(hipGetLastError());
        return 0;
    }
    // a residual input takes the form that prefetches it in the epilogue; a
    // contraction of 64 or more 32-element chunks (the k7 convolutions of the
    // 768- and 384-channel decoder blocks: 168 and 84) stages two chunks per
    // K step (2.92-2.97 -> 2.83 ms per 73-frame window; four per step and two
    // from 32 chunks measured no better)
    static const int deep_ks = [] {
        const char * e = std::getenv("Q3T_VOC_DEEPKS");
        return e ? std::atoi(e) : 2;
    }();
    const bool deep = W.KT * (W.Cp / 32) >= 64 && deep_ks == 2;
    // a deep contraction on the narrowest tile (the upsampler's 4096-deep
    // pwconv2 over 146 rows, narrowed to fill the CUs) stages four chunks per
    // step: its 128-chunk K loop is a chain of load round trips (2.72 -> 2.68
    // ms per window; eight per step no better)
    if (W.KT * (W.Cp / 32) >= 64 && WM == 1 && WN == 1 && deep_ks != 1) {
        hipLaunchKernelGGL((k_conv_gemm<1, 1, 4>), grid, dim3(kGemmT), 0, v->stream, a);
        HIP_OK(hipGetLastError());
        return 0;
    }
#define Q3T_VOC_GEMM(wm, wn)                                                                             \
    do {                                                                                                 \
        if (res) hipLaunchKernelGGL((k_conv_gemm<wm, wn, 1, true>), grid, dim3(kGemmT), 0, v->stream, a); \
        else if (deep) hipLaunchKernelGGL((k_conv_gemm<wm, wn, 2>), grid, dim3(kGemmT), 0, v->stream, a); \
        else hipLaunchKernelGGL((k_conv_gemm<wm, wn>), grid, dim3(kGemmT), 0, v->stream, a);             \
    } while (0)
#define Q3T_VOC_GEMM_WN(wm)                   \
    switch (WN) {                             \
    case 4: Q3T_VOC_GEMM(wm, 4); break;       \
    case 2: Q3T_VOC_GEMM(wm, 2); break;       \
    default: Q3T_VOC_GEMM(wm, 1); break;      \
    }
    switch (WM) {
    case 4: Q3T_VOC_GEMM_WN(4); break;
    case 3: Q3T_VOC_GEMM_WN(3); break;
    case 2: Q3T_VOC_GEMM_WN(2); break;
    default: Q3T_VOC_GEMM_WN(1); break;
    }
#undef Q3T_VOC_GEMM_WN
#undef Q3T_VOC_GEMM
    HIP_OK(hipGetLastError());
    return 0;
}

int prep(q3t_voc * v, const float * x, int32_t xs, int64_t T, int32_t C, int32_t act, const Snake * sn,
         uint16_t * yh, int32_t yhs) {
    const int64_t n = T * C;
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_prep, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, v->stream, x, xs, (int32_t) T, C, act,
                       sn ? sn->ea : nullptr, sn ? sn->eb : nullptr, yh, yhs);
    HIP_OK(hipGetLastError());
    return 0;
}

int rms(q3t_voc * v, const float * x, int32_t xs, int64_t T, int32_t C, const float * w, uint16_t * y, int32_t ys) {
    hipLaunchKernelGGL(k_rms_h, dim3((unsigned) ((T + 3) / 4)), dim3(256), 0, v->stream, x, xs, (int32_t) T, C, w,
                       v->cfg.rms_eps, y, ys);
    HIP_OK(hipGetLastError());
    return 0;
}

// zero the pad channels of an fp16 layout whose width is not a multiple of 32
int clear_pad(q3t_voc * v, uint16_t * p, int64_t rows, int32_t C) {
    if (C % 32 == 0 || rows <= 0) return 0;
    HIP_OK(hipMemsetAsync(p, 0, (size_t) rows * rup(C, 32) * 2, v->stream));
    return 0;
}

int rope_table(q3t_voc * v, int32_t need) {
    if (need <= v->rope_n) return 0;
    const int32_t n = std::max(need, 8192);
    const int32_t hd = v->cfg.latent / v->cfg.n_heads, half = hd / 2;
    std::vector<float> cs((size_t) n * half), sn((size_t) n * half);
    // ggml_rope_cache_init: theta_i = pos * base^(-2i/hd) by cumulative fp32 product
    const float theta_scale = std::pow(v->cfg.rope_theta, -2.0f / (float) hd);
    for (int32_t p = 0; p < n; ++p) {
        float theta = (float) p;
        for (int i = 0; i < half; ++i) {
            cs[(size_t) p * half + i] = std::cos(theta);
            sn[(size_t) p * half + i] = std::sin(theta);
            theta *= theta_scale;
        }
    }
    release(v, v->rope_cos);
    release(v, v->rope_sin);
    v->rope_cos = v->rope_sin = nullptr;
    if (upload(v, &v->rope_cos, cs) || upload(v, &v->rope_sin, sn)) return -1;
    v->rope_n = n;
    return 0;
}

// The input activation each stage applies to the previous stage's rows
// before its first product (fused into the producer's epilogue).
struct InAct { int32_t act; const Snake * sn; };

InAct input_act(q3t_voc * v, const std::string & name) {
    if (name == "dec.6") return {ACT_SNAKE, &v->snake5};
    if (name.size() > 6 && name.rfind("dec.", 0) == 0 && name != "dec.0") {
        const int b = name[4] - '1';
        if (name.compare(5, std::string::npos, ".conv_t") == 0) return {ACT_SNAKE, &v->dec[b].snake};
        const int r = name.back() - '2';
        return {ACT_SNAKE, &v->dec[b].res[r].act1};
    }
    return {ACT_NONE, nullptr};
}

// Buffers for an n-frame segment.
int reserve(q3t_voc * v, int32_t n) {
    if (n <= v->cap_frames) return 0;
    const q3t_voc_config & c = v->cfg;
    size_t xf = 0, hn = 0, mid = 0;
    for (const std::string & s : stage_names(c)) {
        const Shape sh = stage_shape(c, s, n);
        xf = std::max(xf, (size_t) sh.rows * rup(sh.ch, 32));
        hn = std::max(hn, (size_t) sh.rows * rup(sh.ch, 32));
    }
    // transposed-conv outputs can hold more rows than the stage output (upsample)
    mid = std::max(hn, (size_t) stage_shape(c, "upsample.1", n).rows * rup(c.latent, 32));
    const size_t wide = (size_t) stage_shape(c, "upsample.1", n).rows * rup(c.cnx_ffn, 32);
    const size_t audio = (size_t) samples_for(c, n) + 64;
    for (void * p : {(void *) v->xf, (void *) v->qkv, (void *) v->pre_out, (void *) v->audio, (void *) v->h[0],
                     (void *) v->h[1], (void *) v->mid, (void *) v->wide, (void *) v->hq, (void *) v->att,
                     (void *) v->ffn, (void *) v->codes})
        release(v, p);
    const int32_t L = rup(c.latent, 32), H = rup(c.hidden, 32), F = rup(c.ffn, 32);
    int rc = 0;
    rc |= alloc(v, &v->xf, xf);
    rc |= alloc(v, &v->qkv, (size_t) n * 3 * c.latent);
    rc |= alloc(v, &v->pre_out, audio);
    rc |= alloc(v, &v->audio, audio);
    rc |= alloc(v, &v->h[0], hn);
    rc |= alloc(v, &v->h[1], hn);
    rc |= alloc(v, &v->mid, mid);
    rc |= alloc(v, &v->wide, wide);
    rc |= alloc(v, &v->hq, (size_t) n * std::max(H, L));
    rc |= alloc(v, &v->att, (size_t) n * L);
    rc |= alloc(v, &v->ffn, (size_t) n * F);
    rc |= alloc(v, &v->codes, (size_t) n * c.n_codebooks);
    if (rc) return -1;
    HIP_OK(hipMemset(v->h[0], 0, hn * 2));
    HIP_OK(hipMemset(v->h[1], 0, hn * 2));
    HIP_OK(hipMemset(v->mid, 0, mid * 2));
    HIP_OK(hipMemset(v->hq, 0, (size_t) n * std::max(H, L) * 2));
    HIP_OK(hipMemset(v->att, 0, (size_t) n * L * 2));
    HIP_OK(hipMemset(v->ffn, 0, (size_t) n * F * 2));
    v->xf_n = xf; v->h_n = hn; v->mid_n = mid; v->wide_n = wide; v->audio_n = audio;
    v->cap_frames = n;
    return 0;
}

// --------------------------------------------------------------- stages
// Every stage reads rows of T = its input row count: xf (fp32, stride Cp of
// the input width) and/or hin (fp16 act(x), same stride), and leaves its
// output in xf (when yf is wanted or the next stage reads fp32) and hout
// (fp16 nx(y) with nx the next stage's input activation).
struct Io {
    uint16_t * hin, * hout;
    bool want_f32;          // the caller reads the fp32 output in xf
    InAct nx;
};

int st_pre_conv(q3t_voc * v, int64_t n, const Io & io) {
    const int32_t H = rup(v->cfg.hidden, 32), L = rup(v->cfg.latent, 32);
    if (clear_pad(v, io.hout, n, v->cfg.latent)) return -1;
    return gemm(v, v->pre_conv, io.hin, H, (int32_t) n, -2, 1, (int32_t) n, 1, v->pre_conv_b, nullptr, nullptr, 0,
                io.want_f32 ? v->xf : nullptr, L, io.hout, L, io.nx.act, io.nx.sn);
}

int st_input_proj(q3t_voc * v, int64_t n, const Io & io) {
    const int32_t H = rup(v->cfg.hidden, 32), L = rup(v->cfg.latent, 32);
    return gemm(v, v->in_proj, io.hin, L, (int32_t) n, 0, 1, (int32_t) n, 1, v->in_proj_b, nullptr, nullptr, 0,
                v->xf, H, nullptr, 0, ACT_NONE, nullptr);
}

int st_pre_tfm(q3t_voc * v, int l, int64_t n, int32_t pos0) {
    const q3t_voc_config & c = v->cfg;
    const PreLayer & P = v->pre[(size_t) l];
    const int32_t H = rup(c.hidden, 32), L = rup(c.latent, 32), F = rup(c.ffn, 32), Q = 3 * c.latent;
    const int32_t hd = c.latent / c.n_heads;
    if (n > 32768) return fail(v, "decoder window longer than 32768 frames");
    if (rope_table(v, pos0 + (int32_t) n)) return -1;
    if (rms(v, v->xf, H, n, c.hidden, P.attn_norm, v->hq, H)) return -1;
    if (gemm(v, P.qkv, v->hq, H, (int32_t) n, 0, 1, (int32_t) n, 1, nullptr, nullptr, nullptr, 0, v->qkv, Q,
             nullptr, 0, ACT_NONE, nullptr))
        return -1;
    const int64_t nr = n * 2 * (c.latent / hd) * (hd / 2);
    hipLaunchKernelGGL(k_rope_qk, dim3((unsigned) ((nr + 255) / 256)), dim3(256), 0, v->stream, v->qkv, Q, (int32_t) n,
                       c.latent, hd, v->rope_cos, v->rope_sin, pos0);
    HIP_OK(hipGetLastError());
    // windows whose K and V rows fit in LDS take the staged kernel (4 query
    // rows per workgroup, head widths 32 and 64); longer decodes the
    // one-wave-per-row kernel
    const size_t lds = ((size_t) 2 * n * hd + (size_t) 4 * hd + (size_t) 4 * n) * 4;
    const dim3 sg((unsigned) ((n + 3) / 4), (unsigned) c.n_heads);
    const float asc = 1.0f / std::sqrt((float) hd);
    if (lds <= 65536 && hd == 64)
        hipLaunchKernelGGL(k_attn_causal_lds<64>, sg, dim3(256), lds, v->stream, v->qkv, Q, c.latent, (int32_t) n, asc,
                           v->att, L);
    else if (lds <= 65536 && hd == 32)
        hipLaunchKernelGGL(k_attn_causal_lds<32>, sg, dim3(256), lds, v->stream, v->qkv, Q, c.latent, (int32_t) n, asc,
                           v->att, L);
    else
        hipLaunchKernelGGL(k_attn_causal, dim3((unsigned) n, (unsigned) c.n_heads), dim3(64), (size_t) n * 4, v->stream,
                           v->qkv, Q, c.latent, hd, 1.0f / std::sqrt((float) hd), v->att, L);
    HIP_OK(hipGetLastError());
    if (gemm(v, P.wo, v->att, L, (int32_t) n, 0, 1, (int32_t) n, 1, nullptr, P.attn_scale, v->xf, H, v->xf, H,
             nullptr, 0, ACT_NONE, nullptr))
        return -1;
    if (rms(v, v->xf, H, n, c.hidden, P.ffn_norm, v->hq, H)) return -1;
    if (gemm(v, P.gu, v->hq, H, (int32_t) n, 0, 1, (int32_t) n, 1, nullptr, nullptr, nullptr, 0, nullptr, 0, v->ffn,
             F, ACT_SWIGLU, nullptr))
        return -1;
    return gemm(v, P.down, v->ffn, F, (int32_t) n, 0, 1, (int32_t) n, 1, nullptr, P.ffn_scale, v->xf, H, v->xf, H,
                nullptr, 0, ACT_NONE, nullptr);
}

int st_output_proj(q3t_voc * v, int64_t n, const Io & io) {
    const q3t_voc_config & c = v->cfg;
    const int32_t H = rup(c.hidden, 32), L = rup(c.latent, 32);
    if (rms(v, v->xf, H, n, c.hidden, v->final_norm, v->hq, H)) return -1;
    if (clear_pad(v, io.hout, n, c.latent)) return -1;
    return gemm(v, v->out_proj, v->hq, H, (int32_t) n, 0, 1, (int32_t) n, 1, v->out_proj_b, nullptr, nullptr, 0,
                io.want_f32 ? v->xf : nullptr, L, io.hout, L, io.nx.act, io.nx.sn);
}

int st_upsample(q3t_voc * v, int i, int64_t T, const Io & io) {
    const q3t_voc_config & c = v->cfg;
    const UpBlock & U = v->up[i];
    const int32_t L = rup(c.latent, 32), W = rup(c.cnx_ffn, 32);
    const int64_t R = (T - 1) * 2 + c.up_kernel;           // = 2T (kernel 2)
    // y = conv_t(x) + b (fp32: the block's residual and the dwconv input)
    if (gemm(v, U.conv_t, io.hin, L, (int32_t) T, 0, 1, (int32_t) T, 2, U.conv_b, nullptr, nullptr, 0, v->xf, L,
             nullptr, 0, ACT_NONE, nullptr))
        return -1;
    if (clear_pad(v, v->mid, R, c.latent)) return -1;
    hipLaunchKernelGGL(k_dwconv_ln, dim3((unsigned) R), dim3(256), (size_t) c.latent * 4, v->stream, v->xf, L,
                       (int32_t) R, c.latent, U.dw_w, U.dw_b, U.norm_w, U.norm_b, v->mid, L);
    HIP_OK(hipGetLastError());
    if (clear_pad(v, v->wide, R, c.cnx_ffn)) return -1;
    if (gemm(v, U.pw1, v->mid, L, (int32_t) R, 0, 1, (int32_t) R, 1, U.pw1_b, nullptr, nullptr, 0, nullptr, 0, v->wide,
             W, ACT_GELU, nullptr))
        return -1;
    if (clear_pad(v, io.hout, R, c.latent)) return -1;
    return gemm(v, U.pw2, v->wide, W, (int32_t) R, 0, 1, (int32_t) R, 1, U.pw2_b, U.gamma, v->xf, L,
                io.want_f32 ? v->xf : nullptr, L, io.hout, L, io.nx.act, io.nx.sn);
}

int st_dec0(q3t_voc * v, int64_t T, const Io & io) {
    const q3t_voc_config & c = v->cfg;
    const int32_t L = rup(c.latent, 32), D = rup(c.decoder_dim, 32);
    if (clear_pad(v, io.hout, T, c.decoder_dim)) return -1;
    return gemm(v, v->dec0, io.hin, L, (int32_t) T, -6, 1, (int32_t) T, 1, v->dec0_b, nullptr, nullptr, 0,
                io.want_f32 ? v->xf : nullptr, D, io.hout, D, io.nx.act, io.nx.sn);
}

// snake (in hin) + transposed conv: out rows (T - 1) * s, phase p of row
// m*s + p = x[m] . W[p + s] + x[m + 1] . W[p]
int st_conv_t(q3t_voc * v, int b, int64_t T, const Io & io) {
    const DecBlock & B = v->dec[b];
    const int32_t s = v->cfg.rates[b], Ci = rup(B.conv_t.Cp, 32), Co = rup(B.conv_t.N, 32);
    if (clear_pad(v, io.hout, (T - 1) * s, B.conv_t.N)) return -1;
    return gemm(v, B.conv_t, io.hin, Ci, (int32_t) T, 0, 1, (int32_t) (T - 1), s, B.conv_t_b, nullptr, nullptr, 0,
                v->xf, Co, io.hout, Co, io.nx.act, io.nx.sn);
}

// A residual unit of 96 or 192 channels over at least kFuseRows rows in one
// launch (k_conv_gemm<WM, 2, 1, false, true>, one channel tile of 32 WM = C,
// 64-row tiles): the decoder blocks at the 192- and 96-channel widths.
// Q3T_VOC_FUSE=0 runs the two convolutions as separate launches.  Returns 1
// when the unit does not qualify, else 0 or the launch's error.
constexpr int64_t kFuseRows = 1024;

int res_fused(q3t_voc * v, const ResUnit & U, int64_t T, int32_t d, const Io & io, bool last) {
    static const bool off = [] {
        const char * e = std::getenv("Q3T_VOC_FUSE");
        return e && std::strcmp(e, "0") == 0;
    }();
    const int32_t C = U.conv1.N;
    if (off || T < kFuseRows || (C != 96 && C != 192) || U.conv1.Cp != C || U.conv1.Np != C || U.conv1.KT != 7 ||
        U.conv2.Cp != C || U.conv2.Np != C || U.conv2.N != C || U.conv2.KT != 1)
        return 1;
    if (T * C * 4 >= ((int64_t) 1 << 31)) return fail(v, "decode segment too long: a vocoder layer exceeds 2^31 elements");
    ConvArgs a{};
    a.x = io.hin; a.xs = C; a.rows_in = (int32_t) T;
    a.w = U.conv1.w; a.Cp = C; a.KT = 7; a.dil = d; a.off0 = -6 * d;
    a.M = (int32_t) T; a.N = C; a.Np = C; a.ostride = 1;
    a.bias = U.b1; a.act = ACT_SNAKE; a.ea = U.act2.ea; a.eb = U.act2.eb;
    a.w2 = U.conv2.w; a.bias2 = U.b2; a.act2 = io.nx.act;
    a.ea2 = io.nx.sn ? io.nx.sn->ea : nullptr;
    a.eb2 = io.nx.sn ? io.nx.sn->eb : nullptr;
    a.res = v->xf; a.rs = C;
    a.yf = (!last || io.want_f32) ? v->xf : nullptr; a.yfs = C;
    a.yh = io.hout; a.yhs = C;
    const dim3 grid(1, (unsigned) ((T + 63) / 64), 1);
    if (C == 96) hipLaunchKernelGGL((k_conv_gemm<3, 2, 1, false, true>), grid, dim3(kGemmT), 0, v->stream, a);
    else hipLaunchKernelGGL((k_conv_gemm<6, 2, 1, false, true>), grid, dim3(kGemmT), 0, v->stream, a);
    HIP_OK(hipGetLastError());
    return 0;
}

// residual unit r: x + conv2(snake2(conv1(snake1(x)))) with snake1(x) in hin
int st_res(q3t_voc * v, int b, int r, int64_t T, const Io & io, bool last) {
    const ResUnit & U = v->dec[b].res[r];
    const int32_t C = U.conv1.N, Cp = rup(C, 32), d = r == 0 ? 1 : r == 1 ? 3 : 9;
    if (const int rc = res_fused(v, U, T, d, io, last); rc <= 0) return rc;
    if (clear_pad(v, v->mid, T, C)) return -1;
    if (gemm(v, U.conv1, io.hin, Cp, (int32_t) T, -6 * d, d, (int32_t) T, 1, U.b1, nullptr, nullptr, 0, nullptr, 0,
             v->mid, Cp, ACT_SNAKE, &U.act2))
        return -1;
    if (clear_pad(v, io.hout, T, C)) return -1;
    return gemm(v, U.conv2, v->mid, Cp, (int32_t) T, 0, 1, (int32_t) T, 1, U.b2, nullptr, v->xf, Cp,
                (!last || io.want_f32) ? v->xf : nullptr, Cp, io.hout, Cp, io.nx.act, io.nx.sn);
}

int st_out(q3t_voc * v, int64_t T, const uint16_t * hin, float * pre, int64_t drop) {
    const int32_t C = rup(v->cfg.decoder_dim >> 4, 32);
    // up to 96 channels: the rows staged in LDS per 256 samples
    if (C <= kOutMaxC)
        hipLaunchKernelGGL(k_out_conv_lds, dim3((unsigned) ((T + 255) / 256)), dim3(256), 0, v->stream, hin, C,
                           (int32_t) T, C, v->out_w, v->out_b, pre, v->audio, drop);
    else
        hipLaunchKernelGGL(k_out_conv, dim3((unsigned) ((T + 255) / 256)), dim3(256), 0, v->stream, hin, C, (int32_t) T,
                           C, v->out_w, v->out_b, pre, v->audio, drop);
    HIP_OK(hipGetLastError());
    return 0;
}

// Runs stages [first, last] of the chain over an n-frame segment starting at
// position pos0; the input of `first` is already in place (xf and/or
// h[cur]).  want_f32: the last stage leaves its fp32 output in xf (or, for
// dec.6, pre_out).  drop: samples of dec.6 skipped at the start of audio.
int run_chain(q3t_voc * v, const std::vector<std::string> & names, size_t first, size_t last, int64_t n,
              int32_t pos0, int & cur, bool want_f32, int64_t drop) {
    const q3t_voc_config & c = v->cfg;
    for (size_t si = first; si <= last; ++si) {
        const std::string & s = names[si];
        const bool is_last = si == last;
        Io io{v->h[cur], v->h[cur ^ 1], is_last && want_f32,
              is_last ? InAct{ACT_NONE, nullptr} : input_act(v, names[si + 1])};
        int64_t T = si == 0 ? n : stage_shape(c, names[si - 1], n).rows;
        int rc = 0;
        bool flips = true;
        if (s == "latent") {
            flips = false;                        // handled by the caller (k_vq_sum)
        } else if (s == "pre_conv") {
            rc = st_pre_conv(v, T, io);
        } else if (s == "input_proj") {
            rc = st_input_proj(v, T, io);
            flips = false;
        } else if (s.rfind("pre_tfm.", 0) == 0) {
            rc = st_pre_tfm(v, std::stoi(s.substr(8)), T, pos0);
            flips = false;
        } else if (s == "output_proj") {
            rc = st_output_proj(v, T, io);
        } else if (s.rfind("upsample.", 0) == 0) {
            rc = st_upsample(v, s[9] - '0', T, io);
        } else if (s == "dec.0") {
            rc = st_dec0(v, T, io);
        } else if (s == "dec.6") {
            rc = st_out(v, T, io.hin, want_f32 ? v->pre_out : nullptr, drop);
            flips = false;
        } else {
            const int b = s[4] - '1';
            if (s.compare(5, std::string::npos, ".conv_t") == 0) rc = st_conv_t(v, b, T, io);
            else rc = st_res(v, b, s.back() - '2', T, io, s.back() == '4');
        }
        if (rc) return -1;
        if (flips) cur ^= 1;
    }
    return 0;
}

int vq(q3t_voc * v, const int32_t * codes_dev, int64_t n, uint16_t * hout) {
    const q3t_voc_config & c = v->cfg;
    if (clear_pad(v, hout, n, c.hidden)) return -1;
    HIP_OK(hipMemsetAsync(v->bad, 0, 4, v->stream));
    // a workgroup per 256 elements of a frame: one element per thread
    hipLaunchKernelGGL(k_vq_sum, dim3((unsigned) n, (unsigned) ((c.hidden + 255) / 256)), dim3(256), 0, v->stream,
                       codes_dev, c.n_codebooks, (int32_t) n,
                       v->vq_tab, c.codebook_size, c.hidden, v->xf, rup(c.hidden, 32), hout, rup(c.hidden, 32), v->bad);
    HIP_OK(hipGetLastError());
    return 0;
}

int check_bad(q3t_voc * v) {
    int32_t bad = 0;
    HIP_OK(hipMemcpyAsync(&bad, v->bad, 4, hipMemcpyDeviceToHost, v->stream));
    HIP_OK(hipStreamSynchronize(v->stream));
    if (bad) return fail(v, "code out of range");
    return 0;
}

}  // namespace

// ================================================================= C ABI
extern "C" {

q3t_voc * q3t_voc_create(const q3t_voc_config * cfg, int32_t device, const char ** err_out) {
    static std::string last;
    auto bad = [&](const std::string & m) -> q3t_voc * {
        last = m;
        if (err_out) *err_out = last.c_str();
        return nullptr;
    };
    if (!cfg) return bad("config is null");
    const q3t_voc_config & c = *cfg;
    if (c.n_codebooks < 2 || c.codebook_size < 1 || c.codebook_dim < 1 || c.hidden < 1 || c.latent < 1 ||
        c.n_layers < 0 || c.n_heads < 1 || c.ffn < 1 || c.cnx_ffn < 1 || c.decoder_dim < 16)
        return bad("invalid decoder widths");
    if (c.latent % c.n_heads || c.latent / c.n_heads > 64 || (c.latent / c.n_heads) % 2)
        return bad("head_dim must be even and at most 64");
    if (c.up_kernel != 2) return bad("upsample transposed-conv kernel must be 2 (stride 2)");
    for (int i = 0; i < 4; ++i)
        if (c.rates[i] < 1 || c.dec_kernel[i] != 2 * c.rates[i]) return bad("decoder transposed-conv kernels must be 2 * rate");
    if (c.decoder_dim % 16 || (c.decoder_dim >> 4) % 8) return bad("decoder_dim must be a multiple of 128");
    if (c.ffn % 16) return bad("ffn must be a multiple of 16");
    int n_dev = 0;
    if (hipGetDeviceCount(&n_dev) != hipSuccess || n_dev <= device || device < 0) return bad("no HIP device");
    if (hipSetDevice(device) != hipSuccess) return bad("hipSetDevice failed");
    q3t_voc * v = new q3t_voc();
    v->device = device;
    v->cfg = c;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        v->n_cu = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&v->stream, hipStreamNonBlocking) != hipSuccess) {
        delete v;
        return bad("hipStreamCreate failed");
    }
    if (alloc(v, &v->bad, 1)) {
        last = v->err;
        q3t_voc_destroy(v);
        if (err_out) *err_out = last.c_str();
        return nullptr;
    }
    return v;
}

void q3t_voc_destroy(q3t_voc * v) {
    if (!v) return;
    (void) hipSetDevice(v->device);
    if (v->stream) (void) hipStreamSynchronize(v->stream);
    for (void * p : v->allocs) (void) hipFree(p);
    if (v->stream) (void) hipStreamDestroy(v->stream);
    delete v;
}

const char * q3t_voc_last_error(const q3t_voc * v) { return v ? v->err.c_str() : "null decoder"; }

int q3t_voc_set_tensor(q3t_voc * v, const char * name, int32_t type, const void * data, size_t nbytes) {
    if (!v || !name || !data) return -1;
    if (type != 0 && type != 1) return fail(v, std::string("tensor ") + name + ": only F32 and F16 are supported");
    HostTensor & t = v->host[name];
    t.type = type;
    t.bytes.assign((const uint8_t *) data, (const uint8_t *) data + nbytes);
    v->ready = false;
    return 0;
}

int q3t_voc_finalize(q3t_voc * v) {
    if (!v) return -1;
    HIP_OK(hipSetDevice(v->device));
    const q3t_voc_config & c = v->cfg;
    // presence, type and size of every tensor build_graph reads
    struct Want { std::string name; int32_t type; size_t n; };
    std::vector<Want> want;
    auto add = [&](const std::string & n, int32_t ty, size_t cnt) { want.push_back({n, ty, cnt}); };
    auto blk = [](int l, const char * s) { return "tok_dec.pre_tfm.blk." + std::to_string(l) + "." + s; };
    add("tok_dec.vq_first.output_proj.weight", 1, (size_t) c.codebook_dim * c.hidden);
    add("tok_dec.vq_rest.output_proj.weight", 1, (size_t) c.codebook_dim * c.hidden);
    for (int q = 0; q < c.n_codebooks; ++q) {
        const std::string p = q == 0 ? "tok_dec.vq_first.0." : "tok_dec.vq_rest." + std::to_string(q - 1) + ".";
        add(p + "codebook", 1, (size_t) c.codebook_dim * c.codebook_size);
        add(p + "usage", 0, (size_t) c.codebook_size);
    }
    add("tok_dec.pre_conv.weight", 1, (size_t) 3 * c.hidden * c.latent);
    add("tok_dec.pre_conv.bias", 0, (size_t) c.latent);
    add("tok_dec.pre_tfm.input_proj.weight", 1, (size_t) c.latent * c.hidden);
    add("tok_dec.pre_tfm.input_proj.bias", 0, (size_t) c.hidden);
    for (int l = 0; l < c.n_layers; ++l) {
        add(blk(l, "attn_norm.weight"), 0, (size_t) c.hidden);
        for (const char * s : {"attn_q.weight", "attn_k.weight", "attn_v.weight"}) add(blk(l, s), 1, (size_t) c.hidden * c.latent);
        add(blk(l, "attn_output.weight"), 1, (size_t) c.latent * c.hidden);
        add(blk(l, "attn_scale"), 0, (size_t) c.hidden);
        add(blk(l, "ffn_norm.weight"), 0, (size_t) c.hidden);
        add(blk(l, "ffn_gate.weight"), 1, (size_t) c.hidden * c.ffn);
        add(blk(l, "ffn_up.weight"), 1, (size_t) c.hidden * c.ffn);
        add(blk(l, "ffn_down.weight"), 1, (size_t) c.ffn * c.hidden);
        add(blk(l, "ffn_scale"), 0, (size_t) c.hidden);
    }
    add("tok_dec.pre_tfm.norm.weight", 0, (size_t) c.hidden);
    add("tok_dec.pre_tfm.output_proj.weight", 1, (size_t) c.hidden * c.latent);
    add("tok_dec.pre_tfm.output_proj.bias", 0, (size_t) c.latent);
    for (int i = 0; i < 2; ++i) {
        const std::string p = "tok_dec.upsample." + std::to_string(i) + ".";
        add(p + "conv.weight", 1, (size_t) c.up_kernel * c.latent * c.latent);
        add(p + "dwconv.weight", 1, (size_t) 7 * c.latent);
        add(p + "pwconv1.weight", 1, (size_t) c.latent * c.cnx_ffn);
        add(p + "pwconv1.bias", 0, (size_t) c.cnx_ffn);
        add(p + "pwconv2.weight", 1, (size_t) c.cnx_ffn * c.latent);
        for (const char * s : {"conv.bias", "dwconv.bias", "norm.weight", "norm.bias", "pwconv2.bias", "gamma"})
            add(p + s, 0, (size_t) c.latent);
    }
    add("tok_dec.dec.0.conv.weight", 1, (size_t) 7 * c.latent * c.decoder_dim);
    add("tok_dec.dec.0.conv.bias", 0, (size_t) c.decoder_dim);
    int ch = c.decoder_dim;
    for (int b = 0; b < 4; ++b) {
        const std::string p = "tok_dec.dec." + std::to_string(b + 1) + ".";
        const int co = ch / 2;
        add(p + "snake.alpha", 0, (size_t) ch);
        add(p + "snake.beta", 0, (size_t) ch);
        add(p + "conv_t.weight", 1, (size_t) c.dec_kernel[b] * co * ch);
        add(p + "conv_t.bias", 0, (size_t) co);
        for (int r = 2; r <= 4; ++r) {
            const std::string q = p + "res." + std::to_string(r) + ".";
            for (const char * s : {"act1.alpha", "act1.beta", "conv1.bias", "act2.alpha", "act2.beta", "conv2.bias"})
                add(q + s, 0, (size_t) co);
            add(q + "conv1.weight", 1, (size_t) 7 * co * co);
            add(q + "conv2.weight", 1, (size_t) co * co);
        }
        ch = co;
    }
    add("tok_dec.dec.5.snake.alpha", 0, (size_t) ch);
    add("tok_dec.dec.5.snake.beta", 0, (size_t) ch);
    add("tok_dec.dec.6.conv.weight", 1, (size_t) 7 * ch);
    add("tok_dec.dec.6.conv.bias", 0, (size_t) 1);
    for (const Want & w : want) {
        const HostTensor * t = get(v, w.name);
        if (!t) return fail(v, "missing tensor " + w.name);
        if (t->type != w.type || t->bytes.size() != w.n * (w.type == 0 ? 4 : 2))
            return fail(v, "tensor " + w.name + ": unexpected type or size");
    }

    // codebooks normalised by usage (normalize_codebooks :66-100), then
    // projected: tab_q[e] = output_proj_q . cb_q[e] (the VQ's per-code rows)
    const int32_t cdp = rup(c.codebook_dim, 32), H = rup(c.hidden, 32);
    GemmW proj[2];
    if (build_linear(v, proj[0], f16(v, "tok_dec.vq_first.output_proj.weight"), c.codebook_dim, c.hidden) ||
        build_linear(v, proj[1], f16(v, "tok_dec.vq_rest.output_proj.weight"), c.codebook_dim, c.hidden))
        return -1;
    if (alloc(v, &v->vq_tab, (size_t) c.n_codebooks * c.codebook_size * c.hidden)) return -1;
    uint16_t * cbd = nullptr;
    if (alloc(v, &cbd, (size_t) c.codebook_size * cdp)) return -1;
    std::vector<uint16_t> cbh((size_t) c.codebook_size * cdp, 0);
    for (int q = 0; q < c.n_codebooks; ++q) {
        const std::string p = q == 0 ? "tok_dec.vq_first.0." : "tok_dec.vq_rest." + std::to_string(q - 1) + ".";
        const uint16_t * src = f16(v, p + "codebook");
        const float * u = f32(v, p + "usage");
        for (int e = 0; e < c.codebook_size; ++e) {
            float uu = u[e];
            if (uu < 1e-5f) uu = 1e-5f;
            const float inv = 1.0f / uu;
            for (int d = 0; d < c.codebook_dim; ++d) {
                const size_t at = (size_t) e * c.codebook_dim + d;
                _Float16 hv;
                std::memcpy(&hv, &src[at], 2);
                const _Float16 nv = (_Float16) ((float) hv * inv);
                std::memcpy(&cbh[(size_t) e * cdp + d], &nv, 2);
            }
        }
        HIP_OK(hipMemcpy(cbd, cbh.data(), cbh.size() * 2, hipMemcpyHostToDevice));
        if (gemm(v, proj[q == 0 ? 0 : 1], cbd, cdp, c.codebook_size, 0, 1, c.codebook_size, 1, nullptr, nullptr,
                 nullptr, 0, v->vq_tab + (size_t) q * c.codebook_size * c.hidden, c.hidden, nullptr, 0, ACT_NONE,
                 nullptr))
            return -1;
        HIP_OK(hipStreamSynchronize(v->stream));
    }
    release(v, cbd);
    release(v, proj[0].w);
    release(v, proj[1].w);
    (void) H;

    // pre-transformer
    if (build_conv(v, v->pre_conv, f16(v, "tok_dec.pre_conv.weight"), 3, c.hidden, c.latent) ||
        upload_f32(v, &v->pre_conv_b, "tok_dec.pre_conv.bias") ||
        build_linear(v, v->in_proj, f16(v, "tok_dec.pre_tfm.input_proj.weight"), c.latent, c.hidden) ||
        upload_f32(v, &v->in_proj_b, "tok_dec.pre_tfm.input_proj.bias"))
        return -1;
    v->pre.assign((size_t) c.n_layers, PreLayer{});
    for (int l = 0; l < c.n_layers; ++l) {
        PreLayer & P = v->pre[(size_t) l];
        const uint16_t * wq = f16(v, blk(l, "attn_q.weight")), * wk = f16(v, blk(l, "attn_k.weight")),
                       * wv = f16(v, blk(l, "attn_v.weight"));
        const int32_t L = c.latent, K = c.hidden;
        if (build_gemm(v, P.qkv, 3 * L, 1, K, 1, false, [&](int, int n, int, int k) {
                const uint16_t * w = n < L ? wq : n < 2 * L ? wk : wv;
                return w[(size_t) (n % L) * K + k];
            }))
            return -1;
        const uint16_t * wg = f16(v, blk(l, "ffn_gate.weight")), * wu = f16(v, blk(l, "ffn_up.weight"));
        // 16-row groups alternate gate / up (the SwiGLU epilogue pairs tiles 2q, 2q+1)
        if (build_gemm(v, P.gu, 2 * c.ffn, 1, K, 1, true, [&](int, int n, int, int k) {
                const int g = n / 32, w = n % 32;
                const uint16_t * src = w < 16 ? wg : wu;
                return src[(size_t) (g * 16 + (w & 15)) * K + k];
            }))
            return -1;
        if (build_linear(v, P.wo, f16(v, blk(l, "attn_output.weight")), c.latent, c.hidden) ||
            build_linear(v, P.down, f16(v, blk(l, "ffn_down.weight")), c.ffn, c.hidden) ||
            upload_f32(v, &P.attn_norm, blk(l, "attn_norm.weight")) ||
            upload_f32(v, &P.ffn_norm, blk(l, "ffn_norm.weight")) ||
            upload_f32(v, &P.attn_scale, blk(l, "attn_scale")) || upload_f32(v, &P.ffn_scale, blk(l, "ffn_scale")))
            return -1;
    }
    if (upload_f32(v, &v->final_norm, "tok_dec.pre_tfm.norm.weight") ||
        build_linear(v, v->out_proj, f16(v, "tok_dec.pre_tfm.output_proj.weight"), c.hidden, c.latent) ||
        upload_f32(v, &v->out_proj_b, "tok_dec.pre_tfm.output_proj.bias"))
        return -1;

    // upsample blocks: conv_t ne (2, C, C) = [i][o][k]; phase p uses tap k = p
    for (int i = 0; i < 2; ++i) {
        UpBlock & U = v->up[i];
        const std::string p = "tok_dec.upsample." + std::to_string(i) + ".";
        const uint16_t * w = f16(v, p + "conv.weight");
        const int32_t C = c.latent;
        if (build_gemm(v, U.conv_t, C, 1, C, 2, false,
                       [&](int ph, int o, int, int ci) { return w[((size_t) ci * C + o) * 2 + ph]; }))
            return -1;
        std::vector<uint16_t> dw(f16(v, p + "dwconv.weight"), f16(v, p + "dwconv.weight") + (size_t) 7 * C);
        if (upload(v, &U.dw_w, dw) || upload_f32(v, &U.conv_b, p + "conv.bias") ||
            upload_f32(v, &U.dw_b, p + "dwconv.bias") || upload_f32(v, &U.norm_w, p + "norm.weight") ||
            upload_f32(v, &U.norm_b, p + "norm.bias") ||
            build_linear(v, U.pw1, f16(v, p + "pwconv1.weight"), C, c.cnx_ffn) ||
            upload_f32(v, &U.pw1_b, p + "pwconv1.bias") ||
            build_linear(v, U.pw2, f16(v, p + "pwconv2.weight"), c.cnx_ffn, C) ||
            upload_f32(v, &U.pw2_b, p + "pwconv2.bias") || upload_f32(v, &U.gamma, p + "gamma"))
            return -1;
    }
    if (build_conv(v, v->dec0, f16(v, "tok_dec.dec.0.conv.weight"), 7, c.latent, c.decoder_dim) ||
        upload_f32(v, &v->dec0_b, "tok_dec.dec.0.conv.bias"))
        return -1;
    ch = c.decoder_dim;
    for (int b = 0; b < 4; ++b) {
        DecBlock & B = v->dec[b];
        const std::string p = "tok_dec.dec." + std::to_string(b + 1) + ".";
        const int32_t co = ch / 2, s = c.rates[b], K = c.dec_kernel[b];
        const uint16_t * w = f16(v, p + "conv_t.weight");          // [ci][co][k]
        // phase p: tap 0 reads row m (kernel index p + s), tap 1 row m + 1 (index p)
        if (build_gemm(v, B.conv_t, co, 2, ch, s, false, [&](int ph, int o, int tap, int ci) {
                return w[((size_t) ci * co + o) * K + (tap == 0 ? ph + s : ph)];
            }))
            return -1;
        if (upload_snake(v, B.snake, p + "snake.") || upload_f32(v, &B.conv_t_b, p + "conv_t.bias")) return -1;
        for (int r = 0; r < 3; ++r) {
            ResUnit & U = B.res[r];
            const std::string q = p + "res." + std::to_string(r + 2) + ".";
            if (upload_snake(v, U.act1, q + "act1.") || upload_snake(v, U.act2, q + "act2.") ||
                build_conv(v, U.conv1, f16(v, q + "conv1.weight"), 7, co, co) ||
                build_conv(v, U.conv2, f16(v, q + "conv2.weight"), 1, co, co) ||
                upload_f32(v, &U.b1, q + "conv1.bias") || upload_f32(v, &U.b2, q + "conv2.bias"))
                return -1;
        }
        ch = co;
    }
    if (upload_snake(v, v->snake5, "tok_dec.dec.5.snake.")) return -1;
    {
        const int32_t Cp = rup(ch, 32);
        const uint16_t * w = f16(v, "tok_dec.dec.6.conv.weight");   // [0][c][k]
        std::vector<uint16_t> ow((size_t) Cp * 7, 0);
        for (int i = 0; i < ch * 7; ++i) ow[(size_t) i] = w[i];
        if (upload(v, &v->out_w, ow)) return -1;
        v->out_b = f32(v, "tok_dec.dec.6.conv.bias")[0];
    }
    if (rope_table(v, 8192)) return -1;
    HIP_OK(hipDeviceSynchronize());
    v->ready = true;
    return 0;
}

int q3t_voc_reserve(q3t_voc * v, int32_t max_frames) {
    if (!v) return -1;
    if (!v->ready) return fail(v, "Model not loaded");
    if (max_frames < 1) return fail(v, "max_frames must be >= 1");
    HIP_OK(hipSetDevice(v->device));
    return reserve(v, max_frames);
}

int64_t q3t_voc_samples_for_frames(const q3t_voc * v, int32_t n_frames) {
    return v ? samples_for(v->cfg, n_frames) : 0;
}

int q3t_voc_decode_window(q3t_voc * v, const int32_t * codes, int32_t codes_on_device, int32_t n_frames,
                          int32_t start, int32_t end, int32_t context, float * out, int64_t cap, int64_t * n_out) {
    if (!v || !n_out) return -1;
    if (!v->ready) return fail(v, "Model not loaded");
    if (!codes || !out) return fail(v, "null codes or output");
    if (start < 0 || end <= start || end > n_frames) return fail(v, "decode_window: invalid frame range");
    HIP_OK(hipSetDevice(v->device));
    const q3t_voc_config & c = v->cfg;
    const int32_t ctx_start = std::max(0, start - std::max(0, context));
    const int32_t seg = end - ctx_start;
    const int64_t total = samples_for(c, seg);
    const int64_t drop = std::min(samples_for(c, start - ctx_start), total);
    if (total - drop > cap) return fail(v, "decode_window: output buffer too small");
    if (reserve(v, seg)) return -1;
    const int32_t * cd = codes + (size_t) ctx_start * c.n_codebooks;
    if (!codes_on_device) {
        for (int64_t i = 0; i < (int64_t) seg * c.n_codebooks; ++i)
            if (cd[i] < 0 || cd[i] >= c.codebook_size) return fail(v, "code out of range");
        HIP_OK(hipMemcpyAsync(v->codes, cd, (size_t) seg * c.n_codebooks * 4, hipMemcpyHostToDevice, v->stream));
        cd = v->codes;
    }
    int cur = 0;
    if (vq(v, cd, seg, v->h[cur])) return -1;
    const std::vector<std::string> names = stage_names(c);
    if (run_chain(v, names, 1, names.size() - 1, seg, ctx_start, cur, false, drop)) return -1;
    if (check_bad(v)) return -1;
    if (total - drop > 0)
        HIP_OK(hipMemcpyAsync(out, v->audio, (size_t) (total - drop) * 4, hipMemcpyDeviceToHost, v->stream));
    HIP_OK(hipStreamSynchronize(v->stream));
    *n_out = total - drop;
    return 0;
}

int q3t_voc_decode(q3t_voc * v, const int32_t * codes, int32_t codes_on_device, int32_t n_frames, float * out,
                   int64_t cap, int64_t * n_out) {
    if (!v || !n_out) return -1;
    if (n_frames <= 0) { *n_out = 0; return 0; }
    return q3t_voc_decode_window(v, codes, codes_on_device, n_frames, 0, n_frames, 0, out, cap, n_out);
}

int q3t_voc_run_stage(q3t_voc * v, const char * name, const float * in, const int32_t * codes, int64_t T, int64_t C,
                      int32_t pos0, float * out, int64_t cap, int64_t * T_out, int64_t * C_out) {
    if (!v || !name || !T_out || !C_out || !out) return -1;
    if (!v->ready) return fail(v, "Model not loaded");
    HIP_OK(hipSetDevice(v->device));
    const q3t_voc_config & c = v->cfg;
    const std::vector<std::string> names = stage_names(c);
    auto it = std::find(names.begin(), names.end(), std::string(name));
    if (it == names.end()) return fail(v, std::string("unknown stage ") + name);
    const size_t si = (size_t) (it - names.begin());
    // the segment length n whose stage si - 1 has T rows
    int64_t n = -1;
    for (int64_t m = 1; m <= 1 << 16 && n < 0; ++m) {
        const int64_t rows = si == 0 ? m : stage_shape(c, names[si - 1], m).rows;
        if (rows == T) n = m;
        if (rows > T) break;
    }
    if (n < 0) return fail(v, "run_stage: no segment length gives that many input rows");
    if (reserve(v, (int32_t) n)) return -1;
    const Shape osh = stage_shape(c, names[si], n);
    if (osh.rows * osh.ch > cap) return fail(v, "run_stage: output buffer too small");
    int cur = 0;
    if (si == 0) {
        if (!codes) return fail(v, "latent needs codes");
        for (int64_t i = 0; i < T * c.n_codebooks; ++i)
            if (codes[i] < 0 || codes[i] >= c.codebook_size) return fail(v, "code out of range");
        HIP_OK(hipMemcpyAsync(v->codes, codes, (size_t) T * c.n_codebooks * 4, hipMemcpyHostToDevice, v->stream));
        if (vq(v, v->codes, T, v->h[cur])) return -1;
        if (check_bad(v)) return -1;
    } else {
        const Shape ish = stage_shape(c, names[si - 1], n);
        if (!in || C != ish.ch) return fail(v, "run_stage: input width does not match the stage");
        const int32_t Cp = rup((int32_t) C, 32);
        HIP_OK(hipMemsetAsync(v->xf, 0, (size_t) T * Cp * 4, v->stream));
        HIP_OK(hipMemcpy2DAsync(v->xf, (size_t) Cp * 4, in, (size_t) C * 4, (size_t) C * 4, (size_t) T,
                                hipMemcpyHostToDevice, v->stream));
        const InAct ia = input_act(v, names[si]);
        if (clear_pad(v, v->h[cur], T, (int32_t) C)) return -1;
        if (prep(v, v->xf, Cp, T, (int32_t) C, ia.act, ia.sn, v->h[cur], Cp)) return -1;
        if (run_chain(v, names, si, si, n, pos0, cur, true, 0)) return -1;
    }
    const int32_t Cop = rup(osh.ch, 32);
    if (names[si] == "dec.6")
        HIP_OK(hipMemcpyAsync(out, v->pre_out, (size_t) osh.rows * 4, hipMemcpyDeviceToHost, v->stream));
    else
        HIP_OK(hipMemcpy2DAsync(out, (size_t) osh.ch * 4, v->xf, (size_t) Cop * 4, (size_t) osh.ch * 4,
                                (size_t) osh.rows, hipMemcpyDeviceToHost, v->stream));
    HIP_OK(hipStreamSynchronize(v->stream));
    *T_out = osh.rows;
    *C_out = osh.ch;
    return 0;
}

}  // extern "C"
