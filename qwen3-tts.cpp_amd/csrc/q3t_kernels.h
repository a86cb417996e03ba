// q3t_kernels.h -- gfx950 kernels of the talker / code-predictor decode loop.
//
//   k_gemv        Q8_0 / F16 / F16-widened GEMV for 1, 2 or 4 tokens, with a
//                 fused prologue (RMSNorm, activation quantisation into LDS)
//                 and epilogue (store, residual add, bias, bias+SiLU, SwiGLU
//                 of a gate/up pair).  Replaces ggml_rms_norm + ggml_mul +
//                 ggml_mul_mat (+ ggml_add / ggml_silu / ggml_mul) at
//                 src/tts_transformer.cpp:1656-1661, 1732-1750, 1755-1762.
//   k_attention   QK-norm + NEOX RoPE + fp16 KV append + GQA decode attention
//                 for one (query head, token); replaces :1667-1730.
//   k_sample      codec-head / code-predictor sampler on device; replaces the
//                 host sampler at :3109-3184 and sample_or_argmax :2750-2788.
//                 It also gathers the next pass's input rows: the
//                 code-predictor inputs (:2790-2793, :2091) and the talker
//                 step embedding (:3264-3295).
//   k_gemv_r      (q3t_gemv_reg.h) the decode-loop GEMV for 1-2 tokens:
//                 weights prefetched into registers at entry, activation
//                 normalised/quantised per lane in registers.
#pragma once

#include "q3t_numerics.h"

namespace q3t {

enum WeightKind { W_Q8 = 0, W_F16 = 1, W_F16W = 2 };
enum Prologue { PRO_NONE = 0, PRO_NORM = 1 };
enum Epilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_BIAS = 2, EPI_BIAS_SILU = 3, EPI_SWIGLU = 4 };

// Device-resident state of the frame loop (one per context).  The
// codebook-0 sampler opens a frame (frame = next_frame++, talker_pos =
// base_pos + frame); the codebook-15 sampler emits the frame's codes.
struct FrameState {
    int32_t talker_pos;  // position the talker step of this frame writes
    int32_t frame;       // index of the frame being generated
    int32_t done;        // 1 once EOS was sampled or max_frames were opened: every kernel exits early
    int32_t n_emitted;   // frames written to codes_out
    int32_t codes[16];   // codes of the current frame
    int32_t max_frames;  // capacity of codes_out (and of the KV positions reserved for the loop)
    int32_t eos;         // 1 once codebook 0 sampled EOS
    int32_t base_pos;    // talker position of frame 0's step (the prefill length)
    int32_t next_frame;  // frame index the next codebook-0 sampler opens
};

struct SampleParams {
    float    temperature;
    int32_t  top_k;
    float    rep_penalty;
    float    eos_bias;
    int32_t  target_frames;
    int32_t  pad;
    uint64_t seed;
};

struct GemvArgs {
    const void * w;  const uint16_t * wd;    // weight (int8 quants or fp16) + Q8_0 scales
    const void * w2; const uint16_t * w2d;   // second (up) weight for EPI_SWIGLU
    int32_t rows, K;
    const float * x; int32_t x_stride;       // input rows [NT][x_stride]
    const float * norm_w; float eps;         // PRO_NORM
    float * hidden_out; int32_t hidden_stride;  // PRO_NORM: normed rows (block 0 writes)
    float * y; int32_t y_stride;             // output rows [NT][y_stride]
    const float * resid; int32_t resid_stride;
    const float * bias;
    const int32_t * done;
    int32_t pro, epi;
};

// ------------------------------------------------------------------ GEMV
// LDS: 4 doubles of reduction scratch, then the activation of NT tokens:
//   W_Q8  : int8 [NT][K] then float scale [NT][K/32] (fp16-rounded d)
//   W_F16 : fp16 [NT][K] (activation rounded to fp16)
//   W_F16W: fp32 [NT][K]
template <int WT>
__host__ __device__ constexpr size_t act_bytes(int nt, int k) {
    return WT == W_Q8 ? (size_t) nt * k + (size_t) nt * (k / kQK) * 4
         : WT == W_F16 ? (size_t) nt * k * 2 : (size_t) nt * k * 4;
}

// LDS ahead of the activation rows: the RMSNorm partials [NT][4 waves] fp64.
__host__ __device__ constexpr size_t act_red_bytes(int nt) { return (size_t) (nt < 2 ? 2 : nt) * 4 * 8; }

template <int WT, int NT, int NTH = kBlock>
__device__ __forceinline__ void build_act(const GemvArgs & a, double * red, char * act) {
    const int K = a.K, t = threadIdx.x;
    // Elements e = e0 + u*NTH + t (u < U) of all NT rows are loaded together,
    // so their loads are in flight at once; for K <= U*NTH they are loaded
    // once and kept in registers for both passes.
    constexpr int U = NTH >= 1024 ? 1 : 4, NW = NTH / 64;
    const bool once = K <= U * NTH;
    float v[NT][U];
    const auto load = [&](int e0) {
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            const float * x = a.x + (size_t) tok * a.x_stride;
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + u * NTH + t;
                v[tok][u] = e < K ? x[e] : 0.0f;
            }
        }
    };
    if (once) load(0);
    // RMSNorm scales of all NT rows with one pair of workgroup barriers; each
    // thread sums its elements in ascending order, then the order of block_sum_d
    float scales[NT];
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) scales[tok] = 1.0f;
    if (NTH >= 1024 && NT * 64 <= NTH && a.pro == PRO_NORM) {
        // a wave per row: wave w sums the squares of row w (lane l: elements
        // l, l + 64, ... in ascending order, loaded 16 at a time), one wave
        // reduction per wave instead of NT
        const int w = t >> 6, l = t & 63;
        if (w < NT) {
            const float * xr = a.x + (size_t) w * a.x_stride;
            double ss = 0.0;
            for (int e0 = 0; e0 < K; e0 += 16 * 64) {
                float q[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int e = e0 + 64 * i + l;
                    q[i] = e < K ? xr[e] : 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (e0 + 64 * i + l < K) ss += (double) (q[i] * q[i]);
            }
            ss = wave_sum_d(ss);
            // the scale once per row (fp64 division, square root and
            // reciprocal are long instruction sequences), shared through LDS
            const float mean = (float) (ss / (double) K);
            if (l == 0) ((float *) red)[w] = 1.0f / sqrtf(mean + a.eps);
        }
        __syncthreads();
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) scales[tok] = ((const float *) red)[tok];
    } else if (a.pro == PRO_NORM) {
        double ss[NT];
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) ss[tok] = 0.0;
        for (int e0 = 0; e0 < K; e0 += U * NTH) {
            if (!once) load(e0);
#pragma unroll
            for (int tok = 0; tok < NT; ++tok)
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (e0 + u * NTH + t < K) ss[tok] += (double) (v[tok][u] * v[tok][u]);
        }
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) ss[tok] = wave_sum_d(ss[tok]);
        __syncthreads();
        if ((t & 63) == 0)
#pragma unroll
            for (int tok = 0; tok < NT; ++tok) red[tok * NW + (t >> 6)] = ss[tok];
        __syncthreads();
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            const double * rw = red + tok * NW;
            double tot;
            if (NW == 4) {
                tot = (rw[0] + rw[1]) + (rw[2] + rw[3]);
            } else {
                tot = rw[0];
                for (int w = 1; w < NW; ++w) tot += rw[w];
            }
            const float mean = (float) (tot / (double) K);
            scales[tok] = 1.0f / sqrtf(mean + a.eps);
        }
    }
    for (int e0 = 0; e0 < K; e0 += U * NTH) {
        if (!once) load(e0);
        // the gains are read before any store: a store through hidden_out
        // could alias them and would force a reload per row
        float nw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * NTH + t;
            nw[u] = a.pro == PRO_NORM && e < K ? a.norm_w[e] : 1.0f;
        }
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int e = e0 + u * NTH + t;
                if (e >= K) continue;      // K % 32 == 0: a Q8_0 block's 32 lanes agree
                float y = v[tok][u];
                if (a.pro == PRO_NORM) {
                    y = y * scales[tok];
                    y = y * nw[u];
                    if (a.hidden_out && blockIdx.x == 0) a.hidden_out[(size_t) tok * a.hidden_stride + e] = y;
                }
                if (WT == W_Q8) {
                    // the 32 consecutive lanes t..t+31 hold one Q8_0 block
                    float am = fabsf(y);
#pragma unroll
                    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
                    const float d = am / 127.0f;
                    const float id = am != 0.0f ? 127.0f / am : 0.0f;
                    int8_t * q = (int8_t *) act;
                    q[(size_t) tok * K + e] = (int8_t) (int) rintf(y * id);
                    if ((t & 31) == 0) {
                        float * sd = (float *) (act + (size_t) NT * K);
                        sd[tok * (K / kQK) + e / kQK] = round_f16(d);
                    }
                } else if (WT == W_F16) {
                    ((uint16_t *) act)[(size_t) tok * K + e] = f2h(y);
                } else {
                    ((float *) act)[(size_t) tok * K + e] = y;
                }
            }
        }
    }
    __syncthreads();
}

template <int NT>
__device__ __forceinline__ void gemv_store(const GemvArgs & a, int r, const double * acc, const double * acc2) {
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
        const float v = (float) acc[tok];
        float o;
        switch (a.epi) {
            case EPI_RESID: o = v + a.resid[(size_t) tok * a.resid_stride + r]; break;
            case EPI_BIAS: o = v + a.bias[r]; break;
            case EPI_BIAS_SILU: o = silu_q3t(v + a.bias[r]); break;
            case EPI_SWIGLU: o = silu_q3t(v) * (float) acc2[tok]; break;
            default: o = v; break;
        }
        a.y[(size_t) tok * a.y_stride + r] = o;
    }
}

// Lane layout: a row's K/32 blocks are spread over LPR = min(32, K/32)
// consecutive lanes (each lane owns whole 32-element blocks, SLOTS of them
// per row), so one wave covers 64/LPR rows per iteration and every weight
// load instruction reads a contiguous 2 KB (Q8) / 4 KB (F16) span.  The
// per-lane fp64 partials are summed over the LPR lanes with xor shuffles.
template <int WT, int NT, bool DUAL>
__device__ __forceinline__ void gemv_rows(const GemvArgs & a, const char * act) {
    const int K = a.K, BPR = K / kQK;
    const int LPR = BPR < 32 ? BPR : 32;
    const int SLOTS = BPR / LPR;
    const int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lir = lane & (LPR - 1), rsub = lane / LPR;
    const int ngroups = a.rows / RPW;
    for (int g = blockIdx.x * (kBlock / 64) + wave; g < ngroups; g += gridDim.x * (kBlock / 64)) {
        const int r = g * RPW + rsub;
        double acc[NT], acc2[NT];
#pragma unroll
        for (int i = 0; i < NT; ++i) { acc[i] = 0.0; acc2[i] = 0.0; }
        for (int s = 0; s < SLOTS; ++s) {
            const int b = lir + s * LPR;
            if (WT == W_Q8) {
                const int4 * wp = (const int4 *) ((const int8_t *) a.w + (size_t) r * K + b * kQK);
                const int4 w0 = wp[0], w1 = wp[1];
                const float dw = h2f(a.wd[(size_t) r * BPR + b]);
                int4 u0, u1; float du = 0.0f;
                if (DUAL) {
                    const int4 * up = (const int4 *) ((const int8_t *) a.w2 + (size_t) r * K + b * kQK);
                    u0 = up[0]; u1 = up[1];
                    du = h2f(a.w2d[(size_t) r * BPR + b]);
                }
                const int8_t * xq = (const int8_t *) act;
                const float * xd = (const float *) (act + (size_t) NT * K);
#pragma unroll
                for (int tok = 0; tok < NT; ++tok) {
                    const int4 * xp = (const int4 *) (xq + (size_t) tok * K + b * kQK);
                    const int4 x0 = xp[0], x1 = xp[1];
                    const float dx = xd[tok * BPR + b];
                    acc[tok] += (double) (dw * dx) * (double) dot32_i8(w0, w1, x0, x1);
                    if (DUAL) acc2[tok] += (double) (du * dx) * (double) dot32_i8(u0, u1, x0, x1);
                }
            } else {
                const uint16_t * wrow = (const uint16_t *) a.w + (size_t) r * K + b * kQK;
                const uint16_t * urow = DUAL ? (const uint16_t *) a.w2 + (size_t) r * K + b * kQK : nullptr;
#pragma unroll
                for (int c = 0; c < 4; ++c) {       // 4 chunks of 8 halves (16 bytes)
                    const int4 wv = ((const int4 *) wrow)[c];
                    const uint16_t * wh = (const uint16_t *) &wv;
                    int4 uv;
                    if (DUAL) uv = ((const int4 *) urow)[c];
                    const uint16_t * uh = (const uint16_t *) &uv;
#pragma unroll
                    for (int tok = 0; tok < NT; ++tok) {
                        if (WT == W_F16) {
                            const int4 xv = *(const int4 *) ((const uint16_t *) act + (size_t) tok * K + b * kQK + c * 8);
                            const uint16_t * xh = (const uint16_t *) &xv;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                const _Float16 xj = __builtin_bit_cast(_Float16, xh[j]);
                                // exact fp16*fp16 product
                                acc[tok] += (double) hmul_exact(__builtin_bit_cast(_Float16, wh[j]), xj);
                                if (DUAL) acc2[tok] += (double) hmul_exact(__builtin_bit_cast(_Float16, uh[j]), xj);
                            }
                        } else {
                            const float * xf = (const float *) act + (size_t) tok * K + b * kQK + c * 8;
#pragma unroll
                            for (int j = 0; j < 8; ++j) {
                                acc[tok] = fma((double) h2f(wh[j]), (double) xf[j], acc[tok]);
                                if (DUAL) acc2[tok] = fma((double) h2f(uh[j]), (double) xf[j], acc2[tok]);
                            }
                        }
                    }
                }
            }
        }
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            for (int o = LPR / 2; o > 0; o >>= 1) {
                acc[tok] += __shfl_xor(acc[tok], o);
                if (DUAL) acc2[tok] += __shfl_xor(acc2[tok], o);
            }
        }
        if (lir == 0) gemv_store<NT>(a, r, acc, acc2);
    }
}

template <int WT, int NT, bool DUAL>
__global__ __launch_bounds__(kBlock) void k_gemv(GemvArgs a) {
    if (a.done && *a.done) return;
    extern __shared__ __align__(16) char smem[];
    double * red = (double *) smem;
    char * act = smem + act_red_bytes(NT);
    build_act<WT, NT>(a, red, act);
    gemv_rows<WT, NT, DUAL>(a, act);
}

// F16 GEMV of NT rows (the multi-stream heads: 8 or 16 streams) on 1024
// threads, EPI_STORE.  Block b owns output rows [8b, 8b + 8): wave w takes row
// pair w % 4 over K quarter w / 4; lane l row 2 (w % 4) + l / 32 and the
// 8-element chunks (l % 32) + 32 i of its quarter.  Four waves per SIMD hide
// the latency of the exact fp64 accumulation that k_gemv's one row pair per
// wave leaves exposed.  A lane's partials are summed over its row's 32 lanes
// (xor tree), then over the quarters in a fixed order.  Requires rows % 8 == 0
// and K % 32 == 0 (the host checks).
constexpr int kMtThreads = 1024;
template <int NT>
__host__ __device__ constexpr size_t gemv_mt_lds_bytes(int K) {
    return (size_t) NT * 16 * 8 + (size_t) 4 * 8 * NT * 8 + (size_t) NT * K * 2;
}
template <int NT>
__global__ __launch_bounds__(kMtThreads) void k_gemv_mt(GemvArgs a) {
    if (a.done && *a.done) return;
    extern __shared__ __align__(16) char smem[];
    double * red = (double *) smem;                  // [NT][16] RMSNorm partials
    double * part = red + NT * 16;                   // [4 quarters][8 rows][NT]
    char * act = (char *) (part + 4 * 8 * NT);       // fp16 [NT][K]
    build_act<W_F16, NT, kMtThreads>(a, red, act);
    const int K = a.K, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int q = wave >> 2, rl = 2 * (wave & 3) + (lane >> 5), r = blockIdx.x * 8 + rl;
    const int KQ = K / 4, nch = KQ / 8;              // elements / 8-element chunks per quarter
    const uint16_t * wrow = (const uint16_t *) a.w + (size_t) r * K + q * KQ;
    const uint16_t * xq = (const uint16_t *) act + q * KQ;
    double acc[NT];
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) acc[tok] = 0.0;
    for (int c = lane & 31; c < nch; c += 32) {
        const int4 wv = *(const int4 *) (wrow + c * 8);
        const uint16_t * wh = (const uint16_t *) &wv;
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            const int4 xv = *(const int4 *) (xq + (size_t) tok * K + c * 8);
            const uint16_t * xh = (const uint16_t *) &xv;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                acc[tok] += (double) hmul_exact(__builtin_bit_cast(_Float16, wh[j]), __builtin_bit_cast(_Float16, xh[j]));
        }
    }
#pragma unroll
    for (int tok = 0; tok < NT; ++tok)
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) acc[tok] += __shfl_xor(acc[tok], o);
    if ((lane & 31) == 0)
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) part[(q * 8 + rl) * NT + tok] = acc[tok];
    __syncthreads();
    if (t < 8 * NT) {
        const int rr = t / NT, tok = t - rr * NT;
        const double * p = part + rr * NT + tok;
        const double v = (p[0] + p[8 * NT]) + (p[16 * NT] + p[24 * NT]);
        a.y[(size_t) tok * a.y_stride + blockIdx.x * 8 + rr] = (float) v;
    }
}

// ------------------------------------------------------------- attention
struct AttnArgs {
    const float * qkv; int32_t qkv_stride;        // [NT][n_head*hd + 2*n_kv*hd]
    const float * q_norm; const float * k_norm; float eps;
    const float * rope_cos; const float * rope_sin;  // [pos][hd/2]
    uint16_t * kc; uint16_t * vc;                  // layer base, [n_kv_head][n_ctx][hd]
    int32_t n_ctx, n_head, n_kv_head;
    const int32_t * pos_ptr; int32_t pos_const;    // position of token 0
    float * out; int32_t out_stride;               // [NT][n_head*hd]
    const int32_t * done;
    float scale;
    int32_t nt;
    float * probs_out;                             // optional [n_head][n_kv] (token 0)
    // independent streams (blockIdx.z): element offsets per stream; 0 for one stream
    int64_t kv_stream;                             // in kc / vc
    int32_t qkv_stream, out_stream;                // in qkv / out (floats)
    int32_t pos_stream, done_stream;               // in pos_ptr / done (int32)
    // optional Q8_0 copy of the output rows for the next projection:
    // out_q [NT][out_stride] int8, out_dx [NT][out_stride / 32] (same stream offsets)
    int8_t * out_q; float * out_dx;
    // 1: the code predictor's prefill (pos0 = 0, nt = 2), which attends over
    // the F32 rows of this launch (src/tts_transformer.cpp:1999-2012): q, K, V
    // and P stay fp32; the fp16 cache rows are still written
    int32_t f32_new;
    // 1: a bfloat16 cache (q and P are rounded to bfloat16, ggml_mul_mat's
    // conversion of its F32 operand to a BF16 cache's dot type)
    int32_t kv_bf16;
};

constexpr int kHD = 128;

// RMSNorm over one head (hd = 128) held by threads 0..127, then NEOX RoPE;
// returns the rotated value for element threadIdx.x (threads < 128).
__device__ __forceinline__ float head_norm_rope(float v, const float * w, float eps, const float * c,
                                                const float * s, float * tmp, double * red) {
    const int t = threadIdx.x;
    const double ss = t < kHD ? (double) (v * v) : 0.0;
    const double tot = block_sum_d(ss, red);
    const float mean = (float) (tot / (double) kHD);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (t < kHD) { v = v * scale; v = v * w[t]; tmp[t] = v; }
    __syncthreads();
    float o = 0.0f;
    if (t < kHD) {
        const int i = t & 63;
        const float x0 = tmp[i], x1 = tmp[i + 64];
        if (t < 64) { const float p = x0 * c[i], q = x1 * s[i]; o = p - q; }
        else        { const float p = x0 * s[i], q = x1 * c[i]; o = p + q; }
    }
    __syncthreads();
    return o;
}

// head_norm_rope with this thread's operands already loaded: wv = w[t], cv =
// c[t & 63], sv = s[t & 63] (threads < 128); the same arithmetic.
__device__ __forceinline__ float head_norm_rope_v(float v, float wv, float eps, float cv, float sv, float * tmp,
                                                  double * red) {
    const int t = threadIdx.x;
    const double ss = t < kHD ? (double) (v * v) : 0.0;
    const double tot = block_sum_d(ss, red);
    const float mean = (float) (tot / (double) kHD);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (t < kHD) { v = v * scale; v = v * wv; tmp[t] = v; }
    __syncthreads();
    float o = 0.0f;
    if (t < kHD) {
        const int i = t & 63;
        const float x0 = tmp[i], x1 = tmp[i + 64];
        if (t < 64) { const float p = x0 * cv, q = x1 * sv; o = p - q; }
        else        { const float p = x0 * sv, q = x1 * cv; o = p + q; }
    }
    __syncthreads();
    return o;
}

// RMSNorm over one 128-element head held by a wave (lane holds elements
// lane and lane + 64), then NEOX RoPE; returns the two rotated elements.
// The arithmetic of head_norm_rope, with the sum of squares reduced over the
// wave.
__device__ __forceinline__ void wave_norm_rope(float & x0, float & x1, const float * w, float eps, const float * c,
                                               const float * s) {
    const int l = threadIdx.x & 63;
    const double tot = wave_sum_d((double) (x0 * x0) + (double) (x1 * x1));
    const float mean = (float) (tot / (double) kHD);
    const float sc = 1.0f / sqrtf(mean + eps);
    float a0 = x0 * sc, a1 = x1 * sc;
    a0 = a0 * w[l];
    a1 = a1 * w[l + 64];
    const float p0 = a0 * c[l], q0 = a1 * s[l];
    const float p1 = a0 * s[l], q1 = a1 * c[l];
    x0 = p0 - q0;
    x1 = p1 + q1;
}

// Q8_0 quantisation of one value per lane, a block being 32 consecutive lanes
// (d = amax/127 as fp16, q = rint(x * 127/amax)); the block's first lane
// stores the scale.
__device__ __forceinline__ int8_t quant_lane32(float v, float * dx, bool first) {
    float am = fabsf(v);
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    const float d = am / 127.0f;
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    if (first) *dx = round_f16(d);
    return (int8_t) (int) rintf(v * id);
}

__global__ __launch_bounds__(kBlock) void k_attention(AttnArgs a) {
    {
        const int z = blockIdx.z;
        if (a.done && a.done[(size_t) z * a.done_stream]) return;
        a.kc += z * a.kv_stream; a.vc += z * a.kv_stream;
        a.qkv += (size_t) z * a.qkv_stream; a.out += (size_t) z * a.out_stream;
        if (a.out_q) { a.out_q += (size_t) z * a.out_stream; a.out_dx += (size_t) z * (a.out_stream / kQK); }
        if (a.pos_ptr) a.pos_ptr += (size_t) z * a.pos_stream;
    }
    extern __shared__ __align__(16) char smem[];
    double * red = (double *) smem;                   // 4 doubles
    float * fred = (float *) (smem + 32);             // 4 floats
    float * tmp = (float *) (smem + 64);              // 128
    float * qf = tmp + kHD;                           // 128: fp16-rounded rotated q
    float * knew = qf + kHD;                          // [4][128]
    float * vnew = knew + 4 * kHD;                    // [4][128]
    double * pv = (double *) (vnew + 4 * kHD);        // [4 waves][128]
    float * sc = (float *) (pv + 4 * kHD);            // [n_kv] scores, then fp16 probs

    const int h = blockIdx.x, tok = blockIdx.y, t = threadIdx.x;
    const int group = a.n_head / a.n_kv_head, g = h / group;
    const int qd = a.n_head * kHD, kd = a.n_kv_head * kHD;
    const int pos0 = a.pos_ptr ? *a.pos_ptr : a.pos_const;
    const int pos = pos0 + tok, n_kv = pos + 1;

    const int lane = t & 63, wave = t >> 6;
    const int sub = lane & 7, pw = lane >> 3;          // scores: 8 lanes per position
    const int dsub = lane & 15, pq = lane >> 4;        // P.V: 16 lanes per position
    const uint16_t * kbase = a.kc + (size_t) g * a.n_ctx * kHD;
    const uint16_t * vbase = a.vc + (size_t) g * a.n_ctx * kHD;
    // every global operand of the q row, the first new K/V row and the first
    // score and P.V steps is loaded here, once the position is known, so that
    // they cost one memory round trip instead of one per step
    const int i63 = t & 63;
    const float * row0 = a.qkv;
    const float * rowq = a.qkv + (size_t) tok * a.qkv_stride;
    const float qraw = t < kHD ? rowq[h * kHD + t] : 0.0f;
    const float wq = t < kHD ? a.q_norm[t] : 0.0f, wk = t < kHD ? a.k_norm[t] : 0.0f;
    const float cq = t < kHD ? a.rope_cos[(size_t) pos * 64 + i63] : 0.0f;
    const float sq = t < kHD ? a.rope_sin[(size_t) pos * 64 + i63] : 0.0f;
    const float ck0 = t < kHD ? a.rope_cos[(size_t) pos0 * 64 + i63] : 0.0f;
    const float sk0 = t < kHD ? a.rope_sin[(size_t) pos0 * 64 + i63] : 0.0f;
    const float k0raw = t < kHD ? row0[qd + g * kHD + t] : 0.0f;
    const float v0raw = t < kHD ? row0[qd + kd + g * kHD + t] : 0.0f;
    int4 kpre0 = make_int4(0, 0, 0, 0), kpre1 = kpre0, vpre = kpre0;
    if (!a.f32_new) {
        const int jk = wave * 8 + pw, jv = wave * 4 + pq;
        if (jk < n_kv && jk < pos0) {
            const int4 * kp = (const int4 *) (kbase + (size_t) jk * kHD + sub * 16);
            kpre0 = kp[0];
            kpre1 = kp[1];
        }
        if (jv < n_kv && jv < pos0) vpre = *(const int4 *) (vbase + (size_t) jv * kHD + dsub * 8);
    }
    // q of this head/token
    {
        const float o = head_norm_rope_v(qraw, wq, a.eps, cq, sq, tmp, red);
        if (t < kHD) qf[t] = a.f32_new ? o : round_kv(o, a.kv_bf16);
    }
    // k, v of this KV head for the chunk tokens 0..tok (positions >= pos0 are
    // never read from the cache inside this launch)
    for (int j = 0; j <= tok; ++j) {
        const float * row = a.qkv + (size_t) j * a.qkv_stride;
        float o;
        if (j == 0) {
            o = head_norm_rope_v(k0raw, wk, a.eps, ck0, sk0, tmp, red);
        } else {
            const float kvv = t < kHD ? row[qd + g * kHD + t] : 0.0f;
            o = head_norm_rope(kvv, a.k_norm, a.eps, a.rope_cos + (size_t) (pos0 + j) * 64,
                               a.rope_sin + (size_t) (pos0 + j) * 64, tmp, red);
        }
        if (t < kHD) {
            const float vraw = j == 0 ? v0raw : row[qd + kd + g * kHD + t];
            const uint16_t kh = f2kv(o, a.kv_bf16);
            const uint16_t vh = f2kv(vraw, a.kv_bf16);
            knew[j * kHD + t] = a.f32_new ? o : kv2f(kh, a.kv_bf16);
            vnew[j * kHD + t] = a.f32_new ? vraw : kv2f(vh, a.kv_bf16);
            if (j == tok && (h % group) == 0) {
                a.kc[((size_t) g * a.n_ctx + pos) * kHD + t] = kh;
                a.vc[((size_t) g * a.n_ctx + pos) * kHD + t] = vh;
            }
        }
    }
    __syncthreads();

    // scores: 8 lanes per position, 16 dims per lane
    float lmax = -INFINITY;
    if (a.f32_new) {
        // every position is a new fp32 row (pos0 = 0, n_kv <= 16): 4 lanes of
        // wave 0 per position, each a sequential 32-dim partial of exact fp64
        // products, combined (s0 + s1) + (s2 + s3)
        const int j = lane >> 2, s4 = lane & 3;
        double acc = 0.0;
        if (wave == 0 && j < n_kv) {
            const float * kr = knew + j * kHD + s4 * 32;
            const float * qq = qf + s4 * 32;
#pragma unroll
            for (int e = 0; e < 32; ++e) acc = fma((double) qq[e], (double) kr[e], acc);
        }
        acc += __shfl_xor(acc, 1);
        acc += __shfl_xor(acc, 2);
        if (wave == 0 && j < n_kv) {
            const float s = (float) acc * a.scale;
            if (s4 == 0) sc[j] = s;
            lmax = s;
        }
    }
    for (int j0 = 0; !a.f32_new && j0 < n_kv; j0 += 32) {
        const int j = j0 + wave * 8 + pw;
        double acc = 0.0;
        if (j < n_kv) {
            if (j < pos0) {
                const int4 * kp = (const int4 *) (kbase + (size_t) j * kHD + sub * 16);
                const int4 k0 = j0 == 0 ? kpre0 : kp[0], k1 = j0 == 0 ? kpre1 : kp[1];
                const uint16_t * kh0 = (const uint16_t *) &k0;
                const uint16_t * kh1 = (const uint16_t *) &k1;
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += (double) (qf[sub * 16 + e] * kv2f(kh0[e], a.kv_bf16));
#pragma unroll
                for (int e = 0; e < 8; ++e) acc += (double) (qf[sub * 16 + 8 + e] * kv2f(kh1[e], a.kv_bf16));
            } else {
                const float * kr = knew + (j - pos0) * kHD + sub * 16;
#pragma unroll
                for (int e = 0; e < 16; ++e) acc += (double) (qf[sub * 16 + e] * kr[e]);
            }
        }
        acc += __shfl_xor(acc, 4);
        acc += __shfl_xor(acc, 2);
        acc += __shfl_xor(acc, 1);
        if (j < n_kv) {
            const float s = (float) acc * a.scale;
            if (sub == 0) sc[j] = s;
            lmax = fmaxf(lmax, s);
        }
    }
    const float mx = block_max_f(lmax, fred);
    double lsum = 0.0;
    for (int j = t; j < n_kv; j += kBlock) {
        const float e = expf_q3t(sc[j] - mx);
        sc[j] = e;
        lsum += (double) e;
    }
    const double sum = block_sum_d(lsum, red);
    const float inv = (float) (1.0 / sum);
    for (int j = t; j < n_kv; j += kBlock) {
        const float p = sc[j] * inv;
        if (a.probs_out && tok == 0) a.probs_out[(size_t) h * n_kv + j] = p;
        sc[j] = a.f32_new ? p : round_kv(p, a.kv_bf16);
    }
    __syncthreads();

    // P.V: 16 lanes per position, 8 dims per lane, 4 positions per wave step
    double o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = 0.0;
    for (int j0 = 0; j0 < n_kv; j0 += 16) {
        const int j = j0 + wave * 4 + pq;
        if (j < n_kv) {
            const float p = sc[j];
            if (j < pos0) {
                const int4 vv = j0 == 0 ? vpre : *(const int4 *) (vbase + (size_t) j * kHD + dsub * 8);
                const uint16_t * vh = (const uint16_t *) &vv;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] += (double) p * (double) kv2f(vh[e], a.kv_bf16);
            } else {
                // fp16 x fp16 or (prefill) fp32 x fp32: exact in fp64 either way
                const float * vr = vnew + (j - pos0) * kHD + dsub * 8;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e] += (double) p * (double) vr[e];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        o[e] += __shfl_xor(o[e], 16);
        o[e] += __shfl_xor(o[e], 32);
    }
    if (pq == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) pv[wave * kHD + dsub * 8 + e] = o[e];
    }
    __syncthreads();
    if (t < kHD) {
        const double r = (pv[t] + pv[kHD + t]) + (pv[2 * kHD + t] + pv[3 * kHD + t]);
        const float o = (float) r;
        a.out[(size_t) tok * a.out_stride + h * kHD + t] = o;
        if (a.out_q) {
            // Q8_0 block = 32 consecutive threads of a fully active wave
            const size_t e = (size_t) tok * a.out_stride + h * kHD + t;
            a.out_q[e] = quant_lane32(o, a.out_dx + e / kQK, (t & 31) == 0);
        }
    }
}

__host__ __device__ constexpr size_t attn_lds_bytes(int n_ctx) {
    return 64 + (size_t) (2 * kHD + 8 * kHD) * 4 + (size_t) 4 * kHD * 8 + (size_t) n_ctx * 4;
}

// ---------------------------------------------------------------- sampler
struct SampleArgs {
    const float * logits; int32_t vocab;
    int32_t mode;                 // 0: talker codebook 0, 1: code predictor
    int32_t group;                // code-predictor codebook (1..15)
    const SampleParams * params;
    FrameState * st;
    uint8_t * seen;               // talker: codebook-0 tokens already generated
    int32_t eos_id;
    int32_t open_frame;           // mode 0: open a frame (frame loop); 0 for standalone calls
    int32_t * codes_out;          // mode 1, group 15: frame loop emits [frame][16] here (NULL: no emit)
    // input rows of the next pass, gathered once the token is known:
    //   mode 0        stage = [hidden; codec_embd[tok]]          (code-predictor prefill)
    //   mode 1, g<15  stage = code_pred_embd[g-1][tok]            (code-predictor step g)
    //   mode 1, g=15  stage = step embedding of the frame when codes_out is set (talker step)
    float * stage;
    const float * hidden;
    const uint16_t * codec_embd;
    const uint16_t * cp_embd[15];
    const float * trailing; int32_t n_trailing; const float * pad;
    int32_t d;
    // independent streams (blockIdx.x = stream): st and params are arrays;
    // element offsets per stream for the rest (0 for one stream)
    int32_t logits_stream, seen_stream, stage_stream, codes_stream, hidden_stream, trailing_stream, pad_stream;
    const int32_t * n_trailing_arr;   // per-stream trailing-row counts (NULL: n_trailing)
};

constexpr int kSampleThreads = 1024;
constexpr int kMaxVocab = 4096;

__device__ __forceinline__ uint32_t f2key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// LDS scratch of the sampling core for NTH threads.
template <int NTH>
struct SampleScratch {
    uint32_t hist[4][256];                   // one radix histogram per pass
    double dw[NTH / 64], dw2[NTH / 64];
    float fv[NTH / 64];
    int32_t iv[NTH / 64], iv2[NTH / 64];
    uint32_t uv[NTH / 64];
};
constexpr int kMaxSampleVocab = 3072;        // codec vocabulary; the host checks both vocabularies

template <int NTH>
__host__ __device__ constexpr int sample_chunk() { return (kMaxSampleVocab + NTH - 1) / NTH; }

// The sampled path of sample_core on logits held in registers: thread t owns
// the contiguous chunk [t*C, t*C + C), C = ceil(V / NTH), in x[0 .. C)
// (entries at or past V are ignored).  Cross-thread steps are wave
// reductions plus one workgroup barrier each.  Every thread returns the token.
template <int NTH>
__device__ int32_t sample_regs(float (&x)[sample_chunk<NTH>()], int V, float temperature, int top_k, int eos_id,
                               float eff, uint64_t seed, uint32_t frame, uint32_t group, SampleScratch<NTH> & S) {
    constexpr int NW = NTH / 64, MAXC = sample_chunk<NTH>();
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int C = (V + NTH - 1) / NTH;
    float lmax = -INFINITY;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = t * C + c;
        float v = -INFINITY;
        if (c < C && i < V) {
            v = x[c] / temperature;
            if (eff != 0.0f && i == eos_id) v += eff;
        }
        x[c] = v;
        lmax = fmaxf(lmax, v);
    }
    // the maximum survives the top-k filter, so it is taken here
    lmax = wave_max_f(lmax);
    if (lane == 0) S.fv[wave] = lmax;
    const bool topk = top_k > 0 && top_k < V;
    if (topk)
        for (int i = t; i < 4 * 256; i += NTH) (&S.hist[0][0])[i] = 0u;
    __syncthreads();
    float mx = S.fv[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) mx = fmaxf(mx, S.fv[w]);
    if (topk) {
        // radix select of the top_k-th largest key, 8 bits per pass from the
        // top; a pass whose selected bin holds exactly the keys still to go
        // ends the search with that bin's smallest key
        uint32_t k[MAXC];
#pragma unroll
        for (int c = 0; c < MAXC; ++c) k[c] = f2key(x[c]);
        uint32_t prefix = 0, mask = 0, thr_key = 0;
        int remaining = top_k;
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            uint32_t * hist = S.hist[pass];
#pragma unroll
            for (int c = 0; c < MAXC; ++c)
                if (c < C && t * C + c < V && (k[c] & mask) == prefix) atomicAdd(&hist[(k[c] >> shift) & 255u], 1u);
            __syncthreads();
            // every wave finds the bin holding the remaining-th largest key: the
            // highest b >= 1 with count(bins >= b) >= remaining (else bin 0);
            // lane l owns bins 4l .. 4l+3
            int h[4], own = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) { h[e] = (int) hist[4 * lane + e]; own += h[e]; }
            int incl = own;                        // keys in bins of lanes >= lane
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const int o = __shfl_down(incl, off);
                if (lane + off < 64) incl += o;
            }
            int above = incl - own, best = -1, best_above = 0, best_cnt = 0;
#pragma unroll
            for (int e = 3; e >= 0; --e) {
                const int b = 4 * lane + e;
                if (best < 0 && b >= 1 && above + h[e] >= remaining) { best = b; best_above = above; best_cnt = h[e]; }
                above += h[e];
            }
            int bmax = best;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) bmax = max(bmax, __shfl_xor(bmax, off));
            int bin, cnt;
            if (bmax >= 0) {
                const int owner = bmax >> 2;
                bin = bmax;
                remaining -= __shfl(best_above, owner);
                cnt = __shfl(best_cnt, owner);
            } else {
                bin = 0;
                remaining -= __shfl(incl, 0) - __shfl(h[0], 0);
                cnt = __shfl(h[0], 0);
            }
            prefix |= (uint32_t) bin << shift;
            mask |= 255u << shift;
            if (pass == 3) { thr_key = prefix; break; }
            if (cnt == remaining) {
                uint32_t m = 0xffffffffu;
#pragma unroll
                for (int c = 0; c < MAXC; ++c)
                    if (c < C && t * C + c < V && (k[c] & mask) == prefix) m = min(m, k[c]);
#pragma unroll
                for (int off = 32; off > 0; off >>= 1) m = min(m, (uint32_t) __shfl_xor((int) m, off));
                if (lane == 0) S.uv[wave] = m;
                __syncthreads();
                thr_key = S.uv[0];
#pragma unroll
                for (int w = 1; w < NW; ++w) thr_key = min(thr_key, S.uv[w]);
                break;
            }
        }
        const float thr = key2f(thr_key);
#pragma unroll
        for (int c = 0; c < MAXC; ++c)
            if (x[c] < thr) x[c] = -INFINITY;
    }
    // softmax: exp and the fp64 denominator
    double ls = 0.0;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        x[c] = c < C ? expf_q3t(x[c] - mx) : 0.0f;
        ls += (double) x[c];
    }
    ls = wave_sum_d(ls);
    if (lane == 0) S.dw[wave] = ls;
    __syncthreads();
    double sum = S.dw[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) sum += S.dw[w];
    // fp32 probabilities and the inclusive prefix of the per-thread sums (the CDF)
    double lp = 0.0;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        x[c] = (float) ((double) x[c] / sum);
        lp += (double) x[c];
    }
    double incl = lp;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(incl, off);
        if (lane >= off) incl += o;
    }
    if (lane == 63) S.dw2[wave] = incl;
    __syncthreads();
    double base = 0.0, total = 0.0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        if (w < wave) base += S.dw2[w];
        total += S.dw2[w];
    }
    const double u = philox_uniform(seed, frame, group);
    const double target = u * total;
    // the first index whose running sum passes the target, else the last
    // index of positive probability
    double cum = base + (incl - lp);
    int first = 0x7fffffff, last = -1;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = t * C + c;
        if (c < C && i < V && x[c] > 0.0f && first == 0x7fffffff) {
            cum += (double) x[c];
            last = i;
            if (cum > target) first = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        first = min(first, __shfl_xor(first, off));
        last = max(last, __shfl_xor(last, off));
    }
    if (lane == 0) { S.iv[wave] = first; S.iv2[wave] = last; }
    __syncthreads();
    int pick = S.iv[0], lastp = S.iv2[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) { pick = min(pick, S.iv[w]); lastp = max(lastp, S.iv2[w]); }
    __syncthreads();
    return pick != 0x7fffffff ? pick : (lastp >= 0 ? lastp : 0);
}

// Token from prepared logits l[0..V) in LDS (suppression / penalty already
// applied; `eff` is the EOS bias for the talker, 0 otherwise), following
// sample_or_argmax (src/tts_transformer.cpp:2750-2788) and the talker sampler
// (:3146-3183): greedy first-index argmax, or temperature, EOS bias, top-k
// threshold (ties kept), softmax with fp64 denominator, draw against the
// Philox uniform of (seed, frame, group).  Every thread returns the token.
// The greedy path adds the EOS bias into l.
template <int NTH>
__device__ int32_t sample_core(float * l, int V, float temperature, int top_k, int eos_id, float eff,
                               uint64_t seed, uint32_t frame, uint32_t group, SampleScratch<NTH> & S) {
    const int t = threadIdx.x;
    if (temperature <= 0.0f) {
        if (eff != 0.0f && t == 0) l[eos_id] += eff;
        __syncthreads();
        // empty = (-inf, INT_MAX); ascending scan with strict '>' keeps the first maximum
        float bv = -INFINITY; int32_t bi = 0x7fffffff;
        for (int i = t; i < V; i += NTH)
            if (l[i] > bv || (l[i] == bv && i < bi)) { bv = l[i]; bi = i; }
        wave_argmax(bv, bi);
        if ((t & 63) == 0) { S.fv[t >> 6] = bv; S.iv[t >> 6] = bi; }
        __syncthreads();
        float b = S.fv[0]; int32_t i0 = S.iv[0];
        for (int w = 1; w < NTH / 64; ++w)
            if (S.fv[w] > b || (S.fv[w] == b && S.iv[w] < i0)) { b = S.fv[w]; i0 = S.iv[w]; }
        __syncthreads();
        return i0;
    }
    constexpr int MAXC = sample_chunk<NTH>();
    const int C = (V + NTH - 1) / NTH;
    float x[MAXC];
#pragma unroll
    for (int c = 0; c < MAXC; ++c) x[c] = c < C && t * C + c < V ? l[t * C + c] : -INFINITY;
    return sample_regs<NTH>(x, V, temperature, top_k, eos_id, eff, seed, frame, group, S);
}

// The argument block is never modified: its table of code-predictor
// embeddings is indexed by a runtime group, and a modified copy would be
// moved to scratch memory for that.
__global__ __launch_bounds__(kSampleThreads) void k_sample(const SampleArgs a) {
    const int b = blockIdx.x;
    FrameState * st = a.st + b;
    const SampleParams & P = a.params[b];
    const float * logits = a.logits + (size_t) b * a.logits_stream;
    uint8_t * seen = a.seen + (size_t) b * a.seen_stream;
    float * stage = a.stage ? a.stage + (size_t) b * a.stage_stream : nullptr;
    int32_t * codes_out = a.codes_out ? a.codes_out + (size_t) b * a.codes_stream : nullptr;
    const float * hidden = a.hidden ? a.hidden + (size_t) b * a.hidden_stream : nullptr;
    const float * trailing = a.trailing ? a.trailing + (size_t) b * a.trailing_stream : nullptr;
    const float * pad = a.pad ? a.pad + (size_t) b * a.pad_stream : nullptr;
    const int32_t n_trailing = a.n_trailing_arr ? a.n_trailing_arr[b] : a.n_trailing;
    __shared__ int32_t s_frame;
    if (threadIdx.x == 0) {
        int32_t f = st->frame;
        if (a.mode == 0 && a.open_frame && !st->done) {
            f = st->next_frame;
            if (f >= st->max_frames) st->done = 1;
            else { st->frame = f; st->next_frame = f + 1; st->talker_pos = st->base_pos + f; }
        }
        s_frame = st->done ? -1 : f;
    }
    __syncthreads();
    if (s_frame < 0) return;
    __shared__ float l[kMaxVocab];
    __shared__ SampleScratch<kSampleThreads> S;
    const int t = threadIdx.x, V = a.vocab;
    const int frame = s_frame;
    for (int i = t; i < V; i += kSampleThreads) {
        float v = logits[i];
        if (a.mode == 0) {
            if (i >= V - 1024 && i != a.eos_id) v = -INFINITY;
            if (P.rep_penalty != 1.0f && seen[i]) v = v > 0.0f ? v / P.rep_penalty : v * P.rep_penalty;
        }
        l[i] = v;
    }
    float eff = 0.0f;
    if (a.mode == 0) {
        eff = P.eos_bias;
        if (P.target_frames > 0 && frame > P.target_frames) {
            eff += 0.1f * (float) (frame - P.target_frames);
            if (eff > 6.0f) eff = 6.0f;
        }
    }
    __syncthreads();
    const int32_t tok = sample_core<kSampleThreads>(l, V, P.temperature, P.top_k, a.eos_id, eff, P.seed,
                                                    (uint32_t) frame, a.mode == 0 ? 0u : (uint32_t) a.group, S);
    if (t == 0) {
        if (a.mode == 0) {
            st->codes[0] = tok;
            if (tok == a.eos_id) { st->done = 1; st->eos = 1; }
            else seen[tok] = 1;
        } else {
            st->codes[a.group] = tok;
            if (codes_out && a.group == 15) {
                for (int g = 0; g < 15; ++g) codes_out[(size_t) frame * 16 + g] = st->codes[g];
                codes_out[(size_t) frame * 16 + 15] = tok;
                st->n_emitted = frame + 1;
            }
        }
    }
    if (!stage) return;
    const size_t d = (size_t) a.d;
    if (a.mode == 0) {
        if (tok == a.eos_id) return;
        for (int e = t; e < a.d; e += kSampleThreads) {
            stage[e] = hidden[e];
            stage[d + e] = h2f(a.codec_embd[(size_t) tok * d + e]);
        }
    } else if (a.group < 15) {
        const uint16_t * row = a.cp_embd[a.group - 1] + (size_t) tok * d;
        for (int e = t; e < a.d; e += kSampleThreads) stage[e] = h2f(row[e]);
    } else if (codes_out) {
        // step embedding (src/tts_transformer.cpp:3264-3295), summed in the reference order
        __shared__ int32_t sc[16];
        if (t < 15) sc[t] = st->codes[t];
        __syncthreads();
        for (int e = t; e < a.d; e += kSampleThreads) {
            float s = h2f(a.codec_embd[(size_t) sc[0] * d + e]);
            for (int g = 1; g < 15; ++g) s = s + h2f(a.cp_embd[g - 1][(size_t) sc[g] * d + e]);
            s = s + h2f(a.cp_embd[14][(size_t) tok * d + e]);
            const float tr = frame < n_trailing ? trailing[(size_t) frame * d + e] : pad[e];
            stage[e] = s + tr;
        }
    }
}

// code-predictor prefill input rows for a standalone call: [hidden; codec_embd[codes[0]]]
__global__ void k_cp_input(const FrameState * st, const float * hidden, const uint16_t * codec_embd, int32_t d,
                           float * stage) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= d) return;
    stage[e] = hidden[e];
    stage[d + e] = h2f(codec_embd[(size_t) st->codes[0] * d + e]);
}

// The single-pass code predictor's input row (src/tts_transformer.cpp:1801-1808):
// hidden + code_pred.codec_embd[g][codes[g]] for g = 0 .. n-1, added in that
// order in fp32.  Codes are checked on the host.
struct SingleInArgs {
    const float * hidden;
    float * out;
    int32_t d, n;
    int32_t codes[15];
    const uint16_t * embd[15];
};

__global__ void k_cp_single_input(SingleInArgs a) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= a.d) return;
    float v = a.hidden[e];
    for (int g = 0; g < a.n; ++g) v = v + h2f(a.embd[g][(size_t) a.codes[g] * a.d + e]);
    a.out[e] = v;
}

// Attention of one position over itself (src/tts_transformer.cpp:1855-1864):
// the softmax of a single score is exactly 1, so query head h's output is the
// fp32 V row of its KV head h / group.
__global__ void k_v_to_heads(const float * v, int32_t head_dim, int32_t group, int32_t n_head, float * out) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= n_head * head_dim) return;
    const int h = e / head_dim, i = e - h * head_dim;
    out[e] = v[(size_t) (h / group) * head_dim + i];
}

// normed rows for the prefill's all-token hidden output
__global__ __launch_bounds__(kBlock) void k_rmsnorm_rows(const float * x, const float * w, float eps, int32_t d,
                                                        float * y) {
    __shared__ double red[4];
    const float * xr = x + (size_t) blockIdx.x * d;
    double ss = 0.0;
    for (int e = threadIdx.x; e < d; e += kBlock) { const float v = xr[e]; ss += (double) (v * v); }
    const double tot = block_sum_d(ss, red);
    const float mean = (float) (tot / (double) d);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int e = threadIdx.x; e < d; e += kBlock) { float v = xr[e] * scale; y[(size_t) blockIdx.x * d + e] = v * w[e]; }
}

// dequantise a repacked Q8_0 tensor: out = fp32(d) * q
__global__ void k_dequant_q8(const int8_t * q, const uint16_t * d, int64_t n, float * out) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = h2f(d[i / kQK]) * (float) q[i];
}

// gather rows of an fp16 table into fp32 rows (token ids from host copy)
__global__ void k_gather_rows(const uint16_t * table, int64_t dim, const int32_t * ids, int32_t n, float * out) {
    const int r = blockIdx.y;
    for (int64_t e = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; e < dim; e += (int64_t) gridDim.x * blockDim.x)
        out[(size_t) r * dim + e] = h2f(table[(size_t) ids[r] * dim + e]);
}

// x = silu(x) over count elements (fc1 of the text projection after its
// bias add: silu_q3t(v + b), the GEMV's EPI_BIAS_SILU, in two steps).
__global__ void k_silu_rows(float * x, size_t count) {
    for (size_t i = (size_t) blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (size_t) gridDim.x * blockDim.x)
        x[i] = silu_q3t(x[i]);
}

// ---------------------------------------------------- prefill row assembly
// The rows of build_prefill_graph (src/tts_transformer.cpp:1030-1186) and
// build_prefill_graph_icl (:1188-1472): every output row is one source row,
// the sum of two (a + b), or the ICL interleave's (0 + a) + b, each an fp32
// addition in the order the reference's host loops make it.  Sources:
// projected text rows, talker.codec_embd rows (F16, exact in fp32), the
// speaker row, or an ICL reference frame's summed embeddings
// (codec_embd[c0], then + code_pred.codec_embd[cb-1][c_cb] for cb = 1..15 in
// order, :1348-1367).
enum RowSrc : int32_t { RS_PROJ = 0, RS_CODEC = 1, RS_SPEAKER = 2, RS_FRAME = 3 };
enum RowOp : int32_t { RO_COPY = 0, RO_ADD = 1, RO_ZERO_ADD = 2 };
struct RowSpec {
    int32_t op, a_src, a_idx, b_src, b_idx;
};
struct RowTables {
    const float * proj;              // projected text rows [m][d]
    const uint16_t * codec_embd;     // [codec_vocab][d]
    const uint16_t * cp_embd[15];    // [cp_vocab][d] each
    const float * speaker;           // [d]
    const int32_t * frames;          // reference codes [n_frames][16]
    int32_t n_cb, d;
};

__device__ __forceinline__ float row_src(const RowTables & T, int src, int idx, int h) {
    if (src == RS_PROJ) return T.proj[(size_t) idx * T.d + h];
    if (src == RS_CODEC) return h2f(T.codec_embd[(size_t) idx * T.d + h]);
    if (src == RS_SPEAKER) return T.speaker[h];
    const int32_t * f = T.frames + (size_t) idx * 16;
    float r = h2f(T.codec_embd[(size_t) f[0] * T.d + h]);
    for (int cb = 1; cb < 16 && cb < T.n_cb; ++cb) r = r + h2f(T.cp_embd[cb - 1][(size_t) f[cb] * T.d + h]);
    return r;
}

// Block (x, row): out[row] from specs[row].  Every index was range-checked on
// the host.
__global__ void k_prefill_rows(RowTables T, const RowSpec * specs, float * out) {
    const RowSpec s = specs[blockIdx.y];
    for (int h = (int) (blockIdx.x * blockDim.x + threadIdx.x); h < T.d; h += (int) (gridDim.x * blockDim.x)) {
        const float a = row_src(T, s.a_src, s.a_idx, h);
        float o = a;
        if (s.op != RO_COPY) {
            const float b = row_src(T, s.b_src, s.b_idx, h);
            o = s.op == RO_ADD ? a + b : (0.0f + a) + b;
        }
        out[(size_t) blockIdx.y * T.d + h] = o;
    }
}

}  // namespace q3t

#include "q3t_gemv_reg.h"
