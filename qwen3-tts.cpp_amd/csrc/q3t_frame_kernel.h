// q3t_frame_kernel.h -- the whole frame (codebook-0 sample, 2-token
// code-predictor prefill + 14 steps, talker step) as ONE persistent kernel.
//
// Why: at batch 1 every phase of the loop moves a few MB, so a frame of
// ~550 dependent kernels is bound by per-kernel latency (launch, end-of-kernel
// cache maintenance, refetch of the activation), not by HBM bandwidth.  Here
// all workgroups stay resident for the frame and hand data from phase to
// phase through "tagged" 8-byte elements: a producer writes {epoch, fp32
// value} with one 64-bit store, a consumer polls until the epoch matches.
// One round trip per dependency, no atomics, no fences, no barriers.
//
//   - every workgroup runs the same straight-line program of phases; phase
//     p of frame f carries tag ((f + 1) << 12) | p and owns arena slot p;
//   - a workgroup prefetches its phase weights into registers before it
//     polls the phase input, so weight latency hides behind the wait;
//   - workgroup g (< n_kv_head) owns KV head g for attention; the code
//     predictor's 16-position KV cache lives in that workgroup's LDS for the
//     whole frame;
//   - samplers run redundantly in every workgroup that needs the token (all
//     compute the same token from the same tagged logits); workgroup 0
//     alone writes the frame state and the emitted codes;
//   - every wait is bounded: a timeout marks the thread dead (it never waits
//     again), sets an error flag the host reads after the frame, so a bug
//     cannot hang the GPU.
// Numerics are those of the multi-kernel path (q3t_gemv_reg.h, k_attention,
// sample_core): fp64 accumulation of exact terms, identical rounding points.
#pragma once

#include "q3t_kernels.h"

namespace q3t {
namespace fk {

constexpr int kT = 256;                 // threads per workgroup
constexpr int kW = kT / 64;             // waves per workgroup
constexpr int kSlot = 8192;             // tagged elements per phase slot
constexpr int kMaxCtx = 4096;           // talker positions the attention phase can hold in LDS
constexpr unsigned kSpin = 1u << 20;    // polls before a wait gives up
constexpr int kCpLayers = 5;            // code-predictor layers whose KV fits in LDS

struct LayerQ8 {
    const int8_t * qkv; const uint16_t * qkv_d;
    const int8_t * wo; const uint16_t * wo_d;
    const int8_t * wg; const uint16_t * wg_d;
    const int8_t * wu; const uint16_t * wu_d;
    const int8_t * wd; const uint16_t * wd_d;
    const float * attn_norm; const float * ffn_norm; const float * q_norm; const float * k_norm;
};

struct Args {
    const LayerQ8 * talker; const LayerQ8 * cp;
    int32_t n_layers, cp_layers, d, n_head, n_kv_head, ffn, cp_ffn, codec_vocab, cp_vocab, eos_id, n_ctx;
    float eps, attn_scale;
    const uint16_t * codec_embd;
    const uint16_t * cp_embd[15];
    const uint16_t * cp_head[15];
    const uint16_t * codec_head;
    const float * out_norm; const float * cp_out_norm;
    const float * rope_cos; const float * rope_sin; const float * cp_rope_cos; const float * cp_rope_sin;
    uint16_t * kc; uint16_t * vc;            // talker KV, [layer][n_kv_head][n_ctx][128]
    uint64_t * arena;                        // tagged phase slots
    float * logits; float * hidden;          // talker head outputs, read by the next frame
    FrameState * st; const SampleParams * params; uint8_t * seen; int32_t * codes_out;
    const float * trailing; int32_t n_trailing; const float * pad;
    int32_t * err;
};

struct Lds {
    float x[2 * 3072];                      // phase input rows / logits
    float a[2 * 4 * 128];                   // attention: q (2 heads x 2 tok), new k, new v rows
    float sc[2 * kMaxCtx];                  // attention scores / probabilities, 2 heads
    double pv[kW * 128];
    uint16_t cpk[kCpLayers][16 * 128];      // code-predictor KV of this workgroup's KV head, per layer
    uint16_t cpv[kCpLayers][16 * 128];
    double red[kW];
    float fred[kW];
    int32_t codes[16];
    SampleScratch<kT> S;
};

// ---------------------------------------------------------------- tagged I/O
__device__ __forceinline__ uint64_t tload(const uint64_t * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t * p, uint32_t tag, float v) {
    __hip_atomic_store(p, ((uint64_t) tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float twait(const uint64_t * p, uint32_t tag, bool & dead, int32_t * err) {
    uint64_t v = tload(p);
    unsigned n = 0;
    while ((uint32_t) (v >> 32) != tag && !dead) {
        if (++n > kSpin) { dead = true; atomicExch(err, 1); break; }
        __builtin_amdgcn_s_sleep(1);
        v = tload(p);
    }
    return __uint_as_float((uint32_t) v);
}
// Waits for up to kB tagged elements at once: all loads are issued before
// any tag is checked, and a re-poll reloads only the elements still missing,
// so a thread pays about one round trip per batch instead of one per element.
constexpr int kB = 8;
__device__ __forceinline__ void twait_batch(const uint64_t * const (&ptr)[kB], int cnt, uint32_t tag, float (&out)[kB],
                                            bool & dead, int32_t * err) {
    uint64_t v[kB];
#pragma unroll
    for (int k = 0; k < kB; ++k) v[k] = k < cnt ? tload(ptr[k]) : ((uint64_t) tag << 32);
    unsigned n = 0;
    while (!dead) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < kB; ++k) all = all && (uint32_t) (v[k] >> 32) == tag;
        if (all) break;
        if (++n > kSpin) { dead = true; atomicExch(err, 1); break; }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < kB; ++k)
            if ((uint32_t) (v[k] >> 32) != tag) v[k] = tload(ptr[k]);
    }
#pragma unroll
    for (int k = 0; k < kB; ++k) out[k] = __uint_as_float((uint32_t) v[k]);
}

// all threads: rows [nt][n] of a tagged slot (row stride `stride`) into LDS dst [nt][n]
__device__ __forceinline__ void stage(const uint64_t * slot, int nt, int n, int stride, uint32_t tag, float * dst,
                                      bool & dead, int32_t * err) {
    const int total = nt * n;
    for (int e0 = 0; e0 < total; e0 += kB * kT) {
        const uint64_t * ptr[kB];
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const int e = e0 + k * kT + (int) threadIdx.x;
            const int tt = e < total ? e / n : 0, i = e < total ? e - tt * n : 0;
            ptr[k] = slot + (size_t) tt * stride + i;
            if (e < total) cnt = k + 1;
        }
        float val[kB];
        twait_batch(ptr, cnt, tag, val, dead, err);
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const int e = e0 + k * kT + (int) threadIdx.x;
            if (e < total) dst[e] = val[k];
        }
    }
    __syncthreads();
}

__device__ __forceinline__ double wg_sum(double v, double * red) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    double s = red[0];
    for (int w = 1; w < kW; ++w) s += red[w];
    __syncthreads();
    return s;
}
__device__ __forceinline__ float wg_max(float v, float * red) {
    v = wave_max_f(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
    for (int w = 1; w < kW; ++w) s = fmaxf(s, red[w]);
    __syncthreads();
    return s;
}

// ------------------------------------------------------------------- GEMV
// Row groups of a GEMV are dealt to the grid's waves: wave gw takes groups
// gw and gw + nwaves (at most two per wave; the host checks).
template <int SLOTS, bool DUAL>
struct Q8Regs {
    int4 w[2][SLOTS][2], u[2][SLOTS][2];
    float dw[2][SLOTS], du[2][SLOTS];
    uint64_t res[2][2];   // residual elements (tagged) read early by the storing lanes
    int ng;          // groups this wave owns (0..2)
};

template <int SLOTS, bool DUAL>
__device__ __forceinline__ void q8_prefetch(Q8Regs<SLOTS, DUAL> & R, const int8_t * W, const uint16_t * Wd,
                                            const int8_t * U, const uint16_t * Ud, int rows, int K) {
    const int BPR = K / kQK, LPR = BPR / SLOTS, RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, lir = lane & (LPR - 1), rsub = lane / LPR;
    const int groups = rows / RPW;
    const int gw = blockIdx.x * kW + (threadIdx.x >> 6), nw = gridDim.x * kW;
    R.ng = 0;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = gw + gi * nw;
        if (g >= groups) break;
        R.ng = gi + 1;
        const int r = g * RPW + rsub;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const int b = lir + s * LPR;
            const int4 * wp = (const int4 *) (W + (size_t) r * K + b * kQK);
            R.w[gi][s][0] = wp[0]; R.w[gi][s][1] = wp[1];
            R.dw[gi][s] = h2f(Wd[(size_t) r * BPR + b]);
            if (DUAL) {
                const int4 * up = (const int4 *) (U + (size_t) r * K + b * kQK);
                R.u[gi][s][0] = up[0]; R.u[gi][s][1] = up[1];
                R.du[gi][s] = h2f(Ud[(size_t) r * BPR + b]);
            }
        }
    }
}

// Issues the residual loads of the rows this lane will store (EPI_RESID),
// before the phase input is awaited; q8_compute re-polls any not yet tagged.
template <int NT, int SLOTS, bool DUAL>
__device__ __forceinline__ void res_prefetch(Q8Regs<SLOTS, DUAL> & R, int K, const uint64_t * res, int res_stride) {
    const int BPR = K / kQK, LPR = BPR / SLOTS, RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, lir = lane & (LPR - 1), rsub = lane / LPR;
    const int gw = blockIdx.x * kW + (threadIdx.x >> 6), nw = gridDim.x * kW;
    if (lir != 0) return;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) R.res[gi][t] = tload(res + (size_t) t * res_stride + r);
    }
}

__device__ __forceinline__ bool wg_has_rows(int rows, int K, int slots) {
    const int LPR = (K / kQK) / slots, RPW = 64 / LPR;
    return blockIdx.x * kW < rows / RPW;
}

// One lane's 32-element block of token `tok` from LDS x [nt][K].
__device__ __forceinline__ void blk_lds(const float * x, int K, int tok, int blk, float (&v)[32]) {
    const float4 * p = (const float4 *) (x + (size_t) tok * K + blk * kQK);
#pragma unroll
    for (int c = 0; c < 8; ++c) { const float4 q = p[c]; v[4 * c] = q.x; v[4 * c + 1] = q.y; v[4 * c + 2] = q.z; v[4 * c + 3] = q.w; }
}

// Q8_0 GEMV over LDS input x [NT][K] (optionally RMSNorm'd with norm_w),
// epilogue, tagged stores into out [NT][out_stride].  res: residual slot
// (tagged, read by the storing lane) for EPI_RESID.
template <int NT, int SLOTS, bool DUAL>
__device__ __forceinline__ void q8_compute(const Q8Regs<SLOTS, DUAL> & R, int rows, int K, const float * x,
                                           const float * norm_w, float eps, int epi, const uint64_t * res,
                                           uint32_t res_tag, int res_stride, uint64_t * out, uint32_t out_tag,
                                           int out_stride, bool & dead, int32_t * err) {
    if (R.ng == 0) return;
    const int BPR = K / kQK, LPR = BPR / SLOTS, RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, lir = lane & (LPR - 1), rsub = lane / LPR;
    const int gw = blockIdx.x * kW + (threadIdx.x >> 6), nw = gridDim.x * kW;
    float scale[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        scale[t] = 1.0f;
        if (norm_w) {
            double ss = 0.0;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                float v[32];
                blk_lds(x, K, t, lir + s * LPR, v);
#pragma unroll
                for (int j = 0; j < 32; ++j) ss += (double) (v[j] * v[j]);
            }
            ss = group_sum_d(ss, LPR);
            const float mean = (float) (ss / (double) K);
            scale[t] = 1.0f / sqrtf(mean + eps);
        }
    }
    double acc[2][NT], acc2[2][NT];
#pragma unroll
    for (int gi = 0; gi < 2; ++gi)
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[gi][t] = 0.0; acc2[gi][t] = 0.0; }
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int b = lir + s * LPR;
        float nw_[32];
        if (norm_w) {
            const float4 * p = (const float4 *) (norm_w + b * kQK);
#pragma unroll
            for (int c = 0; c < 8; ++c) { const float4 q = p[c]; nw_[4 * c] = q.x; nw_[4 * c + 1] = q.y; nw_[4 * c + 2] = q.z; nw_[4 * c + 3] = q.w; }
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v[32];
            blk_lds(x, K, t, b, v);
            if (norm_w) {
#pragma unroll
                for (int j = 0; j < 32; ++j) { const float y = v[j] * scale[t]; v[j] = y * nw_[j]; }
            }
            float am = 0.0f;
#pragma unroll
            for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(v[j]));
            const float d = am / 127.0f;
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            int q[8];
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const int a0 = (int) rintf(v[4 * c] * id), a1 = (int) rintf(v[4 * c + 1] * id);
                const int a2 = (int) rintf(v[4 * c + 2] * id), a3 = (int) rintf(v[4 * c + 3] * id);
                q[c] = (a0 & 0xff) | ((a1 & 0xff) << 8) | ((a2 & 0xff) << 16) | ((int) ((unsigned) a3 << 24));
            }
            const int4 x0 = make_int4(q[0], q[1], q[2], q[3]), x1 = make_int4(q[4], q[5], q[6], q[7]);
            const float dx = round_f16(d);
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                if (gi >= R.ng) break;
                acc[gi][t] += (double) (R.dw[gi][s] * dx) * (double) dot32_i8(R.w[gi][s][0], R.w[gi][s][1], x0, x1);
                if (DUAL) acc2[gi][t] += (double) (R.du[gi][s] * dx) * (double) dot32_i8(R.u[gi][s][0], R.u[gi][s][1], x0, x1);
            }
        }
    }
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double a1 = group_sum_d(acc[gi][t], LPR);
            const double a2 = DUAL ? group_sum_d(acc2[gi][t], LPR) : 0.0;
            if (lir != 0) continue;
            const float v = (float) a1;
            float o;
            if (epi == EPI_RESID) {
                const uint64_t rv = R.res[gi][t];
                o = v + ((uint32_t) (rv >> 32) == res_tag ? __uint_as_float((uint32_t) rv)
                                                          : twait(res + (size_t) t * res_stride + r, res_tag, dead, err));
            }
            else if (epi == EPI_SWIGLU) o = silu_q3t(v) * (float) a2;
            else o = v;
            tstore(out + (size_t) t * out_stride + r, out_tag, o);
        }
    }
}

// F16 head GEMV (K = d, one slot per lane), RMSNorm'd input row in LDS.
// Outputs tagged (code predictor) or plain (talker: logits, plus the normed
// hidden written by workgroup 0).
__device__ __forceinline__ void f16_head(const uint16_t * W, int rows, int K, const float * x, const float * norm_w,
                                         float eps, uint64_t * out_tagged, uint32_t tag, float * out_plain,
                                         float * hidden_out) {
    const int BPR = K / kQK, LPR = BPR, RPW = 64 / LPR;   // K <= 1024
    const int lane = threadIdx.x & 63, lir = lane & (LPR - 1), rsub = lane / LPR;
    const int groups = rows / RPW;
    const int gw = blockIdx.x * kW + (threadIdx.x >> 6), nw = gridDim.x * kW;
    int4 w[2][4];
    int ng = 0;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = gw + gi * nw;
        if (g >= groups) break;
        ng = gi + 1;
        const int4 * wp = (const int4 *) (W + (size_t) (g * RPW + rsub) * K + lir * kQK);
#pragma unroll
        for (int c = 0; c < 4; ++c) w[gi][c] = wp[c];
    }
    float v[32];
    blk_lds(x, K, 0, lir, v);
    double ss = 0.0;
#pragma unroll
    for (int j = 0; j < 32; ++j) ss += (double) (v[j] * v[j]);
    ss = group_sum_d(ss, LPR);
    const float scale = 1.0f / sqrtf((float) (ss / (double) K) + eps);
    const float4 * np = (const float4 *) (norm_w + lir * kQK);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float4 q = np[c];
        float y;
        y = v[4 * c] * scale; v[4 * c] = y * q.x;
        y = v[4 * c + 1] * scale; v[4 * c + 1] = y * q.y;
        y = v[4 * c + 2] * scale; v[4 * c + 2] = y * q.z;
        y = v[4 * c + 3] * scale; v[4 * c + 3] = y * q.w;
    }
    if (hidden_out && blockIdx.x == 0 && threadIdx.x < LPR) {
#pragma unroll
        for (int j = 0; j < 32; ++j) hidden_out[lir * kQK + j] = v[j];
    }
    if (ng == 0) return;
    double acc[2] = {0.0, 0.0};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float xf = round_f16(v[8 * c + j]);
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                const uint16_t * wh = (const uint16_t *) &w[gi][c];
                acc[gi] += (double) (h2f(wh[j]) * xf);
            }
        }
    }
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        if (gi >= ng) break;
        const double a = group_sum_d(acc[gi], LPR);
        if (lir != 0) continue;
        const int r = (gw + gi * nw) * RPW + rsub;
        if (out_tagged) tstore(out_tagged + r, tag, (float) a);
        else out_plain[r] = (float) a;
    }
}

// -------------------------------------------------------------- attention
// QK-norm + NEOX RoPE of one 128-row held by threads 0..127 (value v);
// returns the rotated element for threads < 128.
__device__ __forceinline__ float norm_rope(float v, const float * w, float eps, const float * c, const float * s,
                                           float * tmp, double * red) {
    const int t = threadIdx.x;
    const double ss = wg_sum(t < 128 ? (double) (v * v) : 0.0, red);
    const float mean = (float) (ss / 128.0);
    const float scale = 1.0f / sqrtf(mean + eps);
    if (t < 128) { float y = v * scale; tmp[t] = y * w[t]; }
    __syncthreads();
    float o = 0.0f;
    if (t < 128) {
        const int i = t & 63;
        const float x0 = tmp[i], x1 = tmp[i + 64];
        if (t < 64) { const float p = x0 * c[i], q = x1 * s[i]; o = p - q; }
        else        { const float p = x0 * s[i], q = x1 * c[i]; o = p + q; }
    }
    __syncthreads();
    return o;
}

// Attention of KV head g = blockIdx.x for its `group` query heads and nt
// tokens at positions pos0.. (causal).  Talker (cp == false): positions
// < pos0 from the HBM cache, new rows appended there; code predictor: all
// rows in this workgroup's LDS.
__device__ void attention_phase(const Args & A, Lds & L, const LayerQ8 & W, int layer, bool cp, int nt, int pos0,
                                const uint64_t * qkv, uint32_t qkv_tag, uint64_t * out, uint32_t out_tag,
                                bool & dead) {
    const int g = blockIdx.x, t = threadIdx.x;
    const int group = A.n_head / A.n_kv_head, qd = A.n_head * 128, kd = A.n_kv_head * 128, qkvd = qd + 2 * kd;
    const float * rc = cp ? A.cp_rope_cos : A.rope_cos;
    const float * rs = cp ? A.cp_rope_sin : A.rope_sin;
    float * qf = L.a;                      // [group][nt][128] rotated, fp16-rounded q
    float * knew = L.a + 4 * 128;          // [nt][128]
    float * vnew = knew + 2 * 128;         // [nt][128]
    float * tmp = L.x;                     // 128 scratch
    uint16_t * kc = A.kc + ((size_t) layer * A.n_kv_head + g) * A.n_ctx * 128;
    uint16_t * vc = A.vc + ((size_t) layer * A.n_kv_head + g) * A.n_ctx * 128;
    // stage this head group's q, k, v rows
    float qraw[2][2], kraw[2], vraw[2];
    {
        // (q0, q1, k, v) of each token, one batch; threads >= 128 load nothing
        const uint64_t * ptr[kB];
        const int tc = t < 128 ? t : 0;
#pragma unroll
        for (int tok = 0; tok < 2; ++tok) {
            const uint64_t * row = qkv + (size_t) (tok < nt ? tok : 0) * kSlot / 2;
            ptr[4 * tok + 0] = row + (g * group + 0) * 128 + tc;
            ptr[4 * tok + 1] = row + (g * group + 1) * 128 + tc;
            ptr[4 * tok + 2] = row + qd + g * 128 + tc;
            ptr[4 * tok + 3] = row + qd + kd + g * 128 + tc;
        }
        float val[kB];
        twait_batch(ptr, t < 128 ? 4 * nt : 0, qkv_tag, val, dead, A.err);
#pragma unroll
        for (int tok = 0; tok < 2; ++tok) {
            qraw[0][tok] = val[4 * tok]; qraw[1][tok] = val[4 * tok + 1];
            kraw[tok] = val[4 * tok + 2]; vraw[tok] = val[4 * tok + 3];
        }
    }
    (void) qkvd;
    for (int tok = 0; tok < nt; ++tok) {
        const int pos = pos0 + tok;
        for (int hq = 0; hq < group; ++hq) {
            const float o = norm_rope(qraw[hq][tok], W.q_norm, A.eps, rc + (size_t) pos * 64, rs + (size_t) pos * 64, tmp, L.red);
            if (t < 128) qf[(hq * 2 + tok) * 128 + t] = round_f16(o);
        }
        const float o = norm_rope(kraw[tok], W.k_norm, A.eps, rc + (size_t) pos * 64, rs + (size_t) pos * 64, tmp, L.red);
        if (t < 128) {
            const uint16_t kh = f2h(o), vh = f2h(vraw[tok]);
            knew[tok * 128 + t] = h2f(kh);
            vnew[tok * 128 + t] = h2f(vh);
            if (cp) { L.cpk[layer][pos * 128 + t] = kh; L.cpv[layer][pos * 128 + t] = vh; }
            else { kc[(size_t) pos * 128 + t] = kh; vc[(size_t) pos * 128 + t] = vh; }
        }
    }
    __syncthreads();
    const int lane = t & 63, wave = t >> 6;
    for (int tok = 0; tok < nt; ++tok) {
        const int n_kv = pos0 + tok + 1;
        // scores for every query head of the group: 8 lanes per position, 16 dims per lane
        const int sub = lane & 7, pw = lane >> 3;
        float lmax[2] = {-INFINITY, -INFINITY};
        for (int j0 = 0; j0 < n_kv; j0 += 8 * kW) {
            const int j = j0 + wave * 8 + pw;
            float kv16[16];
            if (j < n_kv) {
                if (cp) {
#pragma unroll
                    for (int e = 0; e < 16; ++e) kv16[e] = h2f(L.cpk[layer][j * 128 + sub * 16 + e]);
                } else if (j < pos0) {
                    const int4 * kp = (const int4 *) (kc + (size_t) j * 128 + sub * 16);
                    const int4 k0 = kp[0], k1 = kp[1];
                    const uint16_t * a0 = (const uint16_t *) &k0;
                    const uint16_t * a1 = (const uint16_t *) &k1;
#pragma unroll
                    for (int e = 0; e < 8; ++e) { kv16[e] = h2f(a0[e]); kv16[8 + e] = h2f(a1[e]); }
                } else {
#pragma unroll
                    for (int e = 0; e < 16; ++e) kv16[e] = knew[(j - pos0) * 128 + sub * 16 + e];
                }
            }
            for (int hq = 0; hq < group; ++hq) {
                double acc = 0.0;
                if (j < n_kv) {
                    const float * q = qf + (hq * 2 + tok) * 128 + sub * 16;
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc += (double) (q[e] * kv16[e]);
                }
                acc += __shfl_xor(acc, 4);
                acc += __shfl_xor(acc, 2);
                acc += __shfl_xor(acc, 1);
                if (j < n_kv) {
                    const float s = (float) acc * A.attn_scale;
                    if (sub == 0) L.sc[hq * kMaxCtx + j] = s;
                    lmax[hq] = fmaxf(lmax[hq], s);
                }
            }
        }
        for (int hq = 0; hq < group; ++hq) {
            float * sc = L.sc + hq * kMaxCtx;
            const float mx = wg_max(lmax[hq], L.fred);
            double ls = 0.0;
            for (int j = t; j < n_kv; j += kT) { const float e = expf_q3t(sc[j] - mx); sc[j] = e; ls += (double) e; }
            const double sum = wg_sum(ls, L.red);
            const float inv = (float) (1.0 / sum);
            for (int j = t; j < n_kv; j += kT) sc[j] = round_f16(sc[j] * inv);
            __syncthreads();
            // P.V: 16 lanes per position, 8 dims per lane
            const int dsub = lane & 15, pq = lane >> 4;
            double o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = 0.0;
            for (int j0 = 0; j0 < n_kv; j0 += 4 * kW) {
                const int j = j0 + wave * 4 + pq;
                if (j < n_kv) {
                    const float p = sc[j];
                    float vv[8];
                    if (cp) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) vv[e] = h2f(L.cpv[layer][j * 128 + dsub * 8 + e]);
                    } else if (j < pos0) {
                        const int4 q4 = *(const int4 *) (vc + (size_t) j * 128 + dsub * 8);
                        const uint16_t * vh = (const uint16_t *) &q4;
#pragma unroll
                        for (int e = 0; e < 8; ++e) vv[e] = h2f(vh[e]);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; ++e) vv[e] = vnew[(j - pos0) * 128 + dsub * 8 + e];
                    }
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[e] += (double) (p * vv[e]);
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) { o[e] += __shfl_xor(o[e], 16); o[e] += __shfl_xor(o[e], 32); }
            if (pq == 0) {
#pragma unroll
                for (int e = 0; e < 8; ++e) L.pv[wave * 128 + dsub * 8 + e] = o[e];
            }
            __syncthreads();
            if (t < 128) {
                double r = L.pv[t];
                for (int w = 1; w < kW; ++w) r += L.pv[w * 128 + t];
                tstore(out + (size_t) tok * (kSlot / 2) + (g * group + hq) * 128 + t, out_tag, (float) r);
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------- samplers
// codebook-0 token from the talker logits (plain memory, written by the
// previous kernel): suppression window, repetition penalty, EOS bias ramp.
__device__ int32_t sample_cb0(const Args & A, Lds & L, int frame) {
    const SampleParams & P = *A.params;
    const int V = A.codec_vocab;
    for (int i = threadIdx.x; i < V; i += kT) {
        float v = A.logits[i];
        if (i >= V - 1024 && i != A.eos_id) v = -INFINITY;
        if (P.rep_penalty != 1.0f && A.seen[i]) v = v > 0.0f ? v / P.rep_penalty : v * P.rep_penalty;
        L.x[i] = v;
    }
    float eff = P.eos_bias;
    if (P.target_frames > 0 && frame > P.target_frames) {
        eff += 0.1f * (float) (frame - P.target_frames);
        if (eff > 6.0f) eff = 6.0f;
    }
    __syncthreads();
    return sample_core<kT>(L.x, V, P.temperature, P.top_k, A.eos_id, eff, P.seed, (uint32_t) frame, 0u, L.S);
}

// code-predictor token of codebook `group` from tagged head logits
__device__ int32_t sample_cp(const Args & A, Lds & L, const uint64_t * logits, uint32_t tag, int frame, int group,
                             bool & dead) {
    const SampleParams & P = *A.params;
    stage(logits, 1, A.cp_vocab, 0, tag, L.x, dead, A.err);
    return sample_core<kT>(L.x, A.cp_vocab, P.temperature, P.top_k, A.eos_id, 0.0f, P.seed, (uint32_t) frame,
                           (uint32_t) group, L.S);
}

// ------------------------------------------------------------------ layers
template <int NT, int SQ, int SO, int SD>
__device__ void layer_t(const Args & A, Lds & L, const LayerQ8 & W, int layer, bool cp, int pos0, uint32_t tb, int & p,
                        int p_in, bool in_in_lds, int & p_out, bool & dead) {
    const int d = A.d, qd = A.n_head * 128, kd = A.n_kv_head * 128, qkvd = qd + 2 * kd;
    const int ffn = cp ? A.cp_ffn : A.ffn;
    uint64_t * ar = A.arena;
    constexpr int HS = kSlot / 2;          // per-token stride inside a slot
    // QKV (RMSNorm'd input)
    const int p_qkv = p++;
    if (wg_has_rows(qkvd, d, SQ)) {
        Q8Regs<SQ, false> R;
        q8_prefetch<SQ, false>(R, W.qkv, W.qkv_d, nullptr, nullptr, qkvd, d);
        if (!in_in_lds) stage(ar + (size_t) p_in * kSlot, NT, d, HS, tb | p_in, L.x, dead, A.err);
        q8_compute<NT, SQ, false>(R, qkvd, d, L.x, W.attn_norm, A.eps, EPI_STORE, nullptr, 0, 0,
                                  ar + (size_t) p_qkv * kSlot, tb | p_qkv, HS, dead, A.err);
    }
    __syncthreads();
    // attention (workgroup g < n_kv_head owns KV head g)
    const int p_att = p++;
    if ((int) blockIdx.x < A.n_kv_head)
        attention_phase(A, L, W, layer, cp, NT, pos0, ar + (size_t) p_qkv * kSlot, tb | p_qkv,
                        ar + (size_t) p_att * kSlot, tb | p_att, dead);
    __syncthreads();
    // Wo + residual (the block input)
    const int p_wo = p++;
    if (wg_has_rows(d, qd, SO)) {
        Q8Regs<SO, false> R;
        q8_prefetch<SO, false>(R, W.wo, W.wo_d, nullptr, nullptr, d, qd);
        res_prefetch<NT, SO, false>(R, qd, ar + (size_t) p_in * kSlot, HS);
        stage(ar + (size_t) p_att * kSlot, NT, qd, HS, tb | p_att, L.x, dead, A.err);
        q8_compute<NT, SO, false>(R, d, qd, L.x, nullptr, A.eps, EPI_RESID, ar + (size_t) p_in * kSlot, tb | p_in, HS,
                                  ar + (size_t) p_wo * kSlot, tb | p_wo, HS, dead, A.err);
    }
    __syncthreads();
    // gate/up + SwiGLU (RMSNorm'd)
    const int p_gu = p++;
    if (wg_has_rows(ffn, d, SQ)) {
        Q8Regs<SQ, true> R;
        q8_prefetch<SQ, true>(R, W.wg, W.wg_d, W.wu, W.wu_d, ffn, d);
        stage(ar + (size_t) p_wo * kSlot, NT, d, HS, tb | p_wo, L.x, dead, A.err);
        q8_compute<NT, SQ, true>(R, ffn, d, L.x, W.ffn_norm, A.eps, EPI_SWIGLU, nullptr, 0, 0,
                                 ar + (size_t) p_gu * kSlot, tb | p_gu, HS, dead, A.err);
    }
    __syncthreads();
    // down + residual
    const int p_dn = p++;
    if (wg_has_rows(d, ffn, SD)) {
        Q8Regs<SD, false> R;
        q8_prefetch<SD, false>(R, W.wd, W.wd_d, nullptr, nullptr, d, ffn);
        res_prefetch<NT, SD, false>(R, ffn, ar + (size_t) p_wo * kSlot, HS);
        stage(ar + (size_t) p_gu * kSlot, NT, ffn, HS, tb | p_gu, L.x, dead, A.err);
        q8_compute<NT, SD, false>(R, d, ffn, L.x, nullptr, A.eps, EPI_RESID, ar + (size_t) p_wo * kSlot, tb | p_wo, HS,
                                  ar + (size_t) p_dn * kSlot, tb | p_dn, HS, dead, A.err);
    }
    __syncthreads();
    p_out = p_dn;
}

// Publish LDS rows [nt][d] as the tagged slot p (workgroup 0 only): the
// block's residual input for layer 0.
__device__ __forceinline__ void publish(const Args & A, const float * x, int nt, int d, int p, uint32_t tb) {
    if (blockIdx.x != 0) return;
    for (int t = 0; t < nt; ++t)
        for (int i = threadIdx.x; i < d; i += kT) tstore(A.arena + (size_t) p * kSlot + (size_t) t * (kSlot / 2) + i, tb | p, x[t * d + i]);
}

template <int SQ, int SO, int SD>
// The argument block lives in device memory: dynamic indexing into a by-value
// kernel argument (cp_embd[s], cp_head[s]) would copy it to private scratch.
__global__ __launch_bounds__(kT) void k_frame(const Args * __restrict__ Ap, int32_t frame) {
    const Args & A = *Ap;
    __shared__ Lds L;
    bool dead = false;
    FrameState * st = A.st;
    if (st->done) return;
    const uint32_t tb = (uint32_t) (frame + 1) << 12;
    const int d = A.d;
    const int t = threadIdx.x;
    int p = 0;

    // ---- codebook 0 (every workgroup samples the same token).  Workgroup 0
    // writes the frame state only at the end of the kernel: by then every
    // workgroup has finished this sampler (it consumed their later outputs),
    // so none can still be reading `seen`.
    const int32_t tok0 = sample_cb0(A, L, frame);
    if (tok0 == A.eos_id) {
        if (blockIdx.x == 0 && t == 0) { st->frame = frame; st->codes[0] = tok0; st->done = 1; st->eos = 1; }
        return;
    }
    if (t == 0) L.codes[0] = tok0;

    // ---- code predictor: 2-token prefill [hidden; codec_embd[tok0]] + 14 steps
    int code = tok0;
    for (int s = 0; s < 15; ++s) {
        const int p_x = p++;
        if (s == 0) {
            for (int i = t; i < d; i += kT) {
                L.x[i] = A.hidden[i];
                L.x[d + i] = h2f(A.codec_embd[(size_t) tok0 * d + i]);
            }
        } else {
            for (int i = t; i < d; i += kT) L.x[i] = h2f(A.cp_embd[s - 1][(size_t) code * d + i]);
        }
        __syncthreads();
        const int nt = s == 0 ? 2 : 1;
        const int pos0 = s == 0 ? 0 : s + 1;
        publish(A, L.x, nt, d, p_x, tb);
        int p_in = p_x, p_out = p_x;
        for (int l = 0; l < A.cp_layers; ++l) {
            if (nt == 2) layer_t<2, SQ, SO, SD>(A, L, A.cp[l], l, true, pos0, tb, p, p_in, l == 0, p_out, dead);
            else layer_t<1, SQ, SO, SD>(A, L, A.cp[l], l, true, pos0, tb, p, p_in, l == 0, p_out, dead);
            p_in = p_out;
        }
        // head on the last token's normed row
        const int p_head = p++;
        stage(A.arena + (size_t) p_out * kSlot + (size_t) (nt - 1) * (kSlot / 2), 1, d, kSlot / 2, tb | p_out, L.x,
              dead, A.err);
        f16_head(A.cp_head[s], A.cp_vocab, d, L.x, A.cp_out_norm, A.eps, A.arena + (size_t) p_head * kSlot,
                 tb | p_head, nullptr, nullptr);
        __syncthreads();
        code = sample_cp(A, L, A.arena + (size_t) p_head * kSlot, tb | p_head, frame, s + 1, dead);
        if (t == 0) L.codes[s + 1] = code;
        __syncthreads();
    }
    // ---- emit the frame
    if (blockIdx.x == 0 && t < 16) A.codes_out[(size_t) frame * 16 + t] = L.codes[t];

    // ---- talker step on the step embedding
    const int p_x = p++;
    for (int i = t; i < d; i += kT) {
        float s = h2f(A.codec_embd[(size_t) L.codes[0] * d + i]);
        for (int g = 1; g < 16; ++g) s = s + h2f(A.cp_embd[g - 1][(size_t) L.codes[g] * d + i]);
        const float tr = frame < A.n_trailing ? A.trailing[(size_t) frame * d + i] : A.pad[i];
        L.x[i] = s + tr;
    }
    __syncthreads();
    publish(A, L.x, 1, d, p_x, tb);
    const int pos = st->base_pos + frame;
    int p_in = p_x, p_out = p_x;
    for (int l = 0; l < A.n_layers; ++l) {
        layer_t<1, SQ, SO, SD>(A, L, A.talker[l], l, false, pos, tb, p, p_in, l == 0, p_out, dead);
        p_in = p_out;
    }
    stage(A.arena + (size_t) p_out * kSlot, 1, d, kSlot / 2, tb | p_out, L.x, dead, A.err);
    f16_head(A.codec_head, A.codec_vocab, d, L.x, A.out_norm, A.eps, nullptr, 0, A.logits, A.hidden);
    if (blockIdx.x == 0 && t == 0) {
        st->frame = frame;
        st->next_frame = frame + 1;
        st->talker_pos = pos;
        for (int g = 0; g < 16; ++g) st->codes[g] = L.codes[g];
        st->n_emitted = frame + 1;
        A.seen[tok0] = 1;
        if (frame + 1 >= st->max_frames) st->done = 1;
    }
}

}  // namespace fk
}  // namespace q3t
