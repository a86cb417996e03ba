// q3t_gemv_reg.h -- register-path GEMV of the decode loop (1 or 2 tokens).
//
// A batch-1 GEMV of a few MB is bound by latency, not bandwidth: the kernel
// launch, the fetch of the activation the previous kernel wrote, and the
// fetch of the weights.  This kernel therefore
//   1. issues every weight load of its row group at entry (they do not depend
//      on the previous kernel), together with the residual / bias operands;
//   2. loads its input rows (fp32) straight into registers;
//   3. normalises (RMSNorm) and quantises (Q8_0 per 32-block, or fp16
//      rounding) each lane's own blocks in registers -- a lane owns whole
//      32-element blocks, so no LDS staging and no workgroup barrier;
//   4. accumulates exact block terms in fp64, reduces over the row's lanes
//      with xor shuffles and applies the epilogue.
// Lane layout: a row's K/32 blocks are spread over LPR = K/32/SLOTS lanes
// (SLOTS blocks each); a wave covers 64/LPR rows; one row group per wave.
#pragma once

#include "q3t_kernels.h"

namespace q3t {

__device__ __forceinline__ void load_blk(const float * row, int blk, float (&dst)[32]) {
    const float4 * p = (const float4 *) (row + blk * kQK);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float4 v = p[c];
        dst[4 * c] = v.x; dst[4 * c + 1] = v.y; dst[4 * c + 2] = v.z; dst[4 * c + 3] = v.w;
    }
}

__device__ __forceinline__ int pack4(int a, int b, int c, int d) {
    return (a & 0xff) | ((b & 0xff) << 8) | ((c & 0xff) << 16) | ((int) ((unsigned) d << 24));
}

template <int WT, int NT, bool DUAL, int SLOTS, int G>
__global__ __launch_bounds__(kBlock) void k_gemv_r(GemvArgs a) {
    const int K = a.K, BPR = K / kQK;
    const int LPR = BPR / SLOTS;
    const int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lir = lane & (LPR - 1), rsub = lane / LPR;
    const int grp0 = (blockIdx.x * (kBlock / 64) + wave) * G;
    if (grp0 >= a.rows / RPW) return;
    const int ng = min(G, a.rows / RPW - grp0);

    // 1. weights and epilogue operands: independent of the previous kernel
    constexpr int WV = WT == W_Q8 ? 2 : 4;          // int4 per block: 32 int8 / 32 halves
    int4 w[G][SLOTS][WV], u[G][SLOTS][WV];
    float dw[G][SLOTS], du[G][SLOTS];
    float eop[G][NT];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int r = (grp0 + (g < ng ? g : 0)) * RPW + rsub;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const int b = lir + s * LPR;
            if (WT == W_Q8) {
                const int4 * wp = (const int4 *) ((const int8_t *) a.w + (size_t) r * K + b * kQK);
                w[g][s][0] = wp[0]; w[g][s][1] = wp[1];
                dw[g][s] = h2f(a.wd[(size_t) r * BPR + b]);
                if (DUAL) {
                    const int4 * up = (const int4 *) ((const int8_t *) a.w2 + (size_t) r * K + b * kQK);
                    u[g][s][0] = up[0]; u[g][s][1] = up[1];
                    du[g][s] = h2f(a.w2d[(size_t) r * BPR + b]);
                }
            } else {
                const int4 * wp = (const int4 *) ((const uint16_t *) a.w + (size_t) r * K + b * kQK);
#pragma unroll
                for (int c = 0; c < 4; ++c) w[g][s][c] = wp[c];
                if (DUAL) {
                    const int4 * up = (const int4 *) ((const uint16_t *) a.w2 + (size_t) r * K + b * kQK);
#pragma unroll
                    for (int c = 0; c < 4; ++c) u[g][s][c] = up[c];
                }
            }
        }
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            eop[g][tok] = 0.0f;
            if (lir == 0) {
                if (a.epi == EPI_RESID) eop[g][tok] = a.resid[(size_t) tok * a.resid_stride + r];
                else if (a.epi == EPI_BIAS || a.epi == EPI_BIAS_SILU) eop[g][tok] = a.bias[r];
            }
        }
    }
    // a finished frame loop (EOS) still runs the kernels of its graph: they
    // compute on stale but in-bounds inputs and store nothing
    const bool skip = a.done && *a.done;
    const bool writer = !skip && blockIdx.x == 0 && wave == 0 && rsub == 0;

    // 2. RMSNorm scale per token (ggml_rms_norm; the gain is applied per slot)
    float scale[NT];
    float xs[NT][32];                 // the current slot of each token
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
        scale[tok] = 1.0f;
        if (a.pro == PRO_NORM) {
            double ss = 0.0;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                load_blk(a.x + (size_t) tok * a.x_stride, lir + s * LPR, xs[tok]);
#pragma unroll
                for (int j = 0; j < 32; ++j) { const float v = xs[tok][j]; ss += (double) (v * v); }
            }
            ss = group_sum_d(ss, LPR);
            const float mean = (float) (ss / (double) K);
            scale[tok] = 1.0f / sqrtf(mean + a.eps);
        }
    }

    // 3. per slot: activation (normed, quantised / rounded), exact block terms in fp64
    double acc[G][NT], acc2[G][NT];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) { acc[g][tok] = 0.0; acc2[g][tok] = 0.0; }
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        float nw[32];
        if (a.pro == PRO_NORM) load_blk(a.norm_w, lir + s * LPR, nw);
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            // SLOTS == 1 with RMSNorm keeps the slot loaded in step 2
            if (!(SLOTS == 1 && a.pro == PRO_NORM)) load_blk(a.x + (size_t) tok * a.x_stride, lir + s * LPR, xs[tok]);
            float * xv = xs[tok];
            if (a.pro == PRO_NORM) {
#pragma unroll
                for (int j = 0; j < 32; ++j) { const float v = xv[j] * scale[tok]; xv[j] = v * nw[j]; }
                if (a.hidden_out && writer) {
                    float4 * p = (float4 *) (a.hidden_out + (size_t) tok * a.hidden_stride + (lir + s * LPR) * kQK);
#pragma unroll
                    for (int c = 0; c < 8; ++c) p[c] = make_float4(xv[4 * c], xv[4 * c + 1], xv[4 * c + 2], xv[4 * c + 3]);
                }
            }
            if (WT == W_Q8) {
                float am = 0.0f;
#pragma unroll
                for (int j = 0; j < 32; ++j) am = fmaxf(am, fabsf(xv[j]));
                const float d = am / 127.0f;
                const float id = am != 0.0f ? 127.0f / am : 0.0f;
                int q[8];
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    q[c] = pack4((int) rintf(xv[4 * c] * id), (int) rintf(xv[4 * c + 1] * id),
                                 (int) rintf(xv[4 * c + 2] * id), (int) rintf(xv[4 * c + 3] * id));
                const int4 x0 = make_int4(q[0], q[1], q[2], q[3]), x1 = make_int4(q[4], q[5], q[6], q[7]);
                const float dx = round_f16(d);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    acc[g][tok] += (double) (dw[g][s] * dx) * (double) dot32_i8(w[g][s][0], w[g][s][1], x0, x1);
                    if (DUAL) acc2[g][tok] += (double) (du[g][s] * dx) * (double) dot32_i8(u[g][s][0], u[g][s][1], x0, x1);
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        const float xv8 = xv[8 * c + j];
                        const _Float16 xh = __builtin_bit_cast(_Float16, f2h(xv8));
#pragma unroll
                        for (int g = 0; g < G; ++g) {
                            const uint16_t * wh = (const uint16_t *) &w[g][s][c];
                            const uint16_t * uh = (const uint16_t *) &u[g][s][c];
                            if (WT == W_F16) {
                                acc[g][tok] += (double) hmul_exact(__builtin_bit_cast(_Float16, wh[j]), xh);
                                if (DUAL) acc2[g][tok] += (double) hmul_exact(__builtin_bit_cast(_Float16, uh[j]), xh);
                            } else {
                                acc[g][tok] = fma((double) h2f(wh[j]), (double) xv8, acc[g][tok]);
                            }
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            acc[g][tok] = group_sum_d(acc[g][tok], LPR);
            if (DUAL) acc2[g][tok] = group_sum_d(acc2[g][tok], LPR);
        }
        if (lir != 0 || skip || g >= ng) continue;
        const int r = (grp0 + g) * RPW + rsub;
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            const float v = (float) acc[g][tok];
            float o;
            switch (a.epi) {
                case EPI_RESID: o = v + eop[g][tok]; break;
                case EPI_BIAS: o = v + eop[g][tok]; break;
                case EPI_BIAS_SILU: o = silu_q3t(v + eop[g][tok]); break;
                case EPI_SWIGLU: o = silu_q3t(v) * (float) acc2[g][tok]; break;
                default: o = v; break;
            }
            a.y[(size_t) tok * a.y_stride + r] = o;
        }
    }
}

}  // namespace q3t
