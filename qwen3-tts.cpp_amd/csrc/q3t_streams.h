// q3t_streams.h -- decode-shaped kernels of the multi-stream frame loop.
//
// With nb independent utterances advancing together, every talker and
// code-predictor projection of a frame is a GEMM of a few rows (nb, or 2nb
// for the code predictor's 2-token prefill) against one weight matrix that is
// read once for all rows.  The talker attention of a stream reads its own KV
// cache, whose length differs per stream.
//
//   k_gemm_rows  Q8_0 weight x up to 64 activation rows on
//                v_mfma_i32_16x16x32_i8.  A workgroup owns 16 weight rows and
//                every activation row; its 8 waves split K.  The activation
//                rows are read as fp32 and quantised (RMSNorm first where
//                the layer has one) inside the kernel, in the MFMA B-operand
//                layout, so no separate quantisation pass runs.  Block scales
//                are applied in fp64 per MFMA, the waves' partial sums meet
//                in a fixed tree, and the epilogue adds the residual or forms
//                SwiGLU from the paired gate/up matrices.
//   k_attn_gqa   one workgroup (16 waves) per (KV head, stream): QK-norm and
//                NEOX RoPE of the query heads that share the KV head and of
//                the new K, the cache append, and softmax attention over the
//                stream's positions, each K/V row read once for all of the
//                group's query heads.
//
// Numerics are those of the batch-1 path (forward_step,
// src/tts_transformer.cpp:1619-1769): fp64 sums of exact terms rounded once,
// Q8_0 activation quantisation d = amax/127 (fp16), q = rint(x * 127/amax),
// RMSNorm y = (x * scale) * w, attention probabilities rounded to fp16.
#pragma once

#include "q3t_kernels.h"

namespace q3t {
namespace ms {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef double v4d __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int kRows = 16;             // weight rows per MFMA tile (M)
constexpr int kWaves = 4;             // waves per workgroup, each a part of the K slice
constexpr int kThreads = kWaves * 64;
constexpr int kMaxTok = 64;           // activation rows per launch (4 MFMA column tiles)

enum GemmIn { IN_Q8 = 0, IN_NORM = 1, IN_ROUND = 2, IN_WIDE = 3 };
enum GemmOut { OUT_F32 = 0, OUT_RESID = 1, OUT_SWIGLU_Q8 = 2, OUT_SWIGLU_F32 = 3 };

struct GemmArgs {
    const int8_t * W; const uint16_t * Wd;     // [N][K] int8, [N][K/32] fp16 scales
    const int8_t * W2; const uint16_t * W2d;   // SwiGLU: the up matrix (W is gate)
    const uint16_t * H; const uint16_t * H2;   // F16 weights [N][K] (k_gemm_h; H2: the up matrix)
    int32_t N, K;
    const int8_t * q; const float * qdx;       // IN_Q8: activation rows [n][K] int8, scales [n][K/32]
    const float * x; int32_t xs;               // IN_NORM: activation rows [n][xs] fp32
    const float * rscale;                      //          1/sqrt(mean(x^2) + eps) per row, or:
    const double * ss_in; int32_t ss_tiles;    //          the producing GEMM's per-tile sums of squares [tiles][n]
    float eps;
    const float * norm_w;                      //          RMSNorm gain [K]
    int32_t n;                                 // activation rows, <= 16 * NT
    float * y; int32_t ys;                     // OUT_F32 / OUT_RESID rows [n][ys]
    const float * res; int32_t rs;             // OUT_RESID residual rows [n][rs]
    double * ss_out;                           // OUT_RESID: per-tile sums of squares of the rows [tiles][n] (or NULL)
    int8_t * yq; float * ydx;                  // OUT_SWIGLU_Q8 rows [n][N] int8, scales [n][N/32]
    uint64_t * part;                           // split-K partials [tiles][S][2 NV][64] tagged words
    uint32_t * cnt;                            // per-tile arrival counters (S per launch, never reset)
    int32_t * err;                             // set when a split-K wait times out
};

constexpr unsigned kSkSpin = 1u << 20;     // polls before a split-K wait gives up
constexpr int kSsPer = 16;                 // per-tile sums of squares one lane adds (hidden <= 1024)

// Dynamic LDS: weight scales of the slice [NW][MT*16][K/32/S] f32 and the
// cross-wave partials [2][NW][MT][NT][4][64] f64.
__host__ __device__ constexpr size_t gemm_sk_lds_bytes(int nt, int mt, bool dual, int nbs) {
    return (size_t) (dual ? 2 : 1) * mt * kRows * nbs * 4 + (size_t) 2 * (dual ? 2 : 1) * mt * nt * 4 * 64 * 8;
}

// RMSNorm row scale 1/sqrt(mean(x^2) + eps), the sum of squares in fp64 (one
// workgroup per row).  The GEMMs that consume normed rows apply it.
__global__ __launch_bounds__(kBlock) void k_row_scale(const float * __restrict__ x, int32_t xs, int32_t K, float eps,
                                                      float * __restrict__ out) {
    __shared__ double red[4];
    const float * xr = x + (size_t) blockIdx.x * xs;
    double ss = 0.0;
    for (int i = threadIdx.x; i < K; i += kBlock) ss += (double) (xr[i] * xr[i]);
    const double tot = block_sum_d(ss, red);
    if (threadIdx.x == 0) {
        const float mean = (float) (tot / (double) K);
        out[blockIdx.x] = 1.0f / sqrtf(mean + eps);
    }
}

// Quantises the 8 values a lane holds of one (row, Q8_0 block) into the MFMA
// B operand: the 4 lanes l, l^16, l^32, l^48 hold the block's 32 values.
__device__ __forceinline__ long quant8(const float (&v)[8], float & dx) {
    float am = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) am = fmaxf(am, fabsf(v[e]));
    am = fmaxf(am, __shfl_xor(am, 16));
    am = fmaxf(am, __shfl_xor(am, 32));
    const float d = am / 127.0f;
    const float id = am != 0.0f ? 127.0f / am : 0.0f;
    dx = round_f16(d);
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int e = 0; e < 4; ++e) lo |= ((uint32_t) (int) rintf(v[e] * id) & 0xffu) << (8 * e);
#pragma unroll
    for (int e = 0; e < 4; ++e) hi |= ((uint32_t) (int) rintf(v[4 + e] * id) & 0xffu) << (8 * e);
    return (long) (((uint64_t) hi << 32) | lo);
}

// Split-K exchange without fences (S > 1): every workgroup of a tile takes a
// ticket; ticket / S + 1 tags this launch.  All but the last store their
// partial as tagged 32-bit halves (relaxed agent-scope atomics) and return
// false; the last adds the S partials in slice order (so the sum does not
// depend on arrival order), polling each slot until its tags are current, and
// returns true.  The writers hold their tickets already, so every wait ends;
// a bounded poll count guards it anyway.  With S = 1 it returns true.
template <int NV>
__device__ __forceinline__ bool splitk_exchange(double (&acc)[NV], const GemmArgs & a, int tile, int s, int S,
                                                int lane) {
    if (S <= 1) return true;
    uint32_t old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(a.cnt + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = (uint32_t) __builtin_amdgcn_readfirstlane((int) old);
    const uint32_t tag = old / (uint32_t) S + 1u;
    uint64_t * base = a.part + (size_t) tile * S * 2 * NV * 64;
    if (old % (uint32_t) S != (uint32_t) (S - 1)) {
        uint64_t * mine = base + (size_t) s * 2 * NV * 64;
        const uint64_t th = (uint64_t) tag << 32;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
            __hip_atomic_store(mine + (2 * v) * 64 + lane, th | (uint32_t) __double2loint(acc[v]), __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(mine + (2 * v + 1) * 64 + lane, th | (uint32_t) __double2hiint(acc[v]),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return false;
    }
    bool dead = false;
    constexpr int CH = NV < 8 ? NV : 8;          // values summed per pass over the slices
#pragma unroll
    for (int c0 = 0; c0 < NV; c0 += CH) {
        double tot[CH];
#pragma unroll
        for (int v = 0; v < CH; ++v) tot[v] = 0.0;
        for (int ss = 0; ss < S; ++ss) {
            if (ss == s) {
#pragma unroll
                for (int v = 0; v < CH; ++v) tot[v] += acc[c0 + v];
                continue;
            }
            const uint64_t * src = base + ((size_t) ss * 2 * NV + 2 * c0) * 64;
            uint64_t w[2 * CH];
#pragma unroll
            for (int k = 0; k < 2 * CH; ++k)
                w[k] = __hip_atomic_load(src + k * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            unsigned n = 0;
            while (!dead) {
                bool all = true;
#pragma unroll
                for (int k = 0; k < 2 * CH; ++k) all = all && (uint32_t) (w[k] >> 32) == tag;
                if (__all(all)) break;
                if (++n > kSkSpin) { dead = true; atomicExch(a.err, 1); break; }
                __builtin_amdgcn_s_sleep(1);
#pragma unroll
                for (int k = 0; k < 2 * CH; ++k)
                    if ((uint32_t) (w[k] >> 32) != tag)
                        w[k] = __hip_atomic_load(src + k * 64 + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int v = 0; v < CH; ++v)
                tot[v] += __hiloint2double((int) (uint32_t) w[2 * v + 1], (int) (uint32_t) w[2 * v]);
        }
#pragma unroll
        for (int v = 0; v < CH; ++v) acc[c0 + v] = tot[v];
    }
    return true;
}

// Y[t][r] = epi(sum_b fp16(dw[r][b]) * dx[t][b] * sum_k W[r][32b+k] q[t][32b+k]).
// MFMA lane layout (16x16x32 i8): A[m = l%16][k = 8(l/16)..+7], B[k =
// 8(l/16)..+7][n = l%16], D[m = 4(l/16)+i][n = l%16]: lane l's B operand and
// D column are activation row 16j + l%16 of column tile j, so every lane
// applies the activation scales of its own row.
//
// Workgroup (tile, s) owns MT 16-row tiles of W (and of W2), all n activation
// rows and K slice s of S = gridDim.y: blocks [s*nbs, (s+1)*nbs), nbs = K/32/S,
// wave w taking bpw = nbs/4 <= KB of them.  IN_Q8 reads pre-quantised rows;
// IN_NORM reads fp32 rows with their RMSNorm row scales and quantises the
// normed values in registers.  The 4 waves' sums meet in a fixed LDS tree;
// with S > 1 each workgroup stores its fp64 partial, and the last of a tile's
// S workgroups to arrive adds the S partials in slice order (so the result
// does not depend on arrival order), resets the tile's counter and runs the
// epilogue.  OUT_SWIGLU_Q8 needs MT = 2 and DUAL: the tile's 32 rows are one
// Q8_0 block of the next projection's input, quantised in the epilogue.
// Requires N % (16 MT) == 0, (K/32) % (4 S) == 0, K/32/S/4 <= KB, n <= 16 NT
// (the host checks).
template <int NT, int MT, bool DUAL, int IN, int OUT, int KB>
__global__ __launch_bounds__(kThreads) void k_gemm_sk(GemmArgs a) {
    constexpr int NW = DUAL ? 2 : 1;
    constexpr bool QIN = IN == IN_Q8;
    constexpr int NV = NW * MT * NT * 4;             // fp64 partials per lane
    extern __shared__ __align__(16) char smem[];
    const int nb = a.K / kQK, S = gridDim.y, nbs = nb / S, bpw = nbs / kWaves;
    float * sdw = (float *) smem;                     // [NW][MT*16][nbs]
    double * spart = (double *) (sdw + NW * MT * kRows * nbs);   // [2][NV][64]
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int lm = lane & 15, lk = lane >> 4;
    const int tile = blockIdx.x, s = blockIdx.y;
    const int r0 = tile * (MT * kRows), bs = s * nbs, b0 = bs + wave * bpw;

    // weight quants and activations of this wave's blocks, all in flight before any use
    long wa[MT][KB], wb[DUAL ? MT : 1][KB];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int8_t * wr = a.W + (size_t) (r0 + 16 * m + lm) * a.K + 8 * lk;
        const int8_t * wr2 = DUAL ? a.W2 + (size_t) (r0 + 16 * m + lm) * a.K + 8 * lk : nullptr;
#pragma unroll
        for (int i = 0; i < KB; ++i)
            if (i < bpw) {
                wa[m][i] = *(const long *) (wr + (b0 + i) * kQK);
                if (DUAL) wb[m][i] = *(const long *) (wr2 + (b0 + i) * kQK);
            }
    }
    long qb[QIN ? NT : 1][QIN ? KB : 1];
    float qd[QIN ? NT : 1][QIN ? KB : 1];
    float4 xv[QIN ? 1 : NT][QIN ? 1 : KB][2];
    float rsc[QIN ? 1 : NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int tok = 16 * j + lm;
        const bool ok = tok < a.n;
        if (QIN) {
            const int8_t * qr = a.q + (size_t) (ok ? tok : 0) * a.K + 8 * lk;
            const float * dr = a.qdx + (size_t) (ok ? tok : 0) * nb;
#pragma unroll
            for (int i = 0; i < KB; ++i)
                if (i < bpw) {
                    qb[j][i] = ok ? *(const long *) (qr + (b0 + i) * kQK) : 0L;
                    qd[j][i] = ok ? dr[b0 + i] : 0.0f;
                }
        } else {
            const float * xr = a.x + (size_t) (ok ? tok : 0) * a.xs + 8 * lk;
            if (a.ss_in) {
                // RMSNorm row scale from the producer's per-tile sums: lane
                // group lk adds a quarter of the tiles in order, then a fixed
                // pairwise tree ((q0 + q1) + (q2 + q3))
                const int per = a.ss_tiles / 4;   // <= kSsPer (the host checks)
                double sv[kSsPer];
#pragma unroll
                for (int i = 0; i < kSsPer; ++i)
                    sv[i] = ok && i < per ? a.ss_in[(size_t) (lk * per + i) * a.n + tok] : 0.0;
                double part = 0.0;
#pragma unroll
                for (int i = 0; i < kSsPer; ++i) part += sv[i];
                part += __shfl_xor(part, 16);
                part += __shfl_xor(part, 32);
                const float mean = (float) (part / (double) a.K);
                rsc[QIN ? 0 : j] = ok ? 1.0f / sqrtf(mean + a.eps) : 0.0f;
            } else {
                rsc[QIN ? 0 : j] = ok ? a.rscale[tok] : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < KB; ++i) {
                float4 u0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u1 = u0;
                if (ok && i < bpw) {
                    u0 = *(const float4 *) (xr + (b0 + i) * kQK);
                    u1 = *(const float4 *) (xr + (b0 + i) * kQK + 4);
                }
                xv[QIN ? 0 : j][QIN ? 0 : i][0] = u0;
                xv[QIN ? 0 : j][QIN ? 0 : i][1] = u1;
            }
        }
    }
    // OUT_RESID: wave 0 runs the epilogue if this workgroup arrives last; its
    // residual values are loaded now, so the epilogue does not wait on them
    // (no workgroup writes the tile's rows before the last arriver)
    float rres[OUT == OUT_RESID ? NT : 1][OUT == OUT_RESID ? MT : 1][4];
    if constexpr (OUT == OUT_RESID) {
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int tok = 16 * j + lm;
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        rres[j][m][e] = tok < a.n ? a.res[(size_t) tok * a.rs + r0 + 16 * m + 4 * lk + e] : 0.0f;
            }
        }
    }
    // the slice's weight scales: rows r0.. of [N][nb] fp16, blocks bs..bs+nbs-1
    for (int i = t; i < MT * kRows * nbs; i += kThreads) {
        const int rr = i / nbs, bb = i - rr * nbs;
        sdw[i] = h2f(a.Wd[(size_t) (r0 + rr) * nb + bs + bb]);
        if (DUAL) sdw[MT * kRows * nbs + i] = h2f(a.W2d[(size_t) (r0 + rr) * nb + bs + bb]);
    }
    __syncthreads();

    double acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.0;
    const v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        if (i >= bpw) continue;
        const int b = b0 + i, bl = b - bs;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            long bop;
            float dxv;
            if (QIN) {
                bop = qb[j][i];
                dxv = qd[j][i];
            } else {
                // RMSNorm y = (x * scale) * w, then Q8_0 of the block
                const float * nw = a.norm_w + b * kQK + 8 * lk;
                const float4 g0 = *(const float4 *) nw, g1 = *(const float4 *) (nw + 4);
                const float4 u0 = xv[QIN ? 0 : j][QIN ? 0 : i][0], u1 = xv[QIN ? 0 : j][QIN ? 0 : i][1];
                const float xs8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
                const float gs8[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) { const float sv = xs8[e] * rsc[QIN ? 0 : j]; v[e] = sv * gs8[e]; }
                bop = quant8(v, dxv);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                // fp16 x fp16 scale product exact in fp32; times the int32 block sum exact in fp64
                const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(wa[m][i], bop, zero, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float dw = sdw[(16 * m + 4 * lk + e) * nbs + bl];
                    double & ac = acc[((0 * MT + m) * NT + j) * 4 + e];
                    ac = fma((double) (dw * dxv), (double) d[e], ac);
                }
                if (DUAL) {
                    const v4i d2 = __builtin_amdgcn_mfma_i32_16x16x32_i8(wb[m][i], bop, zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float dw = sdw[MT * kRows * nbs + (16 * m + 4 * lk + e) * nbs + bl];
                        double & ac = acc[((1 * MT + m) * NT + j) * 4 + e];
                        ac = fma((double) (dw * dxv), (double) d2[e], ac);
                    }
                }
            }
        }
    }

    // fixed tree over the 4 waves: (0 + 2, 1 + 3), then (0 + 1)
    if (wave >= 2) {
#pragma unroll
        for (int v = 0; v < NV; ++v) spart[((wave - 2) * NV + v) * 64 + lane] = acc[v];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int v = 0; v < NV; ++v) acc[v] += spart[(wave * NV + v) * 64 + lane];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v) spart[v * 64 + lane] = acc[v];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] += spart[v * 64 + lane];

    if (!splitk_exchange<NV>(acc, a, tile, s, gridDim.y, lane)) return;

#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int tok = 16 * j + lm;
        if (OUT == OUT_SWIGLU_Q8) {
            // rows r0 + 16m + 4lk + e of token tok: 8 of the block's 32 values
            float f[MT][4];
            float am = 0.0f;
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float g = (float) acc[((0 * MT + m) * NT + j) * 4 + e];
                    f[m][e] = silu_q3t(g) * (float) acc[(((NW - 1) * MT + m) * NT + j) * 4 + e];
                    am = fmaxf(am, fabsf(f[m][e]));
                }
            am = fmaxf(am, __shfl_xor(am, 16));
            am = fmaxf(am, __shfl_xor(am, 32));
            const float d = am / 127.0f;
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            if (tok < a.n) {
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    uint32_t pk = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) pk |= ((uint32_t) (int) rintf(f[m][e] * id) & 0xffu) << (8 * e);
                    *(uint32_t *) (a.yq + (size_t) tok * a.N + r0 + 16 * m + 4 * lk) = pk;
                }
                if (lk == 0) a.ydx[(size_t) tok * (a.N / kQK) + r0 / kQK] = round_f16(d);
            }
        } else {
            const bool ok = tok < a.n;
            double sq = 0.0;   // this lane's part of the tile's sum of squares of row tok
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float o[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float v = (float) acc[(m * NT + j) * 4 + e];
                    float rv = 0.0f;
                    if constexpr (OUT == OUT_RESID) rv = rres[j][m][e];
                    o[e] = OUT == OUT_RESID && ok ? v + rv : v;
                    sq += (double) (o[e] * o[e]);
                }
                if (ok) *(float4 *) (a.y + (size_t) tok * a.ys + r0 + 16 * m + 4 * lk) = make_float4(o[0], o[1], o[2], o[3]);
            }
            if (OUT == OUT_RESID && a.ss_out) {
                sq += __shfl_xor(sq, 16);
                sq += __shfl_xor(sq, 32);
                if (ok && lk == 0) a.ss_out[(size_t) tile * a.n + tok] = sq;
            }
        }
    }
}


// F16 weights: Y[t][r] = epi(sum_k W[r][k] * x[t][k]) on v_mfma_f64_16x16x4f64,
// the decode counterpart of the prefill's F16 GEMM.  The input rows are the
// F16 contract's: IN_NORM RMSNorm'd (y = (x * scale) * w) and rounded to
// fp16, IN_ROUND rounded to fp16, IN_WIDE fp32 as they are (the widened
// ffn_down); fp16 x fp16 and fp16 x fp32 products are exact in fp64, so every
// output is an fp64 sum of exact terms rounded to fp32 once, the numbers of
// the batch-1 F16 GEMVs.
//
// Same workgroup shape and split-K exchange as k_gemm_sk: workgroup (tile, s)
// owns MT 16-row tiles of W (and of H2), all n activation rows and K slice s,
// wave w taking bpw 32-element chunks of it.  Lane layout (16x16x4 f64):
// A[m = l%16][k = l/16] is activation row 16j + l%16, B[k = l/16][n = l%16]
// weight row 16m + l%16, and step e (0..7) of a chunk gives lane group
// k = l/16 the element 8k + e, so each lane loads 8 contiguous elements of
// its weight row and of its activation row per chunk.  D element r of lane
// l is activation row 16j + 4r + l/16, weight row 16m + l%16.  Epilogues:
// OUT_F32, OUT_RESID (+ per-tile sums of squares of the output rows for the
// next RMSNorm), OUT_SWIGLU_F32 (silu(gate) * up, fp32 rows).
// Requires N % (16 MT) == 0, (K/32) % (4 S) == 0, K/32/S/4 <= KB, n <= 16 NT.
//
// HM: the fast form on v_mfma_f32_16x16x32_f16, fp32 accumulation as ggml's
// F16 mul_mat accumulates: one MFMA per 32-element chunk with the same lane
// operands (A[m = l%16][k = 8(l/16)..+7] activation row 16j + l%16, B[k =
// 8(l/16)..+7][n = l%16] weight row 16m + l%16); D element r of lane l is
// activation row 16j + 4(l/16) + r.  The widened ffn_down input (fp32) goes
// in as two fp16 planes, hi = fp16(x) and lo = fp16(x - hi), so the product
// keeps about 22 bits of x.  The wave tree and split-K exchange add the fp32
// chunk sums in fp64 as before.
template <int NT, int MT, bool DUAL, int IN, int OUT, int KB, bool HM = false>
__global__ __launch_bounds__(kThreads) void k_gemm_h(GemmArgs a) {
    constexpr int NW = DUAL ? 2 : 1;
    constexpr int NA = NW * MT * NT;                  // 16 x 16 accumulators per lane
    constexpr int NV = NA * 4;                        // fp64 partials per lane
    extern __shared__ __align__(16) char smem[];
    const int nb = a.K / kQK, S = gridDim.y, nbs = nb / S, bpw = nbs / kWaves;
    double * spart = (double *) smem;                 // [2][NV][64]
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int lm = lane & 15, lk = lane >> 4;
    const int tile = blockIdx.x, s = blockIdx.y;
    const int r0 = tile * (MT * kRows), b0 = s * nbs + wave * bpw;

    // weights and activations of this wave's chunks, all in flight before any use
    v4i wa[MT][KB], wb[DUAL ? MT : 1][KB];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const uint16_t * wr = a.H + (size_t) (r0 + 16 * m + lm) * a.K + 8 * lk;
        const uint16_t * wr2 = DUAL ? a.H2 + (size_t) (r0 + 16 * m + lm) * a.K + 8 * lk : nullptr;
#pragma unroll
        for (int i = 0; i < KB; ++i)
            if (i < bpw) {
                wa[m][i] = *(const v4i *) (wr + (b0 + i) * kQK);
                if (DUAL) wb[m][i] = *(const v4i *) (wr2 + (b0 + i) * kQK);
            }
    }
    float4 xv[NT][KB][2];
    float rsc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int tok = 16 * j + lm;
        const bool ok = tok < a.n;
        const float * xr = a.x + (size_t) (ok ? tok : 0) * a.xs + 8 * lk;
        rsc[j] = 0.0f;
        if (IN == IN_NORM) {
            if (a.ss_in) {
                // RMSNorm row scale from the producer's per-tile sums: lane
                // group lk adds a quarter of the tiles in order, then a fixed
                // pairwise tree ((q0 + q1) + (q2 + q3))
                const int per = a.ss_tiles / 4;   // <= kSsPer (the host checks)
                double sv[kSsPer];
#pragma unroll
                for (int i = 0; i < kSsPer; ++i)
                    sv[i] = ok && i < per ? a.ss_in[(size_t) (lk * per + i) * a.n + tok] : 0.0;
                double part = 0.0;
#pragma unroll
                for (int i = 0; i < kSsPer; ++i) part += sv[i];
                part += __shfl_xor(part, 16);
                part += __shfl_xor(part, 32);
                const float mean = (float) (part / (double) a.K);
                rsc[j] = ok ? 1.0f / sqrtf(mean + a.eps) : 0.0f;
            } else {
                rsc[j] = ok ? a.rscale[tok] : 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < KB; ++i) {
            float4 u0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), u1 = u0;
            if (ok && i < bpw) {
                u0 = *(const float4 *) (xr + (b0 + i) * kQK);
                u1 = *(const float4 *) (xr + (b0 + i) * kQK + 4);
            }
            xv[j][i][0] = u0;
            xv[j][i][1] = u1;
        }
    }
    // OUT_RESID: the epilogue's residual values, loaded now by wave 0 (as in
    // k_gemm_sk), in the epilogue's (token, row) order
    float rres[OUT == OUT_RESID ? NT : 1][4][OUT == OUT_RESID ? MT : 1];
    if constexpr (OUT == OUT_RESID) {
        if (wave == 0) {
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int tok = HM ? 16 * j + 4 * lk + r : 16 * j + 4 * r + lk;
#pragma unroll
                    for (int m = 0; m < MT; ++m)
                        rres[j][r][m] = tok < a.n ? a.res[(size_t) tok * a.rs + r0 + 16 * m + lm] : 0.0f;
                }
        }
    }

    v4d acc[HM ? 1 : NA];
    v4f accf[HM ? NA : 1];
#pragma unroll
    for (int v = 0; v < (HM ? 1 : NA); ++v) acc[v] = v4d{0.0, 0.0, 0.0, 0.0};
#pragma unroll
    for (int v = 0; v < (HM ? NA : 1); ++v) accf[v] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < KB; ++i) {
        if (i >= bpw) continue;
        const int b = b0 + i;
        // the chunk's activation values as the F16 contract rounds them
        float av[NT][8];
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const float4 u0 = xv[j][i][0], u1 = xv[j][i][1];
            const float xs8[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            if (IN == IN_NORM) {
                const float * nw = a.norm_w + b * kQK + 8 * lk;
                const float4 g0 = *(const float4 *) nw, g1 = *(const float4 *) (nw + 4);
                const float gs8[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) { const float sv = xs8[e] * rsc[j]; av[j][e] = round_f16(sv * gs8[e]); }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) av[j][e] = IN == IN_WIDE ? xs8[e] : round_f16(xs8[e]);
            }
        }
        if (HM) {
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                h8 ah, al;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    ah[e] = (_Float16) av[j][e];
                    al[e] = IN == IN_WIDE ? (_Float16) (av[j][e] - (float) ah[e]) : (_Float16) 0.0f;
                }
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    const h8 w8 = __builtin_bit_cast(h8, wa[m][i]);
                    v4f & c0 = accf[(0 * MT + m) * NT + j];
                    c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, w8, c0, 0, 0, 0);
                    if (IN == IN_WIDE) c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, w8, c0, 0, 0, 0);
                    if (DUAL) {
                        v4f & c1 = accf[(1 * MT + m) * NT + j];
                        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, __builtin_bit_cast(h8, wb[DUAL ? m : 0][i]),
                                                                    c1, 0, 0, 0);
                    }
                }
            }
            continue;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            double bw[MT], bu[DUAL ? MT : 1];
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const v4i & w4 = wa[m][i];
                const uint32_t word = (uint32_t) w4[e >> 1];
                bw[m] = (double) h2f((uint16_t) ((e & 1) ? (word >> 16) : (word & 0xffffu)));
                if (DUAL) {
                    const v4i & u4 = wb[m][i];
                    const uint32_t uw = (uint32_t) u4[e >> 1];
                    bu[DUAL ? m : 0] = (double) h2f((uint16_t) ((e & 1) ? (uw >> 16) : (uw & 0xffffu)));
                }
            }
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const double ad = (double) av[j][e];
#pragma unroll
                for (int m = 0; m < MT; ++m) {
                    acc[(0 * MT + m) * NT + j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad, bw[m], acc[(0 * MT + m) * NT + j], 0, 0, 0);
                    if (DUAL)
                        acc[(1 * MT + m) * NT + j] =
                            __builtin_amdgcn_mfma_f64_16x16x4f64(ad, bu[DUAL ? m : 0], acc[(1 * MT + m) * NT + j], 0, 0, 0);
                }
            }
        }
    }
    double fl[NV];
#pragma unroll
    for (int v = 0; v < NA; ++v)
#pragma unroll
        for (int r = 0; r < 4; ++r) fl[4 * v + r] = HM ? (double) accf[HM ? v : 0][r] : acc[HM ? 0 : v][r];

    // fixed tree over the 4 waves: (0 + 2, 1 + 3), then (0 + 1)
    if (wave >= 2) {
#pragma unroll
        for (int v = 0; v < NV; ++v) spart[((wave - 2) * NV + v) * 64 + lane] = fl[v];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int v = 0; v < NV; ++v) fl[v] += spart[(wave * NV + v) * 64 + lane];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int v = 0; v < NV; ++v) spart[v * 64 + lane] = fl[v];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int v = 0; v < NV; ++v) fl[v] += spart[v * 64 + lane];
    if (!splitk_exchange<NV>(fl, a, tile, s, S, lane)) return;

#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = HM ? 16 * j + 4 * lk + r : 16 * j + 4 * r + lk;
            const bool ok = tok < a.n;
            double sq = 0.0;   // this lane's square of row 16m + lm of token tok, summed over the tile's lanes below
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                const int row = r0 + 16 * m + lm;
                const double g = fl[4 * ((0 * MT + m) * NT + j) + r];
                float o;
                if (OUT == OUT_SWIGLU_F32) {
                    o = silu_q3t((float) g) * (float) fl[4 * (((NW - 1) * MT + m) * NT + j) + r];
                } else {
                    o = (float) g;
                    if constexpr (OUT == OUT_RESID)
                        if (ok) o = o + rres[j][r][m];
                }
                sq += (double) (o * o);
                if (ok) a.y[(size_t) tok * a.ys + row] = o;
            }
            if (OUT == OUT_RESID && a.ss_out) {
                // the tile's sum of squares of token tok: a fixed tree over its 16 lanes
                sq += __shfl_xor(sq, 1);
                sq += __shfl_xor(sq, 2);
                sq += __shfl_xor(sq, 4);
                sq += __shfl_xor(sq, 8);
                if (ok && lm == 0) a.ss_out[(size_t) tile * a.n + tok] = sq;
            }
        }
}

__host__ __device__ constexpr size_t gemm_h_lds_bytes(int nt, int mt, bool dual) {
    return (size_t) 2 * (dual ? 2 : 1) * mt * nt * 4 * 64 * 8;
}

// ------------------------------------------------------------- attention

constexpr int kAWaves = 16;
constexpr int kAThreads = kAWaves * 64;
constexpr int kAU = 4;                // positions per lane in flight

struct GqaArgs {
    const float * qkv; int32_t qkv_stride;     // stream s's row at qkv + s * qkv_stride
    const float * q_norm; const float * k_norm; float eps;
    const float * rope_cos; const float * rope_sin;  // [pos][64]
    uint16_t * kc; uint16_t * vc;              // layer base of stream 0, [n_kv_head][n_ctx][128]
    int64_t kv_stream;                         // elements per stream
    int32_t n_ctx, n_head, n_kv_head;
    const int32_t * pos; int32_t pos_stream;   // position of stream s at pos[s * pos_stream] (NULL: pos_const)
    int32_t pos_const;
    const int32_t * done; int32_t done_stream; // stream s idles while done[s * done_stream] (NULL: never)
    float * out; int32_t out_stride;           // stream s's [n_head * 128] row
    int8_t * out_q; float * out_dx;            // its Q8_0 copy: [n_head * 128] int8, [n_head * 4] scales (NULL: none)
    float scale;
};

__host__ __device__ constexpr size_t attn_gqa_lds_bytes(int g, int n_ctx) {
    // staging: q [g][128], k, v [128] f32; reductions; then max(scores [g][n_ctx]
    // f32, P.V partials [16 waves][g][128] f64)
    return (size_t) (g + 2) * kHD * 4 + 512 +
           ((size_t) g * n_ctx * 4 > (size_t) kAWaves * g * kHD * 8 ? (size_t) g * n_ctx * 4
                                                                    : (size_t) kAWaves * g * kHD * 8);
}

// Workgroup x takes query heads G x .. G x + G - 1 of stream blockIdx.y; with
// G below the group size two or more workgroups share a KV head, read its
// cache each, and only the first appends the new K/V row (the others take
// the new row from their own LDS).  BF: a bfloat16 cache (q and P rounded to
// bfloat16 as well).
template <int G, bool BF = false>
__global__ __launch_bounds__(kAThreads) void k_attn_gqa(GqaArgs a) {
    const int hq0 = blockIdx.x * G, z = blockIdx.y;
    const int gsz = a.n_head / a.n_kv_head, g = hq0 / gsz;
    const bool append = hq0 % gsz == 0;
    if (a.done && a.done[(size_t) z * a.done_stream]) return;
    extern __shared__ __align__(16) char smem[];
    float * qf = (float *) smem;                  // [G][128] fp16-rounded rotated q
    float * knew = qf + G * kHD;                  // [128]
    float * vnew = knew + kHD;                    // [128]
    float * fred = vnew + kHD;                    // [16][G <= 4] wave maxima
    double * dred = (double *) (smem + (size_t) (G + 2) * kHD * 4 + 256);   // [16] sums
    float * sc = (float *) (smem + (size_t) (G + 2) * kHD * 4 + 512);        // [G][n_ctx]
    double * pv = (double *) sc;                  // after the scores are consumed: [16][G][128]

    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int pos = a.pos ? a.pos[(size_t) z * a.pos_stream] : a.pos_const, n_kv = pos + 1;
    const int qd = a.n_head * kHD, kd = a.n_kv_head * kHD;
    const float * row = a.qkv + (size_t) z * a.qkv_stride;
    uint16_t * kbase = a.kc + z * a.kv_stream + (size_t) g * a.n_ctx * kHD;
    uint16_t * vbase = a.vc + z * a.kv_stream + (size_t) g * a.n_ctx * kHD;
    const float * rc = a.rope_cos + (size_t) pos * 64;
    const float * rs = a.rope_sin + (size_t) pos * 64;

    if (wave < G) {
        const int h = hq0 + wave;
        float x0 = row[h * kHD + lane], x1 = row[h * kHD + 64 + lane];
        wave_norm_rope(x0, x1, a.q_norm, a.eps, rc, rs);
        qf[wave * kHD + lane] = round_kv(x0, BF);
        qf[wave * kHD + 64 + lane] = round_kv(x1, BF);
    } else if (wave == G) {
        float x0 = row[qd + g * kHD + lane], x1 = row[qd + g * kHD + 64 + lane];
        wave_norm_rope(x0, x1, a.k_norm, a.eps, rc, rs);
        const uint16_t k0 = f2kv(x0, BF), k1 = f2kv(x1, BF);
        knew[lane] = kv2f(k0, BF);
        knew[lane + 64] = kv2f(k1, BF);
        if (append) {
            kbase[(size_t) pos * kHD + lane] = k0;
            kbase[(size_t) pos * kHD + 64 + lane] = k1;
        }
    } else if (wave == G + 1) {
        const uint16_t v0 = f2kv(row[qd + kd + g * kHD + lane], BF), v1 = f2kv(row[qd + kd + g * kHD + 64 + lane], BF);
        vnew[lane] = kv2f(v0, BF);
        vnew[lane + 64] = kv2f(v1, BF);
        if (append) {
            vbase[(size_t) pos * kHD + lane] = v0;
            vbase[(size_t) pos * kHD + 64 + lane] = v1;
        }
    }
    __syncthreads();

    // scores: 16 lanes per position (8 dims each), 4 positions per wave, kAU in flight
    const int dsub = lane & 15, pq = lane >> 4;
    // fp16 x fp16 products are exact in fp64: fma rounds like the fp32
    // product added in fp64, with one conversion per cached element
    double q[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) q[h][e] = (double) qf[h * kHD + dsub * 8 + e];
    float lmax[G];
#pragma unroll
    for (int h = 0; h < G; ++h) lmax[h] = -INFINITY;
    constexpr int kStep = kAWaves * 4;
    // cache rows of the next kAU positions are in flight while the current ones are used
    int4 kv[kAU], kn[kAU];
#pragma unroll
    for (int u = 0; u < kAU; ++u) {
        const int j = u * kStep + wave * 4 + pq;
        if (j < pos) kv[u] = *(const int4 *) (kbase + (size_t) j * kHD + dsub * 8);
    }
    for (int j0 = 0; j0 < n_kv; j0 += kStep * kAU) {
        if (j0 + kStep * kAU < n_kv) {
#pragma unroll
            for (int u = 0; u < kAU; ++u) {
                const int j = j0 + kStep * kAU + u * kStep + wave * 4 + pq;
                if (j < pos) kn[u] = *(const int4 *) (kbase + (size_t) j * kHD + dsub * 8);
            }
        }
#pragma unroll
        for (int u = 0; u < kAU; ++u) {
            const int j = j0 + u * kStep + wave * 4 + pq;
            double kf[8];
            if (j < pos) {
                const uint16_t * kh = (const uint16_t *) &kv[u];
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] = (double) kv2f(kh[e], BF);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) kf[e] = j == pos ? (double) knew[dsub * 8 + e] : 0.0;
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                double s = 0.0;
#pragma unroll
                for (int e = 0; e < 8; ++e) s = fma(q[h][e], kf[e], s);
                s = group_sum_d(s, 16);
                if (j < n_kv) {
                    const float sv = (float) s * a.scale;
                    if (dsub == 0) sc[h * a.n_ctx + j] = sv;
                    lmax[h] = fmaxf(lmax[h], sv);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kAU; ++u) kv[u] = kn[u];
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const float m = wave_max_f(lmax[h]);
        if (lane == 0) fred[wave * G + h] = m;
    }
    __syncthreads();
    float mx[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        mx[h] = fred[h];
        for (int w = 1; w < kAWaves; ++w) mx[h] = fmaxf(mx[h], fred[w * G + h]);
    }
    // exp and fp64 sums (one head per pass; dred holds 16 wave sums)
    float inv[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        double ls = 0.0;
        for (int j = t; j < n_kv; j += kAThreads) {
            const float e = expf_q3t(sc[h * a.n_ctx + j] - mx[h]);
            sc[h * a.n_ctx + j] = e;
            ls += (double) e;
        }
        ls = wave_sum_d(ls);
        if (lane == 0) dred[wave] = ls;
        __syncthreads();
        double tot = 0.0;
#pragma unroll
        for (int w = 0; w < kAWaves; ++w) tot += dred[w];
        inv[h] = (float) (1.0 / tot);
        __syncthreads();
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
        for (int j = t; j < n_kv; j += kAThreads) sc[h * a.n_ctx + j] = round_kv(sc[h * a.n_ctx + j] * inv[h], BF);
    __syncthreads();

    // P.V: same position mapping; each V row read once for the group's heads
    double o[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] = 0.0;
    int4 vv[kAU], vn[kAU];
#pragma unroll
    for (int u = 0; u < kAU; ++u) {
        const int j = u * kStep + wave * 4 + pq;
        if (j < pos) vv[u] = *(const int4 *) (vbase + (size_t) j * kHD + dsub * 8);
    }
    for (int j0 = 0; j0 < n_kv; j0 += kStep * kAU) {
        if (j0 + kStep * kAU < n_kv) {
#pragma unroll
            for (int u = 0; u < kAU; ++u) {
                const int j = j0 + kStep * kAU + u * kStep + wave * 4 + pq;
                if (j < pos) vn[u] = *(const int4 *) (vbase + (size_t) j * kHD + dsub * 8);
            }
        }
#pragma unroll
        for (int u = 0; u < kAU; ++u) {
            const int j = j0 + u * kStep + wave * 4 + pq;
            if (j >= n_kv) continue;
            double vf[8];
            if (j < pos) {
                const uint16_t * vh = (const uint16_t *) &vv[u];
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = (double) kv2f(vh[e], BF);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = (double) vnew[dsub * 8 + e];
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const double p = (double) sc[h * a.n_ctx + j];
#pragma unroll
                for (int e = 0; e < 8; ++e) o[h][e] = fma(p, vf[e], o[h][e]);
            }
        }
#pragma unroll
        for (int u = 0; u < kAU; ++u) vv[u] = vn[u];
    }
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            o[h][e] += swz16_d(o[h][e]);
            o[h][e] += __shfl_xor(o[h][e], 32);
        }
    __syncthreads();   // the scores are consumed: reuse their LDS for the partials
    if (pq == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) pv[(wave * G + h) * kHD + dsub * 8 + e] = o[h][e];
    }
    __syncthreads();
    if (t < G * kHD) {
        const int h = t / kHD, d = t % kHD;
        double r = 0.0;
#pragma unroll
        for (int w = 0; w < kAWaves; ++w) r += pv[(w * G + h) * kHD + d];
        const float o = (float) r;
        const size_t e = (size_t) z * a.out_stride + (hq0 + h) * kHD + d;
        a.out[e] = o;
        if (a.out_q) a.out_q[e] = quant_lane32(o, a.out_dx + e / kQK, (t & 31) == 0);
    }
}

}  // namespace ms
}  // namespace q3t
