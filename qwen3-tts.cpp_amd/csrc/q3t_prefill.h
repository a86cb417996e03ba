// q3t_prefill.h -- long-prompt talker prefill on MFMA: int8 GEMMs for Q8_0
// layers, f64 GEMMs for F16 layers, f64 causal attention.
//
// The n-token prefill (forward_prefill, src/tts_transformer.cpp:2217-2347 /
// build_prefill_forward_graph :1474-1617) is a real contraction once n is in
// the tens or thousands, so each layer runs as
//   quantise rows (RMSNorm where the layer has one, Q8_0 per 32-block)
//   -> GEMM on v_mfma_i32_16x16x32_i8 (one MFMA = one 32-element Q8_0 block,
//      exact in int32) with the block scales applied in fp64
//   -> K/V rows into the cache -> causal attention over the cache
//   -> quantise -> Wo GEMM (+ residual) -> quantise (+ RMSNorm) -> gate and up
//      GEMMs -> SwiGLU -> quantise -> down GEMM (+ residual).
// Every sum is of exact terms in fp64 rounded once, the contract of the GEMV
// path, so the result equals the chunked GEMV prefill bit for bit.
#pragma once

#include <type_traits>

#include "q3t_kernels.h"

namespace q3t {
namespace pf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef double v4d __attribute__((ext_vector_type(4)));

// Element e (0..7) of eight 16-bit values packed in an int4.
__device__ __forceinline__ uint16_t h8bits(const int4 & v, int e) {
    const int w = (e >> 1) == 0 ? v.x : (e >> 1) == 1 ? v.y : (e >> 1) == 2 ? v.z : v.w;
    return (uint16_t) ((e & 1) ? ((uint32_t) w >> 16) : ((uint32_t) w & 0xffffu));
}

// One row per block: optional RMSNorm (y = (x * scale) * w, scale from the
// fp64 sum of fp32 squares) or, with u, the SwiGLU y = silu(x) * u (x the
// gate rows, u the up rows of the same stride; the numbers of k_swiglu_rows),
// then Q8_0 quantisation per 32-element block (d = amax/127 as fp16, q =
// rint(x * 127/amax)).  q: int8 [n][K]; dx: the fp16-rounded scales as float
// [n][K/32].
__global__ __launch_bounds__(kBlock) void k_quant_rows(const float * __restrict__ x, int32_t xs, int32_t K,
                                                       const float * __restrict__ w, float eps, int8_t * __restrict__ q,
                                                       float * __restrict__ dx, const float * __restrict__ u) {
    __shared__ double red[4];
    const int row = blockIdx.x, t = threadIdx.x;
    const float * xr = x + (size_t) row * xs;
    float scale = 1.0f;
    if (w && !u) {
        double ss = 0.0;
        for (int i = t; i < K; i += kBlock) ss += (double) (xr[i] * xr[i]);
        const double tot = block_sum_d(ss, red);
        const float mean = (float) (tot / (double) K);
        scale = 1.0f / sqrtf(mean + eps);
    }
    // four elements per thread, a block being 8 consecutive lanes (K % 32 == 0
    // keeps every 8-lane group wholly inside or outside the loop)
    const int nb = K / kQK;
    for (int g = t; g < K / 4; g += kBlock) {
        const float4 xv = *(const float4 *) (xr + 4 * g);
        float y[4] = {xv.x, xv.y, xv.z, xv.w};
        if (u) {
            const float4 uv = *(const float4 *) (u + (size_t) row * xs + 4 * g);
            const float uk[4] = {uv.x, uv.y, uv.z, uv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = silu_q3t(y[e]) * uk[e];
        } else if (w) {
            const float4 wv = *(const float4 *) (w + 4 * g);
            const float wk[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) { const float sv = y[e] * scale; y[e] = sv * wk[e]; }
        }
        float am = fmaxf(fmaxf(fabsf(y[0]), fabsf(y[1])), fmaxf(fabsf(y[2]), fabsf(y[3])));
        am = fmaxf(am, __shfl_xor(am, 1));
        am = fmaxf(am, __shfl_xor(am, 2));
        am = fmaxf(am, __shfl_xor(am, 4));
        const float d = am / 127.0f;
        const float id = am != 0.0f ? 127.0f / am : 0.0f;
        int p = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) p |= ((int) rintf(y[e] * id) & 0xff) << (8 * e);
        *(int *) (q + (size_t) row * K + 4 * g) = p;
        if ((g & 7) == 0) dx[(size_t) row * nb + (g >> 3)] = round_f16(d);
    }
}

// Y[t][r] = epi(sum_b fp16(dw[r][b]) * dx[t][b] * sum_k W[r][32b+k] Q[t][32b+k])
// on a (32 IR rows) x (32 JT tokens) tile per workgroup: wave (wr, wt) =
// (wave & 1, wave >> 1) owns IR x JT MFMA tiles of 16 x 16.  Each stage holds
// kGB Q8_0 blocks of the tile's weight and activation rows in LDS (rows padded
// by 8 bytes against bank conflicts) with their scales, double-buffered: the
// next stage's global loads are in flight during this stage's MFMAs.  MFMA
// lane layout (16x16x32 i8): A[m = l%16][k = 8(l/16)..+7], B[k][n = l%16],
// D[m = 4(l/16)+i][n = l%16]; each block's exact int32 sums take the fp16 x
// fp16 scale product (exact in fp32) in an fp64 fma, so the fp64 sum of exact
// terms is rounded to fp32 once.  epi: EPI_STORE or EPI_RESID (res [n][rs],
// rs = 0 broadcasts one row).  Requires N % (32 IR) == 0, K % (32 kGB) == 0.
// A wave skips the MFMAs and epilogue of its 16-token groups that lie wholly
// past n, so the partial last token tile (2,049 rows: one row) costs about
// half a tile, not a whole one.
template <int IR, int JT, int GB>
struct Q8Tile {
    static constexpr int TN = 32 * IR, TM = 32 * JT;
    static constexpr int ROWB = GB * kQK + 8;          // bytes per staged row (padded against bank conflicts)
    static constexpr int A_BYTES = TN * ROWB, B_BYTES = TM * ROWB;
    static constexpr int STAGE = A_BYTES + B_BYTES + (TN + TM) * GB * 4;
    static constexpr int LDS = 2 * STAGE;
};

template <int IR, int JT, int kGB>
__global__ __launch_bounds__(kBlock) void k_gemm_q8(const int8_t * __restrict__ W, const uint16_t * __restrict__ Wd,
                                                    int32_t N, int32_t K, const int8_t * __restrict__ Q,
                                                    const float * __restrict__ dx, int32_t n, float * __restrict__ Y,
                                                    int32_t ys, const float * __restrict__ res, int32_t rs, int32_t epi) {
    using T = Q8Tile<IR, JT, kGB>;
    constexpr int kRowB = T::ROWB;
    __shared__ __align__(16) char smem[T::LDS];
    const int BPR = K / kQK, S = BPR / kGB;
    const int r0 = blockIdx.x * T::TN, t0 = blockIdx.y * T::TM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, wr = wave & 1, wt = wave >> 1;
    const int lm = lane & 15, lk = lane >> 4;
    // staging: 16-byte chunks, kGB * 2 per row (A then B rows), scale pairs
    constexpr int CPR = kGB * kQK / 16;                  // chunks per row
    constexpr int NA = (T::TN * CPR + kBlock - 1) / kBlock, NB = (T::TM * CPR + kBlock - 1) / kBlock;
    int4 ra[NA], rb[NB];
    float sw[kGB], sx[kGB];
#pragma unroll
    for (int g = 0; g < kGB; ++g) { sw[g] = 0.f; sx[g] = 0.f; }
    auto fetch = [&](int st) {
        const int kb = st * kGB;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int c = tid + i * kBlock, row = c / CPR, col = c - row * CPR;
            ra[i] = c < T::TN * CPR ? *(const int4 *) (W + (size_t) (r0 + row) * K + kb * kQK + col * 16) : make_int4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int c = tid + i * kBlock, row = c / CPR, col = c - row * CPR;
            const int tok = t0 + row;
            rb[i] = (c < T::TM * CPR && tok < n) ? *(const int4 *) (Q + (size_t) tok * K + kb * kQK + col * 16)
                                                 : make_int4(0, 0, 0, 0);
        }
        if (tid < T::TN) {
            const uint16_t * p = Wd + (size_t) (r0 + tid) * BPR + kb;
#pragma unroll
            for (int g = 0; g < kGB; ++g) sw[g] = h2f(p[g]);
        }
        if (tid < T::TM) {
            const int tok = t0 + tid;
#pragma unroll
            for (int g = 0; g < kGB; ++g) sx[g] = tok < n ? dx[(size_t) tok * BPR + kb + g] : 0.f;
        }
    };
    auto stash = [&](int buf) {
        char * st = smem + buf * T::STAGE;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int c = tid + i * kBlock, row = c / CPR, col = c - row * CPR;
            if (c < T::TN * CPR) {
                long * d = (long *) (st + row * kRowB + col * 16);   // 8-byte aligned rows
                d[0] = ((const long *) &ra[i])[0];
                d[1] = ((const long *) &ra[i])[1];
            }
        }
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int c = tid + i * kBlock, row = c / CPR, col = c - row * CPR;
            if (c < T::TM * CPR) {
                long * d = (long *) (st + T::A_BYTES + row * kRowB + col * 16);
                d[0] = ((const long *) &rb[i])[0];
                d[1] = ((const long *) &rb[i])[1];
            }
        }
        float * sdw = (float *) (st + T::A_BYTES + T::B_BYTES);   // [kGB][TN]
        float * sdx = sdw + kGB * T::TN;                          // [kGB][TM]
#pragma unroll
        for (int g = 0; g < kGB; ++g) {
            if (tid < T::TN) sdw[g * T::TN + tid] = sw[g];
            if (tid < T::TM) sdx[g * T::TM + tid] = sx[g];
        }
    };

    double acc[IR][JT][4];
#pragma unroll
    for (int i = 0; i < IR; ++i)
#pragma unroll
        for (int j = 0; j < JT; ++j)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[i][j][e] = 0.0;
    const v4i zero = {0, 0, 0, 0};

    fetch(0);
    stash(0);
    __syncthreads();
    for (int st = 0; st < S; ++st) {
        const int buf = st & 1;
        if (st + 1 < S) fetch(st + 1);
        const char * sb = smem + buf * T::STAGE;
        const float * sdw = (const float *) (sb + T::A_BYTES + T::B_BYTES);
        const float * sdx = sdw + kGB * T::TN;
#pragma unroll
        for (int kb = 0; kb < kGB; ++kb) {
            long bq[JT];
            float dxv[JT];
#pragma unroll
            for (int j = 0; j < JT; ++j) {
                const int tl = wt * JT * 16 + j * 16 + lm;
                bq[j] = *(const long *) (sb + T::A_BYTES + tl * kRowB + kb * kQK + 8 * lk);
                dxv[j] = sdx[kb * T::TM + tl];
            }
#pragma unroll
            for (int i = 0; i < IR; ++i) {
                const int rl = wr * IR * 16 + i * 16;
                const long a = *(const long *) (sb + (rl + lm) * kRowB + kb * kQK + 8 * lk);
                float dwv[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) dwv[e] = sdw[kb * T::TN + rl + 4 * lk + e];
#pragma unroll
                for (int j = 0; j < JT; ++j) {
                    if (t0 + (wt * JT + j) * 16 >= n) continue;   // 16 tokens past n (wave-uniform): nothing to add
                    const v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bq[j], zero, 0, 0, 0);
                    // fp16 x fp16 scale product exact in fp32; times the int32 block sum exact in fp64
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[i][j][e] = fma((double) (dwv[e] * dxv[j]), (double) d[e], acc[i][j][e]);
                }
            }
        }
        if (st + 1 < S) stash(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < JT; ++j) {
        const int tok = t0 + wt * JT * 16 + j * 16 + lm;
        if (tok >= n) continue;
#pragma unroll
        for (int i = 0; i < IR; ++i) {
            const int r = r0 + wr * IR * 16 + i * 16 + 4 * lk;
            float4 v = make_float4((float) acc[i][j][0], (float) acc[i][j][1], (float) acc[i][j][2], (float) acc[i][j][3]);
            if (epi == EPI_RESID) {
                const float * rr = res + (size_t) tok * rs + r;
                v.x = v.x + rr[0]; v.y = v.y + rr[1]; v.z = v.z + rr[2]; v.w = v.w + rr[3];
            }
            *(float4 *) (Y + (size_t) tok * ys + r) = v;
        }
    }
}


constexpr int kTile = 64;         // output rows and tokens per workgroup of the F16 GEMM

// F16 weights: Y[t][r] = epi(sum_k W[r][k] * x[t][k]) with x rounded to fp16
// (WIDE = false, the F16-weight contract) or kept fp32 (WIDE = true, the
// widened ffn_down).  Both products are exact in fp64 (11 x 11 or 11 x 24
// significant bits), so the GEMM runs on v_mfma_f64_16x16x4f64: exact
// products summed in fp64 and rounded to fp32 once, the numbers of the GEMV
// path.  (fp16 MFMA would accumulate in fp32.)
//
// A 64-row x 64-token tile per workgroup, K in chunks of KC (32 or 64)
// staged in LDS as fp16 (weights, and activations when !WIDE) or fp32 (WIDE
// activations), double-buffered: chunk c + 1 is loaded into registers while
// chunk c's MFMAs run.  Four waves in a 2 x 2 arrangement, each 32 tokens x
// 32 rows as 2 x 2 MFMA tiles with the tokens as the A operand (m) and the
// weight rows as B (n), so lane l's element r is token 4r + l/16 of its tile
// and row l%16: 16 consecutive lanes store 16 consecutive floats of one
// output row.  Step s (0 .. KC/4 - 1) of a chunk gives lane group k = l/16
// the index (KC/4) k + s, so each lane reads KC/4 contiguous elements of its
// row with 16-byte loads.
// Requires N % 64 == 0, K % KC == 0 (the host checks).
template <bool WIDE, int KC>
struct F16Tile {
    static constexpr int HS = KC + 8;          // LDS row stride (halves) of fp16 rows: conflict-free 16-byte reads
    static constexpr int FS = KC + 4;          // LDS row stride (floats) of fp32 rows
    static constexpr int W_BYTES = kTile * HS * 2;
    static constexpr int X_BYTES = WIDE ? kTile * FS * 4 : kTile * HS * 2;
    static constexpr int STAGE = W_BYTES + X_BYTES;
    static constexpr int E = KC / 4;           // elements per lane group and chunk (= MFMA steps)
    static constexpr int SP = KC / 4;          // elements staged per thread (4 threads per row)
};

// Tail workgroup of the F16 GEMM: 16 weight rows from r0 x the at most 32
// tokens t0 .. n - 1, in 16-token groups.  The four waves take interleaved
// 32-wide K slices straight from global memory (no staging), each keeps fp64
// partials, and the partials are added in wave order through LDS, so the
// result does not depend on timing.  A 1-row remainder then costs 1/16 of a
// 64 x 64 tile instead of a whole one.
template <bool WIDE>
__device__ __forceinline__ void gemm_f16_tail(const uint16_t * __restrict__ W, int K, const float * __restrict__ x,
                                              int xs, int n, int t0, int r0, float * __restrict__ Y, int ys,
                                              const float * __restrict__ res, int rs, char * smem) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, li = lane & 15, lk = lane >> 4;
    const int ng = (n - t0 + 15) >> 4;            // token groups: 1 or 2
    const int ta = t0 + li, tb = t0 + 16 + li;
    const bool oka = ta < n, okb = tb < n;        // rows past n read row n - 1 and multiply zeros
    const uint16_t * wp = W + (size_t) (r0 + li) * K + 8 * lk;
    const float * xa = x + (size_t) (oka ? ta : n - 1) * xs + 8 * lk;
    const float * xb = x + (size_t) (okb ? tb : n - 1) * xs + 8 * lk;
    v4d acc[2] = {v4d{0.0, 0.0, 0.0, 0.0}, v4d{0.0, 0.0, 0.0, 0.0}};
    auto arow = [&](const float * xp, bool ok, int k0, double (&ad)[8]) {
        const float4 p = *(const float4 *) (xp + k0), q = *(const float4 *) (xp + k0 + 4);
        const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ad[e] = ok ? (double) (WIDE ? v[e] : round_f16(v[e])) : 0.0;
    };
#pragma unroll 2
    for (int k0 = 32 * wave; k0 < K; k0 += 128) {
        const int4 wv = *(const int4 *) (wp + k0);
        double ad[8];
        arow(xa, oka, k0, ad);
#pragma unroll
        for (int s = 0; s < 8; ++s)
            acc[0] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad[s], (double) h2f(h8bits(wv, s)), acc[0], 0, 0, 0);
        if (ng > 1) {
            arow(xb, okb, k0, ad);
#pragma unroll
            for (int s = 0; s < 8; ++s)
                acc[1] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad[s], (double) h2f(h8bits(wv, s)), acc[1], 0, 0, 0);
        }
    }
    double * red = (double *) smem;               // [wave][group][r][lane]
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[((wave * 2 + g) * 4 + r) * 64 + lane] = acc[g][r];
    __syncthreads();
    for (int v = t; v < ng * 256; v += kBlock) {
        const int g = v >> 8, r = (v >> 6) & 3, l = v & 63;
        const int tok = t0 + 16 * g + 4 * r + (l >> 4), row = r0 + (l & 15);
        if (tok >= n) continue;
        double sum = 0.0;
#pragma unroll
        for (int w = 0; w < 4; ++w) sum += red[((w * 2 + g) * 4 + r) * 64 + l];
        float o = (float) sum;
        if (res) o = o + res[(size_t) tok * rs + row];
        Y[(size_t) tok * ys + row] = o;
    }
}

// One-dimensional grid: the first (N / 64) * nfull workgroups are 64 x 64
// tiles (weight tile fastest), the rest 16-row tail workgroups over the
// tokens from nfull * 64 on (at most 32 of them).
template <bool WIDE, int KC>
__global__ __launch_bounds__(kBlock) void k_gemm_f16(const uint16_t * __restrict__ W, int32_t N, int32_t K,
                                                     const float * __restrict__ x, int32_t xs, int32_t n,
                                                     float * __restrict__ Y, int32_t ys, const float * __restrict__ res,
                                                     int32_t rs, int32_t nfull) {
    using T = F16Tile<WIDE, KC>;
    constexpr int E = T::E, NW = T::SP / 8, NX = T::SP / 4;
    static_assert(2 * T::STAGE >= 4 * 2 * 4 * 64 * 8, "tail reduction fits the staging LDS");
    __shared__ __align__(16) char smem[2 * T::STAGE];
    const int nx = N / kTile, b = blockIdx.x;
    if (b >= nx * nfull) {
        gemm_f16_tail<WIDE>(W, K, x, xs, n, nfull * kTile, (b - nx * nfull) * 16, Y, ys, res, rs, smem);
        return;
    }
    const int t = threadIdx.x, r0 = (b % nx) * kTile, t0 = (b / nx) * kTile;
    const int lane = t & 63, wave = t >> 6, wr = wave & 1, wt = wave >> 1, li = lane & 15, lk = lane >> 4;
    // staging: thread t loads SP consecutive k of weight row / token t / 4, part t % 4
    const int sr = t >> 2, sp = (t & 3) * T::SP;
    const bool sok = t0 + sr < n;                 // tokens past n load row n - 1 and stage zeros
    const float * sx = x + (size_t) (sok ? t0 + sr : n - 1) * xs + sp;
    const uint16_t * sw = W + (size_t) (r0 + sr) * K + sp;
    v4i rw[NW];                                   // clang vectors: arrays of these stay in registers
    float4 rx[NX];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int u = 0; u < NW; ++u) rw[u] = *(const v4i *) (sw + k0 + 8 * u);
#pragma unroll
        for (int u = 0; u < NX; ++u) rx[u] = *(const float4 *) (sx + k0 + 4 * u);
    };
    auto stash = [&](int buf) {
        char * st = smem + buf * T::STAGE;
#pragma unroll
        for (int u = 0; u < NW; ++u) *(v4i *) (st + (sr * T::HS + sp + 8 * u) * 2) = rw[u];
        if (!sok) {                               // zeroed here, not at the load (which stays in flight)
#pragma unroll
            for (int u = 0; u < NX; ++u) rx[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (WIDE) {
            float * xr = (float *) (st + T::W_BYTES) + sr * T::FS + sp;
#pragma unroll
            for (int u = 0; u < NX; ++u) *(float4 *) (xr + 4 * u) = rx[u];
        } else {
            auto pk = [](float a, float b) { return (int) ((uint32_t) f2h(a) | ((uint32_t) f2h(b) << 16)); };
#pragma unroll
            for (int u = 0; u < NX / 2; ++u) {
                const float4 a = rx[2 * u], b = rx[2 * u + 1];
                *(int4 *) (st + T::W_BYTES + (sr * T::HS + sp + 8 * u) * 2) =
                    make_int4(pk(a.x, a.y), pk(a.z, a.w), pk(b.x, b.y), pk(b.z, b.w));
            }
        }
    };
    v4d acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = v4d{0.0, 0.0, 0.0, 0.0};
    const int C = K / KC;
    fetch(0);
    stash(0);
    __syncthreads();
    for (int ch = 0; ch < C; ++ch) {
        const int buf = ch & 1;
        if (ch + 1 < C) fetch((ch + 1) * KC);
        const char * sb = smem + buf * T::STAGE;
        int4 bw[2][E / 8];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int u = 0; u < E / 8; ++u)
                bw[j][u] = *(const int4 *) (sb + ((wr * 32 + 16 * j + li) * T::HS + E * lk + 8 * u) * 2);
        float ax[2][E];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int tr = wt * 32 + 16 * i + li;
            if (WIDE) {
                const float * xr = (const float *) (sb + T::W_BYTES) + tr * T::FS + E * lk;
#pragma unroll
                for (int u = 0; u < E / 4; ++u) {
                    const float4 q = *(const float4 *) (xr + 4 * u);
                    ax[i][4 * u] = q.x; ax[i][4 * u + 1] = q.y; ax[i][4 * u + 2] = q.z; ax[i][4 * u + 3] = q.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < E / 8; ++u) {
                    const int4 hv = *(const int4 *) (sb + T::W_BYTES + (tr * T::HS + E * lk + 8 * u) * 2);
#pragma unroll
                    for (int e = 0; e < 8; ++e) ax[i][8 * u + e] = h2f(h8bits(hv, e));
                }
            }
        }
#pragma unroll
        for (int s = 0; s < E; ++s) {
            double bd[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) bd[j] = (double) h2f(h8bits(bw[j][s >> 3], s & 7));
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const double ad = (double) ax[i][s];
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad, bd[j], acc[i][j], 0, 0, 0);
            }
        }
        if (ch + 1 < C) stash(buf ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tok = t0 + wt * 32 + 16 * i + 4 * r + lk;
            if (tok >= n) continue;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = r0 + wr * 32 + 16 * j + li;
                float v = (float) acc[i][j][r];
                if (res) v = v + res[(size_t) tok * rs + row];
                Y[(size_t) tok * ys + row] = v;
            }
        }
}

// ------------------------------------------------- F16 GEMM on fp16 MFMA
// The fast form of the F16 prefill GEMM: the reference's F16 mul_mat rounds
// its F32 activation to fp16 and accumulates fp16 x fp16 products in fp32
// (src/tts_transformer.cpp:1474-1617 via ggml), so v_mfma_f32_16x16x32_f16
// with fp32 accumulation is the same class of arithmetic (the exact
// f64-MFMA form above stays selectable; the two differ at fp32 rounding
// level).  Y[t][r] = (sum_k X[t][k] W[r][k]) * xsc[t] (+ res[t][r]).
//   - X arrives as fp16 rows (xh [n][xs]); the widened ffn_down (F32 weights
//     and activation in the reference) adds a low plane xl with
//     xh + xl = x * 2^-e to about 22 bits, the row scaled by a power of two
//     (xsc[t] = 2^e) so that neither plane overflows fp16; each weight
//     fragment then meets both planes, two MFMAs per step;
//   - the workgroup tile is 32 WM weight rows x 32 TT tokens, four waves in
//     a 2 x 2 arrangement, each 16 WM rows x 16 TT tokens as WM x TT MFMA
//     tiles with the weights as A (m = row) and the tokens as B (n = token),
//     so lane l's accumulator holds rows 4 (l/16) .. +3 of token l % 16:
//     one float4 store;
//   - K in stages of 64 staged in LDS as 16-byte chunks, chunk c of row r at
//     position c ^ (r & 7) (8 consecutive rows of one chunk hit distinct
//     banks), double-buffered: stage s + 1's global loads are in flight
//     during stage s's MFMAs;
//   - tokens past n stage zeros and store nothing.
// Requires N % (32 WM) == 0 and K % 64 == 0 (the host checks).
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef float f4v __attribute__((ext_vector_type(4)));
constexpr int kHK = 64;            // K per stage (8 chunks of 8 halves)

__device__ __forceinline__ int hswz(int r, int c) { return r * kHK + ((c ^ (r & 7)) << 3); }

// WM: 16-row MFMA tiles per wave along the weight rows (workgroup rows 32 WM);
// TT: 16-token tiles per wave (workgroup tokens 32 TT); LO: the low plane;
// PD: stages in flight (1: the next stage's loads overlap this stage's
// MFMAs; 2: two register sets, loads issued two stages ahead).
template <int WM, int TT, bool LO, int PD>
struct H16Tile {
    static constexpr int BR = 32 * WM, BT = 32 * TT;         // workgroup tile
    static constexpr int WSUB = BR * kHK, XSUB = BT * kHK;   // halves per stage and plane
    static constexpr int STAGE = WSUB + (LO ? 2 : 1) * XSUB;
    static constexpr int NW = BR * 8 / kBlock;               // W chunks per thread per stage
    static constexpr int NX = BT * 8 / kBlock;               // X chunks per thread per stage and plane
};

template <int WM, int TT, bool LO, int PD>
__global__ __launch_bounds__(kBlock) void k_gemm_h16(const uint16_t * __restrict__ W, int32_t K,
                                                     const uint16_t * __restrict__ xh, const uint16_t * __restrict__ xl,
                                                     int32_t xs, const float * __restrict__ xsc, int32_t n,
                                                     float * __restrict__ Y, int32_t ys, const float * __restrict__ res,
                                                     int32_t rs) {
    using T = H16Tile<WM, TT, LO, PD>;
    __shared__ __align__(16) uint16_t lds[2 * T::STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave & 1, wt = wave >> 1, lm = lane & 15, lk = lane >> 4;
    const int r0 = blockIdx.x * T::BR, t0 = blockIdx.y * T::BT;
    const uint16_t * gw[T::NW];
    int lw[T::NW];
#pragma unroll
    for (int u = 0; u < T::NW; ++u) {
        const int c = tid + u * kBlock, row = c >> 3, ch = c & 7;
        gw[u] = W + (size_t) (r0 + row) * K + ch * 8;
        lw[u] = hswz(row, ch);
    }
    size_t gx[T::NX];                              // element offsets of this thread's X chunks
    int lx[T::NX];
    bool ox[T::NX];
#pragma unroll
    for (int u = 0; u < T::NX; ++u) {
        // tokens past n load row n - 1 (no branch around the load) and stage zeros
        const int c = tid + u * kBlock, row = c >> 3, ch = c & 7;
        ox[u] = t0 + row < n;
        gx[u] = (size_t) (ox[u] ? t0 + row : n - 1) * xs + ch * 8;
        lx[u] = T::WSUB + hswz(row, ch);
    }
    // register sets of the stages in flight, indexed by compile-time
    // constants only (a runtime index would put them in scratch memory)
    v4i rw[PD][T::NW], rx[PD][T::NX], rl[PD][LO ? T::NX : 1];
    auto fetch = [&](auto set_c, int k0) {
        constexpr int set = decltype(set_c)::value;
#pragma unroll
        for (int u = 0; u < T::NW; ++u) rw[set][u] = *(const v4i *) (gw[u] + k0);
#pragma unroll
        for (int u = 0; u < T::NX; ++u) {
            rx[set][u] = *(const v4i *) (xh + gx[u] + k0);
            if (LO) rl[set][LO ? u : 0] = *(const v4i *) (xl + gx[u] + k0);
        }
    };
    auto stash = [&](auto set_c, int buf) {
        constexpr int set = decltype(set_c)::value;
        uint16_t * st = lds + buf * T::STAGE;
#pragma unroll
        for (int u = 0; u < T::NW; ++u) *(v4i *) (st + lw[u]) = rw[set][u];
#pragma unroll
        for (int u = 0; u < T::NX; ++u) {
            v4i a = rx[set][u];
            if (!ox[u]) a = (v4i){0, 0, 0, 0};
            *(v4i *) (st + lx[u]) = a;
            if (LO) {
                v4i b = rl[set][LO ? u : 0];
                if (!ox[u]) b = (v4i){0, 0, 0, 0};
                *(v4i *) (st + T::XSUB + lx[u]) = b;
            }
        }
    };
    f4v acc[WM][TT];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < TT; ++j) acc[i][j] = (f4v){0.f, 0.f, 0.f, 0.f};
    auto mfmas = [&](int buf) {
        const uint16_t * st = lds + buf * T::STAGE;
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            h8v af[WM], bf[TT], bl[LO ? TT : 1];
#pragma unroll
            for (int i = 0; i < WM; ++i) af[i] = *(const h8v *) (st + hswz(wr * 16 * WM + 16 * i + lm, 4 * q + lk));
#pragma unroll
            for (int j = 0; j < TT; ++j) {
                const int off = T::WSUB + hswz(wt * 16 * TT + 16 * j + lm, 4 * q + lk);
                bf[j] = *(const h8v *) (st + off);
                if (LO) bl[LO ? j : 0] = *(const h8v *) (st + T::XSUB + off);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < TT; ++j) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
                    if (LO) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bl[LO ? j : 0], acc[i][j], 0, 0, 0);
                }
        }
        // keep the next stage's LDS stores (and so the wait for its global
        // loads) after this stage's MFMAs: without the barriers the compiler
        // hoists them right behind the loads, which exposes the load latency
        __asm__ volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    };
    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, PD == 2 ? 1 : 0>;
    const int S = K / kHK;
    // stage s computes from LDS buffer s & 1.  PD 1: stage s + 1 is loaded into
    // the one register set during stage s and stashed after its MFMAs.  PD 2:
    // stage s + 2 is loaded into set s & 1 during stage s, while stage s + 1
    // (set (s + 1) & 1, loaded during stage s - 1) is stashed after the MFMAs.
    auto step = [&](int s, auto cur, auto nxt) {
        if (PD == 1 && s + 1 < S) fetch(C0{}, (s + 1) * kHK);
        if (PD == 2 && s + 2 < S) fetch(cur, (s + 2) * kHK);
        mfmas(s & 1);
        if (s + 1 < S) {
            if (PD == 1) stash(C0{}, (s + 1) & 1);
            else stash(nxt, (s + 1) & 1);
        }
        __syncthreads();
    };
    fetch(C0{}, 0);
    stash(C0{}, 0);
    if (PD == 2 && S > 1) fetch(C1{}, kHK);
    __syncthreads();
    for (int s = 0; s < S; s += 2) {
        step(s, C0{}, C1{});
        if (s + 1 < S) step(s + 1, C1{}, C0{});
    }
#pragma unroll
    for (int j = 0; j < TT; ++j) {
        const int tok = t0 + wt * 16 * TT + 16 * j + lm;
        if (tok >= n) continue;
        const float sc = xsc ? xsc[tok] : 1.0f;
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int row = r0 + wr * 16 * WM + 16 * i + 4 * lk;
            float4 v = make_float4(acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
            if (xsc) { v.x *= sc; v.y *= sc; v.z *= sc; v.w *= sc; }
            if (res) {
                const float4 q = *(const float4 *) (res + (size_t) tok * rs + row);
                v.x = v.x + q.x; v.y = v.y + q.y; v.z = v.z + q.z; v.w = v.w + q.w;
            }
            *(float4 *) (Y + (size_t) tok * ys + row) = v;
        }
    }
}

// fp16 rows for the fast GEMM: yh[t][e] = fp16(x[t][e]) (the rounding the
// reference's F16 mul_mat applies to its F32 activation).
__global__ __launch_bounds__(kBlock) void k_rows_h16(const float * __restrict__ x, int32_t xs, int32_t K, int32_t n,
                                                     uint16_t * __restrict__ yh) {
    const size_t cnt = (size_t) n * K;
    for (size_t i = (size_t) blockIdx.x * kBlock + threadIdx.x; i < cnt; i += (size_t) gridDim.x * kBlock) {
        const size_t t = i / K, e = i - t * K;
        yh[i] = f2h(x[t * xs + e]);
    }
}

// RMSNorm rows (k_rmsnorm_rows' numbers) written as fp16: the input of an F16
// GEMM, which rounds it to fp16 anyway.
__global__ __launch_bounds__(kBlock) void k_rmsnorm_rows_h16(const float * __restrict__ x, const float * __restrict__ w,
                                                             float eps, int32_t d, uint16_t * __restrict__ yh) {
    __shared__ double red[4];
    const float * xr = x + (size_t) blockIdx.x * d;
    double ss = 0.0;
    for (int e = threadIdx.x; e < d; e += kBlock) { const float v = xr[e]; ss += (double) (v * v); }
    const double tot = block_sum_d(ss, red);
    const float mean = (float) (tot / (double) d);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int e = threadIdx.x; e < d; e += kBlock) { const float v = xr[e] * scale; yh[(size_t) blockIdx.x * d + e] = f2h(v * w[e]); }
}

// SwiGLU rows f = silu(g) * u (k_swiglu_rows' numbers) as the two fp16 planes
// of the widened ffn_down's fast GEMM: with 2^e the power of two that puts
// the row's largest |f| in [2^13, 2^14), hi = fp16(f * 2^-e) and lo =
// fp16(f * 2^-e - hi) (the difference is exact in fp32), so hi + lo carries
// f * 2^-e to about 22 bits and neither plane can overflow; xsc[row] = 2^e
// undoes the scaling in the GEMM's epilogue.  One workgroup per row, ffn <=
// 16 * kBlock.
__global__ __launch_bounds__(kBlock) void k_swiglu_h16(const float * __restrict__ g, const float * __restrict__ u,
                                                       int32_t ffn, uint16_t * __restrict__ xh,
                                                       uint16_t * __restrict__ xl, float * __restrict__ xsc) {
    __shared__ float red[kBlock / 64];
    constexpr int M = 16;
    const size_t base = (size_t) blockIdx.x * ffn;
    float f[M];
    float am = 0.0f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int e = threadIdx.x + m * kBlock;
        f[m] = e < ffn ? silu_q3t(g[base + e]) * u[base + e] : 0.0f;
        am = fmaxf(am, fabsf(f[m]));
    }
    for (int o = 32; o > 0; o >>= 1) am = fmaxf(am, __shfl_xor(am, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = am;
    __syncthreads();
    am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int ex = (am > 0.0f && am <= 3.0e38f) ? ilogbf(am) - 13 : 0;
    const float down = ldexpf(1.0f, -ex);
    if (threadIdx.x == 0) xsc[blockIdx.x] = ldexpf(1.0f, ex);
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const int e = threadIdx.x + m * kBlock;
        if (e >= ffn) break;
        const float v = f[m] * down;
        const uint16_t h = f2h(v);
        xh[base + e] = h;
        xl[base + e] = f2h(v - h2f(h));
    }
}

// SwiGLU over rows: f = silu(g) * u.
__global__ __launch_bounds__(kBlock) void k_swiglu_rows(const float * __restrict__ g, const float * __restrict__ u,
                                                        float * __restrict__ f, size_t count) {
    for (size_t i = (size_t) blockIdx.x * kBlock + threadIdx.x; i < count; i += (size_t) gridDim.x * kBlock)
        f[i] = silu_q3t(g[i]) * u[i];
}

// K (QK-norm + NEOX RoPE) and V rows of n tokens into the KV cache at
// positions pos0 + tok, fp16 or (bf) bfloat16.  Grid (n, ceil(n_kv_head /
// 4)), one wave per (token, KV head), each lane owning elements lane and
// lane + 64.
__global__ __launch_bounds__(kBlock) void k_kv_rows(const float * __restrict__ qkv, int32_t qkv_stride, int32_t qd,
                                                    int32_t kd, const float * __restrict__ k_norm, float eps,
                                                    const float * __restrict__ rc, const float * __restrict__ rs,
                                                    uint16_t * __restrict__ kc, uint16_t * __restrict__ vc, int32_t n_ctx,
                                                    int32_t pos0, int32_t bf) {
    const int tok = blockIdx.x, g = blockIdx.y * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63, pos = pos0 + tok;
    if (g * kHD >= kd) return;                    // whole wave; no workgroup barrier follows
    const float * row = qkv + (size_t) tok * qkv_stride;
    float x0 = row[qd + g * kHD + l], x1 = row[qd + g * kHD + 64 + l];
    wave_norm_rope(x0, x1, k_norm, eps, rc + (size_t) pos * 64, rs + (size_t) pos * 64);
    const size_t o = ((size_t) g * n_ctx + pos) * kHD;
    kc[o + l] = f2kv(x0, bf);
    kc[o + 64 + l] = f2kv(x1, bf);
    vc[o + l] = f2kv(row[qd + kd + g * kHD + l], bf);
    vc[o + 64 + l] = f2kv(row[qd + kd + g * kHD + 64 + l], bf);
}

// Causal attention of n tokens over the cache (all rows already written).
// Block (h, tok): q-norm + RoPE, scores over positions [0, pos0+tok], fp64
// softmax denominator, fp16 (bf: bfloat16) probabilities, fp64 P.V.
// out [n][qd].
__global__ __launch_bounds__(kBlock) void k_attn_rows(const float * __restrict__ qkv, int32_t qkv_stride,
                                                      const float * __restrict__ q_norm, float eps,
                                                      const float * __restrict__ rc, const float * __restrict__ rs,
                                                      const uint16_t * __restrict__ kc, const uint16_t * __restrict__ vc,
                                                      int32_t n_ctx, int32_t n_head, int32_t n_kv_head, int32_t pos0,
                                                      float scale, float * __restrict__ out, int32_t out_stride,
                                                      int32_t bf) {
    extern __shared__ __align__(16) char smem[];
    double * red = (double *) smem;                   // 4 doubles
    float * fred = (float *) (smem + 32);             // 4 floats
    float * tmp = (float *) (smem + 64);              // 128
    float * qf = tmp + kHD;                           // 128
    double * pv = (double *) (qf + kHD);              // [4 waves][128]
    float * sc = (float *) (pv + 4 * kHD);            // [n_kv]
    const int h = blockIdx.x, tok = blockIdx.y, t = threadIdx.x;
    const int g = h / (n_head / n_kv_head);
    const int pos = pos0 + tok, n_kv = pos + 1;
    {
        const float v = t < kHD ? qkv[(size_t) tok * qkv_stride + h * kHD + t] : 0.0f;
        const float o = head_norm_rope(v, q_norm, eps, rc + (size_t) pos * 64, rs + (size_t) pos * 64, tmp, red);
        if (t < kHD) qf[t] = round_kv(o, bf);
    }
    __syncthreads();
    const int lane = t & 63, wave = t >> 6, sub = lane & 15, pw = lane >> 4;
    const uint16_t * kb = kc + (size_t) g * n_ctx * kHD;
    const uint16_t * vb = vc + (size_t) g * n_ctx * kHD;
    double qd8[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) qd8[e] = (double) qf[sub * 8 + e];
    float lmax = -INFINITY;
    for (int j0 = 0; j0 < n_kv; j0 += 16) {
        const int j = j0 + wave * 4 + pw;
        double acc = 0.0;
        if (j < n_kv) {
            const int4 k4 = *(const int4 *) (kb + (size_t) j * kHD + sub * 8);
            const uint16_t * kh = (const uint16_t *) &k4;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc = fma(qd8[e], (double) kv2f(kh[e], bf), acc);   // exact products
        }
        acc = group_sum_d(acc, 16);
        if (j < n_kv) {
            const float s = (float) acc * scale;
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
    for (int j = t; j < n_kv; j += kBlock) sc[j] = round_kv(sc[j] * inv, bf);
    __syncthreads();
    // P.V: lane owns dims 2*lane, 2*lane+1; wave w takes positions w, w+4, ...
    double o0 = 0.0, o1 = 0.0;
    for (int j = wave; j < n_kv; j += 4) {
        const double p = (double) sc[j];
        const uint32_t w2 = *(const uint32_t *) (vb + (size_t) j * kHD + 2 * lane);
        o0 = fma(p, (double) kv2f((uint16_t) (w2 & 0xffffu), bf), o0);
        o1 = fma(p, (double) kv2f((uint16_t) (w2 >> 16), bf), o1);
    }
    pv[wave * kHD + 2 * lane] = o0;
    pv[wave * kHD + 2 * lane + 1] = o1;
    __syncthreads();
    if (t < kHD) {
        const double r = (pv[t] + pv[kHD + t]) + (pv[2 * kHD + t] + pv[3 * kHD + t]);
        out[(size_t) tok * out_stride + h * kHD + t] = (float) r;
    }
}

// ------------------------------------------- causal attention on f64 MFMA
// The prefill's causal attention as three kernels per layer, for n rows at
// positions n_past.. (the K/V rows of all n tokens already in the cache):
//   k_att_scores  S[h][r][j] = fp32(q_r . k_j) * scale for j <= n_past + r,
//                 one workgroup per (head, 64-row tile) sweeping 64-position
//                 K tiles on v_mfma_f64_16x16x4f64;
//   k_att_softmax per row: maximum, exp, fp64 sum, P = fp16(e / sum) (the
//                 probabilities the reference's KQV product rounds to);
//   k_att_pv      O[r][h*128 + d] = fp32(sum_j P[r][j] V[j][d]) on the same
//                 MFMA, P and V^T staged in LDS per 64-position tile.
// q and k are fp16 values (or bfloat16 with a BF16 cache), so every product
// is exact in fp64 and every sum is an fp64 sum of exact terms, rounded once:
// the numbers of pf::k_attn_rows, whatever order the MFMA adds them in.
// MFMA lane layout (16x16x4 f64): A[m = l%16][k = l/16], B[k = l/16][n =
// l%16], D[m = 4r + l/16][n = l%16] in element r.  Step s of a contraction
// gives lane group k = l/16 the index 32k + s (scores, 128 dims: each lane
// reads 32 contiguous dims of its row) or 16k + s (P.V, 64 positions).
constexpr int kAT = 64;          // rows and positions per attention tile
constexpr int kKS = 136;         // LDS row stride (halves) of a staged K tile: conflict-free 16-byte reads
constexpr int kVS = 72;          // LDS row stride (halves) of staged P and V^T tiles

__device__ __forceinline__ double kvd(uint16_t h, bool bf) { return (double) kv2f(h, bf); }

// grid (n, ceil(n_head / 4)), one wave per (row, head): q of row r, head h
// (QK-norm, NEOX RoPE at position n_past + r) rounded to the cache type, into
// Qh[h][r][128].
__global__ __launch_bounds__(kBlock) void k_att_q(const float * __restrict__ qkv, int32_t qkv_stride,
                                                  const float * __restrict__ q_norm, float eps,
                                                  const float * __restrict__ rc, const float * __restrict__ rs,
                                                  int32_t n, int32_t n_past, int32_t n_head, uint16_t * __restrict__ Qh,
                                                  int32_t bf) {
    const int row = blockIdx.x, h = blockIdx.y * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63, pos = n_past + row;
    if (h >= n_head) return;                      // whole wave; no workgroup barrier follows
    const float * src = qkv + (size_t) row * qkv_stride + h * kHD;
    float x0 = src[l], x1 = src[64 + l];
    wave_norm_rope(x0, x1, q_norm, eps, rc + (size_t) pos * 64, rs + (size_t) pos * 64);
    uint16_t * dst = Qh + ((size_t) h * n + row) * kHD;
    dst[l] = f2kv(x0, bf);
    dst[64 + l] = f2kv(x1, bf);
}

// grid (n_head, Y, 2): workgroup y takes 64-row tiles y and tiles - 1 - y, so
// every workgroup sweeps about the same number of K tiles (the causal sweep
// of tile y is y + 1 tiles long); grid z = grp takes the 64-position K tiles
// at 128 s + 64 grp, so that two workgroups of four waves share each CU and
// one's MFMAs run while the other waits at a barrier.  An odd tile count
// leaves a middle tile: with Y = (tiles + 1) / 2 its own workgroup sweeps
// it; with Y = tiles / 2 (from 3 tiles on) its K steps are dealt out, step
// st to workgroup st mod Y, since score blocks are independent outputs.  The
// latter keeps 2 * n_head * tiles / 2 workgroups (two per CU at 2,049 rows,
// where a workgroup of its own would leave 16 CUs a third one).
// Wave w owns rows 16w..16w+15 of a tile (q from k_att_q): lane (i = l%16,
// k = l/16) holds dims 32k..32k+31 of row 16w + i, and four 16-position
// accumulators.  K tiles are double-buffered in LDS (tile s + 1 loaded into
// registers while tile s's MFMAs run; rows past the tile's last position
// staged as zero).
constexpr int kAttT = 256;       // threads of the MFMA attention kernels

// One 16x16x32 MFMA with fp32 accumulation on fp16 (or, bf, bfloat16)
// operands held as 16-bit patterns: the fast forms of the attention kernels.
template <bool BF>
__device__ __forceinline__ f4v mfma_h32(const int4 & a, const int4 & b, f4v c) {
    const v4i av = (v4i){a.x, a.y, a.z, a.w}, bv = (v4i){b.x, b.y, b.z, b.w};
    if constexpr (BF) {
        typedef __bf16 b8v __attribute__((ext_vector_type(8)));
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8v, av), __builtin_bit_cast(b8v, bv), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8v, av), __builtin_bit_cast(h8v, bv), c, 0, 0, 0);
    }
}

// FAST: the scores of a step on 16x16x32 fp16 (bfloat16) MFMAs with fp32
// accumulation (the reference's F16 K.Q product class) instead of the exact
// f64 MFMA sums: lane (i, k) supplies dims 32c + 8k .. +7 of q row 16w + i as
// A and of position 16 t4 + i as B for MFMA c of 4, and its accumulator
// element r is row 16w + 4k + r, position 16 t4 + i.
__global__ __launch_bounds__(kAttT) void k_att_scores_fast(const uint16_t * __restrict__ Qh,
                                                            const uint16_t * __restrict__ kc, int32_t n_ctx,
                                                            int32_t n_head, int32_t n_kv_head, int32_t n,
                                                            int32_t n_past, float scale, float * __restrict__ S,
                                                            int32_t ls, int32_t bf);

__global__ __launch_bounds__(kAttT) void k_att_scores(const uint16_t * __restrict__ Qh,
                                                       const uint16_t * __restrict__ kc, int32_t n_ctx, int32_t n_head,
                                                       int32_t n_kv_head, int32_t n, int32_t n_past, float scale,
                                                       float * __restrict__ S, int32_t ls, int32_t bf) {
    __shared__ __align__(16) uint16_t kt[2][kAT * kKS];
    const int h = blockIdx.x, tiles = (n + kAT - 1) / kAT, g = h / (n_head / n_kv_head), grp = blockIdx.z;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, i = l & 15, k = l >> 4;
    const int krow = t >> 4, kch = t & 15;                  // staging: positions krow + 16u, 8-dim chunk
    const uint16_t * kbase = kc + (size_t) g * n_ctx * kHD + 8 * kch;
    const int y = blockIdx.y, Y = gridDim.y;
    const bool spread = 2 * Y + 1 == tiles;                     // middle tile's K steps dealt out
    for (int pass = 0; pass < (spread ? 3 : 2); ++pass) {
        const int tile = pass == 0 ? y : pass == 1 ? tiles - 1 - y : Y;
        if (pass == 1 && tile == y) break;                      // the middle tile of an odd count
        const int row0 = tile * kAT, my_row = row0 + 16 * w + i;
        const int lim_tile = n_past + min(row0 + kAT, n) - 1;   // last position any row of the tile sees
        if (lim_tile < 64 * grp) continue;                      // no K tile for this group
        const int nst = (lim_tile - 64 * grp) / (2 * kAT) + 1;
        const int st0 = pass == 2 ? y : 0, sd = pass == 2 ? Y : 1;   // steps st0, st0 + sd, ...
        if (st0 >= nst) continue;
        // q of row my_row, dims 32k .. 32k+31 (fp16 / bfloat16 values, held as fp32)
        float a[32];
        {
            const bool ok = my_row < n;
            const int4 * src = (const int4 *) (Qh + ((size_t) h * n + (ok ? my_row : 0)) * kHD + 32 * k);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int4 v = ok ? src[c] : make_int4(0, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 8; ++e) a[8 * c + e] = kv2f(h8bits(v, e), bf);
            }
        }
        int4 rk[4];
        int kok[4];
        auto fetch = [&](int j0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + krow + 16 * u;
                kok[u] = j <= lim_tile;
                rk[u] = *(const int4 *) (kbase + (size_t) min(j, lim_tile) * kHD);
            }
        };
        auto stash = [&](int buf) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                *(int4 *) (&kt[buf][(krow + 16 * u) * kKS + 8 * kch]) = kok[u] ? rk[u] : make_int4(0, 0, 0, 0);
        };
        fetch(2 * kAT * st0 + 64 * grp);
        stash(0);
        __syncthreads();
        for (int st = st0, it = 0; st < nst; st += sd, ++it) {
            const int buf = it & 1, j0 = 2 * kAT * st + 64 * grp;
            const bool more = st + sd < nst;
            if (more) fetch(j0 + 2 * kAT * sd);
            v4d acc[4];
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) acc[t4] = v4d{0.0, 0.0, 0.0, 0.0};
            // positions past the tile's limit are zero in kt and never stored
#pragma unroll
            for (int c = 0; c < 4; ++c) {                      // dims 32k + 8c .. +7
                int4 kb[4];
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4)
                    kb[t4] = *(const int4 *) (&kt[buf][(16 * t4 + i) * kKS + 32 * k + 8 * c]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const double ad = (double) a[8 * c + e];
#pragma unroll
                    for (int t4 = 0; t4 < 4; ++t4)
                        acc[t4] = __builtin_amdgcn_mfma_f64_16x16x4f64(ad, kvd(h8bits(kb[t4], e), bf), acc[t4], 0, 0, 0);
                }
                // keep the next dims' loads and conversions after these MFMAs (register pressure)
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = row0 + 16 * w + 4 * r + k, j = j0 + 16 * t4 + i;
                    if (row < n && j <= n_past + row)
                        S[((size_t) h * n + row) * ls + j] = (float) acc[t4][r] * scale;
                }
            if (more) stash(buf ^ 1);
            __syncthreads();
        }
    }
}

// The fast form of k_att_scores (see its declaration); same grid, tile
// pairing, K staging and masking.
template <bool BF>
__device__ __forceinline__ void att_scores_fast_body(const uint16_t * __restrict__ Qh, const uint16_t * __restrict__ kc,
                                                     int32_t n_ctx, int32_t n_head, int32_t n_kv_head, int32_t n,
                                                     int32_t n_past, float scale, float * __restrict__ S, int32_t ls,
                                                     uint16_t (*kt)[kAT * kKS]) {
    const int h = blockIdx.x, tiles = (n + kAT - 1) / kAT, g = h / (n_head / n_kv_head), grp = blockIdx.z;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, i = l & 15, k = l >> 4;
    const int krow = t >> 4, kch = t & 15;
    const uint16_t * kbase = kc + (size_t) g * n_ctx * kHD + 8 * kch;
    const int y = blockIdx.y, Y = gridDim.y;
    const bool spread = 2 * Y + 1 == tiles;
    for (int pass = 0; pass < (spread ? 3 : 2); ++pass) {
        const int tile = pass == 0 ? y : pass == 1 ? tiles - 1 - y : Y;
        if (pass == 1 && tile == y) break;
        const int row0 = tile * kAT, my_row = row0 + 16 * w + i;
        const int lim_tile = n_past + min(row0 + kAT, n) - 1;
        if (lim_tile < 64 * grp) continue;
        const int nst = (lim_tile - 64 * grp) / (2 * kAT) + 1;
        const int st0 = pass == 2 ? y : 0, sd = pass == 2 ? Y : 1;
        if (st0 >= nst) continue;
        int4 qa[4];                                             // dims 32c + 8k .. +7 of row my_row
        {
            const bool ok = my_row < n;
            const int4 * src = (const int4 *) (Qh + ((size_t) h * n + (ok ? my_row : 0)) * kHD + 8 * k);
#pragma unroll
            for (int c = 0; c < 4; ++c) qa[c] = ok ? src[4 * c] : make_int4(0, 0, 0, 0);
        }
        int4 rk[4];
        int kok[4];
        auto fetch = [&](int j0) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int j = j0 + krow + 16 * u;
                kok[u] = j <= lim_tile;
                rk[u] = *(const int4 *) (kbase + (size_t) min(j, lim_tile) * kHD);
            }
        };
        auto stash = [&](int buf) {
#pragma unroll
            for (int u = 0; u < 4; ++u)
                *(int4 *) (&kt[buf][(krow + 16 * u) * kKS + 8 * kch]) = kok[u] ? rk[u] : make_int4(0, 0, 0, 0);
        };
        fetch(2 * kAT * st0 + 64 * grp);
        stash(0);
        __syncthreads();
        for (int st = st0, it = 0; st < nst; st += sd, ++it) {
            const int buf = it & 1, j0 = 2 * kAT * st + 64 * grp;
            const bool more = st + sd < nst;
            if (more) fetch(j0 + 2 * kAT * sd);
            f4v acc[4];
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) acc[t4] = (f4v){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int t4 = 0; t4 < 4; ++t4)
                    acc[t4] = mfma_h32<BF>(qa[c], *(const int4 *) (&kt[buf][(16 * t4 + i) * kKS + 32 * c + 8 * k]),
                                           acc[t4]);
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = row0 + 16 * w + 4 * k + r, j = j0 + 16 * t4 + i;
                    if (row < n && j <= n_past + row) S[((size_t) h * n + row) * ls + j] = acc[t4][r] * scale;
                }
            __asm__ volatile("" ::: "memory");
            if (more) stash(buf ^ 1);
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(kAttT) void k_att_scores_fast(const uint16_t * __restrict__ Qh,
                                                            const uint16_t * __restrict__ kc, int32_t n_ctx,
                                                            int32_t n_head, int32_t n_kv_head, int32_t n,
                                                            int32_t n_past, float scale, float * __restrict__ S,
                                                            int32_t ls, int32_t bf) {
    __shared__ __align__(16) uint16_t kt[2][kAT * kKS];
    if (bf) att_scores_fast_body<true>(Qh, kc, n_ctx, n_head, n_kv_head, n, n_past, scale, S, ls, kt);
    else att_scores_fast_body<false>(Qh, kc, n_ctx, n_head, n_kv_head, n, n_past, scale, S, ls, kt);
}

// One row held in registers, R positions per lane (cnt <= 64 R).  Each lane
// adds its terms in position order and lanes past cnt add exact zeros, so the
// sum is the one of the three-pass loop below, whatever R.
template <int R>
__device__ __forceinline__ void softmax_row_reg(const float * __restrict__ sr, uint16_t * __restrict__ pr, int cnt,
                                                int lane, int bf) {
    float v[R];
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int j = lane + 64 * u;
        v[u] = j < cnt ? sr[j] : -INFINITY;
        m = fmaxf(m, v[u]);
    }
    const float mx = wave_max_f(m);
    double sum = 0.0;
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int j = lane + 64 * u;
        v[u] = j < cnt ? expf_q3t(v[u] - mx) : 0.0f;
        sum += (double) v[u];
    }
    const float inv = (float) (1.0 / wave_sum_d(sum));
#pragma unroll
    for (int u = 0; u < R; ++u) {
        const int j = lane + 64 * u;
        if (j < cnt) pr[j] = f2kv(v[u] * inv, bf);
    }
}

// grid (ceil(n / 4), n_head), one wave per row: P[h][r][j] = fp16(exp(S -
// max) / sum) for j <= n_past + r (bfloat16 with a BF16 cache), as
// pf::k_attn_rows rounds it.  Rows of up to 2,560 positions stay in
// registers (one read of S; 16, 32 or 40 per lane by length, so a 2,049-
// position row is not the three-read straggler that ends the launch, and the
// kernel keeps 64 VGPRs, eight waves per SIMD); longer rows are read three
// times.
__global__ __launch_bounds__(kBlock) void k_att_softmax(const float * __restrict__ S, int32_t n, int32_t n_past,
                                                        int32_t ls, uint16_t * __restrict__ P, int32_t bf) {
    const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6), h = blockIdx.y;
    if (row >= n) return;                   // whole wave
    const int cnt = n_past + row + 1;
    const float * sr = S + ((size_t) h * n + row) * ls;
    uint16_t * pr = P + ((size_t) h * n + row) * ls;
    if (cnt <= 64 * 16) { softmax_row_reg<16>(sr, pr, cnt, lane, bf); return; }
    if (cnt <= 64 * 32) { softmax_row_reg<32>(sr, pr, cnt, lane, bf); return; }
    if (cnt <= 64 * 40) { softmax_row_reg<40>(sr, pr, cnt, lane, bf); return; }
    float m = -INFINITY;
    for (int j = lane; j < cnt; j += 64) m = fmaxf(m, sr[j]);
    const float mx = wave_max_f(m);
    double sum = 0.0;
    for (int j = lane; j < cnt; j += 64) sum += (double) expf_q3t(sr[j] - mx);
    const float inv = (float) (1.0 / wave_sum_d(sum));
    for (int j = lane; j < cnt; j += 64) pr[j] = f2kv(expf_q3t(sr[j] - mx) * inv, bf);
}

// grid (n_head, Y, 2), tiles paired as in k_att_scores; grid z = grp takes
// dims 64 grp .. 64 grp + 63.  An odd tile count's middle tile: with Y =
// (tiles + 1) / 2 its own workgroup sweeps it; with Y = tiles / 2 (from 3
// tiles on) its four 16-row groups are dealt out, group q to workgroup q mod
// Y, which stages the tile as usual and sweeps it for those 16 rows only,
// wave w taking dims 16 w .. 16 w + 15 (one accumulator; every output is the
// same sum, in the same order, as in the undealt form).  Four waves: wave w owns rows
// 16w..16w+15 of a tile and dims 64 grp + 4 i + d4 (lane i = l%16, d4 =
// 0..3) as four 16 x 16 accumulators, so each lane reads its four B operands
// of a step with one 8-byte load and stores four consecutive floats.  P tiles
// [row][position] and V tiles [position][dim] are double-buffered in LDS:
// step s + 1's tiles are loaded into registers while step s's MFMAs run.
// Probabilities past a row's last position, and V rows past the tile's last
// position, are staged as zero.
constexpr int kVN = 64 + 8;      // LDS row stride (halves) of a staged V half-tile: conflict-free 16-byte writes
__global__ __launch_bounds__(kAttT, 4) void k_att_pv(const uint16_t * __restrict__ P, int32_t ls,
                                                   const uint16_t * __restrict__ vc, int32_t n_ctx, int32_t n_head,
                                                   int32_t n_kv_head, int32_t n, int32_t n_past,
                                                   float * __restrict__ out, int32_t out_stride, int32_t bf) {
    __shared__ __align__(16) uint16_t pt[2][kAT * kVS];      // [row][position]
    __shared__ __align__(16) uint16_t vt[2][kAT * kVN];      // [position][dim - 64 grp]
    const int h = blockIdx.x, tiles = (n + kAT - 1) / kAT, g = h / (n_head / n_kv_head), grp = blockIdx.z;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, i = l & 15, k = l >> 4;
    const int srow = t >> 3, sch = t & 7;                    // staging: rows / positions srow + 32u, 8-wide chunk
    const uint16_t * vbase = vc + (size_t) g * n_ctx * kHD + 64 * grp + 8 * sch;
    const int y = blockIdx.y, Y = gridDim.y;
    // passes: tiles y and tiles - 1 - y, then (spread) middle-tile row groups y, y + Y, ... < 4
    const int nrg = (2 * Y + 1 == tiles && y < 4) ? (4 - y + Y - 1) / Y : 0;
  for (int pass = 0; pass < 2 + nrg; ++pass) {
    const int rg = pass < 2 ? -1 : y + (pass - 2) * Y;        // row group of the middle tile, or -1
    const int tile = pass == 0 ? y : pass == 1 ? tiles - 1 - y : Y;
    if (pass == 1 && tile == y) continue;                     // the middle tile of an odd count
    const int row0 = tile * kAT, prow = rg < 0 ? 16 * w : 16 * rg;   // first A row of this wave in the tile
    const int lim_tile = n_past + min(row0 + kAT, n) - 1;
    const int nst = lim_tile / kAT + 1;
    int plim[2];
    const uint16_t * prp[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int prw = row0 + srow + 32 * u;
        plim[u] = prw < n ? n_past + prw : -1;
        prp[u] = P + ((size_t) h * n + (prw < n ? prw : 0)) * ls + 8 * sch;
    }
    int4 rp[2], rv[2];
    int pvalid[2], vok[2];
    // loads for step j0 / kAT into registers; the masks are applied at stash
    // time so that the loads stay in flight across the MFMAs
    auto fetch = [&](int j0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            pvalid[u] = min(max(plim[u] - (j0 + 8 * sch) + 1, 0), 8);   // valid positions of the chunk
            rp[u] = *(const int4 *) (prp[u] + (pvalid[u] > 0 ? j0 : 0)); // j0 + 63 < ls: in the row
            const int pos = j0 + srow + 32 * u;
            vok[u] = pos <= lim_tile;
            rv[u] = *(const int4 *) (vbase + (size_t) min(pos, lim_tile) * kHD);
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            int4 v = rp[u];
            const int pv = pvalid[u];
            if (pv < 8) {
                const auto m = [pv](int e) { return (2 * e < pv ? 0xffff : 0) | (2 * e + 1 < pv ? (int) 0xffff0000u : 0); };
                v.x &= m(0); v.y &= m(1); v.z &= m(2); v.w &= m(3);
            }
            *(int4 *) (&pt[buf][(srow + 32 * u) * kVS + 8 * sch]) = v;
            *(int4 *) (&vt[buf][(srow + 32 * u) * kVN + 8 * sch]) = vok[u] ? rv[u] : make_int4(0, 0, 0, 0);
        }
    };
    v4d acc[4];
#pragma unroll
    for (int d4 = 0; d4 < 4; ++d4) acc[d4] = v4d{0.0, 0.0, 0.0, 0.0};
    fetch(0);
    stash(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        if (st + 1 < nst) fetch((st + 1) * kAT);
        int4 pa[2];
        pa[0] = *(const int4 *) (&pt[buf][(prow + i) * kVS + 16 * k]);
        pa[1] = *(const int4 *) (&pt[buf][(prow + i) * kVS + 16 * k + 8]);
        if (rg < 0) {
            const uint16_t * vr = &vt[buf][16 * k * kVN + 4 * i];
#pragma unroll
            for (int s = 0; s < 16; ++s) {                   // position 16k + s of the tile
                const double pd = kvd(h8bits(pa[s >> 3], s & 7), bf);
                const uint2 vv = *(const uint2 *) (vr + s * kVN);
#pragma unroll
                for (int d4 = 0; d4 < 4; ++d4) {
                    const uint32_t word = (d4 >> 1) ? vv.y : vv.x;
                    const uint16_t vh = (uint16_t) ((d4 & 1) ? (word >> 16) : (word & 0xffffu));
                    acc[d4] = __builtin_amdgcn_mfma_f64_16x16x4f64(pd, kvd(vh, bf), acc[d4], 0, 0, 0);
                }
            }
        } else {                                             // rows 16 rg + .., wave w: dims 16 w + i
            const uint16_t * vr = &vt[buf][16 * k * kVN + 16 * w + i];
#pragma unroll
            for (int s = 0; s < 16; ++s)
                acc[0] = __builtin_amdgcn_mfma_f64_16x16x4f64(kvd(h8bits(pa[s >> 3], s & 7), bf), kvd(vr[s * kVN], bf),
                                                              acc[0], 0, 0, 0);
        }
        if (st + 1 < nst) stash(buf ^ 1);
        __syncthreads();
    }
    if (rg < 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 16 * w + 4 * r + k;
            if (row < n)
                *(float4 *) (out + (size_t) row * out_stride + h * kHD + 64 * grp + 4 * i) =
                    make_float4((float) acc[0][r], (float) acc[1][r], (float) acc[2][r], (float) acc[3][r]);
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 16 * rg + 4 * r + k;
            if (row < n) out[(size_t) row * out_stride + h * kHD + 64 * grp + 16 * w + i] = (float) acc[0][r];
        }
    }
  }
}

// The fast form of k_att_pv: P.V on 16x16x32 fp16 (bfloat16) MFMAs with
// fp32 accumulation.  Same grid, tile pairing, P staging and masks; the V
// tile is staged transposed ([dim][position], 8 two-byte stores per 8-dim
// chunk) so that lane (i, k) reads positions 32q + 8k .. +7 of dim 16 b + i as
// one 16-byte B operand, against P row 16w + i (A).  Accumulator b holds dims
// 64 grp + 16 b + i of rows 16w + 4k + r (the middle-tile row groups: wave w's
// dims 16 w + i of rows 16 rg + 4k + r).
constexpr int kVT = 64 + 8;      // LDS row stride (halves) of the transposed V tile
template <bool BF>
__device__ __forceinline__ void att_pv_fast_body(const uint16_t * __restrict__ P, int32_t ls,
                                                 const uint16_t * __restrict__ vc, int32_t n_ctx, int32_t n_head,
                                                 int32_t n_kv_head, int32_t n, int32_t n_past, float * __restrict__ out,
                                                 int32_t out_stride, uint16_t (*pt)[kAT * kVS],
                                                 uint16_t (*vt)[kAT * kVT]) {
    const int h = blockIdx.x, tiles = (n + kAT - 1) / kAT, g = h / (n_head / n_kv_head), grp = blockIdx.z;
    const int t = threadIdx.x, w = t >> 6, l = t & 63, i = l & 15, k = l >> 4;
    const int srow = t >> 3, sch = t & 7;
    const uint16_t * vbase = vc + (size_t) g * n_ctx * kHD + 64 * grp + 8 * sch;
    const int y = blockIdx.y, Y = gridDim.y;
    const int nrg = (2 * Y + 1 == tiles && y < 4) ? (4 - y + Y - 1) / Y : 0;
  for (int pass = 0; pass < 2 + nrg; ++pass) {
    const int rg = pass < 2 ? -1 : y + (pass - 2) * Y;
    const int tile = pass == 0 ? y : pass == 1 ? tiles - 1 - y : Y;
    if (pass == 1 && tile == y) continue;
    const int row0 = tile * kAT, prow = rg < 0 ? 16 * w : 16 * rg;
    const int lim_tile = n_past + min(row0 + kAT, n) - 1;
    const int nst = lim_tile / kAT + 1;
    int plim[2];
    const uint16_t * prp[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int prw = row0 + srow + 32 * u;
        plim[u] = prw < n ? n_past + prw : -1;
        prp[u] = P + ((size_t) h * n + (prw < n ? prw : 0)) * ls + 8 * sch;
    }
    int4 rp[2], rv[2];
    int pvalid[2], vok[2];
    auto fetch = [&](int j0) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            pvalid[u] = min(max(plim[u] - (j0 + 8 * sch) + 1, 0), 8);
            rp[u] = *(const int4 *) (prp[u] + (pvalid[u] > 0 ? j0 : 0));
            const int pos = j0 + srow + 32 * u;
            vok[u] = pos <= lim_tile;
            rv[u] = *(const int4 *) (vbase + (size_t) min(pos, lim_tile) * kHD);
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            int4 v = rp[u];
            const int pv = pvalid[u];
            if (pv < 8) {
                const auto m = [pv](int e) { return (2 * e < pv ? 0xffff : 0) | (2 * e + 1 < pv ? (int) 0xffff0000u : 0); };
                v.x &= m(0); v.y &= m(1); v.z &= m(2); v.w &= m(3);
            }
            *(int4 *) (&pt[buf][(srow + 32 * u) * kVS + 8 * sch]) = v;
            const int4 vv = vok[u] ? rv[u] : make_int4(0, 0, 0, 0);
            const int pos = srow + 32 * u;
#pragma unroll
            for (int e = 0; e < 8; ++e) vt[buf][(8 * sch + e) * kVT + pos] = h8bits(vv, e);
        }
    };
    f4v acc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[b] = (f4v){0.f, 0.f, 0.f, 0.f};
    fetch(0);
    stash(0);
    __syncthreads();
    for (int st = 0; st < nst; ++st) {
        const int buf = st & 1;
        if (st + 1 < nst) fetch((st + 1) * kAT);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const int4 pa = *(const int4 *) (&pt[buf][(prow + i) * kVS + 32 * q + 8 * k]);
            if (rg < 0) {
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    acc[b] = mfma_h32<BF>(pa, *(const int4 *) (&vt[buf][(16 * b + i) * kVT + 32 * q + 8 * k]), acc[b]);
            } else {
                acc[0] = mfma_h32<BF>(pa, *(const int4 *) (&vt[buf][(16 * w + i) * kVT + 32 * q + 8 * k]), acc[0]);
            }
        }
        __asm__ volatile("" ::: "memory");
        if (st + 1 < nst) stash(buf ^ 1);
        __syncthreads();
    }
    if (rg < 0) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = row0 + 16 * w + 4 * k + r;
                if (row < n) out[(size_t) row * out_stride + h * kHD + 64 * grp + 16 * b + i] = acc[b][r];
            }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = row0 + 16 * rg + 4 * k + r;
            if (row < n) out[(size_t) row * out_stride + h * kHD + 64 * grp + 16 * w + i] = acc[0][r];
        }
    }
  }
}

__global__ __launch_bounds__(kAttT, 4) void k_att_pv_fast(const uint16_t * __restrict__ P, int32_t ls,
                                                        const uint16_t * __restrict__ vc, int32_t n_ctx,
                                                        int32_t n_head, int32_t n_kv_head, int32_t n, int32_t n_past,
                                                        float * __restrict__ out, int32_t out_stride, int32_t bf) {
    __shared__ __align__(16) uint16_t pt[2][kAT * kVS];
    __shared__ __align__(16) uint16_t vt[2][kAT * kVT];
    if (bf) att_pv_fast_body<true>(P, ls, vc, n_ctx, n_head, n_kv_head, n, n_past, out, out_stride, pt, vt);
    else att_pv_fast_body<false>(P, ls, vc, n_ctx, n_head, n_kv_head, n, n_past, out, out_stride, pt, vt);
}

__host__ __device__ constexpr size_t attn_rows_lds_bytes(int n_ctx) {
    return 64 + 2 * kHD * sizeof(float) + 4 * kHD * sizeof(double) + (size_t) n_ctx * sizeof(float);
}

}  // namespace pf
}  // namespace q3t
