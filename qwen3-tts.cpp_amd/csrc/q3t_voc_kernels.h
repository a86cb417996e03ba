// q3t_voc_kernels.h -- gfx950 kernels of the audio-tokenizer decoder (the
// vocoder after the frame loop, src/audio_tokenizer_decoder.cpp).
//
// Layout: activations are time-major rows [t][c] with the channel stride
// padded to a multiple of 32 (pad channels hold zeros), so that every
// convolution and linear layer is one GEMM over (tap, channel) on
// v_mfma_f32_16x16x32_f16: the F16 weights times the fp16-rounded activation
// (ggml's F16 im2col / vec_dot_type), accumulated in fp32 as ggml does.
// Element-wise work (bias, layer scale, residual add, snake / GELU / SwiGLU
// and the fp16 rounding of the next layer's input) runs in the GEMM's
// epilogue, so each conv reads its input once and writes its output once.
#pragma once

#include "q3t_numerics.h"

namespace q3t {
namespace voc {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

enum : int32_t { ACT_NONE = 0, ACT_SNAKE = 1, ACT_GELU = 2, ACT_SWIGLU = 3 };

// sin(y)^2 in fp32: Cody-Waite reduction r = y - k pi/2 (k = rint(y 2/pi),
// pi/2 as a three-part sum applied with fused multiply-adds), the degree-9
// Taylor polynomial of sin on |r| <= pi/4 (truncation below 3e-9 relative),
// and sin^2(y) = sin^2(r) for even k, cos^2(r) = 1 - sin^2(r) for odd k.
// Within 4 ulp of the true value (sinf squared: within 3), at about half of
// sinf's instructions.  |y| beyond 2^13 takes sinf.
__device__ __forceinline__ float sin_sq(float y) {
    if (fabsf(y) > 8192.0f) {
        const float s = sinf(y);
        return s * s;
    }
    const float k = rintf(y * 0.636619746685028076171875f);
    float r = fmaf(-k, 1.57079637050628662109375f, y);
    r = fmaf(-k, -4.37113882867379300296306610107421875e-8f, r);
    r = fmaf(-k, -1.715124510005881882e-15f, r);
    const float r2 = r * r;
    float p = fmaf(r2, 2.7557318844628753e-6f, -1.9841270113829523e-4f);
    p = fmaf(r2, p, 8.333333767950535e-3f);
    p = fmaf(r2, p, -0.1666666716337204f);
    const float sn = fmaf(r * r2, p, r);
    const float ss = sn * sn;
    return ((int) k & 1) ? 1.0f - ss : ss;
}

// snake (src/audio_tokenizer_decoder.cpp:402-426): x + sin(x e^a)^2 e^-b,
// with ea = e^alpha and eb = e^-beta per channel (computed on the host).
__device__ __forceinline__ float snake(float x, float ea, float eb) {
    const float sq = sin_sq(x * ea);
    return x + sq * eb;
}

// ggml_gelu's tanh form
__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.79788456080286535587989211986876f, a = 0.044715f;
    return 0.5f * x * (1.0f + tanhf(c * x * (1.0f + a * x * x)));
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + expf(-x)); }

// One GEMM launch: Y[m * ostride + phase][n] = epi(sum_{tap, c} W[phase][n][tap][c]
//                                                   * X[m + off0 + tap * dil][c])
// X rows outside [0, rows_in) are zero (causal padding).  Epilogue, in the
// graph's op order: v = acc; v += bias[n]; v *= scale[n]; v = res[row][n] + v;
// yf[row][n] = v; yh[row][n] = fp16(act(v)).  ACT_SWIGLU pairs 16-channel
// tiles (2q: gate, 2q+1: up, interleaved at upload) and writes
// fp16(silu(gate) * up) at channel 16q + i.
struct ConvArgs {
    const uint16_t * x; int32_t xs, rows_in;
    const uint16_t * w; int32_t Cp, KT, dil, off0;
    int32_t M, N, Np, ostride;
    const float * bias, * scale, * res; int32_t rs;
    float * yf; int32_t yfs;
    uint16_t * yh; int32_t yhs;
    int32_t act;
    const float * ea, * eb;
    // FU launches (a residual unit in one launch): this launch's GEMM is the
    // unit's k7 conv, whose output (+ bias, snake ea/eb, fp16) stays in LDS
    // as the input of the 1-tap conv w2 ([N][N] fp16), whose output takes
    // bias2, the residual res and act2 (ea2, eb2) into yf / yh
    const uint16_t * w2;
    const float * bias2;
    int32_t act2;
    const float * ea2, * eb2;
};

constexpr int kGemmT = 256;    // 4 waves: 2 along channels x 2 along time

// The workgroup tile is 32 WM channels x 32 WN rows; wave (wc, wt) owns WM
// 16-channel tiles x WN 16-row tiles.  Each K step (KS chunks of one tap x 32
// channels) stages the weight rows and the activation rows of the tile in LDS,
// double-buffered, from registers loaded two steps ahead: the loads of step
// s + 2 are issued before step s runs on the matrix cores and stored to LDS
// only after step s + 1 has run, so a load round trip overlaps two steps
// (with the loads of step s + 1 stored right after step s, every step waited
// for its own round trip).  The loads are buffer loads whose range check
// returns zeros: causal padding rows, rows past the launch and chunks past
// the contraction need no branches.  MFMA lane layout (16x16x32):
// A[m = l%16][k = 8(l/16)..+7] (weights, m = channel), B[k][n = l%16]
// (activations, n = time row), D[m = 4(l/16)+e][n = l%16].  The SwiGLU
// pairing needs WM even.  KS = 4 for the small launches (the 73-row
// pre-transformer GEMMs), whose K loop of 16-32 steps would otherwise be a
// chain of load-and-barrier round trips.
template <int WM, int WN, int KS = 1>
struct GemmTile {
    static constexpr int BC = 32 * WM, BT = 32 * WN;
    static constexpr int NA = (BC * 4 + kGemmT - 1) / kGemmT, NB = (BT * 4 + kGemmT - 1) / kGemmT;
    static constexpr int SUB = (BC + BT) * 32;                      // halfs per chunk
    static constexpr int STAGE = KS * SUB;                          // halfs per stage
    static constexpr int TS = WM * 16 + 4;                          // epilogue row stride (floats)
    static constexpr int LDS_STAGE = 2 * STAGE * 2, LDS_EPI = 4 * 16 * TS * 4;
    static constexpr int LDS = LDS_STAGE > LDS_EPI ? LDS_STAGE : LDS_EPI;
};

// LDS slot of 16-byte piece c of tile row r (rows of 4 pieces, 64 bytes):
// piece c sits at c ^ ((r >> 1) & 3), so the pieces c of 8 consecutive rows
// (a fragment read: 8 lanes, rows r0..r0+7) cover all 32 banks, and so do
// 8 consecutive threads writing rows 2q and 2q + 1.
__device__ __forceinline__ int swz(int row, int chunk) { return row * 32 + ((chunk ^ ((row >> 1) & 3)) << 3); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// A buffer resource over `bytes` bytes at p: loads at offsets past `bytes`
// (or at 0x80000000, the out-of-range marker used here) return zeros.  Stride
// 0 (raw addressing: the range check applies to the byte offset); the last
// word, 0x00020000, is the gfx9 format word for untyped 32-bit data.  The host
// keeps every range below 2^31 bytes, so the marker is always out of range.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void * p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *) p, (short) 0, (int) bytes, 0x00020000);
}
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, (int) off, 0, 0);
    return make_uint4(v.x, v.y, v.z, v.w);
}
constexpr uint32_t kOut = 0x80000000u;

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

// The epilogue of a wave's WM x WN tiles of 16 channels x 16 rows (channels
// [ch0, ch0 + 16 WM), rows [t0, t0 + 16 WN)), one 16-row tile at a time
// through the wave's LDS slice `my` (16 x (16 WM + 4) floats, [row][channel]),
// then 64 lanes walk it channel-fastest (coalesced row stores).  LDS is in
// order within a wave, so no barrier is needed.
// RP (A.res set): every residual value of the tiles is loaded before any is
// used, so their reads overlap instead of forming one dependent chain; the
// registers this takes lower the occupancy, which the convolutions without a
// residual (whose K loops need it) keep.
template <int WM, int WN, bool RP>
__device__ __forceinline__ void conv_epilogue(const ConvArgs & A, const v4f (&acc)[WM][WN], float * my, int ch0, int t0,
                                              int phase, int lane) {
    const int lm = lane & 15, lk = lane >> 4;
    constexpr int TC = WM * 16, TS = TC + 4;
    constexpr int IT = 16 * TC / 64;                 // elements per lane of one 16-row tile
    // element k of a lane sits in channel (lane + 64 k) % TC, which repeats
    // with period P in k: the per-channel parameters are loaded once
    constexpr int P = TC / gcd_c(TC, 64);
    static_assert(IT % P == 0, "whole periods");
    float pb[P], ps[P], pa[P], pe[P];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int n = ch0 + (lane + 64 * p) % TC;
        const bool ok = n < A.N;
        pb[p] = A.bias && ok ? A.bias[n] : 0.0f;
        ps[p] = A.scale && ok ? A.scale[n] : 0.0f;
        pa[p] = A.act == ACT_SNAKE && ok ? A.ea[n] : 0.0f;
        pe[p] = A.act == ACT_SNAKE && ok ? A.eb[n] : 0.0f;
    }
    // up to 48 residual values per lane are loaded for all tiles at once,
    // more one 16-row tile at a time
    constexpr bool ALL = WN * IT <= 48;
    constexpr int RJ = RP && ALL ? WN : 1;
    float rv[RJ][RP ? IT : 1];
    // element offsets in 32 bits (the host checks that they fit)
    const uint32_t ost = (uint32_t) A.ostride, ph = (uint32_t) phase;
    auto load_res = [&](int j, int slot) {
#pragma unroll
        for (int k = 0; k < IT; ++k) {
            const int idx = lane + 64 * k, tl = idx / TC, cl = idx - tl * TC;
            const int t = t0 + j * 16 + tl, n = ch0 + cl;
            rv[slot][RP ? k : 0] =
                t < A.M && n < A.N ? A.res[((uint32_t) t * ost + ph) * (uint32_t) A.rs + (uint32_t) n] : 0.0f;
        }
    };
    if (RP && ALL) {
#pragma unroll
        for (int j = 0; j < WN; ++j) load_res(j, RJ > 1 ? j : 0);
    }
#pragma unroll
    for (int j = 0; j < WN; ++j) {
        if (RP && !ALL) load_res(j, 0);
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) my[lm * TS + i * 16 + 4 * lk + e] = acc[i][j][e];
        __builtin_amdgcn_wave_barrier();
        const int tbase = t0 + j * 16;
        if (A.act == ACT_SWIGLU) {
            // tiles 2q (gate) and 2q + 1 (up) of channel group q
            for (int idx = lane; idx < 16 * (TC / 2); idx += 64) {
                const int tl = idx / (TC / 2), ol = idx - tl * (TC / 2);
                const int t = tbase + tl;
                const int pr = ol >> 4, w = ol & 15;
                const int n = ((ch0 >> 1) + pr * 16) + w;
                if (t >= A.M || n >= (A.N >> 1)) continue;
                const float g = my[tl * TS + pr * 32 + w], u = my[tl * TS + pr * 32 + 16 + w];
                A.yh[((uint32_t) t * ost + ph) * (uint32_t) A.yhs + (uint32_t) n] = f2h(silu(g) * u);
            }
        } else {
#pragma unroll
            for (int k = 0; k < IT; ++k) {
                const int idx = lane + 64 * k, tl = idx / TC, cl = idx - tl * TC;
                const int t = tbase + tl, n = ch0 + cl;
                if (t >= A.M || n >= A.N) continue;
                const uint32_t row = (uint32_t) t * ost + ph;
                float v = my[tl * TS + cl];
                if (A.bias) v = v + pb[k % P];
                if (A.scale) v = v * ps[k % P];
                if (RP) v = rv[RJ > 1 ? j : 0][RP ? k : 0] + v;
                else if (A.res) v = A.res[row * (uint32_t) A.rs + (uint32_t) n] + v;
                if (A.yf) A.yf[row * (uint32_t) A.yfs + (uint32_t) n] = v;
                if (A.yh) {
                    float h = v;
                    if (A.act == ACT_SNAKE) h = snake(v, pa[k % P], pe[k % P]);
                    else if (A.act == ACT_GELU) h = gelu_tanh(v);
                    A.yh[row * (uint32_t) A.yhs + (uint32_t) n] = f2h(h);
                }
            }
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// The epilogue straight from the MFMA output layout, for launches whose
// channel count and row strides are multiples of 4 (all but SwiGLU): lane (lm, lk) of tile
// (i, j) holds channels 16 i + 4 lk .. + 3 of row 16 j + lm, so each lane
// loads its 4 residuals and stores its 4 fp32 results as one 16-byte access
// and its 4 fp16 results as one 8-byte access, with the per-channel
// parameters loaded once per tile column i.  No LDS round trip and no
// per-element index arithmetic; the arithmetic per element is conv_epilogue's.
template <int WM, int WN, bool RP>
__device__ __forceinline__ void conv_epilogue_direct(const ConvArgs & A, const v4f (&acc)[WM][WN], int ch0, int t0,
                                                     int phase, int lane) {
    const int lm = lane & 15, lk = lane >> 4;
    const uint32_t ost = (uint32_t) A.ostride, ph = (uint32_t) phase;
    // RP: every residual quad of the wave's tiles is loaded before any is used
    constexpr bool ALLR = RP && WM * WN <= 8;
    float4 rq[ALLR ? WM : 1][ALLR ? WN : 1];
    if (ALLR) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int n0 = ch0 + i * 16 + 4 * lk, t = t0 + j * 16 + lm;
                rq[ALLR ? i : 0][ALLR ? j : 0] =
                    n0 < A.N && t < A.M
                        ? *(const float4 *) (A.res + ((uint32_t) t * ost + ph) * (uint32_t) A.rs + (uint32_t) n0)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
            }
    }
#pragma unroll
    for (int i = 0; i < WM; ++i) {
        const int n0 = ch0 + i * 16 + 4 * lk;
        if (n0 >= A.N) continue;
        const float4 b4 = A.bias ? *(const float4 *) (A.bias + n0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 s4 = A.scale ? *(const float4 *) (A.scale + n0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const bool sn = A.act == ACT_SNAKE;
        const float4 a4 = sn ? *(const float4 *) (A.ea + n0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 e4 = sn ? *(const float4 *) (A.eb + n0) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float bb[4] = {b4.x, b4.y, b4.z, b4.w}, ss[4] = {s4.x, s4.y, s4.z, s4.w};
        const float aa[4] = {a4.x, a4.y, a4.z, a4.w}, ee[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int t = t0 + j * 16 + lm;
            if (t >= A.M) continue;
            const uint32_t row = (uint32_t) t * ost + ph;
            float4 r4 = make_float4(0.f, 0.f, 0.f, 0.f);
            if (ALLR) r4 = rq[ALLR ? i : 0][ALLR ? j : 0];
            else if (A.res) r4 = *(const float4 *) (A.res + row * (uint32_t) A.rs + (uint32_t) n0);
            const float rr[4] = {r4.x, r4.y, r4.z, r4.w};
            float v[4];
            uint16_t h[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float x = acc[i][j][e];
                if (A.bias) x = x + bb[e];
                if (A.scale) x = x * ss[e];
                if (A.res) x = rr[e] + x;
                v[e] = x;
                float y = x;
                if (sn) y = snake(x, aa[e], ee[e]);
                else if (A.act == ACT_GELU) y = gelu_tanh(x);
                h[e] = f2h(y);
            }
            if (A.yf) *(float4 *) (A.yf + row * (uint32_t) A.yfs + (uint32_t) n0) = make_float4(v[0], v[1], v[2], v[3]);
            if (A.yh)
                *(uint2 *) (A.yh + row * (uint32_t) A.yhs + (uint32_t) n0) =
                    make_uint2((uint32_t) h[0] | ((uint32_t) h[1] << 16), (uint32_t) h[2] | ((uint32_t) h[3] << 16));
        }
    }
}

// FU (a whole residual unit, x + conv1(snake2(conv7(snake1(x))))): the
// workgroup's tile holds every channel of its rows (32 WM = N, one channel
// tile), so after the k7 loop it rounds snake2(acc + bias) to fp16 into LDS
// in the layout of a stage's activation rows, runs the 1-tap conv on it with
// the weight fragments read straight from memory (N x N fp16, cache-resident),
// and finishes with the direct epilogue: the intermediate tensor is neither
// written nor read back, and the arithmetic is that of the two launches.
template <int WM, int WN, int KS = 1, bool RP = false, bool FU = false>
__global__ __launch_bounds__(kGemmT) void k_conv_gemm(const ConvArgs A) {
    using G = GemmTile<WM, WN, KS>;
    __shared__ __align__(16) char smem[G::LDS];
    uint16_t * lds = (uint16_t *) smem;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wc = wave & 1, wt = wave >> 1;
    const int lm = lane & 15, lk = lane >> 4;
    const int phase = blockIdx.z;
    const int cb0 = blockIdx.x * G::BC, tb0 = blockIdx.y * G::BT;
    const int CB = A.Cp >> 5, NCH = A.KT * CB, S = (NCH + KS - 1) / KS;
    const uint32_t wrow = (uint32_t) A.KT * (uint32_t) A.Cp * 2u, xrow = (uint32_t) A.xs * 2u;
    const __amdgpu_buffer_rsrc_t wr = rsrc(A.w + (size_t) phase * A.Np * A.KT * A.Cp, (uint32_t) A.Np * wrow);
    const __amdgpu_buffer_rsrc_t xr = rsrc(A.x, (uint32_t) A.rows_in * xrow);

    // this thread's 16-byte pieces of the A (weights) and B (activations) tiles
    uint32_t wo[G::NA];
    int la[G::NA];
    bool oa[G::NA];
#pragma unroll
    for (int r = 0; r < G::NA; ++r) {
        const int c = tid + r * kGemmT, row = c >> 2, col = c & 3;
        oa[r] = c < G::BC * 4;
        wo[r] = (uint32_t) (cb0 + (oa[r] ? row : 0)) * wrow + col * 16;
        la[r] = swz(row, col);
    }
    int tb[G::NB], lb[G::NB];
    uint32_t xo[G::NB];
    bool ob[G::NB];
#pragma unroll
    for (int r = 0; r < G::NB; ++r) {
        const int c = tid + r * kGemmT, row = c >> 2, col = c & 3;
        ob[r] = c < G::BT * 4;
        const int t = tb0 + row;
        tb[r] = (ob[r] && t < A.M) ? t + A.off0 : -(1 << 30);
        xo[r] = col * 16;
        lb[r] = G::BC * 32 + swz(row, col);
    }
    struct Stage {
        uint4 a[KS][G::NA], b[KS][G::NB];
    };
    // fetches run in chunk order, so a cursor (tap, channel offset) replaces
    // a division per chunk; chunk ch's weights start at byte 64 ch of a row
    int f_ch = 0, f_tap = 0, f_cc = 0;
    auto fetch = [&](int s, Stage & R) {
        (void) s;
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            const int tap = f_tap, cc = f_cc;
            const bool in = f_ch < NCH;
            const uint32_t wk = in ? (uint32_t) f_ch * 64u : kOut;
            f_ch += 1;
            f_cc += 32;
            if (f_cc == A.Cp) {
                f_cc = 0;
                f_tap += 1;
            }
#pragma unroll
            for (int r = 0; r < G::NA; ++r) R.a[q][r] = bload(wr, wo[r] + wk);
#pragma unroll
            for (int r = 0; r < G::NB; ++r) {
                const int src = tb[r] + tap * A.dil;
                const bool ok = in && (unsigned) src < (unsigned) A.rows_in;
                R.b[q][r] = bload(xr, ok ? (uint32_t) src * xrow + (uint32_t) cc * 2u + xo[r] : kOut);
            }
        }
    };
    auto stash = [&](int buf, const Stage & R) {
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            uint16_t * st = lds + buf * G::STAGE + q * G::SUB;
#pragma unroll
            for (int r = 0; r < G::NA; ++r)
                if (oa[r]) *(uint4 *) (st + la[r]) = R.a[q][r];
#pragma unroll
            for (int r = 0; r < G::NB; ++r)
                if (ob[r]) *(uint4 *) (st + lb[r]) = R.b[q][r];
        }
    };

    v4f acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf) {
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            const uint16_t * st = lds + buf * G::STAGE + q * G::SUB;
            v8h af[WM], bf[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) af[i] = *(const v8h *) (st + swz(wc * WM * 16 + i * 16 + lm, lk));
#pragma unroll
            for (int j = 0; j < WN; ++j) bf[j] = *(const v8h *) (st + G::BC * 32 + swz(wt * WN * 16 + j * 16 + lm, lk));
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };

    // two register stages: Ra holds the even steps, Rb the odd ones.  The
    // fetches and stores of steps past the end are not skipped (their loads
    // are out of range and return zeros, into buffers no step reads): a
    // branch around a load would cost the compiler's wait counts their
    // precision, and a wait for the newest loads undoes the prefetch.
    // An odd step count runs one more step of zeros (S2 even), so the loop
    // body has no exit between its two halves.
    Stage Ra, Rb;
    const int S2 = S + (S & 1);
    fetch(0, Ra);
    fetch(1, Rb);
    stash(0, Ra);
    __syncthreads();
    for (int s = 0; s < S2; s += 2) {
        fetch(s + 2, Ra);
        compute(0);
        stash(1, Rb);
        __syncthreads();
        fetch(s + 3, Rb);
        compute(1);
        stash(0, Ra);
        __syncthreads();
    }
    if constexpr (FU) {
        static_assert(G::BC * G::BT <= G::LDS / 2, "the intermediate tile fits the stage buffers");
        // the k7 outputs: lane (lm, lk) of tile (i, j) holds channels
        // 16 (WM wc + i) + 4 lk .. + 3 of local row 16 (WN wt + j) + lm, half
        // of a 16-byte piece of that row in chunk n0 / 32
        uint16_t * mid = lds;                       // [N / 32][BT][32], swizzled rows
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int n0 = wc * WM * 16 + i * 16 + 4 * lk;
            const float4 b4 = A.bias ? *(const float4 *) (A.bias + n0) : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 a4 = *(const float4 *) (A.ea + n0), e4 = *(const float4 *) (A.eb + n0);
            const float bb[4] = {b4.x, b4.y, b4.z, b4.w}, aa[4] = {a4.x, a4.y, a4.z, a4.w};
            const float ee[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int rl = wt * WN * 16 + j * 16 + lm;
                uint16_t h[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float x = acc[i][j][e];
                    if (A.bias) x = x + bb[e];
                    h[e] = f2h(snake(x, aa[e], ee[e]));
                }
                *(uint2 *) (mid + (n0 >> 5) * G::BT * 32 + swz(rl, (n0 & 31) >> 3) + (n0 & 7)) =
                    make_uint2((uint32_t) h[0] | ((uint32_t) h[1] << 16), (uint32_t) h[2] | ((uint32_t) h[3] << 16));
            }
        }
        __syncthreads();
        // the 1-tap conv over the tile, chunk by chunk in order
        v4f acc2[WM][WN];
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j) acc2[i][j] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q = 0; q < WM; ++q) {              // N / 32 = WM chunks
            v8h af[WM], bf[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i)
                af[i] = *(const v8h *) (A.w2 + (size_t) (wc * WM * 16 + i * 16 + lm) * (WM * 32) + q * 32 + 8 * lk);
#pragma unroll
            for (int j = 0; j < WN; ++j) bf[j] = *(const v8h *) (mid + q * G::BT * 32 + swz(wt * WN * 16 + j * 16 + lm, lk));
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc2[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc2[i][j], 0, 0, 0);
        }
        ConvArgs B = A;
        B.bias = A.bias2;
        B.scale = nullptr;
        B.act = A.act2;
        B.ea = A.ea2;
        B.eb = A.eb2;
        conv_epilogue_direct<WM, WN, true>(B, acc2, wc * WM * 16, tb0 + wt * WN * 16, phase, lane);
        return;
    }
    if (A.act != ACT_SWIGLU && ((A.N | A.rs | A.yfs | A.yhs) & 3) == 0)
        conv_epilogue_direct<WM, WN, RP>(A, acc, cb0 + wc * WM * 16, tb0 + wt * WN * 16, phase, lane);
    else
        conv_epilogue<WM, WN, RP>(A, acc, (float *) smem + wave * 16 * G::TS, cb0 + wc * WM * 16, tb0 + wt * WN * 16,
                                  phase, lane);
}

// yh[t][c] = fp16(act(x[t][c])) for c < C (the input of a stage whose
// producer is not a fused epilogue: the stage runner, or fp32 rows).
__global__ void k_prep(const float * __restrict__ x, int32_t xs, int32_t T, int32_t C, int32_t act,
                       const float * __restrict__ ea, const float * __restrict__ eb, uint16_t * __restrict__ yh,
                       int32_t yhs) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t) T * C) return;
    const int t = (int) (i / C), c = (int) (i - (int64_t) t * C);
    float v = x[(size_t) t * xs + c];
    if (act == ACT_SNAKE) v = snake(v, ea[c], eb[c]);
    else if (act == ACT_GELU) v = gelu_tanh(v);
    yh[(size_t) t * yhs + c] = f2h(v);
}

// VQ (src/audio_tokenizer_decoder.cpp:663-727): lat[f][d] = tab_0[code_0][d]
// + ((tab_1[code_1][d] + tab_2[code_2][d]) + ...), tab_q = the codebook's
// normalised rows through its output projection (built at finalize).  A code
// outside [0, size) raises *bad and reads row 0.  Workgroup (f, y) takes
// elements y * blockDim.x + i (stride blockDim.x * gridDim.y) of frame f.
__global__ void k_vq_sum(const int32_t * __restrict__ codes, int32_t n_cb, int32_t n, const float * __restrict__ tab,
                         int32_t size, int32_t hidden, float * __restrict__ latf, int32_t lfs,
                         uint16_t * __restrict__ lath, int32_t lhs, int32_t * __restrict__ bad) {
    const int f = blockIdx.x;
    const int32_t * cf = codes + (size_t) f * n_cb;
    // up to 16 codebooks: every table load of an element is issued before the
    // sum, which keeps its order
    constexpr int QM = 16;
    for (int d = blockIdx.y * blockDim.x + threadIdx.x; d < hidden; d += blockDim.x * gridDim.y) {
        float r = 0.0f, first = 0.0f;
        if (n_cb <= QM) {
            float tv[QM];
#pragma unroll
            for (int q = 0; q < QM; ++q) {
                if (q >= n_cb) break;
                int code = cf[q];
                if (code < 0 || code >= size) {
                    if (d == 0) atomicOr(bad, 1);
                    code = 0;
                }
                tv[q] = tab[((size_t) q * size + code) * hidden + d];
            }
#pragma unroll
            for (int q = 0; q < QM; ++q) {
                if (q >= n_cb) break;
                if (q == 0) first = tv[q];
                else if (q == 1) r = tv[q];
                else r = r + tv[q];
            }
        } else {
            for (int q = 0; q < n_cb; ++q) {
                int code = cf[q];
                if (code < 0 || code >= size) {
                    if (d == 0) atomicOr(bad, 1);
                    code = 0;
                }
                const float v = tab[((size_t) q * size + code) * hidden + d];
                if (q == 0) first = v;
                else if (q == 1) r = v;
                else r = r + v;
            }
        }
        const float y = first + r;
        latf[(size_t) f * lfs + d] = y;
        lath[(size_t) f * lhs + d] = f2h(y);
    }
}

// RMSNorm rows (eps, weight) -> fp16: sum of fp32 squares in fp64,
// y = (x * (1 / sqrtf(mean + eps))) * w.  One wave per row.
__global__ void k_rms_h(const float * __restrict__ x, int32_t xs, int32_t T, int32_t C, const float * __restrict__ w,
                        float eps, uint16_t * __restrict__ y, int32_t ys) {
    const int t = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (t >= T) return;
    const float * r = x + (size_t) t * xs;
    // up to 512 channels: all of a lane's loads are issued before its sum,
    // which keeps its order (the terms past C add exact zeros)
    constexpr int RV = 8;
    if (C <= 64 * RV) {
        float xv[RV], wv[RV];
#pragma unroll
        for (int k = 0; k < RV; ++k) {
            const int c = lane + 64 * k;
            xv[k] = c < C ? r[c] : 0.0f;
            wv[k] = c < C ? w[c] : 0.0f;
        }
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < RV; ++k) s += (double) (xv[k] * xv[k]);
        for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
        const float mean = (float) (s / (double) C);
        const float sc = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int k = 0; k < RV; ++k) {
            const int c = lane + 64 * k;
            if (c >= C) break;
            const float v = xv[k] * sc;
            y[(size_t) t * ys + c] = f2h(v * wv[k]);
        }
        return;
    }
    double s = 0.0;
    for (int c = lane; c < C; c += 64) s += (double) (r[c] * r[c]);
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    const float mean = (float) (s / (double) C);
    const float sc = 1.0f / sqrtf(mean + eps);
    for (int c = lane; c < C; c += 64) {
        const float v = r[c] * sc;
        y[(size_t) t * ys + c] = f2h(v * w[c]);
    }
}

// NEOX RoPE in place on the q and k parts of qkv rows [t][3L] (q: [0, L),
// k: [L, 2L)), positions pos0 + t, table rows [pos][hd/2].
__global__ void k_rope_qk(float * __restrict__ qkv, int32_t qs, int32_t T, int32_t L, int32_t hd,
                          const float * __restrict__ cs, const float * __restrict__ sn, int32_t pos0) {
    const int half = hd >> 1;
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int per_row = 2 * (L / hd) * half;           // (q, k) x heads x pairs
    if (i >= (int64_t) T * per_row) return;
    const int t = (int) (i / per_row);
    int r = (int) (i - (int64_t) t * per_row);
    const int part = r / (per_row / 2);
    r -= part * (per_row / 2);
    const int h = r / half, p = r - h * half;
    float * v = qkv + (size_t) t * qs + part * L + h * hd;
    const float c = cs[(size_t) (pos0 + t) * half + p], s = sn[(size_t) (pos0 + t) * half + p];
    const float x0 = v[p], x1 = v[p + half];
    const float a = x0 * c, b = x1 * s, e = x0 * s, f = x1 * c;
    v[p] = a - b;
    v[p + half] = e + f;
}

// Causal F32 attention of one query row (blockIdx.x) and head (blockIdx.y),
// one wave: scores q.k_j (fp64 sums of exact fp32 products, rounded once) *
// scale, softmax with an fp64 denominator, P.V in fp64 -> fp16 row (the
// input of attn_output).  hd <= 64.  Dynamic LDS: T floats.
__global__ __launch_bounds__(64) void k_attn_causal(const float * __restrict__ qkv, int32_t qs, int32_t L, int32_t hd,
                                                    float scale, uint16_t * __restrict__ out, int32_t os) {
    extern __shared__ float p[];
    const int t = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
    const float * q = qkv + (size_t) t * qs + h * hd;
    float mx = -INFINITY;
    for (int j = lane; j <= t; j += 64) {
        const float * k = qkv + (size_t) j * qs + L + h * hd;
        double s = 0.0;
        for (int d = 0; d < hd; ++d) s = fma((double) q[d], (double) k[d], s);
        const float v = (float) s * scale;
        p[j] = v;
        mx = fmaxf(mx, v);
    }
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    double sum = 0.0;
    for (int j = lane; j <= t; j += 64) {
        const float e = expf(p[j] - mx);
        p[j] = e;
        sum += (double) e;
    }
    for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
    const float inv = (float) (1.0 / sum);
    __syncthreads();
    if (lane < hd) {
        double o = 0.0;
        for (int j = 0; j <= t; ++j) o = fma((double) (p[j] * inv), (double) qkv[(size_t) j * qs + 2 * L + h * hd + lane], o);
        out[(size_t) t * os + h * hd + lane] = f2h((float) o);
    }
}

// k_attn_causal for short windows: workgroup (x, h) takes query rows 4x ..
// 4x + 3 of head h, one wave each, with their q rows and the head's K and V
// rows 0 .. 4x + 3 staged in LDS once, and the head width a constant so the
// dot products unroll (the one-wave kernel reads q, K and V from global
// memory inside its dependent fp64 chains).  Every lane computes what it
// computes there, in the same order: scores as sequential fp64 fmas over
// the head dims, the max and fp64 sum over the same lane split and shuffle
// tree, P.V as one dim per lane over the keys in order.  Dynamic LDS:
// (2 T HD + 4 HD + 4 T) floats.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_causal_lds(const float * __restrict__ qkv, int32_t qs, int32_t L, int32_t T,
                                                         float scale, uint16_t * __restrict__ out, int32_t os) {
    extern __shared__ float sm[];
    const int h = blockIdx.y, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int t0 = blockIdx.x * 4, t = t0 + wave;
    const int nrow = min(t0 + 4, T);                  // keys 0 .. nrow - 1 cover every row of the workgroup
    // K transposed ([d][key], stride T), so the lanes of a wave, one key
    // each, read consecutive words; V as rows ([key][d]), read one dim per lane
    float * ks = sm;                                  // [HD][T]
    float * vs = sm + (size_t) T * HD;                // [nrow][HD]
    float * qv = sm + (size_t) 2 * T * HD;            // [4][HD]
    float * p = qv + 4 * HD + (size_t) wave * T;      // [T] per wave
    // 8 elements of K and of V per thread in flight before they are stored
    constexpr int U = 8;
    for (int i0 = threadIdx.x; i0 < nrow * HD; i0 += 256 * U) {
        float kv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + 256 * u, j = i / HD, d = i - j * HD;
            if (i < nrow * HD) {
                kv[u] = qkv[(size_t) j * qs + L + h * HD + d];
                vv[u] = qkv[(size_t) j * qs + 2 * L + h * HD + d];
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int i = i0 + 256 * u, j = i / HD, d = i - j * HD;
            if (i < nrow * HD) {
                ks[(size_t) d * T + j] = kv[u];
                vs[i] = vv[u];
            }
        }
    }
    for (int i = threadIdx.x; i < 4 * HD; i += 256) {
        const int r = t0 + i / HD;
        qv[i] = r < T ? qkv[(size_t) r * qs + h * HD + i % HD] : 0.0f;
    }
    __syncthreads();
    const bool act = t < T;                           // wave-uniform: the last workgroup's spare waves idle
    float inv = 0.0f;
    if (act) {
        const float * q = qv + wave * HD;
        float mx = -INFINITY;
        for (int j = lane; j <= t; j += 64) {
            double s = 0.0;
#pragma unroll
            for (int d = 0; d < HD; ++d) s = fma((double) q[d], (double) ks[(size_t) d * T + j], s);
            const float v = (float) s * scale;
            p[j] = v;
            mx = fmaxf(mx, v);
        }
        for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
        double sum = 0.0;
        for (int j = lane; j <= t; j += 64) {
            const float e = expf(p[j] - mx);
            p[j] = e;
            sum += (double) e;
        }
        for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o);
        inv = (float) (1.0 / sum);
    }
    __syncthreads();
    if (act && lane < HD) {
        double o = 0.0;
        for (int j = 0; j <= t; ++j) o = fma((double) (p[j] * inv), (double) vs[(size_t) j * HD + lane], o);
        out[(size_t) t * os + h * HD + lane] = f2h((float) o);
    }
}

// ConvNeXt front (src/audio_tokenizer_decoder.cpp:515-539): causal depthwise
// k7 over fp16-rounded y, + bias, then LayerNorm over the C channels (eps
// 1e-6, ggml_norm: fp64 mean, centred fp32 values, fp64 variance), * w + b,
// rounded to fp16 for pwconv1.  One workgroup per row; LDS C floats.
__global__ __launch_bounds__(256) void k_dwconv_ln(const float * __restrict__ y, int32_t ys, int32_t T, int32_t C,
                                                   const uint16_t * __restrict__ w, const float * __restrict__ b,
                                                   const float * __restrict__ nw, const float * __restrict__ nb,
                                                   uint16_t * __restrict__ out, int32_t os) {
    extern __shared__ float z[];
    __shared__ double red[4];
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    double s = 0.0;
    for (int c = tid; c < C; c += 256) {
        double acc = 0.0;
        for (int k = 0; k < 7; ++k) {
            const int src = t + k - 6;
            if (src < 0) continue;
            acc += (double) round_f16(y[(size_t) src * ys + c]) * (double) h2f(w[c * 7 + k]);
        }
        const float v = (float) acc + b[c];
        z[c] = v;
        s += (double) v;
    }
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    const float mean = (float) ((red[0] + red[1] + red[2] + red[3]) / (double) C);
    __syncthreads();
    double s2 = 0.0;
    for (int c = tid; c < C; c += 256) {
        const float v = z[c] - mean;
        z[c] = v;
        s2 += (double) (v * v);
    }
    for (int o = 32; o > 0; o >>= 1) s2 += __shfl_xor(s2, o);
    if (lane == 0) red[wave] = s2;
    __syncthreads();
    const float var = (float) ((red[0] + red[1] + red[2] + red[3]) / (double) C);
    const float sc = 1.0f / sqrtf(var + 1e-6f);
    for (int c = tid; c < C; c += 256) {
        float v = z[c] * sc;
        v = v * nw[c];
        out[(size_t) t * os + c] = f2h(v + nb[c]);
    }
}

// k_out_conv with the workgroup's rows staged in LDS: samples t0 .. t0 + 255
// read rows t0 - 6 .. t0 + 255, loaded once and coalesced, stored channel-
// major (xt[c][row]) so that the lanes, one sample each, read consecutive
// halves; the weights as fp64.  Each thread sums taps then channels in the
// order of k_out_conv.  C <= 96.  Static LDS: 96 x 262 halves + 7 x 96
// doubles (55 KB).
constexpr int kOutRows = 256 + 6, kOutMaxC = 96;
__global__ __launch_bounds__(256) void k_out_conv_lds(const uint16_t * __restrict__ x, int32_t xs, int32_t T, int32_t C,
                                                      const uint16_t * __restrict__ w, float bias,
                                                      float * __restrict__ pre, float * __restrict__ out, int64_t drop) {
    __shared__ uint16_t xt[kOutMaxC][kOutRows];
    __shared__ double wd[7][kOutMaxC];
    const int64_t t0 = (int64_t) blockIdx.x * 256;
    for (int i = threadIdx.x; i < C * 7; i += 256) {
        const int c = i / 7, k = i - c * 7;
        wd[k][c] = (double) h2f(w[c * 7 + k]);
    }
    // rows r = 0 .. 261 are samples t0 - 6 + r; eight channels per load
    const int cg = C / 8;
    for (int i = threadIdx.x; i < kOutRows * cg; i += 256) {
        const int r = i / cg, c8 = (i - r * cg) * 8;
        const int64_t src = t0 - 6 + r;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (src >= 0 && src < T) v = *(const uint4 *) (x + src * xs + c8);
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) xt[c8 + e][r] = (uint16_t) (wv[e >> 1] >> (16 * (e & 1)));
    }
    __syncthreads();
    const int64_t t = t0 + threadIdx.x;
    if (t >= T) return;
    double acc = 0.0;
    for (int k = 0; k < 7; ++k) {
        if (t + k - 6 < 0) continue;
        const int r = (int) threadIdx.x + k;
        for (int c = 0; c < C; ++c) acc = fma((double) h2f(xt[c][r]), wd[k][c], acc);
    }
    const float y = (float) acc + bias;
    if (pre) pre[t] = y;
    if (t >= drop) out[t - drop] = tanhf(y);
}

// Output conv (C -> 1, k7, causal) over the fp16 snake'd rows, + bias, tanh.
// pre (optional) keeps the value before tanh; out gets samples t >= drop at
// out[t - drop].  One thread per sample; C % 8 == 0.
__global__ void k_out_conv(const uint16_t * __restrict__ x, int32_t xs, int32_t T, int32_t C,
                           const uint16_t * __restrict__ w, float bias, float * __restrict__ pre,
                           float * __restrict__ out, int64_t drop) {
    const int64_t t = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    double acc = 0.0;
    for (int k = 0; k < 7; ++k) {
        const int64_t src = t + k - 6;
        if (src < 0) continue;
        const uint16_t * r = x + src * xs;
        for (int c = 0; c < C; c += 8) {
            const v8h v = *(const v8h *) (r + c);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc = fma((double) (float) v[e], (double) h2f(w[(c + e) * 7 + k]), acc);
        }
    }
    const float y = (float) acc + bias;
    if (pre) pre[t] = y;
    if (t >= drop) out[t - drop] = tanhf(y);
}

}  // namespace voc
}  // namespace q3t
