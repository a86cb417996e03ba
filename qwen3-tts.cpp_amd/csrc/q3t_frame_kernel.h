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
//   - the phase input is prepared once per workgroup: all 256 threads load
//     it, apply the RMSNorm and quantise it to Q8_0 (or round it to fp16 for
//     the F16 heads) into LDS; the GEMV lanes then only run dot products;
//   - workgroup g (< n_kv_head) owns KV head g for attention; the code
//     predictor's 16-position KV cache lives in that workgroup's LDS for the
//     whole frame;
//   - samplers run redundantly in every workgroup that needs the token (all
//     compute the same token from the same tagged logits); workgroup 0
//     alone writes the frame state and the emitted codes;
//   - every wait is bounded: a timeout marks the thread dead (it never waits
//     again), sets an error flag the host reads after the frame, so a bug
//     cannot hang the GPU.
// The model dimensions are template parameters (hidden D, query width QD =
// 2 x KV width, FFN width FF), so every loop over an activation is unrolled
// into registers.  Numerics are those of the multi-kernel path
// (q3t_gemv_reg.h, k_attention, sample_core): fp64 accumulation of exact
// terms, identical rounding points.
#pragma once

#include "q3t_kernels.h"

namespace q3t {
namespace fk {

constexpr int kT = 256;                 // threads per workgroup
constexpr int kW = kT / 64;             // waves per workgroup
constexpr int kSlot = 8192;             // tagged elements per phase slot
constexpr int kHS = kSlot / 2;          // per-token stride inside a slot
constexpr int kMaxCtx = 4096;           // talker positions the attention phase can hold in LDS
constexpr unsigned kSpin = 1u << 20;    // polls before a wait gives up
constexpr int kCpLayers = 5;            // code-predictor layers whose KV fits in LDS
constexpr int kMaxBlk = 96;             // Q8_0 blocks of the widest GEMV input (3072)

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
    int32_t kv_bf16;                         // talker cache of bfloat16 values (else fp16)
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
    float * cand_val; int32_t * cand_idx;    // talker-head greedy candidates, one per workgroup
    const float * step_in;                   // MODE_TALKER_STEP: the step embedding [D]
    // XCD-parallel program: code-predictor layer 0's QKV rows of every
    // (codebook step s, code), [15][cp_vocab][4096] (null: computed)
    const float * cp_qkv0;
    // 1.7B layout: code_pred.mtp_proj (talker width -> code-predictor width) and its bias
    const int8_t * mtp_w; const uint16_t * mtp_d; const float * mtp_b;
};

// What one launch runs: a whole frame, or one of its two halves alone (the
// reference's separate forward_step and predict_codes_autoregressive calls).
enum : int32_t {
    MODE_FRAME = 0,          // codebook-0 sample, code predictor, talker step; frame state advanced
    MODE_TALKER_STEP = 1,    // talker step on step_in at st->talker_pos -> logits, hidden
    MODE_CODE_PRED = 2,      // code predictor on hidden and st->codes[0] -> st->codes[1..15]
};

// Geometry of a Q8_0 GEMV with input width K: each row is split over LPR
// lanes holding SLOTS blocks each; a wave covers RPW rows ("row group").
template <int K>
struct Geo {
    static constexpr int BPR = K / kQK;
    static constexpr int SLOTS = BPR > 32 ? BPR / 32 : 1;
    static constexpr int LPR = BPR / SLOTS;
    static constexpr int RPW = 64 / LPR;
    static constexpr int G4 = K / 4;                   // groups of 4 consecutive input elements
    static constexpr int CHG = (G4 + kT - 1) / kT;     // groups per thread per token
    static_assert(BPR % SLOTS == 0 && (LPR & (LPR - 1)) == 0 && LPR >= 4 && LPR <= 32 && G4 % 64 == 0,
                  "unsupported GEMV width");
};

// Row groups per wave that a GEMV phase of `rows` rows of input width K needs
// on the 1,024 waves of a 256-workgroup launch; its register sets hold that
// many (the host admits a launch only when its waves cover the rows with it).
template <int K>
constexpr int ngroups(int rows) {
    return (rows / Geo<K>::RPW + 1023) / 1024 < 1 ? 1 : (rows / Geo<K>::RPW + 1023) / 1024;
}

// Thread t's share of NT input rows of width K: groups g = t + c * kT of 4
// consecutive elements (4g .. 4g+3); 8 consecutive threads cover one Q8_0
// block.  Groups with g >= K/4 belong to whole idle waves (K/4 % 64 == 0).
template <int K>
constexpr int kChg = (K / 4 + kT - 1) / kT;        // groups of 4 per thread for width K
template <int NT, int K>
using RowsT = float[NT][kChg<K>][4];
template <int K>
using NormT = float[kChg<K>][4];

struct Lds {
    alignas(16) float x[4096];                  // gathered layer-0 rows [nt][D] / sampler logits
    alignas(16) int8_t qlo[2 * kMaxBlk * 16];   // Q8 input: bytes 0..15 of block b of token t at (t*BPR+b)*16
    alignas(16) int8_t qhi[2 * kMaxBlk * 16];   // bytes 16..31
    float qdx[2 * kMaxBlk];                     // fp16-rounded block scales
    alignas(16) uint16_t hq[4][64 * 8];         // F16 head input: halves 8c..8c+7 of block b at hq[c][b*8]
    float a[2 * 4 * 128];                       // attention: q (2 tok x 2 heads), new k, new v rows
    union {                                     // attention and F16 GEMV inputs are never live together
        alignas(16) float sc[2 * kMaxCtx];      // attention scores / probabilities, 2 heads; P.V partials
        alignas(16) uint16_t hf[2][4][kMaxBlk * 8];   // F16 GEMV input: halves 8c..8c+7 of block b at hf[t][c][b*8]
        alignas(16) float xw[2][8][kMaxBlk * 4];      // widened F16 GEMV input: fp32 4c..4c+3 of block b at xw[t][c][b*4]
    };
    alignas(16) uint16_t cpk[kCpLayers][16 * 128];   // code-predictor KV of this workgroup's KV head
    alignas(16) uint16_t cpv[kCpLayers][16 * 128];
    alignas(16) float att[2][256];              // XCD-parallel layers: this XCD's head-pair attention rows
    float rx[2][32];                            // XCD-parallel layers: this workgroup's slice of the residual stream
    double red[2 * kW];
    float fred[2 * kW];
    int32_t ired[kW];
    int32_t codes[16];
    SampleScratch<kT> S;
};

// ------------------------------------------------------ global accessors
// Every pointer comes from the argument block, so the compiler cannot prove
// its address space and would emit flat accesses, which also count against
// the LDS wait counter: an LDS wait would then stall on weight prefetches in
// flight.  These accessors address the global space explicitly.
#define Q3T_GAS __attribute__((address_space(1)))
typedef int gvi4 __attribute__((ext_vector_type(4)));
typedef float gvf4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ int4 gld4(const void * p) {
    const gvi4 v = *(const Q3T_GAS gvi4 *) p;
    return make_int4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float4 gldf4(const float * p) {
    const gvf4 v = *(const Q3T_GAS gvf4 *) p;
    return make_float4(v.x, v.y, v.z, v.w);
}
template <class T>
__device__ __forceinline__ T gld(const T * p) { return *(const Q3T_GAS T *) p; }
// Non-temporal variants (NTL) for the talker weights, read once per frame:
// they then leave the memory-side cache to the code predictor's weights,
// which every pass of the next frame re-reads.  NTL must be a constant (a
// runtime choice between the two forms folds into one plain load).
template <bool NTL>
__device__ __forceinline__ int4 gld4n(const void * p) {
    gvi4 v;
    if constexpr (NTL) v = __builtin_nontemporal_load((const Q3T_GAS gvi4 *) p);
    else v = *(const Q3T_GAS gvi4 *) p;
    return make_int4(v.x, v.y, v.z, v.w);
}
template <bool NTL, class T>
__device__ __forceinline__ T gldn(const T * p) {
    if constexpr (NTL) return __builtin_nontemporal_load((const Q3T_GAS T *) p);
    else return *(const Q3T_GAS T *) p;
}
template <class T>
__device__ __forceinline__ void gst(T * p, T v) { *(Q3T_GAS T *) p = v; }

// A layer descriptor read through the constant address space, one field at a
// time (an aggregate copy would lose the address space): the kernel never
// writes the descriptors, so the pointers arrive by scalar loads and the
// accesses through them are global ones.
template <class T>
__device__ __forceinline__ T cld(const T * p) { return *(const __attribute__((address_space(4))) T *) p; }
__device__ __forceinline__ LayerQ8 layer_desc(const LayerQ8 * p) {
    return LayerQ8{cld(&p->qkv), cld(&p->qkv_d), cld(&p->wo), cld(&p->wo_d), cld(&p->wg), cld(&p->wg_d),
                   cld(&p->wu), cld(&p->wu_d), cld(&p->wd), cld(&p->wd_d), cld(&p->attn_norm), cld(&p->ffn_norm),
                   cld(&p->q_norm), cld(&p->k_norm)};
}

// ---------------------------------------------------------------- tagged I/O
__device__ __forceinline__ uint64_t tload(const uint64_t * p) {
    return __hip_atomic_load((const Q3T_GAS uint64_t *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void tstore(uint64_t * p, uint32_t tag, float v) {
    __hip_atomic_store((Q3T_GAS uint64_t *) p, ((uint64_t) tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
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

// XCD-local tagged I/O.  The hardware deals the workgroups of a launch to
// the eight XCDs round-robin: workgroup b runs on XCD (b + r) % 8 for a
// rotation r that can differ between launches (the host checks the
// round-robin form before it selects a kernel that relies on it), so the
// workgroups with equal b % 8 always share an XCD, and the eight XCDs have
// separate L2 caches.  Data exchanged only among the workgroups of one
// XCD goes through that XCD's L2: a plain 64-bit store (wavefront scope),
// polled with a load that skips the CU's L1 (system scope: sc0 sc1), at
// about 0.7 us per hand-off against 1.1-1.9 us for the device-scope form.
// A region written this way is only ever written and read by the workgroups
// of one b % 8 class within a launch, and never shares a cache line with
// another class's region.  Were the dealing not round-robin, a reader on
// another XCD would not see the writer's L2 line and its wait would time out
// (error 1): never a stale value, since every tag is unique.
__device__ __forceinline__ uint64_t lload(const uint64_t * p) {
    return __hip_atomic_load((const Q3T_GAS uint64_t *) p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void lstore(uint64_t * p, uint32_t tag, float v) {
    __hip_atomic_store((Q3T_GAS uint64_t *) p, ((uint64_t) tag << 32) | __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WAVEFRONT);
}
// XL: XCD-local (lload / lstore) or device-wide (tload / tstore).
template <bool XL>
__device__ __forceinline__ uint64_t xload(const uint64_t * p) { return XL ? lload(p) : tload(p); }
template <bool XL>
__device__ __forceinline__ void xstore(uint64_t * p, uint32_t tag, float v) {
    if (XL) lstore(p, tag, v);
    else tstore(p, tag, v);
}
template <bool XL>
__device__ __forceinline__ float xwait(const uint64_t * p, uint32_t tag, bool & dead, int32_t * err) {
    uint64_t v = xload<XL>(p);
    unsigned n = 0;
    while ((uint32_t) (v >> 32) != tag && !dead) {
        if (++n > kSpin) { dead = true; atomicExch(err, 1); break; }
        __builtin_amdgcn_s_sleep(1);
        v = xload<XL>(p);
    }
    return __uint_as_float((uint32_t) v);
}

// Waits for up to kB tagged elements at once: all loads are issued before
// any tag is checked, and a re-poll reloads only the elements still missing,
// so a thread pays about one round trip per batch instead of one per element.
constexpr int kB = 8;
template <int N, bool XL = false>
__device__ __forceinline__ void twait_batch(const uint64_t * const (&ptr)[N], int cnt, uint32_t tag, float (&out)[N],
                                            bool & dead, int32_t * err) {
    uint64_t v[N];
    unsigned n = 0;
#pragma unroll
    for (int k = 0; k < N; ++k) v[k] = k < cnt ? xload<XL>(ptr[k]) : ((uint64_t) tag << 32);
    while (!dead) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < N; ++k) all = all && (uint32_t) (v[k] >> 32) == tag;
        if (all) break;
        if (++n > kSpin) { dead = true; atomicExch(err, 1); break; }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < N; ++k)
            if ((uint32_t) (v[k] >> 32) != tag) v[k] = xload<XL>(ptr[k]);
    }
#pragma unroll
    for (int k = 0; k < N; ++k) out[k] = __uint_as_float((uint32_t) v[k]);
}

// Thread t's groups of rows [NT][K] of a tagged slot (row stride ts), in
// batches of up to 12 loads ordered group-major, so the valid loads of a
// thread always form a prefix of each batch.  XL: an XCD-local slot.
template <int NT, int K, bool XL = false>
__device__ __forceinline__ void load_tagged(const uint64_t * slot, uint32_t tag, RowsT<NT, K> & v, bool & dead,
                                            int32_t * err, int ts = kHS) {
    constexpr int CHG = kChg<K>, G4 = K / 4, F = CHG * NT * 4;
    constexpr int NB = F <= 12 ? F : (F % 12 == 0 ? 12 : 8);
    static_assert(F % NB == 0, "batch split");
#pragma unroll
    for (int f0 = 0; f0 < F; f0 += NB) {
        const uint64_t * ptr[NB];
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int f = f0 + k, c = f / (NT * 4), tok = (f / 4) % NT, e = f % 4;
            const int g = (int) threadIdx.x + kT * c;
            const bool ok = g < G4;
            ptr[k] = slot + (size_t) tok * ts + (ok ? 4 * g + e : 0);
            if (ok) cnt = k + 1;
        }
        float val[NB];
        twait_batch<NB, XL>(ptr, cnt, tag, val, dead, err);
#pragma unroll
        for (int k = 0; k < NB; ++k) {
            const int f = f0 + k, c = f / (NT * 4), tok = (f / 4) % NT, e = f % 4;
            v[tok][c][e] = val[k];
        }
    }
}

// The same groups from plain LDS rows x [NT][K].
template <int NT, int K>
__device__ __forceinline__ void load_lds(const float * x, RowsT<NT, K> & v, int ts = K) {
    constexpr int CHG = kChg<K>, G4 = K / 4;
#pragma unroll
    for (int c = 0; c < CHG; ++c) {
        const int g = (int) threadIdx.x + kT * c;
        if (g >= G4) break;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float4 q = *(const float4 *) (x + t * ts + 4 * g);
            v[t][c][0] = q.x; v[t][c][1] = q.y; v[t][c][2] = q.z; v[t][c][3] = q.w;
        }
    }
}

// ------------------------------------------------------ cross-lane helpers

// ------------------------------------------------------- input preparation
// RMSNorm of thread-distributed rows v[NT][K/kT]: y = (x * scale) * w with
// scale = 1/sqrt(mean(fl(x*x)) + eps), the sum of squares accumulated in
// fp64.  Every thread ends with its normed elements.
// The norm weights of this thread's groups, loaded before the phase input
// is awaited.
template <int K>
__device__ __forceinline__ void norm_prefetch(const float * w, NormT<K> & nw) {
#pragma unroll
    for (int c = 0; c < Geo<K>::CHG; ++c) {
        const int g = (int) threadIdx.x + kT * c;
        if (g >= Geo<K>::G4) break;
        const float4 q = gldf4(w + 4 * g);
        nw[c][0] = q.x; nw[c][1] = q.y; nw[c][2] = q.z; nw[c][3] = q.w;
    }
}

// RMSNorm of thread-distributed rows: y = (x * scale) * w with scale =
// 1/sqrt(mean(fl(x*x)) + eps), the sum of squares accumulated in fp64.
// Every thread ends with its normed elements.
template <int NT, int K>
__device__ __forceinline__ void rms_rows(RowsT<NT, K> & v, const NormT<K> & nw, float eps, Lds & L) {
    constexpr int CHG = Geo<K>::CHG, G4 = Geo<K>::G4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        double ss = 0.0;
#pragma unroll
        for (int c = 0; c < CHG; ++c)
            if ((int) threadIdx.x + kT * c < G4)
#pragma unroll
                for (int e = 0; e < 4; ++e) ss += (double) (v[t][c][e] * v[t][c][e]);
        ss = wave_sum_d(ss);
        if (lane == 0) L.red[t * kW + wave] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        double tot = L.red[t * kW];
#pragma unroll
        for (int w2 = 1; w2 < kW; ++w2) tot += L.red[t * kW + w2];
        const float mean = (float) (tot / (double) K);
        const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int c = 0; c < CHG; ++c)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float y = v[t][c][e] * scale;
                v[t][c][e] = y * nw[c][e];
            }
    }
}

// Q8_0 activation quantisation (ggml-cpu x86 quantize_row_q8_0: d =
// amax/127 stored as fp16, q = round-to-nearest-even(x * 127/amax)) of
// thread-distributed rows into LDS.  A block is 8 consecutive threads of 4
// elements, so its amax is a 3-step DPP reduction and the two divisions are
// shared by 4 elements.
template <int NT, int K>
__device__ __forceinline__ void quant_rows(const RowsT<NT, K> & v, Lds & L) {
    constexpr int CHG = kChg<K>, G4 = K / 4, BPR = K / kQK;
    static_assert(K % kQK == 0, "whole Q8_0 blocks");
#pragma unroll
    for (int c = 0; c < CHG; ++c) {
        const int g = (int) threadIdx.x + kT * c;
        if (g >= G4) break;                 // whole 8-lane blocks (K % 32 == 0)
        const int b = g >> 3, eo = (g & 7) * 4;
#pragma unroll
        for (int tok = 0; tok < NT; ++tok) {
            float am = fmaxf(fmaxf(fabsf(v[tok][c][0]), fabsf(v[tok][c][1])), fmaxf(fabsf(v[tok][c][2]), fabsf(v[tok][c][3])));
            am = fmaxf(am, dpp_f<0xB1>(am));
            am = fmaxf(am, dpp_f<0x4E>(am));
            am = fmaxf(am, dpp_f<0x141>(am));
            const float d = am / 127.0f;
            const float id = am != 0.0f ? 127.0f / am : 0.0f;
            int packed = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) packed |= ((int) rintf(v[tok][c][e] * id) & 0xff) << (8 * e);
            int8_t * dst = eo < 16 ? L.qlo : L.qhi;
            *(int *) &dst[(tok * BPR + b) * 16 + (eo & 15)] = packed;
            if ((g & 7) == 0) L.qdx[tok * BPR + b] = round_f16(d);
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------------- GEMV
// Row groups of a GEMV are dealt to the grid's waves: wave gw takes groups
// gw, gw + nwaves, ... (at most NG per wave; the host checks).  NG = 3 only
// for the 1.7B talker's 6144-row gate/up.
template <int K, bool DUAL, int NG = 2>
struct Q8Regs {
    static constexpr int S = Geo<K>::SLOTS;
    int4 w[NG][S][2], u[NG][S][2];
    uint16_t dw[NG][S], du[NG][S];   // fp16 block scales, converted at use so the prefetch never waits
    uint64_t res[NG][2];  // residual elements (tagged) read early by the storing lanes
    int ng;               // groups this wave owns (0..NG)
};

// Row-group owner of wave gw when a phase's groups start at wave `rot`
// (phases that follow a phase with uneven work start where the idle waves are).
__device__ __forceinline__ int rot_wave(int rot) {
    const int nw = gridDim.x * kW;
    const int gw = blockIdx.x * kW + (threadIdx.x >> 6) + nw - rot;
    return gw >= nw ? gw - nw : gw;
}

template <int K, bool DUAL, bool NTL, int NG = 2>
__device__ __forceinline__ void q8_prefetch(Q8Regs<K, DUAL, NG> & R, const int8_t * W, const uint16_t * Wd,
                                            const int8_t * U, const uint16_t * Ud, int rows, int rot) {
    using G = Geo<K>;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int groups = rows / G::RPW;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    R.ng = 0;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const int g = gw + gi * nw;
        if (g >= groups) break;
        R.ng = gi + 1;
        const int r = g * G::RPW + rsub;
#pragma unroll
        for (int s = 0; s < G::SLOTS; ++s) {
            const int b = lir + s * G::LPR;
            const int4 * wp = (const int4 *) (W + (size_t) r * K + b * kQK);
            R.w[gi][s][0] = gld4n<NTL>(wp); R.w[gi][s][1] = gld4n<NTL>(wp + 1);
            R.dw[gi][s] = gldn<NTL>(Wd + (size_t) r * G::BPR + b);
            if (DUAL) {
                const int4 * up = (const int4 *) (U + (size_t) r * K + b * kQK);
                R.u[gi][s][0] = gld4n<NTL>(up); R.u[gi][s][1] = gld4n<NTL>(up + 1);
                R.du[gi][s] = gldn<NTL>(Ud + (size_t) r * G::BPR + b);
            }
        }
    }
}

// Issues the residual loads of the rows this lane will store (EPI_RESID),
// before the phase input is awaited; q8_compute re-polls any not yet tagged.
template <int NT, int K, bool DUAL, int NG = 2>
__device__ __forceinline__ void res_prefetch(Q8Regs<K, DUAL, NG> & R, const uint64_t * res, int rot) {
    using G = Geo<K>;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    if (lir != 0) return;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * G::RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) R.res[gi][t] = tload(res + (size_t) t * kHS + r);
    }
}

// Whether any wave of this workgroup owns a row group.  rot is a multiple of
// kW, so a workgroup's waves stay consecutive in the rotated order and the
// first one owns a group whenever any does.
template <int K>
__device__ __forceinline__ bool wg_has_rows(int rows, int rot) {
    const int nw = gridDim.x * kW;
    int first = (int) blockIdx.x * kW + nw - rot;
    if (first >= nw) first -= nw;
    return first < rows / Geo<K>::RPW;
}

// Q8_0 GEMV over the quantised LDS input, epilogue, tagged stores into
// out [NT][kHS].  res: residual slot (tagged) for EPI_RESID; bias: fp32 per
// row for EPI_BIAS.
template <int NT, int K, bool DUAL, int NG = 2>
__device__ __forceinline__ void q8_compute(const Q8Regs<K, DUAL, NG> & R, const Lds & L, int epi, const uint64_t * res,
                                           uint32_t res_tag, uint64_t * out, uint32_t out_tag, int rot, bool & dead,
                                           int32_t * err, const float * bias = nullptr) {
    using G = Geo<K>;
    if (R.ng == 0) return;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    double acc[NG][NT], acc2[NG][NT];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[gi][t] = 0.0; acc2[gi][t] = 0.0; }
    // the scales enter here: the empty asm keeps their conversion (and the
    // wait for their loads) from being hoisted into the prefetch
    float sw[NG][G::SLOTS], su[NG][G::SLOTS];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
        for (int s = 0; s < G::SLOTS; ++s) {
            uint32_t a = R.dw[gi][s], c = DUAL ? R.du[gi][s] : 0u;
            asm volatile("" : "+v"(a), "+v"(c));
            sw[gi][s] = h2f((uint16_t) a);
            su[gi][s] = h2f((uint16_t) c);
        }
#pragma unroll
    for (int s = 0; s < G::SLOTS; ++s) {
        const int b = lir + s * G::LPR;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int4 x0 = *(const int4 *) &L.qlo[(t * G::BPR + b) * 16];
            const int4 x1 = *(const int4 *) &L.qhi[(t * G::BPR + b) * 16];
            const float dx = L.qdx[t * G::BPR + b];
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
                if (gi >= R.ng) break;
                // d_w * d_x (two fp16 values) is exact in fp32 and its product with
                // the int32 block sum exact in fp64: fma rounds like mul + add
                acc[gi][t] = fma((double) (sw[gi][s] * dx), (double) dot32_i8(R.w[gi][s][0], R.w[gi][s][1], x0, x1),
                                 acc[gi][t]);
                if (DUAL)
                    acc2[gi][t] = fma((double) (su[gi][s] * dx),
                                      (double) dot32_i8(R.u[gi][s][0], R.u[gi][s][1], x0, x1), acc2[gi][t]);
            }
        }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * G::RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double a1 = group_sum_d(acc[gi][t], G::LPR);
            const double a2 = DUAL ? group_sum_d(acc2[gi][t], G::LPR) : 0.0;
            if (lir != 0) continue;
            const float v = (float) a1;
            float o;
            if (epi == EPI_RESID) {
                const uint64_t rv = R.res[gi][t];
                o = v + ((uint32_t) (rv >> 32) == res_tag ? __uint_as_float((uint32_t) rv)
                                                          : twait(res + (size_t) t * kHS + r, res_tag, dead, err));
            } else if (epi == EPI_SWIGLU) {
                o = silu_q3t(v) * (float) a2;
            } else if (epi == EPI_BIAS) {
                o = v + gld(bias + r);
            } else {
                o = v;
            }
            tstore(out + (size_t) t * kHS + r, out_tag, o);
        }
    }
}

// ------------------------------------------------------------- F16 GEMV
// F16 weights (the F16 model's layers): the activation is rounded to fp16
// (or kept fp32 for ffn_down, which the reference widens to F32) and every
// product, exact in fp64, is accumulated in fp64.  Same row geometry as the
// Q8_0 GEMV: a lane holds whole 32-element blocks, 64 bytes each.
template <int K, bool DUAL, int NG = 2>
struct F16Regs {
    static constexpr int S = Geo<K>::SLOTS;
    int4 w[NG][S][4], u[DUAL ? NG : 1][DUAL ? S : 1][4];
    uint64_t res[NG][2];
    int ng;
};

template <int K, bool DUAL, bool NTL, int NG = 2>
__device__ __forceinline__ void f16_prefetch(F16Regs<K, DUAL, NG> & R, const uint16_t * W, const uint16_t * U,
                                             int rows, int rot) {
    using G = Geo<K>;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int groups = rows / G::RPW;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    R.ng = 0;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        const int g = gw + gi * nw;
        if (g >= groups) break;
        R.ng = gi + 1;
        const int r = g * G::RPW + rsub;
#pragma unroll
        for (int s = 0; s < G::SLOTS; ++s) {
            const int b = lir + s * G::LPR;
            const int4 * wp = (const int4 *) (W + (size_t) r * K + b * kQK);
#pragma unroll
            for (int c = 0; c < 4; ++c) R.w[gi][s][c] = gld4n<NTL>(wp + c);
            if (DUAL) {
                const int4 * up = (const int4 *) (U + (size_t) r * K + b * kQK);
#pragma unroll
                for (int c = 0; c < 4; ++c) R.u[DUAL ? gi : 0][DUAL ? s : 0][c] = gld4n<NTL>(up + c);
            }
        }
    }
}

template <int NT, int K, bool DUAL, int NG = 2>
__device__ __forceinline__ void res_prefetch16(F16Regs<K, DUAL, NG> & R, const uint64_t * res, int rot) {
    using G = Geo<K>;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    if (lir != 0) return;
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * G::RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) R.res[gi][t] = tload(res + (size_t) t * kHS + r);
    }
}

// Thread-distributed rows into the F16 GEMV input layout: rounded to fp16
// (WIDE = false) or kept fp32 (WIDE = true).
// The F16 GEMV input rows in LDS, packed by their width K (so one token of
// the 1.7B talker's 6144-wide ffn_down input fits where two 3072-wide rows
// do): fp16 halves 8c..8c+7 of block b of token t at hf_at<K>(t, c, b), the
// widened form's fp32 values 4c..4c+3 at xw_at<K>(t, c, b).
template <int K>
__device__ __forceinline__ uint16_t * hf_at(Lds & L, int t, int c, int b) {
    return &L.hf[0][0][0] + ((t * 4 + c) * (K / kQK) + b) * 8;
}
template <int K>
__device__ __forceinline__ const uint16_t * hf_at(const Lds & L, int t, int c, int b) {
    return &L.hf[0][0][0] + ((t * 4 + c) * (K / kQK) + b) * 8;
}
template <int K>
__device__ __forceinline__ float * xw_at(Lds & L, int t, int c, int b) {
    return &L.xw[0][0][0] + ((t * 8 + c) * (K / kQK) + b) * 4;
}
template <int K>
__device__ __forceinline__ const float * xw_at(const Lds & L, int t, int c, int b) {
    return &L.xw[0][0][0] + ((t * 8 + c) * (K / kQK) + b) * 4;
}

template <int NT, int K, bool WIDE>
__device__ __forceinline__ void f16_rows(const RowsT<NT, K> & v, Lds & L) {
    constexpr int CHG = kChg<K>, G4 = K / 4;
    static_assert(K % kQK == 0, "whole 32-element blocks");
    static_assert(NT * K <= 2 * kMaxBlk * kQK, "F16 GEMV input rows exceed their LDS buffer");
#pragma unroll
    for (int c = 0; c < CHG; ++c) {
        const int g = (int) threadIdx.x + kT * c;
        if (g >= G4) break;
        const int b = g >> 3, e32 = (g & 7) * 4;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (WIDE) {
                *(float4 *) xw_at<K>(L, t, g & 7, b) = make_float4(v[t][c][0], v[t][c][1], v[t][c][2], v[t][c][3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) hf_at<K>(L, t, (e32 + e) >> 3, b)[(e32 + e) & 7] = f2h(v[t][c][e]);
            }
        }
    }
    __syncthreads();
}

// fp16 element j (0..7) of 8 packed in an int4, without taking the register's address
__device__ __forceinline__ float h8(const int4 & v, int j) {
    const int w = (j >> 1) == 0 ? v.x : (j >> 1) == 1 ? v.y : (j >> 1) == 2 ? v.z : v.w;
    return h2f((uint16_t) ((j & 1) ? ((uint32_t) w >> 16) : ((uint32_t) w & 0xffffu)));
}
// The same element as a half value.
__device__ __forceinline__ _Float16 h8h(const int4 & v, int j) {
    const int w = (j >> 1) == 0 ? v.x : (j >> 1) == 1 ? v.y : (j >> 1) == 2 ? v.z : v.w;
    const uint16_t b = (uint16_t) ((j & 1) ? ((uint32_t) w >> 16) : ((uint32_t) w & 0xffffu));
    return __builtin_bit_cast(_Float16, b);
}


template <int NT, int K, bool DUAL, bool WIDE, int NG = 2>
__device__ __forceinline__ void f16_compute(const F16Regs<K, DUAL, NG> & R, const Lds & L, int epi, const uint64_t * res,
                                            uint32_t res_tag, uint64_t * out, uint32_t out_tag, int rot, bool & dead,
                                            int32_t * err, const float * bias = nullptr) {
    using G = Geo<K>;
    if (R.ng == 0) return;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR;
    const int gw = rot_wave(rot), nw = gridDim.x * kW;
    double acc[NG][NT], acc2[NG][NT];
#pragma unroll
    for (int gi = 0; gi < NG; ++gi)
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[gi][t] = 0.0; acc2[gi][t] = 0.0; }
#pragma unroll
    for (int s = 0; s < G::SLOTS; ++s) {
        const int b = lir + s * G::LPR;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // activation elements 8c..8c+7 of block b, every token, kept packed
            // (fp16) or as fp32 until each product is formed
            int4 xp[NT];
            float xa[WIDE ? NT : 1][8];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (WIDE) {
                    const float4 x0 = *(const float4 *) xw_at<K>(L, t, 2 * c, b);
                    const float4 x1 = *(const float4 *) xw_at<K>(L, t, 2 * c + 1, b);
                    float * xr = xa[WIDE ? t : 0];
                    xr[0] = x0.x; xr[1] = x0.y; xr[2] = x0.z; xr[3] = x0.w;
                    xr[4] = x1.x; xr[5] = x1.y; xr[6] = x1.z; xr[7] = x1.w;
                } else {
                    xp[t] = *(const int4 *) hf_at<K>(L, t, c, b);
                }
            }
#pragma unroll
            for (int gi = 0; gi < NG; ++gi) {
                if (gi >= R.ng) break;
                // The packed weights pass through an empty asm here, so their
                // conversions are not hoisted ahead of the input barrier.
                int4 wv = R.w[gi][s][c], uv = R.u[DUAL ? gi : 0][DUAL ? s : 0][c];
                __asm__ volatile("" : "+v"(wv.x), "+v"(wv.y), "+v"(wv.z), "+v"(wv.w));
                if (DUAL) __asm__ volatile("" : "+v"(uv.x), "+v"(uv.y), "+v"(uv.z), "+v"(uv.w));
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float wf = WIDE ? h8(wv, j) : 0.0f, uf = WIDE && DUAL ? h8(uv, j) : 0.0f;
                    const _Float16 wh = h8h(wv, j), uh = DUAL ? h8h(uv, j) : (_Float16) 0.0f;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        if (WIDE) {
                            // fp16 x fp32 is exact in fp64.  It is formed as the fp32 product
                            // plus its fma residual (TwoProduct: exact unless the product is
                            // below 2^-102 and the residual underflows), whose fp64 sum is
                            // exact, then added once.  Fewer live fp64 values than converting
                            // both operands keeps this phase within the register file.
                            const float xf = xa[WIDE ? t : 0][j];
                            const float pr = wf * xf, pe = fmaf(wf, xf, -pr);
                            acc[gi][t] += (double) pr + (double) pe;
                            if (DUAL) {
                                const float qr = uf * xf, qe = fmaf(uf, xf, -qr);
                                acc2[gi][t] += (double) qr + (double) qe;
                            }
                        } else {
                            // fp16 x fp16: exact in fp32
                            const _Float16 xh = h8h(xp[t], j);
                            acc[gi][t] += (double) hmul_exact(wh, xh);
                            if (DUAL) acc2[gi][t] += (double) hmul_exact(uh, xh);
                        }
                    }
                }
            }
            // keep each chunk's loads and conversions next to their use
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int gi = 0; gi < NG; ++gi) {
        if (gi >= R.ng) break;
        const int r = (gw + gi * nw) * G::RPW + rsub;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double a1 = group_sum_d(acc[gi][t], G::LPR);
            const double a2 = DUAL ? group_sum_d(acc2[gi][t], G::LPR) : 0.0;
            if (lir != 0) continue;
            const float v = (float) a1;
            float o;
            if (epi == EPI_RESID) {
                const uint64_t rv = R.res[gi][t];
                o = v + ((uint32_t) (rv >> 32) == res_tag ? __uint_as_float((uint32_t) rv)
                                                          : twait(res + (size_t) t * kHS + r, res_tag, dead, err));
            } else if (epi == EPI_SWIGLU) {
                o = silu_q3t(v) * (float) a2;
            } else if (epi == EPI_BIAS) {
                o = v + gld(bias + r);
            } else {
                o = v;
            }
            tstore(out + (size_t) t * kHS + r, out_tag, o);
        }
    }
}

// ------------------------------------------------------------------ F16 head
// RMSNorm'd input row, rounded to fp16 into LDS (the F16 weight x fp32
// activation contract); workgroup 0 also writes the normed fp32 row to
// hidden_out when given.
template <int K>
__device__ __forceinline__ void head_input(RowsT<1, K> & v, const NormT<K> & nw, float eps, Lds & L,
                                           float * hidden_out) {
    rms_rows<1, K>(v, nw, eps, L);
#pragma unroll
    for (int c = 0; c < Geo<K>::CHG; ++c) {
        const int g = (int) threadIdx.x + kT * c;
        if (g >= Geo<K>::G4) break;
        const int b = g >> 3, e32 = (g & 7) * 4;
        if (hidden_out && blockIdx.x == 0)
            for (int e = 0; e < 4; ++e) gst(hidden_out + 4 * g + e, v[0][c][e]);
#pragma unroll
        for (int e = 0; e < 4; ++e) L.hq[(e32 + e) >> 3][b * 8 + ((e32 + e) & 7)] = f2h(v[0][c][e]);
    }
    __syncthreads();
}

// Codebook-0 logit transforms of the talker sampler (suppression window,
// repetition penalty over the tokens seen so far plus this frame's, EOS
// bias), applied by the head for the next frame's greedy candidate.
struct Cb0Xf {
    int V, eos, tok0;
    float rep, eff;
    const uint8_t * seen;
};

// F16 GEMV (one 32-element block per lane), outputs tagged (code predictor)
// or plain (talker logits).  Every workgroup also publishes its greedy
// candidate: the first maximum over its rows (after the codebook-0
// transforms when xf != nullptr), tagged at cand_tagged[2b], [2b+1] or plain
// in cand_val[b] / cand_idx[b] (neither when both are null).  All threads of
// the workgroup must call it.
// Head geometry: a row is split over LPR lanes holding HS blocks each
// (HS = 2 for the 1.7B talker's 2048-wide rows).
template <int K>
struct HeadGeo {
    static constexpr int BPR = K / kQK;
    static constexpr int LPR = BPR > 32 ? 32 : BPR, HS = BPR / LPR, RPW = 64 / LPR;
    static_assert((LPR & (LPR - 1)) == 0 && BPR % LPR == 0 && HS <= 2, "head width");
};

struct HeadRegs {
    int4 w[2][2][4];      // [row group][block slot][16-byte chunk]
    int ng;
};

// The head rows' weights of this lane, loaded before the head input is awaited.
template <int K, bool NTL>
__device__ __forceinline__ void f16_head_prefetch(const uint16_t * W, int rows, HeadRegs & H) {
    using G = HeadGeo<K>;
    const int lane = threadIdx.x & 63, lir = lane & (G::LPR - 1), rsub = lane / G::LPR, wave = threadIdx.x >> 6;
    const int groups = rows / G::RPW;
    const int gw = blockIdx.x * kW + wave, nw = gridDim.x * kW;
    H.ng = 0;
#pragma unroll
    for (int gi = 0; gi < 2; ++gi) {
        const int g = gw + gi * nw;
        if (g >= groups) break;
        H.ng = gi + 1;
#pragma unroll
        for (int hs = 0; hs < G::HS; ++hs) {
            const int4 * wp = (const int4 *) (W + (size_t) (g * G::RPW + rsub) * K + (lir + hs * G::LPR) * kQK);
#pragma unroll
            for (int c = 0; c < 4; ++c) H.w[gi][hs][c] = gld4n<NTL>(wp + c);
        }
    }
}

template <int K>
__device__ __forceinline__ void f16_head(const HeadRegs & H, int rows, Lds & L, uint64_t * out_tagged,
                                         uint32_t tag, float * out_plain, const Cb0Xf * xf, uint64_t * cand_tagged,
                                         float * cand_val, int32_t * cand_idx) {
    using G = HeadGeo<K>;
    constexpr int LPR = G::LPR, RPW = G::RPW;
    const int lane = threadIdx.x & 63, lir = lane & (LPR - 1), rsub = lane / LPR, wave = threadIdx.x >> 6;
    const int gw = blockIdx.x * kW + wave, nw = gridDim.x * kW;
    const int ng = H.ng;
    (void) rows;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    if (ng > 0) {
        double acc[2] = {0.0, 0.0};
#pragma unroll
        for (int hs = 0; hs < G::HS; ++hs)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int4 x4 = *(const int4 *) &L.hq[c][(lir + hs * LPR) * 8];
                const uint16_t * xh = (const uint16_t *) &x4;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const double xd = (double) h2f(xh[j]);
#pragma unroll
                    for (int gi = 0; gi < 2; ++gi)
                        acc[gi] = fma((double) h8(H.w[gi][hs][c], j), xd, acc[gi]);   // fp16 x fp16: exact product
                }
            }
#pragma unroll
        for (int gi = 0; gi < 2; ++gi) {
            if (gi >= ng) break;
            const double a = group_sum_d(acc[gi], LPR);
            if (lir != 0) continue;
            const int r = (gw + gi * nw) * RPW + rsub;
            if (out_tagged) tstore(out_tagged + r, tag, (float) a);
            else gst(out_plain + r, (float) a);
            float v = (float) a;
            if (xf) {
                if (r >= xf->V - 1024 && r != xf->eos) v = -INFINITY;
                if (xf->rep != 1.0f && (gld(xf->seen + r) || r == xf->tok0)) v = v > 0.0f ? v / xf->rep : v * xf->rep;
                if (r == xf->eos && xf->eff != 0.0f) v = v + xf->eff;
            }
            if (v > bv || (v == bv && r < bi)) { bv = v; bi = r; }
        }
    }
    wave_argmax(bv, bi);
    if (lane == 0) { L.fred[wave] = bv; L.ired[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0 && (cand_tagged || cand_val)) {
        float v = L.fred[0];
        int i = L.ired[0];
#pragma unroll
        for (int w2 = 1; w2 < kW; ++w2) argmax_step(v, i, L.fred[w2], L.ired[w2]);
        if (cand_tagged) {
            tstore(cand_tagged + 2 * blockIdx.x, tag, v);
            tstore(cand_tagged + 2 * blockIdx.x + 1, tag, __int_as_float(i));
        } else {
            gst(cand_val + blockIdx.x, v);
            gst(cand_idx + blockIdx.x, (int32_t) i);
        }
    }
}

// First-index argmax over the workgroups' candidates (values v, indices i
// held by threads t < gridDim.x).
__device__ __forceinline__ int32_t reduce_candidates(float v, int i, Lds & L) {
    wave_argmax(v, i);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { L.fred[wave] = v; L.ired[wave] = i; }
    __syncthreads();
    float bv = L.fred[0];
    int bi = L.ired[0];
#pragma unroll
    for (int w2 = 1; w2 < kW; ++w2) argmax_step(bv, bi, L.fred[w2], L.ired[w2]);
    __syncthreads();
    return bi;
}

// -------------------------------------------------------------- attention
// Code-predictor attention of KV head g = blockIdx.x for its two query heads
// and nt tokens at positions pos0.. (causal); the 16-position KV cache of
// every code-predictor layer lives in this workgroup's LDS.
//
// nt == 2 is the prefill (positions 0 and 1), which attends over the F32
// rows of this call (src/tts_transformer.cpp:1999-2012): q, K, V and P stay
// fp32, every product is exact in fp64, and a score's sum is the four 32-dim
// partials of its quad combined (s0 + s1) + (s2 + s3).  It still writes the
// fp16 cache rows the 14 steps read, where q and P are rounded to fp16.
//
// Wave w owns row w of (q0, q1, k, v): lane l holds elements l and l + 64,
// which are exactly the NEOX rotation pairs, so QK-norm and RoPE need only
// wave reductions; the new K/V rows go straight into the LDS cache.  Then
// waves w and w + 2 both handle query head 2g + (w & 1): each computes the
// (at most 16) scores and the softmax, and forms 64 of the head's 128 output
// dims, so all four waves work and no workgroup barrier is needed.
// XL (XCD-parallel layers): every workgroup of XCD g runs KV head g, reading
// its rows [q0 q1 k v] (512 per token) from the XCD's local QKV region and
// leaving the attention rows in L.att instead of publishing them.
// tab (one token): the QKV row comes from plain memory in the GEMV's layout
// (the layer-0 table) instead of a tagged slot.
template <bool XL>
__device__ __attribute__((always_inline)) void attention_cp(const Args & A, Lds & L, const LayerQ8 & W, int layer,
                                                            int nt, int pos0, int qd, const uint64_t * qkv,
                                                            uint32_t qkv_tag, uint64_t * out, uint32_t out_tag,
                                                            bool & dead, const float * tab = nullptr) {
    const int g = XL ? (int) (blockIdx.x & 7) : (int) blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int kd = qd / 2;
    const bool f32 = nt == 2;              // the prefill: unrounded q, K, V, P
    float * qf = L.a;                      // [tok][head][128] rotated q (fp16-rounded in a step)
    float * kf = L.a + 4 * 128;            // prefill: [tok][128] rotated k, fp32
    float * vf = L.a + 6 * 128;            // prefill: [tok][128] v, fp32
    {
        const int col = XL ? wave * 128 : wave < 2 ? (g * 2 + wave) * 128 : wave == 2 ? qd + g * 128 : qd + kd + g * 128;
        const uint64_t * ptr[kB];
#pragma unroll
        for (int tok = 0; tok < 2; ++tok) {
            const uint64_t * row = qkv + (size_t) (tok < nt ? tok : 0) * (XL ? 512 : kHS) + col;
            ptr[2 * tok] = row + lane;
            ptr[2 * tok + 1] = row + lane + 64;
        }
#pragma unroll
        for (int k = 4; k < kB; ++k) ptr[k] = ptr[0];
        // norm weights and RoPE rows do not depend on the new rows: load them first
        const float * nwp = wave < 2 ? W.q_norm : W.k_norm;
        const float nw0 = gld(nwp + lane), nw1 = gld(nwp + lane + 64);
        float rcv[2], rsv[2];
#pragma unroll
        for (int tok = 0; tok < 2; ++tok) {
            const int pos = pos0 + (tok < nt ? tok : 0);
            rcv[tok] = gld(A.cp_rope_cos + (size_t) pos * 64 + lane);
            rsv[tok] = gld(A.cp_rope_sin + (size_t) pos * 64 + lane);
        }
        float val[kB];
        if (tab) {
            const int tcol = wave < 2 ? (g * 2 + wave) * 128 : wave == 2 ? qd + g * 128 : qd + kd + g * 128;
            val[0] = gld(tab + tcol + lane);
            val[1] = gld(tab + tcol + lane + 64);
        } else {
            twait_batch<kB, XL>(ptr, 2 * nt, qkv_tag, val, dead, A.err);
        }
        for (int tok = 0; tok < nt; ++tok) {
            const int pos = pos0 + tok;
            const float x0 = val[2 * tok], x1 = val[2 * tok + 1];
            if (wave < 3) {
                const double ss = wave_sum_d((double) (x0 * x0) + (double) (x1 * x1));
                const float mean = (float) (ss / 128.0);
                const float scale = 1.0f / sqrtf(mean + A.eps);
                float y0 = x0 * scale, y1 = x1 * scale;
                y0 = y0 * nw0;
                y1 = y1 * nw1;
                const float c = rcv[tok], sn = rsv[tok];
                const float a0 = y0 * c, b0 = y1 * sn, a1 = y0 * sn, b1 = y1 * c;
                const float o0 = a0 - b0, o1 = a1 + b1;
                if (wave < 2) {
                    qf[(tok * 2 + wave) * 128 + lane] = f32 ? o0 : round_f16(o0);
                    qf[(tok * 2 + wave) * 128 + lane + 64] = f32 ? o1 : round_f16(o1);
                } else {
                    L.cpk[layer][pos * 128 + lane] = f2h(o0);
                    L.cpk[layer][pos * 128 + lane + 64] = f2h(o1);
                    if (f32) {
                        kf[tok * 128 + lane] = o0;
                        kf[tok * 128 + lane + 64] = o1;
                    }
                }
            } else {
                L.cpv[layer][pos * 128 + lane] = f2h(x0);
                L.cpv[layer][pos * 128 + lane + 64] = f2h(x1);
                if (f32) {
                    vf[tok * 128 + lane] = x0;
                    vf[tok * 128 + lane + 64] = x1;
                }
            }
        }
    }
    __syncthreads();

    // Scores with 4 lanes per position (32 dims each, quad DPP sum), softmax
    // with wave reductions, P.V with one dim per lane over the positions
    // (unrolled to the cache length; each probability broadcast by readlane).
    const int hq = wave & 1, d = (wave >> 1) * 64 + lane;
    const int jq = lane >> 2, sq = lane & 3;
    const uint16_t * kc = L.cpk[layer];
    const uint16_t * vc = L.cpv[layer];
    for (int tok = 0; tok < nt; ++tok) {
        const int n_kv = pos0 + tok + 1;
        double acc = 0.0;
        if (jq < n_kv) {
            const float * q = qf + (tok * 2 + hq) * 128 + sq * 32;
            if (f32) {
                const float * k = kf + jq * 128 + sq * 32;
#pragma unroll
                for (int c = 0; c < 8; ++c) {
                    const float4 k4 = *(const float4 *) &k[c * 4], q4 = *(const float4 *) &q[c * 4];
                    acc = fma((double) q4.x, (double) k4.x, acc);
                    acc = fma((double) q4.y, (double) k4.y, acc);
                    acc = fma((double) q4.z, (double) k4.z, acc);
                    acc = fma((double) q4.w, (double) k4.w, acc);
                }
            } else {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int4 k4 = *(const int4 *) &kc[jq * 128 + sq * 32 + c * 8];
                    const float4 qa = *(const float4 *) &q[c * 8], qb = *(const float4 *) &q[c * 8 + 4];
                    const float qv[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
                    for (int e = 0; e < 8; ++e) acc = fma((double) qv[e], (double) h8(k4, e), acc);
                }
            }
        }
        acc += dpp_d<0xB1>(acc);
        acc += dpp_d<0x4E>(acc);
        const float sv = jq < n_kv ? (float) acc * A.attn_scale : -INFINITY;
        const float mx = wave_max_f(sv);
        const float ev = jq < n_kv ? expf_q3t(sv - mx) : 0.0f;
        const double sum = wave_sum_d(sq == 0 ? (double) ev : 0.0);
        const float inv = (float) (1.0 / sum);
        const float pr = f32 ? ev * inv : round_f16(ev * inv);
        float vv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) vv[j] = f32 ? (j < 2 ? vf[j * 128 + d] : 0.0f) : h2f(vc[j * 128 + d]);
        double o = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if (j >= n_kv) break;
            const double pj = (double) __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr), j * 4));
            o = fma(pj, (double) vv[j], o);
        }
        if (XL) L.att[tok][hq * 128 + d] = (float) o;
        else tstore(out + (size_t) tok * kHS + (g * 2 + hq) * 128 + d, out_tag, (float) o);
    }
    __syncthreads();
}

// ------------------------------------------------- talker attention (split)
// The talker's attention over its HBM cache runs on every workgroup: b =
// blockIdx.x takes KV head g = b % H and position chunk c = b / H (C = grid/H
// chunks of Lc positions, Lc a multiple of 16).  The softmax is exact as in
// the reference, so its global maximum and sum each need a hand-off:
//   A  stage q (both heads), k, v; scores of the chunk -> chunk maxima
//   B  global maxima -> exp of the chunk, fp64 chunk sums
//   C  global sums (added in chunk order) -> fp16 probabilities -> fp64 P.V
//      partials of the chunk (256 per workgroup, published as 32-bit halves
//      over kPvSlots consecutive slots)
//   D  each workgroup adds the C partials of 8 outputs in chunk order and
//      publishes the attention rows the Wo GEMV reads
// The chunk's cached K and V rows are loaded before the QKV wait (they do not
// depend on the new token), kPre position steps of each.
constexpr int kPre = 4;                      // position steps of K and V prefetched per thread
constexpr int kScoreRow = 1024;              // two-phase form: scores per head row (8 groups x 2 heads in 2 slots)
constexpr int kPvSlots = 16;                 // arena slots phase C spans (256 wg x 512 halves)
constexpr int kMaxChunk = kMaxCtx;           // longest chunk whose scores fit L.sc

struct AttSplit {
    int g, c, C, Lc, j0, j1;
};
__device__ __forceinline__ AttSplit att_split(const Args & A, int n_kv) {
    AttSplit s;
    const int H = A.n_kv_head;
    s.C = (int) gridDim.x / H;
    s.Lc = 16 * ((n_kv + 16 * s.C - 1) / (16 * s.C));
    s.g = (int) blockIdx.x % H;
    s.c = (int) blockIdx.x / H;
    s.j0 = s.c * s.Lc;
    s.j1 = min(s.j0 + s.Lc, n_kv);
    return s;
}

struct KvPre {
    int4 k[kPre], v[kPre];
};

// Position of step i for this lane: 16 lanes per position (8 dims each),
// 4 positions per wave, 16 per workgroup step.
__device__ __forceinline__ int att_pos(const AttSplit & s, int i) {
    return s.j0 + i * 16 + (int) (threadIdx.x >> 6) * 4 + (int) ((threadIdx.x & 63) >> 4);
}

__device__ __forceinline__ void att_prefetch(const Args & A, int layer, const AttSplit & s, int pos0, KvPre & P) {
    if (s.c >= s.C) return;
    const int sub = threadIdx.x & 15;
    const size_t base = ((size_t) layer * A.n_kv_head + s.g) * A.n_ctx * 128;
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int j = att_pos(s, i);
        if (j < s.j1 && j < pos0) {
            P.k[i] = gld4(A.kc + base + (size_t) j * 128 + sub * 8);
            P.v[i] = gld4(A.vc + base + (size_t) j * 128 + sub * 8);
        }
    }
}

// score_out != nullptr (two-phase form): the chunk's scores themselves are
// published at score_out[(2g + h) * kScoreRow + j] instead of its maxima.
// XL (XCD-parallel layers): q, k, v come from this XCD's local QKV region
// ([q0 q1 k v]), and the scores or maxima go to XCD-local regions per KV
// head (maxima at g * 64 + 2c + h).
template <bool XL, bool KB = false>
__device__ __attribute__((always_inline)) void att_scores(const Args & A, Lds & L, const LayerQ8 & W, int layer,
                                                          int pos0, int qd, const AttSplit & s, const KvPre & P,
                                                          const uint64_t * qkv, uint32_t qkv_tag, uint64_t * out,
                                                          uint32_t out_tag, bool & dead, uint64_t * score_out = nullptr) {
    if (s.c >= s.C) return;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, g = s.g;
    const int kd = qd / 2;
    float * qf = L.a;                      // [head][128] rotated, fp16-rounded q
    float * knew = L.a + 2 * 128;          // [128]
    float * vnew = knew + 128;             // [128]
    const size_t base = ((size_t) layer * A.n_kv_head + g) * A.n_ctx * 128;
    constexpr bool bf = KB;               // bfloat16 cache: q, K, V (and P) rounded to bfloat16
    {
        const int col = XL ? wave * 128 : wave < 2 ? (g * 2 + wave) * 128 : wave == 2 ? qd + g * 128 : qd + kd + g * 128;
        const float * nwp = wave < 2 ? W.q_norm : W.k_norm;
        const float nw0 = gld(nwp + lane), nw1 = gld(nwp + lane + 64);
        const float rcv = gld(A.rope_cos + (size_t) pos0 * 64 + lane), rsv = gld(A.rope_sin + (size_t) pos0 * 64 + lane);
        const uint64_t * ptr[2] = {qkv + col + lane, qkv + col + lane + 64};
        float val[2];
        twait_batch<2, XL>(ptr, 2, qkv_tag, val, dead, A.err);
        const float x0 = val[0], x1 = val[1];
        const bool writer = s.c == 0;      // one workgroup per KV head appends the new rows
        if (wave < 3) {
            const double ss = wave_sum_d((double) (x0 * x0) + (double) (x1 * x1));
            const float mean = (float) (ss / 128.0);
            const float scale = 1.0f / sqrtf(mean + A.eps);
            float y0 = x0 * scale, y1 = x1 * scale;
            y0 = y0 * nw0;
            y1 = y1 * nw1;
            const float a0 = y0 * rcv, b0 = y1 * rsv, a1 = y0 * rsv, b1 = y1 * rcv;
            const float o0 = a0 - b0, o1 = a1 + b1;
            if (wave < 2) {
                qf[wave * 128 + lane] = round_kv(o0, bf);
                qf[wave * 128 + lane + 64] = round_kv(o1, bf);
            } else {
                const uint16_t h0 = f2kv(o0, bf), h1 = f2kv(o1, bf);
                knew[lane] = kv2f(h0, bf);
                knew[lane + 64] = kv2f(h1, bf);
                if (writer) {
                    gst(A.kc + base + (size_t) pos0 * 128 + lane, h0);
                    gst(A.kc + base + (size_t) pos0 * 128 + lane + 64, h1);
                }
            }
        } else {
            const uint16_t h0 = f2kv(x0, bf), h1 = f2kv(x1, bf);
            vnew[lane] = kv2f(h0, bf);
            vnew[lane + 64] = kv2f(h1, bf);
            if (writer) {
                gst(A.vc + base + (size_t) pos0 * 128 + lane, h0);
                gst(A.vc + base + (size_t) pos0 * 128 + lane + 64, h1);
            }
        }
    }
    __syncthreads();
    const int sub = lane & 15;
    double q0[8], q1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        q0[e] = (double) qf[sub * 8 + e];
        q1[e] = (double) qf[128 + sub * 8 + e];
    }
    float lm0 = -INFINITY, lm1 = -INFINITY;
    const int steps = s.Lc / 16;
    for (int i = 0; i < steps; ++i) {
        const int j = att_pos(s, i);
        int4 kk = make_int4(0, 0, 0, 0);
        if (i < kPre) {
#pragma unroll
            for (int u = 0; u < kPre; ++u) if (u == i) kk = P.k[u];
        } else if (j < s.j1 && j < pos0) {
            kk = gld4(A.kc + base + (size_t) j * 128 + sub * 8);
        }
        float kv[8];
        if (j == pos0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) kv[e] = knew[sub * 8 + e];
        } else {
            const uint16_t * kh = (const uint16_t *) &kk;
#pragma unroll
            for (int e = 0; e < 8; ++e) kv[e] = kv2f(kh[e], bf);
        }
        // fp16 x fp16 (bfloat16 x bfloat16) products are exact in fp64: fma rounds like mul + add
        double a0 = 0.0, a1 = 0.0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const double kd8 = (double) kv[e];
            a0 = fma(q0[e], kd8, a0);
            a1 = fma(q1[e], kd8, a1);
        }
        a0 = group_sum_d(a0, 16);
        a1 = group_sum_d(a1, 16);
        if (j < s.j1) {
            const float s0 = (float) a0 * A.attn_scale, s1 = (float) a1 * A.attn_scale;
            if (sub == 0) {
                if (score_out) {
                    xstore<XL>(score_out + (size_t) (2 * g) * kScoreRow + j, out_tag, s0);
                    xstore<XL>(score_out + (size_t) (2 * g + 1) * kScoreRow + j, out_tag, s1);
                } else {
                    L.sc[j - s.j0] = s0;
                    L.sc[kMaxChunk + j - s.j0] = s1;
                }
            }
            lm0 = fmaxf(lm0, s0);
            lm1 = fmaxf(lm1, s1);
        }
    }
    if (score_out) return;
    lm0 = wave_max_f(lm0);
    lm1 = wave_max_f(lm1);
    if (lane == 0) { L.fred[wave] = lm0; L.fred[kW + wave] = lm1; }
    __syncthreads();
    if (t < 2) {
        float m = L.fred[t * kW];
#pragma unroll
        for (int w = 1; w < kW; ++w) m = fmaxf(m, L.fred[t * kW + w]);
        if (XL) lstore(out + g * 64 + s.c * 2 + t, out_tag, m);
        else tstore(out + blockIdx.x * 2 + t, out_tag, m);
    }
}

template <bool XL>
__device__ __attribute__((always_inline)) void att_sums(const Args & A, Lds & L, const AttSplit & s,
                                                        const uint64_t * in, uint32_t in_tag, uint64_t * out,
                                                        uint32_t out_tag, bool & dead) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, H = A.n_kv_head;
    float * gm = L.a + 4 * 128;            // [C][2] chunk maxima of this KV head
    if (s.c < s.C) {
        for (int i = t; i < 2 * s.C; i += kT)
            gm[i] = XL ? xwait<true>(in + s.g * 64 + i, in_tag, dead, A.err)
                       : twait(in + (s.g + (i >> 1) * H) * 2 + (i & 1), in_tag, dead, A.err);
    }
    __syncthreads();
    if (s.c >= s.C) return;
    float mx0 = gm[0], mx1 = gm[1];
    for (int c = 1; c < s.C; ++c) { mx0 = fmaxf(mx0, gm[2 * c]); mx1 = fmaxf(mx1, gm[2 * c + 1]); }
    double ls0 = 0.0, ls1 = 0.0;
    const int n = s.j1 - s.j0;
    for (int j = t; j < n; j += kT) {
        const float e0 = expf_q3t(L.sc[j] - mx0), e1 = expf_q3t(L.sc[kMaxChunk + j] - mx1);
        L.sc[j] = e0; L.sc[kMaxChunk + j] = e1;
        ls0 += (double) e0; ls1 += (double) e1;
    }
    ls0 = wave_sum_d(ls0);
    ls1 = wave_sum_d(ls1);
    if (lane == 0) { L.red[wave] = ls0; L.red[kW + wave] = ls1; }
    __syncthreads();
    if (t < 2) {
        double sm = L.red[t * kW];
#pragma unroll
        for (int w = 1; w < kW; ++w) sm += L.red[t * kW + w];
        uint64_t * dst = XL ? out + s.g * 128 + s.c * 4 + 2 * t : out + blockIdx.x * 4 + 2 * t;
        xstore<XL>(dst, out_tag, __int_as_float(__double2loint(sm)));
        xstore<XL>(dst + 1, out_tag, __int_as_float(__double2hiint(sm)));
    }
}

template <bool XL, bool KB = false>
__device__ __attribute__((always_inline)) void att_pv(const Args & A, Lds & L, int layer, int pos0,
                                                      const AttSplit & s, const KvPre & P, const uint64_t * in,
                                                      uint32_t in_tag, uint64_t * out, uint32_t out_tag,
                                                      bool & dead) {
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, H = A.n_kv_head;
    uint32_t * gs = (uint32_t *) (L.a + 4 * 128);   // [C][2 heads][2 halves] chunk sums
    if (s.c < s.C) {
        for (int i = t; i < 4 * s.C; i += kT)
            gs[i] = __float_as_uint(XL ? xwait<true>(in + s.g * 128 + i, in_tag, dead, A.err)
                                       : twait(in + (s.g + (i >> 2) * H) * 4 + (i & 3), in_tag, dead, A.err));
    }
    __syncthreads();
    if (s.c >= s.C) return;
    double sum0 = 0.0, sum1 = 0.0;
    for (int c = 0; c < s.C; ++c) {
        sum0 += __hiloint2double((int) gs[4 * c + 1], (int) gs[4 * c]);
        sum1 += __hiloint2double((int) gs[4 * c + 3], (int) gs[4 * c + 2]);
    }
    const float inv0 = (float) (1.0 / sum0), inv1 = (float) (1.0 / sum1);
    const int n = s.j1 - s.j0;
    for (int j = t; j < n; j += kT) {
        L.sc[j] = round_kv(L.sc[j] * inv0, KB);
        L.sc[kMaxChunk + j] = round_kv(L.sc[kMaxChunk + j] * inv1, KB);
    }
    __syncthreads();
    const int sub = lane & 15;
    const float * vnew = L.a + 3 * 128;
    const size_t base = ((size_t) layer * A.n_kv_head + s.g) * A.n_ctx * 128;
    double o0[8], o1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) { o0[e] = 0.0; o1[e] = 0.0; }
    const int steps = s.Lc / 16;
    for (int i = 0; i < steps; ++i) {
        const int j = att_pos(s, i);
        int4 vv4 = make_int4(0, 0, 0, 0);
        if (i < kPre) {
#pragma unroll
            for (int u = 0; u < kPre; ++u) if (u == i) vv4 = P.v[u];
        } else if (j < s.j1 && j < pos0) {
            vv4 = gld4(A.vc + base + (size_t) j * 128 + sub * 8);
        }
        if (j < s.j1) {
            const double p0 = (double) L.sc[j - s.j0], p1 = (double) L.sc[kMaxChunk + j - s.j0];
            float vv[8];
            if (j == pos0) {
#pragma unroll
                for (int e = 0; e < 8; ++e) vv[e] = vnew[sub * 8 + e];
            } else {
                const uint16_t * vh = (const uint16_t *) &vv4;
#pragma unroll
                for (int e = 0; e < 8; ++e) vv[e] = kv2f(vh[e], KB);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double vd = (double) vv[e];
                o0[e] = fma(p0, vd, o0[e]);
                o1[e] = fma(p1, vd, o1[e]);
            }
        }
    }
    // the 4 positions of a wave step: lanes l, l^16, l^32, l^48 hold the same dims
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        o0[e] += swz16_d(o0[e]);
        o0[e] += __shfl_xor(o0[e], 32);
        o1[e] += swz16_d(o1[e]);
        o1[e] += __shfl_xor(o1[e], 32);
    }
    __syncthreads();                        // the probabilities are consumed: reuse L.sc
    double * part = (double *) L.sc;        // [wave][head][128]
    if (lane < 16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            part[(wave * 2 + 0) * 128 + sub * 8 + e] = o0[e];
            part[(wave * 2 + 1) * 128 + sub * 8 + e] = o1[e];
        }
    }
    __syncthreads();
    {
        const int h = t >> 7, d = t & 127;
        double r = part[h * 128 + d];
#pragma unroll
        for (int w = 1; w < kW; ++w) r += part[(w * 2 + h) * 128 + d];
        uint64_t * dst = out + (size_t) (XL ? s.g * s.C + s.c : (int) blockIdx.x) * 512 + h * 256 + d * 2;
        xstore<XL>(dst, out_tag, __int_as_float(__double2loint(r)));
        xstore<XL>(dst + 1, out_tag, __int_as_float(__double2hiint(r)));
    }
}

// Talker contexts up to kScoreRow positions take two phases instead of four:
//   A  as in the split form, but each chunk workgroup publishes its scores
//      (2 heads x its positions, into two consecutive arena slots);
//   B  every workgroup of KV head g gathers the head group's whole score row,
//      runs the softmax (maximum, exp, fp64 sum, fp16 probabilities; cheap and
//      identical in every workgroup) and forms DPW = 128 * H / grid output
//      dims of both heads over all positions, publishing the attention rows.
// This workgroup's V columns (positions t + 256u) are loaded before the QKV
// wait.  Longer contexts use the four-phase form.
struct KvCols {
    uint16_t v[4][4];                        // V[t + 256u][c*DPW + d]
};

__device__ __forceinline__ bool att_two_phase(const Args & A, int n_kv) {
    const int C = (int) gridDim.x / A.n_kv_head;
    return n_kv <= kScoreRow && C >= 32 && 128 % C == 0 && 2 * A.n_kv_head * kScoreRow <= 2 * kSlot;
}

__device__ __forceinline__ void att2_prefetch(const Args & A, int layer, int pos0, KvCols & P) {
    const int H = A.n_kv_head, C = (int) gridDim.x / H, dpw = 128 / C;
    const int g = (int) blockIdx.x % H, c = (int) blockIdx.x / H;
    if (c >= C) return;
    const size_t base = ((size_t) layer * H + g) * A.n_ctx * 128;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int j = (int) threadIdx.x + u * kT;
#pragma unroll
        for (int d = 0; d < 4; ++d)
            if (d < dpw && j < pos0) P.v[u][d] = gld(A.vc + base + (size_t) j * 128 + c * dpw + d);
    }
}

// XL: the scores come from XCD-local regions, and the attention rows of the
// head pair go to this XCD's local region (out [h * 128 + d]).
template <bool XL, bool KB = false>
__device__ __attribute__((always_inline)) void att2_pv(const Args & A, Lds & L, int pos0, const KvCols & P,
                                                       const uint64_t * scores, uint32_t sc_tag, uint64_t * out,
                                                       uint32_t out_tag, bool & dead) {
    const int H = A.n_kv_head, C = (int) gridDim.x / H, dpw = 128 / C;
    const int g = (int) blockIdx.x % H, c = (int) blockIdx.x / H;
    if (c >= C) return;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6, n_kv = pos0 + 1;
    const float * vnew = L.a + 3 * 128;
    // the head group's score rows into L.sc[h * kMaxChunk + j]
    for (int i0 = 0; i0 < 2 * n_kv; i0 += kB * kT) {
        const uint64_t * ptr[kB];
        int cnt = 0;
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const int i = i0 + k * kT + t;
            const int h = i >= n_kv, j = i - h * n_kv;
            ptr[k] = scores + (size_t) (2 * g + h) * kScoreRow + (i < 2 * n_kv ? j : 0);
            if (i < 2 * n_kv) cnt = k + 1;
        }
        float val[kB];
        twait_batch<kB, XL>(ptr, cnt, sc_tag, val, dead, A.err);
#pragma unroll
        for (int k = 0; k < kB; ++k) {
            const int i = i0 + k * kT + t;
            if (i < 2 * n_kv) {
                const int h = i >= n_kv, j = i - h * n_kv;
                L.sc[h * kMaxChunk + j] = val[k];
            }
        }
    }
    __syncthreads();
    float lm0 = -INFINITY, lm1 = -INFINITY;
    for (int j = t; j < n_kv; j += kT) { lm0 = fmaxf(lm0, L.sc[j]); lm1 = fmaxf(lm1, L.sc[kMaxChunk + j]); }
    lm0 = wave_max_f(lm0);
    lm1 = wave_max_f(lm1);
    if (lane == 0) { L.fred[wave] = lm0; L.fred[kW + wave] = lm1; }
    __syncthreads();
    float mx0 = L.fred[0], mx1 = L.fred[kW];
#pragma unroll
    for (int w = 1; w < kW; ++w) { mx0 = fmaxf(mx0, L.fred[w]); mx1 = fmaxf(mx1, L.fred[kW + w]); }
    double ls0 = 0.0, ls1 = 0.0;
    for (int j = t; j < n_kv; j += kT) {
        const float e0 = expf_q3t(L.sc[j] - mx0), e1 = expf_q3t(L.sc[kMaxChunk + j] - mx1);
        L.sc[j] = e0; L.sc[kMaxChunk + j] = e1;
        ls0 += (double) e0; ls1 += (double) e1;
    }
    ls0 = wave_sum_d(ls0);
    ls1 = wave_sum_d(ls1);
    if (lane == 0) { L.red[wave] = ls0; L.red[kW + wave] = ls1; }
    __syncthreads();
    double sum0 = L.red[0], sum1 = L.red[kW];
#pragma unroll
    for (int w = 1; w < kW; ++w) { sum0 += L.red[w]; sum1 += L.red[kW + w]; }
    const float inv0 = (float) (1.0 / sum0), inv1 = (float) (1.0 / sum1);
    // P.V for this workgroup's dims: thread t owns positions t + 256u
    double o[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int d = 0; d < 4; ++d) o[h][d] = 0.0;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int j = t + u * kT;
        if (j < n_kv) {
            const double p0 = (double) round_kv(L.sc[j] * inv0, KB), p1 = (double) round_kv(L.sc[kMaxChunk + j] * inv1, KB);
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                if (d >= dpw) break;
                // fp16 probability x fp16 value: exact in fp64
                const double vd = (double) (j == pos0 ? vnew[c * dpw + d] : kv2f(P.v[u][d], KB));
                o[0][d] = fma(p0, vd, o[0][d]);
                o[1][d] = fma(p1, vd, o[1][d]);
            }
        }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int d = 0; d < 4; ++d) o[h][d] = wave_sum_d(o[h][d]);
    double * part = (double *) L.sc;       // [wave][head][4] (the probabilities are consumed)
    __syncthreads();
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int d = 0; d < 4; ++d) part[(wave * 2 + h) * 4 + d] = o[h][d];
    }
    __syncthreads();
    if (t < 2 * dpw) {
        const int h = t / dpw, d = t % dpw;
        double r = part[h * 4 + d];
#pragma unroll
        for (int w = 1; w < kW; ++w) r += part[(w * 2 + h) * 4 + d];
        if (XL) lstore(out + h * 128 + c * dpw + d, out_tag, (float) r);
        else tstore(out + (g * 2 + h) * 128 + c * dpw + d, out_tag, (float) r);
    }
}

// Phase D: 8 attention outputs per workgroup (n_head * 128 over the grid),
// each the chunk-ordered fp64 sum of its KV head's C partials.
// XL: workgroup (g, c) combines outputs [8c, 8c + 8) of KV head g's pair
// (256 rows) from the head's XCD-local partials and writes them to the XCD's
// local region (out [o]).
template <bool XL>
__device__ __attribute__((always_inline)) void att_combine(const Args & A, Lds & L, const uint64_t * in,
                                                           uint32_t in_tag, uint64_t * out, uint32_t out_tag,
                                                           bool & dead) {
    const int t = threadIdx.x, H = A.n_kv_head, C = (int) gridDim.x / H;
    const int n_out = XL ? 256 : A.n_head * 128;
    const int opw = XL ? 256 / C : (n_out + (int) gridDim.x - 1) / (int) gridDim.x;   // outputs per workgroup
    const int gx = (int) blockIdx.x % H, cx = (int) blockIdx.x / H;
    uint32_t * w = (uint32_t *) L.sc;        // [opw][C][2]
    for (int i = t; i < opw * 2 * C; i += kT) {
        const int k = i / (2 * C), c = (i >> 1) % C, half = i & 1;
        const int o = (XL ? cx : (int) blockIdx.x) * opw + k;
        uint32_t v = 0;
        if (o < n_out) {
            const int hq = o >> 7, d = o & 127, g = XL ? gx : hq >> 1, hh = hq & 1;
            const size_t src = (size_t) (XL ? g * C + c : g + c * H) * 512 + hh * 256 + d * 2 + half;
            v = __float_as_uint(XL ? xwait<true>(in + src, in_tag, dead, A.err) : twait(in + src, in_tag, dead, A.err));
        }
        w[i] = v;
    }
    __syncthreads();
    if (t < opw) {
        const int o = (XL ? cx : (int) blockIdx.x) * opw + t;
        if (o < n_out) {
            double r = 0.0;
            for (int c = 0; c < C; ++c) r += __hiloint2double((int) w[(t * C + c) * 2 + 1], (int) w[(t * C + c) * 2]);
            xstore<XL>(out + o, out_tag, (float) r);
        }
    }
    __syncthreads();
}

// ------------------------------------------------------------- samplers
// codebook-0 token from the talker logits (plain memory, written by the
// previous kernel): suppression window, repetition penalty, EOS bias ramp.
// Out of line, once per frame, so the sampler's registers stay out of the
// frame program's allocation.
__device__ __attribute__((noinline)) int32_t sample_cb0(const Args & A, Lds & L, int frame) {
    const SampleParams & P = *A.params;
    const int V = A.codec_vocab;
    if (P.temperature <= 0.0f && frame > 0) {
        // greedy: the previous frame's talker head left one transformed
        // candidate per workgroup
        const int t = threadIdx.x;
        const bool in = t < (int) gridDim.x;
        return reduce_candidates(in ? gld(A.cand_val + t) : -INFINITY, in ? gld(A.cand_idx + t) : 0x7fffffff, L);
    }
    for (int i = threadIdx.x; i < V; i += kT) {
        float v = gld(A.logits + i);
        if (i >= V - 1024 && i != A.eos_id) v = -INFINITY;
        if (P.rep_penalty != 1.0f && gld(A.seen + i)) v = v > 0.0f ? v / P.rep_penalty : v * P.rep_penalty;
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

// The sampled draw of sample_cp, kept out of line: its register arrays
// would otherwise raise the register pressure of the whole frame program
// (the greedy decode's phases included).  `dead` is passed through a local of
// the caller so the caller's own flag stays in a register.
__device__ __attribute__((noinline)) int32_t sample_cp_draw(const Args & A, Lds & L, const uint64_t * logits,
                                                             uint32_t tag, int frame, int group, bool & dead) {
    const SampleParams & P = *A.params;
    // sampled: this thread's contiguous chunk of the logits straight into
    // registers (the valid loads of a thread form a prefix of the batch)
    constexpr int MAXC = sample_chunk<kT>();
    const int V = A.cp_vocab, C = (V + kT - 1) / kT, t = threadIdx.x;
    const uint64_t * ptr[MAXC];
    int cnt = 0;
#pragma unroll
    for (int c = 0; c < MAXC; ++c) {
        const int i = t * C + c;
        const bool ok = c < C && i < V;
        ptr[c] = logits + (ok ? i : 0);
        if (ok) cnt = c + 1;
    }
    float x[MAXC];
    twait_batch<MAXC>(ptr, cnt, tag, x, dead, A.err);
    return sample_regs<kT>(x, V, P.temperature, P.top_k, A.eos_id, 0.0f, P.seed, (uint32_t) frame, (uint32_t) group,
                           L.S);
}

// code-predictor token of codebook `group` from tagged head logits
__device__ __attribute__((always_inline)) int32_t sample_cp(const Args & A, Lds & L, const uint64_t * logits, uint32_t tag, int frame, int group,
                             bool & dead) {
    const SampleParams & P = *A.params;
    if (P.temperature <= 0.0f) {
        // greedy: one (value, index) candidate per head workgroup, tagged
        // after the logits in the head slot
        const int t = threadIdx.x;
        float v = -INFINITY;
        int i = 0x7fffffff;
        if (t < (int) gridDim.x) {
            const uint64_t * ptr[kB];
#pragma unroll
            for (int k = 0; k < kB; ++k) ptr[k] = logits + kHS + 2 * t + (k & 1);
            float val[kB];
            twait_batch<kB>(ptr, 2, tag, val, dead, A.err);
            v = val[0];
            i = __float_as_int(val[1]);
        }
        return reduce_candidates(v, i, L);
    }
    bool d2 = dead;
    const int code = sample_cp_draw(A, L, logits, tag, frame, group, d2);
    dead = d2;
    return code;
}

// The talker attention for the context's cache type, chosen once per call
// (KB: bfloat16 cache) rather than per element.
#define Q3T_KV_TYPED(...)                       \
    do {                                        \
        if (A.kv_bf16) {                        \
            constexpr bool KB = true;           \
            __VA_ARGS__;                        \
        } else {                                \
            constexpr bool KB = false;          \
            __VA_ARGS__;                        \
        }                                       \
    } while (0)

// ------------------------------------------------------------------ layers
// One decoder layer (QKV -> attention -> Wo + residual -> gate/up SwiGLU ->
// down + residual) for NT tokens.  The input rows come from tagged slot p_in,
// or (x_lds != nullptr, layer 0) from the rows gathered into LDS.  The
// output is tagged slot p_out.  TK: a talker layer (weights read
// non-temporally).
template <int NT, int D, int QD, int FF, int WT, bool TK>
__device__ __attribute__((always_inline)) void layer_t(const Args & A, Lds & L, const LayerQ8 & W, int layer, bool cp, int pos0, uint32_t tb, int & p,
                        int p_in, const float * x_lds, int & p_out, bool & dead) {
    constexpr int QKVD = 2 * QD;
    uint64_t * ar = A.arena;
    // Wo and down have fewer row groups than waves: they start at the second
    // half of the waves, away from the attention workgroups (0..n_kv_head-1)
    // and from the waves that carry two gate/up groups (the first ones)
    const int rot = (int) (gridDim.x / 2) * kW;
    // talker: this workgroup's chunk of cached K/V rows, loaded now (it does
    // not depend on anything this frame computes)
    KvPre kv;
    KvCols kc2;
    const bool two_phase = !cp && att_two_phase(A, pos0 + 1);
    if (!cp) att_prefetch(A, layer, att_split(A, pos0 + 1), pos0, kv);
    if (two_phase) att2_prefetch(A, layer, pos0, kc2);
    // QKV (RMSNorm'd input)
    const int p_qkv = p++;
    constexpr int NGQ = ngroups<D>(QKVD);
    if (wg_has_rows<D>(QKVD, 0)) {
        Q8Regs<D, false, NGQ> R;
        F16Regs<D, false, NGQ> F;
        if constexpr (WT == W_Q8) q8_prefetch<D, false, TK, NGQ>(R, W.qkv, W.qkv_d, nullptr, nullptr, QKVD, 0);
        else f16_prefetch<D, false, TK, NGQ>(F, (const uint16_t *) W.qkv, nullptr, QKVD, 0);
        NormT<D> nw;
        norm_prefetch<D>(W.attn_norm, nw);
        RowsT<NT, D> v;
        if (x_lds) {
            load_lds<NT, D>(x_lds, v);
        } else {
            load_tagged<NT, D>(ar + (size_t) p_in * kSlot, tb | p_in, v, dead, A.err);
        }
        rms_rows<NT, D>(v, nw, A.eps, L);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, D>(v, L);
            q8_compute<NT, D, false, NGQ>(R, L, EPI_STORE, nullptr, 0, ar + (size_t) p_qkv * kSlot, tb | p_qkv, 0, dead,
                                          A.err);
        } else {
            f16_rows<NT, D, false>(v, L);
            f16_compute<NT, D, false, false, NGQ>(F, L, EPI_STORE, nullptr, 0, ar + (size_t) p_qkv * kSlot, tb | p_qkv, 0,
                                             dead, A.err);
        }
    }
    __syncthreads();
    // attention: code predictor on workgroup g < n_kv_head (KV head g, cache
    // in LDS); talker split over every workgroup in four phases
    int p_att;
    if (cp) {
        p_att = p++;
        if ((int) blockIdx.x < A.n_kv_head)
            attention_cp<false>(A, L, W, layer, NT, pos0, QD, ar + (size_t) p_qkv * kSlot, tb | p_qkv,
                         ar + (size_t) p_att * kSlot, tb | p_att, dead);
        __syncthreads();
    } else if (two_phase) {
        // scores in the two slots p_a, p_a + 1; the other split-phase slots stay
        // unused, so both forms share one phase numbering
        const AttSplit sp = att_split(A, pos0 + 1);
        const int p_a = p;
        p += 2 + kPvSlots;
        p_att = p++;
        Q3T_KV_TYPED(att_scores<false, KB>(A, L, W, layer, pos0, QD, sp, kv, ar + (size_t) p_qkv * kSlot, tb | p_qkv,
                   ar + (size_t) p_a * kSlot, tb | p_a, dead, ar + (size_t) p_a * kSlot));
        __syncthreads();
        Q3T_KV_TYPED(att2_pv<false, KB>(A, L, pos0, kc2, ar + (size_t) p_a * kSlot, tb | p_a, ar + (size_t) p_att * kSlot, tb | p_att, dead));
        __syncthreads();
    } else {
        const AttSplit sp = att_split(A, pos0 + 1);
        const int p_a = p++, p_b = p++, p_c = p;
        p += kPvSlots;
        p_att = p++;
        Q3T_KV_TYPED(att_scores<false, KB>(A, L, W, layer, pos0, QD, sp, kv, ar + (size_t) p_qkv * kSlot, tb | p_qkv,
                   ar + (size_t) p_a * kSlot, tb | p_a, dead));
        __syncthreads();
        att_sums<false>(A, L, sp, ar + (size_t) p_a * kSlot, tb | p_a, ar + (size_t) p_b * kSlot, tb | p_b, dead);
        __syncthreads();
        Q3T_KV_TYPED(att_pv<false, KB>(A, L, layer, pos0, sp, kv, ar + (size_t) p_b * kSlot, tb | p_b, ar + (size_t) p_c * kSlot, tb | p_c,
               dead));
        __syncthreads();
        att_combine<false>(A, L, ar + (size_t) p_c * kSlot, tb | p_c, ar + (size_t) p_att * kSlot, tb | p_att, dead);
    }
    // Wo + residual (the block input)
    const int p_wo = p++;
    constexpr int NGO = ngroups<QD>(D);
    if (wg_has_rows<QD>(D, rot)) {
        RowsT<NT, QD> v;
        if constexpr (WT == W_Q8) {
            Q8Regs<QD, false, NGO> R;
            q8_prefetch<QD, false, TK, NGO>(R, W.wo, W.wo_d, nullptr, nullptr, D, rot);
            res_prefetch<NT, QD, false, NGO>(R, ar + (size_t) p_in * kSlot, rot);
            load_tagged<NT, QD>(ar + (size_t) p_att * kSlot, tb | p_att, v, dead, A.err);
            quant_rows<NT, QD>(v, L);
            q8_compute<NT, QD, false, NGO>(R, L, EPI_RESID, ar + (size_t) p_in * kSlot, tb | p_in,
                                           ar + (size_t) p_wo * kSlot, tb | p_wo, rot, dead, A.err);
        } else {
            F16Regs<QD, false, NGO> F;
            f16_prefetch<QD, false, TK, NGO>(F, (const uint16_t *) W.wo, nullptr, D, rot);
            res_prefetch16<NT, QD, false, NGO>(F, ar + (size_t) p_in * kSlot, rot);
            load_tagged<NT, QD>(ar + (size_t) p_att * kSlot, tb | p_att, v, dead, A.err);
            f16_rows<NT, QD, false>(v, L);
            f16_compute<NT, QD, false, false, NGO>(F, L, EPI_RESID, ar + (size_t) p_in * kSlot, tb | p_in,
                                                   ar + (size_t) p_wo * kSlot, tb | p_wo, rot, dead, A.err);
        }
    }
    __syncthreads();
    // gate/up + SwiGLU (RMSNorm'd); NGU row groups per wave (3 for the 1.7B
    // talker's 6144 rows over 1024 waves)
    constexpr int NGU = ngroups<D>(FF);
    const int p_gu = p++;
    if (wg_has_rows<D>(FF, 0)) {
        Q8Regs<D, true, NGU> R;
        F16Regs<D, true, NGU> F;
        if constexpr (WT == W_Q8) q8_prefetch<D, true, TK, NGU>(R, W.wg, W.wg_d, W.wu, W.wu_d, FF, 0);
        else f16_prefetch<D, true, TK, NGU>(F, (const uint16_t *) W.wg, (const uint16_t *) W.wu, FF, 0);
        NormT<D> nw;
        norm_prefetch<D>(W.ffn_norm, nw);
        RowsT<NT, D> v;
        load_tagged<NT, D>(ar + (size_t) p_wo * kSlot, tb | p_wo, v, dead, A.err);
        rms_rows<NT, D>(v, nw, A.eps, L);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, D>(v, L);
            q8_compute<NT, D, true, NGU>(R, L, EPI_SWIGLU, nullptr, 0, ar + (size_t) p_gu * kSlot, tb | p_gu, 0, dead,
                                         A.err);
        } else {
            f16_rows<NT, D, false>(v, L);
            f16_compute<NT, D, true, false, NGU>(F, L, EPI_SWIGLU, nullptr, 0, ar + (size_t) p_gu * kSlot, tb | p_gu, 0,
                                                 dead, A.err);
        }
    }
    __syncthreads();
    // down + residual (F16: the fp32 activation, ffn_down being widened to F32)
    const int p_dn = p++;
    if (wg_has_rows<FF>(D, rot)) {
        RowsT<NT, FF> v;
        constexpr int NGD = ngroups<FF>(D);
        if constexpr (WT == W_Q8) {
            Q8Regs<FF, false, NGD> R;
            q8_prefetch<FF, false, TK, NGD>(R, W.wd, W.wd_d, nullptr, nullptr, D, rot);
            res_prefetch<NT, FF, false, NGD>(R, ar + (size_t) p_wo * kSlot, rot);
            load_tagged<NT, FF>(ar + (size_t) p_gu * kSlot, tb | p_gu, v, dead, A.err);
            quant_rows<NT, FF>(v, L);
            q8_compute<NT, FF, false, NGD>(R, L, EPI_RESID, ar + (size_t) p_wo * kSlot, tb | p_wo,
                                           ar + (size_t) p_dn * kSlot, tb | p_dn, rot, dead, A.err);
        } else {
            F16Regs<FF, false, NGD> F;
            f16_prefetch<FF, false, TK, NGD>(F, (const uint16_t *) W.wd, nullptr, D, rot);
            res_prefetch16<NT, FF, false, NGD>(F, ar + (size_t) p_wo * kSlot, rot);
            load_tagged<NT, FF>(ar + (size_t) p_gu * kSlot, tb | p_gu, v, dead, A.err);
            f16_rows<NT, FF, true>(v, L);
            f16_compute<NT, FF, false, true, NGD>(F, L, EPI_RESID, ar + (size_t) p_wo * kSlot, tb | p_wo,
                                                  ar + (size_t) p_dn * kSlot, tb | p_dn, rot, dead, A.err);
        }
    }
    __syncthreads();
    p_out = p_dn;
}

// ---------------------------------------------------- XCD-parallel layers
// The 0.6B shapes (hidden 1024, 16 query / 8 KV heads, FFN 3072) on 256
// workgroups, workgroup b in XCD class x = b % 8 (one physical XCD, see the
// XCD-local I/O above) with rank j = b / 8 among the class's 32.  XCD x owns KV head x (query heads 2x, 2x+1) and the FFN
// columns [384x, 384x + 384); a layer is
//   QKV      XCD x: its heads' 512 rows, 16 per workgroup        -> XCD-local
//   attn     code predictor: every workgroup of XCD x, the cache in its
//            LDS; talker: the split attention of KV head x, whose 32 chunk
//            workgroups are XCD x's                            -> XCD-local
//   Wo       rows [32j, 32j+32) over the head pair's 256 inputs: fp64
//            partial sums                                      -> device-wide
//   reduce   rank j of every XCD adds the 8 XCDs' partials of its 32 outputs
//            in XCD order, rounds once, adds its residual slice -> XCD-local
//   gate/up  columns [384x + 12j, +12) of both, SwiGLU          -> XCD-local
//   down     rows [32j, 32j+32) over the XCD's 384 inputs      -> device-wide
//   reduce   as above                                          -> XCD-local
// Each workgroup computes as many GEMV rows per phase as in the row-parallel
// program, but only the two reductions cross XCDs.  Sums stay exact fp64
// sums of exact terms, rounded to fp32 once.
constexpr int kXcd = 8;                // XCDs = KV heads
constexpr int kXcdWg = 32;             // workgroups per XCD

enum XKind : int { XK_QKV = 0, XK_GU = 1, XK_WO = 2, XK_DN = 3 };
// K: the slice of a weight row one phase reads; KS: the full row; LPR lanes
// per row (one 32-element block each, lanes past K/32 idle); NG row groups
// per wave.
template <int KIND> struct XGeo;
template <> struct XGeo<XK_QKV> { static constexpr int K = 1024, KS = 1024, LPR = 32, NG = 2; static constexpr bool DUAL = false; };
template <> struct XGeo<XK_GU> { static constexpr int K = 1024, KS = 1024, LPR = 32, NG = 2; static constexpr bool DUAL = true; };
template <> struct XGeo<XK_WO> { static constexpr int K = 256, KS = 2048, LPR = 8, NG = 1; static constexpr bool DUAL = false; };
template <> struct XGeo<XK_DN> { static constexpr int K = 384, KS = 3072, LPR = 16, NG = 2; static constexpr bool DUAL = false; };

// This lane's row in group gi: weight row r, output index o, offset k0 of
// the slice in the row.  False when the group is past the phase's rows
// (the same for every lane of a wave).
template <int KIND>
__device__ __forceinline__ bool xrow(int gi, int & r, int & o, int & k0) {
    constexpr int RPW = 64 / XGeo<KIND>::LPR;
    const int x = (int) blockIdx.x & 7, j = (int) blockIdx.x >> 3, w = (int) threadIdx.x >> 6;
    const int rsub = ((int) threadIdx.x & 63) / XGeo<KIND>::LPR;
    if (KIND == XK_QKV) {
        // local rows [q head 2x | q head 2x+1 | k | v] of KV head x
        const int lr = j * 16 + (w * 2 + gi) * RPW + rsub;
        r = lr < 256 ? 256 * x + lr : lr < 384 ? 2048 + 128 * x + (lr - 256) : 3072 + 128 * x + (lr - 384);
        o = lr;
        k0 = 0;
        return true;
    } else if (KIND == XK_GU) {
        const int gg = w + gi * 4;          // 6 groups over 4 waves
        const int col = j * 12 + gg * RPW + rsub;
        r = 384 * x + col;
        o = col;
        k0 = 0;
        return gg < 6;
    } else if (KIND == XK_WO) {
        r = o = j * 32 + w * RPW + rsub;
        k0 = 256 * x;
        return true;
    } else {
        r = o = j * 32 + (w * 2 + gi) * RPW + rsub;
        k0 = 384 * x;
        return true;
    }
}

template <int KIND>
struct XRegs {
    int4 w[XGeo<KIND>::NG][2], u[XGeo<KIND>::DUAL ? XGeo<KIND>::NG : 1][2];
    uint16_t dw[XGeo<KIND>::NG], du[XGeo<KIND>::DUAL ? XGeo<KIND>::NG : 1];
    int o[XGeo<KIND>::NG];                 // output index of this lane's row, -1: none
};

// The Q8_0 blocks of this lane's rows, loaded before the phase input is awaited.
template <int KIND, bool NTL>
__device__ __forceinline__ void xq8_prefetch(XRegs<KIND> & R, const int8_t * W, const uint16_t * Wd, const int8_t * U,
                                             const uint16_t * Ud) {
    using G = XGeo<KIND>;
    constexpr int BPR = G::K / kQK;
    const int lir = (int) threadIdx.x & (G::LPR - 1);
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi) {
        int r, o, k0;
        const bool row = xrow<KIND>(gi, r, o, k0);
        R.o[gi] = row ? o : -1;
        R.w[gi][0] = R.w[gi][1] = make_int4(0, 0, 0, 0);
        R.dw[gi] = 0;
        if (G::DUAL) { R.u[G::DUAL ? gi : 0][0] = R.u[G::DUAL ? gi : 0][1] = make_int4(0, 0, 0, 0); R.du[G::DUAL ? gi : 0] = 0; }
        if (!row || lir >= BPR) continue;
        const int4 * wp = (const int4 *) (W + (size_t) r * G::KS + k0 + lir * kQK);
        R.w[gi][0] = gld4n<NTL>(wp);
        R.w[gi][1] = gld4n<NTL>(wp + 1);
        R.dw[gi] = gldn<NTL>(Wd + (size_t) r * (G::KS / kQK) + k0 / kQK + lir);
        if (G::DUAL) {
            const int4 * up = (const int4 *) (U + (size_t) r * G::KS + k0 + lir * kQK);
            R.u[G::DUAL ? gi : 0][0] = gld4n<NTL>(up);
            R.u[G::DUAL ? gi : 0][1] = gld4n<NTL>(up + 1);
            R.du[G::DUAL ? gi : 0] = gldn<NTL>(Ud + (size_t) r * (G::KS / kQK) + k0 / kQK + lir);
        }
    }
}

// The dot products over the quantised LDS input (NT rows of K/32 blocks) and
// the phase's epilogue: QKV stores its rows and gate/up its SwiGLU outputs
// XCD-locally at out[t * ts + o]; Wo and down publish fp64 partial sums
// device-wide at out[((x * 2 + t) * 1024 + o) * 2 + half].
template <int NT, int KIND>
__device__ __forceinline__ void xq8_compute(const XRegs<KIND> & R, const Lds & L, uint64_t * out, int ts,
                                            uint32_t out_tag) {
    using G = XGeo<KIND>;
    constexpr int BPR = G::K / kQK;
    const int lir = (int) threadIdx.x & (G::LPR - 1), x = (int) blockIdx.x & 7;
    const int b = lir < BPR ? lir : 0;
    double acc[G::NG][NT], acc2[G::NG][NT];
    float sw[G::NG], su[G::NG];
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi) {
        // the empty asm keeps the scale conversion (and the wait for its load)
        // out of the prefetch
        uint32_t a = R.dw[gi], c = G::DUAL ? R.du[G::DUAL ? gi : 0] : 0u;
        asm volatile("" : "+v"(a), "+v"(c));
        sw[gi] = h2f((uint16_t) a);
        su[gi] = h2f((uint16_t) c);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int4 x0 = *(const int4 *) &L.qlo[(t * BPR + b) * 16];
        const int4 x1 = *(const int4 *) &L.qhi[(t * BPR + b) * 16];
        const float dx = L.qdx[t * BPR + b];
#pragma unroll
        for (int gi = 0; gi < G::NG; ++gi) {
            // fp16(d_w) * fp16(d_x) is exact in fp32, its product with the int32
            // block sum exact in fp64; lanes past the slice add nothing
            acc[gi][t] = lir < BPR ? (double) (sw[gi] * dx) * (double) dot32_i8(R.w[gi][0], R.w[gi][1], x0, x1) : 0.0;
            acc2[gi][t] = G::DUAL && lir < BPR
                              ? (double) (su[gi] * dx) *
                                    (double) dot32_i8(R.u[G::DUAL ? gi : 0][0], R.u[G::DUAL ? gi : 0][1], x0, x1)
                              : 0.0;
        }
    }
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi) {
        if (R.o[gi] < 0) continue;          // wave-uniform
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double a1 = group_sum_d(acc[gi][t], G::LPR);
            const double a2 = G::DUAL ? group_sum_d(acc2[gi][t], G::LPR) : 0.0;
            if (lir != 0) continue;
            const int o = R.o[gi];
            if (KIND == XK_QKV) {
                lstore(out + t * ts + o, out_tag, (float) a1);
            } else if (KIND == XK_GU) {
                lstore(out + t * ts + o, out_tag, silu_q3t((float) a1) * (float) a2);
            } else {
                uint64_t * dst = out + ((size_t) (x * 2 + t) * 1024 + o) * 2;
                tstore(dst, out_tag, __int_as_float(__double2loint(a1)));
                tstore(dst + 1, out_tag, __int_as_float(__double2hiint(a1)));
            }
        }
    }
}

// F16 layers on the XCD-parallel program: a lane's 32-element block of each
// of its rows as four 16-byte chunks (the same rows and lanes as XRegs).
template <int KIND>
struct XRegs16 {
    int4 w[XGeo<KIND>::NG][4], u[XGeo<KIND>::DUAL ? XGeo<KIND>::NG : 1][4];
    int o[XGeo<KIND>::NG];                 // output index of this lane's row, -1: none
};

template <int KIND, bool NTL>
__device__ __forceinline__ void xf16_prefetch(XRegs16<KIND> & R, const uint16_t * W, const uint16_t * U) {
    using G = XGeo<KIND>;
    constexpr int BPR = G::K / kQK;
    const int lir = (int) threadIdx.x & (G::LPR - 1);
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi) {
        int r, o, k0;
        const bool row = xrow<KIND>(gi, r, o, k0);
        R.o[gi] = row ? o : -1;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            R.w[gi][c] = make_int4(0, 0, 0, 0);
            if (G::DUAL) R.u[G::DUAL ? gi : 0][c] = make_int4(0, 0, 0, 0);
        }
        if (!row || lir >= BPR) continue;
        const int4 * wp = (const int4 *) (W + (size_t) r * G::KS + k0 + lir * kQK);
#pragma unroll
        for (int c = 0; c < 4; ++c) R.w[gi][c] = gld4n<NTL>(wp + c);
        if (G::DUAL) {
            const int4 * up = (const int4 *) (U + (size_t) r * G::KS + k0 + lir * kQK);
#pragma unroll
            for (int c = 0; c < 4; ++c) R.u[G::DUAL ? gi : 0][c] = gld4n<NTL>(up + c);
        }
    }
}

// xq8_compute for F16 weights: the input rows in L.hf (fp16, from f16_rows)
// or, WIDE (the widened ffn_down), L.xw (fp32); each product exact in fp64
// (fp16 x fp16 exact in fp32; fp16 x fp32 as the fp32 product plus its fma
// residual), summed in fp64 as in f16_compute.  Same epilogues and outputs.
template <int NT, int KIND, bool WIDE>
__device__ __forceinline__ void xf16_compute(const XRegs16<KIND> & R, const Lds & L, uint64_t * out, int ts,
                                             uint32_t out_tag) {
    using G = XGeo<KIND>;
    constexpr int BPR = G::K / kQK;
    const int lir = (int) threadIdx.x & (G::LPR - 1), x = (int) blockIdx.x & 7;
    const int b = lir < BPR ? lir : 0;
    double acc[G::NG][NT], acc2[G::NG][NT];
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi)
#pragma unroll
        for (int t = 0; t < NT; ++t) { acc[gi][t] = 0.0; acc2[gi][t] = 0.0; }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        int4 xp[NT];
        float xa[WIDE ? NT : 1][8];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (WIDE) {
                const float4 x0 = *(const float4 *) xw_at<G::K>(L, t, 2 * c, b);
                const float4 x1 = *(const float4 *) xw_at<G::K>(L, t, 2 * c + 1, b);
                float * xr = xa[WIDE ? t : 0];
                xr[0] = x0.x; xr[1] = x0.y; xr[2] = x0.z; xr[3] = x0.w;
                xr[4] = x1.x; xr[5] = x1.y; xr[6] = x1.z; xr[7] = x1.w;
            } else {
                xp[t] = *(const int4 *) hf_at<G::K>(L, t, c, b);
            }
        }
#pragma unroll
        for (int gi = 0; gi < G::NG; ++gi) {
            // the empty asm keeps the weights' conversions after the input barrier
            int4 wv = R.w[gi][c], uv = R.u[G::DUAL ? gi : 0][c];
            __asm__ volatile("" : "+v"(wv.x), "+v"(wv.y), "+v"(wv.z), "+v"(wv.w));
            if (G::DUAL) __asm__ volatile("" : "+v"(uv.x), "+v"(uv.y), "+v"(uv.z), "+v"(uv.w));
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                const float wf = WIDE ? h8(wv, jj) : 0.0f, uf = WIDE && G::DUAL ? h8(uv, jj) : 0.0f;
                const _Float16 wh = h8h(wv, jj), uh = G::DUAL ? h8h(uv, jj) : (_Float16) 0.0f;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    if (WIDE) {
                        const float xf = xa[WIDE ? t : 0][jj];
                        const float pr = wf * xf, pe = fmaf(wf, xf, -pr);
                        acc[gi][t] += (double) pr + (double) pe;
                        if (G::DUAL) {
                            const float qr = uf * xf, qe = fmaf(uf, xf, -qr);
                            acc2[gi][t] += (double) qr + (double) qe;
                        }
                    } else {
                        const _Float16 xh = h8h(xp[t], jj);
                        acc[gi][t] += (double) hmul_exact(wh, xh);
                        if (G::DUAL) acc2[gi][t] += (double) hmul_exact(uh, xh);
                    }
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
    if (lir >= BPR) {                       // lanes past the slice add nothing
#pragma unroll
        for (int gi = 0; gi < G::NG; ++gi)
#pragma unroll
            for (int t = 0; t < NT; ++t) { acc[gi][t] = 0.0; acc2[gi][t] = 0.0; }
    }
#pragma unroll
    for (int gi = 0; gi < G::NG; ++gi) {
        if (R.o[gi] < 0) continue;          // wave-uniform
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const double a1 = group_sum_d(acc[gi][t], G::LPR);
            const double a2 = G::DUAL ? group_sum_d(acc2[gi][t], G::LPR) : 0.0;
            if (lir != 0) continue;
            const int o = R.o[gi];
            if (KIND == XK_QKV) {
                lstore(out + t * ts + o, out_tag, (float) a1);
            } else if (KIND == XK_GU) {
                lstore(out + t * ts + o, out_tag, silu_q3t((float) a1) * (float) a2);
            } else {
                uint64_t * dst = out + ((size_t) (x * 2 + t) * 1024 + o) * 2;
                tstore(dst, out_tag, __int_as_float(__double2loint(a1)));
                tstore(dst + 1, out_tag, __int_as_float(__double2hiint(a1)));
            }
        }
    }
}

// Rank j's 32 outputs of a device-wide partial slot: the 8 XCDs' fp64
// partials added in XCD order and rounded once, plus the residual slice
// L.rx, which takes the sum; the sums also go to the XCD-local row
// outl[t * 1024 + 32j + i].  Thread t = 8i + xs waits for output i's partial
// from XCD xs; the 8 lanes of output i then form ((p0 + p1) + ...) + p7 as a
// sequential scan over DPP shifts (step k: lane k adds lane k - 1's running
// sum to its own partial), so lane 8i + 7 holds the sum, with no LDS round
// trip or workgroup barrier.  That lane keeps L.rx[tok][i].
template <int NT>
__device__ __forceinline__ void xreduce(const Args & A, Lds & L, const uint64_t * part, uint32_t ptag, uint64_t * outl,
                                        uint32_t otag, bool & dead) {
    const int t = (int) threadIdx.x, j = (int) blockIdx.x >> 3;
    const int i = t >> 3, xs = t & 7, o = 32 * j + i;
    const uint64_t * ptr[4];
#pragma unroll
    for (int tok = 0; tok < 2; ++tok) {
        const uint64_t * src = part + ((size_t) (xs * 2 + (tok < NT ? tok : 0)) * 1024 + o) * 2;
        ptr[2 * tok] = src;
        ptr[2 * tok + 1] = src + 1;
    }
    float val[4];
    twait_batch<4>(ptr, 2 * NT, ptag, val, dead, A.err);
#pragma unroll
    for (int tok = 0; tok < NT; ++tok) {
        const double pv = __hiloint2double(__float_as_int(val[2 * tok + 1]), __float_as_int(val[2 * tok]));
        double sm = pv;
#pragma unroll
        for (int k = 1; k < kXcd; ++k) {
            const double prev = dpp_d<0x111>(sm);          // row_shr:1, lane k - 1's running sum
            if (xs == k) sm = prev + pv;
        }
        if (xs == kXcd - 1) {
            const float v = (float) sm + L.rx[tok][i];
            L.rx[tok][i] = v;
            lstore(outl + tok * 1024 + 32 * j + i, otag, v);
        }
    }
}

// One XCD-parallel layer for NT tokens (Q8_0 weights).  Input: the rows
// gathered into LDS (layer 0) or this XCD's local copy of the previous
// layer's output (slot p_in); output: slot p_out (XCD-local copies).  The
// slot numbering keeps one slot per phase (partials: 4, local rows: 2).
// tab_row (code-predictor layer 0 of steps 1..14): the layer's QKV row from
// the table, and rx_row the embedding row whose slice is the residual; the
// QKV phase is skipped.
template <int NT, bool TK, int WT = W_Q8>
__device__ __attribute__((always_inline)) void layer_x(const Args & A, Lds & L, const LayerQ8 & W, int layer, bool cp,
                                                       int pos0, uint32_t tb, int & p, int p_in, const float * x_lds,
                                                       int & p_out, bool & dead, const float * tab_row = nullptr,
                                                       const uint16_t * rx_row = nullptr) {
    constexpr int D = 1024, QD = 2048;
    uint64_t * ar = A.arena;
    const int x = (int) blockIdx.x & 7, j = (int) blockIdx.x >> 3, t = (int) threadIdx.x;
    KvPre kv;
    KvCols kc2;
    const bool two_phase = !cp && att_two_phase(A, pos0 + 1);
    if (!cp) att_prefetch(A, layer, att_split(A, pos0 + 1), pos0, kv);
    if (two_phase) att2_prefetch(A, layer, pos0, kc2);
    // QKV rows of KV head x -> local [NT][512]
    const int p_qkv = p++;
    uint64_t * qkv_l = ar + (size_t) p_qkv * kSlot + x * 1024;
    if (tab_row) {
        if (t < 32) L.rx[0][t] = h2f(gld(rx_row + 32 * j + t));
    } else {
        XRegs<XK_QKV> R;
        XRegs16<XK_QKV> F;
        if constexpr (WT == W_Q8) xq8_prefetch<XK_QKV, TK>(R, W.qkv, W.qkv_d, nullptr, nullptr);
        else xf16_prefetch<XK_QKV, TK>(F, (const uint16_t *) W.qkv, nullptr);
        NormT<D> nw;
        norm_prefetch<D>(W.attn_norm, nw);
        RowsT<NT, D> v;
        if (x_lds) {
            load_lds<NT, D>(x_lds, v);
            if (t < 32 * NT) L.rx[t >> 5][t & 31] = x_lds[(t >> 5) * D + 32 * j + (t & 31)];
        } else {
            load_tagged<NT, D, true>(ar + (size_t) p_in * kSlot + x * 2048, tb | p_in, v, dead, A.err, D);
        }
        rms_rows<NT, D>(v, nw, A.eps, L);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, D>(v, L);
            xq8_compute<NT, XK_QKV>(R, L, qkv_l, 512, tb | p_qkv);
        } else {
            f16_rows<NT, D, false>(v, L);
            xf16_compute<NT, XK_QKV, false>(F, L, qkv_l, 512, tb | p_qkv);
        }
    }
    __syncthreads();
    // attention of KV head x
    int p_att = 0;
    if (cp) {
        p_att = p++;
        attention_cp<true>(A, L, W, layer, NT, pos0, QD, qkv_l, tb | p_qkv, nullptr, 0, dead, tab_row);
    } else if (two_phase) {
        const AttSplit sp = att_split(A, pos0 + 1);
        const int p_a = p;
        p += 2 + kPvSlots;
        p_att = p++;
        Q3T_KV_TYPED(att_scores<true, KB>(A, L, W, layer, pos0, QD, sp, kv, qkv_l, tb | p_qkv, ar + (size_t) p_a * kSlot, tb | p_a, dead,
                         ar + (size_t) p_a * kSlot));
        __syncthreads();
        Q3T_KV_TYPED(att2_pv<true, KB>(A, L, pos0, kc2, ar + (size_t) p_a * kSlot, tb | p_a, ar + (size_t) p_att * kSlot + x * 1024,
                      tb | p_att, dead));
        __syncthreads();
    } else {
        const AttSplit sp = att_split(A, pos0 + 1);
        const int p_a = p++, p_b = p++, p_c = p;
        p += kPvSlots;
        p_att = p++;
        Q3T_KV_TYPED(att_scores<true, KB>(A, L, W, layer, pos0, QD, sp, kv, qkv_l, tb | p_qkv, ar + (size_t) p_a * kSlot, tb | p_a, dead));
        __syncthreads();
        att_sums<true>(A, L, sp, ar + (size_t) p_a * kSlot, tb | p_a, ar + (size_t) p_b * kSlot, tb | p_b, dead);
        __syncthreads();
        Q3T_KV_TYPED(att_pv<true, KB>(A, L, layer, pos0, sp, kv, ar + (size_t) p_b * kSlot, tb | p_b, ar + (size_t) p_c * kSlot,
                     tb | p_c, dead));
        __syncthreads();
        att_combine<true>(A, L, ar + (size_t) p_c * kSlot, tb | p_c, ar + (size_t) p_att * kSlot + x * 1024, tb | p_att,
                          dead);
    }
    // Wo partial sums over the head pair's 256 inputs -> device-wide
    const int p_wo = p;
    p += 4;
    {
        XRegs<XK_WO> R;
        XRegs16<XK_WO> F;
        if constexpr (WT == W_Q8) xq8_prefetch<XK_WO, TK>(R, W.wo, W.wo_d, nullptr, nullptr);
        else xf16_prefetch<XK_WO, TK>(F, (const uint16_t *) W.wo, nullptr);
        RowsT<NT, 256> va;
        if (cp) load_lds<NT, 256>(&L.att[0][0], va, 256);
        else load_tagged<NT, 256, true>(ar + (size_t) p_att * kSlot + x * 1024, tb | p_att, va, dead, A.err, 256);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, 256>(va, L);
            xq8_compute<NT, XK_WO>(R, L, ar + (size_t) p_wo * kSlot, 0, tb | p_wo);
        } else {
            f16_rows<NT, 256, false>(va, L);
            xf16_compute<NT, XK_WO, false>(F, L, ar + (size_t) p_wo * kSlot, 0, tb | p_wo);
        }
    }
    __syncthreads();
    const int p_x1 = p;
    p += 2;
    xreduce<NT>(A, L, ar + (size_t) p_wo * kSlot, tb | p_wo, ar + (size_t) p_x1 * kSlot + x * 2048, tb | p_x1, dead);
    // gate/up + SwiGLU of FFN columns [384x + 12j, +12) -> local [NT][384]
    const int p_gu = p++;
    {
        XRegs<XK_GU> R;
        XRegs16<XK_GU> F;
        if constexpr (WT == W_Q8) xq8_prefetch<XK_GU, TK>(R, W.wg, W.wg_d, W.wu, W.wu_d);
        else xf16_prefetch<XK_GU, TK>(F, (const uint16_t *) W.wg, (const uint16_t *) W.wu);
        NormT<D> nw;
        norm_prefetch<D>(W.ffn_norm, nw);
        RowsT<NT, D> v;
        load_tagged<NT, D, true>(ar + (size_t) p_x1 * kSlot + x * 2048, tb | p_x1, v, dead, A.err, D);
        rms_rows<NT, D>(v, nw, A.eps, L);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, D>(v, L);
            xq8_compute<NT, XK_GU>(R, L, ar + (size_t) p_gu * kSlot + x * 1024, 384, tb | p_gu);
        } else {
            f16_rows<NT, D, false>(v, L);
            xf16_compute<NT, XK_GU, false>(F, L, ar + (size_t) p_gu * kSlot + x * 1024, 384, tb | p_gu);
        }
    }
    __syncthreads();
    // down partial sums over the XCD's 384 FFN inputs -> device-wide
    const int p_dn = p;
    p += 4;
    {
        XRegs<XK_DN> R;
        XRegs16<XK_DN> F;
        if constexpr (WT == W_Q8) xq8_prefetch<XK_DN, TK>(R, W.wd, W.wd_d, nullptr, nullptr);
        else xf16_prefetch<XK_DN, TK>(F, (const uint16_t *) W.wd, nullptr);
        RowsT<NT, 384> vh;
        load_tagged<NT, 384, true>(ar + (size_t) p_gu * kSlot + x * 1024, tb | p_gu, vh, dead, A.err, 384);
        if constexpr (WT == W_Q8) {
            quant_rows<NT, 384>(vh, L);
            xq8_compute<NT, XK_DN>(R, L, ar + (size_t) p_dn * kSlot, 0, tb | p_dn);
        } else {
            // ffn_down widened to F32: the fp32 SwiGLU rows as they are
            f16_rows<NT, 384, true>(vh, L);
            xf16_compute<NT, XK_DN, true>(F, L, ar + (size_t) p_dn * kSlot, 0, tb | p_dn);
        }
    }
    __syncthreads();
    const int p_x2 = p;
    p += 2;
    xreduce<NT>(A, L, ar + (size_t) p_dn * kSlot, tb | p_dn, ar + (size_t) p_x2 * kSlot + x * 2048, tb | p_x2, dead);
    p_out = p_x2;
}

// Publish LDS rows [nt][d] as the tagged slot p (workgroup 0 only): the
// block's residual input for layer 0.
__device__ __forceinline__ void publish(const Args & A, const float * x, int nt, int d, int p, uint32_t tb) {
    if (blockIdx.x != 0) return;
    for (int t = 0; t < nt; ++t)
        for (int i = threadIdx.x; i < d; i += kT)
            tstore(A.arena + (size_t) p * kSlot + (size_t) t * kHS + i, tb | p, x[t * d + i]);
}

// code_pred.mtp_proj: the NT gathered rows of width K in L.x (Q8_0-quantised,
// or rounded to fp16 for an F16 projection) through the projection (rows =
// the code predictor's width) plus its bias, tagged into slot p.
template <int NT, int K, int WT>
__device__ __attribute__((always_inline)) void mtp_phase(const Args & A, Lds & L, int rows, int p, uint32_t tb,
                                                         bool & dead) {
    if (wg_has_rows<K>(rows, 0)) {
        RowsT<NT, K> v;
        if constexpr (WT == W_Q8) {
            Q8Regs<K, false> R;
            q8_prefetch<K, false, false>(R, A.mtp_w, A.mtp_d, nullptr, nullptr, rows, 0);
            load_lds<NT, K>(L.x, v);
            quant_rows<NT, K>(v, L);
            q8_compute<NT, K, false>(R, L, EPI_BIAS, nullptr, 0, A.arena + (size_t) p * kSlot, tb | p, 0, dead, A.err,
                                     A.mtp_b);
        } else {
            F16Regs<K, false> F;
            f16_prefetch<K, false, false>(F, (const uint16_t *) A.mtp_w, nullptr, rows, 0);
            load_lds<NT, K>(L.x, v);
            f16_rows<NT, K, false>(v, L);
            f16_compute<NT, K, false, false>(F, L, EPI_BIAS, nullptr, 0, A.arena + (size_t) p * kSlot, tb | p, 0, dead,
                                             A.err, A.mtp_b);
        }
    }
    __syncthreads();
}

// The head's input: the last token's row of the pass's output slot, normed
// (width K), into L.hq (and, for the talker, the hidden row the next frame's
// code predictor reads).
template <int K, bool XT>
__device__ __attribute__((always_inline)) void head_rows(const Args & A, Lds & L, const float * norm, int p_out,
                                                         int nt, uint32_t tb, float * hidden, bool & dead) {
    NormT<K> nw;
    norm_prefetch<K>(norm, nw);
    RowsT<1, K> v;
    if constexpr (XT)
        load_tagged<1, K, true>(A.arena + (size_t) p_out * kSlot + ((int) blockIdx.x & 7) * 2048 + (size_t) (nt - 1) * K,
                                tb | p_out, v, dead, A.err, K);
    else
        load_tagged<1, K>(A.arena + (size_t) p_out * kSlot + (size_t) (nt - 1) * kHS, tb | p_out, v, dead, A.err);
    head_input<K>(v, nw, A.eps, L, hidden);
}

// The argument block lives in device memory: dynamic indexing into a by-value
// kernel argument (cp_embd[s], cp_head[s]) would copy it to private scratch.
// One workgroup per CU, so one wave per SIMD: the full unified register file
// (256 VGPRs + 256 AGPRs) is available to every wave.
// `frame` indexes the sampler streams and the frame state; `epoch` (distinct
// for every launch since the arena was last cleared) makes the phase tags.
// XT: the XCD-parallel layer program (layer_x; Q8_0 0.6B shapes, 256
// workgroups dealt round-robin over the XCDs).
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID, 0, 4)" : "=s"(v));
    return v;
}

template <int D, int DC, int QD, int FF, int FFC, int WT, bool XT>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_frame(const Args * __restrict__ Ap,
                                                                                         int32_t frame, int32_t epoch,
                                                                                         int32_t mode) {
    const Args & A = *Ap;
    __shared__ Lds L;
    bool dead = false;
    FrameState * st = A.st;
    if (st->done) return;
    const uint32_t tb = (uint32_t) (epoch + 1) << 12;
    const int t = threadIdx.x;
    int p = 0;

    // ---- codebook 0 (every workgroup samples the same token).  Workgroup 0
    // writes the frame state only at the end of the kernel: by then every
    // workgroup has finished this sampler (it consumed their later outputs),
    // so none can still be reading `seen`.
    int32_t tok0 = 0;
    if (mode == MODE_FRAME) {
        tok0 = sample_cb0(A, L, frame);
        if (tok0 == A.eos_id) {
            if (blockIdx.x == 0 && t == 0) { st->frame = frame; st->codes[0] = tok0; st->done = 1; st->eos = 1; }
            return;
        }
    } else if (mode == MODE_CODE_PRED) {
        tok0 = st->codes[0];
    }
    if (t == 0) L.codes[0] = tok0;

    // ---- 16 passes: s = 0..14 code predictor (s = 0 is the 2-token prefill
    // [hidden; codec_embd[tok0]], then one step per codebook), s = 15 the
    // talker step on the summed step embedding.  One call site per layer
    // shape keeps the inlined program small.
    int code = tok0;
    const int pos = mode == MODE_TALKER_STEP ? st->talker_pos : st->base_pos + frame;
    const int s_first = mode == MODE_TALKER_STEP ? 15 : 0, s_last = mode == MODE_CODE_PRED ? 14 : 15;
    for (int s = s_first; s <= s_last; ++s) {
        const bool tk = s == 15;
        const int p_x = p++;
        if (s == 0) {
            for (int i = t; i < D; i += kT) {
                L.x[i] = gld(A.hidden + i);
                L.x[D + i] = h2f(gld(A.codec_embd + (size_t) tok0 * D + i));
            }
        } else if (!tk) {
            if (!(XT && A.cp_qkv0))
                for (int i = t; i < D; i += kT) L.x[i] = h2f(gld(A.cp_embd[s - 1] + (size_t) code * D + i));
        } else if (mode == MODE_TALKER_STEP) {
            for (int i = t; i < D; i += kT) L.x[i] = gld(A.step_in + i);
        } else {
            // emit the frame, then the step embedding (reference summation order)
            if (blockIdx.x == 0 && t < 16) A.codes_out[(size_t) frame * 16 + t] = L.codes[t];
            for (int i = t; i < D; i += kT) {
                float e = h2f(gld(A.codec_embd + (size_t) L.codes[0] * D + i));
                for (int g = 1; g < 16; ++g) e = e + h2f(gld(A.cp_embd[g - 1] + (size_t) L.codes[g] * D + i));
                const float tr = frame < A.n_trailing ? gld(A.trailing + (size_t) frame * D + i) : gld(A.pad + i);
                L.x[i] = e + tr;
            }
        }
        __syncthreads();
        const int nt = s == 0 ? 2 : 1;
        const int pos0 = tk ? pos : s == 0 ? 0 : s + 1;
        int p_in = p_x, p_out = p_x;
        const float * x0 = L.x;
        if constexpr (DC != D) {
            if (!tk) {
                // the 1.7B layout: the code predictor's input rows pass through
                // code_pred.mtp_proj (+ bias) into its own width
                const int p_m = p++;
                if (nt == 2) mtp_phase<2, D, WT>(A, L, DC, p_m, tb, dead);
                else mtp_phase<1, D, WT>(A, L, DC, p_m, tb, dead);
                p_in = p_out = p_m;
                x0 = nullptr;
            }
        }
        if (!XT && x0) publish(A, L.x, nt, tk ? D : DC, p_x, tb);
        const int nl = tk ? A.n_layers : A.cp_layers;
        const LayerQ8 * Ls = tk ? A.talker : A.cp;
        for (int l = 0; l < nl; ++l) {
            const float * x_lds = l == 0 ? x0 : nullptr;
            const LayerQ8 Wl = layer_desc(Ls + l);
            if constexpr (XT) {
                const bool tabl = A.cp_qkv0 && !tk && s > 0 && l == 0;
                const float * tab_row =
                    tabl ? A.cp_qkv0 + ((size_t) (s - 1) * A.cp_vocab + code) * (size_t) (QD + QD) : nullptr;
                const uint16_t * rx_row = tabl ? A.cp_embd[s - 1] + (size_t) code * D : nullptr;
                if (nt == 2) layer_x<2, false, WT>(A, L, Wl, l, true, pos0, tb, p, p_in, x_lds, p_out, dead);
                else if (tk) layer_x<1, true, WT>(A, L, Wl, l, false, pos0, tb, p, p_in, x_lds, p_out, dead);
                else layer_x<1, false, WT>(A, L, Wl, l, true, pos0, tb, p, p_in, x_lds, p_out, dead, tab_row, rx_row);
            } else {
                if (nt == 2) layer_t<2, DC, QD, FFC, WT, false>(A, L, Wl, l, true, pos0, tb, p, p_in, x_lds, p_out, dead);
                else if (tk) layer_t<1, D, QD, FF, WT, true>(A, L, Wl, l, false, pos0, tb, p, p_in, x_lds, p_out, dead);
                else layer_t<1, DC, QD, FFC, WT, false>(A, L, Wl, l, true, pos0, tb, p, p_in, x_lds, p_out, dead);
            }
            p_in = p_out;
        }
        // head on the last token's normed row
        const int p_head = tk ? 0 : p++;
        HeadRegs hr;
        if (tk) {
            f16_head_prefetch<D, true>(A.codec_head, A.codec_vocab, hr);
            head_rows<D, XT>(A, L, A.out_norm, p_out, nt, tb, A.hidden, dead);
        } else {
            f16_head_prefetch<DC, false>(A.cp_head[s], A.cp_vocab, hr);
            head_rows<DC, XT>(A, L, A.cp_out_norm, p_out, nt, tb, nullptr, dead);
        }
        if (tk) {
            const SampleParams & P = *A.params;
            Cb0Xf xf{A.codec_vocab, A.eos_id, L.codes[0], P.rep_penalty, P.eos_bias, A.seen};
            if (P.target_frames > 0 && frame + 1 > P.target_frames) {   // the next frame's EOS-bias ramp
                xf.eff += 0.1f * (float) (frame + 1 - P.target_frames);
                if (xf.eff > 6.0f) xf.eff = 6.0f;
            }
            if (mode == MODE_FRAME)
                f16_head<D>(hr, A.codec_vocab, L, nullptr, 0, A.logits, &xf, nullptr, A.cand_val, A.cand_idx);
            else
                f16_head<D>(hr, A.codec_vocab, L, nullptr, 0, A.logits, nullptr, nullptr, nullptr, nullptr);
        } else {
            uint64_t * hs = A.arena + (size_t) p_head * kSlot;
            f16_head<DC>(hr, A.cp_vocab, L, hs, tb | p_head, nullptr, nullptr, hs + kHS, nullptr, nullptr);
            __syncthreads();
            code = sample_cp(A, L, A.arena + (size_t) p_head * kSlot, tb | p_head, frame, s + 1, dead);
            if (t == 0) L.codes[s + 1] = code;
            __syncthreads();
        }
    }
    if (mode == MODE_CODE_PRED && blockIdx.x == 0 && t == 0)
        for (int g = 1; g < 16; ++g) st->codes[g] = L.codes[g];
    if (mode == MODE_FRAME && blockIdx.x == 0 && t == 0) {
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
