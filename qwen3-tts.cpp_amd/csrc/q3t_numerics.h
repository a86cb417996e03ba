// q3t_numerics.h -- device-side arithmetic shared by every kernel of the
// frame loop.  Each helper rounds exactly where the reference's ggml CPU
// path rounds (fp16 activations, fp16 KV, Q8_0 activation quantisation);
// reductions take exact terms and accumulate in fp64 so that the rounded
// fp32 result does not depend on how the GPU splits the sum.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace q3t {

constexpr int kBlock = 256;   // threads per workgroup for GEMV / attention
constexpr int kQK = 32;       // Q8_0 block length

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
// Exact fp32 product of two fp16 values (at most 22 significant bits, no
// overflow or underflow in fp32) as one mixed-precision fma with a zero addend.
__device__ __forceinline__ float hmul_exact(_Float16 a, _Float16 b) { return __builtin_fmaf((float) a, (float) b, 0.0f); }
// The empty asm makes the fp32 value opaque: without it the compiler folds
// f2h(a * b) into v_fma_mixlo_f16 (one rounding of the exact product to
// fp16), which differs from rounding to fp32 and then to fp16 whenever the
// fp32 product lands exactly on an fp16 tie.
__device__ __forceinline__ uint16_t f2h(float f) {
    __asm__("" : "+v"(f));
    return __half_as_ushort(__float2half_rn(f));
}
__device__ __forceinline__ float round_f16(float f) { return h2f(f2h(f)); }

// bfloat16 (a BF16 talker cache): round to nearest even on the upper 16 bits,
// NaN kept quiet, as ggml's GGML_FP32_TO_BF16; widening is exact.
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t) h << 16); }
__device__ __forceinline__ uint16_t f2bf(float f) {
    const uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((x >> 16) | 64u);
    return (uint16_t) ((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}
// Cache element <-> fp32 for an F16 (bf = false) or BF16 (bf = true) cache.
__device__ __forceinline__ float kv2f(uint16_t h, bool bf) { return bf ? bf2f(h) : h2f(h); }
__device__ __forceinline__ uint16_t f2kv(float f, bool bf) { return bf ? f2bf(f) : f2h(f); }
__device__ __forceinline__ float round_kv(float f, bool bf) { return kv2f(f2kv(f, bf), bf); }

// exp(x): Cody-Waite reduction x = k*ln2 + r (ln2 split hi/lo, fused
// multiply-add), exp(r) by its degree-7 Taylor polynomial in Horner form,
// scaled by 2^k built from the exponent field.  Results below 2^-126 are
// flushed to zero (x < -87); x > 88.7228 overflows to +inf.  Max error
// about 1 ulp; the same steps are restated on the CPU for parity.
__device__ __forceinline__ float expf_q3t(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.72283935546875f) return __int_as_float(0x7f800000);
    const float k = rintf(x * 1.44269504088896341f);
    float r = fmaf(-k, 0.693145751953125f, x);
    r = fmaf(-k, 1.428606765330187e-06f, r);
    float p = 1.98412698412698413e-4f;
    p = fmaf(p, r, 1.38888888888888889e-3f);
    p = fmaf(p, r, 8.33333333333333333e-3f);
    p = fmaf(p, r, 4.16666666666666667e-2f);
    p = fmaf(p, r, 1.66666666666666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    int ki = (int) k;
    if (ki > 127) { p = p * 2.0f; ki -= 1; }
    return p * __int_as_float((ki + 127) << 23);
}

// ggml_silu_f32: x / (1 + e^-x), correctly rounded division.
__device__ __forceinline__ float silu_q3t(float x) { return x / (1.0f + expf_q3t(-x)); }

// Cross-lane moves through DPP (VALU, a few cycles) instead of ds_bpermute.
// ctrl: 0xB1 = quad_perm[1,0,3,2] (xor 1), 0x4E = quad_perm[2,3,0,1] (xor 2),
// 0x141 = row_half_mirror (lane i <-> 7-i), 0x140 = row_mirror (i <-> 15-i).
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const int lo = __builtin_amdgcn_update_dpp(0, __double2loint(v), CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, __double2hiint(v), CTRL, 0xF, 0xF, false);
    return __hiloint2double(hi, lo);
}
// lane i <-> i ^ 16 within each 32-lane half (ds_swizzle bit mode, xor_mask 0x10)
__device__ __forceinline__ double swz16_d(double v) {
    const int lo = __builtin_amdgcn_ds_swizzle(__double2loint(v), 0x401F);
    const int hi = __builtin_amdgcn_ds_swizzle(__double2hiint(v), 0x401F);
    return __hiloint2double(hi, lo);
}
// Sum over each aligned group of n lanes (n = 8, 16 or 32, a power of two
// <= 32).  Every lane of a group ends with the bitwise-same value (each step
// adds a lane's value and its partner's, and fp addition commutes).
__device__ __forceinline__ double group_sum_d(double v, int n) {
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    if (n > 4) v += dpp_d<0x141>(v);
    if (n > 8) v += dpp_d<0x140>(v);
    if (n > 16) v += swz16_d(v);
    return v;
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ double readlane_d(double v, int lane) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                            __builtin_amdgcn_readlane(__double2loint(v), lane));
}

// Wave64 reductions (all 64 lanes active): DPP / swizzle within each 32-lane
// half, then the two halves through readlane.  Every lane gets the same value.
__device__ __forceinline__ double wave_sum_d(double v) {
    v = group_sum_d(v, 32);
    return readlane_d(v, 0) + readlane_d(v, 32);
}
__device__ __forceinline__ float wave_max_f(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
    return fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)),
                 __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32)));
}
// First-index argmax over the wave: (value, index) with the larger value, or
// the smaller index on equal values.  Every lane gets the winner.
__device__ __forceinline__ void argmax_step(float & bv, int & bi, float ov, int oi) {
    if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
}
__device__ __forceinline__ void wave_argmax(float & bv, int & bi) {
    argmax_step(bv, bi, dpp_f<0xB1>(bv), __builtin_amdgcn_update_dpp(0, bi, 0xB1, 0xF, 0xF, false));
    argmax_step(bv, bi, dpp_f<0x4E>(bv), __builtin_amdgcn_update_dpp(0, bi, 0x4E, 0xF, 0xF, false));
    argmax_step(bv, bi, dpp_f<0x141>(bv), __builtin_amdgcn_update_dpp(0, bi, 0x141, 0xF, 0xF, false));
    argmax_step(bv, bi, dpp_f<0x140>(bv), __builtin_amdgcn_update_dpp(0, bi, 0x140, 0xF, 0xF, false));
    argmax_step(bv, bi, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(bv), 0x401F)),
                __builtin_amdgcn_ds_swizzle(bi, 0x401F));
    float v0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 0));
    int i0 = __builtin_amdgcn_readlane(bi, 0);
    argmax_step(v0, i0, __int_as_float(__builtin_amdgcn_readlane(__float_as_int(bv), 32)), __builtin_amdgcn_readlane(bi, 32));
    bv = v0; bi = i0;
}

// Workgroup-wide fp64 sum for 256 threads; every thread gets the same value.
// red: 4 doubles of LDS.
__device__ __forceinline__ double block_sum_d(double v, double * red) {
    v = wave_sum_d(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max_f(float v, float * red) {
    v = wave_max_f(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Eight int8x4 dot products: sum of 32 int8 products, exact in int32.
__device__ __forceinline__ int dot32_i8(const int4 a0, const int4 a1, const int4 b0, const int4 b1) {
    int s = 0;
    s = __builtin_amdgcn_sdot4(a0.x, b0.x, s, false);
    s = __builtin_amdgcn_sdot4(a0.y, b0.y, s, false);
    s = __builtin_amdgcn_sdot4(a0.z, b0.z, s, false);
    s = __builtin_amdgcn_sdot4(a0.w, b0.w, s, false);
    s = __builtin_amdgcn_sdot4(a1.x, b1.x, s, false);
    s = __builtin_amdgcn_sdot4(a1.y, b1.y, s, false);
    s = __builtin_amdgcn_sdot4(a1.z, b1.z, s, false);
    s = __builtin_amdgcn_sdot4(a1.w, b1.w, s, false);
    return s;
}

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC'11).  Returns a uniform double in [0,1) from 53 bits.
__device__ __forceinline__ double philox_uniform(uint64_t key, uint32_t c0, uint32_t c1) {
    uint32_t k0 = (uint32_t) key, k1 = (uint32_t) (key >> 32);
    uint32_t c[4] = {c0, c1, 0u, 0u};
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint64_t p0 = (uint64_t) 0xD2511F53u * c[0];
        const uint64_t p1 = (uint64_t) 0xCD9E8D57u * c[2];
        const uint32_t n0 = (uint32_t) (p1 >> 32) ^ c[1] ^ k0;
        const uint32_t n2 = (uint32_t) (p0 >> 32) ^ c[3] ^ k1;
        c[0] = n0; c[1] = (uint32_t) p1; c[2] = n2; c[3] = (uint32_t) p0;
    }
    return ((double) (c[0] >> 5) * 67108864.0 + (double) (c[1] >> 6)) * (1.0 / 9007199254740992.0);
}

}  // namespace q3t
