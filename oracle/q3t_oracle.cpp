// q3t_oracle.cpp -- CPU restatement of the qwen3-tts.cpp per-frame token loop.
//
// TEST INFRASTRUCTURE ONLY: parity checker and timed CPU baseline.  The
// numerics contract and the reference functions restated are listed in
// q3t_oracle.h.  Written from the reference's behaviour; no reference source
// is reused.  Build: oracle/Makefile (g++ -O3 -ffp-contract=off).

#include "q3t_oracle.h"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <cstring>
#include <functional>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace {

inline uint32_t f2u(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }

float g_f16_table[65536];
struct TableInit {
    TableInit() {
        for (uint32_t i = 0; i < 65536; ++i) g_f16_table[i] = orc_f16_to_f32((uint16_t) i);
    }
} g_table_init;

inline float h2f(uint16_t h) { return g_f16_table[h]; }

// ---------------------------------------------------------------- threads
class Pool {
public:
    explicit Pool(int n) { resize(n); }
    ~Pool() { stop(); }
    void resize(int n) {
        stop();
        n_ = std::max(1, n);
        quit_ = false;
        for (int i = 1; i < n_; ++i) workers_.emplace_back([this, i] { loop(i); });
    }
    int size() const { return n_; }
    // fn(begin, end) over [0, n) split into n_ contiguous chunks.
    void run(int64_t n, const std::function<void(int64_t, int64_t)> & fn) {
        if (n_ == 1 || n < 2) { fn(0, n); return; }
        {
            std::unique_lock<std::mutex> lk(mu_);
            fn_ = &fn; total_ = n; pending_ = n_ - 1; ++gen_;
        }
        cv_.notify_all();
        chunk(0, n, fn);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [this] { return pending_ == 0; });
        fn_ = nullptr;
    }
private:
    void chunk(int idx, int64_t n, const std::function<void(int64_t, int64_t)> & fn) {
        int64_t b = n * idx / n_, e = n * (idx + 1) / n_;
        if (b < e) fn(b, e);
    }
    void loop(int idx) {
        uint64_t seen = 0;
        for (;;) {
            const std::function<void(int64_t, int64_t)> * fn;
            int64_t n;
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return quit_ || gen_ != seen; });
                if (quit_) return;
                seen = gen_; fn = fn_; n = total_;
            }
            chunk(idx, n, *fn);
            std::unique_lock<std::mutex> lk(mu_);
            if (--pending_ == 0) done_cv_.notify_one();
        }
    }
    void stop() {
        { std::unique_lock<std::mutex> lk(mu_); quit_ = true; }
        cv_.notify_all();
        for (auto & t : workers_) t.join();
        workers_.clear();
    }
    int n_ = 1;
    std::vector<std::thread> workers_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const std::function<void(int64_t, int64_t)> * fn_ = nullptr;
    int64_t total_ = 0;
    int pending_ = 0;
    uint64_t gen_ = 0;
    bool quit_ = false;
};

Pool * g_default_pool() { static Pool p(1); return &p; }

// ------------------------------------------------------------ gemv cores
constexpr int QK = 32;
constexpr int QB = 34;   // bytes per Q8_0 block: fp16 d + 32 int8

void quant_act_block(const float * x, uint8_t * out) {
    float amax = 0.0f;
    for (int j = 0; j < QK; ++j) amax = std::max(amax, std::fabs(x[j]));
    const float d  = amax / 127.0f;
    const float id = (amax != 0.0f) ? 127.0f / amax : 0.0f;
    uint16_t dh = orc_f32_to_f16(d);
    std::memcpy(out, &dh, 2);
    int8_t * q = (int8_t *) (out + 2);
    for (int j = 0; j < QK; ++j) q[j] = (int8_t) (int) std::nearbyint(x[j] * id);
}

inline double q8_row_dot(const uint8_t * wrow, const uint8_t * xq, int64_t nb) {
    double acc = 0.0;
    for (int64_t b = 0; b < nb; ++b) {
        const uint8_t * wb = wrow + b * QB;
        const uint8_t * xb = xq + b * QB;
        uint16_t dw, dx;
        std::memcpy(&dw, wb, 2);
        std::memcpy(&dx, xb, 2);
        const int8_t * qw = (const int8_t *) (wb + 2);
        const int8_t * qx = (const int8_t *) (xb + 2);
        int32_t isum = 0;
        for (int j = 0; j < QK; ++j) isum += (int32_t) qw[j] * (int32_t) qx[j];
        acc += ((double) h2f(dw) * (double) h2f(dx)) * (double) isum;
    }
    return acc;
}

inline double f16_row_dot(const uint16_t * w, const float * x, int64_t k) {
    double a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int64_t i = 0;
    for (; i + 8 <= k; i += 8)
        for (int j = 0; j < 8; ++j) a[j] += (double) h2f(w[i + j]) * (double) x[i + j];
    double s = 0.0;
    for (; i < k; ++i) s += (double) h2f(w[i]) * (double) x[i];
    for (int j = 0; j < 8; ++j) s += a[j];
    return s;
}

void gemv_impl(Pool * pool, int type, const void * w, int64_t rows, int64_t k,
               const float * x, int64_t ntok, float * y, int widen) {
    if (type == ORC_TYPE_Q8_0) {
        const int64_t nb = k / QK;
        std::vector<uint8_t> xq((size_t) (ntok * nb * QB));
        for (int64_t t = 0; t < ntok; ++t)
            for (int64_t b = 0; b < nb; ++b)
                quant_act_block(x + t * k + b * QK, xq.data() + (t * nb + b) * QB);
        const uint8_t * wb = (const uint8_t *) w;
        pool->run(rows, [&](int64_t r0, int64_t r1) {
            for (int64_t r = r0; r < r1; ++r)
                for (int64_t t = 0; t < ntok; ++t)
                    y[t * rows + r] = (float) q8_row_dot(wb + r * nb * QB, xq.data() + t * nb * QB, nb);
        });
    } else if (type == ORC_TYPE_F16) {
        std::vector<float> xr((size_t) (ntok * k));
        for (int64_t i = 0; i < ntok * k; ++i)
            xr[i] = widen ? x[i] : h2f(orc_f32_to_f16(x[i]));
        const uint16_t * wh = (const uint16_t *) w;
        pool->run(rows, [&](int64_t r0, int64_t r1) {
            for (int64_t r = r0; r < r1; ++r)
                for (int64_t t = 0; t < ntok; ++t)
                    y[t * rows + r] = (float) f16_row_dot(wh + r * k, xr.data() + t * k, k);
        });
    } else {  // F32 weights
        const float * wf = (const float *) w;
        pool->run(rows, [&](int64_t r0, int64_t r1) {
            for (int64_t r = r0; r < r1; ++r)
                for (int64_t t = 0; t < ntok; ++t) {
                    double s = 0.0;
                    for (int64_t i = 0; i < k; ++i) s += (double) wf[r * k + i] * (double) x[t * k + i];
                    y[t * rows + r] = (float) s;
                }
        });
    }
}

inline float silu(float x) { return x / (1.0f + orc_expf(-x)); }

// -------------------------------------------------------------- philox
inline void mulhilo(uint32_t a, uint32_t b, uint32_t & hi, uint32_t & lo) {
    uint64_t p = (uint64_t) a * (uint64_t) b;
    hi = (uint32_t) (p >> 32);
    lo = (uint32_t) p;
}

// ----------------------------------------------------------- sampling
int32_t sample_probs(const std::vector<float> & p, double u) {
    double total = 0.0;
    for (float v : p) total += (double) v;
    const double target = u * total;
    double cum = 0.0;
    int32_t last = -1;
    for (size_t i = 0; i < p.size(); ++i) {
        if (p[i] > 0.0f) {
            cum += (double) p[i];
            last = (int32_t) i;
            if (cum > target) return (int32_t) i;
        }
    }
    return last < 0 ? 0 : last;
}

// logits already temperature-scaled and biased: top-k, softmax, draw.
int32_t topk_softmax_draw(float * l, int32_t n, int32_t top_k, double u) {
    if (top_k > 0 && top_k < n) {
        std::vector<float> s(l, l + n);
        std::nth_element(s.begin(), s.begin() + (top_k - 1), s.end(), std::greater<float>());
        const float thr = s[top_k - 1];
        for (int32_t i = 0; i < n; ++i)
            if (l[i] < thr) l[i] = -INFINITY;
    }
    float mx = -INFINITY;
    for (int32_t i = 0; i < n; ++i) mx = std::max(mx, l[i]);
    std::vector<float> e(n);
    double sum = 0.0;
    for (int32_t i = 0; i < n; ++i) { e[i] = orc_expf(l[i] - mx); sum += (double) e[i]; }
    for (int32_t i = 0; i < n; ++i) e[i] = (float) ((double) e[i] / sum);
    return sample_probs(e, u);
}

}  // namespace

// ================================================================ C API
extern "C" {

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu;
    const uint32_t mant = h & 0x3ffu;
    if (ex == 0) {
        float v = (float) mant * 5.9604644775390625e-08f;  // mant * 2^-24, exact
        return u2f(f2u(v) | sign);
    }
    if (ex == 31) return u2f(sign | 0x7f800000u | (mant << 13));
    return u2f(sign | ((ex + 112u) << 23) | (mant << 13));
}

uint16_t orc_f32_to_f16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t) ((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u);
    if (ax >= 0x477ff000u) return sign | 0x7c00u;            // >= 65520 -> inf
    if (ax < 0x38800000u) {                                   // < 2^-14: subnormal
        const float v = u2f(ax) * 16777216.0f;                // units of 2^-24, exact
        return sign | (uint16_t) (uint32_t) std::nearbyint(v);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return sign | (uint16_t) h;
}

// bfloat16 <-> fp32 as ggml converts them (GGML_FP32_TO_BF16: round to
// nearest even on the upper 16 bits, NaN kept quiet; the reverse is a shift).
float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t) h << 16); }

uint16_t orc_f32_to_bf16(float f) {
    const uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((x >> 16) | 64u);
    return (uint16_t) ((x + (0x7fffu + ((x >> 16) & 1u))) >> 16);
}

float orc_expf(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.72283935546875f) return INFINITY;
    const float k = std::rint(x * 1.44269504088896341f);
    float r = std::fma(-k, 0.693145751953125f, x);
    r = std::fma(-k, 1.428606765330187e-06f, r);
    float p = 1.98412698412698413e-4f;     // 1/7!
    p = std::fma(p, r, 1.38888888888888889e-3f);   // 1/6!
    p = std::fma(p, r, 8.33333333333333333e-3f);   // 1/5!
    p = std::fma(p, r, 4.16666666666666667e-2f);   // 1/4!
    p = std::fma(p, r, 1.66666666666666667e-1f);   // 1/3!
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    int ki = (int) k;
    if (ki > 127) { p = p * 2.0f; ki -= 1; }
    return p * u2f((uint32_t) (ki + 127) << 23);
}

void orc_quantize_q8_0_weights(const float * x, int64_t n, uint8_t * out) {
    for (int64_t b = 0; b < n / QK; ++b) {
        const float * xb = x + b * QK;
        float amax = 0.0f;
        for (int j = 0; j < QK; ++j) amax = std::max(amax, std::fabs(xb[j]));
        const float d = amax / 127.0f;
        uint16_t dh = orc_f32_to_f16(d);
        std::memcpy(out + b * QB, &dh, 2);
        int8_t * q = (int8_t *) (out + b * QB + 2);
        for (int j = 0; j < QK; ++j) q[j] = d == 0.0f ? 0 : (int8_t) (int) std::round(xb[j] / d);
    }
}

void orc_quantize_q8_0_act(const float * x, int64_t n, uint8_t * out) {
    for (int64_t b = 0; b < n / QK; ++b) quant_act_block(x + b * QK, out + b * QB);
}

void orc_dequantize_q8_0(const uint8_t * blocks, int64_t n, float * out) {
    for (int64_t b = 0; b < n / QK; ++b) {
        uint16_t dh;
        std::memcpy(&dh, blocks + b * QB, 2);
        const float d = h2f(dh);
        const int8_t * q = (const int8_t *) (blocks + b * QB + 2);
        for (int j = 0; j < QK; ++j) out[b * QK + j] = d * (float) q[j];
    }
}

void orc_gemv(int type, const void * w, int64_t rows, int64_t k,
              const float * x, int64_t ntok, float * y, int widen_f16) {
    gemv_impl(g_default_pool(), type, w, rows, k, x, ntok, y, widen_f16);
}

void orc_rmsnorm(const float * x, const float * w, int64_t n, float eps, float * y) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; ++i) sum += (double) (x[i] * x[i]);
    const float mean = (float) (sum / (double) n);
    const float scale = 1.0f / std::sqrt(mean + eps);
    for (int64_t i = 0; i < n; ++i) {
        const float t = x[i] * scale;
        y[i] = w ? t * w[i] : t;
    }
}

void orc_rope_table(float theta_base, int64_t head_dim, int64_t n_pos, float * cos_tab, float * sin_tab) {
    const int64_t half = head_dim / 2;
    const float theta_scale = std::pow(theta_base, -2.0f / (float) head_dim);
    for (int64_t p = 0; p < n_pos; ++p) {
        float theta = (float) p;
        for (int64_t i = 0; i < half; ++i) {
            cos_tab[p * half + i] = std::cos(theta);
            sin_tab[p * half + i] = std::sin(theta);
            theta *= theta_scale;
        }
    }
}

void orc_rope_neox(float * x, int64_t head_dim, const float * c, const float * s) {
    const int64_t half = head_dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float x0 = x[i], x1 = x[i + half];
        const float a = x0 * c[i], b = x1 * s[i];
        const float e = x0 * s[i], f = x1 * c[i];
        x[i] = a - b;
        x[i + half] = e + f;
    }
}

void orc_attention(const float * q, const uint16_t * k, const uint16_t * v,
                   int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_ctx,
                   int64_t n_kv, float * out, float * probs_out) {
    orc_attention_typed(q, k, v, n_head, n_kv_head, hd, n_ctx, n_kv, out, probs_out, 0);
}

// bf16: a BF16 cache.  ggml_mul_mat converts its F32 operand to the cache
// type's dot type, so q and P are rounded to bfloat16 instead of fp16; the
// products of two bfloat16 values (16 significant bits) stay exact in fp64.
void orc_attention_typed(const float * q, const uint16_t * k, const uint16_t * v,
                         int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_ctx,
                         int64_t n_kv, float * out, float * probs_out, int32_t bf16) {
    const float scale = 1.0f / std::sqrt((float) hd);
    const int64_t group = n_head / n_kv_head;
    std::vector<float> qh(hd), s(n_kv);
    std::vector<uint16_t> p16(n_kv);
    auto to_f = [bf16](uint16_t x) { return bf16 ? orc_bf16_to_f32(x) : h2f(x); };
    auto to_h = [bf16](float x) { return bf16 ? orc_f32_to_bf16(x) : orc_f32_to_f16(x); };
    for (int64_t h = 0; h < n_head; ++h) {
        const int64_t kvh = h / group;
        for (int64_t d = 0; d < hd; ++d) qh[d] = to_f(to_h(q[h * hd + d]));
        const uint16_t * kh = k + kvh * n_ctx * hd;
        const uint16_t * vh = v + kvh * n_ctx * hd;
        float mx = -INFINITY;
        for (int64_t j = 0; j < n_kv; ++j) {
            double acc = 0.0;
            for (int64_t d = 0; d < hd; ++d) acc += (double) qh[d] * (double) to_f(kh[j * hd + d]);
            s[j] = (float) acc * scale;
            mx = std::max(mx, s[j]);
        }
        double sum = 0.0;
        for (int64_t j = 0; j < n_kv; ++j) { s[j] = orc_expf(s[j] - mx); sum += (double) s[j]; }
        const float inv = (float) (1.0 / sum);
        for (int64_t j = 0; j < n_kv; ++j) {
            const float p = s[j] * inv;
            if (probs_out) probs_out[h * n_kv + j] = p;
            p16[j] = to_h(p);
        }
        for (int64_t d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (int64_t j = 0; j < n_kv; ++j) acc += (double) to_f(p16[j]) * (double) to_f(vh[j * hd + d]);
            out[h * hd + d] = (float) acc;
        }
    }
}

// The code predictor's 2-token prefill attends over its F32 Kcur/Vcur, not
// over the F16 cache (src/tts_transformer.cpp:1999-2012: K, V are permutes of
// Kcur/Vcur; an F32 src0 in ggml_mul_mat leaves q and P unrounded).  Every
// product of two fp32 values is exact in fp64; the score's 128-term sum is
// taken in one fixed order, four sequential 32-dim partials combined as
// (s0 + s1) + (s2 + s3), the order the device kernels use, so the fp64
// rounding of the sum is the same everywhere.  P.V adds the exact products in
// position order.  Rows j of k and v are at k + j * kv_stride + kvh * hd.
void orc_attention_f32(const float * q, const float * k, const float * v, int64_t kv_stride,
                       int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_kv, float * out) {
    const float scale = 1.0f / std::sqrt((float) hd);
    const int64_t group = n_head / n_kv_head, qtr = hd / 4;
    std::vector<float> s(n_kv);
    for (int64_t h = 0; h < n_head; ++h) {
        const int64_t kvh = h / group;
        const float * qh = q + h * hd;
        float mx = -INFINITY;
        for (int64_t j = 0; j < n_kv; ++j) {
            const float * kj = k + j * kv_stride + kvh * hd;
            double part[4];
            for (int c = 0; c < 4; ++c) {
                double acc = 0.0;
                for (int64_t d = c * qtr; d < (c + 1) * qtr; ++d) acc += (double) qh[d] * (double) kj[d];
                part[c] = acc;
            }
            s[j] = (float) ((part[0] + part[1]) + (part[2] + part[3])) * scale;
            mx = std::max(mx, s[j]);
        }
        double sum = 0.0;
        for (int64_t j = 0; j < n_kv; ++j) { s[j] = orc_expf(s[j] - mx); sum += (double) s[j]; }
        const float inv = (float) (1.0 / sum);
        for (int64_t j = 0; j < n_kv; ++j) s[j] = s[j] * inv;
        for (int64_t d = 0; d < hd; ++d) {
            double acc = 0.0;
            for (int64_t j = 0; j < n_kv; ++j) acc += (double) s[j] * (double) v[j * kv_stride + kvh * hd + d];
            out[h * hd + d] = (float) acc;
        }
    }
}

int32_t orc_argmax(const float * x, int32_t n) {
    int32_t best = 0;
    float bv = x[0];
    for (int32_t i = 1; i < n; ++i)
        if (x[i] > bv) { bv = x[i]; best = i; }
    return best;
}

void orc_philox4x32(uint64_t key, uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t out[4]) {
    uint32_t k0 = (uint32_t) key, k1 = (uint32_t) (key >> 32);
    uint32_t c[4] = {c0, c1, c2, c3};
    for (int r = 0; r < 10; ++r) {
        if (r) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        uint32_t hi0, lo0, hi1, lo1;
        mulhilo(0xD2511F53u, c[0], hi0, lo0);
        mulhilo(0xCD9E8D57u, c[2], hi1, lo1);
        const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
    }
    for (int i = 0; i < 4; ++i) out[i] = c[i];
}

double orc_uniform(uint64_t seed, uint32_t frame, uint32_t group) {
    uint32_t o[4];
    orc_philox4x32(seed, frame, group, 0u, 0u, o);
    return ((double) (o[0] >> 5) * 67108864.0 + (double) (o[1] >> 6)) * (1.0 / 9007199254740992.0);
}

int32_t orc_sample_cb0(float * logits, int32_t vocab, int32_t eos_id,
                       const uint8_t * seen, float rep_penalty, float temperature,
                       int32_t top_k, float eos_bias, int32_t target_frames,
                       int32_t frame, uint64_t seed) {
    for (int32_t i = vocab - 1024; i < vocab; ++i)
        if (i != eos_id) logits[i] = -INFINITY;
    if (rep_penalty != 1.0f && seen) {
        for (int32_t t = 0; t < vocab; ++t) {
            if (!seen[t]) continue;
            if (logits[t] > 0.0f) logits[t] /= rep_penalty;
            else logits[t] *= rep_penalty;
        }
    }
    float eff = eos_bias;
    if (target_frames > 0 && frame > target_frames) {
        eff += 0.1f * (float) (frame - target_frames);
        if (eff > 6.0f) eff = 6.0f;
    }
    if (temperature <= 0.0f) {
        if (eff != 0.0f) logits[eos_id] += eff;
        return orc_argmax(logits, vocab);
    }
    for (int32_t i = 0; i < vocab; ++i) logits[i] /= temperature;
    if (eff != 0.0f) logits[eos_id] += eff;
    return topk_softmax_draw(logits, vocab, top_k, orc_uniform(seed, (uint32_t) frame, 0u));
}

int32_t orc_sample_cp(float * logits, int32_t vocab, float temperature, int32_t top_k,
                      uint64_t seed, uint32_t frame, uint32_t group) {
    if (temperature <= 0.0f) return orc_argmax(logits, vocab);
    for (int32_t i = 0; i < vocab; ++i) logits[i] /= temperature;
    return topk_softmax_draw(logits, vocab, top_k, orc_uniform(seed, frame, group));
}

}  // extern "C"

// =========================================================== model
namespace {

struct Tensor {
    int32_t type = -1;
    const uint8_t * data = nullptr;
    size_t nbytes = 0;
    bool ok() const { return data != nullptr; }
};

struct Layer {
    Tensor attn_norm, q_norm, k_norm, wq, wk, wv, wo, ffn_norm, wg, wu, wd;
};

struct KV {
    std::vector<uint16_t> k, v;   // [layers][n_kv_head][n_ctx][hd], fp16 or (bf16) bfloat16 bits
    int32_t n_ctx = 0;
    int32_t bf16 = 0;
};

}  // namespace

struct orc_model {
    orc_config cfg;
    Pool pool{1};
    std::map<std::string, Tensor> tensors;
    std::vector<Layer> talker, cp;
    std::vector<Tensor> cp_embd, cp_head;
    Tensor text_embd, fc1, fc1_b, fc2, fc2_b, codec_embd, codec_head, out_norm, cp_out_norm;
    Tensor mtp_w, mtp_b;                          // code_pred.mtp_proj (only when cp_hidden != hidden_size)
    KV kv, cp_kv;
    std::vector<float> rope_cos, rope_sin;        // talker theta
    std::vector<float> cp_rope_cos, cp_rope_sin;  // code-predictor theta
    int32_t rope_rows = 0;
    std::vector<float> last_hidden;
    int32_t attn_layer = -1;                      // orc_set_attn_capture
    std::vector<std::vector<float>> attn_rows;    // [n_head][n_kv] per talker step
    std::string err;
};

namespace {

bool fail(orc_model * m, const std::string & e) { m->err = e; return false; }

void ensure_rope(orc_model * m, int32_t n_pos) {
    if (n_pos <= m->rope_rows) return;
    const int64_t half = m->cfg.head_dim / 2;
    m->rope_cos.resize((size_t) n_pos * half); m->rope_sin.resize((size_t) n_pos * half);
    m->cp_rope_cos.resize((size_t) n_pos * half); m->cp_rope_sin.resize((size_t) n_pos * half);
    orc_rope_table(m->cfg.rope_theta, m->cfg.head_dim, n_pos, m->rope_cos.data(), m->rope_sin.data());
    orc_rope_table(m->cfg.cp_rope_theta, m->cfg.head_dim, n_pos, m->cp_rope_cos.data(), m->cp_rope_sin.data());
    m->rope_rows = n_pos;
}

const float * fp(const Tensor & t) { return (const float *) t.data; }

void gemv_t(orc_model * m, const Tensor & w, int64_t rows, int64_t k, const float * x,
            int64_t ntok, float * y, bool is_down = false) {
    gemv_impl(&m->pool, w.type, w.data, rows, k, x, ntok, y, is_down ? 1 : 0);
}

// One transformer layer of width d over ntok consecutive positions starting at
// pos0.  f32_attn: the code predictor's prefill, whose attention reads the
// F32 rows of this call instead of the F16 cache (orc_attention_f32); the
// cache rows are written either way, for the steps that follow.
void layer_forward(orc_model * m, const Layer & L, int64_t d, int64_t ffn, float * x, int64_t ntok, int32_t pos0,
                   KV & kv, int32_t il, const float * rc, const float * rs, bool f32_attn = false,
                   float * probs = nullptr) {
    const orc_config & c = m->cfg;
    const int64_t hd = c.head_dim, nh = c.n_head, nkv = c.n_kv_head;
    const int64_t qd = nh * hd, kd = nkv * hd, half = hd / 2;
    std::vector<float> h(ntok * d), q(ntok * qd), k(ntok * kd), v(ntok * kd), o(ntok * qd), t(ntok * d);
    for (int64_t i = 0; i < ntok; ++i) orc_rmsnorm(x + i * d, fp(L.attn_norm), d, c.rms_eps, h.data() + i * d);
    gemv_t(m, L.wq, qd, d, h.data(), ntok, q.data());
    gemv_t(m, L.wk, kd, d, h.data(), ntok, k.data());
    gemv_t(m, L.wv, kd, d, h.data(), ntok, v.data());
    uint16_t * kc = kv.k.data() + (size_t) il * nkv * kv.n_ctx * hd;
    uint16_t * vc = kv.v.data() + (size_t) il * nkv * kv.n_ctx * hd;
    for (int64_t i = 0; i < ntok; ++i) {
        const int64_t pos = pos0 + i;
        for (int64_t hh = 0; hh < nh; ++hh) {
            float * qh = q.data() + i * qd + hh * hd;
            orc_rmsnorm(qh, fp(L.q_norm), hd, c.rms_eps, qh);
            orc_rope_neox(qh, hd, rc + pos * half, rs + pos * half);
        }
        for (int64_t hh = 0; hh < nkv; ++hh) {
            float * kh = k.data() + i * kd + hh * hd;
            orc_rmsnorm(kh, fp(L.k_norm), hd, c.rms_eps, kh);
            orc_rope_neox(kh, hd, rc + pos * half, rs + pos * half);
            for (int64_t e = 0; e < hd; ++e) {
                const float ve = v[i * kd + hh * hd + e];
                kc[(hh * kv.n_ctx + pos) * hd + e] = kv.bf16 ? orc_f32_to_bf16(kh[e]) : orc_f32_to_f16(kh[e]);
                vc[(hh * kv.n_ctx + pos) * hd + e] = kv.bf16 ? orc_f32_to_bf16(ve) : orc_f32_to_f16(ve);
            }
        }
    }
    if (f32_attn) {
        // causal over this call's rows only (the prefill starts at position 0)
        for (int64_t i = 0; i < ntok; ++i)
            orc_attention_f32(q.data() + i * qd, k.data(), v.data(), kd, nh, nkv, hd, i + 1, o.data() + i * qd);
    } else {
        m->pool.run(ntok, [&](int64_t i0, int64_t i1) {
            for (int64_t i = i0; i < i1; ++i)
                orc_attention_typed(q.data() + i * qd, kc, vc, nh, nkv, hd, kv.n_ctx, pos0 + i + 1,
                                    o.data() + i * qd, ntok == 1 ? probs : nullptr, kv.bf16);
        });
    }
    gemv_t(m, L.wo, d, qd, o.data(), ntok, t.data());
    for (int64_t i = 0; i < ntok * d; ++i) x[i] = t[i] + x[i];
    for (int64_t i = 0; i < ntok; ++i) orc_rmsnorm(x + i * d, fp(L.ffn_norm), d, c.rms_eps, h.data() + i * d);
    std::vector<float> g(ntok * ffn), u(ntok * ffn);
    gemv_t(m, L.wg, ffn, d, h.data(), ntok, g.data());
    gemv_t(m, L.wu, ffn, d, h.data(), ntok, u.data());
    for (int64_t i = 0; i < ntok * ffn; ++i) g[i] = silu(g[i]) * u[i];
    gemv_t(m, L.wd, d, ffn, g.data(), ntok, t.data(), true);
    for (int64_t i = 0; i < ntok * d; ++i) x[i] = t[i] + x[i];
}

// One block of the single-pass code predictor: one row, one position, no
// cache (src/tts_transformer.cpp:1823-1890).  Its attention is softmax over a
// single score, which is exactly 1, times that row's fp32 V: query head h
// gets V of KV head h / group (ggml_mul_mat broadcasts the KV heads over the
// query heads, :1855-1864).  Q, K, their norms and the score do not reach the
// output, so they are not computed.
void layer_single(orc_model * m, const Layer & L, int64_t d, int64_t ffn, float * x) {
    const orc_config & c = m->cfg;
    const int64_t hd = c.head_dim, nh = c.n_head, nkv = c.n_kv_head;
    const int64_t qd = nh * hd, kd = nkv * hd, group = nh / nkv;
    std::vector<float> h(d), v(kd), o(qd), t(d), g(ffn), u(ffn);
    orc_rmsnorm(x, fp(L.attn_norm), d, c.rms_eps, h.data());
    gemv_t(m, L.wv, kd, d, h.data(), 1, v.data());
    for (int64_t hh = 0; hh < nh; ++hh)
        for (int64_t e = 0; e < hd; ++e) o[hh * hd + e] = v[(hh / group) * hd + e];
    gemv_t(m, L.wo, d, qd, o.data(), 1, t.data());
    for (int64_t i = 0; i < d; ++i) x[i] = t[i] + x[i];
    orc_rmsnorm(x, fp(L.ffn_norm), d, c.rms_eps, h.data());
    gemv_t(m, L.wg, ffn, d, h.data(), 1, g.data());
    gemv_t(m, L.wu, ffn, d, h.data(), 1, u.data());
    for (int64_t i = 0; i < ffn; ++i) g[i] = silu(g[i]) * u[i];
    gemv_t(m, L.wd, d, ffn, g.data(), 1, t.data(), true);
    for (int64_t i = 0; i < d; ++i) x[i] = t[i] + x[i];
}

bool resolve(orc_model * m) {
    const orc_config & c = m->cfg;
    auto get = [&](const std::string & n, Tensor & dst) -> bool {
        auto it = m->tensors.find(n);
        if (it == m->tensors.end()) return fail(m, "missing tensor " + n);
        dst = it->second;
        return true;
    };
    auto layer = [&](const std::string & p, Layer & L) -> bool {
        return get(p + "attn_norm.weight", L.attn_norm) && get(p + "attn_q_norm.weight", L.q_norm) &&
               get(p + "attn_k_norm.weight", L.k_norm) && get(p + "attn_q.weight", L.wq) &&
               get(p + "attn_k.weight", L.wk) && get(p + "attn_v.weight", L.wv) &&
               get(p + "attn_output.weight", L.wo) && get(p + "ffn_norm.weight", L.ffn_norm) &&
               get(p + "ffn_gate.weight", L.wg) && get(p + "ffn_up.weight", L.wu) &&
               get(p + "ffn_down.weight", L.wd);
    };
    m->talker.assign(c.n_layers, Layer());
    m->cp.assign(c.cp_layers, Layer());
    m->cp_embd.assign(c.n_codebooks - 1, Tensor());
    m->cp_head.assign(c.n_codebooks - 1, Tensor());
    for (int i = 0; i < c.n_layers; ++i)
        if (!layer("talker.blk." + std::to_string(i) + ".", m->talker[i])) return false;
    for (int i = 0; i < c.cp_layers; ++i)
        if (!layer("code_pred.blk." + std::to_string(i) + ".", m->cp[i])) return false;
    for (int g = 0; g < c.n_codebooks - 1; ++g) {
        if (!get("code_pred.codec_embd." + std::to_string(g) + ".weight", m->cp_embd[g])) return false;
        if (!get("code_pred.lm_head." + std::to_string(g) + ".weight", m->cp_head[g])) return false;
    }
    if (c.cp_hidden != c.hidden_size &&
        !(get("code_pred.mtp_proj.weight", m->mtp_w) && get("code_pred.mtp_proj.bias", m->mtp_b)))
        return false;
    return get("talker.codec_embd.weight", m->codec_embd) && get("talker.codec_head.weight", m->codec_head) &&
           get("talker.output_norm.weight", m->out_norm) && get("code_pred.output_norm.weight", m->cp_out_norm) &&
           get("talker.text_embd.weight", m->text_embd) && get("talker.text_proj.fc1.weight", m->fc1) &&
           get("talker.text_proj.fc1.bias", m->fc1_b) && get("talker.text_proj.fc2.weight", m->fc2) &&
           get("talker.text_proj.fc2.bias", m->fc2_b);
}

void embd_row(const Tensor & t, int64_t dim, int32_t tok, float * out) {
    if (t.type == ORC_TYPE_F16) {
        const uint16_t * r = (const uint16_t *) t.data + (size_t) tok * dim;
        for (int64_t i = 0; i < dim; ++i) out[i] = h2f(r[i]);
    } else {
        std::memcpy(out, (const float *) t.data + (size_t) tok * dim, dim * sizeof(float));
    }
}

// step: forward_step, which keeps the attention row of the capture layer
// (src/tts_transformer.cpp:1719-1724, :2485-2497); forward_prefill keeps none.
bool talker_forward(orc_model * m, const float * embd, int32_t n, int32_t n_past,
                    float * hidden_out, float * logits_out, bool step = false) {
    const orc_config & c = m->cfg;
    if (m->talker.empty() && !resolve(m)) return false;
    if (n_past + n > m->kv.n_ctx) return fail(m, "Context length exceeded");
    ensure_rope(m, m->kv.n_ctx);
    const int64_t d = c.hidden_size;
    std::vector<float> x(embd, embd + (size_t) n * d);
    std::vector<float> probs;
    if (step && m->attn_layer >= 0) probs.resize((size_t) c.n_head * (n_past + 1));
    for (int il = 0; il < c.n_layers; ++il)
        layer_forward(m, m->talker[il], d, c.ffn_size, x.data(), n, n_past, m->kv, il, m->rope_cos.data(),
                      m->rope_sin.data(), false, il == m->attn_layer && !probs.empty() ? probs.data() : nullptr);
    if (!probs.empty()) m->attn_rows.push_back(std::move(probs));
    std::vector<float> hid((size_t) n * d);
    for (int32_t i = 0; i < n; ++i) orc_rmsnorm(x.data() + i * d, fp(m->out_norm), d, c.rms_eps, hid.data() + i * d);
    if (hidden_out) std::memcpy(hidden_out, hid.data(), hid.size() * sizeof(float));
    m->last_hidden.assign(hid.end() - d, hid.end());
    if (logits_out) gemv_t(m, m->codec_head, c.codec_vocab, d, hid.data() + (size_t) (n - 1) * d, 1, logits_out);
    return true;
}

}  // namespace

extern "C" {

orc_model * orc_create(const orc_config * cfg) {
    orc_model * m = new orc_model();
    m->cfg = *cfg;
    return m;
}

void orc_destroy(orc_model * m) { delete m; }

void orc_set_threads(orc_model * m, int32_t n) { m->pool.resize(n); }

int orc_set_tensor(orc_model * m, const char * name, int32_t type, const void * data, size_t nbytes) {
    Tensor t;
    t.type = type; t.data = (const uint8_t *) data; t.nbytes = nbytes;
    m->tensors[name] = t;
    m->talker.clear();
    return 0;
}

int orc_check_complete(orc_model * m) { return resolve(m) ? 0 : -1; }

const char * orc_last_error(const orc_model * m) { return m->err.c_str(); }

int orc_kv_reset(orc_model * m, int32_t n_ctx) {
    const orc_config & c = m->cfg;
    m->kv.n_ctx = n_ctx;
    m->kv.k.assign((size_t) c.n_layers * c.n_kv_head * n_ctx * c.head_dim, 0);
    m->kv.v.assign(m->kv.k.size(), 0);
    m->cp_kv.n_ctx = 16;
    m->cp_kv.k.assign((size_t) c.cp_layers * c.n_kv_head * 16 * c.head_dim, 0);
    m->cp_kv.v.assign(m->cp_kv.k.size(), 0);
    ensure_rope(m, std::max(n_ctx, 16));
    return 0;
}

int orc_kv_set_type(orc_model * m, int32_t type) {
    if (type != 1 && type != 30) { m->err = "talker KV type must be F16 (1) or BF16 (30)"; return -1; }
    m->kv.bf16 = type == 30;
    return 0;
}

int orc_kv_write(orc_model * m, int32_t layer, int32_t n_pos, const uint16_t * k, const uint16_t * v) {
    const orc_config & c = m->cfg;
    if (layer < 0 || layer >= c.n_layers || n_pos < 0 || n_pos > m->kv.n_ctx) {
        m->err = "kv_write: layer or position range outside the cache";
        return -1;
    }
    const int64_t hd = c.head_dim, nkv = c.n_kv_head;
    uint16_t * kc = m->kv.k.data() + (size_t) layer * nkv * m->kv.n_ctx * hd;
    uint16_t * vc = m->kv.v.data() + (size_t) layer * nkv * m->kv.n_ctx * hd;
    for (int64_t p = 0; p < n_pos; ++p)
        for (int64_t h = 0; h < nkv; ++h) {
            std::memcpy(kc + (h * m->kv.n_ctx + p) * hd, k + (p * nkv + h) * hd, hd * sizeof(uint16_t));
            std::memcpy(vc + (h * m->kv.n_ctx + p) * hd, v + (p * nkv + h) * hd, hd * sizeof(uint16_t));
        }
    return 0;
}

int orc_kv_read(orc_model * m, int32_t layer, int32_t n_pos, uint16_t * k, uint16_t * v) {
    const orc_config & c = m->cfg;
    if (layer < 0 || layer >= c.n_layers || n_pos < 0 || n_pos > m->kv.n_ctx) {
        m->err = "kv_read: layer or position range outside the cache";
        return -1;
    }
    const int64_t hd = c.head_dim, nkv = c.n_kv_head;
    const uint16_t * kc = m->kv.k.data() + (size_t) layer * nkv * m->kv.n_ctx * hd;
    const uint16_t * vc = m->kv.v.data() + (size_t) layer * nkv * m->kv.n_ctx * hd;
    for (int64_t p = 0; p < n_pos; ++p)
        for (int64_t h = 0; h < nkv; ++h) {
            std::memcpy(k + (p * nkv + h) * hd, kc + (h * m->kv.n_ctx + p) * hd, hd * sizeof(uint16_t));
            std::memcpy(v + (p * nkv + h) * hd, vc + (h * m->kv.n_ctx + p) * hd, hd * sizeof(uint16_t));
        }
    return 0;
}

int orc_prefill(orc_model * m, const float * embd, int32_t n, int32_t n_past,
                float * hidden_out, float * logits_out) {
    return talker_forward(m, embd, n, n_past, hidden_out, logits_out) ? 0 : -1;
}

int orc_step(orc_model * m, const float * embd, int32_t n_past, float * logits_out, float * hidden_out) {
    return talker_forward(m, embd, 1, n_past, hidden_out, logits_out, true) ? 0 : -1;
}

int orc_set_attn_capture(orc_model * m, int32_t layer) {
    if (layer < -1 || layer >= m->cfg.n_layers) { m->err = "attention capture layer out of range"; return -1; }
    m->attn_layer = layer;
    m->attn_rows.clear();
    return 0;
}

int32_t orc_attn_row_count(const orc_model * m) { return (int32_t) m->attn_rows.size(); }

int32_t orc_attn_row(const orc_model * m, int32_t index, float * out, int64_t cap) {
    if (index < 0 || index >= (int32_t) m->attn_rows.size()) return -1;
    const std::vector<float> & r = m->attn_rows[(size_t) index];
    if (out && cap >= (int64_t) r.size()) std::memcpy(out, r.data(), r.size() * sizeof(float));
    return (int32_t) (r.size() / (size_t) m->cfg.n_head);
}

int orc_code_pred(orc_model * m, const float * hidden, int32_t cb0,
                  float temperature, int32_t top_k, uint64_t seed, uint32_t frame,
                  int32_t * codes_out, float * logits_out) {
    const orc_config & c = m->cfg;
    if (m->talker.empty() && !resolve(m)) return -1;
    if (m->cp_kv.n_ctx < 16) {
        m->cp_kv.n_ctx = 16;
        m->cp_kv.k.assign((size_t) c.cp_layers * c.n_kv_head * 16 * c.head_dim, 0);
        m->cp_kv.v.assign(m->cp_kv.k.size(), 0);
    }
    ensure_rope(m, 16);
    // the inputs are talker-width rows (hidden, codec / code-predictor
    // embeddings); the MTP projection, when present, maps them to the code
    // predictor's width (src/tts_transformer.cpp:1942-1947, :2096-2101)
    const int64_t d = c.hidden_size, dc = c.cp_hidden;
    const bool mtp = dc != d;
    const int32_t V = c.cp_vocab;
    const int ng = c.n_codebooks - 1;
    if (cb0 < 0 || cb0 >= c.codec_vocab) { m->err = "Embedding token ID out of range"; return -1; }
    std::vector<float> in(2 * d), x(2 * dc), hid(dc), logits(V);
    auto project = [&](const float * rows, int64_t n, float * out) {
        if (!mtp) { std::memcpy(out, rows, (size_t) n * d * sizeof(float)); return; }
        gemv_t(m, m->mtp_w, dc, d, rows, n, out);
        for (int64_t i = 0; i < n; ++i)
            for (int64_t j = 0; j < dc; ++j) out[i * dc + j] = out[i * dc + j] + fp(m->mtp_b)[j];
    };
    std::memcpy(in.data(), hidden, d * sizeof(float));
    embd_row(m->codec_embd, d, cb0, in.data() + d);
    project(in.data(), 2, x.data());
    for (int il = 0; il < c.cp_layers; ++il)
        layer_forward(m, m->cp[il], dc, c.cp_ffn, x.data(), 2, 0, m->cp_kv, il, m->cp_rope_cos.data(),
                      m->cp_rope_sin.data(), true);
    orc_rmsnorm(x.data() + dc, fp(m->cp_out_norm), dc, c.rms_eps, hid.data());
    gemv_t(m, m->cp_head[0], V, dc, hid.data(), 1, logits.data());
    if (logits_out) std::memcpy(logits_out, logits.data(), V * sizeof(float));
    codes_out[0] = orc_sample_cp(logits.data(), V, temperature, top_k, seed, frame, 1);
    for (int s = 1; s < ng; ++s) {
        if (codes_out[s - 1] < 0 || codes_out[s - 1] >= V) { m->err = "Embedding token ID out of range"; return -1; }
        embd_row(m->cp_embd[s - 1], d, codes_out[s - 1], in.data());
        project(in.data(), 1, x.data());
        for (int il = 0; il < c.cp_layers; ++il)
            layer_forward(m, m->cp[il], dc, c.cp_ffn, x.data(), 1, s + 1, m->cp_kv, il, m->cp_rope_cos.data(),
                          m->cp_rope_sin.data());
        orc_rmsnorm(x.data(), fp(m->cp_out_norm), dc, c.rms_eps, hid.data());
        gemv_t(m, m->cp_head[s], V, dc, hid.data(), 1, logits.data());
        if (logits_out) std::memcpy(logits_out + (size_t) s * V, logits.data(), V * sizeof(float));
        codes_out[s] = orc_sample_cp(logits.data(), V, temperature, top_k, seed, frame, (uint32_t) (s + 1));
    }
    return 0;
}

int orc_predict_codes(orc_model * m, const float * hidden, const int32_t * prev_codes, float * logits_out) {
    const orc_config & c = m->cfg;
    if (m->talker.empty() && !resolve(m)) return -1;
    const int64_t d = c.hidden_size, dc = c.cp_hidden;
    const int ng = c.n_codebooks - 1;
    // hidden + code_pred.codec_embd[g][prev_codes[g]], added in codebook
    // order in fp32 (:1801-1808)
    std::vector<float> in(hidden, hidden + d), e(d), x(dc);
    for (int g = 0; prev_codes && g < ng; ++g) {
        if (prev_codes[g] < 0 || prev_codes[g] >= c.cp_vocab) { m->err = "Embedding token ID out of range"; return -1; }
        embd_row(m->cp_embd[g], d, prev_codes[g], e.data());
        for (int64_t i = 0; i < d; ++i) in[i] = in[i] + e[i];
    }
    // the MTP projection (:1811-1816); identity in the 0.6B layout
    if (dc != d) {
        gemv_t(m, m->mtp_w, dc, d, in.data(), 1, x.data());
        for (int64_t j = 0; j < dc; ++j) x[j] = x[j] + fp(m->mtp_b)[j];
    } else {
        x = in;
    }
    for (int il = 0; il < c.cp_layers; ++il) layer_single(m, m->cp[il], dc, c.cp_ffn, x.data());
    // the heads read the last layer's row as it is: no output norm (:1881-1888)
    for (int g = 0; g < ng; ++g) gemv_t(m, m->cp_head[g], c.cp_vocab, dc, x.data(), 1, logits_out + (size_t) g * c.cp_vocab);
    return 0;
}

int orc_text_proj(orc_model * m, const int32_t * tokens, int32_t n, float * out) {
    const orc_config & c = m->cfg;
    if (m->talker.empty() && !resolve(m)) return -1;
    const int64_t te = c.text_embd_dim, d = c.hidden_size;
    std::vector<float> e((size_t) n * te), h((size_t) n * te);
    for (int32_t i = 0; i < n; ++i) {
        if (tokens[i] < 0 || tokens[i] >= c.text_vocab) { m->err = "Embedding token ID out of range"; return -1; }
        embd_row(m->text_embd, te, tokens[i], e.data() + (size_t) i * te);
    }
    gemv_t(m, m->fc1, te, te, e.data(), n, h.data());
    for (int32_t i = 0; i < n; ++i)
        for (int64_t j = 0; j < te; ++j) h[i * te + j] = silu(h[i * te + j] + fp(m->fc1_b)[j]);
    gemv_t(m, m->fc2, d, te, h.data(), n, out);
    for (int32_t i = 0; i < n; ++i)
        for (int64_t j = 0; j < d; ++j) out[i * d + j] = out[i * d + j] + fp(m->fc2_b)[j];
    return 0;
}

int orc_embed_row(orc_model * m, const char * table, int32_t index, int32_t token, float * out) {
    if (m->talker.empty() && !resolve(m)) return -1;
    const orc_config & c = m->cfg;
    if (!std::strcmp(table, "codec")) {
        if (token < 0 || token >= c.codec_vocab) return -1;
        embd_row(m->codec_embd, c.hidden_size, token, out);
    } else if (!std::strcmp(table, "cp")) {
        if (token < 0 || token >= c.cp_vocab || index < 0 || index >= c.n_codebooks - 1) return -1;
        embd_row(m->cp_embd[index], c.hidden_size, token, out);
    } else {
        if (token < 0 || token >= c.text_vocab) return -1;
        embd_row(m->text_embd, c.text_embd_dim, token, out);
    }
    return 0;
}

int orc_build_prefill(orc_model * m, const int32_t * text, int32_t n_text,
                      const float * speaker, int32_t language_id,
                      const int32_t * instruct, int32_t n_instruct,
                      float * prefill_out, float * trailing_out, float * pad_out,
                      int32_t * trailing_len_out) {
    const orc_config & c = m->cfg;
    const int64_t d = c.hidden_size;
    if (!text || n_text < 4) { m->err = "Need at least 4 text tokens for prefill"; return -1; }
    int32_t special[3] = {c.tts_bos_id, c.tts_eos_id, c.tts_pad_id};
    std::vector<float> sp(3 * d), role(3 * d), first(d);
    if (orc_text_proj(m, special, 3, sp.data()) || orc_text_proj(m, text, 3, role.data())) return -1;
    const float * bos_e = sp.data(), * eos_e = sp.data() + d, * pad_e = sp.data() + 2 * d;
    std::vector<int32_t> codec_tok;
    if (language_id < 0) codec_tok = {c.codec_nothink_id, c.codec_think_bos_id, c.codec_think_eos_id};
    else codec_tok = {c.codec_think_id, c.codec_think_bos_id, language_id, c.codec_think_eos_id};
    const bool has_spk = speaker != nullptr;
    const int32_t in_len = (int32_t) codec_tok.size() + (has_spk ? 1 : 0) + 2;
    std::vector<float> cin((size_t) in_len * d);
    int32_t row = 0;
    for (int32_t t : codec_tok) {
        if (t < 0 || t >= c.codec_vocab) { m->err = "Embedding token ID out of range"; return -1; }
        embd_row(m->codec_embd, d, t, cin.data() + (size_t) row++ * d);
    }
    if (has_spk) std::memcpy(cin.data() + (size_t) row++ * d, speaker, d * sizeof(float));
    embd_row(m->codec_embd, d, c.codec_pad_id, cin.data() + (size_t) row++ * d);
    embd_row(m->codec_embd, d, c.codec_bos_id, cin.data() + (size_t) row++ * d);
    const int32_t ov_len = in_len - 1;
    if (orc_text_proj(m, text + 3, 1, first.data())) return -1;
    std::vector<float> instr;
    if (instruct && n_instruct > 0) {
        instr.resize((size_t) n_instruct * d);
        if (orc_text_proj(m, instruct, n_instruct, instr.data())) return -1;
    } else {
        n_instruct = 0;
    }
    const int32_t plen = n_instruct + 3 + ov_len + 1;
    float * o = prefill_out;
    if (n_instruct) std::memcpy(o, instr.data(), instr.size() * sizeof(float));
    std::memcpy(o + (size_t) n_instruct * d, role.data(), role.size() * sizeof(float));
    for (int32_t t = 0; t < ov_len; ++t) {
        const float * ovl = (t == ov_len - 1) ? bos_e : pad_e;
        float * dst = o + (size_t) (n_instruct + 3 + t) * d;
        for (int64_t h = 0; h < d; ++h) dst[h] = ovl[h] + cin[(size_t) t * d + h];
    }
    float * last = o + (size_t) (plen - 1) * d;
    for (int64_t h = 0; h < d; ++h) last[h] = first[h] + cin[(size_t) (in_len - 1) * d + h];
    const int32_t n_trail = std::max(0, n_text - 9);
    if (n_trail > 0 && orc_text_proj(m, text + 4, n_trail, trailing_out)) return -1;
    std::memcpy(trailing_out + (size_t) n_trail * d, eos_e, d * sizeof(float));
    std::memcpy(pad_out, pad_e, d * sizeof(float));
    *trailing_len_out = n_trail + 1;
    return plen;
}

int orc_generate_rows(orc_model * m, const float * pre, int32_t plen, const float * trail, int32_t trail_len,
                      const float * pad, const orc_gen_params * p, int32_t * codes_out, float * first_logits_out);
int orc_frames(orc_model * m, const float * first_logits, int32_t n_past, const float * trail, int32_t trail_len,
               const float * pad_row, const orc_gen_params * p, int32_t * codes_out, float * frame_logits_out);

int orc_generate(orc_model * m, const int32_t * text, int32_t n_text,
                 const float * speaker, const orc_gen_params * p,
                 const int32_t * instruct, int32_t n_instruct,
                 int32_t * codes_out, float * first_logits_out) {
    const orc_config & c = m->cfg;
    if (n_text < 4) { m->err = "Need at least 4 text tokens for generation"; return -1; }
    if (p->max_len <= 0) return 0;
    const int64_t d = c.hidden_size;
    std::vector<float> pre((size_t) (std::max(0, n_instruct) + 10) * d);
    std::vector<float> trail((size_t) (std::max(0, n_text - 9) + 1) * d), pad(d);
    int32_t trail_len = 0;
    const int32_t plen = orc_build_prefill(m, text, n_text, speaker, p->language_id, instruct, n_instruct,
                                           pre.data(), trail.data(), pad.data(), &trail_len);
    if (plen < 0) return -1;
    return orc_generate_rows(m, pre.data(), plen, trail.data(), trail_len, pad.data(), p, codes_out, first_logits_out);
}

// generate() from prebuilt prefill rows (src/tts_transformer.cpp:3061-3309;
// generate_icl shares the loop, :3425-3640).
int orc_generate_rows(orc_model * m, const float * pre, int32_t plen, const float * trail, int32_t trail_len,
                      const float * pad_row, const orc_gen_params * p, int32_t * codes_out, float * first_logits_out) {
    const orc_config & c = m->cfg;
    if (p->max_len <= 0) return 0;
    orc_kv_reset(m, plen + p->max_len + 8);
    std::vector<float> logits(c.codec_vocab);
    if (orc_prefill(m, pre, plen, 0, nullptr, logits.data())) return -1;
    if (first_logits_out) std::memcpy(first_logits_out, logits.data(), logits.size() * sizeof(float));
    return orc_frames(m, logits.data(), plen, trail, trail_len, pad_row, p, codes_out, nullptr);
}

// The frame loop of generate() (src/tts_transformer.cpp:3108-3309) from the
// current talker cache: `first_logits` and the normed hidden row left by the
// last prefill or step, the next talker position n_past.
int orc_frames(orc_model * m, const float * first_logits, int32_t n_past, const float * trail, int32_t trail_len,
               const float * pad_row, const orc_gen_params * p, int32_t * codes_out, float * frame_logits_out) {
    const orc_config & c = m->cfg;
    if (p->max_len <= 0) return 0;
    if (m->last_hidden.size() != (size_t) c.hidden_size) { m->err = "frames: no prefill or step has run"; return -1; }
    if (n_past + p->max_len > m->kv.n_ctx) { m->err = "Context length exceeded"; return -1; }
    const int64_t d = c.hidden_size;
    const int32_t ncb = c.n_codebooks;
    std::vector<float> pad(pad_row, pad_row + d);
    std::vector<float> logits(first_logits, first_logits + c.codec_vocab);
    std::vector<uint8_t> seen(c.codec_vocab, 0);
    std::vector<int32_t> frame_codes(ncb), cps(ncb - 1);
    std::vector<std::vector<int32_t>> rep_frames;
    int32_t rep_run_len = 0, rep_run_start = 0;
    int32_t n_frames = 0;
    std::vector<float> step(d), row(d);
    for (int32_t frame = 0; frame < p->max_len; ++frame) {
        if (frame_logits_out)
            std::memcpy(frame_logits_out + (size_t) frame * c.codec_vocab, logits.data(), logits.size() * sizeof(float));
        const int32_t tok = orc_sample_cb0(logits.data(), c.codec_vocab, c.codec_eos_id, seen.data(),
                                           p->repetition_penalty, p->temperature, p->top_k, p->eos_bias,
                                           p->target_frames, frame, p->seed);
        if (tok == c.codec_eos_id) break;
        frame_codes[0] = tok;
        seen[tok] = 1;
        if (orc_code_pred(m, m->last_hidden.data(), tok, p->temperature, p->top_k, p->seed,
                          (uint32_t) frame, cps.data(), nullptr)) return -1;
        for (int g = 1; g < ncb; ++g) frame_codes[g] = cps[g - 1];
        std::memcpy(codes_out + (size_t) n_frames * ncb, frame_codes.data(), ncb * sizeof(int32_t));
        ++n_frames;
        if (p->rep_loop_detect) rep_frames.push_back(frame_codes);
        {
            const size_t nf = rep_frames.size();
            bool is_rep = false;
            for (int back = 1; back <= 6 && !is_rep && (size_t) back < nf; ++back) {
                int matches = 0;
                for (int g = 0; g < ncb; ++g) matches += rep_frames[nf - 1][g] == rep_frames[nf - 1 - back][g];
                if (matches >= 10) is_rep = true;
            }
            if (is_rep) { if (rep_run_len == 0) rep_run_start = (int32_t) (nf - 1); ++rep_run_len; }
            else rep_run_len = 0;
            if (rep_run_len >= 5) { n_frames = rep_run_start; break; }
        }
        if (frame + 1 >= p->max_len) break;
        embd_row(m->codec_embd, d, frame_codes[0], step.data());
        for (int g = 1; g < ncb; ++g) {
            embd_row(m->cp_embd[g - 1], d, frame_codes[g], row.data());
            for (int64_t h = 0; h < d; ++h) step[h] += row[h];
        }
        const float * tr = frame < trail_len ? trail + (size_t) frame * d : pad.data();
        for (int64_t h = 0; h < d; ++h) step[h] += tr[h];
        if (orc_step(m, step.data(), n_past, logits.data(), nullptr)) return -1;
        ++n_past;
    }
    return n_frames;
}

}  // extern "C"
