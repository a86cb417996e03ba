/*
 * q3t_oracle.h -- CPU restatement of the qwen3-tts.cpp per-frame token loop.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path and the timed CPU baseline.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it.  Nothing in the shipped library
 * (qwen3-tts.cpp_amd/) links, loads or calls it.
 *
 * What it restates (reference paths relative to the reference checkout):
 *   talker decode step          src/tts_transformer.cpp:1619-1769 (build_step_graph)
 *   n-token prefill             src/tts_transformer.cpp:1474-1617 (build_prefill_forward_graph)
 *   code-predictor prefill      src/tts_transformer.cpp:1901-2053
 *   code-predictor step         src/tts_transformer.cpp:2055-2215
 *   code-predictor loop/sampler src/tts_transformer.cpp:2711-2976 (sample_or_argmax :2750-2788)
 *   argmax                      src/tts_transformer.cpp:2583-2593
 *   generate() frame loop       src/tts_transformer.cpp:3007-3309
 *   text projection             src/tts_transformer.cpp:963-1028
 *   prefill layout              src/tts_transformer.cpp:1030-1186
 *
 * Numerics contract (the ggml kernels the reference calls are not in the
 * reference checkout; their semantics are restated from upstream ggml):
 *   - activations are fp32;
 *   - Q8_0 weight x fp32 activation: the activation row is quantised per
 *     32-block as ggml-cpu's x86 quantize_row_q8_0 does (d = amax/127 stored
 *     as fp16, q = round-to-nearest-even(x * (127/amax))), block dot products
 *     are exact int32, combined as fp16(d_w)*fp16(d_x)*isum;
 *   - F16 weight x fp32 activation: the activation is rounded to fp16 (RNE);
 *   - F16 ffn_down is widened to fp32 (ggml_cast) so its activation is NOT
 *     rounded (src/tts_transformer.cpp:1746-1748);
 *   - attention over the F16 KV cache rounds q and P to fp16 (F16 src0 in
 *     ggml_mul_mat); the code predictor's 2-token prefill instead attends
 *     over its F32 Kcur/Vcur (src/tts_transformer.cpp:1999-2012), so q, K, V
 *     and P stay fp32 there (orc_attention_f32); it still writes the F16
 *     cache rows the 14 steps read;
 *   - every dot product / sum of squares / softmax denominator accumulates its
 *     (exact) terms in fp64 and rounds to fp32 once.  ggml accumulates in
 *     fp32 SIMD lanes in an order that cannot be reproduced here; fp64
 *     accumulation is at least as accurate and makes the rounded result
 *     independent of summation order, which is what lets a GPU reduction
 *     match this restatement bit for bit;
 *   - exp() is q3t_orc_expf: Cody-Waite range reduction plus a degree-7
 *     Taylor polynomial (Horner with fused multiply-add), flushed to zero
 *     below -87; ggml uses its own SIMD exp approximation;
 *   - RoPE cos/sin come from a table built with the C library's cosf/sinf on
 *     theta_i = pos * base^(-2i/128) formed by cumulative fp32 product
 *     (ggml_rope_cache_init);
 *   - sampling (temperature > 0) uses Philox4x32-10 (Salmon et al., SC'11)
 *     keyed by a caller seed instead of std::mt19937/discrete_distribution,
 *     which cannot be reproduced on a GPU: distributional parity only with
 *     the reference, exact parity with the HIP path.
 *
 * Pinning status (tests/test_oracle.py, tests/test_oracle_model.py): every
 * function here is checked against closed forms, fp64 brute force, the
 * reference's fixture reference/det_prefill_token_types.json, known-answer
 * vectors (Philox), self-consistency (prefill == sequential steps) or an
 * independent float64 numpy forward written from the reference graphs; the
 * frame loop (orc_frames / orc_generate_rows: the greedy codebook-0 rules,
 * the code predictor fed the normed hidden row, the step-embedding order and
 * trailing-row index, the EOS ramp) against a numpy loop written from
 * src/tts_transformer.cpp:3108-3309, with planted loop mistakes that miss.
 * What ggml's own CPU build
 * would decide differently is NOT pinned, because ggml is absent (empty
 * submodule) and the reference's det_*.bin fixtures are absent:
 *   orc_gemv            parity unpinned vs ggml's fp32 SIMD accumulation order
 *   orc_quantize_q8_0_act  parity unpinned vs ggml's build (formula as published)
 *   orc_expf / softmax / SiLU  parity unpinned vs ggml's exp approximation
 *   orc_rope_table      parity unpinned vs ggml_rope_cache_init's recurrence
 *   orc_sample_cb0 / orc_sample_cp (temperature > 0)  distributional parity only
 */
#ifndef Q3T_ORACLE_H
#define Q3T_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (ggml.h enum ggml_type) */
#define ORC_TYPE_F32  0
#define ORC_TYPE_F16  1
#define ORC_TYPE_Q8_0 8

typedef struct orc_config {
    int32_t hidden_size;
    int32_t n_layers;
    int32_t n_head;
    int32_t n_kv_head;
    int32_t head_dim;
    int32_t ffn_size;
    int32_t codec_vocab;
    int32_t n_codebooks;
    int32_t cp_layers;
    int32_t cp_vocab;
    int32_t cp_hidden;
    int32_t cp_ffn;
    int32_t text_vocab;
    int32_t text_embd_dim;
    float   rms_eps;
    float   rope_theta;
    float   cp_rope_theta;
    int32_t codec_pad_id, codec_bos_id, codec_eos_id;
    int32_t tts_bos_id, tts_eos_id, tts_pad_id;
    int32_t codec_think_id, codec_nothink_id, codec_think_bos_id, codec_think_eos_id;
    int32_t english_language_id;
} orc_config;

typedef struct orc_gen_params {
    int32_t max_len;
    int32_t language_id;
    float   repetition_penalty;
    float   temperature;
    int32_t top_k;
    float   eos_bias;
    int32_t target_frames;
    int32_t rep_loop_detect;
    uint64_t seed;
} orc_gen_params;

typedef struct orc_model orc_model;

/* ---- elementwise / kernel-level restatements (unit-test surface) ---- */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
float    orc_expf(float x);
/* converter weight quantisation (scripts/convert_tts_to_gguf.py:304-307 via
 * gguf-py quants): d = amax/127, q = round-half-away(x/d).  out: n/32 blocks
 * of 34 bytes (fp16 d, 32 x int8). */
void orc_quantize_q8_0_weights(const float * x, int64_t n, uint8_t * out);
/* ggml-cpu x86 activation quantisation; out as above. */
void orc_quantize_q8_0_act(const float * x, int64_t n, uint8_t * out);
void orc_dequantize_q8_0(const uint8_t * blocks, int64_t n, float * out);
/* y[t][r] = W[r,:] . x[t][:]; type selects the reference numerics.
 * widen_f16 = 1 selects the F16-as-F32 (ffn_down cast) path. */
void orc_gemv(int type, const void * w, int64_t rows, int64_t k,
              const float * x, int64_t ntok, float * y, int widen_f16);
void orc_rmsnorm(const float * x, const float * w, int64_t n, float eps, float * y);
void orc_rope_neox(float * x, int64_t head_dim, const float * cos_row, const float * sin_row);
void orc_rope_table(float theta_base, int64_t head_dim, int64_t n_pos, float * cos_tab, float * sin_tab);
/* single-query GQA decode attention.  q: [n_head][hd] fp32; k,v: fp16
 * caches laid out [n_kv_head][n_ctx][hd]; first n_kv positions used.
 * out: [n_head][hd].  probs_out (optional): [n_head][n_kv] post-softmax. */
void orc_attention(const float * q, const uint16_t * k, const uint16_t * v,
                   int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_ctx,
                   int64_t n_kv, float * out, float * probs_out);
/* the same over a bfloat16 cache when bf16 != 0 (the configuration-2 timing
 * variant; the reference's cache is F16): q and P are rounded to bfloat16,
 * ggml_mul_mat's conversion of its F32 operand to a BF16 cache's dot type. */
void orc_attention_typed(const float * q, const uint16_t * k, const uint16_t * v,
                         int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_ctx,
                         int64_t n_kv, float * out, float * probs_out, int32_t bf16);
float    orc_bf16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
/* the code predictor's 2-token prefill attention (src/tts_transformer.cpp:
 * 1999-2012): q, K and V are the F32 rows of the call, P stays F32; causal
 * over the first n_kv rows.  k, v: row j of KV head h at
 * k + j * kv_stride + h * hd.  The score's fp64 sum is taken as four
 * sequential 32-dim partials combined (s0 + s1) + (s2 + s3). */
void orc_attention_f32(const float * q, const float * k, const float * v, int64_t kv_stride,
                       int64_t n_head, int64_t n_kv_head, int64_t hd, int64_t n_kv, float * out);
int32_t orc_argmax(const float * x, int32_t n);
/* talker cb0 sampler (src/tts_transformer.cpp:3109-3184); modifies logits. */
int32_t orc_sample_cb0(float * logits, int32_t vocab, int32_t eos_id,
                       const uint8_t * seen, float rep_penalty, float temperature,
                       int32_t top_k, float eos_bias, int32_t target_frames,
                       int32_t frame, uint64_t seed);
/* code-predictor sampler (sample_or_argmax, :2750-2788); modifies logits. */
int32_t orc_sample_cp(float * logits, int32_t vocab, float temperature, int32_t top_k,
                      uint64_t seed, uint32_t frame, uint32_t group);
void orc_philox4x32(uint64_t key, uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t out[4]);
double orc_uniform(uint64_t seed, uint32_t frame, uint32_t group);

/* ---- model-level ---- */
orc_model * orc_create(const orc_config * cfg);
void        orc_destroy(orc_model * m);
void        orc_set_threads(orc_model * m, int32_t n_threads);
/* Borrows `data` (caller keeps it alive).  ggml layout, ne0 contiguous. */
int         orc_set_tensor(orc_model * m, const char * name, int32_t type,
                           const void * data, size_t nbytes);
int         orc_check_complete(orc_model * m);
const char * orc_last_error(const orc_model * m);
int         orc_kv_reset(orc_model * m, int32_t n_ctx);
/* fp16 K/V rows [n_pos][n_kv_head][head_dim] into positions [0, n_pos) of
 * talker layer `layer` (the layout q3t_dev_kv_write takes). */
/* talker cache element type: 1 (F16, the reference's) or 30 (BF16); kept
 * across orc_kv_reset, set it before the cache is filled. */
int         orc_kv_set_type(orc_model * m, int32_t type);
int         orc_kv_write(orc_model * m, int32_t layer, int32_t n_pos, const uint16_t * k, const uint16_t * v);
/* the inverse: rows of positions [0, n_pos) of talker layer `layer`. */
int         orc_kv_read(orc_model * m, int32_t layer, int32_t n_pos, uint16_t * k, uint16_t * v);
/* n-token prefill at positions [n_past, n_past+n).  hidden_out: [n][d]
 * (normed), logits_out: last row [codec_vocab] (may be NULL). */
int orc_prefill(orc_model * m, const float * embd, int32_t n, int32_t n_past,
                float * hidden_out, float * logits_out);
int orc_step(orc_model * m, const float * embd, int32_t n_past,
             float * logits_out, float * hidden_out);
/* Attention-row capture (set_attn_dump, src/tts_transformer.cpp:1719-1724,
 * :2485-2497): with layer in [0, n_layers) every orc_step (also inside
 * orc_frames) keeps that talker layer's post-softmax fp32 row [n_head][n_kv];
 * -1 turns it off.  Either call clears the kept rows.  orc_attn_row copies
 * row `index` when out holds cap >= n_head * n_kv floats and returns n_kv
 * (-1: no such row). */
int     orc_set_attn_capture(orc_model * m, int32_t layer);
int32_t orc_attn_row_count(const orc_model * m);
int32_t orc_attn_row(const orc_model * m, int32_t index, float * out, int64_t cap);
/* 15 codes for codebooks 1..15.  logits_out (optional): [15][cp_vocab]
 * logits as produced by each head before sampling. */
int orc_code_pred(orc_model * m, const float * hidden, int32_t cb0,
                  float temperature, int32_t top_k, uint64_t seed, uint32_t frame,
                  int32_t * codes_out, float * logits_out);
/* Single-pass code predictor (src/tts_transformer.cpp:2531-2581 over
 * build_code_pred_graph :1771-1899): logits_out [15][cp_vocab] of the 15
 * heads on one row hidden (+ the 15 code-predictor embeddings of prev_codes
 * when not NULL) after the MTP projection (if any) and the layers at one
 * position with no cache and no output norm. */
int orc_predict_codes(orc_model * m, const float * hidden, const int32_t * prev_codes, float * logits_out);
int orc_text_proj(orc_model * m, const int32_t * tokens, int32_t n, float * out);
int orc_embed_row(orc_model * m, const char * table, int32_t index, int32_t token, float * out);
/* build_prefill_graph: prefill_out [(n_instruct+10 or 9)][d],
 * trailing_out [max(0,n-9)+1][d], pad_out [d].  Returns prefill_len,
 * writes trailing_len. */
int orc_build_prefill(orc_model * m, const int32_t * text, int32_t n_text,
                      const float * speaker, int32_t language_id,
                      const int32_t * instruct, int32_t n_instruct,
                      float * prefill_out, float * trailing_out, float * pad_out,
                      int32_t * trailing_len_out);
/* generate(): returns number of frames written to codes_out ([max_len][16]);
 * negative on error.  first_logits_out (optional): prefill logits row. */
int orc_generate(orc_model * m, const int32_t * text, int32_t n_text,
                 const float * speaker, const orc_gen_params * p,
                 const int32_t * instruct, int32_t n_instruct,
                 int32_t * codes_out, float * first_logits_out);

/* the generate() frame loop from prebuilt rows (prefill [plen][d],
 * trailing [trail_len][d], tts_pad [d]); used for the ICL layout. */
int orc_generate_rows(orc_model * m, const float * prefill, int32_t plen, const float * trailing,
                      int32_t trail_len, const float * pad, const orc_gen_params * p,
                      int32_t * codes_out, float * first_logits_out);

/* the frame loop alone, from the current talker cache: first_logits and the
 * normed hidden row of the last orc_prefill / orc_step, next position n_past
 * (what q3t_dev_frames_begin continues from).  Returns frames written.
 * frame_logits_out (optional, [max_len][codec_vocab]): the talker logits each
 * frame's codebook-0 sampler starts from, before suppression and penalty. */
int orc_frames(orc_model * m, const float * first_logits, int32_t n_past, const float * trailing,
               int32_t trail_len, const float * pad, const orc_gen_params * p, int32_t * codes_out,
               float * frame_logits_out);

/* ---- audio-tokenizer decoder (vocoder), q3t_vocoder.cpp ----
 * Restates src/audio_tokenizer_decoder.cpp (build_graph :636-843,
 * decode_window :946).  Widths come from the config; tensors are named and
 * laid out as the GGUF's tok_dec.* tensors (ggml ne order, ne0 contiguous).
 * Numerics: fp16-rounded activations into every F16-weight product, exact
 * products summed in fp64 and rounded once; F32 attention; the C library's
 * expf/sinf/tanhf.  Parity with ggml is tolerance-level (its fp32 lane sums
 * and SIMD exp are not restated). */
typedef struct orc_voc_config {
    int32_t n_codebooks;      /* 16 */
    int32_t codebook_size;    /* 2048 */
    int32_t codebook_dim;     /* 256 */
    int32_t hidden;           /* 512: VQ output and pre-transformer width */
    int32_t latent;           /* 1024: pre_conv / attention q,k,v / upsample width */
    int32_t n_layers;         /* 8 */
    int32_t n_heads;          /* 16 (head_dim = latent / n_heads) */
    int32_t ffn;              /* 1024 */
    int32_t cnx_ffn;          /* 4096: ConvNeXt pwconv1 width */
    int32_t up_kernel;        /* 2: upsample conv_t kernel (stride 2) */
    int32_t decoder_dim;      /* 1536 */
    int32_t rates[4];         /* 8 5 4 3 */
    int32_t dec_kernel[4];    /* conv_t kernels, 2 * rate */
    float   rms_eps;          /* 1e-5 */
    float   rope_theta;       /* 1e4 */
} orc_voc_config;

typedef struct orc_voc orc_voc;
orc_voc *    orc_voc_create(const orc_voc_config * cfg);
void         orc_voc_destroy(orc_voc * m);
void         orc_voc_set_threads(orc_voc * m, int32_t n);
const char * orc_voc_last_error(const orc_voc * m);
/* Borrows `data`. */
int          orc_voc_set_tensor(orc_voc * m, const char * name, int32_t type, const void * data, size_t nbytes);
/* checks every tensor, then normalises the codebooks (load_model :318-340) */
int          orc_voc_finalize(orc_voc * m);
int64_t      orc_voc_samples_for_frames(const orc_voc * m, int32_t n_frames);
/* decode_single: codes [n][n_codebooks] at positions pos0..; out holds
 * orc_voc_samples_for_frames(n) floats; latent_out (optional) [n][hidden]. */
int          orc_voc_decode_single(orc_voc * m, const int32_t * codes, int32_t n, int32_t pos0, float * out,
                                   float * latent_out);
int          orc_voc_decode_window(orc_voc * m, const int32_t * codes, int32_t n_frames, int32_t start,
                                   int32_t end, int32_t context, float * out, int64_t cap, int64_t * n_out);
/* one named stage (see orc_voc_set_record for the names) from in [T][C]
 * (or, for "latent", from codes [T][n_codebooks]); out [T_out][C_out]. */
int          orc_voc_run_stage(orc_voc * m, const char * name, const float * in, const int32_t * codes, int64_t T,
                               int64_t C, int32_t pos0, float * out, int64_t cap, int64_t * T_out, int64_t * C_out);
/* stage recording: with on != 0 every decode_single keeps each stage's fp32
 * rows (latent, pre_conv, input_proj, pre_tfm.<l>, output_proj,
 * upsample.<i>, dec.0, dec.<b>.conv_t, dec.<b>.res.<r>, dec.6). */
void         orc_voc_set_record(orc_voc * m, int32_t on);
int32_t      orc_voc_stage_count(const orc_voc * m);
int          orc_voc_stage(const orc_voc * m, int32_t i, char * name, int32_t name_cap, float * out, int64_t cap,
                           int64_t * T, int64_t * C);

#ifdef __cplusplus
}
#endif
#endif
