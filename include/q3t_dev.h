/*
 * q3t_dev.h -- C ABI of the MI355X (gfx950) device layer for the
 * qwen3-tts.cpp per-frame token loop.
 *
 * This is the boundary a maintainer binds when the reference's
 * TTSTransformer (src/tts_transformer.h:198-338) stops building ggml graphs
 * for the talker step and the code predictor and calls the GPU instead.
 * Nothing here uses C++ types, torch types or CUDA names: plain pointers,
 * sizes and int status codes (0 = ok, negative = error; the message is
 * returned by q3t_dev_last_error).
 *
 * Threading: one q3t_dev per host thread, like the reference's
 * TTSTransformer (not thread safe; src/tts_transformer.h:400-404 keeps
 * mutable state and an RNG per instance).  Host pointers are borrowed for
 * the duration of a call; outputs are written into caller-owned buffers.
 *
 * Numerics (shared with the CPU restatement in oracle/): Q8_0 weights take a
 * per-32-block Q8_0-quantised activation (int8 x int8 block dots); F16
 * weights take an fp16-rounded activation; F16 ffn_down takes the fp32
 * activation; every dot product accumulates exact terms in fp64 and rounds
 * once to fp32.  The talker KV cache is fp16 as in the reference (bfloat16
 * on request, q3t_dev_kv_set_type).
 */
#ifndef Q3T_DEV_H
#define Q3T_DEV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define Q3T_TYPE_F32  0   /* ggml GGML_TYPE_F32  */
#define Q3T_TYPE_F16  1   /* ggml GGML_TYPE_F16  */
#define Q3T_TYPE_Q8_0 8   /* ggml GGML_TYPE_Q8_0 */
#define Q3T_TYPE_BF16 30  /* ggml GGML_TYPE_BF16 (talker KV cache only) */

/* Hyperparameters.  Mirrors tts_transformer_config
 * (src/tts_transformer.h:59-103) field for field; values come from the
 * GGUF keys parsed at src/tts_transformer.cpp:228-377. */
typedef struct q3t_config {
    int32_t hidden_size;      /* talker width, 1024 */
    int32_t n_layers;         /* talker blocks, 28 */
    int32_t n_head;           /* query heads, 16 */
    int32_t n_kv_head;        /* KV heads, 8 */
    int32_t head_dim;         /* 128 (the only value the kernels accept) */
    int32_t ffn_size;         /* 3072 */
    int32_t codec_vocab;      /* 3072 */
    int32_t n_codebooks;      /* 16 */
    int32_t cp_layers;        /* code-predictor blocks, 5 */
    int32_t cp_vocab;         /* 2048 */
    int32_t cp_hidden;        /* code predictor width; below hidden_size the
                               * model carries code_pred.mtp_proj (1.7B layout,
                               * src/tts_transformer.cpp:548-553, :1942-1947) */
    int32_t cp_ffn;           /* 3072 */
    int32_t text_vocab;       /* 151936 */
    int32_t text_embd_dim;    /* 2048 */
    float   rms_eps;          /* 1e-6 */
    float   rope_theta;       /* 1e6 */
    float   cp_rope_theta;    /* defaults to rope_theta (:316-324) */
    int32_t codec_pad_id, codec_bos_id, codec_eos_id;
    int32_t tts_bos_id, tts_eos_id, tts_pad_id;
    int32_t codec_think_id, codec_nothink_id, codec_think_bos_id, codec_think_eos_id;
    int32_t english_language_id;
} q3t_config;

/* Per-call sampling controls.  temperature <= 0 selects greedy argmax
 * (first maximum), as in sample_or_argmax (src/tts_transformer.cpp:2750-2788).
 * The reference draws from std::mt19937 (src/tts_transformer.h:403); this
 * layer draws from Philox4x32-10 keyed by `seed` and counted by
 * (frame, codebook), so a run is reproducible. */
typedef struct q3t_sampling {
    float    temperature;
    int32_t  top_k;
    uint64_t seed;
} q3t_sampling;

/* Arguments of the device-resident frame loop: the state generate() keeps
 * across frames (src/tts_transformer.cpp:3092-3106) and its per-call
 * controls (repetition penalty, EOS bias ramp, sampling). */
typedef struct q3t_frame_args {
    const float * trailing;      /* [n_trailing][hidden]: trailing_text_hidden rows */
    int32_t       n_trailing;
    const float * tts_pad;       /* [hidden]: row used once trailing rows run out */
    int32_t       n_past;        /* positions already in the talker KV (prefill length) */
    int32_t       max_len;       /* frames the caller will request at most */
    float         repetition_penalty;
    float         eos_bias;
    int32_t       target_frames;
    q3t_sampling  sampling;
} q3t_frame_args;

typedef struct q3t_dev q3t_dev;

/* Context on HIP device `device` (ordinal).  Replaces the ggml backend and
 * scheduler set up in TTSTransformer::load_model
 * (src/tts_transformer.cpp:68-169, backend choice src/gguf_loader.cpp:154-198). */
int  q3t_dev_create(const q3t_config * cfg, int32_t device, q3t_dev ** out);
/* Frees every device allocation.  Replaces TTSTransformer::unload_model
 * (src/tts_transformer.cpp:25-51). */
void q3t_dev_destroy(q3t_dev * dev);
/* Last error message of this context ("" if none).  Maps onto
 * TTSTransformer::get_error (src/tts_transformer.h:329). */
const char * q3t_dev_last_error(const q3t_dev * dev);

/* One GGUF tensor, ggml layout (ne[0] contiguous), ggml type id.  Names and
 * shapes as create_tensors binds them (src/tts_transformer.cpp:379-668);
 * replaces load_tensor_data's ggml_backend_tensor_set
 * (src/tts_transformer.cpp:670-729).  Q8_0 blocks are repacked in HBM
 * (int8 quants and fp16 scales split) without changing any value. */
int  q3t_dev_upload_tensor(q3t_dev * dev, const char * name, int32_t ggml_type,
                           const int64_t ne[4], const void * data, size_t nbytes);
/* The same upload in row ranges, for loaders that read a GGUF file in
 * bounded pieces instead of holding whole tensors in host memory (the
 * reference's load_tensor_data reads each tensor whole,
 * src/tts_transformer.cpp:670-729): rows [row0, row0 + n_rows) of the ne[1]
 * rows, `data` holding those rows in ggml layout (Q8_0: whole 34-byte
 * blocks), nbytes their size.  A tensor's first range (row0 == 0) allocates
 * it; the ranges must cover every row once (checked before the first compute
 * call: "tensor ... incomplete").  Synchronous: `data` may be reused on
 * return.  Q8_0 blocks are repacked on the device. */
int  q3t_dev_upload_tensor_rows(q3t_dev * dev, const char * name, int32_t ggml_type, const int64_t ne[4],
                                int64_t row0, int64_t n_rows, const void * data, size_t nbytes);
/* The context's pinned host staging buffer for q3t_dev_upload_tensor_rows
 * (at least min_bytes, 64 MiB by default; owned by the context, valid until
 * the next call or q3t_dev_destroy); *cap_out receives its size.  Filling it
 * from the file makes each range one DMA.  NULL on failure. */
void * q3t_dev_staging(q3t_dev * dev, size_t min_bytes, size_t * cap_out);
/* Copies a tensor back in ggml layout (used to check the upload). */
int  q3t_dev_download_tensor(q3t_dev * dev, const char * name, void * data, size_t nbytes);
/* Dequantises a Q8_0 tensor on the device to fp32 [ne1][ne0] (fp32(d)*q). */
int  q3t_dev_dequantize(q3t_dev * dev, const char * name, float * out, size_t n_floats);

/* Talker KV cache of n_ctx positions (fp16 or bfloat16, per layer
 * [n_kv_head][n_ctx][head_dim]).  Replaces init_kv_cache / clear_kv_cache
 * (src/tts_transformer.cpp:731-783).  n_ctx is bounded by the decode
 * attention's LDS (a head's n_ctx fp32 scores in one workgroup: about 38,600
 * positions on gfx950, past the talker's 32,768-position table). */
int  q3t_dev_kv_reserve(q3t_dev * dev, int32_t n_ctx);
int  q3t_dev_kv_clear(q3t_dev * dev);
int32_t q3t_dev_kv_capacity(const q3t_dev * dev);
/* Talker KV element type: Q3T_TYPE_F16 (the reference's, init_kv_cache at
 * src/tts_transformer.cpp:761-768; the default) or Q3T_TYPE_BF16, the cache
 * type as a parameter for timing configuration 2.  With BF16, q and the
 * softmax probabilities are rounded to bfloat16 where the F16 cache rounds
 * them to fp16 (ggml_mul_mat's conversion of its F32 operand to the cache's
 * dot type).  A reserved cache is re-reserved (cleared).  Single steps,
 * prefill and the frame loop (persistent kernel or multi-kernel) take either
 * type; multi-stream decode takes F16 only.  q3t_dev_kv_write rows are then
 * bfloat16 bits. */
int  q3t_dev_kv_set_type(q3t_dev * dev, int32_t type);
/* Attention-row capture, the device side of set_attn_dump / attn_rows
 * (src/tts_transformer.h:224-227; rows captured in forward_step,
 * src/tts_transformer.cpp:1719-1724 and :2485-2497).  layer in
 * [0, n_layers) turns it on for that talker layer, -1 turns it off; either
 * call clears the kept rows and ends an open frame loop (call it before
 * q3t_dev_frames_begin).  While it is on, every talker step (talker_step and
 * each frame of frames_run that is not EOS) keeps the layer's post-softmax
 * fp32 row [n_head][n_kv], heads as blocks of n_kv, n_kv = step position + 1;
 * those steps run on the multi-kernel path and synchronise once per frame. */
int  q3t_dev_set_attn_capture(q3t_dev * dev, int32_t layer);
int32_t q3t_dev_attn_row_count(const q3t_dev * dev);
/* Copies kept row `index` (n_head * n_kv floats) to out when out is non-null
 * (cap: its size in floats); *n_kv_out receives n_kv. */
int  q3t_dev_attn_row(q3t_dev * dev, int32_t index, float * out, int64_t cap, int32_t * n_kv_out);
/* Writes fp16 K/V rows [n_pos][n_kv_head][head_dim] for positions
 * [0, n_pos) of talker layer `layer` (used to pre-fill a cache). */
int  q3t_dev_kv_write(q3t_dev * dev, int32_t layer, int32_t n_pos,
                      const uint16_t * k, const uint16_t * v);

/* n-token talker forward at positions [n_past, n_past+n).
 * embd: [n][hidden].  hidden_out: [n][hidden] normed hidden (NULL ok).
 * logits_out: last row's codec logits [codec_vocab] (NULL ok).
 * Replaces forward_prefill (src/tts_transformer.cpp:2217-2347). */
int  q3t_dev_prefill(q3t_dev * dev, const float * embd, int32_t n, int32_t n_past,
                     float * hidden_out, float * logits_out);
/* One-token talker step at position n_past.  Replaces forward_step
 * (src/tts_transformer.cpp:2379-2509).  Runs as one launch of the
 * persistent frame kernel's talker pass where that kernel applies (else the
 * multi-kernel step; same results). */
int  q3t_dev_talker_step(q3t_dev * dev, const float * embd, int32_t n_past,
                         float * logits_out, float * hidden_out);
/* Single-pass code predictor: replaces TTSTransformer::predict_codes
 * (src/tts_transformer.cpp:2531-2581, graph build_code_pred_graph :1771-1899).
 * One row: hidden [hidden_size] plus, when prev_codes is not NULL, the 15
 * code_pred.codec_embd[g][prev_codes[g]] rows (added in order, fp32); the
 * MTP projection when the layout has one; the code-predictor layers on one
 * position with no cache (each head's attention output is its V row); the 15
 * heads on the last layer's row with no output norm.  logits_out:
 * [15][cp_vocab].  Needs no KV reservation and leaves the frame loop's state
 * alone.  A code outside [0, cp_vocab) fails ("Embedding token ID out of
 * range"). */
int  q3t_dev_predict_codes(q3t_dev * dev, const float * hidden, const int32_t * prev_codes, float * logits_out);
/* Code predictor: 2-token prefill [hidden, codec_embd[cb0]] then 14 steps;
 * codes_out[15] = codebooks 1..15.  logits_out (NULL ok): [15][cp_vocab],
 * each head's logits before sampling.  `frame` keys the sampler's RNG.
 * Replaces predict_codes_autoregressive (src/tts_transformer.cpp:2711-2976).
 * Runs on the persistent frame kernel's code-predictor passes when the talker
 * KV cache is reserved and that kernel applies (else the multi-kernel
 * sequence; same results). */
int  q3t_dev_code_pred(q3t_dev * dev, const float * hidden, int32_t cb0,
                       const q3t_sampling * sampling, uint32_t frame,
                       int32_t * codes_out, float * logits_out);

/* text_proj: fc2(silu(fc1(text_embd[tok]) + b1)) + b2 -> out [n][hidden].
 * Replaces project_text_tokens (src/tts_transformer.cpp:963-1028). */
int  q3t_dev_text_proj(q3t_dev * dev, const int32_t * tokens, int32_t n, float * out);
/* q3t_dev_text_proj without any device allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, results and errors
 * as q3t_dev_text_proj for n <= 64 ids; more ids are rejected with an error.
 * Its work buffers (2 MiB) are a static device array that each GPU holds until
 * the process ends and that every call on that GPU shares: calls that overlap
 * on one GPU (from several contexts or threads) race. */
int  q3t_dev_text_proj_noalloc(q3t_dev * dev, const int32_t * tokens, int32_t n, float * out);
/* Embedding rows as fp32: table 0 = talker.codec_embd, 1 = code_pred.codec_embd[index],
 * 2 = talker.text_embd.  Replaces lookup_embedding_rows /
 * lookup_single_embedding_row (src/tts_transformer.cpp:839-961). */
int  q3t_dev_embed_rows(q3t_dev * dev, int32_t table, int32_t index,
                        const int32_t * tokens, int32_t n, float * out);

/* Prefill rows in one call: build_prefill_graph (src/tts_transformer.cpp:1030-1186).
 * Every text id of the layout (tts bos/eos/pad, the 3 role ids, the first text id,
 * the instruct ids, the trailing ids text[4 .. n-5)) is projected in one batched
 * pass, and the codec overlays are summed on the device.  Outputs: prefill_out
 * [n_prefill][hidden], trailing_out [n_trailing][hidden] (trailing text rows, then
 * tts_eos), tts_pad_out [hidden].  With prefill_out == NULL only the two counts are
 * written (n_prefill = n_instruct + 3 + codec rows, n_trailing = max(0, n - 9) + 1).
 * language_id < 0 selects the no-think codec prefix; speaker_embd may be NULL. */
int  q3t_dev_build_prefill(q3t_dev * dev, const int32_t * text_tokens, int32_t n_tokens,
                           const float * speaker_embd, int32_t language_id,
                           const int32_t * instruct_tokens, int32_t n_instruct,
                           float * prefill_out, int32_t * n_prefill_out,
                           float * trailing_out, int32_t * n_trailing_out, float * tts_pad_out);
/* The voice-clone prefill: build_prefill_graph_icl (src/tts_transformer.cpp:1188-1472).
 * The text stream ref_text[3:-5] ++ text[3:-5] ++ tts_eos is interleaved with the
 * codec stream [codec_bos, reference frames] (each frame the sum of its 16 codebook
 * embeddings, ref_codec_tokens [n_ref_frames][16]) up to the codec length; the rest
 * of the text stream is the trailing text (n_trailing may be 0).  Same output and
 * size-query convention as q3t_dev_build_prefill. */
int  q3t_dev_build_prefill_icl(q3t_dev * dev, const int32_t * text_tokens, int32_t n_tokens,
                               const int32_t * ref_text_tokens, int32_t n_ref_text,
                               const int32_t * ref_codec_tokens, int32_t n_ref_frames,
                               const float * speaker_embd,
                               float * prefill_out, int32_t * n_prefill_out,
                               float * trailing_out, int32_t * n_trailing_out, float * tts_pad_out);

/* Device-resident frame loop (the body of generate(),
 * src/tts_transformer.cpp:3108-3309).  frames_begin takes the logits and
 * normed hidden left on the device by the last q3t_dev_prefill /
 * q3t_dev_talker_step call; frames_run advances up to n_frames frames with
 * one hipGraph launch per frame and one host sync per call, appending
 * [frames][n_codebooks] codes to codes_out.  *eos_out is set once codebook 0
 * samples EOS (the frame that sampled it is not emitted). */
int  q3t_dev_frames_begin(q3t_dev * dev, const q3t_frame_args * args);
int  q3t_dev_frames_run(q3t_dev * dev, int32_t n_frames, int32_t * codes_out,
                        int32_t * n_emitted_out, int32_t * eos_out);
/* Device address of the frame loop's code rows: frame f's n_codebooks codes
 * at + f * n_codebooks, valid for the frames emitted since the last
 * q3t_dev_frames_begin (complete once frames_run returns).  The streaming
 * vocoder reads them in place (q3t_voc_decode_window with codes_on_device),
 * where the reference hands codes_total from its FrameCallback
 * (src/tts_transformer.cpp:3213, src/qwen3_tts.cpp:294) to decode_window.
 * NULL before the first q3t_dev_frames_begin. */
const int32_t * q3t_dev_frame_codes(const q3t_dev * dev);

/* Frame-loop statistics since the last q3t_dev_frames_begin or
 * q3t_dev_streams_begin: GPU time of the frame launches (HIP events around
 * each frames_run / streams_run's launches, in microseconds), the number of
 * frame launches, and which implementation ran them (1 = one persistent
 * cooperative kernel per frame, 3 = the same with its XCD-parallel layer
 * program, 0 = the captured multi-kernel graph, 2 = the multi-stream graph,
 * one launch advancing every stream by a frame).  Instrumentation with no counterpart in the
 * reference; the benchmark and the tests use it. */
int  q3t_dev_frames_stats(q3t_dev * dev, double * gpu_us_out, int64_t * frames_out,
                          int32_t * path_out);

/* Multi-stream decode: n_streams independent generate() frame loops
 * (src/tts_transformer.cpp:3108-3309, one per utterance) advanced together.
 * The reference runs one utterance per TTSTransformer at batch 1; this is
 * the batched form of the same loop, each stream bit-identical to its own
 * q3t_dev_frames_* run (same weights, prompt rows, arguments and seed).
 * Every talker / code-predictor layer runs as one MFMA GEMM over the
 * streams' rows (int8 for Q8_0 layers, f64 for F16 layers), attention and
 * the samplers as one block per stream.  Requires the layer weights to be all
 * Q8_0 or all F16.
 *
 * streams_reserve allocates per-stream KV caches of n_ctx positions (and
 * re-reserves the context's own cache to n_ctx for the shared RoPE tables);
 * stream_prefill runs forward_prefill (:2217-2347) for one stream at n_past 0
 * into its cache; streams_begin takes one q3t_frame_args per stream (n_past
 * = that stream's prompt length); streams_run advances every live stream by
 * up to n_frames frames.  codes_out is [n_streams][n_frames][n_codebooks]:
 * stream b's new frames start at codes_out + b*n_frames*16, their count in
 * n_emitted_out[b], eos_out[b] = 1 once its codebook 0 sampled EOS.  Streams
 * that stopped (EOS or max_len) idle while the others run. */
int  q3t_dev_streams_reserve(q3t_dev * dev, int32_t n_streams, int32_t n_ctx);
int  q3t_dev_stream_prefill(q3t_dev * dev, int32_t stream, const float * embd, int32_t n);
/* Stream b's counterparts of q3t_dev_kv_write and q3t_dev_prefill(n_past):
 * rows [0, n_pos) of talker layer `layer` of the stream's cache, and the
 * prefill of n rows at positions [n_past, n_past+n) over that cache (a stream
 * resumed from a cached history).  stream_prefill is stream_prefill_at with
 * n_past 0. */
int  q3t_dev_stream_kv_write(q3t_dev * dev, int32_t stream, int32_t layer, int32_t n_pos,
                             const uint16_t * k, const uint16_t * v);
int  q3t_dev_stream_prefill_at(q3t_dev * dev, int32_t stream, const float * embd, int32_t n, int32_t n_past);
int  q3t_dev_streams_begin(q3t_dev * dev, const q3t_frame_args * args);
int  q3t_dev_streams_run(q3t_dev * dev, int32_t n_frames, int32_t * codes_out,
                         int32_t * n_emitted_out, int32_t * eos_out);

/* Copies stream `stream`'s talker logits [codec_vocab] into out: the row the
 * stream's next codebook-0 sampler reads (after a streams_run, the logits of
 * its last talker step).  Instrumentation with no counterpart in the
 * reference: tests compare the decode GEMM forms of F16 layers with it. */
int  q3t_dev_stream_logits(q3t_dev * dev, int32_t stream, float * out);

/* Blocks until all work queued by this context has finished. */
int  q3t_dev_sync(q3t_dev * dev);
/* Times `iters` launches of one kernel class of the frame loop with HIP
 * events on the context's stream; writes the average microseconds per
 * launch and the algorithmic bytes one launch moves.  which: 0 = talker
 * gate/up GEMV, 1 = talker QKV GEMV, 2 = talker down GEMV, 3 = talker Wo
 * GEMV, 4 = talker attention (at position min(n_ctx-1, 512)), 5 = a plain
 * 64 MiB device-to-device copy kernel (k_copy16; the calibration point for
 * the HBM byte counters).  Resets the frame-loop state.  Used by the
 * benchmark to report roofline fractions. */
int  q3t_dev_time_kernel(q3t_dev * dev, int32_t which, int32_t iters,
                         double * avg_us_out, double * bytes_out);

#ifdef __cplusplus
}
#endif
#endif
