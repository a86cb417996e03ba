/*
 * q3t_voc.h -- C ABI of the MI355X (gfx950) audio-tokenizer decoder: the
 * vocoder that turns the frame loop's 16-codebook frames into 24 kHz PCM.
 *
 * This is the boundary a maintainer binds when the reference's
 * AudioTokenizerDecoder (src/audio_tokenizer_decoder.h:160-232) stops
 * building its ggml graph and calls the GPU instead; the streaming driver
 * (src/qwen3_tts.cpp:271-316) then feeds decode_window from the device code
 * rows the frame loop already holds (q3t_dev_frame_codes), with no host copy
 * of the codes per frame.  Plain pointers and sizes, int status codes
 * (0 = ok, negative = error; message from q3t_voc_last_error).  One
 * q3t_voc per host thread.
 *
 * Numerics: every F16-weight product (linear layers, 1-D and transposed
 * convolutions) takes the fp16-rounded activation, as ggml's F16 im2col and
 * vec_dot_type do, and accumulates in fp32 on the matrix cores; attention in
 * the pre-transformer is F32; norms accumulate in fp64.  Results agree with
 * the CPU restatement (oracle/q3t_vocoder.cpp) within the tolerances its
 * tests state, not bit for bit.
 */
#ifndef Q3T_VOC_H
#define Q3T_VOC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Widths of the decoder.  Mirrors audio_decoder_config
 * (src/audio_tokenizer_decoder.h:15-29); the fields the reference reads from
 * tensor shapes instead (ConvNeXt width, transposed-conv kernels) are
 * explicit here.  The 12 Hz tokenizer: 16, 2048, 256, 512, 1024, 8, 16,
 * 1024, 4096, 2, 1536, {8,5,4,3}, {16,10,8,6}, 1e-5, 1e4. */
typedef struct q3t_voc_config {
    int32_t n_codebooks;      /* 16 */
    int32_t codebook_size;    /* 2048 */
    int32_t codebook_dim;     /* 256 */
    int32_t hidden;           /* 512: VQ output and pre-transformer width */
    int32_t latent;           /* 1024: pre_conv, attention q/k/v and upsample width */
    int32_t n_layers;         /* 8 */
    int32_t n_heads;          /* 16 (head_dim = latent / n_heads, at most 64) */
    int32_t ffn;              /* 1024 */
    int32_t cnx_ffn;          /* 4096: ConvNeXt pwconv1 width */
    int32_t up_kernel;        /* 2: upsample transposed-conv kernel (stride 2) */
    int32_t decoder_dim;      /* 1536 */
    int32_t rates[4];         /* 8 5 4 3 */
    int32_t dec_kernel[4];    /* 2 * rate */
    float   rms_eps;          /* 1e-5 */
    float   rope_theta;       /* 1e4 */
} q3t_voc_config;

typedef struct q3t_voc q3t_voc;

/* AudioTokenizerDecoder() + the backend set-up of load_model
 * (src/audio_tokenizer_decoder.cpp:38-44, 342-370).  Fails (returns NULL
 * with *err_out set, if given) without a HIP device. */
q3t_voc * q3t_voc_create(const q3t_voc_config * cfg, int32_t device, const char ** err_out);
/* unload_model + ~AudioTokenizerDecoder (:42-64) */
void q3t_voc_destroy(q3t_voc * v);
/* get_error (:232) */
const char * q3t_voc_last_error(const q3t_voc * v);

/* One tok_dec.* tensor of the GGUF (load_model's per-tensor loop,
 * :142-313): ggml type (0 = F32, 1 = F16), ggml layout (ne0 contiguous).
 * The bytes are copied; the caller may free them after q3t_voc_finalize. */
int q3t_voc_set_tensor(q3t_voc * v, const char * name, int32_t type, const void * data, size_t nbytes);
/* The rest of load_model (:314-340): checks every tensor's presence, type
 * and size, normalises the codebooks by their usage (normalize_codebooks,
 * :66-100), lays the weights out for the GEMMs and builds the per-codebook
 * projection tables. */
int q3t_voc_finalize(q3t_voc * v);
/* Device buffers for windows of up to max_frames frames (decode_window
 * grows them on demand; this avoids allocating inside a streaming loop). */
int q3t_voc_reserve(q3t_voc * v, int32_t max_frames);

/* output_samples_for_frames (:845-875) */
int64_t q3t_voc_samples_for_frames(const q3t_voc * v, int32_t n_frames);

/* decode_window (:946-980): decodes frames [max(0, start - context), end)
 * of codes ([n_frames][n_codebooks] int32) at their absolute positions and
 * writes the samples of frames [start, end) to out (cap floats); *n_out =
 * samples written.  codes_on_device = 1: codes is a device pointer (e.g.
 * q3t_dev_frame_codes) read in place, the streaming path; 0: host memory.
 * A code outside [0, codebook_size) fails the call. */
int q3t_voc_decode_window(q3t_voc * v, const int32_t * codes, int32_t codes_on_device, int32_t n_frames,
                          int32_t start, int32_t end, int32_t context, float * out, int64_t cap,
                          int64_t * n_out);
/* decode (:1003-1024): the whole utterance in one pass (out holds
 * q3t_voc_samples_for_frames(n_frames) floats). */
int q3t_voc_decode(q3t_voc * v, const int32_t * codes, int32_t codes_on_device, int32_t n_frames, float * out,
                   int64_t cap, int64_t * n_out);

/* Diagnostic: one stage of the graph from host fp32 rows in [T][C] (codes
 * [T][n_codebooks] for "latent"), the named intermediate tensors of
 * build_graph (:636-843): latent, pre_conv, input_proj, pre_tfm.<l>,
 * output_proj (final norm + projection), upsample.<i>, dec.0,
 * dec.<b>.conv_t (block snake + transposed conv), dec.<b>.res.<r> (r = 2..4),
 * dec.6 (final snake + conv, before tanh).  out gets [T_out][C_out] fp32.
 * Positions (pre_tfm.<l>) start at pos0. */
int q3t_voc_run_stage(q3t_voc * v, const char * name, const float * in, const int32_t * codes, int64_t T,
                      int64_t C, int32_t pos0, float * out, int64_t cap, int64_t * T_out, int64_t * C_out);

#ifdef __cplusplus
}
#endif
#endif
