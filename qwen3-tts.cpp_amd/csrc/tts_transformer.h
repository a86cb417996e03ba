// tts_transformer.h -- drop-in TTSTransformer over the MI355X device layer.
//
// Same class, namespace and public methods as the reference's
// src/tts_transformer.h:198-338, so the pipeline (src/qwen3_tts.cpp) and the
// C API (src/qwen3tts_c_api.cpp) keep calling it unchanged.  The ggml graphs
// are replaced by calls into the C ABI of include/q3t_dev.h: the talker step,
// code predictor, samplers and frame loop run on the GPU; this class keeps
// the reference's host-side control flow (prefill layout, KV sizing rule,
// per-frame callback, repetition-loop truncation) and error reporting
// (bool + get_error()).
#pragma once

#include <cstdint>
#include <functional>
#include <random>
#include <string>
#include <vector>

struct q3t_dev;

namespace qwen3_tts {

// Field for field the reference's tts_transformer_config
// (src/tts_transformer.h:59-103).
struct tts_transformer_config {
    int32_t text_vocab_size = 151936;
    int32_t text_embd_dim = 2048;
    int32_t hidden_size = 1024;
    int32_t n_layers = 28;
    int32_t n_attention_heads = 16;
    int32_t n_key_value_heads = 8;
    int32_t intermediate_size = 3072;
    int32_t head_dim = 128;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 1000000.0f;
    int32_t mrope_section[3] = {24, 20, 20};
    int32_t codec_vocab_size = 3072;
    int32_t n_codebooks = 16;
    int32_t code_pred_layers = 5;
    int32_t code_pred_vocab_size = 2048;
    int32_t code_pred_hidden_size = 1024;
    int32_t code_pred_intermediate_size = 3072;
    float code_pred_rope_theta = 10000.0f;
    int32_t codec_pad_id = 2148;
    int32_t codec_bos_id = 2149;
    int32_t codec_eos_id = 2150;
    int32_t tts_bos_token_id = 151672;
    int32_t tts_eos_token_id = 151673;
    int32_t tts_pad_token_id = 151671;
    int32_t codec_think_id = 2154;
    int32_t codec_nothink_id = 2155;
    int32_t codec_think_bos_id = 2156;
    int32_t codec_think_eos_id = 2157;
    int32_t english_language_id = 2050;
};

class TTSTransformer {
public:
    TTSTransformer();
    ~TTSTransformer();

    bool load_model(const std::string & model_path);
    void set_n_threads(int32_t n_threads);   // no CPU thread pool on this path: accepted and ignored
    void unload_model();
    void set_debug_dump(bool enabled) { debug_dump_ = enabled; }
    void set_attn_dump(const std::string & path, int layer = 27) {
        attn_dump_ = !path.empty(); attn_dump_path_ = path; attn_dump_layer_ = layer;
    }
    const std::vector<std::vector<float>> & attn_rows() const { return attn_rows_; }

    bool init_kv_cache(int32_t n_ctx);
    void clear_kv_cache();
    bool init_code_pred_kv_cache(int32_t n_ctx);
    void clear_code_pred_kv_cache();

    bool forward_text(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd, int32_t n_past,
                      std::vector<float> & output);
    bool forward_prefill(const float * prefill_embd, int32_t n_tokens, int32_t n_past, std::vector<float> & output,
                         std::vector<float> * logits_out = nullptr);
    bool forward_codec(int32_t codec_token, int32_t n_past, std::vector<float> & output);
    bool forward_step(const float * step_embd, int32_t n_past, std::vector<float> & output,
                      std::vector<float> * hidden_out = nullptr);
    bool get_hidden_states(std::vector<float> & hidden) const;
    bool predict_codes(const float * hidden, const int32_t * prev_codes, std::vector<float> & output);
    bool predict_codes_autoregressive(const float * hidden, int32_t codebook_0_token, std::vector<int32_t> & output,
                                      float temperature = 0.9f, int32_t top_k = 50);

    using FrameCallback = std::function<bool(const int32_t *, int32_t, int32_t)>;

    bool generate(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd, int32_t max_len,
                  std::vector<int32_t> & output, int32_t language_id = 2050, float repetition_penalty = 1.05f,
                  float temperature = 0.9f, int32_t top_k = 50, const int32_t * instruct_tokens = nullptr,
                  int32_t n_instruct = 0, float eos_bias = 0.0f, int32_t target_frames = 0,
                  bool rep_loop_detect = false, const FrameCallback & on_frame = nullptr);

    bool generate_icl(const int32_t * text_tokens, int32_t n_tokens, const int32_t * ref_text_tokens,
                      int32_t n_ref_text, const int32_t * ref_codec_tokens, int32_t n_ref_frames,
                      const float * speaker_embd, int32_t max_len, std::vector<int32_t> & output,
                      int32_t language_id = 2050, float repetition_penalty = 1.05f, float temperature = 0.9f,
                      int32_t top_k = 50, float eos_bias = 0.0f, int32_t target_frames = 0,
                      bool rep_loop_detect = true, const FrameCallback & on_frame = nullptr);

    const tts_transformer_config & get_config() const { return config_; }
    const std::string & get_error() const { return error_msg_; }

    bool forward(const int32_t * tokens, int32_t n_tokens, int32_t n_past, std::vector<float> & output);
    bool forward_with_audio(const int32_t * tokens, int32_t n_tokens, const float * audio_embd, int32_t n_audio,
                            int32_t audio_start_pos, int32_t n_past, std::vector<float> & output);

    // Not in the reference: the sampler's RNG seed (the reference seeds
    // std::mt19937 from std::random_device; the device sampler is Philox
    // keyed by this seed, so a fixed seed makes sampled decoding repeatable).
    void set_seed(uint64_t seed) { seed_ = seed; }

    // Not in the reference: the device address of generate()'s code rows
    // (frame f's n_codebooks codes at + f * n_codebooks), complete for every
    // frame passed to the FrameCallback so far.  A streaming vocoder reads
    // them in place (AudioTokenizerDecoder::decode_window_device) instead of
    // the host codes_total the reference's driver hands to decode_window
    // (src/qwen3_tts.cpp:294-306).  NULL before the first generate().
    const int32_t * device_frame_codes() const;

private:
    bool build_prefill_graph(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd,
                             int32_t language_id, std::vector<float> & prefill_embd,
                             std::vector<float> & trailing_text_hidden, std::vector<float> & tts_pad_embed,
                             const int32_t * instruct_tokens = nullptr, int32_t n_instruct = 0);
    bool build_prefill_graph_icl(const int32_t * text_tokens, int32_t n_tokens, const int32_t * ref_text_tokens,
                                 int32_t n_ref_text, const int32_t * ref_codec_tokens, int32_t n_ref_frames,
                                 const float * speaker_embd, std::vector<float> & prefill_embd,
                                 std::vector<float> & trailing_text_hidden, std::vector<float> & tts_pad_embed);
    bool project_text_tokens(const int32_t * text_tokens, int32_t n_tokens, std::vector<float> & output);
    bool lookup_rows(int32_t table, int32_t index, const int32_t * ids, int32_t n, std::vector<float> & out);
    // figures of the QWEN3_TTS_TIMING report
    struct gen_timing;
    bool run_frames(const std::vector<float> & prefill, const std::vector<float> & trailing,
                    const std::vector<float> & pad, int32_t max_len, float repetition_penalty, float temperature,
                    int32_t top_k, float eos_bias, int32_t target_frames, bool rep_loop_detect,
                    const FrameCallback & on_frame, std::vector<int32_t> & output, gen_timing * tm);
    bool dev_ok(int rc);
    bool write_attn_dump();
    static void print_timing(const gen_timing & t);

    q3t_dev * dev_ = nullptr;
    tts_transformer_config config_;
    std::string error_msg_;
    std::vector<float> last_hidden_;
    int32_t kv_n_ctx_ = 0;
    int32_t kv_n_used_ = 0;
    uint64_t seed_ = std::random_device{}();
    uint32_t sample_calls_ = 0;
    bool debug_dump_ = false;
    bool attn_dump_ = false;
    int attn_dump_layer_ = 27;
    std::string attn_dump_path_;
    std::vector<std::vector<float>> attn_rows_;
};

// A GGUF file's hyperparameters as load_model parses them (primary keys, then
// the converter's aliases, then the defaults; src/tts_transformer.cpp:228-377),
// and a check that every talker / code-predictor tensor has a type this build
// loads (F32, F16, Q8_0).  No device is touched.  False with `err` set when
// the file cannot be read or a tensor type is unsupported.
bool load_gguf_config(const std::string & path, tts_transformer_config & out, std::string & err);

}  // namespace qwen3_tts
