// tts_transformer.cpp -- TTSTransformer over the MI355X device layer.
//
// Host control flow restated from the reference (src/tts_transformer.cpp):
// GGUF key parsing (:228-377), prefill layouts (:1030-1472), forward
// wrappers (:2217-2509), the generate()/generate_icl() frame loops
// (:3007-3656).  Every tensor operation goes through include/q3t_dev.h.
#include "tts_transformer.h"

#include "../../include/q3t_dev.h"
#include "gguf_reader.h"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>

namespace qwen3_tts {

namespace {

q3t_config to_dev_config(const tts_transformer_config & c) {
    q3t_config d{};
    d.hidden_size = c.hidden_size; d.n_layers = c.n_layers; d.n_head = c.n_attention_heads;
    d.n_kv_head = c.n_key_value_heads; d.head_dim = c.head_dim; d.ffn_size = c.intermediate_size;
    d.codec_vocab = c.codec_vocab_size; d.n_codebooks = c.n_codebooks; d.cp_layers = c.code_pred_layers;
    d.cp_vocab = c.code_pred_vocab_size; d.cp_hidden = c.code_pred_hidden_size;
    d.cp_ffn = c.code_pred_intermediate_size; d.text_vocab = c.text_vocab_size; d.text_embd_dim = c.text_embd_dim;
    d.rms_eps = c.rms_norm_eps; d.rope_theta = c.rope_theta; d.cp_rope_theta = c.code_pred_rope_theta;
    d.codec_pad_id = c.codec_pad_id; d.codec_bos_id = c.codec_bos_id; d.codec_eos_id = c.codec_eos_id;
    d.tts_bos_id = c.tts_bos_token_id; d.tts_eos_id = c.tts_eos_token_id; d.tts_pad_id = c.tts_pad_token_id;
    d.codec_think_id = c.codec_think_id; d.codec_nothink_id = c.codec_nothink_id;
    d.codec_think_bos_id = c.codec_think_bos_id; d.codec_think_eos_id = c.codec_think_eos_id;
    d.english_language_id = c.english_language_id;
    return d;
}

// GGUF keys and fallbacks of parse_config (src/tts_transformer.cpp:250-374).
void parse_config(const GGUFReader & g, tts_transformer_config & cfg) {
    auto u32 = [&](std::initializer_list<const char *> keys, int32_t def) -> int32_t {
        for (const char * k : keys) { uint32_t v; if (g.get_u32(k, v)) return (int32_t) v; }
        return def;
    };
    auto f32 = [&](std::initializer_list<const char *> keys, float def) -> float {
        for (const char * k : keys) { float v; if (g.get_f32(k, v)) return v; }
        return def;
    };
    cfg.text_vocab_size = u32({"qwen3-tts.text.vocab_size", "qwen3-tts.text_vocab_size"}, 151936);
    cfg.text_embd_dim = u32({"qwen3-tts.text.embedding_dim", "qwen3-tts.text_hidden_size"}, 2048);
    cfg.hidden_size = u32({"qwen3-tts.talker.embedding_length", "qwen3-tts.embedding_length"}, 1024);
    cfg.n_layers = u32({"qwen3-tts.talker.block_count", "qwen3-tts.block_count"}, 28);
    cfg.n_attention_heads = u32({"qwen3-tts.talker.attention.head_count", "qwen3-tts.attention.head_count"}, 16);
    cfg.n_key_value_heads = u32({"qwen3-tts.talker.attention.head_count_kv", "qwen3-tts.attention.head_count_kv"}, 8);
    cfg.intermediate_size = u32({"qwen3-tts.talker.feed_forward_length", "qwen3-tts.feed_forward_length"}, 3072);
    cfg.head_dim = u32({"qwen3-tts.talker.attention.key_length", "qwen3-tts.attention.key_length"}, 128);
    cfg.rms_norm_eps = f32({"qwen3-tts.talker.attention.layer_norm_rms_epsilon",
                            "qwen3-tts.attention.layer_norm_rms_epsilon"}, 1e-6f);
    cfg.rope_theta = f32({"qwen3-tts.talker.rope.freq_base", "qwen3-tts.rope.freq_base"}, 1000000.0f);
    cfg.codec_vocab_size = u32({"qwen3-tts.talker.codec_vocab_size", "qwen3-tts.vocab_size"}, 3072);
    cfg.n_codebooks = u32({"qwen3-tts.talker.num_codebooks", "qwen3-tts.num_code_groups"}, 16);
    cfg.code_pred_layers = u32({"qwen3-tts.code_pred.layer_count", "qwen3-tts.code_predictor.layer_count"}, 5);
    cfg.code_pred_vocab_size = u32({"qwen3-tts.code_pred.vocab_size", "qwen3-tts.code_predictor.vocab_size"}, 2048);
    cfg.code_pred_hidden_size = u32({"qwen3-tts.code_pred.embedding_length",
                                     "qwen3-tts.code_predictor.embedding_length"}, 1024);
    cfg.code_pred_intermediate_size = u32({"qwen3-tts.code_pred.feed_forward_length",
                                           "qwen3-tts.code_predictor.feed_forward_length"}, 3072);
    // code-predictor theta falls back to the talker's (both HF configs use 1e6)
    cfg.code_pred_rope_theta = f32({"qwen3-tts.code_pred.rope.freq_base", "qwen3-tts.code_predictor.rope.freq_base"},
                                   cfg.rope_theta);
    cfg.codec_pad_id = u32({"qwen3-tts.codec.pad_id"}, 2148);
    cfg.codec_bos_id = u32({"qwen3-tts.codec.bos_id"}, 2149);
    cfg.codec_eos_id = u32({"qwen3-tts.codec.eos_id", "qwen3-tts.codec.eos_token_id"}, 2150);
    cfg.tts_bos_token_id = u32({"qwen3-tts.tts_bos_token_id", "qwen3-tts.tts.bos_token_id", "qwen3-tts.tts.bos_id"}, 151672);
    cfg.tts_eos_token_id = u32({"qwen3-tts.tts_eos_token_id", "qwen3-tts.tts.eos_token_id", "qwen3-tts.tts.eos_id"}, 151673);
    cfg.tts_pad_token_id = u32({"qwen3-tts.tts_pad_token_id", "qwen3-tts.tts.pad_token_id", "qwen3-tts.tts.pad_id"}, 151671);
    cfg.codec_think_id = u32({"qwen3-tts.codec.think_id", "qwen3-tts.codec_think_id"}, 2154);
    cfg.codec_nothink_id = u32({"qwen3-tts.codec.nothink_id", "qwen3-tts.codec_nothink_id"}, 2155);
    cfg.codec_think_bos_id = u32({"qwen3-tts.codec.think_bos_id", "qwen3-tts.codec_think_bos_id"}, 2156);
    cfg.codec_think_eos_id = u32({"qwen3-tts.codec.think_eos_id", "qwen3-tts.codec_think_eos_id"}, 2157);
    cfg.english_language_id = u32({"qwen3-tts.language.english_id", "qwen3-tts.codec.language.english_id",
                                   "qwen3-tts.language_id"}, 2050);
}

// The first talker / code-predictor tensor of a type this build cannot load
// (it would otherwise surface later as a missing tensor): false with `err`.
bool check_tensor_types(const GGUFReader & g, std::string & err) {
    for (const GGUFTensorInfo & t : g.tensors()) {
        const bool ours = t.name.rfind("talker.", 0) == 0 || t.name.rfind("code_pred.", 0) == 0;
        if (ours && t.nbytes == 0) {
            err = "unsupported tensor type " + gguf_type_name(t.type) + " for " + t.name +
                  " (this build loads F32, F16 and Q8_0 tensors: convert with --type f16 or q8_0)";
            return false;
        }
    }
    return true;
}

uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

}  // namespace

TTSTransformer::TTSTransformer() = default;

TTSTransformer::~TTSTransformer() { unload_model(); }

const int32_t * TTSTransformer::device_frame_codes() const { return dev_ ? q3t_dev_frame_codes(dev_) : nullptr; }

bool TTSTransformer::dev_ok(int rc) {
    if (rc == 0) return true;
    error_msg_ = dev_ ? q3t_dev_last_error(dev_) : "device not initialised";
    if (error_msg_.empty()) error_msg_ = "device call failed";
    return false;
}

void TTSTransformer::unload_model() {
    if (dev_) { q3t_dev_destroy(dev_); dev_ = nullptr; }
    last_hidden_.clear();
    kv_n_ctx_ = 0;
    kv_n_used_ = 0;
}

void TTSTransformer::set_n_threads(int32_t) {}

bool load_gguf_config(const std::string & path, tts_transformer_config & out, std::string & err) {
    GGUFReader g;
    if (!g.open(path)) { err = g.error(); return false; }
    parse_config(g, out);
    return check_tensor_types(g, err);
}

bool TTSTransformer::load_model(const std::string & model_path) {
    unload_model();
    GGUFReader g;
    if (!g.open(model_path)) { error_msg_ = g.error(); return false; }
    parse_config(g, config_);
    if (!check_tensor_types(g, error_msg_)) return false;
    const q3t_config dc = to_dev_config(config_);
    int device = 0;
    if (const char * e = std::getenv("QWEN3_TTS_DEVICE")) device = std::atoi(e);
    const int rc = q3t_dev_create(&dc, device, &dev_);
    if (rc != 0) {
        error_msg_ = dev_ ? q3t_dev_last_error(dev_) : "no HIP device available for TTSTransformer";
        if (dev_) { q3t_dev_destroy(dev_); dev_ = nullptr; }
        return false;
    }
    // Tensors go to HBM in row ranges through the context's pinned staging
    // buffer (64 MiB): host memory stays bounded whatever the tensor size (the
    // text embedding alone is 622 MB at F16), and each range is one DMA.
    for (const GGUFTensorInfo & t : g.tensors()) {
        if (t.name.find("spk_enc.") != std::string::npos || t.name.find("tok_") != std::string::npos) continue;
        if (t.nbytes == 0) continue;      // not ours (checked above)
        const int64_t rows = t.n_dims >= 2 ? t.ne[1] * t.ne[2] * t.ne[3] : 1;
        const size_t row_bytes = t.nbytes / (size_t) rows;
        size_t cap = 0;
        uint8_t * stage = (uint8_t *) q3t_dev_staging(dev_, row_bytes, &cap);
        if (!stage) { dev_ok(-1); unload_model(); return false; }
        const int64_t per = (int64_t) std::max<size_t>(1, cap / row_bytes);
        for (int64_t r0 = 0; r0 < rows; r0 += per) {
            const int64_t n = std::min(per, rows - r0);
            if (!g.read_tensor_rows(t, r0, n, stage)) { error_msg_ = g.error(); unload_model(); return false; }
            if (!dev_ok(q3t_dev_upload_tensor_rows(dev_, t.name.c_str(), t.type, t.ne, r0, n, stage,
                                                   row_bytes * (size_t) n))) {
                unload_model();
                return false;
            }
        }
    }
    fprintf(stderr, "  TTSTransformer backend: HIP (MI355X frame loop)\n");
    return true;
}

bool TTSTransformer::init_kv_cache(int32_t n_ctx) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!dev_ok(q3t_dev_kv_reserve(dev_, n_ctx))) return false;
    kv_n_ctx_ = n_ctx;
    kv_n_used_ = 0;
    return true;
}

void TTSTransformer::clear_kv_cache() { kv_n_used_ = 0; }

// The device keeps a fixed 16-position code-predictor cache per context
// (the most a frame uses: 2-token prefill + 14 steps).
bool TTSTransformer::init_code_pred_kv_cache(int32_t n_ctx) {
    if (n_ctx > 16) { error_msg_ = "code predictor cache holds 16 positions"; return false; }
    return true;
}

void TTSTransformer::clear_code_pred_kv_cache() {}

bool TTSTransformer::lookup_rows(int32_t table, int32_t index, const int32_t * ids, int32_t n,
                                 std::vector<float> & out) {
    const int32_t dim = table == 2 ? config_.text_embd_dim : config_.hidden_size;
    out.resize((size_t) n * dim);
    return dev_ok(q3t_dev_embed_rows(dev_, table, index, ids, n, out.data()));
}

bool TTSTransformer::project_text_tokens(const int32_t * text_tokens, int32_t n_tokens, std::vector<float> & output) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (n_tokens <= 0) { output.clear(); return true; }
    output.resize((size_t) n_tokens * config_.hidden_size);
    return dev_ok(q3t_dev_text_proj(dev_, text_tokens, n_tokens, output.data()));
}

bool TTSTransformer::forward_prefill(const float * prefill_embd, int32_t n_tokens, int32_t n_past,
                                     std::vector<float> & output, std::vector<float> * logits_out) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!prefill_embd) { error_msg_ = "prefill_embd is null"; return false; }
    if (n_tokens <= 0) { error_msg_ = "n_tokens must be > 0"; return false; }
    if (kv_n_ctx_ == 0 && !init_kv_cache(std::max<int32_t>(256, n_past + n_tokens + 16))) return false;
    if (n_past + n_tokens > kv_n_ctx_) { error_msg_ = "Context length exceeded"; return false; }
    const int32_t d = config_.hidden_size;
    output.resize((size_t) n_tokens * d);
    std::vector<float> logits(config_.codec_vocab_size);
    if (!dev_ok(q3t_dev_prefill(dev_, prefill_embd, n_tokens, n_past, output.data(), logits.data()))) return false;
    last_hidden_.assign(output.end() - d, output.end());
    if (logits_out) *logits_out = logits;
    kv_n_used_ = n_past + n_tokens;
    return true;
}

bool TTSTransformer::forward_text(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd,
                                  int32_t n_past, std::vector<float> & output) {
    if (!text_tokens) { error_msg_ = "text_tokens is null"; return false; }
    if (n_tokens <= 0) { error_msg_ = "n_tokens must be > 0"; return false; }
    std::vector<float> projected;
    if (!project_text_tokens(text_tokens, n_tokens, projected)) return false;
    if (speaker_embd) {
        const int32_t d = config_.hidden_size;
        for (int32_t t = 0; t < n_tokens; ++t)
            for (int32_t h = 0; h < d; ++h) projected[(size_t) t * d + h] += speaker_embd[h];
    }
    return forward_prefill(projected.data(), n_tokens, n_past, output, nullptr);
}

bool TTSTransformer::forward_step(const float * step_embd, int32_t n_past, std::vector<float> & output,
                                  std::vector<float> * hidden_out) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!step_embd) { error_msg_ = "step_embd is null"; return false; }
    if (kv_n_ctx_ == 0 && !init_kv_cache(std::max<int32_t>(256, n_past + 1 + 16))) return false;
    if (n_past + 1 > kv_n_ctx_) { error_msg_ = "Context length exceeded"; return false; }
    output.resize(config_.codec_vocab_size);
    last_hidden_.resize(config_.hidden_size);
    // forward_step keeps the dump layer's attention row (src/tts_transformer.cpp:2485-2497)
    if (!dev_ok(q3t_dev_set_attn_capture(dev_, attn_dump_ ? attn_dump_layer_ : -1))) return false;
    if (!dev_ok(q3t_dev_talker_step(dev_, step_embd, n_past, output.data(), last_hidden_.data()))) return false;
    if (attn_dump_) {
        int32_t n_kv = 0;
        std::vector<float> row((size_t) config_.n_attention_heads * (n_past + 1));
        if (!dev_ok(q3t_dev_attn_row(dev_, 0, row.data(), (int64_t) row.size(), &n_kv))) return false;
        attn_rows_.push_back(std::move(row));
    }
    if (hidden_out) *hidden_out = last_hidden_;
    kv_n_used_ = n_past + 1;
    return true;
}

bool TTSTransformer::forward_codec(int32_t codec_token, int32_t n_past, std::vector<float> & output) {
    std::vector<float> row;
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!lookup_rows(0, 0, &codec_token, 1, row)) return false;
    return forward_step(row.data(), n_past, output, nullptr);
}

bool TTSTransformer::get_hidden_states(std::vector<float> & hidden) const {
    if (last_hidden_.empty()) return false;
    hidden = last_hidden_;
    return true;
}

// The single-pass predictor (src/tts_transformer.cpp:2531-2581): output is
// [15][code_pred_vocab_size] logits; prev_codes, when not null, holds the 15
// previous codes whose code-predictor embeddings join the input row.
bool TTSTransformer::predict_codes(const float * hidden, const int32_t * prev_codes, std::vector<float> & output) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!hidden) { error_msg_ = "hidden is null"; return false; }
    output.resize((size_t) (config_.n_codebooks - 1) * config_.code_pred_vocab_size);
    return dev_ok(q3t_dev_predict_codes(dev_, hidden, prev_codes, output.data()));
}

bool TTSTransformer::predict_codes_autoregressive(const float * hidden, int32_t codebook_0_token,
                                                  std::vector<int32_t> & output, float temperature, int32_t top_k) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (kv_n_ctx_ == 0 && !init_kv_cache(256)) return false;
    output.resize(config_.n_codebooks - 1);
    q3t_sampling s{temperature, top_k, seed_};
    return dev_ok(q3t_dev_code_pred(dev_, hidden, codebook_0_token, &s, sample_calls_++, output.data(), nullptr));
}

bool TTSTransformer::build_prefill_graph(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd,
                                         int32_t language_id, std::vector<float> & prefill_embd,
                                         std::vector<float> & trailing_text_hidden, std::vector<float> & tts_pad_embed,
                                         const int32_t * instruct_tokens, int32_t n_instruct) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!text_tokens) { error_msg_ = "text_tokens is null"; return false; }
    if (n_tokens < 4) { error_msg_ = "Need at least 4 text tokens for prefill"; return false; }
    const int32_t d = config_.hidden_size;
    int32_t n_pre = 0, n_trail = 0;
    if (!dev_ok(q3t_dev_build_prefill(dev_, text_tokens, n_tokens, speaker_embd, language_id, instruct_tokens,
                                      n_instruct, nullptr, &n_pre, nullptr, &n_trail, nullptr)))
        return false;
    prefill_embd.resize((size_t) n_pre * d);
    trailing_text_hidden.resize((size_t) n_trail * d);
    tts_pad_embed.resize(d);
    return dev_ok(q3t_dev_build_prefill(dev_, text_tokens, n_tokens, speaker_embd, language_id, instruct_tokens,
                                        n_instruct, prefill_embd.data(), &n_pre, trailing_text_hidden.data(), &n_trail,
                                        tts_pad_embed.data()));
}

bool TTSTransformer::build_prefill_graph_icl(const int32_t * text_tokens, int32_t n_tokens,
                                             const int32_t * ref_text_tokens, int32_t n_ref_text,
                                             const int32_t * ref_codec_tokens, int32_t n_ref_frames,
                                             const float * speaker_embd, std::vector<float> & prefill_embd,
                                             std::vector<float> & trailing_text_hidden,
                                             std::vector<float> & tts_pad_embed) {
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!text_tokens || n_tokens < 4) { error_msg_ = "ICL: need at least 4 target text tokens"; return false; }
    if (!ref_codec_tokens || n_ref_frames < 1) { error_msg_ = "ICL: need at least 1 reference codec frame"; return false; }
    const int32_t d = config_.hidden_size;
    int32_t n_pre = 0, n_trail = 0;
    if (!dev_ok(q3t_dev_build_prefill_icl(dev_, text_tokens, n_tokens, ref_text_tokens, n_ref_text, ref_codec_tokens,
                                          n_ref_frames, speaker_embd, nullptr, &n_pre, nullptr, &n_trail, nullptr)))
        return false;
    prefill_embd.resize((size_t) n_pre * d);
    trailing_text_hidden.resize((size_t) n_trail * d);
    tts_pad_embed.resize(d);
    return dev_ok(q3t_dev_build_prefill_icl(dev_, text_tokens, n_tokens, ref_text_tokens, n_ref_text,
                                            ref_codec_tokens, n_ref_frames, speaker_embd, prefill_embd.data(), &n_pre,
                                            trailing_text_hidden.data(), &n_trail, tts_pad_embed.data()));
}

// The QWEN3_TTS_TIMING report (src/tts_transformer.h:20-46, printed at
// src/tts_transformer.cpp:3311-3352): compiled in with -DQWEN3_TTS_TIMING as
// in the reference, or switched on at run time with QWEN3_TTS_TIMING=1.  The
// device runs the codebook-0 sampler, the code predictor, the step embedding
// and the talker step of a frame in one launch, so the frame loop is one
// figure (wall time, and the GPU time of the frame launches from HIP events)
// where the reference splits talker and code-predictor graphs.
struct TTSTransformer::gen_timing {
    double build_ms = 0, prefill_ms = 0, frames_ms = 0, frames_gpu_ms = 0, callback_ms = 0, total_ms = 0;
    int32_t prefill_rows = 0, frames = 0, path = -1;
    int64_t launches = 0;
};

namespace {

using timing_clock = std::chrono::steady_clock;

double ms_since(timing_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(timing_clock::now() - t0).count();
}

bool timing_enabled() {
#ifdef QWEN3_TTS_TIMING
    return true;
#else
    static const bool on = [] {
        const char * e = std::getenv("QWEN3_TTS_TIMING");
        return e && *e && std::strcmp(e, "0") != 0;
    }();
    return on;
#endif
}

const char * frame_path_name(int32_t path) {
    switch (path) {
        case 1: return "persistent frame kernel, row-parallel layers";
        case 3: return "persistent frame kernel, XCD-parallel layers";
        case 0: return "captured multi-kernel graph";
        case 2: return "multi-stream graph";
        default: return "none";
    }
}

// QWEN3_TTS_DUMP_CODES=<path> (src/tts_transformer.cpp:3356-3366, 3641-3651):
// after each generate / generate_icl the codes go to <path> as int32 n
// followed by the n int32 codes.  The reference compiles this in with
// -DQWEN3_TTS_DUMP_CODES; here the variable alone turns it on.
void dump_codes(const std::vector<int32_t> & output) {
    const char * path = std::getenv("QWEN3_TTS_DUMP_CODES");
    if (!path || !*path) return;
    FILE * f = fopen(path, "wb");
    if (!f) return;
    const int32_t n = (int32_t) output.size();
    fwrite(&n, sizeof n, 1, f);
    fwrite(output.data(), sizeof(int32_t), output.size(), f);
    fclose(f);
}

}  // namespace

bool TTSTransformer::run_frames(const std::vector<float> & prefill, const std::vector<float> & trailing,
                                const std::vector<float> & pad, int32_t max_len, float repetition_penalty,
                                float temperature, int32_t top_k, float eos_bias, int32_t target_frames,
                                bool rep_loop_detect, const FrameCallback & on_frame, std::vector<int32_t> & output,
                                gen_timing * tm) {
    const tts_transformer_config & cfg = config_;
    const int32_t d = cfg.hidden_size, ncb = cfg.n_codebooks;
    const int32_t plen = (int32_t) (prefill.size() / d);
    const int32_t required = plen + max_len + 8;
    if (kv_n_ctx_ < required || kv_n_ctx_ > std::max<int32_t>(required * 2, 512)) {
        if (!init_kv_cache(required)) return false;
    }
    clear_kv_cache();
    std::vector<float> hidden;
    auto t0 = timing_clock::now();
    if (!forward_prefill(prefill.data(), plen, 0, hidden, nullptr)) return false;
    if (tm) { tm->prefill_ms = ms_since(t0); tm->prefill_rows = plen; }
    q3t_frame_args a{};
    a.trailing = trailing.empty() ? nullptr : trailing.data();
    a.n_trailing = (int32_t) (trailing.size() / d);
    a.tts_pad = pad.data();
    a.n_past = plen;
    a.max_len = max_len;
    a.repetition_penalty = repetition_penalty;
    a.eos_bias = eos_bias;
    a.target_frames = target_frames;
    a.sampling = q3t_sampling{temperature, top_k, seed_};
    if (temperature > 0.0f) seed_ = splitmix64(seed_);   // next call draws a fresh stream
    // attention capture for set_attn_dump (src/tts_transformer.cpp:1719-1724)
    if (!dev_ok(q3t_dev_set_attn_capture(dev_, attn_dump_ ? attn_dump_layer_ : -1))) return false;
    if (!dev_ok(q3t_dev_frames_begin(dev_, &a))) return false;
    // Frames per q3t_dev_frames_run call.  With a callback every frame is
    // handed over before the next one is computed, as the reference does
    // (src/tts_transformer.cpp:3213): an abort wastes no frame and streaming
    // consumers see one frame at a time.  Without one, 8-frame chunks save
    // host synchronisations.  QWEN3_TTS_FRAME_CHUNK overrides both.
    int chunk = on_frame ? 1 : 8;
    if (const char * e = std::getenv("QWEN3_TTS_FRAME_CHUNK")) chunk = std::max(1, std::atoi(e));
    output.clear();
    output.reserve((size_t) max_len * ncb);
    std::vector<int32_t> buf((size_t) chunk * ncb);
    std::vector<std::vector<int32_t>> rep_frames;
    int32_t rep_run_len = 0, rep_run_start = 0;
    int32_t produced = 0, stop_frame = -1;
    t0 = timing_clock::now();
    while (produced < max_len) {
        const int32_t n = std::min(chunk, max_len - produced);
        int32_t got = 0, eos = 0;
        if (!dev_ok(q3t_dev_frames_run(dev_, n, buf.data(), &got, &eos))) return false;
        bool stop = false;
        for (int32_t f = 0; f < got && !stop; ++f) {
            const int32_t * codes = buf.data() + (size_t) f * ncb;
            const int32_t frame = produced + f;
            output.insert(output.end(), codes, codes + ncb);
            if (on_frame) {
                const auto tc = timing_clock::now();
                const bool go_on = on_frame(codes, ncb, frame);
                if (tm) tm->callback_ms += ms_since(tc);
                if (!go_on) { stop = true; stop_frame = frame; break; }
            }
            if (rep_loop_detect) rep_frames.emplace_back(codes, codes + ncb);
            const size_t nf = rep_frames.size();
            bool is_rep = false;
            for (int back = 1; back <= 6 && !is_rep && (size_t) back < nf; ++back) {
                int matches = 0;
                for (int cb = 0; cb < ncb; ++cb) matches += rep_frames[nf - 1][cb] == rep_frames[nf - 1 - back][cb];
                if (matches >= 10) is_rep = true;
            }
            if (is_rep) { if (rep_run_len == 0) rep_run_start = (int32_t) (nf - 1); ++rep_run_len; }
            else rep_run_len = 0;
            if (rep_run_len >= 5) {
                fprintf(stderr, "  Repetition loop detected at frame %d, truncating %d frames\n", (int) (nf - 1),
                        (int) rep_run_len);
                output.resize((size_t) rep_run_start * ncb);
                stop = true;
                stop_frame = frame;
            }
        }
        produced += got;
        if (stop || eos || got < n) break;
    }
    if (tm) {
        tm->frames_ms = ms_since(t0) - tm->callback_ms;
        tm->frames = (int32_t) (output.size() / ncb);
        double gpu_us = 0.0;
        if (q3t_dev_frames_stats(dev_, &gpu_us, &tm->launches, &tm->path) == 0) tm->frames_gpu_ms = gpu_us / 1000.0;
    }
    kv_n_used_ = plen + produced;
    if (attn_dump_) {
        // one row per talker step the reference takes: none for the frame
        // at which the loop stops (callback, repetition loop) or for frames
        // the device computed past it
        int32_t n_rows = q3t_dev_attn_row_count(dev_);
        if (stop_frame >= 0) n_rows = std::min(n_rows, stop_frame);
        attn_rows_.clear();
        for (int32_t i = 0; i < n_rows; ++i) {
            int32_t n_kv = 0;
            if (!dev_ok(q3t_dev_attn_row(dev_, i, nullptr, 0, &n_kv))) return false;
            std::vector<float> row((size_t) n_kv * cfg.n_attention_heads);
            if (!dev_ok(q3t_dev_attn_row(dev_, i, row.data(), (int64_t) row.size(), &n_kv))) return false;
            attn_rows_.push_back(std::move(row));
        }
    }
    return true;
}

bool TTSTransformer::generate(const int32_t * text_tokens, int32_t n_tokens, const float * speaker_embd,
                              int32_t max_len, std::vector<int32_t> & output, int32_t language_id,
                              float repetition_penalty, float temperature, int32_t top_k,
                              const int32_t * instruct_tokens, int32_t n_instruct, float eos_bias,
                              int32_t target_frames, bool rep_loop_detect, const FrameCallback & on_frame) {
    attn_rows_.clear();
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!text_tokens) { error_msg_ = "text_tokens is null"; return false; }
    if (n_tokens < 4) { error_msg_ = "Need at least 4 text tokens for generation"; return false; }
    if (max_len <= 0) { output.clear(); return true; }
    gen_timing timing, * tm = timing_enabled() ? &timing : nullptr;
    const auto t_start = timing_clock::now();
    std::vector<float> prefill, trailing, pad;
    if (!build_prefill_graph(text_tokens, n_tokens, speaker_embd, language_id, prefill, trailing, pad,
                             instruct_tokens, n_instruct))
        return false;
    if (tm) tm->build_ms = ms_since(t_start);
    if (!run_frames(prefill, trailing, pad, max_len, repetition_penalty, temperature, top_k, eos_bias, target_frames,
                    rep_loop_detect, on_frame, output, tm))
        return false;
    dump_codes(output);
    write_attn_dump();
    if (tm) { tm->total_ms = ms_since(t_start); print_timing(*tm); }
    return true;
}

bool TTSTransformer::generate_icl(const int32_t * text_tokens, int32_t n_tokens, const int32_t * ref_text_tokens,
                                  int32_t n_ref_text, const int32_t * ref_codec_tokens, int32_t n_ref_frames,
                                  const float * speaker_embd, int32_t max_len, std::vector<int32_t> & output,
                                  int32_t /*language_id*/, float repetition_penalty, float temperature, int32_t top_k,
                                  float eos_bias, int32_t target_frames, bool rep_loop_detect,
                                  const FrameCallback & on_frame) {
    attn_rows_.clear();
    if (!dev_) { error_msg_ = "Model not loaded"; return false; }
    if (!text_tokens || n_tokens < 4) { error_msg_ = "ICL: need at least 4 target text tokens"; return false; }
    if (!ref_codec_tokens || n_ref_frames < 1) { error_msg_ = "ICL: need at least 1 reference codec frame"; return false; }
    if (max_len <= 0) { output.clear(); return true; }
    gen_timing timing, * tm = timing_enabled() ? &timing : nullptr;
    const auto t_start = timing_clock::now();
    std::vector<float> prefill, trailing, pad;
    if (!build_prefill_graph_icl(text_tokens, n_tokens, ref_text_tokens, n_ref_text, ref_codec_tokens, n_ref_frames,
                                 speaker_embd, prefill, trailing, pad))
        return false;
    if (tm) tm->build_ms = ms_since(t_start);
    if (!run_frames(prefill, trailing, pad, max_len, repetition_penalty, temperature, top_k, eos_bias, target_frames,
                    rep_loop_detect, on_frame, output, tm))
        return false;
    dump_codes(output);
    write_attn_dump();
    if (tm) { tm->total_ms = ms_since(t_start); print_timing(*tm); }
    return true;
}

void TTSTransformer::print_timing(const gen_timing & t) {
    const int nf = t.frames;
    const double per = nf > 0 ? 1.0 / nf : 0.0;
    fprintf(stderr, "\n=== Detailed Generation Timing (%d frames) ===\n", nf);
    fprintf(stderr, "\n  Prefill:\n");
    fprintf(stderr, "    Build rows:       %8.1f ms   (text projection and prompt layout on the device)\n", t.build_ms);
    fprintf(stderr, "    Forward total:    %8.1f ms   (%d rows)\n", t.prefill_ms, t.prefill_rows);
    fprintf(stderr, "\n  Frame loop (codebook-0 sampler, code predictor, step embedding, talker step; total / per-frame):\n");
    fprintf(stderr, "    Implementation:   %s, %lld launches\n", frame_path_name(t.path), (long long) t.launches);
    fprintf(stderr, "    Total:            %8.1f ms   (%.3f ms/frame)\n", t.frames_ms, t.frames_ms * per);
    fprintf(stderr, "      GPU:            %8.1f ms   (%.3f ms/frame)\n", t.frames_gpu_ms, t.frames_gpu_ms * per);
    fprintf(stderr, "      Host and sync:  %8.1f ms   (%.3f ms/frame)\n", t.frames_ms - t.frames_gpu_ms,
            (t.frames_ms - t.frames_gpu_ms) * per);
    fprintf(stderr, "    Callbacks:        %8.1f ms\n", t.callback_ms);
    const double accounted = t.build_ms + t.prefill_ms + t.frames_ms + t.callback_ms;
    fprintf(stderr, "\n  Other/overhead:     %8.1f ms\n", t.total_ms - accounted);
    fprintf(stderr, "  -----------------------------------------\n");
    fprintf(stderr, "  Total generate:     %8.1f ms\n", t.total_ms);
    if (nf > 0)
        fprintf(stderr, "  Throughput:         %8.3f ms/frame (%.1f frames/s)\n", t.total_ms / nf,
                1000.0 * nf / t.total_ms);
}

bool TTSTransformer::forward(const int32_t * tokens, int32_t n_tokens, int32_t n_past, std::vector<float> & output) {
    return forward_text(tokens, n_tokens, nullptr, n_past, output);
}

bool TTSTransformer::forward_with_audio(const int32_t * tokens, int32_t n_tokens, const float *, int32_t, int32_t,
                                        int32_t n_past, std::vector<float> & output) {
    return forward_text(tokens, n_tokens, nullptr, n_past, output);
}

// The ATTD file of the reference (src/tts_transformer.cpp:2978-3005): magic,
// version 1, layer, n_head, n_rows, then per row n_kv and n_kv * n_head
// floats (heads as blocks of n_kv).
bool TTSTransformer::write_attn_dump() {
    if (!attn_dump_ || attn_dump_path_.empty() || attn_rows_.empty()) return true;
    FILE * f = fopen(attn_dump_path_.c_str(), "wb");
    if (!f) {
        fprintf(stderr, "attn-dump: cannot open %s for writing\n", attn_dump_path_.c_str());
        return false;
    }
    const int32_t n_head = config_.n_attention_heads, n_rows = (int32_t) attn_rows_.size(), version = 1;
    const uint32_t magic = 0x41545444u;
    bool ok = fwrite(&magic, 4, 1, f) == 1 && fwrite(&version, 4, 1, f) == 1 &&
              fwrite(&attn_dump_layer_, 4, 1, f) == 1 && fwrite(&n_head, 4, 1, f) == 1 && fwrite(&n_rows, 4, 1, f) == 1;
    for (const std::vector<float> & row : attn_rows_) {
        const int32_t n_kv = (int32_t) (row.size() / (size_t) n_head);
        ok = ok && fwrite(&n_kv, 4, 1, f) == 1 && fwrite(row.data(), sizeof(float), row.size(), f) == row.size();
    }
    ok = fclose(f) == 0 && ok;
    if (!ok) {
        fprintf(stderr, "attn-dump: write to %s failed\n", attn_dump_path_.c_str());
        return false;
    }
    fprintf(stderr, "attn-dump: wrote %d rows (layer %d, %d heads) to %s\n", n_rows, attn_dump_layer_, n_head,
            attn_dump_path_.c_str());
    return true;
}

}  // namespace qwen3_tts
