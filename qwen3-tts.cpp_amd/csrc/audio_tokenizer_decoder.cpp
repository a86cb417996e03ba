// audio_tokenizer_decoder.cpp -- AudioTokenizerDecoder over q3t_voc: GGUF
// loading (src/audio_tokenizer_decoder.cpp:102-370) and the decode /
// decode_window entry points (:877-1024).  No arithmetic here.
#include "audio_tokenizer_decoder.h"

#include "gguf_reader.h"
#include "../../include/q3t_voc.h"

#include <cstdio>
#include <cstring>
#include <map>

namespace qwen3_tts {

namespace {

const GGUFTensorInfo * find(const std::map<std::string, const GGUFTensorInfo *> & m, const std::string & n) {
    auto it = m.find(n);
    return it == m.end() ? nullptr : it->second;
}

}  // namespace

AudioTokenizerDecoder::AudioTokenizerDecoder() = default;

AudioTokenizerDecoder::~AudioTokenizerDecoder() { unload_model(); }

void AudioTokenizerDecoder::unload_model() {
    if (voc_) q3t_voc_destroy(voc_);
    voc_ = nullptr;
}

bool AudioTokenizerDecoder::load_model(const std::string & model_path) {
    unload_model();
    GGUFReader g;
    if (!g.open(model_path)) {
        error_msg_ = g.error();
        return false;
    }
    audio_decoder_config cfg;
    uint32_t u = 0;
    if (g.get_u32("qwen3-tts.tokenizer.sample_rate", u)) cfg.sample_rate = (int32_t) u;
    if (g.get_u32("qwen3-tts.tokenizer.num_codebooks", u)) cfg.n_codebooks = (int32_t) u;
    if (g.get_u32("qwen3-tts.tokenizer.codebook_size", u)) cfg.codebook_size = (int32_t) u;
    std::map<std::string, const GGUFTensorInfo *> dec;
    for (const GGUFTensorInfo & t : g.tensors())
        if (t.name.compare(0, 8, "tok_dec.") == 0) dec[t.name] = &t;
    if (dec.empty()) {
        error_msg_ = "No decoder tensors found in model";
        return false;
    }
    // widths the reference keeps as audio_decoder_config defaults, read from
    // the tensor shapes (equal to the defaults for the 12 Hz tokenizer)
    const GGUFTensorInfo * cb = find(dec, "tok_dec.vq_first.0.codebook");
    const GGUFTensorInfo * op = find(dec, "tok_dec.vq_first.output_proj.weight");
    const GGUFTensorInfo * pc = find(dec, "tok_dec.pre_conv.weight");
    const GGUFTensorInfo * gt = find(dec, "tok_dec.pre_tfm.blk.0.ffn_gate.weight");
    const GGUFTensorInfo * p1 = find(dec, "tok_dec.upsample.0.pwconv1.weight");
    const GGUFTensorInfo * uc = find(dec, "tok_dec.upsample.0.conv.weight");
    const GGUFTensorInfo * d0 = find(dec, "tok_dec.dec.0.conv.weight");
    if (!cb || !op || !pc || !gt || !p1 || !uc || !d0) {
        error_msg_ = "decoder tensors missing";
        return false;
    }
    q3t_voc_config vc{};
    vc.n_codebooks = cfg.n_codebooks;
    vc.codebook_size = (int32_t) cb->ne[1];
    vc.codebook_dim = (int32_t) cb->ne[0];
    vc.hidden = (int32_t) op->ne[2];
    vc.latent = (int32_t) pc->ne[2];
    int32_t n_layers = 0;
    while (find(dec, "tok_dec.pre_tfm.blk." + std::to_string(n_layers) + ".attn_norm.weight")) ++n_layers;
    vc.n_layers = n_layers;
    vc.n_heads = vc.latent / 64;                   // head_dim 64 (docs/model_inspection.txt:789)
    vc.ffn = (int32_t) gt->ne[1];
    vc.cnx_ffn = (int32_t) p1->ne[1];
    vc.up_kernel = (int32_t) uc->ne[0];
    vc.decoder_dim = (int32_t) d0->ne[2];
    for (int i = 0; i < 4; ++i) {
        vc.rates[i] = cfg.upsample_rates[i];
        const GGUFTensorInfo * ct = find(dec, "tok_dec.dec." + std::to_string(i + 1) + ".conv_t.weight");
        vc.dec_kernel[i] = ct ? (int32_t) ct->ne[0] : 2 * cfg.upsample_rates[i];
    }
    vc.rms_eps = cfg.rms_norm_eps;
    vc.rope_theta = cfg.rope_theta;
    const char * err = nullptr;
    voc_ = q3t_voc_create(&vc, 0, &err);
    if (!voc_) {
        error_msg_ = err ? err : "q3t_voc_create failed";
        return false;
    }
    std::vector<uint8_t> buf;
    for (const auto & kv : dec) {
        const GGUFTensorInfo & t = *kv.second;
        if (!g.read_tensor(t, buf)) {
            error_msg_ = g.error();
            unload_model();
            return false;
        }
        if (q3t_voc_set_tensor(voc_, t.name.c_str(), t.type, buf.data(), buf.size()) != 0) {
            error_msg_ = q3t_voc_last_error(voc_);
            unload_model();
            return false;
        }
    }
    if (q3t_voc_finalize(voc_) != 0) {
        error_msg_ = q3t_voc_last_error(voc_);
        unload_model();
        return false;
    }
    cfg.codebook_size = vc.codebook_size;
    cfg.codebook_dim = vc.codebook_dim;
    cfg.latent_dim = vc.latent;
    cfg.hidden_dim = vc.hidden;
    cfg.n_pre_tfm_layers = vc.n_layers;
    cfg.n_heads = vc.n_heads;
    cfg.ffn_dim = vc.ffn;
    cfg.decoder_dim = vc.decoder_dim;
    config_ = cfg;
    fprintf(stderr, "  AudioTokenizerDecoder backend: MI355X (HIP)\n");
    return true;
}

bool AudioTokenizerDecoder::window(const int32_t * codes, int on_device, int32_t n_frames, int32_t start_frame,
                                   int32_t end_frame, int32_t context_frames, std::vector<float> & out_new) {
    if (!voc_) {
        error_msg_ = "Model not loaded";
        return false;
    }
    if (start_frame < 0 || end_frame <= start_frame || end_frame > n_frames) {
        error_msg_ = "decode_window: invalid frame range";
        return false;
    }
    const int32_t ctx_start = start_frame - (context_frames > 0 ? context_frames : 0);
    const int64_t cap = q3t_voc_samples_for_frames(voc_, end_frame - (ctx_start > 0 ? ctx_start : 0));
    const size_t at = out_new.size();
    out_new.resize(at + (size_t) cap);
    int64_t n = 0;
    if (q3t_voc_decode_window(voc_, codes, on_device, n_frames, start_frame, end_frame, context_frames,
                              out_new.data() + at, cap, &n) != 0) {
        out_new.resize(at);
        error_msg_ = q3t_voc_last_error(voc_);
        return false;
    }
    out_new.resize(at + (size_t) n);
    return true;
}

bool AudioTokenizerDecoder::decode_window(const int32_t * codes, int32_t n_frames, int32_t start_frame,
                                          int32_t end_frame, int32_t context_frames, std::vector<float> & out_new) {
    return window(codes, 0, n_frames, start_frame, end_frame, context_frames, out_new);
}

bool AudioTokenizerDecoder::decode_window_device(const int32_t * device_codes, int32_t n_frames,
                                                 int32_t start_frame, int32_t end_frame, int32_t context_frames,
                                                 std::vector<float> & out_new) {
    return window(device_codes, 1, n_frames, start_frame, end_frame, context_frames, out_new);
}

bool AudioTokenizerDecoder::decode(const int32_t * codes, int32_t n_frames, std::vector<float> & samples) {
    if (!voc_) {
        error_msg_ = "Model not loaded";
        return false;
    }
    samples.clear();
    if (n_frames <= 0) return true;
    return window(codes, 0, n_frames, 0, n_frames, 0, samples);
}

}  // namespace qwen3_tts
