// audio_tokenizer_decoder.h -- drop-in AudioTokenizerDecoder (the vocoder)
// over the MI355X device vocoder (include/q3t_voc.h).
//
// Same class name, namespace and public methods as the reference
// (src/audio_tokenizer_decoder.h:160-232), so Qwen3TTS and the streaming
// driver (src/qwen3_tts.cpp:271-316) compile against it unchanged; the
// compute runs in libq3t_hip.so.  One addition: decode_window_device reads the
// codes from device memory, e.g. the frame loop's code rows
// (TTSTransformer::device_frame_codes), so a streaming caller does not copy
// codes to the host per frame.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

struct q3t_voc;

namespace qwen3_tts {

// audio_decoder_config (src/audio_tokenizer_decoder.h:15-29); load_model
// fills it from the GGUF (the three tokenizer keys the reference reads, the
// rest from the tensor shapes, which for the 12 Hz tokenizer equal the
// reference's defaults).
struct audio_decoder_config {
    int32_t sample_rate = 24000;
    int32_t n_codebooks = 16;
    int32_t codebook_size = 2048;
    int32_t codebook_dim = 256;
    int32_t latent_dim = 1024;
    int32_t hidden_dim = 512;
    int32_t n_pre_tfm_layers = 8;
    int32_t n_heads = 16;
    int32_t ffn_dim = 1024;
    int32_t decoder_dim = 1536;
    int32_t upsample_rates[4] = {8, 5, 4, 3};
    float rms_norm_eps = 1e-5f;
    float rope_theta = 10000.0f;
};

class AudioTokenizerDecoder {
public:
    AudioTokenizerDecoder();
    ~AudioTokenizerDecoder();

    bool load_model(const std::string & model_path);
    void unload_model();

    // codes [n_frames][n_codebooks] int32 (row-major); samples at 24 kHz
    bool decode(const int32_t * codes, int32_t n_frames, std::vector<float> & samples);

    // frames [start_frame, end_frame) with context_frames of warm-up before
    // start_frame; appends only the new samples to out_new
    bool decode_window(const int32_t * codes, int32_t n_frames, int32_t start_frame, int32_t end_frame,
                       int32_t context_frames, std::vector<float> & out_new);

    // the same with codes in device memory (no counterpart in the reference)
    bool decode_window_device(const int32_t * device_codes, int32_t n_frames, int32_t start_frame,
                              int32_t end_frame, int32_t context_frames, std::vector<float> & out_new);

    const audio_decoder_config & get_config() const { return config_; }
    const std::string & get_error() const { return error_msg_; }

private:
    bool window(const int32_t * codes, int on_device, int32_t n_frames, int32_t start_frame, int32_t end_frame,
                int32_t context_frames, std::vector<float> & out_new);

    audio_decoder_config config_;
    q3t_voc * voc_ = nullptr;
    std::string error_msg_;
};

}  // namespace qwen3_tts
