// Drives the drop-in AudioTokenizerDecoder (qwen3-tts.cpp_amd/csrc/
// audio_tokenizer_decoder.h) the way the reference's streaming synthesis
// does (src/qwen3_tts.cpp:271-316 and the tail flush :615-633): generate()
// with a FrameCallback that decodes a window every chunk frames with context
// frames of warm-up; here the windows read the frame loop's device code rows
// (TTSTransformer::device_frame_codes).  Also decodes the same windows from
// the host codes and the whole utterance, and the error paths.  Writes raw
// binaries for the pytest wrapper.
//   usage: test_vocoder_dev <tts.gguf> <vocoder.gguf> <inputs.bin> <out_dir>
// inputs.bin: int32 n_text, int32 text[n_text], int32 max_len, int32 chunk, int32 context
#include "audio_tokenizer_decoder.h"
#include "tts_transformer.h"

#include <cstdio>
#include <string>
#include <vector>

static bool dump(const std::string & path, const void * p, size_t n) {
    FILE * f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    std::fwrite(p, 1, n, f);
    std::fclose(f);
    return true;
}

int main(int argc, char ** argv) {
    if (argc < 5) { std::fprintf(stderr, "usage: %s tts.gguf vocoder.gguf inputs.bin out_dir\n", argv[0]); return 2; }
    const std::string out = argv[4];
    FILE * f = std::fopen(argv[3], "rb");
    if (!f) return 2;
    int32_t n_text = 0, max_len = 0, chunk = 0, context = 0;
    std::fread(&n_text, 4, 1, f);
    std::vector<int32_t> text(n_text);
    std::fread(text.data(), 4, n_text, f);
    std::fread(&max_len, 4, 1, f);
    std::fread(&chunk, 4, 1, f);
    std::fread(&context, 4, 1, f);
    std::fclose(f);

    qwen3_tts::TTSTransformer tr;
    if (!tr.load_model(argv[1])) { std::printf("FAIL tts load: %s\n", tr.get_error().c_str()); return 1; }
    qwen3_tts::AudioTokenizerDecoder dec;
    int fails = 0;
    std::vector<float> none;
    if (dec.decode_window(nullptr, 1, 0, 1, 0, none)) { std::printf("FAIL decode before load\n"); ++fails; }
    else std::printf("PASS not loaded: %s\n", dec.get_error().c_str());
    if (!dec.load_model(argv[2])) { std::printf("FAIL vocoder load: %s\n", dec.get_error().c_str()); return 1; }
    const auto & vc = dec.get_config();
    std::printf("PASS vocoder load: codebooks=%d size=%d latent=%d layers=%d decoder_dim=%d\n", vc.n_codebooks,
                vc.codebook_size, vc.latent_dim, vc.n_pre_tfm_layers, vc.decoder_dim);

    // StreamDecoderDriver over the device code rows
    std::vector<int32_t> codes;
    std::vector<float> audio;
    std::vector<int32_t> bounds;             // window ends
    int32_t emitted = 0;
    bool failed = false;
    auto on_frame = [&](const int32_t *, int32_t, int32_t frame) {
        const int32_t n = frame + 1;
        if (n - emitted < chunk) return true;
        std::vector<float> s;
        if (!dec.decode_window_device(tr.device_frame_codes(), n, emitted, n, context, s)) {
            std::printf("FAIL window: %s\n", dec.get_error().c_str());
            failed = true;
            return false;
        }
        audio.insert(audio.end(), s.begin(), s.end());
        emitted = n;
        bounds.push_back(n);
        return true;
    };
    if (!tr.generate(text.data(), n_text, nullptr, max_len, codes, tr.get_config().english_language_id, 1.05f, 0.0f,
                     0, nullptr, 0, 0.0f, 0, false, on_frame)) {
        std::printf("FAIL generate: %s\n", tr.get_error().c_str());
        return 1;
    }
    const int32_t total = (int32_t) codes.size() / 16;
    if (total > emitted) {      // the tail flush
        std::vector<float> s;
        if (!dec.decode_window_device(tr.device_frame_codes(), total, emitted, total, context, s)) {
            std::printf("FAIL tail: %s\n", dec.get_error().c_str());
            ++fails;
        }
        audio.insert(audio.end(), s.begin(), s.end());
        bounds.push_back(total);
    }
    if (failed) ++fails;
    std::printf("PASS streamed %d frames in %zu windows, %zu samples\n", total, bounds.size(), audio.size());

    // the same windows from host codes must give the same samples
    std::vector<float> host;
    int32_t from = 0;
    for (int32_t end : bounds) {
        if (!dec.decode_window(codes.data(), total, from, end, context, host)) { ++fails; break; }
        from = end;
    }
    if (host == audio) std::printf("PASS host-codes windows equal device-codes windows\n");
    else { std::printf("FAIL host-codes windows differ\n"); ++fails; }
    std::vector<float> whole;
    if (!dec.decode(codes.data(), total, whole)) { std::printf("FAIL decode: %s\n", dec.get_error().c_str()); ++fails; }
    std::vector<float> bad;
    if (dec.decode_window(codes.data(), total, 2, total + 1, context, bad)) { std::printf("FAIL bad range accepted\n"); ++fails; }
    else std::printf("PASS bad range: %s\n", dec.get_error().c_str());

    dump(out + "/codes.bin", codes.data(), codes.size() * 4);
    dump(out + "/stream.bin", audio.data(), audio.size() * 4);
    dump(out + "/bounds.bin", bounds.data(), bounds.size() * 4);
    dump(out + "/whole.bin", whole.data(), whole.size() * 4);
    std::printf("%s\n", fails ? "FAILED" : "ALL PASS");
    return fails ? 1 : 0;
}
