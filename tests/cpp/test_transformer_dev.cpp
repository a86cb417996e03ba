// Drives the drop-in TTSTransformer (qwen3-tts.cpp_amd/csrc/tts_transformer.h)
// the way the reference's tests/test_transformer.cpp drives its own: load a
// GGUF, init the KV cache, forward_prefill, then generate() greedy; plus
// generate_icl, predict_codes_autoregressive, predict_codes and the error
// paths.  Writes
// the results as raw binary files that the pytest wrapper compares with the
// CPU oracle.
//   usage: test_transformer_dev <model.gguf> <inputs.bin> <out_dir>
// inputs.bin: int32 n_text, int32 text[n_text], float speaker[hidden],
//             int32 max_len, int32 n_ref_frames, int32 ref_codes[n_ref_frames*16]
#include "tts_transformer.h"

#include <cstdio>
#include <cstring>
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
    if (argc < 4) { std::fprintf(stderr, "usage: %s model.gguf inputs.bin out_dir\n", argv[0]); return 2; }
    const std::string out = argv[3];
    FILE * f = std::fopen(argv[2], "rb");
    if (!f) return 2;
    int32_t n_text = 0, max_len = 0, n_ref = 0;
    std::fread(&n_text, 4, 1, f);
    std::vector<int32_t> text(n_text);
    std::fread(text.data(), 4, n_text, f);

    qwen3_tts::TTSTransformer tr;
    if (!tr.load_model(argv[1])) { std::printf("FAIL load: %s\n", tr.get_error().c_str()); return 1; }
    const auto & cfg = tr.get_config();
    std::printf("PASS load: hidden=%d layers=%d cp_layers=%d\n", cfg.hidden_size, cfg.n_layers, cfg.code_pred_layers);
    std::vector<float> spk(cfg.hidden_size);
    std::fread(spk.data(), 4, cfg.hidden_size, f);
    std::fread(&max_len, 4, 1, f);
    std::fread(&n_ref, 4, 1, f);
    std::vector<int32_t> ref(n_ref * 16);
    std::fread(ref.data(), 4, ref.size(), f);
    std::fclose(f);

    int fails = 0;
    // error paths (reference messages)
    std::vector<int32_t> codes;
    if (tr.generate(text.data(), 3, nullptr, 4, codes)) { std::printf("FAIL short prompt accepted\n"); ++fails; }
    else std::printf("PASS short prompt rejected: %s\n", tr.get_error().c_str());
    std::vector<float> logits, hidden;
    if (!tr.init_kv_cache(64)) { std::printf("FAIL kv: %s\n", tr.get_error().c_str()); return 1; }
    std::vector<float> dummy((size_t) cfg.hidden_size * 70, 0.01f);
    if (tr.forward_prefill(dummy.data(), 70, 0, hidden, &logits)) { std::printf("FAIL context overflow accepted\n"); ++fails; }
    else std::printf("PASS context overflow: %s\n", tr.get_error().c_str());

    // greedy generate
    if (!tr.generate(text.data(), n_text, spk.data(), max_len, codes, cfg.english_language_id, 1.05f, 0.0f, 0)) {
        std::printf("FAIL generate: %s\n", tr.get_error().c_str());
        return 1;
    }
    std::printf("PASS generate: %zu frames\n", codes.size() / 16);
    dump(out + "/codes.bin", codes.data(), codes.size() * 4);

    // callback abort after 3 frames
    int calls = 0;
    std::vector<int32_t> cut;
    tr.generate(text.data(), n_text, spk.data(), max_len, cut, cfg.english_language_id, 1.05f, 0.0f, 0, nullptr, 0,
                0.0f, 0, false, [&](const int32_t *, int32_t n, int32_t frame) { ++calls; return frame < 2 && n == 16; });
    if (cut.size() != 3 * 16 || calls != 3) { std::printf("FAIL callback abort %zu %d\n", cut.size(), calls); ++fails; }
    else std::printf("PASS callback abort\n");

    // attention dump of talker layer 1 over a greedy generate (ATTD file)
    tr.set_attn_dump(out + "/attn.bin", 1);
    std::vector<int32_t> dumped;
    if (!tr.generate(text.data(), n_text, spk.data(), max_len, dumped, cfg.english_language_id, 1.05f, 0.0f, 0) ||
        dumped != codes) {
        std::printf("FAIL attn-dump generate: %s\n", tr.get_error().c_str());
        ++fails;
    } else {
        std::printf("PASS attn-dump generate: %zu rows\n", tr.attn_rows().size());
    }
    tr.set_attn_dump("", 1);

    // code predictor on the last hidden state
    std::vector<int32_t> cp;
    std::vector<float> h;
    tr.get_hidden_states(h);
    if (!tr.predict_codes_autoregressive(h.data(), 5, cp, 0.0f, 0)) { std::printf("FAIL code pred\n"); ++fails; }
    dump(out + "/hidden.bin", h.data(), h.size() * 4);
    dump(out + "/cp.bin", cp.data(), cp.size() * 4);

    // the single-pass predictor on the same row, without and with the
    // previous codes (those of the last generated frame)
    std::vector<float> pl0, pl1;
    const int32_t * prev = codes.size() >= 16 ? codes.data() + codes.size() - 15 : nullptr;
    if (!tr.predict_codes(h.data(), nullptr, pl0) || !prev || !tr.predict_codes(h.data(), prev, pl1)) {
        std::printf("FAIL predict_codes: %s\n", tr.get_error().c_str());
        ++fails;
    } else {
        std::printf("PASS predict_codes: %zu logits\n", pl0.size());
        dump(out + "/pc0.bin", pl0.data(), pl0.size() * 4);
        dump(out + "/pc1.bin", pl1.data(), pl1.size() * 4);
    }
    {
        int32_t bad[15];
        for (int i = 0; i < 15; ++i) bad[i] = 1;
        bad[7] = cfg.code_pred_vocab_size;
        std::vector<float> pl;
        if (tr.predict_codes(h.data(), bad, pl)) { std::printf("FAIL predict_codes accepted a bad code\n"); ++fails; }
        else std::printf("PASS predict_codes bad code: %s\n", tr.get_error().c_str());
    }

    // ICL
    if (n_ref > 0) {
        std::vector<int32_t> icl;
        if (!tr.generate_icl(text.data(), n_text, text.data(), n_text, ref.data(), n_ref, spk.data(), max_len, icl,
                             cfg.english_language_id, 1.05f, 0.0f, 0, 0.0f, 0, false)) {
            std::printf("FAIL generate_icl: %s\n", tr.get_error().c_str());
            ++fails;
        } else {
            std::printf("PASS generate_icl: %zu frames\n", icl.size() / 16);
            dump(out + "/icl.bin", icl.data(), icl.size() * 4);
        }
    }
    std::printf(fails ? "=== FAILED ===\n" : "=== ALL PASS ===\n");
    return fails ? 1 : 0;
}
