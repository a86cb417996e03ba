// CPU check of the facade's GGUF reading (no device): prints the parsed
// hyperparameters of a file as "name value" lines, or "error <message>" and
// exit status 2.  Usage: test_gguf_config <model.gguf>
#include "tts_transformer.h"

#include <cstdio>

int main(int argc, char ** argv) {
    if (argc != 2) { std::fprintf(stderr, "usage: %s model.gguf\n", argv[0]); return 1; }
    qwen3_tts::tts_transformer_config c;
    std::string err;
    if (!qwen3_tts::load_gguf_config(argv[1], c, err)) { std::printf("error %s\n", err.c_str()); return 2; }
    std::printf("hidden_size %d\nn_layers %d\nn_head %d\nn_kv_head %d\nhead_dim %d\nffn_size %d\n", c.hidden_size,
                c.n_layers, c.n_attention_heads, c.n_key_value_heads, c.head_dim, c.intermediate_size);
    std::printf("codec_vocab %d\nn_codebooks %d\ncp_layers %d\ncp_vocab %d\ncp_hidden %d\ncp_ffn %d\n",
                c.codec_vocab_size, c.n_codebooks, c.code_pred_layers, c.code_pred_vocab_size, c.code_pred_hidden_size,
                c.code_pred_intermediate_size);
    std::printf("text_vocab %d\ntext_embd_dim %d\nrms_eps %.9g\nrope_theta %.9g\ncp_rope_theta %.9g\n",
                c.text_vocab_size, c.text_embd_dim, c.rms_norm_eps, c.rope_theta, c.code_pred_rope_theta);
    std::printf("codec_pad_id %d\ncodec_bos_id %d\ncodec_eos_id %d\ntts_bos_id %d\ntts_eos_id %d\ntts_pad_id %d\n",
                c.codec_pad_id, c.codec_bos_id, c.codec_eos_id, c.tts_bos_token_id, c.tts_eos_token_id,
                c.tts_pad_token_id);
    return 0;
}
