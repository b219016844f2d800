/*
 * jieyu_text.h — the host-side text layer behind jieyu_api.h, exported so it
 * can be used (and checked) without a GPU: the byte-level BPE tokenizer
 * (libs/tokenizer_libs/include/tokenizer.h:242-701), model_info.json lookups
 * (libs/json_libs/json.h:57-84) and the model-directory bind
 * (libs/model_libs/pipeline.h:63-153, :395-441).
 *
 * Status returns are 0 / count on success and -1 on error, with the text in
 * jytext_last_error() (per thread).
 */
#ifndef JIEYU_TEXT_H
#define JIEYU_TEXT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define JYTEXT_API __attribute__((visibility("default")))

typedef struct jytext_tokenizer jytext_tokenizer;

JYTEXT_API const char* jytext_last_error(void);

/* Tokenizer::load (tokenizer.h:342-423) */
JYTEXT_API jytext_tokenizer* jytext_tokenizer_load(const char* vocab_json, const char* merges_txt);
JYTEXT_API void jytext_tokenizer_free(jytext_tokenizer* t);
/* vocab_size / bos_id / eos_id / unk_id (tokenizer.h:675-697); any pointer may be NULL */
JYTEXT_API int jytext_tokenizer_info(const jytext_tokenizer* t, int* vocab_size, int* bos, int* eos, int* unk);
/* add_special_token (tokenizer.h:310-327): the piece's id, or -1 if not in the vocabulary */
JYTEXT_API int jytext_tokenizer_add_special(jytext_tokenizer* t, const char* piece);
/* encode (tokenizer.h:594-633) of len bytes of text: returns the number of ids
 * (only the first cap are written) */
JYTEXT_API int jytext_tokenizer_encode(const jytext_tokenizer* t, const char* text, size_t len, int32_t* ids,
                                       int cap);
/* decode (tokenizer.h:635-664): returns the byte count (only the first cap bytes
 * are written, no terminator) */
JYTEXT_API int jytext_tokenizer_decode(const jytext_tokenizer* t, const int32_t* ids, int n, char* out, int cap);

/* read_info_int / read_info_str of a JSON file (pipeline.h:53-57, :157-162) */
JYTEXT_API int jytext_info_int(const char* path, const char* key, int fallback);
/* returns the text length (only the first cap-1 bytes are written, NUL-terminated) */
JYTEXT_API int jytext_info_str(const char* path, const char* key, const char* fallback, char* out, int cap);

/* install_model + bind_model of a model directory, host only.  hp receives
 * {layers, hidden, heads, kv_heads, head_dim, intermediate, vocab, add_bos,
 *  qkv_bias, embed_type, lm_head_type, layer_type} (jieyu_model.h types: 0 f32,
 * 1 f16, 3 q8_0, 5 q4_K, 6 q5_K, 7 q6_K).  -1 and the reference's error text on
 * failure. */
JYTEXT_API int jytext_model_bind(const char* dir, int max_seq, int* hp);

/* GGUF (v2 / v3) file -> model directory: model.bf, model_info.json, vocab.json,
 * merges.txt, as ggufc::convert writes them (libs/gguf_libs/gguf_convert.h:260-421).
 * out_dtype: model.bf dtype of the non-quantized 2-D weights (0 f32, 1 f16, 2 bf16);
 * quant != 0 keeps Q4_K / Q5_K / Q6_K / Q8_0 blocks (q / k rows permuted), else
 * every tensor is dequantized.  info (optional, 16 values) receives {hidden, layers,
 * heads, kv_heads, head_dim, intermediate, vocab, rope_theta, max_position,
 * tensor_count, transposed, permuted, quant, tied_lm_head, eos_id, file_size}.
 * 0, or -1 and the reference's error text. */
JYTEXT_API int jytext_gguf_convert(const char* src, const char* out_dir, int out_dtype, int quant, int verbose,
                                   long long* info);

#ifdef __cplusplus
}
#endif

#endif
