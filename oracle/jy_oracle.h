/*
 * jy_oracle.h — CPU oracle for jieyu's decode path.  TEST INFRASTRUCTURE:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * as the reference results the GPU path is checked against.  The product
 * (libjieyu_amd.so) never links or calls it.
 *
 * A clean-room C restatement of the arithmetic of jieyu's default x86 path
 * (AVX2 + FMA, GCC -O3), operation for operation, so its results are
 * bit-identical to the reference on the same inputs.  Each function cites the
 * reference file:line it restates.  Pinning (tests/test_oracle_*.py):
 *   - golden vectors from the reference compiled in this repository's
 *     oracle/Makefile (oracle/_ref), committed under tests/golden/;
 *   - the reference's own known-answer tests (bind_test fixtures, greedy ids
 *     against the float64 restatement of libs/text/text.h:551-597);
 *   - closed forms and brute force (float64 dots, exhaustive expf, special
 *     cases).
 */
#ifndef JY_ORACLE_H
#define JY_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#include "jieyu_model.h"

#ifdef __cplusplus
extern "C" {
#endif

float jyo_f16_to_f32(uint16_t h);

/* block geometry of a quantized type (libs/matmul_libs/matmul_q.h:35-45) */
int jyo_block_elems(int type);
int jyo_block_bytes(int type);
/* dequant_block: Q8_0 / Q4_K / Q5_K / Q6_K (libs/matmul_libs/matmul_q.h:47-100) */
void jyo_dequant_block(int type, const uint8_t* block, float* dst);
/* decode row dot, 32 virtual FMA lanes (libs/matmul_libs/matmul_q.h:111-132) */
float jyo_q_row_dot(const float* x, const uint8_t* row, int type, int k);
float jyo_q8_row_dot(const float* x, const uint8_t* row, int k);
/* qmat::matmul_q (libs/matmul_libs/matmul_q.h:134-162) */
void jyo_matmul_q(const float* a, const uint8_t* w, float* c, int m, int n, int k, int type);
void jyo_matmul_q8(const float* a, const uint8_t* w, float* c, int m, int n, int k);
/* matmul f32, B = [k][n] (libs/matmul_libs/matmul.h:7-76, x86/x86_classic.txt:1-16) */
void jyo_matmul_f32(int m, int n, int k, const float* A, const float* B, float* C);
/* matmul f16, B = [k][n] halves (libs/matmul_libs/matmul_f16.h:19-41) */
void jyo_matmul_f16(int m, int n, int k, const float* A, const uint16_t* B, float* C);
/* matmul_w dispatch (libs/model_libs/wmat_kernel.h:9-16) */
void jyo_matmul_w(const jy_wmat* w, int m, int n, int k, const float* A, float* C);
/* wmat_row (libs/model_libs/wmat_kernel.h:18-29) */
void jyo_embed_row(const jy_wmat* w, int id, int width, float* dst);

/* rmsnorm (libs/model_libs/rmsnorm/rmsnorm.h:8-78, x86/x86_classic.txt:1-27) */
void jyo_rmsnorm(const float* x, float* y, const float* w, int n, float eps);
/* RoPETable::init (libs/date_libs/date.h:52-66); cos/sin are [max_seq][hd/2] */
void jyo_rope_table(int max_seq, int head_dim, float theta, float* cos_t, float* sin_t);
/* rope_pos (libs/model_libs/rope/rope.h:7-110, x86/x86_classic.txt:1-39) */
void jyo_rope(float* q, int seq, int start_pos, int num_heads, int head_dim, const float* cos_t,
              const float* sin_t);
/* kv_pack_q8 (libs/model_libs/attention/attention_q8.h:20-37) */
void jyo_kv_pack(const float* src, int8_t* dst, float* sc, int heads, int hd, int n);
/* silu (libs/model_libs/silu/silu.h:7-81, x86/x86_classic.txt:1-32) */
void jyo_silu(const float* x, float* y, int n);

/* __KVcache (libs/date_libs/date.h:89-147): int8 [L][max_seq][nkv][hd], fp32 [L][max_seq][nkv] */
typedef struct jyo_kv {
    int num_layers, max_seq, num_kv_heads, head_dim, current_len;
    int8_t* k;
    int8_t* v;
    float* ks;
    float* vs;
} jyo_kv;
int  jyo_kv_init(jyo_kv* kv, int num_layers, int max_seq, int num_kv_heads, int head_dim);
void jyo_kv_free(jyo_kv* kv);

/* attention_q8 with a cache view of one layer (libs/model_libs/attention/attention_q8.h:38-184,
 * x86/x86_classic.txt:1-75).  Packs K,V into the cache, then attends.  Returns 0 / -1. */
int jyo_attention(float* Q, const float* K, const float* V, float* out, int seq, int start_pos,
                  int num_heads, int num_kv_heads, int head_dim, int8_t* kc, float* ksc, int8_t* vc,
                  float* vsc, int cap);

/* transformer_layer (libs/model_libs/transformer_layer.h:10-90); X [seq][hidden] in place */
int jyo_transformer_layer(float* X, const jy_layer_weights* w, const float* cos_t, const float* sin_t,
                          int seq, int hidden, int num_heads, int num_kv_heads, int head_dim,
                          int intermediate, int start_pos, jyo_kv* kv, int layer, float eps);

/* forward_cached (libs/model_libs/forward.h:47-96).  If layer_out != NULL it receives X after
 * every layer, [num_layers][seq][hidden].  Returns 0 / -1 (bad shape / capacity). */
int jyo_forward_cached(const jy_model_desc* m, float* X, const float* cos_t, const float* sin_t, int seq,
                       int start_pos, jyo_kv* kv, float* layer_out);

/* generate_cached / generate (libs/model_libs/generate.h:9-112).  kv == NULL: a private cache of
 * max_seq positions.  last_logits (optional, [vocab]) receives the logits of the final step. */
int jyo_generate(const jy_model_desc* m, const int* prompt_ids, int prompt_len, const int* eos_ids,
                 int num_eos, const float* cos_t, const float* sin_t, int max_seq, int max_new,
                 float temperature, float repetition_penalty, int* out_ids, jyo_kv* kv,
                 float* last_logits);

#ifdef __cplusplus
}
#endif

#endif
