/*
 * jieyu_amd.h — C ABI of the MI355X (gfx950) decode path: HBM-resident
 * weights and int8 KV cache, hand-written HIP kernels, one GPU.
 *
 * These entry points are the device-resident counterparts of jieyu's
 * model_libs forward-step interface.  All take plain pointers and sizes, return
 * an int status (0 / count on success, -1 on error) or a handle (NULL on
 * error); jyhip_last_error() gives the calling thread's last error text.  No
 * C++ exception crosses this boundary.
 *
 * Arithmetic: every kernel reproduces the reference CPU path's operation order
 * and rounding, so outputs are bit-identical to jieyu's AVX2+FMA build on the
 * same inputs (token ids, KV cache bytes, hidden states).
 */
#ifndef JIEYU_AMD_H
#define JIEYU_AMD_H

#include <stddef.h>
#include <stdint.h>

#include "jieyu_model.h"

#ifdef __cplusplus
extern "C" {
#endif

#define JYHIP_API __attribute__((visibility("default")))

typedef struct jyhip_model jyhip_model;
typedef struct jyhip_kv jyhip_kv;

/* token_cb of libs/model_libs/generate.h:8 — return nonzero to stop */
typedef int (*jyhip_token_cb)(int id, void* ud);

typedef struct jyhip_stats {
    double prefill_ms;      /* prompt forward + first token, device time */
    double decode_ms;       /* every later token, device time             */
    int prompt_len;
    int decoded;            /* tokens produced after the first            */
    double upload_ms;       /* host->device weight copy + repack (model)  */
} jyhip_stats;

/* Thread-local text of the last error ("" when none). */
JYHIP_API const char* jyhip_last_error(void);
/* Number of visible HIP devices (0 when none; never an error). */
JYHIP_API int jyhip_device_count(void);
/* Select the device used by subsequent calls of this thread. */
JYHIP_API int jyhip_set_device(int device);

/* Upload a model and precompute its RoPE table for positions [0, max_seq).
 * Mirrors what jieyu's bind_model + RoPETable::init produce
 * (libs/model_libs/pipeline.h:63-153, libs/date_libs/date.h:52-66); 2-D weights
 * must all be JY_Q8_0 or all JY_F32. */
JYHIP_API jyhip_model* jyhip_model_upload(const jy_model_desc* m, int max_seq);
JYHIP_API void jyhip_model_free(jyhip_model* model);
/* Arithmetic mode of a model's kernels (no counterpart in the reference).
 * JYHIP_MODE_EXACT (the default) reproduces the reference's operation order and rounding
 * bit for bit.  The other bits trade that for speed where the specification allows a
 * tolerance (per-layer fp32 hidden states within 1e-3 relative, identical greedy ids):
 *   JYHIP_MODE_SPLIT_ATTN  decode attention split across workgroups over the keys
 *                          (flash-decoding): exact int8 quantisation and int32 q.k, the
 *                          softmax sum and p.v accumulated per slice and merged; up to
 *                          1024 keys one kernel whose workgroups each take all the keys
 *                          and 16 output dims (the sum and p.v per wave, merged in the
 *                          workgroup); prompt rows in the same arithmetic, one workgroup
 *                          per kv head and row;
 *   JYHIP_MODE_SPLIT_MV    decode Q8_0 matvecs of fewer than JYHIP_SPLIT_MV_ROWS rows with
 *                          each row's dot split across waves; larger matrices keep the exact
 *                          kernel's dot order, which measured faster there (e.g. 4096 x
 *                          14336: 15.7 vs 18.9 us; 896 x 4864: 7.2 vs 5.1 us the other way);
 *                          both apply the RMSNorm scale after the dot (linearity);
 *   JYHIP_MODE_MFMA_PREFILL Q8_0 prompt GEMMs (m > 1) on the matrix cores: each activation
 *                          row scaled by a power of two and split into fp16 high + low parts
 *                          (22 significant bits), int8 weights exact in fp16, one fp32 MFMA
 *                          sum per 32-weight block times its scale.  Enabling it builds a
 *                          second copy of every layer's Q8_0 matrices in the matrix-core
 *                          operand order (about 1.13 bytes per weight; kept until the model
 *                          is freed); other weight types keep the exact tiles.
 * Int8 KV bytes and ids are the reference's wherever the fp32 values they come from are. */
#define JYHIP_MODE_EXACT 0
#define JYHIP_MODE_SPLIT_ATTN 1
#define JYHIP_MODE_SPLIT_MV 2
#define JYHIP_MODE_MFMA_PREFILL 4
#define JYHIP_MODE_FAST (JYHIP_MODE_SPLIT_ATTN | JYHIP_MODE_SPLIT_MV | JYHIP_MODE_MFMA_PREFILL)
#define JYHIP_SPLIT_MV_ROWS 2048
/* With both split bits: each decode row of every layer (and, in a session's greedy step, the
 * head) as one persistent kernel whose workgroups hand activations to each other through
 * grid barriers, instead of about six kernels per layer.  Same arithmetic as the split
 * forms; opt-in (measured slower than the separate kernels at the benchmark shapes). */
#define JYHIP_MODE_PERSIST 8
#define JYHIP_MODE_ALL (JYHIP_MODE_SPLIT_ATTN | JYHIP_MODE_SPLIT_MV | JYHIP_MODE_MFMA_PREFILL | JYHIP_MODE_PERSIST)
/* Set the mode (a combination of the bits above) for later calls on the model; sessions
 * capture their decode graphs again after a change.  Returns 0 / -1. */
JYHIP_API int jyhip_model_set_mode(jyhip_model* model, int mode);
JYHIP_API int jyhip_model_mode(const jyhip_model* model);

/* Bytes of 2-D weights (incl. lm_head) one decode step streams. */
JYHIP_API size_t jyhip_model_weight_bytes(const jyhip_model* model);
JYHIP_API double jyhip_model_upload_ms(const jyhip_model* model);

/* __KVcache::init (libs/date_libs/date.h:99-111): zero-filled int8 K/V and fp32
 * scales for num_layers x max_seq x num_kv_heads x head_dim. */
JYHIP_API jyhip_kv* jyhip_kv_create(const jyhip_model* model, int max_seq);
JYHIP_API void jyhip_kv_free(jyhip_kv* kv);
JYHIP_API int jyhip_kv_len(const jyhip_kv* kv);
JYHIP_API int jyhip_kv_set_len(jyhip_kv* kv, int current_len);
/* Copy positions [pos0, pos0+npos) of one layer in jieyu's host layout:
 * k, v int8 [npos][num_kv_heads][head_dim]; ks, vs float [npos][num_kv_heads]. */
JYHIP_API int jyhip_kv_write(jyhip_kv* kv, int layer, int pos0, int npos, const int8_t* k, const float* ks,
                             const int8_t* v, const float* vs);
JYHIP_API int jyhip_kv_read(const jyhip_kv* kv, int layer, int pos0, int npos, int8_t* k, float* ks, int8_t* v,
                            float* vs);

/* forward_cached (libs/model_libs/forward.h:47-96).  X: host [seq][hidden], the
 * embeddings of positions [start_pos, start_pos+seq) on entry, the final-normed
 * hidden states on exit.  layer_out (optional, host [num_layers][seq][hidden])
 * receives X after every layer.  Sets the cache length to start_pos+seq. */
JYHIP_API int jyhip_forward_cached(jyhip_model* model, jyhip_kv* kv, float* X, int seq, int start_pos,
                                   float* layer_out);

/* Bytes of the static per-GPU workspace of jyhip_forward_cached_noalloc. */
#define JYHIP_NOALLOC_SCRATCH_BYTES (16u << 20)

/* jyhip_forward_cached (layer_out aside) without any device allocation.  It has no
 * counterpart in the reference: it is for callers that cannot allocate device memory
 * (tight serving loops, harnesses that forbid hipMalloc).  Like jyhip_forward_cached it
 * copies X from and back to the host and waits for the model's stream, so it cannot be
 * recorded into a caller's HIP graph: it allocates nothing, it is not capturable.
 * Same arguments, checks and results as jyhip_forward_cached with layer_out == NULL.
 * Its workspace is one static array of JYHIP_NOALLOC_SCRATCH_BYTES in each GPU's memory,
 * held until the process ends; a call whose rows and keys need more (a long prompt, a
 * long context) fails with an error that names the size.  Every call on a GPU shares
 * that GPU's array: calls that overlap on one GPU race. */
JYHIP_API int jyhip_forward_cached_noalloc(jyhip_model* model, jyhip_kv* kv, float* X, int seq, int start_pos);

/* generate / generate_cached (libs/model_libs/generate.h:9-112).  kv == NULL
 * uses a private max_seq cache.  Returns the sequence length written to
 * out_ids (prompt + generated), 0 for an empty / too long prompt, -1 on error.
 * out_ids needs max_seq entries.  logits_out (optional, [vocab_size]) receives
 * the logits of the last step. */
JYHIP_API int jyhip_generate(jyhip_model* model, jyhip_kv* kv, const int* prompt_ids, int prompt_len,
                             const int* eos_ids, int num_eos, int max_seq, int max_new, float temperature,
                             float repetition_penalty, int* out_ids, jyhip_token_cb cb, void* cb_ud,
                             float* logits_out, jyhip_stats* stats);

/* The same generation driven step by step (no counterpart in the reference; the
 * decode loop of generate_cached, generate.h:39-87, split so a caller can time
 * or interleave steps).  begin runs the prompt and picks the first token;
 * step produces up to n more (returns how many, 0 when finished); ids copies the
 * sequence so far.  begin returns a finished session (len = what generate()
 * would return) when the prompt is empty/too long or max_new <= 0.  A model holds
 * one generation's token ids and length on the device: once another session (or
 * jyhip_generate) begins on the same model, step on the earlier session returns -1
 * with an error.  forward_cached calls between steps are allowed. */
typedef struct jyhip_session jyhip_session;
JYHIP_API jyhip_session* jyhip_session_begin(jyhip_model* model, jyhip_kv* kv, const int* prompt_ids,
                                             int prompt_len, const int* eos_ids, int num_eos, int max_seq,
                                             int max_new, float temperature, float repetition_penalty);
/* A generation over a cache that already holds kv's current length (c) positions of
 * ids[0 .. n_ids): ids[c .. n_ids) run as one chunk at start_pos c, as forward_cached
 * does (libs/model_libs/forward.h:95), then decoding continues as in begin; the
 * repetition penalty covers only the tokens generated here.  Needs 0 <= c < n_ids.
 * The reference has no such entry (generate_cached, generate.h:31, always starts the
 * cache at 0); it serves decoding after a cache filled by other means (long-context
 * measurement, a conversation's earlier turns). */
JYHIP_API jyhip_session* jyhip_session_resume(jyhip_model* model, jyhip_kv* kv, const int* ids, int n_ids,
                                              const int* eos_ids, int num_eos, int max_seq, int max_new,
                                              float temperature, float repetition_penalty);
JYHIP_API int jyhip_session_step(jyhip_session* s, int n);
JYHIP_API int jyhip_session_remaining(const jyhip_session* s);
JYHIP_API int jyhip_session_len(const jyhip_session* s);
JYHIP_API int jyhip_session_ids(const jyhip_session* s, int* out, int cap);
JYHIP_API int jyhip_session_stats(jyhip_session* s, jyhip_stats* stats);
/* Diagnostics of a session's captured decode graph `which` (0: the graph for lengths past
 * the short-context threshold, 1: up to it); no counterpart in the reference.  Each graph is
 * checked when it is captured (kernel nodes only, one dependency chain, launch shapes within
 * the device's limits, every device buffer the step can address a live allocation on the
 * model's device) and before each jyhip_session_step (no such buffer replaced since capture).
 * Writes info[0] = nodes, info[1] = edges, info[2] = buffers checked; returns 1, 0 when that
 * graph has not been captured, -1 on error (a failed check). */
JYHIP_API int jyhip_session_graph_info(const jyhip_session* s, int which, long long* info);
JYHIP_API void jyhip_session_end(jyhip_session* s);

/* Isolated Q8_0 matvec (decode kernel): y[n] = W[n][:] . x for a [rows][cols/32]x34
 * jieyu matrix.  jyhip_q8_upload keeps `copies` identical device copies so timed
 * runs can rotate through more bytes than the 256 MiB last-level cache. */
typedef struct jyhip_q8mat jyhip_q8mat;
JYHIP_API jyhip_q8mat* jyhip_q8_upload(const void* w, int rows, int cols, int copies);
JYHIP_API void jyhip_q8_free(jyhip_q8mat* m);
JYHIP_API int jyhip_q8_matvec(jyhip_q8mat* m, const float* x, float* y);
/* jyhip_q8_matvec's kernel: JYHIP_MODE_EXACT (the default) or with JYHIP_MODE_SPLIT_MV the
 * split-dot form at any size; with JYHIP_MODE_MFMA_PREFILL jyhip_q8_gemm runs the matrix-core kernel
 * (the first such call builds its copies of the matrix).  Returns 0 / -1. */
JYHIP_API int jyhip_q8_set_mode(jyhip_q8mat* m, int mode);
/* Time `iters` launches (rotating copies) with HIP events on the launch stream:
 * *avg_us = mean kernel-to-kernel time per launch.  variant 0 is the plain
 * matvec; variant 1 is the decode step's gate/up launch of the same kernel
 * (RMSNorm over x, SwiGLU epilogue over interleaved row pairs); variants 2 and 3
 * are the same two launches of the split-dot kernel (JYHIP_MODE_SPLIT_MV); variant 4 is
 * the gate/up launch of the first kernel with the RMSNorm applied after the dot, the form
 * JYHIP_MODE_SPLIT_MV gives the matrices it leaves in the 32-lane order. */
JYHIP_API int jyhip_q8_matvec_time(jyhip_q8mat* m, const float* x, int variant, int iters, double* avg_us);
/* C[mr][rows] = A[mr][cols] W^T (row-major fp32) through the prompt GEMM of the
 * matrix's mode: the exact tiles, or with JYHIP_MODE_MFMA_PREFILL the matrix-core kernel
 * (the generic m > 1 matmul of libs/matmul_libs/matmul_q.h:145-161).  Returns 0 / -1. */
JYHIP_API int jyhip_q8_gemm(jyhip_q8mat* m, int mr, const float* A, float* C);
/* Mean device time in microseconds of `iters` such GEMMs (A uploaded once, the launches
 * cycling through the matrix's copies), the activation split included.  Returns 0 / -1. */
JYHIP_API int jyhip_q8_gemm_time(jyhip_q8mat* m, int mr, const float* A, int iters, double* avg_us);

/* One weight matrix of any bound type in HBM: matmul_w (libs/model_libs/wmat_kernel.h:9-16)
 * with B = w, n output rows, k inputs (f32 / f16 [k][n]; Q8_0 / k-quants [n][k/block]).
 * jyhip_wmat_matmul computes C[m][n] = A[m][k] x B from host buffers in the
 * reference's order for w's type: m == 1 the decode kernel (dot_row_avx2 for
 * quantized rows, matmul_q.h:111-143), m > 1 the prompt GEMM (:145-161; dense
 * [k][n]: the fma chain of matmul.h / matmul_f16.h).  `copies` device copies let
 * jyhip_wmat_time rotate through more bytes than the last-level cache: it times
 * `iters` decode launches with HIP events on the launch stream (mean us). */
typedef struct jyhip_wmat jyhip_wmat;
JYHIP_API jyhip_wmat* jyhip_wmat_upload(const jy_wmat* w, int n, int k, int copies);
JYHIP_API void jyhip_wmat_free(jyhip_wmat* w);
JYHIP_API int jyhip_wmat_matmul(jyhip_wmat* w, int m, const float* A, float* C);
JYHIP_API int jyhip_wmat_time(jyhip_wmat* w, const float* x, int iters, double* avg_us);

#ifdef __cplusplus
}
#endif

#endif
