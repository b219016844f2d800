/*
 * jieyu_synth.h — deterministic synthetic models and inputs.
 *
 * jieyu never quantizes weights itself: Q8_0 only arrives by verbatim copy of
 * GGUF blocks (libs/gguf_libs/gguf_convert.h:201-229).  Random-init Q8 models
 * therefore need a quantizer of their own; only the block FORMAT is jieyu's
 * (libs/matmul_libs/matmul_q.h:35-45, :101-105).  Every consumer (the HIP
 * path, the CPU oracle, the compiled reference) reads the same bytes produced
 * here, so the quantizer's rounding choices do not affect parity.
 *
 * Randomness is counter based (splitmix64 + Box-Muller in double), so a value
 * depends only on (seed, stream, index) and generation is thread-count
 * independent.
 */
#ifndef JIEYU_SYNTH_H
#define JIEYU_SYNTH_H

#include "jieyu_model.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct jy_synth_config {
    int num_layers;
    int hidden;
    int num_heads;
    int num_kv_heads;
    int head_dim;
    int intermediate;
    int vocab_size;
    int rope_theta;     /* integer, as jieyu parses model_info.json */
    int wtype;          /* JY_F32 | JY_Q8_0 for the 2-D weights */
    int qkv_bias;       /* 1: q/k/v biases present (Qwen2-style) */
    int tied;           /* 1: lm_head shares the embedding (Q8_0 only) */
    uint64_t seed;
    float std;          /* weights ~ N(0, std); norms = 1 + N(0, std); biases ~ N(0, std) */
} jy_synth_config;

typedef struct jy_synth_model {
    jy_model_desc desc;
    jy_layer_weights* layers;
    void* arena;        /* owns every tensor */
    size_t arena_bytes;
    size_t weight_bytes; /* bytes a decode step streams for the 2-D weights incl. lm_head */
} jy_synth_model;

/* Build a model in host memory.  Returns 0, or -1 with *out = NULL. */
int  jysyn_create(const jy_synth_config* cfg, jy_synth_model** out);
void jysyn_free(jy_synth_model* m);

/* out[i] = std * N(0,1) for the (seed, stream) sequence, i in [0, n). */
void jysyn_normal_fill(uint64_t seed, uint64_t stream, float std, float* out, size_t n);
/* out[i] = uniform integer in [lo, hi] for the (seed, stream) sequence. */
void jysyn_uniform_int_fill(uint64_t seed, uint64_t stream, int lo, int hi, int* out, size_t n);
/* out[i] = uniform float in [lo, hi) for the (seed, stream) sequence. */
void jysyn_uniform_fill(uint64_t seed, uint64_t stream, float lo, float hi, float* out, size_t n);

/* GGML-convention Q8_0 quantizer: d = amax/127 (stored as fp16, round to
 * nearest even), q = roundf(x * (1/d)).  n must be a multiple of 32. */
void jysyn_quantize_q8_0(const float* x, uint8_t* out, size_t n);

/* IEEE half <-> float (round to nearest even). */
uint16_t jysyn_f32_to_f16(float f);
float    jysyn_f16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif

#endif
