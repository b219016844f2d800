/*
 * jieyu_model.h — host-side description of a decoder model, in the in-memory
 * layouts jieyu's model_libs consume.  Plain C so it can cross any FFI.
 *
 * Mirrors (same slots, same tensor layouts):
 *   WMat          libs/date_libs/wmat.h:32-44
 *   LayerWeights  libs/date_libs/date.h:75-88
 *   the argument list of generate()  libs/model_libs/generate.h:90-104
 *
 * Tensor layouts (as jieyu binds them, libs/model_libs/pipeline.h:124-132):
 *   JY_F32 matrices   : float [in][out]  (matmul B operand, libs/matmul_libs/matmul.h:7)
 *   JY_F16 matrices   : IEEE half [in][out]  (libs/matmul_libs/matmul_f16.h:19-41)
 *   JY_Q8_0 matrices  : [out rows][in/32 blocks] x 34 bytes; a block is the
 *                       little-endian fp16 scale d followed by 32 int8 q,
 *                       w = (float)q * d   (libs/matmul_libs/matmul_q.h:35-45, :101-105)
 *   JY_Q4_K / JY_Q5_K / JY_Q6_K matrices: [out rows][in/256 super-blocks] x
 *                       144 / 176 / 210 bytes, GGML's k-quant blocks
 *                       (libs/matmul_libs/matmul_q.h:35-100, libs/file_libs/q4/q4.h:8-35)
 *   embedding         : [vocab][hidden] (f32 / f16 rows, or quantized rows)
 *   lm_head           : quantized [vocab][hidden], or f32 / f16 [hidden][vocab]
 *                       (libs/model_libs/load_weights.h:137-155)
 *   norm weights, biases: float [n]
 */
#ifndef JIEYU_MODEL_H
#define JIEYU_MODEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight element types.  JY_Q8_0 keeps jieyu's qmat enum value
 * (libs/matmul_libs/matmul_q.h:15); f16 and the k-quants take their model.bf
 * dtype codes (libs/model_libs/bfile.h:26).  Each matrix carries its own type,
 * as jieyu's WMat does. */
enum { JY_F32 = 0, JY_F16 = 1, JY_Q8_0 = 3, JY_Q4_K = 5, JY_Q5_K = 6, JY_Q6_K = 7 };

#define JY_Q8_BLOCK 32     /* weights per Q8_0 block */
#define JY_Q8_BYTES 34     /* bytes per Q8_0 block   */
#define JY_QK_BLOCK 256    /* weights per k-quant super-block */
#define JY_Q4_K_BYTES 144
#define JY_Q5_K_BYTES 176
#define JY_Q6_K_BYTES 210

typedef struct jy_wmat {
    const void* data;   /* NULL = absent */
    int type;           /* JY_F32 | JY_F16 | JY_Q8_0 | JY_Q4_K | JY_Q5_K | JY_Q6_K */
} jy_wmat;

typedef struct jy_layer_weights {
    const float* rms1_weight;          /* input_layernorm            [hidden] */
    jy_wmat Wq, Wk, Wv, Wo;            /* self_attn.{q,k,v,o}_proj            */
    const float* bq;                   /* optional biases (NULL = none)       */
    const float* bk;
    const float* bv;
    const float* rms2_weight;          /* post_attention_layernorm   [hidden] */
    jy_wmat W1, W2, W3;                /* mlp.gate_proj, down_proj, up_proj   */
} jy_layer_weights;

typedef struct jy_model_desc {
    int num_layers;
    int hidden;
    int num_heads;
    int num_kv_heads;
    int head_dim;
    int intermediate;
    int vocab_size;
    float rope_theta;                  /* jieyu reads it as an integer (pipeline.h:59-61) */
    jy_wmat embed;
    jy_wmat lm_head;
    const float* final_rms_weight;     /* model.norm.weight [hidden] */
    const jy_layer_weights* layers;    /* [num_layers] */
} jy_model_desc;

#ifdef __cplusplus
}
#endif

#endif
