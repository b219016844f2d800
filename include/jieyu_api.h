/*
 * jieyu_api.h — jieyu's text C ABI (JieyuAI_api.h:34-67, implemented in
 * main.hpp:85-227), exported by libjieyu_amd.so with the same names,
 * signatures, struct layout, return values and error behaviour.  Generation
 * runs on the GPU: jieyu_load uploads the model to HBM once, every
 * jieyu_generate* call decodes on the device.
 *
 * Return values (main.hpp:153-227):
 *   jieyu_generate / jieyu_generate_jsonl: > 0 tokens generated, 0 nothing
 *   generated (empty prompt or a full context; an error text is still set),
 *   -1 on error (text via jieyu_last_error(h); with h == NULL via
 *   jieyu_last_error(NULL)).  The generated text goes to out, truncated to
 *   cap-1 bytes and NUL-terminated; out may be NULL.
 *
 * Model data is one per process and shared by every handle (main.hpp:15-28):
 * loading another directory replaces it, the last jieyu_free releases it.
 * Calls are serialised by a lock inside the library.
 */
#ifndef JIEYU_API_H
#define JIEYU_API_H

#define JIEYU_AMD_API __attribute__((visibility("default")))

#define JIEYU_PATH_MAX 512
#define JIEYU_ERR_MAX 256

/* JieyuAI_api.h:42-46 — layout is public */
struct jieyu_ctx {
    char dir[JIEYU_PATH_MAX];   /* model directory of this handle        */
    char error[JIEYU_ERR_MAX];  /* last error on this handle ("" = none)  */
    int max_seq;                /* context length                         */
};

#ifdef __cplusplus
#define JIEYU_DEFAULT(v) = v
extern "C" {
#else
#define JIEYU_DEFAULT(v)
#endif

typedef struct jieyu_ctx* jieyu_model;

/* JieyuAI_api.h:49 — max_seq 0: max_position_embeddings of model_info.json
 * clamped to [64, 4096] (main.hpp:63-66).  NULL on failure. */
JIEYU_AMD_API jieyu_model jieyu_load(const char* dir, int max_seq JIEYU_DEFAULT(0));
/* JieyuAI_api.h:50 */
JIEYU_AMD_API void jieyu_free(jieyu_model h);
/* JieyuAI_api.h:51 — h == NULL: this thread's last load error */
JIEYU_AMD_API const char* jieyu_last_error(jieyu_model h);
/* JieyuAI_api.h:52 — "1.0.0" (date_libs/consten_pool.h:14) */
JIEYU_AMD_API const char* jieyu_version(void);
/* JieyuAI_api.h:53 */
JIEYU_AMD_API int jieyu_context_length(jieyu_model h);
/* JieyuAI_api.h:54 */
JIEYU_AMD_API const char* jieyu_model_dir(jieyu_model h);
/* JieyuAI_api.h:55-59 — generate_text (libs/model_libs/pipeline.h:280-374) */
JIEYU_AMD_API int jieyu_generate(jieyu_model h, const char* prompt, char* out, int cap, int max_new,
                                 float temperature, float repetition_penalty);
/* JieyuAI_api.h:60-66 — the name/message lines of a .jsonl file as one prompt
 * (libs/model_libs/jsonl_ochat.h:7-33) */
JIEYU_AMD_API int jieyu_generate_jsonl(jieyu_model h, const char* jsonl, const char* qb, const char* qe, char* out,
                                       int cap, int max_new JIEYU_DEFAULT(256),
                                       float temperature JIEYU_DEFAULT(0.8f),
                                       float repetition_penalty JIEYU_DEFAULT(1.1f));

#ifdef __cplusplus
}
#endif

#endif
