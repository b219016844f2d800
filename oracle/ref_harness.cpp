/*
 * ref_harness.cpp — exposes jieyu's own decode-path functions, compiled from
 * the reference sources where they lie (see oracle/Makefile), behind a small C
 * ABI so tests and bench.py's cpu_baseline leg can call them.  TEST
 * INFRASTRUCTURE ONLY: the product never links it.  The output library lives
 * in oracle/_ref/ and is not committed.
 *
 * Compiled with the reference's own flags (CMakeLists.txt:20-22, :97-105):
 * -std=c++17 -O3 -DNDEBUG -fopenmp, no -march (runtime CPUID dispatch,
 * libs/date_libs/check_cpu.h:15-69).
 */
#include <cmath>
#include <cstring>
#include <ctime>
#include <stdexcept>
#include <vector>

#include "model_libs/generate.h"   /* generate / forward_cached / transformer_layer and every kernel */
#include "main.hpp"                 /* the text C ABI (jieyu_load / jieyu_generate ...), pipeline, tokenizer,
                                       consten_pool */
#include "gguf_libs/gguf_convert.h" /* GGUF -> model directory */

#include "jieyu_model.h"

#define JYREF_API extern "C" __attribute__((visibility("default")))

namespace {

WMat to_wmat(const jy_wmat& w) {
    if (w.data == nullptr) return WMat();
    switch (w.type) {
        case JY_Q8_0: return WMat(w.data, (uint8_t)qmat::Q8_0);
        case JY_Q4_K: return WMat(w.data, (uint8_t)qmat::Q4K);
        case JY_Q5_K: return WMat(w.data, (uint8_t)qmat::Q5K);
        case JY_Q6_K: return WMat(w.data, (uint8_t)qmat::Q6K);
        case JY_F16: return WMat((const uint16_t*)w.data);
        default: return WMat((const float*)w.data);
    }
}

std::vector<LayerWeights> to_layers(const jy_model_desc* m) {
    std::vector<LayerWeights> out((size_t)m->num_layers);
    for (int l = 0; l < m->num_layers; l++) {
        const jy_layer_weights& s = m->layers[l];
        LayerWeights& d = out[(size_t)l];
        d.rms1_weight = s.rms1_weight;
        d.Wq = to_wmat(s.Wq);
        d.Wk = to_wmat(s.Wk);
        d.Wv = to_wmat(s.Wv);
        d.Wo = to_wmat(s.Wo);
        d.bq = s.bq;
        d.bk = s.bk;
        d.bv = s.bv;
        d.rms2_weight = s.rms2_weight;
        d.W1 = to_wmat(s.W1);
        d.W2 = to_wmat(s.W2);
        d.W3 = to_wmat(s.W3);
    }
    return out;
}

}  // namespace

/* ISA tiers the reference will take on this host: bit0 avx2, bit1 fma, bit2 avx-vnni */
JYREF_API int jyref_init(void) {
    static const bool once = (cpu_can.GetCpuCan(), true);
    (void)once;
    return (cpu_can.avx2 ? 1 : 0) | (cpu_can.fma3 ? 2 : 0) | (cpu_can.avxvnni ? 4 : 0);
}

JYREF_API const char* jyref_version(void) { return consten_pool.version.charv.c_str(); }

JYREF_API void jyref_matmul_q8(const float* a, const void* w, float* c, int m, int n, int k) {
    qmat::matmul_q(a, w, c, m, n, k, qmat::Q8_0);
}

/* matmul_w (libs/model_libs/wmat_kernel.h:9-16) for any weight type, and wmat_row
 * (:18-29), the embedding gather */
JYREF_API void jyref_matmul_w(const jy_wmat* w, int m, int n, int k, const float* A, float* C) {
    matmul_w(to_wmat(*w), m, n, k, A, C);
}

JYREF_API void jyref_wmat_row(const jy_wmat* w, int id, int width, float* dst) {
    wmat_row(to_wmat(*w), (size_t)id, width, dst);
}

JYREF_API void jyref_matmul_f32(int m, int n, int k, const float* A, const float* B, float* C) {
    matmul(m, n, k, A, B, C);
}

JYREF_API void jyref_rmsnorm(float* x, float* y, const float* w, int n, float eps) { rmsnorm(x, y, w, n, eps); }

JYREF_API void jyref_rope_table(int max_seq, int head_dim, float theta, float* cos_t, float* sin_t) {
    RoPETable t;
    t.init(max_seq, head_dim, theta);
    std::memcpy(cos_t, t.cos.data(), t.cos.size() * sizeof(float));
    std::memcpy(sin_t, t.sin.data(), t.sin.size() * sizeof(float));
}

JYREF_API void jyref_rope(float* q, int seq, int start_pos, int num_heads, int head_dim, const float* cos_t,
                          const float* sin_t) {
    rope_pos(q, seq, start_pos, num_heads, head_dim, cos_t, sin_t);
}

JYREF_API void jyref_kv_pack(const float* src, int8_t* dst, float* sc, int heads, int hd, int n) {
    kv_pack_q8(src, dst, sc, heads, hd, n);
}

JYREF_API int jyref_attention(float* Q, float* K, float* V, float* out, int seq, int start_pos, int num_heads,
                              int num_kv_heads, int head_dim, int8_t* kc, float* ksc, int8_t* vc, float* vsc,
                              int cap) {
    try {
        attention_q8(Q, K, V, out, seq, start_pos, num_heads, num_kv_heads, head_dim, __KVq{kc, ksc, vc, vsc, cap});
    } catch (const std::exception&) {
        return -1;
    }
    return 0;
}

JYREF_API void jyref_silu(float* x, float* y, int n) { silu(x, y, n); }

/* ---- KV cache (the reference's own __KVcache) -------------------------------- */

JYREF_API void* jyref_kv_create(int num_layers, int max_seq, int num_kv_heads, int head_dim) {
    __KVcache* c = new (std::nothrow) __KVcache();
    if (!c) return nullptr;
    c->init(num_layers, max_seq, num_kv_heads, head_dim);
    return c;
}

JYREF_API void jyref_kv_free(void* kv) { delete (__KVcache*)kv; }

/* raw views: k, v int8 [L][max_seq][nkv][hd]; ks, vs float [L][max_seq][nkv] */
JYREF_API int8_t* jyref_kv_k(void* kv) { return ((__KVcache*)kv)->k.data(); }
JYREF_API int8_t* jyref_kv_v(void* kv) { return ((__KVcache*)kv)->v.data(); }
JYREF_API float* jyref_kv_ks(void* kv) { return ((__KVcache*)kv)->ks.data(); }
JYREF_API float* jyref_kv_vs(void* kv) { return ((__KVcache*)kv)->vs.data(); }
JYREF_API int jyref_kv_len(void* kv) { return ((__KVcache*)kv)->current_len; }
JYREF_API void jyref_kv_set_len(void* kv, int n) { ((__KVcache*)kv)->current_len = n; }

/* ---- model level ----------------------------------------------------------- */

/* forward_cached (libs/model_libs/forward.h:47-96), unrolled here only to hand out
 * X after each transformer_layer call; the per-layer work and the final norm are
 * the reference's own functions. */
JYREF_API int jyref_forward_cached(const jy_model_desc* m, const float* cos_t, const float* sin_t, float* X, int seq,
                                   int start_pos, void* kvp, float* layer_out) {
    __KVcache& cache = *(__KVcache*)kvp;
    std::vector<LayerWeights> L = to_layers(m);
    try {
        if (layer_out == nullptr) {
            forward_cached(X, L.data(), m->num_layers, m->final_rms_weight, cos_t, sin_t, seq, start_pos, cache,
                           m->hidden, m->num_heads, m->num_kv_heads, m->head_dim, m->intermediate);
            return 0;
        }
        if (cache.num_layers < m->num_layers || cache.num_kv_heads != m->num_kv_heads ||
            cache.head_dim != m->head_dim || start_pos < 0 || start_pos + seq > cache.max_seq)
            return -1;
        const size_t H = (size_t)m->hidden;
        for (int l = 0; l < m->num_layers; l++) {
            const LayerWeights& w = L[(size_t)l];
            const __KVq kvq{cache.k_ptr(l, 0), cache.ks_ptr(l, 0), cache.v_ptr(l, 0), cache.vs_ptr(l, 0),
                            cache.max_seq};
            transformer_layer(X, w.rms1_weight, w.Wq, w.Wk, w.Wv, w.Wo, w.bq, w.bk, w.bv, cos_t, sin_t,
                              w.rms2_weight, w.W1, w.W2, w.W3, seq, m->hidden, m->num_heads, m->num_kv_heads,
                              m->head_dim, m->intermediate, start_pos, kvq);
            std::memcpy(layer_out + (size_t)l * seq * H, X, sizeof(float) * seq * H);
        }
        std::vector<float> xn((size_t)seq * H);
        for (int i = 0; i < seq; i++)
            rmsnorm(X + (size_t)i * H, xn.data() + (size_t)i * H, m->final_rms_weight, m->hidden, 1e-5f);
        std::memcpy(X, xn.data(), sizeof(float) * seq * H);
        cache.current_len = start_pos + seq;
    } catch (const std::exception&) {
        return -1;
    }
    return 0;
}

struct cb_state {
    double* stamps;
    int cap;
    int n;
};

static bool stamp_cb(int, void* ud) {
    cb_state* s = (cb_state*)ud;
    if (s->n < s->cap) {
        timespec ts;
        clock_gettime(CLOCK_MONOTONIC, &ts);
        s->stamps[s->n] = (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
    }
    s->n++;
    return false;
}

/* generate (libs/model_libs/generate.h:90-112) or, with kv != NULL, generate_cached
 * (:9-89).  stamps (optional) receives CLOCK_MONOTONIC seconds at every emitted
 * token, the callback the reference's -tokenspeed report uses (pipeline.h:229-237). */
JYREF_API int jyref_generate(const jy_model_desc* m, const int* prompt_ids, int prompt_len, const int* eos_ids,
                             int num_eos, const float* cos_t, const float* sin_t, int max_seq, int max_new,
                             float temperature, float repetition_penalty, int* out_ids, void* kv, double* stamps,
                             int stamps_cap) {
    std::vector<LayerWeights> L = to_layers(m);
    cb_state st{stamps, stamps_cap, 0};
    token_cb cb = stamps ? stamp_cb : nullptr;
    try {
        if (kv == nullptr)
            return generate(prompt_ids, prompt_len, eos_ids, num_eos, to_wmat(m->embed), to_wmat(m->lm_head), L.data(),
                            m->num_layers, m->final_rms_weight, cos_t, sin_t, max_seq, max_new, temperature,
                            m->vocab_size, m->hidden, m->num_heads, m->num_kv_heads, m->head_dim, m->intermediate,
                            out_ids, repetition_penalty, cb, &st);
        return generate_cached(prompt_ids, prompt_len, eos_ids, num_eos, to_wmat(m->embed), to_wmat(m->lm_head),
                               L.data(), m->num_layers, m->final_rms_weight, cos_t, sin_t, max_seq, max_new,
                               temperature, m->vocab_size, m->hidden, m->num_heads, m->num_kv_heads, m->head_dim,
                               m->intermediate, *(__KVcache*)kv, out_ids, repetition_penalty, cb, &st);
    } catch (const std::exception&) {
        return -1;
    }
}

/* ---------------------------------------------------------------- text layer
 * The reference's tokenizer, JSON lookups, model-directory bind and BPE trainer,
 * for the text-path checks.  The C ABI itself (jieyu_load, jieyu_generate, ...) is
 * exported by main.hpp above under its own names. */

JYREF_API void* jyref_tok_load(const char* vocab, const char* merges) {
    auto* t = new json_libs::Tokenizer();
    if (!t->load(vocab, merges)) {
        delete t;
        return nullptr;
    }
    return t;
}

JYREF_API void jyref_tok_free(void* t) { delete (json_libs::Tokenizer*)t; }

JYREF_API int jyref_tok_info(void* t, int* vocab_size, int* bos, int* eos, int* unk) {
    auto* k = (json_libs::Tokenizer*)t;
    *vocab_size = (int)k->vocab_size();
    *bos = k->bos_id();
    *eos = k->eos_id();
    *unk = k->unk_id();
    return 0;
}

JYREF_API int jyref_tok_add_special(void* t, const char* piece) {
    return ((json_libs::Tokenizer*)t)->add_special_token(piece);
}

JYREF_API int jyref_tok_encode(void* t, const char* text, size_t len, int32_t* ids, int cap) {
    const std::vector<int32_t> v = ((json_libs::Tokenizer*)t)->encode(std::string(text, len));
    for (int i = 0; i < (int)v.size() && i < cap; i++) ids[i] = v[(size_t)i];
    return (int)v.size();
}

JYREF_API int jyref_tok_decode(void* t, const int32_t* ids, int n, char* out, int cap) {
    const std::string s = ((json_libs::Tokenizer*)t)->decode(std::vector<int32_t>(ids, ids + n));
    if (cap > 0) memcpy(out, s.data(), std::min<size_t>(s.size(), (size_t)cap));
    return (int)s.size();
}

JYREF_API int jyref_info_int(const char* path, const char* key, int fallback) {
    return pipeline::read_info_int(path, key, fallback);
}

JYREF_API int jyref_info_str(const char* path, const char* key, const char* fallback, char* out, int cap) {
    const std::string v = pipeline::read_info_str(path, key, fallback);
    if (cap > 0) {
        const size_t n = std::min<size_t>(v.size(), (size_t)cap - 1);
        memcpy(out, v.data(), n);
        out[n] = 0;
    }
    return (int)v.size();
}

/* install_model + bind_model; hp as jytext_model_bind's first nine entries */
JYREF_API int jyref_model_bind(const char* dir, int max_seq, int* hp, char* err, int cap) {
    std::string e;
    bool ok = false;
    pipeline::ModelRefs r;
    free_model_map();
    try {
        install_model(std::filesystem::path(dir));
        ok = pipeline::bind_model(r, max_seq, &e);
    } catch (const std::exception& x) {
        e = std::string("装载 model.bf 失败: ") + x.what();
    }
    if (cap > 0) {
        const size_t n = std::min<size_t>(e.size(), (size_t)cap - 1);
        memcpy(err, e.data(), n);
        err[n] = 0;
    }
    if (ok && hp) {
        const int v[9] = {r.num_layers, r.hidden, r.num_heads, r.num_kv_heads, r.head_dim, r.intermediate,
                          r.vocab_size, r.add_bos ? 1 : 0, r.qkv_bias ? 1 : 0};
        memcpy(hp, v, sizeof v);
    }
    r.free();
    free_model_map();
    return ok ? 0 : -1;
}

/* BPETrainer (libs/tokenizer_libs/include/trainer.h:63-132, :370-395) */
JYREF_API int jyref_train_bpe(const char* corpus, int target_vocab, const char* out_dir) {
    json_libs::BPETrainer t(target_vocab);
    if (!t.load_corpus(corpus)) return -1;
    t.train();
    return t.save(out_dir) ? (int)t.vocab_size() : -1;
}

/* write_byte_level_vocab (libs/tokenizer_libs/include/byte_vocab.h:15-38) */
JYREF_API int jyref_write_byte_vocab(const char* vocab, const char* merges) {
    try {
        json_libs::write_byte_level_vocab(vocab, merges);
    } catch (const std::exception&) {
        return -1;
    }
    return 0;
}

/* ggufc::convert (libs/gguf_libs/gguf_convert.h:260-421): 0, or -1 with the error text */
JYREF_API int jyref_gguf_convert(const char* src, const char* out_dir, int out_dtype, int quant, long long* info,
                                 char* err, int cap) {
    try {
        ggufc::Options o;
        o.src = src;
        o.out_dir = out_dir;
        o.out_dtype = (uint8_t)out_dtype;
        o.quant = quant != 0;
        o.verbose = false;
        const ggufc::Result r = ggufc::convert(o);
        if (info) {
            const long long v[16] = {(long long)r.head.hidden, (long long)r.head.layers, r.head.num_heads,
                                     r.head.num_kv_heads, r.head.head_dim, (long long)r.head.intermediate,
                                     (long long)r.head.vocab_size, r.rope_theta, r.max_position,
                                     (long long)r.tensor_count, r.transposed, r.permuted, r.quant,
                                     r.tied_lm_head ? 1 : 0, r.eos_id, (long long)r.file_size};
            std::memcpy(info, v, sizeof v);
        }
        return 0;
    } catch (const std::exception& e) {
        if (err && cap > 0) {
            std::strncpy(err, e.what(), (size_t)cap - 1);
            err[cap - 1] = 0;
        }
        return -1;
    }
}
