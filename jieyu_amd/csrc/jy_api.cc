// jy_api.cc — jieyu's text C ABI (include/jieyu_api.h) and the host-side text
// layer exports (include/jieyu_text.h).
//
// jieyu_load binds the model directory on the host (model.bf, model_info.json,
// vocab.json + merges.txt) and uploads the weights to HBM once; the mapping of
// model.bf is released after the upload.  jieyu_generate* encode the prompt,
// run generate_text's clamps (libs/model_libs/pipeline.h:280-374), decode on
// the device through jyhip_generate with a token callback that turns ids back
// into text and stops at special ids or stop markers, and copy the text out.
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <mutex>
#include <string>
#include <vector>

#include "jieyu_amd.h"
#include "jieyu_api.h"
#include "jieyu_text.h"
#include "jy_text.h"

namespace {

using jytext::ModelDir;
using jytext::Tokenizer;

// The process's one loaded model (main.hpp:15-28, pipeline.h:376-394).
struct Loaded {
    bool ready = false;
    std::string dir;
    Tokenizer tok;
    jyhip_model* dev = nullptr;
    jyhip_kv* kv = nullptr;
    int vocab = 0, max_seq = 0;
    bool add_bos = true;
    int max_new = 256;                // set by every generate call
    float rep_penalty = 1.1f;
    // model_info.json strings (pipeline.h:420-433)
    std::string s_start, s_end, s_text, s_system, s_name, s_user, s_asst, s_bos, s_turn;
    // ids of message_start / message_end / text_end; 0 when the piece is unset or
    // not in the vocabulary (pipeline.h:164-168, :434-436)
    int32_t sp_start = 0, sp_end = 0, sp_text = 0;

    void release() {
        if (kv) jyhip_kv_free(kv);
        if (dev) jyhip_model_free(dev);
        kv = nullptr;
        dev = nullptr;
        tok = Tokenizer();
        ready = false;
    }
};

Loaded& model() {
    static Loaded m;
    return m;
}
int g_handles = 0;
std::mutex g_lock;
thread_local char g_load_error[JIEYU_ERR_MAX] = {0};
thread_local std::string g_text_error;

void set_text(char* dst, size_t cap, const char* src) {
    if (!dst || !cap) return;
    const size_t n = src ? strlen(src) : 0, k = std::min(n, cap - 1);
    if (k) memcpy(dst, src, k);
    dst[k] = '\0';
}
void load_error(const std::string& m) { set_text(g_load_error, JIEYU_ERR_MAX, m.c_str()); }
void handle_error(jieyu_ctx* h, const char* m) { set_text(h->error, JIEYU_ERR_MAX, m); }

int32_t register_special(Tokenizer& t, const std::string& piece) {
    const int32_t id = piece.empty() ? -1 : t.add_special(piece);
    return id < 0 ? 0 : id;
}

// load_model_dir (pipeline.h:395-441) followed by the device upload
bool load_dir(Loaded& m, const std::string& dir, int max_seq, std::string& err) {
    m.dir = dir;
    ModelDir md;
    if (!md.open(dir, max_seq, err)) return false;
    std::string terr;
    if (!m.tok.load(md.vocab_path, md.merges_path, &terr)) {
        err = "分词器加载失败: " + md.vocab_path + " / " + md.merges_path;
        return false;
    }
    if ((int)m.tok.vocab_size() > md.desc.vocab_size)
        fprintf(stderr, "[jieyu_amd] warning: the vocabulary has %zu tokens but the model only %d embedding rows\n",
                m.tok.vocab_size(), md.desc.vocab_size);
    const std::string& info = md.info_path;
    m.s_start = jytext::info_str(info, "message_start", "");
    m.s_end = jytext::info_str(info, "message_end", "");
    m.s_text = jytext::info_str(info, "text_end", "");
    m.s_system = jytext::info_str(info, "system", "");
    m.s_name = jytext::info_str(info, "source_name", "");
    m.s_user = jytext::info_str(info, "user_start", "");
    m.s_asst = jytext::info_str(info, "assistant_start", "");
    m.s_bos = jytext::info_str(info, "bos_text", "");
    m.s_turn = jytext::info_str(info, "turn_end", "");
    m.sp_start = register_special(m.tok, m.s_start);
    m.sp_end = register_special(m.tok, m.s_end);
    m.sp_text = register_special(m.tok, m.s_text);
    register_special(m.tok, m.s_user);
    register_special(m.tok, m.s_asst);
    register_special(m.tok, m.s_bos);
    register_special(m.tok, m.s_turn);
    m.add_bos = md.add_bos;
    m.vocab = md.desc.vocab_size;
    m.max_seq = md.max_seq;

    // every weight type the bind produces (f32, f16, q8_0, q4_K, q5_K, q6_K) runs on
    // the device; the upload reports shapes it cannot run
    const jy_model_desc& d = md.desc;
    m.dev = jyhip_model_upload(&d, m.max_seq);
    if (!m.dev) {
        err = std::string("device upload failed: ") + jyhip_last_error();
        return false;
    }
    m.kv = jyhip_kv_create(m.dev, m.max_seq);
    if (!m.kv) {
        err = std::string("device KV cache: ") + jyhip_last_error();
        return false;
    }
    return true;  // md unmaps model.bf: the weights live in HBM now
}

// marker_at (pipeline.h:191-209): first position of a stop string, or of "<|"
// followed by 1..24 marker characters; npos when none
size_t marker_at(const std::string& s, const std::vector<std::string>& stops) {
    size_t best = std::string::npos;
    for (const std::string& st : stops) {
        const size_t at = s.find(st);
        if (at != std::string::npos && (best == std::string::npos || at < best)) best = at;
    }
    auto marker_char = [](unsigned char c) {
        return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || (c >= '0' && c <= '9') || c == '_' || c == '-';
    };
    for (size_t lt = s.find("<|"); lt != std::string::npos; lt = s.find("<|", lt + 1)) {
        size_t n = 0;
        while (lt + 2 + n < s.size() && n < 24 && marker_char((unsigned char)s[lt + 2 + n])) n++;
        if (n >= 1 && (best == std::string::npos || lt < best)) best = lt;
    }
    return best;
}

// the per-token callback of generate_text (echo_token, pipeline.h:224-255)
struct Sink {
    const Tokenizer* tok;
    std::string* out;
    int32_t sp[3];
    int nsp;
    std::vector<std::string> stops;
};

int on_token(int id, void* ud) {
    Sink* s = static_cast<Sink*>(ud);
    for (int i = 0; i < s->nsp; i++)
        if (id == s->sp[i]) return 1;
    const int32_t one = id;
    *s->out += s->tok->decode(&one, 1);
    const size_t at = marker_at(*s->out, s->stops);
    if (at != std::string::npos) {
        s->out->erase(at);
        return 1;
    }
    return 0;
}

struct DeviceError {
    std::string msg;
};

// generate_text (pipeline.h:280-374): > 0 tokens generated, 0 none, -1 an id
// outside the model's vocabulary
int generate_text(Loaded& m, const std::string& prompt, std::string& out, float temperature) {
    std::vector<int32_t> ids = m.tok.encode(prompt);
    const int32_t bos = m.tok.bos_id();
    if (m.add_bos && bos >= 0 && bos < m.vocab) ids.insert(ids.begin(), bos);
    if (ids.empty()) {
        out.clear();
        return 0;
    }
    long long max_new = m.max_new <= 0 ? m.max_seq : m.max_new;
    for (int32_t id : ids)
        if (id < 0 || id >= m.vocab) return -1;
    int prompt_len = (int)ids.size();
    if (prompt_len > m.max_seq) {
        prompt_len = m.max_seq;
        ids.resize((size_t)prompt_len);
    }
    if (prompt_len + max_new > m.max_seq) max_new = m.max_seq - prompt_len;
    if (max_new <= 0) {
        out.clear();
        return 0;
    }
    // up to three EOS ids: the tokenizer's, text_end's, message_end's
    int32_t eos[3];
    int neos = 0;
    for (long long e : {(long long)m.tok.eos_id(), (long long)m.sp_text, (long long)m.sp_end}) {
        if (e < 0 || e >= m.vocab) continue;
        if (std::find(eos, eos + neos, (int32_t)e) == eos + neos && neos < 3) eos[neos++] = (int32_t)e;
    }
    out.clear();
    Sink sink{&m.tok, &out, {0, 0, 0}, 0, {}};
    for (const std::string* c : {&m.s_start, &m.s_end, &m.s_text, &m.s_user, &m.s_asst, &m.s_turn})
        if (!c->empty()) sink.stops.push_back(*c);
    for (int32_t sp : {m.sp_start, m.sp_end, m.sp_text})
        if (sp != 0) sink.sp[sink.nsp++] = sp;
    std::vector<int> out_ids((size_t)m.max_seq + 1);
    const int len = jyhip_generate(m.dev, m.kv, ids.data(), prompt_len, neos ? eos : nullptr, neos, m.max_seq,
                                   (int)max_new, temperature, m.rep_penalty, out_ids.data(), on_token, &sink,
                                   nullptr, nullptr);
    if (len < 0) throw DeviceError{jyhip_last_error()};
    return len - prompt_len;
}

// json_ochat_build (libs/model_libs/jsonl_ochat.h:7-28): one "name\nmessage" turn
// per line that has either, wrapped in qb/qe (default message_start/end), then
// the assistant opener
std::string jsonl_prompt(const Loaded& m, const std::string& path, const std::string& qb, const std::string& qe) {
    std::string text;
    if (!jytext::read_file(jytext::resolve_path(path), text)) return std::string();
    const std::string pre = qb.empty() ? m.s_start : qb, suf = qe.empty() ? m.s_end : qe;
    std::string feed;
    // lines as jsonl_len / jsonl_sget count them: a trailing newline ends the last line
    size_t start = 0;
    while (start < text.size()) {
        const size_t nl = text.find('\n', start);
        const std::string line = text.substr(start, nl == std::string::npos ? std::string::npos : nl - start);
        jytext::JValue v;
        std::string name, msg;
        if (jytext::json_parse(line, v)) {
            if (const jytext::JValue* x = jytext::json_find(v, "name")) name = jytext::json_text(*x);
            if (const jytext::JValue* x = jytext::json_find(v, "message")) msg = jytext::json_text(*x);
        }
        if (!name.empty() || !msg.empty()) {
            feed += pre + name + '\n';
            feed += msg + suf + '\n';
        }
        if (nl == std::string::npos) break;
        start = nl + 1;
    }
    if (!feed.empty()) {
        if (!m.s_asst.empty())
            feed += m.s_asst;
        else if (m.s_start == "<|im_start|>")
            feed += m.s_start + "assistant\n";
    }
    return feed;
}

int copy_out(const std::string& text, char* out, int cap) {
    if (!out || cap <= 0) return (int)text.size();
    const size_t n = std::min(text.size(), (size_t)cap - 1);
    memcpy(out, text.data(), n);
    out[n] = '\0';
    return (int)text.size();
}

// the shared tail of both generate entry points (main.hpp:156-227)
template <class Run>
int generate_call(jieyu_ctx* h, char* out, int cap, int max_new, float rp, Run&& run) {
    Loaded& m = model();
    handle_error(h, "");
    m.max_new = max_new;
    m.rep_penalty = rp;
    std::string text;
    int produced;
    try {
        produced = run(m, text);
    } catch (const DeviceError& e) {
        handle_error(h, ("device: " + e.msg).c_str());
        return -1;
    } catch (const std::exception& e) {
        handle_error(h, e.what());
        return -1;
    }
    if (produced == -2) {
        handle_error(h, "jsonl_no_srch（文件里没有可用的 name/message）");
        return -1;
    }
    if (produced < 0) {
        handle_error(h, "生成失败（提示词里有超出词表的 token）");
        return -1;
    }
    if (produced == 0) handle_error(h, "没有产出（提示词为空或上下文已满）");
    copy_out(text, out, cap);
    return produced;
}

}  // namespace

extern "C" {

JIEYU_AMD_API jieyu_model jieyu_load(const char* dir, int max_seq) {
    if (!dir) {
        load_error("dir 为空");
        return nullptr;
    }
    std::lock_guard<std::mutex> g(g_lock);
    Loaded& m = model();
    const std::string d = std::filesystem::path(dir).string();
    if (m.ready && m.dir != d) m.release();  // another directory replaces the loaded one
    jieyu_ctx* ctx = new (std::nothrow) jieyu_ctx();
    if (!ctx) {
        load_error("内存不足");
        return nullptr;
    }
    set_text(ctx->dir, JIEYU_PATH_MAX, dir);
    if (max_seq > 0) {
        ctx->max_seq = max_seq;
    } else {
        // max_position_embeddings clamped to [64, 4096] (main.hpp:63-66)
        const int want = jytext::info_int((std::filesystem::path(d) / "model_info.json").string(),
                                          "max_position_embeddings", 1024);
        ctx->max_seq = std::max(64, std::min(want, 4096));
    }
    if (!m.ready) {
        std::string err;
        bool ok;
        try {
            ok = load_dir(m, d, ctx->max_seq, err);
        } catch (const std::exception& e) {
            ok = false;
            err = e.what();
        }
        if (!ok) {
            m.release();
            load_error(err);
            delete ctx;
            return nullptr;
        }
        m.ready = true;
    }
    g_handles++;
    load_error("");
    return ctx;
}

JIEYU_AMD_API void jieyu_free(jieyu_model h) {
    if (!h) return;
    std::lock_guard<std::mutex> g(g_lock);
    if (g_handles > 0 && --g_handles <= 0) model().release();
    delete h;
}

JIEYU_AMD_API const char* jieyu_last_error(jieyu_model h) { return h ? h->error : g_load_error; }

JIEYU_AMD_API const char* jieyu_version(void) { return "1.0.0"; }

JIEYU_AMD_API int jieyu_context_length(jieyu_model h) { return h ? h->max_seq : 0; }

JIEYU_AMD_API const char* jieyu_model_dir(jieyu_model h) { return h ? h->dir : ""; }

JIEYU_AMD_API int jieyu_generate(jieyu_model h, const char* prompt, char* out, int cap, int max_new,
                                 float temperature, float repetition_penalty) {
    if (!h) {
        load_error("句柄为空");
        return -1;
    }
    if (!prompt) {
        handle_error(h, "prompt 为空");
        return -1;
    }
    std::lock_guard<std::mutex> g(g_lock);
    if (!model().ready) {
        handle_error(h, "模型未装载（先 jieyu_load）");
        return -1;
    }
    const std::string p(prompt);
    return generate_call(h, out, cap, max_new, repetition_penalty,
                         [&](Loaded& m, std::string& text) { return generate_text(m, p, text, temperature); });
}

JIEYU_AMD_API int jieyu_generate_jsonl(jieyu_model h, const char* jsonl, const char* qb, const char* qe, char* out,
                                       int cap, int max_new, float temperature, float repetition_penalty) {
    if (!h) {
        load_error("句柄为空");
        return -1;
    }
    if (!jsonl) {
        handle_error(h, "jsonl 路径为空");
        return -1;
    }
    std::lock_guard<std::mutex> g(g_lock);
    if (!model().ready) {
        handle_error(h, "模型未装载（先 jieyu_load）");
        return -1;
    }
    const std::string path(jsonl), b(qb ? qb : ""), e(qe ? qe : "");
    return generate_call(h, out, cap, max_new, repetition_penalty, [&](Loaded& m, std::string& text) {
        text.clear();
        const std::string feed = jsonl_prompt(m, path, b, e);
        if (feed.empty()) return -2;
        return generate_text(m, feed, text, temperature);
    });
}

// ------------------------------------------------------------ jieyu_text.h

struct jytext_tokenizer {
    Tokenizer t;
};

JYTEXT_API const char* jytext_last_error(void) { return g_text_error.c_str(); }

JYTEXT_API jytext_tokenizer* jytext_tokenizer_load(const char* vocab_json, const char* merges_txt) {
    g_text_error.clear();
    if (!vocab_json || !merges_txt) {
        g_text_error = "NULL path";
        return nullptr;
    }
    auto* t = new (std::nothrow) jytext_tokenizer();
    if (!t) return nullptr;
    if (!t->t.load(vocab_json, merges_txt, &g_text_error)) {
        delete t;
        return nullptr;
    }
    return t;
}

JYTEXT_API void jytext_tokenizer_free(jytext_tokenizer* t) { delete t; }

JYTEXT_API int jytext_tokenizer_info(const jytext_tokenizer* t, int* vocab_size, int* bos, int* eos, int* unk) {
    if (!t) return -1;
    if (vocab_size) *vocab_size = (int)t->t.vocab_size();
    if (bos) *bos = t->t.bos_id();
    if (eos) *eos = t->t.eos_id();
    if (unk) *unk = t->t.unk_id();
    return 0;
}

JYTEXT_API int jytext_tokenizer_add_special(jytext_tokenizer* t, const char* piece) {
    return t && piece ? t->t.add_special(piece) : -1;
}

JYTEXT_API int jytext_tokenizer_encode(const jytext_tokenizer* t, const char* text, size_t len, int32_t* ids,
                                       int cap) {
    if (!t || (!text && len)) return -1;
    const std::vector<int32_t> v = t->t.encode(std::string(text ? text : "", len));
    if (ids && cap > 0) std::copy(v.begin(), v.begin() + std::min<size_t>(v.size(), (size_t)cap), ids);
    return (int)v.size();
}

JYTEXT_API int jytext_tokenizer_decode(const jytext_tokenizer* t, const int32_t* ids, int n, char* out, int cap) {
    if (!t || n < 0 || (!ids && n)) return -1;
    const std::string s = t->t.decode(ids, (size_t)n);
    if (out && cap > 0) memcpy(out, s.data(), std::min<size_t>(s.size(), (size_t)cap));
    return (int)s.size();
}

JYTEXT_API int jytext_info_int(const char* path, const char* key, int fallback) {
    return path && key ? jytext::info_int(path, key, fallback) : fallback;
}

JYTEXT_API int jytext_info_str(const char* path, const char* key, const char* fallback, char* out, int cap) {
    const std::string v = path && key ? jytext::info_str(path, key, fallback ? fallback : "")
                                      : std::string(fallback ? fallback : "");
    return copy_out(v, out, cap);
}

JYTEXT_API int jytext_gguf_convert(const char* src, const char* out_dir, int out_dtype, int quant, int verbose,
                                   long long* info) {
    g_text_error.clear();
    if (!src || !out_dir) {
        g_text_error = "src / out_dir is NULL";
        return -1;
    }
    try {
        const jytext::GgufResult r = jytext::gguf_convert(src, out_dir, (uint8_t)out_dtype, quant != 0, verbose != 0);
        if (info) {
            const long long v[16] = {(long long)r.hidden, (long long)r.layers, r.num_heads, r.num_kv_heads, r.head_dim,
                                     (long long)r.intermediate, (long long)r.vocab, r.rope_theta, r.max_position,
                                     (long long)r.tensor_count, r.transposed, r.permuted, r.quant,
                                     r.tied_lm_head ? 1 : 0, r.eos_id, (long long)r.file_size};
            memcpy(info, v, sizeof v);
        }
    } catch (const std::exception& e) {
        g_text_error = e.what();
        return -1;
    }
    return 0;
}

JYTEXT_API int jytext_model_bind(const char* dir, int max_seq, int* hp) {
    g_text_error.clear();
    if (!dir) {
        g_text_error = "dir is NULL";
        return -1;
    }
    ModelDir md;
    if (!md.open(dir, max_seq, g_text_error)) return -1;
    if (hp) {
        const jy_model_desc& d = md.desc;
        const int v[12] = {d.num_layers, d.hidden, d.num_heads, d.num_kv_heads, d.head_dim, d.intermediate,
                           d.vocab_size, md.add_bos ? 1 : 0, d.layers[0].bq ? 1 : 0, d.embed.type, d.lm_head.type,
                           d.layers[0].Wq.type};
        memcpy(hp, v, sizeof v);
    }
    return 0;
}

}  // extern "C"
