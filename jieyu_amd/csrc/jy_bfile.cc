// jy_bfile.cc — model directory loader: model.bf (bfile v2) mapped read-only,
// its tensor table validated, the decoder bound by tensor name.
//
// model.bf (libs/model_libs/bfile.h:17-22, :124-135, :141-187;
// libs/model_libs/install_model.h:17-48), little-endian:
//   0   "JYAIBF"
//   6   u64 hidden        14 u64 layers      22 u8 mode       23 u8 num_heads
//   24  u8 num_kv_heads   25 u8 head_dim     26 u32 intermediate
//   30  u64 vocab         38 u32 version (>= 2 has a tensor table)
//   42  u32 tensor count  46 u32 data offset 50 u32 entry size (104)
//   64  tensor table: {char name[64]; u8 dtype; u8 ndim; u16 pad; u32 shape[4];
//                      u32 pad; u64 offset; u64 nbytes} per tensor
//   data_off + offset: tensor bytes, offsets 64-byte aligned.
// 2-D f32/f16 weights are stored [in][out]; block-quantized ones [out][in/B].
//
// Error texts are the reference's own (load_model_dir / bind_model), so a
// caller that reports or matches them sees the same strings.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <filesystem>
#include <fstream>

#include "jy_text.h"

namespace jytext {

namespace {

uint32_t rd32(const unsigned char* p) { return p[0] | (p[1] << 8) | (p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const unsigned char* p) { return rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

size_t dtype_bytes(uint8_t d) {
    switch (d) {
        case BF_F32: case BF_I32: return 4;
        case BF_F16: case BF_BF16: return 2;
        case BF_I8: return 1;
        default: return 0;
    }
}
size_t block_elems(uint8_t d) {
    switch (d) {
        case BF_Q4K: case BF_Q5K: case BF_Q6K: return 256;
        case BF_Q8_0: return 32;
        default: return 0;
    }
}
size_t block_bytes(uint8_t d) {
    switch (d) {
        case BF_Q4K: return 144;
        case BF_Q5K: return 176;
        case BF_Q6K: return 210;
        case BF_Q8_0: return 34;
        default: return 0;
    }
}
// bytes a tensor of `elems` elements occupies; 0 for an unknown type or a
// partial quantization block
uint64_t tensor_bytes(uint8_t d, uint64_t elems) {
    const size_t be = block_elems(d);
    if (!be) return elems * dtype_bytes(d);
    return elems % be ? 0 : elems / be * block_bytes(d);
}

std::string layer_name(int l, const char* suffix) { return "model.layers." + std::to_string(l) + "." + suffix; }

std::string dims(const uint32_t* s, uint32_t n) {
    std::string t = "[";
    for (uint32_t i = 0; i < n; i++) t += (i ? "," : "") + std::to_string(s[i]);
    return t + "]";
}

}  // namespace

void ModelDir::unmap() {
    if (base_) munmap(const_cast<unsigned char*>(base_), size_);
    base_ = nullptr;
    size_ = 0;
    entries_.clear();
    table_ok = false;
}

const BfEntry* ModelDir::find(const std::string& name) const {
    if (!table_ok) return nullptr;
    for (const BfEntry& e : entries_)
        if (e.name == name.substr(0, 64)) return &e;
    return nullptr;
}

bool ModelDir::install(const std::string& dir, std::string& err) {
    namespace fs = std::filesystem;
    unmap();
    const fs::path d(dir);
    info_path = (d / "model_info.json").string();
    vocab_path = (d / "vocab.json").string();
    merges_path = (d / "merges.txt").string();
    const std::string bf = (d / "model.bf").string();
    auto fail = [&](const char* what) {
        err = std::string("装载 model.bf 失败: ") + what;
        return false;
    };
    std::error_code ec;
    if (!fs::exists(info_path, ec)) return fail("model_info.json not found");
    if (!fs::exists(bf, ec)) return fail("model.bf not found");
    const int fd = ::open(bf.c_str(), O_RDONLY);
    if (fd < 0) return fail("open_Error");
    struct stat st {};
    if (fstat(fd, &st) != 0) {
        ::close(fd);
        return fail("fstat_Error");
    }
    void* map = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);  // the mapping stays valid
    if (map == MAP_FAILED) return fail("mmap_Error");
    base_ = static_cast<const unsigned char*>(map);
    size_ = (size_t)st.st_size;
    if (!std::ifstream(info_path)) return fail("model_info.json open failed");

    // header fields past the end of a short file read as zero
    unsigned char h[64] = {};
    std::memcpy(h, base_, std::min<size_t>(size_, 64));
    if (size_ < 6 || std::memcmp(h, "JYAIBF", 6) != 0) return fail("model.bf magic not match");
    hidden = rd64(h + 6);
    layers = rd64(h + 14);
    mode = h[22];
    num_heads = h[23];
    num_kv_heads = h[24];
    head_dim = h[25];
    intermediate = rd32(h + 26);
    vocab = rd64(h + 30);
    if (size_ < 64 || rd32(h + 38) < 2) return true;  // v1 file: no tensor table, bind() reports it

    // tensor table (bfile.h:153-176)
    const uint32_t count = rd32(h + 42), entry_size = rd32(h + 50);
    data_off_ = rd32(h + 46);
    bool ok = entry_size == 104 && data_off_ >= 64 && data_off_ <= size_ && 64 + (uint64_t)count * 104 <= data_off_;
    for (uint32_t i = 0; ok && i < count; i++) {
        const unsigned char* p = base_ + 64 + (size_t)i * 104;
        BfEntry e;
        e.name.assign(reinterpret_cast<const char*>(p), strnlen(reinterpret_cast<const char*>(p), 64));
        e.dtype = p[64];
        e.ndim = p[65];
        for (int k = 0; k < 4; k++) e.shape[k] = rd32(p + 68 + 4 * k);
        e.offset = rd64(p + 88);
        e.nbytes = rd64(p + 96);
        uint64_t elems = 1;
        for (uint32_t k = 0; k < e.ndim && k < 4; k++) elems *= e.shape[k];
        const bool known = dtype_bytes(e.dtype) || block_elems(e.dtype);
        ok = e.ndim <= 4 && known && tensor_bytes(e.dtype, elems) == e.nbytes && e.offset % 64 == 0 &&
             data_off_ + e.offset + e.nbytes <= size_;
        entries_.push_back(std::move(e));
    }
    if (!ok) {
        entries_.clear();
        return fail("model.bf tensor table broken");
    }
    table_ok = true;
    return true;
}

const float* ModelDir::f32(const std::string& name) const {
    const BfEntry* e = find(name);
    return e && e->dtype == BF_F32 ? static_cast<const float*>(data(e)) : nullptr;
}

// a 2-D weight as the forward pass sees it (load_weights.h:26-35): f32, f16,
// q8_0 and the k-quants, each with its jy type
bool ModelDir::wmat(const std::string& name, jy_wmat& out) const {
    out = jy_wmat{nullptr, JY_F32};
    const BfEntry* e = find(name);
    if (!e) return false;
    switch (e->dtype) {
        case BF_F32: out = jy_wmat{data(e), JY_F32}; return true;
        case BF_Q8_0: out = jy_wmat{data(e), JY_Q8_0}; return true;
        case BF_F16: out = jy_wmat{data(e), JY_F16}; return true;
        case BF_Q4K: out = jy_wmat{data(e), JY_Q4_K}; return true;
        case BF_Q5K: out = jy_wmat{data(e), JY_Q5_K}; return true;
        case BF_Q6K: out = jy_wmat{data(e), JY_Q6_K}; return true;
        default: return false;  // bf16 / i8 / i32 are not weight types
    }
}

bool ModelDir::bind(std::string& err) {
    auto fail = [&](const std::string& m) {
        err = m;
        return false;
    };
    if (!table_ok) return fail("model.bf 没有张量目录,请先用 jieyu -convert 转化");
    desc = jy_model_desc{};
    desc.num_layers = (int)layers;
    desc.hidden = (int)hidden;
    desc.num_heads = num_heads;
    desc.num_kv_heads = num_kv_heads;
    desc.head_dim = head_dim;
    desc.intermediate = (int)intermediate;
    desc.vocab_size = (int)vocab;
    if (desc.num_layers <= 0 || desc.hidden <= 0 || desc.head_dim <= 0 || desc.num_heads <= 0)
        return fail("model.bf 头部超参不合法");
    if (max_seq <= 0) max_seq = 1024;

    // per-layer tensors in slot order (load_weights.h:51-125)
    static const char* const suffix[9] = {"input_layernorm.weight", "self_attn.q_proj.weight",
                                          "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                                          "self_attn.o_proj.weight", "post_attention_layernorm.weight",
                                          "mlp.gate_proj.weight", "mlp.down_proj.weight", "mlp.up_proj.weight"};
    layer_w.assign((size_t)desc.num_layers, jy_layer_weights{});
    for (int l = 0; l < desc.num_layers; l++) {
        jy_layer_weights& w = layer_w[(size_t)l];
        jy_wmat* slot[9] = {nullptr, &w.Wq, &w.Wk, &w.Wv, &w.Wo, nullptr, &w.W1, &w.W2, &w.W3};
        for (int k = 0; k < 9; k++) {
            const std::string name = layer_name(l, suffix[k]);
            bool ok;
            if (k == 0 || k == 5) {
                const float* p = f32(name);
                (k == 0 ? w.rms1_weight : w.rms2_weight) = p;
                ok = p != nullptr;
            } else {
                ok = wmat(name, *slot[k]);
            }
            if (!ok) return fail("缺少张量: " + name);
        }
    }
    for (int l = 0; l < desc.num_layers; l++) {
        jy_layer_weights& w = layer_w[(size_t)l];
        w.bq = f32(layer_name(l, "self_attn.q_proj.bias"));
        w.bk = f32(layer_name(l, "self_attn.k_proj.bias"));
        w.bv = f32(layer_name(l, "self_attn.v_proj.bias"));
    }
    if (!wmat("model.embed_tokens.weight", desc.embed)) return fail("缺少张量: model.embed_tokens.weight");

    // lm_head: lm_head.weight, else the embedding (tied); quantized [vocab][hidden],
    // f32/f16 [hidden][vocab] (load_weights.h:137-155)
    {
        const BfEntry* e = find("lm_head.weight");
        if (!e) e = find("model.embed_tokens.weight");
        const uint64_t V64 = (uint64_t)(int64_t)desc.vocab_size, H64 = (uint64_t)(int64_t)desc.hidden;
        bool ok = e && e->ndim == 2;
        if (ok && block_elems(e->dtype))
            ok = e->shape[0] == V64 && e->shape[1] == H64;
        else if (ok)
            ok = (e->dtype == BF_F32 || e->dtype == BF_F16) && e->shape[0] == H64 && e->shape[1] == V64;
        if (ok) ok = wmat(e->name, desc.lm_head);
        if (!ok) return fail("lm_head.weight 缺失或形状不是 [hidden, vocab]（权重共享时需要转换器补一份转置副本）");
    }
    desc.final_rms_weight = f32("model.norm.weight");
    if (!desc.final_rms_weight) return fail("缺少张量: model.norm.weight");

    // shapes of the embedding, the final norm and layer 0 (pipeline.h:96-138)
    const uint32_t H = (uint32_t)desc.hidden, V = (uint32_t)desc.vocab_size, F = (uint32_t)desc.intermediate;
    const uint32_t q = (uint32_t)(desc.num_heads * desc.head_dim), kv = (uint32_t)(desc.num_kv_heads * desc.head_dim);
    struct Want {
        std::string name;
        uint32_t n;
        uint32_t s[2];
    };
    auto w2 = [&](const char* sfx, uint32_t in, uint32_t out) {
        const std::string name = layer_name(0, sfx);
        const BfEntry* e = find(name);
        const bool blocked = e && block_elems(e->dtype);
        return Want{name, 2, {blocked ? out : in, blocked ? in : out}};
    };
    const Want checks[] = {
        {"model.embed_tokens.weight", 2, {V, H}},
        {"model.norm.weight", 1, {H, 0}},
        {layer_name(0, "input_layernorm.weight"), 1, {H, 0}},
        w2("self_attn.q_proj.weight", H, q),
        w2("self_attn.k_proj.weight", H, kv),
        w2("self_attn.v_proj.weight", H, kv),
        w2("self_attn.o_proj.weight", q, H),
        w2("mlp.gate_proj.weight", H, F),
        w2("mlp.up_proj.weight", H, F),
        w2("mlp.down_proj.weight", F, H),
    };
    auto shape_is = [&](const BfEntry* e, const Want& w) {
        if (!e || e->ndim != w.n) return false;
        for (uint32_t i = 0; i < w.n; i++)
            if (e->shape[i] != w.s[i]) return false;
        return true;
    };
    for (const Want& c : checks) {
        const BfEntry* e = find(c.name);
        if (shape_is(e, c)) continue;
        if (!e) return fail("缺少张量: " + c.name);
        return fail(c.name + " 形状是 " + dims(e->shape, std::min<uint32_t>(e->ndim, 4)) + "，期望 " +
                    dims(c.s, c.n) + "（2D 权重需要转置）");
    }
    const Want bias[] = {{layer_name(0, "self_attn.q_proj.bias"), 1, {q, 0}},
                         {layer_name(0, "self_attn.k_proj.bias"), 1, {kv, 0}},
                         {layer_name(0, "self_attn.v_proj.bias"), 1, {kv, 0}}};
    for (const Want& c : bias) {
        const BfEntry* e = find(c.name);
        if (e && !shape_is(e, c)) return fail("张量形状不对: " + c.name);
    }
    desc.layers = layer_w.data();
    add_bos = info_int(info_path, "add_bos_token", 1) != 0;
    desc.rope_theta = (float)info_int(info_path, "rope_theta", 10000);
    return true;
}

bool ModelDir::open(const std::string& dir, int max_seq_, std::string& err) {
    max_seq = max_seq_;
    if (!install(dir, err)) {
        unmap();
        return false;
    }
    return bind(err);
}

}  // namespace jytext
