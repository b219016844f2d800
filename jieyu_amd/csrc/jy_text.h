// jy_text.h — host-side text layer of the JieyuAI_api.h boundary: the JSON
// reader, the model-directory loader (bfile v2 + model_info.json) and the
// byte-level BPE tokenizer.  Plain C++17, no device code.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "jieyu_model.h"

namespace jytext {

// ---------------------------------------------------------------- files

bool read_file(const std::string& path, std::string& out);
// a path that does not open is retried under ../, ../../ and ../../../
// (libs/json_libs/file_util.h:92-106)
std::string resolve_path(const std::string& path);
std::vector<std::string> split_lines(const std::string& text);

// ---------------------------------------------------------------- UTF-8

std::string utf8_encode(uint32_t cp);
// one code point at p (n bytes available); malformed input decodes as the single
// byte (libs/json_libs/file_util.h:36-73)
void utf8_decode(const char* p, size_t n, uint32_t& cp, size_t& len);

// ---------------------------------------------------------------- JSON

struct JValue {
    enum Kind { Null, Bool, Number, String, Array, Object };
    Kind kind = Null;
    std::string text;  // String: the unescaped text
    std::string raw;   // the value's source text (numbers and literals are read from it)
    std::vector<JValue> items;
    std::vector<std::pair<std::string, JValue>> members;  // in file order
};

// Whole-document parse (libs/json_libs/json_parser.h); false + message on error.
bool json_parse(const std::string& src, JValue& out, std::string* err = nullptr);
// member lookup: an exact top-level key first, then a dotted path a.b.c
const JValue* json_find(const JValue& root, const std::string& key);
// a String's text, else the value's source text
std::string json_text(const JValue& v);

// A JSON file opened once for key lookups (json_file::GetJsonData / GetJsonInt).
class JsonFile {
public:
    bool open(const std::string& path);
    bool loaded() const { return loaded_; }
    const JValue& root() const { return root_; }
    std::string get(const std::string& key) const;                  // "" when absent
    int get_int(const std::string& key, int fallback) const;          // std::stoi rules
    std::string get_str(const std::string& key, const std::string& fallback) const;

private:
    JValue root_;
    bool loaded_ = false;
};

int info_int(const std::string& path, const std::string& key, int fallback);
std::string info_str(const std::string& path, const std::string& key, const std::string& fallback);

// ---------------------------------------------------------------- tokenizer

// Byte-level BPE over vocab.json + merges.txt with special-token splitting
// (libs/tokenizer_libs/include/tokenizer.h:242-701).
class Tokenizer {
public:
    bool load(const std::string& vocab_path, const std::string& merges_path, std::string* err = nullptr);
    std::vector<int32_t> encode(const std::string& text) const;
    std::string decode(const int32_t* ids, size_t n) const;
    std::string piece(int32_t id) const;
    size_t vocab_size() const { return piece_to_id_.size(); }
    int32_t bos_id() const { return bos_; }
    int32_t eos_id() const { return eos_; }
    int32_t unk_id() const { return unk_; }
    // registers a piece already in the vocabulary as unsplittable; its id or -1
    int32_t add_special(const std::string& piece);

private:
    int32_t id_of(const std::string& piece) const;
    int32_t intern(const std::string& piece);
    std::vector<int32_t> merge(std::vector<int32_t> syms) const;
    int find_special(const std::string& text, size_t from, size_t& at, size_t& len) const;

    std::unordered_map<std::string, int32_t> piece_to_id_;
    std::vector<std::string> id_to_piece_;
    std::unordered_map<uint64_t, int32_t> rank_;   // (left id, right id) -> merge rank
    std::vector<int32_t> merged_;                  // rank -> merged token id
    int32_t byte_id_[256] = {};
    int32_t word_end_ = -1, bos_ = -1, eos_ = -1, unk_ = -1;
    std::vector<std::string> special_;
    std::vector<int32_t> special_ids_;
};

// ---------------------------------------------------------------- model directory

struct BfEntry {            // one 104-byte tensor-table record (libs/model_libs/bfile.h:124-135)
    std::string name;
    uint8_t dtype = 0;
    uint32_t ndim = 0;
    uint32_t shape[4] = {0, 0, 0, 0};
    uint64_t offset = 0, nbytes = 0;
};

enum BfType : uint8_t { BF_F32 = 0, BF_F16 = 1, BF_BF16 = 2, BF_I8 = 3, BF_I32 = 4, BF_Q4K = 5, BF_Q5K = 6,
                        BF_Q6K = 7, BF_Q8_0 = 8 };

// A model directory bound the way jieyu's load_model_dir does it
// (libs/model_libs/pipeline.h:63-153, :395-441): model.bf mapped read-only, its
// tensor table validated, the decoder's tensors located by name and checked
// against the header's shape, model_info.json read.
class ModelDir {
public:
    ModelDir() = default;
    ModelDir(const ModelDir&) = delete;
    ModelDir& operator=(const ModelDir&) = delete;
    ~ModelDir() { unmap(); }

    // install_model + bind_model; false + the reference's error text
    bool open(const std::string& dir, int max_seq, std::string& err);
    void unmap();

    // header (bytes 6..37 of model.bf)
    uint64_t hidden = 0, layers = 0, vocab = 0;
    uint8_t mode = 0, num_heads = 0, num_kv_heads = 0, head_dim = 0;
    uint32_t intermediate = 0;
    bool table_ok = false;  // a v2 tensor table is present and valid

    // bound model (valid after open() returns true)
    jy_model_desc desc{};
    std::vector<jy_layer_weights> layer_w;
    int max_seq = 0;
    bool add_bos = true;
    std::string info_path, vocab_path, merges_path;

    const BfEntry* find(const std::string& name) const;
    const void* data(const BfEntry* e) const { return base_ + data_off_ + e->offset; }
    size_t file_size() const { return size_; }
    const std::vector<BfEntry>& entries() const { return entries_; }

private:
    bool install(const std::string& dir, std::string& err);
    bool bind(std::string& err);
    bool wmat(const std::string& name, jy_wmat& out) const;
    const float* f32(const std::string& name) const;

    const unsigned char* base_ = nullptr;
    size_t size_ = 0;
    uint64_t data_off_ = 0;
    std::vector<BfEntry> entries_;
};

// ---------------------------------------------------------------- GGUF

// what ggufc::convert reports (libs/gguf_libs/gguf_convert.h:25-34)
struct GgufResult {
    uint64_t hidden = 0, layers = 0, vocab = 0;
    int num_heads = 0, num_kv_heads = 0, head_dim = 0;
    uint32_t intermediate = 0;
    long long rope_theta = 10000, max_position = 32768;
    size_t tensor_count = 0;
    uint64_t file_size = 0;
    int transposed = 0, permuted = 0, quant = 0;
    bool tied_lm_head = false;
    int eos_id = -1;
    std::string arch;
};

// GGUF file -> model directory (ggufc::convert, libs/gguf_libs/gguf_convert.h:260-421);
// out_dtype is the model.bf dtype of the non-quantized 2-D weights (BF_F32 / BF_F16 /
// BF_BF16), quant keeps Q4_K / Q5_K / Q6_K / Q8_0 blocks as they are.  Throws
// std::runtime_error with the reference's texts.
GgufResult gguf_convert(const std::string& src, const std::string& out_dir, uint8_t out_dtype, bool quant,
                        bool verbose);

}  // namespace jytext
