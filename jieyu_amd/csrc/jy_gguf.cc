// jy_gguf.cc — GGUF (v2 / v3) reader and the GGUF -> model-directory converter
// (libs/gguf_libs/gguf.h, libs/gguf_libs/gguf_convert.h): the other on-disk format
// jieyu's decode path is fed from.  Host C++17, no device code.
//
// The converter writes what jieyu's does, byte for byte:
//   model.bf          bfile v2 (libs/model_libs/bfile.h:276-341): every GGUF tensor
//                     with a Hugging Face name; Q4_K / Q5_K / Q6_K / Q8_0 2-D blocks
//                     copied row by row (quant = true), everything else dequantized
//                     and written as out_dtype, 2-D weights transposed to [in][out]
//                     (the embedding stays [vocab][hidden]); q / k rows permuted from
//                     GGUF's interleaved RoPE halves back to adjacent pairs (perm_row)
//   model_info.json   the header's hyper-parameters and tokenizer markers, merged into
//                     an existing file the way json_file::WriteJsonKey does
//   vocab.json, merges.txt  from tokenizer.ggml.tokens / .merges
// Errors are std::runtime_error with the reference's texts.
//
// How: the header is parsed into a plan (hyper-parameters, the list of output tensors
// with their layouts) and every check, including the source ranges and dequantization
// support of each tensor, runs before the first file is written, so a failed conversion
// writes nothing.  The source is then memory-mapped; quantized rows are copied out of
// the mapping, dense tensors dequantized from it block run by block run, and transposed
// weights produced in panels of whole-block input columns (each panel dequantizes only
// the blocks it covers from every source row).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <set>
#include <stdexcept>

#include "jy_text.h"

namespace jytext {

namespace {

namespace fs = std::filesystem;
using std::runtime_error;
using std::string;
using std::vector;

// ---------------------------------------------------------------- GGUF types (GGML's codes)

enum : uint32_t {
    G_F32 = 0, G_F16 = 1, G_Q4_0 = 2, G_Q4_1 = 3, G_Q5_0 = 6, G_Q5_1 = 7, G_Q8_0 = 8, G_Q8_1 = 9, G_Q2_K = 10,
    G_Q3_K = 11, G_Q4_K = 12, G_Q5_K = 13, G_Q6_K = 14, G_Q8_K = 15, G_IQ4_NL = 20, G_IQ4_XS = 23, G_I8 = 24,
    G_I16 = 25, G_I32 = 26, G_I64 = 27, G_F64 = 28, G_BF16 = 30
};
enum : uint32_t { M_U8 = 0, M_I8, M_U16, M_I16, M_U32, M_I32, M_F32, M_BOOL, M_STR, M_ARR, M_U64, M_I64, M_F64 };

const char* gtype_name(uint32_t t) {
    switch (t) {
        case G_F32: return "f32";
        case G_F16: return "f16";
        case G_BF16: return "bf16";
        case G_Q4_0: return "q4_0";
        case G_Q4_1: return "q4_1";
        case G_Q5_0: return "q5_0";
        case G_Q5_1: return "q5_1";
        case G_Q8_0: return "q8_0";
        case G_Q8_1: return "q8_1";
        case G_Q2_K: return "q2_K";
        case G_Q3_K: return "q3_K";
        case G_Q4_K: return "q4_K";
        case G_Q5_K: return "q5_K";
        case G_Q6_K: return "q6_K";
        case G_IQ4_NL: return "iq4_nl";
        case G_IQ4_XS: return "iq4_xs";
        case G_I8: return "i8";
        case G_I16: return "i16";
        case G_I32: return "i32";
        case G_I64: return "i64";
        case G_F64: return "f64";
        default: return "?";
    }
}

// (elements, bytes) per block; (0, 0) for a type GGUF files may name but jieyu does not know
std::pair<size_t, size_t> gblock(uint32_t t) {
    switch (t) {
        case G_F32: case G_I32: return {1, 4};
        case G_F16: case G_BF16: case G_I16: return {1, 2};
        case G_F64: case G_I64: return {1, 8};
        case G_I8: return {1, 1};
        case G_Q4_0: case G_IQ4_NL: return {32, 18};
        case G_Q4_1: return {32, 20};
        case G_Q5_0: return {32, 22};
        case G_Q5_1: return {32, 24};
        case G_Q8_0: return {32, 34};
        case G_Q8_1: return {32, 36};
        case G_Q2_K: return {256, 84};
        case G_Q3_K: return {256, 110};
        case G_Q4_K: return {256, 144};
        case G_Q5_K: return {256, 176};
        case G_Q6_K: return {256, 210};
        case G_Q8_K: return {256, 292};
        case G_IQ4_XS: return {256, 136};
        default: return {0, 0};
    }
}

uint64_t gtype_bytes(uint32_t t, uint64_t n) {
    const auto [be, bb] = gblock(t);
    if (!be) throw runtime_error(string("gguf: 不认识的量化类型 ") + gtype_name(t));
    if (n % be) throw runtime_error("gguf: 元素个数不是块的整数倍");
    if (n / be > ~0ull / bb) throw runtime_error("gguf: 张量字节数溢出");  // (a corrupt shape)
    return n / be * bb;
}

float h2f(const unsigned char* p) {
    const uint16_t h = (uint16_t)(p[0] | (p[1] << 8));
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31u;
    uint32_t m = h & 0x3FFu, bits;
    if (e == 0 && m == 0) {
        bits = s;
    } else if (e == 0) {  // subnormal: normalise
        int k = 0;
        while (!(m & 0x400u)) {
            m <<= 1;
            k++;
        }
        bits = s | ((uint32_t)(113 - k) << 23) | ((m & 0x3FFu) << 13);
    } else if (e == 31) {
        bits = s | 0x7F800000u | (m << 13);
    } else {
        bits = s | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float bf2f(const unsigned char* p) {
    const uint32_t bits = (uint32_t)(p[0] | (p[1] << 8)) << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void scale_min_k4(int j, const unsigned char* q, int& sc, int& mn) {
    if (j < 4) {
        sc = q[j] & 63;
        mn = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// gguf::dequant (libs/gguf_libs/gguf.h:145-315): n elements of type t to float.  Every
// product below is exact in float, so the one rounding of each sum is the reference's.
void dequant(uint32_t t, const unsigned char* src, float* dst, uint64_t n) {
    switch (t) {
        case G_F32: memcpy(dst, src, (size_t)n * 4); return;
        case G_F16:
            for (uint64_t i = 0; i < n; i++) dst[i] = h2f(src + 2 * i);
            return;
        case G_BF16:
            for (uint64_t i = 0; i < n; i++) dst[i] = bf2f(src + 2 * i);
            return;
        case G_Q8_0:
            for (uint64_t b = 0; b < n / 32; b++) {
                const unsigned char* p = src + b * 34;
                const float d = h2f(p);
                for (int j = 0; j < 32; j++) dst[b * 32 + j] = (float)(int8_t)p[2 + j] * d;
            }
            return;
        case G_Q4_0: case G_Q4_1: case G_Q5_0: case G_Q5_1: {
            const bool min = t == G_Q4_1 || t == G_Q5_1, five = t == G_Q5_0 || t == G_Q5_1;
            const size_t bb = gblock(t).second;
            for (uint64_t b = 0; b < n / 32; b++) {
                const unsigned char* p = src + b * bb;
                const float d = h2f(p), m = min ? h2f(p + 2) : 0.0f;
                uint32_t qh = 0;
                if (five) memcpy(&qh, p + (min ? 4 : 2), 4);
                const unsigned char* q = p + (min ? 4 : 2) + (five ? 4 : 0);
                for (int j = 0; j < 16; j++) {
                    int x0 = q[j] & 0xF, x1 = q[j] >> 4;
                    if (five) {
                        x0 |= (int)(((qh >> j) & 1u) << 4);
                        x1 |= (int)(((qh >> (j + 16)) & 1u) << 4);
                    }
                    if (min) {
                        dst[b * 32 + j] = (float)x0 * d + m;
                        dst[b * 32 + j + 16] = (float)x1 * d + m;
                    } else {
                        const int off = five ? 16 : 8;
                        dst[b * 32 + j] = (float)(x0 - off) * d;
                        dst[b * 32 + j + 16] = (float)(x1 - off) * d;
                    }
                }
            }
            return;
        }
        case G_Q4_K: case G_Q5_K:
            for (uint64_t b = 0; b < n / 256; b++) {
                const unsigned char* p = src + b * (t == G_Q4_K ? 144 : 176);
                const float d = h2f(p), dmin = h2f(p + 2);
                const unsigned char* qh = p + 16;
                const unsigned char* qs = p + (t == G_Q4_K ? 16 : 48);
                float* y = dst + b * 256;
                for (int j = 0; j < 8; j++) {  // 32-weight steps; even j low nibbles, odd j high
                    int sc, mn;
                    scale_min_k4(j, p + 4, sc, mn);
                    const float d1 = d * (float)sc, n1 = dmin * (float)mn;
                    for (int l = 0; l < 32; l++) {
                        const unsigned char qb = qs[(j >> 1) * 32 + l];
                        int q = (j & 1) ? (qb >> 4) : (qb & 0xF);
                        if (t == G_Q5_K && ((qh[l] >> j) & 1)) q += 16;
                        y[32 * j + l] = d1 * (float)q - n1;
                    }
                }
            }
            return;
        case G_Q6_K:
            for (uint64_t b = 0; b < n / 256; b++) {
                const unsigned char* p = src + b * 210;
                const float d = h2f(p + 208);
                float* y = dst + b * 256;
                for (int e = 0; e < 256; e++) {
                    const int half = e >> 7, quarter = (e >> 5) & 3, l = e & 31;
                    const unsigned char qb = p[half * 64 + l + 32 * (quarter & 1)];
                    const int lo = quarter < 2 ? (qb & 0xF) : (qb >> 4);
                    const int hi = (p[128 + half * 32 + l] >> (2 * quarter)) & 3;
                    const int8_t sc = (int8_t)p[192 + half * 8 + l / 16 + 2 * quarter];
                    y[e] = d * (float)sc * (float)((lo | (hi << 4)) - 32);
                }
            }
            return;
        default: throw runtime_error(string("gguf: 还没写这种量化的反量化 ") + gtype_name(t));
    }
}

// ---------------------------------------------------------------- file

struct Meta {
    uint32_t type = 0, elem_type = 0;
    uint64_t n = 0;
    long long i = 0;
    double f = 0.0;
    string s;
    vector<long long> ints;
    vector<double> floats;
    vector<string> strs;
    // as_int / as_float (gguf.h:329-336): the scalar's own field, or an array's first element
    long long as_int(long long d) const { return type != M_ARR ? i : (ints.empty() ? d : ints[0]); }
    double as_float(double d) const { return type != M_ARR ? f : (floats.empty() ? d : floats[0]); }
};

struct GTensor {
    string name;
    uint32_t type = 0;
    vector<uint64_t> shape;
    uint64_t offset = 0, n_elem = 0, nbytes = 0;
};

class Reader {
public:
    Reader(std::istream& in, uint64_t size) : in_(in), size_(size) {}
    void bytes(void* p, size_t n) {
        if (!n) return;
        in_.read(static_cast<char*>(p), (std::streamsize)n);
        if (!in_) throw runtime_error("gguf: 文件被截断");
    }
    uint64_t u(int n) {
        unsigned char b[8];
        bytes(b, (size_t)n);
        uint64_t v = 0;
        for (int k = 0; k < n; k++) v |= (uint64_t)b[k] << (8 * k);
        return v;
    }
    string str(bool v3) {
        const uint64_t n = v3 ? u(8) : u(4);
        // a length past the end of the file is a truncated file (checked before allocating)
        if (n > size_) throw runtime_error("gguf: 文件被截断");
        string s((size_t)n, '\0');
        bytes(&s[0], (size_t)n);
        return s;
    }
    void scalar(uint32_t t, Meta& m) {
        switch (t) {
            case M_U8: m.i = (long long)u(1); break;
            case M_I8: m.i = (long long)(int8_t)u(1); break;
            case M_U16: m.i = (long long)u(2); break;
            case M_I16: m.i = (long long)(int16_t)u(2); break;
            case M_U32: m.i = (long long)u(4); break;
            case M_I32: m.i = (long long)(int32_t)u(4); break;
            case M_F32: {
                const uint32_t v = (uint32_t)u(4);
                float x;
                memcpy(&x, &v, 4);
                m.f = (double)x;
                break;
            }
            case M_BOOL: m.i = u(1) != 0 ? 1 : 0; break;
            case M_U64: case M_I64: m.i = (long long)u(8); break;
            case M_F64: {
                const uint64_t v = u(8);
                memcpy(&m.f, &v, 8);
                break;
            }
            default: throw runtime_error("gguf: 不认识的元数据类型 " + std::to_string(t));
        }
    }
    // meta_value (gguf.h:423-458)
    void value(bool v3, Meta& m) {
        m.type = (uint32_t)u(4);
        if (m.type == M_STR) {
            m.s = str(v3);
            return;
        }
        if (m.type != M_ARR) {
            scalar(m.type, m);
            return;
        }
        m.elem_type = (uint32_t)u(4);
        m.n = v3 ? u(8) : u(4);
        if (m.elem_type == M_ARR) throw runtime_error("gguf: 不支持嵌套数组");
        for (uint64_t k = 0; k < m.n; k++) {
            if (m.elem_type == M_STR) {
                m.strs.push_back(str(v3));
                continue;
            }
            Meta e;
            scalar(m.elem_type, e);
            if (m.elem_type == M_F32 || m.elem_type == M_F64)
                m.floats.push_back(e.f);
            else
                m.ints.push_back(e.i);
        }
    }

private:
    std::istream& in_;
    uint64_t size_;
};

struct GFile {
    string path;
    uint32_t version = 0;
    uint64_t align = 32, data_off = 0, file_size = 0;
    vector<std::pair<string, Meta>> kvs;
    vector<GTensor> tensors;

    const Meta* meta(const string& k) const {
        for (const auto& kv : kvs)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    const GTensor* find(const string& n) const {
        for (const GTensor& t : tensors)
            if (t.name == n) return &t;
        return nullptr;
    }
};

// gguf::open (gguf.h:495-541)
GFile gguf_open(const string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw runtime_error("gguf: 打不开 " + path);
    f.seekg(0, std::ios::end);
    const uint64_t size = (uint64_t)f.tellg();
    f.seekg(0);
    Reader r(f, size);
    GFile g;
    g.path = path;
    g.file_size = size;
    char magic[4];
    r.bytes(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) throw runtime_error("gguf: magic 不是 GGUF");
    g.version = (uint32_t)r.u(4);
    if (g.version < 2 || g.version > 3) throw runtime_error("gguf: 只支持 v2/v3，遇到 v" + std::to_string(g.version));
    const bool v3 = g.version == 3;
    const uint64_t nt = v3 ? r.u(8) : r.u(4), nk = v3 ? r.u(8) : r.u(4);
    for (uint64_t k = 0; k < nk; k++) {
        string key = r.str(v3);
        Meta m;
        r.value(v3, m);
        g.kvs.emplace_back(std::move(key), std::move(m));
    }
    for (uint64_t k = 0; k < nt; k++) {
        GTensor t;
        t.name = r.str(v3);
        const uint32_t nd = (uint32_t)r.u(4);
        if (nd == 0 || nd > 4) throw runtime_error("gguf: 维度数不对 " + t.name);
        t.n_elem = 1;
        for (uint32_t d = 0; d < nd; d++) {
            t.shape.push_back(r.u(8));
            // model.bf keeps 32-bit dims, and a zero dim leaves the writer's loops over the
            // others with nothing to bound them
            if (t.shape.back() == 0 || t.shape.back() > 0xFFFFFFFFull)
                throw runtime_error("gguf: 张量维度不对 " + t.name);
            // (a corrupt shape whose element count wraps would pass every range check)
            if (t.n_elem > ~0ull / t.shape.back()) throw runtime_error("gguf: 张量元素个数溢出 " + t.name);
            t.n_elem *= t.shape.back();
        }
        t.type = (uint32_t)r.u(4);
        t.offset = r.u(8);
        t.nbytes = gtype_bytes(t.type, t.n_elem);
        g.tensors.push_back(std::move(t));
    }
    if (const Meta* al = g.meta("general.alignment")) {
        const long long a = al->as_int(32);
        if (a > 0) g.align = (uint64_t)a;
    }
    const uint64_t here = (uint64_t)f.tellg();
    // (an alignment past the file's size would wrap the data offset: such a file has no data)
    if (g.align > size) throw runtime_error("gguf: general.alignment 超出文件大小");
    g.data_off = (here + g.align - 1) / g.align * g.align;
    return g;
}

// ---------------------------------------------------------------- output formats

uint16_t f2h(float v) {  // converter.h:55-79: truncating exponent logic, mantissa rounded half up
    uint32_t b;
    memcpy(&b, &v, 4);
    const uint32_t sign = (b >> 31) << 15, exp = (b >> 23) & 0xFFu;
    uint32_t man = b & 0x7FFFFFu;
    if (exp == 0xFFu) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    int e = (int)exp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man = (man | 0x800000u) >> (unsigned)(1 - e);
        return (uint16_t)(sign | ((man + 0x1000u) >> 13));
    }
    uint32_t hm = (man + 0x1000u) >> 13;
    if (hm == 0x400u) {
        hm = 0;
        if (++e >= 31) return (uint16_t)(sign | 0x7C00u);
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | hm);
}

uint16_t f2bf(float v) {  // converter.h:81-86: + 0x8000 unless inf / nan
    uint32_t b;
    memcpy(&b, &v, 4);
    if ((b & 0x7F800000u) != 0x7F800000u) b += 0x8000u;
    return (uint16_t)(b >> 16);
}

// float values in a model.bf dtype, little-endian, appended to `out`
void encode_values(const float* v, size_t n, uint8_t dtype, vector<unsigned char>& out) {
    if (n == 0) return;  // (a tensor with a zero dimension: nothing to append, and v may be null)
    const size_t at = out.size();
    if (dtype == BF_F32) {
        out.resize(at + n * 4);
        memcpy(out.data() + at, v, n * 4);
        return;
    }
    out.resize(at + n * 2);
    unsigned char* o = out.data() + at;
    for (size_t i = 0; i < n; i++) {
        const uint16_t h = dtype == BF_F16 ? f2h(v[i]) : f2bf(v[i]);
        o[2 * i] = (unsigned char)h;
        o[2 * i + 1] = (unsigned char)(h >> 8);
    }
}

size_t bf_elem_bytes(uint8_t d) { return d == BF_F32 || d == BF_I32 ? 4 : (d == BF_F16 || d == BF_BF16) ? 2 : d == BF_I8 ? 1 : 0; }

// GGUF stores q / k rows with each head's RoPE pairs split into halves; jieyu's
// rope_at takes adjacent pairs, so output row r of a head reads source row
// perm_row(r) (gguf_convert.h:67-70)
uint64_t perm_row(uint64_t r, int hd) {
    const uint64_t h = r / hd, k = r % hd;
    return h * hd + ((k & 1) ? hd / 2 + k / 2 : k / 2);
}

bool dequant_known(uint32_t t) {
    switch (t) {
        case G_F32: case G_F16: case G_BF16: case G_Q8_0: case G_Q4_0: case G_Q4_1: case G_Q5_0: case G_Q5_1:
        case G_Q4_K: case G_Q5_K: case G_Q6_K: return true;
        default: return false;
    }
}

// The source file mapped read-only: every tensor's bytes are a pointer into it.
class Mapped {
public:
    explicit Mapped(const string& path) {
        fd_ = ::open(path.c_str(), O_RDONLY);
        if (fd_ < 0) throw runtime_error("gguf: 打不开 " + path);
        struct stat st;
        if (fstat(fd_, &st) != 0) throw runtime_error("gguf: 打不开 " + path);
        size_ = (uint64_t)st.st_size;
        if (size_) {
            void* p = mmap(nullptr, (size_t)size_, PROT_READ, MAP_PRIVATE, fd_, 0);
            if (p == MAP_FAILED) throw runtime_error("gguf: 打不开 " + path);
            base_ = static_cast<const unsigned char*>(p);
        }
    }
    ~Mapped() {
        if (base_) munmap(const_cast<unsigned char*>(base_), (size_t)size_);
        if (fd_ >= 0) ::close(fd_);
    }
    Mapped(const Mapped&) = delete;
    Mapped& operator=(const Mapped&) = delete;
    const unsigned char* data() const { return base_; }
    uint64_t size() const { return size_; }

private:
    int fd_ = -1;
    const unsigned char* base_ = nullptr;
    uint64_t size_ = 0;
};

// One tensor of the output: where its values come from and how they are laid out.
//   raw        quantized 2-D blocks kept: source row j (or perm_row(j) for q / k) per row
//   transposed a 2-D weight dequantized, GGUF's [out rows][in] written as [in][out]
//   pairs      q / k: rows (or a bias's elements) back in adjacent RoPE pair order
struct OutTensor {
    string name;
    const GTensor* src = nullptr;
    uint8_t dtype = BF_F32;
    vector<uint32_t> shape;
    uint64_t bytes = 0;
    bool raw = false, transposed = false, pairs = false;
};

uint64_t bf_tensor_bytes(uint8_t d, uint64_t elems) {
    if (d == BF_Q4K || d == BF_Q5K || d == BF_Q6K)
        return elems % 256 ? ~0ull : elems / 256 * (d == BF_Q4K ? 144 : d == BF_Q5K ? 176 : 210);
    if (d == BF_Q8_0) return elems % 32 ? ~0ull : elems / 32 * 34;
    const size_t eb = bf_elem_bytes(d);
    return eb ? elems * eb : ~0ull;
}

constexpr size_t kFlushBytes = 16u << 20;  // output buffered in pieces of about this size

void flush_if(std::ostream& f, vector<unsigned char>& buf, bool all) {
    if (buf.empty() || (!all && buf.size() < kFlushBytes)) return;
    f.write(reinterpret_cast<const char*>(buf.data()), (std::streamsize)buf.size());
    buf.clear();
}

// a tensor's bytes in model.bf order, read from the mapped source (bounds checked when
// the conversion was planned)
void write_tensor(const unsigned char* file, uint64_t data_off, const OutTensor& o, int hd, std::ostream& f) {
    const GTensor& t = *o.src;
    const unsigned char* src = file + data_off + t.offset;
    const auto [be, bb] = gblock(t.type);
    vector<unsigned char> buf;
    buf.reserve(kFlushBytes + (1u << 20));
    if (o.raw) {
        const uint64_t rows = t.shape[1], row_bytes = t.shape[0] / be * bb;
        for (uint64_t j = 0; j < rows; j++) {
            const unsigned char* r = src + (o.pairs ? perm_row(j, hd) : j) * row_bytes;
            buf.insert(buf.end(), r, r + row_bytes);
            flush_if(f, buf, false);
        }
        flush_if(f, buf, true);
        return;
    }
    vector<float> vals;
    if (!o.transposed) {
        if (o.pairs) {  // a q / k bias: whole, then reordered
            vector<float> v((size_t)t.n_elem);
            dequant(t.type, src, v.data(), t.n_elem);
            vals.resize(v.size());
            for (uint64_t i = 0; i < t.n_elem; i++) vals[(size_t)i] = v[(size_t)perm_row(i, hd)];
            encode_values(vals.data(), vals.size(), o.dtype, buf);
            flush_if(f, buf, true);
            return;
        }
        // in source order, a run of whole blocks at a time
        const uint64_t run = std::max<uint64_t>(1, (1u << 20) / be) * be;
        for (uint64_t e0 = 0; e0 < t.n_elem; e0 += run) {
            const uint64_t n = std::min(run, t.n_elem - e0);
            vals.resize((size_t)n);
            dequant(t.type, src + e0 / be * bb, vals.data(), n);
            encode_values(vals.data(), (size_t)n, o.dtype, buf);
            flush_if(f, buf, false);
        }
        flush_if(f, buf, true);
        return;
    }
    // transposed: output row c (input column c) holds every source row's element c.  The
    // output goes out in panels of `width` input columns (whole quant blocks); a panel is
    // filled by dequantizing, for each source row, only the blocks it covers.
    const uint64_t in_dim = t.shape[0], out_dim = t.shape[1], row_bytes = in_dim / be * bb;
    uint64_t width = (32u << 20) / (4 * std::max<uint64_t>(out_dim, 1)) / be * be;
    width = std::min(std::max<uint64_t>(width, be), in_dim);
    vector<float> panel, piece((size_t)width);
    for (uint64_t c0 = 0; c0 < in_dim; c0 += width) {
        const uint64_t w = std::min(width, in_dim - c0);
        panel.resize((size_t)(w * out_dim));
        for (uint64_t j = 0; j < out_dim; j++) {
            const unsigned char* r = src + (o.pairs ? perm_row(j, hd) : j) * row_bytes + c0 / be * bb;
            dequant(t.type, r, piece.data(), w);
            for (uint64_t c = 0; c < w; c++) panel[(size_t)(c * out_dim + j)] = piece[(size_t)c];
        }
        encode_values(panel.data(), panel.size(), o.dtype, buf);
        flush_if(f, buf, true);
    }
}

void put_le(unsigned char* p, uint64_t v, int n) {
    for (int k = 0; k < n; k++) p[k] = (unsigned char)(v >> (8 * k));
}
uint64_t align64(uint64_t v) { return (v + 63) & ~uint64_t(63); }

// model.bf, bfile v2 (libs/model_libs/bfile.h:276-341): a 64-byte header, a 104-byte
// entry per tensor, the data at 64-byte aligned offsets after the (aligned) table.
// The tensor entries were checked when the conversion was planned.
void write_model_bf(const string& path, const GgufResult& r, const Mapped& file, uint64_t data_off,
                    const vector<OutTensor>& ts) {
    const uint64_t table = align64(64 + 104 * (uint64_t)ts.size());
    vector<unsigned char> head((size_t)table, 0);
    memcpy(head.data(), "JYAIBF", 6);
    put_le(&head[6], r.hidden, 8);
    put_le(&head[14], r.layers, 8);
    head[22] = 1;
    head[23] = (unsigned char)r.num_heads;
    head[24] = (unsigned char)r.num_kv_heads;
    head[25] = (unsigned char)r.head_dim;
    put_le(&head[26], r.intermediate, 4);
    put_le(&head[30], r.vocab, 8);
    put_le(&head[38], 2, 4);
    put_le(&head[42], ts.size(), 4);
    put_le(&head[46], table, 4);
    put_le(&head[50], 104, 4);
    vector<uint64_t> at(ts.size());
    uint64_t pos = 0;
    for (size_t i = 0; i < ts.size(); i++) {
        at[i] = pos;
        pos = align64(pos + ts[i].bytes);
        unsigned char* e = &head[64 + 104 * i];
        memcpy(e, ts[i].name.data(), ts[i].name.size());
        e[64] = ts[i].dtype;
        e[65] = (unsigned char)ts[i].shape.size();
        for (size_t d = 0; d < ts[i].shape.size(); d++) put_le(e + 68 + 4 * d, ts[i].shape[d], 4);
        put_le(e + 88, at[i], 8);
        put_le(e + 96, ts[i].bytes, 8);
    }
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    if (!f) throw runtime_error("bfile: 无法写入 " + path);
    f.write(reinterpret_cast<const char*>(head.data()), (std::streamsize)head.size());
    uint64_t done = 0;
    static const char zeros[64] = {};
    for (size_t i = 0; i < ts.size(); i++) {
        f.write(zeros, (std::streamsize)(at[i] - done));  // < 64 bytes of alignment
        write_tensor(file.data(), data_off, ts[i], r.head_dim, f);
        done = at[i] + ts[i].bytes;
    }
    f.flush();
    if (!f) throw runtime_error("bfile: 写入失败 " + path);
}

// ---------------------------------------------------------------- model_info.json

// is_json_number (libs/json_libs/json_value.h:107-150)
bool json_number(const string& t) {
    size_t i = 0;
    const size_t n = t.size();
    if (i < n && t[i] == '-') i++;
    if (i >= n) return false;
    if (t[i] == '0') {
        if (++i < n && t[i] >= '0' && t[i] <= '9') return false;
    } else if (t[i] >= '1' && t[i] <= '9') {
        while (i < n && t[i] >= '0' && t[i] <= '9') i++;
    } else {
        return false;
    }
    if (i < n && t[i] == '.') {
        const size_t d = ++i;
        while (i < n && t[i] >= '0' && t[i] <= '9') i++;
        if (i == d) return false;
    }
    if (i < n && (t[i] == 'e' || t[i] == 'E')) {
        if (++i < n && (t[i] == '+' || t[i] == '-')) i++;
        const size_t d = i;
        while (i < n && t[i] >= '0' && t[i] <= '9') i++;
        if (i == d) return false;
    }
    return i == n;
}

void json_escape(string& out, const string& s) {
    out.push_back('"');
    for (const unsigned char c : s) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (c < 0x20u) {
                    char b[8];
                    snprintf(b, sizeof b, "\\u%04x", (unsigned)c);
                    out += b;
                } else {
                    out.push_back((char)c);
                }
        }
    }
    out.push_back('"');
}

// write_value (libs/json_libs/json_value.h:54-105): two-space indentation, "key": value
void json_write(string& out, const JValue& v, int level) {
    switch (v.kind) {
        case JValue::Null: out += "null"; return;
        case JValue::Bool: case JValue::Number: out += v.raw.empty() ? string("null") : v.raw; return;
        case JValue::String: json_escape(out, v.text); return;
        case JValue::Array:
            if (v.items.empty()) {
                out += "[]";
                return;
            }
            out += "[\n";
            for (size_t i = 0; i < v.items.size(); i++) {
                out.append((size_t)(level + 1) * 2, ' ');
                json_write(out, v.items[i], level + 1);
                out += i + 1 < v.items.size() ? ",\n" : "\n";
            }
            out.append((size_t)level * 2, ' ');
            out += "]";
            return;
        case JValue::Object:
            if (v.members.empty()) {
                out += "{}";
                return;
            }
            out += "{\n";
            for (size_t i = 0; i < v.members.size(); i++) {
                out.append((size_t)(level + 1) * 2, ' ');
                json_escape(out, v.members[i].first);
                out += ": ";
                json_write(out, v.members[i].second, level + 1);
                out += i + 1 < v.members.size() ? ",\n" : "\n";
            }
            out.append((size_t)level * 2, ' ');
            out += "}";
            return;
    }
}

// model_info.json as json_file::SetJsonWay + WriteJsonKey leave it (libs/json_libs/
// json.h:20-47, :146-176, :240-313) after a run of flat key writes: an existing document
// keeps its other members and their order (a key already present is updated in place, a
// new one appended); a missing or blank file starts as an empty object; a file that does
// not parse is left as it is.  Values are typed as make_value (json_parser.h:291-320)
// types them.
JValue info_value(const string& value) {
    JValue v;
    if (json_number(value)) {
        v.kind = JValue::Number;
        v.raw = value;
    } else if (value == "true" || value == "false") {
        v.kind = JValue::Bool;
        v.raw = value;
    } else if (value == "null") {
        v.kind = JValue::Null;
    } else if (value.empty() || (value[0] != '{' && value[0] != '[') || !json_parse(value, v)) {
        v = JValue();
        v.kind = JValue::String;
        v.text = value;
    }
    return v;
}

void merge_info(const string& path, const vector<std::pair<string, string>>& entries) {
    const string file = resolve_path(path);
    string text;
    JValue doc;
    if (!(read_file(file, text) && json_parse(text, doc))) {
        if (text.find_first_not_of(" \t\r\n") != string::npos) return;  // unparsable: untouched
        doc = JValue();
        doc.kind = JValue::Object;
    }
    for (const auto& [key, value] : entries) {
        auto it = std::find_if(doc.members.begin(), doc.members.end(), [&](const auto& m) { return m.first == key; });
        if (it != doc.members.end())
            it->second = info_value(value);
        else
            doc.members.emplace_back(key, info_value(value));
    }
    string out;
    json_write(out, doc, 0);
    out.push_back('\n');
    std::ofstream f(file, std::ios::binary | std::ios::trunc);
    f.write(out.data(), (std::streamsize)out.size());
}

// ---------------------------------------------------------------- names

const char* suffix_map(const string& s) {
    static const std::pair<const char*, const char*> m[] = {
        {"attn_norm.weight", "input_layernorm.weight"},   {"attn_q.weight", "self_attn.q_proj.weight"},
        {"attn_q.bias", "self_attn.q_proj.bias"},         {"attn_k.weight", "self_attn.k_proj.weight"},
        {"attn_k.bias", "self_attn.k_proj.bias"},         {"attn_v.weight", "self_attn.v_proj.weight"},
        {"attn_v.bias", "self_attn.v_proj.bias"},         {"attn_output.weight", "self_attn.o_proj.weight"},
        {"ffn_norm.weight", "post_attention_layernorm.weight"}, {"ffn_gate.weight", "mlp.gate_proj.weight"},
        {"ffn_down.weight", "mlp.down_proj.weight"},      {"ffn_up.weight", "mlp.up_proj.weight"},
    };
    for (const auto& p : m)
        if (s == p.first) return p.second;
    return nullptr;
}

// GGUF tensor name -> the Hugging Face name model.bf uses (gguf_convert.h:88-103); "" = skipped
string hf_name(const string& n) {
    if (n == "token_embd.weight") return "model.embed_tokens.weight";
    if (n == "output_norm.weight") return "model.norm.weight";
    if (n == "output.weight") return "lm_head.weight";
    if (n.size() > 4 && n.compare(0, 4, "blk.") == 0) {
        const size_t b = n.find('.', 4);
        if (b == string::npos) return "";
        const string idx = n.substr(4, b - 4);
        if (idx.empty() || idx.find_first_not_of("0123456789") != string::npos) return "";
        const char* sfx = suffix_map(n.substr(b + 1));
        return sfx ? "model.layers." + idx + "." + sfx : "";
    }
    return "";
}

int quant_code(uint32_t t) {
    switch (t) {
        case G_Q4_K: return BF_Q4K;
        case G_Q5_K: return BF_Q5K;
        case G_Q6_K: return BF_Q6K;
        case G_Q8_0: return BF_Q8_0;
        default: return -1;
    }
}

const char* dtype_name(uint8_t d) {
    switch (d) {
        case BF_F32: return "f32";
        case BF_F16: return "f16";
        case BF_BF16: return "bf16";
        case BF_I8: return "i8";
        case BF_I32: return "i32";
        case BF_Q4K: return "q4_K";
        case BF_Q5K: return "q5_K";
        case BF_Q6K: return "q6_K";
        case BF_Q8_0: return "q8_0";
        default: return "?";
    }
}

}  // namespace

namespace {

// ---------------------------------------------------------------- the plan

// Hyper-parameters from the header (llama.cpp's `<arch>.` keys), with the embedding's
// shape, the token list and the block names standing in for missing ones, and the
// checks model_info.json's fields need (gguf_convert.h:260-421 gives the texts)
void read_hyper(const GFile& g, GgufResult& r) {
    auto num = [&](const string& key, long long fallback) {
        const Meta* m = g.meta(r.arch + "." + key);
        return m ? m->as_int(fallback) : fallback;
    };
    long long hidden = num("embedding_length", 0), blocks = num("block_count", 0);
    const long long ffn = num("feed_forward_length", 0), heads = num("attention.head_count", 0);
    const long long kv_heads = num("attention.head_count_kv", heads);
    long long head_dim = num("attention.key_length", 0);
    const Meta* fb = g.meta(r.arch + ".rope.freq_base");
    const double theta = fb ? fb->as_float(10000.0) : 10000.0;
    const long long ctx = num("context_length", 1024);

    long long vocab = 0;
    if (const GTensor* e = g.find("token_embd.weight"); e && e->shape.size() >= 2) {
        if (hidden <= 0) hidden = (long long)e->shape[0];
        vocab = (long long)e->shape[1];
    }
    if (vocab <= 0)
        if (const Meta* tk = g.meta("tokenizer.ggml.tokens")) vocab = (long long)tk->n;
    if (blocks <= 0)
        for (const GTensor& t : g.tensors)
            if (t.name.rfind("blk.", 0) == 0 && t.name.size() > 4) blocks = std::max(blocks, atoll(t.name.c_str() + 4) + 1);

    if (hidden <= 0 || vocab <= 0 || blocks <= 0 || ffn <= 0)
        throw runtime_error("gguf: 超参不全（hidden / layers / intermediate / vocab）");
    if (heads <= 0) throw runtime_error("gguf: 没有 attention.head_count");
    if (head_dim <= 0) head_dim = hidden / heads;
    if (heads > 255 || kv_heads > 255 || head_dim > 255)
        throw runtime_error("gguf: num_heads / num_kv_heads / head_dim 必须落在 1..255");
    if (kv_heads <= 0 || heads % kv_heads) throw runtime_error("gguf: num_heads 必须能被 num_kv_heads 整除");
    if (hidden != heads * head_dim) printf("[警告] hidden(%lld) != num_heads*head_dim(%lld)\n", hidden, heads * head_dim);

    r.hidden = (uint64_t)hidden;
    r.layers = (uint64_t)blocks;
    r.num_heads = (int)(uint8_t)heads;
    r.num_kv_heads = (int)(uint8_t)kv_heads;
    r.head_dim = (int)(uint8_t)head_dim;
    r.intermediate = (uint32_t)ffn;
    r.vocab = (uint64_t)vocab;
    r.rope_theta = (long long)std::fabs(theta);
    r.max_position = ctx;
}

// every output tensor, in GGUF tensor order, then the tied head when the file has no
// output.weight; the counters of the report
vector<OutTensor> plan_tensors(const GFile& g, uint8_t out_dtype, bool quant, GgufResult& r,
                               vector<string>& skipped) {
    for (const GTensor& t : g.tensors)
        if (t.shape.size() == 2 && t.shape[0] % gblock(t.type).first)
            throw runtime_error("gguf: " + t.name + " 的行长不是量化块的整数倍");
    vector<OutTensor> out;
    auto add_dense = [&](const GTensor& t, const string& name, bool transposed, bool pairs, uint8_t dtype) {
        OutTensor o;
        o.name = name;
        o.src = &t;
        o.dtype = dtype;
        o.transposed = transposed;
        o.pairs = pairs;
        if (t.shape.size() == 1)
            o.shape = {(uint32_t)t.shape[0]};
        else if (transposed)  // [in][out]
            o.shape = {(uint32_t)t.shape[0], (uint32_t)t.shape[1]};
        else  // the embedding: [vocab][hidden]
            o.shape = {(uint32_t)(t.shape.size() > 1 ? t.shape[1] : 0), (uint32_t)t.shape[0]};
        o.bytes = bf_elem_bytes(dtype);
        for (uint32_t d : o.shape) o.bytes *= d;
        out.push_back(std::move(o));
        if (transposed) r.transposed++;
    };
    for (const GTensor& t : g.tensors) {
        const string hf = hf_name(t.name);
        if (hf.empty()) {
            skipped.push_back(t.name);
            continue;
        }
        const bool two_d = t.shape.size() == 2, embedding = t.name == "token_embd.weight";
        const bool pairs = t.name.find(".attn_q.") != string::npos || t.name.find(".attn_k.") != string::npos;
        const int code = two_d ? quant_code(t.type) : -1;
        if (quant && code >= 0) {
            OutTensor o;
            o.name = hf;
            o.src = &t;
            o.dtype = (uint8_t)code;
            o.raw = true;
            o.pairs = pairs;
            o.shape = {(uint32_t)t.shape[1], (uint32_t)t.shape[0]};
            o.bytes = t.nbytes;
            out.push_back(std::move(o));
            r.quant++;
        } else {
            add_dense(t, hf, two_d && !embedding, pairs, two_d ? out_dtype : (uint8_t)BF_F32);
        }
        if (pairs) r.permuted++;
    }
    if (!g.find("output.weight")) {
        const GTensor* e = g.find("token_embd.weight");
        if (!e) throw runtime_error("gguf: 既没有 output.weight 也没有 token_embd.weight");
        r.tied_lm_head = true;
        if (!(quant && quant_code(e->type) >= 0)) add_dense(*e, "lm_head.weight", true, false, out_dtype);
    }
    return out;
}

// what would stop model.bf from being written, found before anything is: the entry
// checks of bfile's writer (check_tensor_meta, bfile.h:258-273), then per tensor in output
// order a source range past the end of the file or a type with no dequantization
void check_tensors(const GFile& g, const vector<OutTensor>& ts, int hd) {
    if (align64(64 + 104 * (uint64_t)ts.size()) > 0xFFFFFFFFull) throw runtime_error("bfile: 张量太多");
    for (const OutTensor& o : ts) {
        if (o.name.empty() || o.name.size() > 63) throw runtime_error("bfile: 张量名长度必须 1..63: " + o.name);
        if (o.shape.size() > 4) throw runtime_error("bfile: 维度超过 4: " + o.name);
        if (o.dtype > BF_Q8_0) throw runtime_error("bfile: 不认识的 dtype: " + o.name);
        uint64_t elems = 1;
        for (uint32_t d : o.shape) elems *= d;
        if (bf_tensor_bytes(o.dtype, elems) != o.bytes) throw runtime_error("bfile: shape 与数据长度不符: " + o.name);
    }
    for (const OutTensor& o : ts) {
        // start = data_off + offset, formed only where it cannot wrap
        if (g.data_off > g.file_size || o.src->offset > g.file_size - g.data_off)
            throw runtime_error("bfile: 写张量失败: " + o.name);
        const uint64_t start = g.data_off + o.src->offset;
        if (o.src->nbytes > g.file_size - start)
            throw runtime_error("bfile: 写张量失败: " + o.name);
        if (!o.raw && !dequant_known(o.src->type))
            throw runtime_error(string("gguf: 还没写这种量化的反量化 ") + gtype_name(o.src->type));
    }
    // perm_row reads source rows h * hd + k for k < hd of every head: the q / k rows (or a
    // bias's elements) must be whole heads of an even head_dim, or it would read past the
    // tensor.  jieyu's converter does not check this (gguf_convert.h:67-70 indexes blindly).
    for (const OutTensor& o : ts) {
        if (!o.pairs) continue;
        const uint64_t n = o.src->shape.size() == 2 ? o.src->shape[1] : o.src->shape[0];
        if (hd <= 0 || hd % 2 || n % (uint64_t)hd)
            throw runtime_error("gguf: " + o.src->name + " 的行数不是偶数 head_dim(" + std::to_string(hd) +
                                ") 的整数倍");
    }
}

// model_info.json's keys, in the order jieyu's converter writes them
vector<std::pair<string, string>> info_entries(const GFile& g, const GgufResult& r, const string& src,
                                               uint8_t out_dtype, bool quant) {
    vector<std::pair<string, string>> e = {
        {"hidden_size", std::to_string(r.hidden)},
        {"layer_count", std::to_string(r.layers)},
        {"mode", "1"},
        {"num_heads", std::to_string(r.num_heads)},
        {"num_kv_heads", std::to_string(r.num_kv_heads)},
        {"head_dim", std::to_string(r.head_dim)},
        {"intermediate_size", std::to_string(r.intermediate)},
        {"vocab_size", std::to_string(r.vocab)},
        {"rope_theta", std::to_string(r.rope_theta)},
        {"max_position_embeddings", std::to_string(r.max_position)},
        {"dtype", quant ? string("quant") : string(dtype_name(out_dtype))},
        {"add_bos_token", "0"},
        {"rope_style", "adjacent_after_permute"},
        {"source_arch", r.arch},
        {"source_file", fs::path(src).filename().string()},
    };
    if (const Meta* nm = g.meta("general.name"); nm && !nm->s.empty()) e.emplace_back("source_name", nm->s);
    const Meta* tk = g.meta("tokenizer.ggml.tokens");
    if (!tk) return e;
    const std::set<string> vocab(tk->strs.begin(), tk->strs.end());
    // the chat markers: the first of each list the vocabulary holds
    const std::pair<const char*, vector<const char*>> markers[] = {
        {"message_start", {"<|im_start|>", "<|start_header_id|>"}},
        {"message_end", {"<|im_end|>", "<|eot_id|>", "<|end_of_turn|>"}},
        {"text_end", {"<|endoftext|>", "<|end_of_text|>", "</s>"}},
    };
    for (const auto& [key, cands] : markers)
        for (const char* c : cands)
            if (vocab.count(c)) {
                e.emplace_back(key, c);
                break;
            }
    // DeepSeek's template: markers spelled with U+FF5C (fullwidth vertical line) and
    // U+2581 (lower one eighth block)
    const string bar = "\xEF\xBD\x9C", low = "\xE2\x96\x81";
    auto marker = [&](const string& inner) { return "<" + bar + inner + bar + ">"; };
    const string user = marker("User"), assistant = marker("Assistant");
    if (vocab.count(user) && vocab.count(assistant)) {
        e.emplace_back("template", "deepseek");
        e.emplace_back("bos_text", marker("begin" + low + "of" + low + "sentence"));
        e.emplace_back("user_start", user);
        e.emplace_back("assistant_start", assistant);
        e.emplace_back("turn_end", marker("end" + low + "of" + low + "sentence"));
    }
    return e;
}

}  // namespace

// GGUF file -> model directory, as jieyu's converter (ggufc::convert,
// libs/gguf_libs/gguf_convert.h:260-421) leaves it.  Everything that can fail is checked
// before the first file is written, so a failed conversion writes nothing.
GgufResult gguf_convert(const std::string& src, const std::string& out_dir, uint8_t out_dtype, bool quant,
                        bool verbose) {
    const GFile g = gguf_open(src);
    GgufResult r;
    const Meta* arch = g.meta("general.architecture");
    r.arch = arch && !arch->s.empty() ? arch->s : string("llama");
    if (verbose) printf("GGUF v%u  %s  tensors %zu\n", g.version, r.arch.c_str(), g.tensors.size());
    read_hyper(g, r);
    vector<string> skipped;
    const vector<OutTensor> tensors = plan_tensors(g, out_dtype, quant, r, skipped);
    if (verbose && !skipped.empty()) {
        printf("  skipped %zu unknown tensors:", skipped.size());
        for (size_t i = 0; i < skipped.size() && i < 6; i++) printf(" %s", skipped[i].c_str());
        printf(skipped.size() > 6 ? " ...\n" : "\n");
    }
    check_tensors(g, tensors, r.head_dim);
    const Meta* tokens = g.meta("tokenizer.ggml.tokens");
    if (!tokens || tokens->strs.empty()) throw runtime_error("gguf: 没有 tokenizer.ggml.tokens，抽不出词表");
    r.eos_id = (int)(g.meta("tokenizer.ggml.eos_token_id") ? g.meta("tokenizer.ggml.eos_token_id")->as_int(-1) : -1);
    if (r.eos_id < 0)
        r.eos_id = (int)(g.meta("tokenizer.ggml.bos_token_id") ? g.meta("tokenizer.ggml.bos_token_id")->as_int(-1) : -1);

    // the files
    fs::create_directories(out_dir);
    const fs::path dir(out_dir);
    {
        const Mapped file(src);
        write_model_bf((dir / "model.bf").string(), r, file, g.data_off, tensors);
    }
    r.tensor_count = tensors.size();
    r.file_size = fs::file_size(dir / "model.bf");
    merge_info((dir / "model_info.json").string(), info_entries(g, r, src, out_dtype, quant));

    // vocab.json: {"piece": id, ...} one per line, only '"' and '\\' escaped;
    // merges.txt: the version line, then the merge rules (gguf_convert.h:231-258)
    string vocab = "{\n";
    for (size_t i = 0; i < tokens->strs.size(); i++) {
        if (i) vocab += ",\n";
        vocab += "  \"";
        for (const char c : tokens->strs[i]) {
            if (c == '"' || c == '\\') vocab.push_back('\\');
            vocab.push_back(c);
        }
        vocab += "\": " + std::to_string(i);
    }
    vocab += "\n}\n";
    string merges = "#version: 0.2\n";
    if (const Meta* mg = g.meta("tokenizer.ggml.merges"))
        for (const string& m : mg->strs) merges += m + "\n";
    for (const auto& [name, text] : {std::pair<const char*, const string*>{"vocab.json", &vocab},
                                     std::pair<const char*, const string*>{"merges.txt", &merges}}) {
        std::ofstream f((dir / name).string(), std::ios::binary | std::ios::trunc);
        if (!f) throw runtime_error(string("gguf: 写不了 ") + name);
        f.write(text->data(), (std::streamsize)text->size());
    }
    if (verbose) printf("  vocab %zu tokens, eos=%d\n", tokens->strs.size(), r.eos_id);
    return r;
}

}  // namespace jytext
