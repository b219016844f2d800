// jy_json.cc — files, UTF-8 and the JSON reader used by the model-directory
// loader and the tokenizer.  Follows what jieyu's json_libs accepts and returns
// (libs/json_libs/json_parser.h, json.h, file_util.h), so model_info.json and
// vocab.json read the same: numbers are kept as their source text, strings
// are unescaped (\uXXXX with surrogate pairs), lookups try the exact key and
// then a dotted path.
#include <cstdio>
#include <fstream>
#include <sstream>
#include <stdexcept>

#include "jy_text.h"

namespace jytext {

bool read_file(const std::string& path, std::string& out) {
    std::ifstream in(path, std::ios::binary);
    if (!in) return false;
    std::ostringstream ss;
    ss << in.rdbuf();
    out = ss.str();
    return true;
}

static bool readable(const std::string& path) {
    std::ifstream in(path, std::ios::binary);
    return static_cast<bool>(in);
}

std::string resolve_path(const std::string& path) {
    if (path.empty() || readable(path)) return path;
    std::string up;
    for (int i = 0; i < 3; i++) {
        up += "../";
        if (readable(up + path)) return up + path;
    }
    return path;
}

std::vector<std::string> split_lines(const std::string& text) {
    std::vector<std::string> lines;
    size_t at = 0;
    while (at < text.size()) {
        const size_t nl = text.find('\n', at);
        if (nl == std::string::npos) {
            lines.push_back(text.substr(at));
            break;
        }
        lines.push_back(text.substr(at, nl - at));
        at = nl + 1;
    }
    return lines;
}

std::string utf8_encode(uint32_t cp) {
    std::string s;
    if (cp < 0x80u) {
        s += (char)cp;
    } else if (cp < 0x800u) {
        s += (char)(0xC0u | (cp >> 6));
        s += (char)(0x80u | (cp & 0x3Fu));
    } else if (cp < 0x10000u) {
        s += (char)(0xE0u | (cp >> 12));
        s += (char)(0x80u | ((cp >> 6) & 0x3Fu));
        s += (char)(0x80u | (cp & 0x3Fu));
    } else {
        s += (char)(0xF0u | (cp >> 18));
        s += (char)(0x80u | ((cp >> 12) & 0x3Fu));
        s += (char)(0x80u | ((cp >> 6) & 0x3Fu));
        s += (char)(0x80u | (cp & 0x3Fu));
    }
    return s;
}

void utf8_decode(const char* p, size_t n, uint32_t& cp, size_t& len) {
    const unsigned char* u = reinterpret_cast<const unsigned char*>(p);
    const unsigned b0 = u[0];
    cp = b0;
    len = 1;
    auto cont = [&](size_t i) { return (u[i] & 0xC0u) == 0x80u; };
    if (b0 < 0x80u) return;
    // the lead byte picks the length; a short buffer or a bad continuation byte
    // leaves the lead byte on its own
    if ((b0 & 0xE0u) == 0xC0u) {
        if (n >= 2 && cont(1)) {
            cp = ((b0 & 0x1Fu) << 6) | (u[1] & 0x3Fu);
            len = 2;
        }
    } else if ((b0 & 0xF0u) == 0xE0u) {
        if (n >= 3 && cont(1) && cont(2)) {
            cp = ((b0 & 0x0Fu) << 12) | ((u[1] & 0x3Fu) << 6) | (u[2] & 0x3Fu);
            len = 3;
        }
    } else if ((b0 & 0xF8u) == 0xF0u) {
        if (n >= 4 && cont(1) && cont(2) && cont(3)) {
            cp = ((b0 & 0x07u) << 18) | ((u[1] & 0x3Fu) << 12) | ((u[2] & 0x3Fu) << 6) | (u[3] & 0x3Fu);
            len = 4;
        }
    }
}

namespace {

struct Reader {
    const std::string& s;
    size_t i = 0;
    std::string err;

    explicit Reader(const std::string& src) : s(src) {}

    bool bad(const char* m) {
        if (err.empty()) err = m;
        return false;
    }
    void ws() {
        while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) i++;
    }
    bool eat(char c) {
        if (i < s.size() && s[i] == c) {
            i++;
            return true;
        }
        return false;
    }
    bool hex4(uint32_t& v) {
        if (i + 4 > s.size()) return bad("truncated \\u escape");
        v = 0;
        for (int k = 0; k < 4; k++) {
            const char c = s[i + k];
            uint32_t d;
            if (c >= '0' && c <= '9') d = c - '0';
            else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
            else return bad("non-hex digit in \\u escape");
            v = v * 16 + d;
        }
        i += 4;
        return true;
    }
    bool str(std::string& out) {
        if (!eat('"')) return bad("expected '\"'");
        out.clear();
        while (i < s.size()) {
            const char c = s[i++];
            if (c == '"') return true;
            if (c != '\\') {
                out += c;
                continue;
            }
            if (i >= s.size()) break;
            const char e = s[i++];
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    uint32_t cp;
                    if (!hex4(cp)) return false;
                    // a high surrogate followed by \u: combine when the second is a low
                    // surrogate, otherwise the second escape is consumed and dropped
                    if (cp >= 0xD800u && cp <= 0xDBFFu && i + 1 < s.size() && s[i] == '\\' && s[i + 1] == 'u') {
                        i += 2;
                        uint32_t lo;
                        if (!hex4(lo)) return false;
                        if (lo >= 0xDC00u && lo <= 0xDFFFu) cp = 0x10000u + ((cp - 0xD800u) << 10) + (lo - 0xDC00u);
                    }
                    out += utf8_encode(cp);
                    break;
                }
                default: return bad("bad escape");
            }
        }
        return bad("unterminated string");
    }
    bool literal(const char* word, JValue::Kind k, JValue& v) {
        const size_t n = std::char_traits<char>::length(word);
        if (s.compare(i, n, word) == 0 && i + n <= s.size()) {
            i += n;
            v.kind = k;
            return true;
        }
        return bad("bad literal");
    }
    bool value(JValue& v) {
        ws();
        if (i >= s.size()) return bad("unexpected end");
        const size_t begin = i;
        const char c = s[i];
        bool ok;
        if (c == '{') {
            ok = object(v);
        } else if (c == '[') {
            ok = array(v);
        } else if (c == '"') {
            v.kind = JValue::String;
            ok = str(v.text);
        } else if (c == 't') {
            ok = literal("true", JValue::Bool, v);
        } else if (c == 'f') {
            ok = literal("false", JValue::Bool, v);
        } else if (c == 'n') {
            ok = literal("null", JValue::Null, v);
        } else {
            // any run of number characters; its text is interpreted by the reader
            while (i < s.size() && ((s[i] >= '0' && s[i] <= '9') || s[i] == '-' || s[i] == '+' || s[i] == '.' ||
                                    s[i] == 'e' || s[i] == 'E'))
                i++;
            ok = i > begin ? (v.kind = JValue::Number, true) : bad("bad number");
        }
        if (!ok) return false;
        v.raw = s.substr(begin, i - begin);
        return true;
    }
    bool object(JValue& v) {
        v.kind = JValue::Object;
        if (!eat('{')) return bad("expected '{'");
        ws();
        if (eat('}')) return true;
        for (;;) {
            ws();
            std::string key;
            if (!str(key)) return false;
            ws();
            if (!eat(':')) return bad("expected ':'");
            JValue m;
            if (!value(m)) return false;
            v.members.emplace_back(std::move(key), std::move(m));
            ws();
            if (eat(',')) continue;
            if (eat('}')) return true;
            return bad("expected ',' or '}'");
        }
    }
    bool array(JValue& v) {
        v.kind = JValue::Array;
        if (!eat('[')) return bad("expected '['");
        ws();
        if (eat(']')) return true;
        for (;;) {
            JValue m;
            if (!value(m)) return false;
            v.items.push_back(std::move(m));
            ws();
            if (eat(',')) continue;
            if (eat(']')) return true;
            return bad("expected ',' or ']'");
        }
    }
};

}  // namespace

bool json_parse(const std::string& src, JValue& out, std::string* err) {
    Reader r(src);
    out = JValue();
    r.ws();
    bool ok = r.value(out);
    if (ok) {
        r.ws();
        if (r.i != src.size()) ok = r.bad("trailing content");
    }
    if (!ok) {
        out = JValue();
        if (err) *err = r.err;
    }
    return ok;
}

static const JValue* member(const JValue& obj, const std::string& key) {
    for (const auto& m : obj.members)
        if (m.first == key) return &m.second;
    return nullptr;
}

const JValue* json_find(const JValue& root, const std::string& key) {
    if (root.kind != JValue::Object) return nullptr;
    if (const JValue* v = member(root, key)) return v;
    if (key.find('.') == std::string::npos) return nullptr;
    const JValue* cur = &root;
    size_t start = 0;
    for (;;) {
        const size_t dot = key.find('.', start);
        const std::string part = key.substr(start, dot == std::string::npos ? std::string::npos : dot - start);
        if (part.empty() || cur->kind != JValue::Object) return nullptr;
        cur = member(*cur, part);
        if (!cur) return nullptr;
        if (dot == std::string::npos) return cur;
        start = dot + 1;
    }
}

std::string json_text(const JValue& v) {
    if (v.kind == JValue::String) return v.text;
    if (!v.raw.empty()) return v.raw;
    // values built in memory never reach here: every parsed value has its source text
    return v.kind == JValue::Null ? "null" : std::string();
}

bool JsonFile::open(const std::string& path) {
    loaded_ = false;
    root_ = JValue();
    std::string text;
    if (path.empty() || !read_file(resolve_path(path), text)) return false;
    loaded_ = json_parse(text, root_);
    return loaded_;
}

std::string JsonFile::get(const std::string& key) const {
    if (!loaded_) return std::string();
    const JValue* v = json_find(root_, key);
    return v ? json_text(*v) : std::string();
}

std::string JsonFile::get_str(const std::string& key, const std::string& fallback) const {
    if (!loaded_) return fallback;
    const JValue* v = json_find(root_, key);
    return v ? json_text(*v) : fallback;
}

int JsonFile::get_int(const std::string& key, int fallback) const {
    const std::string t = get(key);
    if (t.empty()) return fallback;
    try {
        return std::stoi(t);  // leading integer of the text ("5e5" reads 5)
    } catch (...) {
        return fallback;
    }
}

int info_int(const std::string& path, const std::string& key, int fallback) {
    JsonFile j;
    if (!j.open(path)) return fallback;
    return j.get_int(key, fallback);
}

std::string info_str(const std::string& path, const std::string& key, const std::string& fallback) {
    JsonFile j;
    if (!j.open(path)) return fallback;
    const std::string v = j.get(key);
    return v.empty() ? fallback : v;
}

}  // namespace jytext
