// jy_tokenizer.cc — byte-level BPE tokenizer of jieyu's text path
// (libs/tokenizer_libs/include/tokenizer.h).  Same vocabulary rules, word
// splitting, merge order and special-token matching, so prompts encode to the
// same ids and ids decode to the same bytes.
//
//  * Bytes map to code points GPT-2 style: printable Latin-1 bytes
//    (33..126, 161..172, 174..255) are themselves, the other 68 bytes take
//    256, 257, ... in byte order (tokenizer.h:64-100).
//  * vocab.json maps pieces to ids; merges.txt lists "left right" pairs, a
//    pair's rank is its line order.  Pieces named by merges but absent from the
//    vocabulary are appended after the largest id, as are the BOS / EOS / UNK
//    pieces (tokenizer.h:342-423).
//  * Text splits into words: whitespace runs, single punctuation code points,
//    and runs of other code points; a lone ' ' joins the word or punctuation
//    mark after it (tokenizer.h:150-220).
//  * Each word's byte ids (plus "</w>" when the vocabulary has it) merge lowest
//    rank first, leftmost first (tokenizer.h:482-592).
//  * Special pieces split the text first: the earliest occurrence wins, the
//    longer piece on a tie (tokenizer.h:458-480, :594-633).
#include <algorithm>
#include <cstdlib>
#include <queue>

#include "jy_text.h"

namespace jytext {

namespace {

const char kBos[] = "<\xEF\xBD\x9C" "begin\xE2\x96\x81of\xE2\x96\x81sentence\xEF\xBD\x9C>";
const char kEos[] = "<\xEF\xBD\x9C" "end\xE2\x96\x81of\xE2\x96\x81sentence\xEF\xBD\x9C>";
const char kUnk[] = "<unk>";
const char kWordEnd[] = "</w>";

bool byte_is_printable(int b) { return (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255); }

struct ByteMap {
    std::string to_piece[256];
    int to_byte[68];
    ByteMap() {
        int slot = 0;
        for (int b = 0; b < 256; b++) {
            if (byte_is_printable(b)) {
                to_piece[b] = utf8_encode((uint32_t)b);
            } else {
                to_piece[b] = utf8_encode(256u + (uint32_t)slot);
                to_byte[slot++] = b;
            }
        }
    }
};

const ByteMap& byte_map() {
    static const ByteMap m;
    return m;
}

// code point of a piece back to its byte, -1 when it is not a byte-level code point
int cp_to_byte(uint32_t cp) {
    if (cp < 256u) return byte_is_printable((int)cp) ? (int)cp : -1;
    return cp - 256u < 68u ? byte_map().to_byte[cp - 256u] : -1;
}

bool is_space(uint32_t c) { return c == 0x20 || (c >= 0x09 && c <= 0x0D) || c == 0x3000; }

bool is_punct(uint32_t c) {
    return (c >= 0x21 && c <= 0x2F) || (c >= 0x3A && c <= 0x40) || (c >= 0x5B && c <= 0x60) ||
           (c >= 0x7B && c <= 0x7E) || (c >= 0x2010 && c <= 0x2027) || (c >= 0x2030 && c <= 0x205E) ||
           (c >= 0x3001 && c <= 0x303F) || (c >= 0xFF01 && c <= 0xFF0F) || (c >= 0xFF1A && c <= 0xFF20) ||
           (c >= 0xFF3B && c <= 0xFF40) || (c >= 0xFF5B && c <= 0xFF65);
}

uint32_t cp_at(const std::string& s, size_t i, size_t& len) {
    uint32_t c;
    utf8_decode(s.data() + i, s.size() - i, c, len);
    return c;
}

// end of the run starting at i whose code points satisfy keep()
template <class P>
size_t run_end(const std::string& s, size_t i, P keep) {
    while (i < s.size()) {
        size_t n;
        if (!keep(cp_at(s, i, n))) break;
        i += n;
    }
    return i;
}

// [begin, end) byte ranges of the words of s
std::vector<std::pair<size_t, size_t>> words(const std::string& s) {
    std::vector<std::pair<size_t, size_t>> out;
    auto plain = [](uint32_t c) { return !is_space(c) && !is_punct(c); };
    size_t i = 0;
    while (i < s.size()) {
        size_t n;
        const uint32_t c = cp_at(s, i, n);
        size_t end;
        if (is_space(c)) {
            end = run_end(s, i, is_space);
            if (end - i == 1 && s[i] == ' ' && end < s.size()) {
                // one plain space: it leads the next punctuation mark or word
                size_t m;
                const uint32_t next = cp_at(s, end, m);
                end = is_punct(next) ? end + m : run_end(s, end, plain);
            }
        } else if (is_punct(c)) {
            end = i + n;
        } else {
            end = run_end(s, i, plain);
        }
        out.emplace_back(i, end);
        i = end;
    }
    return out;
}

uint64_t pair_key(int32_t a, int32_t b) { return ((uint64_t)(uint32_t)a << 32) | (uint32_t)b; }

}  // namespace

int32_t Tokenizer::id_of(const std::string& p) const {
    auto it = piece_to_id_.find(p);
    return it == piece_to_id_.end() ? -1 : it->second;
}

int32_t Tokenizer::intern(const std::string& p) {
    const int32_t have = id_of(p);
    if (have >= 0) return have;
    const int32_t id = (int32_t)id_to_piece_.size();
    id_to_piece_.push_back(p);
    piece_to_id_.emplace(p, id);
    return id;
}

int32_t Tokenizer::add_special(const std::string& p) {
    if (p.empty()) return -1;
    const int32_t id = id_of(p);
    if (id < 0) return -1;
    if (std::find(special_.begin(), special_.end(), p) == special_.end()) {
        special_.push_back(p);
        special_ids_.push_back(id);
    }
    return id;
}

std::string Tokenizer::piece(int32_t id) const {
    return id >= 0 && (size_t)id < id_to_piece_.size() ? id_to_piece_[id] : std::string();
}

bool Tokenizer::load(const std::string& vocab_path, const std::string& merges_path, std::string* err) {
    *this = Tokenizer();
    auto fail = [&](const std::string& m) {
        if (err) *err = m;
        return false;
    };
    std::string merges_text;
    if (!read_file(resolve_path(merges_path), merges_text)) return fail("cannot read " + merges_path);
    std::string vocab_text;
    JValue vocab;
    std::string perr;
    if (!read_file(resolve_path(vocab_path), vocab_text)) return fail("cannot read " + vocab_path);
    if (!json_parse(vocab_text, vocab, &perr)) return fail("vocab.json: " + perr);
    if (vocab.kind != JValue::Object) return fail("vocab.json is not an object");
    size_t entries = 0;
    for (const auto& m : vocab.members) {
        // the id is the leading integer of the value's text; others are skipped
        const std::string t = json_text(m.second);
        char* end = nullptr;
        const long id = std::strtol(t.c_str(), &end, 10);
        if (end == t.c_str() || id < 0) continue;
        if ((size_t)id >= id_to_piece_.size()) id_to_piece_.resize((size_t)id + 1);
        id_to_piece_[(size_t)id] = m.first;
        piece_to_id_.emplace(m.first, (int32_t)id);  // the first id of a repeated piece stays
        entries++;
    }
    if (entries == 0) return fail("vocab.json is empty");

    bos_ = intern(kBos);
    eos_ = intern(kEos);
    unk_ = intern(kUnk);
    word_end_ = id_of(kWordEnd);
    for (int b = 0; b < 256; b++) {
        const int32_t id = id_of(byte_map().to_piece[b]);
        byte_id_[b] = id >= 0 ? id : unk_;
    }

    for (std::string line : split_lines(merges_text)) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line.empty() || line[0] == '#') continue;
        const size_t sp = line.find(' ');
        if (sp == std::string::npos) continue;
        const std::string left = line.substr(0, sp), right = line.substr(sp + 1);
        if (right.empty()) continue;
        const int32_t l = intern(left), r = intern(right);
        const uint64_t k = pair_key(l, r);
        if (rank_.count(k)) continue;
        const int32_t m = intern(left + right);
        rank_.emplace(k, (int32_t)merged_.size());
        merged_.push_back(m);
    }

    special_ = {kBos, kEos, kUnk};
    std::sort(special_.begin(), special_.end(), [](const std::string& a, const std::string& b) {
        return a.size() != b.size() ? a.size() > b.size() : a < b;
    });
    for (const std::string& p : special_) special_ids_.push_back(intern(p));
    return true;
}

int Tokenizer::find_special(const std::string& text, size_t from, size_t& at, size_t& len) const {
    int best = -1;
    for (size_t i = 0; i < special_.size(); i++) {
        const size_t p = text.find(special_[i], from);
        if (p == std::string::npos) continue;
        if (best < 0 || p < at || (p == at && special_[i].size() > len)) {
            best = (int)i;
            at = p;
            len = special_[i].size();
        }
    }
    return best;
}

// Merge adjacent symbols, lowest rank first and leftmost among equal ranks.  A
// doubly linked list over the symbols plus a min-heap of (rank, position)
// candidates; a candidate is stale once either symbol of its pair changed.
std::vector<int32_t> Tokenizer::merge(std::vector<int32_t> sym) const {
    const int n = (int)sym.size();
    if (n < 2 || rank_.empty()) return sym;
    std::vector<int> prev(n), next(n);
    std::vector<uint32_t> gen(n, 0);
    std::vector<char> live(n, 1);
    for (int i = 0; i < n; i++) {
        prev[i] = i - 1;
        next[i] = i + 1 < n ? i + 1 : -1;
    }
    struct Cand {
        int32_t rank;
        int pos;
        uint32_t gen;
    };
    auto later = [](const Cand& a, const Cand& b) { return a.rank != b.rank ? a.rank > b.rank : a.pos > b.pos; };
    std::priority_queue<Cand, std::vector<Cand>, decltype(later)> heap(later);
    auto rank_at = [&](int p) -> int32_t {
        if (p < 0 || next[p] < 0) return -1;
        auto it = rank_.find(pair_key(sym[p], sym[next[p]]));
        return it == rank_.end() ? -1 : it->second;
    };
    auto offer = [&](int p) {
        const int32_t r = rank_at(p);
        if (r >= 0) heap.push({r, p, gen[p]});
    };
    for (int i = 0; i + 1 < n; i++) offer(i);
    while (!heap.empty()) {
        const Cand c = heap.top();
        heap.pop();
        const int p = c.pos;
        if (!live[p] || gen[p] != c.gen || rank_at(p) != c.rank) continue;
        const int q = next[p];
        sym[p] = merged_[(size_t)c.rank];
        live[q] = 0;
        next[p] = next[q];
        if (next[q] >= 0) prev[next[q]] = p;
        gen[p]++;
        if (prev[p] >= 0) gen[prev[p]]++;
        if (prev[p] >= 0) offer(prev[p]);
        offer(p);
    }
    std::vector<int32_t> out;
    for (int i = 0; i >= 0; i = next[i])
        if (live[i]) out.push_back(sym[i]);
    return out;
}

std::vector<int32_t> Tokenizer::encode(const std::string& text) const {
    std::vector<int32_t> ids;
    size_t cur = 0;
    while (cur < text.size()) {
        size_t at = 0, len = 0;
        const int sp = find_special(text, cur, at, len);
        const size_t stop = sp >= 0 ? at : text.size();
        if (stop > cur) {
            const std::string seg = text.substr(cur, stop - cur);
            for (const auto& w : words(seg)) {
                if (w.second <= w.first) continue;
                std::vector<int32_t> sym;
                sym.reserve(w.second - w.first + 1);
                for (size_t i = w.first; i < w.second; i++) sym.push_back(byte_id_[(unsigned char)seg[i]]);
                if (word_end_ >= 0) sym.push_back(word_end_);
                const std::vector<int32_t> m = merge(std::move(sym));
                ids.insert(ids.end(), m.begin(), m.end());
            }
        }
        if (sp < 0) break;
        ids.push_back(special_ids_[(size_t)sp]);
        cur = at + len;
    }
    return ids;
}

std::string Tokenizer::decode(const int32_t* ids, size_t n) const {
    std::string out;
    for (size_t k = 0; k < n; k++) {
        const int32_t id = ids[k];
        if (id < 0 || (size_t)id >= id_to_piece_.size()) continue;
        const std::string& p = id_to_piece_[(size_t)id];
        if (id == bos_ || id == eos_ || id == unk_) {
            out += p;  // these three print as written
            continue;
        }
        size_t end = p.size();
        if (end >= 4 && p.compare(end - 4, 4, kWordEnd) == 0) end -= 4;
        for (size_t i = 0; i < end;) {
            uint32_t cp;
            size_t len;
            utf8_decode(p.data() + i, end - i, cp, len);
            const int b = cp_to_byte(cp);
            if (b >= 0) out += (char)b;
            i += len;
        }
    }
    return out;
}

}  // namespace jytext
