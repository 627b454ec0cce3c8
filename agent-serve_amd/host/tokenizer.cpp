// Byte-level BPE (the reference's tokenizer.cpp:43-239), restated:
//   * every byte stands for a printable code point (GPT-2's table: bytes 33-126, 161-172
//     and 174-255 stand for themselves, the other 68 for 256, 257, ... in byte order);
//   * the text is cut at special tokens ("<...>" vocabulary entries, longest first);
//   * other chunks are cut into pieces (the reference's approximate pre-tokenizer, quirks
//     included: a whitespace run keeps only its last character, glued to the word after
//     it), and each piece is merged pairwise by merge rank, lowest rank first;
//   * a merged symbol missing from the vocabulary falls back to the stand-ins of its bytes.
#include "tokenizer.hpp"

#include <algorithm>
#include <climits>

namespace tfh {
namespace {

// The "C" locale's character classes, which the reference's <cctype> calls use.
bool is_space(unsigned char c) { return c == ' ' || (c >= '\t' && c <= '\r'); }
bool is_alpha(unsigned char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z'); }
bool is_digit(unsigned char c) { return c >= '0' && c <= '9'; }
bool is_word(unsigned char c) { return is_alpha(c) || is_digit(c) || c == '\''; }

std::string utf8(int cp) {
    std::string s;
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
    return s;
}

bool printable_byte(int b) { return (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255); }

// The reference's pre-tokenizer (tokenizer.cpp:94-130).
std::vector<std::string> pieces(const std::string& s) {
    std::vector<std::string> out;
    const size_t n = s.size();
    size_t i = 0;
    while (i < n) {
        const unsigned char c = (unsigned char)s[i];
        size_t j = i + 1;
        if (is_space(c)) {
            while (j < n && is_space((unsigned char)s[j])) ++j;
            if (j < n) {
                // the run's last whitespace character goes with the word after it; the
                // characters before it are dropped
                size_t k = j;
                while (k < n && is_word((unsigned char)s[k])) ++k;
                out.push_back(s.substr(j - 1, k - j + 1));
                i = k;
            } else {
                out.push_back(s.substr(i));
                i = n;
            }
            continue;
        }
        if (is_alpha(c) || c == '\'') {
            while (j < n && is_word((unsigned char)s[j])) ++j;
        } else if (is_digit(c)) {
            while (j < n && is_digit((unsigned char)s[j])) ++j;
        }
        out.push_back(s.substr(i, j - i));
        i = j;
    }
    return out;
}

}  // namespace

Tokenizer::Tokenizer(const GgufFile& g) : char_byte_(1 << 16, -1) {
    int extra = 0;
    for (int b = 0; b < 256; ++b) {
        const int cp = printable_byte(b) ? b : 256 + extra++;
        byte_char_[(size_t)b] = utf8(cp);
        char_byte_[(size_t)cp] = b;
    }
    vocab_ = g.arr_str("tokenizer.ggml.tokens");
    id_of_.reserve(vocab_.size());
    for (size_t i = 0; i < vocab_.size(); ++i) id_of_[vocab_[i]] = (int)i;  // a repeated string keeps its last id
    const auto& merges = g.arr_str("tokenizer.ggml.merges");
    merge_rank_.reserve(merges.size());
    for (size_t i = 0; i < merges.size(); ++i) merge_rank_[merges[i]] = (int)i;
    bos_ = (int)g.u64("tokenizer.ggml.bos_token_id", 1);
    eos_ = (int)g.u64("tokenizer.ggml.eos_token_id", 2);
    add_bos_ = g.boolean("tokenizer.ggml.add_bos_token", true);
    for (const auto& t : vocab_)
        if (t.size() >= 3 && t.front() == '<' && t.back() == '>') specials_.push_back(t);
    std::stable_sort(specials_.begin(), specials_.end(),
                     [](const std::string& a, const std::string& b) { return a.size() > b.size(); });
}

// Length of the first (longest) special token starting at pos, 0 if none.
size_t Tokenizer::special_at(const std::string& text, size_t pos) const {
    for (const auto& sp : specials_)
        if (pos + sp.size() <= text.size() && text.compare(pos, sp.size(), sp) == 0) return sp.size();
    return 0;
}

std::vector<int> Tokenizer::bpe(const std::string& piece) const {
    const auto whole = id_of_.find(piece);
    if (whole != id_of_.end()) return {whole->second};
    // one symbol per byte, as its stand-in character
    std::vector<std::string> sym;
    sym.reserve(piece.size());
    for (unsigned char b : piece) sym.push_back(byte_char_[b]);
    while (sym.size() > 1) {
        int best = INT_MAX;
        size_t at = 0;
        for (size_t i = 0; i + 1 < sym.size(); ++i) {
            const auto r = merge_rank_.find(sym[i] + " " + sym[i + 1]);
            if (r != merge_rank_.end() && r->second < best) {
                best = r->second;
                at = i;
            }
        }
        if (best == INT_MAX) break;
        sym[at] += sym[at + 1];
        sym.erase(sym.begin() + (std::ptrdiff_t)at + 1);
    }
    std::vector<int> ids;
    for (const auto& s : sym) {
        const auto it = id_of_.find(s);
        if (it != id_of_.end()) {
            ids.push_back(it->second);
            continue;
        }
        // not in the vocabulary: the stand-in of each byte of the symbol's own text
        for (unsigned char b : s) {
            const auto f = id_of_.find(byte_char_[b]);
            if (f != id_of_.end()) ids.push_back(f->second);
        }
    }
    return ids;
}

std::vector<int> Tokenizer::encode(const std::string& text, bool add_bos) const {
    std::vector<int> ids;
    if (add_bos && add_bos_) ids.push_back(bos_);
    if (vocab_.empty()) return ids;
    size_t i = 0;
    while (i < text.size()) {
        size_t len = special_at(text, i);
        if (len == 0) {
            // plain text up to the next special token
            size_t j = i + 1;
            while (j < text.size() && special_at(text, j) == 0) ++j;
            len = j - i;
        }
        const std::string chunk = text.substr(i, len);
        i += len;
        const auto it = id_of_.find(chunk);
        if (it != id_of_.end()) {
            ids.push_back(it->second);
            continue;
        }
        for (const auto& p : pieces(chunk)) {
            const auto more = bpe(p);
            ids.insert(ids.end(), more.begin(), more.end());
        }
    }
    return ids;
}

std::string Tokenizer::decode_one(int id) const {
    if (id < 0 || id >= (int)vocab_.size()) return "";
    const std::string& t = vocab_[(size_t)id];
    std::string out;
    size_t i = 0;
    while (i < t.size()) {
        const unsigned char c = (unsigned char)t[i];
        int cp, len;
        if (c < 0x80) {
            cp = c;
            len = 1;
        } else if ((c & 0xE0) == 0xC0 && i + 1 < t.size()) {
            cp = ((c & 0x1F) << 6) | ((unsigned char)t[i + 1] & 0x3F);
            len = 2;
        } else if ((c & 0xF0) == 0xE0 && i + 2 < t.size()) {
            cp = ((c & 0x0F) << 12) | (((unsigned char)t[i + 1] & 0x3F) << 6) | ((unsigned char)t[i + 2] & 0x3F);
            len = 3;
        } else {
            out += (char)c;  // not a character the table knows: the byte itself
            ++i;
            continue;
        }
        const int b = char_byte_[(size_t)cp];
        if (b >= 0)
            out += (char)b;
        else
            out.append(t, i, (size_t)len);
        i += (size_t)len;
    }
    return out;
}

std::string Tokenizer::decode(const std::vector<int>& ids) const {
    std::string s;
    for (int id : ids) s += decode_one(id);
    return s;
}

}  // namespace tfh
