// Byte-level BPE tokenizer over a GGUF's vocabulary: the Tokenizer of the reference
// (tokenizer.hpp:8-33, tokenizer.cpp:43-239) with the same API and the same ids, so that
// `--prompt` gives the GPU backend the prompt the reference would run.
#pragma once
#include <array>
#include <string>
#include <unordered_map>
#include <vector>

#include "gguf.hpp"

namespace tfh {

class Tokenizer {
public:
    explicit Tokenizer(const GgufFile& g);

    std::vector<int> encode(const std::string& text, bool add_bos) const;
    std::string decode(const std::vector<int>& ids) const;
    std::string decode_one(int id) const;

    int bos() const { return bos_; }
    int eos() const { return eos_; }
    int n_vocab() const { return (int)vocab_.size(); }

private:
    std::vector<std::string> vocab_;
    std::unordered_map<std::string, int> id_of_;
    std::unordered_map<std::string, int> merge_rank_;  // "left right" -> rank
    std::vector<std::string> specials_;                // "<...>" tokens, longest first
    std::array<std::string, 256> byte_char_;           // byte -> its printable stand-in (UTF-8)
    std::vector<int> char_byte_;                       // stand-in code point -> byte, -1 if none
    int bos_ = 1, eos_ = 2;
    bool add_bos_ = true;

    size_t special_at(const std::string& text, size_t pos) const;
    std::vector<int> bpe(const std::string& piece) const;
};

}  // namespace tfh
