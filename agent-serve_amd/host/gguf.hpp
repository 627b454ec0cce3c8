// GGUF v2/v3 reader (mmap) and tensor-type tables for the tinferno token loop.
//
// Follows the container layout the reference parses in gguf.cpp:88-168 (header,
// key/value section, tensor-info section, aligned data section) and the dtype
// tables of tensor.cpp:18-77. Weights stay in the mapping; the HIP backend copies
// them to HBM at model load.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

namespace tfh {

// ggml type ids used by the token loop (tensor.cpp:18-28).
enum GgmlType : int { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q8_0 = 8, GGML_Q6_K = 14 };

const char* ggml_type_name(int t);
bool ggml_type_known(int t);
int ggml_blck_size(int t);        // elements per block (tensor.cpp:42-53)
size_t ggml_blck_nbytes(int t);   // bytes per block (tensor.cpp:55-64)
size_t ggml_row_nbytes(int t, int64_t ne0);  // throws if ne0 is not a block multiple (tensor.cpp:66-70)

struct TensorInfo {
    std::string name;
    int type = GGML_F32;
    int ndim = 0;
    int64_t ne[4] = {1, 1, 1, 1};  // ggml order: ne[0] is the row length (K for weights)
    uint64_t offset = 0;           // relative to the data section
    const uint8_t* data = nullptr; // into the mapping
    size_t nbytes = 0;
    int64_t cols() const { return ne[0]; }
    int64_t rows() const {
        int64_t r = 1;
        for (int i = 1; i < ndim; ++i) r *= ne[i];
        return r;
    }
};

class GgufFile {
public:
    explicit GgufFile(const std::string& path);
    ~GgufFile();
    GgufFile(const GgufFile&) = delete;
    GgufFile& operator=(const GgufFile&) = delete;

    const TensorInfo* find(const std::string& name) const;
    const TensorInfo& must(const std::string& name) const;  // throws "missing tensor <name>"

    uint64_t u64(const std::string& key, uint64_t def = 0) const;
    float f32(const std::string& key, float def = 0) const;
    std::string str(const std::string& key, const std::string& def = "") const;
    bool boolean(const std::string& key, bool def = false) const;
    size_t arr_len(const std::string& key) const;  // length of an array value, 0 if absent
    const std::vector<std::string>& arr_str(const std::string& key) const;

    const std::string& arch() const { return arch_; }
    const std::vector<TensorInfo>& tensors() const { return tensors_; }
    size_t file_size() const { return size_; }
    size_t weight_bytes() const;  // sum of tensor nbytes (gguf.cpp:219-223)

private:
    void* map_ = nullptr;
    size_t size_ = 0;
    int fd_ = -1;
    std::string arch_;
    std::vector<TensorInfo> tensors_;
    std::unordered_map<std::string, size_t> by_name_;
    std::unordered_map<std::string, uint64_t> u64_;
    std::unordered_map<std::string, float> f32_;
    std::unordered_map<std::string, std::string> str_;
    std::unordered_map<std::string, bool> bool_;
    std::unordered_map<std::string, size_t> arr_len_;
    std::unordered_map<std::string, std::vector<std::string>> arr_str_;
};

}  // namespace tfh
