#include "gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>

namespace tfh {

const char* ggml_type_name(int t) {
    switch (t) {
        case GGML_F32: return "F32";
        case GGML_F16: return "F16";
        case GGML_Q4_0: return "Q4_0";
        case GGML_Q4_1: return "Q4_1";
        case GGML_Q8_0: return "Q8_0";
        case GGML_Q6_K: return "Q6_K";
    }
    return "?";
}

bool ggml_type_known(int t) {
    return t == GGML_F32 || t == GGML_F16 || t == GGML_Q4_0 || t == GGML_Q4_1 || t == GGML_Q8_0 ||
           t == GGML_Q6_K;
}

int ggml_blck_size(int t) {
    switch (t) {
        case GGML_Q4_0:
        case GGML_Q4_1:
        case GGML_Q8_0: return 32;
        case GGML_Q6_K: return 256;
        default: return 1;
    }
}

size_t ggml_blck_nbytes(int t) {
    switch (t) {
        case GGML_F32: return 4;
        case GGML_F16: return 2;
        case GGML_Q4_0: return 18;
        case GGML_Q4_1: return 20;
        case GGML_Q8_0: return 34;
        case GGML_Q6_K: return 210;
    }
    return 0;
}

size_t ggml_row_nbytes(int t, int64_t ne0) {
    const int bs = ggml_blck_size(t);
    if (ne0 % bs != 0) throw std::runtime_error("row length not divisible by block size");
    return (size_t)(ne0 / bs) * ggml_blck_nbytes(t);
}

namespace {

// Bounds-checked little-endian reader over the mapping.
struct Reader {
    const uint8_t* p;
    const uint8_t* end;
    void need(size_t n) const {
        if ((size_t)(end - p) < n) throw std::runtime_error("GGUF truncated");
    }
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p, sizeof(T));
        p += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > (uint64_t)(end - p)) throw std::runtime_error("GGUF string overflow");
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
};

// Scalar sizes of GGUF value types 0..12 (8 = string, 9 = array are variable).
size_t scalar_size(uint32_t type) {
    switch (type) {
        case 0: case 1: case 7: return 1;
        case 2: case 3: return 2;
        case 4: case 5: case 6: return 4;
        case 10: case 11: case 12: return 8;
    }
    return 0;
}

void skip(Reader& r, uint32_t type);

void skip_array(Reader& r) {
    const uint32_t et = r.get<uint32_t>();
    const uint64_t n = r.get<uint64_t>();
    const size_t sz = scalar_size(et);
    if (sz) {
        if (n > (uint64_t)(r.end - r.p) / sz) throw std::runtime_error("GGUF truncated");
        r.p += n * sz;
        return;
    }
    for (uint64_t i = 0; i < n; ++i) skip(r, et);
}

void skip(Reader& r, uint32_t type) {
    if (type == 8) {
        r.str();
    } else if (type == 9) {
        skip_array(r);
    } else {
        const size_t sz = scalar_size(type);
        if (!sz) throw std::runtime_error("unknown GGUF type");
        r.need(sz);
        r.p += sz;
    }
}

uint64_t read_int(Reader& r, uint32_t type) {
    switch (type) {
        case 0: return r.get<uint8_t>();
        case 1: return (uint64_t)(int64_t)r.get<int8_t>();
        case 2: return r.get<uint16_t>();
        case 3: return (uint64_t)(int64_t)r.get<int16_t>();
        case 4: return r.get<uint32_t>();
        case 5: return (uint64_t)(int64_t)r.get<int32_t>();
        case 10: return r.get<uint64_t>();
        case 11: return (uint64_t)r.get<int64_t>();
    }
    throw std::runtime_error("not an integer GGUF value");
}

}  // namespace

GgufFile::GgufFile(const std::string& path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("cannot open " + path);
    struct stat st {};
    if (fstat(fd_, &st) != 0) {
        ::close(fd_);
        throw std::runtime_error("fstat failed: " + path);
    }
    size_ = (size_t)st.st_size;
    if (size_ == 0) {
        ::close(fd_);
        throw std::runtime_error("GGUF truncated");
    }
    map_ = mmap(nullptr, size_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (map_ == MAP_FAILED) {
        map_ = nullptr;
        ::close(fd_);
        throw std::runtime_error("mmap failed: " + path);
    }
    try {
        const uint8_t* base = (const uint8_t*)map_;
        Reader r{base, base + size_};
        if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("not a GGUF file: " + path);
        const uint32_t version = r.get<uint32_t>();
        if (version != 2 && version != 3) throw std::runtime_error("unsupported GGUF version");
        const uint64_t n_tensors = r.get<uint64_t>();
        const uint64_t n_kv = r.get<uint64_t>();
        for (uint64_t i = 0; i < n_kv; ++i) {
            std::string key = r.str();
            const uint32_t type = r.get<uint32_t>();
            switch (type) {
                case 0: case 1: case 2: case 3: case 4: case 5: case 10: case 11:
                    u64_[key] = read_int(r, type);
                    break;
                case 6: f32_[key] = r.get<float>(); break;
                case 12: f32_[key] = (float)r.get<double>(); break;
                case 7: bool_[key] = r.get<uint8_t>() != 0; break;
                case 8: str_[key] = r.str(); break;
                case 9: {
                    const uint8_t* save = r.p;
                    const uint32_t et = r.get<uint32_t>();
                    const uint64_t n = r.get<uint64_t>();
                    arr_len_[key] = (size_t)n;
                    if (et == 8) {
                        if (n > (uint64_t)(r.end - r.p) / 8) throw std::runtime_error("GGUF truncated");
                        auto& a = arr_str_[key];
                        a.resize((size_t)n);
                        for (uint64_t j = 0; j < n; ++j) a[j] = r.str();
                    } else {
                        r.p = save;
                        skip_array(r);
                    }
                    break;
                }
                default: skip(r, type); break;
            }
        }
        arch_ = str("general.architecture", "llama");
        uint64_t align = u64("general.alignment", 32);
        if (align == 0) align = 32;

        tensors_.resize((size_t)n_tensors);
        for (uint64_t i = 0; i < n_tensors; ++i) {
            TensorInfo& t = tensors_[i];
            t.name = r.str();
            t.ndim = (int)r.get<uint32_t>();
            if (t.ndim < 1 || t.ndim > 4) throw std::runtime_error("bad ndim for " + t.name);
            for (int d = 0; d < t.ndim; ++d) t.ne[d] = (int64_t)r.get<uint64_t>();
            t.type = (int)r.get<uint32_t>();
            if (!ggml_type_known(t.type))
                throw std::runtime_error("unsupported ggml type " + std::to_string(t.type));
            t.offset = r.get<uint64_t>();
            t.nbytes = (size_t)t.rows() * ggml_row_nbytes(t.type, t.ne[0]);
            by_name_[t.name] = (size_t)i;
        }
        const size_t hdr = (size_t)(r.p - base);
        const size_t data_off = (hdr + align - 1) / align * align;
        for (auto& t : tensors_) {
            const size_t abs = data_off + (size_t)t.offset;
            if (abs > size_ || t.nbytes > size_ - abs)
                throw std::runtime_error("tensor out of range: " + t.name);
            t.data = base + abs;
        }
    } catch (...) {
        munmap(map_, size_);
        ::close(fd_);
        map_ = nullptr;
        fd_ = -1;
        throw;
    }
}

GgufFile::~GgufFile() {
    if (map_) munmap(map_, size_);
    if (fd_ >= 0) ::close(fd_);
}

const TensorInfo* GgufFile::find(const std::string& name) const {
    auto it = by_name_.find(name);
    return it == by_name_.end() ? nullptr : &tensors_[it->second];
}

const TensorInfo& GgufFile::must(const std::string& name) const {
    const TensorInfo* t = find(name);
    if (!t) throw std::runtime_error("missing tensor " + name);
    return *t;
}

uint64_t GgufFile::u64(const std::string& key, uint64_t def) const {
    auto it = u64_.find(key);
    return it == u64_.end() ? def : it->second;
}

float GgufFile::f32(const std::string& key, float def) const {
    auto it = f32_.find(key);
    return it == f32_.end() ? def : it->second;
}

std::string GgufFile::str(const std::string& key, const std::string& def) const {
    auto it = str_.find(key);
    return it == str_.end() ? def : it->second;
}

bool GgufFile::boolean(const std::string& key, bool def) const {
    auto it = bool_.find(key);
    return it == bool_.end() ? def : it->second;
}

size_t GgufFile::arr_len(const std::string& key) const {
    auto it = arr_len_.find(key);
    return it == arr_len_.end() ? 0 : it->second;
}

const std::vector<std::string>& GgufFile::arr_str(const std::string& key) const {
    static const std::vector<std::string> empty;
    auto it = arr_str_.find(key);
    return it == arr_str_.end() ? empty : it->second;
}

size_t GgufFile::weight_bytes() const {
    size_t n = 0;
    for (const auto& t : tensors_) n += t.nbytes;
    return n;
}

}  // namespace tfh
