// GGUF v3 reader (see gguf.h). Layout of a GGUF file:
//   u32 magic "GGUF", u32 version, u64 n_tensors, u64 n_kv,
//   n_kv x (string key, u32 value type, value),
//   n_tensors x (string name, u32 n_dims, u64 dims[n_dims], u32 ggml type, u64 offset),
//   padding to general.alignment, then the data section (offsets are relative to it).
// Strings are u64 length + bytes; arrays are u32 element type + u64 count + elements.
#include "gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <stdexcept>

namespace flint {
namespace gguf {
namespace {

// metadata value types of the format
enum : uint32_t {
    T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STRING, T_ARRAY, T_U64, T_I64, T_F64,
};

struct TypeRow {
    uint32_t id;
    const char *name;
    BlockGeom geom;
};
// ggml's block sizes (ggml-common.h) for the types the reference's loader accepts
constexpr TypeRow kTypes[] = {
    {0, "F32", {1, 4}},          {1, "F16", {1, 2}},        {2, "Q4_0", {32, 18}},      {8, "Q8_0", {32, 34}},
    {10, "Q2_K", {256, 84}},     {11, "Q3_K", {256, 110}},  {12, "Q4_K", {256, 144}},   {13, "Q5_K", {256, 176}},
    {14, "Q6_K", {256, 210}},    {16, "IQ2_XXS", {256, 66}}, {17, "IQ2_XS", {256, 74}}, {18, "IQ3_XXS", {256, 98}},
    {19, "IQ1_S", {256, 50}},    {20, "IQ4_NL", {32, 18}},  {21, "IQ3_S", {256, 110}},  {22, "IQ2_S", {256, 82}},
    {23, "IQ4_XS", {256, 136}},  {29, "IQ1_M", {256, 56}},  {30, "BF16", {1, 2}},
};

class Reader {
public:
    Reader(const uint8_t *p, size_t n) : p_(p), end_(p + n), begin_(p) {}
    template <typename T>
    T get() {
        need(sizeof(T));
        T v;
        std::memcpy(&v, p_, sizeof(T));
        p_ += sizeof(T);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        need(n);
        std::string s((const char *)p_, (size_t)n);
        p_ += n;
        return s;
    }
    uint64_t offset() const { return (uint64_t)(p_ - begin_); }

private:
    void need(uint64_t n) const {
        if ((uint64_t)(end_ - p_) < n) throw std::runtime_error("gguf: unexpected end of file");
    }
    const uint8_t *p_, *end_, *begin_;
};

bool integral(uint32_t t) {
    return t == T_U8 || t == T_I8 || t == T_U16 || t == T_I16 || t == T_U32 || t == T_I32 || t == T_U64 ||
           t == T_I64;
}

int64_t get_integral(Reader &r, uint32_t t) {
    switch (t) {
        case T_U8: return r.get<uint8_t>();
        case T_I8: return r.get<int8_t>();
        case T_U16: return r.get<uint16_t>();
        case T_I16: return r.get<int16_t>();
        case T_U32: return r.get<uint32_t>();
        case T_I32: return r.get<int32_t>();
        case T_U64: return (int64_t)r.get<uint64_t>();
        default: return r.get<int64_t>();
    }
}

Value get_value(Reader &r, uint32_t t) {
    Value v;
    if (integral(t)) {
        v.kind = Value::INT;
        v.i = get_integral(r, t);
        return v;
    }
    switch (t) {
        case T_F32: v.kind = Value::FLOAT; v.f = r.get<float>(); return v;
        case T_F64: v.kind = Value::FLOAT; v.f = r.get<double>(); return v;
        case T_BOOL: v.kind = Value::BOOL; v.b = r.get<uint8_t>() != 0; return v;
        case T_STRING: v.kind = Value::STRING; v.s = r.str(); return v;
        case T_ARRAY: {
            const uint32_t et = r.get<uint32_t>();
            const uint64_t n = r.get<uint64_t>();
            if (integral(et)) {
                v.kind = Value::INT_ARRAY;
                for (uint64_t k = 0; k < n; k++) v.ia.push_back(get_integral(r, et));
            } else if (et == T_F32 || et == T_F64) {
                v.kind = Value::FLOAT_ARRAY;
                for (uint64_t k = 0; k < n; k++) v.fa.push_back(et == T_F32 ? r.get<float>() : r.get<double>());
            } else if (et == T_BOOL) {
                v.kind = Value::BOOL_ARRAY;
                for (uint64_t k = 0; k < n; k++) v.ba.push_back(r.get<uint8_t>() != 0);
            } else if (et == T_STRING) {
                v.kind = Value::STRING_ARRAY;
                for (uint64_t k = 0; k < n; k++) v.sa.push_back(r.str());
            } else {
                throw std::runtime_error("gguf: unsupported array element type");
            }
            return v;
        }
    }
    throw std::runtime_error("gguf: unknown metadata type " + std::to_string(t));
}

}  // namespace

bool block_geom(uint32_t type, BlockGeom *g) {
    for (const TypeRow &t : kTypes)
        if (t.id == type) {
            *g = t.geom;
            return true;
        }
    return false;
}

const char *type_name(uint32_t type) {
    for (const TypeRow &t : kTypes)
        if (t.id == type) return t.name;
    return "?";
}

uint64_t Tensor::n_rows() const {
    uint64_t n = 1;
    for (size_t d = 1; d < dims.size(); d++) n *= dims[d];
    return n;
}

uint64_t Tensor::row_bytes() const {
    BlockGeom g{};
    block_geom(type, &g);
    return dims.empty() ? 0 : dims[0] / g.elems * g.bytes;
}

File::File(const std::string &path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) throw std::runtime_error("cannot open " + path);
    struct stat st {};
    if (fstat(fd_, &st) != 0) {
        ::close(fd_);
        throw std::runtime_error("cannot open " + path);
    }
    size_ = (size_t)st.st_size;
    void *m = size_ ? mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd_, 0) : MAP_FAILED;
    if (m == MAP_FAILED) {
        ::close(fd_);
        if (size_ == 0) throw std::runtime_error("gguf: unexpected end of file");
        throw std::runtime_error("mmap failed: " + path);
    }
    base_ = (const uint8_t *)m;
    try {
        Reader r(base_, size_);
        if (r.get<uint32_t>() != 0x46554747u) throw std::runtime_error("not a GGUF file: " + path);
        if (r.get<uint32_t>() < 3) throw std::runtime_error("unsupported GGUF version");
        const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
        for (uint64_t k = 0; k < n_kv; k++) {
            std::string key = r.str();
            const uint32_t t = r.get<uint32_t>();
            meta_[key] = get_value(r, t);
        }
        struct Info {
            std::string name;
            std::vector<uint64_t> dims;
            uint32_t type;
            uint64_t rel;
        };
        std::vector<Info> infos;
        for (uint64_t k = 0; k < n_tensors; k++) {
            Info in;
            in.name = r.str();
            const uint32_t nd = r.get<uint32_t>();
            for (uint32_t d = 0; d < nd; d++) in.dims.push_back(r.get<uint64_t>());
            in.type = r.get<uint32_t>();
            in.rel = r.get<uint64_t>();
            infos.push_back(std::move(in));
        }
        const uint64_t align = has("general.alignment") ? (uint64_t)get_int("general.alignment") : 32;
        if (align == 0) throw std::runtime_error("gguf: general.alignment is 0");
        const uint64_t data0 = (r.offset() + align - 1) / align * align;
        for (Info &in : infos) {
            BlockGeom g{};
            if (!block_geom(in.type, &g)) throw std::runtime_error("unsupported ggml type " + std::to_string(in.type));
            Tensor t;
            t.name = std::move(in.name);
            t.type = in.type;
            t.dims = std::move(in.dims);
            uint64_t n = 1;
            for (uint64_t d : t.dims) {
                if (d != 0 && n > UINT64_MAX / d) throw std::runtime_error("tensor out of bounds: " + t.name);
                n *= d;
            }
            t.offset = data0 + in.rel;
            t.nbytes = n / g.elems * g.bytes;
            if (t.offset < data0 || t.offset + t.nbytes > size_ || t.offset + t.nbytes < t.offset)
                throw std::runtime_error("tensor out of bounds: " + t.name);
            t.data = base_ + t.offset;
            index_[t.name] = tensors_.size();
            tensors_.push_back(std::move(t));
        }
    } catch (...) {
        munmap((void *)base_, size_);
        ::close(fd_);
        throw;
    }
}

File::~File() {
    munmap((void *)base_, size_);
    ::close(fd_);
}

const Value &File::value(const std::string &key) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) throw std::runtime_error("gguf: missing key " + key);
    return it->second;
}

static std::runtime_error wrong_type(const std::string &key) {
    return std::runtime_error("gguf: key " + key + " has the wrong type");
}

int64_t File::get_int(const std::string &key) const {
    const Value &v = value(key);
    if (v.kind != Value::INT) throw wrong_type(key);
    return v.i;
}

double File::get_float(const std::string &key) const {
    const Value &v = value(key);
    if (v.kind == Value::INT) return (double)v.i;
    if (v.kind != Value::FLOAT) throw wrong_type(key);
    return v.f;
}

bool File::get_bool(const std::string &key) const {
    const Value &v = value(key);
    if (v.kind != Value::BOOL) throw wrong_type(key);
    return v.b;
}

const std::string &File::get_string(const std::string &key) const {
    const Value &v = value(key);
    if (v.kind != Value::STRING) throw wrong_type(key);
    return v.s;
}

const std::vector<uint8_t> &File::get_bool_array(const std::string &key) const {
    const Value &v = value(key);
    if (v.kind != Value::BOOL_ARRAY) throw wrong_type(key);
    return v.ba;
}

const Tensor *File::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

const Tensor &File::tensor(const std::string &name) const {
    const Tensor *t = find(name);
    if (!t) throw std::runtime_error("missing tensor " + name);
    return *t;
}

}  // namespace gguf
}  // namespace flint
