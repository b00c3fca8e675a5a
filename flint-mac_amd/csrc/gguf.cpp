// GGUF v3 reader (see gguf.h), written from the format description:
//
//   header      u32 magic "GGUF" | u32 version | u64 tensor count | u64 key/value count
//   key/values  string key | u32 value type | value
//   tensor info string name | u32 rank | u64 dims[rank] | u32 ggml type | u64 offset
//   padding     to general.alignment (32 when the key is absent)
//   data        tensor offsets are relative to its start
//
// Strings are a u64 byte count and the bytes; an array is a u32 element type, a u64
// count and the elements. Every scalar metadata type is a fixed-width little-endian
// number, so one table (width and class per type id) drives the decoding of scalars
// and of scalar arrays alike. Error texts are the ones the reference's reader gives
// (/root/reference/src/gguf.cpp), so callers see the same messages.
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

using std::runtime_error;

// ---- metadata value types -------------------------------------------------------------

enum Class : uint8_t { NONE, UNSIGNED, SIGNED, REAL, FLAG };
struct Scalar {
    uint8_t width;  // bytes in the file
    Class cls;
};
constexpr uint32_t kString = 8, kArray = 9;
// indexed by the format's value-type id; ids 8 (string) and 9 (array) are not scalars
constexpr Scalar kScalars[] = {
    {1, UNSIGNED}, {1, SIGNED}, {2, UNSIGNED}, {2, SIGNED}, {4, UNSIGNED}, {4, SIGNED}, {4, REAL},
    {1, FLAG},     {0, NONE},   {0, NONE},     {8, UNSIGNED}, {8, SIGNED}, {8, REAL},
};
constexpr uint32_t kNumTypes = sizeof(kScalars) / sizeof(kScalars[0]);

const Scalar *scalar_of(uint32_t type) {
    return type < kNumTypes && kScalars[type].cls != NONE ? &kScalars[type] : nullptr;
}

// ---- ggml tensor types ----------------------------------------------------------------

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

const TypeRow *type_row(uint32_t id) {
    for (const TypeRow &t : kTypes)
        if (t.id == id) return &t;
    return nullptr;
}

// ---- the byte stream ------------------------------------------------------------------

// A window over the mapped file that hands out byte ranges front to back.
struct Span {
    const uint8_t *at, *end;

    const uint8_t *take(uint64_t n) {
        if ((uint64_t)(end - at) < n) throw runtime_error("gguf: unexpected end of file");
        const uint8_t *p = at;
        at += n;
        return p;
    }
    uint64_t left() const { return (uint64_t)(end - at); }
    uint32_t u32() { return (uint32_t)bits(take(4), 4); }
    uint64_t u64() { return bits(take(8), 8); }
    std::string text() {
        const uint64_t n = u64();
        return std::string((const char *)take(n), (size_t)n);
    }
    static uint64_t bits(const uint8_t *p, int width) {
        uint64_t u = 0;
        std::memcpy(&u, p, width);  // the format is little-endian, as is the host
        return u;
    }
};

// One fixed-width scalar (bytes at p) as an integer, a real or a flag.
int64_t to_int(const uint8_t *p, const Scalar &s) {
    const uint64_t u = Span::bits(p, s.width);
    if (s.cls == SIGNED && s.width < 8) {
        const int shift = 64 - 8 * s.width;
        return (int64_t)(u << shift) >> shift;
    }
    return (int64_t)u;
}
double to_real(const uint8_t *p, const Scalar &s) {
    if (s.width == 4) {
        float f;
        std::memcpy(&f, p, 4);
        return f;
    }
    double d;
    std::memcpy(&d, p, 8);
    return d;
}

// Append one scalar to the value: a scalar value when `array` is false, an element of
// the array of that class otherwise.
void put(Value &v, const uint8_t *p, const Scalar &s, bool array) {
    switch (s.cls) {
        case UNSIGNED:
        case SIGNED:
            if (array) v.ia.push_back(to_int(p, s)); else v.i = to_int(p, s);
            break;
        case REAL:
            if (array) v.fa.push_back(to_real(p, s)); else v.f = to_real(p, s);
            break;
        default:
            if (array) v.ba.push_back(*p != 0); else v.b = *p != 0;
            break;
    }
}

Value::Kind kind_of(Class c, bool array) {
    switch (c) {
        case UNSIGNED:
        case SIGNED: return array ? Value::INT_ARRAY : Value::INT;
        case REAL: return array ? Value::FLOAT_ARRAY : Value::FLOAT;
        default: return array ? Value::BOOL_ARRAY : Value::BOOL;
    }
}

Value decode(Span &in, uint32_t type) {
    Value v;
    if (const Scalar *s = scalar_of(type)) {
        v.kind = kind_of(s->cls, false);
        put(v, in.take(s->width), *s, false);
        return v;
    }
    if (type == kString) {
        v.kind = Value::STRING;
        v.s = in.text();
        return v;
    }
    if (type != kArray) throw runtime_error("gguf: unknown metadata type " + std::to_string(type));
    const uint32_t elem = in.u32();
    const uint64_t count = in.u64();
    if (const Scalar *s = scalar_of(elem)) {
        // the whole array must be in the file before anything is allocated for it
        if (count > in.left() / s->width) throw runtime_error("gguf: unexpected end of file");
        v.kind = kind_of(s->cls, true);
        const uint8_t *p = in.take(count * s->width);
        for (uint64_t k = 0; k < count; k++) put(v, p + k * s->width, *s, true);
        return v;
    }
    if (elem != kString) throw runtime_error("gguf: unsupported array element type");
    v.kind = Value::STRING_ARRAY;
    for (uint64_t k = 0; k < count; k++) v.sa.push_back(in.text());
    return v;
}

// Bytes of a tensor of the given dims in blocks of geometry g, or throws.
uint64_t tensor_bytes(const std::vector<uint64_t> &dims, const BlockGeom &g, const std::string &name) {
    uint64_t n = 1;
    for (uint64_t d : dims) {
        if (d != 0 && n > UINT64_MAX / d) throw runtime_error("tensor out of bounds: " + name);
        n *= d;
    }
    const uint64_t blocks = n / g.elems;
    if (n % g.elems != 0 || blocks > UINT64_MAX / g.bytes) throw runtime_error("tensor out of bounds: " + name);
    return blocks * g.bytes;
}

}  // namespace

bool block_geom(uint32_t type, BlockGeom *g) {
    const TypeRow *t = type_row(type);
    if (t) *g = t->geom;
    return t != nullptr;
}

const char *type_name(uint32_t type) {
    const TypeRow *t = type_row(type);
    return t ? t->name : "?";
}

uint64_t Tensor::n_rows() const {
    uint64_t n = 1;
    for (size_t d = 1; d < dims.size(); d++) n *= dims[d];
    return n;
}

uint64_t Tensor::row_bytes() const {
    const TypeRow *t = type_row(type);
    return dims.empty() || !t ? 0 : dims[0] / t->geom.elems * t->geom.bytes;
}

File::File(const std::string &path) : path_(path) {
    fd_ = ::open(path.c_str(), O_RDONLY);
    struct stat st {};
    if (fd_ < 0 || fstat(fd_, &st) != 0) {
        if (fd_ >= 0) ::close(fd_);
        throw runtime_error("cannot open " + path);
    }
    size_ = (size_t)st.st_size;
    if (size_ == 0) {
        ::close(fd_);
        throw runtime_error("gguf: unexpected end of file");
    }
    void *m = mmap(nullptr, size_, PROT_READ, MAP_SHARED, fd_, 0);
    if (m == MAP_FAILED) {
        ::close(fd_);
        throw runtime_error("mmap failed: " + path);
    }
    base_ = (const uint8_t *)m;
    try {
        parse();
    } catch (...) {
        munmap((void *)base_, size_);
        ::close(fd_);
        throw;
    }
}

void File::parse() {
    Span in{base_, base_ + size_};
    if (in.u32() != 0x46554747u) throw runtime_error("not a GGUF file: " + path_);
    if (in.u32() < 3) throw runtime_error("unsupported GGUF version");
    const uint64_t n_tensors = in.u64(), n_kv = in.u64();
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = in.text();
        const uint32_t type = in.u32();
        meta_[std::move(key)] = decode(in, type);
    }
    // The tensor table. `offset` holds the offset into the data section until the
    // section's start is known (it follows the table, aligned).
    for (uint64_t k = 0; k < n_tensors; k++) {
        Tensor t;
        t.name = in.text();
        const uint32_t rank = in.u32();
        if (rank > in.left() / 8) throw runtime_error("gguf: unexpected end of file");
        t.dims.resize(rank);
        for (uint64_t &d : t.dims) d = in.u64();
        t.type = in.u32();
        t.offset = in.u64();
        tensors_.push_back(std::move(t));
    }
    const uint64_t align = has("general.alignment") ? (uint64_t)get_int("general.alignment") : 32;
    if (align == 0) throw runtime_error("gguf: general.alignment is 0");
    const uint64_t table_end = (uint64_t)(in.at - base_);
    const uint64_t data0 = (table_end + align - 1) / align * align;
    for (size_t i = 0; i < tensors_.size(); i++) {
        Tensor &t = tensors_[i];
        const TypeRow *row = type_row(t.type);
        if (!row) throw runtime_error("unsupported ggml type " + std::to_string(t.type));
        t.nbytes = tensor_bytes(t.dims, row->geom, t.name);
        const uint64_t rel = t.offset;
        t.offset = data0 + rel;
        if (t.offset < rel || t.offset > size_ || t.nbytes > size_ - t.offset)
            throw runtime_error("tensor out of bounds: " + t.name);
        t.data = base_ + t.offset;
        index_[t.name] = i;
    }
}

File::~File() {
    munmap((void *)base_, size_);
    ::close(fd_);
}

const Value &File::value(const std::string &key) const {
    auto it = meta_.find(key);
    if (it == meta_.end()) throw runtime_error("gguf: missing key " + key);
    return it->second;
}

// a value of the expected kind, or "gguf: key ... has the wrong type"
const Value &File::typed(const std::string &key, int kind) const {
    const Value &v = value(key);
    if (v.kind != kind) throw runtime_error("gguf: key " + key + " has the wrong type");
    return v;
}

int64_t File::get_int(const std::string &key) const { return typed(key, Value::INT).i; }

double File::get_float(const std::string &key) const {
    const Value &v = value(key);
    return v.kind == Value::INT ? (double)v.i : typed(key, Value::FLOAT).f;
}

bool File::get_bool(const std::string &key) const { return typed(key, Value::BOOL).b; }

const std::string &File::get_string(const std::string &key) const { return typed(key, Value::STRING).s; }

const std::vector<uint8_t> &File::get_bool_array(const std::string &key) const {
    return typed(key, Value::BOOL_ARRAY).ba;
}

const Tensor *File::find(const std::string &name) const {
    auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

const Tensor &File::tensor(const std::string &name) const {
    const Tensor *t = find(name);
    if (!t) throw runtime_error("missing tensor " + name);
    return *t;
}

}  // namespace gguf
}  // namespace flint
