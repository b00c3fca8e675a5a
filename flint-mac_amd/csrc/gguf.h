// Read-only GGUF v3 reader: the file is memory-mapped once; metadata is decoded
// into typed values and the tensor table into (name, ggml type, dims, bytes).
// Reads the format the reference parses at /root/reference/src/gguf.cpp:137-194
// (header, key/value section, tensor infos, data section aligned to
// general.alignment, default 32) and reports the same error messages.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <unordered_map>
#include <vector>

namespace flint {
namespace gguf {

// ggml type ids and block geometry (elements, bytes per block) of every type the
// reference's loader knows (/root/reference/src/gguf.h:14-19, gguf.cpp:112-124).
struct BlockGeom {
    int elems, bytes;
};
// false if the id is not a known type
bool block_geom(uint32_t type, BlockGeom *g);
const char *type_name(uint32_t type);

// One metadata value. Integers of every width decode to i, f32/f64 to f; arrays keep
// their element kind.
struct Value {
    enum Kind { INT, FLOAT, BOOL, STRING, INT_ARRAY, FLOAT_ARRAY, BOOL_ARRAY, STRING_ARRAY } kind = INT;
    int64_t i = 0;
    double f = 0;
    bool b = false;
    std::string s;
    std::vector<int64_t> ia;
    std::vector<double> fa;
    std::vector<uint8_t> ba;
    std::vector<std::string> sa;
};

struct Tensor {
    std::string name;
    uint32_t type = 0;
    std::vector<uint64_t> dims;  // ggml order: dims[0] is the row length
    uint64_t offset = 0;         // from the start of the file
    uint64_t nbytes = 0;
    const uint8_t *data = nullptr;  // into the mapping

    uint64_t n_rows() const;     // product of dims[1..]
    uint64_t row_bytes() const;  // bytes of dims[0] elements
};

class File {
public:
    explicit File(const std::string &path);  // throws std::runtime_error
    ~File();
    File(const File &) = delete;
    File &operator=(const File &) = delete;

    const std::string &path() const { return path_; }
    bool has(const std::string &key) const { return meta_.count(key) != 0; }
    int64_t get_int(const std::string &key) const;
    double get_float(const std::string &key) const;  // an integer value converts
    bool get_bool(const std::string &key) const;
    const std::string &get_string(const std::string &key) const;
    const std::vector<uint8_t> &get_bool_array(const std::string &key) const;

    const Tensor *find(const std::string &name) const;
    const Tensor &tensor(const std::string &name) const;  // throws "missing tensor <name>"
    const std::vector<Tensor> &tensors() const { return tensors_; }

private:
    void parse();  // header, metadata and tensor table of the mapped file
    const Value &value(const std::string &key) const;
    const Value &typed(const std::string &key, int kind) const;

    std::string path_;
    int fd_ = -1;
    const uint8_t *base_ = nullptr;
    size_t size_ = 0;
    std::unordered_map<std::string, Value> meta_;
    std::vector<Tensor> tensors_;
    std::unordered_map<std::string, size_t> index_;
};

}  // namespace gguf
}  // namespace flint
