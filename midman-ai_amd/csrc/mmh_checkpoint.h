// Safetensors headers and model checkpoints: the format on the host
// (host_safetensors.cpp) and the streaming between files and HBM
// (checkpoint.hip). Host-only declarations.
#pragma once

#include <unistd.h>

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "mmh_error.h"

namespace mmh {

struct Context;
namespace st {

// A parsed header value: the restricted JSON of a safetensors header.
struct Json {
    enum Kind { Object, Array, String, Number } kind = Object;
    std::vector<std::pair<std::string, Json>> obj;
    std::vector<Json> arr;
    std::string str;
    uint64_t num = 0;
};

struct Entry {
    std::string name;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0, numel = 0;
};

// Entries sorted by data offset (file order) and the string metadata.
struct Header {
    std::vector<Entry> entries;
    std::map<std::string, std::string> metadata;
    uint64_t header_len = 0, data_len = 0;
};

struct TensorSpec {
    std::string name;
    std::vector<uint64_t> shape;
};

[[noreturn]] void parse_fail(const std::string &m);
void write_json_string(std::string &out, const std::string &text);
// Validates the header of a file whose data section has data_len bytes.
Header parse_header(const uint8_t *header, uint64_t header_len, uint64_t data_len);
// A whole file in memory: prefix, header, data.
Header parse_prefix_and_header(const uint8_t *bytes, uint64_t len);
// The header text (padded) for tensors in the given order.
std::string build_header(const std::vector<TensorSpec> &sorted,
                         const std::map<std::string, std::string> &metadata);

}  // namespace st

// One parameter of the flat weight layout: reference name, shape, offset.
struct ParamSpec {
    std::string name;
    std::vector<uint64_t> shape;
    int64_t offset;
    int64_t numel;
};

// File I/O that fails with MMH_ERR_OTHER and the path and errno text.
std::string io_error(const std::string &path, const std::string &what);
void write_all(int fd, const void *p, size_t n, const std::string &path);
// n bytes at offset off (pread); a short file is an error.
void read_all(int fd, void *p, size_t n, uint64_t off, const std::string &path);
// A file descriptor closed when it goes out of scope.
struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

std::vector<ParamSpec> model_param_specs(int64_t vocab, int64_t d, int64_t layers, int64_t kv,
                                         int64_t ff, bool tie);
void save_checkpoint(Context &ctx, const float *weights_dev, const std::vector<ParamSpec> &specs,
                     const std::map<std::string, std::string> &user_meta,
                     const std::string &path);
void load_checkpoint(Context &ctx, const std::vector<ParamSpec> &specs, int64_t n_params,
                     const std::string &path, float *dst_dev,
                     std::map<std::string, std::string> *meta_out);

}  // namespace mmh
