// Safetensors files on the host (midman-checkpoint: safetensors.rs, json.rs,
// params.rs): the header reader and writer, the model checkpoint's parameter
// layout, file I/O helpers and the TensorFile objects of the C ABI. Host code
// only (built with g++, and with the sanitizers by build_sanitized.py);
// checkpoint.hip streams the weights between these files and HBM.
//
// The format rules are the reference's:
//   * an 8-byte little-endian header length N, N bytes of JSON, then the data;
//   * the header is a JSON object restricted to objects, arrays, strings and
//     non-negative integers (json.rs:1-9), nesting depth <= 8, no duplicate keys;
//   * every tensor entry has exactly dtype "F32", shape and data_offsets, the
//     offsets span shape * 4 bytes, and sorted by offset the ranges tile the data
//     with no gap, overlap or trailing byte (safetensors.rs:255-300, 380-445);
//   * written files sort tensors by name, write __metadata__ first with its keys
//     sorted, escape strings as serde_json does (json.rs:51-67) and pad the header
//     with spaces to a multiple of 8 (safetensors.rs:140-214).
// A model checkpoint (params.rs:36-210) names every parameter as the reference
// does (embed_tokens.weight, blocks.{i}.attn_norm.weight,
// blocks.{i}.attn.{q,k,v,o}_proj.weight, blocks.{i}.mlp_norm.weight,
// blocks.{i}.mlp.{gate,up,down}_proj.weight, final_norm.weight, lm_head.weight)
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>

#include "mmh_checkpoint.h"

namespace mmh {
namespace st {

void parse_fail(const std::string &m) { fail(MMH_ERR_OTHER, "safetensors file: " + m); }

namespace {

constexpr uint64_t kMaxHeader = 100000000;  // safetensors.rs:38
constexpr int kMaxDepth = 8;                 // json.rs:18

// ---- json.rs: the restricted reader ------------------------------------------
struct Parser {
    const uint8_t *b;
    size_t n, pos = 0;

    [[noreturn]] void err(const std::string &m) const {
        parse_fail(m + " at byte " + std::to_string(pos));
    }
    int peek() const { return pos < n ? b[pos] : -1; }
    void ws() {
        while (pos < n && (b[pos] == ' ' || b[pos] == '\t' || b[pos] == '\n' || b[pos] == '\r'))
            ++pos;
    }
    void expect(uint8_t c) {
        if (peek() != c) err(std::string("expected `") + (char)c + "`");
        ++pos;
    }
    Json value(int depth) {
        if (depth > kMaxDepth) err("nesting is too deep");
        const int c = peek();
        if (c == '{') return object(depth);
        if (c == '[') return array(depth);
        if (c == '"') {
            Json v;
            v.kind = Json::String;
            v.str = string();
            return v;
        }
        if (c >= '0' && c <= '9') {
            Json v;
            v.kind = Json::Number;
            v.num = number();
            return v;
        }
        if (c == '-') err("negative numbers are not allowed");
        if (c < 0) err("unexpected end of the header");
        err("unexpected character");
    }
    Json object(int depth) {
        expect('{');
        ws();
        Json v;
        v.kind = Json::Object;
        if (peek() == '}') {
            ++pos;
            return v;
        }
        std::set<std::string> seen;
        for (;;) {
            ws();
            if (peek() != '"') err("expected a string key");
            std::string key = string();
            if (!seen.insert(key).second) err("duplicate key `" + key + "`");
            ws();
            expect(':');
            ws();
            Json item = value(depth + 1);
            v.obj.emplace_back(std::move(key), std::move(item));
            ws();
            const int c = peek();
            if (c == ',') {
                ++pos;
            } else if (c == '}') {
                ++pos;
                return v;
            } else {
                err("expected `,` or `}`");
            }
        }
    }
    Json array(int depth) {
        expect('[');
        ws();
        Json v;
        v.kind = Json::Array;
        if (peek() == ']') {
            ++pos;
            return v;
        }
        for (;;) {
            ws();
            v.arr.push_back(value(depth + 1));
            ws();
            const int c = peek();
            if (c == ',') {
                ++pos;
            } else if (c == ']') {
                ++pos;
                return v;
            } else {
                err("expected `,` or `]`");
            }
        }
    }
    uint64_t number() {
        const size_t start = pos;
        while (peek() >= '0' && peek() <= '9') ++pos;
        if (pos - start > 1 && b[start] == '0') err("numbers must not have leading zeros");
        const int c = peek();
        if (c == '.' || c == 'e' || c == 'E') err("fractions and exponents are not allowed");
        uint64_t v = 0;
        for (size_t i = start; i < pos; ++i) {
            const uint64_t d = b[i] - '0';
            if (v > (UINT64_MAX - d) / 10) err("number is too large");
            v = v * 10 + d;
        }
        return v;
    }
    uint32_t hex4() {
        if (pos + 4 > n) err("unterminated escape");
        uint32_t v = 0;
        for (int i = 0; i < 4; ++i) {
            const int c = b[pos + i];
            int d;
            if (c >= '0' && c <= '9') d = c - '0';
            else if (c >= 'a' && c <= 'f') d = c - 'a' + 10;
            else if (c >= 'A' && c <= 'F') d = c - 'A' + 10;
            else err("bad hex digit in an escape");
            v = v * 16 + (uint32_t)d;
        }
        pos += 4;
        return v;
    }
    static void put_utf8(std::string &out, uint32_t cp) {
        if (cp < 0x80) {
            out.push_back((char)cp);
        } else if (cp < 0x800) {
            out.push_back((char)(0xc0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3f)));
        } else if (cp < 0x10000) {
            out.push_back((char)(0xe0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
            out.push_back((char)(0x80 | (cp & 0x3f)));
        } else {
            out.push_back((char)(0xf0 | (cp >> 18)));
            out.push_back((char)(0x80 | ((cp >> 12) & 0x3f)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3f)));
            out.push_back((char)(0x80 | (cp & 0x3f)));
        }
    }
    std::string string() {
        expect('"');
        std::string out;
        for (;;) {
            const int c = peek();
            if (c < 0) err("unterminated string");
            ++pos;
            if (c == '"') break;
            if (c == '\\') {
                const int e = peek();
                if (e < 0) err("unterminated escape");
                ++pos;
                switch (e) {
                    case '"': out.push_back('"'); break;
                    case '\\': out.push_back('\\'); break;
                    case '/': out.push_back('/'); break;
                    case 'b': out.push_back('\b'); break;
                    case 'f': out.push_back('\f'); break;
                    case 'n': out.push_back('\n'); break;
                    case 'r': out.push_back('\r'); break;
                    case 't': out.push_back('\t'); break;
                    case 'u': {
                        const uint32_t first = hex4();
                        uint32_t cp = first;
                        if (first >= 0xd800 && first <= 0xdbff) {
                            if (!(peek() == '\\' && pos + 1 < n && b[pos + 1] == 'u'))
                                err("unpaired surrogate in an escape");
                            pos += 2;
                            const uint32_t second = hex4();
                            if (second < 0xdc00 || second > 0xdfff)
                                err("unpaired surrogate in an escape");
                            cp = 0x10000 + ((first - 0xd800) << 10) + (second - 0xdc00);
                        } else if (first >= 0xdc00 && first <= 0xdfff) {
                            err("unpaired surrogate in an escape");
                        }
                        put_utf8(out, cp);
                        break;
                    }
                    default:
                        --pos;
                        err("unknown escape");
                }
                continue;
            }
            if (c < 0x20) {
                --pos;
                err("control character in a string");
            }
            out.push_back((char)c);
        }
        return out;
    }
};

bool valid_utf8(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        size_t len;
        uint32_t cp;
        if (c < 0x80) {
            ++i;
            continue;
        } else if ((c & 0xe0) == 0xc0) {
            len = 2;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            len = 3;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (i + len > n) return false;
        for (size_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) ||
            cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff))
            return false;
        i += len;
    }
    return true;
}

bool mul_ok(uint64_t a, uint64_t b, uint64_t *out) {
    if (a != 0 && b > UINT64_MAX / a) return false;
    *out = a * b;
    return true;
}

}  // namespace

// json.rs:51-67: the escapes serde_json writes.
void write_json_string(std::string &out, const std::string &text) {
    out.push_back('"');
    for (unsigned char c : text) {
        switch (c) {
            case '"': out += "\\\""; break;
            case '\\': out += "\\\\"; break;
            case '\b': out += "\\b"; break;
            case '\f': out += "\\f"; break;
            case '\n': out += "\\n"; break;
            case '\r': out += "\\r"; break;
            case '\t': out += "\\t"; break;
            default:
                if (c < 0x20) {
                    char buf[8];
                    snprintf(buf, sizeof buf, "\\u%04x", (unsigned)c);
                    out += buf;
                } else {
                    out.push_back((char)c);
                }
        }
    }
    out.push_back('"');
}

// safetensors.rs:255-330 (from_bytes) and :380-445 (read_entry), given the
// header bytes and the length of what follows them.
Header parse_header(const uint8_t *header, uint64_t header_len, uint64_t data_len) {
    Header h;
    h.header_len = header_len;
    h.data_len = data_len;
    if (header_len == 0 || header[0] != '{') parse_fail("the header must start with `{`");
    if (!valid_utf8(header, header_len)) parse_fail("the header is not valid UTF-8");
    Parser p{header, (size_t)header_len};
    p.ws();
    Json root = p.value(0);
    p.ws();
    if (p.pos != p.n) p.err("unexpected data after the top-level value");
    if (root.kind != Json::Object) parse_fail("the header must be a JSON object");
    for (auto &kv : root.obj) {
        const std::string &key = kv.first;
        Json &val = kv.second;
        if (key == "__metadata__") {
            if (val.kind != Json::Object) parse_fail("`__metadata__` must be an object of strings");
            for (auto &m : val.obj) {
                if (m.second.kind != Json::String)
                    parse_fail("metadata value for `" + m.first + "` must be a string");
                h.metadata[m.first] = m.second.str;
            }
            continue;
        }
        if (val.kind != Json::Object) parse_fail("the entry for `" + key + "` must be an object");
        const Json *dtype = nullptr, *shape = nullptr, *offs = nullptr;
        for (auto &f : val.obj) {
            if (f.first == "dtype") dtype = &f.second;
            else if (f.first == "shape") shape = &f.second;
            else if (f.first == "data_offsets") offs = &f.second;
            else parse_fail("the entry for `" + key + "` has an unknown field `" + f.first + "`");
        }
        if (!dtype || !shape || !offs)
            parse_fail("the entry for `" + key + "` must have `dtype`, `shape` and `data_offsets`");
        if (dtype->kind != Json::String) parse_fail("the dtype of `" + key + "` must be a string");
        if (dtype->str != "F32")
            parse_fail("tensor `" + key + "` has dtype `" + dtype->str + "`; only F32 is supported");
        if (shape->kind != Json::Array) parse_fail("the shape of `" + key + "` must be an array");
        Entry e;
        e.name = key;
        for (auto &d : shape->arr) {
            if (d.kind != Json::Number) parse_fail("the shape of `" + key + "` must hold only integers");
            e.shape.push_back(d.num);
        }
        if (offs->kind != Json::Array || offs->arr.size() != 2 ||
            offs->arr[0].kind != Json::Number || offs->arr[1].kind != Json::Number)
            parse_fail("the data_offsets of `" + key + "` must be two integers");
        e.begin = offs->arr[0].num;
        e.end = offs->arr[1].num;
        uint64_t count = 1, bytes = 0;
        for (uint64_t d : e.shape)
            if (!mul_ok(count, d, &count)) parse_fail("the shape of `" + key + "` is too large");
        if (!mul_ok(count, 4, &bytes)) parse_fail("the shape of `" + key + "` is too large");
        if (e.end < e.begin || e.end - e.begin != bytes)
            parse_fail("tensor `" + key + "` has a shape that needs " + std::to_string(bytes) +
                       " bytes, but its data_offsets [" + std::to_string(e.begin) + ", " +
                       std::to_string(e.end) + "] do not span that");
        e.numel = count;
        h.entries.push_back(std::move(e));
    }
    std::stable_sort(h.entries.begin(), h.entries.end(), [](const Entry &a, const Entry &b) {
        return a.begin != b.begin ? a.begin < b.begin : a.end < b.end;
    });
    uint64_t expected = 0;
    for (const Entry &e : h.entries) {
        if (e.begin != expected)
            parse_fail("tensor `" + e.name + "` starts at byte " + std::to_string(e.begin) +
                       " where byte " + std::to_string(expected) +
                       " was expected: the data ranges must tile the data with no gap or overlap");
        expected = e.end;
    }
    if (expected != data_len)
        parse_fail("the tensors cover " + std::to_string(expected) +
                   " bytes but the data section has " + std::to_string(data_len));
    return h;
}

Header parse_prefix_and_header(const uint8_t *bytes, uint64_t len) {
    if (len < 8) parse_fail("the file is shorter than its 8-byte length prefix");
    uint64_t hl = 0;
    std::memcpy(&hl, bytes, 8);
    if (hl > kMaxHeader)
        parse_fail("the header claims " + std::to_string(hl) +
                   " bytes, over the format's limit of 100000000");
    if (hl > len - 8)
        parse_fail("the header claims " + std::to_string(hl) + " bytes but the file has only " +
                   std::to_string(len - 8) + " after the prefix");
    return parse_header(bytes + 8, hl, len - 8 - hl);
}

// safetensors.rs:150-190: __metadata__ first (keys sorted), then the tensors in
// the given (name-sorted) order, offsets consecutive, spaces to a multiple of 8.
std::string build_header(const std::vector<TensorSpec> &sorted,
                         const std::map<std::string, std::string> &metadata) {
    std::string h = "{";
    bool first = true;
    if (!metadata.empty()) {
        h += "\"__metadata__\":{";
        bool f = true;
        for (auto &kv : metadata) {
            if (!f) h.push_back(',');
            f = false;
            write_json_string(h, kv.first);
            h.push_back(':');
            write_json_string(h, kv.second);
        }
        h.push_back('}');
        first = false;
    }
    uint64_t begin = 0;
    for (const TensorSpec &t : sorted) {
        uint64_t count = 1, bytes = 0;
        for (uint64_t d : t.shape)
            if (!mul_ok(count, d, &count)) fail(MMH_ERR_ARGUMENT, "the tensors are too large to address");
        if (!mul_ok(count, 4, &bytes) || begin + bytes < begin)
            fail(MMH_ERR_ARGUMENT, "the tensors are too large to address");
        const uint64_t end = begin + bytes;
        if (!first) h.push_back(',');
        first = false;
        write_json_string(h, t.name);
        h += ":{\"dtype\":\"F32\",\"shape\":[";
        for (size_t i = 0; i < t.shape.size(); ++i) {
            if (i) h.push_back(',');
            h += std::to_string(t.shape[i]);
        }
        h += "],\"data_offsets\":[" + std::to_string(begin) + "," + std::to_string(end) + "]}";
        begin = end;
    }
    h.push_back('}');
    h.append((8 - h.size() % 8) % 8, ' ');
    if (h.size() > kMaxHeader)
        fail(MMH_ERR_ARGUMENT, "the header is " + std::to_string(h.size()) +
                                   " bytes, over the format's limit of 100000000");
    return h;
}

}  // namespace st

// ---- model checkpoint layout (params.rs) --------------------------------------

std::vector<ParamSpec> model_param_specs(int64_t vocab, int64_t d, int64_t layers, int64_t kv,
                                         int64_t ff, bool tie) {
    std::vector<ParamSpec> out;
    int64_t off = 0;
    auto add = [&](std::string name, std::vector<uint64_t> shape) {
        uint64_t n = 1;
        for (uint64_t s : shape) n *= s;
        out.push_back({std::move(name), std::move(shape), off, (int64_t)n});
        off += (int64_t)n;
    };
    add("embed_tokens.weight", {(uint64_t)vocab, (uint64_t)d});
    for (int64_t l = 0; l < layers; ++l) {
        const std::string b = "blocks." + std::to_string(l) + ".";
        add(b + "attn_norm.weight", {(uint64_t)d});
        add(b + "attn.q_proj.weight", {(uint64_t)d, (uint64_t)d});
        add(b + "attn.k_proj.weight", {(uint64_t)d, (uint64_t)kv});
        add(b + "attn.v_proj.weight", {(uint64_t)d, (uint64_t)kv});
        add(b + "attn.o_proj.weight", {(uint64_t)d, (uint64_t)d});
        add(b + "mlp_norm.weight", {(uint64_t)d});
        add(b + "mlp.gate_proj.weight", {(uint64_t)d, (uint64_t)ff});
        add(b + "mlp.up_proj.weight", {(uint64_t)d, (uint64_t)ff});
        add(b + "mlp.down_proj.weight", {(uint64_t)ff, (uint64_t)d});
    }
    add("final_norm.weight", {(uint64_t)d});
    if (!tie) add("lm_head.weight", {(uint64_t)d, (uint64_t)vocab});
    return out;
}

// ---- file I/O ------------------------------------------------------------------


std::string io_error(const std::string &path, const std::string &what) {
    return path + ": " + what + ": " + std::strerror(errno);
}

void write_all(int fd, const void *p, size_t n, const std::string &path) {
    const char *c = static_cast<const char *>(p);
    while (n) {
        const ssize_t w = ::write(fd, c, n);
        if (w < 0) {
            if (errno == EINTR) continue;
            fail(MMH_ERR_OTHER, io_error(path, "write"));
        }
        c += w;
        n -= (size_t)w;
    }
}

void read_all(int fd, void *p, size_t n, uint64_t off, const std::string &path) {
    char *c = static_cast<char *>(p);
    while (n) {
        const ssize_t r = ::pread(fd, c, n, (off_t)off);
        if (r < 0) {
            if (errno == EINTR) continue;
            fail(MMH_ERR_OTHER, io_error(path, "read"));
        }
        if (r == 0) fail(MMH_ERR_OTHER, path + ": unexpected end of file");
        c += r;
        n -= (size_t)r;
        off += (uint64_t)r;
    }
}

}  // namespace mmh

// ---- TensorFile (safetensors.rs:68-330) over the C ABI ------------------------

namespace mmh {
namespace {

struct TensorFileObj {
    struct Tensor {
        std::string name;
        std::vector<uint64_t> shape;
        std::vector<float> data;
    };
    std::vector<Tensor> tensors;  // insertion order, or file order when parsed
    std::map<std::string, std::string> metadata;
};

std::mutex g_tf_mutex;
std::vector<std::unique_ptr<TensorFileObj>> g_tfs;  // handle = index + 1

TensorFileObj &tf(mmh_handle h) {
    std::lock_guard<std::mutex> lock(g_tf_mutex);
    if (h <= 0 || (size_t)h > g_tfs.size() || !g_tfs[(size_t)h - 1])
        fail(MMH_ERR_ARGUMENT, "invalid tensor file handle " + std::to_string(h));
    return *g_tfs[(size_t)h - 1];
}

mmh_handle register_tf(std::unique_ptr<TensorFileObj> t) {
    std::lock_guard<std::mutex> lock(g_tf_mutex);
    g_tfs.push_back(std::move(t));
    return (mmh_handle)g_tfs.size();
}

std::unique_ptr<TensorFileObj> from_bytes(const uint8_t *bytes, uint64_t len) {
    st::Header h = st::parse_prefix_and_header(bytes, len);
    auto t = std::make_unique<TensorFileObj>();
    t->metadata = h.metadata;
    const uint8_t *data = bytes + 8 + h.header_len;
    for (const st::Entry &e : h.entries) {
        TensorFileObj::Tensor x;
        x.name = e.name;
        x.shape = e.shape;
        x.data.resize((size_t)e.numel);
        if (e.numel) std::memcpy(x.data.data(), data + e.begin, (size_t)(e.end - e.begin));
        t->tensors.push_back(std::move(x));
    }
    return t;
}

void copy_out(const std::string &s, char *buf, uint32_t cap, uint32_t *len) {
    if (len) *len = (uint32_t)s.size();
    if (buf && cap) std::memcpy(buf, s.data(), std::min<size_t>(cap, s.size()));
}

}  // namespace
}  // namespace mmh

using namespace mmh;

extern "C" {

int32_t mmh_tensorfile_create(mmh_handle *out) {
    return guard([&] {
        if (!out) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        *out = register_tf(std::make_unique<TensorFileObj>());
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_parse(const uint8_t *bytes, uint64_t len, mmh_handle *out) {
    return guard([&] {
        if (!out) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
        if (!bytes && len) fail(MMH_ERR_ARGUMENT, "bytes is a null pointer");
        static const uint8_t none = 0;
        *out = register_tf(from_bytes(bytes ? bytes : &none, len));
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_push(mmh_handle h, const char *name, uint32_t name_len,
                            const uint64_t *shape, int32_t rank, const float *data, uint64_t n) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if (!name && name_len) fail(MMH_ERR_ARGUMENT, "name is a null pointer");
        if (rank < 0 || (rank > 0 && !shape)) fail(MMH_ERR_ARGUMENT, "bad shape");
        if (!data && n) fail(MMH_ERR_ARGUMENT, "data is a null pointer");
        std::string nm(name ? name : "", name_len);
        if (nm == "__metadata__")
            fail(MMH_ERR_ARGUMENT, "`__metadata__` is reserved and cannot name a tensor");
        for (auto &x : t.tensors)
            if (x.name == nm) fail(MMH_ERR_ARGUMENT, "two tensors are named `" + nm + "`");
        uint64_t count = 1;
        bool ok = true;
        for (int32_t i = 0; i < rank; ++i) {
            if (shape[i] != 0 && count > UINT64_MAX / shape[i]) ok = false;
            count *= shape[i];
        }
        if (!ok || count != n)
            fail(MMH_ERR_SHAPE, "TensorFile::push: tensor `" + nm + "` has a shape of " +
                                    std::to_string(count) + " values but " + std::to_string(n) +
                                    " values");
        TensorFileObj::Tensor x;
        x.name = nm;
        x.shape.assign(shape, shape + rank);
        x.data.assign(data, data + n);
        t.tensors.push_back(std::move(x));
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_set_metadata(mmh_handle h, const char *key, uint32_t key_len,
                                    const char *value, uint32_t value_len) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if ((!key && key_len) || (!value && value_len))
            fail(MMH_ERR_ARGUMENT, "key or value is a null pointer");
        t.metadata[std::string(key ? key : "", key_len)] = std::string(value ? value : "", value_len);
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_count(mmh_handle h, int64_t *n_tensors, int64_t *n_metadata) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if (n_tensors) *n_tensors = (int64_t)t.tensors.size();
        if (n_metadata) *n_metadata = (int64_t)t.metadata.size();
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_tensor(mmh_handle h, int64_t i, char *name, uint32_t name_cap,
                              uint32_t *name_len, int32_t *rank, uint64_t *shape,
                              int32_t shape_cap, uint64_t *numel) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if (i < 0 || (size_t)i >= t.tensors.size()) fail(MMH_ERR_INDEX, "tensor index out of range");
        const auto &x = t.tensors[(size_t)i];
        copy_out(x.name, name, name_cap, name_len);
        if (rank) *rank = (int32_t)x.shape.size();
        if (shape)
            for (size_t k = 0; k < x.shape.size() && (int32_t)k < shape_cap; ++k) shape[k] = x.shape[k];
        if (numel) *numel = (uint64_t)x.data.size();
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_read(mmh_handle h, int64_t i, float *out, uint64_t n) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if (i < 0 || (size_t)i >= t.tensors.size()) fail(MMH_ERR_INDEX, "tensor index out of range");
        const auto &x = t.tensors[(size_t)i];
        if (n != x.data.size()) fail(MMH_ERR_SHAPE, "read: wrong value count");
        if (n) {
            if (!out) fail(MMH_ERR_ARGUMENT, "out is a null pointer");
            std::memcpy(out, x.data.data(), (size_t)n * 4);
        }
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_metadata(mmh_handle h, int64_t i, char *key, uint32_t key_cap,
                                uint32_t *key_len, char *value, uint32_t value_cap,
                                uint32_t *value_len) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        if (i < 0 || (size_t)i >= t.metadata.size()) fail(MMH_ERR_INDEX, "metadata index out of range");
        auto it = t.metadata.begin();
        std::advance(it, i);
        copy_out(it->first, key, key_cap, key_len);
        copy_out(it->second, value, value_cap, value_len);
        return MMH_OK;
    });
}

// TensorFile::to_bytes (safetensors.rs:140-214): out may be NULL to learn the size.
int32_t mmh_tensorfile_serialize(mmh_handle h, uint8_t *out, uint64_t cap, uint64_t *len) {
    return guard([&] {
        TensorFileObj &t = tf(h);
        std::vector<const TensorFileObj::Tensor *> sorted;
        for (auto &x : t.tensors) sorted.push_back(&x);
        std::sort(sorted.begin(), sorted.end(),
                  [](const TensorFileObj::Tensor *a, const TensorFileObj::Tensor *b) {
                      return a->name < b->name;
                  });
        std::vector<st::TensorSpec> specs;
        uint64_t data_bytes = 0;
        for (auto *x : sorted) {
            specs.push_back({x->name, x->shape});
            data_bytes += (uint64_t)x->data.size() * 4;
        }
        const std::string header = st::build_header(specs, t.metadata);
        const uint64_t total = 8 + header.size() + data_bytes;
        if (len) *len = total;
        if (!out) return MMH_OK;
        if (cap < total) fail(MMH_ERR_SHAPE, "serialize: the buffer holds " + std::to_string(cap) +
                                                 " bytes, the file needs " + std::to_string(total));
        const uint64_t hl = header.size();
        std::memcpy(out, &hl, 8);
        std::memcpy(out + 8, header.data(), header.size());
        uint8_t *p = out + 8 + header.size();
        for (auto *x : sorted) {
            if (x->data.empty()) continue;  // an empty vector's data() may be null
            std::memcpy(p, x->data.data(), x->data.size() * 4);
            p += x->data.size() * 4;
        }
        return MMH_OK;
    });
}

int32_t mmh_tensorfile_destroy(mmh_handle h) {
    return guard([&] {
        std::lock_guard<std::mutex> lock(g_tf_mutex);
        if (h <= 0 || (size_t)h > g_tfs.size() || !g_tfs[(size_t)h - 1])
            fail(MMH_ERR_ARGUMENT, "invalid tensor file handle " + std::to_string(h));
        g_tfs[(size_t)h - 1].reset();
        return MMH_OK;
    });
}

}  // extern "C"
