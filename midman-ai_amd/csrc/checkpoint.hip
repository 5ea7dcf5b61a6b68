// Model checkpoints streamed between HBM and safetensors files (params.rs:36-210,
// safetensors.rs:220-300): a load never builds host tensors and a save never
// holds more than two pinned staging chunks on the host. The file format
// itself (header reader and writer, parameter layout, I/O helpers) is host code
// in host_safetensors.cpp.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <map>
#include <set>

#include "mmh_checkpoint.h"
#include "mmh_internal.h"

namespace mmh {

namespace {

// Two pinned host chunks with an event each: the device side of a chunk's copy
// runs while the other chunk is filled or drained by the file.
struct Staging {
    static constexpr size_t kChunk = size_t(64) << 20;
    void *buf[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    bool busy[2] = {false, false};
    Staging() {
        for (int i = 0; i < 2; ++i) {
            check_hip(hipHostMalloc(&buf[i], kChunk, hipHostMallocDefault), "pinned staging alloc");
            check_hip(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "event");
        }
    }
    ~Staging() {
        for (int i = 0; i < 2; ++i) {
            if (done[i]) {
                (void)hipEventSynchronize(done[i]);
                (void)hipEventDestroy(done[i]);
            }
            if (buf[i]) (void)hipHostFree(buf[i]);
        }
    }
    void *acquire(int i) {
        if (busy[i]) check_hip(hipEventSynchronize(done[i]), "staging wait");
        busy[i] = false;
        return buf[i];
    }
    void issued(int i, hipStream_t s) {
        check_hip(hipEventRecord(done[i], s), "staging event");
        busy[i] = true;
    }
};

}  // namespace

// save_parameters (params.rs:36-80) from device weights: header in memory, data
// streamed in name order through the pinned chunks, written to <path>.tmp,
// flushed and renamed over path (safetensors.rs:220-250).
void save_checkpoint(Context &ctx, const float *weights_dev, const std::vector<ParamSpec> &specs,
                     const std::map<std::string, std::string> &user_meta,
                     const std::string &path) {
    for (const char *reserved : {"format", "checkpoint_version"})
        if (user_meta.count(reserved))
            fail(MMH_ERR_ARGUMENT, std::string("metadata key `") + reserved +
                                       "` is set by the checkpoint writer");
    std::map<std::string, std::string> meta = user_meta;
    meta["format"] = "midman-checkpoint";
    meta["checkpoint_version"] = "1";
    std::vector<const ParamSpec *> order;
    for (const ParamSpec &s : specs) order.push_back(&s);
    std::sort(order.begin(), order.end(),
              [](const ParamSpec *a, const ParamSpec *b) { return a->name < b->name; });
    std::vector<st::TensorSpec> ts;
    for (const ParamSpec *s : order) ts.push_back({s->name, s->shape});
    const std::string header = st::build_header(ts, meta);

    const std::string tmp = path + ".tmp";
    Fd f;
    f.fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (f.fd < 0) fail(MMH_ERR_OTHER, io_error(tmp, "create"));
    try {
        const uint64_t hl = header.size();
        write_all(f.fd, &hl, 8, tmp);
        write_all(f.fd, header.data(), header.size(), tmp);
        Staging stg;
        check_hip(hipStreamSynchronize(ctx.stream), "save sync");
        // Flattened list of (device source, bytes) pieces in file order.
        int slot = 0;
        int pending = -1;
        size_t pending_bytes = 0;
        auto drain = [&]() {
            if (pending < 0) return;
            check_hip(hipEventSynchronize(stg.done[pending]), "staging wait");
            stg.busy[pending] = false;
            write_all(f.fd, stg.buf[pending], pending_bytes, tmp);
            pending = -1;
        };
        for (const ParamSpec *s : order) {
            const char *src = reinterpret_cast<const char *>(weights_dev + s->offset);
            size_t left = (size_t)s->numel * 4;
            while (left) {
                const size_t n = std::min(left, Staging::kChunk);
                void *dst = stg.acquire(slot);
                check_hip(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, ctx.stream),
                          "checkpoint download");
                stg.issued(slot, ctx.stream);
                drain();  // the other chunk's bytes go to the file while this one copies
                pending = slot;
                pending_bytes = n;
                slot ^= 1;
                src += n;
                left -= n;
            }
        }
        drain();
        if (::fsync(f.fd) != 0) fail(MMH_ERR_OTHER, io_error(tmp, "fsync"));
        if (::close(f.fd) != 0) {
            f.fd = -1;
            fail(MMH_ERR_OTHER, io_error(tmp, "close"));
        }
        f.fd = -1;
        if (::rename(tmp.c_str(), path.c_str()) != 0) fail(MMH_ERR_OTHER, io_error(path, "rename"));
    } catch (...) {
        if (f.fd >= 0) {
            ::close(f.fd);
            f.fd = -1;
        }
        ::unlink(tmp.c_str());
        throw;
    }
}

// check_header + load_parameters (params.rs:82-210) into a fresh device buffer
// of n_params floats; the caller swaps it in only when this returns.
void load_checkpoint(Context &ctx, const std::vector<ParamSpec> &specs, int64_t n_params,
                     const std::string &path, float *dst_dev,
                     std::map<std::string, std::string> *meta_out) {
    Fd f;
    f.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) fail(MMH_ERR_OTHER, io_error(path, "open"));
    struct stat stt;
    if (::fstat(f.fd, &stt) != 0) fail(MMH_ERR_OTHER, io_error(path, "stat"));
    const uint64_t size = (uint64_t)stt.st_size;
    if (size < 8) st::parse_fail("the file is shorter than its 8-byte length prefix");
    uint64_t hl = 0;
    read_all(f.fd, &hl, 8, 0, path);
    if (hl > 100000000)
        st::parse_fail("the header claims " + std::to_string(hl) +
                       " bytes, over the format's limit of 100000000");
    if (hl > size - 8)
        st::parse_fail("the header claims " + std::to_string(hl) + " bytes but the file has only " +
                       std::to_string(size - 8) + " after the prefix");
    std::vector<uint8_t> hb((size_t)hl);
    if (hl) read_all(f.fd, hb.data(), (size_t)hl, 8, path);
    st::Header h = st::parse_header(hb.data(), hl, size - 8 - hl);

    // params.rs:87-120
    auto fit = h.metadata.find("format");
    if (fit == h.metadata.end())
        fail(MMH_ERR_OTHER, "checkpoint: the file has no `format` entry, so it is not a "
                            "midman-checkpoint file");
    if (fit->second != "midman-checkpoint")
        fail(MMH_ERR_OTHER, "checkpoint: `format` is `" + fit->second + "`, not `midman-checkpoint`");
    auto vit = h.metadata.find("checkpoint_version");
    if (vit == h.metadata.end()) fail(MMH_ERR_OTHER, "checkpoint: the file has no `checkpoint_version` entry");
    const std::string &vt = vit->second;
    if (vt.empty() || vt.size() > 10 || !std::all_of(vt.begin(), vt.end(), ::isdigit) ||
        std::stoull(vt) > 0xffffffffull)
        fail(MMH_ERR_OTHER, "checkpoint: `checkpoint_version` is `" + vt + "`, not a whole number");
    if (std::stoull(vt) != 1)
        fail(MMH_ERR_OTHER, "checkpoint: version " + vt + " is not supported (this build reads 1)");

    // params.rs:132-190: every parameter present with its shape, nothing else.
    std::map<std::string, const st::Entry *> by_name;
    for (const st::Entry &e : h.entries) by_name[e.name] = &e;
    std::vector<std::string> missing;
    for (const ParamSpec &s : specs) {
        auto it = by_name.find(s.name);
        if (it == by_name.end()) {
            missing.push_back(s.name);
            continue;
        }
        if (it->second->shape != s.shape)
            fail(MMH_ERR_SHAPE, "load_parameters: `" + s.name +
                                    "` has another shape in the checkpoint than in the model");
    }
    auto list = [](const std::vector<std::string> &names) {
        std::string t;
        for (size_t i = 0; i < names.size() && i < 5; ++i) t += (i ? ", `" : "`") + names[i] + "`";
        if (names.size() > 5) t += " and " + std::to_string(names.size() - 5) + " more";
        return t;
    };
    if (!missing.empty())
        fail(MMH_ERR_ARGUMENT, "the checkpoint is missing " + std::to_string(missing.size()) +
                                   " tensor(s) the model needs: " + list(missing));
    std::set<std::string> wanted;
    for (const ParamSpec &s : specs) wanted.insert(s.name);
    std::vector<std::string> extra;
    for (const st::Entry &e : h.entries)
        if (!wanted.count(e.name)) extra.push_back(e.name);
    if (!extra.empty())
        fail(MMH_ERR_ARGUMENT, "the checkpoint holds " + std::to_string(extra.size()) +
                                   " tensor(s) the model does not have: " + list(extra));
    int64_t total = 0;
    for (const ParamSpec &s : specs) total += s.numel;
    if (total != n_params) fail(MMH_ERR_OTHER, "checkpoint: parameter layout mismatch");

    // Stream the data section in file order straight into the device buffer.
    std::map<std::string, const ParamSpec *> spec_of;
    for (const ParamSpec &s : specs) spec_of[s.name] = &s;
    Staging stg;
    int slot = 0;
    const uint64_t data0 = 8 + hl;
    for (const st::Entry &e : h.entries) {
        const ParamSpec *s = spec_of[e.name];
        char *dst = reinterpret_cast<char *>(dst_dev + s->offset);
        uint64_t left = e.end - e.begin, at = data0 + e.begin;
        while (left) {
            const size_t n = (size_t)std::min<uint64_t>(left, Staging::kChunk);
            void *buf = stg.acquire(slot);
            read_all(f.fd, buf, n, at, path);
            check_hip(hipMemcpyAsync(dst, buf, n, hipMemcpyHostToDevice, ctx.stream),
                      "checkpoint upload");
            stg.issued(slot, ctx.stream);
            slot ^= 1;
            dst += n;
            at += n;
            left -= n;
        }
    }
    check_hip(hipStreamSynchronize(ctx.stream), "checkpoint upload sync");
    if (meta_out) *meta_out = h.metadata;
}

}  // namespace mmh
