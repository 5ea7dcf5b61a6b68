// Token shards (midman-data/src/shard.rs), training sequences and the seeded
// batcher (src/batch.rs), and their C-ABI. Host code: the shard is a file
// format and the batcher an order over it; the ids it hands out go to the
// device through the model's staging (model.hip).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <mutex>

#include "mmh_data.h"
#include "mmh_error.h"
#include "mmh_host.h"

namespace mmh {

namespace {

constexpr char kMagic[8] = {'M', 'M', 'T', 'O', 'K', 'E', 'N', 'S'};
constexpr uint32_t kVersion = 1;             // shard.rs:16
constexpr uint64_t kHeader = 8 + 4 * 4 + 8;  // shard.rs:22
constexpr uint64_t kChecksum = 32;           // shard.rs:23

[[noreturn]] void invalid(const std::string &m) {
    fail(MMH_ERR_ARGUMENT, "invalid argument: " + m);
}
[[noreturn]] void parse_error(const std::string &m) {
    fail(MMH_ERR_OTHER, "failed to parse token shard: " + m);
}
[[noreturn]] void io_error(const std::string &path, int err) {
    fail(MMH_ERR_OTHER, "I/O error: " + path + ": " + std::strerror(err));
}

std::string below_message(uint32_t token, uint64_t at, uint32_t vocab) {
    return "token " + std::to_string(token) + " at position " + std::to_string(at) +
           " is not below the vocabulary size " + std::to_string(vocab);
}

void put32(uint8_t *p, uint32_t v) {
    for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i));
}
uint32_t get32(const uint8_t *p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}

struct Fd {
    int fd = -1;
    ~Fd() {
        if (fd >= 0) ::close(fd);
    }
};

// The permutation of pass `epoch` (batch.rs:244-248): the Fisher-Yates
// shuffle of 0..n (rng.rs:108-113) by Rng::seed_from_u64(seed).fork(epoch).
void permutation(uint64_t n, uint64_t seed, uint64_t epoch, std::vector<uint64_t> &order) {
    order.resize(n);
    for (uint64_t i = 0; i < n; ++i) order[i] = i;
    HostRng base = HostRng::seed(seed);
    HostRng r = base.fork(epoch);
    for (uint64_t i = n; i-- > 1;) std::swap(order[i], order[r.below(i + 1)]);
}

}  // namespace

TokenShard TokenShard::make(uint32_t vocab, uint32_t eos, std::vector<uint32_t> tokens) {
    // shard.rs:66-83
    if (vocab == 0) invalid("the vocabulary size is 0");
    if (eos >= vocab)
        invalid("the end-of-text id " + std::to_string(eos) +
                " is not below the vocabulary size " + std::to_string(vocab));
    for (size_t i = 0; i < tokens.size(); ++i)
        if (tokens[i] >= vocab) invalid(below_message(tokens[i], i, vocab));
    TokenShard s;
    s.vocab = vocab;
    s.eos = eos;
    s.tokens = std::move(tokens);
    return s;
}

uint64_t TokenShard::file_bytes() const { return kHeader + tokens.size() * width() + kChecksum; }

void TokenShard::to_bytes(uint8_t *out) const {
    // shard.rs:112-135: magic, version, width, vocab, eos, count, ids, SHA-256.
    const uint32_t w = width();
    std::memcpy(out, kMagic, 8);
    put32(out + 8, kVersion);
    put32(out + 12, w);
    put32(out + 16, vocab);
    put32(out + 20, eos);
    const uint64_t n = tokens.size();
    for (int i = 0; i < 8; ++i) out[24 + i] = (uint8_t)(n >> (8 * i));
    uint8_t *p = out + kHeader;
    if (w == 2) {
        for (uint64_t i = 0; i < n; ++i) {
            p[2 * i] = (uint8_t)tokens[i];
            p[2 * i + 1] = (uint8_t)(tokens[i] >> 8);
        }
    } else {
        for (uint64_t i = 0; i < n; ++i) put32(p + 4 * i, tokens[i]);
    }
    const uint64_t body = kHeader + n * w;
    sha256(out, body, out + body);
}

TokenShard TokenShard::from_bytes(const uint8_t *b, uint64_t len) {
    // shard.rs:146-223, the checks in the same order and with the same reasons
    if (len < kHeader + kChecksum)
        parse_error(std::to_string(len) + " bytes is shorter than the smallest shard, " +
                    std::to_string(kHeader + kChecksum));
    if (std::memcmp(b, kMagic, 8) != 0) parse_error("the file does not start with `MMTOKENS`");
    const uint32_t version = get32(b + 8);
    if (version != kVersion)
        fail(MMH_ERR_OTHER, "token shard version " + std::to_string(version) +
                                " is not supported (this build supports " +
                                std::to_string(kVersion) + ")");
    const uint32_t width = get32(b + 12), vocab = get32(b + 16), eos = get32(b + 20);
    uint64_t count = 0;
    for (int i = 0; i < 8; ++i) count |= (uint64_t)b[24 + i] << (8 * i);
    if (vocab == 0) parse_error("the vocabulary size is 0");
    const uint32_t want = vocab <= 65536 ? 2 : 4;
    if (width != want)
        parse_error("token width " + std::to_string(width) +
                    " is not the one for a vocabulary of " + std::to_string(vocab) + " ids (" +
                    std::to_string(want) + ")");
    if (eos >= vocab)
        parse_error("the end-of-text id " + std::to_string(eos) +
                    " is not below the vocabulary size " + std::to_string(vocab));
    // count * width + header + checksum, without overflow
    const bool fits = count <= (UINT64_MAX - kHeader - kChecksum) / width &&
                      count * width + kHeader + kChecksum == len;
    if (!fits)
        parse_error(std::to_string(count) + " tokens of " + std::to_string(width) +
                    " bytes do not make a file of " + std::to_string(len) + " bytes");
    const uint64_t body = len - kChecksum;
    uint8_t digest[32];
    sha256(b, body, digest);
    if (std::memcmp(digest, b + body, 32) != 0)
        parse_error("the checksum does not match: the file is damaged");
    TokenShard s;
    s.vocab = vocab;
    s.eos = eos;
    s.tokens.resize(count);
    const uint8_t *p = b + kHeader;
    if (width == 2) {
        for (uint64_t i = 0; i < count; ++i)
            s.tokens[i] = (uint32_t)p[2 * i] | (uint32_t)p[2 * i + 1] << 8;
    } else {
        for (uint64_t i = 0; i < count; ++i) s.tokens[i] = get32(p + 4 * i);
    }
    for (uint64_t i = 0; i < count; ++i)
        if (s.tokens[i] >= vocab) parse_error(below_message(s.tokens[i], i, vocab));
    return s;
}

void TokenShard::save(const std::string &path) const {
    // shard.rs:233-254: write <path>.tmp, flush it to disk, rename it over
    // path; on failure remove the temporary file.
    const std::string tmp = path + ".tmp";
    std::vector<uint8_t> bytes(file_bytes());
    to_bytes(bytes.data());
    int err = 0;
    {
        Fd f;
        f.fd = ::open(tmp.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
        if (f.fd < 0) io_error(path, errno);
        size_t done = 0;
        while (done < bytes.size() && !err) {
            const ssize_t w = ::write(f.fd, bytes.data() + done, bytes.size() - done);
            if (w < 0) {
                if (errno != EINTR) err = errno;
            } else {
                done += (size_t)w;
            }
        }
        if (!err && ::fsync(f.fd) != 0) err = errno;
        if (!err) {
            const int fd = f.fd;
            f.fd = -1;
            if (::close(fd) != 0) err = errno;
        }
    }
    if (!err && ::rename(tmp.c_str(), path.c_str()) != 0) err = errno;
    if (err) {
        ::unlink(tmp.c_str());
        io_error(path, err);
    }
}

TokenShard TokenShard::load(const std::string &path) {
    // shard.rs:256-260: read the whole file, then from_bytes.
    Fd f;
    f.fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (f.fd < 0) io_error(path, errno);
    struct stat st;
    if (::fstat(f.fd, &st) != 0) io_error(path, errno);
    std::vector<uint8_t> bytes((size_t)st.st_size);
    size_t done = 0;
    while (done < bytes.size()) {
        const ssize_t r = ::read(f.fd, bytes.data() + done, bytes.size() - done);
        if (r < 0) {
            if (errno == EINTR) continue;
            io_error(path, errno);
        }
        if (r == 0) break;
        done += (size_t)r;
    }
    bytes.resize(done);
    return from_bytes(bytes.data(), bytes.size());
}

std::shared_ptr<const Sequences> Sequences::make(
    std::vector<std::shared_ptr<const TokenShard>> shards, uint64_t seq_len) {
    // batch.rs:45-70
    if (seq_len == 0) invalid("a sequence must have at least one token");
    for (size_t n = 0; n < shards.size(); ++n) {
        const TokenShard &s = *shards[n], &f = *shards[0];
        if (s.vocab != f.vocab || s.eos != f.eos)
            invalid("shard " + std::to_string(n) + " has vocabulary size " +
                    std::to_string(s.vocab) + " and end-of-text " + std::to_string(s.eos) +
                    ", but shard 0 has " + std::to_string(f.vocab) + " and " +
                    std::to_string(f.eos));
    }
    auto q = std::make_shared<Sequences>();
    q->seq_len = seq_len;
    uint64_t total = 0;
    for (const auto &s : shards) {
        if (s->tokens.size() > seq_len) total += (s->tokens.size() - 1) / seq_len;
        q->ends.push_back(total);
    }
    q->shards = std::move(shards);
    return q;
}

const uint32_t *Sequences::window(uint64_t i) const {
    // batch.rs:96-104: the first shard whose end is past i
    if (i >= len()) return nullptr;
    const size_t s = (size_t)(std::upper_bound(ends.begin(), ends.end(), i) - ends.begin());
    const uint64_t before = s ? ends[s - 1] : 0;
    return shards[s]->tokens.data() + (i - before) * seq_len;
}

std::unique_ptr<Batcher> Batcher::make(std::shared_ptr<const Sequences> data, uint64_t batch,
                                       uint64_t seed) {
    // batch.rs:161-172
    if (batch == 0) invalid("a batch must have at least one sequence");
    if (data->len() < batch)
        invalid("there are " + std::to_string(data->len()) +
                " sequences, fewer than one batch of " + std::to_string(batch));
    auto b = std::make_unique<Batcher>();
    b->data = std::move(data);
    b->batch = batch;
    b->seed = seed;
    permutation(b->data->len(), seed, 0, b->order);
    return b;
}

void Batcher::seek(uint64_t e, uint64_t done) {
    // batch.rs:196-208
    if (done > batches_per_epoch())
        invalid(std::to_string(done) + " batches done is more than the " +
                std::to_string(batches_per_epoch()) + " in a pass");
    if (e != epoch) permutation(data->len(), seed, e, order);
    epoch = e;
    position = done;
}

void Batcher::next_batch(uint32_t *inputs, uint32_t *targets, uint64_t *epoch_out,
                   uint64_t *index_out) {
    // batch.rs:211-239
    if (position == batches_per_epoch()) {
        ++epoch;
        position = 0;
        permutation(data->len(), seed, epoch, order);
    }
    const uint64_t seq = data->seq_len;
    for (uint64_t r = 0; r < batch; ++r) {
        const uint32_t *w = data->window(order[position * batch + r]);
        std::memcpy(inputs + r * seq, w, seq * 4);
        std::memcpy(targets + r * seq, w + 1, seq * 4);
    }
    if (epoch_out) *epoch_out = epoch;
    if (index_out) *index_out = position;
    ++position;
}

// ---- handle registries -------------------------------------------------------

namespace {

template <class T>
struct Registry {
    std::mutex mu;
    std::vector<std::shared_ptr<T>> items;  // handle = index + 1
    const char *what;

    explicit Registry(const char *w) : what(w) {}
    std::shared_ptr<T> get(mmh_handle h) {
        std::lock_guard<std::mutex> lock(mu);
        if (h <= 0 || (size_t)h > items.size() || !items[(size_t)h - 1])
            fail(MMH_ERR_ARGUMENT, std::string("invalid ") + what + " handle " +
                                       std::to_string(h));
        return items[(size_t)h - 1];
    }
    mmh_handle add(std::shared_ptr<T> t) {
        std::lock_guard<std::mutex> lock(mu);
        items.push_back(std::move(t));
        return (mmh_handle)items.size();
    }
    void remove(mmh_handle h) {
        std::lock_guard<std::mutex> lock(mu);
        if (h <= 0 || (size_t)h > items.size() || !items[(size_t)h - 1])
            fail(MMH_ERR_ARGUMENT, std::string("invalid ") + what + " handle " +
                                       std::to_string(h));
        items[(size_t)h - 1].reset();
    }
};

Registry<const TokenShard> g_shards("token shard");
Registry<const Sequences> g_sequences("sequences");
Registry<Batcher> g_batchers("batcher");
Registry<Sha256> g_hashers("sha256");

template <class T>
void need(const T *p, const char *name) {
    if (!p) fail(MMH_ERR_ARGUMENT, std::string(name) + " is a null pointer");
}

std::string path_of(const char *path) {
    if (!path) fail(MMH_ERR_ARGUMENT, "path is a null pointer");
    return std::string(path);
}

}  // namespace

std::shared_ptr<const Sequences> sequences_of(mmh_handle h) { return g_sequences.get(h); }

Batcher &batcher_of(mmh_handle h) { return *g_batchers.get(h); }

}  // namespace mmh

using namespace mmh;

extern "C" {

int32_t mmh_sha256(const uint8_t *data, uint64_t len, uint8_t *digest) {
    return guard([&] {
        if (len) need(data, "data");
        need(digest, "digest");
        sha256(data, (size_t)len, digest);
        return MMH_OK;
    });
}

int32_t mmh_sha256_new(mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        *out = g_hashers.add(std::make_shared<Sha256>());
        return MMH_OK;
    });
}

int32_t mmh_sha256_update(mmh_handle h, const uint8_t *data, uint64_t len) {
    return guard([&] {
        if (len) need(data, "data");
        g_hashers.get(h)->update(data, (size_t)len);
        return MMH_OK;
    });
}

int32_t mmh_sha256_finalize(mmh_handle h, uint8_t *digest) {
    return guard([&] {
        need(digest, "digest");
        g_hashers.get(h)->finalize(digest);
        g_hashers.remove(h);
        return MMH_OK;
    });
}

int32_t mmh_sha256_select(int32_t mode, int32_t *in_use) {
    return guard([&] {
        if (mode < 0 || mode > 2) fail(MMH_ERR_ARGUMENT, "sha256 mode must be 0, 1 or 2");
        const int v = sha256_select(mode);
        if (in_use) *in_use = v;
        return MMH_OK;
    });
}

int32_t mmh_shard_create(uint32_t vocab_size, uint32_t eos, const uint32_t *tokens, uint64_t n,
                         mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        if (n) need(tokens, "tokens");
        std::vector<uint32_t> t(tokens, tokens + n);
        *out = g_shards.add(std::make_shared<TokenShard>(TokenShard::make(vocab_size, eos,
                                                                          std::move(t))));
        return MMH_OK;
    });
}

int32_t mmh_shard_parse(const uint8_t *bytes, uint64_t len, mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        if (len) need(bytes, "bytes");
        static const uint8_t empty = 0;
        *out = g_shards.add(
            std::make_shared<TokenShard>(TokenShard::from_bytes(len ? bytes : &empty, len)));
        return MMH_OK;
    });
}

int32_t mmh_shard_load(const char *path, mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        *out = g_shards.add(std::make_shared<TokenShard>(TokenShard::load(path_of(path))));
        return MMH_OK;
    });
}

int32_t mmh_shard_save(mmh_handle shard, const char *path) {
    return guard([&] {
        g_shards.get(shard)->save(path_of(path));
        return MMH_OK;
    });
}

int32_t mmh_shard_info(mmh_handle shard, uint32_t *vocab_size, uint32_t *eos, uint64_t *len,
                       uint32_t *token_width, uint64_t *file_bytes) {
    return guard([&] {
        auto s = g_shards.get(shard);
        if (vocab_size) *vocab_size = s->vocab;
        if (eos) *eos = s->eos;
        if (len) *len = s->tokens.size();
        if (token_width) *token_width = s->width();
        if (file_bytes) *file_bytes = s->file_bytes();
        return MMH_OK;
    });
}

int32_t mmh_shard_tokens(mmh_handle shard, uint32_t *out, uint64_t n) {
    return guard([&] {
        auto s = g_shards.get(shard);
        if (n != s->tokens.size())
            fail(MMH_ERR_SHAPE, "the shard holds " + std::to_string(s->tokens.size()) +
                                    " tokens, not " + std::to_string(n));
        if (n) {
            need(out, "out");
            std::memcpy(out, s->tokens.data(), n * 4);
        }
        return MMH_OK;
    });
}

int32_t mmh_shard_serialize(mmh_handle shard, uint8_t *out, uint64_t cap, uint64_t *len) {
    return guard([&] {
        auto s = g_shards.get(shard);
        const uint64_t n = s->file_bytes();
        if (len) *len = n;
        if (!out) return MMH_OK;  // size query
        if (cap < n)
            fail(MMH_ERR_SHAPE, "the file takes " + std::to_string(n) + " bytes, the buffer " +
                                    std::to_string(cap));
        s->to_bytes(out);
        return MMH_OK;
    });
}

int32_t mmh_shard_destroy(mmh_handle shard) {
    return guard([&] {
        g_shards.remove(shard);
        return MMH_OK;
    });
}

int32_t mmh_sequences_create(const mmh_handle *shards, int64_t n_shards, uint64_t seq_len,
                             mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        if (n_shards < 0) fail(MMH_ERR_ARGUMENT, "n_shards is negative");
        if (n_shards) need(shards, "shards");
        std::vector<std::shared_ptr<const TokenShard>> v;
        for (int64_t i = 0; i < n_shards; ++i) v.push_back(g_shards.get(shards[i]));
        *out = g_sequences.add(Sequences::make(std::move(v), seq_len));
        return MMH_OK;
    });
}

int32_t mmh_sequences_info(mmh_handle seqs, uint64_t *len, uint64_t *seq_len,
                           int64_t *vocab_size) {
    return guard([&] {
        auto q = g_sequences.get(seqs);
        if (len) *len = q->len();
        if (seq_len) *seq_len = q->seq_len;
        if (vocab_size) *vocab_size = q->vocab();
        return MMH_OK;
    });
}

int32_t mmh_sequences_window(mmh_handle seqs, uint64_t index, uint32_t *out) {
    return guard([&] {
        need(out, "out");
        auto q = g_sequences.get(seqs);
        const uint32_t *w = q->window(index);
        if (!w)
            fail(MMH_ERR_INDEX, "sequences index " + std::to_string(index) +
                                    " is out of range (must be below " +
                                    std::to_string(q->len()) + ")");
        std::memcpy(out, w, (q->seq_len + 1) * 4);
        return MMH_OK;
    });
}

int32_t mmh_sequences_destroy(mmh_handle seqs) {
    return guard([&] {
        g_sequences.remove(seqs);
        return MMH_OK;
    });
}

int32_t mmh_batcher_create(mmh_handle seqs, uint64_t batch_size, uint64_t seed,
                           mmh_handle *out) {
    return guard([&] {
        need(out, "out");
        *out = g_batchers.add(
            std::shared_ptr<Batcher>(Batcher::make(g_sequences.get(seqs), batch_size, seed)));
        return MMH_OK;
    });
}

int32_t mmh_batcher_info(mmh_handle batcher, uint64_t *batches_per_epoch, uint64_t *epoch,
                         uint64_t *position, uint64_t *batch_size, uint64_t *seq_len) {
    return guard([&] {
        auto b = g_batchers.get(batcher);
        if (batches_per_epoch) *batches_per_epoch = b->batches_per_epoch();
        if (epoch) *epoch = b->epoch;
        if (position) *position = b->position;
        if (batch_size) *batch_size = b->batch;
        if (seq_len) *seq_len = b->data->seq_len;
        return MMH_OK;
    });
}

int32_t mmh_batcher_seek(mmh_handle batcher, uint64_t epoch, uint64_t batches_done) {
    return guard([&] {
        g_batchers.get(batcher)->seek(epoch, batches_done);
        return MMH_OK;
    });
}

int32_t mmh_batcher_next(mmh_handle batcher, uint32_t *inputs, uint32_t *targets,
                         uint64_t *epoch, uint64_t *index) {
    return guard([&] {
        need(inputs, "inputs");
        need(targets, "targets");
        g_batchers.get(batcher)->next_batch(inputs, targets, epoch, index);
        return MMH_OK;
    });
}

int32_t mmh_batcher_destroy(mmh_handle batcher) {
    return guard([&] {
        g_batchers.remove(batcher);
        return MMH_OK;
    });
}

}  // extern "C"
