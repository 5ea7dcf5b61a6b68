// Token shards, training sequences and the seeded batcher (midman-data
// src/shard.rs, src/batch.rs), host side. data.hip implements them and their
// C-ABI; model.hip feeds batches from them to the device training step.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "../../include/midman_hip.h"

namespace mmh {

// shard.rs:53-260: a run of token ids for one vocabulary.
struct TokenShard {
    uint32_t vocab = 0;
    uint32_t eos = 0;
    std::vector<uint32_t> tokens;

    // TokenShard::new: MMH_ERR_ARGUMENT for an empty vocabulary, eos or a
    // token not below it.
    static TokenShard make(uint32_t vocab, uint32_t eos, std::vector<uint32_t> tokens);
    uint32_t width() const { return vocab <= 65536 ? 2 : 4; }
    uint64_t file_bytes() const;
    void to_bytes(uint8_t *out) const;  // file_bytes() bytes
    static TokenShard from_bytes(const uint8_t *bytes, uint64_t len);
    void save(const std::string &path) const;
    static TokenShard load(const std::string &path);
};

// batch.rs:31-104: windows of seq_len + 1 tokens every seq_len tokens of
// each shard, never across shards.
struct Sequences {
    std::vector<std::shared_ptr<const TokenShard>> shards;
    uint64_t seq_len = 0;
    std::vector<uint64_t> ends;  // sequences in this shard and all before it

    static std::shared_ptr<const Sequences> make(
        std::vector<std::shared_ptr<const TokenShard>> shards, uint64_t seq_len);
    uint64_t len() const { return ends.empty() ? 0 : ends.back(); }
    // The window of sequence i (seq_len + 1 ids), or nullptr.
    const uint32_t *window(uint64_t i) const;
    // The shards' vocabulary, or -1 with no shards.
    int64_t vocab() const { return shards.empty() ? -1 : (int64_t)shards[0]->vocab; }
};

// batch.rs:144-240: batches of `batch` sequences, each pass over the data in
// the order permutation(len, seed, epoch).
struct Batcher {
    std::shared_ptr<const Sequences> data;
    uint64_t batch = 0, seed = 0, epoch = 0;
    uint64_t position = 0;  // batches of this epoch handed out
    std::vector<uint64_t> order;

    static std::unique_ptr<Batcher> make(std::shared_ptr<const Sequences> data, uint64_t batch,
                                         uint64_t seed);
    uint64_t batches_per_epoch() const { return data->len() / batch; }
    void seek(uint64_t epoch, uint64_t done);
    // next_batch: batch * seq_len inputs and targets, row after row; the
    // batch's epoch and index.
    void next_batch(uint32_t *inputs, uint32_t *targets, uint64_t *epoch_out,
                    uint64_t *index_out);
};

std::shared_ptr<const Sequences> sequences_of(mmh_handle h);
Batcher &batcher_of(mmh_handle h);

}  // namespace mmh
