"""Token shards, sequences and the batcher through the library's C ABI (host
code, no GPU), against the reference's own tests (midman-data src/shard.rs
:268-456, src/batch.rs:250-420, tests/reference_vectors.rs) and the oracle.

The SHA-256 vectors are the reference's fixture
(crates/midman-data/tests/fixtures/sha256_vectors.txt), with the messages
rebuilt from the formula reference_vectors.rs:13-15 states.
"""
import ctypes
import hashlib
import math
import os
import struct
import tempfile

import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as mo

U64P = ctypes.POINTER(ctypes.c_uint64)
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def vectors():
    out = []
    with open(os.path.join(GOLDEN, "sha256_vectors.txt")) as f:
        for line in f:
            n, digest = line.split()
            out.append((int(n), digest))
    return out


def message(n):
    return bytes((31 * j + 7 * n + 5) % 256 for j in range(n))


# ---- SHA-256 --------------------------------------------------------------------------

def test_the_fixture_covers_every_small_length_and_some_large_ones():
    lengths = [n for n, _ in vectors()]
    assert set(range(301)) <= set(lengths) and 100003 in lengths and len(lengths) == 309


def test_the_fixture_is_hashlibs_sha256():
    """The fixture and the message formula pin each other against a textbook
    implementation (Python's hashlib)."""
    for n, digest in vectors():
        assert hashlib.sha256(message(n)).hexdigest() == digest, n


@pytest.mark.parametrize("mode", [1, 2])
def test_every_vector_matches_in_one_shot_and_in_pieces(mode):
    used = mh.sha256_select(mode)
    if mode == 2 and used != 2:
        mh.sha256_select(0)
        pytest.skip("this CPU has no SHA extensions")
    try:
        for n, digest in vectors():
            data = message(n)
            assert mh.sha256(data).hex() == digest, f"length {n}"
            for piece in (1, 3, 63, 64, 65, 1000):
                if piece == 1 and n > 4096:
                    continue
                h = mh.Sha256()
                for a in range(0, n, piece):
                    h.update(data[a:a + piece])
                assert h.finalize().hex() == digest, f"length {n}, pieces of {piece}"
    finally:
        mh.sha256_select(0)


def test_both_paths_agree_on_large_random_inputs():
    r = np.random.default_rng(1)
    data = r.integers(0, 256, 3 << 20, dtype=np.uint8).tobytes()
    want = hashlib.sha256(data).digest()
    for mode in (1, 2):
        mh.sha256_select(mode)
        assert mh.sha256(data) == want
    mh.sha256_select(0)


# ---- the shard file -------------------------------------------------------------------

def shard(vocab, tokens, eos=0):
    return mh.TokenShard(vocab, eos, tokens)


def craft(version, width, vocab, eos, count, payload):
    """File contents with every header field given and a correct checksum
    (shard.rs:274-285)."""
    body = b"MMTOKENS" + struct.pack("<IIIIQ", version, width, vocab, eos, count) + bytes(payload)
    return body + hashlib.sha256(body).digest()


def parse_error(data):
    with pytest.raises(mh.MidmanError) as e:
        mh.TokenShard.from_bytes(data)
    return e.value.message


def test_the_file_has_exactly_this_layout():
    b = mh.TokenShard(300, 256, [1, 2, 3, 256]).to_bytes()
    assert b[:-32].hex() == ("4d4d544f4b454e53" "01000000" "02000000" "2c010000" "00010000"
                             "0400000000000000" "0100020003000001")
    assert b[-32:] == hashlib.sha256(b[:-32]).digest()
    assert len(b) == 32 + 8 + 32
    # the shard.rs:46-50 doc example
    s = mh.TokenShard(300, 256, [5, 6, 7, 256, 9, 256])
    assert mh.TokenShard.from_bytes(s.to_bytes()) == s
    assert len(s.to_bytes()) == 32 + 6 * 2 + 32


def test_four_byte_ids_are_used_above_65536():
    b = shard(65537, [65536, 7]).to_bytes()
    assert b[12:16] == struct.pack("<I", 4) and len(b) == 32 + 8 + 32
    assert b[32:36] == struct.pack("<I", 65536)
    b = shard(65536, [65535, 7]).to_bytes()
    assert b[12:16] == struct.pack("<I", 2) and len(b) == 32 + 4 + 32
    assert b[32:34] == struct.pack("<H", 65535)


@pytest.mark.parametrize("vocab,tokens", [
    (256, [0, 255, 1, 2, 3]), (65536, [0, 65535, 40000]), (65537, [0, 65536, 40000]),
    (4_000_000_000, [0, 3_999_999_999, 1_234_567_890]), (300, [])])
def test_round_trips_in_both_widths_and_empty(vocab, tokens):
    original = shard(vocab, tokens)
    again = mh.TokenShard.from_bytes(original.to_bytes())
    assert again == original
    assert again.tokens().tolist() == tokens
    assert (again.vocab_size(), again.eos(), len(again)) == (vocab, 0, len(tokens))
    assert again.is_empty() == (not tokens)


def test_construction_checks_the_vocabulary():
    with pytest.raises(mh.ArgumentError):
        mh.TokenShard(0, 0, [])
    with pytest.raises(mh.ArgumentError):
        mh.TokenShard(10, 10, [])
    with pytest.raises(mh.ArgumentError) as e:
        mh.TokenShard(10, 3, [1, 2, 10, 4])
    assert "token 10 at position 2" in e.value.message
    mh.TokenShard(10, 9, [9, 0])


def test_the_reader_refuses_a_wrong_header_each_with_its_reason():
    good = craft(1, 2, 300, 256, 2, [1, 0, 2, 0])
    mh.TokenShard.from_bytes(good)
    bad = b"X" + good[1:]
    assert "MMTOKENS" in parse_error(bad)
    for version in (2, 0):
        msg = parse_error(craft(version, 2, 300, 256, 2, [1, 0, 2, 0]))
        assert f"version {version} is not supported (this build supports 1)" in msg
    for width in (0, 1, 3, 4, 8):
        msg = parse_error(craft(1, width, 300, 256, 2, [1, 0, 2, 0, 0, 0, 0, 0]))
        assert "token width" in msg, (width, msg)
    assert "token width" in parse_error(craft(1, 2, 65537, 0, 1, [1, 0]))
    assert "vocabulary size is 0" in parse_error(craft(1, 2, 0, 0, 0, []))
    assert "end-of-text" in parse_error(craft(1, 2, 300, 300, 0, []))
    mh.TokenShard.from_bytes(craft(1, 2, 300, 299, 0, []))


def test_the_reader_refuses_a_wrong_length_for_every_cut_and_extension():
    good = shard(300, [1, 2, 3, 4, 5]).to_bytes()
    for cut in range(len(good)):
        with pytest.raises(mh.MidmanError):
            mh.TokenShard.from_bytes(good[:cut])
    assert "do not make a file" in parse_error(good + b"\0")
    assert "3 tokens" in parse_error(craft(1, 2, 300, 0, 3, [1, 0, 2, 0]))
    for count in (2**64 - 1, (2**64 - 1) // 2, 1 << 62):
        assert "do not make a file" in parse_error(craft(1, 2, 300, 0, count, []))


def test_the_reader_refuses_damage_anywhere_in_the_file():
    good = shard(300, [1, 2, 3, 4, 5]).to_bytes()
    for index in range(len(good)):
        for bit in (0, 7):
            bad = bytearray(good)
            bad[index] ^= 1 << bit
            with pytest.raises(mh.MidmanError):
                mh.TokenShard.from_bytes(bytes(bad))
    bad = bytearray(good)
    bad[34] ^= 0x10
    assert "checksum" in parse_error(bytes(bad))


def test_a_token_outside_the_vocabulary_is_refused_even_with_a_valid_checksum():
    assert "token 300 at position 1" in parse_error(craft(1, 2, 300, 0, 3, [1, 0, 44, 1, 2, 0]))


def test_save_and_load_round_trip_and_replace_atomically():
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "a.mmtokens")
        first = shard(300, [1, 2, 3])
        first.save(path)
        assert mh.TokenShard.load(path) == first
        second = shard(300, [4, 5, 6, 7])
        second.save(path)
        assert mh.TokenShard.load(path) == second
        assert not os.path.exists(path + ".tmp")
        assert open(path, "rb").read() == second.to_bytes()
        with pytest.raises(mh.MidmanError) as e:
            first.save(os.path.join(d, "nope", "b.mmtokens"))
        assert "I/O error" in e.value.message and "nope" in e.value.message
        with pytest.raises(mh.MidmanError) as e:
            mh.TokenShard.load(os.path.join(d, "absent.mmtokens"))
        assert "I/O error" in e.value.message and "absent.mmtokens" in e.value.message
        data = bytearray(open(path, "rb").read())
        data[40] ^= 1
        open(path, "wb").write(bytes(data))
        with pytest.raises(mh.MidmanError) as e:
            mh.TokenShard.load(path)
        assert e.value.message.startswith("failed to parse token shard")


@pytest.mark.parametrize("vocab", [2, 300, 65536, 65537, 4_000_000_000])
def test_files_are_the_oracles_bytes_and_parse_like_it(vocab):
    r = np.random.default_rng(vocab % 1000)
    for n in (0, 1, 7, 1000):
        t = r.integers(0, vocab, n, dtype=np.uint64).astype(np.uint32)
        eos = int(r.integers(0, vocab))
        b = mh.TokenShard(vocab, eos, t).to_bytes()
        assert b == mo.shard_bytes(vocab, eos, t)
        v, e, got = mo.shard_parse(b)
        assert (v, e) == (vocab, eos) and np.array_equal(got, t)


def test_the_oracle_refuses_what_the_library_refuses():
    good = mo.shard_bytes(300, 0, [1, 2, 3, 4, 5])
    cases = [good[:10], b"X" + good[1:], craft(2, 2, 300, 0, 0, []), craft(1, 4, 300, 0, 0, []),
             craft(1, 2, 300, 300, 0, []), good + b"\0", craft(1, 2, 300, 0, 3, [1, 0, 2, 0]),
             good[:40] + bytes([good[40] ^ 1]) + good[41:],
             craft(1, 2, 300, 0, 3, [1, 0, 44, 1, 2, 0])]
    keys = ["shorter", "MMTOKENS", "version 2", "token width", "end-of-text",
            "do not make a file", "3 tokens", "checksum", "token 300 at position 1"]
    for data, key in zip(cases, keys):
        with pytest.raises(ValueError) as e:
            mo.shard_parse(data)
        assert key in str(e.value)
        assert key in parse_error(data)


# ---- sequences ------------------------------------------------------------------------

def stream(n, vocab):
    return mh.TokenShard(vocab, vocab - 1, [t % (vocab - 1) for t in range(n)])


def sequences(tokens, seq_len):
    return mh.Sequences([stream(tokens, 1000)], seq_len)


def test_windows_start_every_seq_len_tokens_and_overlap_by_one():
    s = sequences(21, 4)
    assert len(s) == 5
    for i in range(5):
        assert s.window(i).tolist() == list(range(4 * i, 4 * i + 5))
    assert s.window(5) is None
    assert s.seq_len() == 4 and s.vocab_size() == 1000
    # the batch.rs:22-28 doc example
    q = mh.Sequences([mh.TokenShard(100, 99, list(range(11)))], 4)
    assert len(q) == 2 and q.window(0).tolist() == [0, 1, 2, 3, 4]
    assert q.window(1).tolist() == [4, 5, 6, 7, 8]


def test_every_token_is_a_target_exactly_once_and_the_remainder_is_dropped():
    s = sequences(23, 4)
    assert len(s) == 5
    targets = np.concatenate([s.window(i)[1:] for i in range(len(s))])
    assert targets.tolist() == list(range(1, 21))


def test_the_count_is_exact_at_the_edges():
    for tokens, expected in [(0, 0), (1, 0), (4, 0), (5, 1), (8, 1), (9, 2), (13, 3)]:
        assert len(sequences(tokens, 4)) == expected, tokens
    assert sequences(4, 4).is_empty()
    assert len(sequences(5, 4).window(0)) == 5
    assert len(sequences(10, 1)) == 9


def test_windows_never_cross_from_one_shard_to_the_next():
    shards = [mh.TokenShard(1000, 999, list(range(a, b)))
              for a, b in [(0, 10), (100, 109), (200, 203), (300, 306)]]
    s = mh.Sequences(shards, 4)
    assert len(s) == 5
    assert [s.window(i).tolist() for i in range(5)] == [
        [0, 1, 2, 3, 4], [4, 5, 6, 7, 8], [100, 101, 102, 103, 104],
        [104, 105, 106, 107, 108], [300, 301, 302, 303, 304]]


def test_no_shards_and_bad_arguments():
    none = mh.Sequences([], 4)
    assert none.is_empty() and none.vocab_size() is None and none.window(0) is None
    with pytest.raises(mh.ArgumentError):
        mh.Sequences([stream(10, 100)], 0)
    other_vocab = mh.TokenShard(200, 199, [1] * 10)
    other_eos = mh.TokenShard(100, 98, [1] * 10)
    with pytest.raises(mh.ArgumentError) as e:
        mh.Sequences([stream(10, 100), other_vocab], 4)
    assert "shard 1" in e.value.message
    with pytest.raises(mh.ArgumentError):
        mh.Sequences([stream(10, 100), other_eos], 4)


def test_a_sequence_outlives_the_shard_handles():
    shards = [stream(50, 1000), stream(30, 1000)]
    s = mh.Sequences(shards, 8)
    want = [s.window(i).tolist() for i in range(len(s))]
    for sh in shards:
        sh.close()
    assert [s.window(i).tolist() for i in range(len(s))] == want


def test_windows_match_the_oracle():
    r = np.random.default_rng(5)
    toks = [r.integers(0, 500, n).astype(np.uint32) for n in (0, 3, 17, 100, 64, 65, 9)]
    for seq_len in (1, 4, 8, 16, 64):
        s = mh.Sequences([mh.TokenShard(500, 0, t) for t in toks], seq_len)
        wins = mo.sequence_windows(toks, seq_len)
        assert len(s) == len(wins)
        for i, (sh, a) in enumerate(wins):
            assert np.array_equal(s.window(i), toks[sh][a:a + seq_len + 1])


# ---- the batcher ----------------------------------------------------------------------

def test_batches_hold_inputs_and_the_next_tokens_as_targets():
    b = mh.Batcher(sequences(101, 5), 4, 1)
    for _ in range(12):
        batch = b.next_batch()
        assert (batch.batch, batch.seq) == (4, 5)
        assert batch.inputs.size == batch.targets.size == 20
        x, y = batch.inputs.reshape(4, 5), batch.targets.reshape(4, 5)
        assert np.array_equal(y, x + 1)
        assert np.array_equal(x[:, 1:], y[:, :4])


def test_the_doc_example():
    s = mh.Sequences([mh.TokenShard(100, 99, [t % 90 for t in range(41)])], 4)
    b = mh.Batcher(s, 3, 7)
    assert b.batches_per_epoch() == 3
    batch = b.next_batch()
    assert (batch.batch, batch.seq, batch.inputs.size) == (3, 4, 12)


def test_one_epoch_uses_each_sequence_at_most_once_and_skips_the_remainder():
    s = sequences(1 + 4 * 23, 4)
    assert len(s) == 23
    b = mh.Batcher(s, 5, 9)
    assert b.batches_per_epoch() == 4
    seen = set()
    for index in range(4):
        batch = b.next_batch()
        assert (batch.epoch, batch.index) == (0, index)
        seen |= {int(batch.inputs[r * 4]) for r in range(5)}
    assert len(seen) == 20
    batch = b.next_batch()
    assert (batch.epoch, batch.index) == (1, 0)


def test_every_sequence_is_used_over_enough_epochs():
    b = mh.Batcher(sequences(1 + 4 * 23, 4), 5, 3)
    seen = set()
    for _ in range(40):
        batch = b.next_batch()
        seen |= {int(batch.inputs[r * 4]) for r in range(5)}
    assert len(seen) == 23


def test_the_order_depends_on_the_seed_and_the_epoch_alone():
    def run(seed):
        b = mh.Batcher(sequences(1 + 4 * 40, 4), 4, seed)
        return [b.next_batch() for _ in range(25)]
    assert run(11) == run(11)
    assert run(11) != run(12)
    batches = run(11)
    assert batches[0].epoch == 0 and batches[10].epoch == 1
    assert not np.array_equal(batches[0].inputs, batches[10].inputs)
    assert not np.array_equal(batches[0].inputs, batches[20].inputs)


def test_seeking_continues_exactly_where_a_run_left_off():
    def make():
        return mh.Batcher(sequences(1 + 4 * 37, 4), 4, 5)
    straight = make()
    all_ = [straight.next_batch() for _ in range(40)]
    for k in range(31):
        first = make()
        for _ in range(k):
            first.next_batch()
        second = make()
        second.seek(first.epoch(), first.position())
        for want in all_[k:k + 8]:
            assert second.next_batch() == want, k


def test_batcher_arguments():
    s = sequences(1 + 4 * 10, 4)
    with pytest.raises(mh.ArgumentError):
        mh.Batcher(s, 0, 1)
    with pytest.raises(mh.ArgumentError) as e:
        mh.Batcher(s, 11, 1)
    assert "there are 10 sequences, fewer than one batch of 11" in e.value.message
    b = mh.Batcher(s, 3, 1)
    with pytest.raises(mh.ArgumentError) as e:
        b.seek(0, 4)
    assert "4 batches done is more than the 3 in a pass" in e.value.message
    b.seek(5, 3)  # the end of a pass: the next batch opens pass 6
    batch = b.next_batch()
    assert (batch.epoch, batch.index) == (6, 0)


@pytest.mark.parametrize("shape", [
    # (shard lengths, seq_len, batch, seed, batches)
    ((1 + 4 * 37,), 4, 4, 5, 40),
    ((100, 3, 250, 64, 1000), 16, 3, 1234, 90),
    ((5000,), 128, 4, 1, 30),
    ((17, 17, 17), 1, 7, 2**63 + 5, 20),
])
def test_batches_are_the_oracles_bit_for_bit(shape):
    lengths, seq_len, batch, seed, count = shape
    r = np.random.default_rng(len(lengths))
    toks = [r.integers(0, 1000, n).astype(np.uint32) for n in lengths]
    b = mh.Batcher(mh.Sequences([mh.TokenShard(1000, 999, t) for t in toks], seq_len), batch,
                   seed)
    for x, y, e, i in mo.batches(toks, seq_len, batch, seed, count):
        got = b.next_batch()
        assert (got.epoch, got.index) == (e, i)
        assert np.array_equal(got.inputs, x) and np.array_equal(got.targets, y)


# ---- oracle pins for fork / shuffle (rng.rs:108-119) ------------------------------------

def test_fork_of_stream_zero_is_a_seed_from_the_next_draw():
    a, b = mo.rng(77), mo.rng(77)
    f = mo.Rng()
    mo.lib().mmo_rng_fork(a, 0, f)
    g = mo.rng(mo.lib().mmo_rng_next_u64(b))
    assert [mo.lib().mmo_rng_next_u64(f) for _ in range(8)] == \
        [mo.lib().mmo_rng_next_u64(g) for _ in range(8)]
    # both parents advanced by one draw
    assert mo.lib().mmo_rng_next_u64(a) == mo.lib().mmo_rng_next_u64(b)


def test_the_stream_multiplier_is_the_golden_ratio_constant():
    # floor(2^64 / phi) = floor(2^63 (sqrt 5 - 1)) from the integer square root
    # of 5 * 2^126; then fork(s) = seed(next ^ s * C) for a stream s = 1.
    c = math.isqrt(5 << 126) - (1 << 63)
    assert c == 0x9E3779B97F4A7C15
    a, b = mo.rng(9), mo.rng(9)
    f = mo.Rng()
    mo.lib().mmo_rng_fork(a, 1, f)
    g = mo.rng(mo.lib().mmo_rng_next_u64(b) ^ c)
    assert mo.lib().mmo_rng_next_u64(f) == mo.lib().mmo_rng_next_u64(g)


def fisher_yates(draws, n):
    items = list(range(n))
    for i, j in zip(range(n - 1, 0, -1), draws):
        items[i], items[j] = items[j], items[i]
    return tuple(items)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5])
def test_the_shuffle_is_a_bijection_from_draws_to_permutations(n):
    import itertools
    tuples = itertools.product(*[range(i + 1) for i in range(n - 1, 0, -1)])
    perms = {fisher_yates(t, n) for t in tuples}
    assert len(perms) == math.factorial(n)


def test_the_oracle_shuffle_is_fisher_yates_over_its_draws():
    for seed in range(20):
        for n in (1, 2, 5, 13):
            a, b = mo.rng(seed), mo.rng(seed)
            items = np.arange(n, dtype=np.uint64)
            mo.lib().mmo_rng_shuffle_u64(a, items.ctypes.data_as(U64P), n)
            draws = [mo.lib().mmo_rng_below(b, i + 1) for i in range(n - 1, 0, -1)]
            assert tuple(int(v) for v in items) == fisher_yates(draws, n)


def test_the_reference_shuffle_test_on_the_oracle():
    # rng.rs:216-228: a permutation that depends on the seed
    def shuffled(seed):
        items = np.arange(50, dtype=np.uint64)
        mo.lib().mmo_rng_shuffle_u64(mo.rng(seed), items.ctypes.data_as(U64P), 50)
        return items.tolist()
    a, b = shuffled(3), shuffled(4)
    assert sorted(a) == list(range(50)) and a != list(range(50)) and a != b


def test_eval_rows_follow_the_even_spacing():
    # trainer.rs:236-249 for a few shapes, against the formula's properties:
    # distinct, ascending, first row 0, within range
    for n, bs, mb in [(10, 3, 100), (10, 20, 5), (1000, 4, 8), (7, 7, 1)]:
        rows = mo.eval_rows(n, bs, mb)
        flat = [i for b in rows for i in b]
        assert flat[0] == 0 and flat == sorted(set(flat)) and flat[-1] < n
        assert len(rows) == min(mb, n // min(bs, n))
