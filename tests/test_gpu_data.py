"""Training and evaluation fed by token shards through the batcher
(Trainer::step trainer.rs:162-183, Trainer::evaluate :218-258), on the
device through the C ABI."""
import os
import tempfile

import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as mo

pytestmark = pytest.mark.gpu

SMOKE = mh.PRESETS["smoke"]
ADAM = (0.9, 0.99, 1e-8, 0.01, 1.0)  # beta1, beta2, eps, weight_decay, clip_norm


def ocfg(config):
    return mo.config(*[int(x) for x in config[:7]], theta=config[7], eps=config[8],
                     tie=bool(config[9]))


def token_streams(vocab, lengths, seed):
    r = np.random.default_rng(seed)
    return [r.integers(0, vocab, n).astype(np.uint32) for n in lengths]


def saved_shards(d, vocab, toks):
    """Writes each stream as a shard file and reads it back, as a run would."""
    out = []
    for n, t in enumerate(toks):
        p = os.path.join(d, f"shard-{n:05}.mmtokens")
        mh.TokenShard(vocab, vocab - 1, t).save(p)
        out.append(mh.TokenShard.load(p))
    return out


def test_steps_from_shards_are_train_steps_on_the_oracles_batches(ctx):
    """Each Trainer::step takes the batcher's next batch: the same losses,
    norms and weights as train_step on the oracle's batch order, bit for bit."""
    vocab, seq, batch, seed = 256, 32, 2, 1234
    toks = token_streams(vocab, [700, 90, 400], 3)
    steps = 20  # past one pass: 21 + 2 + 12 = 35 sequences, 17 batches per pass
    print(f"\n[case] smoke {steps} steps from shards, B{batch} T{seq}", flush=True)
    with tempfile.TemporaryDirectory() as d:
        shards = saved_shards(d, vocab, toks)
    data = mh.Sequences(shards, seq)
    batcher = mh.Batcher(data, batch, seed)
    a = mh.Model.new(ctx, SMOKE, 7)
    b = mh.Model.new(ctx, SMOKE, 7)
    try:
        a.set_optimizer(*ADAM)
        b.set_optimizer(*ADAM)
        want = mo.batches(toks, seq, batch, seed, steps)
        for s, (x, y, e, i) in enumerate(want):
            lr = mh.warmup_cosine_lr(0.003, 0.0003, 3, steps, s)
            got = a.train_next(batcher, lr)
            ref = b.train_step(x.astype(np.int32), y.astype(np.int32), batch, seq, lr)
            assert got[2:] == (e, i)
            assert got[:2] == ref, s
        assert np.array_equal(a.weights(), b.weights())
        assert a.optimizer_steps() == steps
    finally:
        a.close()
        b.close()


def test_losses_from_shards_match_the_oracle(ctx):
    """The device steps against the oracle's forward, backward, clip and AdamW
    on the same batches."""
    vocab, seq, batch, seed = 256, 16, 3, 5
    toks = token_streams(vocab, [500, 260], 11)
    c = ocfg(SMOKE)
    w = mo.init_weights(c, mo.rng(9))
    data = mh.Sequences([mh.TokenShard(vocab, vocab - 1, t) for t in toks], seq)
    batcher = mh.Batcher(data, batch, seed)
    m = mh.Model.from_weights(ctx, SMOKE, w)
    wo = w.copy()
    mom1, mom2 = np.zeros_like(w), np.zeros_like(w)
    steps = 0
    try:
        m.set_optimizer(*ADAM)
        for x, y, e, i in mo.batches(toks, seq, batch, seed, 4):
            loss, norm, ge, gi = m.train_next(batcher, 0.002)
            assert (ge, gi) == (e, i)
            # Trainer::update (trainer.rs:185-207): loss, backward, clip, AdamW
            want_loss, g = mo.forward_backward(c, wo, x.astype(np.int32), y.astype(np.int32),
                                               batch, seq)
            f = mo.ctypes.c_float()
            assert mo.lib().mmo_clip_global_norm(mo.fp(g), g.size, ADAM[4],
                                                 mo.ctypes.byref(f)) == mo.OK
            want_norm = f.value
            steps = mo.adamw_step(c, wo, g, mom1, mom2, 0.002, *ADAM[:4], steps)
            assert abs(loss - want_loss) <= 1e-5 * abs(want_loss)
            assert abs(norm - want_norm) <= 1e-4 * abs(want_norm)
        assert np.median(np.abs(m.weights() - wo)) <= 1e-6
    finally:
        m.close()


def test_a_failed_step_leaves_the_batcher_where_it_was(ctx):
    vocab, seq = 256, 8
    data = mh.Sequences([mh.TokenShard(vocab, 0, token_streams(vocab, [200], 1)[0])], seq)
    batcher = mh.Batcher(data, 2, 3)
    other = mh.Batcher(data, 2, 3)
    m = mh.Model.new(ctx, SMOKE, 1)
    try:
        with pytest.raises(mh.ArgumentError):  # no optimizer yet
            m.train_next(batcher, 0.001)
        assert (batcher.epoch(), batcher.position()) == (0, 0)
        m.set_optimizer(*ADAM)
        m.train_next(batcher, 0.001)
        other.next_batch()
        with pytest.raises(mh.ArgumentError):  # a learning rate AdamW refuses
            m.train_next(batcher, -1.0)
        assert (batcher.epoch(), batcher.position()) == (0, 1)
        assert m.optimizer_steps() == 1
        _, _, e, i = m.train_next(batcher, 0.001)
        assert (e, i) == (0, 1)
        want = other.next_batch()
        got = mh.Batcher(data, 2, 3)
        got.seek(0, 1)
        assert got.next_batch() == want
    finally:
        m.close()


def test_a_non_finite_step_is_stopped_and_the_batcher_goes_back(ctx):
    c = ocfg(SMOKE)
    w = mo.init_weights(c, mo.rng(2))
    w[: c.d_model * c.vocab_size] = np.nan  # the whole embedding table
    data = mh.Sequences([mh.TokenShard(256, 0, token_streams(256, [100], 4)[0])], 8)
    batcher = mh.Batcher(data, 2, 1)
    m = mh.Model.from_weights(ctx, SMOKE, w)
    try:
        m.set_optimizer(*ADAM)
        with pytest.raises(mh.Stopped):
            m.train_next(batcher, 0.001)
        assert (batcher.epoch(), batcher.position()) == (0, 0)
        assert m.optimizer_steps() == 0
    finally:
        m.close()


def test_the_data_must_fit_the_model(ctx):
    m = mh.Model.new(ctx, SMOKE, 1)  # vocab 256, max_seq_len 128
    try:
        m.set_optimizer(*ADAM)
        wrong_vocab = mh.Sequences([mh.TokenShard(300, 0, list(range(100)))], 8)
        with pytest.raises(mh.ArgumentError) as e:
            m.train_next(mh.Batcher(wrong_vocab, 2, 1), 0.001)
        assert "vocabulary of 300 and the model 256" in e.value.message
        too_long = mh.Sequences([mh.TokenShard(256, 0, [1] * 600)], 129)
        with pytest.raises(mh.ArgumentError) as e:
            m.train_next(mh.Batcher(too_long, 2, 1), 0.001)
        assert "longer than the model's 128" in e.value.message
        with pytest.raises(mh.ArgumentError) as e:
            m.evaluate(mh.Sequences([], 8), 2, 4)
        assert "no tokens" in e.value.message
        empty = mh.Sequences([mh.TokenShard(256, 0, [1] * 5)], 8)
        with pytest.raises(mh.ArgumentError) as e:
            m.evaluate(empty, 2, 4)
        assert "nothing to evaluate" in e.value.message
        ok = mh.Sequences([mh.TokenShard(256, 0, [1] * 100)], 8)
        with pytest.raises(mh.ArgumentError):
            m.evaluate(ok, 2, 0)
    finally:
        m.close()


@pytest.mark.parametrize("n_tokens,batch_size,max_batches", [
    (1 + 16 * 37, 4, 3), (1 + 16 * 37, 4, 100), (1 + 16 * 5, 8, 2), (1 + 16 * 9, 3, 2)])
def test_evaluate_is_the_mean_loss_over_evenly_spaced_sequences(ctx, n_tokens, batch_size,
                                                                max_batches):
    seq = 16
    toks = token_streams(256, [n_tokens], 8)
    data = mh.Sequences([mh.TokenShard(256, 255, toks[0])], seq)
    wins = mo.sequence_windows(toks, seq)
    c = ocfg(SMOKE)
    w = mo.init_weights(c, mo.rng(4))
    m = mh.Model.from_weights(ctx, SMOKE, w)
    try:
        loss, nb, nt = m.evaluate(data, batch_size, max_batches)
        rows = mo.eval_rows(len(wins), batch_size, max_batches)
        assert (nb, nt) == (len(rows), len(rows) * len(rows[0]) * seq)
        device, oracle = 0.0, 0.0
        for r in rows:
            x = np.concatenate([toks[0][wins[i][1]:wins[i][1] + seq] for i in r]).astype(np.int32)
            y = np.concatenate([toks[0][wins[i][1] + 1:wins[i][1] + seq + 1]
                                for i in r]).astype(np.int32)
            device += float(m.loss(x, y, len(r), seq))
            oracle += float(mo.forward_loss(c, w, x, y, len(r), seq, want_logits=False)[0])
        assert loss == np.float32(device / len(rows))
        assert abs(loss - oracle / len(rows)) <= 1e-5 * abs(loss)
    finally:
        m.close()
