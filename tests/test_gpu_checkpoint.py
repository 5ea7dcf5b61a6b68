"""Model checkpoints straight between HBM and safetensors files
(midman-checkpoint params.rs; the reference's end-to-end tests in
crates/midman-checkpoint/tests/model_roundtrip.rs:35-80)."""
import os
import struct
import tempfile

import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as mo

pytestmark = pytest.mark.gpu

SMOKE = mh.PRESETS["smoke"]
TINY = mh.PRESETS["tiny"]


def ids(vocab, n):
    return np.array([(i * 7 + 3) % vocab for i in range(n)], np.int32)  # model_roundtrip.rs:23-26


def logits_bits(m, vocab):
    return m.forward(ids(vocab, 32), 2, 16).view(np.uint32)


@pytest.fixture
def tmpdir_path():
    with tempfile.TemporaryDirectory() as d:
        yield d


def test_a_saved_model_loads_into_another_and_computes_the_same_logits(ctx, tmpdir_path):
    src = mh.Model.new(ctx, SMOKE, 1)
    dst = mh.Model.new(ctx, SMOKE, 2)
    try:
        a, b = logits_bits(src, 256), logits_bits(dst, 256)
        assert not np.array_equal(a, b)
        path = os.path.join(tmpdir_path, "smoke.safetensors")
        src.save_checkpoint(path, {"step": "0"})
        assert not os.path.exists(path + ".tmp")
        f = mh.TensorFile.load(path)
        assert f.metadata() == {"checkpoint_version": "1", "format": "midman-checkpoint",
                                "step": "0"}
        t = f.tensors()
        assert len(t) == len(mh.parameter_names(SMOKE))
        assert sum(v.size for _, _, v in t) == src.num_parameters()
        dst.load_checkpoint(path)
        assert np.array_equal(logits_bits(dst, 256), a)
        assert np.array_equal(dst.weights(), src.weights())
        again = mh.Model.from_checkpoint(ctx, SMOKE, path)
        try:
            assert np.array_equal(logits_bits(again, 256), a)
        finally:
            again.close()
    finally:
        src.close()
        dst.close()


@pytest.mark.parametrize("config", [SMOKE, [12, 16, 2, 2, 1, 32, 16, 10000.0, 1e-5, 0]])
def test_the_device_file_is_the_reference_writers_bytes(ctx, tmpdir_path, config):
    """The file streamed from HBM equals TensorFile serialization (itself
    byte-identical to the reference package's files) of the reference-init
    weights under the reference's names."""
    c = mo.config(*[int(x) for x in config[:7]], theta=config[7], eps=config[8],
                  tie=bool(config[9]))
    w = mo.init_weights(c, mo.rng(5))
    m = mh.Model.new(ctx, config, 5)
    try:
        path = os.path.join(tmpdir_path, "m.safetensors")
        m.save_checkpoint(path, {"step": "7", "tokens_seen": "128"})
        data = open(path, "rb").read()
    finally:
        m.close()
    f = mh.TensorFile()
    for name, (off, size, _), shape in zip(mh.parameter_names(config), mo.param_segments(c),
                                          _shapes(config)):
        f.push(name, shape, w[off:off + size])
    for k, v in {"step": "7", "tokens_seen": "128", "format": "midman-checkpoint",
                 "checkpoint_version": "1"}.items():
        f.set_metadata(k, v)
    assert data == f.to_bytes()


def _shapes(config):
    V, d, L, H, Hkv, ff = (int(x) for x in config[:6])
    kv = Hkv * (d // H)
    s = [[V, d]]
    for _ in range(L):
        s += [[d], [d, d], [d, kv], [d, kv], [d, d], [d], [d, ff], [d, ff], [ff, d]]
    s.append([d])
    if not config[9]:
        s.append([d, V])
    return s


def test_saving_twice_gives_identical_files(ctx, tmpdir_path):
    m = mh.Model.new(ctx, SMOKE, 1)
    try:
        a, b = (os.path.join(tmpdir_path, n) for n in ("a", "b"))
        m.save_checkpoint(a)
        m.save_checkpoint(b)
        assert open(a, "rb").read() == open(b, "rb").read()
    finally:
        m.close()


def test_a_checkpoint_of_another_model_is_refused_and_changes_nothing(ctx, tmpdir_path):
    smoke = mh.Model.new(ctx, SMOKE, 1)
    tiny = mh.Model.new(ctx, TINY, 2)
    try:
        path = os.path.join(tmpdir_path, "smoke")
        smoke.save_checkpoint(path)
        before = logits_bits(tiny, 4096)
        with pytest.raises(mh.MidmanError):
            tiny.load_checkpoint(path)
        assert np.array_equal(logits_bits(tiny, 4096), before)
    finally:
        smoke.close()
        tiny.close()


def test_strict_loading_and_its_messages(ctx, tmpdir_path):
    m = mh.Model.new(ctx, SMOKE, 1)
    try:
        w0 = m.weights()
        with pytest.raises(mh.ArgumentError):
            m.save_checkpoint(os.path.join(tmpdir_path, "x"), {"format": "mine"})
        with pytest.raises(mh.MidmanError) as e:
            m.load_checkpoint(os.path.join(tmpdir_path, "missing.safetensors"))
        assert "missing.safetensors" in e.value.message

        def write(tensors, meta):
            f = mh.TensorFile()
            for n, s, v in tensors:
                f.push(n, s, v)
            for k, v in meta.items():
                f.set_metadata(k, v)
            p = os.path.join(tmpdir_path, "crafted")
            open(p, "wb").write(f.to_bytes())
            return p

        full = [(n, s, w0[o:o + z]) for n, s, (o, z, _) in
                zip(mh.parameter_names(SMOKE), _shapes(SMOKE),
                    mo.param_segments(mo.preset("smoke")))]
        good = {"format": "midman-checkpoint", "checkpoint_version": "1"}
        with pytest.raises(mh.MidmanError) as e:
            m.load_checkpoint(write(full, {"checkpoint_version": "1"}))
        assert "format" in e.value.message
        with pytest.raises(mh.MidmanError) as e:
            m.load_checkpoint(write(full, {"format": "midman-checkpoint", "checkpoint_version": "2"}))
        assert "version" in e.value.message
        with pytest.raises(mh.ArgumentError) as e:
            m.load_checkpoint(write(full[1:], good))
        assert "missing 1" in e.value.message and "embed_tokens.weight" in e.value.message
        with pytest.raises(mh.ArgumentError) as e:
            m.load_checkpoint(write(full + [("extra", [1], [1.0])], good))
        assert "`extra`" in e.value.message
        bad_shape = list(full)
        n, s, v = bad_shape[0]  # embed_tokens [V, d] given as [d, V]
        bad_shape[0] = (n, [s[1], s[0]], v)
        with pytest.raises(mh.ShapeError):
            m.load_checkpoint(write(bad_shape, good))
        assert np.array_equal(m.weights(), w0)
        # and a crafted but valid one loads
        m.load_checkpoint(write(full, good))
        assert np.array_equal(m.weights(), w0)
    finally:
        m.close()


def test_a_loaded_model_trains_like_the_original(ctx, tmpdir_path):
    """Checkpoint -> another model -> one Lab step gives the reference's native
    golden loss and gradient norm (engine.test.mjs:25-26): the weights the file
    holds are the ones the model computes with, packed copies included."""
    config = [12, 16, 2, 2, 1, 32, 16, 10000.0, 1e-5, 1]
    src = mh.Model.new(ctx, config, 2024)
    x, y = src.lab_tokens(2, 12)
    path = os.path.join(tmpdir_path, "lab")
    src.save_checkpoint(path)
    src.close()
    m = mh.Model.new(ctx, config, 9)
    try:
        m.load_checkpoint(path)
        m.set_optimizer(0.9, 0.99, 1e-8, 0.01, 1.0)
        l0, n0 = m.train_step(x, y, 2, 12, 0.002)
        assert abs(l0 - 2.493498) <= 1e-4 * 2.493498
        assert abs(n0 - 1.0999628) <= 1e-4 * 1.0999628
    finally:
        m.close()
