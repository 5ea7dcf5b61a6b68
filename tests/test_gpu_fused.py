"""GPU parity of the fused loss-only forward (fused_forward.hip: the whole of
model.rs:127-183 as one persistent launch, per-XCD teams of workgroups),
and the guard bands around every region of its arena.

Every case runs the same model and tokens through the fused launch
(MMH_PATH_AUTO) and through the per-operation kernels (MMH_PATH_PER_OP) and
compares both with the oracle. Tolerances: fused vs oracle <= 1e-4 relative
(the stated loss target); fused vs per-operation <= 2e-6 relative (two f32
paths of the same arithmetic in different orders); repeated fused runs and
staged runs bit-identical (fixed reduction orders, no atomics on data).
"""
import numpy as np
import pytest

import midman_hip as mh
import mm_oracle as O

pytestmark = pytest.mark.gpu


def oracle_config(cfg):
    return O.config(*[int(v) for v in cfg[:7]], float(cfg[7]), float(cfg[8]), bool(cfg[9]))


def both_paths(m, x, y, batch, seq):
    # every shape here fits the fused kernel: PATH_AUTO must take it (on an
    # MI355X the context's XCD probe passes), PATH_PER_OP must not
    m.set_forward_path(mh.PATH_AUTO)
    fused = float(m.loss(x, y, batch, seq))
    assert m.last_forward_fused()
    again = float(m.loss(x, y, batch, seq))
    m.set_forward_path(mh.PATH_PER_OP)
    per_op = float(m.loss(x, y, batch, seq))
    assert not m.last_forward_fused()
    m.set_forward_path(mh.PATH_AUTO)
    return fused, again, per_op


@pytest.mark.parametrize("preset,batch,seq", [("tiny", 8, 256), ("smoke", 2, 32), ("smoke", 4, 128)])
def test_fused_presets(ctx, preset, batch, seq):
    print(f"\n[fused] {preset} B{batch} T{seq} seed 0", flush=True)
    cfg = mh.PRESETS[preset]
    m = mh.Model.new(ctx, cfg, 0)
    try:
        x, y = m.lab_tokens(batch, seq)
        fused, again, per_op = both_paths(m, x, y, batch, seq)
        c = oracle_config(cfg)
        w_ref, _, _ = O.lab_setup(c, 0, batch, seq)
        ref = float(O.forward_loss(c, w_ref, x, y, batch, seq, want_logits=False)[0])
        print(f"  fused {fused:.7f} per-op {per_op:.7f} oracle {ref:.7f}", flush=True)
        assert fused == again
        assert abs(fused - per_op) <= 2e-6 * per_op
        assert abs(fused - ref) <= 1e-4 * ref
    finally:
        m.close()


@pytest.mark.parametrize("cfg,batch,seq", [
    # hd 32, GQA, untied head, V ending inside a 256-row block, ragged T:
    # XCD 0 owns sequences 0 and 8, the others one each
    ([1000, 128, 2, 4, 2, 96, 64, 10000.0, 1e-5, 0], 9, 45),
    # hd 16, one token: a single row in the whole launch
    ([50, 64, 2, 4, 4, 40, 16, 10000.0, 1e-5, 1], 1, 1),
    # d 256 (K = 256 steps over both K-groups), 8 heads of 32, 2 kv heads,
    # ff 100 (gate/up padded to 128 pairs), 16 sequences: two per XCD
    ([300, 256, 1, 8, 2, 100, 64, 500.0, 1e-6, 1], 16, 64),
    # T = 257: nine key tiles, so a wave walks two; a one-row last block
    ([257, 64, 1, 4, 2, 64, 300, 10000.0, 1e-5, 1], 2, 257),
    # 20 sequences of 33 rows: XCDs 0-3 own three, 4-7 two; partial blocks
    ([77, 96, 2, 3, 1, 36, 40, 10000.0, 1e-5, 0], 20, 33),
])
def test_fused_shapes_against_oracle(ctx, cfg, batch, seq):
    print(f"\n[fused] {cfg[:7]} tie={cfg[9]} B{batch} T{seq}", flush=True)
    c = oracle_config(cfg)
    w = O.init_weights(c, O.rng(41), std=0.1)
    r = np.random.default_rng(batch * 1000 + seq)
    x = r.integers(0, cfg[0], batch * seq).astype(np.int32)
    y = r.integers(0, cfg[0], batch * seq).astype(np.int32)
    m = mh.Model.from_weights(ctx, cfg, w)
    try:
        fused, again, per_op = both_paths(m, x, y, batch, seq)
        ref = float(O.forward_loss(c, w, x, y, batch, seq, want_logits=False)[0])
        print(f"  fused {fused:.7f} per-op {per_op:.7f} oracle {ref:.7f}", flush=True)
        assert fused == again
        assert abs(fused - per_op) <= 2e-6 * per_op
        assert abs(fused - ref) <= 1e-4 * ref
        # every region of the fused arena (and of the activations) kept its
        # guard bands (kernels_avx.rs:368-390)
        assert m.broken_guards() == 0
    finally:
        m.close()


def test_fused_staged_runs_and_reshapes(ctx):
    # run_staged launches the fused kernel directly on every call; runs interleaved
    # with eager fused runs, per-operation runs and a run at another shape
    # (the arena is laid out again) must keep returning the eager loss.
    cfg = mh.PRESETS["tiny"]
    print("\n[fused staged] tiny B8 T256 / B3 T100", flush=True)
    m = mh.Model.new(ctx, cfg, 7)
    try:
        x, y = m.lab_tokens(8, 256)
        x2, y2 = m.lab_tokens(3, 100)
        eager = float(m.loss(x, y, 8, 256))
        eager2 = float(m.loss(x2, y2, 3, 100))
        for i in range(8):
            m.stage(x, y, 8, 256)
            m.run_staged(8, 256)
            assert m.read_loss() == eager, i
            assert m.last_forward_fused()
            if i % 3 == 1:
                assert float(m.loss(x2, y2, 3, 100)) == eager2
            if i % 3 == 2:
                m.set_forward_path(mh.PATH_PER_OP)
                assert abs(float(m.loss(x, y, 8, 256)) - eager) <= 2e-6 * eager
                m.set_forward_path(mh.PATH_AUTO)
    finally:
        m.close()


def test_forward_path_argument(ctx):
    m = mh.Model.new(ctx, mh.PRESETS["smoke"], 1)
    try:
        with pytest.raises(mh.MidmanError):
            m.set_forward_path(2)
    finally:
        m.close()


def test_unfit_model_and_logits_stay_per_op(ctx):
    # heads of 64 (outside the fused kernel) and a logits-producing forward
    # run on the per-operation kernels even under PATH_AUTO
    cfg = [64, 128, 1, 2, 2, 64, 32, 10000.0, 1e-5, 1]
    m = mh.Model.new(ctx, cfg, 3)
    try:
        x, y = m.lab_tokens(2, 16)
        m.loss(x, y, 2, 16)
        assert not m.last_forward_fused()
    finally:
        m.close()
    m = mh.Model.new(ctx, mh.PRESETS["smoke"], 3)
    try:
        x, y = m.lab_tokens(2, 16)
        m.loss(x, y, 2, 16)
        assert m.last_forward_fused()
        m.forward(x, 2, 16)
        assert not m.last_forward_fused()
    finally:
        m.close()


def test_fused_failure_is_redone_on_the_per_op_kernels(ctx):
    # The fused kernel's bounded waits give up once its error word is set (a
    # wait that reached its bound sets it; here the host presets it, so every
    # workgroup still runs to its end). The forward is then redone on the
    # per-operation kernels from the staged ids: the loss is the
    # per-operation loss bit for bit, the word and the counters are cleared,
    # and the next fused launch (mmh_model_loss or a staged run) is right again.
    cfg = mh.PRESETS["tiny"]
    print("\n[fused failure] tiny B8 T256 seed 0, error word preset", flush=True)
    m = mh.Model.new(ctx, cfg, 0)
    try:
        x, y = m.lab_tokens(8, 256)
        m.set_forward_path(mh.PATH_PER_OP)
        per_op = float(m.loss(x, y, 8, 256))
        m.set_forward_path(mh.PATH_AUTO)
        fused = float(m.loss(x, y, 8, 256))
        assert m.last_forward_fused()
        assert m.fused_fallbacks() == (0, 0)

        # mmh_model_loss: the redo happens before it returns
        m.inject_fused_error(8)
        assert float(m.loss(x, y, 8, 256)) == per_op
        assert not m.last_forward_fused()
        n, e = m.fused_fallbacks()
        assert n == 1 and e & 8, (n, e)
        assert float(m.loss(x, y, 8, 256)) == fused
        assert m.last_forward_fused()

        # staged runs (a direct launch each); the preset word reaches a staged run
        m.stage(x, y, 8, 256)
        for _ in range(3):
            m.run_staged(8, 256)
            assert m.read_loss() == fused
            assert m.last_forward_fused()
        m.inject_fused_error(8)
        m.run_staged(8, 256)
        assert m.read_loss() == per_op
        assert m.fused_fallbacks()[0] == 2
        for _ in range(2):
            m.run_staged(8, 256)
            assert m.read_loss() == fused
            assert m.last_forward_fused()

        # a failed staged run whose loss is not read before new ids are staged
        # is redone first; the runs after it are right
        m.inject_fused_error(16)
        m.run_staged(8, 256)
        m.stage(x, y, 8, 256)
        n, e = m.fused_fallbacks()
        assert n == 3 and e & 16, (n, e)
        m.run_staged(8, 256)
        assert m.read_loss() == fused
        assert m.broken_guards() == 0
    finally:
        m.close()


@pytest.mark.parametrize("batch,fits", [(4160, True), (4161, False)])
def test_fused_loss_slot_bound(ctx, batch, fits):
    # The fused launch's last workgroup parks one f64 sum per (sequence,
    # 32-row block) in a 4160-slot LDS stage before adding them in order; a
    # shape with more blocks than that stays on the per-operation kernels.
    cfg = mh.PRESETS["smoke"]
    print(f"\n[fused slots] smoke B{batch} T1 seed 0", flush=True)
    m = mh.Model.new(ctx, cfg, 0)
    try:
        x, y = m.lab_tokens(batch, 1)
        got = float(m.loss(x, y, batch, 1))
        assert m.last_forward_fused() == fits
        c = oracle_config(cfg)
        w_ref, _, _ = O.lab_setup(c, 0, batch, 1)
        ref = float(O.forward_loss(c, w_ref, x, y, batch, 1, want_logits=False)[0])
        print(f"  device {got:.7f} oracle {ref:.7f}", flush=True)
        assert abs(got - ref) <= 1e-4 * ref
        assert m.broken_guards() == 0
    finally:
        m.close()


def test_team_slots_from_the_dispatch_order_match_the_atomic_slots(ctx):
    # The context's probe decides how the fused launch's workgroups get their
    # per-XCD team slots: from the dispatch order (blockIdx / 8, checked by
    # every launch) or from one returning atomic each. Both give the same
    # tasks to the same XCD teams, so the same loss bit for bit, with no
    # launch redone. MMH_FUSED_ATOMIC_SLOTS=1 at context creation forces the
    # atomic slots.
    import os
    teams, rr = ctx.fused_slots()
    print(f"\n[fused slots] default context: teams {teams}, round-robin {rr}", flush=True)
    assert teams
    os.environ["MMH_FUSED_ATOMIC_SLOTS"] = "1"
    try:
        actx = mh.Context(0)
    finally:
        del os.environ["MMH_FUSED_ATOMIC_SLOTS"]
    try:
        assert actx.fused_slots() == (True, False)
        cfg = mh.PRESETS["tiny"]
        losses = []
        for c in (ctx, actx):
            m = mh.Model.new(c, cfg, 0)
            try:
                x, y = m.lab_tokens(8, 256)
                m.stage(x, y, 8, 256)
                for _ in range(3):
                    m.run_staged(8, 256)
                staged = m.read_loss()
                direct = float(m.loss(x, y, 8, 256))
                assert m.last_forward_fused()
                assert m.fused_fallbacks()[0] == 0
                assert np.float32(staged) == np.float32(direct)
                losses.append(np.float32(direct))
            finally:
                m.close()
        print(f"  loss {float(losses[0]):.7f} (slot mode of the default context), "
              f"{float(losses[1]):.7f} (atomic slots)", flush=True)
        assert losses[0].view(np.uint32) == losses[1].view(np.uint32)
    finally:
        actx.close()
