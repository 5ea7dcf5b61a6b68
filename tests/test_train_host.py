"""Host-side training entry points of the C ABI (no GPU needed): the
warmup-cosine schedule (schedule.rs:25-66) against the reference's own values
and the oracle."""
import pytest

import midman_hip as mh
import mm_oracle as mo


def test_schedule_matches_reference_values(goldens):
    s = goldens["warmup_cosine"]
    for step, want in s["values"]:
        got = mh.warmup_cosine_lr(s["max_lr"], s["min_lr"], s["warmup"], s["total"], step)
        assert abs(got - want) < s["tol"], (step, got, want)


def test_schedule_matches_oracle_bit_for_bit():
    for args in ((0.03, 0.003, 15, 150), (1e-3, 1e-4, 4, 14), (0.5, 0.0, 0, 10)):
        for step in range(0, 160, 3):
            assert mh.warmup_cosine_lr(*args, step) == mo.warmup_cosine_lr(*args, step)


@pytest.mark.parametrize("args", [(0.0, 0.0, 0, 10), (float("nan"), 0.0, 0, 10),
                                  (1.0, -0.1, 0, 10), (1.0, 2.0, 0, 10), (1.0, 0.0, 10, 10),
                                  (1.0, 0.0, 11, 10), (1.0, 0.0, 0, 0)])
def test_schedule_rejects_what_the_reference_rejects(args):
    # schedule.rs:122-129
    with pytest.raises(mh.ArgumentError):
        mh.warmup_cosine_lr(*args, 0)
