"""bench.py's synthetic inputs follow the seeded streams the benchmark configs
name (CPU only: the library's host RNG against the oracle's)."""
import os
import sys

import numpy as np

import midman_hip as mh
import mm_oracle as O

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import bench  # noqa: E402


def test_block_inputs_follow_the_seeded_stream():
    # x ~ N(0,1) from Rng(0); then q, k, v, o, gate, up, down ~ N(0,0.02) from
    # the same stream (0.02 * normal() in f32); norm weights 1
    B, T, d, H, ff = (bench.BLOCK[k] for k in ("B", "T", "d", "H", "ff"))
    for hkv in (16, 8):
        kv = hkv * (d // H)
        x, w = bench.block_inputs(mh, hkv)
        r = O.rng(0)
        assert np.array_equal(x, O.randn((B, T, d), 1.0, r))
        parts = [np.ones(d, np.float32), O.randn((d, d), 0.02, r), O.randn((d, kv), 0.02, r),
                 O.randn((d, kv), 0.02, r), O.randn((d, d), 0.02, r), np.ones(d, np.float32),
                 O.randn((d, ff), 0.02, r), O.randn((d, ff), 0.02, r), O.randn((ff, d), 0.02, r)]
        want = np.concatenate([p.reshape(-1) for p in parts])
        assert w.dtype == np.float32 and w.shape == want.shape
        assert np.array_equal(w.view(np.uint32), want.view(np.uint32)), hkv
