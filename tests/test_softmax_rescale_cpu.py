"""The planted-key inputs of test_gpu_softmax_rescale.py catch a broken rescale.

CPU only.  A float64 model of each kernel's softmax schedule (64-key tiles,
a maximum that moves lazily, p = 2^(s - m) with fp16's overflow) runs over
the planted inputs and is compared with the oracle (src/model/math.rs:102-155
restated in oracle/sr_oracle.c) at the GPU tests' tolerance.  The faithful
model passes; the same model with one step of the rescale dropped (O not
rescaled, l not rescaled, or the maximum never moved) fails.  So a kernel
with such a mistake cannot pass the GPU tests on these inputs.
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_softmax_rescale import (LN2, PlantedSeq, falling_plants, gammas,
                                      rising_plants, threshold_plants, transformed_q)

ATOL, RTOL = 2e-3, 1e-2
F16_MAX = 65504.0


class _HostPool:
    page_tokens = 64
    _max_tokens = 4096

    def __init__(self):
        self.n = 0

    def open(self):
        self.n += 1
        return self.n - 1

    def append(self, seq, keys, values):
        pass


def _scores_log2(qt_row_head, keys, dim):
    return (keys @ qt_row_head.astype(np.float64)) / math.sqrt(dim) / LN2


def _fp16_p(x):
    # p = 2^x rounded to fp16: beyond the range it is infinite
    p = np.exp2(np.minimum(x, 1024.0))
    return np.where(p > F16_MAX, np.inf, p)


def model_softmax(s, vals, schedule, bug=None):
    """o = sum p v / sum p over keys in 64-key tiles, as the kernels order it.

    schedule "sum_bound": the ping-pong prefill kernel (maximum of the first
    tile, raised when a 32-key half of a tile sums above 2^15).
    schedule "lazy8": the lock-step prefill and verify kernels (raised when a
    tile's maximum is more than 8 above it)."""
    m, l, o = -np.inf, 0.0, np.zeros(vals.shape[1])
    for t0 in range(0, len(s), 64):
        st, vt = s[t0:t0 + 64], vals[t0:t0 + 64]
        mx = st.max()
        alpha = 1.0
        if t0 == 0:
            m = mx  # both schedules: the first tile sets the maximum (l = o = 0 before it)
            p = _fp16_p(st - m)
        elif schedule == "lazy8":
            if mx > m + 8.0 and bug != "never_move":
                alpha, m = 2.0 ** (m - mx), mx
            p = _fp16_p(st - m)
        else:
            p = _fp16_p(st - m)
            if bug != "never_move" and not (p[:32].sum() <= 32768.0 and p[32:].sum() <= 32768.0):
                shift = max(mx - m, 0.0)
                m += shift
                alpha = 2.0 ** -shift
                p = _fp16_p(st - m)
        l = l * (1.0 if bug == "l_not_rescaled" else alpha) + p.sum()
        o = o * (1.0 if bug == "o_not_rescaled" else alpha) + p @ vt
    return o / l


def _case(schedule_heads, plants_of, ctx, rows, seed):
    rng = np.random.default_rng(seed)
    heads, kv_heads, dim = schedule_heads
    pool = _HostPool()
    pool._max_tokens = ctx + rows
    gq, gk = gammas(rng, dim)
    seq = PlantedSeq(rng, pool, heads, kv_heads, dim, ctx, rows, plants_of(rows, heads), gq=gq)
    exp = O.attention_rows(seq.q, seq.k, seq.v, seq.pos.astype(np.int64), seq.ref, heads=heads,
                           kv_heads=kv_heads, dim=dim, rotary_dim=dim, theta=1e6, eps=1e-6,
                           q_norm=gq, k_norm=gk, threads=8)
    # the cache after the call: context plus the rows' normalised, rotated keys (bf16)
    n = len(seq.ref)
    keys = np.empty((n, kv_heads * dim), np.float64)
    vals = np.empty((n, kv_heads * dim), np.float64)
    for t in range(n):
        keys[t], vals[t] = seq.ref.get(t)
    qt = transformed_q(seq.q, seq.pos, heads, dim, dim, 1e6, gq)
    return seq, exp.reshape(rows, heads, dim), keys, vals, qt


def _run_models(case, schedule, heads, kv_heads, dim, rows_heads):
    seq, exp, keys, vals, qt = case
    g = heads // kv_heads
    bad = {None: 0, "o_not_rescaled": 0, "l_not_rescaled": 0, "never_move": 0}
    for r, h in rows_heads:
        kv = h // g
        vis = seq.ctx + r + 1
        s = _scores_log2(qt[r, h], keys[:vis, kv * dim:(kv + 1) * dim], dim)
        vv = vals[:vis, kv * dim:(kv + 1) * dim]
        for bug in bad:
            with np.errstate(invalid="ignore", over="ignore"):
                got = model_softmax(s, vv, schedule, bug)
            e = exp[r, h]
            ok = np.isfinite(got).all() and np.all(np.abs(got - e) <= ATOL + RTOL * np.abs(e))
            bad[bug] += 0 if ok else 1
    return bad


@pytest.mark.parametrize("schedule", ["sum_bound", "lazy8"])
def test_rising_plants_catch_a_dropped_rescale(schedule):
    heads, kv_heads, dim = 8, 2, 128
    rows = 24
    case = _case((heads, kv_heads, dim),
                 lambda r, h: rising_plants(r, h, (64, 256, 448), (10.0, 20.0, 40.0)), 640, rows,
                 seed=11)
    planted = [(r, (7 * r) % heads) for r in range(rows)]
    bad = _run_models(case, schedule, heads, kv_heads, dim, planted)
    assert bad[None] == 0, bad
    for bug in ("o_not_rescaled", "l_not_rescaled", "never_move"):
        assert bad[bug] == len(planted), (bug, bad)


def test_threshold_plants_catch_a_dropped_rescale_in_the_sum_bound_schedule():
    heads, kv_heads, dim = 8, 2, 128
    gaps = (5.0, 7.9, 8.1, 12.0, 14.9, 15.1, 15.9, 16.1, 17.0, 30.0)
    rows = 20
    case = _case((heads, kv_heads, dim), lambda r, h: threshold_plants(r, h, 128, gaps), 400,
                 rows, seed=12)
    planted = [(r, (5 * r + 1) % heads) for r in range(rows)]
    bad = _run_models(case, "sum_bound", heads, kv_heads, dim, planted)
    assert bad[None] == 0, bad
    # rows whose plant crosses the 2^15 sum bound (gap >= 15.1) move the
    # maximum, so a dropped O or l rescale shows there; never moving it shows
    # where p itself leaves fp16's range (gap > log2(65504) = 15.9993)
    crossing = sum(1 for r in range(rows) if gaps[r % len(gaps)] >= 15.1)
    overflow = sum(1 for r in range(rows) if gaps[r % len(gaps)] >= 16.1)
    assert bad["o_not_rescaled"] >= crossing and bad["l_not_rescaled"] >= crossing, bad
    assert bad["never_move"] >= overflow, bad


def test_falling_plants_agree_with_the_oracle():
    # a first-tile maximum 12 or 40 log2 units above every later key: the
    # later probabilities underflow in fp16 without moving the output
    heads, kv_heads, dim = 8, 2, 128
    rows = 16
    case = _case((heads, kv_heads, dim), lambda r, h: falling_plants(r, h, (12.0, 40.0)), 300,
                 rows, seed=13)
    planted = [(r, (3 * r + 2) % heads) for r in range(rows)]
    for schedule in ("sum_bound", "lazy8"):
        bad = _run_models(case, schedule, heads, kv_heads, dim, planted)
        assert bad[None] == 0, (schedule, bad)
