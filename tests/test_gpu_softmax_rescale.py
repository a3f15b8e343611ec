"""GPU parity of the online-softmax rescale paths, through the C-ABI.

The reference keeps one running maximum m per (row, query head) and, for
every key whose score beats it, rescales the running sum and output by
e^(m - m') before adding the key (src/model/math.rs:133-152).  The MI355X
kernels move their maximum less often:

* the pipelined prefill kernel (G = 2, 4, 8 at head_dim 128, pages of 64
  tokens or more) and the ping-pong prefill kernel (G = 1, and G = 2, 4 on
  smaller pages) keep the row maximum of their first 64-key tile and raise
  it only when a lane's partial sum of a tile's probabilities exceeds 2^15 (a
  score about 15 log2 units above the kept maximum, or many keys a little
  lower);
* the lock-step prefill kernel (other group sizes and head dims) and the
  verify kernel raise it when a tile's maximum is more than 8 log2 units
  above it;
* the decode kernel raises it whenever a chunk's maximum is larger.

With q and k ~ N(0, 1) after RMSNorm the scores are ~N(0, 1) nats, so a key
after the first tile never beats the first tile's maximum by more than about
2 log2 units and random inputs reach only the first-tile branch.  These
cases plant keys into the cached context: a planted key for (row r, query
head h) is the direction of r's normalised and rotated q for head h, scaled
so that its score for (r, h) is r's first-tile maximum plus a chosen number
of log2 units.  Plants after the first tile raise the maximum (by 10, 20 and
40 log2 units in turn, across the thresholds above, or with a whole tile of
equal scores); plants inside the first tile make every later tile fall far
below the kept maximum.  Each case is checked against the oracle at the
bf16-path tolerance |d| <= 2e-3 + 1e-2 * |ref|, and asserts which kernels
ran (a call whose operands left the fp16 range would be recomputed on the
split-K decode path and would no longer test the kernel it names).
"""
import math
import os
import zlib

import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_attention import close, new_pool

pytestmark = pytest.mark.gpu

LN2 = math.log(2.0)
EPS = 1e-6
ORACLE_THREADS = min(16, os.cpu_count() or 1)


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


def transformed_q(q_raw, pos, heads, dim, rotary, theta, gq):
    """q after the QK-RMSNorm and RoPE of Attention::forward (native.rs:629-636)."""
    out = np.empty((q_raw.shape[0], heads, dim), np.float32)
    for r in range(q_raw.shape[0]):
        x = q_raw[r]
        if gq is not None:
            x = O.rms_norm(x, gq, EPS, False)
        out[r] = O.apply_rope(x, dim, pos[r].astype(np.int64), theta, rotary).reshape(heads, dim)
    return out


class PlantedSeq:
    """One sequence: a cached context with planted keys, plus new rows.

    plants: (row, head, position, gap) tuples.  Plants at positions below 64
    (the first key tile) are applied first; every plant's score for its
    (row, head) is then set to the row's first-tile maximum plus gap log2
    units (gap may be negative)."""

    def __init__(self, rng, pool, heads, kv_heads, dim, ctx, rows, plants, *, rotary=None,
                 theta=1e6, gq=None, first_tile_gap=None):
        self.heads, self.kv_heads, self.dim, self.rows = heads, kv_heads, dim, rows
        rotary = rotary or dim
        g = heads // kv_heads
        width = kv_heads * dim
        self.q = rng.standard_normal((rows, heads * dim)).astype(np.float32)
        self.k = rng.standard_normal((rows, width)).astype(np.float32)
        self.v = rng.standard_normal((rows, width)).astype(np.float32)
        self.pos = np.array([[ctx + r] * 3 for r in range(rows)], np.int32)
        qt = transformed_q(self.q, self.pos, heads, dim, rotary, theta, gq)
        ck = rng.standard_normal((ctx, width)).astype(np.float32)
        cv = rng.standard_normal((ctx, width)).astype(np.float32)
        seen = set()
        for _, h, p, _ in plants:
            key = (p, h // g)
            assert p < ctx and key not in seen, f"plant position {key} reused or past the context"
            seen.add(key)
        ck = O.bf16_round(ck)

        def plant(r, h, p, target):
            kv = h // g
            u = qt[r, h].astype(np.float64)
            # score(r, h) = q . k / sqrt(dim) (math.rs:126) = target
            k = u * (target * math.sqrt(dim) / float(u @ u))
            ck[p, kv * dim:(kv + 1) * dim] = O.bf16_round(k.astype(np.float32))

        def first_max(r, h):
            kv = h // g
            s = ck[:64, kv * dim:(kv + 1) * dim].astype(np.float64) @ qt[r, h].astype(np.float64)
            return float(s.max()) / math.sqrt(dim)

        early = [pl for pl in plants if pl[2] < 64]
        late = [pl for pl in plants if pl[2] >= 64]
        for r, h, p, gap in early:
            plant(r, h, p, first_max(r, h) + gap * LN2)
        for r, h, p, gap in late:
            plant(r, h, p, first_max(r, h) + gap * LN2)
        self.seq = pool.open()
        self.ref = O.KvCache(width, pool._max_tokens, pool.page_tokens, bf16=True)
        cv = O.bf16_round(cv)
        pool.append(self.seq, ck, cv)
        self.ref.append_many(ck, cv)
        self.ctx = ctx


def run_planted(pkg, backend, pool, seqs, *, rotary=None, theta=1e6, gq=None, gk=None,
                expect=(), forbid=()):
    heads, kv_heads, dim = seqs[0].heads, seqs[0].kv_heads, seqs[0].dim
    rotary = rotary or dim
    q = np.concatenate([s.q for s in seqs])
    k = np.concatenate([s.k for s in seqs])
    v = np.concatenate([s.v for s in seqs])
    pos = np.concatenate([s.pos for s in seqs])
    out = np.zeros((q.shape[0], heads * dim), np.float32)
    backend.timing(True)
    try:
        pkg.attention_forward(backend, pool, [s.seq for s in seqs], [s.rows for s in seqs],
                              q, k, v, pos, out, heads=heads, kv_heads=kv_heads, head_dim=dim,
                              rotary_dim=rotary, rope_theta=theta, eps=EPS, q_norm=gq,
                              k_norm=gk)
        ran = backend.kernel_times()
    finally:
        backend.timing(False)
    for name in expect:
        assert name in ran, f"{name} did not run (ran: {sorted(ran)})"
    for name in forbid:
        assert name not in ran, f"{name} ran (ran: {sorted(ran)})"
    r0 = 0
    for s in seqs:
        exp = O.attention_rows(q[r0:r0 + s.rows], k[r0:r0 + s.rows], v[r0:r0 + s.rows],
                               pos[r0:r0 + s.rows].astype(np.int64), s.ref, heads=heads,
                               kv_heads=kv_heads, dim=dim, rotary_dim=rotary, theta=theta,
                               eps=EPS, q_norm=gq, k_norm=gk, threads=ORACLE_THREADS)
        close(out[r0:r0 + s.rows], exp, what=f"seq {s.seq} ctx {s.ctx}")
        r0 += s.rows
    return ran


def gammas(rng, dim):
    return ((1 + 0.02 * rng.standard_normal(dim)).astype(np.float32),
            (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32))


def rising_plants(rows, heads, bands, gaps):
    """Every row gets one plant per band (a band per gap, rising), for the
    query head (7 r) mod heads, at band start + r."""
    out = []
    for r in range(rows):
        h = (7 * r) % heads
        for b0, gap in zip(bands, gaps):
            out.append((r, h, b0 + r, gap))
    return out


def threshold_plants(rows, heads, start, gaps):
    """One plant per row, at gaps[r % len(gaps)], one tile or more after key 0."""
    return [(r, (5 * r + 1) % heads, start + r, gaps[r % len(gaps)]) for r in range(rows)]


def dense_tile_plants(heads, kv_heads, tile_start, gap, rows):
    """For row r < kv_heads: 64 equal planted scores (a whole tile) for the
    first head of KV head r.  Each p is 2^gap, finite in fp16 for gap 10, but
    the tile's sum 64 * 2^gap is not below 2^15."""
    g = heads // kv_heads
    return [(r, r * g, tile_start + j, gap) for r in range(min(rows, kv_heads)) for j in range(64)]


def falling_plants(rows, heads, gaps):
    """A plant inside the first tile (position r < 64): every later tile's
    maximum is far below the kept one."""
    return [(r, (3 * r + 2) % heads, r, gaps[r % len(gaps)]) for r in range(min(rows, 64))]


PP = ("attn_prefill_pp_kernel",)
PIPE = ("attn_prefill_pipe_kernel",)
LOCKSTEP = ("attn_prefill_kernel",)
NOT_DECODE = ("attn_decode_kernel",)


# ---------------------------------------------------------------------------
# prefill: the pipelined kernel (G = 2, 4, 8; head_dim 128; pages >= 64) and
# the ping-pong kernel (G = 1; G = 2, 4 on 16-token pages)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("heads,kv_heads,page,kernel", [(32, 8, 64, PIPE), (8, 8, 64, PP),
                                                        (16, 8, 64, PIPE), (64, 8, 64, PIPE),
                                                        (32, 8, 16, PP)])
def test_prefill_rising_maxima(pkg, backend, rng, heads, kv_heads, page, kernel):
    # every row's maximum rises three times after the first tile: +10, +20
    # and +40 log2 units over its first-tile maximum
    pool = new_pool(pkg, backend, kv_heads, 128, page_tokens=page, max_tokens=1024, seqs=1)
    gq, gk = gammas(rng, 128)
    rows = 128
    plants = rising_plants(rows, heads, (64, 256, 448), (10.0, 20.0, 40.0))
    s = PlantedSeq(rng, pool, heads, kv_heads, 128, 640, rows, plants, gq=gq)
    run_planted(pkg, backend, pool, [s], gq=gq, gk=gk, expect=kernel, forbid=NOT_DECODE)
    pool.destroy()


@pytest.mark.parametrize("page,kernel", [(64, PIPE), (16, PP)])
def test_prefill_thresholds_dense_tile_and_falls(pkg, backend, rng, page, kernel):
    # one call, three sequences at G = 4: single plants across the lazy and
    # fp16-sum thresholds, a whole tile of equal planted scores (sum 2^16
    # with every p finite), and first-tile plants 12 and 40 log2 units above
    # every later key
    heads, kv_heads, dim = 32, 8, 128
    pool = new_pool(pkg, backend, kv_heads, dim, page_tokens=page, max_tokens=1024, seqs=3)
    gq, gk = gammas(rng, dim)
    gaps = (5.0, 7.9, 8.1, 12.0, 14.9, 15.1, 15.9, 16.1, 17.0, 30.0)
    a = PlantedSeq(rng, pool, heads, kv_heads, dim, 400, 96,
                   threshold_plants(96, heads, 128, gaps), gq=gq)
    b = PlantedSeq(rng, pool, heads, kv_heads, dim, 300, 64,
                   dense_tile_plants(heads, kv_heads, 128, 10.0, 64), gq=gq)
    c = PlantedSeq(rng, pool, heads, kv_heads, dim, 500, 80,
                   falling_plants(80, heads, (12.0, 40.0)), gq=gq)
    run_planted(pkg, backend, pool, [a, b, c], gq=gq, gk=gk, expect=kernel, forbid=NOT_DECODE)
    pool.destroy()


# ---------------------------------------------------------------------------
# prefill: the lock-step kernel (G = 3, 5, 7; head_dim 64 and 256), and a
# group of 16 heads (run as two groups of 8 on the pipelined kernel)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("heads,kv_heads,dim,kernel", [(12, 4, 128, LOCKSTEP),
                                                       (10, 2, 128, LOCKSTEP),
                                                       (32, 2, 128, PIPE),
                                                       (14, 2, 64, LOCKSTEP),
                                                       (8, 2, 256, LOCKSTEP)])
def test_lockstep_prefill_rising_thresholds_and_falls(pkg, backend, rng, heads, kv_heads, dim,
                                                      kernel):
    pool = new_pool(pkg, backend, kv_heads, dim, max_tokens=1024, seqs=3)
    gq, gk = gammas(rng, dim)
    a = PlantedSeq(rng, pool, heads, kv_heads, dim, 640, 96,
                   rising_plants(96, heads, (64, 256, 448), (10.0, 20.0, 40.0)), gq=gq)
    gaps = (7.9, 8.1, 9.0, 16.0, 25.0)
    b = PlantedSeq(rng, pool, heads, kv_heads, dim, 300, 40,
                   threshold_plants(40, heads, 96, gaps)
                   + [(r, (5 * r + 1) % heads, 200 + r, gaps[r % len(gaps)] + 9.0)
                      for r in range(40)], gq=gq)
    c = PlantedSeq(rng, pool, heads, kv_heads, dim, 200, 48,
                   falling_plants(48, heads, (12.0, 40.0)), gq=gq)
    run_planted(pkg, backend, pool, [a, b, c], gq=gq, gk=gk, expect=kernel, forbid=NOT_DECODE)
    pool.destroy()


# ---------------------------------------------------------------------------
# MTP verify (2..15 rows): split-K partitions, each with its own maximum
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("heads,kv_heads,rows,dim", [(64, 8, 5, 128), (32, 8, 3, 128),
                                                     (40, 8, 9, 128), (64, 8, 9, 128),
                                                     (16, 2, 5, 256), (16, 2, 9, 256)])
def test_verify_sinks_in_later_partitions(pkg, backend, rng, heads, kv_heads, rows, dim):
    # partitions are at least 256 keys, so a 6000-token context is cut into
    # many; every (row, head) gets a planted key at +10, +20 or +40 log2
    # units somewhere in the context, most of them past the first partition,
    # and a second sequence has first-tile plants above every later key.
    # 64 / 8 with 9 rows runs as two row slices; head_dim 256 splits each
    # workgroup's output dims over two waves that share the softmax
    pool = new_pool(pkg, backend, kv_heads, dim, page_tokens=16, max_tokens=8192, seqs=2)
    gq, gk = gammas(rng, dim)
    ctx = 6000
    plants = []
    gaps = (10.0, 20.0, 40.0)
    for r in range(rows):
        for h in range(heads):
            i = r * heads + h
            plants.append((r, h, 64 + (i * 97) % (ctx - 64), gaps[i % 3]))
    # (position, KV head) pairs must be distinct
    seen, uniq = set(), []
    g = heads // kv_heads
    for pl in plants:
        key = (pl[2], pl[1] // g)
        if key not in seen:
            seen.add(key)
            uniq.append(pl)
    a = PlantedSeq(rng, pool, heads, kv_heads, dim, ctx, rows, uniq, gq=gq)
    b = PlantedSeq(rng, pool, heads, kv_heads, dim, 3000, rows,
                   falling_plants(rows, heads, (12.0, 40.0)), gq=gq)
    run_planted(pkg, backend, pool, [a, b], gq=gq, gk=gk, expect=("attn_verify_kernel",),
                forbid=NOT_DECODE)
    pool.destroy()


# ---------------------------------------------------------------------------
# decode (1 row): split-K segments and the combine kernel
# ---------------------------------------------------------------------------

def test_decode_sinks_in_later_segments(pkg, backend, rng):
    heads, kv_heads, dim = 32, 8, 128
    pool = new_pool(pkg, backend, kv_heads, dim, max_tokens=8192, seqs=4)
    gq, gk = gammas(rng, dim)
    seqs = []
    for n, ctx in enumerate((7000, 3000, 5000)):
        plants = [(0, h, 64 + ((h * 211 + n * 37) % (ctx - 64)), (10.0, 20.0, 40.0)[h % 3])
                  for h in range(heads)]
        seqs.append(PlantedSeq(rng, pool, heads, kv_heads, dim, ctx, 1, plants, gq=gq))
    seqs.append(PlantedSeq(rng, pool, heads, kv_heads, dim, 4000, 1,
                           [(0, h, h, 40.0) for h in range(heads)], gq=gq))
    run_planted(pkg, backend, pool, seqs, gq=gq, gk=gk, expect=("attn_decode_kernel",))
    pool.destroy()


# ---------------------------------------------------------------------------
# BASELINE config 3 at its last chunk: 4 sequences, context 3584, 512 rows
# ---------------------------------------------------------------------------

def test_qwen3_8b_prefill_last_chunk_at_context_3584(pkg, backend, rng):
    # chunk 7 of 4 x 4096 in chunks of 512: rows at positions 3584..4095 see
    # 3585..4096 keys (math.rs:102-155 with the append order of native.rs:637)
    heads, kv_heads, dim, ctx, rows = 32, 8, 128, 3584, 512
    pool = new_pool(pkg, backend, kv_heads, dim, max_tokens=4096, seqs=4)
    gq, gk = gammas(rng, dim)
    seqs = [PlantedSeq(rng, pool, heads, kv_heads, dim, ctx, rows, [], gq=gq) for _ in range(4)]
    for s in seqs:
        s.q = O.bf16_round(s.q)
        s.k = O.bf16_round(s.k)
        s.v = O.bf16_round(s.v)
    run_planted(pkg, backend, pool, seqs, gq=gq, gk=gk, expect=PIPE, forbid=NOT_DECODE)
    pool.destroy()
