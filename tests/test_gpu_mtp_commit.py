"""MTP commit without a re-forward, through the C-ABI.

The reference's decode_round verifies 1 + d draft rows on the target model,
accepts the first j of them (greedy), restores the checkpoint and runs the j
committed tokens through the model again (src/engine/speculative.rs:176-259,
the re-forward at :242-247).  Here the verify call leaves enough behind to
land on "state after row j" directly:

* attention layers: kv_truncate to the context plus j rows;
* GDN layers: a KEEP_ROWS gdn_forward (which records each row's decay,
  correction and key and keeps the pre-call state buffer), then gdn_rollback.

The tests check the rolled-back GDN state and conv history against the
oracle run of the first j rows from the pre-call snapshot (|d| <= 1e-4 +
1e-4 |ref|, the history bit for bit) and against re-forwarding those rows on
a fork (bit for bit: the rollback applies the forward's element-wise
operations), and that decoding continues from there as the oracle does.
"""
import zlib
import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_gdn import Layer, close, oracle_rows, plugin_rows
from test_gpu_attention import ATOL, RTOL, new_pool

pytestmark = pytest.mark.gpu


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


def gdn_rows_keep(pkg, backend, pool, L, seqs, rows, x):
    qkv, z, a, b = x
    out = np.zeros((qkv.shape[0], L.hv * L.dv), np.float32)
    pkg.gdn_forward(backend, pool, seqs, rows, qkv, z, a, b, L.a_log, L.dt_bias, L.conv, L.norm,
                    out, eps=1e-6, keep_rows=True)
    return out


def rows_of(x, lo, hi):
    return tuple(t[lo:hi] for t in x)


def test_gdn_rollback_to_every_row_of_a_verify_call(pkg, backend, rng):
    L = Layer(rng, 2, 4, 128, 128, 4)
    pool = pkg.GdnState(backend, 2, 4, 128, 128, 4, 8, keep_rows=8)
    s = pool.open()
    # context: 20 rows (chunked prefill path), then a snapshot for the checks
    plugin_rows(pkg, backend, pool, L, [s], [20], L.inputs(rng, 20))
    snap_m, snap_h = pool.read(s)
    pre = pool.fork(s)
    x = L.inputs(rng, 5)
    out = gdn_rows_keep(pkg, backend, pool, L, [s], [5], x)
    state, hist = snap_m.copy(), snap_h.copy()
    close(out, oracle_rows(L, x, state, hist), what="KEEP_ROWS outputs")
    for j in (2, 0, 5, 4, 1, 3):
        pool.rollback(s, j)
        m, h = pool.read(s)
        st, hi = snap_m.copy(), snap_h.copy()
        if j:
            oracle_rows(L, rows_of(x, 0, j), st, hi)
        close(m, st, what=f"state after rollback to row {j}")
        assert np.array_equal(h, hi), f"history after rollback to row {j}"
        f = pool.fork(pre)
        if j:
            plugin_rows(pkg, backend, pool, L, [f], [j], rows_of(x, 0, j))
        fm, fh = pool.read(f)
        assert np.array_equal(m, fm), f"rollback to row {j} differs from re-forwarding {j} rows"
        assert np.array_equal(h, fh)
        pool.close(f)
    # commit 3 rows, then decode on: the same as the oracle from state 3
    pool.rollback(s, 3)
    st, hi = snap_m.copy(), snap_h.copy()
    oracle_rows(L, rows_of(x, 0, 3), st, hi)
    nxt = L.inputs(rng, 1)
    got = plugin_rows(pkg, backend, pool, L, [s], [1], nxt)
    close(got, oracle_rows(L, nxt, st, hi), what="decode after the commit")
    m, h = pool.read(s)
    close(m, st, what="state after the commit and one decode")
    assert np.array_equal(h, hi)
    pool.destroy()


def test_gdn_rollback_batch_and_errors(pkg, backend, rng):
    L = Layer(rng, 2, 4, 128, 128, 4)
    pool = pkg.GdnState(backend, 2, 4, 128, 128, 4, 6, keep_rows=6)
    seqs = [pool.open() for _ in range(3)]
    snaps = []
    for s in seqs:
        plugin_rows(pkg, backend, pool, L, [s], [3], L.inputs(rng, 3))
        snaps.append(pool.read(s))
    rows = [6, 1, 4]
    x = L.inputs(rng, sum(rows))
    gdn_rows_keep(pkg, backend, pool, L, seqs, rows, x)
    r0 = 0
    for s, r, (sm, sh), j in zip(seqs, rows, snaps, (3, 0, 4)):
        pool.rollback(s, j)
        m, h = pool.read(s)
        st, hi = sm.copy(), sh.copy()
        if j:
            oracle_rows(L, rows_of(x, r0, r0 + j), st, hi)
        close(m, st, what=f"sequence {s} rolled back to row {j}")
        assert np.array_equal(h, hi)
        r0 += r
    with pytest.raises(pkg.PluginError):
        pool.rollback(seqs[0], 7)                       # more rows than the call had
    plugin_rows(pkg, backend, pool, L, [seqs[0]], [1], L.inputs(rng, 1))
    with pytest.raises(pkg.PluginError):
        pool.rollback(seqs[0], 0)                       # last call was not KEEP_ROWS
    with pytest.raises(pkg.PluginError):
        gdn_rows_keep(pkg, backend, pool, L, [seqs[1]], [7], L.inputs(rng, 7))  # > keep_rows
    plain = pkg.GdnState(backend, 2, 4, 128, 128, 4, 1)
    p = plain.open()
    with pytest.raises(pkg.PluginError):
        gdn_rows_keep(pkg, backend, plain, L, [p], [2], L.inputs(rng, 2))  # no keep_rows
    plain.destroy()
    pool.destroy()


def test_hybrid_commit_attention_truncate_and_gdn_rollback(pkg, backend, rng):
    # one attention layer (Qwen3.5 full-attention geometry at small size) and
    # one GDN layer verify 1 + 4 rows; the first 2 are accepted; after
    # kv_truncate and gdn_rollback the next decode token of both layers equals
    # the oracle's decode after the 2 committed rows
    heads, kvh, dim, ctx, rows, j = 16, 4, 128, 300, 5, 2
    kv = new_pool(pkg, backend, kvh, dim, page_tokens=16, max_tokens=1024, seqs=2)
    seq = kv.open()
    ref = O.KvCache(kvh * dim, 1024, 16, bf16=True)
    ck = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    cv = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    kv.append(seq, ck, cv)
    ref.append_many(ck, cv)
    gq = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    kw = dict(heads=heads, kv_heads=kvh, head_dim=dim, rotary_dim=64, rope_theta=1e7,
              q_norm=gq, k_norm=gk, gated=True, norm_offset=True)
    okw = dict(heads=heads, kv_heads=kvh, dim=dim, rotary_dim=64, theta=1e7, q_norm=gq,
               k_norm=gk, gated=True, threads=8)
    q = rng.standard_normal((rows + 1, heads * dim * 2)).astype(np.float32)
    k = rng.standard_normal((rows + 1, kvh * dim)).astype(np.float32)
    v = rng.standard_normal((rows + 1, kvh * dim)).astype(np.float32)
    pos = np.array([[ctx + r] * 3 for r in range(rows)] + [[ctx + j] * 3], np.int32)
    out = np.zeros((rows, heads * dim), np.float32)
    pkg.attention_forward(backend, kv, [seq], [rows], q[:rows], k[:rows], v[:rows], pos[:rows],
                          out, **kw)
    L = Layer(rng, 2, 4, 128, 128, 4)
    gdn = pkg.GdnState(backend, 2, 4, 128, 128, 4, 2, keep_rows=8)
    g = gdn.open()
    plugin_rows(pkg, backend, gdn, L, [g], [7], L.inputs(rng, 7))
    gm, gh = gdn.read(g)
    x = L.inputs(rng, rows)
    gdn_rows_keep(pkg, backend, gdn, L, [g], [rows], x)
    # commit j rows: truncate the cache, roll the recurrent state back
    kv.truncate(seq, ctx + j)
    gdn.rollback(g, j)
    # next token (it follows the j committed rows)
    a1 = np.zeros((1, heads * dim), np.float32)
    pkg.attention_forward(backend, kv, [seq], [1], q[rows:], k[rows:], v[rows:], pos[rows:],
                          a1, **kw)
    nxt = L.inputs(rng, 1)
    g1 = plugin_rows(pkg, backend, gdn, L, [g], [1], nxt)
    # oracle: the j committed rows, then the next row
    O.attention_rows(q[:j], k[:j], v[:j], pos[:j].astype(np.int64), ref, **okw)
    exp_a = O.attention_rows(q[rows:], k[rows:], v[rows:], pos[rows:].astype(np.int64), ref,
                             **okw)
    err = np.abs(a1 - exp_a)
    assert (err <= ATOL + RTOL * np.abs(exp_a)).all(), err.max()
    st, hi = gm.copy(), gh.copy()
    oracle_rows(L, rows_of(x, 0, j), st, hi)
    close(g1, oracle_rows(L, nxt, st, hi), what="GDN decode after the commit")
    assert kv.len(seq) == ctx + j + 1
    kv.destroy()
    gdn.destroy()
