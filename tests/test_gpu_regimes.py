"""GPU parity in the regimes the BASELINE shapes run, through the C-ABI.

* MTP verify at BASELINE config 5's context: 131072 cached tokens in 16-token
  pages handed out in a random order (the pool's page_order_seed), four
  sequences so that each key partition of the verify kernel spans about 16k
  keys (the page ids of a partition are staged in LDS);
* calls with more than 64 sequences, which the plugin splits into launches of
  at most 64 (their metadata travels in the kernel arguments), for decode,
  verify and prefill rows in one call;
* errors of an asynchronous call reported by the next synchronous call.

Attention is held to the bf16-path tolerance |d| <= 2e-3 + 1e-2 * |ref|
against the CPU oracle (src/model/math.rs:102-155 with bf16 KV storage).
"""
import zlib
import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_attention import Case, close, new_pool, run_case

pytestmark = pytest.mark.gpu


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def gammas(rng, dim):
    return ((1 + 0.02 * rng.standard_normal(dim)).astype(np.float32),
            (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32))


def test_verify_at_131072_cached_tokens_random_page_order(pkg, backend, rng):
    # 64 Q / 8 KV heads, head_dim 128, 1 + 4 rows, context
    # 131072, page 16, pages in a random permutation of the pool.  The four
    # sequences are forks of one filled cache (shared pages, as after a
    # checkpoint), each verifying its own five rows.
    heads, kvh, dim, ctx, rows, page, nseq = 64, 8, 128, 131072, 5, 16, 4
    width = kvh * dim
    max_tokens = ctx + rows
    pages = (ctx // page) + nseq * 2 + 8
    pool = pkg.KvCache(backend, kvh, dim, page, pages, max_tokens, nseq,
                       page_order_seed=0x5A5A0005)
    ref = O.KvCache(width, max_tokens, page, bf16=True)
    base = pool.open()
    step = 8192
    for start in range(0, ctx, step):
        kk = O.bf16_round(rng.standard_normal((step, width), dtype=np.float32))
        vv = O.bf16_round(rng.standard_normal((step, width), dtype=np.float32))
        pool.append(base, kk, vv)
        ref.append_many(kk, vv)
    seqs = [base] + [pool.fork(base) for _ in range(nseq - 1)]
    gq, gk = gammas(rng, dim)
    q = rng.standard_normal((nseq * rows, heads * dim)).astype(np.float32)
    k = rng.standard_normal((nseq * rows, width)).astype(np.float32)
    v = rng.standard_normal((nseq * rows, width)).astype(np.float32)
    pos = np.array([[ctx + r] * 3 for _ in range(nseq) for r in range(rows)], np.int32)
    out = np.zeros((nseq * rows, heads * dim), np.float32)
    kw = dict(heads=heads, kv_heads=kvh, rotary_dim=dim, eps=1e-6, q_norm=gq, k_norm=gk)
    pkg.attention_forward(backend, pool, seqs, [rows] * nseq, q, k, v, pos, out,
                          head_dim=dim, rope_theta=1e6, **kw)
    for i, s in enumerate(seqs):
        assert pool.len(s) == ctx + rows
        r = slice(i * rows, (i + 1) * rows)
        exp = O.attention_rows(q[r], k[r], v[r], pos[r].astype(np.int64), ref, dim=dim,
                               theta=1e6, threads=16, **kw)
        ref.truncate(ctx)
        close(out[r], exp, what=f"verify sequence {i} at context {ctx}")
    pool.destroy()


def test_decode_call_with_more_than_64_sequences(pkg, backend, rng):
    # 100 sequences of one decode row each: two decode launches (64 + 36), and
    # more page-table entries than travel inline
    nseq = 100
    pool = new_pool(pkg, backend, 8, 128, page_tokens=16, max_tokens=512, seqs=nseq)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, 32, 8, 128, ctx=int(c), rows=1)
             for c in rng.integers(0, 400, size=nseq)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_one_call_with_more_than_64_sequences_per_route(pkg, backend, rng, torch_mod):
    # 70 decode (1 row), 70 verify (2..6 rows) and 70 prefill (16..40 rows)
    # sequences in one call, interleaved: each route splits into launches of
    # at most 64 sequences; device pointers, bf16 inputs
    n = 70
    pool = new_pool(pkg, backend, 8, 128, page_tokens=16, max_tokens=512, seqs=3 * n)
    gq, gk = gammas(rng, 128)
    rows = ([1] * n + [int(r) for r in rng.integers(2, 7, size=n)] +
            [int(r) for r in rng.integers(16, 41, size=n)])
    order = rng.permutation(len(rows))
    cases = [Case(rng, pool, 32, 8, 128, ctx=int(rng.integers(0, 300)), rows=rows[i])
             for i in order]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk, bf16_inputs=True,
             device=True, torch=torch_mod)
    pool.destroy()


def test_async_error_is_reported_by_the_next_synchronous_call(pkg, backend, rng, torch_mod):
    # an ASYNC prefill call whose V holds a value beyond the fp16 operand range
    # advances its sequence and flags the condition; the next synchronous call
    # reports it (before changing anything) instead of taking it for its own,
    # and after the caller truncates and repeats the call synchronously the
    # rows match the oracle
    torch = torch_mod
    pool = new_pool(pkg, backend, 8, 128, max_tokens=512, seqs=3)
    gq, gk = gammas(rng, 128)
    c = Case(rng, pool, 32, 8, 128, ctx=10, rows=32)
    c.v[3, 9] = -3.0e5
    other = Case(rng, pool, 32, 8, 128, ctx=40, rows=20)
    kw = dict(heads=32, kv_heads=8, head_dim=128, rotary_dim=128, rope_theta=1e6)
    tq, tk, tv = (torch.from_numpy(x).cuda() for x in (c.q, c.k, c.v))
    tp = torch.from_numpy(c.pos).cuda()
    to = torch.zeros((32, 32 * 128), device="cuda")
    tgq, tgk = torch.from_numpy(gq).cuda(), torch.from_numpy(gk).cuda()
    pkg.attention_forward(backend, pool, [c.seq], [32], tq, tk, tv, tp, to, q_norm=tgq,
                          k_norm=tgk, asynchronous=True, **kw)
    assert pool.len(c.seq) == 42
    out = np.zeros((20, 32 * 128), np.float32)
    with pytest.raises(pkg.PluginError) as err:
        pkg.attention_forward(backend, pool, [other.seq], [20], other.q, other.k, other.v,
                              other.pos, out, q_norm=gq, k_norm=gk, **kw)
    assert "fp16 range" in str(err.value)
    assert pool.len(other.seq) == 40  # the failing call changed nothing
    # the report cleared the condition: the same call now runs
    run_case(pkg, backend, pool, [other], rotary=128, gq=gq, gk=gk)
    pool.truncate(c.seq, 10)
    run_case(pkg, backend, pool, [c], rotary=128, gq=gq, gk=gk)
    assert pool.len(c.seq) == 42
    pool.destroy()
