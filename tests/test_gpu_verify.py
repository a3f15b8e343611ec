"""GPU parity of the multi-row (MTP verify) path, through the C-ABI.

Calls with 2..15 rows for a sequence take the split-K verify kernel: each
cached K/V tile is read once for all rows and query heads of a workgroup, on
MFMA, and partition records are merged by a combine pass.  A workgroup holds
up to 64 query vectors (rows x heads/kv_heads); beyond that the rows run as
slices of 64 / G rows (1 + 8 drafts at G = 8: two slices).  head_dim 64, 128
and 256 (Qwen3.5 full attention, whose MTP the reference runs:
src/model/mtp.rs:110-112).  Row r of a sequence sees its context plus rows
0..r (src/model/native.rs:637-638).  Checked against the CPU oracle with bf16
KV storage at |d| <= 2e-3 + 1e-2 * |ref|, and the kernels that ran are
checked (no row falls back to the row-serial decode kernel).
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


def gammas(rng, dim):
    return ((1 + 0.02 * rng.standard_normal(dim)).astype(np.float32),
            (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32))


def interleaved_cases(rng, pool, heads, kvh, dim, ctxs, rows, chunk=16):
    """Sequences whose cached pages interleave (appended chunk by chunk in a
    random sequence order), like a long-running server's paged pool."""
    cases = [Case(rng, pool, heads, kvh, dim, ctx=0, rows=r) for r in rows]
    width = kvh * dim
    remaining = list(ctxs)
    filled = [0] * len(cases)
    while any(remaining):
        order = [i for i in range(len(cases)) if remaining[i]]
        rng.shuffle(order)
        for i in order:
            n = min(chunk * int(rng.integers(1, 4)), remaining[i])
            kk = O.bf16_round(rng.standard_normal((n, width)).astype(np.float32))
            vv = O.bf16_round(rng.standard_normal((n, width)).astype(np.float32))
            pool.append(cases[i].seq, kk, vv)
            cases[i].ref.append_many(kk, vv)
            remaining[i] -= n
            filled[i] += n
    for c, n in zip(cases, filled):
        c.pos = np.array([[n + r] * 3 for r in range(c.rows)], np.int32)
    return cases


@pytest.mark.parametrize("rows", [2, 5, 8])
def test_verify_qwen3_32b_shape_interleaved_pages(pkg, backend, rng, rows):
    # BASELINE config 5 geometry (64 Q / 8 KV heads, head_dim 128, 16-token
    # pages spread over the pool) at a few thousand tokens of context
    pool = new_pool(pkg, backend, 8, 128, page_tokens=16, max_tokens=4096, seqs=4)
    gq, gk = gammas(rng, 128)
    cases = interleaved_cases(rng, pool, 64, 8, 128, [3000, 1777, 64, 0], [rows] * 4)
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_verify_gqa4_up_to_15_rows_and_mixed_batch(pkg, backend, rng):
    pool = new_pool(pkg, backend, 8, 128, page_tokens=64, max_tokens=8192, seqs=4)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, 32, 8, 128, ctx=5000, rows=15),
             Case(rng, pool, 32, 8, 128, ctx=700, rows=3),
             Case(rng, pool, 32, 8, 128, ctx=20, rows=1),
             Case(rng, pool, 32, 8, 128, ctx=255, rows=9)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_verify_gated_and_small_head_dim(pkg, backend, rng):
    # Qwen3.5-style gate at head_dim 128 and a Qwen2-style head_dim 64 (G 7)
    pool = new_pool(pkg, backend, 4, 128, max_tokens=2048, seqs=2)
    gq = (0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(128)).astype(np.float32)
    cases = [Case(rng, pool, 16, 4, 128, ctx=900, rows=4, gated=True),
             Case(rng, pool, 16, 4, 128, ctx=33, rows=6, gated=True)]
    run_case(pkg, backend, pool, cases, rotary=128, theta=1e7, gq=gq, gk=gk, gated=True,
             offset=True)
    pool.destroy()
    pool = new_pool(pkg, backend, 2, 64, page_tokens=32, max_tokens=2048, seqs=2)
    cases = [Case(rng, pool, 14, 2, 64, ctx=1000, rows=9, qk_norm=False),
             Case(rng, pool, 14, 2, 64, ctx=5, rows=2, qk_norm=False)]
    run_case(pkg, backend, pool, cases, rotary=64)
    pool.destroy()


def test_verify_equals_row_by_row_decode(pkg, backend, rng):
    # invariant (speculative.rs:201-202): verifying the drafts in one call ==
    # feeding them one decode step at a time
    heads, kvh, dim, ctx, rows = 64, 8, 128, 2500, 5
    pool = new_pool(pkg, backend, kvh, dim, page_tokens=16, max_tokens=4096, seqs=2)
    gq, gk = gammas(rng, dim)
    base = pool.open()
    ck = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    cv = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    pool.append(base, ck, cv)
    fork = pool.fork(base)
    q = rng.standard_normal((rows, heads * dim)).astype(np.float32)
    k = rng.standard_normal((rows, kvh * dim)).astype(np.float32)
    v = rng.standard_normal((rows, kvh * dim)).astype(np.float32)
    pos = np.array([[ctx + r] * 3 for r in range(rows)], np.int32)
    kw = dict(heads=heads, kv_heads=kvh, head_dim=dim, rotary_dim=dim, rope_theta=1e6,
              q_norm=gq, k_norm=gk)
    whole = np.zeros((rows, heads * dim), np.float32)
    pkg.attention_forward(backend, pool, [base], [rows], q, k, v, pos, whole, **kw)
    single = np.zeros_like(whole)
    for r in range(rows):
        o = np.zeros((1, heads * dim), np.float32)
        pkg.attention_forward(backend, pool, [fork], [1], q[r:r + 1], k[r:r + 1], v[r:r + 1],
                              pos[r:r + 1], o, **kw)
        single[r] = o[0]
    close(whole, single, what="verify vs row-by-row decode")
    ka, va = pool.read(base)
    kb, vb = pool.read(fork)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    pool.destroy()


def test_verify_beyond_fp16_range_recomputes(pkg, backend, rng):
    pool = new_pool(pkg, backend, 8, 128, max_tokens=1024, seqs=2)
    gq, gk = gammas(rng, 128)
    a = Case(rng, pool, 32, 8, 128, ctx=300, rows=5)
    a.v[2, 40] = 1.0e5
    run_case(pkg, backend, pool, [a], rotary=128, gq=gq, gk=gk)
    pool.destroy()


def run_verify_only(pkg, backend, pool, cases, **kw):
    """run_case, asserting that the call took the verify kernel and no
    row-serial decode launch."""
    backend.timing(True)
    try:
        out = run_case(pkg, backend, pool, cases, **kw)
        ran = backend.kernel_times()
    finally:
        backend.timing(False)
    assert "attn_verify_kernel" in ran and "attn_decode_kernel" not in ran, sorted(ran)
    return out


@pytest.mark.parametrize("rows", [5, 9])
def test_verify_qwen35_head_dim_256(pkg, backend, rng, rows):
    # Qwen3.5 full-attention geometry, the model the reference's MTP runs
    # (mtp.rs:110-112): 16 Q / 2 KV heads (G = 8), head_dim 256, q/gate
    # interleaved, norm offset, partial rotary 64 with interleaved MRoPE,
    # theta 1e7; 1 + 4 and 1 + 8 drafts (speculative.rs:12 caps drafts at 8):
    # 40 and 72 query vectors per KV head, the latter in two row slices
    pool = new_pool(pkg, backend, 2, 256, page_tokens=16, max_tokens=4096, seqs=3)
    gq = (0.02 * rng.standard_normal(256)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(256)).astype(np.float32)
    cases = interleaved_cases(rng, pool, 16, 2, 256, [3000, 777, 40], [rows] * 3)
    for c in cases:
        c.q = rng.standard_normal((c.rows, 16 * 256 * 2)).astype(np.float32)
        p0 = int(c.pos[0, 0])
        c.pos = np.array([[p0 + r, p0 + r + 3, p0 + r + 7] for r in range(c.rows)], np.int32)
    run_verify_only(pkg, backend, pool, cases, rotary=64, theta=1e7, gq=gq, gk=gk, gated=True,
                    offset=True, mrope=(11, 11, 10))
    pool.destroy()


@pytest.mark.parametrize("rows", [9, 15])
def test_verify_more_than_64_query_vectors(pkg, backend, rng, rows):
    # 64 Q / 8 KV heads (G = 8) at head_dim 128: 1 + 8 drafts (72 vectors)
    # and 15 rows (120), two row slices of 8 rows each
    pool = new_pool(pkg, backend, 8, 128, page_tokens=16, max_tokens=4096, seqs=3)
    gq, gk = gammas(rng, 128)
    cases = interleaved_cases(rng, pool, 64, 8, 128, [2500, 300, 0], [rows, rows, 2])
    run_verify_only(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


@pytest.mark.parametrize("heads,kvh,dim,rows", [(64, 8, 128, 9), (16, 2, 256, 9),
                                                 (16, 2, 256, 5)])
def test_sliced_and_wide_verify_equal_row_by_row_decode(pkg, backend, rng, heads, kvh, dim, rows):
    # speculative.rs:201-202: verifying the drafts in one call == feeding them
    # one decode step at a time, for the row-sliced and head_dim 256 forms
    ctx = 1900
    pool = new_pool(pkg, backend, kvh, dim, page_tokens=16, max_tokens=4096, seqs=2)
    gq, gk = gammas(rng, dim)
    base = pool.open()
    ck = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    cv = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    pool.append(base, ck, cv)
    fork = pool.fork(base)
    q = rng.standard_normal((rows, heads * dim)).astype(np.float32)
    k = rng.standard_normal((rows, kvh * dim)).astype(np.float32)
    v = rng.standard_normal((rows, kvh * dim)).astype(np.float32)
    pos = np.array([[ctx + r] * 3 for r in range(rows)], np.int32)
    kw = dict(heads=heads, kv_heads=kvh, head_dim=dim, rotary_dim=dim, rope_theta=1e6,
              q_norm=gq, k_norm=gk)
    whole = np.zeros((rows, heads * dim), np.float32)
    pkg.attention_forward(backend, pool, [base], [rows], q, k, v, pos, whole, **kw)
    single = np.zeros_like(whole)
    for r in range(rows):
        o = np.zeros((1, heads * dim), np.float32)
        pkg.attention_forward(backend, pool, [fork], [1], q[r:r + 1], k[r:r + 1], v[r:r + 1],
                              pos[r:r + 1], o, **kw)
        single[r] = o[0]
    close(whole, single, what="verify vs row-by-row decode")
    pool.destroy()
