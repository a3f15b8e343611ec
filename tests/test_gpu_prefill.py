"""GPU parity of the chunked-prefill path (MFMA kernels), through the C-ABI.

Calls with at least 16 new rows for a sequence take the prefill kernels: the
rows' K/V are appended first, then every row attends causally to the context
plus the rows before it (src/model/native.rs:627-643, math.rs:102-155).  Each
case is checked against the CPU oracle on the same seeded inputs with bf16 KV
storage, at the bf16-path tolerance |d| <= 2e-3 + 1e-2 * |ref|.
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
    gq = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    return gq, gk


@pytest.mark.parametrize("page", [16, 64])
def test_qwen3_8b_prefill_chunks_host_pointers(pkg, backend, rng, page):
    # BASELINE prefill geometry (32 Q / 8 KV, head_dim 128, QK-norm + RoPE
    # theta 1e6) at small lengths: a fresh prompt and a chunk after a context
    # that ends mid-page and mid-tile
    pool = new_pool(pkg, backend, 8, 128, page_tokens=page, max_tokens=2048, seqs=2)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, 32, 8, 128, ctx=0, rows=130),
             Case(rng, pool, 32, 8, 128, ctx=515, rows=64)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_qwen3_8b_prefill_bf16_device_pointers(pkg, backend, rng, torch_mod):
    pool = new_pool(pkg, backend, 8, 128, max_tokens=4096, seqs=3)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, 32, 8, 128, ctx=1024, rows=512),
             Case(rng, pool, 32, 8, 128, ctx=37, rows=200),
             Case(rng, pool, 32, 8, 128, ctx=0, rows=16)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk, bf16_inputs=True,
             device=True, torch=torch_mod)
    pool.destroy()


@pytest.mark.parametrize("heads,kv_heads", [(8, 8), (8, 4), (12, 4), (10, 2), (24, 4), (32, 4)])
def test_prefill_gqa_group_sizes(pkg, backend, rng, heads, kv_heads):
    # G = 1, 2, 3, 5, 6, 8 query heads per KV head (a workgroup holds G heads,
    # and 4/G row blocks when G < 4)
    pool = new_pool(pkg, backend, kv_heads, 128, max_tokens=1024, seqs=2)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, heads, kv_heads, 128, ctx=77, rows=150),
             Case(rng, pool, heads, kv_heads, 128, ctx=300, rows=33)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


@pytest.mark.parametrize("heads,kv_heads,rotary", [(16, 8, 64), (32, 8, 96), (16, 4, 32)])
def test_prefill_partial_rotary_group_sizes(pkg, backend, rng, heads, kv_heads, rotary):
    # head_dim 128 with partial rotary (math.rs:52-99: dims past rotary_dim
    # unrotated) for G = 2 and 4, where the workgroup's RoPE table is staged
    # in LDS for the q side
    pool = new_pool(pkg, backend, kv_heads, 128, max_tokens=1024, seqs=2)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, heads, kv_heads, 128, ctx=77, rows=150),
             Case(rng, pool, heads, kv_heads, 128, ctx=300, rows=33)]
    run_case(pkg, backend, pool, cases, rotary=rotary, gq=gq, gk=gk)
    pool.destroy()


def test_qwen2_shape_prefill_without_qk_norm(pkg, backend, rng):
    # Qwen2-0.5B attention: 14 Q / 2 KV heads (G = 7), head_dim 64, no QK-norm
    pool = new_pool(pkg, backend, 2, 64, page_tokens=32, max_tokens=1024, seqs=2)
    cases = [Case(rng, pool, 14, 2, 64, ctx=30, rows=50, qk_norm=False),
             Case(rng, pool, 14, 2, 64, ctx=511, rows=100, qk_norm=False)]
    run_case(pkg, backend, pool, cases, rotary=64)
    pool.destroy()


def test_qwen35_gated_partial_rope_prefill(pkg, backend, rng):
    # Qwen3.5 full-attention layer: q/gate interleaved per head, norm offset,
    # head_dim 256 with rotary_dim 64, interleaved MRoPE sections, theta 1e7
    pool = new_pool(pkg, backend, 2, 256, max_tokens=1024, seqs=2)
    gq = (0.02 * rng.standard_normal(256)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(256)).astype(np.float32)
    cases = [Case(rng, pool, 8, 2, 256, ctx=100, rows=40, gated=True, pos_axes=(0, 3, 7)),
             Case(rng, pool, 8, 2, 256, ctx=0, rows=70, gated=True, pos_axes=(0, 3, 7))]
    run_case(pkg, backend, pool, cases, rotary=64, theta=1e7, gq=gq, gk=gk, gated=True,
             offset=True, mrope=(11, 11, 10))
    pool.destroy()


@pytest.mark.parametrize("heads,kv_heads,gated,qk_norm", [(16, 4, True, True),
                                                          (16, 8, True, True),
                                                          (32, 4, False, False)])
def test_head_dim_128_gate_mrope_offset_and_no_norm(pkg, backend, rng, heads, kv_heads,
                                                    gated, qk_norm):
    # head_dim 128 at page 64 (the pipelined kernel's shapes, G = 4, 2, 8):
    # the per-head q/gate interleave with the sigmoid gate on the output,
    # MRoPE sections over a partial rotary span with the norm offset, and a
    # layer without QK-norm
    pool = new_pool(pkg, backend, kv_heads, 128, max_tokens=1024, seqs=2)
    if qk_norm:
        gq = (0.02 * rng.standard_normal(128)).astype(np.float32)
        gk = (0.02 * rng.standard_normal(128)).astype(np.float32)
        extra = dict(rotary=96, theta=1e7, gq=gq, gk=gk, offset=True, mrope=(16, 16, 16))
        axes = (0, 3, 7)
    else:
        extra = dict(rotary=128)
        axes = None
    cases = [Case(rng, pool, heads, kv_heads, 128, ctx=100, rows=70, gated=gated,
                  qk_norm=qk_norm, pos_axes=axes),
             Case(rng, pool, heads, kv_heads, 128, ctx=0, rows=150, gated=gated,
                  qk_norm=qk_norm, pos_axes=axes)]
    backend.timing(True)
    try:
        run_case(pkg, backend, pool, cases, gated=gated, **extra)
        ran = backend.kernel_times()
    finally:
        backend.timing(False)
    assert "attn_prefill_pipe_kernel" in ran, sorted(ran)
    pool.destroy()


def test_mixed_batch_prefill_decode_and_verify_rows(pkg, backend, rng):
    # one call: a prefill chunk, a decode row and a 5-row verify block
    pool = new_pool(pkg, backend, 8, 128, max_tokens=2048, seqs=3)
    gq, gk = gammas(rng, 128)
    cases = [Case(rng, pool, 32, 8, 128, ctx=200, rows=96),
             Case(rng, pool, 32, 8, 128, ctx=1500, rows=1),
             Case(rng, pool, 32, 8, 128, ctx=640, rows=5)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


@pytest.mark.parametrize("heads,kv_heads,dim,page", [(32, 2, 128, 16), (24, 2, 128, 64),
                                                     (18, 2, 128, 64), (22, 2, 64, 16),
                                                     (64, 4, 128, 64)])
def test_gqa_groups_larger_than_8(pkg, backend, rng, heads, kv_heads, dim, page):
    # math.rs:109-127 takes any heads that kv_heads divides: query head h
    # reads KV head h / (heads / kv_heads).  Groups of G = 16, 12, 9, 11 and
    # 16 query heads (64 / 4, the Qwen3-235B shape) run as groups of at most
    # 8 sharing one cache head; one call holds a prefill chunk, a decode row
    # and a verify block (3 rows), each against the oracle.
    pool = new_pool(pkg, backend, kv_heads, dim, page_tokens=page, max_tokens=1024, seqs=5)
    gq, gk = gammas(rng, dim)
    cases = [Case(rng, pool, heads, kv_heads, dim, ctx=150, rows=40),
             Case(rng, pool, heads, kv_heads, dim, ctx=333, rows=1),
             Case(rng, pool, heads, kv_heads, dim, ctx=97, rows=3)]
    run_case(pkg, backend, pool, cases, rotary=dim, gq=gq, gk=gk)
    # decode and 2-row verify calls of their own (no prefill row in the call,
    # so their page-table entries travel in the append kernel's arguments)
    more = [Case(rng, pool, heads, kv_heads, dim, ctx=500, rows=1),
            Case(rng, pool, heads, kv_heads, dim, ctx=64, rows=2)]
    run_case(pkg, backend, pool, more, rotary=dim, gq=gq, gk=gk)
    pool.destroy()


def test_prefill_whole_equals_chunked_then_decode(pkg, backend, rng):
    # invariants (native.rs:431-455): one 96-row call == chunks of 32 + 64,
    # and a decode row after either matches the oracle
    heads, kvh, dim, ctx, rows = 32, 8, 128, 70, 96
    pool = new_pool(pkg, backend, kvh, dim, max_tokens=1024, seqs=2)
    gq, gk = gammas(rng, dim)
    base = pool.open()
    ck = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    cv = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    pool.append(base, ck, cv)
    fork = pool.fork(base)
    q = rng.standard_normal((rows + 1, heads * dim)).astype(np.float32)
    k = rng.standard_normal((rows + 1, kvh * dim)).astype(np.float32)
    v = rng.standard_normal((rows + 1, kvh * dim)).astype(np.float32)
    pos = np.array([[ctx + r] * 3 for r in range(rows + 1)], np.int32)
    kw = dict(heads=heads, kv_heads=kvh, head_dim=dim, rotary_dim=dim, rope_theta=1e6,
              q_norm=gq, k_norm=gk)
    whole = np.zeros((rows, heads * dim), np.float32)
    pkg.attention_forward(backend, pool, [base], [rows], q[:rows], k[:rows], v[:rows],
                          pos[:rows], whole, **kw)
    chunked = np.zeros_like(whole)
    for a, b in ((0, 32), (32, 96)):
        o = np.zeros((b - a, heads * dim), np.float32)
        pkg.attention_forward(backend, pool, [fork], [b - a], q[a:b], k[a:b], v[a:b], pos[a:b],
                              o, **kw)
        chunked[a:b] = o
    close(chunked, whole, atol=1e-6, rtol=1e-6, what="chunked vs whole")
    ref = O.KvCache(kvh * dim, 1024, 64, bf16=True)
    ref.append_many(ck, cv)
    exp = O.attention_rows(q, k, v, pos.astype(np.int64), ref, heads=heads, kv_heads=kvh,
                           dim=dim, rotary_dim=dim, theta=1e6, eps=1e-6, q_norm=gq, k_norm=gk,
                           threads=8)
    close(whole, exp[:rows], what="whole vs oracle")
    for seq in (base, fork):
        o = np.zeros((1, heads * dim), np.float32)
        pkg.attention_forward(backend, pool, [seq], [1], q[rows:], k[rows:], v[rows:],
                              pos[rows:], o, **kw)
        close(o, exp[rows:], what="decode after prefill")
    assert pool.len(base) == pool.len(fork) == ctx + rows + 1
    pool.destroy()


def test_prefill_rejects_non_finite_and_keeps_lengths(pkg, backend, rng):
    pool = new_pool(pkg, backend, 8, 128, max_tokens=512, seqs=2)
    gq, gk = gammas(rng, 128)
    a = Case(rng, pool, 32, 8, 128, ctx=40, rows=20)
    b = Case(rng, pool, 32, 8, 128, ctx=10, rows=33)
    kw = dict(heads=32, kv_heads=8, head_dim=128, rotary_dim=128, rope_theta=1e6, q_norm=gq,
              k_norm=gk)
    q = np.concatenate([a.q, b.q])
    k = np.concatenate([a.k, b.k])
    v = np.concatenate([a.v, b.v])
    pos = np.concatenate([a.pos, b.pos])
    out = np.zeros((53, 32 * 128), np.float32)
    bad_v = v.copy()
    bad_v[30, 5] = np.nan           # a row of the second sequence (state.rs:56-58)
    with pytest.raises(pkg.PluginError) as err:
        pkg.attention_forward(backend, pool, [a.seq, b.seq], [20, 33], q, k, bad_v, pos, out,
                              **kw)
    assert err.value.status == 1
    assert pool.len(a.seq) == 40 and pool.len(b.seq) == 10
    bad_q = q.copy()
    bad_q[3, :128] = np.inf         # non-finite norm variance (math.rs:39-41)
    with pytest.raises(pkg.PluginError) as err:
        pkg.attention_forward(backend, pool, [a.seq, b.seq], [20, 33], bad_q, k, v, pos, out,
                              **kw)
    assert err.value.status == 1
    assert pool.len(a.seq) == 40 and pool.len(b.seq) == 10
    # the same call with clean inputs matches the oracle
    run_case(pkg, backend, pool, [a, b], rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_prefill_values_beyond_fp16_range_are_recomputed(pkg, backend, rng, torch_mod):
    # finite bf16 K/V beyond the fp16 operand range of the MFMA kernel: a
    # synchronous call recomputes those rows on the f32 split-K path and
    # still matches the oracle; an asynchronous call reports the condition
    pool = new_pool(pkg, backend, 8, 128, max_tokens=512, seqs=3)
    gq, gk = gammas(rng, 128)
    a = Case(rng, pool, 32, 8, 128, ctx=50, rows=40)
    b = Case(rng, pool, 32, 8, 128, ctx=20, rows=24)
    a.v[7, 130] = 2.0e5           # a value row 7.. of sequence a attends to
    run_case(pkg, backend, pool, [a, b], rotary=128, gq=gq, gk=gk)
    assert pool.len(a.seq) == 90 and pool.len(b.seq) == 44

    c = Case(rng, pool, 32, 8, 128, ctx=10, rows=32)
    c.v[3, 9] = -3.0e5
    torch = torch_mod
    tq, tk, tv = (torch.from_numpy(x).cuda() for x in (c.q, c.k, c.v))
    tp = torch.from_numpy(c.pos).cuda()
    to = torch.zeros((32, 32 * 128), device="cuda")
    pkg.attention_forward(backend, pool, [c.seq], [32], tq, tk, tv, tp, to, heads=32,
                          kv_heads=8, head_dim=128, rotary_dim=128, rope_theta=1e6,
                          q_norm=torch.from_numpy(gq).cuda(), k_norm=torch.from_numpy(gk).cuda(),
                          asynchronous=True)
    with pytest.raises(pkg.PluginError) as err:
        backend.synchronize()
    assert "fp16 range" in str(err.value)
    pool.destroy()
