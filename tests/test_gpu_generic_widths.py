"""GPU parity at head widths the tuned kernels are not built for, through the C-ABI.

The reference takes any attention head_dim (src/model/math.rs:109-124) and
any GDN key/value width (math.rs:201-210); its own tests run head_dim 4 and
8 and GDN widths 2 and 3 (src/model/spec.rs:539, :567-572).  Head widths other
than 64/128/256, GDN key widths other than 128 and value widths that are not
a multiple of 16 run on the plain f32 kernels (attn_generic.hip,
gdn_generic_kernel).  Tolerances as the tuned paths: attention
|d| <= 2e-3 + 1e-2 |ref| (bf16 KV storage), GDN |d| <= 1e-4 + 1e-4 |ref|.
"""
import zlib

import numpy as np
import pytest

from oracle import pyoracle as O
from test_gpu_attention import Case, close as attn_close, new_pool, run_case
from test_gpu_gdn import Layer, close as gdn_close, oracle_rows, plugin_rows

pytestmark = pytest.mark.gpu


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dim,heads,kvh,rotary", [(4, 4, 2, 4), (8, 2, 1, 4), (2, 3, 1, 2),
                                                  (80, 16, 4, 80), (96, 12, 2, 48),
                                                  (100, 8, 8, 100), (192, 16, 2, 64),
                                                  (320, 6, 3, 320), (512, 4, 1, 512)])
def test_generic_width_decode_verify_prefill(pkg, backend, rng, dim, heads, kvh, rotary):
    # one call with a decode row, a 5-row verify and a 40-row prefill chunk,
    # over cached contexts that cross page edges
    pool = new_pool(pkg, backend, kvh, dim, page_tokens=16, max_tokens=512, seqs=3)
    gq = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    cases = [Case(rng, pool, heads, kvh, dim, ctx=70, rows=1, max_tokens=512),
             Case(rng, pool, heads, kvh, dim, ctx=33, rows=5, max_tokens=512),
             Case(rng, pool, heads, kvh, dim, ctx=0, rows=40, max_tokens=512)]
    run_case(pkg, backend, pool, cases, rotary=rotary, gq=gq, gk=gk)
    for c, n in zip(cases, (71, 38, 40)):
        assert pool.len(c.seq) == n
    # the appended rows read back as the oracle's bf16 cache rows
    k_dev, v_dev = pool.read(cases[2].seq, 0, 40)
    for t in (0, 17, 39):
        k_ref, v_ref = cases[2].ref.get(t)
        attn_close(k_dev[t], k_ref, atol=1e-6, rtol=2 ** -8, what=f"appended k {t}")
        assert np.array_equal(v_dev[t], v_ref)
    pool.destroy()


def test_generic_width_gated_mrope_bf16_device(pkg, backend, rng, torch_mod):
    # a Qwen3.5-style gated layer at head_dim 160: (1 + w) norms, partial
    # rotary 64, interleaved MRoPE with distinct axes, bf16 device inputs
    dim = 160
    pool = new_pool(pkg, backend, 2, dim, max_tokens=1024, seqs=2)
    gq = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(dim)).astype(np.float32)
    cases = [Case(rng, pool, 8, 2, dim, ctx=300, rows=3, gated=True, pos_axes=(0, 5, 9)),
             Case(rng, pool, 8, 2, dim, ctx=2, rows=1, gated=True, pos_axes=(0, 2, 1))]
    run_case(pkg, backend, pool, cases, rotary=64, theta=1e7, gq=gq, gk=gk, gated=True,
             offset=True, mrope=(11, 11, 10), bf16_inputs=True, device=True, torch=torch_mod)
    pool.destroy()


def test_generic_width_no_norm_and_fork(pkg, backend, rng):
    # no QK-norm; a fork shares the pages and both branches go on separately
    # (the copy-on-write of the shared partial page)
    dim = 48
    pool = new_pool(pkg, backend, 2, dim, page_tokens=16, max_tokens=256, seqs=3)
    base = Case(rng, pool, 4, 2, dim, ctx=21, rows=2, qk_norm=False, max_tokens=256)
    run_case(pkg, backend, pool, [base], rotary=dim)
    fork = pool.fork(base.seq)
    k0, v0 = pool.read(base.seq, 0, 23)
    for branch in range(2):
        c = Case(rng, pool, 4, 2, dim, ctx=0, rows=3, qk_norm=False, max_tokens=256)
        pool.close(c.seq)
        c.seq = base.seq if branch == 0 else fork
        c.ref = O.KvCache(2 * dim, 256, 16, bf16=True)
        c.ref.append_many(k0, v0)
        c.pos = c.pos + 23
        run_case(pkg, backend, pool, [c], rotary=dim)
    kf, _ = pool.read(fork, 0, 23)
    assert np.array_equal(kf, k0), "the fork's first 23 rows stay the shared ones"
    pool.truncate(fork, 10)
    assert pool.len(fork) == 10 and pool.len(base.seq) == 26
    pool.destroy()


def test_generic_width_non_finite_k_is_rejected(pkg, backend, rng):
    dim = 24
    pool = new_pool(pkg, backend, 1, dim, max_tokens=64, seqs=1)
    c = Case(rng, pool, 2, 1, dim, ctx=5, rows=2, qk_norm=False, max_tokens=64)
    c.k[1, 3] = np.inf
    with pytest.raises(pkg.PluginError):
        run_case(pkg, backend, pool, [c], rotary=dim)
    assert pool.len(c.seq) == 5, "a rejected call leaves the length as it was"
    pool.destroy()


def test_width_limits(pkg, backend):
    with pytest.raises(pkg.PluginError):
        new_pool(pkg, backend, 1, 513, max_tokens=64, seqs=1)
    with pytest.raises(pkg.PluginError):
        pkg.GdnState(backend, 1, 1, 513, 64, 4, 1)


# ---------------------------------------------------------------------------
# GDN
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("dk,dv,hk,hv,K", [(2, 3, 1, 2, 4), (64, 64, 2, 4, 4), (96, 80, 1, 3, 3),
                                            (128, 100, 2, 2, 4), (256, 256, 1, 2, 4),
                                            (512, 24, 1, 1, 2), (40, 128, 2, 4, 1)])
def test_generic_gdn_widths_decode_and_prefill(pkg, backend, rng, dk, dv, hk, hv, K):
    L = Layer(rng, hk, hv, dk, dv, K)
    L.a_log = (0.5 * rng.standard_normal(hv)).astype(np.float32)
    L.dt_bias = (0.5 * rng.standard_normal(hv)).astype(np.float32)
    L.norm = (1 + 0.1 * rng.standard_normal(dv)).astype(np.float32)
    pool = pkg.GdnState(backend, hk, hv, dk, dv, K, 2)
    a, b = pool.open(), pool.open()
    ma = np.zeros((hv, dv, dk), np.float32)
    ha = np.zeros((L.C, K - 1), np.float32)
    mb = (0.02 * rng.standard_normal((hv, dv, dk))).astype(np.float32)
    hb = (0.5 * rng.standard_normal((L.C, K - 1))).astype(np.float32)
    pool.write(b, mb, hb)
    for step, (ra, rb) in enumerate(((40, 1), (1, 9), (3, 1))):
        xa, xb = L.inputs(rng, ra), L.inputs(rng, rb)
        x = tuple(np.concatenate([u, v]) for u, v in zip(xa, xb))
        got = plugin_rows(pkg, backend, pool, L, [a, b], [ra, rb], x)
        gdn_close(got[:ra], oracle_rows(L, xa, ma, ha), what=f"seq a step {step}")
        gdn_close(got[ra:], oracle_rows(L, xb, mb, hb), what=f"seq b step {step}")
    for s, (m, h) in ((a, (ma, ha)), (b, (mb, hb))):
        gm, gh = pool.read(s)
        gdn_close(gm, m, what="state")
        assert np.array_equal(gh, h), "conv history"
    pool.destroy()


@pytest.mark.parametrize("dk,dv", [(64, 48), (96, 100)])
def test_generic_gdn_rollback_equals_oracle_and_reforward(pkg, backend, rng, dk, dv):
    L = Layer(rng, 1, 2, dk, dv, 4)
    pool = pkg.GdnState(backend, 1, 2, dk, dv, 4, 4, keep_rows=9)
    s = pool.open()
    plugin_rows(pkg, backend, pool, L, [s], [12], L.inputs(rng, 12))
    snap_m, snap_h = pool.read(s)
    pre = pool.fork(s)
    x = L.inputs(rng, 9)
    qkv, z, a, b = x
    out = np.zeros((9, L.hv * L.dv), np.float32)
    pkg.gdn_forward(backend, pool, [s], [9], qkv, z, a, b, L.a_log, L.dt_bias, L.conv, L.norm,
                    out, eps=1e-6, keep_rows=True)
    st, hi = snap_m.copy(), snap_h.copy()
    gdn_close(out, oracle_rows(L, x, st, hi), what="KEEP_ROWS outputs")
    for j in (4, 0, 9, 1):
        pool.rollback(s, j)
        m, h = pool.read(s)
        st, hi = snap_m.copy(), snap_h.copy()
        if j:
            oracle_rows(L, tuple(t[:j] for t in x), st, hi)
        gdn_close(m, st, what=f"state after rollback to row {j}")
        assert np.array_equal(h, hi), f"history after rollback to row {j}"
        f = pool.fork(pre)
        if j:
            plugin_rows(pkg, backend, pool, L, [f], [j], tuple(t[:j] for t in x))
        fm, fh = pool.read(f)
        assert np.array_equal(m, fm), f"rollback to row {j} differs from re-forwarding {j} rows"
        assert np.array_equal(h, fh)
        pool.close(f)
    pool.destroy()


# ---------------------------------------------------------------------------
# the generic path's own limits
# ---------------------------------------------------------------------------

def test_generic_width_more_rows_than_one_grid_holds(pkg, backend, rng, torch_mod):
    # 66,000 rows of one sequence in one call: the generic kernels cover at
    # most 65,535 rows per launch (grid y) and run the rest in a second
    # launch, after every row's append.  Every V row is the same vector c, so
    # each row's output is c whatever its softmax weights (sum p c / sum p).
    torch = torch_mod
    dim, rows = 4, 66000
    pool = new_pool(pkg, backend, 1, dim, page_tokens=64, max_tokens=rows, seqs=1)
    s = pool.open()
    c = O.bf16_round(np.array([0.75, -1.5, 2.0, 0.125], np.float32))
    q = torch.from_numpy(rng.standard_normal((rows, dim)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((rows, dim)).astype(np.float32)).cuda()
    v = torch.from_numpy(np.tile(c, (rows, 1))).cuda()
    pos = torch.arange(rows, dtype=torch.int32, device="cuda").view(rows, 1).repeat(1, 3).contiguous()
    out = torch.zeros((rows, dim), dtype=torch.float32, device="cuda")
    pkg.attention_forward(backend, pool, [s], [rows], q, k, v, pos, out, heads=1, kv_heads=1,
                          head_dim=dim, rotary_dim=dim, rope_theta=1e6)
    got = out.cpu().numpy()
    assert pool.len(s) == rows
    # f32 sums over up to 66k weights: each row's sum p c / sum p keeps c to
    # a few e-5 relative (recursive summation errs by at most rows * 2^-24);
    # a row the second launch missed would read 0, a wrong V row another vector
    err = np.abs(got - c[None, :])
    assert err.max() <= 1e-3 * np.abs(c).max(), f"max abs {err.max():.3e} (row {err.max(1).argmax()})"
    assert np.abs(got[65535:] - c).max() <= 1e-3 * np.abs(c).max()
    # both launches appended: the first and the last rows read back as stored
    kd, vd = pool.read(s, rows - 2, 2)
    assert np.array_equal(vd, np.tile(c, (2, 1)))
    pool.destroy()


def test_generic_width_no_alloc_entry_point_equals_ordinary(pkg, backend, rng, torch_mod):
    # the same generic-width call through both entry points, on forked copies
    # of the same sequences: bit for bit
    import ctypes as C
    torch = torch_mod
    dim, heads, kvh = 80, 4, 2
    pool = new_pool(pkg, backend, kvh, dim, page_tokens=16, max_tokens=256, seqs=4)
    a, b = pool.open(), pool.open()
    ck = O.bf16_round(rng.standard_normal((30, kvh * dim)).astype(np.float32))
    cv = O.bf16_round(rng.standard_normal((30, kvh * dim)).astype(np.float32))
    pool.append(a, ck, cv)
    fa, fb = pool.fork(a), pool.fork(b)
    rows = [3, 20]
    n = sum(rows)
    q = torch.from_numpy(rng.standard_normal((n, heads * dim)).astype(np.float32)).cuda()
    k = torch.from_numpy(rng.standard_normal((n, kvh * dim)).astype(np.float32)).cuda()
    v = torch.from_numpy(rng.standard_normal((n, kvh * dim)).astype(np.float32)).cuda()
    pos = torch.tensor([[30 + r] * 3 for r in range(3)] + [[r] * 3 for r in range(20)],
                       dtype=torch.int32, device="cuda")
    g = torch.from_numpy((1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)).cuda()
    outs = []
    for seqs, entry in (([a, b], "safetyraise_kernel_attention_forward"),
                        ([fa, fb], "safetyraise_kernel_attention_forward_noalloc")):
        P = pkg.plugin
        args = P.AttentionArgs()
        args.struct_size = C.sizeof(P.AttentionArgs)
        args.flags = P.DEVICE_POINTERS | P.QK_NORM | P.MROPE_INTERLEAVED
        args.heads, args.kv_heads, args.head_dim, args.rotary_dim = heads, kvh, dim, dim
        args.eps, args.rope_theta = 1e-6, 1e6
        args.num_seqs = 2
        ids = (C.c_uint32 * 2)(*seqs)
        nr = (C.c_uint32 * 2)(*rows)
        args.seq_ids, args.seq_rows = ids, nr
        args.q, args.k, args.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
        args.q_norm = args.k_norm = g.data_ptr()
        args.positions = pos.data_ptr()
        out = torch.zeros((n, heads * dim), dtype=torch.float32, device="cuda")
        args.out = out.data_ptr()
        args.kv = pool.handle
        backend.check(getattr(backend.lib, entry)(backend.context, C.byref(args)), entry)
        outs.append(out.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    assert pool.len(a) == pool.len(fa) == 33 and pool.len(b) == pool.len(fb) == 20
    pool.destroy()


def test_generic_width_more_sequences_than_one_launch_holds(pkg, backend, rng):
    # 70 sequences in one call: the generic kernels take 64 sequences per
    # launch (their argument block), so the call runs as two launch pairs
    dim = 40
    pool = new_pool(pkg, backend, 1, dim, page_tokens=16, max_tokens=64, seqs=70)
    ctxs = [int(rng.integers(0, 20)) for _ in range(70)]
    cases = [Case(rng, pool, 3, 1, dim, ctx=ctx, rows=1 + (i % 3), max_tokens=64)
             for i, ctx in enumerate(ctxs)]
    run_case(pkg, backend, pool, cases, rotary=dim)
    for c, ctx in zip(cases, ctxs):
        assert pool.len(c.seq) == ctx + c.rows
    pool.destroy()


def test_generic_gdn_more_sequences_than_one_launch_holds(pkg, backend, rng):
    # 70 sequences of one decode row each at key width 64 (the generic GDN
    # kernel), from distinct seeded states
    L = Layer(rng, 1, 2, 64, 48, 4)
    n = 70
    pool = pkg.GdnState(backend, 1, 2, 64, 48, 4, n)
    seqs, states = [], []
    for _ in range(n):
        s = pool.open()
        m = (0.05 * rng.standard_normal((2, 48, 64))).astype(np.float32)
        h = (0.5 * rng.standard_normal((L.C, 3))).astype(np.float32)
        pool.write(s, m, h)
        seqs.append(s)
        states.append((m, h))
    xs = [L.inputs(rng, 1) for _ in range(n)]
    x = tuple(np.concatenate([u[i] for u in xs]) for i in range(4))
    got = plugin_rows(pkg, backend, pool, L, seqs, [1] * n, x)
    for i, (m, h) in enumerate(states):
        gdn_close(got[i:i + 1], oracle_rows(L, xs[i], m, h), what=f"sequence {i}")
        gm, gh = pool.read(seqs[i])
        gdn_close(gm, m, what=f"state {i}")
        assert np.array_equal(gh, h), f"history {i}"
    pool.destroy()
