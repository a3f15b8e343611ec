"""GPU parity of the attention path and the paged KV cache, through the C-ABI.

Every case runs the same seeded inputs through the plugin and through the CPU
oracle (with bf16 KV storage, since the plugin stores K/V in bf16) and
compares with the bf16-path tolerance |d| <= 2e-3 + 1e-2 * |ref|.
"""
import zlib
import numpy as np
import pytest

from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def close(actual, expected, atol=ATOL, rtol=RTOL, what=""):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} outside tolerance, "
                           f"max abs {err.max():.3e}")


def make_pool(pkg, backend, kv_heads, head_dim, page_tokens=64, max_tokens=4096, seqs=8,
              pages=None):
    if pages is None:
        pages = seqs * ((max_tokens + page_tokens - 1) // page_tokens) + 8
    return pkg.KvCache(backend, kv_heads, head_dim, page_tokens, pages, max_tokens, seqs)


class Case:
    """One sequence: cached context plus new rows, mirrored on the oracle."""

    def __init__(self, rng, pool, heads, kv_heads, dim, ctx, rows, *, gated=False,
                 qk_norm=True, pos0=None, pos_axes=None, max_tokens=None):
        self.heads, self.kv_heads, self.dim = heads, kv_heads, dim
        width = kv_heads * dim
        self.seq = pool.open()
        self.ref = O.KvCache(width, max_tokens or pool_max(pool), pool.page_tokens, bf16=True)
        if ctx:
            ck = O.bf16_round(rng.standard_normal((ctx, width)).astype(np.float32))
            cv = O.bf16_round(rng.standard_normal((ctx, width)).astype(np.float32))
            pool.append(self.seq, ck, cv)
            self.ref.append_many(ck, cv)
        qw = heads * dim * (2 if gated else 1)
        self.q = rng.standard_normal((rows, qw)).astype(np.float32)
        self.k = rng.standard_normal((rows, width)).astype(np.float32)
        self.v = rng.standard_normal((rows, width)).astype(np.float32)
        p0 = ctx if pos0 is None else pos0
        if pos_axes is None:
            self.pos = np.array([[p0 + r] * 3 for r in range(rows)], np.int32)
        else:
            self.pos = np.array([[p0 + r + o for o in pos_axes] for r in range(rows)], np.int32)
        self.rows = rows


def pool_max(pool):
    return pool._max_tokens


def run_case(pkg, backend, pool, cases, *, rotary, theta=1e6, gq=None, gk=None, gated=False,
             offset=False, mrope=None, bf16_inputs=False, device=False, torch=None):
    q = np.concatenate([c.q for c in cases])
    k = np.concatenate([c.k for c in cases])
    v = np.concatenate([c.v for c in cases])
    pos = np.concatenate([c.pos for c in cases])
    heads, kv_heads, dim = cases[0].heads, cases[0].kv_heads, cases[0].dim
    if bf16_inputs:
        q, k, v = O.bf16_round(q), O.bf16_round(k), O.bf16_round(v)
    out = np.zeros((q.shape[0], heads * dim), np.float32)
    args = dict(heads=heads, kv_heads=kv_heads, head_dim=dim, rotary_dim=rotary,
                rope_theta=theta, eps=1e-6, q_norm=gq, k_norm=gk, gated=gated,
                norm_offset=offset, mrope_section=mrope or (0, 0, 0))
    if device:
        dt = torch.bfloat16 if bf16_inputs else torch.float32
        tq = torch.from_numpy(q).to("cuda").to(dt)
        tk = torch.from_numpy(k).to("cuda").to(dt)
        tv = torch.from_numpy(v).to("cuda").to(dt)
        tp = torch.from_numpy(pos).to("cuda")
        to = torch.zeros(out.shape, dtype=torch.float32, device="cuda")
        tgq = torch.from_numpy(gq).cuda() if gq is not None else None
        tgk = torch.from_numpy(gk).cuda() if gk is not None else None
        args.update(q_norm=tgq, k_norm=tgk)
        pkg.attention_forward(backend, pool, [c.seq for c in cases], [c.rows for c in cases],
                              tq, tk, tv, tp, to, **args)
        out = to.cpu().numpy()
    else:
        pkg.attention_forward(backend, pool, [c.seq for c in cases], [c.rows for c in cases],
                              q, k, v, pos, out, **args)
    r0 = 0
    for c in cases:
        exp = O.attention_rows(q[r0:r0 + c.rows], k[r0:r0 + c.rows], v[r0:r0 + c.rows],
                               pos[r0:r0 + c.rows].astype(np.int64), c.ref, heads=heads,
                               kv_heads=kv_heads, dim=dim, rotary_dim=rotary, theta=theta,
                               eps=1e-6, q_norm=gq, k_norm=gk, gated=gated,
                               mrope_section=mrope, threads=8)
        close(out[r0:r0 + c.rows], exp, what=f"seq {c.seq} ctx {len(c.ref) - c.rows}")
        r0 += c.rows
    return out


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def new_pool(pkg, backend, kv_heads, dim, page_tokens=64, max_tokens=4096, seqs=8):
    pool = make_pool(pkg, backend, kv_heads, dim, page_tokens, max_tokens, seqs)
    pool._max_tokens = max_tokens
    return pool


# ---------------------------------------------------------------------------
# KV cache semantics (src/engine/state.rs, src/gpu.rs:6467-6518)
# ---------------------------------------------------------------------------

def test_kv_append_read_layout(pkg, backend):
    # src/gpu.rs:6467-6488: token rows [kv_head][dim] read back unchanged; the
    # reference vector's head_dim 2 sits in the first two dims of each head.
    pool = new_pool(pkg, backend, 2, 64, page_tokens=16, max_tokens=8, seqs=2)
    seq = pool.open()
    rows_k = np.zeros((2, 128), np.float32)
    rows_v = np.zeros((2, 128), np.float32)
    rows_k[0, [0, 1, 64, 65]] = [1, 2, 10, 20]
    rows_v[0, [0, 1, 64, 65]] = [3, 4, 30, 40]
    rows_k[1, [0, 1, 64, 65]] = [5, 6, 50, 60]
    rows_v[1, [0, 1, 64, 65]] = [7, 8, 70, 80]
    pool.append(seq, rows_k[:1], rows_v[:1])
    pool.append(seq, rows_k[1:], rows_v[1:])
    k, v = pool.read(seq)
    assert pool.len(seq) == 2
    compact_k = k.reshape(2, 2, 64)[:, :, :2].transpose(1, 0, 2).ravel()
    compact_v = v.reshape(2, 2, 64)[:, :, :2].transpose(1, 0, 2).ravel()
    assert list(compact_k) == [1, 2, 5, 6, 10, 20, 50, 60]
    assert list(compact_v) == [3, 4, 7, 8, 30, 40, 70, 80]
    assert np.array_equal(k, rows_k) and np.array_equal(v, rows_v)
    pool.destroy()


def rounding_rows(rng, rows, width, big=True):
    """f32 rows whose bf16 rounding covers exact ties (even and odd kept
    halves), one ulp either side of a tie, random low bits, f32 denormals and
    (big=True) values next to the largest finite bf16."""
    hi = rng.standard_normal((rows, width)).astype(np.float32).view(np.uint32) & np.uint32(0xFFFF0000)
    picks = np.array([0x8000, 0x7FFF, 0x8001, 0x0000, 0xFFFF], np.uint32)
    low = np.where(rng.random(hi.shape) < 0.5, rng.choice(picks, size=hi.shape),
                   rng.integers(0, 1 << 16, size=hi.shape, dtype=np.uint32))
    x = (hi | low.astype(np.uint32)).view(np.float32).copy()
    special = [1e-40, -3e-39, 1.1754942e-38, 5e-45, -1e-10, 6e4, 0.0, -0.0]
    if big:
        special += [3.38e38, -3.3e38]
    x[0, :len(special)] = np.array(special, np.float32)
    return x


def bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


@pytest.mark.parametrize("rows", [1, 40])
def test_cache_append_rounds_to_nearest_even_bit_exact(pkg, backend, rng, rows):
    # the cache stores bf16 rounded to nearest even (the oracle's bf16_round);
    # both K and V of a plain append are the inputs themselves
    pool = new_pool(pkg, backend, 2, 128, page_tokens=16, max_tokens=64, seqs=1)
    seq = pool.open()
    k = rounding_rows(rng, rows, 256)
    v = rounding_rows(rng, rows, 256)
    pool.append(seq, k, v)
    rk, rv = pool.read(seq)
    assert np.array_equal(bits(rk), bits(O.bf16_round(k)))
    assert np.array_equal(bits(rv), bits(O.bf16_round(v)))
    pool.destroy()


@pytest.mark.parametrize("rows", [1, 40])
def test_attention_append_rounds_v_to_nearest_even_bit_exact(pkg, backend, rng, rows):
    # the V rows an attention call appends (decode for 1 row, the prefill
    # append kernel for 40) are the inputs rounded to bf16, bit for bit
    pool = new_pool(pkg, backend, 8, 128, max_tokens=256, seqs=1)
    gq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    case = Case(rng, pool, 32, 8, 128, ctx=20, rows=rows)
    case.v = rounding_rows(rng, rows, 8 * 128, big=False)
    run_case(pkg, backend, pool, [case], rotary=128, gq=gq, gk=gk)
    _, rv = pool.read(case.seq, 20, rows)
    assert np.array_equal(bits(rv), bits(O.bf16_round(case.v)))
    pool.destroy()


def test_kv_truncate_restores_without_losing_prior_rows(pkg, backend):
    # src/gpu.rs:6490-6518
    pool = new_pool(pkg, backend, 1, 64, page_tokens=16, max_tokens=8, seqs=2)
    seq = pool.open()
    row = lambda a, b: np.array([[a, b] + [0.0] * 62], np.float32)
    pool.append(seq, row(1, 2), row(3, 4))
    pool.append(seq, row(5, 6), row(7, 8))
    snapshot = pool.len(seq)
    pool.append(seq, row(9, 10), row(11, 12))
    assert pool.len(seq) == 3
    pool.truncate(seq, snapshot)
    pool.append(seq, row(13, 14), row(15, 16))
    k, v = pool.read(seq)
    assert list(k[:, :2].ravel()) == [1, 2, 5, 6, 13, 14]
    assert list(v[:, :2].ravel()) == [3, 4, 7, 8, 15, 16]
    pool.destroy()


@pytest.mark.parametrize("scale", [1, 4])
def test_kv_snapshot_isolated_across_partial_and_full_pages(pkg, backend, scale):
    # src/engine/state.rs tests: width 2 (dims 0..1 of one 64-wide head), 9
    # tokens max, fork = checkpoint().  The reference pages hold 4 tokens; the
    # pool's smallest page is 16, so scale 4 multiplies every token count by 4
    # to keep the same full-page / partial-page pattern (scale 1 keeps the
    # reference's counts, all inside one page).
    n_max, n_fork, n_trunc = 9 * scale, 3 * scale, 2 * scale
    pool = new_pool(pkg, backend, 1, 64, page_tokens=16, max_tokens=n_max, seqs=4)
    seq = pool.open()
    row = lambda a, b: np.array([[a, b] + [0.0] * 62], np.float32)
    for n in range(n_fork):
        pool.append(seq, row(n, 1.0), row(2.0, n))
    saved = pool.fork(seq)
    for n in range(n_fork, n_max):
        pool.append(seq, row(n, 1.0), row(2.0, n))
    with pytest.raises(pkg.PluginError):
        pool.append(seq, row(1, 1), row(1, 1))
    pool.truncate(seq, n_trunc)
    pool.append(seq, row(99, 99), row(88, 88))
    assert list(pool.read(saved, n_trunc, 1)[0][0, :2]) == [float(n_trunc), 1.0]
    assert list(pool.read(seq, n_trunc, 1)[0][0, :2]) == [99.0, 99.0]
    with pytest.raises(pkg.PluginError):
        pool.read(saved, n_fork, 1)
    with pytest.raises(pkg.PluginError):
        pool.truncate(seq, n_trunc + 2)
    pool.truncate(seq, 0)
    assert pool.len(seq) == 0
    # the snapshot still reads its own rows after the original moved on
    k, _ = pool.read(saved)
    assert list(k[:, 0]) == [float(n) for n in range(n_fork)]
    pool.destroy()


def test_kv_pool_rejects_unsupported_page_sizes(pkg, backend):
    for pt in (4, 24, 100):
        with pytest.raises(pkg.PluginError):
            pkg.KvCache(backend, 1, 64, pt, 8, 64, 1)


def test_kv_append_rejects_non_finite_and_keeps_length(pkg, backend):
    pool = new_pool(pkg, backend, 1, 64, page_tokens=16, max_tokens=8, seqs=1)
    seq = pool.open()
    good = np.ones((1, 64), np.float32)
    pool.append(seq, good, good)
    bad = good.copy()
    bad[0, 5] = np.nan
    with pytest.raises(pkg.PluginError) as err:
        pool.append(seq, bad, good)
    assert err.value.status == 1
    assert pool.len(seq) == 1
    pool.destroy()


@pytest.mark.parametrize("heads,page", [(16, 16), (16, 64), (32, 16), (32, 64)])
@pytest.mark.parametrize("rows", [1, 3, 20])
def test_non_finite_bits_past_the_length_are_never_read(pkg, backend, rng, heads, page, rows):
    # A rejected append leaves its rows in the slots past the length (the
    # length stays, as the reference's does).  The kernels load whole chunks
    # and tiles, so the slots past the last token are read; their scores are
    # masked and their V must not turn the output into NaN (0 * NaN).  G = 2
    # and G = 4; decode (1 row), verify (3) and prefill (20); pages of 16 and
    # 64 tokens.
    pool = new_pool(pkg, backend, 8, 128, page_tokens=page, max_tokens=512, seqs=2)
    gq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    case = Case(rng, pool, heads, 8, 128, ctx=37, rows=rows)
    nan = np.full((80, 8 * 128), np.nan, np.float32)
    with pytest.raises(pkg.PluginError):
        pool.append(case.seq, nan, nan)
    assert pool.len(case.seq) == 37
    out = run_case(pkg, backend, pool, [case], rotary=128, gq=gq, gk=gk)
    assert np.isfinite(out).all()
    pool.destroy()


# ---------------------------------------------------------------------------
# attention parity
# ---------------------------------------------------------------------------

def test_c1_qwen2_decode_host_pointers(pkg, backend, rng):
    # Qwen2-0.5B shape, 14 Q / 2 KV heads, head_dim 64,
    # RoPE theta 1e6, no QK-norm, 511 cached tokens + the new one at 511, f32.
    pool = new_pool(pkg, backend, 2, 64, max_tokens=1024, seqs=1)
    case = Case(rng, pool, 14, 2, 64, ctx=511, rows=1, qk_norm=False)
    run_case(pkg, backend, pool, [case], rotary=64)
    # the appended row is the normalised/roped k rounded to bf16, as the oracle stores it
    k_dev, v_dev = pool.read(case.seq, 511, 1)
    k_ref, v_ref = case.ref.get(511)
    close(k_dev[0], k_ref, atol=1e-6, rtol=2 ** -8, what="appended k")
    assert np.array_equal(v_dev[0], v_ref)
    pool.destroy()


@pytest.mark.parametrize("bf16_inputs", [False, True])
def test_qwen3_8b_decode_batch_device_pointers(pkg, backend, rng, torch_mod, bf16_inputs):
    # BASELINE config 2 shape: 32 Q / 8 KV, head_dim 128, QK-norm gamma
    # 1 + N(0, 0.02), theta 1e6; lengths chosen around page/split edges.
    lengths = [1, 2, 63, 64, 65, 1023, 1025, 4097, 20000, 32768]
    pool = new_pool(pkg, backend, 8, 128, max_tokens=32800, seqs=len(lengths))
    gq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    cases = [Case(rng, pool, 32, 8, 128, ctx=L - 1, rows=1) for L in lengths]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk, bf16_inputs=bf16_inputs,
             device=True, torch=torch_mod)
    for c, L in zip(cases, lengths):
        assert pool.len(c.seq) == L
    pool.destroy()


def test_qwen35_gated_partial_rope_mrope(pkg, backend, rng):
    # Qwen3.5 full-attention layer: q/gate interleaved per head, (1 + w) norms,
    # partial rotary 0.25 of 256, interleaved MRoPE with distinct axes.
    pool = new_pool(pkg, backend, 2, 256, max_tokens=2048, seqs=2)
    gq = (0.02 * rng.standard_normal(256)).astype(np.float32)
    gk = (0.02 * rng.standard_normal(256)).astype(np.float32)
    cases = [Case(rng, pool, 8, 2, 256, ctx=700, rows=1, gated=True, pos_axes=(0, 5, 9)),
             Case(rng, pool, 8, 2, 256, ctx=3, rows=1, gated=True, pos_axes=(0, 2, 1))]
    run_case(pkg, backend, pool, cases, rotary=64, theta=1e7, gq=gq, gk=gk, gated=True,
             offset=True, mrope=(11, 11, 10))
    pool.destroy()


@pytest.mark.parametrize("ctx,rows,page", [(300, 5, 64), (1000, 37, 64), (0, 9, 64),
                                           (300, 5, 16), (1000, 37, 32)])
def test_multi_row_call_is_causal_row_by_row(pkg, backend, rng, ctx, rows, page):
    # row r sees the context plus rows 0..r (native.rs:637-638); ctx 0 is a
    # fresh prompt
    pool = new_pool(pkg, backend, 8, 128, page_tokens=page, max_tokens=2048, seqs=2)
    gq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    cases = [Case(rng, pool, 32, 8, 128, ctx=ctx, rows=rows),
             Case(rng, pool, 32, 8, 128, ctx=17, rows=1)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_large_positions_match_reference_angle(pkg, backend, rng):
    # positions near 131072: one f32 ulp of the angle is ~0.008 rad, so this
    # fails unless the device uses the reference's exact f32 angle
    pool = new_pool(pkg, backend, 8, 128, max_tokens=1024, seqs=3)
    gq = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(128)).astype(np.float32)
    cases = [Case(rng, pool, 64, 8, 128, ctx=200, rows=1, pos0=131071),
             Case(rng, pool, 64, 8, 128, ctx=90, rows=5, pos0=131072 + 4000)]
    run_case(pkg, backend, pool, cases, rotary=128, gq=gq, gk=gk)
    pool.destroy()


def test_single_calls_equal_one_multi_row_call(pkg, backend, rng):
    # invariant: decode row by row == one call with all rows (whole == chunked),
    # each within the bf16-path tolerance of the oracle
    heads, kvh, dim, ctx, rows = 32, 8, 128, 500, 6
    pool = new_pool(pkg, backend, kvh, dim, max_tokens=1024, seqs=2)
    gq = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    gk = (1 + 0.02 * rng.standard_normal(dim)).astype(np.float32)
    base = pool.open()
    ck = O.bf16_round(rng.standard_normal((ctx, kvh * dim)).astype(np.float32))
    pool.append(base, ck, ck)
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
    # the 6-row call runs the multi-row verify kernel (fp16 MFMA operands),
    # the single rows the f32 split-K kernel: both against the oracle
    ref = O.KvCache(kvh * dim, 1024, 64, bf16=True)
    ref.append_many(ck, ck)
    exp = O.attention_rows(q, k, v, pos.astype(np.int64), ref, heads=heads, kv_heads=kvh,
                           dim=dim, rotary_dim=dim, theta=1e6, eps=1e-6, q_norm=gq, k_norm=gk,
                           threads=8)
    close(whole, exp, what="multi-row call vs oracle")
    close(single, exp, what="single rows vs oracle")
    close(single, whole, what="single vs whole")
    assert pool.len(base) == pool.len(fork) == ctx + rows
    pool.destroy()


def test_attention_error_paths(pkg, backend, rng):
    pool = new_pool(pkg, backend, 2, 64, page_tokens=16, max_tokens=40, seqs=2)
    case = Case(rng, pool, 4, 2, 64, ctx=38, rows=1, qk_norm=False)
    out = np.zeros((1, 256), np.float32)
    kw = dict(heads=4, kv_heads=2, head_dim=64, rotary_dim=64, rope_theta=1e6)
    # non-finite key: rejected, length unchanged (state.rs:56-58)
    bad_k = case.k.copy()
    bad_k[0, 3] = np.inf
    with pytest.raises(pkg.PluginError) as err:
        pkg.attention_forward(backend, pool, [case.seq], [1], case.q, bad_k, case.v, case.pos,
                              out, **kw)
    assert err.value.status == 1 and pool.len(case.seq) == 38
    # capacity: 38 + 3 > 40 (state.rs:53-55)
    q3 = np.repeat(case.q, 3, 0)
    k3 = np.repeat(case.k, 3, 0)
    p3 = np.array([[38 + r] * 3 for r in range(3)], np.int32)
    with pytest.raises(pkg.PluginError):
        pkg.attention_forward(backend, pool, [case.seq], [3], q3, k3, k3, p3,
                              np.zeros((3, 256), np.float32), **kw)
    # empty input (ensure_room), heads not a multiple of kv_heads, odd rotary dim
    with pytest.raises(pkg.PluginError):
        pkg.attention_forward(backend, pool, [case.seq], [0], case.q, case.k, case.v, case.pos,
                              out, **kw)
    with pytest.raises(pkg.PluginError):
        pkg.attention_forward(backend, pool, [case.seq], [1], case.q, case.k, case.v, case.pos,
                              out, **{**kw, "heads": 3})
    with pytest.raises(pkg.PluginError):
        pkg.attention_forward(backend, pool, [case.seq], [1], case.q, case.k, case.v, case.pos,
                              out, **{**kw, "rotary_dim": 63})
    # a valid call still works afterwards and matches the oracle
    run_case(pkg, backend, pool, [case], rotary=64)
    pool.destroy()


def test_capabilities_advertise_the_extension(pkg, backend):
    caps = backend.capabilities
    assert caps.abi_version == 1 and caps.struct_size >= 40
    assert caps.device_kind == 3
    assert caps.dtype_mask == (1 << 1) | (1 << 2) | (1 << 3)  # F32, F16, BF16 projections
    assert backend.supports(pkg.CAP_ATTENTION) and backend.supports(pkg.CAP_GDN)
    assert np.array_equal(backend.linear(np.ones((2, 2), np.float32), np.ones((1, 2), np.float32)),
                          np.full((1, 2), 2.0, np.float32))
    # quantised weight formats (dtype 4 and up) stay on the engine's matmul
    with pytest.raises(pkg.PluginError) as err:
        backend.create_weight(np.ones((2, 2), np.uint16), 4)
    assert err.value.status == 2
