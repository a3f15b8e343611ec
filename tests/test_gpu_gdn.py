"""GPU parity of the gated-delta-net path through the C-ABI.

f32 path: |d| <= 1e-4 + 1e-4 * |ref| against the CPU oracle on the same
seeded inputs, for outputs, the recurrent state and the conv history.
"""
import zlib
import numpy as np
import pytest

from oracle import pyoracle as O

pytestmark = pytest.mark.gpu

ATOL = RTOL = 1e-4


def close(actual, expected, atol=ATOL, rtol=RTOL, what=""):
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} off, max abs {err.max():.3e}"


class Layer:
    """Seeded GDN layer weights (BASELINE config 4 draws)."""

    def __init__(self, rng, hk, hv, dk=128, dv=128, K=4):
        self.hk, self.hv, self.dk, self.dv, self.K = hk, hv, dk, dv, K
        self.C = 2 * hk * dk + hv * dv
        self.a_log = np.zeros(hv, np.float32)
        self.dt_bias = np.zeros(hv, np.float32)
        self.conv = (rng.standard_normal((self.C, K)) / 2).astype(np.float32)
        self.norm = np.ones(dv, np.float32)

    def inputs(self, rng, rows):
        return (rng.standard_normal((rows, self.C)).astype(np.float32),
                rng.standard_normal((rows, self.hv * self.dv)).astype(np.float32),
                rng.standard_normal((rows, self.hv)).astype(np.float32),
                rng.standard_normal((rows, self.hv)).astype(np.float32))


def oracle_rows(L, x, state, hist):
    qkv, z, a, b = x
    return O.gdn_rows(qkv, z, a, b, L.a_log, L.dt_bias, L.conv, L.K, L.norm, 1e-6,
                      key_heads=L.hk, value_heads=L.hv, key_dim=L.dk, value_dim=L.dv,
                      history=hist, state=state)


def plugin_rows(pkg, backend, pool, L, seqs, rows, x):
    qkv, z, a, b = x
    out = np.zeros((qkv.shape[0], L.hv * L.dv), np.float32)
    pkg.gdn_forward(backend, pool, seqs, rows, qkv, z, a, b, L.a_log, L.dt_bias, L.conv, L.norm,
                    out, eps=1e-6)
    return out


@pytest.fixture
def rng(request):
    return np.random.default_rng(zlib.crc32(request.node.name.encode()))


def seeded_state(rng, L):
    return ((0.02 * rng.standard_normal((L.hv, L.dv, L.dk))).astype(np.float32),
            (0.5 * rng.standard_normal((L.C, L.K - 1))).astype(np.float32))


def test_gdn_decode_batch8_matches_oracle(pkg, backend, rng):
    # BASELINE config 4 decode: Hk 16 / Hv 32, d 128, conv 4, batch 8, one token
    # per step; several steps so the history ring and the state carry over
    L = Layer(rng, 16, 32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 8)
    seqs, refs = [], []
    for _ in range(8):
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        seqs.append(s)
        refs.append((m.copy(), h.copy()))
    for step in range(3):
        x = L.inputs(rng, 8)
        got = plugin_rows(pkg, backend, pool, L, seqs, [1] * 8, x)
        for i, (m, h) in enumerate(refs):
            exp = oracle_rows(L, tuple(t[i:i + 1] for t in x), m, h)
            close(got[i], exp[0], what=f"step {step} seq {i}")
    for s, (m, h) in zip(seqs, refs):
        gm, gh = pool.read(s)
        close(gm, m, what="state")
        close(gh, h, atol=0, rtol=0, what="history")
    pool.destroy()


def test_gdn_prefill_chunks_and_mixed_rows(pkg, backend, rng):
    # chunked prefill (64-row chunks) on one sequence next to a decode row on
    # another, in the same calls
    L = Layer(rng, 16, 32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 4)
    a, b = pool.open(), pool.open()
    ma, ha = np.zeros((L.hv, L.dv, L.dk), np.float32), np.zeros((L.C, 3), np.float32)
    mb, hb = seeded_state(rng, L)
    pool.write(b, mb, hb)
    for chunk in range(3):
        xa = L.inputs(rng, 64)
        xb = L.inputs(rng, 1)
        x = tuple(np.concatenate([u, v]) for u, v in zip(xa, xb))
        got = plugin_rows(pkg, backend, pool, L, [a, b], [64, 1], x)
        close(got[:64], oracle_rows(L, xa, ma, ha), what=f"prefill chunk {chunk}")
        close(got[64:], oracle_rows(L, xb, mb, hb), what=f"decode row {chunk}")
    close(pool.read(a)[0], ma, what="prefill state")
    pool.destroy()


def test_gdn_small_heads_and_kernel_sizes(pkg, backend, rng):
    # key groups of 1 and 4, conv kernels 1 (no history) and 3, value_dim 32
    for hk, hv, K in ((2, 2, 1), (1, 4, 3)):
        L = Layer(rng, hk, hv, 128, 32, K)
        pool = pkg.GdnState(backend, hk, hv, 128, 32, K, 2)
        s = pool.open()
        m = np.zeros((hv, 32, 128), np.float32)
        h = np.zeros((L.C, K - 1), np.float32)
        x = L.inputs(rng, 10)
        close(plugin_rows(pkg, backend, pool, L, [s], [10], x), oracle_rows(L, x, m, h),
              what=f"hk {hk} hv {hv} K {K}")
        close(pool.read(s)[0], m, what="state")
        pool.destroy()


def test_gdn_fork_is_an_independent_snapshot(pkg, backend, rng):
    L = Layer(rng, 2, 4, 128, 16, 4)
    pool = pkg.GdnState(backend, 2, 4, 128, 16, 4, 3)
    s = pool.open()
    x1 = L.inputs(rng, 5)
    plugin_rows(pkg, backend, pool, L, [s], [5], x1)
    snap_m, snap_h = pool.read(s)
    f = pool.fork(s)
    x2 = L.inputs(rng, 3)
    plugin_rows(pkg, backend, pool, L, [s], [3], x2)
    fm, fh = pool.read(f)
    assert np.array_equal(fm, snap_m) and np.array_equal(fh, snap_h)
    # replaying x2 on the fork reproduces the original's result exactly
    out_f = plugin_rows(pkg, backend, pool, L, [f], [3], x2)
    sm, sh = pool.read(s)
    fm, fh = pool.read(f)
    assert np.array_equal(fm, sm) and np.array_equal(fh, sh)
    assert out_f.shape == (3, 4 * 16)
    # and matches the oracle run from the same snapshot
    # (SequenceState::checkpoint then Gdn::forward, native.rs:720-742)
    state = np.zeros((4, 16, 128), np.float32)
    hist = np.zeros((L.C, L.K - 1), np.float32)
    oracle_rows(L, x1, state, hist)
    close(snap_m, state, what="snapshot state")
    close(snap_h, hist, what="snapshot history")
    exp = oracle_rows(L, x2, state, hist)
    close(out_f, exp, what="fork replay output")
    close(fm, state, what="fork state")
    close(fh, hist, what="fork history")
    pool.destroy()


def test_gdn_error_paths(pkg, backend, rng):
    with pytest.raises(pkg.PluginError):
        pkg.GdnState(backend, 2, 3, 128, 16, 4, 1)   # value_heads % key_heads
    with pytest.raises(pkg.PluginError):
        pkg.GdnState(backend, 1, 1, 600, 16, 4, 1)   # key_dim above 512
    with pytest.raises(pkg.PluginError):
        pkg.GdnState(backend, 1, 1, 128, 0, 4, 1)    # empty value heads
    with pytest.raises(pkg.PluginError):
        pkg.GdnState(backend, 1, 1, 128, 16, 9, 1)   # conv kernel above 8
    L = Layer(rng, 1, 1, 128, 16, 4)
    pool = pkg.GdnState(backend, 1, 1, 128, 16, 4, 1)
    s = pool.open()
    with pytest.raises(pkg.PluginError):
        plugin_rows(pkg, backend, pool, L, [s], [0], L.inputs(rng, 1))
    with pytest.raises(pkg.PluginError):
        plugin_rows(pkg, backend, pool, L, [s + 1], [1], L.inputs(rng, 1))
    pool.destroy()


def run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, what):
    """One call over several sequences; each checked against the oracle
    (outputs, then the states and histories the oracle carried)."""
    xs = [L.inputs(rng, n) for n in rows]
    x = tuple(np.concatenate(parts) for parts in zip(*xs))
    got = plugin_rows(pkg, backend, pool, L, seqs, rows, x)
    off = 0
    for i, (n, (m, h)) in enumerate(zip(rows, refs)):
        close(got[off:off + n], oracle_rows(L, xs[i], m, h), what=f"{what} seq {i} ({n} rows)")
        off += n
    for i, (s, (m, h)) in enumerate(zip(seqs, refs)):
        gm, gh = pool.read(s)
        close(gm, m, what=f"{what} state {i}")
        close(gh, h, atol=0, rtol=0, what=f"{what} history {i}")


def test_gdn_chunked_form_ragged_rows_seeded_state(pkg, backend, rng):
    # calls with more than 8 rows run the chunked (WY) form in chunks of 32:
    # full, partial and multi-chunk sequences next to a decode row, from
    # seeded states, over consecutive calls; non-zero A_log and dt_bias
    L = Layer(rng, 16, 32)
    L.a_log = (0.3 * rng.standard_normal(L.hv)).astype(np.float32)
    L.dt_bias = (0.3 * rng.standard_normal(L.hv)).astype(np.float32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 4)
    seqs, refs = [], []
    for _ in range(4):
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        seqs.append(s)
        refs.append((m.copy(), h.copy()))
    for call, rows in enumerate(([64, 45, 1, 9], [32, 100, 33, 1], [17, 1, 64, 31])):
        run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, f"call {call}")
    pool.destroy()


def test_gdn_decode_kernel_conv_sizes(pkg, backend, rng):
    # decode-sized calls (at most 8 rows per sequence, Dv 128) with conv
    # kernels other than 4 (run-time taps) and 4 itself (compile-time taps),
    # over two calls so the history carries: outputs, states, histories
    for hk, hv, K in ((2, 8, 1), (1, 4, 3), (2, 4, 6), (4, 8, 4)):
        L = Layer(rng, hk, hv, 128, 128, K)
        pool = pkg.GdnState(backend, hk, hv, 128, 128, K, 3)
        seqs, refs = [], []
        for _ in range(3):
            s = pool.open()
            m, h = seeded_state(rng, L)
            pool.write(s, m, h)
            seqs.append(s)
            refs.append((m.copy(), h.copy()))
        for call, rows in enumerate(([1, 8, 3], [2, 1, 1])):
            run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, f"hk {hk} hv {hv} K {K} call {call}")
        pool.destroy()


def test_gdn_chunked_form_key_groups_and_conv_sizes(pkg, backend, rng):
    # key groups of 1 and 4, conv kernels 1 (no history), 2 and 6
    for hk, hv, K in ((4, 4, 1), (1, 4, 2), (2, 8, 6)):
        L = Layer(rng, hk, hv, 128, 128, K)
        pool = pkg.GdnState(backend, hk, hv, 128, 128, K, 2)
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        run_batch(pkg, backend, pool, L, [s], [70], [(m, h)], rng, f"hk {hk} hv {hv} K {K}")
        pool.destroy()


def test_gdn_chunked_equals_token_serial_and_bf16_device(pkg, backend, rng):
    # invariant: one 96-row call == the same rows one at a time (decode
    # kernel), within the f32 tolerance; then bf16 device inputs, async
    import torch
    L = Layer(rng, 16, 32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 3)
    a = pool.open()
    m, h = seeded_state(rng, L)
    pool.write(a, m, h)
    b = pool.fork(a)
    x = L.inputs(rng, 96)
    whole = plugin_rows(pkg, backend, pool, L, [a], [96], x)
    serial = np.concatenate([plugin_rows(pkg, backend, pool, L, [b], [1],
                                         tuple(t[r:r + 1] for t in x)) for r in range(96)])
    close(whole, serial, what="chunked vs token-serial")
    close(pool.read(a)[0], pool.read(b)[0], what="state chunked vs token-serial")
    c = pool.open()
    m, h = seeded_state(rng, L)
    pool.write(c, m, h)
    qkv, z, av, bv = (O.bf16_round(t) for t in L.inputs(rng, 80))
    exp = oracle_rows(L, (qkv, z, av, bv), m, h)
    dev = [torch.from_numpy(t).to(torch.bfloat16).cuda() for t in (qkv, z, av, bv)]
    out = torch.zeros((80, L.hv * L.dv), device="cuda")
    w = [torch.from_numpy(t).cuda() for t in (L.a_log, L.dt_bias, L.conv, L.norm)]
    pkg.gdn_forward(backend, pool, [c], [80], *dev, *w, out, eps=1e-6, asynchronous=True)
    backend.synchronize()
    close(out.cpu().numpy(), exp, what="bf16 device inputs")
    close(pool.read(c)[0], m, what="bf16 state")
    pool.destroy()


def test_gdn_device_views_at_odd_offsets(pkg, backend, rng):
    # device z, norm weights and output as views one element into their
    # buffers (4-byte but not 8-byte aligned), f32 and bf16 z: the norm/gate
    # kernel's two-dims-per-lane path needs 8-byte alignment and must fall
    # back to the scalar path here; prefill- and decode-sized calls
    import torch
    L = Layer(rng, 16, 32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 2)
    for rows, bf16, odd_qkv in ((40, False, False), (40, True, False), (3, False, False),
                                (40, False, True)):
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        qkv, z, av, bv = L.inputs(rng, rows)
        if bf16:
            qkv, z, av, bv = (O.bf16_round(t) for t in (qkv, z, av, bv))
        exp = oracle_rows(L, (qkv, z, av, bv), m, h)
        dt = torch.bfloat16 if bf16 else torch.float32

        def odd(t, dtype):
            flat = torch.from_numpy(np.ascontiguousarray(t).ravel()).to(dtype)
            buf = torch.zeros(flat.numel() + 1, dtype=dtype, device="cuda")
            buf[1:] = flat.cuda()
            return buf[1:].view(t.shape)

        # a qkv view one element in is not 16-byte aligned: such a call takes
        # the row-block kernel instead of the chunked form
        dev = [odd(qkv, dt) if odd_qkv else torch.from_numpy(qkv).to(dt).cuda(), odd(z, dt),
               torch.from_numpy(av).to(dt).cuda(), torch.from_numpy(bv).to(dt).cuda()]
        w = [torch.from_numpy(t).cuda() for t in (L.a_log, L.dt_bias, L.conv)] + [odd(L.norm, torch.float32)]
        out = odd(np.zeros((rows, L.hv * L.dv), np.float32), torch.float32)
        pkg.gdn_forward(backend, pool, [s], [rows], *dev, *w, out, eps=1e-6)
        close(out.cpu().numpy(), exp, what=f"rows {rows} bf16 {bf16} odd qkv {odd_qkv}")
        close(pool.read(s)[0], m, what=f"state rows {rows} bf16 {bf16} odd qkv {odd_qkv}")
        pool.close(s)
    pool.destroy()


def test_gdn_chunked_form_more_than_64_sequences(pkg, backend, rng):
    # 70 sequences in one call with more than 8 rows somewhere, so every one
    # takes the chunked form: two launch batches (64 + 6 sequences) that
    # reuse one set of chunk records; 1..40 rows each (one or two chunks,
    # full and partial), seeded states
    L = Layer(rng, 2, 4)
    pool = pkg.GdnState(backend, 2, 4, 128, 128, 4, 70)
    seqs, refs = [], []
    for _ in range(70):
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        seqs.append(s)
        refs.append((m.copy(), h.copy()))
    rows = [int(r) for r in rng.integers(1, 41, size=70)]
    rows[3] = 40
    run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, "70 sequences")
    pool.destroy()


def test_gdn_chunked_form_long_calls_take_the_one_workgroup_prep(pkg, backend, rng):
    # a call with more (chunk, value head) records than half the CUs takes
    # the prep form with one workgroup per record (fewer take two): 5 chunks
    # x 32 value heads, conv kernel 3 (run-time taps), f32 host inputs, then
    # bf16 device inputs with a partial last chunk, then a short call
    import torch
    L = Layer(rng, 16, 32, 128, 128, 3)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 3, 2)
    s = pool.open()
    m, h = seeded_state(rng, L)
    pool.write(s, m, h)
    run_batch(pkg, backend, pool, L, [s], [160], [(m, h)], rng, "160 rows f32")
    qkv, z, av, bv = (O.bf16_round(t) for t in L.inputs(rng, 150))
    exp = oracle_rows(L, (qkv, z, av, bv), m, h)
    dev = [torch.from_numpy(t).to(torch.bfloat16).cuda() for t in (qkv, z, av, bv)]
    out = torch.zeros((150, L.hv * L.dv), device="cuda")
    w = [torch.from_numpy(t).cuda() for t in (L.a_log, L.dt_bias, L.conv, L.norm)]
    pkg.gdn_forward(backend, pool, [s], [150], *dev, *w, out, eps=1e-6)
    close(out.cpu().numpy(), exp, what="150 rows bf16")
    gm, gh = pool.read(s)
    close(gm, m, what="state after 150 rows")
    close(gh, h, atol=0, rtol=0, what="history after 150 rows")
    run_batch(pkg, backend, pool, L, [s], [40], [(m, h)], rng, "40 rows after")
    pool.destroy()


def test_gdn_non_unit_norm_weights(pkg, backend, rng):
    # non-unit per-head norm weights (the other tests use ones): a
    # decode-sized call (norm in the head kernel), chunked calls of 128 and
    # 129 rows, then 3 + 129 rows in one call (chunked form, then the norm
    # kernel), each against the oracle with the state carried
    L = Layer(rng, 16, 32)
    L.norm = (1 + 0.1 * rng.standard_normal(L.dv)).astype(np.float32)
    pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 2)
    a, b = pool.open(), pool.open()
    ra, rb = seeded_state(rng, L), seeded_state(rng, L)
    pool.write(a, *ra)
    pool.write(b, *rb)
    for call, (seqs, rows, refs) in enumerate((([a], [5], [ra]), ([a], [128], [ra]),
                                               ([a], [129], [ra]), ([a, b], [3, 129], [ra, rb]))):
        run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, f"call {call} rows {rows}")
    pool.destroy()


def test_gdn_non_finite_output_is_reported(pkg, backend, rng):
    # an infinite value input makes the row's delta-rule output non-finite,
    # which the per-head RMSNorm rejects (math.rs:39-41): a decode-sized call
    # (norm in the head kernel) and chunked calls of 64 and 160 rows (norm
    # kernel); the error word is cleared by the report, so a clean call
    # afterwards succeeds
    L = Layer(rng, 2, 4)
    pool = pkg.GdnState(backend, 2, 4, 128, 128, 4, 4)
    for rows in (3, 64, 160):
        s = pool.open()
        x = L.inputs(rng, rows)
        x[0][rows // 2, 2 * L.hk * L.dk + 5] = np.inf  # a value channel of head 0
        with pytest.raises(pkg.PluginError, match="variance"):
            plugin_rows(pkg, backend, pool, L, [s], [rows], x)
        pool.close(s)
    s = pool.open()
    m = np.zeros((L.hv, L.dv, L.dk), np.float32)
    h = np.zeros((L.C, L.K - 1), np.float32)
    x = L.inputs(rng, 64)
    close(plugin_rows(pkg, backend, pool, L, [s], [64], x), oracle_rows(L, x, m, h),
          what="clean call after the errors")
    pool.destroy()


def test_gdn_chunked_form_long_recurrence(pkg, backend, rng):
    # BASELINE config 4's prefill shape on one sequence: 2048 rows in 32
    # calls of 64 rows, each call and the final state against the oracle
    # with the state carried.  Once with the config's decays and once with
    # slow ones (A_log -4: alpha about 0.99 per row), so the state keeps a
    # long memory of the rounding of the chunked form's products
    for a_log in (0.0, -4.0):
        L = Layer(rng, 16, 32)
        L.a_log = np.full(L.hv, a_log, np.float32)
        pool = pkg.GdnState(backend, 16, 32, 128, 128, 4, 1)
        s = pool.open()
        m = np.zeros((L.hv, L.dv, L.dk), np.float32)
        h = np.zeros((L.C, L.K - 1), np.float32)
        for call in range(32):
            x = L.inputs(rng, 64)
            close(plugin_rows(pkg, backend, pool, L, [s], [64], x), oracle_rows(L, x, m, h),
                  what=f"A_log {a_log} call {call}")
        gm, gh = pool.read(s)
        close(gm, m, what=f"A_log {a_log} state after 2048 rows")
        close(gh, h, atol=0, rtol=0, what=f"A_log {a_log} history after 2048 rows")
        pool.destroy()
