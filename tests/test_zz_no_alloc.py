"""The no-allocation attention entry point against the ordinary one, through the C-ABI.

safetyraise_kernel_attention_forward_noalloc runs the same kernels as
safetyraise_kernel_attention_forward with its scratch in a fixed per-GPU
region, so on identical sequences and inputs its outputs must equal the
ordinary entry point's bit for bit.  Two calls in a row (the second smaller)
check that the region's leftovers from one call do not leak into the next.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    return torch


def make_args(pkg, pool, seqs, rows, q, k, v, pos, out, gq, gk):
    P = pkg.plugin
    a = P.AttentionArgs()
    a.struct_size = C.sizeof(P.AttentionArgs)
    a.flags = P.DEVICE_POINTERS | P.QK_NORM | P.INPUT_BF16 | P.MROPE_INTERLEAVED
    a.heads, a.kv_heads, a.head_dim, a.rotary_dim = 32, 8, 128, 128
    a.eps, a.rope_theta = 1e-6, 1e6
    a.num_seqs = len(seqs)
    a._ids = (C.c_uint32 * len(seqs))(*seqs)
    a._rows = (C.c_uint32 * len(seqs))(*rows)
    a.seq_ids, a.seq_rows = a._ids, a._rows
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.q_norm, a.k_norm = gq.data_ptr(), gk.data_ptr()
    a.positions = pos.data_ptr()
    a.out = out.data_ptr()
    a.kv = pool.handle
    return a


def one_call(pkg, backend, torch, pool, ctxs, rows, seed):
    """The same call through both entry points on forked copies of the same
    sequences; returns (ordinary output, no-alloc output)."""
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    base, fork = [], []
    for c in ctxs:
        s = pool.open()
        if c:
            kk = torch.randn((c, 8 * 128), generator=gen, device="cuda").bfloat16()
            vv = torch.randn((c, 8 * 128), generator=gen, device="cuda").bfloat16()
            pool.append(s, kk, vv)
        base.append(s)
        fork.append(pool.fork(s))
    n = sum(rows)
    q = torch.randn((n, 32 * 128), generator=gen, device="cuda").bfloat16()
    k = torch.randn((n, 8 * 128), generator=gen, device="cuda").bfloat16()
    v = torch.randn((n, 8 * 128), generator=gen, device="cuda").bfloat16()
    pos = torch.tensor([[c + r] * 3 for c, nr in zip(ctxs, rows) for r in range(nr)],
                       dtype=torch.int32, device="cuda")
    gq = (1 + 0.02 * torch.randn(128, generator=gen, device="cuda")).float()
    gk = (1 + 0.02 * torch.randn(128, generator=gen, device="cuda")).float()
    out_a = torch.full((n, 32 * 128), float("nan"), device="cuda")
    out_b = torch.full((n, 32 * 128), float("nan"), device="cuda")
    lib = backend.lib
    a = make_args(pkg, pool, base, rows, q, k, v, pos, out_a, gq, gk)
    backend.check(lib.safetyraise_kernel_attention_forward(backend.context, C.byref(a)),
                  "attention_forward")
    b = make_args(pkg, pool, fork, rows, q, k, v, pos, out_b, gq, gk)
    backend.check(lib.safetyraise_kernel_attention_forward_noalloc(backend.context, C.byref(b)),
                  "attention_forward_noalloc")
    for s, f, c, r in zip(base, fork, ctxs, rows):
        assert pool.len(s) == c + r and pool.len(f) == c + r
    result = out_a.cpu().numpy(), out_b.cpu().numpy()
    for s in base + fork:
        pool.close(s)
    return result


def test_noalloc_equals_attention_forward_on_two_calls(pkg, backend, torch_mod):
    torch = torch_mod
    pool = pkg.KvCache(backend, 8, 128, 64, 2048, 8192, 32)
    # a mixed call: decode rows (split-K records), verify rows (partition
    # records and the RoPE table) and prefill rows (the RoPE table)
    a, b = one_call(pkg, backend, torch, pool, [3000, 17, 1200, 0, 700], [1, 1, 5, 40, 3], 1)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)
    # a smaller second call on the same region
    a, b = one_call(pkg, backend, torch, pool, [90, 2500], [1, 2], 2)
    assert np.isfinite(a).all()
    assert np.array_equal(a, b)
    pool.destroy()


def test_noalloc_rejects_host_pointers_and_oversized_calls(pkg, backend, torch_mod):
    torch = torch_mod
    P = pkg.plugin
    lib = backend.lib
    pool = pkg.KvCache(backend, 8, 128, 64, 2400, 150000, 2)
    s = pool.open()
    # host pointers would need a staging allocation
    q = np.zeros((1, 32 * 128), np.float32)
    kv = np.zeros((1, 8 * 128), np.float32)
    pos = np.zeros((1, 3), np.int32)
    out = np.zeros((1, 32 * 128), np.float32)
    a = P.AttentionArgs()
    a.struct_size = C.sizeof(P.AttentionArgs)
    a.flags = P.MROPE_INTERLEAVED
    a.heads, a.kv_heads, a.head_dim, a.rotary_dim = 32, 8, 128, 128
    a.eps, a.rope_theta = 1e-6, 1e6
    a.num_seqs = 1
    ids = (C.c_uint32 * 1)(s)
    one = (C.c_uint32 * 1)(1)
    a.seq_ids, a.seq_rows = ids, one
    a.q, a.k, a.v = q.ctypes.data, kv.ctypes.data, kv.ctypes.data
    a.positions, a.out, a.kv = pos.ctypes.data, out.ctypes.data, pool.handle
    assert lib.safetyraise_kernel_attention_forward_noalloc(backend.context, C.byref(a)) == 1
    assert pool.len(s) == 0
    # a prefill call whose RoPE table (rows x 64 pairs x 8 bytes) exceeds the
    # 64 MiB region is refused before any kernel runs; the sequence keeps its
    # length and stays usable
    n = 140000
    tq = torch.empty((n, 32 * 128), device="cuda", dtype=torch.bfloat16)
    tk = torch.empty((n, 8 * 128), device="cuda", dtype=torch.bfloat16)
    tp = torch.zeros((n, 3), device="cuda", dtype=torch.int32)
    to = torch.empty((n, 32 * 128), device="cuda")
    rows = (C.c_uint32 * 1)(n)
    a.flags = P.DEVICE_POINTERS | P.INPUT_BF16 | P.MROPE_INTERLEAVED
    a.seq_rows = rows
    a.q, a.k, a.v = tq.data_ptr(), tk.data_ptr(), tk.data_ptr()
    a.positions, a.out = tp.data_ptr(), to.data_ptr()
    st = lib.safetyraise_kernel_attention_forward_noalloc(backend.context, C.byref(a))
    assert st == pkg.plugin.STATUS_OUT_OF_MEMORY
    text = lib.safetyraise_kernel_last_error(backend.context).decode()
    assert "scratch" in text
    assert pool.len(s) == 0
    del tq, tk, tp, to
    pool.destroy()


def test_calls_under_graph_capture_are_refused(pkg, backend, torch_mod):
    # a call advances the sequences' lengths and page lists on the host when
    # it is made, so a captured call could not be replayed: both entry points
    # refuse while the context's stream captures, before touching anything,
    # and the sequence is unchanged and usable afterwards
    torch = torch_mod
    P = pkg.plugin
    lib = backend.lib
    pool = pkg.KvCache(backend, 8, 128, 64, 64, 1024, 2)
    s = pool.open()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    q = torch.randn((1, 32 * 128), generator=gen, device="cuda").bfloat16()
    k = torch.randn((1, 8 * 128), generator=gen, device="cuda").bfloat16()
    pos = torch.zeros((1, 3), dtype=torch.int32, device="cuda")
    gq = torch.ones(128, device="cuda")
    out = torch.zeros((1, 32 * 128), device="cuda")
    a = make_args(pkg, pool, [s], [1], q, k, k, pos, out, gq, gq)
    a.flags |= P.ASYNC
    x = torch.zeros(4, device="cuda")
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    backend.set_stream(stream.cuda_stream)
    try:
        with torch.cuda.graph(graph, stream=stream):
            x.add_(1.0)
            st_plain = lib.safetyraise_kernel_attention_forward(backend.context, C.byref(a))
            text = lib.safetyraise_kernel_last_error(backend.context).decode()
            st_noalloc = lib.safetyraise_kernel_attention_forward_noalloc(backend.context,
                                                                          C.byref(a))
    finally:
        backend.set_stream(None)
    assert st_plain == P.STATUS_INVALID_ARGUMENT and st_noalloc == P.STATUS_INVALID_ARGUMENT
    assert "graph" in text
    assert pool.len(s) == 0
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(x, torch.ones(4, device="cuda"))
    # outside capture the same call runs
    a.flags &= ~P.ASYNC
    backend.check(lib.safetyraise_kernel_attention_forward_noalloc(backend.context, C.byref(a)),
                  "attention_forward_noalloc")
    assert pool.len(s) == 1
    assert torch.isfinite(out).all()
    pool.destroy()
