"""Seeded sweeps of attention shapes through the C-ABI, against the oracle.

Each case draws its geometry from its own seed: query heads per KV head
G = 1..8, head width 64, 128 or 256, page size 16, 64 or 128 tokens, full or
half rotary width, with or without QK-norm, and (some cases) the Qwen3.5 form:
per-head q/gate interleave, norm offset and interleaved MRoPE sections.  A
call holds one to three sequences, each with its own cached context and at
least 16 new rows, so it takes the prefill kernels (the reference's row loop,
src/model/native.rs:627-643; every row's keys appended before any row
attends).  Row counts and contexts fall on and off the 32-row blocks, the
64-key tiles and the page boundaries.  The mixed sweep draws calls whose
sequences take different kernels in one call: 1 new row (decode), 2..15
(MTP verify) and 16 or more (prefill).  Tolerance as the other bf16-path
tests: |d| <= 2e-3 + 1e-2 |ref|.
"""
import numpy as np
import pytest

from test_gpu_attention import Case, new_pool, run_case

pytestmark = pytest.mark.gpu

SWEEP = 64
MIXED = 32


def draw(case_id, mixed=False):
    rng = np.random.default_rng((0x5EED2000 if mixed else 0x5EED0000) + case_id)
    g = int(rng.integers(1, 9))
    dim = int(rng.choice([64, 128, 128, 256]))
    # query width heads * dim at most 4096, so the oracle stays fast
    kv_choices = [k for k in (1, 2, 4, 8) if g * k * dim <= 4096]
    kv_heads = int(rng.choice(kv_choices))
    page = int(rng.choice([16, 64, 64, 128]))
    rotary = dim if rng.random() < 0.6 else dim // 2
    qwen35 = rng.random() < 0.25
    qk_norm = qwen35 or rng.random() < 0.75
    nseq = int(rng.integers(1, 4))
    seqs = []
    for _ in range(nseq + (1 if mixed else 0)):
        ctx = int(rng.choice([0, rng.integers(1, 64), rng.integers(64, 700)]))
        if mixed:
            rows = int(rng.choice([1, rng.integers(2, 16), rng.integers(16, 100)]))
            ctx = max(ctx, 1) if rows == 1 else ctx
        else:
            rows = int(rng.choice([16, rng.integers(17, 64), rng.integers(64, 200)]))
        seqs.append((ctx, rows))
    return rng, dict(g=g, dim=dim, kv_heads=kv_heads, page=page, rotary=rotary, qwen35=qwen35,
                     qk_norm=qk_norm, seqs=seqs)


def run_drawn(pkg, backend, case_id, mixed):
    rng, c = draw(case_id, mixed)
    heads, kv_heads, dim = c["g"] * c["kv_heads"], c["kv_heads"], c["dim"]
    print(f"case {case_id} (mixed {mixed}): {c}", flush=True)
    max_tokens = max(ctx + rows for ctx, rows in c["seqs"]) + 8
    pool = new_pool(pkg, backend, kv_heads, dim, page_tokens=c["page"], max_tokens=max_tokens,
                    seqs=len(c["seqs"]))
    extra = dict(rotary=c["rotary"])
    axes = None
    if c["qwen35"]:
        # norm weights around 0 with the offset; MRoPE sections over the
        # rotary pairs (interleaved), positions differing per axis
        half = c["rotary"] // 2
        sec = (half - 2 * (half // 3), half // 3, half // 3)
        extra.update(theta=1e7, offset=True, gated=True, mrope=sec,
                     gq=(0.02 * rng.standard_normal(dim)).astype(np.float32),
                     gk=(0.02 * rng.standard_normal(dim)).astype(np.float32))
        axes = (0, 3, 7)
    elif c["qk_norm"]:
        extra.update(gq=(1 + 0.02 * rng.standard_normal(dim)).astype(np.float32),
                     gk=(1 + 0.02 * rng.standard_normal(dim)).astype(np.float32))
    cases = [Case(rng, pool, heads, kv_heads, dim, ctx=ctx, rows=rows, gated=c["qwen35"],
                  qk_norm=c["qk_norm"], pos_axes=axes, max_tokens=max_tokens)
             for ctx, rows in c["seqs"]]
    run_case(pkg, backend, pool, cases, **extra)
    pool.destroy()


@pytest.mark.parametrize("case_id", range(SWEEP))
def test_prefill_shape_sweep(pkg, backend, case_id):
    run_drawn(pkg, backend, case_id, mixed=False)


@pytest.mark.parametrize("case_id", range(MIXED))
def test_mixed_rows_sweep(pkg, backend, case_id):
    run_drawn(pkg, backend, case_id, mixed=True)
