"""Seeded sweep of gated-delta-net layer shapes through the C-ABI, against the oracle.

Each case draws its layer from its own seed: key heads 1..16 with 1, 2 or 4
value heads per key head, key and value widths (128, which takes the tuned
kernels, or 48..96, which take the generic ones), conv kernel 1..6, non-zero
A_log and dt_bias, non-unit norm weights and seeded states and histories.
Then three consecutive calls over one to four sequences, each sequence with
1 row (decode), 2..8 or 9..100 rows (the chunked form), so the recurrence,
the conv history and the state carry across calls of different forms
(math.rs:158-239, native.rs:737-740).  f32 path: outputs and states within
|d| <= 1e-4 + 1e-4 |ref|, conv histories bit-exact after every call.
"""
import numpy as np
import pytest

from test_gpu_gdn import Layer, run_batch, seeded_state

pytestmark = pytest.mark.gpu

SWEEP = 48


def draw(case_id):
    rng = np.random.default_rng(0x6D450000 + case_id)
    hk = int(rng.choice([1, 2, 4, 16]))
    ratio = int(rng.choice([1, 2, 4]))
    tuned = rng.random() < 0.6
    dk = 128 if tuned else int(rng.choice([64, 96]))
    dv = 128 if tuned else int(rng.choice([48, 64, 80]))
    # the oracle's token-serial cost grows with hv * dv * dk
    while hk * ratio * dv * dk > 16 * 128 * 128 and hk > 1:
        hk //= 2
    K = int(rng.integers(1, 7))
    nseq = int(rng.integers(1, 5))
    calls = []
    for _ in range(3):
        calls.append([int(rng.choice([1, rng.integers(2, 9), rng.integers(9, 101)]))
                      for _ in range(nseq)])
    return rng, dict(hk=hk, hv=hk * ratio, dk=dk, dv=dv, K=K, calls=calls)


@pytest.mark.parametrize("case_id", range(SWEEP))
def test_gdn_shape_sweep(pkg, backend, case_id):
    rng, c = draw(case_id)
    print(f"case {case_id}: {c}", flush=True)
    L = Layer(rng, c["hk"], c["hv"], dk=c["dk"], dv=c["dv"], K=c["K"])
    L.a_log = (0.3 * rng.standard_normal(L.hv)).astype(np.float32)
    L.dt_bias = (0.3 * rng.standard_normal(L.hv)).astype(np.float32)
    L.norm = (1 + 0.1 * rng.standard_normal(L.dv)).astype(np.float32)
    nseq = len(c["calls"][0])
    pool = pkg.GdnState(backend, L.hk, L.hv, L.dk, L.dv, L.K, nseq)
    seqs, refs = [], []
    for _ in range(nseq):
        s = pool.open()
        m, h = seeded_state(rng, L)
        pool.write(s, m, h)
        seqs.append(s)
        refs.append((m.copy(), h.copy()))
    for call, rows in enumerate(c["calls"]):
        run_batch(pkg, backend, pool, L, seqs, rows, refs, rng, f"case {case_id} call {call}")
    pool.destroy()
