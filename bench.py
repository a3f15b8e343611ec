"""Benchmark of the MI355X attention / GDN hot path on one GPU.

    python bench.py [--steps K] [--warmup W] [--workload decode] [--layers 36]

Prints ONE JSON line.  The default workload is BASELINE config 2 (Qwen3-8B
decode attention: 32 Q / 8 KV heads, head_dim 128, QK-RMSNorm + RoPE theta
1e6, bf16 paged KV, 16 sequences with context ~U[1024, 32768]); one step is
one decode token through all 36 layers' attention (36 plugin calls on 36
independent caches).  Inputs and caches are resident in HBM before timing.

`value` is algorithmic HBM bytes per step / step time.  `roofline` is for
the dominant kernel (attn_decode_kernel<128,4>): algorithmic bytes per launch
/ its average launch duration measured with HIP events on the stream the
plugin launches on.  `cpu_baseline` times the CPU oracle (the C restatement
of the reference's src/model/math.rs) on the same cache contents, one layer,
on the host cores of this machine.
"""
from __future__ import annotations

import argparse
import ctypes as C
import importlib
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
MFMA_BF16_PEAK_TFS = 2500.0  # dense bf16
METRIC = "decode attn HBM GB/s (% peak) + prefill attn TFLOP/s, Qwen3-8B GQA shape"
PROFILES = ROOT / "profiles"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="decode", choices=["decode", "prefill", "copy"])
    p.add_argument("--no-prefill", action="store_true",
                   help="decode workload only (skip the prefill figure of the same line)")
    p.add_argument("--prefill-steps", type=int, default=5)
    p.add_argument("--layers", type=int, default=36)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--seed", type=int, default=0x5A5A0001)
    return p.parse_args()


def traffic_from_profiles(kernel_tag: str):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary, if any."""
    f = PROFILES / f"{kernel_tag}_traffic.json"
    if not f.exists():
        return None
    try:
        return json.loads(f.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def bench_decode(args, torch, pkg):
    heads, kvh, dim, nseq, layers = 32, 8, 128, 16, args.layers
    rng = np.random.default_rng(args.seed)
    lengths = rng.integers(1024, 32768, size=nseq, endpoint=True)
    total_steps = args.warmup + args.steps
    max_tokens = int(lengths.max()) + total_steps + 1
    page = 64
    pages = int(sum((L + total_steps + page) // page + 1 for L in lengths)) + 8

    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()  # default priority
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)

    pools, seqs = [], []
    for _ in range(layers):
        pool = pkg.KvCache(backend, kvh, dim, page, pages, max_tokens, nseq)
        ids = []
        for L in lengths:
            s = pool.open()
            k = torch.randn((int(L), kvh * dim), generator=gen, device="cuda", dtype=torch.bfloat16)
            v = torch.randn((int(L), kvh * dim), generator=gen, device="cuda", dtype=torch.bfloat16)
            pool.append(s, k, v, flags=pkg.ASYNC)
            ids.append(s)
            del k, v
        pools.append(pool)
        seqs.append(ids)
    backend.synchronize()

    gq = (1 + 0.02 * torch.randn(dim, generator=gen, device="cuda")).float()
    gk = (1 + 0.02 * torch.randn(dim, generator=gen, device="cuda")).float()
    q = torch.randn((layers, nseq, heads * dim), generator=gen, device="cuda")
    k = torch.randn((layers, nseq, kvh * dim), generator=gen, device="cuda")
    v = torch.randn((layers, nseq, kvh * dim), generator=gen, device="cuda")
    out = torch.empty((layers, nseq, heads * dim), device="cuda")
    base = torch.from_numpy(lengths.astype(np.int32)).cuda()
    positions = [(base + s).view(nseq, 1).repeat(1, 3).contiguous() for s in range(total_steps)]

    P = pkg.plugin
    flags = (P.DEVICE_POINTERS | P.ASYNC | P.QK_NORM | P.MROPE_INTERLEAVED)
    ids_c = [(C.c_uint32 * nseq)(*s) for s in seqs]
    rows_c = (C.c_uint32 * nseq)(*([1] * nseq))

    def make_args(step, layer):
        a = P.AttentionArgs()
        a.struct_size = C.sizeof(P.AttentionArgs)
        a.flags = flags
        a.heads, a.kv_heads, a.head_dim, a.rotary_dim = heads, kvh, dim, dim
        a.eps, a.rope_theta = 1e-6, 1e6
        a.num_seqs = nseq
        a.seq_ids = ids_c[layer]
        a.seq_rows = rows_c
        a.q, a.k, a.v = q[layer].data_ptr(), k[layer].data_ptr(), v[layer].data_ptr()
        a.q_norm, a.k_norm = gq.data_ptr(), gk.data_ptr()
        a.positions = positions[step].data_ptr()
        a.out = out[layer].data_ptr()
        a.kv = pools[layer].handle
        return a

    all_args = [[make_args(s, l) for l in range(layers)] for s in range(total_steps)]
    fwd = backend.lib.safetyraise_kernel_attention_forward
    ctx = backend.context

    def step_bytes(step):
        ctx_tokens = int((lengths + step + 1).sum())  # every row sees len+1 keys
        io = nseq * (heads * dim * 4 * 2 + kvh * dim * 4 * 2 + 3 * 4)
        return ctx_tokens * kvh * dim * 2 * 2 + io

    for s in range(args.warmup):
        for l in range(layers):
            st = fwd(ctx, C.byref(all_args[s][l]))
            if st != 0:
                backend.check(st, "attention_forward")
    backend.synchronize()

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps * layers)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    i = 0
    for s in range(args.warmup, total_steps):
        for l in range(layers):
            ev[i][0].record(stream)
            st = fwd(ctx, C.byref(all_args[s][l]))
            ev[i][1].record(stream)
            i += 1
            if st != 0:
                backend.check(st, "attention_forward")
    t1.record(stream)
    torch.cuda.synchronize()
    backend.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / args.steps
    bytes_total = sum(step_bytes(s) for s in range(args.warmup, total_steps)) * layers
    value = bytes_total / (total_ms * 1e-3) / 1e9
    launch_us = np.array([a.elapsed_time(b) * 1e3 for a, b in ev])
    per_launch_bytes = bytes_total / len(ev)
    achieved = per_launch_bytes / (launch_us.mean() * 1e-6) / 1e9

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline_decode(pkg, pools[0], seqs[0], lengths + total_steps, q[0], k[0], v[0],
                                  positions[-1], gq, gk, heads, kvh, dim)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-8b decode attention (BASELINE config 2), 36 layers per step",
            "heads": heads, "kv_heads": kvh, "head_dim": dim, "seqs": nseq,
            "context_lens": [int(x) for x in lengths], "kv_dtype": "bf16", "page_tokens": page,
            "layers": layers, "qk_norm": True, "rope_theta": 1e6,
        },
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "us_per_layer": round(ms_per_step * 1e3 / layers, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("attn_decode_qwen3_8b"),
            # one decode call = the split-K kernel plus its small combine pass;
            # the events bracket both (rocprofv3 lists them separately)
            "kernel": "attn_decode_kernel<128,4> + attn_combine_kernel<128,4>",
            "launch_us_mean": round(float(launch_us.mean()), 2),
            "bytes_per_launch": int(per_launch_bytes),
        },
        "cpu_baseline": cpu,
    }
    for p in pools:
        p.destroy()
    backend.close()
    return result


def cpu_baseline_decode(pkg, pool, seqs, lens, q, k, v, pos, gq, gk, heads, kvh, dim):
    """Times the CPU oracle on one layer of the same workload (same cache rows)."""
    from oracle import pyoracle as O

    qn, kn, vn = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    pn = pos.cpu().numpy().astype(np.int64)
    gqn, gkn = gq.cpu().numpy(), gk.cpu().numpy()
    nthreads = min(os.cpu_count() or 1, 16)
    t_single = t_multi = 0.0
    nbytes = 0
    for i, s in enumerate(seqs):
        length = pool.len(s)
        keys, vals = pool.read(s, 0, length)
        cache = O.KvCache(kvh * dim, length + 2, 64, bf16=True)
        cache.append_many(keys, vals)
        del keys, vals
        for threads in (1, nthreads):
            c = cache.clone()
            t = time.perf_counter()
            O.attention_rows(qn[i:i + 1], kn[i:i + 1], vn[i:i + 1], pn[i:i + 1], c, heads=heads,
                             kv_heads=kvh, dim=dim, rotary_dim=dim, theta=1e6, eps=1e-6,
                             q_norm=gqn, k_norm=gkn, threads=threads)
            dt = time.perf_counter() - t
            if threads == 1:
                t_single += dt
            else:
                t_multi += dt
        nbytes += (length + 1) * kvh * dim * 2 * 2
    return {
        "value": round(nbytes / t_single / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"one layer of the same workload: 16 sequences, one decode row each, "
                   f"{int(sum(lens))} cached tokens read back from the GPU cache; f32 oracle "
                   f"over bf16-valued K/V; bytes counted as bf16 like the GPU figure"),
        "us_per_layer": round(t_single * 1e6, 1),
        "all_cores": {"value": round(nbytes / t_multi / 1e9, 3), "cores": nthreads,
                      "us_per_layer": round(t_multi * 1e6, 1)},
    }


def bench_prefill(args, torch, pkg, steps, warmup):
    """Qwen3-8B chunked causal prefill attention.

    4 sequences x 4096 tokens appended in chunks of 512 (8 calls of 4 x 512
    rows), 32 Q / 8 KV heads, head_dim 128, QK-RMSNorm + RoPE theta 1e6, bf16
    inputs ~N(0,1), bf16 KV.  One step is the whole 4096-token prefill of one
    layer (the cache is truncated to empty before each step).  FLOPs count the
    causal work exactly: 4 * head_dim per (query row, visible key, q head).
    """
    heads, kvh, dim, nseq, total, chunk = 32, 8, 128, 4, 4096, 512
    nchunk = total // chunk
    page = 64
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0002)
    pool = pkg.KvCache(backend, kvh, dim, page, nseq * (total // page) + 8, total, nseq)
    ids = [pool.open() for _ in range(nseq)]
    gq = (1 + 0.02 * torch.randn(dim, generator=gen, device="cuda")).float()
    gk = (1 + 0.02 * torch.randn(dim, generator=gen, device="cuda")).float()
    rows = nseq * chunk
    q = torch.randn((nchunk, rows, heads * dim), generator=gen, device="cuda").bfloat16()
    k = torch.randn((nchunk, rows, kvh * dim), generator=gen, device="cuda").bfloat16()
    v = torch.randn((nchunk, rows, kvh * dim), generator=gen, device="cuda").bfloat16()
    out = torch.empty((rows, heads * dim), device="cuda")
    positions = []
    for c in range(nchunk):
        p1 = torch.arange(c * chunk, (c + 1) * chunk, dtype=torch.int32, device="cuda")
        positions.append(p1.repeat(nseq).view(rows, 1).repeat(1, 3).contiguous())

    P = pkg.plugin
    flags = (P.DEVICE_POINTERS | P.ASYNC | P.QK_NORM | P.INPUT_BF16 | P.MROPE_INTERLEAVED)
    ids_c = (C.c_uint32 * nseq)(*ids)
    rows_c = (C.c_uint32 * nseq)(*([chunk] * nseq))

    def make_args(c):
        a = P.AttentionArgs()
        a.struct_size = C.sizeof(P.AttentionArgs)
        a.flags = flags
        a.heads, a.kv_heads, a.head_dim, a.rotary_dim = heads, kvh, dim, dim
        a.eps, a.rope_theta = 1e-6, 1e6
        a.num_seqs = nseq
        a.seq_ids = ids_c
        a.seq_rows = rows_c
        a.q, a.k, a.v = q[c].data_ptr(), k[c].data_ptr(), v[c].data_ptr()
        a.q_norm, a.k_norm = gq.data_ptr(), gk.data_ptr()
        a.positions = positions[c].data_ptr()
        a.out = out.data_ptr()
        a.kv = pool.handle
        return a

    chunk_args = [make_args(c) for c in range(nchunk)]
    fwd = backend.lib.safetyraise_kernel_attention_forward
    ctx = backend.context

    def chunk_flops(c):
        # per (seq, q head): 4 * dim * sum_{i<512} (512 c + i + 1)
        return 4 * dim * (chunk * chunk * c + chunk * (chunk + 1) // 2) * nseq * heads

    step_flops = sum(chunk_flops(c) for c in range(nchunk))

    def run_step(events=None):
        for s in ids:
            pool.truncate(s, 0)
        for c in range(nchunk):
            if events is not None:
                events[c][0].record(stream)
            st = fwd(ctx, C.byref(chunk_args[c]))
            if events is not None:
                events[c][1].record(stream)
            if st != 0:
                backend.check(st, "attention_forward")

    for _ in range(warmup):
        run_step()
    backend.synchronize()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(nchunk)] for _ in range(steps)]
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for s in range(steps):
        run_step(ev[s])
    t1.record(stream)
    torch.cuda.synchronize()
    backend.synchronize()
    total_ms = t0.elapsed_time(t1)
    ms_per_step = total_ms / steps
    tflops = step_flops / (ms_per_step * 1e-3) / 1e12
    per_chunk_us = np.array([[a.elapsed_time(b) * 1e3 for a, b in row] for row in ev]).mean(0)
    call_tflops = step_flops / (per_chunk_us.sum() * 1e-6) / 1e12
    result = {
        "workload": "qwen3-8b chunked causal prefill attention (BASELINE config 3): 4 x 4096 "
                    "tokens in chunks of 512, one layer per step",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "pct_of_mfma_peak": round(100 * tflops / MFMA_BF16_PEAK_TFS, 2),
        "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gflop_per_step": round(step_flops / 1e9, 2),
        "dtype": "bf16 MFMA, f32 accumulate and softmax",
        "chunk_us": [round(float(x), 1) for x in per_chunk_us],
        "roofline": {
            "bound": "mfma",
            "achieved": round(call_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFS,
            "unit": "TFLOP/s",
            "frac": round(call_tflops / MFMA_BF16_PEAK_TFS, 4),
            "traffic": traffic_from_profiles("attn_prefill_qwen3_8b"),
            "kernel": "kv_append_rows_kernel<128> + attn_prefill_kernel<128,4>",
            "launch_us_mean": round(float(per_chunk_us.mean()), 2),
            "flops_per_step": int(step_flops),
        },
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_prefill(q, k, v, positions, gq, gk, heads, kvh, dim,
                                                      chunk)
    pool.destroy()
    backend.close()
    return result


def cpu_baseline_prefill(q, k, v, positions, gq, gk, heads, kvh, dim, chunk):
    """CPU oracle on a bounded sample: chunk 0 of sequence 0 (512 rows, empty cache)."""
    from oracle import pyoracle as O

    qn = q[0, :chunk].float().cpu().numpy()
    kn = k[0, :chunk].float().cpu().numpy()
    vn = v[0, :chunk].float().cpu().numpy()
    pn = positions[0][:chunk].cpu().numpy().astype(np.int64)
    gqn, gkn = gq.cpu().numpy(), gk.cpu().numpy()
    flops = 4 * dim * (chunk * (chunk + 1) // 2) * heads
    nthreads = min(os.cpu_count() or 1, 16)
    res = {}
    for threads in (1, nthreads):
        cache = O.KvCache(kvh * dim, chunk, 64, bf16=True)
        t = time.perf_counter()
        O.attention_rows(qn, kn, vn, pn, cache, heads=heads, kv_heads=kvh, dim=dim,
                         rotary_dim=dim, theta=1e6, eps=1e-6, q_norm=gqn, k_norm=gkn,
                         threads=threads)
        res[threads] = time.perf_counter() - t
    return {
        "value": round(flops / res[1] / 1e9, 3),
        "unit": "GFLOP/s",
        "cores": 1,
        "kind": "port",
        "sample": "chunk 0 of sequence 0 (512 rows on an empty cache, 32 heads) of the same "
                  "inputs; f32 oracle with bf16 KV storage",
        "ms": round(res[1] * 1e3, 1),
        "all_cores": {"value": round(flops / res[nthreads] / 1e9, 3), "cores": nthreads,
                      "ms": round(res[nthreads] * 1e3, 1)},
    }


def bench_copy(args, torch):
    """Calibration: a plain device copy of a known size (for PMC byte counters)."""
    nbytes = 1 << 30
    a = torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").normal_()
    b = torch.empty_like(a)
    for _ in range(args.warmup):
        b.copy_(a)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        b.copy_(a)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / args.steps
    return {"metric": "device copy GB/s (calibration)", "value": round(2 * nbytes / ms / 1e6, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
            "config": {"workload": "copy 1 GiB read + 1 GiB write"}}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested)", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)
    pkg = importlib.import_module("safetyraise-lmengine_amd")
    if args.workload == "decode":
        result = bench_decode(args, torch, pkg)
        if not args.no_prefill:
            result["prefill"] = bench_prefill(args, torch, pkg, args.prefill_steps, 2)
    elif args.workload == "prefill":
        result = bench_prefill(args, torch, pkg, args.steps, args.warmup)
        result = {"metric": "prefill attn TFLOP/s, Qwen3-8B GQA shape", "n_gpus": 1,
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                  "data": "synthetic", "config": {"workload": result.pop("workload")}, **result}
    else:
        result = bench_copy(args, torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
