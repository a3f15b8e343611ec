"""Benchmark of the MI355X attention / GDN hot path on one GPU.

    python bench.py [--steps K] [--warmup W] [--workload decode] [--layers 36]

Prints ONE JSON line.  The default workload is BASELINE config 2 (Qwen3-8B
decode attention: 32 Q / 8 KV heads, head_dim 128, QK-RMSNorm + RoPE theta
1e6, bf16 paged KV, 16 sequences with context ~U[1024, 32768]); one step is
one decode token through all 36 layers' attention (36 plugin calls on 36
independent caches).  Inputs and caches are resident in HBM before timing.

`value` is algorithmic HBM bytes per step / step time.  `roofline` is for
the dominant kernel (attn_decode_kernel<128,4>): algorithmic bytes per launch
/ its average launch duration, measured in a second pass with the plugin's
kernel timing (HIP start/stop events of each dispatch, recorded on the stream
the plugin launches on); `kernels` lists every kernel of that pass with its
launches per call and mean duration.  `cpu_baseline` times the CPU oracle
(the C restatement of the reference's src/model/math.rs) on the same cache
contents, one layer, on the host cores of this machine.  The other workloads
on the line (prefill, verify, gdn_decode, gdn_prefill, linear) are measured
the same way.
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
    p.add_argument("--workload", default="decode",
                   choices=["decode", "prefill", "verify", "verify-qwen3.5", "gdn-decode",
                            "gdn-prefill", "linear", "linear-prefill", "copy"])
    p.add_argument("--rows", type=int, default=5, help="verify rows per sequence (1 + drafts)")
    p.add_argument("--no-prefill", action="store_true",
                   help="decode workload only (skip the prefill figure of the same line)")
    p.add_argument("--prefill-steps", type=int, default=10)
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


def mfma_from_profiles(kernel_tag: str, kernels, launch_us: dict):
    """MFMA use of the leg's kernels from the committed rocprofv3 SQ-counter
    summary (profiles/<tag>_pmc.json): the counted MFMA busy fraction
    (SQ_VALU_MFMA_BUSY_CYCLES over 4 SIMDs x CUs x elapsed cycles), the MFMA
    FLOPs issued per launch (SQ_INSTS_VALU_MFMA_MOPS_* x 512, fixed by the
    workload's shapes) and, with this run's launch durations, the issued rate
    and the time those MFMAs take at the dense peak of their type."""
    f = PROFILES / f"{kernel_tag}_pmc.json"
    if not f.exists():
        return None
    try:
        prof = json.loads(f.read_text())["kernels"]
    except (OSError, ValueError, KeyError):
        return None
    out = {"source": f"profiles/{kernel_tag}_pmc.json", "kernels": {}}
    at_peak_us = run_us = 0.0
    for prefix in kernels:
        found = [(n, d) for n, d in prof.items() if n.startswith(prefix) and "mfma_util" in d]
        if not found or prefix not in launch_us:
            continue
        name, d = found[0]
        c = d["counters_mean_per_dispatch"]
        f32_flops = 512 * c.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)
        half_flops = d["mfma_flops_issued"] - f32_flops
        us = launch_us[prefix]
        peak_us = 1e6 * (f32_flops / (MFMA_F32_PEAK_TFS * 1e12)
                         + half_flops / (MFMA_BF16_PEAK_TFS * 1e12))
        at_peak_us += peak_us
        run_us += us
        out["kernels"][name] = {
            "pmc_mfma_util": d["mfma_util"],
            "mfma_flops_issued_per_launch": d["mfma_flops_issued"],
            "issued_tflops_this_run": round(d["mfma_flops_issued"] / (us * 1e-6) / 1e12, 2),
            "valu_non_mfma_per_mfma": d["valu_non_mfma_per_mfma"],
            "lds_bank_conflict_frac": d["lds_bank_conflict_frac_of_lds_active"],
        }
    if not out["kernels"]:
        return None
    # the share of the kernels' time their MFMAs would take at the dense peak
    # of each type (f32 157.3, fp16/bf16 2500 TFLOP/s)
    out["issued_at_peak_frac_of_time"] = round(at_peak_us / run_us, 4)
    return out


def _load_roctx():
    """The ROCTx range API: `rocprofv3 --marker-trace` records the ranges, and
    without a profiler the calls do nothing.  None when the library is absent."""
    for name in ("librocprofiler-sdk-roctx.so.1", "/opt/rocm/lib/librocprofiler-sdk-roctx.so.1"):
        try:
            lib = C.CDLL(name)
        except OSError:
            continue
        lib.roctxRangePushA.argtypes = [C.c_char_p]
        lib.roctxRangePushA.restype = C.c_int
        lib.roctxRangePop.restype = C.c_int
        return lib
    return None


_ROCTX = _load_roctx()


def region_begin(name: str) -> None:
    """Opens a ROCTx range around a bench region (the timed steps or the
    kernel-timing pass), called with the stream idle: a kernel trace of the
    run then tells that region's dispatches from the rest."""
    if _ROCTX is not None:
        _ROCTX.roctxRangePushA(name.encode())


def region_end() -> None:
    """Closes the range region_begin opened (after a synchronize)."""
    if _ROCTX is not None:
        _ROCTX.roctxRangePop()


def kernel_pass(backend, run, calls, name):
    """Runs `run()` (which makes `calls` plugin calls) with the plugin's kernel
    timing on: each launch's device duration from the start/stop timestamps of
    its own dispatch (hipExtLaunchKernelGGL events on the plugin's stream), the
    figure a profiler's kernel trace records.  The pass follows the timed
    steps directly, with the GPU in the same state; the events stay out of
    the timed steps, where they would slow the host's launches.  `name`
    labels the pass's ROCTx range.  Returns {kernel name: {"per_call":
    launches per call, "us": mean duration}}."""
    backend.timing(True)  # synchronizes the stream
    region_begin(f"{name} timing pass")
    try:
        run()
        times = backend.kernel_times()  # synchronizes the stream
    finally:
        region_end()
        backend.timing(False)
    return {name: {"per_call": round(n / calls, 3), "us": round(us, 2)}
            for name, (n, us) in times.items()}


def bench_decode(args, torch, pkg):
    heads, kvh, dim, nseq, layers = 32, 8, 128, 16, args.layers
    rng = np.random.default_rng(args.seed)
    lengths = rng.integers(1024, 32768, size=nseq, endpoint=True)
    total_steps = args.warmup + args.steps
    event_steps = total_steps + args.steps  # a second pass times each call
    max_tokens = int(lengths.max()) + event_steps + 1
    page = 64
    pages = int(sum((L + event_steps + page) // page + 1 for L in lengths)) + 8

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
    positions = [(base + s).view(nseq, 1).repeat(1, 3).contiguous() for s in range(event_steps)]

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

    all_args = [[make_args(s, l) for l in range(layers)] for s in range(event_steps)]
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

    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("decode timed")
    t0.record(stream)
    for s in range(args.warmup, total_steps):
        for l in range(layers):
            st = fwd(ctx, C.byref(all_args[s][l]))
            if st != 0:
                backend.check(st, "attention_forward")
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    total_ms = t0.elapsed_time(t1)
    # kernel durations in a second pass of the same number of steps (the
    # timing events stay out of the timed region); each call there sees
    # `steps` more keys per sequence

    def second_pass():
        for s in range(total_steps, event_steps):
            for l in range(layers):
                st = fwd(ctx, C.byref(all_args[s][l]))
                if st != 0:
                    backend.check(st, "attention_forward")

    kernels = kernel_pass(backend, second_pass, args.steps * layers, "decode")
    ms_per_step = total_ms / args.steps
    bytes_total = sum(step_bytes(s) for s in range(args.warmup, total_steps)) * layers
    value = bytes_total / (total_ms * 1e-3) / 1e9
    launch_us = kernels["attn_decode_kernel"]["us"]
    per_launch_bytes = sum(step_bytes(s) for s in range(total_steps, event_steps)) / args.steps
    achieved = per_launch_bytes / (launch_us * 1e-6) / 1e9

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
            # the split-K kernel reads every cached K/V byte; its small
            # combine pass merges the per-slice records (listed in `kernels`)
            "kernel": "attn_decode_kernel<128,4,true>",
            "launch_us_mean": round(float(launch_us), 2),
            "bytes_per_launch": int(per_launch_bytes),
        },
        "kernels": kernels,
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

    def run_step():
        for s in ids:
            pool.truncate(s, 0)
        for c in range(nchunk):
            st = fwd(ctx, C.byref(chunk_args[c]))
            if st != 0:
                backend.check(st, "attention_forward")

    for _ in range(warmup):
        run_step()
    backend.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("prefill timed")
    t0.record(stream)
    for s in range(steps):
        run_step()
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    total_ms = t0.elapsed_time(t1)
    # kernel durations (the roofline's launch figure) come from a second pass
    # with the plugin's kernel timing on; one untimed step queued first brings
    # the GPU back from idle
    run_step()

    def second_pass():
        for s in range(steps):
            run_step()

    kernels = kernel_pass(backend, second_pass, steps * nchunk, "prefill")
    ms_per_step = total_ms / steps
    tflops = step_flops / (ms_per_step * 1e-3) / 1e12
    # the attention kernel of the call: the launch route picks it by shape
    attn_name = max((n for n in kernels if n.startswith("attn_prefill")),
                    key=lambda n: kernels[n]["us"] * kernels[n]["per_call"])
    attn_us = kernels[attn_name]["us"]
    call_tflops = step_flops / nchunk / (attn_us * 1e-6) / 1e12
    result = {
        "workload": "qwen3-8b chunked causal prefill attention (BASELINE config 3): 4 x 4096 "
                    "tokens in chunks of 512, one layer per step",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "pct_of_mfma_peak": round(100 * tflops / MFMA_BF16_PEAK_TFS, 2),
        "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gflop_per_step": round(step_flops / 1e9, 2),
        # K and V are the cache's bf16 values converted exactly to fp16 while
        # staged; q and P are rounded to fp16 (the fp16 MFMA has the bf16 rate)
        "dtype": "fp16 MFMA operands (v_mfma_f32_32x32x16_f16) over the bf16 cache, "
                 "f32 accumulate and softmax",
        "roofline": {
            "bound": "mfma",
            "achieved": round(call_tflops, 2),
            "peak": MFMA_BF16_PEAK_TFS,
            "unit": "TFLOP/s",
            "frac": round(call_tflops / MFMA_BF16_PEAK_TFS, 4),
            "traffic": traffic_from_profiles("attn_prefill_qwen3_8b"),
            # (the pipelined kernel is templated on the group size only)
            "kernel": (f"{attn_name}<4>" if attn_name == "attn_prefill_pipe_kernel"
                       else f"{attn_name}<128,4,true>"),
            "launch_us_mean": round(float(attn_us), 2),
            "flops_per_launch": int(step_flops // nchunk),
            "flops_per_step": int(step_flops),
            "mfma_util": mfma_from_profiles("attn_prefill_qwen3_8b", [attn_name],
                                            {attn_name: float(attn_us)}),
        },
        "kernels": kernels,
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


MFMA_F32_PEAK_TFS = 157.3  # MI355X dense fp32 matrix
GDN_KERNEL_CHUNK = 32  # rows per chunk of the chunked GDN kernels (kCk in gdn_kernels.hip)


def gdn_layer_setup(torch, pkg, backend, gen, hk, hv, dk, dv, K, nseq):
    """Seeded GDN layer (BASELINE config 4 draws: A_log 0, dt_bias 0, conv ~N(0,1)/2,
    norm 1) and a state pool whose sequences start from a N(0, 0.02) state."""
    C_ = 2 * hk * dk + hv * dv
    layer = {
        "a_log": torch.zeros(hv, device="cuda"),
        "dt_bias": torch.zeros(hv, device="cuda"),
        "conv": (torch.randn((C_, K), generator=gen, device="cuda") / 2),
        "norm": torch.ones(dv, device="cuda"),
    }
    pool = pkg.GdnState(backend, hk, hv, dk, dv, K, nseq)
    ids = [pool.open() for _ in range(nseq)]
    return layer, pool, ids, C_


def gdn_args(pkg, pool, ids_c, rows_c, nseq, x, layer, out, asynchronous=True):
    P = pkg.plugin
    a = P.GdnArgs()
    a.struct_size = C.sizeof(P.GdnArgs)
    a.flags = P.DEVICE_POINTERS | (P.ASYNC if asynchronous else 0)
    a.eps = 1e-6
    a.num_seqs = nseq
    a.seq_ids, a.seq_rows = ids_c, rows_c
    qkv, z, av, bv = x
    a.qkv, a.z, a.a, a.b = qkv.data_ptr(), z.data_ptr(), av.data_ptr(), bv.data_ptr()
    a.a_log, a.dt_bias = layer["a_log"].data_ptr(), layer["dt_bias"].data_ptr()
    a.conv_weight, a.norm = layer["conv"].data_ptr(), layer["norm"].data_ptr()
    a.out = out.data_ptr()
    a.state = pool.handle
    return a


def bench_gdn_decode(args, torch, pkg, steps, warmup, layers=64):
    """BASELINE config 4, decode: Qwen3.5-style GDN, Hk 16 / Hv 32, d 128, conv 4,
    batch 8, one token per sequence; one step = one token through `layers`
    independent GDN layers.  HBM-bound: algorithmic bytes = state read + write,
    conv history read + write, the inputs, the conv weights and the output."""
    hk, hv, dk, dv, K, nseq = 16, 32, 128, 128, 4, 8
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0003)
    rng = np.random.default_rng(0x5A5A0003)
    P = pkg.plugin
    pools, all_args, layer_w = [], [], []
    total = warmup + steps
    outs = torch.empty((layers, nseq, hv * dv), device="cuda")
    for l in range(layers):
        layer, pool, ids, C_ = gdn_layer_setup(torch, pkg, backend, gen, hk, hv, dk, dv, K, nseq)
        for s in ids:
            m = (0.02 * rng.standard_normal((hv, dv, dk))).astype(np.float32)
            hst = (0.5 * rng.standard_normal((C_, K - 1))).astype(np.float32)
            pool.write(s, m, hst)
        xs = [(torch.randn((nseq, C_), generator=gen, device="cuda"),
               torch.randn((nseq, hv * dv), generator=gen, device="cuda"),
               torch.randn((nseq, hv), generator=gen, device="cuda"),
               torch.randn((nseq, hv), generator=gen, device="cuda")) for _ in range(2)]
        ids_c = (C.c_uint32 * nseq)(*ids)
        rows_c = (C.c_uint32 * nseq)(*([1] * nseq))
        all_args.append([gdn_args(pkg, pool, ids_c, rows_c, nseq, xs[i], layer, outs[l])
                         for i in range(2)])
        pools.append((pool, ids_c, rows_c, xs))
        layer_w.append(layer)
    backend.synchronize()
    fwd = backend.lib.safetyraise_kernel_gdn_forward
    ctx = backend.context

    def run(step):
        for l in range(layers):
            st = fwd(ctx, C.byref(all_args[l][step & 1]))
            if st != 0:
                backend.check(st, "gdn_forward")

    for s in range(warmup):
        run(s)
    backend.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("gdn-decode timed")
    t0.record(stream)
    for s in range(steps):
        run(warmup + s)
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    # kernel durations in a second pass, outside the timed region, after one
    # untimed step
    run(warmup + steps)

    def second_pass():
        for s in range(steps):
            run(warmup + steps + 1 + s)

    kernels = kernel_pass(backend, second_pass, steps * layers, "gdn-decode")
    C_ = 2 * hk * dk + hv * dv
    per_layer = (2 * nseq * hv * dv * dk * 4          # state read + write
                 + 2 * nseq * C_ * (K - 1) * 4        # conv history read + write
                 + nseq * (C_ + hv * dv + 2 * hv) * 4  # qkv, z, a, b
                 + C_ * K * 4                         # conv weights
                 + nseq * hv * dv * 4)                # output
    ms = t0.elapsed_time(t1) / steps
    head_name = next(n for n in kernels if n.startswith("gdn_head"))
    call_us = kernels[head_name]["us"]
    value = per_layer * layers / (ms * 1e-3) / 1e9
    achieved = per_layer / (call_us * 1e-6) / 1e9
    result = {
        "workload": f"qwen3.5 GDN decode (BASELINE config 4): Hk 16 / Hv 32, d 128, conv 4, "
                    f"batch 8, {layers} layers per step",
        "value": round(value, 2), "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "dtype": "f32",
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("gdn_decode_qwen35"),
            "kernel": "gdn_head_kernel<512, ConvK<4>>",
            "launch_us_mean": round(float(call_us), 2),
            "bytes_per_launch": int(per_layer),
        },
        "kernels": kernels,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_gdn(pools[0][0], pools[0][1], pools[0][3][0],
                                                  layer_w[0], hk, hv, dk, dv, K, nseq, 1,
                                                  per_layer, "GB/s")
    for pool, *_ in pools:
        pool.destroy()
    backend.close()
    return result


def bench_gdn_prefill(args, torch, pkg, steps, warmup):
    """BASELINE config 4, prefill: 2 sequences x 2048 tokens in chunks of 64 (32 calls
    per layer); one step = the whole prefill of one layer from a zero state.  Two
    kernels run the chunked (WY) form of the delta rule in chunks of 32 rows on f32
    MFMA: gdn_chunk_prep_kernel (everything that does not involve the state, for all
    chunks of a call at once) and gdn_chunk_scan_kernel (the products with the
    state, chunk after chunk); the roofline's duration is the sum of their mean
    durations per call.  `value` counts the token-serial work, 7 * Dk * Dv per (row, value head)
    (decay, predict, correct, read), independent of the chunking; the roofline
    counts the chunked form's own FLOPs at its chunk size C = 32:
    4 C^2 Dk + 2/3 C^3 + 4 C^2 Dv + 8 C Dk Dv + 2 C^2 Dv per (sequence, value head,
    chunk)."""
    hk, hv, dk, dv, K, nseq, total, chunk = 16, 32, 128, 128, 4, 2, 2048, 64
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0004)
    layer, pool, ids, C_ = gdn_layer_setup(torch, pkg, backend, gen, hk, hv, dk, dv, K, nseq)
    nchunk = total // chunk
    rows = nseq * chunk
    xs = [(torch.randn((rows, C_), generator=gen, device="cuda"),
           torch.randn((rows, hv * dv), generator=gen, device="cuda"),
           torch.randn((rows, hv), generator=gen, device="cuda"),
           torch.randn((rows, hv), generator=gen, device="cuda")) for _ in range(nchunk)]
    out = torch.empty((rows, hv * dv), device="cuda")
    zero_m = np.zeros((hv, dv, dk), np.float32)
    zero_h = np.zeros((C_, K - 1), np.float32)
    fwd = backend.lib.safetyraise_kernel_gdn_forward
    ctx = backend.context

    def make(ids_now):
        ids_c = (C.c_uint32 * nseq)(*ids_now)
        rows_c = (C.c_uint32 * nseq)(*([chunk] * nseq))
        return [gdn_args(pkg, pool, ids_c, rows_c, nseq, xs[c], layer, out) for c in range(nchunk)]

    state = {"ids": ids, "args": make(ids)}

    def reset():
        # a fresh prompt: new sequences start from a zero state and history
        for s in state["ids"]:
            pool.close(s)
        state["ids"] = [pool.open() for _ in range(nseq)]
        state["args"] = make(state["ids"])

    def run():
        for c in range(nchunk):
            st = fwd(ctx, C.byref(state["args"][c]))
            if st != 0:
                backend.check(st, "gdn_forward")

    for _ in range(warmup):
        reset()
        run()
    backend.synchronize()
    total_ms = 0.0
    for s in range(steps):
        reset()  # host bookkeeping and a state clear, outside the timed region
        backend.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        region_begin("gdn-prefill timed")
        t0.record(stream)
        run()
        t1.record(stream)
        torch.cuda.synchronize()
        region_end()
        total_ms += t0.elapsed_time(t1)
    backend.synchronize()
    # kernel durations in a second pass, outside the timed region

    def second_pass():
        for s in range(steps):
            reset()
            run()

    kernels = kernel_pass(backend, second_pass, steps * nchunk, "gdn-prefill")
    ms = total_ms / steps
    flops = 7 * dk * dv * hv * nseq * total
    tflops = flops / (ms * 1e-3) / 1e12
    # the roofline's algorithmic count: the chunked (WY) form's FLOPs at the
    # chunk the kernel runs, C = 32 rows (each 64-row call is two chunks):
    # 4 C^2 Dk + 2/3 C^3 + 4 C^2 Dv + 8 C Dk Dv + 2 C^2 Dv per (sequence, value
    # head, chunk); the token-serial count is reported beside it
    ck = GDN_KERNEL_CHUNK
    chunked_form = ((4 * ck * ck * dk + 2 * ck ** 3 / 3 + 4 * ck * ck * dv + 8 * ck * dk * dv
                     + 2 * ck * ck * dv) * nseq * hv * (total // ck))
    chunk_us = kernels["gdn_chunk_prep_kernel"]["us"] + kernels["gdn_chunk_scan_kernel"]["us"]
    chunk_tf = chunked_form / nchunk / (chunk_us * 1e-6) / 1e12
    serial_tf = flops / nchunk / (chunk_us * 1e-6) / 1e12
    result = {
        "workload": "qwen3.5 GDN prefill (BASELINE config 4): 2 x 2048 tokens in chunks of 64, "
                    "one layer per step, from a zero state",
        "value": round(tflops, 3), "unit": "TFLOP/s",
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "gflop_per_step_token_serial": round(flops / 1e9, 2),
        "gflop_per_step_chunked_form": round(chunked_form / 1e9, 2),
        "dtype": "f32: chunked WY form, prep and scan on v_mfma_f32_16x16x4f32",
        "roofline": {
            # achieved: the reference's own (token-serial) f32 work over the
            # chunked kernels' time, against the f32 matrix peak: the arithmetic
            # the path must reproduce, whatever form computes it
            "bound": "mfma", "achieved": round(serial_tf, 3), "peak": MFMA_F32_PEAK_TFS,
            "unit": "TFLOP/s", "frac": round(serial_tf / MFMA_F32_PEAK_TFS, 4),
            "flops_counted": "token-serial: 7 Dk Dv per (row, value head)",
            "chunked_form_tflops": round(chunk_tf, 3),
            "chunked_form_frac": round(chunk_tf / MFMA_F32_PEAK_TFS, 4),
            "traffic": traffic_from_profiles("gdn_prefill_qwen35"),
            "kernel": "gdn_chunk_prep_kernel<ConvK<4>, true> + gdn_chunk_scan_kernel (the "
                      "call's chunked form, its prep with two workgroups per record: sum of the "
                      "two kernels' mean durations)",
            "launch_us_mean": round(float(chunk_us), 2),
            "flops_per_launch": int(flops / nchunk),
            "flops_per_step": int(flops),
            "chunked_form_flops_per_step": int(chunked_form),
            "mfma_util": mfma_from_profiles(
                "gdn_prefill_qwen35", ["gdn_chunk_prep_kernel", "gdn_chunk_scan_kernel"],
                {n: float(kernels[n]["us"]) for n in ("gdn_chunk_prep_kernel",
                                                      "gdn_chunk_scan_kernel")}),
        },
        "kernels": kernels,
    }
    if not args.no_cpu:
        ids_c = (C.c_uint32 * nseq)(*state["ids"])
        result["cpu_baseline"] = cpu_baseline_gdn(pool, ids_c, xs[0][0], layer, hk, hv, dk, dv,
                                                  K, 1, chunk, 7 * dk * dv * hv * chunk,
                                                  "GFLOP/s")
    pool.destroy()
    backend.close()
    return result


def cpu_baseline_gdn(pool, ids_c, qkv_dev, layer, hk, hv, dk, dv, K, nseq, rows, work, unit):
    """CPU oracle on `nseq` sequences x `rows` rows of the same layer shape, from
    the GPU pool's current state: 1 thread (the reference's row loop is
    serial) and all cores (min(cores, 16) threads, value heads split over
    them: the same arithmetic per head)."""
    from oracle import pyoracle as O

    rng = np.random.default_rng(7)
    C_ = 2 * hk * dk + hv * dv
    conv = layer["conv"].cpu().numpy()
    a_log = layer["a_log"].cpu().numpy()
    dt_bias = layer["dt_bias"].cpu().numpy()
    norm = layer["norm"].cpu().numpy()
    from concurrent.futures import ThreadPoolExecutor

    nthreads = min(os.cpu_count() or 1, 16)
    inputs = []
    for i in range(nseq):
        m, hst = pool.read(ids_c[i])
        inputs.append((m, hst, rng.standard_normal((rows, C_)).astype(np.float32),
                       rng.standard_normal((rows, hv * dv)).astype(np.float32),
                       rng.standard_normal((rows, hv)).astype(np.float32),
                       rng.standard_normal((rows, hv)).astype(np.float32)))

    def one(item, threads):
        m, hst, qkv, z, a, b = item
        O.gdn_rows(qkv, z, a, b, a_log, dt_bias, conv, K, norm, 1e-6, key_heads=hk,
                   value_heads=hv, key_dim=dk, value_dim=dv, history=hst.copy(),
                   state=m.copy(), threads=threads)

    t0 = time.perf_counter()
    for item in inputs:
        one(item, 1)
    t = time.perf_counter() - t0
    # all cores: the sequences side by side (ctypes releases the GIL), each
    # with its value heads split over its share of the threads
    per_seq = max(1, nthreads // nseq)
    with ThreadPoolExecutor(min(nseq, nthreads)) as ex:
        t0 = time.perf_counter()
        list(ex.map(lambda item: one(item, per_seq), inputs))
        tm = time.perf_counter() - t0
    scale = 1e9 if unit in ("GB/s", "GFLOP/s") else 1.0
    per_item = work / nseq if unit == "GB/s" else work
    return {"value": round(per_item * nseq / t / scale, 3), "unit": unit, "cores": 1,
            "kind": "port",
            "sample": f"{nseq} sequence(s) x {rows} row(s) of the same layer shape, f32 oracle",
            "ms": round(t * 1e3, 2),
            "all_cores": {"value": round(per_item * nseq / tm / scale, 3),
                          "cores": min(nthreads, nseq * per_seq), "ms": round(tm * 1e3, 2)}}


# Qwen3-8B decoder layer projections (out, in): q, k, v, o, gate, up, down
LINEAR_SHAPES = ((4096, 4096), (1024, 4096), (1024, 4096), (4096, 4096),
                 (12288, 4096), (12288, 4096), (4096, 12288))


def bench_linear(args, torch, pkg, steps, warmup, rows=16):
    """ABI v1 linear (the next component after the attention / GDN rows): the
    seven projections of one Qwen3-8B decoder layer (bf16 weights, 386 MB)
    for a decode batch of 16 rows, through the device-pointer entry
    (safetyraise_kernel_linear_device), inputs resident on the GPU.  One step =
    the seven calls.  HBM-bound: algorithmic bytes = the weights plus the f32
    inputs and outputs."""
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0006)
    weights, xs, ys = [], [], []
    for out_f, in_f in LINEAR_SHAPES:
        w = (torch.randn((out_f, in_f), generator=gen, device="cuda") * 0.02).bfloat16()
        bits = w.view(torch.int16).cpu().numpy().view(np.uint16)
        weights.append(backend.create_weight(bits, pkg.DTYPE_BF16))
        xs.append(torch.randn((rows, in_f), generator=gen, device="cuda"))
        ys.append(torch.empty((rows, out_f), device="cuda"))
        del w, bits
    fn = backend.lib.safetyraise_kernel_linear_device
    ctx = backend.context

    def run(which=range(len(LINEAR_SHAPES))):
        for i in which:
            out_f, in_f = LINEAR_SHAPES[i]
            st = fn(ctx, weights[i].handle, C.c_void_p(xs[i].data_ptr()), rows, in_f,
                    C.c_void_p(ys[i].data_ptr()), rows, out_f)
            if st != 0:
                backend.check(st, "linear_device")

    for _ in range(warmup):
        run()
    backend.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("linear timed")
    t0.record(stream)
    for _ in range(steps):
        run()
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    run()
    # kernel durations in a second pass over the same rotation of all seven
    # calls (386 MB of weights, more than the 256 MB Infinity Cache, so every
    # call streams its weight from HBM, as in the timed steps).  The roofline
    # kernel is the gate/up plan (12288 x 4096, the only calls with 3 tiles
    # per wave); timing the two big calls alone would leave 201 MB of weights
    # cached between calls and overstate the HBM rate.
    kernels = kernel_pass(backend, lambda: [run() for _ in range(steps)],
                          steps * len(LINEAR_SHAPES), "linear")
    per_call = [o * i * 2 + rows * (i + o) * 4 for o, i in LINEAR_SHAPES]
    per_step = sum(per_call)
    ms = t0.elapsed_time(t1) / steps
    value = per_step / (ms * 1e-3) / 1e9
    big_us = kernels["linear_kernel_t3"]["us"]
    achieved = per_call[4] / (big_us * 1e-6) / 1e9
    result = {
        "workload": f"Qwen3-8B decoder-layer projections (q/k/v/o/gate/up/down, bf16 weights, "
                    f"386 MB), {rows} rows, f32 in/out, device pointers",
        "value": round(value, 2), "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "dtype": "f32",
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("linear_qwen3_8b"),
            "kernel": "linear_kernel<3, true, 3, 8, 2, true> (the 12288 x 4096 gate/up calls: bf16 "
                      "weight, 3 output tiles per wave, 8 waves)",
            "launch_us_mean": round(float(big_us), 2),
            "bytes_per_launch": int(per_call[4]),
        },
        "kernels": kernels,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_linear(weights[0], xs[0], rows)
    for w in weights:
        w.destroy()
    backend.close()
    return result


def bench_linear_prefill(args, torch, pkg, steps, warmup, rows=2048):
    """ABI v1 linear at a prefill chunk's row count: the seven projections of
    one Qwen3-8B decoder layer (bf16 weights) for 2048 rows, through the
    device-pointer entry.  One step = the seven calls.  These calls take the
    tiled product (x split once into three bf16 parts, then 128 x 128 output
    tiles on v_mfma_f32_16x16x32_bf16).  `value` counts the f32 product's own
    FLOPs, 2 rows in out per call; the roofline counts the MFMA work, three
    bf16 passes per exact product, against the dense bf16 peak."""
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0007)
    weights, xs, ys = [], [], []
    for out_f, in_f in LINEAR_SHAPES:
        w = (torch.randn((out_f, in_f), generator=gen, device="cuda") * 0.02).bfloat16()
        bits = w.view(torch.int16).cpu().numpy().view(np.uint16)
        weights.append(backend.create_weight(bits, pkg.DTYPE_BF16))
        xs.append(torch.randn((rows, in_f), generator=gen, device="cuda"))
        ys.append(torch.empty((rows, out_f), device="cuda"))
        del w, bits
    fn = backend.lib.safetyraise_kernel_linear_device
    ctx = backend.context

    def run():
        for i, (out_f, in_f) in enumerate(LINEAR_SHAPES):
            st = fn(ctx, weights[i].handle, C.c_void_p(xs[i].data_ptr()), rows, in_f,
                    C.c_void_p(ys[i].data_ptr()), rows, out_f)
            if st != 0:
                backend.check(st, "linear_device")

    for _ in range(warmup):
        run()
    backend.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("linear-prefill timed")
    t0.record(stream)
    for _ in range(steps):
        run()
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    kernels = kernel_pass(backend, lambda: [run() for _ in range(steps)],
                          steps * len(LINEAR_SHAPES), "linear-prefill")
    ms = t0.elapsed_time(t1) / steps
    flops = [2 * rows * o * i for o, i in LINEAR_SHAPES]
    tflops = sum(flops) / (ms * 1e-3) / 1e12
    # the tiled products: linear_gemm_wide_kernel for calls with many
    # outputs, linear_gemm_kernel for the others; their mean launch over all
    # calls, weighted by the share of calls each takes
    tiled = [kernels[k] for k in ("linear_gemm_wide_kernel", "linear_gemm_kernel") if k in kernels]
    gemm_us = sum(k["per_call"] * k["us"] for k in tiled) / sum(k["per_call"] for k in tiled)
    # the roofline: the MFMA work of one call (3 passes) over the mean
    # tiled-kernel launch, the calls' FLOPs averaged the same way
    launch_flops = sum(flops) / len(flops)
    mfma_tf = 3 * launch_flops / (gemm_us * 1e-6) / 1e12
    result = {
        "workload": f"Qwen3-8B decoder-layer projections (q/k/v/o/gate/up/down, bf16 weights), "
                    f"{rows} rows, f32 in/out, device pointers",
        "value": round(tflops, 2), "unit": "TFLOP/s",
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "dtype": "f32 products, exact (x split in three bf16 parts on v_mfma_f32_16x16x32_bf16)",
        "roofline": {
            "bound": "mfma", "achieved": round(mfma_tf, 2), "peak": MFMA_BF16_PEAK_TFS,
            "unit": "TFLOP/s", "frac": round(mfma_tf / MFMA_BF16_PEAK_TFS, 4),
            "traffic": None,
            "kernel": "linear_gemm_wide_kernel + linear_gemm_kernel (all seven calls; achieved = "
                      "3 bf16 MFMA passes per exact product, the calls' mean FLOPs over the mean "
                      "launch)",
            "launch_us_mean": round(float(gemm_us), 2),
            "flops_per_launch": int(3 * launch_flops),
            "exact_product_tflops_per_launch": round(launch_flops / (gemm_us * 1e-6) / 1e12, 2),
            "fp32_matrix_peak": MFMA_F32_PEAK_TFS,
            "mfma_util": mfma_from_profiles(
                "linear_prefill_qwen3_8b", [k for k in ("linear_gemm_wide_kernel",
                                                        "linear_gemm_kernel") if k in kernels],
                {k: float(kernels[k]["us"]) for k in ("linear_gemm_wide_kernel",
                                                      "linear_gemm_kernel") if k in kernels}),
        },
        "kernels": kernels,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_linear_prefill(xs[0])
    for w in weights:
        w.destroy()
    backend.close()
    return result


def cpu_baseline_linear(weight, x_dev, rows):
    """The oracle's linear (the reference CPU plugin's loop, 1 thread) on the q
    projection (4096 x 4096 bf16) for 4 of the rows, as weight GB/s."""
    from oracle import pyoracle as O

    out_f, in_f = LINEAR_SHAPES[0]
    rng = np.random.default_rng(11)
    bits = (rng.integers(0, 1 << 16, size=(out_f, in_f), dtype=np.uint32) & 0x3fff).astype(np.uint16)
    x = x_dev[:4].cpu().numpy()
    t0 = time.perf_counter()
    O.linear(x, bits, 3)
    t = time.perf_counter() - t0
    call_bytes = out_f * in_f * 2  # the weight stream the GPU figure counts, per call
    return {"value": round(call_bytes / (t / 4 * rows) / 1e9, 3), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": "q projection (4096 x 4096 bf16) for 4 rows, f32 oracle (the reference "
                      "plugin's loop), scaled to the 16-row call",
            "ms": round(t * 1e3, 2)}


def cpu_baseline_linear_prefill(x_dev):
    """The oracle's linear (the reference CPU plugin's loop) on the q
    projection (4096 x 4096 bf16): 4 rows on 1 thread, and 4 rows per thread on
    min(cores, 16) threads at once (ctypes releases the GIL), as GFLOP/s of the
    f32 product (2 rows x out x in per call, the GPU figure's count)."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import pyoracle as O

    out_f, in_f = LINEAR_SHAPES[0]
    rng = np.random.default_rng(12)
    bits = (rng.integers(0, 1 << 16, size=(out_f, in_f), dtype=np.uint32) & 0x3fff).astype(np.uint16)
    nthreads = min(os.cpu_count() or 1, 16)
    x = x_dev[:4 * nthreads].cpu().numpy()
    t0 = time.perf_counter()
    O.linear(x[:4], bits, 3)
    t1 = time.perf_counter() - t0
    with ThreadPoolExecutor(nthreads) as ex:
        t0 = time.perf_counter()
        list(ex.map(lambda i: O.linear(x[4 * i:4 * i + 4], bits, 3), range(nthreads)))
        tm = time.perf_counter() - t0
    flops = 2 * 4 * out_f * in_f
    return {"value": round(flops / t1 / 1e9, 3), "unit": "GFLOP/s", "cores": 1, "kind": "port",
            "sample": "q projection (4096 x 4096 bf16) for 4 rows per thread, f32 oracle (the "
                      "reference plugin's loop)",
            "ms": round(t1 * 1e3, 2),
            "all_cores": {"value": round(nthreads * flops / tm / 1e9, 3), "cores": nthreads,
                          "ms": round(tm * 1e3, 2)}}


# verify shapes: (heads, kv heads, head_dim, rotary_dim, theta, gated)
VERIFY_SHAPES = {
    # BASELINE config 5
    "qwen3-32b": (64, 8, 128, 128, 1e6, False),
    # Qwen3.5 full attention (the model the reference's MTP runs,
    # src/model/mtp.rs:110-112): q/gate interleaved, partial rotary 64, theta 1e7
    "qwen3.5": (16, 2, 256, 64, 1e7, True),
}


def bench_verify(args, torch, pkg, steps, warmup, rows=5, shape="qwen3-32b"):
    """long-context MTP speculative-verify attention, Qwen3-32B
    shape: 64 Q / 8 KV heads, head_dim 128, 1 + 4 draft rows per sequence (row j
    sees 131072 + j + 1 keys), batch 4, context 131072, paged bf16 KV in 16-token
    pages whose ids are a seeded random permutation of the pool (the pool's
    page_order_seed), so no two consecutive pages of a sequence are adjacent
    except by chance.  One step = one verify call; the drafts are truncated away
    afterwards (the next step verifies at the same context).  Inputs ~N(0,1) are
    taken as normalised (no QK-norm); RoPE is applied as part of the fused path.
    shape "qwen3.5": the same workload at the Qwen3.5 full-attention geometry
    (16 Q / 2 KV heads, head_dim 256, gated); rows 9 = 1 + 8 drafts, the
    engine's cap (src/engine/speculative.rs:12)."""
    heads, kvh, dim, rotary, theta, gated = VERIFY_SHAPES[shape]
    nseq, ctx_len, page = 4, 131072, 16
    backend = pkg.NativeBackend.load()
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    backend.set_stream(stream.cuda_stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5A5A0005)
    max_tokens = ctx_len + rows + 16
    pool = pkg.KvCache(backend, kvh, dim, page, nseq * (max_tokens // page + 2) + 8, max_tokens,
                       nseq, page_order_seed=0x5A5A0005)
    ids = [pool.open() for _ in range(nseq)]
    kfull = torch.randn((ctx_len, kvh * dim), generator=gen, device="cuda", dtype=torch.bfloat16)
    vfull = torch.randn((ctx_len, kvh * dim), generator=gen, device="cuda", dtype=torch.bfloat16)
    for s_ in ids:
        pool.append(s_, kfull, vfull, flags=pkg.ASYNC)
    backend.synchronize()
    del kfull, vfull
    qw = heads * dim * (2 if gated else 1)
    q = torch.randn((nseq * rows, qw), generator=gen, device="cuda")
    k = torch.randn((nseq * rows, kvh * dim), generator=gen, device="cuda")
    v = torch.randn((nseq * rows, kvh * dim), generator=gen, device="cuda")
    out = torch.empty((nseq * rows, heads * dim), device="cuda")
    pos = torch.tensor([[ctx_len + r] * 3 for _ in range(nseq) for r in range(rows)],
                       dtype=torch.int32, device="cuda")
    P = pkg.plugin
    a = P.AttentionArgs()
    a.struct_size = C.sizeof(P.AttentionArgs)
    a.flags = P.DEVICE_POINTERS | P.ASYNC | P.MROPE_INTERLEAVED | (P.GATED if gated else 0)
    a.heads, a.kv_heads, a.head_dim, a.rotary_dim = heads, kvh, dim, rotary
    a.eps, a.rope_theta = 1e-6, theta
    a.num_seqs = nseq
    a.seq_ids = (C.c_uint32 * nseq)(*ids)
    a.seq_rows = (C.c_uint32 * nseq)(*([rows] * nseq))
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    a.positions = pos.data_ptr()
    a.out = out.data_ptr()
    a.kv = pool.handle
    fwd = backend.lib.safetyraise_kernel_attention_forward
    ctx = backend.context

    def run():
        st = fwd(ctx, C.byref(a))
        if st != 0:
            backend.check(st, "attention_forward")
        for s_ in ids:
            pool.truncate(s_, ctx_len)  # host bookkeeping only

    # each call streams 2.1 GB from HBM: under this load the GPU's clocks
    # settle within the first ~3 ms (about ten calls, each call about 15 %
    # slower than the first ones), so the timed steps and the timing pass
    # both start after at least that much
    warmup = max(warmup, 10)
    for _ in range(warmup):
        run()
    backend.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    region_begin("verify timed")
    t0.record(stream)
    for s_ in range(steps):
        run()
    t1.record(stream)
    torch.cuda.synchronize()
    region_end()
    backend.synchronize()
    ms = t0.elapsed_time(t1) / steps
    # kernel durations in a second pass (outside the timed region), after two
    # untimed calls that bring the GPU back from idle
    run()
    run()

    def second_pass():
        for _ in range(steps):
            run()

    kernels = kernel_pass(backend, second_pass, steps, "verify")
    call_us = kernels["attn_verify_kernel"]["us"]
    keys = sum(ctx_len + j + 1 for j in range(rows))  # per sequence, summed over rows
    nbytes = nseq * (ctx_len + rows) * kvh * dim * 2 * 2
    flops = nseq * heads * 4 * dim * keys
    gbs = nbytes / (ms * 1e-3) / 1e9
    achieved = nbytes / (call_us * 1e-6) / 1e9
    workload = ("qwen3-32b MTP verify attention (BASELINE config 5): 64 Q / 8 KV heads, "
                "d 128, 1 + 4 rows, batch 4, context 131072, 16-token pages in a random "
                "permutation of the pool") if shape == "qwen3-32b" else (
        f"{shape} MTP verify attention: {heads} Q / {kvh} KV heads, d {dim}, gated, rotary "
        f"{rotary}, 1 + {rows - 1} rows ({-(-rows // (64 // (heads // kvh)))} row slice(s) of "
        f"at most 64 query vectors), batch 4, context 131072, 16-token pages in a random "
        f"permutation of the pool")
    result = {
        "workload": workload,
        "value": round(gbs, 2), "unit": "GB/s",
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "dtype": "fp16 MFMA operands over the bf16 cache, f32 accumulate and softmax",
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (traffic_from_profiles("attn_verify_qwen3_32b")
                        if shape == "qwen3-32b" else None),
            "kernel": f"attn_verify_kernel<{dim}>",
            "launch_us_mean": round(float(call_us), 2),
            "bytes_per_launch": int(nbytes),
        },
        "kernels": kernels,
    }
    if not args.no_cpu and shape == "qwen3-32b":
        result["cpu_baseline"] = cpu_baseline_verify(pool, ids[0], q, k, v, pos, heads, kvh, dim,
                                                     rows, ctx_len)
    pool.destroy()
    backend.close()
    return result


def cpu_baseline_verify(pool, seq, q, k, v, pos, heads, kvh, dim, rows, ctx_len,
                        sample=16384):
    """CPU oracle on a bounded sample: the 5 verify rows of sequence 0 over the first
    `sample` cached tokens (read back from the GPU cache)."""
    from oracle import pyoracle as O

    keys, vals = pool.read(seq, 0, sample)
    cache = O.KvCache(kvh * dim, sample + rows, 64, bf16=True)
    cache.append_many(keys, vals)
    del keys, vals
    qn, kn, vn = q[:rows].cpu().numpy(), k[:rows].cpu().numpy(), v[:rows].cpu().numpy()
    pn = pos[:rows].cpu().numpy().astype(np.int64) - ctx_len + sample
    nthreads = min(os.cpu_count() or 1, 16)
    res = {}
    for threads in (1, nthreads):
        c = cache.clone()
        t = time.perf_counter()
        O.attention_rows(qn, kn, vn, pn, c, heads=heads, kv_heads=kvh, dim=dim, rotary_dim=dim,
                         theta=1e6, eps=1e-6, threads=threads)
        res[threads] = time.perf_counter() - t
    nbytes = sum(sample + j + 1 for j in range(rows)) * kvh * dim * 2 * 2
    return {"value": round(nbytes / res[1] / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"sequence 0, {rows} verify rows over the first {sample} cached tokens "
                      f"(bytes counted per row, as bf16)",
            "ms": round(res[1] * 1e3, 1),
            "all_cores": {"value": round(nbytes / res[nthreads] / 1e9, 3), "cores": nthreads,
                          "ms": round(res[nthreads] * 1e3, 1)}}


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
            result["verify"] = bench_verify(args, torch, pkg, 30, 10)
            result["verify"]["qwen3.5_d256"] = {
                f"rows_{r}": bench_verify(args, torch, pkg, 30, 10, rows=r, shape="qwen3.5")
                for r in (5, 9)}
            result["gdn_decode"] = bench_gdn_decode(args, torch, pkg, 20, 3)
            result["gdn_prefill"] = bench_gdn_prefill(args, torch, pkg, 10, 2)
            result["linear"] = bench_linear(args, torch, pkg, 50, 5)
            result["linear"]["prefill_rows"] = bench_linear_prefill(args, torch, pkg, 3, 1)
    elif args.workload in ("verify", "verify-qwen3.5"):
        shape = "qwen3-32b" if args.workload == "verify" else "qwen3.5"
        result = bench_verify(args, torch, pkg, args.steps, args.warmup, rows=args.rows,
                              shape=shape)
        result = {"metric": "MTP verify attention GB/s", "n_gpus": 1, "higher_is_better": True,
                  "scaling": "weak", "vs_baseline": None, "data": "synthetic",
                  "config": {"workload": result.pop("workload")}, **result}
    elif args.workload in ("gdn-decode", "gdn-prefill"):
        fn = bench_gdn_decode if args.workload == "gdn-decode" else bench_gdn_prefill
        result = fn(args, torch, pkg, args.steps, args.warmup)
        result = {"metric": "GDN " + args.workload[4:] + " " + result["unit"], "n_gpus": 1,
                  "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
                  "data": "synthetic", "config": {"workload": result.pop("workload")}, **result}
    elif args.workload == "linear":
        result = bench_linear(args, torch, pkg, args.steps, args.warmup)
        result = {"metric": "linear weight-stream GB/s", "n_gpus": 1, "higher_is_better": True,
                  "scaling": "weak", "vs_baseline": None, "data": "synthetic",
                  "config": {"workload": result.pop("workload")}, **result}
    elif args.workload == "linear-prefill":
        result = bench_linear_prefill(args, torch, pkg, args.steps, args.warmup)
        result = {"metric": "linear TFLOP/s at 2048 rows", "n_gpus": 1, "higher_is_better": True,
                  "scaling": "weak", "vs_baseline": None, "data": "synthetic",
                  "config": {"workload": result.pop("workload")}, **result}
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
