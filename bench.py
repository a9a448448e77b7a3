#!/usr/bin/env python3
"""Benchmark of the paged FP8-KV decode attention step on one MI355X.

Workload (one "step" = one decode-attention call for one layer): batch 256,
32 query / 8 KV heads, head_dim 128, block_size 256, context lengths
floor(exp(U(ln 512, ln 8192))), fragmented block tables over a 4096-block
pool per layer, FP8 e4m3fn KV with a per-tensor scale, bf16 queries.  Steps
rotate over --layers distinct layer pools (default 8, i.e. 16 GiB of FP8 KV)
so the working set is far larger than the 256 MiB Infinity Cache.

Prints ONE JSON line.  `value` is the algorithmic HBM throughput of the step
(every visible K/V byte once + q + out + used block-table entries +
context_lens, divided by the step time measured with HIP events on the
launch stream).  `roofline` compares that with the 8 TB/s HBM peak,
`cpu_baseline` times the reference's PyTorch decode path
(decode_torch_optimized semantics, restated in oracle/) on a bounded sample
of the same workload on the host CPU.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--kv fp8|bf16]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO / "mini-kvllm_amd"), str(REPO)):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "paged FP8-KV decode attn HBM GB/s (% of peak) at bs=256; e2e decode tok/s"
PEAK_HBM_GBPS = 8000.0
HEAD_DIM = 128


KV_DESC = {"fp8": "per-tensor e4m3fn", "bf16": "bf16",
           "fp8_token": "e4m3fn codes, fp32 scale per token and kv head",
           "int8_token": "int8 codes, fp32 scale per token and kv head"}


ROUTE_NAMES = {0: "stream-K", 1: "split-K", 2: "workgroup"}
DECODE_CONFIGS = ("fp32_decode_b4", "fp8_decode_b32", "fp8_decode_b60_engine_shape", "bf16_decode_b256",
                  "fp8_decode_b256_d64")
EXTRAS = ("configs", "e2e", "append", "prefill", "latency", "producer", "mixed", "copy", "gather")


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kv", choices=["fp8", "bf16", "fp8_token", "int8_token"], default="fp8",
                    help="KV format: per-tensor FP8 (the headline), bf16, or per-token-head "
                         "FP8 / INT8 (kv_cache_dtype fp8_per_token_head / int8_per_token_head)")
    ap.add_argument("--layers", type=int, default=8, help="distinct layer pools rotated per step")
    ap.add_argument("--split-tokens", type=int, default=0)
    ap.add_argument("--batch", type=int, default=256)
    ap.add_argument("--num-heads", type=int, default=32)
    ap.add_argument("--num-kv-heads", type=int, default=8)
    ap.add_argument("--cpu-seqs", type=int, default=64,
                    help="sequences in the CPU-baseline sample (0 = skip the CPU baseline)")
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--extra", default="all",
                    help="secondary measurements to run: 'all' or a comma list of "
                         "configs, e2e, append, prefill, latency, producer, mixed, copy, gather")
    ap.add_argument("--decode-configs", default="all",
                    help="configs extra: 'all' or a comma list of " + ", ".join(DECODE_CONFIGS))
    ap.add_argument("--skip-headline", action="store_true",
                    help="run only the secondary measurements (for profiling them); the printed "
                         "line then has no headline value")
    ap.add_argument("--e2e-no-baselines", action="store_true",
                    help="e2e extra: time only the mkv engine with captured decode (for profiling "
                         "it), not the eager and PyTorch-attention engines beside it")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run a plain device copy of this many MiB (5 times) and exit; "
                         "its rocprofv3 FETCH_SIZE/WRITE_SIZE calibrate the PMC byte counts")
    args = ap.parse_args(argv)
    if args.no_extra:
        args.extra_set = set()
    elif args.extra == "all":
        args.extra_set = set(EXTRAS)
    else:
        args.extra_set = {x.strip() for x in args.extra.split(",") if x.strip()}
        unknown = args.extra_set - set(EXTRAS)
        if unknown:
            ap.error(f"--extra: unknown measurement(s) {sorted(unknown)}; choose from {list(EXTRAS)}")
    if args.decode_configs == "all":
        args.decode_config_set = set(DECODE_CONFIGS)
    else:
        args.decode_config_set = {x.strip() for x in args.decode_configs.split(",") if x.strip()}
        unknown = args.decode_config_set - set(DECODE_CONFIGS)
        if unknown:
            ap.error(f"--decode-configs: unknown {sorted(unknown)}; choose from {list(DECODE_CONFIGS)}")
    return args


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def settle(fn, stream, first: int = 0, chunk: int = 16, tol: float = 0.005, window: int = 4,
           max_steps: int = 960) -> dict:
    """Run fn(i) in chunks of `chunk` calls until the GPU's step time is
    steady, i.e. the last `window` chunk means agree within `tol`, or
    `max_steps` calls have run.  On the MI355X a memory-bound step that starts
    after an idle GPU runs fast for about a millisecond, slows down by up to
    30% and then recovers over 50-100 further steps (the power controller
    finding its operating point), and keeps gaining ~1% over the next few
    hundred; timing a short window inside that transient measures the
    controller, not the kernel (three chunks within 1.5% stopped ~1.5% above
    the time the step keeps over a 200-step run).  Returns the calls made and
    the chunk means (µs)."""
    import torch

    means = []
    i = first
    while i - first < max_steps:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(chunk):
            fn(i)
            i += 1
        b.record(stream)
        b.synchronize()
        means.append(a.elapsed_time(b) * 1e3 / chunk)
        if len(means) >= window and max(means[-window:]) <= min(means[-window:]) * (1 + tol):
            break
    return {"steps": i - first, "chunk_means_us": [round(m, 1) for m in means]}


def time_launches(fn, steps: int, warmup: int, stream, settle_first: bool = False):
    """Average ms per call of fn(i), timed with events on `stream`.  With
    settle_first, the warm-up is followed by settle() and the result is
    (ms, settle record)."""
    import torch

    for i in range(warmup):
        fn(i)
    rec = settle(fn, stream, first=warmup) if settle_first else None
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return (ms, rec) if settle_first else ms


def step_percentiles(fn, steps: int, stream) -> dict:
    """p10/p50/p90 of single-step times (µs), one event pair per step."""
    import torch

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        fn(i)
        b.record(stream)
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    pick = lambda f: round(t[min(len(t) - 1, int(f * len(t)))], 2)
    return {"p10_us": pick(0.1), "p50_us": pick(0.5), "p90_us": pick(0.9), "steps": steps}


def box_copy_gbps(dev, stream, mib: int = 2048) -> float:
    """Read+write bandwidth of a plain device copy on this GPU (a measured
    on-box reference, next to the 8 TB/s datasheet peak)."""
    import torch

    src = torch.ones(mib << 20, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    ms = time_launches(lambda i: dst.copy_(src), 10, 2, stream)
    del src, dst
    return 2 * (mib << 20) / (ms * 1e-3) / 1e9


def box_read_gbps(dev, stream, mib: int = 2048) -> dict:
    """Read rate of a plain streaming kernel on this GPU (mkv_stream_read_probe:
    non-temporal 16-byte loads, the decode's KV load type, over a 2 GiB buffer
    read once per launch, no writes but one checksum dword per wave); the best
    of a few grid sizes (many waves with a few loads each read fastest).  The
    measured ceiling for the decode's HBM reads."""
    import torch

    import mkv

    nbytes = mib << 20
    buf = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    best = None
    for grid in (32768, 65536, 131072, 262144):
        sink = torch.empty(int(mkv._lib.query("mkv_stream_read_probe_sink_words", grid)),
                           dtype=torch.int32, device=dev)
        ms = time_launches(lambda i: mkv._lib.call("mkv_stream_read_probe", buf.data_ptr(), nbytes,
                                                    sink.data_ptr(), grid, stream.cuda_stream),
                           10, 2, stream)
        gbps = nbytes / (ms * 1e-3) / 1e9
        if best is None or gbps > best["GBps"]:
            best = {"GBps": round(gbps, 1), "grid": grid, "bytes": nbytes, "us": round(ms * 1e3, 1)}
        del sink
    del buf
    return best


def prefill_extra(dev, stream, cpu: bool = True) -> dict:
    """Chunked prefill over the paged cache: the 8 prefill sequences of the
    mixed-batch workload (prior context U[0, 4096], 512-row chunks), 32 q / 8
    kv heads, bf16 q; bf16, per-tensor FP8, per-token-head FP8 and INT8 KV.  FLOPs are algorithmic (4*D per
    visible key per row and head); peak is dense fp16/bf16 MFMA."""
    import torch

    from mkv import attention as A
    from mkv import workloads as W

    pm = W.prefill_mixed(seed=4)
    sel = [i for i, d in enumerate(pm["is_decode"]) if not d]
    cu = pm["cu_seqlens_q"]
    rows = torch.cat([torch.arange(int(cu[i]), int(cu[i + 1])) for i in sel])
    ctx = pm["context_lens"][sel]
    bt = pm["block_tables"][sel]
    pos = pm["positions"][rows]
    cu_p = torch.zeros(len(sel) + 1, dtype=torch.int32)
    cu_p[1:] = torch.cumsum(torch.tensor([pm["query_lens"][i] for i in sel]), 0)
    flops = W.alg_flops_prefill(ctx, cu_p, pos, 32)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(rows.numel(), 32, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    dev_meta = (bt.to(dev), ctx.to(dev), cu_p.to(dev), pos.to(dev))
    out = {"workload": (f"{len(sel)} sequences x 512 query rows, prior context "
                        f"{[int(c) - 512 for c in ctx]}, {flops / 1e9:.1f} GFLOP")}
    for name, dt in (("bf16", torch.bfloat16), ("fp8", torch.float8_e4m3fn),
                     ("fp8_token", torch.float8_e4m3fn), ("int8_token", torch.int8)):
        kc = torch.empty(pm["num_blocks"], pm["block_size"], 8, HEAD_DIM, dtype=dt, device=dev)
        vc = torch.empty_like(kc)
        kw = {}
        if name.endswith("_token"):
            mode = "fp8_per_token_head" if name == "fp8_token" else "int8_per_token_head"
            kst = torch.empty(pm["num_blocks"], pm["block_size"], 8, dtype=torch.float32, device=dev)
            vst = torch.empty_like(kst)
            W.fill_pools_per_token_head_on_device(kc, vc, kst, vst, 400, mode)
            kw = dict(k_scale=kst, v_scale=vst, kv_cache_dtype=mode)
        else:
            ks = W.fill_pool_on_device(kc, 400)
            vs = W.fill_pool_on_device(vc, 401)
            if name == "fp8":
                kw = dict(k_scale=torch.tensor([ks], device=dev), v_scale=torch.tensor([vs], device=dev),
                          kv_cache_dtype="fp8_per_tensor")
        args = (q, kc, vc, *dev_meta[:2], dev_meta[2], dev_meta[3], 1.0 / math.sqrt(HEAD_DIM), 32, 8,
                HEAD_DIM, pm["block_size"])
        # (settled first, as the headline step: a launch series that starts
        # from an idle GPU runs through the power controller's transient)
        ms, rec = time_launches(lambda i: A.paged_attention_prefill_triton(*args, **kw), 20, 3, stream,
                                settle_first=True)
        tf = flops / (ms * 1e-3) / 1e12
        out[f"{name}_kv"] = {"us": round(ms * 1e3, 1), "TFLOPs": round(tf, 1),
                             "frac_of_2500_TFLOPs": round(tf / 2500.0, 4), "settle_steps": rec["steps"]}
        if name != "bf16":
            # 1-byte caches: also against the 5.0 PF dense FP8 (and INT8) MFMA
            # peak; the kernel converts the codes exactly to 16-bit operands
            # and runs the fp16 / bf16 MFMA, whose peak is the 2.5 PF above
            out[f"{name}_kv"]["frac_of_5000_TFLOPs_fp8_peak"] = round(tf / 5000.0, 4)
        if name == "bf16" and cpu:
            out["cpu_baseline"] = cpu_prefill_baseline(q, kc, vc, bt, ctx, cu_p, pos, pm["block_size"])
        del kc, vc
    out["full_prefill"] = full_prefill_extra(dev, stream, cpu)
    return out


def full_prefill_extra(dev, stream, cpu: bool = True) -> dict:
    """Causal varlen prefill over fresh contiguous bf16 q/k/v
    (mkv.flash_attention_prefill, the reference's flash_attention_prefill):
    the end-to-end workload's prompts (60, lengths U[32, 512], 16 q / 8 kv
    heads) and 8 prompts of 4096 tokens (32 q / 8 kv heads).  FLOPs are
    algorithmic (4*D per visible key per row and head)."""
    import torch

    from mkv import attention as A

    res = {}
    for name, lens, hq in (("prompts60_16q", None, 16), ("8x4096_32q", [4096] * 8, 32)):
        g = torch.Generator().manual_seed(5)
        if lens is None:
            lens = torch.randint(32, 513, (60,), generator=g).tolist()
        cu = torch.zeros(len(lens) + 1, dtype=torch.int32)
        cu[1:] = torch.cumsum(torch.tensor(lens), 0)
        T = int(cu[-1])
        q = torch.randn(T, hq, HEAD_DIM, generator=g).to(torch.bfloat16)
        k = torch.randn(T, 8, HEAD_DIM, generator=g).to(torch.bfloat16)
        v = torch.randn(T, 8, HEAD_DIM, generator=g).to(torch.bfloat16)
        qd, kd, vd, cud = q.to(dev), k.to(dev), v.to(dev), cu.to(dev)
        flops = sum(n * (n + 1) // 2 for n in lens) * hq * 4 * HEAD_DIM
        sm = 1.0 / math.sqrt(HEAD_DIM)
        ms, rec = time_launches(lambda i: A.flash_attention_prefill(qd, kd, vd, cud, sm, hq, 8, HEAD_DIM),
                                20, 3, stream, settle_first=True)
        tf = flops / (ms * 1e-3) / 1e12
        res[name] = {"tokens": T, "GFLOP": round(flops / 1e9, 1), "us": round(ms * 1e3, 1),
                     "TFLOPs": round(tf, 1), "frac_of_2500_TFLOPs": round(tf / 2500.0, 4),
                     "settle_steps": rec["steps"]}
        if cpu and name == "prompts60_16q":
            # the reference's torch form (pytorch_standard_attention semantics, fp32) on 8 prompts
            from oracle import reference as R
            n = 8
            cu8 = cu[: n + 1]
            t8 = int(cu8[-1])
            t = _median_time(lambda: R.flash_prefill_ref(q[:t8], k[:t8], v[:t8], cu8, sm, hq, 8,
                                                           compute_dtype=torch.float32))
            f8 = sum(x * (x + 1) // 2 for x in lens[:n]) * hq * 4 * HEAD_DIM
            res[name]["cpu_baseline"] = {"value": round(f8 / t / 1e9, 2), "unit": "GFLOP/s",
                                         "cores": _cpu_threads(), "kind": "port",
                                         "sample": f"first {n} prompts ({t8} tokens), median of 3: {t * 1e3:.1f} ms"}
    return res


def _cpu_threads() -> int:
    import torch

    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    torch.set_num_threads(threads)
    return threads


def _median_time(fn, reps: int = 3) -> float:
    fn()  # warm-up
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_prefill_baseline(q, kc, vc, bt, ctx, cu_p, pos, bs) -> dict:
    """The reference's CPU prefill semantics (oracle paged_prefill_ref in
    fp32: per-sequence gather, causal masked matmul / softmax, the paged
    prefix included) on the first sequence of the chunked-prefill workload,
    all 32 query heads."""
    import torch

    from mkv import workloads as W
    from oracle import reference as R

    threads = _cpu_threads()
    n = int(cu_p[1])
    blocks = bt[0][bt[0] >= 0].to(torch.int64)
    idx = blocks.to(kc.device)
    kh, vh = kc.index_select(0, idx).cpu(), vc.index_select(0, idx).cpu()
    bt_h = torch.arange(blocks.numel(), dtype=torch.int32).view(1, -1)
    qh = q[:n].cpu()
    cu_h = torch.tensor([0, n], dtype=torch.int32)
    ctx_h, pos_h = ctx[:1], pos[:n]
    sm = 1.0 / math.sqrt(HEAD_DIM)
    t = _median_time(lambda: R.paged_prefill_ref(qh, kh, vh, bt_h, ctx_h, cu_h, pos_h, sm, 32, 8,
                                                  compute_dtype=torch.float32))
    fl = W.alg_flops_prefill(ctx_h, cu_h, pos_h, 32)
    return {"value": round(fl / t / 1e9, 2), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"sequence 0: {n} rows after a prior of {int(ctx[0]) - n} tokens, 32 q / 8 kv "
                       f"heads, bf16 KV, paged_prefill_ref in fp32, median of 3: {t:.3f} s "
                       f"({fl / 1e9:.1f} GFLOP)")}


def cpu_append_baseline(key, value, slots, ks: float, vs: float) -> dict:
    """The reference's FP8 append semantics on the host cores (oracle
    store_kvcache_fp8_ref: fp32 divide, clamp, e4m3fn cast, scatter into the
    pool) for the 4096-token append workload."""
    import torch

    from mkv import workloads as W
    from oracle import reference as R

    threads = _cpu_threads()
    kp = torch.zeros(1024, 256, 8, HEAD_DIM, dtype=torch.float8_e4m3fn)
    vp = torch.zeros_like(kp)
    kst, vst = torch.tensor([ks]), torch.tensor([vs])
    t = _median_time(lambda: R.store_kvcache_fp8_ref(key, value, kp, vp, kst, vst, slots))
    ab = W.alg_bytes_append(slots, 8, 2, 1)
    return {"value": round(ab / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole workload ({slots.numel()} tokens), median of 3: {t * 1e3:.1f} ms"}


def gather_extra(kc, meta, dev, stream, cpu: bool = True) -> dict:
    """Block-table gather (mkv.gather_kv; the reference's torch form is
    benchmark_decoding.py:166-178) of one layer's K pool of the decode
    workload into a zero-padded (batch, max_len, Hkv, D) tensor, max_len =
    the longest context rounded up to a block.  Algorithmic bytes: the
    visible rows read once, every output row written once, the table
    entries read once."""
    from mkv import attention as A

    bs = meta["block_size"]
    lens = meta["context_lens"]
    max_len = (int(lens.max()) + bs - 1) // bs * bs
    row = kc.shape[2] * kc.shape[3] * kc.element_size()
    nblk = (lens + bs - 1) // bs
    alg = int(lens.sum()) * row + lens.numel() * max_len * row + int(nblk.sum()) * 4
    bt, ctx = meta["block_tables"].to(dev), meta["context_lens"].to(dev)
    ms = time_launches(lambda i: A.gather_kv(kc, bt, ctx, max_len), 20, 3, stream)
    res = {"workload": f"{lens.numel()} sequences, context sum {int(lens.sum())}, max_len {max_len}, "
                       f"{row}-byte rows ({kc.dtype}), block {bs}",
           "us": round(ms * 1e3, 1), "GBps": round(alg / ms / 1e6, 1),
           "frac_of_8000_GBps": round(alg / ms / 1e6 / 8000.0, 4)}
    if cpu:
        # the reference's torch form on the host cores, per sequence: the
        # blocks' rows by index, cut to the context, zero-padded to max_len
        import torch
        n = 32
        pool = kc.view(torch.uint8).cpu()
        tbl, cl = meta["block_tables"][:n], lens[:n]
        threads = _cpu_threads()

        def host_gather():
            outh = torch.zeros(n, max_len, *pool.shape[2:], dtype=pool.dtype)
            for b in range(n):
                L = int(cl[b])
                nb = (L + bs - 1) // bs
                idx = tbl[b, :nb].to(torch.int64)
                outh[b, :L] = pool[idx].reshape(nb * bs, *pool.shape[2:])[:L]
            return outh
        t = _median_time(host_gather)
        cab = int(cl.sum()) * row + n * max_len * row + int(nblk[:n].sum()) * 4
        res["cpu_baseline"] = {"value": round(cab / t / 1e9, 3), "unit": "GB/s", "cores": threads,
                               "kind": "port", "sample": f"first {n} sequences, median of 3: {t * 1e3:.1f} ms"}
    return res


def cpu_copy_append_baseline(key, value, slots) -> dict:
    """The reference's copy append semantics on the host cores (oracle
    store_kvcache_ref: index-assign of every valid row into the pool) for
    the 4096-token append workload."""
    import torch

    from mkv import workloads as W
    from oracle import reference as R

    threads = _cpu_threads()
    kp = torch.zeros(1024, 256, 8, HEAD_DIM, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    t = _median_time(lambda: R.store_kvcache_ref(key, value, kp, vp, slots))
    ab = W.alg_bytes_append(slots, 8, 2, 2)
    return {"value": round(ab / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"the whole workload ({slots.numel()} tokens), median of 3: {t * 1e3:.1f} ms"}


def cpu_mixed_baseline(q, kc, vc, m, n_decode: int = 16) -> dict:
    """The reference's CPU path for the mixed batch on a bounded sample: its
    first prefill chunk (paged_prefill_ref in fp32, the paged prefix
    included) and its first n_decode decode rows (decode_torch_optimized
    semantics, micro-batch 16), all 32 query heads; GFLOP/s of the sample's
    algorithmic FLOPs."""
    import torch

    from mkv import workloads as W
    from oracle import reference as R

    threads = _cpu_threads()
    cu = m["cu_seqlens_q"].tolist()
    pre = [i for i, d in enumerate(m["is_decode"]) if not d][0]
    dec = [i for i, d in enumerate(m["is_decode"]) if d][:n_decode]
    seqs = [pre] + dec
    bt = m["block_tables"][seqs]
    used = sorted({int(x) for x in bt.flatten() if x >= 0})
    remap = {p: i for i, p in enumerate(used)}
    bt_c = bt.clone()
    bt_c.apply_(lambda x: remap[x] if x >= 0 else -1)
    idx = torch.tensor(used, device=kc.device)
    kh, vh = kc.index_select(0, idx).cpu(), vc.index_select(0, idx).cpu()
    ctx = m["context_lens"][seqs]
    a, b = cu[pre], cu[pre + 1]
    qp = q[a:b].float().cpu()
    cu_p = torch.tensor([0, b - a], dtype=torch.int32)
    pos_p = m["positions"][a:b]
    qd = q[torch.tensor([cu[i] for i in dec], device=q.device)].float().cpu()
    sm = 1.0 / math.sqrt(HEAD_DIM)

    def run():
        R.paged_prefill_ref(qp, kh, vh, bt_c[:1], ctx[:1], cu_p, pos_p, sm, 32, 8,
                            compute_dtype=torch.float32)
        R.decode_torch_optimized_ref(qd, kh, vh, bt_c[1:], ctx[1:], sm, 32, 8, HEAD_DIM,
                                     m["block_size"], micro_batch=16)

    t = _median_time(run)
    fl = W.alg_flops_prefill(ctx[:1], cu_p, pos_p, 32) + int(ctx[1:].sum()) * 32 * 4 * HEAD_DIM
    return {"value": round(fl / t / 1e9, 2), "unit": "GFLOP/s", "cores": threads, "kind": "port",
            "sample": (f"the first prefill chunk ({b - a} rows after {int(ctx[0]) - (b - a)} tokens) and the "
                       f"first {len(dec)} decode rows, bf16 KV upcast to fp32, median of 3: {t:.3f} s "
                       f"({fl / 1e9:.1f} GFLOP); CPU {cpu_model()}")}


def mixed_batch_extra(dev, stream, cpu: bool = True) -> dict:
    """Attention over the mixed-batch workload (8 prefill chunks of 512 rows
    after priors U[0, 4096] and 120 decode rows with contexts U[256, 4096],
    shuffled; 32 q / 8 kv heads, bf16 q), K/V already appended, two routes
    of mkv.Attention: "split" (the reference's index_select -> decode kernel
    + prefill kernel -> index_copy_, attention.py:1711-1760), "unified"
    (one prefill launch over every row) and "overlap" (split, with the decode
    rows on a second stream beside the prefill kernel)."""
    import torch

    from mkv import attention as A
    from mkv import context as C
    from mkv import workloads as W

    m = W.prefill_mixed(seed=4)
    T = int(m["cu_seqlens_q"][-1])
    flops = W.alg_flops_prefill(m["context_lens"], m["cu_seqlens_q"], m["positions"], 32)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(T, 32, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    split = C.split_mixed_decode_prefill_metadata(m["cu_seqlens_q"].tolist(), m["query_lens"],
                                                   m["is_decode"])
    split.decode_token_indices_tensor = torch.tensor(split.decode_token_indices, device=dev)
    split.decode_seq_indices_tensor = torch.tensor(split.decode_seq_indices, device=dev)
    split.prefill_token_indices_tensor = torch.tensor(split.prefill_token_indices, device=dev)
    split.prefill_seq_indices_tensor = torch.tensor(split.prefill_seq_indices, device=dev)
    split.prefill_cu_seqlens_q_tensor = torch.tensor(split.prefill_cu_seqlens_q, dtype=torch.int32,
                                                     device=dev)
    res = {"workload": f"{T} rows: 8 x 512-row prefill chunks + 120 decode rows, 32 q / 8 kv heads; "
                       "*_with_append_us: each row's own K/V (bf16) appended in the timed step first"}
    # each row's slot: its position through its sequence's block table
    bs_m = m["block_size"]
    seq_of_row = torch.repeat_interleave(torch.arange(len(m["query_lens"])), torch.tensor(m["query_lens"]))
    pos = m["positions"]
    slots = (m["block_tables"][seq_of_row, pos // bs_m].to(torch.int64) * bs_m + pos % bs_m).to(dev)
    k_new = torch.randn(T, 8, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    v_new = torch.randn(T, 8, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    for name, dt in (("bf16", torch.bfloat16), ("fp8", torch.float8_e4m3fn)):
        kc = torch.empty(m["num_blocks"], m["block_size"], 8, HEAD_DIM, dtype=dt, device=dev)
        vc = torch.empty_like(kc)
        ks = W.fill_pool_on_device(kc, 500)
        vs = W.fill_pool_on_device(vc, 501)
        layer = A.Attention(32, HEAD_DIM, num_kv_heads=8, block_size=m["block_size"])
        layer.k_cache, layer.v_cache = kc, vc
        if name == "fp8":
            layer.kv_cache_dtype = "fp8_per_tensor"
            layer.k_scale = torch.tensor([ks], device=dev)
            layer.v_scale = torch.tensor([vs], device=dev)
        C.set_context(True, cu_seqlens_q=m["cu_seqlens_q"].to(dev), max_seqlen_q=512,
                      slot_mapping=None, context_lens=m["context_lens"].to(dev),
                      block_tables=m["block_tables"].to(dev), positions=m["positions"].to(dev),
                      mixed_attention_split=split, is_full_prefill=False)
        try:
            row = {}
            for route in ("split", "unified", "overlap"):
                layer.mixed_batch = route
                ms, _ = time_launches(lambda i: layer(q, q, q, kv_appended=True), 20, 3, stream,
                                      settle_first=True)
                row[f"{route}_us"] = round(ms * 1e3, 1)
            row["best_speedup_vs_split"] = round(row["split_us"] / min(row["unified_us"], row["overlap_us"]), 2)
            # rooflines of the default (unified) launch: the prefill rows are
            # MFMA work, the decode rows HBM reads; both fractions are given
            us = row["unified_us"]
            ekv = 2 if name == "bf16" else 1
            kv_bytes = int(m["context_lens"].sum()) * 8 * HEAD_DIM * 2 * ekv + T * 32 * HEAD_DIM * 4
            row["roofline"] = {
                "alg_flops": flops, "alg_kv_bytes": kv_bytes,
                "TFLOPs": round(flops / us / 1e6, 1), "frac_of_2500_TFLOPs": round(flops / us / 1e6 / 2500, 4),
                **({"frac_of_5000_TFLOPs_fp8_peak": round(flops / us / 1e6 / 5000, 4)} if name != "bf16" else {}),
                "GBps": round(kv_bytes / us / 1e3, 1),
                "frac_of_8000_GBps": round(kv_bytes / us / 1e3 / PEAK_HBM_GBPS, 4),
                "bound": "mfma" if flops / 2.5e15 > kv_bytes / 8e12 else "hbm"}
            if name == "bf16" and cpu:
                row["cpu_baseline"] = cpu_mixed_baseline(q, kc, vc, m)
            # the engine's step: the rows' own K/V appended first (store, then attend)
            C.set_context(True, cu_seqlens_q=m["cu_seqlens_q"].to(dev), max_seqlen_q=512,
                          slot_mapping=slots, context_lens=m["context_lens"].to(dev),
                          block_tables=m["block_tables"].to(dev), positions=m["positions"].to(dev),
                          mixed_attention_split=split, is_full_prefill=False)
            for route in ("split", "unified"):
                layer.mixed_batch = route
                ms, _ = time_launches(lambda i: layer(q, k_new, v_new), 20, 3, stream, settle_first=True)
                row[f"{route}_with_append_us"] = round(ms * 1e3, 1)
        finally:
            C.reset_context()
        res[f"{name}_kv"] = row
        del kc, vc
    return res


def graph_time_us(fn, reps: int = 20, replays: int = 10) -> float:
    """Device time per call of fn (µs), from replays of a HIP graph that
    holds `reps` back-to-back calls: for launches shorter than the host's
    enqueue time, where an eager loop would time the host.  The replays are
    settled first (chunks of 4 until four chunk means agree within 1%, at
    most 200 replays), as the headline step is: a series that starts from
    an idle GPU runs through the power controller's transient."""
    import torch

    from mkv.decode_state import graph_capture

    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with graph_capture(g):
        for _ in range(reps):
            fn()
    for _ in range(3):
        g.replay()
    settle(lambda i: g.replay(), torch.cuda.current_stream(), chunk=4, tol=0.01, max_steps=200)
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(replays):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / (reps * replays)


def cpu_decode_baseline(q, kc, vc, bt, ctx, scale, num_heads, num_kv_heads, bs, ks, vs,
                        nbytes: int, what: str, head_dim: int = HEAD_DIM):
    """The reference's PyTorch decode path (decode_torch_optimized semantics,
    benchmark_decoding.py:145-198, restated in the oracle) on host tensors,
    micro-batches of 16 sequences, median of 3.  Returns (record, output)."""
    from oracle import reference as R

    threads = _cpu_threads()
    out = {}

    def run():
        out["o"] = R.decode_torch_optimized_ref(q, kc, vc, bt, ctx, scale, num_heads, num_kv_heads,
                                                head_dim, bs, ks, vs, micro_batch=16)

    t = _median_time(run)
    return ({"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
             "sample": f"{what}; median of 3: {t:.3f} s; CPU {cpu_model()}, os.cpu_count {os.cpu_count()}"},
            out["o"])


def configs_extra(dev, stream, cpu: bool = True, which=DECODE_CONFIGS) -> dict:
    """The other decode configurations of the workload set, each with its
    algorithmic bytes, HBM roofline fraction, the reference's CPU decode path
    timed on the same inputs, and the largest difference from it:
    fp32 decode at batch 4 (16 q / 8 kv heads, pool of 64 blocks, contexts
    U[64, 2048]); FP8 decode at batch 32 (32 q / 8 kv heads) over the pool the
    4096-token FP8 append workload leaves (every slot filled first, then the
    append); the end-to-end engine's decode shape under the library's choice
    and each schedule; the batch-256 decode workload with a bf16 cache.
    Each line runs the library's choice of schedule (split_tokens 0) and
    names it.  `which` selects a subset (names as in DECODE_CONFIGS)."""
    import torch

    import mkv
    from mkv import attention as A
    from mkv import workloads as W

    def route(B, Hq, Hkv, mb, bs, kv_dtype):
        return ROUTE_NAMES[mkv._lib.query("mkv_paged_decode_route", B, Hq, Hkv, mb, bs, HEAD_DIM, kv_dtype, 0, 0)]

    res = {}
    # fp32 decode, batch 4
    if "fp32_decode_b4" in which:
        w = W.decode_small(seed=1)
        q, kc, vc = w["q"].to(dev), w["k_cache"].to(dev), w["v_cache"].to(dev)
        bt, ctx = w["block_tables"].to(dev), w["context_lens"].to(dev)
        out = torch.empty_like(q)
        fn = lambda: A._decode(q, kc, vc, bt, ctx, w["scale"], 16, 8, HEAD_DIM, out=out)
        us = graph_time_us(fn)
        nb = W.alg_bytes_decode(w["context_lens"], 256, 16, 8, kv_bytes=4, q_bytes=4)
        row = {"workload": f"fp32 KV and q, batch 4, 16 q / 8 kv heads, contexts {w['context_lens'].tolist()}",
               "us": round(us, 2), "algorithmic_bytes": nb, "GBps": round(nb / us / 1e3, 1),
               "frac_of_8000_GBps": round(nb / us / 1e3 / PEAK_HBM_GBPS, 4),
               "note": "35 MB of KV: the step is launch- and latency-bound and the bytes fit the "
                       "256 MB Infinity Cache, so this is not an HBM rate",
               "library_route": route(4, 16, 8, w["block_tables"].shape[1], 256, mkv._lib.DTYPE_F32)}
        if cpu:
            rec, o = cpu_decode_baseline(w["q"], w["k_cache"], w["v_cache"], w["block_tables"],
                                         w["context_lens"], w["scale"], 16, 8, 256, None, None, nb,
                                         "the whole workload, fp32")
            row["cpu_baseline"] = rec
            row["max_abs_err_vs_cpu"] = float((out.cpu() - o).abs().max())
        res["fp32_decode_b4"] = row
        del q, kc, vc

    # FP8 decode, batch 32, over the appended pool
    if "fp8_decode_b32" in which:
        w = W.decode_fp8_b32(seed=2)
        N, bs = w["num_blocks"], w["block_size"]
        kp = torch.zeros(N, bs, 8, HEAD_DIM, dtype=torch.float8_e4m3fn, device=dev)
        vp = torch.zeros_like(kp)
        ks, vs = torch.ones(1, device=dev), torch.ones(1, device=dev)
        A.store_kvcache_fp8(w["fill_key"].to(dev), w["fill_value"].to(dev), kp, vp, ks, vs,
                            w["fill_slots"].to(dev), bs, "fp8_per_tensor")
        A.store_kvcache_fp8(w["key"].to(dev), w["value"].to(dev), kp, vp, ks, vs,
                            w["slot_mapping"].to(dev), bs, "fp8_per_tensor")
        q = w["q"].to(dev)
        bt, ctx = w["block_tables"].to(dev), w["context_lens"].to(dev)
        out = torch.empty_like(q)
        fn = lambda: A._decode(q, kp, vp, bt, ctx, w["scale"], 32, 8, HEAD_DIM, ks, vs, out=out)
        us = graph_time_us(fn)
        nb = W.alg_bytes_decode(w["context_lens"], bs, 32, 8, kv_bytes=1)
        row = {"workload": f"FP8 per-tensor KV (scales {float(ks):.6g} / {float(vs):.6g}), bf16 q, batch 32, "
                           f"32 q / 8 kv heads, contexts U[256, 4096] sum {int(w['context_lens'].sum())}",
               "us": round(us, 2), "algorithmic_bytes": nb, "GBps": round(nb / us / 1e3, 1),
               "frac_of_8000_GBps": round(nb / us / 1e3 / PEAK_HBM_GBPS, 4),
               "library_route": route(32, 32, 8, w["block_tables"].shape[1], bs, mkv._lib.DTYPE_FP8E4M3)}
        if cpu:
            rec, o = cpu_decode_baseline(w["q"].float(), kp.cpu(), vp.cpu(), w["block_tables"],
                                         w["context_lens"], w["scale"], 32, 8, bs, float(ks), float(vs),
                                         nb, "the whole batch, fp32 on the dequantised cache")
            row["cpu_baseline"] = rec
            row["max_abs_err_vs_cpu"] = float((out.float().cpu() - o).abs().max())
        res["fp8_decode_b32"] = row
        del kp, vp

    # FP8 decode at the end-to-end engine's decode shape (60 rows of 300-800
    # tokens, 16 q / 8 kv heads, 4-block tables: the engine pads each decode
    # step's tables to its longest sequence, rounded up to a power of two):
    # the library's choice (the workgroup route here) and each schedule
    if "fp8_decode_b60_engine_shape" in which:
        g = torch.Generator().manual_seed(11)
        ctx = torch.randint(300, 801, (60,), generator=g)
        N = 60 * 4 + 16
        bt = W.fragmented_block_tables(ctx, 256, N, g, max_blocks=4).to(dev)
        kp = torch.empty(N, 256, 8, HEAD_DIM, dtype=torch.float8_e4m3fn, device=dev)
        vp = torch.empty_like(kp)
        W.fill_pool_on_device(kp, 3001)
        W.fill_pool_on_device(vp, 3002)
        qd = torch.randn(60, 16, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
        sc = torch.full((1,), 0.0125, device=dev)
        ctxd = ctx.to(dev)
        out = torch.empty_like(qd)
        nb = W.alg_bytes_decode(ctx, 256, 16, 8, kv_bytes=1, q_bytes=2)
        row = {"workload": f"FP8 per-tensor KV, bf16 q, batch 60, 16 q / 8 kv heads, contexts U[300, 800] "
                           f"sum {int(ctx.sum())}, 4-block tables (the end-to-end engine's decode shape)",
               "algorithmic_bytes": nb,
               "library_route": ROUTE_NAMES[mkv._lib.query("mkv_paged_decode_route", 60, 16, 8, 4, 256,
                                                           HEAD_DIM, mkv._lib.DTYPE_FP8E4M3, 0, 0)]}
        for name, st in (("library", 0), ("stream_k", A.DECODE_STREAM), ("split_k_256", 256),
                         ("workgroup", A.DECODE_WORKGROUP)):
            fn = lambda st=st: A._decode(qd, kp, vp, bt, ctxd, 0.088, 16, 8, HEAD_DIM, sc, sc,
                                         split_tokens=st, out=out)
            us = graph_time_us(fn)
            row[name] = {"us": round(us, 2), "GBps": round(nb / us / 1e3, 1),
                         "frac_of_8000_GBps": round(nb / us / 1e3 / PEAK_HBM_GBPS, 4)}
        # The whole decode step of one layer from its qkv rows (bf16): the
        # producer (q/k RMSNorm, rotary embedding, FP8 append at each row's
        # last position) and the attention, as two calls and in one launch
        from mkv import producer as P

        qkv = (torch.randn(60, 32 * HEAD_DIM, generator=g)).to(torch.bfloat16).to(dev)
        inv = 1000000.0 ** (-torch.arange(0, HEAD_DIM, 2, dtype=torch.float64) / HEAD_DIM)
        ang = torch.arange(4096, dtype=torch.float64)[:, None] * inv[None, :]
        cs = torch.cat([ang.cos(), ang.sin()], dim=1).to(torch.bfloat16).to(dev)  # [cos | sin] rows
        nw_ = (torch.rand(HEAD_DIM, generator=g) + 0.5).to(torch.bfloat16).to(dev)
        pos = (ctx - 1).to(dev)
        btc = bt.cpu()
        slots = torch.tensor([int(btc[b, (int(ctx[b]) - 1) // 256]) * 256 + (int(ctx[b]) - 1) % 256
                              for b in range(60)], device=dev)
        sc._mkv_calibrated = True

        def producer_step():
            return P.qkv_norm_rope_append(qkv, pos, 16, 8, HEAD_DIM, cs, kp, vp, slots, 256, q_norm_weight=nw_,
                                          k_norm_weight=nw_, kv_cache_dtype="fp8_per_tensor", k_scale=sc,
                                          v_scale=sc)[0]

        def two_calls():
            A._decode(producer_step(), kp, vp, bt, ctxd, 0.088, 16, 8, HEAD_DIM, sc, sc, out=out)

        def one_launch():
            P.qkv_norm_rope_append_decode(qkv, pos, 16, 8, HEAD_DIM, cs, kp, vp, slots, 256, bt, ctxd, 0.088,
                                          q_norm_weight=nw_, k_norm_weight=nw_, kv_cache_dtype="fp8_per_tensor",
                                          k_scale=sc, v_scale=sc, out=out)
        row["decode_step_from_qkv"] = {
            "what": "producer (q/k norm, rotary, FP8 append of each row's new token) + attention, "
                    "library schedule",
            "two_calls_us": round(graph_time_us(two_calls), 2),
            "one_launch_us": round(graph_time_us(one_launch), 2),
            "producer_alone_us": round(graph_time_us(producer_step), 2)}
        # the same step over bf16 pools of the same shape (kv_cache_dtype 'auto')
        kb = torch.empty(N, 256, 8, HEAD_DIM, dtype=torch.bfloat16, device=dev)
        vb = torch.empty_like(kb)
        W.fill_pool_on_device(kb, 3003)
        W.fill_pool_on_device(vb, 3004)

        def two_calls_bf16():
            q16 = P.qkv_norm_rope_append(qkv, pos, 16, 8, HEAD_DIM, cs, kb, vb, slots, 256, q_norm_weight=nw_,
                                         k_norm_weight=nw_)[0]
            A._decode(q16, kb, vb, bt, ctxd, 0.088, 16, 8, HEAD_DIM, out=out)

        def one_launch_bf16():
            P.qkv_norm_rope_append_decode(qkv, pos, 16, 8, HEAD_DIM, cs, kb, vb, slots, 256, bt, ctxd, 0.088,
                                          q_norm_weight=nw_, k_norm_weight=nw_, out=out)
        row["decode_step_from_qkv_bf16_cache"] = {
            "what": "the same step over bf16 KV pools of the same shape",
            "two_calls_us": round(graph_time_us(two_calls_bf16), 2),
            "one_launch_us": round(graph_time_us(one_launch_bf16), 2)}
        del kb, vb
        # and over FP8 pools with per-token-head scales (one per slot and KV head)
        kt = torch.empty(N, 256, 8, HEAD_DIM, dtype=torch.float8_e4m3fn, device=dev)
        vt = torch.empty_like(kt)
        kst = torch.empty(N, 256, 8, dtype=torch.float32, device=dev)
        vst = torch.empty_like(kst)
        W.fill_pools_per_token_head_on_device(kt, vt, kst, vst, 3005, "fp8_per_token_head")

        def two_calls_tok():
            qt = P.qkv_norm_rope_append(qkv, pos, 16, 8, HEAD_DIM, cs, kt, vt, slots, 256, q_norm_weight=nw_,
                                        k_norm_weight=nw_, kv_cache_dtype="fp8_per_token_head", k_scale=kst,
                                        v_scale=vst)[0]
            A._decode(qt, kt, vt, bt, ctxd, 0.088, 16, 8, HEAD_DIM, kst, vst, out=out, per_token_head=True)

        def one_launch_tok():
            P.qkv_norm_rope_append_decode(qkv, pos, 16, 8, HEAD_DIM, cs, kt, vt, slots, 256, bt, ctxd, 0.088,
                                          q_norm_weight=nw_, k_norm_weight=nw_, kv_cache_dtype="fp8_per_token_head",
                                          k_scale=kst, v_scale=vst, out=out)
        row["decode_step_from_qkv_fp8_per_token_head_cache"] = {
            "what": "the same step over FP8 pools with per-token-head scales (the two calls' decode on the "
                    "library's route for those scales)",
            "two_calls_us": round(graph_time_us(two_calls_tok), 2),
            "one_launch_us": round(graph_time_us(one_launch_tok), 2)}
        res["fp8_decode_b60_engine_shape"] = row
        del kp, vp, kt, vt

    # bf16 decode, the batch-256 workload
    if "bf16_decode_b256" in which:
        meta = W.decode_b256_metadata(seed=3)
        N, bs = meta["num_blocks"], meta["block_size"]
        pools = []
        for l in range(4):
            kc = torch.empty(N, bs, 8, HEAD_DIM, dtype=torch.bfloat16, device=dev)
            vc = torch.empty_like(kc)
            W.fill_pool_on_device(kc, 2000 + 2 * l)
            W.fill_pool_on_device(vc, 2001 + 2 * l)
            pools.append((kc, vc))
        g = torch.Generator().manual_seed(3)
        q = torch.randn(256, 32, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
        bt, ctx = meta["block_tables"].to(dev), meta["context_lens"].to(dev)
        out = torch.empty_like(q)
        sm = 1.0 / math.sqrt(HEAD_DIM)

        def step(i):
            kc, vc = pools[i % len(pools)]
            A._decode(q, kc, vc, bt, ctx, sm, 32, 8, HEAD_DIM, out=out)

        ms, rec_settle = time_launches(step, 40, 5, stream, settle_first=True)
        nb = W.alg_bytes_decode(meta["context_lens"], bs, 32, 8, kv_bytes=2)
        row = {"workload": "the batch-256 decode workload (32 q / 8 kv heads, contexts log-U[512, 8192]) "
                           "with bf16 KV, 4 rotating layer pools (16 GiB)",
               "us": round(ms * 1e3, 2), "algorithmic_bytes": nb, "GBps": round(nb / ms / 1e6, 1),
               "frac_of_8000_GBps": round(nb / ms / 1e6 / PEAK_HBM_GBPS, 4), "settle": rec_settle}
        if cpu:
            step(0)
            torch.cuda.synchronize()
            kc, vc = pools[0]
            n = 32
            used = sorted({int(x) for x in meta["block_tables"][:n].flatten() if x >= 0})
            remap = {p: i for i, p in enumerate(used)}
            idx = torch.tensor(used, device=dev)
            bt_c = meta["block_tables"][:n].clone()
            bt_c.apply_(lambda x: remap[x] if x >= 0 else -1)
            nbs = W.alg_bytes_decode(meta["context_lens"][:n], bs, 32, 8, kv_bytes=2)
            rec, o = cpu_decode_baseline(q[:n].float().cpu(), kc.index_select(0, idx).cpu(),
                                         vc.index_select(0, idx).cpu(), bt_c, meta["context_lens"][:n],
                                         sm, 32, 8, bs, None, None, nbs,
                                         f"first {n} of 256 sequences, fp32 on the upcast bf16 cache")
            row["cpu_baseline"] = rec
            row["max_abs_err_vs_cpu"] = float((out[:n].float().cpu() - o).abs().max())
        res["bf16_decode_b256"] = row
        del pools

    # head_dim 64 (the Llama-3.2-1B attention shape: 32 q / 8 kv heads): the
    # batch-256 decode workload's contexts and tables, FP8 per-tensor KV
    if "fp8_decode_b256_d64" in which:
        meta = W.decode_b256_metadata(seed=3)
        N, bs, D64 = meta["num_blocks"], meta["block_size"], 64
        pools = []
        for l in range(8):
            kc = torch.empty(N, bs, 8, D64, dtype=torch.float8_e4m3fn, device=dev)
            vc = torch.empty_like(kc)
            ks_ = W.fill_pool_on_device(kc, 2100 + 2 * l)
            vs_ = W.fill_pool_on_device(vc, 2101 + 2 * l)
            pools.append((kc, vc, torch.tensor([ks_], device=dev), torch.tensor([vs_], device=dev)))
        g = torch.Generator().manual_seed(3)
        q = torch.randn(256, 32, D64, generator=g).to(torch.bfloat16).to(dev)
        bt, ctx = meta["block_tables"].to(dev), meta["context_lens"].to(dev)
        out = torch.empty_like(q)
        sm = 1.0 / math.sqrt(D64)

        def step64(i):
            kc, vc, ksd, vsd = pools[i % len(pools)]
            A._decode(q, kc, vc, bt, ctx, sm, 32, 8, D64, ksd, vsd, out=out)

        ms, rec_settle = time_launches(step64, 40, 5, stream, settle_first=True)
        nb = W.alg_bytes_decode(meta["context_lens"], bs, 32, 8, kv_bytes=1, head_dim=D64)
        row = {"workload": "the batch-256 decode workload's contexts (log-U[512, 8192]) and tables at head_dim 64, "
                           "32 q / 8 kv heads (Llama-3.2-1B), FP8 per-tensor KV, bf16 q, 8 rotating layer pools",
               "us": round(ms * 1e3, 2), "algorithmic_bytes": nb, "GBps": round(nb / ms / 1e6, 1),
               "frac_of_8000_GBps": round(nb / ms / 1e6 / PEAK_HBM_GBPS, 4), "settle": rec_settle,
               "library_route": ROUTE_NAMES[mkv._lib.query("mkv_paged_decode_route", 256, 32, 8, meta["max_blocks"],
                                                           bs, D64, mkv._lib.DTYPE_FP8E4M3, 0, 0)]}
        if cpu:
            step64(0)
            torch.cuda.synchronize()
            kc, vc, ksd, vsd = pools[0]
            n = 32
            used = sorted({int(x) for x in meta["block_tables"][:n].flatten() if x >= 0})
            remap = {p: i for i, p in enumerate(used)}
            idx = torch.tensor(used, device=dev)
            bt_c = meta["block_tables"][:n].clone()
            bt_c.apply_(lambda x: remap[x] if x >= 0 else -1)
            nbs = W.alg_bytes_decode(meta["context_lens"][:n], bs, 32, 8, kv_bytes=1, head_dim=D64)
            rec, o = cpu_decode_baseline(q[:n].float().cpu(), kc.index_select(0, idx).cpu(),
                                         vc.index_select(0, idx).cpu(), bt_c, meta["context_lens"][:n],
                                         sm, 32, 8, bs, float(ksd), float(vsd), nbs,
                                         f"first {n} of 256 sequences, fp32 on the dequantised cache",
                                         head_dim=D64)
            row["cpu_baseline"] = rec
            row["max_abs_err_vs_cpu"] = float((out[:n].float().cpu() - o).abs().max())
        res["fp8_decode_b256_d64"] = row
        del pools
    return res


def e2e_extra(dev, baselines: bool = True) -> dict:
    """The end-to-end engine workload: a random-init Qwen3-0.6B-shaped model
    (28 layers, hidden 1024, 16 q / 8 kv heads, head_dim 128, intermediate
    3072, vocab 151936, bf16 weights N(0, 0.02), seed 5) generating 256
    tokens (temperature 1.0, EOS ignored) for each of 60 prompts of uniform
    random token ids with lengths U[32, 512], through mkv.engine: continuous
    batching of up to 64 sequences, chunked prefill under a 1024-token budget,
    FP8 per-tensor KV in 256-token blocks, decode steps replayed from
    captured graphs.  One untimed run first (graph capture, GEMM
    heuristics), then the timed run; e2e decode tok/s = generated tokens /
    wall time of the whole generate."""
    import torch

    from mkv import engine as E

    g = torch.Generator().manual_seed(5)
    lens = torch.randint(32, 513, (60,), generator=g).tolist()
    prompts = [torch.randint(0, 151936, (L,), generator=g).tolist() for L in lens]
    cfg = E.ModelConfig()
    model = E.Qwen3Model(cfg, dev, seed=5, block_size=256)
    # decode schedule: the library's choice (the workgroup route for these 60
    # rows: one workgroup per sequence and KV head, waves merged in LDS)
    eng = E.Engine(model, num_blocks=512, max_num_seqs=64, max_num_batched_tokens=1024,
                   kv_cache_dtype="fp8_per_tensor", max_model_len=4096, seed=0)
    eng.generate(prompts, max_tokens=256)  # warm-up: captures the decode graphs
    eng.stats.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    outs = eng.generate(prompts, max_tokens=256)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    res = eng.summary(wall)
    assert res["generated_tokens"] == 60 * 256 and all(len(o) == 256 for o in outs)
    res["workload"] = (f"Qwen3-0.6B shape (28 layers, hidden 1024, 16/8 heads, D 128, I 3072, vocab "
                       f"151936), bf16 random weights; 60 prompts of {sum(lens)} tokens (32-512), "
                       "256 output tokens each, T 1.0; max_num_seqs 64, max_num_batched_tokens "
                       "1024, FP8 per-tensor KV, block 256, chunked prefill, captured decode")
    if not baselines:  # (--e2e-no-baselines: a profile of this engine alone)
        return res
    # the same engine with eager decode steps (no captured graphs)
    # (every engine gets the same full warm-up run as the captured one, so
    # that first-use GEMM heuristics for the larger batch shapes stay out of
    # its timed run)
    eager = E.Engine(model, num_blocks=512, max_num_seqs=64, max_num_batched_tokens=1024,
                     kv_cache_dtype="fp8_per_tensor", max_model_len=4096, seed=0, use_graphs=False)
    eager.generate(prompts, max_tokens=256)  # warm-up
    eager.stats.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    eager.generate(prompts, max_tokens=256)
    torch.cuda.synchronize()
    eres = eager.summary(time.perf_counter() - t0)
    res["mkv_eager_engine"] = {k: eres[k] for k in ("e2e_decode_tok_s", "decode_only_tok_s", "wall_s")}
    # the same captured engine with the reference's most accurate KV mode,
    # FP8 codes with one scale per slot and KV head (each decode step's
    # producer and per-token-head decode in one launch per layer)
    ptok = E.Engine(model, num_blocks=512, max_num_seqs=64, max_num_batched_tokens=1024,
                    kv_cache_dtype="fp8_per_token_head", max_model_len=4096, seed=0)
    ptok.generate(prompts, max_tokens=256)  # warm-up
    ptok.stats.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ptok.generate(prompts, max_tokens=256)
    torch.cuda.synchronize()
    pres = ptok.summary(time.perf_counter() - t0)
    res["mkv_engine_fp8_per_token_head_kv"] = {k: pres[k] for k in ("e2e_decode_tok_s", "decode_only_tok_s",
                                                                     "wall_s")}
    del eng, eager, ptok, model
    torch.cuda.empty_cache()
    # the same engine and workload with the reference's PyTorch attention on the GPU
    base_model = _torch_attention_model()(cfg, dev, seed=5, block_size=256)
    base = E.Engine(base_model, num_blocks=512, max_num_seqs=64, max_num_batched_tokens=1024,
                    kv_cache_dtype="fp8_per_tensor", max_model_len=4096, seed=0, use_graphs=False)
    base.generate(prompts, max_tokens=256)  # warm-up (the same full run)
    base.stats.clear()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    bouts = base.generate(prompts, max_tokens=256)
    torch.cuda.synchronize()
    bwall = time.perf_counter() - t0
    assert all(len(o) == 256 for o in bouts)
    bres = base.summary(bwall)
    res["torch_attention_engine"] = {
        "e2e_decode_tok_s": bres["e2e_decode_tok_s"], "decode_only_tok_s": bres["decode_only_tok_s"],
        "wall_s": bres["wall_s"],
        # like for like: both engines eager (the PyTorch attention reads
        # lengths on the host, so it cannot be captured); the captured mkv
        # engine's figure adds graph replay on top
        "speedup_of_mkv_eager": round(res["mkv_eager_engine"]["e2e_decode_tok_s"] / bres["e2e_decode_tok_s"], 2),
        "speedup_of_mkv_captured": round(res["e2e_decode_tok_s"] / bres["e2e_decode_tok_s"], 2),
        "what": "the same engine, producer, FP8 append, GEMMs and workload (eager decode steps), after the same "
                "full warm-up run; attention by the reference's PyTorch semantics in fp32 on the dequantised "
                "cache on the GPU (decode_torch_optimized, pytorch_standard_attention over the paged prefix)"}
    del base, base_model
    torch.cuda.empty_cache()
    return res


def _torch_attention_model():
    """mkv.engine's model with its attention computed by the reference's
    PyTorch semantics on the GPU, in fp32 on dequantised K/V: decode as
    decode_torch_optimized (benchmark_decoding.py:145-198: the batch's blocks
    gathered into a zero-padded (B, Lmax, Hkv, D), GQA by repeat_interleave,
    matmul, mask, softmax, matmul), prefill chunks and mixed items per
    sequence as pytorch_standard_attention (benchmark_prefilling.py:9-52)
    over the paged prefix with visible = min(context, position + 1)
    (attention.py:747).  It reads the layer's own cache after the same
    producer and append, so only the attention differs.  A baseline for the
    end-to-end workload, which the reference's engine cannot run (FP8 KV
    with chunked prefill raises, attention.py:1704-1708)."""
    import torch

    from mkv import context as C
    from mkv import engine as E

    class TorchAttentionModel(E.Qwen3Model):
        fuse_decode_step = False  # every step's attention through attention() below

        def attention(self, li, q, k, v):
            ctx = C.current_context()
            att = self.layers[li]["attn"]
            cfg = self.cfg
            Hq, Hkv, D, bs = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim, self.block_size
            G = Hq // Hkv
            sm = 1.0 / math.sqrt(D)
            fp8 = att.kv_cache_dtype == "fp8_per_tensor"
            kc, vc = att.k_cache, att.v_cache

            def gather(idx, n_tok):  # (..., nb) block ids -> fp32 K, V (..., n_tok, Hkv, D)
                shp = idx.shape[:-1] + (idx.shape[-1] * bs, Hkv, D)
                kk = kc[idx].reshape(shp)[..., :n_tok, :, :].float()
                vv = vc[idx].reshape(shp)[..., :n_tok, :, :].float()
                if fp8:
                    kk, vv = kk * att.k_scale, vv * att.v_scale
                return kk, vv

            out = torch.empty(q.shape[0], Hq, D, dtype=torch.float32, device=q.device)
            qf = q.float().view(-1, Hq, D)
            if not ctx.is_prefill:
                lens = ctx.context_lens
                B = lens.shape[0]
                L = max(int(lens.max()), 1)
                idx = ctx.block_tables[:, :(L + bs - 1) // bs].long().clamp_min(0)
                kk, vv = gather(idx, L)
                kk = kk.repeat_interleave(G, dim=2).permute(0, 2, 3, 1).contiguous()  # (B, Hq, D, L)
                vv = vv.repeat_interleave(G, dim=2).permute(0, 2, 1, 3).contiguous()  # (B, Hq, L, D)
                sc = torch.matmul(qf[:B].unsqueeze(2), kk).squeeze(2) * sm
                mask = torch.arange(L, device=q.device)[None, :] >= lens[:, None]
                p = torch.softmax(sc.masked_fill(mask[:, None, :], float("-inf")), -1).nan_to_num_(0.0)
                out[:B] = torch.matmul(p.unsqueeze(2), vv).squeeze(2)
            else:
                cu = ctx.cu_seqlens_q.tolist()
                lens = ctx.context_lens.tolist()
                for si in range(len(cu) - 1):
                    a, b, c = cu[si], cu[si + 1], int(lens[si])
                    if b == a:
                        continue
                    idx = ctx.block_tables[si, :(c + bs - 1) // bs].long().clamp_min(0)
                    kk, vv = gather(idx, c)
                    kk = kk.repeat_interleave(G, dim=1).permute(1, 2, 0).contiguous()  # (Hq, D, c)
                    vv = vv.repeat_interleave(G, dim=1).permute(1, 0, 2).contiguous()  # (Hq, c, D)
                    sc = torch.matmul(qf[a:b].permute(1, 0, 2).contiguous(), kk) * sm  # (Hq, n, c)
                    vis = torch.clamp(ctx.positions[a:b] + 1, max=c)
                    mask = torch.arange(c, device=q.device)[None, :] >= vis[:, None]
                    p = torch.softmax(sc.masked_fill(mask[None], float("-inf")), -1)
                    out[a:b] = torch.matmul(p, vv).permute(1, 0, 2)
            return out.to(q.dtype).reshape(q.shape[0], Hq * D)

    return TorchAttentionModel


def producer_extra(dev, stream) -> dict:
    """The fused producer (q/k RMSNorm + rotary + FP8 per-tensor append) for
    one layer, 16 q / 8 kv heads, head_dim 128, bf16 qkv, fp32 cos/sin table,
    at 256 tokens (a decode batch) and 4096 tokens (a prefill chunk), against
    the reference's sequence of operations on the same GPU: the q/k/v split,
    LayerNorm.rms_forward on q and k, apply_rotary_pos_emb, the contiguous
    copies of k and v (qwen3.py:85-118, attention.py:1664-1665) in eager torch,
    then the FP8 append.  Bytes are algorithmic: qkv rows, positions, cos/sin
    rows and slots read once, q and the FP8 K/V rows written once."""
    import torch

    from mkv import attention as A
    from mkv import producer as P

    Hq, Hkv, D, bs = 16, 8, HEAD_DIM, 256
    res = {"workload": "one layer, 16 q / 8 kv heads, head_dim 128, bf16 qkv, FP8 per-tensor KV"}
    g = torch.Generator().manual_seed(12)
    cs = (torch.arange(4096, dtype=torch.float32)[:, None] *
          (1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float32) / D)))[None, :])
    cs = torch.cat([cs.cos(), cs.sin()], dim=-1).to(dev)
    qw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    kw = (torch.rand(D, generator=g) + 0.5).to(torch.bfloat16).to(dev)
    for T in (256, 4096):
        qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16).to(dev)
        pos = torch.randint(0, 4096, (T,), generator=g).to(dev)
        slots = torch.randperm(1024 * bs, generator=g)[:T].to(torch.int64).to(dev)
        kc = torch.zeros(1024, bs, Hkv, D, dtype=torch.float8_e4m3fn, device=dev)
        vc = torch.zeros_like(kc)
        ks, vs = torch.ones(1, device=dev), torch.ones(1, device=dev)
        fused = lambda i: P.qkv_norm_rope_append(qkv, pos, Hq, Hkv, D, cs, kc, vc, slots, bs,
                                                 q_norm_weight=qw, k_norm_weight=kw,
                                                 kv_cache_dtype="fp8_per_tensor", k_scale=ks,
                                                 v_scale=vs)
        fused(0)  # first use: calibrates the scales

        def unfused(i):
            q, k, v = qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1)
            q, k, v = q.view(-1, Hq, D), k.view(-1, Hkv, D), v.view(-1, Hkv, D)

            def rms(x, w):
                var = x.pow(2).mean(dim=-1, keepdim=True) + 1e-5
                return x / var.sqrt() * w

            def rope(x, c, s_):
                x1, x2 = x.chunk(2, dim=-1)
                return torch.cat([x1 * c - x2 * s_, x1 * s_ + x2 * c], dim=-1)

            q, k = rms(q, qw), rms(k, kw)
            c, s_ = cs[pos].chunk(2, dim=-1)
            c, s_ = c.unsqueeze(1), s_.unsqueeze(1)
            q, k = rope(q, c, s_), rope(k, c, s_)
            A.store_kvcache_fp8(k.contiguous(), v.contiguous(), kc, vc, ks, vs, slots, bs,
                                "fp8_per_tensor")
            return q

        ms_f = time_launches(fused, 50, 5, stream)
        ms_u = time_launches(unfused, 20, 3, stream)
        nbytes = T * ((Hq + 2 * Hkv) * D * 2 + 8 + D * 4 + 8) + T * Hq * D * 2 + T * 2 * Hkv * D
        res[f"T{T}"] = {"fused_us": round(ms_f * 1e3, 2), "fused_GBps": round(nbytes / ms_f / 1e6, 1),
                        "reference_ops_us": round(ms_u * 1e3, 2), "speedup": round(ms_u / ms_f, 2),
                        "algorithmic_bytes": nbytes}
        del kc, vc
    return res


def decode_step_latency(dev, batches=(1, 8, 32), layers: int = 28, ctx0: int = 700,
                        steps: int = 30) -> dict:
    """Wall time of one decode step's attention work for a 28-layer stack
    (16 q / 8 kv heads, head_dim 128, block 256, FP8 KV, contexts ~700
    tokens), two ways:
      eager: the reference runner's per-step host work (prepare_decode,
        model_runner.py:621-640: Python lists -> pinned tensors -> device)
        followed by every layer's append + decode launched one by one;
      graph: the device-side metadata advance (mkv_decode_metadata) and all
        layers captured once per batch bucket and replayed (mkv.decode_state).
    Both synchronise at the end of each step; the attention kernels are the
    same.  Only the attention path runs (no projections or MLP)."""
    import torch

    from mkv import attention as A
    from mkv import decode_state as DS

    Hq, Hkv, bs = 16, 8, 256
    max_rows = max(batches)
    # lengths ctx0 + 37 b grow by one token per step (steps + 3 warm-up)
    max_blocks = (ctx0 + 37 * max_rows + steps + 3 + bs - 1) // bs
    N = max_rows * max_blocks + 8
    sm = 1.0 / math.sqrt(HEAD_DIM)
    g = torch.Generator().manual_seed(9)
    pools = []
    for _ in range(layers):
        kc = torch.zeros(N, bs, Hkv, HEAD_DIM, dtype=torch.float8_e4m3fn, device=dev)
        pools.append((kc, torch.zeros_like(kc), torch.full((1,), 0.02, device=dev),
                      torch.full((1,), 0.02, device=dev)))
    q = torch.randn(max_rows, Hq, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    kv = torch.randn(max_rows, Hkv, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    out = torch.empty(layers, max_rows, Hq, HEAD_DIM, dtype=torch.bfloat16, device=dev)

    def layers_fn(rows, slot, ctx, bt):
        for li, (kc, vc, ks, vs) in enumerate(pools):
            A.store_kvcache_fp8(kv[:rows], kv[:rows], kc, vc, ks, vs, slot, bs, "fp8_per_tensor")
            A._decode(q[:rows], kc, vc, bt, ctx, sm, Hq, Hkv, HEAD_DIM, ks, vs, out=out[li, :rows])

    res = {"workload": (f"{layers} layers x (FP8 append + decode), {Hq} q / {Hkv} kv heads, "
                        f"head_dim {HEAD_DIM}, block {bs}, contexts ~{ctx0} tokens; wall time per "
                        f"step incl. host work, synchronised; median of {steps}")}
    for B in batches:
        tables = [[b * max_blocks + j for j in range(max_blocks)] for b in range(B)]
        lens = [ctx0 + 37 * b for b in range(B)]
        # eager, reference-style host metadata every step
        times = []
        for it in range(steps + 3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            cur = [L + it for L in lens]
            ctx_l = list(cur)
            slot_l = [tables[b][(L - 1) // bs] * bs + (L - 1) % bs for b, L in enumerate(cur)]
            nb = max((L + bs - 1) // bs for L in cur)
            bt_l = [tables[b][:nb] for b in range(B)]
            slot = torch.tensor(slot_l, dtype=torch.long, pin_memory=True).to(dev, non_blocking=True)
            ctx = torch.tensor(ctx_l, dtype=torch.long, pin_memory=True).to(dev, non_blocking=True)
            bt = torch.tensor(bt_l, dtype=torch.int32, pin_memory=True).to(dev, non_blocking=True)
            layers_fn(B, slot, ctx, bt)
            torch.cuda.synchronize()
            if it >= 3:
                times.append(time.perf_counter() - t0)
        eager_us = statistics.median(times) * 1e6
        # device metadata + captured graph
        meta = DS.DecodeMetadata(max_rows, max_blocks, bs, N, dev)
        graphs = DS.DecodeGraphs(meta, layers_fn, buckets=[B])
        graphs.capture()
        for b in range(B):
            meta.set_row(b, tables[b], lens[b])
        times = []
        for it in range(steps + 3):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            graphs.run(B)
            torch.cuda.synchronize()
            if it >= 3:
                times.append(time.perf_counter() - t0)
        graph_us = statistics.median(times) * 1e6
        res[f"batch{B}"] = {"eager_host_metadata_us": round(eager_us, 1),
                            "graph_device_metadata_us": round(graph_us, 1),
                            "speedup": round(eager_us / graph_us, 2)}
        del graphs, meta
    return res


def cpu_baseline(kcs, vcs, scale_kv, q, meta, n_seqs: int) -> dict:
    """The reference's PyTorch decode path on the host cores, on the first
    n_seqs sequences of the workload (one micro-batch of 16 at a time)."""
    import torch

    from mkv import workloads as W
    from oracle import reference as R

    threads = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        threads = min(threads, int(env))
    torch.set_num_threads(threads)
    ctx = meta["context_lens"][:n_seqs]
    bt = meta["block_tables"][:n_seqs]
    bs = meta["block_size"]
    # copy just the sample's blocks to host memory, re-indexed compactly
    used = sorted({int(x) for x in bt[bt >= 0]})
    remap = {p: i for i, p in enumerate(used)}
    idx = torch.tensor(used, dtype=torch.int64, device=kcs.device)
    kc = kcs.index_select(0, idx).cpu()
    vc = vcs.index_select(0, idx).cpu()
    bt_c = bt.clone()
    for (i, j), p in zip(torch.nonzero(bt >= 0).tolist(), bt[bt >= 0].tolist()):
        bt_c[i, j] = remap[int(p)]
    qc = q[:n_seqs].float().cpu()
    ks, vs = scale_kv if scale_kv else (None, None)
    sm = 1.0 / math.sqrt(HEAD_DIM)

    def run():
        return R.decode_torch_optimized_ref(qc, kc, vc, bt_c, ctx, sm, 32, 8, HEAD_DIM, bs,
                                            ks, vs, micro_batch=16)

    run()  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = statistics.median(times)
    nbytes = W.alg_bytes_decode(ctx, bs, 32, 8, kv_bytes=kcs.element_size())
    return {
        "value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"first {n_seqs} of 256 sequences (context sum {int(ctx.sum())}), "
                   f"decode_torch_optimized semantics in fp32 on dequantised KV, micro-batch 16, "
                   f"median of 3; {t:.3f} s per sample; CPU {cpu_model()}, os.cpu_count "
                   f"{os.cpu_count()}"),
    }


def traffic_from_profiles(name: str):
    """HBM bytes per launch measured by a committed rocprofv3 PMC run, if any."""
    p = REPO / "profiles" / name
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("traffic_bytes_per_launch")
    except (ValueError, OSError):
        return None


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the decode path is per-GPU work and this build runs "
              f"no collectives, so --gpus {args.gpus} (WORLD_SIZE={world}) is not supported; "
              f"run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import mkv
    from mkv import attention as A
    from mkv import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mib > 0:
        n = args.copy_probe_mib << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": n, "launches": 5}), flush=True)
        return 0
    meta = W.decode_b256_metadata(seed=3, batch=args.batch,
                                  num_blocks=max(4096, 16 * args.batch))
    N, bs = meta["num_blocks"], meta["block_size"]
    kv_dtype = {"fp8": torch.float8_e4m3fn, "bf16": torch.bfloat16,
                "fp8_token": torch.float8_e4m3fn, "int8_token": torch.int8}[args.kv]
    per_token = args.kv in ("fp8_token", "int8_token")
    token_mode = {"fp8_token": "fp8_per_token_head", "int8_token": "int8_per_token_head"}.get(args.kv)
    layers = []
    for l in range(args.layers):
        kc = torch.empty(N, bs, args.num_kv_heads, HEAD_DIM, dtype=kv_dtype, device=dev)
        vc = torch.empty_like(kc)
        if per_token:
            ksd = torch.empty(N, bs, args.num_kv_heads, device=dev)
            vsd = torch.empty_like(ksd)
            W.fill_pools_per_token_head_on_device(kc, vc, ksd, vsd, 1000 + l, token_mode)
            layers.append((kc, vc, (ksd, vsd), None))
            continue
        ks = W.fill_pool_on_device(kc, 1000 + 2 * l)
        vs = W.fill_pool_on_device(vc, 1001 + 2 * l)
        sc = (torch.tensor([ks], device=dev), torch.tensor([vs], device=dev)) if ks else (None, None)
        layers.append((kc, vc, sc, (ks, vs) if ks else None))
    g = torch.Generator().manual_seed(3)
    Hq, Hkv = args.num_heads, args.num_kv_heads
    q = torch.randn(args.batch, Hq, HEAD_DIM, generator=g).to(torch.bfloat16).to(dev)
    bt = meta["block_tables"].to(dev)
    ctx = meta["context_lens"].to(dev)
    out = torch.empty_like(q)
    sm = 1.0 / math.sqrt(HEAD_DIM)
    stream = torch.cuda.current_stream(dev)

    def step(i):
        kc, vc, (ksd, vsd), _ = layers[i % len(layers)]
        A._decode(q, kc, vc, bt, ctx, sm, Hq, Hkv, HEAD_DIM, ksd, vsd,
                  split_tokens=args.split_tokens, out=out, per_token_head=per_token)

    nbytes = W.alg_bytes_decode(meta["context_lens"], bs, Hq, Hkv, kv_bytes=kv_dtype.itemsize,
                                scale_bytes=4 if per_token else 0)
    if args.skip_headline:
        # a profiling run of the extras: the headline step is not timed
        result = {"headline": "skipped (--skip-headline)"}
    else:
        torch.cuda.synchronize()
        t_wall = time.perf_counter()
        ms, settle_rec = time_launches(step, args.steps, args.warmup, stream, settle_first=True)
        t_wall = time.perf_counter() - t_wall
        gbps = nbytes / (ms * 1e-3) / 1e9
        pct = step_percentiles(step, 100, stream)
        if args.split_tokens > 0 or args.batch > 8192:
            split = mkv._lib.query("mkv_paged_decode_split_tokens", args.batch, Hkv, meta["max_blocks"], bs,
                                   args.split_tokens)
            schedule = f"split-K, {split}-token splits (paged_decode_mfma16_kernel + paged_decode_merge_kernel)"
        else:
            schedule = ("stream-K over 32-token tile columns, persistent grid, groups of Hkv waves "
                        "with one KV head per wave (paged_decode_stream_kernel + paged_decode_stream_merge_kernel)")

        result = {
            "metric": METRIC,
            "value": round(gbps, 2),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(ms, 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": {"fp8": "fp8", "bf16": "bf16", "fp8_token": "fp8", "int8_token": "int8"}[args.kv],
            "data": "synthetic (seeded N(0,1) KV pools and queries, seeded context lengths/tables)",
            "config": {
                "workload": (f"paged decode attention, batch {args.batch}, {Hq} q / {Hkv} kv heads, head_dim 128, "
                             f"block 256, ctx floor(exp(U(ln512, ln8192))) sum {int(meta['context_lens'].sum())}, "
                             f"fragmented tables over {N} blocks, {args.kv} KV "
                             f"({KV_DESC[args.kv]}), bf16 q/out, "
                             f"{args.layers} rotating layer pools"),
                "batch": args.batch, "num_heads": Hq, "num_kv_heads": Hkv, "head_dim": HEAD_DIM,
                "block_size": bs, "schedule": schedule, "algorithmic_bytes_per_step": nbytes,
            },
            "roofline": {
                "bound": "hbm", "achieved": round(gbps, 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                "frac": round(gbps / PEAK_HBM_GBPS, 4),
                # measured for the default workload only (profiles/decode_b256_<kv>_pmc.json)
                "traffic": (traffic_from_profiles(f"decode_b256_{args.kv}_pmc.json")
                            if (args.batch, Hq, Hkv, args.split_tokens) == (256, 32, 8, 0) else None),
                "timed_unit": "one decode step: main kernel + its merge kernel, HIP events on the launch stream",
            },
            "wall_s_timed_region": round(t_wall, 3),
            # untimed steps after the warm-up, run until the step time is steady
            "settle": settle_rec,
            "step_time": pct,
        }

    wanted = args.extra_set
    if wanted:
        extra = {}
        # the small decode configurations first: they are latency-bound and
        # cache-resident, and the appends' writes ahead of them leave the
        # caches full of dirty lines (fp32 batch 4: 21 µs alone, 25-29 µs
        # right after the append lines)
        if "configs" in wanted:
            extra["decode_configs"] = configs_extra(dev, stream, cpu=args.cpu_seqs > 0,
                                                    which=args.decode_config_set)
        # KV append + FP8 quantisation: 4096 tokens (5% padding) and 65536 tokens
        for T in ((4096, 65536) if "append" in wanted else ()):
            w = W.append_fp8(seed=2, num_tokens=T) if T == 4096 else None
            if w is None:
                gg = torch.Generator().manual_seed(20)
                kk = torch.randn(T, 8, HEAD_DIM, generator=gg).to(torch.bfloat16)
                vv = torch.randn(T, 8, HEAD_DIM, generator=gg).to(torch.bfloat16)
                sl = torch.randperm(1024 * 256, generator=gg)[:T].to(torch.int64)
                w = dict(key=kk, value=vv, slot_mapping=sl)
            kd, vd, sd = w["key"].to(dev), w["value"].to(dev), w["slot_mapping"].to(dev)
            kp = torch.zeros(1024, 256, 8, HEAD_DIM, dtype=torch.float8_e4m3fn, device=dev)
            vp = torch.zeros_like(kp)
            ksd = torch.tensor([0.05], device=dev)
            vsd = torch.tensor([0.05], device=dev)
            ams, _ = time_launches(lambda i: A._append(kd, vd, kp, vp, sd, ksd, vsd), 50, 5, stream,
                                   settle_first=True)
            ab = W.alg_bytes_append(w["slot_mapping"], 8, 2, 1)
            # us: eager launches (host enqueue included: at 4096 tokens the
            # kernel is shorter than the wrapper's host work); graph_us: device
            # time per call from graph replays of back-to-back calls
            gus = graph_time_us(lambda: A._append(kd, vd, kp, vp, sd, ksd, vsd))
            extra[f"append_fp8_T{T}"] = {"us": round(ams * 1e3, 2), "GBps": round(ab / ams / 1e6, 1),
                                         "graph_us": round(gus, 2), "graph_GBps": round(ab / gus / 1e3, 1)}
            if T == 4096 and args.cpu_seqs > 0:
                extra[f"append_fp8_T{T}"]["cpu_baseline"] = cpu_append_baseline(
                    w["key"], w["value"], w["slot_mapping"], 0.05, 0.05)
            del kp, vp
            # the copy append (bf16 rows into a bf16 pool) on the same tokens
            kp = torch.zeros(1024, 256, 8, HEAD_DIM, dtype=torch.bfloat16, device=dev)
            vp = torch.zeros_like(kp)
            cms, _ = time_launches(lambda i: A._append(kd, vd, kp, vp, sd), 50, 5, stream,
                                   settle_first=True)
            cab = W.alg_bytes_append(w["slot_mapping"], 8, 2, 2)
            gus = graph_time_us(lambda: A._append(kd, vd, kp, vp, sd))
            extra[f"append_copy_T{T}"] = {"us": round(cms * 1e3, 2), "GBps": round(cab / cms / 1e6, 1),
                                          "graph_us": round(gus, 2), "graph_GBps": round(cab / gus / 1e3, 1)}
            if T == 4096 and args.cpu_seqs > 0:
                extra[f"append_copy_T{T}"]["cpu_baseline"] = cpu_copy_append_baseline(
                    w["key"], w["value"], w["slot_mapping"])
            del kp, vp
        if "e2e" in wanted:
            extra["e2e_engine"] = e2e_extra(dev, baselines=not args.e2e_no_baselines)
        if "prefill" in wanted:
            extra["prefill_chunked"] = prefill_extra(dev, stream, cpu=args.cpu_seqs > 0)
        if "latency" in wanted:
            extra["decode_step_latency"] = decode_step_latency(dev)
        if "producer" in wanted:
            extra["producer_fused"] = producer_extra(dev, stream)
        if "mixed" in wanted:
            extra["mixed_batch"] = mixed_batch_extra(dev, stream, cpu=args.cpu_seqs > 0)
        if "gather" in wanted:
            extra["gather_kv"] = gather_extra(layers[0][0], meta, dev, stream, cpu=args.cpu_seqs > 0)
        if "copy" in wanted:
            extra["box_copy_GBps"] = round(box_copy_gbps(dev, stream), 1)
            extra["box_read"] = box_read_gbps(dev, stream)
            if "value" in result:
                extra["box_read"]["headline_frac_of_box_read"] = round(
                    result["value"] / extra["box_read"]["GBps"], 4)
        result["extra"] = extra

    if args.cpu_seqs > 0 and not per_token and not args.skip_headline:
        kc0, vc0, _, scales = layers[0]
        result["cpu_baseline"] = cpu_baseline(kc0, vc0, scales, q, meta, args.cpu_seqs)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
