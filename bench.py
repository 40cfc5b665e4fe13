#!/usr/bin/env python
"""Benchmark of the paged-KV attention path on one MI355X.

Headline (the JSON line's `value`): paged decode at serving scale -- 256 sequences,
Lk ~ U[1024, 8192], 16 q / 8 kv heads, head_dim 128, bf16, 256-key blocks from a
shuffled pool. One step is one Attention.forward in decode mode: store_kvcache of
the 256 new tokens, then paged decode attention over all 256 sequences. `value` is
the KV bytes the step must read (sum Lk * 2 * 2048 B) divided by the measured step
time, in GB/s; all inputs are resident in HBM before the timed region starts.

`roofline` is the decode attention call alone, timed per launch with HIP events on
the stream it is launched on. `cpu_baseline` is the CPU oracle (torch on all host
cores) on a bounded sample of the same workload. `kernels` reports every other
configuration (store, mixed chunked prefill + decode, shared-prefix decode, the fused
q/k norm + RoPE + store producer). `e2e` is the serving configuration: offline continuous
batching of 256 requests on a random-init Qwen3-0.6B-geometry model (greedy, ignore_eos),
output tokens per second of generate() (the reference's bench.py:67-72 formula).

    python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--no-cpu-baseline] [--no-e2e]
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT / "nano-vllm-diy_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "paged decode attn KV GB/s (% HBM peak) + e2e gen tok/s, Qwen3-0.6B shape"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
SCALE = 128 ** -0.5


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


_FLUSH = None


def flush_caches():
    """Read 512 MiB so no K/V line of the previous launch is still in L2 or the 256 MB
    Infinity Cache (in a real step the 27 other layers' KV pass through in between). A
    read leaves clean lines, so the timed kernel pays no write-back for the flush."""
    import torch

    global _FLUSH
    if _FLUSH is None:
        _FLUSH = torch.ones(128 << 20, dtype=torch.float32, device="cuda")
    _FLUSH.sum()


def timed_launches(fn, reps: int, warmup: int = 3, cold: bool = True):
    """Mean and median GPU time (ms) of fn() measured with events on the current stream;
    cold=True flushes the caches before every launch (outside the timed interval)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        if cold:
            flush_caches()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    ts = [a.elapsed_time(b) for a, b in evs]
    return statistics.fmean(ts), statistics.median(ts)


def attention_call(w, sub=None, shared: bool = True):
    """Closure running the path's attention op on workload w, or on a sub-batch of it, as
    Attention.forward runs it: the batch's shared-prefix length from its block reference
    counts (what an engine passes) is the cache hint and, when above 0, selects the
    shared-prefix decode path (shared=False keeps the plain split-K path)."""
    import pagedkv

    q, cu_q, cu_k, bt, mq, mk = (w.q, w.cu_seqlens_q, w.cu_seqlens_k, w.block_tables,
                                 w.max_seqlen_q, w.max_seqlen_k) if sub is None else sub
    hint = w.shared_prefix_keys
    sp = hint if shared and hint > 0 else None
    out = pagedkv.varlen_attention(q, w.k_cache, w.v_cache, cu_q, cu_k, mq, mk, SCALE, True, bt,
                                   cached_prefix_keys=hint, shared_prefix_keys=sp)

    def fn():
        pagedkv.varlen_attention(q, w.k_cache, w.v_cache, cu_q, cu_k, mq, mk, SCALE, True, bt, out=out,
                                 cached_prefix_keys=hint, shared_prefix_keys=sp)
    return fn


def sub_batch(w, keep):
    """(q, cu_seqlens_q, cu_seqlens_k, block_tables, max_q, max_k) of the sequences i with keep(i)."""
    import itertools

    import torch

    ids = [i for i in range(len(w.q_lens)) if keep(i)]
    cu_q = w.cu_seqlens_q.cpu().tolist()
    rows = [r for i in ids for r in range(cu_q[i], cu_q[i + 1])]
    dev = w.q.device
    q = w.q.index_select(0, torch.tensor(rows, dtype=torch.long, device=dev))
    lq = [w.q_lens[i] for i in ids]
    lk = [w.k_lens[i] for i in ids]
    cq = torch.tensor([0, *itertools.accumulate(lq)], dtype=torch.int32, device=dev)
    ck = torch.tensor([0, *itertools.accumulate(lk)], dtype=torch.int32, device=dev)
    bt = w.block_tables.index_select(0, torch.tensor(ids, dtype=torch.long, device=dev)).contiguous()
    return q, cq, ck, bt, max(lq), max(lk)


def _host_sub_batch(w, ids):
    """CPU copies of what the oracle needs for sequences `ids` of w: only the blocks they
    read (renumbered), their query / new K / V rows, slots, lengths and block tables."""
    import itertools
    import math

    import torch

    bt = w.block_tables.cpu()
    nblk = {b: math.ceil(w.k_lens[b] / 256) for b in ids}
    blocks = sorted({int(x) for b in ids for x in bt[b, :nblk[b]].tolist()})
    remap = {old: new for new, old in enumerate(blocks)}
    idx = torch.tensor(blocks, dtype=torch.long, device=w.k_cache.device)
    kc0 = w.k_cache.index_select(0, idx).cpu()
    vc0 = w.v_cache.index_select(0, idx).cpu()
    bt_sub = torch.full((len(ids), max(nblk.values())), -1, dtype=torch.int32)
    for j, b in enumerate(ids):
        bt_sub[j, :nblk[b]] = torch.tensor([remap[int(x)] for x in bt[b, :nblk[b]].tolist()], dtype=torch.int32)
    cu = w.cu_seqlens_q.cpu().tolist()
    rows = [r for b in ids for r in range(cu[b], cu[b + 1])]
    ridx = torch.tensor(rows, dtype=torch.long, device=w.q.device)
    slots = w.slot_mapping.cpu()[rows]
    new_slots = torch.tensor([-1 if int(x) < 0 else remap[int(x) // 256] * 256 + int(x) % 256 for x in slots],
                             dtype=torch.int32)
    q, k, v = (t.index_select(0, ridx).cpu() for t in (w.q, w.k, w.v))
    cu_q = torch.tensor([0, *itertools.accumulate(w.q_lens[b] for b in ids)], dtype=torch.int32)
    cu_k = torch.tensor([0, *itertools.accumulate(w.k_lens[b] for b in ids)], dtype=torch.int32)
    return q, k, v, kc0, vc0, new_slots, cu_q, cu_k, bt_sub


def cpu_oracle_time(w, ids, reps: int = 3, store_only: bool = False) -> float:
    """Median wall time (s) of the oracle (CPU torch, all host threads) running Attention.forward
    on sequences `ids` of w: store of their new K/V rows, then paged attention."""
    import torch

    import oracle  # CPU baseline leg only

    torch.set_num_threads(os.cpu_count() or 1)
    q, k, v, kc0, vc0, slots, cu_q, cu_k, bt = _host_sub_batch(w, ids)
    times = []
    for _ in range(reps):
        kc, vc = kc0.clone(), vc0.clone()
        t0 = time.perf_counter()
        oracle.store_kvcache(k, v, kc, vc, slots)
        if not store_only:
            oracle.varlen_attention(q, kc, vc, cu_q, cu_k, SCALE, True, bt)
        times.append(time.perf_counter() - t0)
    return statistics.median(times)


def cpu_baseline_decode(w, max_seqs: int, reps: int = 3):
    """Oracle (CPU torch, all cores) on the first max_seqs sequences of w: store + attention."""
    import torch

    ids = list(range(min(max_seqs, len(w.q_lens))))
    med = cpu_oracle_time(w, ids, reps)
    kv_bytes = sum(w.k_lens[b] * 2 * 2048 for b in ids)
    return {"value": round(kv_bytes / med / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"CPU oracle (torch fp32 on {torch.get_num_threads()} threads, store + paged decode) "
                      f"on {len(ids)} of the 256 sequences ({kv_bytes / 1e9:.3f} GB of KV), "
                      f"median of {reps} runs = {med:.3f} s"}


def cpu_baselines(dev, gpu_kernels: dict | None, reps: int = 3) -> dict:
    """The oracle on the host cores for every other configuration, on the same seeded inputs
    as the GPU measurements, each the full batch of its configuration (median of `reps`
    runs): algorithmic GB/s (store, decode) or GFLOP/s (chunked prefill), and the GPU's
    rate over the CPU's where the GPU figure was measured in this run."""
    import torch

    from pagedkv.workloads import make_workload

    res = {"cores": torch.get_num_threads(), "kind": "port",
           "what": "oracle/paged_kv.py (torch fp32) on all host threads: store of the new K/V rows, then "
                   "paged attention, as Attention.forward; median of %d runs" % reps}
    g = gpu_kernels or {}

    def entry(name, sec, work, unit, gpu_key=None, gpu_field=None):
        rate = work / sec / 1e9
        e = {"s": round(sec, 4), unit: round(rate, 3)}
        if gpu_key in g and gpu_field in g[gpu_key]:
            e["gpu_over_cpu"] = round(g[gpu_key][gpu_field] / rate, 1)
        res[name] = e

    ws = make_workload("cfg1_store", dev)
    entry("cfg1_store", cpu_oracle_time(ws, [0], reps, store_only=True), ws.store_bytes(), "GB/s",
          "cfg1_store", "GB/s")
    del ws
    wd = make_workload("cfg1_decode", dev)
    entry("cfg1_decode", cpu_oracle_time(wd, list(range(len(wd.q_lens))), reps), wd.decode_kv_bytes(), "GB/s",
          "cfg1_forward_step", "GB/s")
    del wd
    w3 = make_workload("cfg3", dev)
    dec = [i for i, lq in enumerate(w3.q_lens) if lq == 1]
    pre = [i for i, lq in enumerate(w3.q_lens) if lq > 1]
    entry("cfg3_decode", cpu_oracle_time(w3, dec, reps), w3.decode_kv_bytes(), "GB/s", "cfg3_decode", "GB/s")
    entry("cfg3_prefill", cpu_oracle_time(w3, pre, reps), w3.prefill_flops(), "GFLOP/s", "cfg3_prefill", "TFLOP/s")
    if "gpu_over_cpu" in res["cfg3_prefill"]:        # TFLOP/s over GFLOP/s
        res["cfg3_prefill"]["gpu_over_cpu"] = round(res["cfg3_prefill"]["gpu_over_cpu"] * 1000, 1)
    del w3
    w4 = make_workload("cfg4", dev)
    sec = cpu_oracle_time(w4, list(range(len(w4.q_lens))), reps)
    entry("cfg4_decode", sec, w4.decode_kv_bytes(), "GB/s", "cfg4_decode", "logical_GB/s")
    res["cfg4_decode"]["unique_GB/s"] = round(w4.decode_unique_kv_bytes() / sec / 1e9, 3)
    res["cfg4_decode"]["unique_block_GB/s"] = round(w4.decode_unique_block_bytes() / sec / 1e9, 3)
    return res


def prefill_probe(dev) -> int:
    """5 calls each of cfg3's prefill part, the prefill_steady batch and the dense 16384-token
    prompt batch (counter passes)."""
    import torch

    from pagedkv.workloads import make_workload

    for name in ("cfg3", "prefill_steady"):
        w = make_workload(name, dev)
        call = attention_call(w, sub_batch(w, lambda i: w.q_lens[i] > 1)) if name == "cfg3" else attention_call(w)
        for _ in range(5):
            call()
        torch.cuda.synchronize()
        log(f"[bench] prefill probe: {name} done")
        del w
    fn, _, _ = dense_prefill_call(dev)
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    log("[bench] prefill probe: dense done")
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-e2e", action="store_true", help="skip the end-to-end serving run")
    ap.add_argument("--e2e-only", action="store_true",
                    help="only the end-to-end serving run (prints its JSON object), for profiling")
    ap.add_argument("--cpu-seqs", type=int, default=256, help="sequences in the CPU-baseline sample")
    ap.add_argument("--prefill-probe", action="store_true",
                    help="only run 5 cfg3 prefill calls and 5 prefill_steady calls, for rocprofv3 --pmc passes")
    ap.add_argument("--pmc-probe", nargs="?", const="cfg2", default=None,
                    choices=("cfg2", "cfg4", "decode_serve", "store_16384", "cfg2_tp2", "cfg2_tp8"),
                    help="only run 5 calls of one workload (default: the cfg2 decode call) and 5 copies "
                         "of 1 GiB (the counter calibration), for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE "
                         "passes")
    ap.add_argument("--no-pmc", action="store_true",
                    help="take roofline.traffic from profiles/traffic.json instead of measuring it")
    ap.add_argument("--call-probe", default=None,
                    help="only run 5 cold-cache calls of each named workload (comma-separated: cfg2, "
                         "cfg2_tp2/4/8, cfg4, decode_serve, cfg3, cfg3_prefill, prefill_steady, dense_prefill, "
                         "store_16384), one at a time, for a rocprofv3 --kernel-trace of each call's launches")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the paged-KV path is not sharded across GPUs "
              f"(asked for --gpus {args.gpus}); run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import pagedkv
    from pagedkv.workloads import make_workload

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.e2e_only:
        print(json.dumps(run_e2e(dev)), flush=True)
        return 0
    if args.prefill_probe:
        return prefill_probe(dev)
    if args.pmc_probe:
        return pmc_probe(dev, args.pmc_probe)
    if args.call_probe:
        return call_probe(dev, args.call_probe.split(","))
    log("[bench] building cfg2 (256 seqs, Lk ~ U[1024, 8192]) on the GPU")
    w = make_workload("cfg2", dev)
    kv_bytes = w.decode_kv_bytes()
    store_bytes = w.store_bytes()
    ctx = w.ctx
    out = torch.empty_like(w.q)
    pagedkv.reserve_workspace(len(w.q_lens), 16, 128, 1, w.max_seqlen_k, dev)

    def store():
        pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, ctx.slot_mapping)

    def attend():
        pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                 ctx.max_seqlen_q, ctx.max_seqlen_k, SCALE, True, ctx.block_tables, out=out,
                                 cached_prefix_keys=ctx.cached_prefix_keys)

    log(f"[bench] warmup {args.warmup} steps")
    for _ in range(args.warmup):
        store()
        attend()
    torch.cuda.synchronize()

    log(f"[bench] timing {args.steps} steps")
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for a, b in evs:
        store()
        a.record()
        attend()
        b.record()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    attn_ms = [a.elapsed_time(b) for a, b in evs]
    ms_per_step = elapsed * 1e3 / args.steps
    value = kv_bytes / (elapsed / args.steps) / 1e9
    attn_mean = statistics.fmean(attn_ms)
    achieved = kv_bytes / (attn_mean * 1e-3) / 1e9
    log(f"[bench] step {ms_per_step:.3f} ms, decode call {attn_mean:.3f} ms -> {achieved:.1f} GB/s")

    # HBM bytes per decode call on this workload: two rocprofv3 --pmc passes (FETCH_SIZE,
    # WRITE_SIZE) run now, in child processes; if the profiler is missing or a pass fails, the
    # value recorded in profiles/ by the same passes
    traffic, traffic_source = None, None
    if not args.no_pmc:
        log("[bench] HBM traffic of the decode call: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes")
        traffic, traffic_source = pmc_traffic("cfg2")
    if traffic is None:
        tfile = ROOT / "profiles" / "traffic.json"
        if tfile.exists():
            traffic = json.loads(tfile.read_text()).get("cfg2_decode_call_hbm_bytes")
            traffic_source = (f"profiles/traffic.json (recorded by the same passes; a pass in this run: "
                              f"{traffic_source or 'skipped'})")
    log(f"[bench] traffic {traffic} B per call ({traffic_source})")

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
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "paged decode, 256 seqs, Lk~U[1024,8192], 16q/8kv heads, head_dim 128, "
                        "block 256, shuffled pool; step = store 256 tokens + decode attention",
            "num_seqs": len(w.q_lens),
            "kv_bytes_per_step": kv_bytes,
            "store_bytes_per_step": store_bytes,
            "num_blocks": int(w.k_cache.shape[0]),
            "cached_prefix_keys": ctx.cached_prefix_keys,
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "pk_varlen_attention decode call = decode_split_kernel + decode_combine_kernel",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_over_algorithmic": round(traffic / kv_bytes, 4) if traffic else None,
            "traffic_source": traffic_source,
            "launch_ms_mean": round(attn_mean, 4),
            "launch_ms_median": round(statistics.median(attn_ms), 4),
        },
    }

    if not args.no_extra:
        result["kernels"] = extra_configs(dev, w)
    del w
    torch.cuda.empty_cache()

    if not args.no_e2e:
        log("[bench] e2e: 256 requests on a random-init Qwen3-0.6B")
        result["e2e"] = run_e2e(dev)
        torch.cuda.empty_cache()

    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle on host cores)")
        wc = make_workload("cfg2", dev)
        result["cpu_baseline"] = cpu_baseline_decode(wc, args.cpu_seqs)
        del wc
        log("[bench] CPU baselines of the other configurations")
        result["cpu_baselines"] = cpu_baselines(dev, result.get("kernels"))
    print(json.dumps(result), flush=True)
    return 0


def run_e2e(dev, seed: int = 5) -> dict:
    """Offline continuous batching, the serving configuration: 256 requests, prompt ids
    U[0, 151936), prompt and output lengths U[100, 1024], ignore_eos, greedy, block 256,
    16384-token budget. The timed region is generate() (requests added inside it, as in the
    reference's bench.py:67-72); model init and graph capture are outside."""
    import torch

    from pagedkv.engine import LLMEngine
    from pagedkv.qwen3 import Qwen3Config
    from pagedkv.workloads import serving_requests

    cfg = Qwen3Config()
    t0 = time.perf_counter()
    eng = LLMEngine(cfg, device=dev, num_blocks=2048, block_size=256,
                    max_num_batched_tokens=16384, seed=seed)
    torch.cuda.synchronize()
    init_s = time.perf_counter() - t0
    prompts, max_tokens = serving_requests(seed, 256, cfg.vocab_size)
    outs, st = eng.generate(prompts, max_tokens, ignore_eos=True)
    assert [len(o) for o in outs] == max_tokens
    res = {"tok_per_s": round(st.tok_per_s, 1), "output_tokens": st.output_tokens,
           "wall_s": round(st.wall_s, 3), "steps": st.steps, "decode_steps": st.decode_steps,
           "prefill_steps": st.prefill_steps, "prefill_tokens": st.prefill_tokens,
           "init_and_capture_s": round(init_s, 2),
           "workload": "256 requests, prompt ids U[0,151936), prompt/output lengths U[100,1024], "
                       "ignore_eos, greedy; random-init Qwen3-0.6B geometry (28 layers, hidden "
                       "1024, 16q/8kv heads, head_dim 128, FFN 3072, vocab 151936), bf16, "
                       "block 256, 16384-token budget, 128 live sequences"}
    log(f"[bench] e2e {res['tok_per_s']} tok/s ({st.output_tokens} tokens in {st.wall_s:.2f} s)")
    del eng
    return res


def pmc_probe(dev, name: str) -> int:
    """5 calls of one workload's path, then 5 device copies of exactly 1 GiB: the copy gives
    the factor between what FETCH_SIZE / WRITE_SIZE report and the bytes moved. Workloads:
    cfg2 / cfg2_tp2 / cfg2_tp8 (the decode call at the full heads or a tensor-parallel
    rank's share), cfg4 (the shared-prefix call), decode_serve (128 sequences of 100-2048
    keys: the flat grid), store_16384 (store_kvcache of a 16384-token prefill step)."""
    import torch

    from pagedkv.workloads import TP_HEADS, make_workload

    if name == "store_16384":
        fn, nbytes = store_call(dev, 16384)
        info = {"store_bytes": nbytes}
    else:
        base, _, tp = name.partition("_tp")
        w = make_workload(base, dev, heads=TP_HEADS[int(tp) if tp else 1])
        fn = attention_call(w)
        info = {"kv_bytes": w.decode_kv_bytes()}
        if base == "cfg4":
            info["unique_bytes"] = w.decode_unique_kv_bytes()
    for _ in range(5):
        fn()
    src = torch.ones(1 << 29, dtype=torch.int16, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"pmc_probe": name, **info, "copy_bytes": 1 << 30}), flush=True)
    return 0


def pmc_traffic(name: str, timeout_s: float = 150.0):
    """HBM bytes per call of one workload's path, measured now: rocprofv3 --pmc FETCH_SIZE,
    then WRITE_SIZE, each over a child `bench.py --pmc-probe NAME` (6 calls of the path, then
    5 device copies of 1 GiB). Each counter's per-dispatch value (KiB) for the path's kernels
    is scaled by the factor that makes it read 1 GiB for the copies, and the per-dispatch
    means of the path's kernels are summed (one launch of each per call). Returns
    (bytes, how) or (None, why not). A pass that does not finish in timeout_s is killed with
    its process group."""
    import csv
    import glob
    import shutil
    import signal
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if exe is None:
        return None, "rocprofv3 not found"
    scaled, factors = {}, {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        with tempfile.TemporaryDirectory(dir="/tmp") as d:
            cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", d, "-o", "p", "--",
                   sys.executable, str(ROOT / "bench.py"), "--pmc-probe", name]
            try:
                p = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp"), stdout=subprocess.DEVNULL,
                                     stderr=subprocess.DEVNULL, start_new_session=True)
            except OSError as e:
                return None, f"{counter} pass not started ({e})"
            try:
                p.wait(timeout=timeout_s)
            except subprocess.TimeoutExpired:
                os.killpg(p.pid, signal.SIGKILL)
                p.wait()
                return None, f"{counter} pass killed after {timeout_s:.0f} s"
            # (the profiler may exit non-zero after writing whole results: the CSV decides)
            files = glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)
            if not files:
                return None, f"{counter} pass wrote no counters (exit {p.returncode})"
            with open(files[0]) as f:
                got = pmc_call_bytes(csv.DictReader(f), counter)
        if got is None:
            return None, f"{counter} pass: no path or copy dispatches in the counters"
        scaled[counter], factors[counter] = got
    total = int(round(scaled["FETCH_SIZE"] + scaled["WRITE_SIZE"]))
    return total, (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes in this run over bench.py --pmc-probe "
                   f"{name}: {scaled['FETCH_SIZE']:.0f} B read + {scaled['WRITE_SIZE']:.0f} B written per call "
                   f"(factors {factors['FETCH_SIZE']} / {factors['WRITE_SIZE']} from the 1 GiB copies)")


def pmc_call_bytes(rows, counter: str):
    """(bytes per call, factor) from rocprofv3 counter rows of a --pmc-probe run: the mean
    per-dispatch value (KiB) of each library kernel, summed over the kernels, times the factor
    that makes the large device copies (the probe's 1 GiB copies: the copy dispatches of at
    least half the largest one's count) read or write 1 GiB. None without such rows."""
    per_kernel, copies = {}, []
    for r in rows:
        if r.get("Counter_Name") != counter:
            continue
        v = float(r["Counter_Value"])
        k = r["Kernel_Name"]
        if "pk::" in k:
            per_kernel.setdefault(k, []).append(v)
        elif "copyBuffer" in k:
            copies.append(v)
    big = [v for v in copies if v >= 0.5 * max(copies)] if copies else []
    if not per_kernel or not big or statistics.median(big) <= 0:
        return None
    factor = (1 << 30) / (statistics.median(big) * 1024)
    return sum(statistics.fmean(v) for v in per_kernel.values()) * 1024 * factor, round(factor, 4)


def call_probe(dev, names) -> int:
    """Per workload: one warm call, then 5 calls each after a cache flush and followed by a
    synchronize, so a kernel trace shows every launch of one call (and the gaps between them)
    on its own."""
    import torch

    from pagedkv.workloads import TP_HEADS, make_workload

    for name in names:
        if name == "store_16384":
            fn = store_call(dev, 16384)[0]
        elif name == "dense_prefill":
            fn = dense_prefill_call(dev)[0]
        elif name == "cfg3_prefill":
            w = make_workload("cfg3", dev)
            fn = attention_call(w, sub_batch(w, lambda i: w.q_lens[i] > 1))
        else:
            base, _, tp = name.partition("_tp")
            fn = attention_call(make_workload(base, dev, heads=TP_HEADS[int(tp) if tp else 1]))
        fn()
        torch.cuda.synchronize()
        for _ in range(5):
            flush_caches()
            torch.cuda.synchronize()
            fn()
            torch.cuda.synchronize()
        print(json.dumps({"call_probe": name, "calls": 5}), flush=True)
    return 0


def producer_call(dev, n: int, seed: int = 6):
    """Fused q/k norm + RoPE + K/V store for n tokens of the Qwen3-0.6B attention geometry.

    Algorithmic bytes per token: the fused qkv row (Hq + 2 Hkv) D 2 B read, q (Hq D 2 B)
    and the K and V cache rows (2 Hkv D 2 B) written, the position (8 B), the slot (4 B)
    and the token's fp32 cos/sin row (D 4 B) read.
    """
    import torch

    import pagedkv
    from pagedkv.workloads import BLOCK_SIZE, HEAD_DIM, HKV, HQ

    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn(n, (HQ + 2 * HKV) * HEAD_DIM, generator=g, device=dev).to(torch.bfloat16)
    cs = pagedkv.rope_cos_sin(40960, HEAD_DIM, 1000000.0, dev)
    pos = torch.randint(0, 40960, (n,), generator=g, device=dev)
    nb = (n + BLOCK_SIZE - 1) // BLOCK_SIZE * 2
    kc = torch.empty(nb, BLOCK_SIZE, HKV, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)
    slots = torch.randperm(nb * BLOCK_SIZE, generator=g, device=dev)[:n].to(torch.int32)
    qw = torch.ones(HEAD_DIM, dtype=torch.bfloat16, device=dev)
    kw = torch.ones(HEAD_DIM, dtype=torch.bfloat16, device=dev)
    q_out = torch.empty(n, HQ, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    per_token = (HQ + 2 * HKV) * HEAD_DIM * 2 + HQ * HEAD_DIM * 2 + 2 * HKV * HEAD_DIM * 2 + 8 + 4 + HEAD_DIM * 4

    def fn():
        pagedkv.qk_norm_rope_store(qkv, pos, cs, HQ, HKV, HEAD_DIM, qw, kw, 1e-6, kc, vc, slots,
                                   q_out=q_out)
    return fn, n * per_token


def store_call(dev, n: int, seed: int = 8):
    """store_kvcache of n new tokens as a prefill step of the serving engine issues it: k
    contiguous, v the strided view of the fused qkv row (row stride 4096 elements,
    qwen3.py:80-88), slots filling whole cache blocks popped from a shuffled pool. Bytes:
    4 n R + 4 n (read K and V rows, write them, read the slot)."""
    import torch

    import pagedkv
    from pagedkv.workloads import BLOCK_SIZE, HEAD_DIM, HKV, HQ, ROW_BYTES

    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn(n, (HQ + 2 * HKV) * HEAD_DIM, generator=g, device=dev).to(torch.bfloat16)
    k = qkv[:, HQ * HEAD_DIM:(HQ + HKV) * HEAD_DIM].reshape(n, HKV, HEAD_DIM).clone()
    v = qkv[:, (HQ + HKV) * HEAD_DIM:].view(n, HKV, HEAD_DIM)
    nb = 2 * ((n + BLOCK_SIZE - 1) // BLOCK_SIZE)
    blocks = torch.randperm(nb, generator=torch.Generator().manual_seed(seed))[:nb // 2]
    slots = (blocks.repeat_interleave(BLOCK_SIZE) * BLOCK_SIZE +
             torch.arange(BLOCK_SIZE).repeat(nb // 2))[:n].to(torch.int32).to(dev)
    kc = torch.empty(nb, BLOCK_SIZE, HKV, HEAD_DIM, dtype=torch.bfloat16, device=dev)
    vc = torch.empty_like(kc)

    def fn():
        pagedkv.store_kvcache(k, v, kc, vc, slots)
    return fn, 4 * n * ROW_BYTES + 4 * n


def dense_prefill_call(dev, seed: int = 5, budget: int = 16384):
    """The serving run's first prefill step in dense (flat) mode, as the reference runs a
    batch of fresh prompts (block_tables None, cu_seqlens_k == cu_seqlens_q,
    model_runner.py:211-212): the first prompts of the serving workload up to the
    16384-token budget, the last one cut to fit (a chunk with no cached keys is still
    fresh). q (N, 16, 128), k contiguous, v the strided qkv view. Returns the call, its
    causal flops and the prompt lengths."""
    import itertools

    import torch

    import pagedkv
    from pagedkv.workloads import HEAD_DIM, HKV, HQ, serving_requests

    prompts, _ = serving_requests(seed, 256)
    lens, tot = [], 0
    for p in prompts:
        take = min(len(p), budget - tot)
        if take <= 0:
            break
        lens.append(take)
        tot += take
    g = torch.Generator(device=dev).manual_seed(seed)
    qkv = torch.randn(tot, (HQ + 2 * HKV) * HEAD_DIM, generator=g, device=dev).to(torch.bfloat16)
    q = qkv[:, :HQ * HEAD_DIM].reshape(tot, HQ, HEAD_DIM).clone()
    k = qkv[:, HQ * HEAD_DIM:(HQ + HKV) * HEAD_DIM].reshape(tot, HKV, HEAD_DIM).clone()
    v = qkv[:, (HQ + HKV) * HEAD_DIM:].view(tot, HKV, HEAD_DIM)
    cu = torch.tensor([0, *itertools.accumulate(lens)], dtype=torch.int32, device=dev)
    out = torch.empty_like(q)
    flops = sum(4 * HQ * HEAD_DIM * (lq * (lq + 1) // 2) for lq in lens)

    def fn():
        pagedkv.varlen_attention(q, k, v, cu, cu, max(lens), max(lens), SCALE, True, None, out=out)
    return fn, flops, lens


def linear_calls(dev, rows: int, seed: int = 7):
    """The four decode-step projections of one Qwen3-0.6B decoder layer on `rows` tokens,
    each with its fused epilogue: qkv (store), o + residual RMSNorm, gate/up + SiLU * mul,
    down + residual RMSNorm. Algorithmic bytes per call: the weight (n_out x k bf16), x,
    the outputs and, for the norm epilogue, the residual read and written."""
    import torch

    import pagedkv

    g = torch.Generator(device=dev).manual_seed(seed)
    H, Q, I, QKV = 1024, 2048, 3072, 4096
    rnd = lambda *shape, s=1.0: (torch.randn(*shape, generator=g, device=dev) * s).to(torch.bfloat16)
    x_h, x_q, x_i = rnd(rows, H), rnd(rows, Q), rnd(rows, I)
    res, nw = rnd(rows, H), torch.ones(H, dtype=torch.bfloat16, device=dev)
    w_qkv, w_o, w_gu, w_d = rnd(QKV, H, s=0.02), rnd(H, Q, s=0.02), rnd(2 * I, H, s=0.02), rnd(H, I, s=0.02)
    y_qkv = torch.empty(rows, QKV, dtype=torch.bfloat16, device=dev)
    y_i = torch.empty(rows, I, dtype=torch.bfloat16, device=dev)
    y_h, r_h = torch.empty(rows, H, dtype=torch.bfloat16, device=dev), torch.empty(rows, H, dtype=torch.bfloat16,
                                                                                   device=dev)
    b = 2
    return [
        ("qkv", lambda: pagedkv.linear(x_h, w_qkv, out=y_qkv), b * (QKV * H + rows * (H + QKV))),
        ("o_norm", lambda: pagedkv.linear_add_rmsnorm(x_q, w_o, res, nw, 1e-6, out=y_h, residual_out=r_h),
         b * (H * Q + rows * (Q + 4 * H) + H)),
        ("gate_up_silu", lambda: pagedkv.linear_silu_mul(x_h, w_gu, out=y_i), b * (2 * I * H + rows * (H + I))),
        ("down_norm", lambda: pagedkv.linear_add_rmsnorm(x_i, w_d, res, nw, 1e-6, out=y_h, residual_out=r_h),
         b * (H * I + rows * (I + 4 * H) + H)),
    ]


def extra_configs(dev, w2):
    """Per-kernel measurements of the other configurations (events, mean of 20 launches)."""
    import torch

    import pagedkv
    from pagedkv.workloads import make_workload

    res = {}
    # cfg2 store of the 256 new tokens
    ms, _ = timed_launches(lambda: pagedkv.store_kvcache(w2.k, w2.v, w2.k_cache, w2.v_cache, w2.slot_mapping), 20)
    res["cache_state"] = "cold: 512 MiB read before every timed launch"
    res["cfg2_store"] = {"ms": round(ms, 5), "GB/s": round(w2.store_bytes() / ms / 1e6, 1)}

    # the store at a prefill step's size (the serving run's 16384-token budget)
    fn, nbytes = store_call(dev, 16384)
    ms, _ = timed_launches(fn, 20)
    res["store_16384"] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
                          "frac": round(nbytes / ms / 1e6 / HBM_PEAK_GBS, 4), "bytes": nbytes}

    log("[bench] cfg1")
    ws = make_workload("cfg1_store", dev)
    ms, _ = timed_launches(lambda: pagedkv.store_kvcache(ws.k, ws.v, ws.k_cache, ws.v_cache, ws.slot_mapping), 20)
    res["cfg1_store"] = {"ms": round(ms, 5), "GB/s": round(ws.store_bytes() / ms / 1e6, 1)}
    wd = make_workload("cfg1_decode", dev)
    ms, _ = timed_launches(attention_call(wd), 20)
    res["cfg1_decode"] = {"ms": round(ms, 5), "GB/s": round(wd.decode_kv_bytes() / ms / 1e6, 1)}
    # the drop-in's decode step (store + decode): Attention.forward does both in one launch
    fwd = pagedkv.Attention(128, 16, 8, SCALE)
    fwd.k_cache, fwd.v_cache = wd.k_cache, wd.v_cache
    ms, _ = timed_launches(lambda: fwd(wd.q, wd.k, wd.v, wd.ctx), 20)
    res["cfg1_forward_step"] = {"ms": round(ms, 5), "GB/s": round(wd.decode_kv_bytes() / ms / 1e6, 1)}

    log("[bench] cfg3")
    w3 = make_workload("cfg3", dev)
    ms, _ = timed_launches(attention_call(w3), 20)
    res["cfg3_mixed"] = {"ms": round(ms, 5)}
    n_dec = sum(1 for lq in w3.q_lens if lq == 1)
    ms_p, _ = timed_launches(attention_call(w3, sub_batch(w3, lambda i: w3.q_lens[i] > 1)), 20)
    fl = w3.prefill_flops()
    res["cfg3_prefill"] = {"ms": round(ms_p, 5), "TFLOP/s": round(fl / ms_p / 1e9, 2),
                           "mfma_frac": round(fl / ms_p / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4), "flops": fl}
    ws_ = make_workload("prefill_steady", dev)
    ms_s, _ = timed_launches(attention_call(ws_), 10)
    fl_s = ws_.prefill_flops()
    res["prefill_steady"] = {"ms": round(ms_s, 5), "TFLOP/s": round(fl_s / ms_s / 1e9, 2),
                             "mfma_frac": round(fl_s / ms_s / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4), "flops": fl_s,
                             "batch": "16 chunks of 1024 tokens over 4096-token cached prefixes"}
    del ws_
    ms_d, _ = timed_launches(attention_call(w3, sub_batch(w3, lambda i: w3.q_lens[i] == 1)), 20)
    kvb = w3.decode_kv_bytes()
    res["cfg3_decode"] = {"ms": round(ms_d, 5), "GB/s": round(kvb / ms_d / 1e6, 1), "seqs": n_dec}

    fn, fl_d, lens = dense_prefill_call(dev)
    ms_dp, _ = timed_launches(fn, 20)
    res["dense_prefill_16384"] = {"ms": round(ms_dp, 5), "TFLOP/s": round(fl_d / ms_dp / 1e9, 2),
                                  "mfma_frac": round(fl_d / ms_dp / 1e9 / MFMA_BF16_PEAK_TFLOPS, 4),
                                  "flops": fl_d, "batch": f"{len(lens)} fresh prompts, {sum(lens)} tokens "
                                  "(the serving run's first prefill step), flat K/V, causal"}

    log("[bench] decode at one tensor-parallel rank's share of the heads")
    from pagedkv.workloads import TP_HEADS
    for tp in (2, 4, 8):
        hq, hkv = TP_HEADS[tp]
        wt = make_workload("cfg2", dev, heads=(hq, hkv))
        ms, _ = timed_launches(attention_call(wt), 20)
        gbs = wt.decode_kv_bytes() / ms / 1e6
        res[f"cfg2_tp{tp}"] = {"ms": round(ms, 5), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                               "heads": f"{hq}q/{hkv}kv", "kv_bytes": wt.decode_kv_bytes()}
        del wt
        torch.cuda.empty_cache()

    wv = make_workload("decode_serve", dev)
    ms, _ = timed_launches(attention_call(wv), 20)
    res["decode_serve_128"] = {"ms": round(ms, 5), "GB/s": round(wv.decode_kv_bytes() / ms / 1e6, 1),
                               "frac": round(wv.decode_kv_bytes() / ms / 1e6 / HBM_PEAK_GBS, 4),
                               "kv_bytes": wv.decode_kv_bytes(),
                               "batch": "128 sequences of U[100, 2048] keys (the serving run's decode steps): "
                                        "flat grid + combine"}
    del wv

    log("[bench] producer")
    for n in (256, 16384):
        fn, nbytes = producer_call(dev, n)
        ms, _ = timed_launches(fn, 20)
        res[f"producer_{n}"] = {"ms": round(ms, 5), "GB/s": round(nbytes / ms / 1e6, 1),
                                "bytes": nbytes}

    log("[bench] decode-step linear layers")
    for rows in (1, 128):
        layer = {}
        for name, fn, nbytes in linear_calls(dev, rows):
            ms, _ = timed_launches(fn, 20)
            layer[name] = {"us": round(ms * 1000, 2), "GB/s": round(nbytes / ms / 1e6, 1), "bytes": nbytes}
        res[f"linear_{rows}rows"] = layer

    log("[bench] cfg4")
    w4 = make_workload("cfg4", dev)
    ms, _ = timed_launches(attention_call(w4), 20)
    # unique: (2048 + sum of the suffixes) * 2R, the distinct keys; unique_block: the distinct
    # cache blocks read, whole; logical: sum Lk * 2R, every sequence's keys
    cfg4_bytes = {"unique": w4.decode_unique_kv_bytes(), "unique_block": w4.decode_unique_block_bytes(),
                  "logical": w4.decode_kv_bytes()}

    def cfg4_entry(ms, path):
        e = {"ms": round(ms, 5)}
        for k, b in cfg4_bytes.items():
            e[f"{k}_GB/s"] = round(b / ms / 1e6, 1)
        e["unique_frac"] = round(cfg4_bytes["unique"] / ms / 1e6 / HBM_PEAK_GBS, 4)
        e["path"] = path
        return e
    res["cfg4_decode"] = cfg4_entry(ms, "shared-prefix decode (the 8 shared blocks once per kv head, on MFMA) "
                                        "+ flat grid over the suffixes")
    ms, _ = timed_launches(attention_call(w4, shared=False), 20)
    res["cfg4_decode_plain"] = cfg4_entry(ms, "split-K over every key of every sequence")
    res["cfg4_bytes"] = cfg4_bytes
    return res


if __name__ == "__main__":
    sys.exit(main())
