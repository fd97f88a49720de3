"""Benchmark of the MI355X paged-KV attention path.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20]

Headline workload (one step = one paged decode attention call over the
whole batch, inputs resident in HBM): Qwen3-8B head layout (32 q / 8 kv
heads, d 128, bf16), 64 sequences with context ~ U{512..4096}, 16-token
pages from a seeded permutation.  Four KV pools (> 2 GB total) are rotated
so the 256 MB Infinity Cache cannot hold the working set.

value = algorithmic decode bytes per step (visible K/V rows + q in + o out +
page ids) / measured time per step, in GB/s.  Secondary figures (chunked
prefill TFLOP/s, fused RoPE+append GB/s, DFlash block, mixed step,
long-context decode) are reported under "secondary".
The CPU baseline is the oracle's LibTorch-CPU restatement of the reference's
ATen attention on the same decode batch.

Prints one JSON line on stdout; progress goes to stderr.
"""

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flashengine.cpp_amd")]

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "paged decode attn HBM GB/s (% of 8 TB/s); prefill attn TFLOP/s, Qwen3-8B"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic():
    """HBM bytes per decode step (decode kernel + split-KV merge) from the
    committed rocprofv3 summary of this workload: DRAM read and write
    request counters summed over every channel, used raw (no calibration
    factor); None if the summary is absent."""
    path = os.path.join(ROOT, "profiles", "decode_qwen3_8b_hbm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("decode_step_traffic_bytes"):
            return int(float(line.split("=")[1]))
    return None


def event_block_means_ms(fn, blocks, iters):
    """Mean ms per call of each of `blocks` consecutive blocks of `iters`
    calls, one event between blocks on the current stream (an event marker
    between single launches adds about 2 us to each, so the statistic is
    taken over blocks)."""
    import torch

    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(blocks + 1)]
    ev[0].record()
    for j in range(blocks):
        for i in range(iters):
            fn(j * iters + i)
        ev[j + 1].record()
    torch.cuda.synchronize()
    return [ev[j].elapsed_time(ev[j + 1]) / iters for j in range(blocks)]


def event_time_ms(fn, iters, warmup):
    """Average ms per call of fn() over `iters` calls, timed with events on
    the current stream (the stream the library launches on)."""
    import torch

    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / iters


DECODE_SEED = 2   # context lengths and page permutation of the headline decode batch
POOL_SEED = 1234  # K/V cache contents
Q_SEED = 4321     # query rows


def make_pools(b, n, dev, dtype):
    import torch

    g = torch.Generator(device=dev).manual_seed(POOL_SEED)
    shape = (b.blocks + 1, b.page, b.hkv, 128)
    pools = []
    for _ in range(n):
        kc = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)
        vc = torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)
        pools.append((kc, vc))
    return pools


ROPE_THETA = 1e6  # Qwen3


def make_rope_pools(b, n, dev):
    """Decode pools filled the way the engine fills them: for every context
    token, raw q / k / v ~ N(0,1) (bf16), k and q rotated at the token's
    position with theta 1e6 and k / v written to the token's page slot by
    the fused RoPE + paged append (src/cuda_model.cpp:94-95), the RoPE table
    built on the device (src/cuda_model.cpp:44-47).  Returns the pools and
    the decode query rows: q of each sequence's last token, rotated at
    position len - 1.  Slots outside every sequence (page tails, the dummy
    page) hold zeros and are never read."""
    import torch

    import feattn
    from feattn import workloads as W

    fill = W.Batch(hq=b.hq, hkv=b.hkv, page=b.page, blocks=b.blocks, starts=[0] * b.batch,
                   qlens=list(b.lens), tables=b.tables)
    W.build_metadata(fill)
    rows = fill.rows
    max_pos = max(b.lens)
    table = torch.empty(max_pos, 128, device=dev)
    feattn.rope_table(table, max_pos, 128, ROPE_THETA)
    pos = torch.from_numpy(fill.positions).to(dev)
    slots = torch.from_numpy(fill.slots).to(dev)
    last_rows = torch.tensor([fill.qo[i + 1] - 1 for i in range(b.batch)], device=dev)
    g = torch.Generator(device=dev).manual_seed(POOL_SEED)
    shape = (b.blocks + 1, b.page, b.hkv, 128)
    pools, q_dec = [], None
    for _ in range(n):
        kc = torch.zeros(shape, device=dev, dtype=torch.bfloat16)
        vc = torch.zeros_like(kc)
        q = torch.randn(rows, b.hq, 128, generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn(rows, b.hkv, 128, generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn(rows, b.hkv, 128, generator=g, device=dev).to(torch.bfloat16)
        feattn.rope_append(q, k, v, kc, vc, pos, slots, table, rows, b.hq, b.hkv, 128, True, max_pos,
                           b.cache_slots)
        if q_dec is None:
            q_dec = q[last_rows].contiguous()
        del q, k, v
        pools.append((kc, vc))
    torch.cuda.synchronize()
    return pools, q_dec


def attn_setup(b, dev, dtype, causal, npools):
    import torch

    import feattn

    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), dtype == torch.bfloat16,
                       b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    pools = make_pools(b, npools, dev, dtype)
    gq = torch.Generator(device=dev).manual_seed(Q_SEED)
    q = torch.randn(b.rows, b.hq, 128, generator=gq, device=dev).to(dtype)
    out = torch.empty_like(q)
    lse = torch.empty(b.rows, b.hq, device=dev)

    def step(i):
        kc, vc = pools[i % len(pools)]
        plan.run(q, kc, vc, out, causal=causal, lse=lse)

    return plan, step


def decode_headline(steps, warmup, dev):
    """The headline step: one attention call over the decode batch, pools
    rotated.  Returns the batch, the mean ms per step of the timed region
    (value), the median over 10 further blocks of `steps` steps of each
    block's mean, and the algorithmic bytes per step."""
    import torch

    import feattn
    from feattn import workloads as W

    b = W.qwen3_8b_decode(seed=DECODE_SEED)
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    pools, q = make_rope_pools(b, 4, dev)
    out = torch.empty_like(q)
    lse = torch.empty(b.rows, b.hq, device=dev)

    def step(i):
        kc, vc = pools[i % len(pools)]
        plan.run(q, kc, vc, out, causal=True, lse=lse)

    ms = event_time_ms(step, steps, warmup)
    per_step = event_block_means_ms(step, 10, steps)
    nbytes = W.decode_bytes(b)

    # The engine prepares the plan every step (cuda_model.cpp:141): host
    # planning, the metadata copy from pinned memory and the attention call,
    # with the host arrays converted to C arrays once as a caller would hold them.
    meta = [feattn._i32(x) for x in (b.qo, b.kv, b.pages, b.last)]

    def step_prepared(i):
        plan.prepare(*meta, b.batch, b.rows)
        step(i)

    ms_prep = event_time_ms(step_prepared, steps, warmup)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
    plan.close()
    del pools
    return b, ms, statistics.median(per_step), nbytes, ms_prep


def secondary(dev, only=None):
    """Other workload shapes: ms per call and throughput.  `only` selects one
    of prefill / dflash / mixed / long / graph."""
    import torch

    import feattn
    from feattn import workloads as W

    res = {}
    want = lambda name: only is None or only == name

    # chunked prefill (causal within chunk, full over prefix) + fused RoPE/append
    b = W.qwen3_8b_prefill()
    if not want("prefill"):
        b = None
    if b is not None:
        _prefill(b, dev, res)
    if want("dflash"):
        _dflash(dev, res)
    if want("mixed"):
        _mixed(dev, res)
    if want("long"):
        _long(dev, res)
    if want("graph"):
        _graph(dev, res)
    return res


def _prefill(b, dev, res):
    import torch

    import feattn
    from feattn import workloads as W

    plan, step = attn_setup(b, dev, torch.bfloat16, True, 1)
    ms = event_time_ms(step, 20, 3)
    flops = W.attention_flops(b, True)
    plan.close()
    k = torch.randn(b.rows, b.hkv, 128, device=dev).to(torch.bfloat16)
    v = torch.randn_like(k)
    q = torch.randn(b.rows, b.hq, 128, device=dev).to(torch.bfloat16)
    kc = torch.zeros(b.blocks + 1, 16, b.hkv, 128, device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    pos = torch.from_numpy(b.positions).to(dev)
    slots = torch.from_numpy(b.slots).to(dev)
    table = W.rope_table(8192, 1e6).to(dev)
    ra = lambda i: feattn.rope_append(q, k, v, kc, vc, pos, slots, table, b.rows, b.hq, b.hkv, 128,
                                      True, 8192, b.cache_slots)
    ms_ra = event_time_ms(ra, 20, 3)
    # the reference's two calls (src/cuda_model.cpp:94-95), each on its own
    ro = lambda i: feattn.rope(q, k, pos, table, b.rows, b.hq, b.hkv, 128, True, 8192)
    ms_ro = event_time_ms(ro, 20, 3)
    st = lambda i: feattn.store(k, v, kc, vc, slots, b.rows, b.hkv * 128, True, b.cache_slots)
    ms_st = event_time_ms(st, 20, 3)
    # the same new tokens through the fused q/k RMSNorm + RoPE + append of a
    # [rows][q | k | v] projection (src/cuda_model.cpp:91-95 in one pass)
    qkv = torch.randn(b.rows, (b.hq + 2 * b.hkv) * 128, device=dev).to(torch.bfloat16)
    qw = torch.ones(128, device=dev, dtype=torch.bfloat16)
    q_out = torch.empty_like(q)
    nra = lambda i: feattn.norm_rope_append(qkv, qkv.shape[1], qw, qw, 1e-6, q_out, kc, vc, pos, slots, table,
                                            b.rows, b.hq, b.hkv, True, 8192, b.cache_slots)
    ms_nra = event_time_ms(nra, 20, 3)
    res["prefill_qwen3_8b"] = {
        "workload": "8 seqs, prefix U[0,2048], chunks >=64 summing to 8192, causal, bf16",
        "attn_ms": round(ms, 4), "attn_tflops": round(flops / ms / 1e9, 2),
        "attn_frac_of_bf16_peak": round(flops / ms / 1e9 / BF16_PEAK_TFLOPS, 4),
        "gflop": round(flops / 1e9, 2),
        "rope_append_ms": round(ms_ra, 4),
        "rope_append_gbs": round(W.rope_append_bytes(b) / ms_ra / 1e6, 1),
        "rope_ms": round(ms_ro, 4), "rope_gbs": round(W.rope_bytes(b) / ms_ro / 1e6, 1),
        "store_ms": round(ms_st, 4), "store_gbs": round(W.store_bytes(b) / ms_st / 1e6, 1),
        "norm_rope_append_ms": round(ms_nra, 4),
        "norm_rope_append_gbs": round(W.norm_rope_append_bytes(b) / ms_nra / 1e6, 1)}
    log("prefill", res["prefill_qwen3_8b"])


def _dflash(dev, res):
    import torch

    from feattn import workloads as W

    # DFlash non-causal 16-row blocks, bf16 and fp16
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        b = W.dflash_block()
        plan, step = attn_setup(b, dev, dt, False, 1)
        ms = event_time_ms(step, 20, 3)
        flops = W.attention_flops(b, False)
        nbytes = sum(b.lens) * W.kv_bytes_per_token(b.hkv) + 2 * b.rows * b.hq * 128 * 2
        res[f"dflash_block_{name}"] = {
            "workload": "32 seqs x 16-row non-causal block over ctx U[2048,16384]",
            "ms": round(ms, 4), "gbs": round(nbytes / ms / 1e6, 1),
            "tflops": round(flops / ms / 1e9, 2)}
        plan.close()
        log("dflash", name, res[f"dflash_block_{name}"])


def _mixed(dev, res):
    import torch

    from feattn import workloads as W

    # mixed decode + prefill (Qwen3-30B-A3B heads: 32 q / 4 kv)
    b = W.qwen3_30b_mixed()
    plan, step = attn_setup(b, dev, torch.bfloat16, True, 1)
    ms = event_time_ms(step, 10, 2)
    dec = W.Batch(hq=32, hkv=4, page=16, blocks=b.blocks, starts=b.starts[:256],
                  qlens=b.qlens[:256], tables=b.tables[:256])
    W.build_metadata(dec)
    pre = W.Batch(hq=32, hkv=4, page=16, blocks=b.blocks, starts=b.starts[256:],
                  qlens=b.qlens[256:], tables=b.tables[256:])
    W.build_metadata(pre)
    t_bw = W.decode_bytes(dec) / (HBM_PEAK_GBS * 1e6)
    t_mf = W.attention_flops(pre, True) / (BF16_PEAK_TFLOPS * 1e9)
    res["mixed_qwen3_30b"] = {
        "workload": "256 decode (ctx U[1024,8192]) + 2 x 1024-token chunks over 4096, hkv 4",
        "ms": round(ms, 4), "roofline_max_ms": round(max(t_bw, t_mf), 4),
        "roofline_sum_ms": round(t_bw + t_mf, 4), "frac_of_max_bound": round(max(t_bw, t_mf) / ms, 4)}
    plan.close()
    log("mixed", res["mixed_qwen3_30b"])


def _graph(dev, res):
    import torch

    import feattn
    from feattn import workloads as W

    # the headline decode batch as the engine runs decode steps: the plan
    # prepared in graph mode outside capture, the attention calls of a step
    # (one per layer; here 8 layers over 4 KV pools) captured in one HIP
    # graph and replayed (src/cuda_model.cpp:150-157); ms is per call
    layers = 8
    b = W.qwen3_8b_decode()
    plan = feattn.Plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
    plan.prepare(b.qo, b.kv, b.pages, b.last, b.batch, b.rows, graph=True)
    pools = make_pools(b, 4, dev, torch.bfloat16)
    q = torch.randn(b.rows, b.hq, 128, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    lse = torch.empty(b.rows, b.hq, device=dev)

    def step():
        for i in range(layers):
            kc, vc = pools[i % len(pools)]
            plan.run(q, kc, vc, out, causal=True, lse=lse)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    ms = event_time_ms(lambda i: graph.replay(), 20, 3) / layers
    res["decode_graph_replay"] = {"workload": "headline decode batch, 8 attention calls per captured graph",
                                  "ms": round(ms, 4), "gbs": round(W.decode_bytes(b) / ms / 1e6, 1)}
    log("graph", res["decode_graph_replay"])
    del graph
    plan.close()


def _long(dev, res):
    import torch

    from feattn import workloads as W

    # long-context decode (split-KV)
    b = W.long_decode()
    plan, step = attn_setup(b, dev, torch.bfloat16, True, 1)
    ms = event_time_ms(step, 20, 3)
    res["long_decode_32k"] = {"workload": "16 seqs x 32768 tokens decode", "ms": round(ms, 4),
                              "gbs": round(W.decode_bytes(b) / ms / 1e6, 1)}
    plan.close()
    log("long", res["long_decode_32k"])


def copy_calibration(dev, mib=1024):
    """A plain device copy of known size (read + write of `mib` MiB), timed:
    the practical bandwidth reference, and the kernel on which the DRAM
    request counters' byte formulas are checked (exactly `mib` MiB read and
    written)."""
    import torch

    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    ms = event_time_ms(lambda i: dst.copy_(src), 10, 2)
    del src, dst
    return {"bytes_per_copy": 2 * n, "ms": round(ms, 4), "gbs": round(2 * n / ms / 1e6, 1)}


def host_cpu():
    """The host the CPU baseline runs on: model name from /proc/cpuinfo, the
    CPUs this process may run on (what `nproc` reports), os.cpu_count() and
    OMP_NUM_THREADS."""
    model = platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"model": model, "nproc": len(os.sched_getaffinity(0)), "os_cpu_count": os.cpu_count(),
            "omp_num_threads": int(omp) if omp and omp.isdigit() else None}


def oracle_time(b, q, kc, vc, causal, runs=4):
    """Median wall time of the oracle's prepare_plan and attention over
    runs - 1 calls after one warm-up call."""
    import torch

    from oracle import aten_attention as A

    times, prep = [], []
    for it in range(runs):
        t0 = time.perf_counter()
        p = A.create_plan(b.hq, b.hkv, 128, b.page, b.batch, b.max_pages(), True, b.blocks)
        A.prepare_plan(p, b.qo, b.kv, b.pages, b.last, b.batch, b.rows)
        t1 = time.perf_counter()
        out = torch.empty_like(q)
        A.attention(p, q, kc, vc, out, causal)
        t2 = time.perf_counter()
        if it:
            prep.append(t1 - t0)
            times.append(t2 - t1)
        log(f"cpu baseline run {it}: prepare {t1 - t0:.3f}s attention {t2 - t1:.3f}s")
    return statistics.median(times), statistics.median(prep)


def cpu_baseline(b):
    """Oracle (LibTorch-CPU restatement of the reference ATen attention,
    sequence by sequence) on the full decode batch and on the full chunked
    prefill batch: median of 3 after 1 warm-up each, with as many threads as
    this process may use (nproc, capped by OMP_NUM_THREADS when set)."""
    import torch

    from feattn import workloads as W

    host = host_cpu()
    threads = host["nproc"]
    if host["omp_num_threads"]:
        threads = min(threads, host["omp_num_threads"])
    torch.set_num_threads(threads)
    q, kc, vc = W.make_tensors(b, seed=7)
    t, tp = oracle_time(b, q, kc, vc, True)
    pb = W.qwen3_8b_prefill()
    pq, pkc, pvc = W.make_tensors(pb, seed=8)
    pt, ptp = oracle_time(pb, pq, pkc, pvc, True)
    pflops = W.attention_flops(pb, True)
    return {
        "value": round(W.decode_bytes(b) / t / 1e9, 3), "unit": "GB/s",
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": "full 64-sequence decode batch (same metadata, seeded bf16 inputs); "
                  "LibTorch-CPU restatement of src/portable_gpu_ops.cpp attention; median of 3 "
                  "after 1 warmup",
        "attention_s": round(t, 4), "prepare_plan_s": round(tp, 4),
        "prefill": {"value": round(pflops / pt / 1e9, 2), "unit": "GFLOP/s",
                    "sample": "full chunked prefill batch (8 seqs, 8192 query rows, causal), the "
                              "same restatement, sequence by sequence; median of 3 after 1 warmup",
                    "attention_s": round(pt, 4), "prepare_plan_s": round(ptp, 4)},
        "cpu": host, "torch": torch.__version__}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["prefill", "dflash", "mixed", "long", "graph"],
                    help="run one secondary workload only (for profiling); no headline line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this attention library has no multi-GPU mode "
              "(sequences and kv heads shard across GPUs without any exchange)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import feattn

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    feattn.lib()
    log("library", feattn.version())
    if args.only:
        print(json.dumps(secondary(dev, args.only)), flush=True)
        return

    b, ms, ms_med, nbytes, ms_prep = decode_headline(args.steps, args.warmup, dev)
    gbs = nbytes / ms / 1e6
    log(f"decode: {ms * 1e3:.1f} us/step, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of peak); "
        f"median of 10 further blocks of {args.steps} steps: {ms_med * 1e3:.1f} us/step; "
        f"with prepare every step: {ms_prep * 1e3:.1f} us/step")
    sec = {} if args.no_secondary else secondary(dev)
    sec["copy_calibration"] = copy_calibration(dev)
    log("copy", sec["copy_calibration"])
    cpu = None if args.no_cpu else cpu_baseline(b)

    line = {
        "metric": METRIC, "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "Qwen3-8B-shape paged decode attention: 64 seqs, ctx U[512,4096] "
                               "(seeded), hq 32 / hkv 8 / d 128, 16-token pages, bf16, 4 rotated "
                               "KV pools; every context token's raw q/k/v ~ N(0,1), q and k rotated "
                               "at the token's position (RoPE theta 1e6) and k/v written to its page "
                               "slot by the fused RoPE + paged append; the decode rows are the last "
                               "token's q",
                   "rope_theta": ROPE_THETA,
                   "batch": b.batch, "context_tokens": sum(b.lens), "pages": b.blocks,
                   "seeds": {"lengths_and_pages": DECODE_SEED, "kv_pools": POOL_SEED, "q": Q_SEED}},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(),
                     "algorithmic_bytes": nbytes,
                     "timed": "one fe_attn_run per step (attn_decode_kernel + attn_merge_kernel, "
                              "the whole attention call), HIP events on the launch stream; "
                              "achieved = algorithmic bytes / mean step time of the timed region; "
                              "traffic = DRAM read + write request counters of both kernels, "
                              "profiles/decode_qwen3_8b_hbm_traffic.txt",
                     "ms_per_step_mean": round(ms, 5),
                     "ms_per_step_median": round(ms_med, 5),
                     "median_of": f"the mean step times of 10 further blocks of {args.steps} steps "
                                  f"({10 * args.steps} launches) after the timed region",
                     "ms_per_step_with_prepare": round(ms_prep, 5),
                     "gbs_with_prepare": round(nbytes / ms_prep / 1e6, 2),
                     "with_prepare": "fe_attn_plan_prepare (host planning + metadata copy from "
                                     "pinned host memory) before every fe_attn_run, as the engine "
                                     "steps; not the headline value"},
        "cpu_baseline": cpu,
        "secondary": sec,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
