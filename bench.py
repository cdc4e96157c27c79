"""Benchmark of the DeepSeek-V4 attention pre-processing hot path on one MI355X.

A "step" is one call of fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert over
one batch of the headline workload c2 (T=8192 prefill tokens from 4 sequences,
H=64, D=512, rope 64, 16384 x 64-slot FP8 cache), inputs already resident in
HBM.  Prints ONE JSON line with tokens/s, the HBM roofline fraction of the
kernel (algorithmic bytes / HIP-event kernel time / 8 TB/s) and the reference
PyTorch path timed on this host's CPU cores on a bounded sample of the same
workload.

    python bench.py [--steps K] [--warmup W] [--config 0..4] [--op main|inv_rope]
"""
import argparse
import json
import math
import os
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (os.path.join(ROOT, "flaggems-vllm_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)

METRIC = "tokens/s and achieved HBM GB/s (% of roofline) at T=8192, H=64, D=512"
HBM_PEAK_GBPS = 8000.0
PROFILES = os.path.join(ROOT, "profiles")


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, help="main-op workload c0..c4 (default c2)")
    ap.add_argument("--op", choices=["main", "inv_rope", "gather", "rmsnorm", "indexer",
                                     "slot_mapping", "mla", "indexer_k", "indexer_k_gather", "mqa_logits",
                                     "paged_mqa_logits", "topk", "einsum", "mla_sparse", "copy"],
                    default="main",
                    help="copy: torch device copy of 512 MiB, the HBM calibration kernel")
    ap.add_argument("--tma", action="store_true", help="inv_rope: packed UE8M0 scales")
    ap.add_argument("--inv-shape", default="8192,64,8",
                    help="inv_rope: num_tokens,num_heads,n_groups (the reference benchmark's shapes are 1,8,1 "
                         "and 16,64,8, with --tma)")
    ap.add_argument("--fp4", action="store_true", help="indexer, mqa_logits, paged_mqa_logits: MXFP4 q instead of FP8")
    ap.add_argument("--mla-case", choices=["decode", "extra512", "extra8192"], default="decode",
                    help="mla: the reference benchmark's MODEL1 sparse-decode case")
    ap.add_argument("--mla-batch", type=int, default=0,
                    help="mla: batch rows instead of the case's 512 (the case's other sizes kept)")
    ap.add_argument("--mla-heads", type=int, default=0, choices=[0, 64, 128],
                    help="mla: query heads instead of the case's 64")
    ap.add_argument("--indexer-case", choices=["0", "1", "2", "3", "large"], default="3",
                    help="indexer_k / indexer_k_gather: the reference benchmark's shape 0..3 (default its "
                         "largest) or 'large' (65536 tokens, head_dim 512)")
    ap.add_argument("--fp16", action="store_true", help="indexer_k: float16 keys instead of bfloat16")
    ap.add_argument("--mqa-shape", default="4096,8192",
                    help="mqa_logits: M,N (default the reference benchmark's largest, 4096 x 8192)")
    ap.add_argument("--paged-shape", default="256,1,8192",
                    help="paged_mqa_logits: batch,next_n,context (reference benchmark shapes)")
    ap.add_argument("--topk-case", choices=["decode", "prefill", "prefill_short"], default="decode",
                    help="topk: top_k_per_row at the reference benchmark's largest decode shape (496 x 262144, "
                         "k 512), its full-vocabulary prefill (64 x 129280, k 1024) or its many short rows "
                         "(16383 x 4095, row stride 4352, k 512)")
    ap.add_argument("--einsum-case", default="flash,8192",
                    help="einsum: group,b with group flash (h 8, r 4096, d 1024) or pro (h 16, r 7168, d 1024) "
                         "and b the batch (the reference benchmark's groups and batches 1..32768)")
    ap.add_argument("--mla-sparse-case", default="v32_8k",
                    help="mla_sparse: flash_mla_sparse_fwd at a reference benchmark case (s_q 4096, sink): "
                         "v32_{8,32,64,96,128}k (topk 2048, h_q 128, d_qk 576), h64_{8,32,48,64}k (topk 512, "
                         "h_q 64, d_qk 512) or h128_{8,32,48,64}k (topk 1024, h_q 128, d_qk 512)")
    ap.add_argument("--cpu-sample-tokens", type=int, default=8192)
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="repeat the CPU sample until this much CPU time is spent (min 3 runs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--ref-shapes", action="store_true",
                    help="with --op gather|rmsnorm|indexer|slot_mapping|inv_rope: time the op at every shape of "
                         "the reference benchmark for it and print a table")
    ap.add_argument("--grid", action="store_true",
                    help="main op over the reference benchmark's grid (T x H); one JSON line per point "
                         "and a markdown table, instead of the single headline line")
    ap.add_argument("--grid-max-tokens", type=int, default=131072)
    ap.add_argument("--eager", action="store_true",
                    help="host cost of eager calls of the main op and the sibling at decode sizes "
                         "(T 1..64, H 64 and 128); a markdown table instead of the headline line")
    return ap.parse_args()


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 PMC summary
    profiles/<kernel>_<workload>_pmc.md (line 'traffic_bytes_per_launch: N'),
    or None when no such summary exists."""
    path = os.path.join(PROFILES, f"{kernel}_{workload}_pmc.md")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read())
    return float(m.group(1)) if m else None


MALL_BYTES = 256 << 20  # MI355X Infinity Cache (MALL)


def mall_sets(bytes_call):
    """How many input sets the timed calls rotate through: enough that
    consecutive calls touch more than twice the 256 MB MALL, so each call
    streams from HBM rather than from what the previous calls left in the
    cache (at most 16; one set when a call alone moves 512 MB or more)."""
    return max(1, min(16, -(-2 * MALL_BYTES // bytes_call)))


def rotating(make_step, bytes_call):
    """(step, sets): step() calls make_step(i)'s closure for set i = 0, 1, ...
    in turn; set 0 is built first, the others are fresh device copies."""
    k = mall_sets(bytes_call)
    steps = [make_step(i) for i in range(k)]
    state = {"i": 0}

    def step():
        steps[state["i"]]()
        state["i"] = (state["i"] + 1) % k

    return step, k


def time_gpu(fn, steps, warmup):
    """Seconds per step: (host wall clock of the eager loop, kernel time, how the
    kernel time was taken).

    The eager loop of `steps` calls through the public API gives the step time.
    The kernel time comes from HIP events around replays of a HIP graph that
    holds the same `steps` calls, so that the host-side cost of the Python
    wrappers (tens of microseconds, more than some of these kernels take) leaves
    no idle gaps between the launches being timed.  The graph is replayed back
    to back until about 2 ms of GPU work lie between the events (once for
    calls of 40 us or more at 50 steps), so that the graph's own launch does not
    weigh on short calls; each replay runs exactly `steps` calls.  Where capture
    is not possible, the eager loop's events are used instead.
    """
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    eager = start.elapsed_time(end) / 1000.0 / steps
    try:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            for _ in range(steps):
                fn()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replays = max(1, min(32, math.ceil(2e-3 / max(steps * eager, 1e-9))))
        start.record()
        for _ in range(replays):
            graph.replay()
        end.record()
        torch.cuda.synchronize()
        return (wall / steps, start.elapsed_time(end) / 1000.0 / (steps * replays),
                f"hip graph of the timed steps, {replays} back-to-back replay(s)")
    except RuntimeError as e:
        print(f"bench.py: graph capture unavailable ({e}); kernel time from the eager loop", file=sys.stderr)
        return wall / steps, eager, "events around the eager loop"


def median_call_us(fn, calls):
    """Median over `calls` eager calls of the time between HIP events recorded
    on the launch stream before and after each call (one event chain, so the
    intervals tile the loop).  It is the kernel's duration where the kernel
    outlasts the wrapper's host cost (the main op's c2-c4); for shorter kernels
    the intervals also hold the GPU's wait for the next launch."""
    import torch

    ev = [torch.cuda.Event(enable_timing=True) for _ in range(calls + 1)]
    fn()
    torch.cuda.synchronize()
    ev[0].record()
    for i in range(calls):
        fn()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return statistics.median(ev[i].elapsed_time(ev[i + 1]) * 1000.0 for i in range(calls))


def eager_loop_us(fn, calls):
    """GPU time per call of `calls` back-to-back eager calls: one pair of HIP
    events around the whole loop, divided by `calls`.  This is the rate a host
    loop of eager calls sustains, max(host cost, kernel) per call, without the
    host time that recording an event after every call adds."""
    import torch

    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(calls):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) * 1000.0 / calls


def _repeat(run, seconds):
    """Median wall time of run(), repeated until `seconds` are spent (3..200 runs)."""
    times = []
    while len(times) < 3 or (sum(times) < seconds and len(times) < 200):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline_main(w, sample_tokens, seconds):
    """The reference's PyTorch formulation (oracle.torch_ref) on the host CPU,
    over the first `sample_tokens` tokens of the workload with all heads;
    median over repeated runs, tokens/s."""
    import torch

    from oracle import torch_ref

    n = min(sample_tokens, w.num_tokens)
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    q = w.q[:n].clone()

    def run():
        torch_ref.qnorm_rope_kv_insert(q, w.kv[:n], w.k_cache, w.slot_mapping[:n],
                                       w.position_ids[:n], w.cos_sin_cache, w.eps, w.block_size)

    t, reps = _repeat(run, seconds)
    return {"value": n / t, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first {n} of {w.num_tokens} tokens of {w.name}, all {w.num_heads} heads: "
                      f"torch CPU restatement of the reference's torch oracle (oracle/torch_ref.py), "
                      f"median of {reps} runs, {t:.3f} s per run"}


def cpu_baseline_inv(w, tma, sample_tokens, seconds):
    import torch

    from oracle import torch_ref

    n = min(sample_tokens, w.o.shape[0])
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)

    def run():
        torch_ref.inv_rope_fp8_quant(w.o[:n], w.positions[:n], w.cos_sin_cache, w.n_groups,
                                     w.heads_per_group, tma_aligned_scales=tma)

    t, reps = _repeat(run, seconds)
    return {"value": n / t, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"first {n} of {w.o.shape[0]} tokens, torch CPU restatement "
                      f"(oracle/torch_ref.py), median of {reps} runs, {t:.3f} s per run"}


def cpu_baseline_mla(w, sample_rows, seconds):
    """The reference's portable MODEL1 algorithm restated in torch
    (oracle.torch_ref) on the host CPU, over the first `sample_rows` batch
    rows; decode rows (batch x seq_q) per second."""
    import torch

    from oracle import torch_ref

    n = min(sample_rows, w.q.shape[0])
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    sub = lambda t: None if t is None else t[:n]
    kw = dict(topk_length=sub(w.topk_length), attn_sink=w.attn_sink,
              extra_k_cache=w.extra_k_cache, extra_indices=sub(w.extra_indices),
              extra_topk_length=sub(w.extra_topk_length))

    def run():
        torch_ref.sparse_mla_decode_model1(w.q[:n], w.k_cache, w.indices[:n], **kw)

    t, reps = _repeat(run, seconds)
    rows = n * w.q.shape[1]
    return {"value": rows / t, "unit": "decode rows/s", "cores": cores, "kind": "port",
            "sample": f"first {n} of {w.q.shape[0]} batch rows of {w.name}, all heads: torch CPU "
                      f"restatement of the reference's portable MODEL1 kernel (oracle/torch_ref.py), "
                      f"median of {reps} runs, {t:.3f} s per run"}


def cpu_baseline_port(run, units, unit, sample, seconds):
    """Median wall time of a torch CPU restatement (oracle.torch_ref) run on a
    bounded sample; `units` of the metric per run."""
    import torch

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t, reps = _repeat(run, seconds)
    return {"value": units / t, "unit": unit, "cores": cores, "kind": "port",
            "sample": f"{sample}: torch CPU restatement (oracle/torch_ref.py), median of {reps} runs, "
                      f"{t:.3f} s per run"}


# The reference benchmark's shapes for the main op
# (benchmark/test_fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert.py:137-163):
# positions = arange(T), slot_mapping = arange(T), 64-slot blocks, max_pos =
# max(4096, T) with the rope base chosen by max_pos (:170-192).
GRID_TOKENS = [1, 4, 17, 64, 1024, 2048, 8192, 32768, 65536, 98304, 131072]
GRID_HEADS = [64, 128]


def run_grid(args):
    """Times the main op at every point of the reference benchmark's grid with
    inputs drawn on the device like the reference benchmark's, rotating device
    copies for calls under 512 MB (mall_sets), graph-replay kernel time."""
    import torch

    import flaggems_vllm
    from flaggems_vllm import testing as W

    dev = torch.device("cuda:0")
    op = flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
    rows = []
    for T in [t for t in GRID_TOKENS if t <= args.grid_max_tokens]:
        for H in GRID_HEADS:
            max_pos = max(4096, T)
            base = 10000.0 if max_pos <= 8192 else 20000.0 if max_pos <= 32768 else 40000.0 \
                if max_pos <= 65536 else 60000.0 if max_pos <= 98304 else 100000.0
            cs = W.make_cos_sin_cache(max_pos, base=base).to(dev)
            pos = torch.arange(T, dtype=torch.int64, device=dev)
            slots = torch.arange(T, dtype=torch.int64, device=dev)
            nblk = (T + 63) // 64 + 1
            bytes_call = W.main_op_bytes(T, H, T)
            gen = torch.Generator(device=dev).manual_seed(T * 1000 + H)

            def make_step(i):
                q = torch.randn(T, H, 512, generator=gen, device=dev, dtype=torch.bfloat16)
                kv = torch.randn(T, 512, generator=gen, device=dev, dtype=torch.bfloat16)
                cache = torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8, device=dev)
                return lambda: op(q, kv, cache, slots, pos, cs, 1e-6, 64)

            step, n_sets = rotating(make_step, bytes_call)
            steps = args.steps if T >= 8192 else max(args.steps, 200)
            _, t_kernel, timing = time_gpu(step, steps, args.warmup)
            median_us = median_call_us(step, max(20, min(steps, 200)))
            loop_us = eager_loop_us(step, max(20, min(steps, 200)))
            host_us = host_us_per_call(step, max(20, min(steps, 200)))
            gbps = bytes_call / t_kernel / 1e9
            span = n_sets * bytes_call
            row = {"op": "fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert", "num_tokens": T, "num_heads": H,
                   "kernel_us": t_kernel * 1e6, "kernel_us_median_per_call": median_us,
                   "eager_loop_us_per_call": loop_us, "host_us_per_eager_call": host_us,
                   "bytes_per_call": bytes_call, "gbps": gbps, "frac_of_8tbps": gbps / HBM_PEAK_GBPS,
                   "tokens_per_s": T / t_kernel, "input_sets": n_sets,
                   "mall": "cold" if n_sets == 1 or span > 2 * MALL_BYTES else "warm", "steps": steps,
                   "kernel_timing": timing}
            print(json.dumps(row), flush=True)
            rows.append(row)
            del step
            torch.cuda.empty_cache()
    print("\n| T | H | MB per call | input sets | µs per call (graph) | µs per call, eager loop (events around "
          "the loop) | µs median per eager call (an event after every call) | host µs per eager call | GB/s "
          "| % of 8 TB/s | tokens/s |")
    print("|---|---|---|---|---|---|---|---|---|---|---|")
    for r in rows:
        sets = f"{r['input_sets']}" + (" (MALL-warm)" if r["mall"] == "warm" else "")
        print(f"| {r['num_tokens']} | {r['num_heads']} | {r['bytes_per_call'] / 1e6:.2f} | {sets} "
              f"| {r['kernel_us']:.2f} | {r['eager_loop_us_per_call']:.2f} | {r['kernel_us_median_per_call']:.2f} "
              f"| {r['host_us_per_eager_call']:.2f} "
              f"| {r['gbps']:.0f} | {100 * r['frac_of_8tbps']:.1f} | {r['tokens_per_s']:.3g} |", flush=True)


# The reference benchmarks' own shapes for the ops beside the main op
# (benchmark/test_deepseek_v4_attention_dequantize_and_gather_k_cache.py:75-81,
# benchmark/test_deepseek_v4_attention_fused_q_kv_rmsnorm.py:58-66,
# benchmark/test_fused_indexer_q_rope_quant.py:139-143 with NUM_HEADS 8 (:24),
# benchmark/test_slot_mapping_perf.py:35-50, benchmark/test_fused_inv_rope_fp8_quant.py:100).
REF_SHAPES = {
    "gather": [(1, 512, 128), (2, 1024, 256), (4, 2048, 512), (4, 2048, 2048), (8, 4096, 1024)],
    "rmsnorm": [(1, 1536, 512), (32, 1536, 512), (128, 1536, 512), (512, 1536, 512), (2048, 1536, 512),
                (32, 64 * 576, 576), (128, 64 * 576, 576)],
    "indexer": [(1, 8, False), (32, 8, False), (32, 8, True)],
    "slot_mapping": [(4, 8192, 128), (8, 8192, 128), (12, 8192, 128), (16, 8192, 128), (4, 8192, 16),
                     (32, 8192, 128), (128, 8192, 128), (8, 8192, 16), (8, 16384, 128), (1, 8192, 128)],
    "inv_rope": [(1, 8, 1, True), (16, 64, 8, True)],
}


def run_ref_shapes(args):
    """Times one op at every shape of its reference benchmark, with inputs drawn
    on the device as that benchmark draws them; rotating device copies for
    small calls (mall_sets), graph-replay kernel time and the eager loop."""
    import torch

    import flaggems_vllm
    from flaggems_vllm import testing as W

    dev = torch.device("cuda:0")
    op = args.op
    if op not in REF_SHAPES:
        raise SystemExit(f"--ref-shapes covers {', '.join(REF_SHAPES)}")
    rows = []
    for shape in REF_SHAPES[op]:
        gen = torch.Generator(device=dev).manual_seed(hash(shape) & 0xFFFF)
        if op == "gather":
            batch, seq_len, gather_len = shape
            nblk = batch * ((seq_len + 63) // 64)
            desc = f"batch {batch}, seq_len {seq_len}, gather_len {gather_len}"
            bytes_call = W.gather_bytes(batch * gather_len)

            def make_step(i, batch=batch, seq_len=seq_len, gather_len=gather_len, nblk=nblk):
                out = torch.empty(batch, gather_len, 512, dtype=torch.bfloat16, device=dev)
                cache = torch.zeros(nblk, 64 * W.HEAD_BYTES, dtype=torch.uint8, device=dev)
                sl = torch.full((batch,), seq_len, dtype=torch.int32, device=dev)
                gl = torch.full((batch,), gather_len, dtype=torch.int32, device=dev)
                bt = torch.arange(nblk, dtype=torch.int32, device=dev).view(batch, -1)
                return lambda: flaggems_vllm.dequantize_and_gather_k_cache(out, cache, sl, gl, bt, 64, 0, 64, 448, 8)
        elif op == "rmsnorm":
            tokens, qdim, kvdim = shape
            desc = f"tokens {tokens}, q {qdim}, kv {kvdim}"
            bytes_call = W.rmsnorm_bytes(tokens, qdim, kvdim)

            def make_step(i, tokens=tokens, qdim=qdim, kvdim=kvdim):
                qr = torch.randn(tokens, qdim, generator=gen, device=dev, dtype=torch.bfloat16)
                kv = torch.randn(tokens, kvdim, generator=gen, device=dev, dtype=torch.bfloat16)
                qw = torch.randn(qdim, generator=gen, device=dev, dtype=torch.bfloat16)
                kw = torch.randn(kvdim, generator=gen, device=dev, dtype=torch.bfloat16)
                return lambda: flaggems_vllm.fused_q_kv_rmsnorm(qr, kv, qw, kw, 1e-6)
        elif op == "indexer":
            tokens, heads, fp4 = shape
            desc = f"tokens {tokens}, heads {heads}, head_dim 128, {'MXFP4' if fp4 else 'FP8'}"
            bytes_call = W.indexer_bytes(tokens, heads, 128, fp4)
            cs = W.make_cos_sin_cache(4096).to(dev).to(torch.bfloat16)

            def make_step(i, tokens=tokens, heads=heads, fp4=fp4, cs=cs):
                q = torch.randn(tokens, heads, 128, generator=gen, device=dev, dtype=torch.bfloat16)
                pos = torch.randint(0, 4096, (tokens,), generator=gen, device=dev, dtype=torch.int64)
                wts = torch.randn(tokens, heads, generator=gen, device=dev, dtype=torch.bfloat16)
                return lambda: flaggems_vllm.fused_indexer_q_rope_quant(pos, q, cs, wts, 128 ** -0.5, heads ** -0.5,
                                                                        use_fp4=fp4)
        elif op == "slot_mapping":
            nreq, maxtok, bs = shape
            tlen = 200
            desc = f"{nreq} requests of {tlen} tokens, max_num_tokens {maxtok}, block size {bs}"
            bytes_call = nreq * tlen * (4 + 4 + 8) + (maxtok - nreq * tlen) * 8 + 4 * (nreq + 1)

            def make_step(i, nreq=nreq, maxtok=maxtok, bs=bs, tlen=tlen):
                qsl = torch.arange(0, tlen * (nreq + 1), tlen, dtype=torch.int32, device=dev)
                pos = torch.arange(tlen, dtype=torch.int32, device=dev).repeat(nreq)
                maxb = (16384 + bs - 1) // bs + 1
                btab = (torch.arange(nreq * maxb, dtype=torch.int32, device=dev) % 900).view(nreq, maxb)
                out = torch.full((maxtok,), -1, dtype=torch.int64, device=dev)
                return lambda: flaggems_vllm.compute_slot_mapping_parallel(tlen * nreq, maxtok, qsl, nreq, pos, btab,
                                                                           out, block_size=bs)
        else:
            T, H, G, tma = shape
            desc = f"tokens {T}, heads {H}, groups {G}, {'packed UE8M0' if tma else 'fp32'} scales"
            bytes_call = W.inv_rope_bytes(T, H, tma)

            def make_step(i, T=T, H=H, G=G, tma=tma):
                wi = W.make_inv_rope_workload(T, H, G, seed=i).to(dev)
                return lambda: flaggems_vllm.fused_inv_rope_fp8_quant(wi.o, wi.positions, wi.cos_sin_cache, G, H // G,
                                                                      tma_aligned_scales=tma)
        step, n_sets = rotating(make_step, bytes_call)
        steps = max(args.steps, 200)
        _, t_kernel, timing = time_gpu(step, steps, args.warmup)
        loop_us = eager_loop_us(step, steps)
        gbps = bytes_call / t_kernel / 1e9
        row = {"op": op, "shape": list(shape), "desc": desc, "kernel_us": t_kernel * 1e6,
               "eager_loop_us_per_call": loop_us, "bytes_per_call": bytes_call, "gbps": gbps,
               "frac_of_8tbps": gbps / HBM_PEAK_GBPS, "input_sets": n_sets, "kernel_timing": timing}
        print(json.dumps(row), flush=True)
        rows.append(row)
        del step
        torch.cuda.empty_cache()
    print("\n| shape | bytes per call | input sets | µs per call (graph) | µs per call, eager loop | GB/s "
          "| % of 8 TB/s |")
    print("|---|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {r['desc']} | {r['bytes_per_call']} | {r['input_sets']} | {r['kernel_us']:.2f} "
              f"| {r['eager_loop_us_per_call']:.2f} | {r['gbps']:.0f} | {100 * r['frac_of_8tbps']:.1f} |", flush=True)


def host_us_per_call(fn, calls):
    """Host wall time per call of `calls` back-to-back eager calls (no
    synchronisation inside the loop), microseconds."""
    import torch

    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(calls):
        fn()
    t1 = time.perf_counter()
    torch.cuda.synchronize()
    return (t1 - t0) / calls * 1e6


def run_eager(args):
    """Eager host cost of the two ops at decode sizes: per-call intervals
    between HIP events (median) and host wall time per call, beside the
    graph-replay kernel time; the main op through the Python drop-in and
    through torch.ops."""
    import torch

    import flaggems_vllm
    from flaggems_vllm import testing as W

    dev = torch.device("cuda:0")
    main_op = flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
    torch_op = torch.ops.flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert
    calls = 2000
    rows = []
    for T in (1, 4, 17, 64):
        for H in (64, 128):
            g = torch.Generator(device=dev).manual_seed(T * 1000 + H)
            q = torch.randn(T, H, 512, generator=g, device=dev, dtype=torch.bfloat16)
            kv = torch.randn(T, 512, generator=g, device=dev, dtype=torch.bfloat16)
            cs = W.make_cos_sin_cache(4096).to(dev)
            pos = torch.arange(T, dtype=torch.int64, device=dev)
            cache = torch.zeros(T // 64 + 2, 64 * W.HEAD_BYTES, dtype=torch.uint8, device=dev)
            a = (q, kv, cache, pos, pos, cs, 1e-6, 64)
            o = torch.randn(T, H, 512, generator=g, device=dev, dtype=torch.bfloat16)
            sib = (o, pos, cs, 8, H // 8)
            r = {"num_tokens": T, "num_heads": H}
            _, t_kernel, _ = time_gpu(lambda: main_op(*a), 200, args.warmup)
            r["main_kernel_us"] = t_kernel * 1e6
            r["main_loop_us"] = eager_loop_us(lambda: main_op(*a), calls)
            r["main_event_median_us"] = median_call_us(lambda: main_op(*a), calls)
            r["main_host_us"] = host_us_per_call(lambda: main_op(*a), calls)
            r["main_torch_ops_host_us"] = host_us_per_call(lambda: torch_op(*a), calls)
            r["sibling_loop_us"] = eager_loop_us(lambda: flaggems_vllm.fused_inv_rope_fp8_quant(*sib), calls)
            r["sibling_event_median_us"] = median_call_us(lambda: flaggems_vllm.fused_inv_rope_fp8_quant(*sib),
                                                          calls)
            r["sibling_host_us"] = host_us_per_call(lambda: flaggems_vllm.fused_inv_rope_fp8_quant(*sib), calls)
            print(json.dumps(r), flush=True)
            rows.append(r)
    print("\n| T | H | main: kernel µs (graph) | main: µs per call, eager loop (events around the loop) "
          "| main: µs median per eager call (an event after every call) | main: host µs per call "
          "| main via torch.ops: host µs per call | sibling: µs per call, eager loop | sibling: µs median per "
          "eager call (an event after every call) | sibling: host µs per call |")
    print("|---|---|---|---|---|---|---|---|---|---|")
    for r in rows:
        print(f"| {r['num_tokens']} | {r['num_heads']} | {r['main_kernel_us']:.2f} | {r['main_loop_us']:.2f} "
              f"| {r['main_event_median_us']:.2f} | {r['main_host_us']:.2f} | {r['main_torch_ops_host_us']:.2f} "
              f"| {r['sibling_loop_us']:.2f} | {r['sibling_event_median_us']:.2f} | {r['sibling_host_us']:.2f} |",
              flush=True)


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this op needs no exchange between GPUs "
              "(tokens and heads shard independently), and this build runs on single-GPU "
              "boxes. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch

    import flaggems_vllm
    from flaggems_vllm import testing as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.ref_shapes:
        run_ref_shapes(args)
        return
    if args.grid:
        run_grid(args)
        return
    if args.eager:
        run_eager(args)
        return
    from oracle import torch_ref

    cpu_case = None  # (run, units per run, unit, sample) for ops timed by cpu_baseline_port

    if args.op == "main":
        w_cpu = W.make_workload(args.config)
        w = w_cpu.to(dev)
        T, H, nv = w.num_tokens, w.num_heads, w.num_inserted
        bytes_call = w.bytes_per_call()

        def make_step(i):
            a = (w if i == 0 else w_cpu.to(dev)).args()
            return lambda: flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*a)

        kernel = "qnorm_rope_kv_insert_kernel"
        workload = f"c{args.config}"
        config = {"workload": f"c{args.config}: fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert, "
                              f"T={T}, H={H}, D=512 (448 nope + 64 rope), kv rows inserted={nv}, "
                              f"cache {w.k_cache.shape[0]} blocks x {w.block_size} slots x 584 B",
                  "num_tokens": T, "num_heads": H, "head_dim": 512, "rope_dim": 64,
                  "inserted_tokens": nv, "cache_block_size": w.block_size,
                  "io": "bf16 q/kv in, bf16 q out, fp8-e4m3 + UE8M0 cache"}
    elif args.op == "gather":
        # c2's cache after the insert; gather every position of its 4 sequences
        w_cpu = W.make_workload(args.config)
        w = w_cpu.to(dev)
        flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*w.args())
        m = w_cpu.meta
        bt, seq_lens = m["block_table"].to(dev), m["seq_lens"].to(dev)
        rows = int(m["seq_lens"].max())
        T = int(m["seq_lens"].sum())
        bytes_call = W.gather_bytes(T)

        def make_step(i):
            wi = w
            if i:
                wi = w_cpu.to(dev)
                flaggems_vllm.fused_deepseek_v4_qnorm_rope_kv_rope_quant_insert(*wi.args())
            out = torch.empty(bt.shape[0], rows, 512, dtype=torch.bfloat16, device=dev)
            return lambda: flaggems_vllm.dequantize_and_gather_k_cache(out, wi.k_cache, seq_lens, None, bt,
                                                                       wi.block_size)

        kernel, workload = "dequantize_gather_kernel", f"c{args.config}_whole_seqs"
        config = {"workload": f"dequantize_and_gather_k_cache: all positions of c{args.config}'s "
                              f"{bt.shape[0]} sequences ({T} rows) from its 584 B/token FP8 cache",
                  "rows": T, "num_reqs": int(bt.shape[0])}
        cache_cpu = w.k_cache.cpu()
        n0 = int(m["seq_lens"][0])
        out_cpu = torch.empty(1, n0, 512, dtype=torch.bfloat16)
        cpu_case = (lambda: torch_ref.dequantize_and_gather_k_cache(
                        out_cpu, cache_cpu, m["seq_lens"][:1], None, m["block_table"][:1], w.block_size),
                    n0, "tokens/s", f"the first of {bt.shape[0]} sequences ({n0} rows)")
    elif args.op == "rmsnorm":
        # DeepSeek-V4 q LoRA rank 1536 and kv latent 512 for c2's 8192 tokens
        g = torch.Generator().manual_seed(0)
        T = 8192
        qr = W.randn_bf16((T, 1536), g).to(dev)
        kvr = W.randn_bf16((T, 512), g).to(dev)
        qw = W.randn_bf16((1536,), g).to(dev)
        kw = W.randn_bf16((512,), g).to(dev)
        bytes_call = W.rmsnorm_bytes(T, 1536, 512)

        def make_step(i):
            x = (qr, kvr) if i == 0 else (qr.clone(), kvr.clone())
            return lambda: flaggems_vllm.fused_q_kv_rmsnorm(x[0], x[1], qw, kw, 1e-6)

        kernel, workload = "fused_q_kv_rmsnorm_kernel", "T8192_q1536_kv512"
        config = {"workload": "fused_q_kv_rmsnorm T=8192, q 1536, kv 512, bf16 weights",
                  "num_tokens": T}
        nc = min(args.cpu_sample_tokens, T)
        cq, ck, cqw, ckw = qr[:nc].cpu(), kvr[:nc].cpu(), qw.cpu(), kw.cpu()
        cpu_case = (lambda: torch_ref.fused_q_kv_rmsnorm(cq, ck, cqw, ckw, 1e-6), nc, "tokens/s",
                    f"first {nc} of {T} tokens")
    elif args.op == "indexer":
        # DeepSeek-V4 sparse indexer: 64 index heads of 128 dims for c2's 8192 tokens
        g = torch.Generator().manual_seed(0)
        T, H = 8192, 64
        iq = W.randn_bf16((T, H, 128), g).to(dev)
        pos = torch.randint(0, 65536, (T,), generator=g).to(dev)
        cs = W.make_cos_sin_cache(65536).to(dev)
        iw = W.randn_bf16((T, H), g).to(dev)
        bytes_call = W.indexer_bytes(T, H, 128, args.fp4)

        def make_step(i):
            x = (pos, iq, iw) if i == 0 else (pos.clone(), iq.clone(), iw.clone())
            return lambda: flaggems_vllm.fused_indexer_q_rope_quant(x[0], x[1], cs, x[2], 128 ** -0.5,
                                                                    H ** -0.5, use_fp4=args.fp4)

        kernel = "indexer_token_kernel"  # one token per workgroup (H = 64)
        workload = "T8192_H64_D128" + ("_mxfp4" if args.fp4 else "_fp8")
        config = {"workload": f"fused_indexer_q_rope_quant T=8192, H=64, D=128, "
                              f"{'MXFP4' if args.fp4 else 'FP8'}", "num_tokens": T}
        nc = min(args.cpu_sample_tokens, 1024, T)  # ~1 s per run on 8 cores
        cpos, ciq, ccs, ciw = pos[:nc].cpu(), iq[:nc].cpu(), cs.cpu(), iw[:nc].cpu()
        cpu_case = (lambda: torch_ref.fused_indexer_q_rope_quant(cpos, ciq, ccs, ciw, 128 ** -0.5, H ** -0.5,
                                                                 use_fp4=args.fp4),
                    nc, "tokens/s", f"first {nc} of {T} tokens, all {H} heads")
    elif args.op == "slot_mapping":
        # slots of c4's ragged batch (64 requests) from its block tables
        w_cpu = W.make_workload(4 if args.config == 2 else args.config)
        m = w_cpu.meta
        qsl = torch.zeros(m["new_lens"].numel() + 1, dtype=torch.int32)
        qsl[1:] = torch.cumsum(m["new_lens"], 0)
        T = w_cpu.num_tokens
        qsl_d, pos_d = qsl.to(dev), w_cpu.position_ids.to(dev)
        bt_d = m["block_table"].to(dev)
        out = torch.empty(T, dtype=torch.int64, device=dev)
        bytes_call = T * (8 + 4 + 8) + 4 * qsl.numel()

        def step():
            flaggems_vllm.compute_slot_mapping_parallel(T, T, qsl_d, qsl.numel() - 1, pos_d, bt_d,
                                                        out, 64)

        kernel, workload = "slot_mapping_kernel", f"{w_cpu.name}"
        config = {"workload": f"compute_slot_mapping_parallel over {w_cpu.name}: {T} tokens, "
                              f"{qsl.numel() - 1} requests", "num_tokens": T}
        nreq = min(8, qsl.numel() - 1)
        ns = int(qsl[nreq])
        cpu_case = (lambda: torch_ref.slot_mapping(ns, qsl[:nreq + 1], w_cpu.position_ids, m["block_table"], 64),
                    ns, "tokens/s", f"the first {nreq} of {qsl.numel() - 1} requests ({ns} tokens; "
                                    f"the reference test's per-request loop)")
    elif args.op == "mla":
        # the reference benchmark's MODEL1 sparse decode (batch 512, 64 heads, top-k 128)
        mla_kw = dict(W.MLA_CASES[args.mla_case])
        if args.mla_batch:
            mla_kw["batch"] = args.mla_batch
        if args.mla_heads:
            mla_kw["heads"] = args.mla_heads
        w_cpu = W.make_mla_workload(seed=0, name=args.mla_case, q_scale=0.1, **mla_kw)
        w = w_cpu.to(dev)
        B, SQ, HQ = w.q.shape[:3]
        T = B * SQ
        bytes_call = W.mla_bytes(w_cpu)
        flops_call = W.mla_flops(w_cpu)
        meta, _ = flaggems_vllm.get_mla_metadata()

        def make_step(i):
            wi = w if i == 0 else w_cpu.to(dev)
            out = torch.empty(B, SQ, HQ, 512, dtype=torch.bfloat16, device=dev)
            kw = wi.kwargs()
            return lambda: flaggems_vllm.flash_mla_with_kvcache(wi.q, wi.k_cache, None, None, 512, meta,
                                                                is_fp8_kvcache=True, indices=wi.indices,
                                                                out=out, **kw)

        from flaggems_vllm import _native

        query = _native.lib().fgv_sparse_mla_decode_workspace_bytes
        etopk = w.extra_indices.shape[-1] if w.extra_indices is not None else 0
        entries = w.extra_k_cache.shape[0] * w.extra_k_cache.shape[1] if w.extra_k_cache is not None else 0
        grid = _native.lib().fgv_sparse_mla_decode_grid(B, SQ, HQ, w.indices.shape[-1], etopk)
        expanded = query(B, SQ, HQ, w.indices.shape[-1], etopk, entries) > query(B, SQ, HQ, w.indices.shape[-1],
                                                                                  etopk, 0)
        kernel = {0: "sparse_mla_decode_kernel", 1: "sparse_mla_decode_split_kernel",
                  2: "sparse_mla_decode_pair_kernel"}[grid]
        workload = (f"mla_{args.mla_case}" + (f"_b{B}" if args.mla_batch else "")
                    + (f"_h{HQ}" if args.mla_heads else ""))
        case = W.MLA_CASES[args.mla_case]
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        items = B * SQ * (HQ // 64)
        order = ("items in runs per XCD" if items <= cus else
                 "long items paired with short on shared CUs" if items <= 2 * cus else
                 "longest first in windows of 256" if items <= 4 * cus else "items in order")
        config = {"workload": f"flash_mla_with_kvcache sparse MODEL1 decode '{args.mla_case}': "
                              f"batch {B}, seq_q {SQ}, {HQ} heads, top-k {case['topk']} over "
                              f"{case['num_pages']} pages of 64 x 584 B, top-k lengths, attention sink"
                              + (f", extra top-k {case['extra_topk']} over {case['extra_pages']} pages "
                                 f"of {case['extra_page']}" if "extra_topk" in case else ""),
                  "batch": B, "seq_q": SQ, "num_heads": HQ, "attended_entries": w_cpu.used_tokens(),
                  "flops_per_call": flops_call,
                  "schedule": {0: f"one workgroup per (row, 64-head block): {items} items on {cus} CUs, {order}",
                               1: "balanced split grid + combine kernel",
                               2: "paired grid: one 8-wave workgroup per CU, both halves on each item, "
                                  "a short item after a long one"}[grid]
                              + ("; extra cache expanded to bf16 once per call" if expanded else "")}
    elif args.op == "indexer_k":
        # indexer key quantise + insert at the reference benchmark's shapes
        # (benchmark/test_indexer_k_quant_and_cache.py:97-102)
        if args.indexer_case == "large":
            T, nblk, bs, hd = 65536, 4096, 16, 512
        else:
            T, nblk, bs, hd = W.INDEXER_K_INSERT_CASES[int(args.indexer_case)]
        dtype = torch.float16 if args.fp16 else torch.bfloat16
        k_cpu, cache_cpu, slots_cpu = W.make_indexer_k_insert(T, nblk, bs, hd, dtype)
        bytes_call = W.indexer_k_insert_bytes(T - 1, hd)  # the last token is padding (slot -1)
        k_d, slots_d = k_cpu.to(dev), slots_cpu.to(dev)

        def make_step(i):
            x = (k_d, cache_cpu.to(dev), slots_d) if i == 0 else (k_d.clone(), cache_cpu.to(dev), slots_d.clone())
            return lambda: flaggems_vllm.indexer_k_quant_and_cache(x[0], x[1], x[2], 128, "ue8m0")

        kernel = "indexer_k_quant_kernel"
        workload = f"T{T}_hd{hd}_bs{bs}" + ("_fp16" if args.fp16 else "_bf16")
        config = {"workload": f"indexer_k_quant_and_cache T={T}, head_dim={hd}, {nblk} blocks x {bs} slots, "
                              f"{'fp16' if args.fp16 else 'bf16'} keys, UE8M0 scales", "num_tokens": T,
                  "head_dim": hd, "block_size": bs}
        nc = min(T, 8192)
        ck, cc, cs_ = k_cpu[:nc], cache_cpu.clone(), slots_cpu[:nc]
        cpu_case = (lambda: torch_ref.indexer_k_quant_and_cache(ck, cc, cs_, 128, "ue8m0"), nc, "tokens/s",
                    f"first {nc} of {T} tokens")
    elif args.op == "indexer_k_gather":
        # gather of a batch's cached indexer keys at the reference benchmark's
        # shapes (benchmark/test_cp_gather_indexer_k_quant_cache.py:125-131)
        if args.indexer_case == "large":
            B, L, bs, hd = 64, 1024, 16, 512
        else:
            B, L, bs, hd = W.INDEXER_K_GATHER_CASES[int(args.indexer_case)]
        cache_cpu, kf_cpu, ks_cpu, bt_cpu, cu_cpu = W.make_indexer_k_gather([L] * B, bs, hd)
        T = B * L
        bytes_call = W.indexer_k_gather_bytes(T, hd)
        bt_d, cu_d = bt_cpu.to(dev), cu_cpu.to(dev)

        def make_step(i):
            c, kf, ks = cache_cpu.to(dev), kf_cpu.to(dev), ks_cpu.to(dev)
            return lambda: flaggems_vllm.cp_gather_indexer_k_quant_cache(c, kf, ks, bt_d, cu_d)

        kernel = "indexer_k_gather_kernel"
        workload = f"B{B}_L{L}_hd{hd}_bs{bs}"
        config = {"workload": f"cp_gather_indexer_k_quant_cache batch={B} x {L} tokens, head_dim={hd}, "
                              f"block {bs}", "num_tokens": T, "batch": B, "head_dim": hd, "block_size": bs}
        nb = max(1, min(B, 8192 // L))
        ck2, cs2 = kf_cpu[:nb * L].clone(), ks_cpu[:nb * L].clone()
        cpu_case = (lambda: torch_ref.cp_gather_indexer_k_quant_cache(cache_cpu, ck2, cs2, bt_cpu[:nb],
                                                                      cu_cpu[:nb + 1]),
                    nb * L, "tokens/s", f"first {nb} of {B} requests ({nb * L} tokens; the reference "
                                        f"test's per-token loop)")
    elif args.op == "mqa_logits":
        # the sparse indexer's prefill logits at the reference benchmark's
        # largest shape (benchmark/test_fp8_fp4_mqa_logits.py:61-72), H = 64, D = 128
        M, N = (int(x) for x in args.mqa_shape.split(","))
        q, kv, w, ks, ke = W.make_mqa_logits_inputs(M, N, fp4=args.fp4)
        d = ((q[0].to(dev), q[1].to(dev) if q[1] is not None else None), (kv[0].to(dev), kv[1].to(dev)),
             w.to(dev), ks.to(dev), ke.to(dev))
        T = M
        flops_call = W.mqa_logits_flops(M, N)
        bytes_call = M * 64 * (68 if args.fp4 else 128) + M * 64 * 4 + N * 132 + 4 * M * N

        def step():  # MFMA-bound: q (M x 8 KiB) and K stay cache-resident by design
            flaggems_vllm.fp8_fp4_mqa_logits(*d[:2], d[2], d[3], d[4], clean_logits=True)

        kernel = "mqa_logits_kernel"
        workload = f"M{M}_N{N}_H64" + ("_mxfp4" if args.fp4 else "_fp8")
        config = {"workload": f"fp8_fp4_mqa_logits M={M} queries x N={N} keys, H=64, D=128, "
                              f"{'MXFP4' if args.fp4 else 'FP8'} q, FP8 k, clean_logits (ks=0, ke=N)",
                  "num_queries": M, "num_keys": N, "flops_per_call": flops_call}
        nc = max(1, min(M, 4))
        qc = (q[0][:nc], q[1][:nc] if q[1] is not None else None)
        cpu_case = (lambda: torch_ref.mqa_logits(qc, kv, w[:nc], ks[:nc], ke[:nc], True), nc, "queries/s",
                    f"first {nc} of {M} queries against all {N} keys (the reference test's float32 loop)")
    elif args.op == "paged_mqa_logits":
        # the sparse indexer's decode logits over the paged key cache at a
        # reference benchmark shape (benchmark/test_fp8_fp4_paged_mqa_logits.py:31-40)
        B, nn, L = (int(x) for x in args.paged_shape.split(","))
        q, cache, w, ctx, bt = W.make_paged_mqa_inputs(B, nn, L, fp4=args.fp4)
        T = B * nn
        mml = W.PAGED_MAX_MODEL_LEN
        bytes_call = W.paged_mqa_logits_bytes(ctx.reshape(-1), T, 64, mml, args.fp4)
        flops_call = int(ctx.reshape(-1).sum()) * 2 * 64 * 128
        dq = (q[0].to(dev), q[1].to(dev) if q[1] is not None else None)
        d_w, d_ctx, d_bt = w.to(dev), ctx.to(dev), bt.to(dev)

        def make_step(i):
            c = cache.to(dev)
            return lambda: flaggems_vllm.fp8_fp4_paged_mqa_logits(dq, c, d_w, d_ctx, d_bt, None, mml)

        kernel = "paged_mqa_logits_kernel"
        workload = f"B{B}_N{nn}_L{L}" + ("_mxfp4" if args.fp4 else "_fp8")
        config = {"workload": f"fp8_fp4_paged_mqa_logits batch={B}, next_n={nn}, contexts ~{L} "
                              f"(uniform 0.7-1.3x), 64-entry blocks, max_model_len {mml}, H=64, D=128, "
                              f"{'MXFP4' if args.fp4 else 'FP8'} q", "rows": T,
                  "context_positions": int(ctx.reshape(-1).sum()), "flops_per_call": flops_call}
        nb = 1
        qc = (q[0][:nb], q[1][:nb] if q[1] is not None else None)
        cpu_case = (lambda: torch_ref.paged_mqa_logits(qc, cache, w[:nb * nn], ctx[:nb], bt[:nb], mml, False),
                    nb * nn, "rows/s", f"first {nb} of {B} sequences (the reference test's per-row gather "
                                       f"and float32 loop)")
    elif args.op == "topk":
        # the sparse indexer's top-k per row at the reference benchmark's shapes
        # (benchmark/test_top_k_per_row_decode.py:70-83, benchmark/test_top_k_per_row_prefill.py:122-132)
        R, V, k, s0 = {"decode": (496, 262144, 512, 262144), "prefill": (64, 129280, 1024, 129280),
                       "prefill_short": (16383, 4095, 512, 4352)}[args.topk_case]
        g = torch.Generator().manual_seed(42)
        buf_cpu = torch.randn((R - 1) * s0 + V, generator=g)
        T = R
        bytes_call = R * V * 4 + R * k * 4 + R * 8

        def make_step(i):
            buf = buf_cpu.to(dev)
            lg = torch.as_strided(buf, (R, V), (s0, 1))
            idx = torch.empty((R, k), dtype=torch.int32, device=dev)
            if args.topk_case == "decode":
                seq = torch.full((R,), V, dtype=torch.int32, device=dev)
                return lambda: flaggems_vllm.top_k_per_row_decode(lg, 1, seq, idx, R, s0, 1, k)
            st = torch.zeros(R, dtype=torch.int32, device=dev)
            en = torch.full((R,), V, dtype=torch.int32, device=dev)
            return lambda: flaggems_vllm.top_k_per_row_prefill(lg, st, en, idx, R, s0, 1, k)

        from flaggems_vllm import _native

        split = _native.lib().fgv_top_k_per_row_workspace_bytes(R, V, k) > 0
        kernel = "top_k_part_kernel" if split else "top_k_per_row_kernel"
        workload = f"{args.topk_case}_R{R}_V{V}_k{k}"
        config = {"workload": f"top_k_per_row_{'decode' if args.topk_case == 'decode' else 'prefill'} "
                              f"{R} rows x {V} float32 logits (row stride {s0}), top_k {k}, full rows",
                  "rows": R, "vocab": V, "top_k": k,
                  "schedule": "rows split into parts of 16384 + merge kernel (kernel_us covers both)" if split
                  else "one workgroup per row"}
        nr = max(1, min(R, 8 if V > 100000 else 256))
        lg_cpu = torch.as_strided(buf_cpu, (R, V), (s0, 1))[:nr].contiguous()
        cpu_case = (lambda: torch.topk(lg_cpu, k, dim=1, largest=True, sorted=False), nr, "rows/s",
                    f"first {nr} of {R} rows: torch.topk on the CPU (the reference test's reference)")
    elif args.op == "einsum":
        # the block-FP8 grouped projection at the reference benchmark's shapes
        # (benchmark/test_fp8_einsum.py: (h, r, d) groups flash / pro, batches 1..32768)
        grp, eb = args.einsum_case.split(",")
        H, R, D = {"flash": (8, 4096, 1024), "pro": (16, 7168, 1024)}[grp]
        Bt = int(eb)
        g = torch.Generator().manual_seed(0)

        def codes(*shape):
            c = torch.randint(0, 256, shape, generator=g, dtype=torch.uint8)
            c[(c & 0x7F) == 0x7F] = 0x38
            return c.view(torch.float8_e4m3fn)

        x_cpu, y_cpu = codes(Bt, H, R), codes(H, D, R)
        xs_cpu = torch.ldexp(torch.ones(Bt, H, R // 128), torch.randint(-12, -5, (Bt, H, R // 128), generator=g))
        ys_cpu = torch.rand(H, D // 128, R // 128, generator=g) * 2 ** -6 + 2 ** -9
        T = Bt
        bytes_call = Bt * H * R + Bt * H * (R // 128) * 4 + H * D * R + H * (D // 128) * (R // 128) * 4 + Bt * H * D * 2
        flops_call = 2 * Bt * H * R * D

        def make_step(i):
            x, xs, y, ys = x_cpu.to(dev), xs_cpu.to(dev), y_cpu.to(dev), ys_cpu.to(dev)
            out = torch.empty((Bt, H, D), dtype=torch.bfloat16, device=dev)
            return lambda: flaggems_vllm.fp8_einsum("bhr,hdr->bhd", x, xs, y, ys, out=out)

        # the launcher's choice (fp8_einsum.hip launch_einsum): split-K tiles when the wrapper's
        # workspace query asks for one; else skinny up to 64 rows, and up to 128 while 128-row tiles
        # would fill fewer than half of the 256 CUs
        from flaggems_vllm import _native

        split = _native.lib().fgv_fp8_einsum_workspace_bytes(Bt, H, R, D) > 0
        skinny = not split and (Bt <= 64 or (Bt <= 128 and 2 * ((Bt + 127) // 128) * (D // 128) * H < 256))
        kernel = "fp8_einsum_skinny_kernel" if skinny else "fp8_einsum_tile_kernel"
        workload = f"{grp}_b{Bt}"
        config = {"workload": f"fp8_einsum 'bhr,hdr->bhd' {grp}: b {Bt}, h {H}, r {R}, d {D}, e4m3fn x and y, "
                              f"float32 128 / 128x128 block scales, bf16 out",
                  "b": Bt, "h": H, "r": R, "d": D, "flops_per_call": flops_call,
                  "schedule": "split-K tiles + fp8_einsum_reduce_kernel (kernel_us covers both)" if split
                  else "one workgroup per output tile"}
        nb = max(1, min(Bt, 16))
        xd = x_cpu[:nb].float() * xs_cpu[:nb].repeat_interleave(128, dim=2)
        yd = (y_cpu.float() * ys_cpu.repeat_interleave(128, dim=1).repeat_interleave(128, dim=2))
        cpu_case = (lambda: torch.einsum("bhr,hdr->bhd", xd, yd), nb, "rows/s",
                    f"first {nb} of {Bt} rows: the reference test's dequantise-then-einsum in float32 on the CPU "
                    f"(dequantisation outside the timing)")
    elif args.op == "mla_sparse":
        # sparse MLA prefill at a reference benchmark case
        # (benchmark/test_flash_mla_sparse_fwd.py:105-121: s_q 4096 with the attention sink)
        s_kv, topk, h_q, d_qk = W.MLA_SPARSE_CASES[args.mla_sparse_case]
        T = 4096
        w_cpu = W.make_mla_sparse_inputs(T, s_kv, topk, h_q=h_q, d_qk=d_qk, have_attn_sink=True, seed=0,
                                         sm_scale=d_qk ** -0.5)
        bytes_call = W.mla_sparse_bytes(w_cpu)
        flops_call = W.mla_sparse_flops(w_cpu)

        def make_step(i):
            wd = w_cpu.to(dev)
            return lambda: flaggems_vllm.flash_mla_sparse_fwd(*wd.args())

        kernel = "sparse_mla_prefill_kernel"
        workload = args.mla_sparse_case
        config = {"workload": f"flash_mla_sparse_fwd s_q {T}, s_kv {s_kv}, topk {topk}, h_q {h_q}, d_qk {d_qk}, "
                              f"d_v 512, attention sink", "s_q": T, "s_kv": s_kv, "topk": topk, "h_q": h_q,
                  "d_qk": d_qk, "flops_per_call": flops_call,
                  "gather_bytes_note": "bytes_per_call counts each attended kv row once per 64-head block; "
                                       "the rows are re-read from L2 / MALL, not HBM"}
        nt = 16
        sub = [w_cpu.q[:nt], w_cpu.kv, w_cpu.indices[:nt], w_cpu.sm_scale, w_cpu.attn_sink]
        cpu_case = (lambda: torch_ref.flash_mla_sparse_fwd(*sub), nt, "tokens/s",
                    f"first {nt} of {T} tokens: the reference test's torch definition in float32 on the CPU")
    elif args.op == "copy":
        n = 512 << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        T, bytes_call = n, 2 * n

        def step():
            dst.copy_(src)

        kernel, workload = "copy", "512MiB"
        config = {"workload": "calibration: torch device copy, 512 MiB read + 512 MiB write"}
        args.no_cpu_baseline = True
    else:
        T_inv, H_inv, G_inv = (int(x) for x in args.inv_shape.split(","))
        w_cpu = W.make_inv_rope_workload(T_inv, H_inv, G_inv, seed=0)
        w = w_cpu.to(dev)
        T, H = w.o.shape[0], w.o.shape[1]
        bytes_call = W.inv_rope_bytes(T, H, args.tma)

        def make_step(i):
            wi = w if i == 0 else w_cpu.to(dev)
            return lambda: flaggems_vllm.fused_inv_rope_fp8_quant(wi.o, wi.positions, wi.cos_sin_cache,
                                                                  wi.n_groups, wi.heads_per_group,
                                                                  tma_aligned_scales=args.tma)

        kernel = "inv_rope_fp8_quant_kernel"
        workload = f"T{T}_H{H}_G{G_inv}" + ("_ue8m0" if args.tma else "_f32")
        config = {"workload": f"fused_inv_rope_fp8_quant T={T}, H={H}, G={G_inv}, "
                              f"{'packed UE8M0' if args.tma else 'fp32'} scales",
                  "num_tokens": T, "num_heads": H, "n_groups": G_inv}

    n_sets = 1
    if args.op in ("main", "gather", "rmsnorm", "indexer", "mla", "inv_rope", "indexer_k", "indexer_k_gather",
                   "paged_mqa_logits", "topk", "einsum", "mla_sparse"):
        step, n_sets = rotating(make_step, bytes_call)
    if n_sets == 1:
        config["input_sets"] = "one input set"
    else:
        span = n_sets * bytes_call
        config["input_sets"] = (f"{n_sets} rotating device copies of the inputs ({span / 1e6:.0f} MB of calls "
                                + ("in turn > 2 x 256 MB MALL)" if span > 2 * MALL_BYTES
                                   else "in turn, within the 256 MB MALL: cache-warm)"))
    ms_step, t_kernel, timing = time_gpu(step, args.steps, args.warmup)
    median_us = median_call_us(step, max(20, args.steps))
    achieved = bytes_call / t_kernel / 1e9
    if args.op in ("mla", "mla_sparse"):
        config["mfma_tflops"] = flops_call / t_kernel / 1e12
        config["mfma_frac_of_bf16_dense_peak"] = flops_call / t_kernel / 2.5e15
    if args.op in ("mqa_logits", "paged_mqa_logits", "einsum"):
        config["mfma_tflops"] = flops_call / t_kernel / 1e12
        config["mfma_frac_of_fp8_dense_peak"] = flops_call / t_kernel / 5.0e15
    traffic = measured_traffic(kernel, workload)
    result = {
        "metric": METRIC,
        "value": T / ms_step,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"mla": "bf16", "mla_sparse": "bf16", "slot_mapping": "int64", "copy": "u8", "indexer_k_gather": "u8",
                  "mqa_logits": "fp4 x fp8 -> f32" if args.fp4 else "fp8 -> f32",
                  "paged_mqa_logits": "fp4 x fp8 -> f32" if args.fp4 else "fp8 -> f32",
                  "einsum": "fp8 -> f32 -> bf16"}.get(args.op, "f32"),
        "data": ("synthetic: seeded q ~ N(0,1)/10 bf16, cache NoPE ~ N(0,0.1) quantised to e4m3 + "
                 "E8M0 per 64, RoPE ~ N(0,0.1) bf16, uniform indices and top-k lengths, sink ~ N(0,1)"
                 if args.op == "mla" else
                 "synthetic: seeded N(0,1) keys, distinct random slots (last one -1), cache pre-filled with "
                 "e4m3 codes of N(0,1) and scales U[0.01, 1.01) as the reference's tests fill it"
                 if args.op in ("indexer_k", "indexer_k_gather") else
                 "synthetic: seeded q, k ~ N(0,1) (bf16, then e4m3fn or MXFP4 q and per-token FP8 k), "
                 "weights N(0,1) (|N(0,1)| dense), as the reference's tests draw them"
                 if args.op in ("mqa_logits", "paged_mqa_logits") else
                 "synthetic: seeded N(0,1) float32 logits, as the reference's benchmark draws them"
                 if args.op == "topk" else
                 "synthetic: seeded uniform finite e4m3fn codes, power-of-two x scales 2^-12..2^-6, "
                 "y block scales U[2^-9, 2^-9 + 2^-6)"
                 if args.op == "einsum" else
                 "synthetic: seeded q, kv ~ N(0,1)/10 + offset (bf16), index rows distinct random ids "
                 "(arithmetic progressions mod s_kv), sink ~ N(0,1) with +-inf entries, as the reference's "
                 "benchmark draws them"
                 if args.op == "mla_sparse" else
                 "synthetic: seeded N(0,1) bf16 q/kv, fp32 cos/sin (theta 1e4), vLLM-style paged slots"),
        "config": config,
        "kernel_us": t_kernel * 1e6,
        "kernel_timing": timing,
        "kernel_us_median_per_call": median_us,
        "gbps": achieved,
        "bytes_per_call": bytes_call,
        "bytes_per_token": bytes_call / T,
        # HBM read + write bytes from the committed rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE,
        # calibrated), per token and over the kernel time measured here
        "traffic_bytes_per_token": traffic / T if traffic else None,
        "traffic_gbps": traffic / t_kernel / 1e9 if traffic else None,
        "roofline": ({"bound": "mfma", "achieved": flops_call / t_kernel / 1e12, "peak": 5000.0,
                      "unit": "TFLOP/s", "frac": flops_call / t_kernel / 5.0e15, "traffic": traffic,
                      "kernel": kernel, "peak_note": "MI355X dense FP8 MFMA"}
                     if args.op == "mqa_logits" or (args.op == "einsum" and flops_call / bytes_call > 625) else
                     {"bound": "mfma", "achieved": flops_call / t_kernel / 1e12, "peak": 2500.0,
                      "unit": "TFLOP/s", "frac": flops_call / t_kernel / 2.5e15, "traffic": traffic,
                      "kernel": kernel, "peak_note": "MI355X dense bf16 MFMA"}
                     if args.op == "mla_sparse" else
                     {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                      "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic,
                      "kernel": kernel}),
    }
    if not args.no_cpu_baseline:
        if args.op == "main":
            result["cpu_baseline"] = cpu_baseline_main(w_cpu, args.cpu_sample_tokens,
                                                       args.cpu_seconds)
        elif args.op == "mla":
            result["cpu_baseline"] = cpu_baseline_mla(w_cpu, 64, args.cpu_seconds)
        elif cpu_case is not None:
            result["cpu_baseline"] = cpu_baseline_port(*cpu_case, args.cpu_seconds)
        else:
            result["cpu_baseline"] = cpu_baseline_inv(w_cpu, args.tma, args.cpu_sample_tokens,
                                                      args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
