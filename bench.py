"""Benchmark of the MI355X attention backend for gemma4-rs.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one global-layer decode-attention call (Gemma 4 E2B shape: 8 query
heads sharing 1 KV head, head_dim 512, proportional NEOX RoPE, context 4096,
query at position 4095), on f32 inputs already resident in HBM.  Each step
reads a different copy of the K/V cache from a pool larger than the 256 MB
Infinity Cache, so every step streams its K/V from HBM.

Printed: one JSON line.  `value` is the achieved HBM bandwidth of the step in
GB/s (algorithmic bytes: the K and V rows attended, q and the output, each
once); `ms_per_step` is the wall time per step; `roofline` relates the decode
kernels' time to MI355X's 8 TB/s; `cpu_baseline` is the oracle (the C
restatement of the reference's CPU attention, same `concat` copy and per-head
thread pool) timed on this host's cores on a bounded sample of the same step.
`workloads` carries the other measured shapes (sliding decode, the 35-layer
stack, 2048-token prefill, the ragged 32-sequence batch, the layer drivers with
their fused input preparation, the Q8_0 mat-vecs of the output head and a
projection).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "gemma4-rs_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
F32_MFMA_PEAK_TFLOPS = 157.3
N_HEADS, N_KV = 8, 1
EPS = 1e-6
LOCAL_BASE, GLOBAL_BASE = 10000.0, 1000000.0
WINDOW = 512
MALL_BYTES = 256 << 20


def decode_bytes(rows, d):
    """Algorithmic bytes of one decode step: K and V rows once, q and out."""
    return rows * 2 * N_KV * d * 4 + 2 * N_HEADS * d * 4


def prefill_flops(N, window, d):
    """4 * heads * d FLOP per attended (query, key) pair (QK^T and PV)."""
    pairs = sum(min(i + 1, window) if window else i + 1 for i in range(N))
    return 4 * N_HEADS * d * pairs


class Prep:
    """Synthetic inputs built on the device with the backend's own kernels:
    N(0,1) draws, per-head RMS norm (unit weight), NEOX RoPE."""

    def __init__(self, ctx, torch, seed):
        self.ctx, self.torch = ctx, torch
        self.gen = torch.Generator(device="cuda")
        self.gen.manual_seed(seed)

    def randn(self, *shape):
        return self.torch.randn(*shape, device="cuda", generator=self.gen, dtype=self.torch.float32)

    def rows(self, n_rows, d, pos0, base, freqs, rope=True, heads=1):
        x = self.randn(n_rows, heads * d)
        self.ctx.rms_norm_rows(x, n_rows * heads, d, None, EPS, x)
        if rope:
            self.ctx.rope_neox_rows(x, n_rows, heads, d, d, pos0, base, freqs)
        return x

    def rope_freqs(self, d):
        return self.torch.rand(d // 2, device="cuda", generator=self.gen) * 7.0 + 1.0


def time_steps(torch, fn, steps, warmup, block=1):
    """Runs `warmup` eager steps, captures steps 0..block-1 into one HIP graph,
    then times exactly `steps` steps (whole graph replays, the remainder
    eagerly) between synchronisations.  fn(i) launches step i on the current
    stream.  Returns (wall seconds, event seconds) for the timed steps."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(block):
            fn(i)
    torch.cuda.synchronize()
    graph.replay()  # first replay uploads the graph
    torch.cuda.synchronize()
    replays, rest = divmod(steps, block)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for _ in range(replays):
        graph.replay()
    for i in range(rest):
        fn(i)
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) * 1e-3


def bench_global_decode(ctx, torch, prep, steps, warmup, T=4096, d=512):
    freqs = prep.rope_freqs(d)
    per_copy = 2 * T * d * 4
    copies = max(2, int(1.5 * MALL_BYTES // per_copy) + 1)
    Ks, Vs = [], []
    for _ in range(copies):
        Ks.append(prep.rows(T, d, 0, GLOBAL_BASE, freqs))
        Vs.append(prep.rows(T, d, 0, 0.0, None, rope=False))
    q = prep.rows(1, d, T - 1, GLOBAL_BASE, freqs, heads=N_HEADS)
    out = torch.zeros(N_HEADS * d, device="cuda")

    def step(i):
        c = i % copies
        ctx.attend_decode(q, Ks[c], Vs[c], 0, T, N_HEADS, N_KV, d, out)

    wall, ev = time_steps(torch, step, steps, warmup, block=copies)
    ctx.check_status()
    # the same step with one resident copy (served from the Infinity Cache)
    wall_w, ev_w = time_steps(torch, lambda i: ctx.attend_decode(q, Ks[0], Vs[0], 0, T, N_HEADS, N_KV, d, out),
                              steps, warmup, block=copies)
    host = {"q": q.cpu().numpy(), "K": Ks[0].cpu().numpy(), "V": Vs[0].cpu().numpy()}
    return {"wall": wall, "event": ev, "wall_warm": wall_w, "event_warm": ev_w, "copies": copies,
            "bytes": decode_bytes(T, d), "host": host}


def bench_sliding_decode(ctx, torch, prep, steps, warmup, T=64, d=256):
    K = prep.rows(T, d, 0, LOCAL_BASE, None)
    V = prep.rows(T, d, 0, 0.0, None, rope=False)
    q = prep.rows(1, d, T - 1, LOCAL_BASE, None, heads=N_HEADS)
    out = torch.zeros(N_HEADS * d, device="cuda")
    wall, ev = time_steps(torch, lambda i: ctx.attend_decode(q, K, V, 0, T, N_HEADS, N_KV, d, out), steps, warmup,
                          block=20)
    ctx.check_status()
    return {"us_per_layer": ev / steps * 1e6, "wall_us_per_layer": wall / steps * 1e6,
            "bytes": decode_bytes(T, d)}


def bench_stack(ctx, torch, prep, g4hip, steps, warmup, ctx_len=8192):
    """35-layer E2B stack, one decode step at position ctx_len-1: each layer's
    attention over its source layer's cache (owners 0..14, shared 15..34)."""
    n_layers, shared = 35, 20
    freqs = prep.rope_freqs(512)
    caches = {}
    plan = []
    total_bytes = 0
    for layer in range(n_layers):
        glob = g4hip.layer_attention_kind(n_layers, layer) == "global"
        d = 512 if glob else 256
        src = g4hip.kv_source_layer(n_layers, shared, layer)
        if src == layer:
            caches[layer] = (prep.rows(ctx_len, d, 0, GLOBAL_BASE if glob else LOCAL_BASE, freqs if glob else None),
                             prep.rows(ctx_len, d, 0, 0.0, None, rope=False))
        r = g4hip.windowed_len(ctx_len, WINDOW) if not glob else range(0, ctx_len)
        q = prep.rows(1, d, ctx_len - 1, GLOBAL_BASE if glob else LOCAL_BASE, freqs if glob else None,
                      heads=N_HEADS)
        plan.append((src, r.start, r.stop, d, q, torch.zeros(N_HEADS * d, device="cuda")))
        total_bytes += decode_bytes(r.stop - r.start, d)

    def step(i):
        for src, b, e, d, q, out in plan:
            K, V = caches[src]
            ctx.attend_decode(q, K, V, b, e, N_HEADS, N_KV, d, out)

    wall, ev = time_steps(torch, step, steps, warmup)
    ctx.check_status()
    n_glob = sum(1 for p in plan if p[3] == 512)
    return {"us_per_stack": ev / steps * 1e6, "wall_us_per_stack": wall / steps * 1e6,
            "us_per_layer_mean": ev / steps / n_layers * 1e6, "bytes_per_stack": total_bytes,
            "gbs": total_bytes / (ev / steps) / 1e9, "layers": n_layers, "global_layers": n_glob}


def bench_prefill(ctx, torch, prep, steps, warmup, N=2048):
    """Causal prefill of an N-token prompt through one sliding and one global
    layer.  The timed steps replay as one captured graph (a graph per step
    adds a launch gap of about 4 us to each 0.1-0.4 ms step), after
    `warmup` untimed steps: the clocks need tens of milliseconds of this
    load to settle (global layer 348 us after 2 warm-up steps, 322 us after
    50, measured in one process)."""
    res = {}
    total_flops, total_s = 0, 0.0
    for name, d, window, base in (("sliding_d256_W512", 256, WINDOW, LOCAL_BASE), ("global_d512", 512, 0, GLOBAL_BASE)):
        freqs = prep.rope_freqs(d) if not window else None
        K = prep.rows(N, d, 0, base, freqs)
        V = prep.rows(N, d, 0, 0.0, None, rope=False)
        q = prep.rows(N, d, 0, base, freqs, heads=N_HEADS)
        out = torch.zeros(N * N_HEADS * d, device="cuda")
        wall, ev = time_steps(torch, lambda i: ctx.attend_prefill(q, K, V, 0, N, window, N_HEADS, N_KV, d, out),
                              steps, warmup, block=steps)
        ctx.check_status()
        fl = prefill_flops(N, window, d)
        res[name] = {"us": ev / steps * 1e6, "tflops": fl / (ev / steps) / 1e12, "flops": fl}
        total_flops += fl
        total_s += ev / steps
    res["both_layers_tflops"] = total_flops / total_s / 1e12
    res["frac_of_f32_mfma_peak"] = res["both_layers_tflops"] / F32_MFMA_PEAK_TFLOPS
    return res


def bench_layer_steps(ctx, torch, prep, steps, warmup, T=4096, N=2048):
    """The launches of the layer drivers, input preparation included: a
    global-layer decode step over T rows as g4_layer_attention runs it (one
    fused launch, g4_decode_step_fused: q norm + RoPE, the new row's k/v norm +
    RoPE and its append, attention over the T rows, plus the split merge),
    beside the two-launch form it replaced (g4_prepare_qkv, then
    g4_attend_decode); and a 2048-token prompt through one sliding and one
    global layer (g4_layer_prefill: the fused preparation of all N tokens with
    their appends, then the prefill).  The cache rows written are the same
    each step, so the steps replay as a graph."""
    res = {}
    d = 512
    freqs = prep.rope_freqs(d)
    K = prep.rows(T, d, 0, GLOBAL_BASE, freqs)
    V = prep.rows(T, d, 0, 0.0, None, rope=False)
    q, k, v = prep.randn(N_HEADS * d), prep.randn(N_KV * d), prep.randn(N_KV * d)
    wq, wk = torch.ones(d, device="cuda"), torch.ones(d, device="cuda")
    out = torch.zeros(N_HEADS * d, device="cuda")
    row = (T - 1) * N_KV * d
    k_row, v_row = K.view(-1)[row:], V.view(-1)[row:]

    def fused(i):
        ctx.decode_step_fused(q, k, v, wq, wk, EPS, GLOBAL_BASE, freqs, T - 1, K, V, N_KV * d, T, k_row, v_row,
                              N_HEADS, N_KV, d, out)

    wall, ev = time_steps(torch, fused, steps, warmup, block=20)
    ctx.check_status()
    res["decode_global_d512_ctx4096_layer_step"] = {"us_per_layer": ev / steps * 1e6,
                                                    "wall_us_per_layer": wall / steps * 1e6,
                                                    "note": "K/V resident (one copy): one fused launch + merge"}

    def two_launch(i):
        # The preparation works in place: repeated steps re-prepare q/k/v
        # (the norm keeps them bounded), as the step's own launches would.
        ctx.prepare_qkv(q, k, v, 1, T - 1, N_HEADS, N_KV, d, wq, wk, EPS, GLOBAL_BASE, freqs,
                        k_rows=k_row, v_rows=v_row, row_stride=N_KV * d)
        ctx.attend_decode(q, K, V, 0, T, N_HEADS, N_KV, d, out)

    wall, ev = time_steps(torch, two_launch, steps, warmup, block=20)
    ctx.check_status()
    res["decode_global_d512_ctx4096_two_launch_step"] = {
        "us_per_layer": ev / steps * 1e6,
        "note": "the same step as a preparation launch, then the decode"}
    del K, V
    total_flops, total_s = 0, 0.0
    psteps = max(5, steps // 20)
    for name, d, window, base in (("sliding_d256_W512", 256, WINDOW, LOCAL_BASE), ("global_d512", 512, 0, GLOBAL_BASE)):
        f = prep.rope_freqs(d) if not window else None
        Kc = torch.zeros(N * N_KV * d, device="cuda")
        Vc = torch.zeros(N * N_KV * d, device="cuda")
        q, k, v = prep.randn(N * N_HEADS * d), prep.randn(N * N_KV * d), prep.randn(N * N_KV * d)
        wq, wk = torch.ones(d, device="cuda"), torch.ones(d, device="cuda")
        out = torch.zeros(N * N_HEADS * d, device="cuda")

        def pstep(i):
            ctx.prepare_qkv(q, k, v, N, 0, N_HEADS, N_KV, d, wq, wk, EPS, base, f, k_rows=Kc, v_rows=Vc,
                            row_stride=N_KV * d)
            ctx.attend_prefill(q, Kc, Vc, 0, N, window, N_HEADS, N_KV, d, out)

        wall, ev = time_steps(torch, pstep, psteps, max(2, warmup // 4), block=psteps)
        ctx.check_status()
        fl = prefill_flops(N, window, d)
        res[f"prefill_2048_{name}_layer"] = {"us": ev / psteps * 1e6, "tflops": fl / (ev / psteps) / 1e12}
        total_flops += fl
        total_s += ev / psteps
    res["prefill_2048_both_layers_tflops_with_preparation"] = total_flops / total_s / 1e12
    return res


def bench_matvec(ctx, torch, steps, warmup, rows=262144, cols=1536, cap=30.0):
    """The output head of E2B as the reference benchmarks it
    (crates/llm-backend-cpu/examples/bench_matvec.rs): a 262,144 x 1536 Q8_0
    matrix (428 MB, larger than the Infinity Cache) against the quantized
    final hidden state, with the logit soft-cap fused; plus the E2B global
    layer's q projection (4096 x 1536)."""
    res = {}
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    for name, r, c, softcap in (("logits_262144x1536_softcap", rows, cols, cap), ("q_proj_4096x1536", 4096, cols, None)):
        nb = c // 32
        w = torch.randint(-127, 128, (r, nb, 34), dtype=torch.int32, device="cuda", generator=gen).to(torch.uint8)
        w[:, :, 0:2] = torch.tensor([0x1F, 0x21], dtype=torch.uint8, device="cuda")  # f16 scale ~0.01
        w = w.reshape(-1)
        x = torch.randn(c, device="cuda", generator=gen)
        out = torch.empty(r, device="cuda")

        def step(i):  # quantize_q8_0 + mat-vec (+ soft-cap), one launch
            if softcap is None:
                ctx.project_q8_0(w, r, c, x, out)
            else:
                ctx.logits_q8_0(w, r, c, x, softcap, out)

        wall, ev = time_steps(torch, step, steps, warmup, block=10)
        nbytes = r * nb * 34 + c * 4 + r * 4
        res[name] = {"us": ev / steps * 1e6, "gbs": nbytes / (ev / steps) / 1e9, "bytes": nbytes,
                     "frac_of_hbm_peak": nbytes / (ev / steps) / 1e9 / HBM_PEAK_GBS}
        del w
    return res


def bench_ragged(ctx, torch, prep, steps, warmup, B=32, seed=2024):
    import numpy as np
    lens = np.random.default_rng(seed).integers(1024, 32768 + 1, size=B).astype(np.int64)
    res = {}
    for name, d, glob in (("global_d512", 512, True), ("sliding_d256_W512", 256, False)):
        freqs = prep.rope_freqs(d) if glob else None
        base = GLOBAL_BASE if glob else LOCAL_BASE
        row0 = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        begin = np.array([0 if glob else max(0, int(L) - WINDOW) for L in lens], np.int64)
        total = int(lens.sum())
        K = prep.rows(total, d, 0, base, freqs)  # positions are not per-sequence here: timing only
        V = prep.rows(total, d, 0, 0.0, None, rope=False)
        q = prep.rows(B, d, 0, base, freqs, heads=N_HEADS)
        out = torch.zeros(B * N_HEADS * d, device="cuda")
        t_row0, t_b, t_e = (torch.from_numpy(a).cuda() for a in (row0, begin, lens))
        max_len = int((lens - begin).max())
        wall, ev = time_steps(torch, lambda i: ctx.attend_decode_batch(q, K, V, t_row0, t_b, t_e, max_len, N_HEADS,
                                                                       N_KV, d, out), steps, warmup)
        ctx.check_status()
        nbytes = sum(decode_bytes(int(lens[s] - begin[s]), d) for s in range(B))
        res[name] = {"us": ev / steps * 1e6, "gbs": nbytes / (ev / steps) / 1e9, "bytes": nbytes,
                     "frac_of_hbm_peak": nbytes / (ev / steps) / 1e9 / HBM_PEAK_GBS}
        del K, V
        torch.cuda.empty_cache()
    res["lengths"] = {"min": int(lens.min()), "max": int(lens.max()), "mean": float(lens.mean())}
    return res


def bench_copy(torch, steps, nbytes=256 << 20):
    """A plain device-to-device copy of known size: the reference point that
    scales the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    src = torch.empty(nbytes // 4, device="cuda").uniform_()
    dst = torch.empty_like(src)
    wall, ev = time_steps(torch, lambda i: dst.copy_(src), steps, 2)
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": ev / steps * 1e6,
            "gbs": 2 * nbytes / (ev / steps) / 1e9}


def measured_traffic(profile="decode_global_d512_ctx4096.txt"):
    """HBM bytes per decode step (split + merge kernels) from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary, or None if it is absent."""
    path = os.path.join(ROOT, "profiles", profile)
    if not os.path.exists(path):
        return None
    total = 0.0
    for line in open(path):
        f = line.split()
        if len(f) >= 3 and "decode_" in line and "_kernel" in line:
            try:
                total += (float(f[-2]) + float(f[-1])) * 1e6
            except ValueError:
                continue
    return int(total) if total else None


def cpu_baseline(host, bytes_per_step, seconds):
    """The oracle's attend over the same K/V, with the reference's per-row
    `concat` copy and per-head pool, timed for about `seconds`."""
    import numpy as np
    from oracle import pyoracle as orc

    q = np.ascontiguousarray(host["q"].reshape(-1))
    rows = orc.RowPointers(np.ascontiguousarray(host["K"]), np.ascontiguousarray(host["V"]))
    out = np.zeros_like(q)
    pool = orc.pool_threads()
    threads_used = min(pool, N_HEADS)  # attention hands out one head per chunk (pool.rs:170-171)
    res = {}
    for label, threads in (("pool", 0), ("single_thread", 1)):
        rows.attend(q, 0, rows.T, N_HEADS, N_KV, out, threads=threads)  # warm
        n, t0 = 0, time.perf_counter()
        while True:
            rows.attend(q, 0, rows.T, N_HEADS, N_KV, out, threads=threads)
            n += 1
            el = time.perf_counter() - t0
            if (el >= seconds / 2 and n >= 3) or el >= seconds:
                break
        res[label] = {"us_per_step": el / n * 1e6, "gbs": bytes_per_step / (el / n) / 1e9, "calls": n}
    return res, threads_used


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-workloads", action="store_true", help="only the headline step")
    ap.add_argument("--only", choices=["global", "sliding", "stack", "prefill", "ragged", "layer", "matvec", "copy"],
                    help="run one workload alone (for profiling); prints its result.  'copy' is a "
                         "plain 256 MiB device copy, the reference point for HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the backend runs on a single MI355X (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    import g4hip

    torch.cuda.init()
    if args.only:
        with g4hip.Context(0) as ctx:
            prep = Prep(ctx, torch, 1234)
            k = max(20, args.steps // 4)
            fn = {"global": lambda: bench_global_decode(ctx, torch, prep, args.steps, args.warmup),
                  "sliding": lambda: bench_sliding_decode(ctx, torch, prep, args.steps, args.warmup),
                  "stack": lambda: bench_stack(ctx, torch, prep, g4hip, k, 5),
                  "prefill": lambda: bench_prefill(ctx, torch, prep, max(5, k // 10), args.warmup),
                  "ragged": lambda: bench_ragged(ctx, torch, prep, max(5, k // 4), 2),
                  "layer": lambda: bench_layer_steps(ctx, torch, prep, args.steps, args.warmup),
                  "matvec": lambda: bench_matvec(ctx, torch, max(20, k // 2), args.warmup),
                  "copy": lambda: bench_copy(torch, max(5, k // 4))}[args.only]
            res = fn()
            res.pop("host", None)
            print(json.dumps({"only": args.only, "result": res}))
        return
    with g4hip.Context(0) as ctx:
        prep = Prep(ctx, torch, 1234)
        g = bench_global_decode(ctx, torch, prep, args.steps, args.warmup)
        step_s = g["event"] / args.steps
        achieved = g["bytes"] / step_s / 1e9
        workloads = {}
        if not args.no_workloads:
            k = max(20, args.steps // 4)
            workloads["sliding_decode_d256_ctx64"] = bench_sliding_decode(ctx, torch, prep, args.steps, args.warmup)
            workloads["e2b_stack_35_layers_ctx8192"] = bench_stack(ctx, torch, prep, g4hip, k, 5)
            workloads["prefill_2048"] = bench_prefill(ctx, torch, prep, max(5, k // 10), args.warmup)
            workloads["ragged_decode_B32"] = bench_ragged(ctx, torch, prep, max(5, k // 4), 2)
            workloads["layer_drivers"] = bench_layer_steps(ctx, torch, prep, args.steps, args.warmup)
            workloads["q8_0_matvec"] = bench_matvec(ctx, torch, max(20, k // 2), args.warmup)
        workloads["global_decode_d512_ctx4096_warm"] = {
            "us_per_layer": g["event_warm"] / args.steps * 1e6,
            "gbs": g["bytes"] / (g["event_warm"] / args.steps) / 1e9,
            "note": "one resident K/V copy, served from the Infinity Cache"}
        cpu, threads_used = cpu_baseline(g["host"], g["bytes"], args.cpu_seconds)

    line = {
        "metric": "decode-attn µs/layer + achieved HBM GB/s; prefill-attn TFLOP/s (1× MI355X)",
        "value": round(achieved, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["wall"] / args.steps * 1e3, 6),
        "us_per_layer": round(step_s * 1e6, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "global-layer decode attention, 8 q heads / 1 kv head, head_dim 512, context 4096, "
                               "proportional NEOX RoPE inputs", "context": 4096, "head_dim": 512, "n_heads": N_HEADS,
                   "n_kv_heads": N_KV, "kv_copies_rotated": g["copies"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(),
                     "kernel": "decode step: split-K kernel + merge kernel",
                     "bytes_per_launch": g["bytes"],
                     "traffic_source": "profiles/decode_global_d512_ctx4096.txt (rocprofv3 --pmc, "
                                       "scaled by profiles/hbm_counter_calibration.txt)"},
        "cpu_baseline": {"value": round(cpu["pool"]["gbs"], 3), "unit": "GB/s", "cores": threads_used,
                         "kind": "port",
                         "sample": f"{cpu['pool']['calls']} calls of the same step (us/step "
                                   f"{cpu['pool']['us_per_step']:.0f}); single thread "
                                   f"{cpu['single_thread']['gbs']:.3f} GB/s ({cpu['single_thread']['us_per_step']:.0f}"
                                   f" us/step); host has {os.cpu_count()} logical CPUs"},
        "workloads": workloads,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
