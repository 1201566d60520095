"""Benchmark of the MI355X attention backend for gemma4-rs.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME]

Every decode and prefill shape of the five benchmark configurations runs on
f32 inputs already resident in HBM; the timed steps are replays of captured
HIP graphs, timed with HIP events on the stream the kernels run on.

The headline step is the largest configuration: a ragged batch of 32
independent sequences (context lengths U[1024, 32768], seed 2024), one
decode token each, through a global layer (head_dim 512, whole contexts,
2.04 GB of K/V) and a sliding layer (head_dim 256, window 512), one launch
per layer.  `value` is the step's achieved HBM bandwidth in GB/s
(algorithmic bytes: the K and V rows attended, q and the output, each once);
`roofline` relates the global layer's launch -- the dominant kernel -- to
MI355X's 8 TB/s; `cpu_baseline` is the oracle (the C restatement of the
reference's CPU attention with its `concat` copy and per-head thread pool)
running the reference's per-sequence loop on this host's cores.

`configs` carries each measured workload, keyed in this order, with its own roofline and
CPU baseline: 1 sliding decode over 64 keys, 2 global decode over 4096 keys
(HBM-cold: K/V copies rotated), 3 the 35-layer E2B stack at context 8192
(cold and resident), 4 a 2048-token prefill through a sliding and a global
layer (MFMA-bound), 5 the ragged batch.  `workloads` adds the layer drivers
with their fused input preparation, chunked prompts deep into a long context
(split-f16 and f32 products), the Q8_0 mat-vecs and the launch,
streaming-read and matrix-pipe floors.  HBM byte counters come from the committed rocprofv3
summaries under profiles/.
"""
import argparse
import ctypes
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
F16_MFMA_PEAK_TFLOPS = 2500.0
# The prefill's split-f16 form executes 3 f16 MFMA products per score product
# and 4 per weight x value product: 3.5 per counted product on average, so its
# algorithmic ceiling is the dense f16 peak / 3.5.
SPLIT_F16_PRODUCTS = 3.5
SPLIT_PEAK_TFLOPS = F16_MFMA_PEAK_TFLOPS / SPLIT_F16_PRODUCTS
N_HEADS, N_KV = 8, 1
EPS = 1e-6
LOCAL_BASE, GLOBAL_BASE = 10000.0, 1000000.0
WINDOW = 512
MALL_BYTES = 256 << 20
RAGGED_SEED, RAGGED_B = 2024, 32
METRIC = "decode-attn µs/layer + achieved HBM GB/s; prefill-attn TFLOP/s (1× MI355X)"
# How the timed CPU restatement is built (oracle/Makefile); the GPU host's
# AVX2 level stands in for -march=native, since the library is built
# elsewhere and shipped to that host.
ORACLE_BUILD = "gcc -O3 -march=x86-64-v3 -ffp-contract=off -fno-fast-math (oracle/Makefile)"


def decode_bytes(rows, d):
    """Algorithmic bytes of one decode step: K and V rows once, q and out."""
    return rows * 2 * N_KV * d * 4 + 2 * N_HEADS * d * 4


def prefill_flops(N, window, d):
    """4 * heads * d FLOP per attended (query, key) pair (QK^T and PV)."""
    pairs = sum(min(i + 1, window) if window else i + 1 for i in range(N))
    return 4 * N_HEADS * d * pairs


def roofline_hbm(nbytes, seconds, traffic=None, **extra):
    gbs = nbytes / seconds / 1e9
    r = {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic}
    r.update(extra)
    return r


def ragged_lengths():
    import numpy as np
    return np.random.default_rng(RAGGED_SEED).integers(1024, 32768 + 1, size=RAGGED_B).astype(np.int64)


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


WARM_SECONDS = 0.1


def time_steps(torch, fn, steps, warmup, warm_seconds=WARM_SECONDS):
    """Runs at least `warmup` eager steps and at least `warm_seconds` of them
    (the clocks need tens of milliseconds of a load to settle: a step timed
    after a handful of warm-up calls reads slow), captures the `steps` timed
    steps into one HIP graph and times one replay of it between
    synchronisations, with HIP events on the current stream (where fn(i)
    launches step i) and with the host clock.  Returns (wall seconds, event
    seconds) for the `steps` steps."""
    t0, i = time.perf_counter(), 0
    while i < warmup or time.perf_counter() - t0 < warm_seconds:
        fn(i)
        i += 1
        if i >= warmup and i % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            fn(i)
    torch.cuda.synchronize()
    graph.replay()  # the first replay uploads the graph
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    graph.replay()
    end.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, start.elapsed_time(end) * 1e-3


# ----------------------------------------------------------------- GPU side
def bench_sliding_decode(ctx, torch, prep, steps, warmup, T=64, d=256):
    """One sliding-layer decode over 64 keys (147 KB; its
    rows stay cached between steps: a launch-latency figure)."""
    K = prep.rows(T, d, 0, LOCAL_BASE, None)
    V = prep.rows(T, d, 0, 0.0, None, rope=False)
    q = prep.rows(1, d, T - 1, LOCAL_BASE, None, heads=N_HEADS)
    out = torch.zeros(N_HEADS * d, device="cuda")
    wall, ev = time_steps(torch, lambda i: ctx.attend_decode(q, K, V, 0, T, N_HEADS, N_KV, d, out), steps, warmup)
    ctx.check_status()
    host = {"q": q.cpu().numpy(), "K": K.cpu().numpy(), "V": V.cpu().numpy()}
    return {"us_per_layer": ev / steps * 1e6, "wall_us_per_layer": wall / steps * 1e6, "bytes": decode_bytes(T, d),
            "cache": "resident (147 KB, read every step)", "host": host}


def bench_global_decode(ctx, torch, prep, steps, warmup, T=4096, d=512):
    """One global-layer decode over 4096 keys.  Each step
    reads one of `copies` K/V copies (more than 1.5x the 256 MB Infinity
    Cache between two reads of a copy), so its K/V come from HBM; the same
    step on one resident copy is reported beside it."""
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

    wall, ev = time_steps(torch, step, steps, warmup)
    ctx.check_status()
    wall_w, ev_w = time_steps(torch, lambda i: ctx.attend_decode(q, Ks[0], Vs[0], 0, T, N_HEADS, N_KV, d, out),
                              steps, warmup)
    host = {"q": q.cpu().numpy(), "K": Ks[0].cpu().numpy(), "V": Vs[0].cpu().numpy()}
    return {"us_per_layer": ev / steps * 1e6, "wall_us_per_layer": wall / steps * 1e6,
            "us_per_layer_resident": ev_w / steps * 1e6, "bytes": decode_bytes(T, d),
            "cache": f"HBM-cold: {min(copies, steps)} K/V copies of {per_copy >> 20} MiB rotated", "host": host}


def bench_host_attend(ctx, torch, prep, steps, warmup=3):
    """g4_attend, the form of `attend` over host buffers (model.rs:348-366
    takes slices): per call it allocates device buffers, copies q, K and V
    in, decodes, copies the output back and frees.  Timed on the host clock
    around whole calls, at the shapes of the 64-key sliding decode and the
    4096-key global decode; the rate counts the bytes that cross PCIe."""
    res = {}
    for name, T, d, base, glob in (("sliding_d256_ctx64", 64, 256, LOCAL_BASE, False),
                                   ("global_d512_ctx4096", 4096, 512, GLOBAL_BASE, True)):
        freqs = prep.rope_freqs(d) if glob else None
        K = prep.rows(T, d, 0, base, freqs).cpu().numpy()
        V = prep.rows(T, d, 0, 0.0, None, rope=False).cpu().numpy()
        q = prep.rows(1, d, T - 1, base, freqs, heads=N_HEADS).cpu().numpy()
        for _ in range(warmup):
            ctx.attend(q, K, V, N_HEADS, N_KV)
        t0 = time.perf_counter()
        for _ in range(steps):
            ctx.attend(q, K, V, N_HEADS, N_KV)
        s = (time.perf_counter() - t0) / steps
        nbytes = (2 * q.size + K.size + V.size) * 4
        res[name] = {"us_per_call": round(s * 1e6, 1), "pcie_bytes": nbytes, "gbs": round(nbytes / s / 1e9, 3),
                     "note": "host buffers in and out (pageable), device buffers allocated and freed per call"}
    return res


def stack_plan(g4hip, ctx_len):
    """The E2B stack's per-layer (source layer, kv range, head_dim, global)."""
    n_layers, shared = 35, 20
    plan = []
    for layer in range(n_layers):
        glob = g4hip.layer_attention_kind(n_layers, layer) == "global"
        d = 512 if glob else 256
        src = g4hip.kv_source_layer(n_layers, shared, layer)
        r = g4hip.windowed_len(ctx_len, WINDOW) if not glob else range(0, ctx_len)
        plan.append((layer, src, r.start, r.stop, d, glob))
    return plan


def bench_stack(ctx, torch, prep, g4hip, steps, warmup, ctx_len=8192, cold=True, want_host=False):
    """The 35-layer E2B stack, one decode step at position
    ctx_len - 1: each layer's attention over its source layer's cache
    (owners 0..14, layers 15..34 reading 13/14), one call per layer.  Cold:
    the 15 owners' caches exist in `copies` copies, one per step in turn, so
    the 108 MiB of K/V one step reads come from HBM; resident: one copy."""
    plan = stack_plan(g4hip, ctx_len)
    freqs = prep.rope_freqs(512)
    unique = sum(decode_bytes(e - b, d) for (l, s, b, e, d, g) in plan if s == l)
    copies = max(2, int(1.5 * MALL_BYTES // unique) + 1) if cold else 1
    caches = []
    for c in range(copies):
        caches.append({})
        for layer, src, b, e, d, glob in plan:
            if src == layer:
                caches[c][layer] = (prep.rows(ctx_len, d, 0, GLOBAL_BASE if glob else LOCAL_BASE,
                                              freqs if glob else None),
                                    prep.rows(ctx_len, d, 0, 0.0, None, rope=False))
    qs = [prep.rows(1, d, ctx_len - 1, GLOBAL_BASE if glob else LOCAL_BASE, freqs if glob else None, heads=N_HEADS)
          for (layer, src, b, e, d, glob) in plan]
    outs = [torch.zeros(N_HEADS * d, device="cuda") for (layer, src, b, e, d, glob) in plan]
    total_bytes = sum(decode_bytes(e - b, d) for (l, s, b, e, d, g) in plan)

    def step(i):
        cc = caches[i % copies]
        for (layer, src, b, e, d, glob), q, out in zip(plan, qs, outs):
            K, V = cc[src]
            ctx.attend_decode(q, K, V, b, e, N_HEADS, N_KV, d, out)

    wall, ev = time_steps(torch, step, steps, warmup)
    ctx.check_status()
    res = {"us_per_stack": ev / steps * 1e6, "wall_us_per_stack": wall / steps * 1e6,
           "us_per_layer_mean": ev / steps / len(plan) * 1e6, "bytes_per_stack": total_bytes,
           "unique_bytes_per_stack": unique, "layers": len(plan),
           "global_layers": sum(1 for p in plan if p[5]),
           "cache": (f"HBM-cold: {min(copies, steps)} copies of the owners' K/V rotated" if cold else
                     "resident: one copy, re-read every step")}
    if want_host:
        res["host"] = {"plan": plan, "q": [q.cpu().numpy() for q in qs],
                       "kv": {l: (K.cpu().numpy(), V.cpu().numpy()) for l, (K, V) in caches[0].items()}}
    return res


def bench_layer_stack(ctx, torch, prep, g4hip, steps, warmup, ctx_len=8192, want_host=False):
    """The per-token attention segment of the whole E2B stack as the engine
    runs it through the layer driver: one g4_layer_attention call per layer
    (model.rs:394-410: q norm + RoPE; on the 15 owner layers the new row's
    k/v norm + RoPE and its append; the view and window; attention), 35
    calls per token, each one fused launch plus the split merge.  Owners
    start with ctx_len - 1 rows; every step decodes the next token (the
    caches grow by one row per step: the timed steps sit at contexts
    ctx_len + warm-up steps onward).  q, k and v are raw (pre-norm) draws,
    the norm weights ones, the global layers' RoPE factors E2B's
    proportional ones."""
    hp = g4hip.G4Hparams.e2b()
    plan = stack_plan(g4hip, ctx_len)
    extra = 8192  # rows of room for warm-up and timed steps
    widths = [d if src == layer else 0 for (layer, src, b, e, d, glob) in plan]
    cache = g4hip.KvCache(ctx, widths, ctx_len + extra)
    host = {}
    try:
        freqs = torch.tensor(g4hip.proportional_rope_freq_factors(512, 0.25), device="cuda")
        for layer, src, b, e, d, glob in plan:
            if src == layer:
                K = prep.rows(ctx_len - 1, d, 0, GLOBAL_BASE if glob else LOCAL_BASE, freqs if glob else None)
                V = prep.rows(ctx_len - 1, d, 0, 0.0, None, rope=False)
                cache.append_rows(layer, K, V, ctx_len - 1)
                if want_host:
                    host[layer] = (K.cpu().numpy(), V.cpu().numpy())
                del K, V
        qs = [prep.randn(N_HEADS * d) for (layer, src, b, e, d, glob) in plan]
        ks = [prep.randn(N_KV * d) for (layer, src, b, e, d, glob) in plan]
        vs = [prep.randn(N_KV * d) for (layer, src, b, e, d, glob) in plan]
        ones = {256: torch.ones(256, device="cuda"), 512: torch.ones(512, device="cuda")}
        outs = [torch.zeros(N_HEADS * d, device="cuda") for (layer, src, b, e, d, glob) in plan]
        state = {"pos": ctx_len - 1}

        def step(i):
            pos = state["pos"]
            for (layer, src, b, e, d, glob), q, k, v, out in zip(plan, qs, ks, vs, outs):
                cache.layer_attention(hp, layer, pos, q, k, v, ones[d], ones[d], freqs, out)
            state["pos"] = pos + 1

        first = state["pos"]
        wall, ev = time_steps(torch, step, steps, warmup, warm_seconds=0.05)
        ctx.check_status()
        timed_from = state["pos"] - steps
        res = {"us_per_token": ev / steps * 1e6, "wall_us_per_token": wall / steps * 1e6,
               "us_per_layer_mean": ev / steps / len(plan) * 1e6, "layers": len(plan),
               "contexts": [timed_from + 1, timed_from + steps],
               "note": "35 g4_layer_attention calls per token (fused preparation + append + attention, then the "
                       "split merge); owners' K/V resident; warm-up steps from context "
                       f"{first + 1}, timed steps at the contexts given",
               "profile": "profiles/decode_e2b_stack_35_layers_ctx8192_layer_attention.txt"}
        if want_host:
            res["host"] = {"plan": plan, "kv": host, "ctx_len": ctx_len,
                           "q": [q.cpu().numpy() for q in qs], "k": [k.cpu().numpy() for k in ks],
                           "v": [v.cpu().numpy() for v in vs], "freqs": freqs.cpu().numpy()}
        return res
    finally:
        cache.close()
        torch.cuda.empty_cache()


def bench_prefill(ctx, torch, prep, steps, warmup, N=2048, want_host=False):
    """A causal prefill of an N-token prompt through one
    sliding and one global layer.  All timed steps replay as one captured
    graph after at least 50 untimed steps: the clocks need tens of
    milliseconds of this load to settle (global layer 348 us after 2 warm-up
    steps, 322 us after 50, measured in one process)."""
    warmup = max(warmup, 50)
    res = {}
    host = {}
    total_flops, total_s = 0, 0.0
    for name, d, window, base in (("sliding_d256_W512", 256, WINDOW, LOCAL_BASE), ("global_d512", 512, 0, GLOBAL_BASE)):
        freqs = prep.rope_freqs(d) if not window else None
        K = prep.rows(N, d, 0, base, freqs)
        V = prep.rows(N, d, 0, 0.0, None, rope=False)
        q = prep.rows(N, d, 0, base, freqs, heads=N_HEADS)
        out = torch.zeros(N * N_HEADS * d, device="cuda")
        wall, ev = time_steps(torch, lambda i: ctx.attend_prefill(q, K, V, 0, N, window, N_HEADS, N_KV, d, out),
                              steps, warmup)
        ctx.check_status()
        fl = prefill_flops(N, window, d)
        res[name] = {"us": ev / steps * 1e6, "tflops": fl / (ev / steps) / 1e12, "flops": fl}
        total_flops += fl
        total_s += ev / steps
        if want_host:
            host[name] = (q.cpu().numpy(), K.cpu().numpy(), V.cpu().numpy(), window, d)
        del K, V, q, out
    res["both_layers_us"] = total_s * 1e6
    res["both_layers_tflops"] = total_flops / total_s / 1e12
    res["frac_of_split_f16_peak"] = res["both_layers_tflops"] / SPLIT_PEAK_TFLOPS
    res["frac_of_f32_mfma_peak"] = res["both_layers_tflops"] / F32_MFMA_PEAK_TFLOPS
    if want_host:
        res["host"] = host
    return res


def bench_prefill_chunks(ctx, torch, prep, steps, warmup):
    """Chunked prompts deep into a long context on a global layer (d=512):
    256 tokens at position 16384 and 2048 tokens at position 30720, each in
    the split-f16 form (the default) and with f32 MFMA products only
    (g4_set_prefill_exact), FLOPs counted as for configuration 4."""
    res = {}
    try:
        for name, d, window, pos0, N in (("global_d512_chunk256_at16384", 512, 0, 16384, 256),
                                         ("global_d512_chunk2048_at30720", 512, 0, 30720, 2048)):
            K = prep.rows(pos0 + N, d, 0, GLOBAL_BASE, prep.rope_freqs(d))
            V = prep.rows(pos0 + N, d, 0, 0.0, None, rope=False)
            q = prep.rows(N, d, pos0, GLOBAL_BASE, prep.rope_freqs(d), heads=N_HEADS)
            out = torch.zeros(N * N_HEADS * d, device="cuda")
            fl = sum(4 * N_HEADS * d * (min(p + 1, window) if window else p + 1) for p in range(pos0, pos0 + N))
            r = {"flops": fl}
            for form, exact in (("split_f16", 0), ("f32", 1)):
                ctx.set_prefill_exact(exact)
                wall, ev = time_steps(torch, lambda i: ctx.attend_prefill(q, K, V, pos0, N, window, N_HEADS, N_KV, d,
                                                                          out), steps, warmup)
                ctx.check_status()
                r[form] = {"us": ev / steps * 1e6, "tflops": fl / (ev / steps) / 1e12,
                           "frac_of_split_f16_peak": fl / (ev / steps) / 1e12 / SPLIT_PEAK_TFLOPS}
            res[name] = r
            del K, V, q, out
    finally:
        ctx.set_prefill_exact(0)
    torch.cuda.empty_cache()
    return res


def bench_ragged(ctx, torch, prep, steps, warmup, want_host=False):
    """The ragged batch of 32 sequences, global layer (whole contexts,
    2.04 GB of K/V, larger than the Infinity Cache: HBM-cold by size) and
    sliding layer (the last 512 rows of each sequence, 34 MB: resident
    between steps).  Timed per layer and as the whole step (both layers)."""
    import numpy as np
    lens = ragged_lengths()
    row0 = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    total = int(lens.sum())
    layers = {}
    host = {}
    for name, d, glob in (("global_d512", 512, True), ("sliding_d256_W512", 256, False)):
        freqs = prep.rope_freqs(d) if glob else None
        base = GLOBAL_BASE if glob else LOCAL_BASE
        begin = np.array([0 if glob else max(0, int(L) - WINDOW) for L in lens], np.int64)
        K = prep.rows(total, d, 0, base, freqs)  # positions are not per-sequence here: timing only
        V = prep.rows(total, d, 0, 0.0, None, rope=False)
        q = prep.rows(RAGGED_B, d, 0, base, freqs, heads=N_HEADS)
        out = torch.zeros(RAGGED_B * N_HEADS * d, device="cuda")
        t_row0, t_b, t_e = (torch.from_numpy(a).cuda() for a in (row0, begin, lens))
        max_len = int((lens - begin).max())
        nbytes = sum(decode_bytes(int(lens[s] - begin[s]), d) for s in range(RAGGED_B))

        def call(i, q=q, K=K, V=V, t_row0=t_row0, t_b=t_b, t_e=t_e, max_len=max_len, d=d, out=out):
            ctx.attend_decode_batch(q, K, V, t_row0, t_b, t_e, max_len, N_HEADS, N_KV, d, out)

        layers[name] = {"call": call, "bytes": nbytes, "keep": (K, V, q, out, t_row0, t_b, t_e)}
        if want_host:
            host[name] = (q.cpu().numpy(), K.cpu().numpy(), V.cpu().numpy(), begin.copy(), d)
    res = {}
    for name, L in layers.items():
        wall, ev = time_steps(torch, L["call"], steps, warmup)
        ctx.check_status()
        res[name] = {"us": ev / steps * 1e6, "gbs": L["bytes"] / (ev / steps) / 1e9, "bytes": L["bytes"],
                     "frac_of_hbm_peak": L["bytes"] / (ev / steps) / 1e9 / HBM_PEAK_GBS}

    def step(i):
        for L in layers.values():
            L["call"](i)

    wall, ev = time_steps(torch, step, steps, warmup)
    ctx.check_status()
    nbytes = sum(L["bytes"] for L in layers.values())
    res["step"] = {"us": ev / steps * 1e6, "wall_us": wall / steps * 1e6, "bytes": nbytes,
                   "gbs": nbytes / (ev / steps) / 1e9}
    res["lengths"] = {"min": int(lens.min()), "max": int(lens.max()), "mean": float(lens.mean()),
                      "seed": RAGGED_SEED}
    res["cache"] = "global layer HBM-cold by size (2.04 GB); sliding layer resident (34 MB re-read every step)"
    if want_host:
        res["host"] = {"lens": lens, "layers": host}
    del layers
    torch.cuda.empty_cache()
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

    wall, ev = time_steps(torch, fused, steps, warmup)
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

    wall, ev = time_steps(torch, two_launch, steps, warmup)
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

        wall, ev = time_steps(torch, pstep, psteps, max(2, warmup // 4))
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

        wall, ev = time_steps(torch, step, steps, warmup)
        nbytes = r * nb * 34 + c * 4 + r * 4
        res[name] = {"us": ev / steps * 1e6, "gbs": nbytes / (ev / steps) / 1e9, "bytes": nbytes,
                     "frac_of_hbm_peak": nbytes / (ev / steps) / 1e9 / HBM_PEAK_GBS}
        del w
    return res


def floors_lib():
    path = os.path.join(ROOT, "gemma4-rs_amd", "lib", "libg4floors.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(path)
    lib.g4f_empty.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.g4f_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.g4f_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.g4f_lds_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    lib.g4f_mix.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def bench_floors(torch, steps, warmup):
    """The floors the decode kernels are measured against: an empty kernel
    of 256 workgroups x 512 threads (the decode split grid's shape) per
    launch in a captured graph, and streaming reads of 1 MiB (a sliding
    layer's K/V, resident), 16 MiB (a 4096-key global layer's, HBM-cold:
    copies rotated), 32 MiB (about the ragged batch's 32 sliding windows,
    resident in the Infinity Cache) and 1 GiB (HBM-cold by size), each one
    launch of 2048 x 256 threads with 16-byte non-temporal loads; and the
    matrix-pipe rates the prefill kernels are read against: MFMAs alone, fed
    from LDS, and beside independent VALU work."""
    lib = floors_lib()

    def check(rc):
        if rc:
            raise RuntimeError("floors kernel launch failed")

    stream = lambda: torch.cuda.current_stream().cuda_stream
    res = {}
    wall, ev = time_steps(torch, lambda i: check(lib.g4f_empty(256, 512, stream())), steps, warmup)
    res["empty_kernel_256x512"] = {"us_per_launch": ev / steps * 1e6}
    sink = torch.zeros(2048, device="cuda")
    for name, nbytes, copies in (("read_1MiB_resident", 1 << 20, 1), ("read_16MiB_cold", 16 << 20, 24),
                                 ("read_32MiB_resident", 32 << 20, 1), ("read_1GiB", 1 << 30, 1)):
        bufs = [torch.ones(nbytes // 4, device="cuda") for _ in range(copies)]
        wall, ev = time_steps(torch, lambda i: check(lib.g4f_read(bufs[i % copies].data_ptr(), nbytes,
                                                                  sink.data_ptr(), 2048, stream())), steps, warmup)
        res[name] = {"us": ev / steps * 1e6, "gbs": nbytes / (ev / steps) / 1e9}
        del bufs
    # Matrix-pipe rate: two independent accumulator chains per wave, 1 or 2
    # waves per SIMD (the prefill kernels run 2); cycles per MFMA per SIMD at
    # the 2.4 GHz peak clock.
    iters = 4096
    msink = torch.zeros(512 * 256, device="cuda")
    for name, f16, flop in (("mfma_16x16x32_f16", 1, 16384), ("mfma_16x16x4_f32", 0, 2048)):
        for wps in (1, 2):
            grid = 256 * wps
            wall, ev = time_steps(torch, lambda i: check(lib.g4f_mfma(f16, grid, iters, msink.data_ptr(), stream())),
                                  max(1, steps // 10), max(1, warmup // 10))
            s = ev / max(1, steps // 10)
            per_simd = wps * 2 * iters
            res[f"{name}_{wps}_waves_per_simd"] = {
                "us": s * 1e6, "cycles_per_mfma_at_2400mhz": s * 2.4e9 / per_simd,
                "tflops": grid * 4 * 2 * iters * flop / s / 1e12}
    # The pipe fed from LDS: one 1 KiB operand (16 bytes per lane) read per
    # one or two MFMAs, 16x16x32 (16 cycles of matrix work per instruction at
    # peak) or 32x32x16 (32); four accumulators per wave.  A 16x16x32 fed one
    # operand per instruction needs 256 B/clk of LDS per CU at peak.
    lsteps = max(1, steps // 10)
    for mode, (shape, mpr) in enumerate((("16x16x32", 0), ("16x16x32", 1), ("16x16x32", 2), ("32x32x16", 0),
                                         ("32x32x16", 1), ("32x32x16", 2))):
        flop = 16384 if shape == "16x16x32" else 32768
        for wps in (1, 2):
            grid = 256 * wps
            lit = 1024
            wall, ev = time_steps(torch, lambda i: check(lib.g4f_lds_mfma(mode, grid, lit, msink.data_ptr(),
                                                                          stream())), lsteps, 1)
            s = ev / lsteps
            per_simd = wps * 8 * lit * max(mpr, 1)
            cyc = s * 2.4e9 / per_simd
            r = {"us": round(s * 1e6, 2), "cycles_per_mfma_at_2400mhz": round(cyc, 2),
                 "tflops": round(grid * 4 * 8 * lit * max(mpr, 1) * flop / s / 1e12, 1)}
            if mpr:
                r["lds_bytes_per_clk_per_cu"] = round(4 * wps * 8 * lit * 1024 / (s * 2.4e9), 1)
            res[f"lds_fed_mfma_{shape}_{mpr}_per_read_{wps}_waves_per_simd"] = r
    # MFMA / VALU overlap (g4f_mix): one workgroup of eight waves per CU; an
    # MFMA wave issues 4 x mit 16x16x32 f16 MFMAs, an FMA wave 16 x mit f32
    # FMAs, an interleaving wave k FMAs after each of its 4 x mit MFMAs.
    mit = 4096
    for name, mode, k in (("mfma_2_waves_per_simd", 0, 1), ("mfma_1_wave_per_simd", 1, 1),
                          ("fma_1_wave_per_simd", 2, 1), ("mfma_wave_and_fma_wave_per_simd", 3, 1),
                          ("interleaved_1_fma_per_mfma_1_wave", 4, 1), ("interleaved_2_fma_per_mfma_1_wave", 4, 2),
                          ("interleaved_4_fma_per_mfma_1_wave", 4, 4), ("interleaved_1_fma_per_mfma_2_waves", 5, 1),
                          ("interleaved_2_fma_per_mfma_2_waves", 5, 2), ("interleaved_4_fma_per_mfma_2_waves", 5, 4)):
        wall, ev = time_steps(torch, lambda i: check(lib.g4f_mix(mode, k, 256, mit, msink.data_ptr(), stream())),
                              lsteps, 1)
        s = ev / lsteps
        mfma_per_simd = 4 * mit * (2 if mode in (0, 5) else 0 if mode == 2 else 1)
        r = {"us": round(s * 1e6, 2)}
        if mfma_per_simd:
            r["cycles_per_mfma_at_2400mhz"] = round(s * 2.4e9 / mfma_per_simd, 2)
        res[f"overlap_{name}"] = r
    del msink
    torch.cuda.empty_cache()
    return res


def bench_copy(torch, steps, nbytes=256 << 20):
    """A plain device-to-device copy of known size: the reference point that
    scales the FETCH_SIZE / WRITE_SIZE counters to bytes."""
    src = torch.empty(nbytes // 4, device="cuda").uniform_()
    dst = torch.empty_like(src)
    wall, ev = time_steps(torch, lambda i: dst.copy_(src), steps, 2)
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": ev / steps * 1e6,
            "gbs": 2 * nbytes / (ev / steps) / 1e9}


# ------------------------------------------------------------- profiles/
def profile_summary(name):
    """Per-kernel figures from a committed profiles/ summary: {kernel:
    {"avg_us": ..., "read_mb": ..., "written_mb": ..., counters...}}."""
    path = os.path.join(ROOT, "profiles", name)
    out = {}
    if not os.path.exists(path):
        return out
    section = None
    for line in open(path):
        s = line.strip()
        if s.startswith("kernel") and "avg us" in s:
            section = "trace"
            continue
        if s.startswith("kernel") and "read MB" in s:
            section = "bytes"
            continue
        if s.startswith("kernel") and "mfma busy" in s:
            section = "mfma"
            continue
        if not s or not (s.startswith("void g4::") or s.startswith("g4::")):
            if not s:
                section = None
            continue
        f = s.split()
        try:
            if section == "trace":
                out.setdefault(" ".join(f[:-3]), {})["avg_us"] = float(f[-2])
            elif section == "bytes":
                d = out.setdefault(" ".join(f[:-2]), {})
                d["read_mb"], d["written_mb"] = float(f[-2]), float(f[-1])
            elif section == "mfma":
                d = out.setdefault(" ".join(f[:-2]), {})
                d["mfma_busy"], d["mfma_tflops"] = float(f[-2]), float(f[-1])
        except ValueError:
            continue
    return out


def traffic_bytes(name, kernels=None):
    """HBM bytes (read + written) per step from a profiles/ summary: of the
    named kernels (substring match, one dispatch each), or with kernels None
    the summary's whole-step total (every dispatch of a step); None when the
    summary does not hold them."""
    if kernels is None:
        path = os.path.join(ROOT, "profiles", name)
        if not os.path.exists(path):
            return None
        for line in open(path):
            f = line.split()
            if line.strip().startswith("per step: read"):
                return int((float(f[3]) + float(f[6])) * 1e6)
        return None
    prof = profile_summary(name)
    total, found = 0.0, False
    for k, v in prof.items():
        if any(sub in k for sub in kernels) and "read_mb" in v:
            total += (v["read_mb"] + v["written_mb"]) * 1e6
            found = True
    return int(total) if found else None


def summarize(base, fetch_scale=2.0, write_scale=1.0):
    """The profiles/ tables from rocprofv3 CSV output under `base`:
    trace/run_kernel_stats.csv (--kernel-trace --stats), fetch/ and write/
    run_counter_collection.csv (--pmc FETCH_SIZE, --pmc WRITE_SIZE; KiB per
    dispatch, scaled by a plain copy's reading: FETCH_SIZE counts half the
    bytes a copy reads, profiles/hbm_counter_calibration.txt) and, when
    present, mfma/ (--pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16
    SQ_BUSY_CYCLES GRBM_GUI_ACTIVE).  Returns the text."""
    import collections
    import csv

    def short(k):
        return k.replace("(anonymous namespace)::", "").split("(")[0]

    def ours(n):
        return n.startswith("void g4::") or n.startswith("g4::")

    lines = []
    stats = os.path.join(base, "trace", "run_kernel_stats.csv")
    avg = {}
    if os.path.exists(stats):
        rows = list(csv.DictReader(open(stats)))
        tot = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
        lines.append("  kernel                                                        calls     avg us  share")
        for r in rows:
            n = short(r["Name"])
            avg[n] = float(r["AverageNs"])
            if ours(n):
                lines.append(f"  {n:<60} {int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>10.3f} "
                             f"{100 * float(r['TotalDurationNs']) / tot:>5.1f}%")

    def counters(sub):
        path = os.path.join(base, sub, "run_counter_collection.csv")
        if not os.path.exists(path):
            return None
        acc = collections.defaultdict(lambda: collections.defaultdict(list))
        for r in csv.DictReader(open(path)):
            n = short(r["Kernel_Name"])
            if ours(n):
                acc[n][r["Counter_Name"]].append(float(r["Counter_Value"]))
        return {n: {c: sum(v) / len(v) for c, v in d.items()} for n, d in acc.items()}

    f, w = counters("fetch"), counters("write")
    if f is not None and w is not None:
        lines += ["", "  kernel                                                          read MB  written MB"]
        for n in f:
            rd = f[n].get("FETCH_SIZE", 0) * 1024 * fetch_scale / 1e6
            wr = w.get(n, {}).get("WRITE_SIZE", 0) * 1024 * write_scale / 1e6
            lines.append(f"  {n:<60} {rd:>10.3f} {wr:>11.3f}")
    m = counters("mfma")
    if m:
        lines += ["", "  kernel                                                        mfma busy  TFLOP/s"]
        for n, d in m.items():
            g = d.get("GRBM_GUI_ACTIVE", 0)
            mops = d.get("SQ_INSTS_VALU_MFMA_MOPS_F16") or d.get("SQ_INSTS_VALU_MFMA_MOPS_F32")
            if not mops or not g or n not in avg:
                continue
            busy = d["SQ_VALU_MFMA_BUSY_CYCLES"] / (g / 8 * 1024)
            lines.append(f"  {n:<60} {busy:>9.3f} {mops * 512 / (avg[n] * 1e-9) / 1e12:>8.1f}")
    return "\n".join(lines)


# ---------------------------------------------------------- CPU baseline
class CpuTimer:
    """Times the oracle's attend (the reference's attend with its `concat`
    copy and per-head pool) on this host's cores."""

    def __init__(self):
        from oracle import pyoracle as orc
        self.orc = orc
        self.pool = orc.pool_threads()
        self.threads = min(self.pool, N_HEADS)  # one head per chunk (pool.rs:170-171)

    def loop(self, fn, seconds, min_calls=2):
        fn()  # warm
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if (n >= min_calls and el >= seconds) or el >= 4 * seconds:
                return el / n, n

    def rows(self, K, V):
        import numpy as np
        return self.orc.RowPointers(np.ascontiguousarray(K), np.ascontiguousarray(V))


def cpu_decode(cpu, host, T, nbytes, seconds):
    """Single-sequence decode (64 keys at d=256, 4096 keys at d=512): attend over T rows."""
    import numpy as np
    q = np.ascontiguousarray(host["q"].reshape(-1))
    rows = cpu.rows(host["K"], host["V"])
    out = np.zeros_like(q)
    s, n = cpu.loop(lambda: rows.attend(q, 0, T, N_HEADS, N_KV, out), seconds)
    s1, n1 = cpu.loop(lambda: rows.attend(q, 0, T, N_HEADS, N_KV, out, threads=1), seconds / 2)
    return {"value": round(nbytes / s / 1e9, 4), "unit": "GB/s", "us_per_layer": round(s * 1e6, 1),
            "cores": cpu.threads, "kind": "port", "build": ORACLE_BUILD,
            "sample": f"{n} calls of the same step; single thread {nbytes / s1 / 1e9:.3f} GB/s "
                      f"({s1 * 1e6:.0f} us/step); host has {os.cpu_count()} logical CPUs"}


def cpu_stack(cpu, host, nbytes, seconds):
    """The E2B stack on the CPU: the reference's layer loop, one attend per layer
    over its source layer's rows (model.rs:407-410)."""
    import numpy as np
    rows = {l: cpu.rows(K, V) for l, (K, V) in host["kv"].items()}
    qs = [np.ascontiguousarray(q.reshape(-1)) for q in host["q"]]
    outs = [np.zeros_like(q) for q in qs]

    def stack():
        for (layer, src, b, e, d, glob), q, out in zip(host["plan"], qs, outs):
            rows[src].attend(q, b, e, N_HEADS, N_KV, out)

    s, n = cpu.loop(stack, seconds)
    return {"value": round(nbytes / s / 1e9, 4), "unit": "GB/s", "us_per_stack": round(s * 1e6, 1),
            "cores": cpu.threads, "kind": "port", "build": ORACLE_BUILD,
            "sample": f"{n} whole stacks (35 attend calls each, resident in host memory); "
                      f"host has {os.cpu_count()} logical CPUs"}


def cpu_layer_stack(cpu, host, seconds):
    """The E2B stack's per-token attention segment on the CPU, as the
    reference's layer loop runs it (model.rs:394-410): per layer the q (and
    on owners k, v) norm + RoPE (or_prepare_rows, the oracle's norm_heads and
    rope_heads), the append into the owner's rows, then attend -- with its
    `concat` copy and per-head pool -- over the window's rows.  Each step is
    the next token, as on the GPU."""
    import numpy as np
    orc = cpu.orc
    ctx_len = host["ctx_len"]
    cap = ctx_len + 4096
    caches, rows = {}, {}
    for layer, (K, V) in host["kv"].items():
        Kc = np.zeros((cap, K.shape[1]), np.float32)
        Vc = np.zeros((cap, V.shape[1]), np.float32)
        Kc[:K.shape[0]], Vc[:V.shape[0]] = K, V
        caches[layer] = (Kc, Vc)
        rows[layer] = cpu.rows(Kc, Vc)
    freqs = host["freqs"]
    ones = {256: np.ones(256, np.float32), 512: np.ones(512, np.float32)}
    state = {"pos": ctx_len - 1}

    def step():
        pos = state["pos"]
        for (layer, src, b, e, d, glob), q0, k0, v0 in zip(host["plan"], host["q"], host["k"], host["v"]):
            base = GLOBAL_BASE if glob else LOCAL_BASE
            f = freqs if glob else None
            q = orc.prepare_rows(q0.reshape(1, -1).copy(), d, ones[d], EPS, pos, base, f)[0]
            if src == layer:
                caches[layer][0][pos] = orc.prepare_rows(k0.reshape(1, -1).copy(), d, ones[d], EPS, pos, base, f)[0]
                caches[layer][1][pos] = orc.prepare_rows(v0.reshape(1, -1).copy(), d, None, EPS, 0, 0.0, None)[0]
            begin = 0 if glob else max(0, pos + 1 - WINDOW)
            out = np.zeros(N_HEADS * d, np.float32)
            rows[src].attend(q, begin, pos + 1, N_HEADS, N_KV, out)
        state["pos"] = pos + 1

    s, n = cpu.loop(step, seconds, min_calls=1)
    return {"value": round(s * 1e6, 1), "unit": "us/token", "cores": cpu.threads, "kind": "port",
            "build": ORACLE_BUILD,
            "sample": f"{n + 1} consecutive tokens from context {ctx_len} (35 layers each: preparation, append "
                      f"and attend); host has {os.cpu_count()} logical CPUs"}


def cpu_prefill(cpu, host, seconds, stride=8):
    """Prefill on the CPU: the reference's prompt loop, one attend per token
    (crates/llm-gemma4/src/impl_/generate.rs:37-41), on every `stride`-th
    position of the 2048-token prompt; TFLOP/s from the sampled positions'
    own FLOPs."""
    import numpy as np
    res = {}
    tot_fl, tot_s = 0, 0.0
    for name, (q, K, V, window, d) in host.items():
        rows = cpu.rows(K, V)
        N = q.shape[0]
        pos = list(range(stride - 1, N, stride))
        qs = [np.ascontiguousarray(q[i]) for i in pos]
        out = np.zeros(N_HEADS * d, np.float32)
        ranges = [(max(0, i + 1 - window) if window else 0, i + 1) for i in pos]
        fl = sum(4 * N_HEADS * d * (e - b) for b, e in ranges)

        def prompt():
            for qi, (b, e) in zip(qs, ranges):
                rows.attend(qi, b, e, N_HEADS, N_KV, out)

        s, n = cpu.loop(prompt, seconds / 2, min_calls=1)
        res[name] = {"tflops": fl / s / 1e12, "us_per_token": s / len(pos) * 1e6}
        tot_fl += fl
        tot_s += s
    return {"value": round(tot_fl / tot_s / 1e12, 6), "unit": "TFLOP/s", "cores": cpu.threads, "kind": "port",
            "build": ORACLE_BUILD, "layers": res,
            "sample": f"the prompt loop at every {stride}th position (256 of 2048 tokens per layer, their own "
                      f"FLOPs); host has {os.cpu_count()} logical CPUs"}


def cpu_ragged(cpu, host, nbytes, seconds):
    """The ragged batch on the CPU: the reference's engine is single-sequence, so the
    batch is a loop over the 32 sequences, one attend each per layer."""
    import numpy as np
    lens = host["lens"]
    row0 = np.concatenate([[0], np.cumsum(lens)[:-1]])
    calls = []
    for name, (q, K, V, begin, d) in host["layers"].items():
        rows = cpu.rows(K, V)
        outs = np.zeros(N_HEADS * d, np.float32)
        for s in range(len(lens)):
            calls.append((rows, np.ascontiguousarray(q[s]), int(row0[s] + begin[s]), int(row0[s] + lens[s]), outs))

    def batch():
        for rows, q, b, e, out in calls:
            rows.attend(q, b, e, N_HEADS, N_KV, out)

    s, n = cpu.loop(batch, seconds, min_calls=1)
    return {"value": round(nbytes / s / 1e9, 4), "unit": "GB/s", "us_per_step": round(s * 1e6, 1),
            "cores": cpu.threads, "kind": "port", "build": ORACLE_BUILD,
            "sample": f"{n} whole steps (64 attend calls: 32 sequences x 2 layers); host has "
                      f"{os.cpu_count()} logical CPUs"}


# ------------------------------------------------------------------ main
ONLY = ["sliding", "global", "stack", "stackwarm", "layerstack", "prefill", "chunks", "ragged", "layer", "matvec",
        "floors", "copy", "host"]


def run_only(args, torch, g4hip):
    with g4hip.Context(0) as ctx:
        prep = Prep(ctx, torch, 1234)
        k = max(20, args.steps // 4)
        fn = {"sliding": lambda: bench_sliding_decode(ctx, torch, prep, args.steps, args.warmup),
              "global": lambda: bench_global_decode(ctx, torch, prep, args.steps, args.warmup),
              "stack": lambda: bench_stack(ctx, torch, prep, g4hip, k, 5, cold=True),
              "stackwarm": lambda: bench_stack(ctx, torch, prep, g4hip, k, 5, cold=False),
              "layerstack": lambda: bench_layer_stack(ctx, torch, prep, g4hip, k, 5),
              "prefill": lambda: bench_prefill(ctx, torch, prep, min(args.steps, 20), args.warmup),
              "ragged": lambda: bench_ragged(ctx, torch, prep, max(5, k // 4), 2),
              "layer": lambda: bench_layer_steps(ctx, torch, prep, args.steps, args.warmup),
              "chunks": lambda: bench_prefill_chunks(ctx, torch, prep, 10, 3),
              "matvec": lambda: bench_matvec(ctx, torch, max(20, k // 2), args.warmup),
              "floors": lambda: bench_floors(torch, max(20, k), 5),
              "host": lambda: bench_host_attend(ctx, torch, prep, 20),
              "copy": lambda: bench_copy(torch, max(5, k // 4))}[args.only]
        res = fn()
        res.pop("host", None)
        print(json.dumps({"only": args.only, "result": res}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=3.0,
                    help="CPU-baseline sample per configuration (seconds, about)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--only", choices=ONLY,
                    help="run one workload alone (for profiling) and print its result; 'copy' is a plain "
                         "256 MiB device copy, the reference point for HBM byte counters")
    ap.add_argument("--summarize", metavar="DIR",
                    help="print the profiles/ tables reduced from rocprofv3 CSV output under DIR (trace/, fetch/, "
                         "write/, mfma/) and exit; needs no GPU")
    args = ap.parse_args()
    if args.summarize:
        print(summarize(args.summarize))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU: the backend runs on a single MI355X, and no run here uses a second "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)

    import torch
    import g4hip

    torch.cuda.init()
    if args.only:
        run_only(args, torch, g4hip)
        return
    steps, warmup = args.steps, args.warmup
    k = max(20, steps // 4)
    want = not args.no_cpu
    with g4hip.Context(0) as ctx:
        prep = Prep(ctx, torch, 1234)
        c5 = bench_ragged(ctx, torch, prep, steps, warmup, want_host=want)
        c1 = bench_sliding_decode(ctx, torch, prep, steps, warmup)
        c2 = bench_global_decode(ctx, torch, prep, steps, warmup)
        c3 = bench_stack(ctx, torch, prep, g4hip, k, 5, cold=True)
        c3w = bench_stack(ctx, torch, prep, g4hip, k, 5, cold=False, want_host=want)
        c3l = bench_layer_stack(ctx, torch, prep, g4hip, k, 5, want_host=want)
        c4 = bench_prefill(ctx, torch, prep, min(steps, 20), warmup, want_host=want)
        workloads = {"layer_drivers": bench_layer_steps(ctx, torch, prep, steps, warmup),
                     "prefill_long_context": bench_prefill_chunks(ctx, torch, prep, 10, 3),
                     "q8_0_matvec": bench_matvec(ctx, torch, max(20, k // 2), warmup),
                     "floors": bench_floors(torch, k, 5),
                     "host_buffer_attend": bench_host_attend(ctx, torch, prep, 20)}
    cpu = {}
    if want:
        timer = CpuTimer()
        sec = args.cpu_seconds
        cpu["5"] = cpu_ragged(timer, c5["host"], c5["step"]["bytes"], sec)
        cpu["1"] = cpu_decode(timer, c1["host"], 64, c1["bytes"], sec / 2)
        cpu["2"] = cpu_decode(timer, c2["host"], 4096, c2["bytes"], sec)
        cpu["3"] = cpu_stack(timer, c3w["host"], c3w["bytes_per_stack"], sec)
        cpu["layer_stack"] = cpu_layer_stack(timer, c3l["host"], sec)
        cpu["4"] = cpu_prefill(timer, c4["host"], sec)
    for r in (c1, c2, c3w, c3l, c4, c5):
        r.pop("host", None)
    c3l["attention_only_stack_us_resident"] = round(c3w["us_per_stack"], 2)
    c3l["cpu_baseline"] = cpu.get("layer_stack")
    workloads["layer_drivers"]["e2b_stack_35_layers_ctx8192_layer_attention"] = c3l

    # The headline: the ragged batch of 32 sequences, both layers per step.
    step_s = c5["step"]["us"] * 1e-6
    g5 = c5["global_d512"]
    prof5 = "decode_ragged_b32_ctx1k-32k.txt"
    headline_roof = roofline_hbm(g5["bytes"], g5["us"] * 1e-6,
                                 traffic_bytes(prof5, ["decode_stream_kernel<512", "decode_merge_kernel<3, 512"]),
                                 kernel="global layer of the batch: decode_stream_kernel<512> + its merge",
                                 bytes_per_launch=g5["bytes"], us_per_launch=round(g5["us"], 3),
                                 traffic_source=f"profiles/{prof5} (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, scaled "
                                                "by profiles/hbm_counter_calibration.txt)")
    prof2 = "decode_global_d512_ctx4096.txt"
    prof3 = "decode_e2b_stack_35_layers_ctx8192.txt"
    prof4 = profile_summary("prefill_2048_sliding_and_global.txt")
    mfma = {k2: v for k2, v in prof4.items() if "prefill_kernel" in k2 and "mfma_busy" in v}
    configs = {
        "1_sliding_decode_d256_ctx64": {
            "us_per_layer": round(c1["us_per_layer"], 3), "wall_us_per_layer": round(c1["wall_us_per_layer"], 3),
            "cache": c1["cache"],
            "roofline": roofline_hbm(c1["bytes"], c1["us_per_layer"] * 1e-6,
                                     traffic_bytes("decode_sliding_d256_ctx64.txt"),
                                     bytes_per_launch=c1["bytes"], note="launch-latency-bound: 147 KB per call"),
            "cpu_baseline": cpu.get("1")},
        "2_global_decode_d512_ctx4096": {
            "us_per_layer": round(c2["us_per_layer"], 3), "wall_us_per_layer": round(c2["wall_us_per_layer"], 3),
            "us_per_layer_resident": round(c2["us_per_layer_resident"], 3), "cache": c2["cache"],
            "roofline": roofline_hbm(c2["bytes"], c2["us_per_layer"] * 1e-6, traffic_bytes(prof2),
                                     bytes_per_launch=c2["bytes"], kernel="decode_split_kernel<512> + merge"),
            "cpu_baseline": cpu.get("2")},
        "3_e2b_stack_35_layers_ctx8192": {
            "us_per_stack": round(c3["us_per_stack"], 2), "us_per_layer_mean": round(c3["us_per_layer_mean"], 3),
            "wall_us_per_stack": round(c3["wall_us_per_stack"], 2), "cache": c3["cache"],
            "us_per_stack_resident": round(c3w["us_per_stack"], 2),
            "bytes_per_stack": c3["bytes_per_stack"], "unique_bytes_per_stack": c3["unique_bytes_per_stack"],
            "roofline": roofline_hbm(c3["bytes_per_stack"], c3["us_per_stack"] * 1e-6,
                                     traffic_bytes(prof3), bytes_per_launch=c3["bytes_per_stack"],
                                     note="35 calls (70 launches); bytes count every layer's rows once, "
                                          "shared layers re-reading layers 13/14"),
            "cpu_baseline": cpu.get("3")},
        "4_prefill_2048": {
            "sliding_d256_W512": {k2: round(v, 3) for k2, v in c4["sliding_d256_W512"].items()},
            "global_d512": {k2: round(v, 3) for k2, v in c4["global_d512"].items()},
            "both_layers_us": round(c4["both_layers_us"], 2),
            "roofline": {"bound": "mfma", "achieved": round(c4["both_layers_tflops"], 2),
                         "peak": round(SPLIT_PEAK_TFLOPS, 2), "unit": "TFLOP/s",
                         "frac": round(c4["frac_of_split_f16_peak"], 4),
                         "peak_note": "dense f16 MFMA peak 2500 TFLOP/s / 3.5 f16 products per counted product "
                                      "(3 per score, 4 per weight x value); counted FLOPs = 4 x 8 heads x d per "
                                      "attended pair",
                         "frac_of_f32_mfma_peak": round(c4["frac_of_f32_mfma_peak"], 4),
                         "traffic": traffic_bytes("prefill_2048_sliding_and_global.txt"),
                         "traffic_note": "HBM bytes of one step (both layers' K/V split, prefill and merge "
                                         "launches) from the rocprofv3 FETCH_SIZE / WRITE_SIZE passes in profiles/",
                         "dtype": "f32 in and out; products as split-f16 MFMAs (v_mfma_f32_16x16x32_f16 on f16 hi "
                                  "+ lo halves of each operand), f32 accumulation; units whose inputs the split "
                                  "does not carry use v_mfma_f32_16x16x4f32",
                         "mfma_busy_counter": {k2: v["mfma_busy"] for k2, v in mfma.items()} or None,
                         "mfma_source": "profiles/prefill_2048_sliding_and_global.txt (SQ_VALU_MFMA_BUSY_CYCLES)"},
            "cpu_baseline": cpu.get("4")},
        "5_ragged_decode_b32": {
            "global_d512": {k2: round(v, 4) for k2, v in c5["global_d512"].items()},
            "sliding_d256_W512": {k2: round(v, 4) for k2, v in c5["sliding_d256_W512"].items()},
            "step_us": round(c5["step"]["us"], 2),
            # In the step the sliding layer runs after the global layer, whose
            # 2 GB stream evicts its 34 MB from the Infinity Cache: its share of
            # the step is an HBM-cold read, unlike its own (resident) timing.
            "sliding_in_step_us": round(c5["step"]["us"] - c5["global_d512"]["us"], 2),
            "lengths": c5["lengths"], "cache": c5["cache"],
            "roofline": headline_roof, "cpu_baseline": cpu.get("5")},
    }
    line = {
        "metric": METRIC,
        "value": round(c5["step"]["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(c5["step"]["wall_us"] * 1e-3, 6),
        "us_per_layer": {"global_d512": round(g5["us"], 3), "sliding_d256_W512": round(c5["sliding_d256_W512"]["us"], 3)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "ragged decode: 32 sequences with context lengths U[1024, 32768] (seed 2024), one "
                               "token each, through a global layer (head_dim 512, whole contexts) and a sliding "
                               "layer (head_dim 256, window 512), 8 q heads / 1 kv head, one launch per layer",
                   "batch": RAGGED_B, "head_dims": [512, 256], "n_heads": N_HEADS, "n_kv_heads": N_KV,
                   "parallelism": "single GPU"},
        "roofline": headline_roof,
        "cpu_baseline": cpu.get("5"),
        "configs": configs,
        "workloads": workloads,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
