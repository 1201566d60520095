"""The device entry points inside captured HIP graphs.

A serving loop captures its per-token work once and replays it.  Each test
warms the call up eagerly (so that workspaces and prefill unit tables
exist), captures it, then replays the graph several times with new inputs
copied in between -- eager work and synchronisations between the replays --
and checks every replay against an eager call on the same inputs, bit for
bit (the kernels are deterministic).
"""
import numpy as np
import pytest
import torch

import inputs as I

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def replay_and_check(ctx, run, inputs, outputs, fresh, n=4):
    """run() launches the work on the current stream reading `inputs`
    (tensors) and writing `outputs`; fresh(i) gives new input values."""
    run()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for i in range(n):
        for t, v in zip(inputs, fresh(i)):
            t.copy_(v)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outputs]
        for o in outputs:
            o.fill_(float("nan"))
        run()  # eager, same inputs
        torch.cuda.synchronize()
        for a, b in zip(got, outputs):
            assert torch.equal(a, b), f"replay {i} differs from the eager call"
    ctx.check_status()


@pytest.mark.parametrize("T,d", [(4096, 512), (512, 256), (40, 256)])
def test_decode_in_a_graph(ctx, T, d):
    rng = np.random.default_rng(T + d)
    q = dev(rng.standard_normal(8 * d).astype(np.float32))
    K = dev(rng.standard_normal((T, d)).astype(np.float32))
    V = dev(rng.standard_normal((T, d)).astype(np.float32))
    out = torch.zeros(8 * d, device="cuda")
    replay_and_check(ctx, lambda: ctx.attend_decode(q, K, V, 0, T, 8, 1, d, out), [q, K], [out],
                     lambda i: [torch.randn(8 * d, device="cuda"), torch.randn(T, d, device="cuda")])


def test_ragged_stream_decode_in_a_graph(ctx):
    lens = np.array([5, 40, 20000, 3000, 700] * 4, np.int64)
    d = 512
    rng = np.random.default_rng(1)
    total = int(lens.sum())
    K = dev(rng.standard_normal((total, d)).astype(np.float32))
    V = dev(rng.standard_normal((total, d)).astype(np.float32))
    q = dev(rng.standard_normal((len(lens), 8 * d)).astype(np.float32))
    row0 = dev(np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64))
    begin = dev(np.zeros(len(lens), np.int64))
    end = dev(lens)
    out = torch.zeros(len(lens) * 8 * d, device="cuda")
    replay_and_check(ctx, lambda: ctx.attend_decode_batch(q, K, V, row0, begin, end, int(lens.max()), 8, 1, d, out),
                     [q], [out], lambda i: [torch.randn(len(lens), 8 * d, device="cuda")])


@pytest.mark.parametrize("d,window", [(512, 0), (256, 512)])
def test_prefill_in_a_graph(ctx, d, window):
    N = 300
    rng = np.random.default_rng(d)
    q = dev(rng.standard_normal((N, 8 * d)).astype(np.float32))
    K = dev(rng.standard_normal((N, d)).astype(np.float32))
    V = dev(rng.standard_normal((N, d)).astype(np.float32))
    out = torch.zeros(N * 8 * d, device="cuda")
    replay_and_check(ctx, lambda: ctx.attend_prefill(q, K, V, 0, N, window, 8, 1, d, out), [q, V], [out],
                     lambda i: [torch.randn(N, 8 * d, device="cuda"), torch.randn(N, d, device="cuda")])


def test_prepare_and_decode_step_in_a_graph(ctx):
    """A global layer step: fused q/k/v preparation with the append into the
    cache, then the decode over the cache."""
    d, T = 512, 1024
    rng = np.random.default_rng(7)
    K = dev(rng.standard_normal((T, d)).astype(np.float32))
    V = dev(rng.standard_normal((T, d)).astype(np.float32))
    q, k, v = (dev(rng.standard_normal(n).astype(np.float32)) for n in (8 * d, d, d))
    wq, wk = dev(rng.uniform(0.5, 1.5, d).astype(np.float32)), dev(rng.uniform(0.5, 1.5, d).astype(np.float32))
    freqs = dev(I.rope_freqs(3, d))
    out = torch.zeros(8 * d, device="cuda")
    qs, ks, vs = q.clone(), k.clone(), v.clone()

    def run():
        q.copy_(qs), k.copy_(ks), v.copy_(vs)  # the preparation works in place
        ctx.prepare_qkv(q, k, v, 1, T - 1, 8, 1, d, wq, wk, 1e-6, I.GLOBAL_BASE, freqs,
                        k_rows=K.view(-1)[(T - 1) * d:], v_rows=V.view(-1)[(T - 1) * d:], row_stride=d)
        ctx.attend_decode(q, K, V, 0, T, 8, 1, d, out)

    replay_and_check(ctx, run, [qs, ks, vs], [out],
                     lambda i: [torch.randn(8 * d, device="cuda"), torch.randn(d, device="cuda"),
                                torch.randn(d, device="cuda")])


@pytest.mark.parametrize("rows,cols", [(4096, 1536), (70000, 1536)])
def test_q8_0_matvecs_in_a_graph(ctx, rows, cols):
    """Small matrices quantize inside the mat-vec; large ones quantize into
    the context's workspace first (a second kernel in the graph)."""
    w = dev(I.q8_0_bytes(np.random.default_rng(rows).uniform(-1, 1, rows * cols).astype(np.float32)))
    up = dev(I.q8_0_bytes(np.random.default_rng(rows + 1).uniform(-1, 1, rows * cols).astype(np.float32)))
    x = torch.randn(cols, device="cuda")
    a, b = torch.zeros(rows, device="cuda"), torch.zeros(rows, device="cuda")

    def run():
        ctx.logits_q8_0(w, rows, cols, x, 30.0, a)
        ctx.gated_ffn_q8_0(w, up, rows, cols, x, b)

    replay_and_check(ctx, run, [x], [a, b], lambda i: [torch.randn(cols, device="cuda") * (i + 1)])


def test_fused_decode_step_in_a_graph(ctx):
    """A global layer step as g4_layer_attention runs it: one launch that
    prepares q and the new row, appends the row and attends (plus the merge)."""
    d, T = 512, 2048
    rng = np.random.default_rng(9)
    K = dev(rng.standard_normal((T, d)).astype(np.float32))
    V = dev(rng.standard_normal((T, d)).astype(np.float32))
    q, k, v = (dev(rng.standard_normal(n).astype(np.float32)) for n in (8 * d, d, d))
    wq, wk = dev(rng.uniform(0.5, 1.5, d).astype(np.float32)), dev(rng.uniform(0.5, 1.5, d).astype(np.float32))
    freqs = dev(I.rope_freqs(4, d))
    out = torch.zeros(8 * d, device="cuda")

    def run():
        ctx.decode_step_fused(q, k, v, wq, wk, 1e-6, I.GLOBAL_BASE, freqs, T - 1, K, V, d, T,
                              K.view(-1)[(T - 1) * d:], V.view(-1)[(T - 1) * d:], 8, 1, d, out)

    replay_and_check(ctx, run, [q, k, v], [out],
                     lambda i: [torch.randn(8 * d, device="cuda"), torch.randn(d, device="cuda"),
                                torch.randn(d, device="cuda")])
