"""Chunked prefill on the GPU against the oracle.

The reference has no batched prefill: a prompt runs one token at a time
(crates/llm-gemma4/src/impl_/generate.rs:37-41), so query i of a chunk must
equal the oracle's attend over exactly the rows a decode at position
pos0 + i sees (eng/mod.rs:10-36).  Tolerance as for decode: 1e-4 relative
(crates/llm-gemma4/tests/synthetic_generate.rs:74-83).
"""
import numpy as np
import pytest
import torch

import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def prefill(ctx, q, K, V, pos0, N, window, d):
    out = torch.zeros(N * 8 * d, device="cuda")
    ctx.attend_prefill(dev(q), dev(K), dev(V), pos0, N, window, 8, 1, d, out)
    ctx.check_status()
    return out.cpu().numpy().reshape(N, 8 * d)


def case(seed, rows, d, glob):
    freqs = I.rope_freqs(seed + 1, d) if glob else None
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    K, V = I.kv_rows(seed, rows, d, base, freqs)
    q = I.queries(seed + 2, rows, d, base, freqs, 0)
    return q, K, V


@pytest.mark.parametrize("d,window", [(256, 8), (256, 0), (512, 0), (512, 5), (256, 512)])
@pytest.mark.parametrize("pos0,N", [(0, 40), (17, 23)])
def test_prefill_every_query(ctx, d, window, pos0, N):
    q, K, V = case(11 + d + window, pos0 + N, d, d == 512)
    got = prefill(ctx, q[pos0:], K, V, pos0, N, window, d)
    for i in range(N):
        b, e = I.attended_range(pos0 + i, window)
        assert I.rel_err(got[i], orc.attend(q[pos0 + i], K[b:e], V[b:e], 8, 1)) <= TOL, i


@pytest.mark.parametrize("name,d,window", [("config4_sliding_W512", 256, 512), ("config4_global", 512, 0)])
def test_config4_prefill_2048(ctx, name, d, window):
    """2048-token prompt; every window/causal boundary row plus a seeded sample."""
    print(f"[case] {name}", flush=True)
    N = 2048
    q, K, V = case(4000 + d, N, d, d == 512)
    got = prefill(ctx, q, K, V, 0, N, window, d)
    rows = sorted(set([0, 1, 2, 15, 16, 17, 510, 511, 512, 513, 1023, 1024, 1535, 2046, 2047]) |
                  set(np.random.default_rng(8).integers(0, N, 96).tolist()))
    worst = 0.0
    for i in rows:
        b, e = I.attended_range(i, window)
        worst = max(worst, I.rel_err(got[i], orc.attend(q[i], K[b:e], V[b:e], 8, 1)))
    print(f"[parity] {name}: worst rel err {worst:.2e} over {len(rows)} rows")
    assert worst <= TOL
    assert np.all(np.isfinite(got))


def test_prefill_never_reads_future_or_out_of_window_rows(ctx):
    """Rows after the chunk and before the first window hold NaN."""
    d, W, pos0, N = 256, 64, 200, 50
    q, K, V = case(5, pos0 + N + 30, d, False)
    K[pos0 + N:] = np.nan
    V[pos0 + N:] = np.nan
    first = I.attended_range(pos0, W)[0]
    K[:first] = np.nan
    V[:first] = np.nan
    got = prefill(ctx, q[pos0:pos0 + N], K, V, pos0, N, W, d)
    assert np.all(np.isfinite(got))
    for i in (0, 1, N // 2, N - 1):
        b, e = I.attended_range(pos0 + i, W)
        assert I.rel_err(got[i], orc.attend(q[pos0 + i], K[b:e], V[b:e], 8, 1)) <= TOL


@pytest.mark.parametrize("d,window,pos0,N", [(512, 0, 6000, 64), (512, 0, 0, 700), (256, 512, 3000, 300),
                                             (512, 0, 12000, 24)])
def test_prefill_long_contexts_and_unit_lengths(ctx, d, window, pos0, N):
    """Chunks deep into a long context and chunk lengths whose unit table
    uses other unit lengths than the 2048-token prompt's (the lengths are
    chosen per shape); sampled rows against the oracle."""
    print(f"[case] prefill d={d} W={window} pos0={pos0} N={N}", flush=True)
    q, K, V = case(900 + d + pos0, pos0 + N, d, d == 512)
    got = prefill(ctx, q[pos0:], K, V, pos0, N, window, d)
    rows = sorted({0, 1, N // 2, N - 2, N - 1} | set(np.random.default_rng(pos0).integers(0, N, 12).tolist()))
    for i in rows:
        b, e = I.attended_range(pos0 + i, window)
        assert I.rel_err(got[i], orc.attend(q[pos0 + i], K[b:e], V[b:e], 8, 1)) <= TOL, i


@pytest.mark.parametrize("pos0,N,window,d", [(0, 4096, 0, 512), (16384, 256, 0, 512), (0, 1024, 0, 512),
                                             (0, 300, 0, 512), (5000, 333, 512, 256)])
def test_prefill_schedule_forms(ctx, pos0, N, window, d):
    """The host schedule takes several forms (a 4096-token causal prompt pairs
    whole blocks, a deep 256-token chunk cuts every block into 8 units, 1024
    and 300 tokens are packed stream-K with many split blocks); the rows of
    the blocks cut into the most units -- merged from the most partials --
    and of some whole blocks are checked against the oracle."""
    import g4hip
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units, _ = g4hip.prefill_schedule(pos0, N, window, d, 1, cus)
    n_units = np.bincount(units[:, 0], minlength=(N + 7) // 8)
    order = np.argsort(-n_units, kind="stable")
    blocks = list(order[:3]) + [b for b in order[::-1] if n_units[b] == 1][:1]
    print(f"[case] prefill schedule pos0={pos0} N={N} W={window} d={d}: units {len(units)}, "
          f"most per block {n_units.max()}, checked blocks {blocks}", flush=True)
    q, K, V = case(77 + d + pos0 + N, pos0 + N, d, d == 512)
    got = prefill(ctx, q[pos0:], K, V, pos0, N, window, d)
    rows = sorted({i for b in blocks for i in range(8 * b, min(8 * b + 8, N))})
    for i in rows:
        b, e = I.attended_range(pos0 + i, window)
        assert I.rel_err(got[i], orc.attend(q[pos0 + i], K[b:e], V[b:e], 8, 1)) <= TOL, i
