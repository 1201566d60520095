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

import g4hip
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


def check_all_rows(name, got, q, K, V, pos0, window):
    """Every query of the chunk against the oracle's token-at-a-time loop
    (generate.rs:37-41): the same non-finite outputs, and the finite ones
    within the tolerance."""
    ref, status = orc.attend_prefill(q, K, V, pos0, window, 8, 1)
    assert not status.any(), f"{name}: oracle softmax failed on rows {np.nonzero(status)[0][:8]}"
    fin_ref, fin_got = np.isfinite(ref), np.isfinite(got)
    bad = np.nonzero((fin_ref != fin_got).any(axis=1))[0]
    assert bad.size == 0, f"{name}: finite/non-finite pattern differs on rows {bad[:8]}"
    both = np.where(fin_ref, ref, 0.0), np.where(fin_got, got, 0.0)
    worst = max(I.rel_err(both[1][i], both[0][i]) for i in range(ref.shape[0]))
    print(f"[parity] {name}: worst rel err {worst:.2e} over all {ref.shape[0]} rows, "
          f"{int((~fin_ref).sum())} non-finite outputs", flush=True)
    assert worst <= TOL
    return worst


@pytest.mark.parametrize("name,d,window", [("sliding_d256_W512", 256, 512), ("global_d512", 512, 0)])
def test_prefill_2048_every_row(ctx, name, d, window):
    """2048-token prompt: every query row against the oracle."""
    print(f"[case] {name}", flush=True)
    N = 2048
    q, K, V = case(4000 + d, N, d, d == 512)
    got = prefill(ctx, q, K, V, 0, N, window, d)
    assert np.all(np.isfinite(got))
    check_all_rows(name, got, q, K, V, 0, window)


@pytest.mark.parametrize("d,window,pos0,N", [(256, 64, 200, 48), (512, 0, 96, 40), (256, 512, 1000, 64)])
def test_prefill_non_finite_v_reaches_only_the_queries_that_attend_it(ctx, d, window, pos0, N):
    """A NaN or +inf V value in a row that some queries of a position block
    attend and others mask: the reference multiplies only attended rows
    (model.rs:339-341), so the masking queries stay finite.  Rows at the
    causal edge (a key inside the block) and at the window edge (the first
    key some of the block's queries still see)."""
    print(f"[case] prefill non-finite V d={d} W={window} pos0={pos0} N={N}", flush=True)
    q, K, V = case(31 + d + pos0, pos0 + N, d, d == 512)
    P0 = pos0 + 16                  # a position block inside the chunk
    causal = P0 + 3                 # attended by P0+3.., masked for P0..P0+2
    V[causal, 5] = np.nan
    V[causal, d - 1] = np.inf
    if window:
        edge = P0 + 4 - window      # attended by ..P0+3, masked for P0+4..
        V[edge, 7] = np.inf
        V[edge, 100] = np.nan
    got = prefill(ctx, q[pos0:], K, V, pos0, N, window, d)
    check_all_rows(f"non-finite V d={d} W={window}", got, q[pos0:], K, V, pos0, window)
    # The block's first three queries mask the causal-edge row, its last four
    # the window-edge row: those dims stay finite in every head.
    heads = np.arange(8) * d
    for i in range(P0 - pos0, P0 - pos0 + 3):
        assert np.all(np.isfinite(got[i][np.concatenate([heads + 5, heads + d - 1])])), i
    if window:
        for i in range(P0 - pos0 + 4, P0 - pos0 + 8):
            assert np.all(np.isfinite(got[i][np.concatenate([heads + 7, heads + 100])])), i


@pytest.mark.parametrize("d,window", [(256, 512), (256, 16), (512, 0)])
def test_prefill_non_finite_scores_fail_the_call(ctx, d, window):
    """A NaN or +inf score (here from one K value) in a row that some query
    attends fails the call with "softmax input is not finite", as that
    query's softmax does in the token-at-a-time loop (model.rs:362-364,
    ops.rs:116-121); a -inf score is only a zero weight.  q's dim 3 is made
    positive so that an infinite K value there gives a score of its sign."""
    pos0, N, row = 37, 45, 37 + 20
    q, K, V = case(77 + d + window, pos0 + N, d, d == 512)
    q = np.ascontiguousarray(q).copy()
    q.reshape(pos0 + N, 8, d)[:, :, 3] = np.abs(q.reshape(pos0 + N, 8, d)[:, :, 3]) + 0.5
    for name, value, fails in [("nan", np.nan, True), ("+inf", np.inf, True), ("-inf", -np.inf, False)]:
        print(f"[case] prefill non-finite score {name} d={d} W={window}", flush=True)
        Kx = K.copy()
        Kx[row, 3] = value
        ref, status = orc.attend_prefill(q[pos0:], Kx, V, pos0, window, 8, 1)
        assert bool(status.any()) == fails, name
        out = torch.zeros(N * 8 * d, device="cuda")
        ctx.attend_prefill(dev(q[pos0:]), dev(Kx), dev(V), pos0, N, window, 8, 1, d, out)
        if fails:
            with pytest.raises(g4hip.EngError, match="softmax input is not finite"):
                ctx.check_status()
        else:
            ctx.check_status()
            check_all_rows(f"-inf score d={d} W={window}", out.cpu().numpy().reshape(N, 8 * d), q[pos0:], Kx, V,
                           pos0, window)


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
