"""Decode attention on the GPU against the oracle, through the C ABI.

Tolerance (floating point): max |gpu - oracle| <= 1e-4 * max(|gpu|, |oracle|, 1),
the reference's own assert_relative_eq (crates/llm-gemma4/tests/synthetic_generate.rs:74-83).
The attended index set is checked exactly where the caller derives it.
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


def run_decode(ctx, q, K, V, begin, end, n_heads, n_kv, d, scale=1.0):
    out = torch.zeros(n_heads * d, device="cuda")
    ctx.attend_decode(dev(q), dev(K), dev(V), begin, end, n_heads, n_kv, d, out, scale=scale)
    ctx.check_status()
    return out.cpu().numpy()


@pytest.mark.parametrize("name,T,d,glob", [("sliding_d256_ctx64", 64, 256, False),
                                           ("global_d512_ctx4096", 4096, 512, True)])
def test_measured_decode_workloads(ctx, name, T, d, glob):
    print(f"[case] {name}", flush=True)
    q, K, V, _ = I.decode_case(1000 + T, T, d, glob)
    begin, end = I.attended_range(T - 1, 0 if glob else I.WINDOW)
    assert (begin, end) == (0, T)
    out = run_decode(ctx, q, K, V, begin, end, 8, 1, d)
    ref = orc.attend(q, K[begin:end], V[begin:end], 8, 1)
    floor = np.max(np.abs(ref - orc.attend_f64(q, K[begin:end], V[begin:end], 8, 1)))
    err = I.rel_err(out, ref)
    print(f"[parity] {name}: rel err {err:.2e} (f32-vs-f64 floor of the oracle {floor:.2e})")
    assert err <= TOL


@pytest.mark.parametrize("T,d", [(131072, 512), (65536, 256)])
def test_decode_longest_contexts(ctx, T, d):
    """Gemma 4's longest context, one sequence: 256 splits of 512 keys (16
    pairs per workgroup) on the global layer, and a whole-history d=256
    cache of 64K rows; every row attended, against the oracle, and the
    allocation-free form (its static scratch holds this plan) gives the same
    bits."""
    print(f"[case] decode T={T} d={d}", flush=True)
    q, K, V, _ = I.decode_case(31 + T, T, d, d == 512)
    out = run_decode(ctx, q, K, V, 0, T, 8, 1, d)
    ref = orc.attend_rows(q, K, V, 8, 1, threads=8)  # bit-equal to attend (test_oracle), one head per thread
    err = I.rel_err(out, ref)
    print(f"[parity] decode T={T} d={d}: rel err {err:.2e}", flush=True)
    assert err <= TOL
    o2 = torch.zeros(8 * d, device="cuda")
    ctx.attend_decode_noalloc(dev(q), dev(K), dev(V), 0, T, 8, 1, d, o2)
    ctx.check_status()
    assert np.array_equal(o2.cpu().numpy(), out)


@pytest.mark.parametrize("d", [256, 512])
@pytest.mark.parametrize("T", [1, 2, 15, 16, 17, 33, 100, 511, 512, 513, 1000])
def test_decode_lengths(ctx, d, T):
    q, K, V, _ = I.decode_case(7 * T + d, T, d, d == 512)
    out = run_decode(ctx, q, K, V, 0, T, 8, 1, d)
    assert I.rel_err(out, orc.attend(q, K, V, 8, 1)) <= TOL


@pytest.mark.parametrize("T,chunk", [(3000, 16), (3000, 32), (3000, 48), (3000, 80), (3000, 256), (3000, 4096),
                                     (5000, 16), (1500, 16), (700, 16), (4200, 0), (8300, 0), (12400, 0)])
def test_decode_split_counts(ctx, T, chunk):
    """Split-K partials merge to the same result for any split size (a
    multiple of 16 keys, not only powers of two): the merge's shapes for 12
    to 313 splits (two batches) and a single split; 0 = the automatic size,
    which just past 256 x a power of two is no longer a power of two
    (4200 keys: 32, 8300: 48, 12400: 64 keys per split)."""
    d = 512
    q, K, V, _ = I.decode_case(55 + T, T, d, True)
    ctx.set_decode_chunk(chunk)
    try:
        out = run_decode(ctx, q, K, V, 0, T, 8, 1, d)
    finally:
        ctx.set_decode_chunk(0)
    assert I.rel_err(out, orc.attend(q, K, V, 8, 1)) <= TOL


def test_sliding_window_inside_longer_cache(ctx):
    """A sliding layer at position 1000 reads rows 489..1000 of its full-history cache."""
    d, pos = 256, 1000
    K, V = I.kv_rows(77, pos + 1, d, I.LOCAL_BASE, None)
    q = I.queries(78, 1, d, I.LOCAL_BASE, None, pos)[0]
    begin, end = I.attended_range(pos, I.WINDOW)
    assert range(begin, end) == orc.windowed_len(pos + 1, 512) == range(489, 1001)
    K[begin] = q[:d]  # the first row inside the window dominates head 0's softmax
    K[:begin] = np.nan  # rows outside the window must never be read
    V[:begin] = np.nan
    out = run_decode(ctx, q, K, V, begin, end, 8, 1, d)
    ref = orc.attend(q, K[begin:end], V[begin:end], 8, 1)
    assert I.rel_err(out, ref) <= TOL
    # so a window one row short is a clearly different answer
    short = orc.attend(q, K[begin + 1:end], V[begin + 1:end], 8, 1)
    assert I.rel_err(short, ref) > 0.1


@pytest.mark.parametrize("n_heads,n_kv,d,T", [(4, 2, 8, 5), (4, 2, 16, 9), (8, 1, 64, 300), (2, 2, 16, 16),
                                              (16, 2, 256, 200), (6, 4, 32, 7)])
def test_other_shapes(ctx, n_heads, n_kv, d, T):
    rng = np.random.default_rng(n_heads * 1000 + d + T)
    q = rng.standard_normal(n_heads * d).astype(np.float32)
    K = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    out = run_decode(ctx, q, K, V, 0, T, n_heads, n_kv, d, scale=0.3)
    assert I.rel_err(out, orc.attend(q, K, V, n_heads, n_kv, 0.3)) <= TOL


def test_host_attend_mirror(ctx):
    """g4_attend takes the same arguments as the reference's attend (model.rs:348)."""
    q, K, V, _ = I.decode_case(5, 200, 256, False)
    out = ctx.attend(q, K, V, 8, 1, 1.0)
    assert I.rel_err(out, orc.attend(q, K, V, 8, 1)) <= TOL
    rng = np.random.default_rng(2)
    q2 = rng.standard_normal(4 * 16).astype(np.float32)
    K2 = rng.standard_normal((7, 2 * 16)).astype(np.float32)
    V2 = rng.standard_normal((7, 2 * 16)).astype(np.float32)
    assert I.rel_err(ctx.attend(q2, K2, V2, 4, 2, 1.0), orc.attend(q2, K2, V2, 4, 2)) <= TOL


def test_host_attend_q_length_not_a_multiple_of_heads(ctx):
    """head_dim = q.len() / n_heads; a q with a remainder leaves the heads'
    concatenation shorter than q, and attend returns Compute("softmax input
    is not finite") (model.rs:349, 362-364) -- the oracle and the backend."""
    rng = np.random.default_rng(9)
    d = 16
    q = rng.standard_normal(8 * d + 3).astype(np.float32)
    K = rng.standard_normal((5, d)).astype(np.float32)
    V = rng.standard_normal((5, d)).astype(np.float32)
    with pytest.raises(orc.OracleError, match="softmax input is not finite"):
        orc.attend(q, K, V, 8, 1)
    with pytest.raises(g4hip.EngError, match="softmax input is not finite"):
        ctx.attend(q, K, V, 8, 1, 1.0)


@pytest.mark.parametrize("d", [256, 512, 16])
def test_non_finite_softmax_is_an_error(ctx, d):
    n_kv = 1
    T = 40
    rng = np.random.default_rng(3)
    q = rng.standard_normal(8 * d).astype(np.float32)
    K = rng.standard_normal((T, d)).astype(np.float32)
    V = rng.standard_normal((T, d)).astype(np.float32)
    for poison in ("q_nan", "k_inf"):
        q2, K2 = q.copy(), K.copy()
        if poison == "q_nan":
            q2[5] = np.nan
        else:
            K2[17, 3] = np.inf
        with pytest.raises(orc.OracleError, match="softmax input is not finite"):
            orc.attend(q2, K2, V, 8, n_kv)
        out = torch.zeros(8 * d, device="cuda")
        ctx.attend_decode(dev(q2), dev(K2), dev(V), 0, T, 8, n_kv, d, out)
        with pytest.raises(g4hip.EngError, match="softmax input is not finite") as e:
            ctx.check_status()
        assert e.value.kind == "Compute"
    # the status is cleared once reported
    ctx.attend_decode(dev(q), dev(K), dev(V), 0, T, 8, n_kv, d, torch.zeros(8 * d, device="cuda"))
    ctx.check_status()


def test_empty_context_is_an_error(ctx):
    with pytest.raises(g4hip.EngError, match="softmax input is not finite"):
        ctx.attend(np.ones(8 * 256, np.float32), np.zeros((0, 256), np.float32), np.zeros((0, 256), np.float32),
                   8, 1, 1.0)


@pytest.mark.parametrize("d,glob", [(512, True), (256, False)])
def test_ragged_batch_32_sequences_1k_to_32k(ctx, d, glob):
    """32 sequences, lengths U[1024, 32768], one launch per layer type."""
    print(f"[case] ragged batch d={d}", flush=True)
    lens = I.ragged_lengths(2024)
    B = lens.size
    freqs = I.rope_freqs(99, d) if glob else None
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    row0 = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    total = int(lens.sum())
    # every sequence's own cache, packed one after another
    begin = np.array([I.attended_range(int(L) - 1, 0 if glob else I.WINDOW)[0] for L in lens], np.int64)
    end = lens.copy()
    # Rows a sequence does not attend hold NaN: reading one would poison the result.
    K = np.full((total, d), np.nan, np.float32)
    V = np.full((total, d), np.nan, np.float32)
    for s in range(B):
        n = int(end[s] - begin[s])
        k, v = I.kv_rows(3000 + s, n, d, base, freqs, pos0=int(begin[s]))
        K[row0[s] + begin[s]:row0[s] + end[s]] = k
        V[row0[s] + begin[s]:row0[s] + end[s]] = v
    q = np.stack([I.queries(5000 + s, 1, d, base, freqs, int(lens[s]) - 1)[0] for s in range(B)])
    out = torch.zeros(B * 8 * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(begin), dev(end), int((end - begin).max()),
                            8, 1, d, out)
    ctx.check_status()
    got = out.cpu().numpy().reshape(B, -1)
    worst = 0.0
    for s in range(B):
        rows = slice(row0[s] + begin[s], row0[s] + end[s])
        worst = max(worst, I.rel_err(got[s], orc.attend(q[s], K[rows], V[rows], 8, 1)))
    print(f"[parity] ragged d={d}: worst rel err {worst:.2e}")
    assert worst <= TOL


def test_ragged_range_longer_than_bound_is_reported(ctx):
    d = 256
    K, V = I.kv_rows(1, 64, d, I.LOCAL_BASE, None)
    q = I.queries(2, 2, d, I.LOCAL_BASE, None, 63)
    out = torch.zeros(2 * 8 * d, device="cuda")
    begin = np.array([0, 0], np.int64)
    end = np.array([64, 10], np.int64)
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), None, dev(begin), dev(end), 32, 8, 1, d, out)
    with pytest.raises(g4hip.EngError) as e:
        ctx.check_status()
    assert e.value.kind == "ContextTooLong"


def _ragged_case(seed, lens, d, n_heads=8, n_kv=1, gap=3):
    """Packed caches of several sequences (NaN rows between them) and their queries."""
    rng = np.random.default_rng(seed)
    B = len(lens)
    width = n_kv * d
    row0 = np.zeros(B, np.int64)
    at = 0
    for s in range(B):
        row0[s] = at
        at += int(lens[s]) + gap
    K = np.full((at, width), np.nan, np.float32)
    V = np.full((at, width), np.nan, np.float32)
    for s in range(B):
        K[row0[s]:row0[s] + lens[s]] = rng.standard_normal((int(lens[s]), width), dtype=np.float32)
        V[row0[s]:row0[s] + lens[s]] = rng.standard_normal((int(lens[s]), width), dtype=np.float32)
    q = rng.standard_normal((B, n_heads * d), dtype=np.float32) * 0.2
    return q, K, V, row0


# Batches with B * max_len >= 32 * 4 * 256 take the streamed path (one
# workgroup per CU walking the concatenated 32-key pairs); smaller ones, or
# more than 1024 sequences, the per-sequence split grid.
@pytest.mark.parametrize("name,lens,d,n_heads,n_kv", [
    ("stream_short_and_long", [5, 40, 20000], 256, 8, 1),
    ("stream_one_key_each", [1, 1, 1, 1, 9000], 512, 8, 1),
    ("stream_fewer_pairs_than_cus", [328] + [1] * 99, 256, 8, 1),
    ("stream_many_short", list(range(1, 301)), 256, 8, 1),  # many whole sequences per workgroup
    ("stream_two_kv_heads", [700, 33, 8000, 64, 1], 256, 16, 2),
    ("stream_odd_pairs", [16, 48, 80, 40000, 17, 31, 33], 512, 8, 1),
    ("split_two_short", [5, 40], 256, 8, 1),
    ("split_one_key_each", [1, 1, 1, 1], 512, 8, 1),
    ("split_over_stream_limit", [7] * 1030 + [300], 256, 8, 1),
])
def test_ragged_batch_shapes(ctx, name, lens, d, n_heads, n_kv):
    print(f"[case] ragged {name} d={d} B={len(lens)}", flush=True)
    lens = np.array(lens, np.int64)
    q, K, V, row0 = _ragged_case(len(lens) * 7 + d, lens, d, n_heads, n_kv)
    B = len(lens)
    begin = np.zeros(B, np.int64)
    out = torch.zeros(B * n_heads * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(begin), dev(lens), int(lens.max()),
                            n_heads, n_kv, d, out)
    ctx.check_status()
    got = out.cpu().numpy().reshape(B, -1)
    worst = 0.0
    for s in range(B):
        rows = slice(row0[s], row0[s] + lens[s])
        worst = max(worst, I.rel_err(got[s], orc.attend(q[s], K[rows], V[rows], n_heads, n_kv)))
    print(f"[parity] ragged {name}: worst rel err {worst:.2e}")
    assert worst <= TOL


@pytest.mark.parametrize("name,lens,d", [
    ("stream", [16, 48, 80, 40000, 17, 31, 33], 512),
    ("split", [5, 40, 700], 256),
])
def test_ragged_batch_softmax_scale(ctx, name, lens, d):
    """attend's score scale (model.rs:326-343) through the batched forms:
    the stream-K kernel (a batch with a 40000-key sequence) and the split
    grid, against the oracle with the same scale."""
    print(f"[case] ragged {name} d={d} scale 0.3", flush=True)
    lens = np.array(lens, np.int64)
    q, K, V, row0 = _ragged_case(len(lens) * 11 + d, lens, d)
    B = len(lens)
    out = torch.zeros(B * 8 * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(np.zeros(B, np.int64)), dev(lens), int(lens.max()),
                            8, 1, d, out, scale=0.3)
    ctx.check_status()
    got = out.cpu().numpy().reshape(B, -1)
    worst = 0.0
    for s in range(B):
        rows = slice(row0[s], row0[s] + lens[s])
        worst = max(worst, I.rel_err(got[s], orc.attend(q[s], K[rows], V[rows], 8, 1, scale=0.3)))
    print(f"[parity] ragged {name} scale 0.3: worst rel err {worst:.2e}")
    assert worst <= TOL


@pytest.mark.parametrize("chunk", [64, 16, 48, 80])
def test_ragged_batch_with_set_split_size(ctx, chunk):
    """A split size set by the caller selects the per-sequence split grid;
    the merge folds 1 to 313 splits per sequence (at 16 keys: 94, 2, 21,
    256 and 313, the last in two batches)."""
    lens = np.array([1500, 20, 333, 4096, 1, 5000], np.int64)
    d = 512
    q, K, V, row0 = _ragged_case(77, lens, d)
    out = torch.zeros(len(lens) * 8 * d, device="cuda")
    ctx.set_decode_chunk(chunk)
    try:
        ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(np.zeros(len(lens), np.int64)), dev(lens),
                                int(lens.max()), 8, 1, d, out)
        ctx.check_status()
    finally:
        ctx.set_decode_chunk(0)
    got = out.cpu().numpy().reshape(len(lens), -1)
    for s in range(len(lens)):
        rows = slice(row0[s], row0[s] + lens[s])
        assert I.rel_err(got[s], orc.attend(q[s], K[rows], V[rows], 8, 1)) <= TOL


def test_ragged_empty_range_is_an_error(ctx):
    lens = np.array([100, 0, 50], np.int64)
    d = 256
    q, K, V, row0 = _ragged_case(5, np.maximum(lens, 1), d)
    out = torch.zeros(3 * 8 * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(np.zeros(3, np.int64)), dev(lens), 100, 8, 1, d,
                            out)
    with pytest.raises(g4hip.EngError, match="softmax input is not finite"):
        ctx.check_status()
