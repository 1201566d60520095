"""Seeded random shapes against the oracle, beyond the hand-picked cases:
chunked prefill at random (pos0, N, window) for both head widths, and
ragged decode batches of random sizes, lengths and windows (through the
streamed path and the per-sequence split grid, whichever the launcher
picks).  Every query row and every sequence is checked, to the tolerance
of the other parity tests: 1e-4 relative
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


def _prefill_shapes():
    rng = np.random.default_rng(20261202)
    shapes = []
    for i in range(12):
        d = (256, 512)[i % 2]
        window = int(rng.choice([0, 512, 1, 7, 100, 4096])) if d == 256 else int(rng.choice([0, 0, 33]))
        shapes.append((d, window, int(rng.integers(0, 3000)), int(rng.integers(1, 400))))
    return shapes


@pytest.mark.parametrize("d,window,pos0,N", _prefill_shapes())
def test_prefill_random_shapes(ctx, d, window, pos0, N):
    print(f"[case] prefill sweep d={d} W={window} pos0={pos0} N={N}", flush=True)
    freqs = I.rope_freqs(pos0 + 1, d) if d == 512 else None
    base = I.GLOBAL_BASE if d == 512 else I.LOCAL_BASE
    K, V = I.kv_rows(3 * pos0 + N, pos0 + N, d, base, freqs)
    q = I.queries(5 * pos0 + N, N, d, base, freqs, pos0)
    out = torch.zeros(N * 8 * d, device="cuda")
    ctx.attend_prefill(dev(q), dev(K), dev(V), pos0, N, window, 8, 1, d, out)
    ctx.check_status()
    got = out.cpu().numpy().reshape(N, 8 * d)
    ref, status = orc.attend_prefill(q, K, V, pos0, window, 8, 1)
    assert not status.any()
    worst = max(I.rel_err(got[i], ref[i]) for i in range(N))
    print(f"[parity] prefill sweep d={d} W={window} pos0={pos0} N={N}: worst rel err {worst:.2e}")
    assert worst <= TOL


def _ragged_shapes():
    rng = np.random.default_rng(4242)
    shapes = []
    for i in range(10):
        d = (256, 512)[i % 2]
        B = int(rng.choice([1, 2, 5, 17, 40, 100]))
        hi = int(rng.choice([40, 600, 5000, 20000]))
        hi = max(1, min(hi, 120000 // B))  # keeps the host arrays and the oracle small
        window = int(rng.choice([0, 512])) if d == 256 else 0
        shapes.append((d, window, rng.integers(1, hi + 1, size=B).astype(np.int64).tolist()))
    return shapes


@pytest.mark.parametrize("d,window,lens", _ragged_shapes())
def test_ragged_decode_random_batches(ctx, d, window, lens):
    lens = np.array(lens, np.int64)
    B = lens.size
    print(f"[case] ragged sweep d={d} W={window} B={B} max={lens.max()} total={lens.sum()}", flush=True)
    rng = np.random.default_rng(int(lens.sum()) + d)
    gap = 2  # NaN rows between the sequences' caches: reading one poisons the result
    row0 = np.zeros(B, np.int64)
    at = 0
    for s in range(B):
        row0[s] = at
        at += int(lens[s]) + gap
    K = np.full((at, d), np.nan, np.float32)
    V = np.full((at, d), np.nan, np.float32)
    for s in range(B):
        K[row0[s]:row0[s] + lens[s]] = rng.standard_normal((int(lens[s]), d), dtype=np.float32)
        V[row0[s]:row0[s] + lens[s]] = rng.standard_normal((int(lens[s]), d), dtype=np.float32)
    q = rng.standard_normal((B, 8 * d), dtype=np.float32) * 0.1
    begin = np.array([I.attended_range(int(L) - 1, window)[0] for L in lens], np.int64)
    out = torch.zeros(B * 8 * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(begin), dev(lens), int((lens - begin).max()),
                            8, 1, d, out)
    ctx.check_status()
    got = out.cpu().numpy().reshape(B, -1)
    worst = 0.0
    for s in range(B):
        rows = slice(row0[s] + begin[s], row0[s] + lens[s])
        worst = max(worst, I.rel_err(got[s], orc.attend(q[s], K[rows], V[rows], 8, 1)))
    print(f"[parity] ragged sweep d={d} W={window} B={B}: worst rel err {worst:.2e}")
    assert worst <= TOL
