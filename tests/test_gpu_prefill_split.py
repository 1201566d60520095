"""Prefill with split-f16 products against the oracle, and the per-unit choice
between the split form and f32 MFMAs.

The split form carries each f32 operand as an f16 hi + lo pair (three f16
MFMA products per f32 product, f32 accumulation).  It must meet the same
bar as the f32 form: every query row within 1e-4 relative of the oracle's
token-at-a-time loop (crates/llm-gemma4/src/impl_/generate.rs:37-41, the
tolerance of crates/llm-gemma4/tests/synthetic_generate.rs:74-83).  A work
unit whose q rows or K/V tiles hold a value the split does not carry
(|x| >= 2^15, NaN, inf) runs with f32 MFMAs; those rows then equal the
f32-only mode bit for bit, since both modes share the unit schedule.
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


def run(ctx, q, K, V, pos0, N, window, d, exact, scale=1.0):
    ctx.set_prefill_exact(exact)
    try:
        out = torch.zeros(N * 8 * d, device="cuda")
        ctx.attend_prefill(dev(q), dev(K), dev(V), pos0, N, window, 8, 1, d, out, scale=scale)
        ctx.check_status()
        return out.cpu().numpy().reshape(N, 8 * d)
    finally:
        ctx.set_prefill_exact(0)


def case(seed, rows, d):
    glob = d == 512
    freqs = I.rope_freqs(seed + 1, d) if glob else None
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    K, V = I.kv_rows(seed, rows, d, base, freqs)
    q = I.queries(seed + 2, rows, d, base, freqs, 0)
    return q, K, V


def worst_vs_oracle(got, q, K, V, pos0, window, unit=1.0, scale=1.0):
    """Worst rel_err over all rows, both sides divided by `unit` (the
    magnitude of V, so that the measure's floor of 1 does not hide errors
    of small outputs)."""
    ref, status = orc.attend_prefill(q, K, V, pos0, window, 8, 1, scale=scale)
    assert not status.any()
    assert np.all(np.isfinite(got))
    return max(I.rel_err(got[i] / unit, ref[i] / unit) for i in range(ref.shape[0]))


@pytest.mark.parametrize("scale", [0.0625, 2.5])
@pytest.mark.parametrize("d,window,pos0,N", [(256, 512, 600, 128), (512, 0, 300, 96), (256, 8, 5, 40)])
def test_softmax_scale(ctx, d, window, pos0, N, scale):
    """A score scale other than Gemma's 1 (attend's `scale`, model.rs:326-343):
    both forms against the oracle's token loop with the same scale, within
    1e-4 or -- where larger scores put the reference's own f32 rounding
    near that -- no further from exact (f64) attention than twice the
    oracle's own distance from it (the bar of the large-score tests)."""
    from test_gpu_prefill_deep import f64_prefill

    print(f"[case] d={d} W={window} pos0={pos0} N={N} scale={scale}", flush=True)
    q, K, V = case(7700 + d + pos0 + N, pos0 + N, d)
    ref, status = orc.attend_prefill(q[pos0:], K, V, pos0, window, 8, 1, scale=scale)
    assert not status.any()
    exact64 = f64_prefill(q[pos0:].astype(np.float64) * scale, K, V, pos0, window)
    floor = max(I.rel_err(ref[i], exact64[i]) for i in range(N))
    for form, ex in (("split-f16", 0), ("f32", 1)):
        got = run(ctx, q[pos0:], K, V, pos0, N, window, d, ex, scale)
        assert np.all(np.isfinite(got))
        w_ref = max(I.rel_err(got[i], ref[i]) for i in range(N))
        w_64 = max(I.rel_err(got[i], exact64[i]) for i in range(N))
        print(f"[parity] scale {scale} {form}: vs oracle {w_ref:.2e}, vs f64 {w_64:.2e}; oracle vs f64 {floor:.2e}",
              flush=True)
        assert w_ref <= TOL or w_64 <= 2.0 * floor, form
    split = run(ctx, q[pos0:], K, V, pos0, N, window, d, 0, scale)
    # The scale reached the kernels: the unscaled outputs differ.
    assert not np.allclose(split, run(ctx, q[pos0:], K, V, pos0, N, window, d, 0), rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("d,window,pos0,N", [(256, 512, 0, 2048), (512, 0, 0, 2048), (256, 512, 3000, 256),
                                             (512, 0, 5000, 200), (256, 64, 37, 91), (512, 5, 0, 33)])
def test_split_and_f32_forms_both_match_the_oracle(ctx, d, window, pos0, N):
    print(f"[case] d={d} W={window} pos0={pos0} N={N}", flush=True)
    q, K, V = case(7000 + d + pos0 + N, pos0 + N, d)
    split = run(ctx, q[pos0:], K, V, pos0, N, window, d, 0)
    exact = run(ctx, q[pos0:], K, V, pos0, N, window, d, 1)
    ws = worst_vs_oracle(split, q[pos0:], K, V, pos0, window)
    we = worst_vs_oracle(exact, q[pos0:], K, V, pos0, window)
    print(f"[parity] split-f16 worst {ws:.2e}, f32 worst {we:.2e}", flush=True)
    assert ws <= TOL and we <= TOL
    # The split form ran: its rounding differs from the f32 form's somewhere.
    assert not np.array_equal(split, exact)


@pytest.mark.parametrize("d,window", [(256, 512), (512, 0)])
def test_out_of_range_q_row_sends_its_block_to_f32(ctx, d, window):
    """One q value of 40000 (above the split's 2^15): the units of that
    position block run in f32, bit-equal to the f32-only mode; every row
    still matches the oracle."""
    pos0, N = 0, 512
    q, K, V = case(8100 + d, N, d)
    row = 203  # position block 25 (8 positions per block)
    q[row, 3 * d + 17] = 40000.0
    split = run(ctx, q, K, V, pos0, N, window, d, 0)
    exact = run(ctx, q, K, V, pos0, N, window, d, 1)
    blk = slice(8 * (row // 8), 8 * (row // 8) + 8)
    assert np.array_equal(split[blk], exact[blk])
    assert not np.array_equal(split[:blk.start], exact[:blk.start])
    w = worst_vs_oracle(split, q, K, V, pos0, window)
    print(f"[parity] worst {w:.2e}", flush=True)
    assert w <= TOL


@pytest.mark.parametrize("d,window,value", [(256, 512, 32768.0), (512, 0, -50000.0), (512, 0, 32767.0)])
def test_out_of_range_kv_values(ctx, d, window, value):
    """A K or V value at or beyond 2^15 sends the units that read its tile to
    f32; one just below it stays in the split form.  Rows match the oracle
    either way."""
    pos0, N = 0, 640
    q, K, V = case(8200 + d, N, d)
    K[300, 11] = value
    V[301, d - 5] = value
    split = run(ctx, q, K, V, pos0, N, window, d, 0)
    w = worst_vs_oracle(split, q, K, V, pos0, window)
    print(f"[parity] value {value}: worst {w:.2e}", flush=True)
    assert w <= TOL
    exact = run(ctx, q, K, V, pos0, N, window, d, 1)
    # Blocks that attend no key of tiles 18 (rows 288..303) end before row
    # 288: they never read the odd tile and keep the split form.
    assert not np.array_equal(split[:288], exact[:288])


def test_blocks_mixing_split_and_f32_units_merge_alike(ctx):
    """2048-token global prompt with one K value of 40000 in tile 62 (rows
    992..1007): the units that read that tile run in f32, the other units of
    the same position blocks in the split form, and the merge combines both
    kinds of partial (the split form's weights carry 2^7, which its partials
    fold into m).  Every row against the oracle."""
    import g4hip
    d, window, N, tile = 512, 0, 2048, 62
    units, _ = g4hip.prefill_schedule(0, N, window, d, 1, 256)
    by_block = {}
    for b, lo, hi, _slot in units:
        by_block.setdefault(int(b), []).append((int(lo), int(hi)))
    mixed = [b for b, us in by_block.items()
             if len(us) > 1 and any(lo <= tile < hi for lo, hi in us) and any(not lo <= tile < hi for lo, hi in us)]
    assert mixed, "the schedule no longer splits long blocks"
    q, K, V = case(8500, N, d)
    K[16 * tile + 5, 100] = 40000.0
    split = run(ctx, q, K, V, 0, N, window, d, 0)
    w = worst_vs_oracle(split, q, K, V, 0, window)
    print(f"[parity] {len(mixed)} mixed blocks; worst {w:.2e}", flush=True)
    assert w <= TOL


@pytest.mark.parametrize("d,window", [(256, 512), (512, 0)])
def test_small_q_and_k(ctx, d, window):
    """q and K scaled by 2^-10: about one element in twenty has a subnormal
    f16 hi half, and every lo half would be subnormal without its 2^11
    scale.  Scores are then ~2^-20 of their usual size, yet the outputs
    (normal V) must still match the oracle at 1e-4."""
    pos0, N = 0, 300
    q, K, V = case(8300 + d, N, d)
    s = np.float32(2.0 ** -10)
    split = run(ctx, q * s, K * s, V, pos0, N, window, d, 0)
    w = worst_vs_oracle(split, q * s, K * s, V, pos0, window)
    print(f"[parity] worst {w:.2e}", flush=True)
    assert w <= TOL


@pytest.mark.parametrize("d,window", [(256, 512), (512, 0)])
def test_small_values_everywhere(ctx, d, window):
    """q, K and V scaled by 2^-12, by the reference's measure (max |diff| /
    max(|a|, |b|, 1)).  V's lo half is not scaled: its error, at most 2^-25
    per element, reaches an output weighted by p/l <= 1, so far below the
    tolerance; in units of V's own scale it stays under 2^-12."""
    pos0, N = 0, 300
    q, K, V = case(8400 + d, N, d)
    s = np.float32(2.0 ** -12)
    q, K, V = q * s, K * s, V * s
    split = run(ctx, q, K, V, pos0, N, window, d, 0)
    w = worst_vs_oracle(split, q, K, V, pos0, window)
    wu = worst_vs_oracle(split, q, K, V, pos0, window, unit=float(s))
    print(f"[parity] worst {w:.2e}; {wu:.2e} in units of 2^-12", flush=True)
    assert w <= TOL and wu <= 2.0 ** -12


def test_exact_flag_rejects_other_values(ctx):
    import g4hip
    with pytest.raises(g4hip.EngError):
        ctx.set_prefill_exact(2)
