"""The prefill kernel's work schedule (g4_prefill_schedule, host only).

Query p attends keys [max(0, p+1-W), p] (W = 0: [0, p]) -- the sets
LocalWindowPolicy / GlobalPolicy give (crates/llm-gemma4/src/eng/mod.rs:10-36).
The kernel computes position blocks of 8 queries against 16-key tiles, so
block b needs exactly the tiles that hold a key some query of the block
attends; the schedule must cover each of them exactly once, in at most 8
pieces (the merge kernel's limit), and spread the tiles evenly over the
workgroups.  No GPU is touched here."""
import numpy as np
import pytest

import g4hip

SHAPES = [  # pos0, N, window, head_dim, n_kv_heads
    (0, 2048, 0, 512, 1), (0, 2048, 512, 256, 1), (0, 4096, 0, 512, 1), (0, 1024, 0, 512, 1),
    (16384, 256, 0, 512, 1), (8192, 2048, 512, 256, 1), (0, 1, 0, 512, 1), (0, 7, 512, 256, 1),
    (0, 300, 0, 512, 1), (150, 90, 100, 512, 2), (5000, 333, 512, 256, 2), (0, 2048, 0, 512, 2),
    (100000, 64, 0, 512, 1), (0, 16384, 0, 512, 1),
]


def needed_tiles(pos0, N, window):
    """Per block, the set of 16-key tiles holding a key one of its queries attends."""
    out = []
    for b in range((N + 7) // 8):
        tiles = set()
        for p in range(pos0 + 8 * b, min(pos0 + 8 * b + 8, pos0 + N)):
            lo = max(0, p + 1 - window) if window else 0
            tiles.update(range(lo // 16, p // 16 + 1))
        out.append(tiles)
    return out


@pytest.mark.parametrize("pos0,N,window,d,n_kv", SHAPES)
def test_schedule_covers_every_attended_tile_once(pos0, N, window, d, n_kv):
    units, bins = g4hip.prefill_schedule(pos0, N, window, d, n_kv, 256)
    need = needed_tiles(pos0, N, window)
    got = [[] for _ in need]
    for b, lo, hi, slot in units:
        assert 0 <= b < len(need) and lo < hi
        got[b].extend(range(lo, hi))
    for b, tiles in enumerate(need):
        assert sorted(got[b]) == sorted(tiles), b  # each needed tile once, nothing else

    # workgroups: contiguous, non-empty ranges over the unit table, at most
    # one per CU per KV head
    assert bins[0] == 0 and bins[-1] == len(units)
    assert np.all(np.diff(bins) >= 1)
    assert len(bins) - 1 <= 256 // n_kv

    # a block computed by one unit has no partial slot; a split block's
    # units have distinct slots, and no block has more than 8 units
    slots = {}
    for b, lo, hi, slot in units:
        slots.setdefault(int(b), []).append(int(slot))
    all_slots = []
    for b, s in slots.items():
        assert len(s) <= 8
        if len(s) == 1:
            assert s == [-1]
        else:
            assert min(s) >= 0 and len(set(s)) == len(s)
            assert sorted(s) == list(range(min(s), min(s) + len(s)))  # merge reads them as a run
            all_slots += s
    assert sorted(all_slots) == list(range(len(all_slots)))


def bin_tiles(units, bins):
    return np.array([int((units[bins[w]:bins[w + 1], 2] - units[bins[w]:bins[w + 1], 1]).sum())
                     for w in range(len(bins) - 1)])


@pytest.mark.parametrize("N", [1024, 2048, 4096, 16384])
def test_causal_prompts_are_balanced(N):
    """A causal prompt's blocks range from 1 to N/16 tiles; the busiest
    workgroup gets at most 10% more tiles than the average plus a few."""
    units, bins = g4hip.prefill_schedule(0, N, 0, 512, 1, 256)
    t = bin_tiles(units, bins)
    ideal = t.sum() / 256
    assert len(t) <= 256
    assert t.max() <= 1.10 * ideal + 4, (t.max(), ideal)


def test_sliding_prompt_is_not_split():
    """With a 512-key window every block needs at most 33 tiles: one unit
    each, no partials (a merge would cost more than the balance gains)."""
    units, bins = g4hip.prefill_schedule(0, 2048, 512, 256, 1, 256)
    assert len(units) == 256 and np.all(units[:, 3] == -1)


def test_schedule_rejects_bad_shapes():
    for args in [(0, 0, 0, 512), (0, 16, 0, 128), (-1, 16, 0, 512), (0, 16, -1, 256)]:
        with pytest.raises(g4hip.EngError):
            g4hip.prefill_schedule(*args)
    with pytest.raises(g4hip.EngError):
        g4hip.prefill_schedule(0, 16, 0, 512, 0, 256)
