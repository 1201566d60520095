"""Sliding-window rings in the device ContextMemory (g4_kv_create_ring).

The reference's sliding owners keep their whole history
(crates/llm-eng/src/context_memory.rs:11-86); a ring keeps only the last R
positions.  Attention must not see the difference: the layer drivers run on
a ring cache and on a whole-history cache with the same inputs must give the
same bits, and a ring's rows must be the last R appended rows."""
import numpy as np
import pytest
import torch

import g4hip

pytestmark = pytest.mark.gpu


class Raw:
    """A raw device address, for the binding's pointer arguments."""

    def __init__(self, addr):
        self.addr = addr

    def data_ptr(self):
        return self.addr


def read_rows(ctx, addr, n_floats):
    """The n floats at a device address (copied out with x + 0)."""
    out = torch.empty(n_floats, device="cuda")
    ctx.port_add(Raw(addr), torch.zeros(n_floats, device="cuda"), n_floats, out)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def test_ring_holds_the_last_positions(ctx):
    w, R, cap = 256, 24, 400
    cache = g4hip.KvCache(ctx, [w], cap, ring_rows=[R])
    rng = np.random.default_rng(5)
    K = np.zeros((0, w), np.float32)
    V = np.zeros((0, w), np.float32)
    try:
        for n in [5, 7, 30, 1, 13, 24, 2, 50, 3, 25]:
            k = rng.standard_normal((n, w)).astype(np.float32)
            v = rng.standard_normal((n, w)).astype(np.float32)
            cache.append_rows(0, dev(k), dev(v), n)
            K, V = np.concatenate([K, k]), np.concatenate([V, v])
            total = len(K)
            assert cache.len(0) == total
            lo = max(0, total - R)
            for b in (lo, (lo + total) // 2, total - 1):
                kp, vp, stride = cache.view_rows(0, b, total)
                assert stride == w
                assert np.array_equal(read_rows(ctx, kp, (total - b) * w), K[b:total].ravel())
                assert np.array_equal(read_rows(ctx, vp, (total - b) * w), V[b:total].ravel())
            if lo > 0:
                with pytest.raises(g4hip.EngError, match="left layer 0's ring of 24 rows"):
                    cache.view_rows(0, lo - 1, total)
                with pytest.raises(g4hip.EngError, match="keeps only its last 24 rows"):
                    cache.view(0, total)
            else:  # not wrapped yet: the whole-history view still holds
                kp, _, _ = cache.view(0, total)
                assert np.array_equal(read_rows(ctx, kp, total * w), K.ravel())
            with pytest.raises(g4hip.EngError) as e:
                cache.view_rows(0, lo, total + 1)
            assert e.value.kind == "ContextTooLong"
        # positions still count up to the capacity
        big = cap - len(K) + 1
        with pytest.raises(g4hip.EngError) as e:
            cache.append_rows(0, dev(np.zeros((big, w))), dev(np.zeros((big, w))), big)
        assert e.value.kind == "ContextTooLong" and e.value.fields == (cap + 1, cap)
    finally:
        cache.close()


def hparams():
    # 7 layers: 0-3 sliding, 4 global, then 5 (sliding) and 6 (global) share
    # the K/V of layers 3 and 4.
    return g4hip.G4Hparams(7, 8, 1, 256, 512, 16, 2, 10000.0, 1000000.0, 1e-6)


def test_ring_cache_attends_like_the_whole_history(ctx):
    hp = hparams()
    R = 24  # window 16 + chunks of up to 8 tokens - 1 = 23
    widths = [256, 256, 256, 256, 512]
    full = g4hip.KvCache(ctx, widths, 256)
    ring = g4hip.KvCache(ctx, widths, 256, ring_rows=[R, R, R, R, 0])
    rng = np.random.default_rng(11)
    dims = [512 if g4hip.layer_attention_kind(7, l) == "global" else 256 for l in range(7)]
    norms = {d: (dev(rng.uniform(0.5, 1.5, d)), dev(rng.uniform(0.5, 1.5, d))) for d in (256, 512)}
    freqs = dev(rng.uniform(1.0, 8.0, 256))
    steps = [("prefill", 0, 8)] + [("decode", p, 1) for p in range(8, 64)] + [("prefill", 64, 8)] + \
            [("decode", p, 1) for p in range(72, 100)] + [("prefill", 100, 5)]
    try:
        for kind, pos, n in steps:
            for layer in range(7):
                d = dims[layer]
                qkv = [rng.standard_normal(n * m * d).astype(np.float32) for m in (8, 1, 1)]
                outs = []
                for cache in (full, ring):
                    q, k, v = (dev(x) for x in qkv)
                    out = torch.zeros(n * 8 * d, device="cuda")
                    qw, kw = norms[d]
                    if kind == "prefill":
                        src = cache.layer_prefill(hp, layer, pos, n, q, k, v, qw, kw, freqs, out)
                        rng_ = None
                    else:
                        src, rng_ = cache.layer_attention(hp, layer, pos, q, k, v, qw, kw, freqs, out)
                    ctx.check_status()
                    outs.append((src, rng_, out))
                (s0, r0, o0), (s1, r1, o1) = outs
                assert (s0, r0) == (s1, r1)
                assert torch.equal(o0, o1), f"{kind} at {pos}, layer {layer}"
        # a chunk longer than a ring, and one whose window reaches evicted rows
        d = 256
        q, k, v = dev(np.ones(30 * 8 * d)), dev(np.ones(30 * d)), dev(np.ones(30 * d))
        out = torch.zeros(30 * 8 * d, device="cuda")
        with pytest.raises(g4hip.EngError, match="do not fit layer 0's ring of 24 rows"):
            ring.layer_prefill(hp, 0, 105, 30, q, k, v, *norms[d], freqs, out)
        with pytest.raises(g4hip.EngError, match="have left layer 0's ring"):
            ring.layer_prefill(hp, 0, 105, 12, q, k, v, *norms[d], freqs, out)
    finally:
        full.close()
        ring.close()
