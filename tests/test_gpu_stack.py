"""The layer attention segment (model.rs:386-411) on the device, through the
35-layer E2B stack with its shared K/V, against the oracle's restatement.

Each call normalises and rotates q (and k, v on owner layers), appends to
the device KvCache, views the source layer, applies the window and attends.
The attended set -- source layer and row range -- must match exactly.
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
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def widths(hp):
    """Row width of each layer's own cache (0 for layers that share one)."""
    out = []
    for l in range(hp.n_layers):
        src = orc.kv_source_layer(hp.n_layers, hp.shared_kv_layers, l)
        glob = orc.layer_attention_kind(hp.n_layers, l) == "global"
        out.append(hp.n_kv_heads * (hp.head_dim_global if glob else hp.head_dim_local) if src == l else 0)
    return out


def run_stack(ctx, hp_g, hp_o, history, positions, seed):
    """Fills owner caches with `history` prepared rows, then steps the stack
    through `positions`; returns the worst relative error."""
    rng = np.random.default_rng(seed)
    ws = widths(hp_o)
    cap = history + len(positions)
    cache = g4hip.KvCache(ctx, ws, cap)
    ocache = orc.KvCache()
    freqs = I.rope_freqs(seed + 3, hp_o.head_dim_global)
    dfreqs = dev(freqs)
    worst = 0.0
    try:
        for l, w in enumerate(ws):
            if not w:
                continue
            glob = orc.layer_attention_kind(hp_o.n_layers, l) == "global"
            d = hp_o.head_dim_global if glob else hp_o.head_dim_local
            K, V = I.kv_rows(seed + 100 + l, history, d, I.GLOBAL_BASE if glob else I.LOCAL_BASE,
                             freqs if glob else None)
            if history:
                cache.append_rows(l, dev(K), dev(V), history)
            for t in range(history):
                ocache.append(l, K[t], V[t])
        for pos in positions:
            for l in range(hp_o.n_layers):
                glob = orc.layer_attention_kind(hp_o.n_layers, l) == "global"
                d = hp_o.head_dim_global if glob else hp_o.head_dim_local
                q = rng.standard_normal(hp_o.n_heads * d).astype(np.float32)
                k = rng.standard_normal(hp_o.n_kv_heads * d).astype(np.float32)
                v = rng.standard_normal(hp_o.n_kv_heads * d).astype(np.float32)
                wq = rng.uniform(0.5, 1.5, d).astype(np.float32)
                wk = rng.uniform(0.5, 1.5, d).astype(np.float32)
                ref, src, rng_kv, _, _, _ = ocache.layer_attention(hp_o, l, pos, q, k, v, wq, wk,
                                                                   freqs if glob else None)
                out = torch.zeros(hp_o.n_heads * d, device="cuda")
                gsrc, grange = cache.layer_attention(hp_g, l, pos, dev(q), dev(k), dev(v), dev(wq), dev(wk),
                                                     dfreqs if glob else None, out)
                ctx.check_status()
                assert (gsrc, grange) == (src, rng_kv), (l, pos)
                worst = max(worst, I.rel_err(out.cpu().numpy(), ref))
    finally:
        cache.close()
    return worst


def test_synthetic_model_shape_generation(ctx):
    """The reference's synthetic model shape (synthetic_generate.rs:12-34):
    7 layers, 4 Q / 2 KV heads, widths 8/16, window 8, 2 shared layers."""
    hp_o = orc.Hparams(7, 4, 2, 8, 16, 8, 2, 10000.0, 1000000.0, 1e-6)
    hp_g = g4hip.G4Hparams(7, 4, 2, 8, 16, 8, 2, 10000.0, 1000000.0, 1e-6)
    worst = run_stack(ctx, hp_g, hp_o, 0, list(range(20)), 31)
    assert worst <= TOL


def test_e2b_stack_decode_at_8192(ctx):
    """The E2B stack: 35 layers, owners hold 8191 rows, one decode step at
    position 8191 through every layer (shared layers read 13 / 14)."""
    print("[case] E2B stack ctx 8192", flush=True)
    worst = run_stack(ctx, g4hip.G4Hparams.e2b(), orc.Hparams.e2b(), 8191, [8191], 77)
    print(f"[parity] E2B stack: worst rel err {worst:.2e}")
    assert worst <= TOL


def test_e2b_stack_short_generation(ctx):
    """Positions 0..39 through the E2B stack from an empty cache."""
    worst = run_stack(ctx, g4hip.G4Hparams.e2b(), orc.Hparams.e2b(), 0, list(range(40)), 5)
    assert worst <= TOL


def test_kv_cache_view_errors(ctx):
    cache = g4hip.KvCache(ctx, [4, 4, 0], 8)
    try:
        with pytest.raises(g4hip.EngError) as e:
            cache.view(0, 1)
        assert e.value.kind == "MissingLayer" and e.value.message == "layer 0 has no cached K/V"
        assert e.value.fields[0] == 0
        cache.view(2, 0)
        row = dev(np.ones(4))
        for _ in range(3):
            cache.append(1, row, row)
        with pytest.raises(g4hip.EngError) as e:
            cache.view(0, 1)  # layer 0 exists (appending to 1 created it) but is empty
        assert e.value.kind == "ContextTooLong" and e.value.fields == (1, 0)
        cache.view(1, 3)
        with pytest.raises(g4hip.EngError) as e:
            cache.view(1, 4)
        assert e.value.message == "context length 4 exceeds configured max 3"
        cache.clear()
        with pytest.raises(g4hip.EngError) as e:
            cache.view(1, 1)
        assert e.value.kind == "MissingLayer"
    finally:
        cache.close()


def _copy_out(ptr, n):
    """n floats at device address ptr, copied with hipMemcpy (test plumbing)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.zeros(n, np.float32)
    assert hip.hipMemcpy(out.ctypes.data, ptr, 4 * n, 2) == 0  # hipMemcpyDeviceToHost
    return out


def test_kv_cache_scalar_fixture(ctx):
    """kv_vs_recompute.rs:13-35 on the device cache: append a row, view the prefix."""
    import json
    import os
    k = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))[
        "kv_cache_scalar_fixture"]
    cache = g4hip.KvCache(ctx, [1], 4)
    try:
        outs = []
        for t in range(3):
            cache.append(0, dev([k["ks"][t]]), dev([k["vs"][t]]))
            torch.cuda.synchronize()
            kp, vp, stride = cache.view(0, t + 1)
            assert stride == 1
            ks, vs = _copy_out(kp, t + 1), _copy_out(vp, t + 1)
            acc = 0.0
            for i in range(t + 1):
                acc += (k["qs"][t] * float(ks[i])) * float(vs[i])
            outs.append(acc)
        assert np.allclose(outs, k["toy_outputs"], atol=k["abs_tol"])
        assert cache.len(0) == 3
    finally:
        cache.close()
