"""The fused layer decode step (g4_decode_step_fused, what g4_layer_attention
runs for head_dim 256/512 and 8 query heads per KV head): the decode kernel
prepares q -- and on an owner layer the new row's k and v, which it appends
-- itself (model.rs:394-410).

Against the two-launch form (g4_prepare_qkv, then g4_attend_decode over the
appended cache): the appended row must be the same bits, q/k/v must be left
as given, and the output must match the oracle's attend over the prepared
rows within the reference's tolerance (synthetic_generate.rs:74-83).  The
cache row the kernel appends is not read by it: it holds NaN beforehand."""
import numpy as np
import pytest
import torch

import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4
EPS = 1e-6


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


CASES = [  # d, attended rows, position of the last row, owner layer, KV heads
    (512, 4096, 4095, True, 1), (512, 1, 0, True, 1), (512, 40, 39, True, 1), (512, 64, 63, True, 1),
    (512, 65, 64, True, 1), (512, 9000, 8999, True, 1), (256, 512, 1200, True, 1), (256, 17, 16, True, 1),
    (256, 512, 700, False, 1), (512, 3000, 2999, False, 1), (512, 300, 299, True, 2), (256, 100, 99, False, 2),
    (512, 8300, 8299, False, 1),  # 48-key splits: a context just past 256 x 32
]


@pytest.mark.parametrize("d,n,pos,owner,n_kv", CASES)
def test_fused_step_matches_prepare_then_decode(ctx, d, n, pos, owner, n_kv):
    print(f"[case] fused step d={d} rows={n} position={pos} owner={owner} kv={n_kv}", flush=True)
    rng = np.random.default_rng(d + n + pos + n_kv)
    n_heads = 8 * n_kv
    glob = d == 512
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    freqs = I.rope_freqs(d + 1, d) if glob else None
    stride = n_kv * d
    q = (rng.standard_normal(n_heads * d) * 2).astype(np.float32)
    k = (rng.standard_normal(n_kv * d) * 2).astype(np.float32)
    v = (rng.standard_normal(n_kv * d) * 2).astype(np.float32)
    wq = rng.uniform(0.5, 1.5, d).astype(np.float32)
    wk = rng.uniform(0.5, 1.5, d).astype(np.float32)
    rows = rng.standard_normal((n, stride)).astype(np.float32)
    vrows = rng.standard_normal((n, stride)).astype(np.float32)

    # the two-launch form: prepare (appending row n-1 on an owner layer), then decode
    K1, V1 = dev(rows), dev(vrows)
    q1, k1, v1 = dev(q), dev(k), dev(v)
    ctx.prepare_qkv(q1, k1 if owner else None, v1 if owner else None, 1, pos, n_heads, n_kv, d, dev(wq), dev(wk),
                    EPS, base, dev(freqs) if glob else None,
                    k_rows=K1.view(-1)[(n - 1) * stride:] if owner else None,
                    v_rows=V1.view(-1)[(n - 1) * stride:] if owner else None, row_stride=stride)
    ref_out = torch.zeros(n_heads * d, device="cuda")
    ctx.attend_decode(q1, K1, V1, 0, n, n_heads, n_kv, d, ref_out)

    # the fused step over a cache whose new row is NaN until the kernel writes it
    rows2, vrows2 = rows.copy(), vrows.copy()
    if owner:
        rows2[n - 1] = np.nan
        vrows2[n - 1] = np.nan
    K2, V2 = dev(rows2), dev(vrows2)
    q2, k2, v2 = dev(q), dev(k), dev(v)
    out = torch.zeros(n_heads * d, device="cuda")
    ctx.decode_step_fused(q2, k2 if owner else None, v2, dev(wq), dev(wk), EPS, base, dev(freqs) if glob else None,
                          pos, K2, V2, stride, n, K2.view(-1)[(n - 1) * stride:] if owner else None,
                          V2.view(-1)[(n - 1) * stride:] if owner else None, n_heads, n_kv, d, out)
    ctx.check_status()

    # q/k/v untouched; the appended row is the prepared row, bit for bit
    assert np.array_equal(host(q2), q) and np.array_equal(host(k2), k) and np.array_equal(host(v2), v)
    if owner:
        assert np.array_equal(host(K2)[n - 1], host(K1)[n - 1])
        assert np.array_equal(host(V2)[n - 1], host(V1)[n - 1])
    got = host(out)
    assert I.rel_err(got, host(ref_out)) <= TOL
    ref = orc.attend(host(q1), host(K1), host(V1), n_heads, n_kv)
    assert I.rel_err(got, ref) <= TOL


def test_fused_step_rejects_other_shapes(ctx):
    import g4hip
    d, n = 128, 10
    z = torch.zeros(8 * d, device="cuda")
    K = torch.zeros(n * d, device="cuda")
    with pytest.raises(g4hip.EngError, match="8 query heads per KV head"):
        ctx.decode_step_fused(z, None, None, None, None, EPS, 10000.0, None, n - 1, K, K, d, n, None, None, 8, 1, d,
                              torch.zeros(8 * d, device="cuda"))
    with pytest.raises(g4hip.EngError, match="n_rows"):
        ctx.decode_step_fused(z, None, None, None, None, EPS, 10000.0, None, 3, K, K, d, n, None, None, 8, 1, 256,
                              torch.zeros(8 * 256, device="cuda"))


def _copy_out(ptr, n):
    """n floats at device address ptr (hipMemcpy, test plumbing)."""
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    out = np.zeros(n, np.float32)
    assert hip.hipMemcpy(out.ctypes.data, ptr, 4 * n, 2) == 0  # hipMemcpyDeviceToHost
    return out


@pytest.mark.parametrize("layer,ring", [(0, False), (4, False), (0, True)])
def test_layer_attention_past_the_cache_fails_like_the_reference(ctx, layer, ring):
    """model.rs:394-407 appends the new row, then views position + 1 rows: a
    position past the cached rows fails at the view with ContextTooLong and
    leaves the appended row in the cache.  The device cache must end in the
    same state as the oracle's: same error fields, same length, same row."""
    import g4hip
    print(f"[case] layer_attention past the cache, layer {layer}", flush=True)
    hp_g = g4hip.G4Hparams(7, 8, 1, 256, 512, 16, 2, 10000.0, 1000000.0, 1e-6)
    hp_o = orc.Hparams(7, 8, 1, 256, 512, 16, 2, 10000.0, 1000000.0, 1e-6)
    d = 512 if layer == 4 else 256
    rng = np.random.default_rng(40 + layer)
    freqs = I.rope_freqs(7, 512)
    cache = g4hip.KvCache(ctx, [256, 256, 256, 256, 512], 64, ring_rows=[24, 24, 24, 24, 0] if ring else None)
    ocache = orc.KvCache()
    try:
        hist = 3
        K = rng.standard_normal((hist, d)).astype(np.float32)
        V = rng.standard_normal((hist, d)).astype(np.float32)
        cache.append_rows(layer, dev(K), dev(V), hist)
        for t in range(hist):
            ocache.append(layer, K[t], V[t])
        q, k, v = (rng.standard_normal(m * d).astype(np.float32) for m in (8, 1, 1))
        wq, wk = (rng.uniform(0.5, 1.5, d).astype(np.float32) for _ in range(2))
        f = freqs if d == 512 else None
        pos = 10
        with pytest.raises(orc.OracleError) as oe:
            ocache.layer_attention(hp_o, layer, pos, q, k, v, wq, wk, f)
        out = torch.zeros(8 * d, device="cuda")
        with pytest.raises(g4hip.EngError) as ge:
            cache.layer_attention(hp_g, layer, pos, dev(q), dev(k), dev(v), dev(wq), dev(wk),
                                  dev(f) if f is not None else None, out)
        ctx.check_status()
        assert ge.value.kind == "ContextTooLong" and oe.value.code == 2
        assert ge.value.message == oe.value.message == "context length 11 exceeds configured max 4"
        assert ge.value.fields == (11, 4)
        assert cache.len(layer) == hist + 1
        ok, ov = ocache.view(layer, hist + 1)
        kp, vp, stride = cache.view(layer, hist + 1)
        gk = _copy_out(kp, (hist + 1) * d).reshape(hist + 1, d)
        gv = _copy_out(vp, (hist + 1) * d).reshape(hist + 1, d)
        assert np.array_equal(gk[:hist], ok[:hist]) and np.array_equal(gv, ov)  # V has no RoPE: bit-exact
        assert np.max(np.abs(gk[hist] - ok[hist])) < 2e-5  # device sin/cos vs host libm, same angles
        # the cache keeps working: the next position attends all five rows
        q, k, v = (rng.standard_normal(m * d).astype(np.float32) for m in (8, 1, 1))
        ref, src, rr, _, _, _ = ocache.layer_attention(hp_o, layer, hist + 1, q, k, v, wq, wk, f)
        gsrc, grange = cache.layer_attention(hp_g, layer, hist + 1, dev(q), dev(k), dev(v), dev(wq), dev(wk),
                                             dev(f) if f is not None else None, out)
        ctx.check_status()
        assert (gsrc, grange) == (src, rr) and cache.len(layer) == hist + 2
        assert I.rel_err(host(out), ref) <= TOL
    finally:
        cache.close()


def test_layer_attention_on_a_cache_longer_than_the_position(ctx):
    """A cache that already holds more rows than the position: the append
    pushes the new row after them (context_memory.rs:44-51) and the view
    takes the first position + 1 rows (model.rs:405-407), so the step attends
    cached rows only.  On a ring the new row and its mirror copy go to its
    own slot: a later window that reads the row through the mirror must see
    it.  Whole-history cache, ring cache and oracle agree."""
    import g4hip
    print("[case] layer_attention, cache longer than the position", flush=True)
    hp_g = g4hip.G4Hparams(7, 8, 1, 256, 512, 16, 2, 10000.0, 1000000.0, 1e-6)
    hp_o = orc.Hparams(7, 8, 1, 256, 512, 16, 2, 10000.0, 1000000.0, 1e-6)
    d, layer, hist, R = 256, 0, 30, 24
    rng = np.random.default_rng(77)
    widths = [256, 256, 256, 256, 512]
    full = g4hip.KvCache(ctx, widths, 64)
    ringc = g4hip.KvCache(ctx, widths, 64, ring_rows=[R, R, R, R, 0])
    ocache = orc.KvCache()
    try:
        K = rng.standard_normal((hist, d)).astype(np.float32)
        V = rng.standard_normal((hist, d)).astype(np.float32)
        for c in (full, ringc):
            c.append_rows(layer, dev(K), dev(V), hist)
        for t in range(hist):
            ocache.append(layer, K[t], V[t])
        wq, wk = (rng.uniform(0.5, 1.5, d).astype(np.float32) for _ in range(2))
        # position 27 appends row 30 and attends rows [12, 28); position 31
        # attends [16, 32), which holds row 30 -- on the ring, from its mirror.
        for pos in (27, 31, 32):
            q, k, v = (rng.standard_normal(m * d).astype(np.float32) for m in (8, 1, 1))
            ref, src, rr, _, _, _ = ocache.layer_attention(hp_o, layer, pos, q, k, v, wq, wk, None)
            outs = []
            for c in (full, ringc):
                out = torch.zeros(8 * d, device="cuda")
                gsrc, grange = c.layer_attention(hp_g, layer, pos, dev(q), dev(k), dev(v), dev(wq), dev(wk), None, out)
                ctx.check_status()
                assert (gsrc, grange) == (src, rr), pos
                outs.append(host(out))
            print(f"[parity] position {pos}: rows {rr}, rel err {I.rel_err(outs[0], ref):.2e}", flush=True)
            assert I.rel_err(outs[0], ref) <= TOL, pos
            assert np.array_equal(outs[0], outs[1]), pos
        assert full.len(layer) == ringc.len(layer) == hist + 3
    finally:
        full.close()
        ringc.close()
