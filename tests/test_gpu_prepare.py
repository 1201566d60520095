"""The fused attention-input preparation (model.rs:394-406: q/k/v norm, RoPE,
append) and the whole-layer prefill driver built on it, on the GPU.

The fused kernel must give bit-for-bit what the separate norm and RoPE
kernels give (same operations in the same order), match the oracle's
norm_heads/rope_heads, and leave the appended cache rows equal to the
prepared k/v.  The layer prefill driver, run layer after layer over a prompt
chunk, must reproduce the reference's token-at-a-time loop
(generate.rs:37-41) as the oracle runs it: same source layer per layer,
outputs within the reference's own tolerance.
"""
import numpy as np
import pytest
import torch

import g4hip
import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4  # synthetic_generate.rs:74-83
ROPE_TOL = 2e-5  # device sin/cos differ from the host libm by ulps; the angles are the same


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


PREP_CASES = [
    # d, n_heads, n_kv, global, n_tokens, pos0
    (256, 8, 1, False, 1, 63),
    (512, 8, 1, True, 1, 4095),
    (512, 8, 1, True, 37, 100),
    (256, 8, 1, False, 300, 0),
    (512, 8, 1, True, 301, 5000),  # a prompt chunk (several tokens per workgroup), ragged last group
    (256, 4, 1, False, 67, 0),     # 6 head rows per token
    (16, 4, 2, True, 5, 0),
    (8, 4, 2, False, 3, 7),
    (128, 16, 2, True, 2, 32767),
]


@pytest.mark.parametrize("d,n_heads,n_kv,glob,n_tokens,pos0", PREP_CASES)
def test_prepare_matches_separate_kernels_and_oracle(ctx, d, n_heads, n_kv, glob, n_tokens, pos0):
    print(f"[case] prepare d={d} heads={n_heads}/{n_kv} tokens={n_tokens} pos0={pos0}", flush=True)
    rng = np.random.default_rng(d * 7 + n_tokens + pos0)
    q = (rng.standard_normal((n_tokens, n_heads * d)) * 2).astype(np.float32)
    k = (rng.standard_normal((n_tokens, n_kv * d)) * 2).astype(np.float32)
    v = (rng.standard_normal((n_tokens, n_kv * d)) * 2).astype(np.float32)
    wq = rng.uniform(0.5, 1.5, d).astype(np.float32)
    wk = rng.uniform(0.5, 1.5, d).astype(np.float32)
    freqs = I.rope_freqs(d, d) if glob else None
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    eps = 1e-6
    stride = n_kv * d + 3  # padded cache rows
    fq, fk, fv = dev(q), dev(k), dev(v)
    kc = torch.full(((n_tokens + 2) * stride,), float("nan"), device="cuda")
    vc = torch.full(((n_tokens + 2) * stride,), float("nan"), device="cuda")
    dfreqs = None if freqs is None else dev(freqs)
    # rows 1.. of the cache: the kernel must write exactly n_tokens rows there
    ctx.prepare_qkv(fq, fk, fv, n_tokens, pos0, n_heads, n_kv, d, dev(wq), dev(wk), eps, base, dfreqs,
                    k_rows=kc[stride:], v_rows=vc[stride:], row_stride=stride)
    # the same through the separate kernels
    sq, sk, sv = dev(q), dev(k), dev(v)
    ctx.rms_norm_rows(sq, n_tokens * n_heads, d, dev(wq), eps, sq)
    ctx.rope_neox_rows(sq, n_tokens, n_heads, d, d, pos0, base, dfreqs)
    ctx.rms_norm_rows(sk, n_tokens * n_kv, d, dev(wk), eps, sk)
    ctx.rms_norm_rows(sv, n_tokens * n_kv, d, None, eps, sv)
    ctx.rope_neox_rows(sk, n_tokens, n_kv, d, d, pos0, base, dfreqs)
    gq, gk, gv = host(fq), host(fk), host(fv)
    assert np.array_equal(gq, host(sq))
    assert np.array_equal(gk, host(sk))
    assert np.array_equal(gv, host(sv))
    kr = host(kc).reshape(n_tokens + 2, stride)
    vr = host(vc).reshape(n_tokens + 2, stride)
    assert np.array_equal(kr[1:n_tokens + 1, :n_kv * d], gk)
    assert np.array_equal(vr[1:n_tokens + 1, :n_kv * d], gv)
    # nothing else of the cache is touched
    assert np.isnan(kr[0]).all() and np.isnan(kr[n_tokens + 1]).all() and np.isnan(kr[:, n_kv * d:]).all()
    assert np.isnan(vr[0]).all() and np.isnan(vr[n_tokens + 1]).all() and np.isnan(vr[:, n_kv * d:]).all()
    # against the oracle: norm_heads then rope_heads per token (model.rs:395-404)
    for t in range(n_tokens):
        p = pos0 + t
        oq = orc.rope_heads(np.concatenate([orc.rms_norm(h, wq, eps) for h in q[t].reshape(n_heads, d)]), d, p,
                            base, freqs)
        ok = orc.rope_heads(np.concatenate([orc.rms_norm(h, wk, eps) for h in k[t].reshape(n_kv, d)]), d, p,
                            base, freqs)
        ov = np.concatenate([orc.rms_norm(h, None, eps) for h in v[t].reshape(n_kv, d)])
        assert np.max(np.abs(gq[t] - oq)) < ROPE_TOL
        assert np.max(np.abs(gk[t] - ok)) < ROPE_TOL
        assert np.array_equal(gv[t], ov)  # no RoPE on V: bit-exact


def test_prepare_q_only_leaves_k_and_v(ctx):
    d, n_heads = 512, 8
    rng = np.random.default_rng(3)
    q = rng.standard_normal(n_heads * d).astype(np.float32)
    k = rng.standard_normal(d).astype(np.float32)
    fq, fk, fv = dev(q), dev(k), dev(k)
    ctx.prepare_qkv(fq, None, None, 1, 9, n_heads, 1, d, None, None, 1e-6, I.LOCAL_BASE)
    oq = orc.rope_heads(np.concatenate([orc.rms_norm(h, None, 1e-6) for h in q.reshape(n_heads, d)]), d, 9,
                        I.LOCAL_BASE)
    assert np.max(np.abs(host(fq) - oq)) < ROPE_TOL
    assert np.array_equal(host(fk), k) and np.array_equal(host(fv), k)


def test_prepare_errors(ctx):
    x = torch.zeros(64, device="cuda")
    with pytest.raises(g4hip.EngError, match="invalid RoPE inputs"):
        ctx.prepare_qkv(x, None, None, 1, 0, 4, 1, 15, None, None, 1e-6, I.LOCAL_BASE)  # odd width
    with pytest.raises(g4hip.EngError, match="invalid RoPE inputs"):
        ctx.prepare_qkv(x, None, None, 1, 0, 4, 1, 16, None, None, 1e-6, 0.0)
    with pytest.raises(g4hip.EngError, match="invalid RMS norm inputs"):
        ctx.prepare_qkv(x, None, None, 1, 0, 4, 1, 16, None, None, -1.0, I.LOCAL_BASE)
    with pytest.raises(g4hip.EngError, match="cache rows"):
        ctx.prepare_qkv(x, x, x, 1, 0, 2, 1, 16, None, None, 1e-6, I.LOCAL_BASE, k_rows=x, v_rows=x, row_stride=8)
    with pytest.raises(g4hip.EngError, match="above 1024"):
        ctx.prepare_qkv(torch.zeros(2048, device="cuda"), None, None, 1, 0, 1, 1, 2048, None, None, 1e-6,
                        I.LOCAL_BASE)


# ------------------------------------------------------- whole-layer prefill
def widths(hp):
    out = []
    for l in range(hp.n_layers):
        src = orc.kv_source_layer(hp.n_layers, hp.shared_kv_layers, l)
        glob = orc.layer_attention_kind(hp.n_layers, l) == "global"
        out.append(hp.n_kv_heads * (hp.head_dim_global if glob else hp.head_dim_local) if src == l else 0)
    return out


def run_prefill(ctx, hp_g, hp_o, history, chunks, seed):
    """Owner caches get `history` prepared rows; then each chunk (a list of
    positions, consecutive) runs layer after layer through g4_layer_prefill
    on the device, and token after token, layer after layer, through the
    oracle's layer segment.  Returns the worst relative error."""
    rng = np.random.default_rng(seed)
    ws = widths(hp_o)
    total = history + sum(len(c) for c in chunks)
    cache = g4hip.KvCache(ctx, ws, total)
    ocache = orc.KvCache()
    freqs = I.rope_freqs(seed + 3, hp_o.head_dim_global)
    dfreqs = dev(freqs)
    worst = 0.0
    L = hp_o.n_layers

    def dim(l):
        return hp_o.head_dim_global if orc.layer_attention_kind(L, l) == "global" else hp_o.head_dim_local

    try:
        for l, w in enumerate(ws):
            if not w or not history:
                continue
            glob = orc.layer_attention_kind(L, l) == "global"
            K, V = I.kv_rows(seed + 100 + l, history, dim(l), I.GLOBAL_BASE if glob else I.LOCAL_BASE,
                             freqs if glob else None)
            cache.append_rows(l, dev(K), dev(V), history)
            for t in range(history):
                ocache.append(l, K[t], V[t])
        for chunk in chunks:
            n, pos0 = len(chunk), chunk[0]
            assert chunk == list(range(pos0, pos0 + n))
            qs = [rng.standard_normal((n, hp_o.n_heads * dim(l))).astype(np.float32) for l in range(L)]
            ks = [rng.standard_normal((n, hp_o.n_kv_heads * dim(l))).astype(np.float32) for l in range(L)]
            vs = [rng.standard_normal((n, hp_o.n_kv_heads * dim(l))).astype(np.float32) for l in range(L)]
            wq = [rng.uniform(0.5, 1.5, dim(l)).astype(np.float32) for l in range(L)]
            wk = [rng.uniform(0.5, 1.5, dim(l)).astype(np.float32) for l in range(L)]
            refs = [[None] * n for _ in range(L)]
            srcs = [None] * L
            for i, pos in enumerate(chunk):  # the reference's order: token-major
                for l in range(L):
                    glob = orc.layer_attention_kind(L, l) == "global"
                    out, src, _, _, _, _ = ocache.layer_attention(hp_o, l, pos, qs[l][i], ks[l][i], vs[l][i], wq[l],
                                                                  wk[l], freqs if glob else None)
                    refs[l][i] = out
                    srcs[l] = src
            for l in range(L):  # the device: layer-major, one call per layer
                glob = orc.layer_attention_kind(L, l) == "global"
                out = torch.zeros(n * hp_o.n_heads * dim(l), device="cuda")
                src = cache.layer_prefill(hp_g, l, pos0, n, dev(qs[l]), dev(ks[l]), dev(vs[l]), dev(wq[l]),
                                          dev(wk[l]), dfreqs if glob else None, out)
                assert src == srcs[l], l
                ctx.check_status()
                got = host(out).reshape(n, -1)
                for i in range(n):
                    worst = max(worst, I.rel_err(got[i], refs[l][i]))
    finally:
        cache.close()
    return worst


def test_layer_prefill_synthetic_model_shape(ctx):
    """The reference's synthetic model shape (synthetic_generate.rs:12-34), a
    prompt of 20 in chunks of 7, 1 and 12 (window 8, shared layers)."""
    hp_o = orc.Hparams(7, 4, 2, 8, 16, 8, 2, 10000.0, 1000000.0, 1e-6)
    hp_g = g4hip.G4Hparams(7, 4, 2, 8, 16, 8, 2, 10000.0, 1000000.0, 1e-6)
    worst = run_prefill(ctx, hp_g, hp_o, 0, [list(range(0, 7)), [7], list(range(8, 20))], 11)
    print(f"[parity] layer prefill, synthetic shape: worst rel err {worst:.2e}")
    assert worst <= TOL


def test_layer_prefill_e2b_prompt(ctx):
    """A 48-token prompt through the 35-layer E2B stack from an empty cache."""
    print("[case] layer prefill E2B 0..47", flush=True)
    worst = run_prefill(ctx, g4hip.G4Hparams.e2b(), orc.Hparams.e2b(), 0, [list(range(48))], 21)
    print(f"[parity] layer prefill, E2B prompt 48: worst rel err {worst:.2e}")
    assert worst <= TOL


def test_layer_prefill_e2b_chunk_across_the_window(ctx):
    """History of 500 rows, then a chunk at positions 500..539: sliding layers'
    windows start moving inside the chunk."""
    print("[case] layer prefill E2B 500..539", flush=True)
    worst = run_prefill(ctx, g4hip.G4Hparams.e2b(), orc.Hparams.e2b(), 500, [list(range(500, 540))], 23)
    print(f"[parity] layer prefill, E2B chunk across the window: worst rel err {worst:.2e}")
    assert worst <= TOL


def test_layer_prefill_errors(ctx):
    hp = g4hip.G4Hparams.e2b()
    cache = g4hip.KvCache(ctx, widths(orc.Hparams.e2b()), 16)
    try:
        q = torch.zeros(4 * 8 * 256, device="cuda")
        k = torch.zeros(4 * 256, device="cuda")
        out = torch.zeros_like(q)
        # layer 0 holds no rows yet: the first token (position 2) would view 3 rows of 1
        with pytest.raises(g4hip.EngError) as e:
            cache.layer_prefill(hp, 0, 2, 4, q, k, k, None, None, None, out)
        assert e.value.kind == "ContextTooLong" and e.value.fields == (3, 1)
        # beyond the capacity of 16 rows
        with pytest.raises(g4hip.EngError) as e:
            cache.layer_prefill(hp, 0, 0, 17, torch.zeros(17 * 8 * 256, device="cuda"),
                                torch.zeros(17 * 256, device="cuda"), torch.zeros(17 * 256, device="cuda"),
                                None, None, None, torch.zeros(17 * 8 * 256, device="cuda"))
        assert e.value.kind == "ContextTooLong" and e.value.fields == (17, 16)
        # a shared layer before its source has the rows
        with pytest.raises(g4hip.EngError) as e:
            cache.layer_prefill(hp, 15, 0, 4, q, k, k, None, None, None, out)
        assert e.value.kind == "MissingLayer"
        assert cache.len(0) == 0
        assert cache.layer_prefill(hp, 0, 0, 0, q, k, k, None, None, None, out) == 0
    finally:
        cache.close()
