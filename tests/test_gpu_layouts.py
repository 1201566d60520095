"""Cache layouts other than one KV head per unpadded row, on the GPU
against the oracle: rows padded beyond n_kv_heads * head_dim (`row_stride`)
and two KV heads per row (heads h read KV head h * n_kv / n_heads,
model.rs:329), through the decode (split and stream-K), prefill and the
layer drivers' building blocks.  Tolerance 1e-4 relative
(crates/llm-gemma4/tests/synthetic_generate.rs:74-83)."""
import numpy as np
import pytest
import torch

import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
TOL = 1e-4


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def padded(rng, T, n_kv, d, pad):
    """K or V rows [T][n_kv*d + pad]: the padding holds NaN, which no head may read."""
    x = np.full((T, n_kv * d + pad), np.nan, np.float32)
    x[:, :n_kv * d] = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    return x


@pytest.mark.parametrize("T,d,n_heads,n_kv,pad", [(100, 512, 8, 1, 32), (4096, 512, 8, 1, 64), (777, 256, 16, 2, 16),
                                                  (64, 256, 8, 1, 4), (3000, 512, 16, 2, 128)])
def test_decode_padded_rows_and_two_kv_heads(ctx, T, d, n_heads, n_kv, pad):
    print(f"[case] decode T={T} d={d} heads {n_heads}/{n_kv} pad {pad}", flush=True)
    rng = np.random.default_rng(T + d + pad)
    K, V = padded(rng, T, n_kv, d, pad), padded(rng, T, n_kv, d, pad)
    q = rng.standard_normal(n_heads * d).astype(np.float32) * 0.05
    out = torch.zeros(n_heads * d, device="cuda")
    ctx.attend_decode(dev(q), dev(K), dev(V), 0, T, n_heads, n_kv, d, out, row_stride=n_kv * d + pad)
    ctx.check_status()
    ref = orc.attend(q, K[:, :n_kv * d], V[:, :n_kv * d], n_heads, n_kv)
    assert I.rel_err(out.cpu().numpy(), ref) <= TOL


def test_ragged_stream_padded_rows_two_kv_heads(ctx):
    d, n_heads, n_kv, pad = 512, 16, 2, 32
    lens = np.array([50, 3000, 7, 1200, 16, 2500] * 6, np.int64)
    rng = np.random.default_rng(3)
    total = int(lens.sum())
    K, V = padded(rng, total, n_kv, d, pad), padded(rng, total, n_kv, d, pad)
    q = rng.standard_normal((len(lens), n_heads * d)).astype(np.float32) * 0.05
    row0 = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    out = torch.zeros(len(lens) * n_heads * d, device="cuda")
    ctx.attend_decode_batch(dev(q), dev(K), dev(V), dev(row0), dev(np.zeros(len(lens), np.int64)), dev(lens),
                            int(lens.max()), n_heads, n_kv, d, out, row_stride=n_kv * d + pad)
    ctx.check_status()
    got = out.cpu().numpy().reshape(len(lens), -1)
    for s in range(len(lens)):
        r = slice(row0[s], row0[s] + lens[s])
        ref = orc.attend(q[s], K[r, :n_kv * d], V[r, :n_kv * d], n_heads, n_kv)
        assert I.rel_err(got[s], ref) <= TOL, s


@pytest.mark.parametrize("d,window,n_heads,n_kv,pad", [(512, 0, 8, 1, 64), (256, 64, 8, 1, 8), (256, 0, 16, 2, 32),
                                                       (512, 100, 16, 2, 16)])
def test_prefill_padded_rows_and_two_kv_heads(ctx, d, window, n_heads, n_kv, pad):
    print(f"[case] prefill d={d} W={window} heads {n_heads}/{n_kv} pad {pad}", flush=True)
    pos0, N = 150, 90
    rng = np.random.default_rng(d + window + pad)
    K, V = padded(rng, pos0 + N, n_kv, d, pad), padded(rng, pos0 + N, n_kv, d, pad)
    q = rng.standard_normal((N, n_heads * d)).astype(np.float32) * 0.05
    out = torch.zeros(N * n_heads * d, device="cuda")
    ctx.attend_prefill(dev(q), dev(K), dev(V), pos0, N, window, n_heads, n_kv, d, out, row_stride=n_kv * d + pad)
    ctx.check_status()
    got = out.cpu().numpy().reshape(N, -1)
    for i in range(0, N, 7):
        b, e = I.attended_range(pos0 + i, window)
        ref = orc.attend(q[i], K[b:e, :n_kv * d], V[b:e, :n_kv * d], n_heads, n_kv)
        assert I.rel_err(got[i], ref) <= TOL, i
