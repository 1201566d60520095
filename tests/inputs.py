"""Seeded synthetic inputs for the five measured attention workloads.

q, K and V are f32 draws from N(0, 1) (numpy's PCG64 generator, seeded),
prepared as the engine prepares them before attention (model.rs:395-404):
per-head RMS norm with unit weight for q and K, RMS norm without weight for V,
NEOX RoPE for q at its position and for K row t at position t (base 1e4 on
sliding layers; base 1e6 divided by rope_freqs on global layers).  The same
buffers go to the oracle and to the device.
"""
import numpy as np

from oracle import pyoracle as orc

N_HEADS, N_KV = 8, 1
EPS = 1e-6
LOCAL_BASE, GLOBAL_BASE = 10000.0, 1000000.0
WINDOW = 512


def normal(seed, shape):
    return np.random.default_rng(seed).standard_normal(shape, dtype=np.float32)


def rope_freqs(seed, head_dim=512):
    """A seeded U[1, 8] rope_freqs vector (one divisor per NEOX pair)."""
    return np.random.default_rng(seed).uniform(1.0, 8.0, head_dim // 2).astype(np.float32)


def kv_rows(seed, n_rows, head_dim, base, freqs, pos0=0):
    """K and V cache rows for positions pos0..pos0+n_rows-1 (n_kv_heads = 1)."""
    k = normal(seed, (n_rows, N_KV * head_dim))
    v = normal(seed + 1, (n_rows, N_KV * head_dim))
    orc.prepare_rows(k, head_dim, None, EPS, pos0, base, freqs)
    orc.prepare_rows(v, head_dim, None, EPS, 0, 0.0, None)
    return k, v


def queries(seed, n, head_dim, base, freqs, pos0):
    """n query rows [n, n_heads*head_dim], row i at position pos0 + i."""
    q = normal(seed, (n, N_HEADS * head_dim))
    orc.prepare_rows(q, head_dim, None, EPS, pos0, base, freqs)
    return q


def decode_case(seed, T, head_dim, global_layer, query_pos=None, freqs=None):
    """One decode step over rows 0..T-1 of a fresh cache; the query sits at
    position T-1 unless given.  Returns (q [8*d], K [T, d], V [T, d], freqs)."""
    if global_layer and freqs is None:
        freqs = rope_freqs(seed + 7, head_dim)
    base = GLOBAL_BASE if global_layer else LOCAL_BASE
    k, v = kv_rows(seed, T, head_dim, base, freqs if global_layer else None)
    pos = T - 1 if query_pos is None else query_pos
    q = queries(seed + 2, 1, head_dim, base, freqs if global_layer else None, pos)[0]
    return q, k, v, freqs


def ragged_lengths(seed, B=32, lo=1024, hi=32768):
    """B context lengths drawn uniformly from [lo, hi]."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=B).astype(np.int64)


def attended_range(pos, window):
    """[begin, end) a decode at `pos` attends: window 0 = global."""
    end = pos + 1
    begin = max(0, end - window) if window else 0
    return begin, end


def rel_err(a, b):
    """max |a-b| / max(|a|, |b|, 1): the reference's assert_relative_eq measure
    (crates/llm-gemma4/tests/synthetic_generate.rs:74-83)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1.0)
    return float(np.max(np.abs(a - b) / scale)) if a.size else 0.0


# ------------------------------------------------- mat-vec inputs (Q8_0, BF16)
def lcg_values(seed, n):
    """The reference mat-vec tests' input generator
    (crates/llm-backend-cpu/tests/matvec.rs:9-18): a 64-bit LCG, values in [-1, 1)."""
    out = np.empty(n, np.float32)
    state = seed
    for i in range(n):
        state = (state * 6364136223846793005 + 1) % (1 << 64)
        out[i] = np.float32(state >> 40) / np.float32(1 << 23) - np.float32(1.0)
    return out


def q8_0_bytes(weights):
    """Q8_0 bytes of a row-major matrix as the reference tests build them
    (tests/matvec.rs:21-31): per 32 values an f16 scale max|w|/127, then the
    values w/scale rounded half away from zero (NaN -> 0), saturated."""
    blocks = np.asarray(weights, np.float32).reshape(-1, 32)
    scale = np.abs(blocks).max(axis=1) / np.float32(127.0)
    with np.errstate(invalid="ignore", divide="ignore"):
        q = blocks / scale[:, None]
    r = np.where(np.isnan(q), 0.0, np.sign(q) * np.floor(np.abs(q) + 0.5))
    qi = np.clip(r, -128, 127).astype(np.int8)
    out = np.empty((blocks.shape[0], 34), np.uint8)
    out[:, :2] = scale.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = qi.view(np.uint8)
    return out.reshape(-1)
