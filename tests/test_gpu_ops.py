"""Attention-input preparation (per-head RMS norm, NEOX RoPE) and the
ComputePort methods on the GPU, against the oracle and the reference's own
known answers (crates/llm-backend-cpu/tests/ops_smoke.rs)."""
import json
import math
import os

import numpy as np
import pytest
import torch

import g4hip
import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu
KATS = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


@pytest.mark.parametrize("width,rows,weighted", [(256, 9, True), (512, 8, True), (512, 3, False), (8, 5, True),
                                                 (2, 1, True), (1000, 4, False)])
def test_rms_norm_rows_matches_oracle(ctx, width, rows, weighted):
    rng = np.random.default_rng(width + rows)
    x = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
    w = rng.uniform(0.5, 2.0, width).astype(np.float32) if weighted else None
    out = torch.zeros(rows * width, device="cuda")
    ctx.rms_norm_rows(dev(x), rows, width, None if w is None else dev(w), 1e-6, out)
    got = out.cpu().numpy().reshape(rows, width)
    ref = np.stack([orc.rms_norm(x[r], w, 1e-6) for r in range(rows)])
    # The device sums the f64 squares in a tree, the reference in sequence;
    # both are exact or far below f32 resolution, so the results are bit-equal.
    assert np.array_equal(got, ref)


def test_rms_norm_known_answers(ctx):
    k = KATS["rms_norm_weighted"]
    out = torch.zeros(2, device="cuda")
    ctx.port_rms_norm(dev(k["x"]), dev(k["weight"]), 2, 0.0, out)
    assert np.all(np.abs(out.cpu().numpy() - np.array(k["expected"])) < k["abs_tol"])
    k = KATS["rms_norm_unit_weight"]
    ctx.port_rms_norm(dev(k["x"]), dev(k["weight"]), 2, 0.0, out)
    assert np.all(np.abs(out.cpu().numpy() - np.array(k["expected"])) < k["abs_tol"])


@pytest.mark.parametrize("d,n_heads,glob", [(256, 8, False), (512, 8, True), (512, 1, True), (16, 4, True)])
@pytest.mark.parametrize("pos0", [0, 1, 4095, 32767])
def test_rope_rows_matches_oracle(ctx, d, n_heads, glob, pos0):
    rng = np.random.default_rng(d + pos0)
    n_tokens = 3
    x = rng.standard_normal((n_tokens, n_heads * d)).astype(np.float32)
    freqs = I.rope_freqs(1, d) if glob else None
    base = I.GLOBAL_BASE if glob else I.LOCAL_BASE
    t = dev(x)
    ctx.rope_neox_rows(t, n_tokens, n_heads, d, d, pos0, base, None if freqs is None else dev(freqs))
    got = t.cpu().numpy()
    ref = np.stack([orc.rope_heads(x[i], d, pos0 + i, base, freqs) for i in range(n_tokens)])
    # same angles (same f32 recurrence); sin/cos of the device libm differ by ulps
    assert np.max(np.abs(got - ref)) < 2e-5


def test_rope_with_e2b_proportional_factors(ctx):
    d = 512
    f = orc.proportional_rope_freq_factors(d, 0.25)
    x = np.random.default_rng(0).standard_normal(8 * d).astype(np.float32)
    t = dev(x)
    ctx.rope_neox_rows(t, 1, 8, d, d, 4095, I.GLOBAL_BASE, dev(f))
    got = t.cpu().numpy()
    assert np.max(np.abs(got - orc.rope_heads(x, d, 4095, I.GLOBAL_BASE, f))) < 2e-5
    # pairs 64.. (factor 1e30) are left as they were
    h = got.reshape(8, d)
    assert np.allclose(h[:, 64:256], x.reshape(8, d)[:, 64:256], atol=1e-6)


def test_rope_known_answers_and_errors(ctx):
    k = KATS["rope_neox_pairs_halves"]
    t = dev(k["x"])
    ctx.rope_neox_rows(t, 1, 1, 5, k["n_rot"], k["position"], k["base"])
    x = t.cpu().numpy()
    assert np.all(np.abs(x - np.array([math.cos(2), math.cos(0.2), math.sin(2), math.sin(0.2), 7.0])) < k["abs_tol"])
    k = KATS["rope_neox_huge_factors"]
    t = dev(k["x"])
    ctx.rope_neox_rows(t, 1, 1, 4, 4, k["position"], k["base"], dev(k["freq_factors"]))
    x = t.cpu().numpy()
    assert abs(x[0] - (math.cos(5) - 3 * math.sin(5))) < k["x0_abs_tol"]
    assert abs(x[1] - 2.0) < 1e-6 and abs(x[3] - 4.0) < 1e-6
    k = KATS["rope_pos1_base1_dims2"]
    t = dev(k["x"])
    ctx.port_rope(t, 2, 1, 1.0, 2)
    x = t.cpu().numpy()
    assert abs(x[0] - math.cos(1.0)) < 1e-6 and abs(x[1] - math.sin(1.0)) < 1e-6
    with pytest.raises(g4hip.EngError, match="invalid RoPE inputs"):
        ctx.port_rope(t, 2, 1, 1.0, 3)
    with pytest.raises(g4hip.EngError, match="invalid RoPE inputs"):
        ctx.port_rope(t, 2, 1, 0.0, 2)


@pytest.mark.parametrize("length,dims", [(50001, 40000), (8194, 8194)])
def test_port_rope_wide_rows(ctx, length, dims):
    """ComputePort::rope over rows wider than one LDS table chunk (4096
    pairs): the angle recurrence carries across chunks, values past dims
    stay as they were."""
    x = np.random.default_rng(length).standard_normal(length).astype(np.float32)
    t = dev(x)
    ctx.port_rope(t, length, 12345, 10000.0, dims)
    got = t.cpu().numpy()
    ref = orc.rope_neox(x, 12345, 10000.0, dims)
    assert np.max(np.abs(got - ref)) < 2e-5
    assert np.array_equal(got[dims:], x[dims:])


def test_compute_port_methods(ctx):
    """CpuPort's behaviour (crates/llm-backend-cpu/src/port.rs) on device buffers."""
    out = torch.zeros(4, device="cuda")
    ctx.port_matmul(dev([1, 2, 3, 4]), dev([5, 6, 7, 8]), 2, 2, 2, out)  # ops_smoke.rs:16-24
    assert out.cpu().tolist() == [19.0, 22.0, 43.0, 50.0]
    k = KATS["softmax_1_2"]
    sm = torch.zeros(2, device="cuda")
    ctx.port_softmax(dev(k["x"]), 2, sm)
    assert np.all(np.abs(sm.cpu().numpy() - np.array(k["expected"])) < k["abs_tol"])
    with pytest.raises(g4hip.EngError, match="softmax input is not finite"):
        ctx.port_softmax(dev([1.0, float("nan")]), 2, sm)
    with pytest.raises(g4hip.EngError, match="non-empty"):
        ctx.port_softmax(dev([1.0]), 0, sm)
    add = torch.zeros(2, device="cuda")
    ctx.port_add(dev([1, 2]), dev([3, 4]), 2, add)  # ops_smoke.rs:86-88
    assert add.cpu().tolist() == [4.0, 6.0]
    rng = np.random.default_rng(1)
    a = rng.standard_normal((33, 17)).astype(np.float32)
    b = rng.standard_normal((17, 9)).astype(np.float32)
    mm = torch.zeros(33 * 9, device="cuda")
    ctx.port_matmul(dev(a), dev(b), 33, 9, 17, mm)
    ref = np.zeros((33, 9), np.float32)
    for k_ in range(17):  # the reference's loop order: sequential inner sum
        ref += a[:, k_:k_ + 1] * b[k_:k_ + 1, :]
    assert np.array_equal(mm.cpu().numpy().reshape(33, 9), ref)
