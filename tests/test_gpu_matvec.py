"""The mat-vec kernels over GGUF weight formats (crates/llm-backend-cpu/src/matvec.rs)
on the GPU against the oracle.

Integer and sum-order work is checked bit for bit: Q8_0 activation
quantization, the Q8_0 mat-vec with quantized or f32 activations (f32 and
f64 sums), BF16 and F32 mat-vecs.  The fused GELU gate and the logit
soft-cap go through tanh, whose device implementation may differ from the
host libm by an ulp; they are checked within a few f32 ulps (fp16 GELU
table: one f16 ulp), and fused against separate device steps bit for bit,
as the reference's own test does (tests/matvec.rs:84-99).  Shapes cover the
reference tests' inputs, the E2B projections (1536 -> 2048/4096, FFN
6144 <-> 1536, the 262,144-row output head in a cut-down form) and the
edges of the kernels' tiling.
"""
import numpy as np
import pytest
import torch

import g4hip
import inputs as I
from oracle import pyoracle as orc

pytestmark = pytest.mark.gpu


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def q8_activation(ctx, x):
    n = x.size
    xs = torch.empty(n // 32, device="cuda")
    xq = torch.empty(n, dtype=torch.int8, device="cuda")
    ctx.quantize_q8_0(dev(x.astype(np.float32)), n, xs, xq)
    return xs, xq


def matrix(seed, rows, cols):
    if rows * cols <= 64 * 256:
        return I.lcg_values(seed, rows * cols)
    return np.random.default_rng(seed).uniform(-1.0, 1.0, rows * cols).astype(np.float32)


def test_quantize_q8_0_bit_exact(ctx):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 200) * 10.0 ** rng.integers(-3, 4, 32 * 200)).astype(np.float32)
    x[32:64] = 0.0
    x[64] = np.nan
    x[96 + 5] = np.inf
    x[128:160] = 1e-30
    x[160:192] = 127.0 * np.arange(32) / 31.0
    xs, xq = q8_activation(ctx, x)
    ref_s, ref_q = orc.quantize_q8_0(x)
    assert np.array_equal(host(xs).view(np.uint32), ref_s.view(np.uint32))
    assert np.array_equal(host(xq), ref_q)
    # tests/matvec.rs:40-49
    blk = np.zeros(32, np.float32)
    blk[:3] = [127.0, 2.5, -3.5]
    xs, xq = q8_activation(ctx, blk)
    assert list(host(xs)) == [1.0] and list(host(xq)[:4]) == [127, 2, -4, 0]


SHAPES = [
    (64, 256),     # the reference tests' shape
    (300, 256),
    (2048, 1536),  # E2B q projection of a sliding layer
    (1536, 6144),  # FFN down: 192 blocks a row
    (77, 512),
    (5, 8192),     # 256 blocks a row
    (33, 96),      # cols not a multiple of 256: the row-per-lane kernel
    (1, 32),
    (4099, 1536),  # rows not a multiple of the row tile
]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_matvec_q8_0_bit_exact(ctx, rows, cols):
    print(f"[case] q8_0 {rows}x{cols}", flush=True)
    w = I.q8_0_bytes(matrix(rows + cols, rows, cols))
    x = I.lcg_values(2, cols) if cols <= 4096 else np.random.default_rng(2).uniform(-1, 1, cols).astype(np.float32)
    xs, xq = q8_activation(ctx, x)
    out = torch.empty(rows, device="cuda")
    ctx.matvec_q8_0(dev(w), rows, cols, xs, xq, out)
    ref = orc.matvec_q8_0(w, rows, cols, host(xs), host(xq))
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(300, 256), (1000, 1536), (13, 96)])
def test_softcap_and_geglu(ctx, rows, cols):
    gate = I.q8_0_bytes(matrix(5, rows, cols) * 4.0)
    up = I.q8_0_bytes(matrix(6, rows, cols))
    x = I.lcg_values(7, cols)
    xs, xq = q8_activation(ctx, x)
    hxs, hxq = host(xs), host(xq)
    dg, du = dev(gate), dev(up)
    g = torch.empty(rows, device="cuda")
    ctx.matvec_q8_0(dg, rows, cols, xs, xq, g)
    # soft-cap: within a few ulps of the oracle (device tanh)
    for cap in (30.0, 2.0):
        capped = torch.empty(rows, device="cuda")
        ctx.matvec_q8_0(dg, rows, cols, xs, xq, capped, softcap=cap)
        ref = orc.matvec_q8_0(gate, rows, cols, hxs, hxq, softcap=cap)
        assert np.max(np.abs(host(capped) - ref)) <= 4e-7 * cap
    # GELU gate: within a few ulps; the fp16 table within one f16 ulp
    out = torch.empty(rows, device="cuda")
    ctx.geglu_q8_0(dg, du, rows, cols, xs, xq, out)
    ref = orc.geglu_q8_0(gate, up, rows, cols, hxs, hxq)
    got = host(out)
    assert np.all(np.abs(got - ref) <= 4e-7 * np.maximum(np.abs(ref), 1.0))
    ctx.geglu_q8_0(dg, du, rows, cols, xs, xq, out, fp16_gelu=True)
    ref16 = orc.geglu_q8_0(gate, up, rows, cols, hxs, hxq, fp16_gelu=True)
    assert np.all(np.abs(host(out) - ref16) <= 2.0 ** -10 * np.maximum(np.abs(ref16), 1.0) * 2)
    # fused == separate steps on the device (tests/matvec.rs:84-99)
    u = torch.empty(rows, device="cuda")
    ctx.matvec_q8_0(du, rows, cols, xs, xq, u)
    ctx.geglu_q8_0(dg, du, rows, cols, xs, xq, out)
    hg, hu = host(g), host(u)
    assert np.max(np.abs(got - np.array([orc.gelu_tanh(a) * b for a, b in zip(hg, hu)], np.float32))) <= \
        4e-7 * max(1.0, float(np.max(np.abs(got))))


@pytest.mark.parametrize("rows,cols", [(64, 256), (333, 1536), (7, 96)])
@pytest.mark.parametrize("f64_sums", [False, True])
def test_matvec_q8_0_f32_activations_bit_exact(ctx, rows, cols, f64_sums):
    w = I.q8_0_bytes(matrix(1, rows, cols))
    x = I.lcg_values(2, cols)
    out = torch.empty(rows, device="cuda")
    ctx.matvec_q8_0_f32(dev(w), rows, cols, dev(x), out, f64_sums=f64_sums)
    ref = orc.matvec_q8_0_f32(w, rows, cols, x, f64_sums=f64_sums)
    assert np.array_equal(host(out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(1, 2), (17, 96), (1031, 1024)])
def test_bf16_and_f32_matvecs_bit_exact(ctx, rows, cols):
    w = matrix(3, rows, cols)
    x = I.lcg_values(4, cols)
    out = torch.empty(rows, device="cuda")
    ctx.matvec_f32(dev(w), rows, cols, dev(x), out)
    assert np.array_equal(host(out).view(np.uint32), orc.matvec_f32(w, rows, cols, x).view(np.uint32))
    wb = np.array([orc.f32_to_bf16(v) for v in w], np.uint16) if w.size < 100000 else \
        ((w.view(np.uint32) + 0x7FFF + ((w.view(np.uint32) >> 16) & 1)) >> 16).astype(np.uint16)
    ctx.matvec_bf16(dev(wb), rows, cols, dev(x), out)
    assert np.array_equal(host(out).view(np.uint32), orc.matvec_bf16(wb, rows, cols, x).view(np.uint32))


def test_bf16_known_answer(ctx):
    """tests/matvec.rs:109-120: x is rounded to bf16 before the product."""
    w = np.array([orc.f32_to_bf16(2.0), orc.f32_to_bf16(-0.5)], np.uint16)
    out = torch.empty(1, device="cuda")
    ctx.matvec_bf16(dev(w), 1, 2, dev(np.array([1.0 + 1.0 / 256.0, 4.0], np.float32)), out)
    assert host(out)[0] == 2.0 * 1.0 - 0.5 * 4.0


def test_shape_errors(ctx):
    out = torch.empty(8, device="cuda")
    with pytest.raises(g4hip.EngError, match="f32 weight has 6 elements, expected 4 rows of 2"):
        ctx.matvec_f32(dev(np.ones(6, np.float32)), 4, 2, dev(np.ones(2, np.float32)), out)
    with pytest.raises(g4hip.EngError, match="Q8_0 activation length 31 is not a multiple of 32"):
        ctx.quantize_q8_0(dev(np.ones(31, np.float32)), 31, out, out)
    xs, xq = q8_activation(ctx, np.ones(32, np.float32))
    with pytest.raises(g4hip.EngError, match="Q8_0 weight has 34 elements, expected 2 rows of 34"):
        ctx.matvec_q8_0(dev(np.zeros(34, np.uint8)), 2, 32, xs, xq, out)
    with pytest.raises(g4hip.EngError, match="Q8_0 row length 33 is not a multiple of 32"):
        ctx.matvec_q8_0_f32(dev(np.zeros(34, np.uint8)), 1, 33, dev(np.ones(33, np.float32)), out)
    with pytest.raises(g4hip.EngError, match="BF16 weight has 3 elements, expected 1 rows of 2"):
        ctx.matvec_bf16(dev(np.zeros(3, np.uint16)), 1, 2, dev(np.ones(2, np.float32)), out)


@pytest.mark.parametrize("rows,cols", [(64, 256), (2048, 1536), (300, 96), (3, 8192)])
def test_fused_quantization_entries_equal_the_two_step_calls(ctx, rows, cols):
    """project / gated FFN / logits with the activation quantized inside the
    call: bit for bit the quantize_q8_0 + mat-vec pair (model.rs:211-212,
    236-237, 447).  An f32 activation that is not 16-byte aligned and column
    counts outside the LDS-staged kernel take the two-step route inside."""
    gate = dev(I.q8_0_bytes(matrix(8, rows, cols)))
    up = dev(I.q8_0_bytes(matrix(9, rows, cols)))
    xh = np.random.default_rng(rows).standard_normal(cols + 1).astype(np.float32)
    for x in (dev(xh[:cols]), dev(xh)[1:]):  # aligned, then 4 bytes off
        xs = torch.empty(cols // 32, device="cuda")
        xq = torch.empty(cols, dtype=torch.int8, device="cuda")
        ctx.quantize_q8_0(x, cols, xs, xq)
        a, b = torch.empty(rows, device="cuda"), torch.empty(rows, device="cuda")
        ctx.matvec_q8_0(gate, rows, cols, xs, xq, a)
        ctx.project_q8_0(gate, rows, cols, x, b)
        assert torch.equal(a, b)
        ctx.matvec_q8_0(gate, rows, cols, xs, xq, a, softcap=30.0)
        ctx.logits_q8_0(gate, rows, cols, x, 30.0, b)
        assert torch.equal(a, b)
        for f16 in (False, True):
            ctx.geglu_q8_0(gate, up, rows, cols, xs, xq, a, fp16_gelu=f16)
            ctx.gated_ffn_q8_0(gate, up, rows, cols, x, b, fp16_gelu=f16)
            assert torch.equal(a, b)


def test_empty_rows(ctx):
    """cols == 0: every output is the empty sum (the reference's -0.0, through
    the soft-cap or the GELU gate), with no element read -- for the calls that
    quantize the activation inside, and for the quantized-activation ones."""
    rows = 5
    e8 = np.zeros(0, np.uint8)
    ef, ei = np.zeros(0, np.float32), np.zeros(0, np.int8)
    w = torch.empty(0, dtype=torch.uint8, device="cuda")
    x = torch.empty(0, device="cuda")
    xs, xq = torch.empty(0, device="cuda"), torch.empty(0, dtype=torch.int8, device="cuda")
    out = torch.full((rows,), 7.0, device="cuda")

    def bits(t):
        return host(t).view(np.uint32)

    ref = orc.matvec_q8_0(e8, rows, 0, ef, ei).view(np.uint32)
    ctx.project_q8_0(w, rows, 0, x, out)
    assert np.array_equal(bits(out), ref)
    ctx.matvec_q8_0(w, rows, 0, xs, xq, out)
    assert np.array_equal(bits(out), ref)
    ref = orc.matvec_q8_0(e8, rows, 0, ef, ei, softcap=30.0).view(np.uint32)
    ctx.logits_q8_0(w, rows, 0, x, 30.0, out)
    assert np.array_equal(bits(out), ref)
    for f16 in (False, True):
        ref = orc.geglu_q8_0(e8, e8, rows, 0, ef, ei, fp16_gelu=f16).view(np.uint32)
        ctx.gated_ffn_q8_0(w, w, rows, 0, x, out, fp16_gelu=f16)
        assert np.array_equal(bits(out), ref)
