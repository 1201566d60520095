"""Pins the oracle's restatement of the mat-vec kernels over GGUF weight
formats (crates/llm-backend-cpu/src/matvec.rs, dequant.rs, ops.rs:79-103).

The checks are the reference's own tests (crates/llm-backend-cpu/tests/matvec.rs:
known answers, agreement with the dequantized product, fused == separate,
shape errors) on the same inputs, plus independent references: numpy's
IEEE half conversion for every f16 bit pattern and a large set of f32
values, and closed forms of GELU-tanh and the soft-cap in f64.
test_planted_mistakes_are_caught rebuilds the oracle with one plausible
mistake at a time and shows one of these checks fails.
"""
import math
import os
import subprocess
import sys

import numpy as np
import pytest

import inputs as I
from oracle import pyoracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))


values = I.lcg_values  # the reference tests' generator (tests/matvec.rs:9-18)
q8_0_bytes = I.q8_0_bytes  # and their Q8_0 quantizer (tests/matvec.rs:21-31)


def naive(w, x, rows):
    return (np.asarray(w, np.float64).reshape(rows, -1) @ np.asarray(x, np.float64)).astype(np.float64)


# ------------------------------------------------------------- conversions
def test_f16_conversions_match_ieee_half():
    bits = np.arange(1 << 16, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10.0) ** rng.integers(-9, 6, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 65519.99, 1e9, -1e9, 5.960464477539063e-08, 2.98e-08, 2.9802322e-08,
                  1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 6.1035156e-05, 6.097555e-05, np.inf, -np.inf], np.float32),
        (np.arange(1 << 16, dtype=np.uint32) << 13).view(np.float32)[:30000] + np.float32(0),  # halfway cases
    ]).astype(np.float32)
    with np.errstate(over="ignore"):
        ref16 = xs.astype(np.float16).view(np.uint16)
    got16 = np.array([orc.f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got16, ref16)


def test_bf16_known_answers():
    """tests/matvec.rs:109-120"""
    assert orc.f32_to_bf16(1.0) == 0x3F80
    assert orc.f32_to_bf16(1.0 + 1.0 / 256.0) == 0x3F80  # halfway: ties to even
    assert orc.f32_to_bf16(1.0 + 3.0 / 256.0) == 0x3F82
    assert orc.bf16_to_f32(0x3F82) == 1.015625
    w = np.array([orc.f32_to_bf16(2.0), orc.f32_to_bf16(-0.5)], np.uint16)
    assert np.array_equal(orc.matvec_bf16(w, 1, 2, [1.0 + 1.0 / 256.0, 4.0]), np.array([2.0 * 1.0 - 0.5 * 4.0], np.float32))


# ----------------------------------------------------------- quantization
def test_quantize_q8_0_known_answer():
    """tests/matvec.rs:40-49: scale max/127, round half to even."""
    block = np.zeros(32, np.float32)
    block[:3] = [127.0, 2.5, -3.5]
    scales, quants = orc.quantize_q8_0(block)
    assert list(scales) == [1.0]
    assert list(quants[:4]) == [127, 2, -4, 0]


def test_quantize_q8_0_scales_are_half_roundings():
    x = values(11, 32 * 40) * np.float32(3.0)
    x[32:64] = 0.0  # an all-zero block: scale 0, quants 0
    scales, quants = orc.quantize_q8_0(x)
    maxes = np.abs(x.reshape(-1, 32)).max(axis=1)
    exact = maxes / np.float32(127.0)
    assert np.array_equal(scales, exact.astype(np.float16).astype(np.float32))
    assert not np.array_equal(scales, exact)  # most f32 scales are not halves
    inv = np.where(exact == 0, np.float32(0), np.float32(1) / np.where(exact == 0, 1, exact)).astype(np.float32)
    assert np.array_equal(quants, np.rint(x.reshape(-1, 32) * inv[:, None]).astype(np.int8).reshape(-1))
    assert np.all(quants[32:64] == 0) and scales[1] == 0.0


# ---------------------------------------------------------------- mat-vecs
def test_q8_0_matvec_equals_the_dequantized_product():
    """tests/matvec.rs:51-67"""
    rows, cols = 64, 256
    w = q8_0_bytes(values(1, rows * cols))
    xs, xq = orc.quantize_q8_0(values(2, cols))
    xd = (xq.reshape(-1, 32).astype(np.float32) * xs[:, None]).reshape(-1)
    expected = naive(orc.dequant_q8_0(w), xd, rows)
    got = orc.matvec_q8_0(w, rows, cols, xs, xq)
    assert np.max(np.abs(got - expected)) < 1e-4


def test_q8_0_matvec_with_f32_activations_equals_the_dequantized_product():
    """tests/matvec.rs:69-82"""
    rows, cols = 64, 256
    w = q8_0_bytes(values(1, rows * cols))
    x = values(2, cols)
    expected = naive(orc.dequant_q8_0(w), x, rows)
    assert np.max(np.abs(orc.matvec_q8_0_f32(w, rows, cols, x) - expected)) < 1e-4
    assert np.max(np.abs(orc.matvec_q8_0_f32(w, rows, cols, x, f64_sums=True) - expected)) < 1e-4
    # the f64 sums round once: they are the f64 product rounded to f32
    assert np.max(np.abs(orc.matvec_q8_0_f32(w, rows, cols, x, f64_sums=True) - expected)) <= \
        np.max(np.abs(expected)) * 2.0 ** -23


def test_fused_kernels_give_the_same_bits_as_separate_steps():
    """tests/matvec.rs:84-99: geglu == gelu(gate) * up, softcap after the mat-vec."""
    rows, cols = 300, 256
    gate = q8_0_bytes(values(5, rows * cols))
    up = q8_0_bytes(values(6, rows * cols))
    xs, xq = orc.quantize_q8_0(values(7, cols))
    g = orc.matvec_q8_0(gate, rows, cols, xs, xq)
    u = orc.matvec_q8_0(up, rows, cols, xs, xq)
    separate = np.array([orc.gelu_tanh(a) * b for a, b in zip(g, u)], np.float32)
    assert np.array_equal(orc.geglu_q8_0(gate, up, rows, cols, xs, xq), separate)
    capped = np.array([orc.softcap(v, 2.0) for v in g], np.float32)
    assert np.array_equal(orc.matvec_q8_0(gate, rows, cols, xs, xq, softcap=2.0), capped)


def test_q8_0_matvec_is_close_to_the_f32_product():
    """tests/matvec.rs:101-112"""
    rows, cols = 64, 256
    w = values(1, rows * cols)
    x = values(2, cols)
    xs, xq = orc.quantize_q8_0(x)
    got = orc.matvec_q8_0(q8_0_bytes(w), rows, cols, xs, xq)
    assert np.max(np.abs(got - naive(w, x, rows))) < 0.25


def test_f32_matvec_of_many_rows():
    """tests/matvec.rs:114-126"""
    rows, cols = 1031, 1024
    w, x = values(3, rows * cols), values(4, cols)
    got = orc.matvec_f32(w, rows, cols, x)
    assert got.shape == (rows,) and np.max(np.abs(got - naive(w, x, rows))) < 1e-3


def test_bf16_matvec_uses_rounded_inputs():
    rng = np.random.default_rng(5)
    rows, cols = 17, 96
    w = np.array([orc.f32_to_bf16(v) for v in rng.standard_normal(rows * cols)], np.uint16)
    x = rng.standard_normal(cols).astype(np.float32)
    wd = np.array([orc.bf16_to_f32(b) for b in w], np.float64)
    xr = np.array([orc.bf16_to_f32(orc.f32_to_bf16(v)) for v in x], np.float64)
    got = orc.matvec_bf16(w, rows, cols, x)
    assert np.max(np.abs(got - naive(wd, xr, rows))) < 1e-4
    assert np.max(np.abs(got - naive(wd, x, rows))) > 1e-5  # the rounding of x shows


def test_shape_mismatches_are_errors():
    """tests/matvec.rs:128-132 and the reference's messages."""
    with pytest.raises(orc.OracleError, match="f32 weight has 6 elements, expected 4 rows of 2"):
        orc.matvec_f32(np.ones(6), 4, 2, [1.0, 1.0])
    with pytest.raises(orc.OracleError, match="Q8_0 activation length 31 is not a multiple of 32"):
        orc.quantize_q8_0(np.ones(31))
    with pytest.raises(orc.OracleError, match="Q8_0 weight has 34 elements, expected 2 rows of 34"):
        orc.matvec_q8_0(np.zeros(34, np.uint8), 2, 32, [1.0], np.zeros(32, np.int8))
    with pytest.raises(orc.OracleError, match="Q8_0 row length 33 is not a multiple of 32"):
        orc.matvec_q8_0_f32(np.zeros(34, np.uint8), 1, 33, np.ones(33))


# ------------------------------------------------------------- activations
def test_gelu_and_softcap_closed_forms():
    xs = np.linspace(-12.0, 12.0, 481)
    for x in xs:
        x32 = float(np.float32(x))
        exact = 0.5 * x32 * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (x32 + 0.044715 * x32 ** 3)))
        assert abs(orc.gelu_tanh(x32) - exact) <= 4e-7 * max(1.0, abs(exact))
        t = orc.gelu_tanh_fp16_table(x32)
        if x32 <= -10.0:
            assert t == 0.0
        elif x32 >= 10.0:
            assert t == x32
        else:
            assert t == float(np.float16(orc.gelu_tanh(float(np.float16(x32)))))
        for cap in (30.0, 2.0):
            assert abs(orc.softcap(x32, cap) - cap * math.tanh(x32 / cap)) <= 4e-7 * cap


# ------------------------------------------------------------- planted bugs
PLANTS = {
    "G4_PLANT_Q8_ROUND_AWAY": "test_quantize_q8_0_known_answer",
    "G4_PLANT_Q8_SCALE_F32": "test_quantize_q8_0_scales_are_half_roundings",
    "G4_PLANT_SOFTCAP": "test_gelu_and_softcap_closed_forms",
    "G4_PLANT_GELU_COEF": "test_gelu_and_softcap_closed_forms",
    "G4_PLANT_BF16_TRUNC": "test_bf16_known_answers",
}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_planted_mistakes_are_caught(plant, tmp_path):
    """Each plausible mistake, planted in a copy of the oracle, fails a check above."""
    root = os.path.dirname(HERE)
    so = tmp_path / "liboracle.so"
    subprocess.run(["gcc", "-O1", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", f"-D{plant}", "-o", str(so),
                    os.path.join(root, "oracle", "g4_oracle.c"), os.path.join(root, "oracle", "g4_oracle_matvec.c"),
                    "-lm", "-lpthread"], check=True)
    env = dict(os.environ, G4_ORACLE_LIB=str(so))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        f"{__file__}::{PLANTS[plant]}"], env=env, cwd=root, capture_output=True, text=True)
    assert r.returncode != 0, f"{plant} was not caught by {PLANTS[plant]}:\n{r.stdout[-2000:]}"
