"""Pins the oracle (the C restatement of the reference's attention path) to
what fixes it independently of its own code:

- the known-answer vectors of the reference's own tests
  (tests/golden/reference_kats.json, read from the cited lines);
- closed forms of attention (one row, equal keys, a dominant score, the GQA
  head -> KV-head map) and an f64 brute force written as the textbook
  softmax(q.K^T).V with numpy;
- invariants (RoPE preserves each pair's norm, RMS norm output has unit RMS,
  softmax sums to one and is shift invariant).

test_planted_mistakes rebuilds the oracle with one plausible mistake at a
time and shows the checks here catch each.
"""
import json
import math
import os
import subprocess
import sys

import numpy as np
import pytest

from oracle import pyoracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


# --------------------------------------------------------------- primitives
def test_rms_norm_known_answers():
    k = KATS["rms_norm_unit_weight"]
    out = orc.rms_norm(k["x"], k["weight"], k["eps"])
    assert np.all(np.abs(out - np.array(k["expected"], np.float32)) < k["abs_tol"])
    k = KATS["rms_norm_weighted"]
    out = orc.rms_norm(k["x"], k["weight"], k["eps"])
    assert np.all(np.abs(out - np.array(k["expected"], np.float32)) < k["abs_tol"])
    k = KATS["rms_norm_unweighted"]
    out = orc.rms_norm(k["x"], None, k["eps"])
    assert abs(out[0] - k["expected_first"]) < k["abs_tol"]
    k = KATS["rms_norm_weight_length_mismatch_is_error"]
    with pytest.raises(orc.OracleError, match="invalid RMS norm inputs"):
        orc.rms_norm(k["x"], k["weight"], 0.0)


def test_rms_norm_output_has_unit_rms():
    x = np.random.default_rng(3).standard_normal(512).astype(np.float32) * 7.5
    y = orc.rms_norm(x, None, 0.0)
    assert abs(math.sqrt(float(np.mean(y.astype(np.float64) ** 2))) - 1.0) < 1e-6


def test_dot_f32_matches_f64_sum():
    k = KATS["dot_f32_vs_f64_sum"]
    for n in k["lengths"]:
        i = np.arange(n, dtype=np.float32)
        a = np.sin(i * np.float32(k["a_step"])).astype(np.float32)
        b = np.cos(i * np.float32(k["b_step"])).astype(np.float32)
        expected = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
        assert abs(orc.dot_f32(a, b) - expected) < k["abs_tol"], n


def test_softmax_known_answer_and_invariants():
    k = KATS["softmax_1_2"]
    out = orc.softmax_f32(k["x"])
    assert np.all(np.abs(out - np.array(k["expected"], np.float32)) < k["abs_tol"])
    x = np.random.default_rng(5).standard_normal(300).astype(np.float32) * 20
    p = orc.softmax_f32(x)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    assert np.allclose(orc.softmax_f32(x + np.float32(13.0)), p, rtol=1e-4, atol=1e-7)
    with pytest.raises(orc.OracleError, match="non-empty"):
        orc.softmax_f32(np.zeros(0, np.float32))
    with pytest.raises(orc.OracleError, match="not finite"):
        orc.softmax_f32(np.array([1.0, np.nan], np.float32))
    with pytest.raises(orc.OracleError, match="not finite"):
        orc.softmax_f32(np.array([1.0, np.inf], np.float32))
    with pytest.raises(orc.OracleError, match="not finite"):
        orc.softmax_f32(np.array([-np.inf, -np.inf], np.float32))
    assert np.allclose(orc.softmax_f32(np.array([0.0, -np.inf], np.float32)), [1.0, 0.0])


def test_rope_known_answers():
    k = KATS["rope_pos1_base1_dims2"]
    x = orc.rope_neox(k["x"], k["position"], k["base"], k["n_rot"])
    assert abs(x[0] - math.cos(1.0)) < k["abs_tol"] and abs(x[1] - math.sin(1.0)) < k["abs_tol"]
    k = KATS["rope_neox_pairs_halves"]
    x = orc.rope_neox(k["x"], k["position"], k["base"], k["n_rot"])
    expected = [math.cos(2), math.cos(0.2), math.sin(2), math.sin(0.2), 7.0]
    assert np.all(np.abs(x - np.array(expected, np.float32)) < k["abs_tol"])
    assert x[4] == 7.0
    k = KATS["rope_neox_huge_factors"]
    x = orc.rope_neox(k["x"], k["position"], k["base"], k["n_rot"], k["freq_factors"])
    assert abs(x[0] - (math.cos(5) - 3 * math.sin(5))) < k["x0_abs_tol"]
    assert abs(x[1] - k["x1"]) < k["unrotated_abs_tol"] and abs(x[3] - k["x3"]) < k["unrotated_abs_tol"]
    with pytest.raises(orc.OracleError, match="invalid RoPE inputs"):
        orc.rope_neox([1.0, 2.0, 3.0], 1, 100.0, 3)
    with pytest.raises(orc.OracleError, match="invalid RoPE inputs"):
        orc.rope_neox([1.0, 2.0], 1, 0.0, 2)


def test_rope_rotates_each_pair_by_its_closed_form_angle():
    """Pair i of a d-wide head turns by pos * base^(-2i/d) / f_i; the f32
    recurrence drifts from the f64 closed form by well under 1e-3 rad."""
    d, pos, base = 512, 4095, 1e6
    f = np.random.default_rng(9).uniform(1, 8, d // 2).astype(np.float32)
    x = np.zeros(d, np.float32)
    x[: d // 2] = 1.0  # unit vector on each pair's first axis
    y = orc.rope_neox(x, pos, base, d, f).astype(np.float64)
    got = np.arctan2(y[d // 2:], y[: d // 2])
    want = pos * base ** (-2.0 * np.arange(d // 2) / d) / f.astype(np.float64)
    diff = np.angle(np.exp(1j * (got - want)))
    assert np.max(np.abs(diff)) < 1e-3
    # each pair keeps its norm
    z = np.random.default_rng(10).standard_normal(d).astype(np.float32)
    w = orc.rope_neox(z, pos, base, d, f).astype(np.float64)
    n0 = np.hypot(z[: d // 2], z[d // 2:])
    n1 = np.hypot(w[: d // 2], w[d // 2:])
    assert np.max(np.abs(n0 - n1)) < 1e-5
    # position 0 is the identity
    assert np.array_equal(orc.rope_neox(z, 0, base, d, f), z)


# ------------------------------------------------------------------ policies
def test_e2b_layer_kinds_head_dims_and_windows():
    hp = KATS["e2b_hyperparams"]
    glob = [l for l in range(hp["n_layers"]) if orc.layer_attention_kind(hp["n_layers"], l) == "global"]
    assert glob == KATS["e2b_layer_kinds"]["global_layers"]
    for layer, d in KATS["e2b_head_dims"]["head_dim"].items():
        assert orc.head_dim(hp["n_layers"], int(layer), hp["head_dim_local"], hp["head_dim_global"]) == d
    w = KATS["windowed_len_1000_512"]
    assert orc.windowed_len(w["seq_len"], w["window"]) == range(*w["range"])
    assert orc.windowed_len(3, 512) == range(0, 3)


def test_e2b_kv_sources_and_errors():
    n = KATS["e2b_hyperparams"]["n_layers"]
    shared = KATS["e2b_hyperparams"]["shared_kv_layers"]
    k = KATS["e2b_kv_sources"]
    for layer in range(n):
        src = orc.kv_source_layer(n, shared, layer)
        if layer in k["owners"]:
            assert src == layer
        else:
            kind = orc.layer_attention_kind(n, layer)
            assert src == (k["shared_global_source"] if kind == "global" else k["shared_local_source"])
    msgs = {
        "LayerOutOfRange": "must be within n_layers",
        "TooManySharedLayers": "leave no layer",
        "NoEarlierLayerOfSameKind": "no earlier layer of the same attention kind",
    }
    for case in KATS["kv_source_errors"]["cases"]:
        with pytest.raises(orc.OracleError, match=msgs[case["error"]]):
            orc.kv_source_layer(n, case["shared_kv_layers"], case["layer"])
    syn = KATS["synthetic_model_kv_sharing"]
    assert [orc.kv_source_layer(syn["n_layers"], syn["shared_kv_layers"], l) for l in range(syn["n_layers"])] == \
        syn["kv_sources"]


def test_proportional_rope_freq_factors_closed_form():
    k = KATS["proportional_rope_freq_factors_512_025"]
    f = orc.proportional_rope_freq_factors(k["head_dim"], k["p"])
    assert f.size == k["ones"] + k["frozen"]
    assert np.all(f[: k["ones"]] == 1.0) and np.all(f[k["ones"]:] == np.float32(k["frozen_value"]))


# ------------------------------------------------------------------ KvCache
def test_kv_cache_scalar_fixture_and_errors():
    k = KATS["kv_cache_scalar_fixture"]
    cache = orc.KvCache()
    outs = []
    for t in range(3):
        cache.append(0, [k["ks"][t]], [k["vs"][t]])
        ks, vs = cache.view(0, t + 1)
        acc = 0.0
        for i in range(t + 1):
            acc += (k["qs"][t] * float(ks[i, 0])) * float(vs[i, 0])
        outs.append(acc)
    assert np.allclose(outs, k["toy_outputs"], atol=k["abs_tol"])
    empty = orc.KvCache()
    with pytest.raises(orc.OracleError, match="layer 0 has no cached K/V"):
        empty.view(KATS["kv_view_missing_layer"]["layer"], KATS["kv_view_missing_layer"]["len"])
    assert empty.view(3, 0)[0].shape[0] == 0
    with pytest.raises(orc.OracleError, match="context length 4 exceeds configured max 3"):
        cache.view(0, 4)
    cache.append(2, [1.0], [2.0])  # creates layers 0..2; layer 1 exists but is empty
    with pytest.raises(orc.OracleError, match="context length 1 exceeds configured max 0"):
        cache.view(1, 1)


# ------------------------------------------------------------------ attention
def f64_attention(q, K, V, n_heads, n_kv, scale=1.0):
    """softmax(q.K^T * scale).V per head in f64 (textbook form, numpy)."""
    d = q.size // n_heads
    T = K.shape[0]
    K3 = K.astype(np.float64).reshape(T, n_kv, d)
    V3 = V.astype(np.float64).reshape(T, n_kv, d)
    out = np.zeros((n_heads, d))
    for h in range(n_heads):
        kv = h * n_kv // n_heads
        s = K3[:, kv, :] @ q.astype(np.float64)[h * d:(h + 1) * d] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ V3[:, kv, :]
    return out.reshape(-1)


@pytest.mark.parametrize("n_heads,n_kv,d,T,scale", [(8, 1, 16, 9, 0.7), (4, 2, 8, 5, 0.7), (2, 2, 16, 16, 0.7),
                                                    (8, 1, 256, 64, 0.7), (8, 1, 256, 64, 8.0)])
def test_attend_matches_f64_brute_force(n_heads, n_kv, d, T, scale):
    rng = np.random.default_rng(n_heads * 100 + T)
    q = rng.standard_normal(n_heads * d).astype(np.float32)
    K = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    V = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    out = orc.attend(q, K, V, n_heads, n_kv, scale)
    ref = f64_attention(q, K, V, n_heads, n_kv, scale)
    # Unnormalised inputs at scale 8 give scores of several hundred, where f32
    # rounding of the score alone moves the weights by ~1e-5.
    assert np.max(np.abs(out - ref)) < (1e-5 if scale < 1 else 1e-4)
    assert np.max(np.abs(orc.attend_f64(q, K, V, n_heads, n_kv, scale) - ref)) < 1e-12
    assert np.array_equal(orc.attend_rows(q, K, V, n_heads, n_kv, scale, threads=1), out)
    assert np.array_equal(orc.attend_rows(q, K, V, n_heads, n_kv, scale, threads=0), out)


def test_attend_closed_forms():
    rng = np.random.default_rng(1)
    n_heads, n_kv, d = 4, 2, 8
    q = rng.standard_normal(n_heads * d).astype(np.float32)
    # one row: every head returns its KV head's value row
    K = rng.standard_normal((1, n_kv * d)).astype(np.float32)
    V = rng.standard_normal((1, n_kv * d)).astype(np.float32)
    out = orc.attend(q, K, V, n_heads, n_kv).reshape(n_heads, d)
    for h in range(n_heads):
        kv = h * n_kv // n_heads  # heads 0,1 -> KV head 0; heads 2,3 -> KV head 1
        assert np.array_equal(out[h], V[0, kv * d:(kv + 1) * d])
    # equal keys: the mean of the value rows
    T = 6
    K = np.tile(rng.standard_normal((1, n_kv * d)).astype(np.float32), (T, 1))
    V = rng.standard_normal((T, n_kv * d)).astype(np.float32)
    out = orc.attend(q, K, V, n_heads, n_kv).reshape(n_heads, d)
    for h in range(n_heads):
        kv = h * n_kv // n_heads
        assert np.allclose(out[h], V[:, kv * d:(kv + 1) * d].mean(0), atol=1e-6)
    # a dominant score selects its row
    K = np.zeros((T, n_kv * d), np.float32)
    K[3] = 50.0 * np.sign(np.concatenate([q[:d], q[2 * d:3 * d]]))
    out = orc.attend(q, K, V, n_heads, n_kv).reshape(n_heads, d)
    assert np.allclose(out[0], V[3, :d], atol=1e-6) and np.allclose(out[2], V[3, d:], atol=1e-6)


def test_attend_failures_match_the_reference():
    q = np.ones(16, np.float32)
    K = np.ones((3, 2), np.float32)
    V = np.ones((3, 2), np.float32)
    with pytest.raises(orc.OracleError, match="softmax input is not finite"):
        orc.attend(q, np.zeros((0, 2), np.float32), np.zeros((0, 2), np.float32), 8, 1)
    qn = q.copy()
    qn[3] = np.nan
    with pytest.raises(orc.OracleError, match="softmax input is not finite"):
        orc.attend(qn, K, V, 8, 1)
    Ki = K.copy()
    Ki[1, 0] = np.inf
    with pytest.raises(orc.OracleError, match="softmax input is not finite"):
        orc.attend(q, Ki, V, 8, 1)
    # a -inf score just gets zero weight
    Km = K.copy()
    Km[1, 0] = -np.inf
    out = orc.attend(q, Km, V, 8, 1)
    assert np.all(np.isfinite(out))


@pytest.mark.parametrize("n_heads,n_kv,d,pos0,N,window", [(4, 2, 8, 0, 24, 0), (4, 2, 8, 7, 20, 5),
                                                        (8, 1, 16, 3, 30, 8), (8, 1, 16, 0, 12, 1)])
def test_attend_prefill_is_the_token_loop(n_heads, n_kv, d, pos0, N, window):
    """or_attend_prefill (the prompt run one token at a time, generate.rs:37-41)
    equals attend over each query's range, bit for bit, on any thread count;
    the range [p+1-W or 0, p+1) is the decode's (eng/mod.rs:10-36), and a
    NaN key fails exactly the queries that attend its row."""
    rng = np.random.default_rng(pos0 * 31 + N + window)
    q = rng.standard_normal((N, n_heads * d)).astype(np.float32)
    K = rng.standard_normal((pos0 + N, n_kv * d)).astype(np.float32)
    V = rng.standard_normal((pos0 + N, n_kv * d)).astype(np.float32)
    out, status = orc.attend_prefill(q, K, V, pos0, window, n_heads, n_kv, threads=1)
    assert not status.any()
    for i in range(N):
        p = pos0 + i
        b = max(0, p + 1 - window) if window else 0
        assert np.array_equal(out[i], orc.attend(q[i], K[b:p + 1], V[b:p + 1], n_heads, n_kv)), i
        assert np.max(np.abs(out[i] - f64_attention(q[i], K[b:p + 1], V[b:p + 1], n_heads, n_kv, 1.0))) < 1e-5
    out3, status3 = orc.attend_prefill(q, K, V, pos0, window, n_heads, n_kv, threads=3)
    assert np.array_equal(out3, out) and not status3.any()
    # NaN in key row r: queries at positions p >= r whose window still holds r fail.
    r = pos0 + N // 2
    Kb = K.copy()
    Kb[r, 0] = np.nan
    _, st = orc.attend_prefill(q, Kb, V, pos0, window, n_heads, n_kv, threads=2)
    for i in range(N):
        p = pos0 + i
        sees = r <= p and (window == 0 or r > p - window)
        assert bool(st[i]) == sees, (i, st[i])


@pytest.mark.parametrize("n_heads,n_kv,d,pos0,N,window", [(8, 1, 32, 200, 37, 0), (8, 1, 32, 130, 29, 100),
                                                        (4, 2, 16, 0, 70, 0), (8, 1, 16, 61, 9, 1)])
def test_blocked_prefill_is_the_token_loop(n_heads, n_kv, d, pos0, N, window):
    """or_attend_prefill_blocked (the checker's fast loop nest: groups of 4
    queries walking 64-key chunks together) equals or_attend_prefill bit for
    bit -- outputs, statuses and the untouched heads of a failing query --
    on ranges that cross chunk and group edges, on any thread count."""
    rng = np.random.default_rng(pos0 + 7 * N + window)
    q = rng.standard_normal((N, n_heads * d)).astype(np.float32)
    K = rng.standard_normal((pos0 + N, n_kv * d)).astype(np.float32)
    V = rng.standard_normal((pos0 + N, n_kv * d)).astype(np.float32)
    ref, st = orc.attend_prefill(q, K, V, pos0, window, n_heads, n_kv, threads=1, blocked=False)
    for threads in (1, 3):
        out, st2 = orc.attend_prefill(q, K, V, pos0, window, n_heads, n_kv, threads=threads, blocked=True)
        assert np.array_equal(out.view(np.uint32), ref.view(np.uint32)) and np.array_equal(st, st2)
    # A NaN key row and a +inf value row: the same failing queries, the same
    # bits everywhere else (NaN outputs included).
    r = pos0 + N // 2
    Kb, Vb = K.copy(), V.copy()
    Kb[r, 1] = np.nan
    Vb[r - 1, 0] = np.inf
    ref, st = orc.attend_prefill(q, Kb, Vb, pos0, window, n_heads, n_kv, threads=2, blocked=False)
    out, st2 = orc.attend_prefill(q, Kb, Vb, pos0, window, n_heads, n_kv, threads=2, blocked=True)
    assert np.array_equal(st, st2) and st.any()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    # A sample of the rows at their own positions: the same bits as the chunk.
    pick = np.arange(1, N, 3)
    out_s, st_s = orc.attend_prefill(q[pick], Kb, Vb, 0, window, n_heads, n_kv, threads=2, positions=pos0 + pick)
    assert np.array_equal(st_s, st[pick]) and np.array_equal(out_s.view(np.uint32), ref[pick].view(np.uint32))


def test_optimised_build_is_bit_identical(tmp_path):
    """The shipped oracle (-O3 -march=x86-64-v3, vectorised) gives the same
    bits as an -O0 build of the same sources: without -ffast-math the
    compiler may not reassociate a sum or fuse a product, so vectorising
    the 16-lane dot and the elementwise loops changes no result."""
    root = os.path.dirname(HERE)
    so = tmp_path / "liboracle_O0.so"
    subprocess.run(["gcc", "-O0", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-o", str(so),
                    os.path.join(root, "oracle", "g4_oracle.c"), os.path.join(root, "oracle", "g4_oracle_matvec.c"),
                    "-lm", "-lpthread"], check=True)
    script = """
import sys, numpy as np
sys.path.insert(0, sys.argv[1])
from oracle import pyoracle as orc
rng = np.random.default_rng(5)
q = rng.standard_normal((24, 8 * 40)).astype(np.float32)
K = rng.standard_normal((90, 40)).astype(np.float32)
V = rng.standard_normal((90, 40)).astype(np.float32)
x = rng.standard_normal(300).astype(np.float32)
outs = [orc.attend(q[0], K[:77], V[:77], 8, 1), orc.attend_prefill(q, K, V, 66, 0, 8, 1, threads=2)[0],
        orc.attend_prefill(q, K, V, 66, 9, 8, 1, threads=2, blocked=False)[0],
        orc.rms_norm(x, None, 1e-6), orc.rope_neox(x[:64].copy(), 37, 10000.0, 64),
        np.array([orc.dot_f32(x[:141], x[141:282])], np.float32), orc.softmax_f32(x[:50])]
np.savez(sys.argv[2], *outs)
"""
    res = {}
    for name, lib in (("O0", str(so)), ("O3", os.path.join(root, "oracle", "liboracle.so"))):
        npz = tmp_path / f"{name}.npz"
        subprocess.run([sys.executable, "-c", script, root, str(npz)], env=dict(os.environ, G4_ORACLE_LIB=lib),
                       check=True)
        z = np.load(npz)
        res[name] = [z[k] for k in sorted(z.files, key=lambda f: int(f.split("_")[1]))]
    for a, b in zip(res["O0"], res["O3"]):
        assert a.dtype == np.float32 and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_layer_attention_segment_matches_its_parts():
    """or_layer_attention (model.rs:386-411) equals norm -> rope -> append ->
    view -> window -> attend done by hand, and reports the attended set."""
    hp = orc.Hparams(7, 4, 2, 8, 16, 8, 2, 10000.0, 1000000.0, 1e-6)  # synthetic_generate.rs:12-34
    rng = np.random.default_rng(4)
    freqs = orc.proportional_rope_freq_factors(16, 0.25)
    cache = orc.KvCache()
    manual = {}
    for pos in range(12):
        for layer in range(7):
            glob = orc.layer_attention_kind(7, layer) == "global"
            d = 16 if glob else 8
            q = rng.standard_normal(4 * d).astype(np.float32)
            k = rng.standard_normal(2 * d).astype(np.float32)
            v = rng.standard_normal(2 * d).astype(np.float32)
            wq = rng.uniform(0.5, 1.5, d).astype(np.float32)
            wk = rng.uniform(0.5, 1.5, d).astype(np.float32)
            out, src, rng_kv, qn, kn, vn = cache.layer_attention(hp, layer, pos, q, k, v, wq, wk,
                                                                 freqs if glob else None)
            base = 1e6 if glob else 1e4
            qh = orc.rope_heads(orc.norm_heads(q, d, wq, 1e-6), d, pos, base, freqs if glob else None)
            assert np.array_equal(qh, qn)
            expect_src = orc.kv_source_layer(7, 2, layer)
            assert src == expect_src
            if src == layer:
                kh = orc.rope_heads(orc.norm_heads(k, d, wk, 1e-6), d, pos, base, freqs if glob else None)
                manual.setdefault(layer, ([], []))
                manual[layer][0].append(kh)
                manual[layer][1].append(orc.norm_heads(v, d, None, 1e-6))
            assert rng_kv == (range(0, pos + 1) if glob else orc.windowed_len(pos + 1, 8))
            Ks = np.array(manual[src][0])[rng_kv.start:rng_kv.stop]
            Vs = np.array(manual[src][1])[rng_kv.start:rng_kv.stop]
            assert np.array_equal(out, orc.attend(qh, Ks, Vs, 4, 2))


# ------------------------------------------------------------- planted bugs
PLANTS = {
    "G4_PLANT_GQA_MAP": "test_attend_closed_forms",
    "G4_PLANT_WINDOW": "test_e2b_layer_kinds_head_dims_and_windows",
    "G4_PLANT_ROPE_SIGN": "test_rope_known_answers",
    "G4_PLANT_RMS_WEIGHT_SHIFT": "test_rms_norm_known_answers",
    "G4_PLANT_PV_STRIDE": "test_attend_closed_forms",
    "G4_PLANT_SOFTMAX_NO_MAX": "test_attend_matches_f64_brute_force",
    "G4_PLANT_KV_SOURCE": "test_e2b_kv_sources_and_errors",
}


@pytest.mark.parametrize("plant", sorted(PLANTS))
def test_planted_mistakes_are_caught(plant, tmp_path):
    """Each plausible mistake, planted in a copy of the oracle, fails a check above."""
    root = os.path.dirname(HERE)
    so = tmp_path / "liboracle.so"
    subprocess.run(["gcc", "-O1", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", f"-D{plant}",
                    "-o", str(so), os.path.join(root, "oracle", "g4_oracle.c"),
                    os.path.join(root, "oracle", "g4_oracle_matvec.c"), "-lm", "-lpthread"], check=True)
    env = dict(os.environ, G4_ORACLE_LIB=str(so))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                        f"{__file__}::{PLANTS[plant]}"], env=env, cwd=root, capture_output=True, text=True)
    assert r.returncode != 0, f"{plant} was not caught by {PLANTS[plant]}:\n{r.stdout[-2000:]}"
