"""Writes reference_kats.json: the known-answer vectors of gemma4-rs's own tests
for the attention path, read out of the cited test lines.

Run in a container that has the gemma4-rs checkout at /root/reference:

    python tests/golden/extract_reference_kats.py

Each entry records the file:line it was read from.  Only numbers and integer
tables are taken (data, not code); the expected values are copied verbatim
from the literal in the cited line, so the fixture can be re-derived and
diffed whenever the reference changes.
"""
import json
import os
import re
import sys

REF = os.environ.get("G4_REFERENCE_ROOT", "/root/reference")
HERE = os.path.dirname(os.path.abspath(__file__))

NUM = r"-?\d[\d_]*(?:\.[\d_]+)?(?:e-?\d+)?"


def line(path, lineno):
    with open(os.path.join(REF, path)) as f:
        return f.read().splitlines()[lineno - 1]


def num(text):
    """A Rust float/int literal (`0.848_528_15`, `1.0_f32`, `2_048`) as float."""
    text = re.sub(r"_?f(32|64)$", "", text.strip())
    return float(text.replace("_", ""))


def lists(path, lineno):
    """Every `[a, b, ...]` literal on the cited line, as lists of floats."""
    out = []
    for body in re.findall(r"\[([^\[\]]*)\]", line(path, lineno)):
        items = [x for x in body.split(",") if x.strip()]
        if items and all(re.fullmatch(NUM + r"(_?f(32|64))?", x.strip()) for x in items):
            out.append([num(x) for x in items])
    return out


def expected_tol(path, lineno):
    """(expected, tolerance) from an `(x - EXPECTED).abs() < TOL` assertion."""
    m = re.search(r"- (" + NUM + r")\)\.abs\(\) < (" + NUM + r")", line(path, lineno))
    return num(m.group(1)), num(m.group(2))


def tol(path, lineno):
    """The last `< TOL` bound on the cited line."""
    return num(re.findall(r"< (" + NUM + r")", line(path, lineno))[-1])


def factor(path, lineno):
    """The `* STEP` multiplier of an `(i as f32 * STEP)` expression."""
    return num(re.search(r"as f32 \* (" + NUM + r")\)", line(path, lineno)).group(1))


def cite(path, lo, hi=None):
    return f"{path}:{lo}" + (f"-{hi}" if hi else "")


def main():
    ops = "crates/llm-backend-cpu/tests/ops_smoke.rs"
    lp = "crates/llm-gemma4/tests/layer_pattern.rs"
    idea = "crates/llm-gemma4/src/idea/mod.rs"
    syn = "crates/llm-gemma4/tests/synthetic_generate.rs"
    kvr = "crates/llm-eng/tests/kv_vs_recompute.rs"

    # Sanity: the cited lines still say what this script expects.
    assert "rms_norm_f32(&x, &weight, 0.0)" in line(ops, 40)
    assert "Some(&[2.0, 0.5])" in line(ops, 48)
    assert "for len in" in line(ops, 59)
    assert "softmax_f32(&a)" in line(ops, 90)
    assert "rope_f32(&mut values, 1, 1.0, 2)" in line(ops, 95)
    assert "rope_neox(&mut x, 2, 100.0, 4, None)" in line(ops, 104)
    assert "rope_neox(&mut x, 5, 100.0, 4, Some(&[1.0, 1e30]))" in line(ops, 116)
    assert "windowed_len(1000, 512)" in line(lp, 49)
    assert "2_048" in line(lp, 44)
    assert "let qs" in line(kvr, 15) and "let vs" in line(kvr, 17)
    assert "n_layers: 7" in line(syn, 16)

    kats = {
        "rms_norm_unit_weight": {
            "cite": cite(ops, 35, 44),
            "x": lists(ops, 37)[0], "weight": lists(ops, 38)[0], "eps": 0.0,
            "expected": [expected_tol(ops, 42)[0], expected_tol(ops, 43)[0]],
            "abs_tol": expected_tol(ops, 42)[1],
        },
        "rms_norm_weighted": {
            "cite": cite(ops, 46, 50),
            "x": lists(ops, 48)[0], "weight": lists(ops, 48)[1], "eps": 0.0,
            "expected": [expected_tol(ops, 49)[0], expected_tol(ops, 50)[0]],
            "abs_tol": expected_tol(ops, 49)[1],
        },
        "rms_norm_unweighted": {
            "cite": cite(ops, 52, 53),
            "x": lists(ops, 52)[0], "eps": 0.0,
            "expected_first": expected_tol(ops, 53)[0], "abs_tol": expected_tol(ops, 53)[1],
        },
        "rms_norm_weight_length_mismatch_is_error": {
            "cite": cite(ops, 54), "x": lists(ops, 54)[0], "weight": lists(ops, 54)[1],
        },
        "dot_f32_vs_f64_sum": {
            "cite": cite(ops, 57, 65),
            "lengths": [int(v) for v in lists(ops, 59)[0]],
            "a_step": factor(ops, 60), "b_step": factor(ops, 61),
            "a_fn": "sin", "b_fn": "cos", "abs_tol": tol(ops, 63),
        },
        "softmax_1_2": {
            "cite": cite(ops, 86, 92),
            "x": lists(ops, 86)[0],
            "expected": [expected_tol(ops, 91)[0], expected_tol(ops, 92)[0]],
            "abs_tol": expected_tol(ops, 91)[1],
        },
        "rope_pos1_base1_dims2": {
            "cite": cite(ops, 94, 97),
            "x": lists(ops, 94)[0], "position": 1, "base": 1.0, "n_rot": 2,
            "expected_fns": ["cos(1)", "sin(1)"], "abs_tol": tol(ops, 96),
        },
        "rope_neox_pairs_halves": {
            "cite": cite(ops, 100, 111),
            "x": lists(ops, 103)[0], "position": 2, "base": 100.0, "n_rot": 4,
            "expected_fns": ["cos(2)", "cos(0.2)", "sin(2)", "sin(0.2)", "7"],
            "abs_tol": tol(ops, 106),
        },
        "rope_neox_huge_factors": {
            "cite": cite(ops, 113, 119),
            "x": lists(ops, 115)[0], "position": 5, "base": 100.0, "n_rot": 4,
            "freq_factors": [1.0, 1e30],
            "x0_expected_fn": "cos(5) - 3*sin(5)", "x0_abs_tol": tol(ops, 117),
            "x1": 2.0, "x3": 4.0, "unrotated_abs_tol": tol(ops, 118),
        },
        "e2b_hyperparams": {
            "cite": cite(idea, 48, 68),
            "n_layers": 35, "vocab_size": 262144, "d_model": 1536, "n_heads": 8,
            "n_kv_heads": 1, "head_dim_local": 256, "head_dim_global": 512, "ple_dim": 256,
            "sliding_window": 512, "shared_kv_layers": 20, "local_rope_base": 10000.0,
            "global_p": 0.25, "global_rope_base": 1000000.0, "rms_norm_eps": 1e-6,
        },
        "e2b_layer_kinds": {
            "cite": cite(lp, 20, 34),
            "global_layers": [l for l in range(35) if l % 5 == 4],
            "rule": "global iff layer % 5 == 4 or layer == 34",
        },
        "e2b_head_dims": {
            "cite": cite(lp, 36, 45),
            "head_dim": {"0": 256, "4": 512, "34": 512},
            "q_width_local": int(num(line(lp, 44).split(",")[-1].strip(" );"))),
        },
        "windowed_len_1000_512": {
            "cite": cite(lp, 47, 52),
            "seq_len": 1000, "window": 512, "range": [488, 1000], "global_range": [0, 1000],
        },
        "e2b_kv_sources": {
            "cite": cite(lp, 54, 67),
            "owners": list(range(15)),
            "shared_local_source": 13, "shared_global_source": 14,
        },
        "kv_source_errors": {
            "cite": cite(lp, 69, 86),
            "cases": [
                {"shared_kv_layers": 20, "layer": 35, "error": "LayerOutOfRange"},
                {"shared_kv_layers": 35, "layer": 0, "error": "TooManySharedLayers"},
                {"shared_kv_layers": 31, "layer": 34, "error": "NoEarlierLayerOfSameKind"},
            ],
        },
        "synthetic_model_kv_sharing": {
            "cite": cite(syn, 12, 34),
            "n_layers": 7, "n_heads": 4, "n_kv_heads": 2, "head_dim_local": 8,
            "head_dim_global": 16, "sliding_window": 8, "shared_kv_layers": 2,
            "kv_sources": [0, 1, 2, 3, 4, 3, 4],
            "global_layers": [4, 6],
        },
        "kv_cache_scalar_fixture": {
            "cite": cite(kvr, 13, 35),
            "qs": lists(kvr, 15)[0], "ks": lists(kvr, 16)[0], "vs": lists(kvr, 17)[0],
            "toy_outputs": [0.5, -3.0, -1.5], "abs_tol": 1e-6,
        },
        "kv_view_missing_layer": {
            "cite": "crates/llm-eng/src/context_memory.rs:109-116",
            "layer": 0, "len": 1, "error": "MissingLayer",
        },
        "proportional_rope_freq_factors_512_025": {
            "cite": "crates/llm-gemma4/tests/e2b_smoke.rs:27-40; crates/llm-gemma4/src/idea/mod.rs:162-165",
            "head_dim": 512, "p": 0.25, "ones": 64, "frozen": 192, "frozen_value": 1e30,
        },
        "synthetic_generate_tolerance": {
            "cite": cite(syn, 74, 83),
            "relative_tol": 1e-4, "scale": "max(|a|, |b|, 1)",
        },
    }
    # The scalar fixture of kv_vs_recompute is reproduced from its own toy
    # attention (acc += (q*k)*v over the viewed prefix).
    qs, ks, vs = (kats["kv_cache_scalar_fixture"][k] for k in ("qs", "ks", "vs"))
    toy = []
    for t in range(3):
        acc = 0.0
        for i in range(t + 1):
            acc += (qs[t] * ks[i]) * vs[i]
        toy.append(acc)
    assert toy == kats["kv_cache_scalar_fixture"]["toy_outputs"], toy

    out = os.path.join(HERE, "reference_kats.json")
    with open(out, "w") as f:
        json.dump(kats, f, indent=1, sort_keys=True)
    print(f"wrote {out} ({len(kats)} entries)")


if __name__ == "__main__":
    sys.exit(main())
