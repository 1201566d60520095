"""The C-ABI library loads, exports every entry point include/g4attn.h
declares, and its host-side policy functions agree with the reference's
known answers.  No GPU is touched here."""
import json
import os
import re

import pytest

import g4hip
from oracle import pyoracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def declared_functions():
    text = open(g4hip.HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(g4_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_entry_point():
    lib = g4hip.lib()
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding knows every one of them
    assert set(names) <= set(g4hip._SIGS), set(names) - set(g4hip._SIGS)


def test_policies_match_reference_known_answers():
    hp = KATS["e2b_hyperparams"]
    n = hp["n_layers"]
    glob = [l for l in range(n) if g4hip.layer_attention_kind(n, l) == "global"]
    assert glob == KATS["e2b_layer_kinds"]["global_layers"]
    for layer in range(n):
        assert g4hip.kv_source_layer(n, hp["shared_kv_layers"], layer) == orc.kv_source_layer(
            n, hp["shared_kv_layers"], layer)
    syn = KATS["synthetic_model_kv_sharing"]
    assert [g4hip.kv_source_layer(syn["n_layers"], syn["shared_kv_layers"], l)
            for l in range(syn["n_layers"])] == syn["kv_sources"]
    w = KATS["windowed_len_1000_512"]
    assert g4hip.windowed_len(w["seq_len"], w["window"]) == range(*w["range"])
    k = KATS["proportional_rope_freq_factors_512_025"]
    f = g4hip.proportional_rope_freq_factors(k["head_dim"], k["p"])
    assert f == list(orc.proportional_rope_freq_factors(k["head_dim"], k["p"]))


def test_kv_share_errors_carry_the_reference_messages():
    n = KATS["e2b_hyperparams"]["n_layers"]
    for case in KATS["kv_source_errors"]["cases"]:
        with pytest.raises(g4hip.EngError) as err:
            g4hip.kv_source_layer(n, case["shared_kv_layers"], case["layer"])
        with pytest.raises(orc.OracleError) as ref:
            orc.kv_source_layer(n, case["shared_kv_layers"], case["layer"])
        assert err.value.kind == "Compute"  # model.rs:398 maps KvShareError to Compute
        assert err.value.message == ref.value.message


def test_product_does_not_reference_the_oracle():
    """The HIP library and its binding never load or call the oracle."""
    root = os.path.dirname(HERE)
    pkg = os.path.join(root, "gemma4-rs_amd")
    for dirpath, _, files in os.walk(pkg):
        for f in files:
            if f.endswith((".hip", ".h", ".py", ".cpp")) or f == "Makefile":
                text = open(os.path.join(dirpath, f)).read()
                assert "oracle" not in text.lower(), os.path.join(dirpath, f)
    data = open(g4hip.LIB_PATH, "rb").read()
    assert b"liboracle" not in data and b"or_attend" not in data
