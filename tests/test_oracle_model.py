"""Pins the oracle's orchestration (oracle/model.py) and the host-side tables.

The fixtures were written by tests/golden/make_golden.py from the reference's
own model.py / config.py / weights.py, driven over the same oracle C kernels,
so the oracle must reproduce them bit for bit: per-token logits, chunked
prefill, greedy and seeded-sampling streams, chosen experts and adaptive widths,
chosen blocks per head, and cache metadata.  The reference's own invariants
(tests/test_inference.py:52-69) are checked on top.
"""
import json

import numpy as np
import pytest

from miracle_hip import ModelConfig, presets, synthetic
from miracle_hip.weights import expected_shapes
from oracle.config import OracleConfig, inverse_frequencies, weight_shapes
from oracle.model import OracleModel


def _load(golden_dir, name):
    z = np.load(golden_dir / f"micro_{name}.npz")
    bundle = json.loads(str(z["bundle"]))
    weights = synthetic.micro_weights(bundle)
    scale = float(z["router_scale"])
    if scale:
        for k in list(weights):
            if ".router." in k and k.endswith(".weight"):
                weights[k] = (weights[k] * np.float32(scale)).astype(np.float32)
    return z, bundle, weights


def pytest_generate_tests(metafunc):
    if "variant" in metafunc.fixturenames:
        from conftest import GOLDEN
        metafunc.parametrize("variant", sorted(p.stem[len("micro_"):] for p in GOLDEN.glob("micro_*.npz")))


def _expert_log(trace):
    out = []
    for rec in trace:
        if rec[0] == "experts":
            out.append((rec[1], -1))
            out.extend((rec[1], e) for e in rec[3])
    return np.asarray(out, np.int64).reshape(-1, 2)


def _block_masks(trace, cfg, heads):
    lc = cfg.source["long_context"]
    masks = []
    for rec in trace:
        if rec[0] != "blocks":
            continue
        count = rec[2] + 1
        length = min(cfg.window, count)
        blocks = -(-count // lc["global_block_size"])
        m = np.zeros((heads, length + blocks), bool)
        m[:, :length] = True
        for h, chosen in enumerate(rec[3]):
            m[h, [length + b for b in chosen]] = True
        masks.append(m)
    return masks


def test_oracle_reproduces_reference_micro(golden_dir, variant):
    z, bundle, weights = _load(golden_dir, variant)
    ids = z["ids"]
    trace = []
    model = OracleModel(bundle, weights, context_length=32, trace=trace)
    logits = model.prefill(ids, return_all=True)
    np.testing.assert_array_equal(logits, z["logits"])
    cfg = model.cfg
    meta = json.loads(str(z["meta"]))
    if "ring_length" in meta:
        assert [s["ring"].length for s in model.layers] == meta["ring_length"]
        assert [s["ring"].start for s in model.layers] == meta["ring_start"]
    if "relay_count" in meta:
        assert [s["relay"]["count"] for s in model.layers] == meta["relay_count"]
    if "latent_rows" in meta:
        assert [s["latent"].shape[0] for s in model.layers] == meta["latent_rows"]
        assert [s["positions"] for s in model.layers] == meta["positions"]
        assert [s["counts"] for s in model.layers] == meta["counts"]
        assert [s["memory_size"] for s in model.layers] == meta["memory_size"]
    if "loop_counts" in meta:
        assert [[lp["ring"].count for lp in s["loops"]] for s in model.layers] == meta["loop_counts"]
    if cfg.family == "heavy-medium-2.0":
        np.testing.assert_array_equal(_expert_log(trace), z["experts"])
        ours = _block_masks(trace, cfg, cfg.query_heads)
        widths = z["block_mask_widths"]
        assert [m.shape[1] for m in ours] == widths.tolist()
        for i, m in enumerate(ours):
            np.testing.assert_array_equal(m, z["block_masks"][i, :, :widths[i]])
    model.reset()
    chunked = np.concatenate([model.prefill(ids[:5], return_all=True), model.prefill(ids[5:], return_all=True)])
    np.testing.assert_array_equal(chunked, z["chunked"])
    assert model.generate(list(ids[:4]), max_new_tokens=8) == z["greedy"].tolist()
    assert model.generate([1, 3], max_new_tokens=4, temperature=0.8, top_k=5, top_p=0.9, seed=7) == \
        z["sampled"].tolist()


def test_oracle_invariants_cache_bounds_and_decode_equals_prefill():
    # reference tests/test_inference.py:52-69
    bundle = presets.micro("flashnano-1.5")
    model = OracleModel(bundle, synthetic.micro_weights(bundle), context_length=12)
    ids = [1, 3, 5, 8, 2, 9, 11, 10, 9, 7, 6, 4]
    whole = model.prefill(ids, return_all=True)
    assert model.layers[0]["ring"].length == 4 and model.layers[1]["ring"].length == 12
    with pytest.raises(ValueError, match="context_length"):
        model.decode(1)
    assert model.position == 12
    model.reset()
    np.testing.assert_array_equal(np.stack([model.decode(i) for i in ids]), whole)
    model.reset()
    for bad in ([32], [-1], [1.5], [[1]], [], [True]):
        with pytest.raises(ValueError):
            model.prefill(bad)
        assert model.position == 0


def test_oracle_workload_tiny(golden_dir):
    z = np.load(golden_dir / "workload_flashnano-1.5-tiny.npz")
    wl = presets.workload("flashnano-1.5-tiny")
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    np.testing.assert_array_equal(z["prompt"], synthetic.prompt_ids(4096, 32, wl["seed"]))
    model = OracleModel(wl["config"], weights, context_length=wl["context"])
    np.testing.assert_array_equal(model.prefill(z["prompt"]), z["last_logits"])
    assert model.generate(list(z["prompt"]), max_new_tokens=16) == z["greedy"].tolist()


def test_rope_tables_match_reference(golden_dir):
    cases = json.loads((golden_dir / "rope_cases.json").read_text())
    tables = np.load(golden_dir / "rope_tables.npz")
    for name, bundle in cases.items():
        np.testing.assert_array_equal(inverse_frequencies(OracleConfig.from_bundle(bundle)), tables[name], name)
        np.testing.assert_array_equal(ModelConfig.from_dict(bundle).inverse_frequencies(), tables[name], name)


def test_rope_table_closed_form():
    cfg = OracleConfig.from_bundle(presets.workload("flashnano-1.7")["config"])
    inv = inverse_frequencies(cfg)
    np.testing.assert_allclose(inv, 5e5 ** (-np.arange(0, 128, 2) / 128), rtol=2e-6)


def test_shape_tables_match_reference(golden_dir):
    shapes = json.loads((golden_dir / "shapes.json").read_text())
    for family, items in shapes.items():
        want = [(k, tuple(v)) for k, v in items]
        bundle = presets.micro(family)
        assert list(expected_shapes(ModelConfig.from_dict(bundle)).items()) == want
        assert list(weight_shapes(OracleConfig.from_bundle(bundle)).items()) == want


def test_native_configs_parse_like_reference(golden_dir):
    parsed = json.loads((golden_dir / "configs.json").read_text())
    for name, case in parsed.items():
        got = ModelConfig.from_dict(case["input"]).to_dict()
        got["global_layers"] = list(got["global_layers"])
        assert json.loads(json.dumps(got)) == case["parsed"], name
