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


def test_oracle_seat_matches_a_prefilled_model():
    # seat() stands a model at a position without running the prompt (timing of
    # decode steps at long positions); with the rings' rows replaced by those a
    # real prefill left, the next decode must be the prefilled model's, bit for
    # bit (ring count, start and position agree, also for a wrapped local ring).
    bundle = presets.micro("flashnano-1.5")
    weights = synthetic.micro_weights(bundle)
    ids = [1, 3, 5, 8, 2, 9, 11, 10, 9]
    real = OracleModel(bundle, weights, context_length=12)
    real.prefill(ids[:8])
    seated = OracleModel(bundle, weights, context_length=12)
    seated.seat(8, seed=3)
    assert seated.position == 8
    for a, b in zip(real.layers, seated.layers):
        assert (a["ring"].count, a["ring"].length, a["ring"].start) == (b["ring"].count, b["ring"].length,
                                                                        b["ring"].start)
        assert np.all(b["ring"].k[:b["ring"].length] != 0)
        b["ring"].k[:] = a["ring"].k
        b["ring"].v[:] = a["ring"].v
    np.testing.assert_array_equal(seated.decode(ids[8]), real.decode(ids[8]))
    with pytest.raises(ValueError):
        seated.seat(12)
    latent = presets.micro("flashnano-1.6")
    with pytest.raises(ValueError, match="beyond the K/V rings"):
        OracleModel(latent, synthetic.micro_weights(latent), context_length=12).seat(4)



@pytest.mark.parametrize("family", ["flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlighting-2.0"])
def test_oracle_bf16_bits_equal_widened_weights(family):
    """The oracle holds BF16 matrices as bits and widens them where it uses
    them; given the same weights already widened to FP32 it must compute the
    same logits.  (flashnano-1.6 reads its learned CBR queries through an
    RMSNorm rather than a projection: unwidened bits there are integers and
    the relay rows come out wrong.)"""
    config = dict(presets.micro(family), hidden_size=64, query_heads=4, kv_heads=2, head_dim=16, ffn_dim=96,
                  vocab_size=64, max_positions=64)
    if family == "flashnano-1.6":
        config.update(cbr_chunk_size=4, cbr_slots=2)
    if family == "flashlighting-2.0":
        config.update(latent_dim=16)
    weights = synthetic.synthetic_weights(config, 23, "bf16")
    bits = {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()}
    wide = {k: ((v.astype(np.uint32) << 16).view(np.float32) if v.dtype == np.uint16 else v) for k, v in bits.items()}
    assert any(v.dtype == np.uint16 and v.ndim == 2 for v in bits.values())
    ids = synthetic.prompt_ids(64, 20, 23)
    got = OracleModel(config, bits, context_length=32).prefill(ids, return_all=True)
    want = OracleModel(config, wide, context_length=32).prefill(ids, return_all=True)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)

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


# A heavy-medium-2.0 geometry with a real block choice (7 blocks, 3 kept) and
# adaptive width 2..4 over 16 experts.
_FOLLOW = {"family": "heavy-medium-2.0", "vocab_size": 64, "hidden_size": 32, "layers": 2, "query_heads": 4,
           "kv_heads": 2, "head_dim": 8, "ffn_dim": 16, "max_positions": 64, "window": 8, "latent_dim": 8,
           "inner_loop_steps": 2, "rope_theta": 1000000.0,
           "source": {"routed_experts": 16, "router_groups": 4, "router_top_k_max": 4, "router_top_k_min": 2,
                      "shared_experts": 1, "router_temperature": 1.0,
                      "long_context": {"global_block_size": 4, "global_slots": 3, "rope_local_fraction": 0.6,
                                       "alibi_slope_scale": 0.015}},
           "backend_format": 1}


def follow_record(trace, cfg, positions):
    """The oracle's own choices in the device's record layout
    (mr_model_choices): width, experts in chosen order, blocks per head."""
    s = cfg.source
    kmax, slots = s["router_top_k_max"], s["long_context"]["global_slots"]
    rec = np.full((positions, cfg.layers, cfg.inner_loop_steps, 1 + kmax + cfg.query_heads * slots), -1, np.int32)
    blocks = [r for r in trace if r[0] == "blocks"]
    experts = [r for r in trace if r[0] == "experts"]
    i = 0
    for pos in range(positions):
        for layer in range(cfg.layers):
            for loop in range(cfg.inner_loop_steps):
                b, e = blocks[i], experts[i]
                assert (b[1], b[2], e[1], e[2]) == (layer, pos, layer, pos)
                r = rec[pos, layer, loop]
                r[0] = e[4]
                r[1:1 + e[4]] = e[3]
                for h, chosen in enumerate(b[3]):
                    r[1 + kmax + h * slots: 1 + kmax + h * slots + len(chosen)] = chosen
                i += 1
    return rec


def _follow_setup():
    weights = synthetic.synthetic_weights(_FOLLOW, 5, "bf16")
    weights = {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()}
    ids = synthetic.prompt_ids(64, 40, 5)
    trace = []
    base = OracleModel(_FOLLOW, weights, context_length=64, trace=trace)
    logits = base.prefill(ids, return_all=True)
    return weights, ids, logits, trace, base.cfg


def test_oracle_follow_own_choices_changes_nothing():
    weights, ids, logits, trace, cfg = _follow_setup()
    rec = follow_record(trace, cfg, len(ids))
    assert (rec[:, :, :, 1 + 4:] >= 0).sum() > 0
    model = OracleModel(_FOLLOW, weights, context_length=64, follow=rec)
    np.testing.assert_array_equal(model.prefill(ids, return_all=True), logits)
    assert model.adopted == [] and model.mismatches == []


def test_oracle_follow_rejects_a_wrong_choice_and_adopts_a_near_tie():
    weights, ids, logits, trace, cfg = _follow_setup()
    rec = follow_record(trace, cfg, len(ids))
    # an expert outside the top-k at position 20, layer 1, loop 0 (a planted wrong routing)
    r = rec[20, 1, 0]
    experts = [r for r in trace if r[0] == "experts" and r[1] == 1 and r[2] == 20][0]
    outsider = next(e for e in range(16) if e not in experts[3])
    r[1] = outsider
    wrong = OracleModel(_FOLLOW, weights, context_length=64, follow=rec)
    np.testing.assert_array_equal(wrong.prefill(ids, return_all=True), logits)   # keeps its own choice
    assert [m[:4] for m in wrong.mismatches] == [("experts", 1, 20, 0)] and wrong.adopted == []
    # a swapped pair of blocks for one head (a planted wrong block choice)
    rec = follow_record(trace, cfg, len(ids))
    b = rec[30, 0, 1, 1 + 4: 1 + 4 + 3]
    blocks_now = -(-31 // 4)
    b[0] = next(x for x in range(blocks_now) if x not in b)
    wrong = OracleModel(_FOLLOW, weights, context_length=64, follow=rec)
    wrong.prefill(ids, return_all=True)
    assert [m[:5] for m in wrong.mismatches] == [("blocks", 0, 30, 1, 0)]
    # with a tolerance wide enough to call it a near-tie, the same choice is adopted
    loose = OracleModel(_FOLLOW, weights, context_length=64, follow=rec)
    loose.NEAR_TIE = 1e3
    out = loose.prefill(ids, return_all=True)
    assert [a[:5] for a in loose.adopted] == [("blocks", 0, 30, 1, 0)] and loose.mismatches == []
    assert loose.adopted[0][5] < 0
    np.testing.assert_array_equal(out[:30], logits[:30])
    assert not np.array_equal(out[30:], logits[30:])


def test_oracle_follow_adopts_expert_order_and_traces_its_own():
    weights, ids, logits, trace, cfg = _follow_setup()
    rec = follow_record(trace, cfg, len(ids))
    r = rec[25, 0, 1]
    assert r[0] >= 2
    r[1], r[2] = r[2], r[1]                        # the two most probable experts swapped
    loose_trace = []
    loose = OracleModel(_FOLLOW, weights, context_length=64, follow=rec, trace=loose_trace)
    loose.NEAR_TIE = 1e3
    loose.prefill(ids, return_all=True)
    assert [a[:4] for a in loose.adopted] == [("experts", 0, 25, 1)] and loose.mismatches == []
    assert follow_record(loose_trace, cfg, len(ids))[25, 0, 1].tolist() == \
        follow_record(trace, cfg, len(ids))[25, 0, 1].tolist()
    strict = OracleModel(_FOLLOW, weights, context_length=64, follow=rec)
    np.testing.assert_array_equal(strict.prefill(ids, return_all=True), logits)
    assert [m[:4] for m in strict.mismatches] == [("experts", 0, 25, 1)]


def test_oracle_follow_width_moves_only_to_the_other_rounding():
    """A rounding near-tie of the adaptive width can move it by one, to the
    other rounding of its raw value; a followed width two away, or one away on
    the wrong side, is a mismatch even where every value counts as a near-tie."""
    weights, ids, logits, trace, cfg = _follow_setup()
    rec = follow_record(trace, cfg, len(ids))

    def plant(at, width):
        p, l, i = at
        planted = follow_record(trace, cfg, len(ids))
        own = planted[p, l, i, 1:1 + planted[p, l, i, 0]].tolist()
        extra = [e for e in range(16) if e not in own]
        planted[p, l, i, 0] = width
        planted[p, l, i, 1:1 + 4] = -1
        planted[p, l, i, 1:1 + width] = (own + extra)[:width]
        loose = OracleModel(_FOLLOW, weights, context_length=64, follow=planted)
        loose.NEAR_TIE = 1e3
        loose.prefill(ids, return_all=True)
        return [e[:4] for e in loose.adopted], [e[:4] for e in loose.mismatches]

    # width kmax = 4 (raw >= 1.5): its other rounding is 3 at most, never 2
    at = tuple(int(v) for v in np.argwhere(rec[:, :, :, 0] == 4)[0])
    event = [("experts", at[1], at[0], at[2])]
    assert plant(at, 2) == ([], event)
    # width 3 (raw in [0.5, 1.5]): exactly one of 2 and 4 is the other rounding
    at = tuple(int(v) for v in np.argwhere(rec[:, :, :, 0] == 3)[0])
    event = [("experts", at[1], at[0], at[2])]
    outcomes = sorted([plant(at, 2), plant(at, 4)])
    assert outcomes == [([], event), (event, [])]


@pytest.mark.parametrize("slots", [2, 0])
def test_oracle_latent_kv_cache_equals_recompute(slots):
    """The oracle's per-row latent K/V cache (each row's key and value kept
    from the step it was appended or merged on) gives the same bits as the
    reference's recompute-every-row form (model.py:160-163), through merges
    into the memory slots (slots 2) and through drops (slots 0), on BF16 and
    FP32 weights."""
    bundle = dict(presets.micro("flashlighting-2.0"), memory_slots=slots)
    ids = [(7 * i + 3) % 32 for i in range(24)]
    for weights in (synthetic.micro_weights(bundle),
                    {k: (v.bits if hasattr(v, "bits") else v)
                     for k, v in synthetic.synthetic_weights(bundle, 9, "bf16").items()}):
        plain = OracleModel(bundle, weights, context_length=32)
        cached = OracleModel(bundle, weights, context_length=32, latent_kv_cache=True)
        want = plain.prefill(ids, return_all=True)
        np.testing.assert_array_equal(cached.prefill(ids, return_all=True), want)
        np.testing.assert_array_equal(cached.decode(5), plain.decode(5))
        assert [len(s["positions"]) for s in cached.layers] == [len(s["positions"]) for s in plain.layers]
