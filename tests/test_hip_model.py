"""MiracleModel on the GPU against the reference's golden fixtures and the oracle.

Tolerances (the contract's): per-token logits within atol 2e-5 / rtol 2e-4 on
the micro and tiny configurations, rtol 1e-3 (atol 1e-4) on the larger ones;
greedy and seeded-sampling token streams identical; the reference's invariants
(decode == prefill bit for bit, context overflow rejected without advancing,
bad inputs rejected before any step) exact.
"""
import json

import numpy as np
import pytest

from miracle_hip import MiracleModel, ModelConfig, presets, synthetic
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu

GQA = ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlite-2.0", "flashlighting-2.0")


def _variants():
    from conftest import GOLDEN
    names = sorted(p.stem[len("micro_"):] for p in GOLDEN.glob("micro_*.npz"))
    return [n for n in names if n.rsplit("-untied", 1)[0] in GQA]


def _micro(golden_dir, name):
    z = np.load(golden_dir / f"micro_{name}.npz")
    bundle = json.loads(str(z["bundle"]))
    return z, ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle)


@pytest.mark.parametrize("variant", _variants())
def test_micro_matches_reference(backend, golden_dir, variant):
    z, cfg, weights = _micro(golden_dir, variant)
    print("case", variant, flush=True)
    model = MiracleModel(cfg, weights, backend=backend, context_length=32)
    ids = z["ids"]
    np.testing.assert_allclose(model.prefill(ids, return_all=True), z["logits"], atol=2e-5, rtol=2e-4)
    model.reset()
    chunked = np.concatenate([model.prefill(ids[:5], return_all=True), model.prefill(ids[5:], return_all=True)])
    np.testing.assert_allclose(chunked, z["chunked"], atol=2e-5, rtol=2e-4)
    assert model.generate(list(ids[:4]), max_new_tokens=8) == z["greedy"].tolist()
    assert model.generate([1, 3], max_new_tokens=4, temperature=0.8, top_k=5, top_p=0.9, seed=7) == \
        z["sampled"].tolist()


def test_cache_reset_bounds_and_decode_equals_prefill(backend):
    # reference tests/test_inference.py:52-69
    bundle = presets.micro("flashnano-1.5")
    model = MiracleModel(ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle), backend=backend,
                         context_length=12)
    ids = [1, 3, 5, 8, 2, 9, 11, 10, 9, 7, 6, 4]
    whole = model.prefill(ids, return_all=True)
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


def test_generation_is_repeatable_and_validates_before_reset(backend):
    # reference tests/test_inference.py:87-99
    bundle = presets.micro("flashnano-1.5")
    model = MiracleModel(ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle), backend=backend,
                         context_length=12)
    a = model.generate([1, 3], max_new_tokens=4, temperature=.8, top_k=5, top_p=.9, seed=7)
    assert a == model.generate([1, 3], max_new_tokens=4, temperature=.8, top_k=5, top_p=.9, seed=7)
    position = model.position
    for kwargs in ({"max_new_tokens": -1}, {"max_new_tokens": 12}, {"temperature": float("nan")}, {"top_p": 0}):
        with pytest.raises(ValueError):
            model.generate([1, 3], **kwargs)
        assert model.position == position
    greedy = model.generate([1], max_new_tokens=1)[0]
    assert model.generate([1], max_new_tokens=4, eos_token_id=greedy) == [greedy]
    assert model.position == 1
    assert model.generate([1], max_new_tokens=0) == []


def test_failed_step_poisons_until_reset(backend):
    bundle = presets.micro("flashnano-1.7")
    model = MiracleModel(ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle), backend=backend,
                         context_length=16)
    model.prefill([1, 2])
    backend.fail_next()
    with pytest.raises(RuntimeError):
        model.decode(3)
    with pytest.raises(RuntimeError, match="reset"):
        model.decode(3)
    model.reset()
    model.prefill([1, 2])


def test_workload_tiny_matches_reference(backend, golden_dir):
    z = np.load(golden_dir / "workload_flashnano-1.5-tiny.npz")
    wl = presets.workload("flashnano-1.5-tiny")
    cfg = ModelConfig.from_dict(wl["config"])
    model = MiracleModel(cfg, synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"]), backend=backend,
                         context_length=wl["context"])
    np.testing.assert_allclose(model.prefill(z["prompt"]), z["last_logits"], atol=2e-5, rtol=2e-4)
    assert model.generate(list(z["prompt"]), max_new_tokens=16) == z["greedy"].tolist()


_WORKLOAD_CACHE = {}


def _workload(name, prompt):
    """Weights, prompt and oracle results for a workload geometry (cached)."""
    if name not in _WORKLOAD_CACHE:
        wl = presets.workload(name)
        weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
        ids = synthetic.prompt_ids(wl["config"]["vocab_size"], prompt, wl["seed"])
        ref = OracleModel(wl["config"], {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                          context_length=wl["context"])
        want = ref.prefill(ids, return_all=True)
        stream = ref.generate(list(ids), max_new_tokens=6)
        _WORKLOAD_CACHE[name] = (wl, weights, ids, want, stream)
    return _WORKLOAD_CACHE[name]


@pytest.mark.parametrize("mode", ["persistent", "graph"])
@pytest.mark.parametrize("name,prompt", [("flashnano-1.5-tiny", 70), ("flashnano-1.5-mid", 40), ("flashnano-1.7", 12)])
def test_workload_geometry_matches_oracle(backend, name, prompt, mode):
    """Full-size geometry (weights as drawn for the workload) on a short prompt:
    logits of every prompt token and a greedy stream against the oracle, for
    both step implementations.  The tiny prompt (70 tokens) wraps its 64-key
    local ring."""
    wl, weights, ids, want, stream = _workload(name, prompt)
    print("case", name, mode, flush=True)
    model = MiracleModel(ModelConfig.from_dict(wl["config"]), weights, backend=backend, context_length=wl["context"])
    model.engine.set_step_mode(mode)
    assert model.engine.step_mode() == mode
    tol = dict(atol=2e-5, rtol=2e-4) if wl["dtype"] == "f32" else dict(rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, **tol)
    assert model.generate(list(ids), max_new_tokens=6) == stream


# flashnano-1.7 geometries whose persistent step runs several key splits per
# head and splits the query heads of a KV head over units (4 per local KV head,
# 2 per global one); the D=128 one also deals those units XCD by XCD.
SPLIT_MID = {"family": "flashnano-1.7", "vocab_size": 1000, "hidden_size": 1024, "layers": 4, "query_heads": 8,
             "kv_heads": 2, "global_kv_heads": 4, "head_dim": 128, "ffn_dim": 1024, "max_positions": 1024,
             "window": 256, "global_layers": [2, 4], "rope_theta": 500000.0, "backend_format": 1}


@pytest.mark.parametrize("dim,prompt", [(128, 300), (32, 600)])
def test_persistent_split_units_match_oracle(backend, dim, prompt):
    """Persistent step kernel with up to 10 active key splits and query-head
    groups per KV head (prompts past the local ring): logits of every prompt
    position and a greedy stream against the oracle."""
    config = SPLIT_MID if dim == 128 else dict(SPLIT_MID, hidden_size=256, head_dim=32, ffn_dim=512, window=512)
    weights = synthetic.synthetic_weights(config, 31, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], prompt, 31)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=1024)
    want = ref.prefill(ids, return_all=True)
    print("case split units", dim, prompt, flush=True)
    model = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=1024)
    assert model.engine.step_mode() == "persistent"
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    assert model.generate(list(ids), max_new_tokens=6) == ref.generate(list(ids), max_new_tokens=6)


def test_persistent_decode_equals_prefill(backend):
    """The exact-mode invariant (decode == prefill, bit for bit) on the
    persistent path, which reduces across workgroups in a fixed order."""
    wl = presets.workload("flashnano-1.5-tiny")
    model = MiracleModel(ModelConfig.from_dict(wl["config"]),
                         synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"]), backend=backend,
                         context_length=128)
    assert model.engine.step_mode() == "persistent"
    ids = synthetic.prompt_ids(4096, 20, 5)
    whole = model.prefill(ids, return_all=True)
    model.reset()
    np.testing.assert_array_equal(np.stack([model.decode(int(i)) for i in ids]), whole)


def test_traced_persistent_step_changes_nothing(backend):
    """A step run with the phase timeline (mr_model_trace_step) decodes like an
    untraced one: the greedy stream through it equals the untraced stream, and
    every workgroup stamps every phase's entry."""
    config = SPLIT_MID
    weights = synthetic.synthetic_weights(config, 31, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 300, 31)
    plain = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=1024)
    plain.prefill(ids)
    want = plain.engine.generate_greedy(6, -1)
    traced = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=1024)
    assert traced.engine.step_mode() == "persistent"
    traced.prefill(ids)
    head = traced.engine.generate_greedy(2, -1)
    t = traced.engine.trace_step()
    tail = traced.engine.generate_greedy(3, -1)
    assert list(head) == list(want[:2]) and list(tail) == list(want[3:6])
    assert t.ndim == 3 and t.shape[2] == 5
    assert np.all(np.isfinite(t[:, :, 0]))                # every workgroup enters every phase
    assert np.all(np.isfinite(t[:, :, 1]).any(axis=1))   # every phase stages inputs on some workgroup
    assert np.all(np.isfinite(t[:, :, 2]).any(axis=1))   # and ends on some workgroup
    assert np.all(np.nanmax(t[:, :, 2], axis=1) >= np.nanmin(t[:, :, 0], axis=1))


def _heavy_variants():
    from conftest import GOLDEN
    return sorted(p.stem[len("micro_"):] for p in GOLDEN.glob("micro_heavy-medium-2.0*.npz"))


def _choice_logs(choices, cfg):
    """Expert log and block masks in the reference trace's order (per position,
    layer and inner loop: attention blocks, then experts)."""
    s = cfg.source
    kmax, slots, block = s["router_top_k_max"], s["long_context"]["global_slots"], \
        s["long_context"]["global_block_size"]
    experts, masks = [], []
    for pos in range(choices.shape[0]):
        count = pos + 1
        length, blocks = min(cfg.window, count), -(-count // block)
        for layer in range(cfg.layers):
            for loop in range(cfg.inner_loop_steps):
                rec = choices[pos, layer, loop]
                m = np.zeros((cfg.query_heads, length + blocks), bool)
                m[:, :length] = True
                for h in range(cfg.query_heads):
                    chosen = rec[1 + kmax + h * slots: 1 + kmax + (h + 1) * slots]
                    m[h, [length + b for b in chosen if b >= 0]] = True
                masks.append(m)
                experts.append((layer, -1))
                experts.extend((layer, int(e)) for e in rec[1:1 + rec[0]])
    return np.asarray(experts, np.int64).reshape(-1, 2), masks


@pytest.mark.parametrize("variant", _heavy_variants())
def test_heavy_micro_matches_reference(backend, golden_dir, variant):
    """heavy-medium-2.0 on device: logits, chunked prefill, streams, and the
    routed experts / adaptive widths / global blocks bit-exact against the
    reference's own trace."""
    from test_oracle_model import _load
    z, bundle, weights = _load(golden_dir, variant)
    print("case", variant, flush=True)
    cfg = ModelConfig.from_dict(bundle)
    model = MiracleModel(cfg, weights, backend=backend, context_length=32)
    ids = z["ids"]
    np.testing.assert_allclose(model.prefill(ids, return_all=True), z["logits"], atol=2e-5, rtol=2e-4)
    experts, masks = _choice_logs(model.engine.choices(), cfg)
    np.testing.assert_array_equal(experts, z["experts"])
    widths = z["block_mask_widths"]
    assert [m.shape[1] for m in masks] == widths.tolist()
    for i, m in enumerate(masks):
        np.testing.assert_array_equal(m, z["block_masks"][i, :, :widths[i]])
    model.reset()
    chunked = np.concatenate([model.prefill(ids[:5], return_all=True), model.prefill(ids[5:], return_all=True)])
    np.testing.assert_allclose(chunked, z["chunked"], atol=2e-5, rtol=2e-4)
    assert model.generate(list(ids[:4]), max_new_tokens=8) == z["greedy"].tolist()
    assert model.generate([1, 3], max_new_tokens=4, temperature=0.8, top_k=5, top_p=0.9, seed=7) == \
        z["sampled"].tolist()


HEAVY_MID = {"family": "heavy-medium-2.0", "vocab_size": 512, "hidden_size": 256, "layers": 2, "query_heads": 4,
             "kv_heads": 2, "head_dim": 64, "ffn_dim": 128, "max_positions": 256, "window": 32, "latent_dim": 32,
             "inner_loop_steps": 2, "rope_theta": 1000000.0,
             "source": {"routed_experts": 16, "router_groups": 4, "router_top_k_max": 4, "router_top_k_min": 2,
                        "shared_experts": 1, "router_temperature": 1.0,
                        "long_context": {"global_block_size": 16, "global_slots": 3, "rope_local_fraction": 0.6,
                                         "alibi_slope_scale": 0.015}},
             "backend_format": 1}


def test_heavy_geometry_matches_oracle(backend):
    """A BF16 heavy-medium-2.0 geometry over 100 tokens (window overflow, seven
    blocks, three chosen per head, 16 experts in 4 groups with adaptive width
    2..4) against the oracle: logits, greedy stream, and every routing choice
    bit-exact."""
    from test_oracle_model import _block_masks, _expert_log
    weights = synthetic.synthetic_weights(HEAVY_MID, 11, "bf16")
    ids = synthetic.prompt_ids(HEAVY_MID["vocab_size"], 100, 11)
    trace = []
    ref = OracleModel(HEAVY_MID, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=160, trace=trace)
    want = ref.prefill(ids, return_all=True)
    cfg = ModelConfig.from_dict(HEAVY_MID)
    model = MiracleModel(cfg, weights, backend=backend, context_length=160)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    experts, masks = _choice_logs(model.engine.choices(), cfg)
    np.testing.assert_array_equal(experts, _expert_log(trace))
    ref_masks = _block_masks(trace, ref.cfg, cfg.query_heads)
    assert len(masks) == len(ref_masks)
    for ours, theirs in zip(masks, ref_masks):
        np.testing.assert_array_equal(ours, theirs)
    stream = ref.generate(list(ids), max_new_tokens=8)
    assert model.generate(list(ids), max_new_tokens=8) == stream


def test_heavy_general_paths_match_oracle(backend):
    """heavy-medium-2.0 with a latent width the fused K/V prologue does not take
    (36: the projection runs as a GEMV and k_heavy_prep follows) and head dim 48
    (the single-workgroup attention instead of the split one): logits, every
    routing and block choice bit-exact, and the greedy stream, against the
    oracle."""
    from test_oracle_model import _block_masks, _expert_log
    config = dict(HEAVY_MID, latent_dim=36, head_dim=48)
    weights = synthetic.synthetic_weights(config, 19, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 70, 19)
    trace = []
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=128, trace=trace)
    want = ref.prefill(ids, return_all=True)
    cfg = ModelConfig.from_dict(config)
    model = MiracleModel(cfg, weights, backend=backend, context_length=128)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    experts, masks = _choice_logs(model.engine.choices(), cfg)
    np.testing.assert_array_equal(experts, _expert_log(trace))
    ref_masks = _block_masks(trace, ref.cfg, cfg.query_heads)
    assert len(masks) == len(ref_masks)
    for ours, theirs in zip(masks, ref_masks):
        np.testing.assert_array_equal(ours, theirs)
    assert model.generate(list(ids), max_new_tokens=6) == ref.generate(list(ids), max_new_tokens=6)


LIGHT_MID = {"family": "flashlighting-2.0", "vocab_size": 512, "hidden_size": 256, "layers": 2, "query_heads": 4,
             "kv_heads": 4, "head_dim": 64, "ffn_dim": 384, "max_positions": 4096, "window": 24, "latent_dim": 32,
             "memory_slots": 4, "rope_theta": 1000000.0,
             "source": {"rope_scaling_type": "yarn", "rope_scaling_factor": 4.0, "max_position_embeddings": 64},
             "backend_format": 1}


@pytest.mark.parametrize("slots", [4, 0])
def test_lighting_geometry_matches_oracle(backend, slots):
    """A BF16 flashlighting-2.0 geometry over 90 tokens: YaRN RoPE, latent rows
    past the window merged into memory slots (or dropped without slots), against
    the oracle's logits and greedy stream."""
    config = dict(LIGHT_MID, memory_slots=slots)
    weights = synthetic.synthetic_weights(config, 13, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 90, 13)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=128)
    want = ref.prefill(ids, return_all=True)
    model = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=128)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    assert model.generate(list(ids), max_new_tokens=8) == ref.generate(list(ids), max_new_tokens=8)



def test_lighting_split_attention_matches_oracle(backend):
    """The split-key latent attention (64 memory rows per workgroup, merged per
    head) over a window of 150 rows and 8 memory slots: 230 tokens fill three
    splits, push rows past the window (masked) and merge the oldest into the
    slots; logits and greedy stream against the oracle."""
    config = dict(LIGHT_MID, window=150, memory_slots=8)
    weights = synthetic.synthetic_weights(config, 17, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 230, 17)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=256)
    want = ref.prefill(ids, return_all=True)
    model = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=256)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    assert model.generate(list(ids), max_new_tokens=8) == ref.generate(list(ids), max_new_tokens=8)


def test_lighting_general_paths_match_oracle(backend):
    """flashlighting-2.0 with a latent width the fused row kernel does not take
    (36: prologue, projection GEMV and cache-row kernels apart) and head dim 48
    (the single-workgroup attention instead of the split one), with merges into
    memory slots: logits and greedy stream against the oracle."""
    config = dict(LIGHT_MID, latent_dim=36, head_dim=48, hidden_size=192)
    weights = synthetic.synthetic_weights(config, 23, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 80, 23)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=128)
    want = ref.prefill(ids, return_all=True)
    model = MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=128)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, rtol=1e-3, atol=1e-4)
    assert model.generate(list(ids), max_new_tokens=6) == ref.generate(list(ids), max_new_tokens=6)


def test_step_timeout_falls_back_to_graph_mode(backend):
    """A persistent step whose wait times out (reported from the host-side
    status check, no kernel is made to wait) fails with a timeout error,
    poisons the model until reset(), and the reset switches it to graph mode,
    whose results are the same to the tolerance."""
    from miracle_hip import HIPError
    wl = presets.workload("flashnano-1.5-tiny")
    cfg = ModelConfig.from_dict(wl["config"])
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    model = MiracleModel(cfg, weights, backend=backend, context_length=64)
    assert model.engine.step_mode() == "persistent"
    ids = [5, 9, 2, 7]
    want = model.prefill(ids, return_all=True)
    model.reset()
    model.prefill(ids[:2])
    model.engine.debug_step_timeout()
    with pytest.raises(HIPError, match="timed out"):
        model.decode(ids[2])
    with pytest.raises(RuntimeError, match="reset"):
        model.decode(ids[2])
    model.reset()
    assert model.engine.step_mode() == "graph"
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, atol=2e-5, rtol=2e-4)
    model.close()


def test_weight_cache_budget_and_untied_head(backend):
    # reference tests/test_inference.py:72-84: a 4 KiB weight budget gives the
    # same logits (here every weight is resident in HBM whatever the budget)
    bundle = dict(presets.micro("flashnano-1.5"), tie_embeddings=False, vocab_size=161)
    cfg = ModelConfig.from_dict(bundle)
    weights = synthetic.micro_weights(bundle)
    rng = np.random.default_rng(4)
    weights["embed"] = rng.normal(0, .1, (161, 16)).astype(np.float32)
    weights["output"] = rng.normal(0, .1, (161, 16)).astype(np.float32)
    tiled = MiracleModel(cfg, weights, backend=backend, context_length=16, weight_cache_bytes=4096)
    full = MiracleModel(cfg, weights, backend=backend, context_length=16)
    np.testing.assert_array_equal(tiled.prefill([1, 5, 8]), full.prefill([1, 5, 8]))
    assert tiled.weight_cache.used <= 4096 and tiled.weight_cache.budget == 4096
    assert tiled.weight_cache.resident == sum(np.asarray(v).nbytes for v in weights.values())
    with pytest.raises(ValueError, match="weight_cache_bytes"):
        MiracleModel(cfg, weights, backend=backend, context_length=16, weight_cache_bytes=4095)


def test_close_releases_models_before_their_backend():
    """HIPBackend.close() closes the backend's models first, then its context;
    closing either twice is harmless, and a backend made afterwards works."""
    from miracle_hip import HIPBackend
    bundle = presets.micro("flashnano-1.7")
    cfg = ModelConfig.from_dict(bundle)
    weights = synthetic.micro_weights(bundle)
    b1 = HIPBackend()
    m1 = MiracleModel(cfg, weights, backend=b1, context_length=16)
    want = m1.prefill([1, 2, 3])
    b1.close()                       # closes m1, then the context
    assert m1.engine.handle is None
    b1.close()
    m1.close()
    m1.close()
    b2 = HIPBackend()
    with MiracleModel(cfg, weights, backend=b2, context_length=16) as m2:
        np.testing.assert_array_equal(m2.prefill([1, 2, 3]), want)
    b2.close()


def test_context_destroyed_under_a_live_model():
    """Through the C ABI: mr_ctx_destroy while a model still uses the context
    drops only the caller's reference (the model holds its own), so the model
    keeps running, and mr_model_destroy then releases the context."""
    from miracle_hip import HIPBackend
    bundle = presets.micro("flashnano-1.7")
    cfg = ModelConfig.from_dict(bundle)
    weights = synthetic.micro_weights(bundle)
    backend = HIPBackend()
    model = MiracleModel(cfg, weights, backend=backend, context_length=16)
    want = model.prefill([1, 2, 3])
    lib = backend.lib
    ctx, backend.ctx = backend.ctx, None      # the caller's reference, taken over here
    assert lib.mr_ctx_destroy(ctx) == 0
    model.reset()
    np.testing.assert_array_equal(model.prefill([1, 2, 3]), want)   # mr_model_forward on the live model
    handle, model.engine.handle = model.engine.handle, None
    assert lib.mr_model_destroy(handle) == 0   # the last reference: the context goes with it
