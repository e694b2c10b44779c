"""Batched prefill on the GPU against the reference's fixtures, the oracle and
the exact token loop.

The batched path runs each layer once per prompt chunk (projections as MFMA
GEMMs with FP32-faithful BF16 term products, causal windowed attention over the
chunk plus the ring), so it sums in another order than the token loop and is
held to the contract's tolerances rather than to bit equality: logits within
atol 2e-5 / rtol 2e-4 on the micro and tiny configurations (FP32 weights),
rtol 1e-3 / atol 1e-4 on the BF16 geometries; greedy streams identical.
"""
import json

import numpy as np
import pytest

from miracle_hip import MiracleModel, ModelConfig, presets, synthetic

pytestmark = pytest.mark.gpu

BATCHED = ("flashnano-1.5", "flashnano-1.7", "flashlite-2.0")


def _variants():
    from conftest import GOLDEN
    names = sorted(p.stem[len("micro_"):] for p in GOLDEN.glob("micro_*.npz"))
    return [n for n in names if n.rsplit("-untied", 1)[0] in BATCHED]


@pytest.mark.parametrize("variant", _variants())
def test_batched_micro_matches_reference(backend, golden_dir, variant):
    """Reference fixtures of the micro models (window 4, so the 12-token prompt
    wraps every local ring twice): whole, chunked and last-token prefill, then
    a greedy stream whose prompt goes through the batched path."""
    z = np.load(golden_dir / f"micro_{variant}.npz")
    bundle = json.loads(str(z["bundle"]))
    print("case", variant, flush=True)
    model = MiracleModel(ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle), backend=backend,
                         context_length=32, prefill_mode="batched")
    ids = z["ids"]
    tol = dict(atol=2e-5, rtol=2e-4)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), z["logits"], **tol)
    model.reset()
    chunked = np.concatenate([model.prefill(ids[:5], return_all=True), model.prefill(ids[5:], return_all=True)])
    np.testing.assert_allclose(chunked, z["chunked"], **tol)
    model.reset()
    np.testing.assert_allclose(model.prefill(ids), z["logits"][-1], **tol)
    assert model.generate(list(ids[:4]), max_new_tokens=8) == z["greedy"].tolist()


@pytest.mark.parametrize("name,prompt", [("flashnano-1.5-tiny", 70), ("flashnano-1.5-mid", 40), ("flashnano-1.7", 12)])
def test_batched_workload_geometry_matches_oracle(backend, name, prompt):
    """Full-size geometries on short prompts against the oracle (the tiny one
    wraps its 64-key local ring), then a greedy stream."""
    from test_hip_model import _workload
    wl, weights, ids, want, stream = _workload(name, prompt)
    print("case", name, flush=True)
    model = MiracleModel(ModelConfig.from_dict(wl["config"]), weights, backend=backend, context_length=wl["context"],
                         prefill_mode="batched")
    tol = dict(atol=2e-5, rtol=2e-4) if wl["dtype"] == "f32" else dict(rtol=1e-3, atol=1e-4)
    np.testing.assert_allclose(model.prefill(ids, return_all=True), want, **tol)
    assert model.generate(list(ids), max_new_tokens=6) == stream


def test_batched_split_prompt_matches_whole(backend):
    """Chunk invariance at tolerance: a prompt appended in three uneven parts
    (each reading the previous parts' keys from the rings, one part shorter
    than the window, one longer) against the whole prompt."""
    wl = presets.workload("flashnano-1.5-tiny")
    model = MiracleModel(ModelConfig.from_dict(wl["config"]),
                         synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"]), backend=backend,
                         context_length=512, prefill_mode="batched")
    ids = synthetic.prompt_ids(4096, 300, 11)
    whole = model.prefill(ids, return_all=True)
    model.reset()
    parts = np.concatenate([model.prefill(ids[:37], return_all=True), model.prefill(ids[37:201], return_all=True),
                            model.prefill(ids[201:], return_all=True)])
    np.testing.assert_allclose(parts, whole, atol=2e-5, rtol=2e-4)


def test_batched_full_prompt_matches_token_loop(backend):
    """flashnano-1.7 at its full 4096-token prompt (every local ring wraps
    four times; the global layers attend over up to 4096 keys): batched
    prefill against the exact token loop, whose agreement with the oracle the
    geometry tests establish.  All 4096 rows of logits, then the position and a
    greedy continuation from the batched prompt."""
    wl = presets.workload("flashnano-1.7")
    cfg = ModelConfig.from_dict(wl["config"])
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    ids = synthetic.prompt_ids(cfg.vocab_size, wl["prompt"], wl["seed"])
    print("case flashnano-1.7 prompt", len(ids), flush=True)
    model = MiracleModel(cfg, weights, backend=backend, context_length=wl["context"])
    exact = model.prefill(ids, return_all=True)
    exact_stream = model.generate(list(ids), max_new_tokens=8)
    model.reset()
    model.prefill_mode = "batched"
    batched = model.prefill(ids, return_all=True)
    assert model.position == len(ids)
    np.testing.assert_allclose(batched, exact, rtol=1e-3, atol=1e-4)
    assert model.generate(list(ids), max_new_tokens=8) == exact_stream
