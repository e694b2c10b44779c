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

BATCHED = ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlite-2.0")


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


def test_batched_fp16_term_inputs_at_extreme_scales(backend):
    """The down and O projections take the SwiGLU output and the attended
    values as FP16 terms whose row scales are bounds fixed before those rows
    exist: |y|^2 ng nu from the FFN input's norm and the gate and up weights'
    row norms, and the largest |v| of every KV head.  Stretch both on the
    flashnano-1.5 mid geometry (BF16): layer 0's gate and up rows x 2^10 and
    its FFN gain x 2^4 (SwiGLU outputs near 10^9, their bound 140-220 times
    higher), layer 1's values of KV head 0 x 2^12 (every other head's
    outputs 2^12 below the scale's bound), and one prompt token's embedding
    row x 2^8.  The batched prefill still matches the exact token loop."""
    from miracle_hip.weights import BF16Array, bf16_bits
    wl = presets.workload("flashnano-1.5-mid")
    cfg = wl["config"]
    weights = synthetic.synthetic_weights(cfg, 29, "bf16")
    ids = synthetic.prompt_ids(cfg["vocab_size"], 300, 29)

    def scale(name, factor, rows=slice(None)):   # powers of two: exact in BF16
        w = weights[name][:]
        w[rows] *= np.float32(factor)
        weights[name] = BF16Array(bf16_bits(w))

    scale("layers.0.ffn.gate", 2.0 ** 10)
    scale("layers.0.ffn.up", 2.0 ** 10)
    weights["layers.0.f_norm"] = weights["layers.0.f_norm"] * np.float32(16.0)
    scale("layers.1.v", 2.0 ** 12, slice(0, cfg["head_dim"]))
    scale("embed", 2.0 ** 8, slice(int(ids[5]), int(ids[5]) + 1))
    runs = {}
    for mode in ("exact", "batched"):
        with MiracleModel(ModelConfig.from_dict(cfg), weights, backend=backend, context_length=1024,
                          prefill_mode=mode) as model:
            runs[mode] = model.prefill(ids, return_all=True)
    assert np.all(np.isfinite(runs["batched"]))
    np.testing.assert_allclose(runs["batched"], runs["exact"], rtol=1e-3, atol=1e-4)


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



# flashnano-1.6 with CBR chunks of 16 rows pooled into 4 relay rows each, a
# 64-key local window and one global layer.
CBR_MID = {"family": "flashnano-1.6", "cbr_chunk_size": 16, "cbr_slots": 4, "vocab_size": 1000, "hidden_size": 512,
           "layers": 3, "query_heads": 8, "kv_heads": 2, "head_dim": 64, "ffn_dim": 1024, "max_positions": 2048,
           "window": 64, "global_layers": [3], "rope_theta": 10000.0, "backend_format": 1}


@pytest.mark.parametrize("dim,parts", [(64, None), (128, [(0, 37), (37, 150), (150, 300)])])
def test_batched_cbr_geometry_matches_oracle(backend, dim, parts):
    """flashnano-1.6 batched (BF16) over 300 tokens, whole and in chunks that
    start and end inside CBR chunks (their pooling reads the pending rows of
    the previous call): logits of every position against the oracle, then the
    greedy stream, whose decode steps pool and read the relay the batched path
    left."""
    from oracle.model import OracleModel
    config = dict(CBR_MID, head_dim=dim, query_heads=CBR_MID["hidden_size"] // dim)
    weights = synthetic.synthetic_weights(config, 17, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 300, 17)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=512)
    want = ref.prefill(ids, return_all=True)
    stream = ref.generate(list(ids), max_new_tokens=8)
    print("case cbr batched", dim, parts, flush=True)
    with MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=512,
                      prefill_mode="batched") as model:
        if parts:
            got = np.concatenate([model.prefill(ids[a:b], return_all=True) for a, b in parts])
        else:
            got = model.prefill(ids, return_all=True)
        np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4)
        assert model.generate(list(ids), max_new_tokens=8) == stream


def test_batched_cbr_long_prompt_matches_token_loop(backend):
    """flashnano-1.6 over a 2000-token prompt (124 CBR chunks, so up to 496
    relay rows join each row's softmax): batched against the exact token loop,
    every 16th row of logits, the decode step that follows, then the greedy
    continuation."""
    weights = synthetic.synthetic_weights(CBR_MID, 19, "bf16")
    ids = synthetic.prompt_ids(CBR_MID["vocab_size"], 2000, 19)
    print("case cbr long prompt", len(ids), flush=True)
    with MiracleModel(ModelConfig.from_dict(CBR_MID), weights, backend=backend, context_length=2048) as model:
        exact = model.prefill(ids, return_all=True)[::16].copy()
        exact_last = model.prefill([int(np.argmax(exact[-1]))])
        exact_stream = model.generate(list(ids), max_new_tokens=6)
        model.reset()
        model.prefill_mode = "batched"
        batched = model.prefill(ids, return_all=True)[::16].copy()
        assert model.position == len(ids)
        np.testing.assert_allclose(batched, exact, rtol=1e-3, atol=1e-4)
        np.testing.assert_allclose(model.prefill([int(np.argmax(exact[-1]))]), exact_last, rtol=1e-3, atol=1e-4)
        assert model.generate(list(ids), max_new_tokens=6) == exact_stream

def _heavy_against_oracle(model, cfg, config, weights, ids, context, parts=None):
    """Device first (its logits, greedy stream and recorded choices), then the
    oracle following the device's choices within its near-tie band."""
    from oracle.model import OracleModel
    if parts:
        got = np.concatenate([model.prefill(ids[a:b], return_all=True) for a, b in parts])
    else:
        got = model.prefill(ids, return_all=True)
    stream = model.generate(list(ids), max_new_tokens=6)
    choices = model.engine.choices()
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=context, follow=choices)
    want = ref.prefill(ids, return_all=True)
    tok, want_stream = int(np.argmax(want[-1])), []
    for i in range(6):
        want_stream.append(tok)
        if tok == cfg.eos_token_id or i == 5:
            break
        tok = int(np.argmax(ref.decode(tok)))
    print("near-ties adopted", ref.adopted, "mismatches", ref.mismatches, flush=True)
    assert ref.mismatches == [] and len(ref.adopted) <= 2
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4)
    assert stream == want_stream


@pytest.mark.parametrize("parts", [None, [(0, 37), (37, 100)]])
def test_batched_heavy_geometry_matches_oracle(backend, parts):
    """heavy-medium-2.0 batched (BF16, head dim 64, 16 experts in 4 groups with
    adaptive width 2..4, blocks of 16 with 3 kept, window 32) over 100 tokens,
    whole and in two chunks (the second reads the first's rings and block
    sums): logits of every position, the greedy stream, and every block and
    expert choice against the oracle."""
    from test_hip_model import HEAVY_MID
    weights = synthetic.synthetic_weights(HEAVY_MID, 11, "bf16")
    ids = synthetic.prompt_ids(HEAVY_MID["vocab_size"], 100, 11)
    cfg = ModelConfig.from_dict(HEAVY_MID)
    print("case heavy batched", parts, flush=True)
    with MiracleModel(cfg, weights, backend=backend, context_length=160, prefill_mode="batched") as model:
        _heavy_against_oracle(model, cfg, HEAVY_MID, weights, ids, 160, parts)


def test_batched_heavy_micro_takes_token_loop(backend, golden_dir):
    """The reference's micro heavy model (head dim 4) is outside the batched
    kernels' geometry: under prefill_mode="batched" it takes the token loop and
    matches the reference's fixture."""
    from test_oracle_model import _load
    z, bundle, weights = _load(golden_dir, "heavy-medium-2.0")
    with MiracleModel(ModelConfig.from_dict(bundle), weights, backend=backend, context_length=32,
                      prefill_mode="batched") as model:
        np.testing.assert_allclose(model.prefill(z["ids"], return_all=True), z["logits"], atol=2e-5, rtol=2e-4)


@pytest.mark.parametrize("slots,parts", [(4, None), (4, [(0, 20), (20, 31), (31, 90)]), (0, None),
                                         (0, [(0, 30), (30, 90)])])
def test_batched_lighting_geometry_matches_oracle(backend, slots, parts):
    """flashlighting-2.0 batched (BF16, YaRN, window 24 with 4 memory slots or
    none) over 90 tokens: whole, and in chunks that begin before, at and after
    the first merge (or drop); logits of every position and the greedy stream
    against the oracle."""
    from oracle.model import OracleModel
    from test_hip_model import LIGHT_MID
    config = dict(LIGHT_MID, memory_slots=slots)
    weights = synthetic.synthetic_weights(config, 13, "bf16")
    ids = synthetic.prompt_ids(config["vocab_size"], 90, 13)
    ref = OracleModel(config, {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()},
                      context_length=128)
    want = ref.prefill(ids, return_all=True)
    stream = ref.generate(list(ids), max_new_tokens=8)
    print("case lighting batched", slots, parts, flush=True)
    with MiracleModel(ModelConfig.from_dict(config), weights, backend=backend, context_length=128,
                      prefill_mode="batched") as model:
        if parts:
            got = np.concatenate([model.prefill(ids[a:b], return_all=True) for a, b in parts])
        else:
            got = model.prefill(ids, return_all=True)
        np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-4)
        assert model.generate(list(ids), max_new_tokens=8) == stream


def test_batched_lighting_full_prompt_matches_token_loop(backend):
    """flashlighting-2.0's full 8192-token prompt in two chunks (the second
    starts before the first merge at 4608 and ends 3584 merges later) batched
    against the exact token loop: every 64th row of logits, the decode step
    that follows (it reads the latent memory the batched path left, with a
    merged row pending), then the greedy continuation.  (heavy-medium-2.0 has
    no such check: its routing has near-ties, where two exact FP32 orders may
    choose differently and the paths then part; its batched prompts are
    checked against the oracle following the device's choices.)"""
    name = "flashlighting-2.0"
    wl = presets.workload(name)
    cfg = ModelConfig.from_dict(wl["config"])
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    ids = synthetic.prompt_ids(cfg.vocab_size, wl["prompt"], wl["seed"])
    print("case", name, "prompt", len(ids), flush=True)
    with MiracleModel(cfg, weights, backend=backend, context_length=wl["context"]) as model:
        exact = model.prefill(ids, return_all=True)[::64].copy()
        exact_last = model.prefill([int(np.argmax(exact[-1]))])   # position len(ids)
        exact_stream = model.generate(list(ids), max_new_tokens=6)
        model.reset()
        model.prefill_mode = "batched"
        batched = model.prefill(ids, return_all=True)[::64].copy()
        assert model.position == len(ids)
        np.testing.assert_allclose(batched, exact, rtol=1e-3, atol=1e-4)
        np.testing.assert_allclose(model.prefill([int(np.argmax(exact[-1]))]), exact_last, rtol=1e-3, atol=1e-4)
        assert model.generate(list(ids), max_new_tokens=6) == exact_stream
