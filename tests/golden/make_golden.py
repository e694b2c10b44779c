"""Write the golden fixtures in tests/golden/ from the reference's own Python.

Run in the build container only (the reference is not present anywhere else):

    python tests/golden/make_golden.py [/root/reference]
    python tests/golden/make_golden.py names     # only native_names.json

It imports the reference package ``miracle_reasoning`` from the given tree and
drives its own ``MiracleModel`` (model.py), ``ModelConfig`` (config.py) and
``expected_shapes`` (weights.py) -- the parts that no closed form pins.  The
reference's OpenCL runtime cannot run here (no OpenCL device), so its kernels
are supplied by the oracle's C restatement (oracle/device.py), which the
closed-form kernel tests pin separately.  Only inputs and outputs are written:
token ids, logits, greedy / sampled streams, routing and block decisions,
cache metadata, RoPE tables, shape tables and parsed configs.
"""
from __future__ import annotations

import json
import sys
from collections.abc import Mapping
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "miraclereasoning-cpu_amd"))

from miracle_hip import presets, synthetic  # noqa: E402
from oracle.device import OracleDevice  # noqa: E402


class Recorder(Mapping):
    """Weight mapping that logs which routed experts each MoE call reads."""

    def __init__(self, weights):
        self.weights, self.log, self.on = weights, [], False

    def __iter__(self):
        return iter(self.weights)

    def __len__(self):
        return len(self.weights)

    def __getitem__(self, key):
        # Count only the projection calls (WeightCache.linear), not cache fills.
        if self.on and sys._getframe(1).f_code.co_name == "linear":
            parts = key.split(".")
            if key.endswith("router.coarse.weight"):
                self.log.append((int(parts[1]), -1))        # start of one MoE call
            elif ".experts." in key and key.endswith(".gate"):
                self.log.append((int(parts[1]), int(parts[3])))
        return self.weights[key]


def run_family(ref, name, bundle, weights, ids):
    cfg = ref.ModelConfig.from_dict(bundle)
    rec = Recorder(weights)
    dev = OracleDevice()
    masks = []
    heads = cfg.query_heads

    def observe(a):
        # heavy-medium's masked [heads, window + blocks] score matrix, uploaded by _heavy_attention.
        if sys._getframe(2).f_code.co_name == "_heavy_attention":
            masks.append(np.isfinite(a))

    model = ref.MiracleModel(cfg, rec, backend=dev, context_length=32)
    rec.on = True
    dev.observe = observe
    expert_log_start = len(rec.log)
    logits = model.prefill(np.asarray(ids), return_all=True)
    experts = rec.log[expert_log_start:]
    block_masks = list(masks)
    meta = {}
    if cfg.family in ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlite-2.0"):
        meta["ring_length"] = [s["ring"].length for s in model.states]
        meta["ring_start"] = [s["ring"].start for s in model.states]
        if cfg.family == "flashnano-1.6":
            meta["relay_count"] = [s["relay"].count for s in model.states]
    if cfg.family == "flashlighting-2.0":
        meta["latent_rows"] = [int(s["latent"].shape[0]) for s in model.states]
        meta["positions"] = [list(map(int, s["positions"])) for s in model.states]
        meta["counts"] = [list(map(float, s["counts"])) for s in model.states]
        meta["memory_size"] = [int(s["memory_size"]) for s in model.states]
    if cfg.family == "heavy-medium-2.0":
        meta["loop_counts"] = [[lp["ring"].count for lp in s["loops"]] for s in model.states]
    model.reset()
    rec.on = False
    dev.observe = None
    chunked = np.concatenate([model.prefill(np.asarray(ids[:5]), return_all=True),
                              model.prefill(np.asarray(ids[5:]), return_all=True)])
    greedy = model.generate(list(ids[:4]), max_new_tokens=8)
    sampled = model.generate([1, 3], max_new_tokens=4, temperature=0.8, top_k=5, top_p=0.9, seed=7)
    out = dict(ids=np.asarray(ids, np.int64), logits=logits.astype(np.float32),
               chunked=chunked.astype(np.float32), greedy=np.asarray(greedy, np.int64),
               sampled=np.asarray(sampled, np.int64), meta=np.asarray(json.dumps(meta)))
    if cfg.family == "heavy-medium-2.0":
        out["experts"] = np.asarray(experts, np.int64).reshape(-1, 2)
        out["block_masks"] = pad_masks(block_masks)
        out["block_mask_widths"] = np.asarray([m.shape[1] for m in block_masks], np.int64)
    return out


def pad_masks(masks):
    width = max(m.shape[1] for m in masks)
    out = np.zeros((len(masks), masks[0].shape[0], width), bool)
    for i, m in enumerate(masks):
        out[i, :, :m.shape[1]] = m
    return out


def rope_cases():
    base = dict(backend_format=1, vocab_size=32, hidden_size=512, layers=2, query_heads=4, kv_heads=2,
                head_dim=128, ffn_dim=24, max_positions=16384, window=4)
    cases = {
        "1.5_theta1e4_d32": dict(base, family="flashnano-1.5", hidden_size=128, head_dim=32, rope_theta=1e4),
        "1.7_theta5e5_d128": dict(base, family="flashnano-1.7", rope_theta=5e5),
        "1.7_yarn": dict(base, family="flashnano-1.7", rope_theta=5e5,
                         source={"rope_scaling": {"type": "yarn", "factor": 4.0, "orig_max_position": 4096,
                                                  "beta_fast": 32, "beta_slow": 1}}),
        "1.7_yarn_narrow": dict(base, family="flashnano-1.7", rope_theta=1e4, hidden_size=32, head_dim=8,
                                source={"rope_scaling": {"type": "yarn", "factor": 2.0, "orig_max_position": 64,
                                                         "beta_fast": 4, "beta_slow": 2}}),
        "lighting_yarn4": dict(base, family="flashlighting-2.0", latent_dim=256,
                               source={"rope_scaling_type": "yarn", "rope_scaling_factor": 4,
                                       "max_position_embeddings": 4096}),
        "lighting_yarn_default": dict(base, family="flashlighting-2.0", latent_dim=256),
        "lighting_linear": dict(base, family="flashlighting-2.0", latent_dim=256,
                                source={"rope_scaling_type": "linear", "rope_scaling_factor": 3.0}),
        "lighting_ntk": dict(base, family="flashlighting-2.0", latent_dim=256,
                             source={"rope_scaling_type": "dynamic_ntk", "rope_scaling_factor": 4.0,
                                     "max_position_embeddings": 4096,
                                     "extension_max_position_embeddings": 16384}),
        "lighting_none": dict(base, family="flashlighting-2.0", latent_dim=256,
                              source={"rope_scaling_type": "none"}),
        "heavy_split": dict(base, family="heavy-medium-2.0", latent_dim=256, hidden_size=2048,
                            source={"routed_experts": 4, "router_groups": 2, "router_top_k_min": 1,
                                    "router_top_k_max": 2, "shared_experts": 1,
                                    "long_context": {"global_block_size": 64, "global_slots": 8,
                                                     "rope_local_fraction": 0.6}}),
    }
    return cases


def native_configs():
    """Native training-config dicts exercising from_dict's detection and aliases."""
    return {
        "native_15": {"model_type": "miracle_flashnano", "vocab_size": 32, "hidden_size": 16,
                      "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
                      "intermediate_size": 24, "max_position_embeddings": 32, "local_window_size": 4,
                      "global_attention_layers": [2]},
        "native_16": {"vocab_size": 32, "hidden_size": 16, "layers": 2, "query_heads": 4, "kv_heads": 2,
                      "head_dim": 4, "ffn_dim": 24, "max_positions": 32, "window": 4, "cbr_chunk_size": 3,
                      "cbr_slots": 2},
        "native_17": {"vocab_size": 32, "hidden_size": 16, "layers": 2, "query_heads": 4, "kv_heads": 2,
                      "global_kv_heads": 4, "head_dim": 4, "ffn_dim": 24, "local_window": 4,
                      "max_positions": 32, "global_layer_indices_1based": [2]},
        "native_lite": {"model_type": "miracle_dense", "vocab_size": 32, "hidden_size": 16,
                        "num_hidden_layers": 2, "num_attention_heads": 4, "num_key_value_heads": 2,
                        "head_dim": 4, "intermediate_size": 24, "max_position_embeddings": 32,
                        "attention_window": 4},
        "native_lighting": {"vocab_size": 32, "hidden_size": 16, "num_layers": 2, "num_attention_heads": 4,
                            "num_key_value_heads": 2, "kv_latent_dim": 8, "intermediate_size": 24,
                            "max_position_embeddings": 32, "attention_window": 4, "attention_memory_slots": 2},
        "native_heavy": {"vocab_size": 32, "hidden_size": 16, "num_layers": 2, "num_attention_heads": 4,
                         "num_kv_heads": 2, "head_dim": 4, "latent_kv_dim": 8, "routed_experts": 4,
                         "shared_experts": 1, "expert_intermediate_size": 12, "router_groups": 2,
                         "router_top_k_min": 1, "router_top_k_max": 2,
                         "long_context": {"target_context": 32, "local_window": 4, "global_block_size": 3,
                                          "global_slots": 2}},
    }


def native_name_cases():
    """Micro bundles of every family, tied and untied, with and without Q/K
    norms: the switches the native checkpoint names depend on."""
    cases = {}
    for f in sorted(presets.MICRO):
        for tied in (True, False):
            for qk in (True, False):
                cases[f"{f}-{'tied' if tied else 'untied'}-{'qk' if qk else 'noqk'}"] = dict(
                    presets.micro(f), tie_embeddings=tied, qk_norm=qk)
    return cases


def write_native_names(ref):
    """native_names.json: the reference's own native checkpoint name table
    (weights.py:145-208) for each case of native_name_cases()."""
    from miracle_reasoning.weights import native_names
    out = {}
    for name, bundle in native_name_cases().items():
        try:
            cfg = ref.ModelConfig.from_dict(bundle)
        except ValueError:           # a family that requires Q/K norms
            continue
        out[name] = {"bundle": bundle, "names": native_names(cfg)}
    (HERE / "native_names.json").write_text(json.dumps(out, indent=0, sort_keys=True))
    print("wrote native_names.json", len(out), "cases")


def main():
    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 and sys.argv[1] != "names" else "/root/reference")
    sys.path.insert(0, str(ref_root))
    import miracle_reasoning as ref
    from miracle_reasoning.weights import expected_shapes

    if "names" in sys.argv[1:]:      # only the native name table
        write_native_names(ref)
        return

    ids = list(presets.MICRO_IDS)
    variants = {}
    for f in presets.MICRO:
        variants[f] = (presets.micro(f), None)
        # An untied random head keeps greedy streams from repeating the last token.
        variants[f + "-untied"] = (dict(presets.micro(f), tie_embeddings=False), None)
    # Router weights scaled so probabilities spread and the adaptive width varies.
    variants["heavy-medium-2.0-spread"] = (presets.micro("heavy-medium-2.0"), 30.0)
    # The same heavy geometry with inner blocks of 2 and 3 kept blocks, top-k width 1..3.
    spread3 = presets.micro("heavy-medium-2.0")
    spread3["source"]["router_top_k_max"] = 3
    spread3["source"]["long_context"] = {"global_block_size": 2, "global_slots": 3, "alibi_slope_scale": 0.5}
    variants["heavy-medium-2.0-blocks"] = (dict(spread3, tie_embeddings=False), 30.0)
    for name, (bundle, router_scale) in variants.items():
        weights = synthetic.micro_weights(bundle)
        if router_scale is not None:
            for k in list(weights):
                if ".router." in k and k.endswith(".weight"):
                    weights[k] = (weights[k] * np.float32(router_scale)).astype(np.float32)
        out = run_family(ref, name, bundle, weights, ids)
        np.savez_compressed(HERE / f"micro_{name}.npz", bundle=np.asarray(json.dumps(bundle)),
                            router_scale=np.float32(router_scale or 0), **out)
        print("wrote", name, out["logits"].shape, out["greedy"].tolist())

    # Measurement workload "flashnano-1.5-tiny": 32-token prompt + 16 greedy tokens.
    wl = presets.workload("flashnano-1.5-tiny")
    cfg = ref.ModelConfig.from_dict(wl["config"])
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    prompt = synthetic.prompt_ids(cfg.vocab_size, wl["prompt"], wl["seed"])
    model = ref.MiracleModel(cfg, weights, backend=OracleDevice(), context_length=wl["context"])
    last = model.prefill(prompt)
    stream = model.generate(list(prompt), max_new_tokens=16)
    np.savez_compressed(HERE / "workload_flashnano-1.5-tiny.npz", prompt=prompt, last_logits=last.astype(np.float32),
                        greedy=np.asarray(stream, np.int64))
    print("wrote workload tiny", stream)

    tables = {}
    for name, bundle in rope_cases().items():
        tables[name] = ref.ModelConfig.from_dict(bundle).inverse_frequencies()
    np.savez_compressed(HERE / "rope_tables.npz", **tables)
    (HERE / "rope_cases.json").write_text(json.dumps(rope_cases(), indent=1, sort_keys=True))

    shapes = {}
    for f in presets.MICRO:
        c = ref.ModelConfig.from_dict(presets.micro(f))
        shapes[f] = [[k, list(v)] for k, v in expected_shapes(c).items()]
    (HERE / "shapes.json").write_text(json.dumps(shapes, indent=0))

    parsed = {}
    for name, data in native_configs().items():
        parsed[name] = {"input": data, "parsed": ref.ModelConfig.from_dict(data).to_dict()}
    (HERE / "configs.json").write_text(json.dumps(parsed, indent=1, sort_keys=True))
    write_native_names(ref)
    print("done")


if __name__ == "__main__":
    main()
