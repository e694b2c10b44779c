"""Named model geometries: five measurement workloads and one micro model per family.

All are bundle-format dicts (``backend_format: 1``), loadable by
``ModelConfig.from_dict``.  Fields that the workload descriptions leave open are
fixed here once, so every fixture and every measurement uses the same values.
"""
from __future__ import annotations

import copy


def _bundle(**fields):
    fields.setdefault("backend_format", 1)
    return fields


def _every(n, layers):
    return tuple(range(n, layers + 1, n))


WORKLOADS = {
    # 4 layers, alternating window-64 local / global; FP32 weights (seed 0).
    "flashnano-1.5-tiny": dict(
        config=_bundle(family="flashnano-1.5", vocab_size=4096, hidden_size=256, layers=4, query_heads=8,
                       kv_heads=2, head_dim=32, ffn_dim=768, max_positions=2048, window=64,
                       global_layers=(2, 4), rope_theta=1e4),
        dtype="f32", seed=0, context=2048, prompt=32, new_tokens=64),
    # 19 layers, every 4th global, rest window 512; BF16 (seed 1).
    "flashnano-1.5-mid": dict(
        config=_bundle(family="flashnano-1.5", vocab_size=32000, hidden_size=1024, layers=19, query_heads=16,
                       kv_heads=4, head_dim=64, ffn_dim=2816, max_positions=2048, window=512,
                       global_layers=_every(4, 19), rope_theta=1e4),
        dtype="bf16", seed=1, context=2048, prompt=512, new_tokens=256),
    # flashnano-1.5-mid's geometry with CBR: chunks of 64 positions pooled into 4 relay
    # rows per layer; BF16 (seed 1).
    "flashnano-1.6-mid": dict(
        config=_bundle(family="flashnano-1.6", vocab_size=32000, hidden_size=1024, layers=19, query_heads=16,
                       kv_heads=4, head_dim=64, ffn_dim=2816, max_positions=2048, window=512,
                       global_layers=_every(4, 19), rope_theta=1e4, cbr_chunk_size=64, cbr_slots=4),
        dtype="bf16", seed=1, context=2048, prompt=1024, new_tokens=256),
    # 24 layers, every 4th global, rest ring window 1024; 4 local / 8 global KV heads;
    # split-half RoPE theta 5e5; BF16 (seed 2).
    "flashnano-1.7": dict(
        config=_bundle(family="flashnano-1.7", vocab_size=32000, hidden_size=2048, layers=24, query_heads=16,
                       kv_heads=4, global_kv_heads=8, head_dim=128, ffn_dim=5632, max_positions=8192,
                       window=1024, global_layers=_every(4, 24), rope_theta=5e5),
        dtype="bf16", seed=2, context=8192, prompt=4096, new_tokens=512),
    # 16 layers, latent 256, YaRN x4 over a 4096 native length; window 4096 + 512 memory slots,
    # 16 KV heads, theta 1e6, residual (2L)^-1/2; BF16 (seed 3).
    "flashlighting-2.0": dict(
        config=_bundle(family="flashlighting-2.0", vocab_size=32000, hidden_size=2048, layers=16,
                       query_heads=16, kv_heads=16, head_dim=128, ffn_dim=5632, max_positions=16384,
                       window=4096, latent_dim=256, memory_slots=512, rope_theta=1e6,
                       residual_scale=(2 * 16) ** -0.5,
                       source={"rope_scaling_type": "yarn", "rope_scaling_factor": 4,
                               "max_position_embeddings": 4096}),
        dtype="bf16", seed=3, context=16384, prompt=8192, new_tokens=256),
    # 12 layers, latent 256, window 512, blocks of 64 with top-8; 64 routed experts in 8 groups,
    # top-6 (fixed width) + 2 shared, expert FFN 1024; 2 inner loops; 16/4 heads, d 128; BF16 (seed 4).
    "heavy-medium-2.0": dict(
        config=_bundle(family="heavy-medium-2.0", vocab_size=32000, hidden_size=2048, layers=12,
                       query_heads=16, kv_heads=4, head_dim=128, ffn_dim=1024, max_positions=8192,
                       window=512, latent_dim=256, inner_loop_steps=2, rope_theta=1e6,
                       source={"routed_experts": 64, "router_groups": 8, "router_top_k_max": 6,
                               "router_top_k_min": 6, "shared_experts": 2, "router_temperature": 1.0,
                               "long_context": {"global_block_size": 64, "global_slots": 8,
                                                "rope_local_fraction": 0.6, "alibi_slope_scale": 0.015}}),
        dtype="bf16", seed=4, context=8192, prompt=2048, new_tokens=256),
}

# Micro geometry of the reference's unit tests: V32 h16 L2, 4 Q / 2 KV heads, d 4,
# FFN 24, 32 positions, window 4, layer 2 global (tests/test_inference.py:15-22,
# tests/make_reference.py:19-71 for the per-family extras).
_MICRO_BASE = dict(vocab_size=32, hidden_size=16, layers=2, query_heads=4, kv_heads=2, head_dim=4,
                   ffn_dim=24, max_positions=32, window=4, global_layers=(2,))

MICRO = {
    "flashnano-1.5": _bundle(family="flashnano-1.5", **_MICRO_BASE),
    "flashnano-1.6": _bundle(family="flashnano-1.6", cbr_chunk_size=3, cbr_slots=2, **_MICRO_BASE),
    "flashnano-1.7": _bundle(family="flashnano-1.7", global_kv_heads=4, **_MICRO_BASE),
    "flashlite-2.0": _bundle(family="flashlite-2.0", residual_scale=0.5, **_MICRO_BASE),
    "flashlighting-2.0": _bundle(family="flashlighting-2.0", latent_dim=8, memory_slots=2,
                                 **dict(_MICRO_BASE, global_layers=())),
    "heavy-medium-2.0": _bundle(
        family="heavy-medium-2.0", latent_dim=8, inner_loop_steps=2,
        **dict(_MICRO_BASE, global_layers=(), ffn_dim=12),
        source={"routed_experts": 4, "router_groups": 2, "router_top_k_min": 1, "router_top_k_max": 2,
                "shared_experts": 1,
                "long_context": {"global_block_size": 3, "global_slots": 2}}),
}

MICRO_IDS = (1, 5, 3, 7, 11, 9, 4, 17, 8, 6, 10, 12)


def workload(name):
    return copy.deepcopy(WORKLOADS[name])


def micro(family):
    return copy.deepcopy(MICRO[family])
