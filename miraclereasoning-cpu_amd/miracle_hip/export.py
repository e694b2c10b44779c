"""Checkpoint -> standalone bundle (``config.json`` + ``model.safetensors``
under canonical names), offline and without executing anything stored in the
checkpoint.

Same inputs and outcome as the reference's exporter (export.py:41-80): a
JSON or YAML config (native or bundle keys), and weights as safetensors, a
sharded safetensors index, a numpy ``.npz`` or a PyTorch state dict (loaded
with ``weights_only=True``).  The bundle keeps each tensor's stored dtype, so
BF16 checkpoints stay BF16 (the HIP engine keeps BF16 resident in HBM and
widens in registers); ``widen=True`` writes FP32 throughout, the reference's
own bundle format.  Both load in either implementation.
"""
from __future__ import annotations

import json
from collections.abc import Mapping
from pathlib import Path

import numpy as np

from .config import ModelConfig
from .weights import BF16Array, SafeTensors, ShardedSafeTensors, adapt_weights, write_safetensors

_WRAPPERS = ("state_dict", "model_state_dict", "parameters", "model")


class _StateDict(Mapping):
    """A PyTorch state dict seen as numpy arrays, one tensor converted at a
    time: bfloat16 keeps its bits (BF16Array), float16 and float32 are viewed
    as they are, other dtypes are cast to float32 when read."""

    def __init__(self, tensors):
        self.tensors = tensors

    def __iter__(self):
        return iter(self.tensors)

    def __len__(self):
        return len(self.tensors)

    def __getitem__(self, key):
        import torch
        t = self.tensors[key].detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            return BF16Array(t.view(torch.int16).numpy().view(np.uint16))
        if t.dtype in (torch.float16, torch.float32):
            return t.numpy()
        return t.float().numpy()


def _read_config(path, family):
    text = path.read_text(encoding="utf-8")
    if path.suffix.lower() in (".yaml", ".yml"):
        import yaml
        values = yaml.safe_load(text)
    else:
        values = json.loads(text)
    return ModelConfig.from_dict(values, family)


def _open_weights(checkpoint):
    name = checkpoint.name
    if name.endswith(".safetensors.index.json"):
        return ShardedSafeTensors(checkpoint)
    if checkpoint.suffix == ".safetensors":
        return SafeTensors(checkpoint)
    if checkpoint.suffix == ".npz":
        return np.load(checkpoint, allow_pickle=False)
    import torch
    payload = torch.load(checkpoint, map_location="cpu", weights_only=True, mmap=True)
    if isinstance(payload, dict):
        for key in _WRAPPERS:
            if isinstance(payload.get(key), dict):
                payload = payload[key]
                break
    if not isinstance(payload, dict) or not all(isinstance(v, torch.Tensor) for v in payload.values()):
        raise ValueError("Checkpoint must contain a tensor state_dict (or parameters/model wrapper)")
    return _StateDict(payload)


def export_checkpoint(checkpoint, config_path, output, *, family=None, widen=False):
    """Write ``output/config.json`` and ``output/model.safetensors``; returns the
    parsed ``ModelConfig``.  Every tensor and shape is checked before anything
    is written, and neither file is replaced unless both are complete."""
    checkpoint, config_path, output = Path(checkpoint), Path(config_path), Path(output)
    config = _read_config(config_path, family)
    weights = adapt_weights(config, _open_weights(checkpoint))
    target = output / "model.safetensors"
    if target.exists() and checkpoint.resolve() == target.resolve():
        raise ValueError("Export output must differ from the input checkpoint path")
    output.mkdir(parents=True, exist_ok=True)
    from .weights import expected_shapes
    staged = output / "model.safetensors.export"
    config_staged = output / "config.json.export"
    try:
        write_safetensors(staged, {name: weights[name] for name in expected_shapes(config)}, widen=widen)
        config_staged.write_text(json.dumps(config.to_dict(), indent=2, ensure_ascii=False) + "\n",
                                 encoding="utf-8")
        staged.replace(target)
        config_staged.replace(output / "config.json")
    finally:
        staged.unlink(missing_ok=True)
        config_staged.unlink(missing_ok=True)
    return config
