"""Loading checkpoints onto the GPU (reference: MiracleModel.from_pretrained,
model.py:58-72; weights.py:14-99, 145-208; config.py:100-117) and the command
line over HIP (cli.py:30-95).

The workload geometries are written to disk as a BF16 safetensors bundle, a
sharded index and a native-name npz (with a native config.json whose family is
auto-detected); each must load with ``from_pretrained`` into a model whose
logits equal, bit for bit, those of the same weights handed over in memory.
"""
import json

import numpy as np
import pytest

from miracle_hip import MiracleModel, ModelConfig, presets, synthetic
from miracle_hip.cli import main
from miracle_hip.weights import BF16Array, SafeTensors, native_names, write_safetensors

pytestmark = pytest.mark.gpu

IDS = [3, 141, 59, 26, 535, 89, 79, 323, 846, 264, 338, 327]


def _write_bundle(directory, config, weights):
    directory.mkdir()
    (directory / "config.json").write_text(json.dumps(config.to_dict()))
    write_safetensors(directory / "model.safetensors", weights)


@pytest.fixture(scope="module")
def mid():
    wl = presets.workload("flashnano-1.5-mid")
    return ModelConfig.from_dict(wl["config"]), synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])


def test_bundle_and_shards_load_bit_exact(backend, tmp_path, mid):
    config, weights = mid
    with MiracleModel(config, weights, backend=backend, context_length=64) as model:
        want = model.prefill(IDS, return_all=True)
        stream = model.generate(IDS, max_new_tokens=4)
    _write_bundle(tmp_path / "bundle", config, weights)
    assert SafeTensors(tmp_path / "bundle" / "model.safetensors").entries["layers.0.q"][1] == "BF16"
    with MiracleModel.from_pretrained(tmp_path / "bundle", backend=backend, context_length=64) as loaded:
        assert loaded.weight_cache.resident == 2 * sum(v.bits.size for v in weights.values()
                                                       if isinstance(v, BF16Array)) + \
            4 * sum(np.asarray(v).size for v in weights.values() if not isinstance(v, BF16Array))
        np.testing.assert_array_equal(loaded.prefill(IDS, return_all=True), want)
    # the same tensors over three shards and an index
    shards = tmp_path / "sharded"
    shards.mkdir()
    (shards / "config.json").write_text(json.dumps(config.to_dict()))
    names = list(weights)
    parts = [names[i::3] for i in range(3)]
    weight_map = {}
    for i, part in enumerate(parts):
        write_safetensors(shards / f"part-{i}.safetensors", {k: weights[k] for k in part})
        weight_map.update({k: f"part-{i}.safetensors" for k in part})
    (shards / "model.safetensors.index.json").write_text(json.dumps({"weight_map": weight_map}))
    with MiracleModel.from_pretrained(shards, backend=backend, context_length=64) as loaded:
        np.testing.assert_array_equal(loaded.prefill(IDS, return_all=True), want)
    # the command line on the bundle
    assert main(["generate", str(tmp_path / "bundle"), "--ids", " ".join(map(str, IDS)), "--max-new-tokens", "4",
                 "--context-length", "64"]) == 0


def test_cli_generate_and_devices(backend, tmp_path, mid, capsys):
    config, weights = mid
    with MiracleModel(config, weights, backend=backend, context_length=64) as model:
        stream = model.generate(IDS, max_new_tokens=5)
        sampled = model.generate(IDS, max_new_tokens=5, temperature=0.7, top_k=20, top_p=0.9, seed=3)
    _write_bundle(tmp_path / "bundle", config, weights)
    capsys.readouterr()
    assert main(["generate", str(tmp_path / "bundle"), "--ids", ",".join(map(str, IDS)), "--max-new-tokens", "5",
                 "--context-length", "64"]) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["token_ids"] == stream and out["device"]["arch"].startswith("gfx950")
    assert main(["generate", str(tmp_path / "bundle"), "--ids", ",".join(map(str, IDS)), "--max-new-tokens", "5",
                 "--context-length", "64", "--temperature", "0.7", "--top-k", "20", "--top-p", "0.9",
                 "--seed", "3"]) == 0
    assert json.loads(capsys.readouterr().out)["token_ids"] == sampled
    assert main(["devices"]) == 0
    devices = json.loads(capsys.readouterr().out)
    assert devices and all(d["arch"].startswith("gfx950") for d in devices)
    assert main(["generate", str(tmp_path / "bundle"), "--ids", "999999", "--context-length", "64"]) == 2
    assert "vocabulary" in capsys.readouterr().err


@pytest.mark.parametrize("case", ["native_15", "native_16", "native_17", "native_heavy", "native_lighting",
                                  "native_lite"])
def test_native_npz_with_native_config_loads_bit_exact(backend, golden_dir, tmp_path, case):
    """A checkpoint under the training repository's names with a native
    config.json (the reference's own native configs; the family is detected
    from their keys) loads like the weights handed over in memory."""
    native_config = json.loads((golden_dir / "configs.json").read_text())[case]["input"]
    config = ModelConfig.from_dict(native_config)
    weights = synthetic.micro_weights(config)
    names = native_names(config)
    directory = tmp_path / case
    directory.mkdir()
    np.savez(directory / "model.npz", **{names[k]: v for k, v in weights.items()})
    (directory / "config.json").write_text(json.dumps(native_config))
    ids = [i % config.vocab_size for i in IDS[:6]]
    with MiracleModel(config, weights, backend=backend, context_length=16) as model:
        want = model.prefill(ids, return_all=True)
    with MiracleModel.from_pretrained(directory, backend=backend, context_length=16) as loaded:
        assert loaded.config == config
        np.testing.assert_array_equal(loaded.prefill(ids, return_all=True), want)


def test_exported_bundles_load_on_the_gpu(backend, tmp_path, mid):
    """Export (reference export.py:41-80) of the flashnano-1.5 mid workload
    from a native-name PyTorch BF16 state dict and from a native-name npz: the
    BF16-keeping bundle loads with from_pretrained into a model whose logits
    equal the in-memory model's bit for bit; the widened FP32 bundle (the
    reference's own format) runs the FP32-weight kernels on the same values,
    so its logits agree within the BF16 tolerance and its greedy stream is the
    same.  The command line's export writes the same bundle."""
    torch = pytest.importorskip("torch")
    from miracle_hip.export import export_checkpoint
    config, weights = mid
    with MiracleModel(config, weights, backend=backend, context_length=64) as model:
        want = model.prefill(IDS, return_all=True)
        stream = model.generate(IDS, max_new_tokens=4)
    names = native_names(config)
    state = {}
    for key, value in weights.items():
        if isinstance(value, BF16Array):
            state[names[key]] = torch.from_numpy(value.bits.view(np.int16)).view(torch.bfloat16)
        else:
            state[names[key]] = torch.from_numpy(np.asarray(value, np.float32))
    torch.save({"model_state_dict": state}, tmp_path / "ckpt.pt")
    (tmp_path / "config.json").write_text(json.dumps(config.to_dict()))
    print("case export torch state dict -> BF16 bundle", flush=True)
    assert export_checkpoint(tmp_path / "ckpt.pt", tmp_path / "config.json", tmp_path / "bf16") == config
    assert SafeTensors(tmp_path / "bf16" / "model.safetensors").entries["layers.0.q"][1] == "BF16"
    with MiracleModel.from_pretrained(tmp_path / "bf16", backend=backend, context_length=64) as loaded:
        np.testing.assert_array_equal(loaded.prefill(IDS, return_all=True), want)
        assert loaded.generate(IDS, max_new_tokens=4) == stream
    print("case export widened FP32 bundle (command line)", flush=True)
    assert main(["export", "--checkpoint", str(tmp_path / "ckpt.pt"), "--config", str(tmp_path / "config.json"),
                 "--output", str(tmp_path / "f32"), "--fp32"]) == 0
    assert SafeTensors(tmp_path / "f32" / "model.safetensors").entries["layers.0.q"][1] == "F32"
    with MiracleModel.from_pretrained(tmp_path / "f32", backend=backend, context_length=64) as loaded:
        np.testing.assert_allclose(loaded.prefill(IDS, return_all=True), want, rtol=1e-3, atol=1e-4)
        assert loaded.generate(IDS, max_new_tokens=4) == stream
    print("case export native npz (FP32 values) -> bundle", flush=True)
    del state
    native = tmp_path / "native"
    native.mkdir()
    np.savez(native / "model.npz", **{names[k]: np.asarray(v, np.float32) for k, v in weights.items()})
    assert export_checkpoint(native / "model.npz", tmp_path / "config.json", tmp_path / "npz") == config
    assert SafeTensors(tmp_path / "npz" / "model.safetensors").entries["layers.0.q"][1] == "F32"
    with MiracleModel.from_pretrained(tmp_path / "npz", backend=backend, context_length=64) as loaded:
        np.testing.assert_allclose(loaded.prefill(IDS, return_all=True), want, rtol=1e-3, atol=1e-4)
        assert loaded.generate(IDS, max_new_tokens=4) == stream
