"""Checkpoint formats, export and the command line, on the CPU.

Restates the reference's tests/test_weights_config.py:15-72 (safetensors round
trips with exact BF16 widening, truncated and malformed headers rejected,
sharded indexes with path containment, native-name export to a bundle,
``inspect``, config round trip and validation) over this package's readers and
writer, plus what the BF16-keeping writer adds: stored bits survive a round
trip, and ``widen=True`` gives the reference's FP32 bundle.
"""
import json
import struct
from dataclasses import replace

import numpy as np
import pytest

from miracle_hip import ModelConfig, presets, synthetic
from miracle_hip.cli import main
from miracle_hip.export import export_checkpoint
from miracle_hip.weights import (BF16Array, SafeTensors, ShardedSafeTensors, adapt_weights, bf16_bits,
                                 expected_shapes, native_names, write_safetensors)


def _tiny():
    bundle = presets.micro("flashnano-1.5")
    return ModelConfig.from_dict(bundle), synthetic.micro_weights(bundle)


def test_safetensors_roundtrip_and_bfloat16(tmp_path):
    arrays = {"x": np.arange(21, dtype=np.float32).reshape(3, 7), "scale": np.ones(7, np.float32)}
    write_safetensors(tmp_path / "f32.safetensors", arrays)
    mapped = SafeTensors(tmp_path / "f32.safetensors")
    for name, expected in arrays.items():
        np.testing.assert_array_equal(mapped[name], expected)
    # a BF16 file written by hand: widening is exact, whole and sliced
    bits = (arrays["x"].view(np.uint32) >> 16).astype("<u2")
    header = json.dumps({"x": {"dtype": "BF16", "shape": [3, 7], "data_offsets": [0, bits.nbytes]}}).encode()
    (tmp_path / "bf16.safetensors").write_bytes(struct.pack("<Q", len(header)) + header + bits.tobytes())
    bf16 = SafeTensors(tmp_path / "bf16.safetensors")["x"]
    assert isinstance(bf16, BF16Array)
    np.testing.assert_array_equal(bf16[1:2], arrays["x"][1:2])
    np.testing.assert_array_equal(np.asarray(bf16), arrays["x"])


def test_writer_keeps_stored_bits_or_widens(tmp_path):
    rng = np.random.default_rng(3)
    values = rng.normal(size=(5, 9)).astype(np.float32)
    tensors = {"b": BF16Array(bf16_bits(values)), "h": values.astype(np.float16), "f": values,
               "g": np.ones(9, np.float32)}
    write_safetensors(tmp_path / "kept.safetensors", tensors)
    kept = SafeTensors(tmp_path / "kept.safetensors")
    assert {k: kept.entries[k][1] for k in tensors} == {"b": "BF16", "h": "F16", "f": "F32", "g": "F32"}
    np.testing.assert_array_equal(kept["b"].bits, tensors["b"].bits)
    np.testing.assert_array_equal(kept["h"], tensors["h"])
    np.testing.assert_array_equal(kept["f"], values)
    write_safetensors(tmp_path / "wide.safetensors", tensors, widen=True)
    wide = SafeTensors(tmp_path / "wide.safetensors")
    assert {wide.entries[k][1] for k in tensors} == {"F32"}
    np.testing.assert_array_equal(wide["b"], np.asarray(tensors["b"]))
    np.testing.assert_array_equal(wide["h"], tensors["h"].astype(np.float32))
    assert wide.offset % 8 == 0 and kept.offset % 8 == 0
    assert not list(tmp_path.glob("*.partial"))


@pytest.mark.parametrize("payload", [b"", struct.pack("<Q", 1024) + b"{}",
                                     struct.pack("<Q", 62) +
                                     b'{"x":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}}'])
def test_truncated_weights_rejected(tmp_path, payload):
    path = tmp_path / "bad.safetensors"
    path.write_bytes(payload)
    with pytest.raises((ValueError, KeyError)):
        SafeTensors(path)


def _raw(tmp_path, header):
    text = json.dumps(header).encode()
    path = tmp_path / "raw.safetensors"
    path.write_bytes(struct.pack("<Q", len(text)) + text + bytes(16))
    return path


@pytest.mark.parametrize("entry", [
    {"dtype": "I8", "shape": [2], "data_offsets": [0, 2]},            # unsupported dtype
    {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]},           # extent disagrees with the shape
    {"dtype": "F32", "shape": [8], "data_offsets": [0, 32]},          # past the end of the file
    {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]},          # negative dimension
])
def test_malformed_entries_rejected(tmp_path, entry):
    with pytest.raises(ValueError):
        SafeTensors(_raw(tmp_path, {"x": entry}))


def test_overlapping_tensors_rejected(tmp_path):
    header = {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]},
              "b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}
    with pytest.raises(ValueError, match="Overlapping"):
        SafeTensors(_raw(tmp_path, header))


def test_shards_and_path_containment(tmp_path):
    write_safetensors(tmp_path / "part.safetensors", {"x": np.ones((3,), np.float32)})
    index = tmp_path / "model.safetensors.index.json"
    index.write_text(json.dumps({"weight_map": {"x": "part.safetensors"}}))
    np.testing.assert_array_equal(ShardedSafeTensors(index)["x"], np.ones(3))
    index.write_text(json.dumps({"weight_map": {"x": "../outside.safetensors"}}))
    with pytest.raises(ValueError, match="escapes"):
        ShardedSafeTensors(index)
    index.write_text(json.dumps({"weight_map": {"y": "part.safetensors"}}))
    with pytest.raises(ValueError, match="does not contain"):
        ShardedSafeTensors(index)


@pytest.mark.parametrize("family", sorted(presets.MICRO))
def test_native_names_resolve_every_tensor(family):
    config = ModelConfig.from_dict(presets.micro(family))
    weights = synthetic.micro_weights(presets.micro(family))
    names = native_names(config)
    assert set(names) == set(expected_shapes(config))
    assert len(set(names.values())) == len(names)
    native = {names[k]: v for k, v in weights.items()}
    adapted = adapt_weights(config, native)
    for key, value in weights.items():
        np.testing.assert_array_equal(adapted[key], value)
    native.pop(names["norm"])
    with pytest.raises(ValueError, match="Missing"):
        adapt_weights(config, native)


def test_native_names_equal_the_reference_table(golden_dir):
    """native_names equals the reference's own table (weights.py:145-208),
    written by tests/golden/make_golden.py for every family, tied and untied,
    with and without Q/K norms where the family allows both."""
    import json
    cases = json.loads((golden_dir / "native_names.json").read_text())
    assert {c.rsplit("-", 2)[0] for c in cases} == set(presets.MICRO)
    for name, case in cases.items():
        assert native_names(ModelConfig.from_dict(case["bundle"])) == case["names"], name


def test_export_native_npz_to_bundle_and_inspect(tmp_path, capsys):
    config, weights = _tiny()
    source, output = tmp_path / "native", tmp_path / "bundle"
    source.mkdir()
    names = native_names(config)
    np.savez(source / "model.npz", **{names[k]: v for k, v in weights.items()})
    (source / "config.json").write_text(json.dumps(config.to_dict()))
    assert export_checkpoint(source / "model.npz", source / "config.json", output) == config
    bundle = SafeTensors(output / "model.safetensors")
    assert list(bundle) == list(expected_shapes(config))
    for key, value in weights.items():
        np.testing.assert_array_equal(bundle[key], value)
    assert ModelConfig.from_dict(json.loads((output / "config.json").read_text())) == config
    assert main(["inspect", str(output)]) == 0
    shown = json.loads(capsys.readouterr().out)
    assert shown["family"] == config.family
    assert shown["inference_parameters"] == sum(v.size for v in weights.values())
    with pytest.raises(ValueError, match="differ"):
        export_checkpoint(output / "model.safetensors", output / "config.json", output)


def test_export_torch_state_dict_keeps_bfloat16(tmp_path):
    torch = pytest.importorskip("torch")
    bundle = presets.micro("flashnano-1.7")
    config = ModelConfig.from_dict(bundle)
    weights = synthetic.synthetic_weights(bundle, 7, "bf16")
    names = native_names(config)
    state = {}
    for key, value in weights.items():
        if isinstance(value, BF16Array):
            state[names[key]] = torch.from_numpy(value.bits.astype(np.int16)).view(torch.bfloat16)
        else:
            state[names[key]] = torch.from_numpy(np.asarray(value, np.float64))   # cast to FP32 on export
    torch.save({"model_state_dict": state}, tmp_path / "ckpt.pt")
    yaml = pytest.importorskip("yaml")
    (tmp_path / "config.yaml").write_text(yaml.safe_dump(json.loads(json.dumps(config.to_dict()))))
    export_checkpoint(tmp_path / "ckpt.pt", tmp_path / "config.yaml", tmp_path / "out")
    out = SafeTensors(tmp_path / "out" / "model.safetensors")
    for key, value in weights.items():
        if isinstance(value, BF16Array):
            assert out.entries[key][1] == "BF16"
            np.testing.assert_array_equal(out[key].bits, value.bits)
        else:
            assert out.entries[key][1] == "F32"
            np.testing.assert_array_equal(out[key], value)
    torch.save([1, 2], tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="state_dict"):
        export_checkpoint(tmp_path / "bad.pt", tmp_path / "config.yaml", tmp_path / "out2")


def test_cli_errors_exit_with_status_2(tmp_path, capsys):
    assert main(["inspect", str(tmp_path / "missing")]) == 2
    assert "error:" in capsys.readouterr().err
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "miracle_neural"}))
    assert main(["inspect", str(tmp_path)]) == 2
    config, weights = _tiny()
    (tmp_path / "config.json").write_text(json.dumps(config.to_dict()))
    assert main(["generate", str(tmp_path), "--prompt", "hello"]) == 2
    assert "--tokenizer" in capsys.readouterr().err


def test_config_roundtrip_and_validation():
    config, _ = _tiny()
    assert ModelConfig.from_dict(json.loads(json.dumps(config.to_dict()))) == config
    for changes in ({"head_dim": 3}, {"query_heads": 3}, {"layers": True}, {"window": 0},
                    {"norm_eps": float("nan")}, {"global_layers": (0,)}, {"family": "miracle-neural"}):
        with pytest.raises(ValueError):
            replace(config, **changes)
    with pytest.raises(ValueError, match="scope"):
        ModelConfig.from_dict({"model_type": "miracle_neural"})
