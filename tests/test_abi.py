"""CPU checks of the drop-in boundary: the built library loads and exports every
function include/miracle_hip.h declares; the Python binding's signature table
covers them; the backend refuses to run without a gfx950 GPU (no fallback);
weights are validated before any device work."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from miracle_hip import HIPBackend, HIPError, MiracleModel, ModelConfig, presets, synthetic
from miracle_hip import hip

HEADER = Path(__file__).resolve().parents[1] / "include" / "miracle_hip.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^MR_API [^;]*?\b(mr_\w+)\(", text, re.M)))


def test_header_declares_the_abi():
    names = declared()
    assert "mr_model_forward" in names and "mr_linear" in names and len(names) >= 30


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(hip.library_path()))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    covered = set(hip._SIGNATURES) | {"mr_last_error"}
    assert set(declared()) <= covered, set(declared()) - covered


def test_descriptor_layout_matches_header():
    # mr_model_desc: 19 int32, 3 float, 7 int32, 2 float, 2 uint64, 4 float -> 31*4 + 4 pad + 16 + 16 = 160
    assert ctypes.sizeof(hip.ModelDesc) == 160
    assert ctypes.sizeof(hip._DeviceInfo) == 256 + 64 + 16 + 24


def test_no_gpu_means_hip_error_not_fallback():
    if hip.list_devices():
        pytest.skip("a GPU is visible")
    with pytest.raises(HIPError, match="no CPU fallback"):
        HIPBackend()


def test_bad_weights_rejected_before_device_allocation():
    # reference tests/test_inference.py:102-106
    bundle = presets.micro("flashnano-1.5")
    weights = synthetic.micro_weights(bundle)
    weights["layers.0.k"] = np.zeros((7, 16), np.float32)
    with pytest.raises(ValueError, match="expected"):
        MiracleModel(ModelConfig.from_dict(bundle), weights)


def test_weight_name_mapping_covers_every_family():
    from miracle_hip.model import weight_target
    from miracle_hip.weights import expected_shapes
    for family in presets.MICRO:
        for name in expected_shapes(ModelConfig.from_dict(presets.micro(family))):
            kind, layer, expert = weight_target(name)
            assert 0 <= kind < 29 and layer >= -1 and expert >= -1
