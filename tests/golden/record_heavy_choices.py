"""Record the HIP engine's heavy-medium-2.0 routing and block choices over the
workload's 2048-token prompt and a 6-token greedy stream (run on an MI355X):

    python tests/golden/record_heavy_choices.py OUT.npz

The oracle at this length takes longer than a GPU test may run, so the check
is split: this script records what the device chose; make_workload_golden.py
then runs the oracle in the build container following that record (adopting a
recorded choice only where it is a valid choice within the oracle's near-tie
band, logging anything else as a mismatch) and writes the fixture that
tests/test_hip_workloads.py compares the device against.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO / "miraclereasoning-cpu_amd"))

from miracle_hip import MiracleModel, ModelConfig, presets, synthetic  # noqa: E402

PROMPT = 2048
STREAM = 6


def main(out):
    wl = presets.workload("heavy-medium-2.0")
    cfg = ModelConfig.from_dict(wl["config"])
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    ids = synthetic.prompt_ids(cfg.vocab_size, PROMPT, wl["seed"])
    with MiracleModel(cfg, weights, context_length=wl["context"], prefill_mode="batched") as model:
        last = model.prefill(ids)
        stream = model.generate(list(ids), max_new_tokens=STREAM)
        choices = model.engine.choices()
    np.savez_compressed(out, prompt=np.int64(PROMPT), choices=choices, stream=np.asarray(stream, np.int64),
                        last=np.asarray(last, np.float32))
    print(f"recorded {choices.shape} choices, stream {stream}", flush=True)


if __name__ == "__main__":
    main(sys.argv[1])
