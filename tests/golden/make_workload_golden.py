"""Write oracle fixtures for the measured workloads at their full prompt length.

Run in the build container (CPU only; the oracle is the checker):

    python tests/golden/make_workload_golden.py [flashnano-1.7]

For each named workload it builds the frozen synthetic weights and prompt
(miracle_hip.presets / miracle_hip.synthetic), runs the oracle's token loop
(oracle/model.py over oracle/kernels.c, the reference's per-token path) over
the whole prompt and then greedy decoding, and writes
``workload_<name>-p<prompt>.npz`` with

* ``prompt``, ``seed``, ``ids_sum``: the prompt length, the workload seed and
  the sum of the prompt ids (a check that the same ids are regenerated);
* ``last``: FP32 logits of the last prompt position;
* ``decode``: FP32 logits of the next ``DECODE`` positions, each after feeding
  the previous greedy token (the positions ``bench.py`` decodes at);
* ``stream``: the greedy stream of ``STREAM`` tokens that continues the prompt
  (generate's rule: argmax, stop at EOS).

heavy-medium-2.0 (2048-token prompt) makes discrete choices whose near-ties
two exact FP32 evaluations in different orders can break either way, so its
fixture follows a record of the device's own choices:

    python tests/golden/make_workload_golden.py heavy-medium-2.0 RECORD.npz

where RECORD.npz comes from tests/golden/record_heavy_choices.py on an
MI355X.  The oracle follows the record where it is a valid choice within its
near-tie band and logs anything else as a mismatch (the script then refuses
to write); the fixture keeps the validated record (``choices``), the adopted
near-ties (``adopted``: position, layer, inner loop, head or -1 for experts;
``adopted_gap``), the smallest decision margins, and the oracle's ``last``
logits and greedy ``stream`` along that path.

Only inputs and outputs are written.  The oracle takes 10-40 minutes per
workload on 8 cores at these lengths, far too long for a GPU test, which
compares against these fixtures instead.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "miraclereasoning-cpu_amd"))

from miracle_hip import presets, synthetic  # noqa: E402
from oracle.model import OracleModel  # noqa: E402

DECODE = 4
STREAM = 8
# flashlighting-2.0 at 4700 tokens: its latent memory is full (window 4096 + 512 memory slots +
# the new row = 4609 rows, compacting every step), as at the bench's positions 8192.., at a
# prompt length the oracle can reach (with its per-row latent K/V cache, pinned bit-exact against
# the recomputing form).
PROMPTS = {"flashnano-1.7": 4096, "flashlighting-2.0": 4700}


def _bits(weights):
    return {k: (v.bits if hasattr(v, "bits") else v) for k, v in weights.items()}


def fixture_path(name, prompt):
    return HERE / f"workload_{name}-p{prompt}.npz"


def write(name, prompt):
    wl = presets.workload(name)
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    ids = synthetic.prompt_ids(wl["config"]["vocab_size"], prompt, wl["seed"])
    ref = OracleModel(wl["config"], _bits(weights), context_length=wl["context"],
                      latent_kv_cache=wl["config"]["family"] == "flashlighting-2.0")
    t0 = time.time()
    last = None
    for begin in range(0, prompt, 256):
        last = ref.prefill(ids[begin:begin + 256])
        print(f"{name}: oracle {min(begin + 256, prompt)}/{prompt} tokens, {time.time() - t0:.0f} s", flush=True)
    eos = ref.cfg.eos_token_id
    stream, decode, logits = [], [], last
    for i in range(STREAM):
        tok = int(np.argmax(logits))
        stream.append(tok)
        if tok == eos or i == STREAM - 1:
            break
        logits = ref.decode(tok)
        if len(decode) < DECODE:
            decode.append(logits)
    path = fixture_path(name, prompt)
    np.savez(path, prompt=np.int64(prompt), seed=np.int64(wl["seed"]), ids_sum=np.int64(np.sum(ids, dtype=np.int64)),
             last=np.asarray(last, np.float32), decode=np.asarray(decode, np.float32),
             stream=np.asarray(stream, np.int64))
    print(f"{name}: wrote {path.name}: stream {stream}, {time.time() - t0:.0f} s", flush=True)


def write_heavy(record_path):
    import math
    name = "heavy-medium-2.0"
    rec = np.load(record_path)
    prompt, choices = int(rec["prompt"]), rec["choices"]
    wl = presets.workload(name)
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    ids = synthetic.prompt_ids(wl["config"]["vocab_size"], prompt, wl["seed"])
    trace = []
    ref = OracleModel(wl["config"], _bits(weights), context_length=wl["context"], trace=trace, follow=choices)
    t0 = time.time()
    last = None
    for begin in range(0, prompt, 128):
        last = ref.prefill(ids[begin:begin + 128])
        print(f"{name}: oracle {min(begin + 128, prompt)}/{prompt} tokens, {time.time() - t0:.0f} s, "
              f"adopted {len(ref.adopted)}, mismatches {len(ref.mismatches)}", flush=True)
    eos = ref.cfg.eos_token_id
    stream, logits = [], last
    for i in range(len(rec["stream"])):
        tok = int(np.argmax(logits))
        stream.append(tok)
        if tok == eos or i == len(rec["stream"]) - 1:
            break
        logits = ref.decode(tok)
    if ref.mismatches:
        raise SystemExit(f"mismatches against the record: {ref.mismatches[:10]}")
    blocks = [r for r in trace if r[0] == "blocks"]
    experts = [r for r in trace if r[0] == "experts"]
    real = [r[4] for r in blocks if math.isfinite(r[4])]
    adopted = np.asarray([(a[2], a[1], a[3], a[4] if a[0] == "blocks" else -1) for a in ref.adopted],
                         np.int64).reshape(-1, 4)
    gaps = np.asarray([a[-1] for a in ref.adopted], np.float64)
    path = HERE / f"workload_{name}-p{prompt}.npz"
    np.savez_compressed(path, prompt=np.int64(prompt), seed=np.int64(wl["seed"]),
                        ids_sum=np.int64(np.sum(ids, dtype=np.int64)), choices=choices.astype(np.int8),
                        adopted=adopted, adopted_gap=gaps, decisions=np.int64(len(blocks) + len(experts)),
                        block_margin=np.float64(min(real)), router_margin=np.float64(min(r[5] for r in experts)),
                        last=np.asarray(last, np.float32), stream=np.asarray(stream, np.int64))
    print(f"{name}: wrote {path.name} ({path.stat().st_size} bytes): stream {stream} (device {rec['stream'].tolist()}), "
          f"{len(blocks) + len(experts)} decisions, adopted {ref.adopted}, {time.time() - t0:.0f} s", flush=True)


if __name__ == "__main__":
    if sys.argv[1:2] == ["heavy-medium-2.0"]:
        write_heavy(sys.argv[2])
    else:
        for n in sys.argv[1:] or sorted(PROMPTS):
            write(n, PROMPTS[n])
