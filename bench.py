#!/usr/bin/env python3
"""flashnano-1.7 on one MI355X: bs=1 greedy decode tokens/s (+ fraction of the HBM
roofline) and prefill tokens/s.

Workload (seed 2, BF16 random-init weights, synthetic prompt ids): 24 layers,
every 4th global, local ring window 1024, hidden 2048, 16 Q heads x d128,
4 local / 8 global KV heads, split-half RoPE theta 5e5, FFN 5632, vocab 32000,
context 8192.  A 4096-token prompt is prefilled, then K greedy decode steps run
on device (a step = one token through all 24 layers + LM head + argmax; only
the token id crosses to the host).  Default K = 511 = the decode passes of a
512-token generation, positions 4096..4606.

Prints one JSON line.  `value` is decode tokens/s with weights and KV cache
resident in HBM.  `roofline` is for the dominant kernel, timed live with HIP
events: in the persistent step mode the step kernel itself (one launch = one
token, algorithmic bytes B(P) averaged over the decode positions); in the graph
and eager modes the fused RMSNorm + gate/up GEMV + SwiGLU (46.2 MB per launch).
`cpu_baseline` times the oracle (a C restatement of the
reference's OpenCL kernels, FP32 weights resident, the reference's token loop)
on this host's cores for a bounded sample of steps at the GPU's decode positions
(the oracle's K/V rings seated with synthetic rows up to the prompt length), with
the host's CPU model.
"""
import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "miraclereasoning-cpu_amd"))

import numpy as np  # noqa: E402

from miracle_hip import ModelConfig, presets, synthetic  # noqa: E402

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0
WORKLOAD = "flashnano-1.7"
METRIC = "bs=1 decode tok/s + % of HBM roofline; prefill tok/s (flashnano-1.7)"


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def weight_bytes(cfg, dtype_bytes=2):
    """Stored bytes of every tensor read by one decode step (norm gains are FP32)."""
    from miracle_hip.weights import expected_shapes
    total = 0
    for name, shape in expected_shapes(cfg).items():
        n = int(np.prod(shape))
        total += n * (4 if len(shape) == 1 else dtype_bytes)
    return total


def decode_bytes(cfg, context, position, dtype_bytes=2):
    """Algorithmic HBM bytes of one decode step at `position` (0-based).

    GQA families: every projection weight once, the LM head, one embedding
    row, the KV rows the attention reads (FP32), the new K/V rows, the logits.
    flashlighting-2.0: the same weights; the key and value cache rows of every
    latent-memory row (min(position + 1, window + memory slots)).
    heavy-medium-2.0: per inner-loop pass the attention weights, the router and
    the active experts (top-k max routed + shared) again; the window rows and
    the block sums of keys (all blocks) and values (the chosen ones) of that
    pass's cache."""
    from miracle_hip.weights import expected_shapes
    h, d, V = cfg.hidden_size, cfg.head_dim, cfg.vocab_size
    head = V * h * dtype_bytes
    fixed = head + h * dtype_bytes + V * 4   # LM head, embedding row, logits
    shapes = expected_shapes(cfg)

    def tensor(name):
        n = int(np.prod(shapes[name]))
        return n * (4 if len(shapes[name]) == 1 else dtype_bytes)

    if cfg.family == "heavy-medium-2.0":
        src = cfg.source
        active = src["router_top_k_max"] + src["shared_experts"]
        lc = src["long_context"]
        total = fixed + tensor("norm")
        for layer in range(cfg.layers):
            pre = f"layers.{layer}."
            attn = sum(tensor(pre + k) for k in ("a_norm", "q", "o", "latent", "kv_up", "f_norm"))
            router = sum(tensor(n) for n in shapes if n.startswith(pre + "router."))
            expert = sum(tensor(pre + f"experts.0.{k}") for k in ("gate", "up", "down"))
            kvw = cfg.kv_heads * d
            blocks = -(-(position + 1) // lc["global_block_size"])
            kv = (2 * min(position + 1, cfg.window) + blocks + min(lc["global_slots"], blocks) + 4) * kvw * 4
            total += cfg.inner_loop_steps * (attn + router + active * expert + kv)
        return total
    body = weight_bytes(cfg, dtype_bytes) - V * h * dtype_bytes * (1 if cfg.tie_embeddings else 2)
    kv = 0
    for layer in range(cfg.layers):
        kvw = cfg.layer_kv_heads(layer) * d
        if cfg.family == "flashlighting-2.0":
            rows = min(position + 1, cfg.window + cfg.memory_slots)
        else:
            rows = min(position + 1, min(cfg.layer_window(layer) or context, context))
        kv += 2 * rows * kvw * 4 + 2 * kvw * 4
    return body + fixed + kv


def prefill_flops(cfg, context, tokens):
    """Algorithmic FLOPs of a batched prefill of `tokens` from position 0: the
    projections (2 per weight per token), attention scores and mixing
    (4 * query heads * head_dim per query-key pair inside each layer's window,
    and per relay row a query sees in flashnano-1.6) and the LM head of the
    last token."""
    h, d, hq, f, V = cfg.hidden_size, cfg.head_dim, cfg.query_heads, cfg.ffn_dim, cfg.vocab_size
    proj = attn = 0
    for layer in range(cfg.layers):
        kvw = cfg.layer_kv_heads(layer) * d
        proj += h * (hq * d + 2 * kvw) + hq * d * h + 3 * h * f
        cap = min(cfg.layer_window(layer) or context, context)
        keys = sum(min(t + 1, cap) for t in range(tokens))
        if cfg.family == "flashnano-1.6":
            keys += sum((t // cfg.cbr_chunk_size) * cfg.cbr_slots for t in range(tokens))
        attn += 4 * hq * d * keys
    return 2 * tokens * proj + attn + 2 * h * V


def gate_up_bytes(cfg):
    """Algorithmic bytes of one fused RMSNorm + gate/up GEMV + SwiGLU launch."""
    h, f = cfg.hidden_size, cfg.ffn_dim
    return 2 * f * h * 2 + h * 4 + h * 4 + f * 4   # weights + hidden + gain + activations out


def host_cpu():
    """Model name of the host CPU (the first `model name` of /proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_baseline(name, wl, weights, budget_s, position):
    """Oracle token steps on the host (FP32 weights resident, all affine cores),
    at the GPU's decode positions: the oracle is seated at `position` with
    synthetic K/V rows in every ring (GQA families), so each step attends over
    the same row counts as the GPU's decode step there."""
    from oracle import kernels as K
    from oracle.model import OracleModel
    widened = {k: np.asarray(v, dtype=np.float32) for k, v in weights.items()}
    model = OracleModel(wl["config"], widened, context_length=wl["context"])
    ids = synthetic.prompt_ids(wl["config"]["vocab_size"], 256, wl["seed"])
    try:
        model.seat(position, seed=wl["seed"])
        seated = True
    except ValueError:
        seated = False
    start = model.position
    model.step(int(ids[0]))          # first touch of every page of the weights
    n, t0 = 0, time.perf_counter()
    while n < 255 and (n < 4 or time.perf_counter() - t0 < budget_s):
        model.step(int(ids[n + 1]))
        n += 1
    elapsed = time.perf_counter() - t0
    where = (f"positions {start + 1}..{start + n}, rings seated with synthetic K/V rows" if seated
             else f"positions {start + 1}..{start + n}")
    return {"value": round(n / elapsed, 3), "unit": "tok/s", "cores": K.threads(), "kind": "port",
            "cpu": host_cpu(),
            "sample": f"{n} token steps ({where}) of {name} through the oracle's C restatement of "
                      f"the reference kernels, FP32 weights resident, the reference's token-by-token loop; "
                      f"{elapsed:.1f} s"}


def summarize_trace(path, steps):
    """Per-kernel decode summary of a rocprofv3 kernel trace (csv) of this
    bench in eager or graph step mode: the dispatches of the last `steps`
    greedy decode steps (after the steps + 1-th last greedy choice, k_argmax,
    which ends a step), as a markdown table."""
    import collections
    import csv
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]))
    rows.sort()
    ends = [i for i, r in enumerate(rows) if "k_argmax" in r[2]]
    steps = max(1, min(steps, len(ends) - 1))
    dec = rows[ends[-steps - 1] + 1:ends[-1] + 1]
    span = (dec[-1][1] - dec[0][0]) / 1e3
    agg = collections.defaultdict(lambda: [0, 0.0])
    for t0, t1, n in dec:
        n = n.replace("mr::(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        agg[n][0] += 1
        agg[n][1] += (t1 - t0) / 1e3
    tot = sum(v[1] for v in agg.values())
    print(f"decode steps {steps}, span {span:.1f} us ({span / steps:.1f} us per step), kernel time {tot:.1f} us")
    print("| Kernel | Calls per step | Avg µs | µs per step | % of kernel time |")
    print("|---|---|---|---|---|")
    for n, (c, us) in sorted(agg.items(), key=lambda x: -x[1][1]):
        print(f"| `{n}` | {c / steps:.1f} | {us / c:.1f} | {us / steps:.1f} | {100 * us / tot:.1f} |")
    return 0


def summarize_traffic(fetch_csv, write_csv, steps, prompt, commit, name=WORKLOAD):
    """HBM bytes per persistent decode step from two rocprofv3 counter runs of
    this bench with --traffic-probe (FETCH_SIZE, then WRITE_SIZE, in KiB per
    dispatch): the last `steps` k_step dispatches (the timed greedy steps, at
    positions prompt .. prompt + steps - 1), each counter scaled by what it
    reads for the probe's copy of 268,435,456 bytes (the largest copy
    dispatch).  Prints the JSON that bench.py reads into roofline.traffic."""
    import csv

    def read(path, counter):
        rows = []
        with open(path) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter:
                    rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
        rows.sort()
        copy = max(v for _, k, v in rows if "copyBuffer" in k)
        step = [v for _, k, v in rows if "k_step" in k][-steps:]
        return copy, float(np.mean(step)), len(step)

    out = {"kernel": "k_step", "workload": name, "step_mode": "persistent", "commit": commit,
           "positions": [prompt, prompt + steps - 1]}
    total = 0.0
    for key, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        copy_kib, step_kib, n = read(path, counter)
        scale = 268435456 / (copy_kib * 1024)
        out[f"copy_{key}_kib"] = round(copy_kib, 2)
        out[f"step_{key}_kib"] = round(step_kib, 2)
        out[f"{key}_scale"] = round(scale, 6)
        out[f"{key}_bytes"] = int(step_kib * 1024 * scale)
        out["dispatches"] = n
        total += step_kib * 1024 * scale
    out["traffic_bytes"] = int(total)
    print(json.dumps(out, indent=1))
    return 0


def trace_summary(model, cfg, steps, dump=None):
    """Per-phase anatomy of `steps` persistent decode steps (mr_model_trace_step)
    from the model's current position, as a markdown table: for each phase kind
    of local and of global layers, the mean time from the previous phase's last
    workgroup to store its outputs to this phase's last ("phase"), and from that
    same instant to the median workgroup having its input staged ("input") and
    the median first stream wave having stored its rows ("rows")."""
    kinds = ("qkv", "attention", "o", "gate_up", "down")
    acc = {}
    first_pos = model.engine.position()
    raw = []
    for _ in range(steps):
        t = model.engine.trace_step()          # [phases, grid, 5]
        raw.append(t)
        ends = np.nanmax(t[:, :, 2], axis=1)
        total = ends[-1] - np.nanmin(t[0, :, 0])
        acc.setdefault(("step", "-"), []).append((total, np.nan, np.nan))
        for p in range(1, t.shape[0]):
            if p == t.shape[0] - 1:
                key = ("head", "-")
            else:
                layer, k = divmod(p - 1, 5)
                key = (kinds[k], "global" if cfg.layer_window(layer) is None else "local")
            prev = ends[p - 1]
            ready = np.nanmedian(t[p, :, 1]) - prev
            rows = np.nanmedian(t[p, :, 3]) - prev if np.any(np.isfinite(t[p, :, 3])) else np.nan
            acc.setdefault(key, []).append((ends[p] - prev, ready, rows))
    print(f"persistent decode step anatomy: {steps} steps from position {first_pos}, "
          f"{cfg.layers} layers ({sum(cfg.layer_window(i) is None for i in range(cfg.layers))} global)")
    print("| Phase | Layers | Phase µs (mean) | Input staged µs (median WG) | Rows stored µs (median first stream "
          "wave) | Count |")
    print("|---|---|---|---|---|---|")
    order = [(k, s) for k in kinds for s in ("local", "global")] + [("head", "-"), ("step", "-")]

    def fmt(col):
        return "" if np.all(np.isnan(col)) else f"{np.nanmean(col):.2f}"

    for key in order:
        if key not in acc:
            continue
        v = np.array(acc[key])
        print(f"| {key[0]} | {key[1]} | {v[:, 0].mean():.2f} | {fmt(v[:, 1])} | {fmt(v[:, 2])} | {len(v)} |")
    if dump:
        np.save(dump, np.stack(raw))
    return 0


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(presets.WORKLOADS), default=WORKLOAD,
                    help="the measured configuration (default: the headline flashnano-1.7)")
    ap.add_argument("--steps", type=int, default=511, help="timed decode steps")
    ap.add_argument("--warmup", type=int, default=16, help="untimed decode steps before timing")
    ap.add_argument("--prompt", type=int, default=None, help="prompt length (default: the workload's 4096)")
    ap.add_argument("--prefill-mode", choices=("exact", "batched"), default="batched",
                    help="batched: one pass per layer over the prompt (MFMA GEMMs, windowed attention); "
                         "exact: the reference's token loop")
    ap.add_argument("--cpu-seconds", type=float, default=20.0, help="CPU-baseline budget; 0 skips it")
    ap.add_argument("--kernel-reps", type=int, default=3)
    ap.add_argument("--traffic-probe", action="store_true",
                    help="copy 256 MiB device to device once before decoding (the reference dispatch for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--step-mode", choices=("persistent", "graph", "eager"), default="persistent",
                    help="persistent: one cooperative kernel per token step; graph: five kernels per layer "
                         "replayed from a hipGraph; eager: the same kernels launched one by one")
    ap.add_argument("--summarize-trace", metavar="CSV", default=None,
                    help="print the per-kernel summary of the last --steps decode steps in a rocprofv3 kernel "
                         "trace of this bench and exit")
    ap.add_argument("--prefill-only", action="store_true",
                    help="time the prompt's prefill only, print its JSON summary and exit (for counter profiles)")
    ap.add_argument("--trace-steps", type=int, default=0,
                    help="after the prefill, trace this many persistent decode steps phase by phase, print the "
                         "per-phase anatomy (markdown) and exit")
    ap.add_argument("--summarize-traffic", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "COMMIT"), default=None,
                    help="print the per-step HBM traffic JSON (profiles/k_step_<workload>_traffic.json) from two "
                         "rocprofv3 --pmc runs of this bench with --traffic-probe (FETCH_SIZE, WRITE_SIZE) over "
                         "the last --steps step dispatches; COMMIT names the build measured")
    ap.add_argument("--trace-dump", metavar="NPY", default=None,
                    help="with --trace-steps: also save the raw timestamps [steps, phases, workgroups, 5] in µs: "
                         "GEMV phases (entry, input staged, last stream wave stored, first stream wave stored, "
                         "unused); attention phases (entry, Q/K/V cells staged, end, partial stored, a merging "
                         "unit's first partial cells seen)")
    args = ap.parse_args()
    if args.summarize_trace:
        return summarize_trace(args.summarize_trace, args.steps)
    if args.summarize_traffic:
        fetch_csv, write_csv, commit = args.summarize_traffic
        return summarize_traffic(fetch_csv, write_csv, args.steps, args.prompt or presets.workload(WORKLOAD)["prompt"],
                                 commit)
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (this path has no multi-GPU "
              "sharding: bs=1 decode of one sequence runs on one GPU).", file=sys.stderr)
        return 2

    from miracle_hip import HIPBackend, MiracleModel

    name = args.workload
    wl = presets.workload(name)
    cfg = ModelConfig.from_dict(wl["config"])
    gqa = cfg.family in ("flashnano-1.5", "flashnano-1.6", "flashnano-1.7", "flashlite-2.0")
    prefill_mode = args.prefill_mode   # every family has the batched path
    prompt_len = args.prompt or wl["prompt"]
    if prompt_len + (0 if args.prefill_only else args.warmup + args.steps) > wl["context"]:
        raise SystemExit("prompt + warmup + steps exceed the context")
    log("generating synthetic weights")
    weights = synthetic.synthetic_weights(wl["config"], wl["seed"], wl["dtype"])
    prompt = synthetic.prompt_ids(cfg.vocab_size, prompt_len, wl["seed"])
    backend = HIPBackend()
    log(f"device {backend.device.name} {backend.device.arch}, {backend.device.compute_units} CUs")
    model = MiracleModel(cfg, weights, backend=backend, context_length=wl["context"],
                         prefill_mode=args.prefill_mode)
    eng = model.engine
    eng.set_step_mode(args.step_mode)
    step_mode = eng.step_mode()
    log(f"step mode {step_mode}")

    # Prefill: the whole prompt, logits of the last token.
    log(f"prefill {prompt_len} tokens ({prefill_mode})")
    # First launches, graph capture and the batched workspace outside the timed region.
    model.prefill(prompt if prefill_mode == "batched" else prompt[:8])
    model.reset()
    t0 = time.perf_counter()
    model.prefill(prompt)
    prefill_s = time.perf_counter() - t0
    pf_flops = prefill_flops(cfg, wl["context"], prompt_len) if gqa else None
    log(f"prefill {prompt_len / prefill_s:.1f} tok/s" +
        (f", {pf_flops / prefill_s / 1e12:.1f} TFLOP/s algorithmic" if pf_flops else ""))
    if args.prefill_only:
        print(json.dumps({"workload": name, "prompt": prompt_len, "mode": prefill_mode,
                          "tok_s": round(prompt_len / prefill_s, 1), "seconds": round(prefill_s, 4),
                          "algorithmic_tflop": round(pf_flops / 1e12, 3) if pf_flops else None,
                          "achieved_tflops": round(pf_flops / prefill_s / 1e12, 1) if pf_flops else None}),
              flush=True)
        return 0
    if args.trace_steps:
        eng.generate_greedy(args.warmup + 1, -1)    # first launches outside the traced steps
        return trace_summary(model, cfg, args.trace_steps, args.trace_dump)

    if args.traffic_probe:
        n = 64 * 1024 * 1024
        src, dst = backend.empty((n,)), backend.empty((n,))
        backend.copy(src, dst)
        backend.finish()
        del src, dst
        log("traffic probe: copied 268435456 bytes device to device")

    # Warm-up decode steps (captures the greedy step graph), then a fresh sequence.
    eng.generate_greedy(args.warmup + 1, -1)
    model.reset()
    model.prefill(prompt)
    backend.finish()
    t0 = time.perf_counter()
    tokens = eng.generate_greedy(args.steps + 1, -1)      # 1 choice from prefill + `steps` decode steps
    decode_s = time.perf_counter() - t0
    device_ms = eng.last_decode_ms()
    assert len(tokens) == args.steps + 1
    if eng.step_mode() != step_mode:   # a failed persistent step falls back to graph mode
        raise SystemExit(f"bench: the step mode changed from {step_mode} to {eng.step_mode()} while decoding")
    tok_s = args.steps / decode_s
    positions = range(prompt_len, prompt_len + args.steps)
    avg_bytes = float(np.mean([decode_bytes(cfg, wl["context"], p) for p in positions]))
    log(f"decode {tok_s:.1f} tok/s, {avg_bytes * tok_s / 1e9:.1f} GB/s algorithmic")

    # Per-kernel device time (HIP events) of the per-layer kernels, each launched
    # for every layer in turn.
    kinds = ("qkv", "attention", "o", "gate_up", "down", "head") if gqa else ("head",)
    kernels = {k: eng.time_kernel(k, args.kernel_reps) for k in kinds}
    if step_mode == "persistent":
        # The dominant (and only) kernel of a decode step is the step kernel.
        # HBM traffic per launch comes from the committed rocprofv3 counter
        # summary of this kernel and workload (FETCH_SIZE + WRITE_SIZE, scaled
        # by a copy of known size); it is not measured in this run.
        step_ms = device_ms / args.steps
        traffic, measured = None, None
        tf = ROOT / "profiles" / f"k_step_{name}_traffic.json"
        if tf.exists():
            rec = json.loads(tf.read_text())
            traffic = rec.get("traffic_bytes")
            measured = {k: rec.get(k) for k in ("commit", "positions")}
        roof = {"kernel": f"persistent decode step ({cfg.layers} layers + LM head + greedy choice)", "bound": "hbm",
                "achieved": round(avg_bytes / (step_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(avg_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_measured": measured, "algorithmic_bytes": int(avg_bytes), "avg_ms": round(step_ms, 5)}
    elif not gqa:
        # heavy / latent families: the graph-captured step (many small kernels) as one unit
        step_ms = device_ms / args.steps
        roof = {"kernel": f"graph-captured decode step ({cfg.layers} layers + LM head + greedy choice)",
                "bound": "hbm", "achieved": round(avg_bytes / (step_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(avg_bytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes": int(avg_bytes), "avg_ms": round(step_ms, 5)}
    else:
        gu_ms = kernels["gate_up"]
        gu_gbs = gate_up_bytes(cfg) / (gu_ms * 1e-3) / 1e9
        roof = {"kernel": "gemv gate/up + SwiGLU (RMSNorm prologue)", "bound": "hbm", "achieved": round(gu_gbs, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes": gate_up_bytes(cfg), "avg_ms": round(gu_ms, 5)}
    result = {
        "metric": METRIC if name == WORKLOAD else METRIC.replace(WORKLOAD, name), "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(1e3 * decode_s / args.steps, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": name, "weights": f"{wl['dtype']} random-init seed {wl['seed']}", "prompt": prompt_len,
                   "decode_positions": [prompt_len, prompt_len + args.steps - 1], "context": wl["context"],
                   "prefill_mode": prefill_mode, "step_mode": step_mode},
        "decode_hbm": {"algorithmic_bytes_per_token": int(avg_bytes),
                       "achieved_gbs": round(avg_bytes * tok_s / 1e9, 1),
                       "peak_gbs": HBM_PEAK_GBS, "frac": round(avg_bytes * tok_s / 1e9 / HBM_PEAK_GBS, 4)},
        "prefill": {"tok_s": round(prompt_len / prefill_s, 1), "seconds": round(prefill_s, 4),
                    "mode": prefill_mode,
                    "algorithmic_tflop": round(pf_flops / 1e12, 3) if pf_flops else None,
                    "achieved_tflops": round(pf_flops / prefill_s / 1e12, 1) if pf_flops else None,
                    "peak_bf16_dense_tflops": MFMA_BF16_PEAK_TFLOPS,
                    "frac": round(pf_flops / prefill_s / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4) if pf_flops else None},
        "roofline": roof,
        "decode_device_ms": round(device_ms, 3),
        "layer_kernels_ms": {k: round(v, 5) for k, v in kernels.items()},
        "greedy_head": tokens[:8],
    }
    if args.cpu_seconds > 0:
        log("cpu baseline")
        result["cpu_baseline"] = cpu_baseline(name, wl, weights, args.cpu_seconds, prompt_len)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
