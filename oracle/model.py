"""ORACLE (test infrastructure only): one sequence's forward path on the CPU.

A restatement of the reference engine (miracle_reasoning/model.py) over the
C kernels in oracle/kernels.c, numpy arrays standing in for device buffers.
Host control (MoE routing, block top-k, latent compaction bookkeeping) is the
same numpy float32 arithmetic the reference performs on its host.

Pinned by: golden per-token logits, greedy streams, chosen experts / active
widths, chosen blocks and latent-cache metadata, written by
tests/golden/make_golden.py from the reference's own model.py for micro
configurations of all six families (tests/test_oracle_model.py), and by the
reference's invariants (decode == prefill bit-exact, ring lengths, relay count,
latent rows, loop caches; tests/test_inference.py:42-69 of the reference).
"""
from __future__ import annotations

import math

import numpy as np

from . import kernels as K
from .config import OracleConfig, inverse_frequencies, weight_shapes


class _Ring:
    """Circular KV buffer: slot of the next row is count % capacity (model.py:15-33)."""

    def __init__(self, capacity, width):
        self.k = np.zeros((capacity, width), np.float32)
        self.v = np.zeros((capacity, width), np.float32)
        self.capacity, self.count = capacity, 0

    def push(self, key, value):
        slot = self.count % self.capacity
        self.k[slot] = key.reshape(-1)
        self.v[slot] = value.reshape(-1)
        self.count += 1

    @property
    def length(self):
        return min(self.count, self.capacity)

    @property
    def start(self):
        return (self.count - self.length) % self.capacity


def _widen(array):
    """Weights are held as FP32 or as BF16 bits (uint16); 1-D tensors are widened."""
    if array.dtype == np.uint16:
        return (array.astype(np.uint32) << 16).view(np.float32)
    return np.asarray(array, np.float32)


class OracleModel:
    """Same call surface as the reference engine: prefill / decode / generate / reset.

    ``weights`` maps canonical names to FP32 arrays or BF16 bit arrays (uint16).
    ``trace`` (optional list) receives per-step routing and block-selection
    records for parity checks of discrete decisions.

    ``follow`` (optional): another implementation's record of its heavy-medium
    choices, int32 [positions, layers, inner loops, record] with a record of
    (width, the experts in chosen order, -1 past the width, then per query head
    its chosen blocks ascending, -1 padded).  Two exact FP32 evaluations of the
    same formulas in different summation orders differ in the last bits, so a
    choice between values that close can come out either way.  Where the
    recorded choice differs from the oracle's own, the oracle checks it against
    its own values: if it is a valid choice within ``NEAR_TIE`` (relative to
    the compared values) the oracle adopts it, so both continue on the same
    path, and logs the event in ``adopted``; otherwise it keeps its own choice
    and logs the event in ``mismatches``.
    """

    NEAR_TIE = 1e-4

    def __init__(self, config, weights, context_length=None, trace=None, follow=None, latent_kv_cache=False):
        cfg = config if isinstance(config, OracleConfig) else OracleConfig.from_bundle(config)
        # FlashLighting: the reference recomputes every latent row's key and
        # value at every step (model.py:160-163).  Row r's key and value
        # depend only on its latent and stored position (every kernel involved
        # computes each row on its own), so with latent_kv_cache a row keeps
        # them from the step it was appended (or merged) on: the same bits at
        # a fraction of the cost, for long prompts; pinned against the
        # recomputing form by tests/test_oracle_model.py.
        self.latent_kv_cache = latent_kv_cache
        self.cfg = cfg
        self.ctx = context_length if context_length is not None else min(2048, cfg.max_positions)
        if not 0 < self.ctx <= cfg.max_positions:
            raise ValueError("context_length out of range")
        self.w = {}
        for name, shape in weight_shapes(cfg).items():
            a = weights[name]
            a = np.ascontiguousarray(a if getattr(a, "dtype", None) == np.uint16 else np.asarray(a, np.float32))
            if tuple(a.shape) != shape:
                raise ValueError(f"{name}: expected {shape}, got {a.shape}")
            self.w[name] = _widen(a) if len(shape) == 1 else a
        self.freq = inverse_frequencies(cfg)
        self.trace = trace
        self.follow = follow
        self.adopted, self.mismatches = [], []
        self._loop = 0
        self.reset()

    # ---------------------------------------------------------------- helpers
    def reset(self):
        self.position = 0
        self.failed = False
        self.layers = [dict() for _ in range(self.cfg.layers)]

    def seat(self, position, seed=0):
        """Place a GQA model (flashnano-1.5 / 1.7 / lite) at `position` with
        synthetic standard-normal K/V rows in every layer's ring, as if
        `position` tokens had been pushed: the next step then attends over the
        same row counts as a decode step at that position.  For timing only;
        the rows stand for no token sequence."""
        c = self.cfg
        if c.family in ("flashnano-1.6", "heavy-medium-2.0", "flashlighting-2.0"):
            raise ValueError(f"seat: {c.family} keeps state beyond the K/V rings")
        if not 0 <= position < self.ctx:
            raise ValueError("seat: position outside the context")
        rng = np.random.default_rng(seed)
        self.reset()
        for layer, state in enumerate(self.layers):
            ring = state["ring"] = _Ring(min(c.window_of(layer) or self.ctx, self.ctx),
                                         c.kv_heads_of(layer) * c.head_dim)
            rows = min(position, ring.capacity)
            ring.k[:rows] = rng.standard_normal((rows, ring.k.shape[1]), np.float32)
            ring.v[:rows] = rng.standard_normal((rows, ring.v.shape[1]), np.float32)
            ring.count = position
        self.position = position

    def _rms(self, x, name, width=None, eps=None):
        c = self.cfg
        return K.rms(x, self.w[name] if name else None, width or c.hidden_size,
                     c.norm_eps if eps is None else eps)

    def _rope(self, x, positions, heads):
        return K.rope(x, self.freq, positions, heads, self.cfg.head_dim, self.cfg.split_half)

    def _mlp(self, x, root):
        g = K.linear(x, self.w[root + "gate"])
        u = K.linear(x, self.w[root + "up"])
        return K.linear(K.swiglu(g, u), self.w[root + "down"])

    # ------------------------------------------------ GQA (1.5 / 1.6 / 1.7 / lite)
    def _gqa(self, x, layer, state, pos):
        c, p = self.cfg, f"layers.{layer}."
        kvh = c.kv_heads_of(layer)
        q = K.linear(x, self.w[p + "q"])
        k = K.linear(x, self.w[p + "k"])
        v = K.linear(x, self.w[p + "v"])
        if c.qk_norm:
            q = self._rms(q, p + "q_norm", c.head_dim)
            k = self._rms(k, p + "k_norm", c.head_dim)
        q = self._rope(q, pos, c.query_heads)
        k = self._rope(k, pos, kvh)
        ring = state.get("ring")
        if ring is None:
            ring = state["ring"] = _Ring(min(c.window_of(layer) or self.ctx, self.ctx), kvh * c.head_dim)
        ring.push(k, v)
        relay = state.get("relay")
        attended = K.attention(q, ring.k, ring.v, c.query_heads, kvh, c.head_dim, ring.start, ring.length,
                               relay["k"] if relay else None, relay["v"] if relay else None,
                               relay["count"] if relay else 0)
        if c.family == "flashnano-1.6":
            self._cbr(x, layer, state, kvh)
        return K.linear(attended, self.w[p + "o"])

    def _cbr(self, x, layer, state, kvh):
        """Chunk pooling into relay keys (model.py:118-144)."""
        c, p = self.cfg, f"layers.{layer}."
        chunk, slots, h = c.cbr_chunk_size, c.cbr_slots, c.hidden_size
        if "pending" not in state:
            state["pending"] = np.zeros((min(chunk, self.ctx), h), np.float32)
        row = self.position % chunk
        state["pending"][row] = x.reshape(-1)
        if row != chunk - 1:
            return
        # the learned queries as FP32 values (the reference reads them widened,
        # model.py:126); BF16 ones are held as bits like every matrix here
        queries = K.rms(_widen(self.w[p + "cbr"]), None, h, c.cbr_norm_eps)
        probs = K.softmax(K.pool_scores(state["pending"], queries, chunk, slots, h))
        pooled, anchors = K.pool_mix(state["pending"], probs, chunk, slots, h, self.position + 1 - chunk)
        key = K.linear(pooled, self.w[p + "k"])
        value = K.linear(pooled, self.w[p + "v"])
        key = self._rope(self._rms(key, p + "k_norm", c.head_dim), anchors, kvh)
        relay = state.get("relay")
        if relay is None:
            cap = (self.ctx // chunk) * slots
            width = kvh * c.head_dim
            relay = state["relay"] = {"k": np.zeros((cap, width), np.float32),
                                      "v": np.zeros((cap, width), np.float32), "count": 0}
        n = relay["count"]
        relay["k"][n:n + slots] = key
        relay["v"][n:n + slots] = value
        relay["count"] = n + slots

    # ------------------------------------------------------- flashlighting-2.0
    def _lighting(self, x, layer, state, pos):
        """Latent attention with memory compaction (model.py:146-190)."""
        c, p = self.cfg, f"layers.{layer}."
        q = self._rope(self._rms(K.linear(x, self.w[p + "q"]), p + "q_norm", c.head_dim), pos, c.query_heads)
        latent = self._rms(K.linear(x, self.w[p + "latent"]), p + "latent_norm", c.latent_dim)
        old = state.get("latent")
        rows = latent if old is None else np.concatenate([old, latent])
        n1 = rows.shape[0]
        positions = state.get("positions", []) + [self.position]
        counts = state.get("counts", []) + [1.0]
        key_pos = np.asarray(positions, np.float32)

        def kv(r, at):
            return (self._rope(self._rms(K.linear(r, self.w[p + "k"]), p + "k_norm", c.head_dim), at, c.kv_heads),
                    K.linear(r, self.w[p + "v"]))

        if self.latent_kv_cache:
            # rows [lo, hi) of two buffers hold the cached keys and values in
            # row order; rows leave at the front and arrive at the back, and the
            # live rows move to the front when the back is reached
            if old is None:
                cap = 2 * (c.window + c.memory_slots + 2)
                state.update(kbuf=np.zeros((cap, c.kv_heads * c.head_dim), np.float32),
                             vbuf=np.zeros((cap, c.kv_heads * c.head_dim), np.float32), lo=0, hi=0)
            kb, vb = state["kbuf"], state["vbuf"]
            if state["hi"] == kb.shape[0]:
                n = state["hi"] - state["lo"]
                kb[:n], vb[:n] = kb[state["lo"]:state["hi"]].copy(), vb[state["lo"]:state["hi"]].copy()
                state.update(lo=0, hi=n)
            kb[state["hi"]], vb[state["hi"]] = (a.reshape(-1) for a in kv(latent, key_pos[-1:]))
            state["hi"] += 1
            key, value = kb[state["lo"]:state["hi"]], vb[state["lo"]:state["hi"]]
        else:
            key, value = kv(rows, key_pos)
        s = K.scores(q, key, None, c.query_heads, c.kv_heads, c.head_dim, n1, 0, n1, 0)
        K.latent_mask(s, key_pos, c.query_heads, n1, state.get("memory_size", 0), self.position - c.window + 1)
        attended = K.mix(K.softmax(s), value, None, c.query_heads, c.kv_heads, c.head_dim, n1, 0, n1, 0)
        overflow = max(0, n1 - c.window)
        if c.memory_slots == 0 and overflow:
            rows, positions, counts, memory = rows[overflow:], positions[overflow:], counts[overflow:], 0
            if self.latent_kv_cache:
                state["lo"] += overflow
        elif overflow > c.memory_slots:
            a, b = np.float32(counts[0]), np.float32(counts[1])
            merged = K.merge_rows(rows[:2], c.latent_dim, float(a), float(b))
            rows = np.concatenate([merged[None, :], rows[2:]])
            centre = np.float32(np.float32(positions[0]) * a + np.float32(positions[1]) * b) / np.float32(a + b)
            positions = [int(np.rint(centre))] + positions[2:]
            counts = [float(a + b)] + counts[2:]
            memory = c.memory_slots
            if self.latent_kv_cache:   # rows 0 and 1 become the merged row at its rounded position
                k0, v0 = kv(np.ascontiguousarray(merged[None, :]), np.asarray(positions[:1], np.float32))
                state["lo"] += 1
                state["kbuf"][state["lo"]], state["vbuf"][state["lo"]] = k0.reshape(-1), v0.reshape(-1)
        else:
            memory = overflow
        state.update(latent=np.ascontiguousarray(rows), positions=positions, counts=counts, memory_size=memory)
        return K.linear(attended, self.w[p + "o"])

    # -------------------------------------------------------- heavy-medium-2.0
    def _heavy_attention(self, x, layer, state, pos):
        """Window + block-mean sparse attention (model.py:192-229)."""
        c, p = self.cfg, f"layers.{layer}."
        d, H, kvh = c.head_dim, c.query_heads, c.kv_heads
        width = kvh * d
        q = K.rms(K.linear(x, self.w[p + "q"]), None, d, 1e-6)
        kv = K.linear(K.linear(x, self.w[p + "latent"]), self.w[p + "kv_up"])
        key, value = kv[:, :width], kv[:, width:]
        q = self._rope(q, pos, H)
        key = self._rope(K.rms(key, None, d, 1e-6), pos, kvh)
        ring = state.get("ring")
        if ring is None:
            ring = state["ring"] = _Ring(self.ctx, width)
        ring.push(key, value)
        count = ring.count
        length = min(c.window, count)
        start = count - length
        lc = c.source["long_context"]
        block = lc["global_block_size"]
        blocks = (count + block - 1) // block
        mk = K.block_means(ring.k, count, width, block)
        mv = K.block_means(ring.v, count, width, block)
        s = K.scores(q, ring.k, mk, H, kvh, d, ring.capacity, start, length, blocks)
        ends = np.minimum((np.arange(blocks) + 1) * block - 1, self.position)
        slope = np.float32(lc.get("alibi_slope_scale", 0.015) / math.sqrt(d))
        s[:, length:] -= slope * np.log1p((self.position - ends).astype(np.float32))
        keep = min(lc["global_slots"], blocks)
        order = np.argsort(-s[:, length:], axis=1, kind="stable")
        if self.trace is not None:
            # margin: smallest score gap across the slot boundary over the heads
            # (inf when every block is kept, so there is no choice to flip)
            ranked = np.take_along_axis(s[:, length:], order, axis=1)
            margin = float((ranked[:, keep - 1] - ranked[:, keep]).min()) if blocks > keep else math.inf
            self.trace.append(("blocks", layer, self.position, [sorted(order[h, :keep].tolist()) for h in range(H)],
                               margin))
        kept = [order[h, :keep] for h in range(H)]
        if self.follow is not None and blocks > keep:
            self._follow_blocks(layer, s[:, length:], kept, blocks)
        for h in range(H):
            drop = np.ones(blocks, bool)
            drop[kept[h]] = False
            s[h, length + np.flatnonzero(drop)] = -np.inf
        attended = K.mix(K.softmax(s), ring.v, mv, H, kvh, d, ring.capacity, start, length, blocks)
        return K.linear(attended, self.w[p + "o"])

    def _moe(self, x, layer):
        """Grouped adaptive routing + experts + shared experts (model.py:231-255)."""
        c, p, s = self.cfg, f"layers.{layer}.", self.cfg.source
        E, G = s["routed_experts"], s["router_groups"]
        coarse = K.linear(x, self.w[p + "router.coarse.weight"])[0]
        fine = K.linear(x, self.w[p + "router.fine.weight"])[0]
        coarse = coarse + (self.w[p + "router.coarse.bias"] + self.w[p + "router.group_bias"])
        fine = fine + (self.w[p + "router.fine.bias"] + self.w[p + "router.expert_bias"])
        size = -(-E // G)
        group_of = np.minimum(np.arange(E) // size, G - 1)
        logits = (fine + coarse[group_of]) / np.float32(max(s.get("router_temperature", 1.0), 1e-4))
        probs = K.softmax(logits.reshape(1, -1))[0]
        kmax, kmin = s["router_top_k_max"], s["router_top_k_min"]
        chosen = np.argsort(-probs, kind="stable")[:kmax]
        weights = probs[chosen].copy()
        confidence = weights[0] - weights[min(kmax - 1, 1)]
        entropy = -(probs * np.log(np.maximum(probs, np.float32(1e-9)))).sum()
        spread = np.rint((np.float32(1) - confidence) * np.float32(2)
                         + entropy / max(np.float32(np.log(E)), np.float32(1)))
        active = int(np.clip(kmin + spread, kmin, kmax))
        own, own_active = chosen[:active].tolist(), active
        if self.follow is not None:
            raw = float((np.float32(1) - confidence) * np.float32(2) + entropy / max(np.float32(np.log(E)),
                                                                                   np.float32(1)))
            chosen, active = self._follow_experts(layer, probs, chosen, active, raw)
            weights = probs[chosen].copy()
        weights[active:] = 0
        weights /= max(weights.sum(), np.float32(1e-9))
        if self.trace is not None:
            # margins: the smallest probability gap between neighbours among the
            # top kmax + 1 (the chosen order and the cut), and how far the
            # adaptive width's value lies from a rounding boundary
            ranked = probs[np.argsort(-probs, kind="stable")[:kmax + 1]]
            order_gap = float(np.min(ranked[:-1] - ranked[1:])) if ranked.size > 1 else math.inf
            raw = float((np.float32(1) - confidence) * np.float32(2) + entropy / max(np.float32(np.log(E)),
                                                                                   np.float32(1)))
            width_gap = abs(raw - math.floor(raw) - 0.5) if kmin < kmax else math.inf
            self.trace.append(("experts", layer, self.position, own, own_active, order_gap, width_gap))
        out = np.zeros_like(x)
        for e, wgt in zip(chosen[:active], weights[:active]):
            out = K.axpy(out, self._mlp(x, p + f"experts.{e}."), float(wgt))
        for e in range(s["shared_experts"]):
            out = K.axpy(out, self._mlp(x, p + f"shared.{e}."), c.residual_scale / max(s["shared_experts"], 1))
        return out

    def _follow_blocks(self, layer, scores, kept, blocks):
        """Adopt the followed per-head block sets that are valid within NEAR_TIE."""
        c = self.cfg
        kmax, slots = c.source["router_top_k_max"], c.source["long_context"]["global_slots"]
        rec = self.follow[self.position, layer, self._loop]
        for h in range(len(kept)):
            dev = rec[1 + kmax + h * slots: 1 + kmax + (h + 1) * slots]
            dev = np.sort(dev[dev >= 0]).astype(np.int64)
            if np.array_equal(dev, np.sort(kept[h])):
                continue
            event = ("blocks", layer, self.position, self._loop, h)
            if dev.size != kept[h].size or dev.size == 0 or dev[-1] >= blocks or np.unique(dev).size != dev.size:
                self.mismatches.append(event + (math.nan,))
                continue
            rest = np.setdiff1d(np.arange(blocks), dev)
            inside, outside = float(scores[h, dev].min()), float(scores[h, rest].max())
            gap = inside - outside            # < 0: the followed set ranks a lower score above a higher one
            if gap >= -self.NEAR_TIE * max(1.0, abs(outside)):
                kept[h] = dev
                self.adopted.append(event + (gap,))
            else:
                self.mismatches.append(event + (gap,))

    def _follow_experts(self, layer, probs, chosen, active, raw):
        """The followed routing (chosen order and width) if valid within
        NEAR_TIE, else the oracle's own; returns (chosen[:kmax], width)."""
        s = self.cfg.source
        kmin, kmax, E = s["router_top_k_min"], s["router_top_k_max"], s["routed_experts"]
        rec = self.follow[self.position, layer, self._loop]
        width = int(rec[0])
        dev = rec[1:1 + width].astype(np.int64) if kmin <= width <= kmax else np.zeros(0, np.int64)
        if width == active and np.array_equal(dev, chosen[:active]):
            return chosen, active
        event = ("experts", layer, self.position, self._loop)
        if dev.size == 0 or dev.min() < 0 or dev.max() >= E or np.unique(dev).size != dev.size:
            self.mismatches.append(event + (math.nan,))
            return chosen, active
        tol = self.NEAR_TIE * float(probs.max())
        pd = probs[dev]
        gap = float(np.min(pd[:-1] - pd[1:])) if dev.size > 1 else math.inf   # the chosen order
        rest = np.setdiff1d(np.arange(E), dev)
        if rest.size:
            gap = min(gap, float(pd[-1] - probs[rest].max()))                  # the cut
        # a rounding near-tie moves the width only to the other rounding of raw
        # (floor or floor + 1 around the .5 boundary, clipped like the width)
        near = abs(raw - math.floor(raw) - 0.5) <= self.NEAR_TIE * max(1.0, abs(raw))
        roundings = {int(np.clip(kmin + math.floor(raw) + d, kmin, kmax)) for d in (0, 1)}
        width_ok = width == active or (near and width in roundings)
        if gap >= -tol and width_ok:
            tail = [e for e in np.argsort(-probs, kind="stable") if e not in set(dev.tolist())]
            self.adopted.append(event + (gap,))
            return np.concatenate([dev, np.asarray(tail, np.int64)])[:kmax], width
        self.mismatches.append(event + (gap,))
        return chosen, active

    # --------------------------------------------------------------- one token
    def step(self, token):
        """One token through every layer; returns the final-normed hidden row."""
        c = self.cfg
        hidden = _widen(np.asarray(self.w["embed"][token:token + 1]))
        pos = np.asarray([self.position], np.float32)
        rs = c.residual_scale
        for layer, state in enumerate(self.layers):
            p = f"layers.{layer}."
            if c.family == "heavy-medium-2.0":
                loops = state.setdefault("loops", [dict() for _ in range(c.inner_loop_steps)])
                scale = rs / math.sqrt(c.inner_loop_steps)
                for self._loop, inner in enumerate(loops):
                    hidden = K.axpy(hidden, self._heavy_attention(self._rms(hidden, p + "a_norm"), layer, inner, pos),
                                    scale)
                    hidden = K.axpy(hidden, self._moe(self._rms(hidden, p + "f_norm"), layer), scale)
            elif c.family == "flashlighting-2.0":
                x = self._rms(hidden, p + "a_norm")
                attended = self._lighting(x, layer, state, pos)
                ag = float(self.w[p + "attention_gate"][0])
                fg = float(self.w[p + "ffn_gate"][0])
                branch = K.axpy(np.zeros_like(hidden), attended, ag)
                branch = K.axpy(branch, self._mlp(x, p + "ffn."), fg)
                hidden = K.axpy(hidden, branch, rs)
            else:
                hidden = K.axpy(hidden, self._gqa(self._rms(hidden, p + "a_norm"), layer, state, pos), rs)
                hidden = K.axpy(hidden, self._mlp(self._rms(hidden, p + "f_norm"), p + "ffn."), rs)
        self.position += 1
        return self._rms(hidden, "norm")

    def head(self, hidden):
        return K.linear(hidden, self.w["embed" if self.cfg.tie_embeddings else "output"])[0]

    # ------------------------------------------------------------- public API
    def _ids(self, ids):
        a = np.asarray(ids)
        if a.ndim != 1 or a.size == 0 or a.dtype.kind not in "iu":
            raise ValueError("input_ids must be a non-empty 1D integer sequence")
        if np.any(a < 0) or np.any(a >= self.cfg.vocab_size):
            raise ValueError("input token is outside the vocabulary")
        return a

    def prefill(self, ids, return_all=False):
        toks = self._ids(ids)
        if self.failed:
            raise RuntimeError("A previous device operation failed; call reset() before reusing this model")
        if self.position + len(toks) > self.ctx:
            raise ValueError("input would exceed context_length; reset or allocate a larger context")
        rows = []
        try:
            for i, t in enumerate(toks):
                hidden = self.step(int(t))
                if return_all or i == len(toks) - 1:
                    rows.append(self.head(hidden))
        except Exception:
            self.failed = True
            raise
        return np.stack(rows) if return_all else rows[0]

    def decode(self, token):
        return self.prefill([token])

    def generate(self, ids, max_new_tokens=32, temperature=0.0, top_k=0, top_p=1.0, seed=17, eos_token_id=None):
        """Greedy or seeded sampling with the reference's numpy stream (model.py:318-357)."""
        toks = self._ids(ids)
        if type(max_new_tokens) is not int or max_new_tokens < 0:
            raise ValueError("max_new_tokens must be a non-negative integer")
        if not math.isfinite(temperature) or temperature < 0:
            raise ValueError("temperature must be finite and non-negative")
        if type(top_k) is not int or top_k < 0 or not math.isfinite(top_p) or not 0 < top_p <= 1:
            raise ValueError("top_k must be non-negative and top_p must be in (0,1]")
        eos = self.cfg.eos_token_id if eos_token_id is None else eos_token_id
        if type(eos) is not int or not 0 <= eos < self.cfg.vocab_size:
            raise ValueError("eos_token_id is outside vocabulary")
        if len(toks) + max(0, max_new_tokens - 1) > self.ctx:
            raise ValueError("prompt plus requested generation exceeds context_length")
        self.reset()
        if max_new_tokens == 0:
            return []
        rng = np.random.default_rng(seed)
        out = []
        logits = self.prefill(toks)
        for i in range(max_new_tokens):
            if not np.all(np.isfinite(logits)):
                raise FloatingPointError("non-finite output logits")
            if temperature == 0:
                tok = int(np.argmax(logits))
            else:
                order = np.argsort(-logits, kind="stable")
                if top_k:
                    order = order[:top_k]
                z = logits[order].astype(np.float64) / temperature
                pr = np.exp(z - z.max())
                pr /= pr.sum()
                cut = min(len(order), int(np.searchsorted(np.cumsum(pr), top_p)) + 1)
                order, pr = order[:cut], pr[:cut]
                tok = int(rng.choice(order, p=pr / pr.sum()))
            out.append(tok)
            if tok == eos or i + 1 == max_new_tokens:
                break
            logits = self.decode(tok)
        return out
