"""Feature-major BSGS linear engine (reference llama3fhe/operators/linear/
operator.py:46-436, config.py:47-317, weight.py:272-366).

A square weight ``W`` (dimension D) acts on every token lane of a
feature-major ciphertext as ``y = W x`` through its D generalised diagonals:
``y = sum_g rot_{g B lanes}( sum_b pt[g, b] * rot_{b lanes}(x) )`` with B baby
steps and D / B giant steps.  The diagonals are encoded chunk by chunk
(``max_plaintext_rows`` rows, i.e. a few giant groups, at a time), each chunk
is aligned by one rotation of ``giant_base * B * lanes``, and the chunk sums
are added before one rescale.

Execution on this backend:
* the baby rotations of all inputs come from one batched hoisted call (one
  ModUp per input, each baby key read once for the batch) and are cached by
  the operator across chunks (and across weights applied to the same input);
* a chunk's plaintexts are packed and encoded on the device straight from
  the resident weight (``easyfhe.packing``), once for all inputs;
* the chunk's MAC and its giant Horner chain run for all inputs at once
  (``fhe.hoisted_mac_sum_many``): each plaintext word is read once per chunk,
  each baby word once per 8 giant groups.
"""

from __future__ import annotations

import time
from dataclasses import dataclass

import numpy as np

from easyfhe import fhe
from easyfhe import packing
from easyfhe.tensor import DeviceTensor

_CACHE_MODES = {"none", "middle", "plain", "both"}
_HOIST_STRATEGIES = {"normal", "ext_normal", "ext_double_hoist"}
_RAW_WEIGHT_POLICIES = {"device", "host"}


@dataclass(frozen=True)
class LinearChunk:
    index: int
    giant_base: int
    giant_count: int

    @property
    def name(self) -> str:
        return f"chunk.{int(self.index)}"


def _check_schedule(baby_steps: int, anchor: int, rows: int) -> None:
    """One check of the BSGS schedule fields shared by the plan and the config."""
    if int(baby_steps) < 1:
        raise ValueError(f"a BSGS schedule needs at least one baby step (got {baby_steps})")
    if not (int(anchor) == -1 or int(anchor) >= 2):
        raise ValueError(f"the baby anchor is -1 (off) or a block of two or more steps "
                         f"(got {anchor})")
    if int(rows) < int(baby_steps):
        raise ValueError(f"a chunk of {rows} plaintext rows cannot hold the {baby_steps} "
                         "diagonals of one giant group")


@dataclass(frozen=True)
class LinearPlan:
    """The physical BSGS schedule of one D-wide linear (config.py:158-273)."""

    dimension: int
    token_lanes: int
    baby_steps: int
    baby_anchor_step: int
    max_plaintext_rows: int

    def __post_init__(self) -> None:
        if int(self.dimension) < 1 or int(self.token_lanes) < 1:
            raise ValueError(f"a linear plan needs a positive width and lane count "
                             f"(got {self.dimension}, {self.token_lanes})")
        _check_schedule(self.baby_steps, self.baby_anchor_step, self.max_plaintext_rows)
        if int(self.dimension) % int(self.baby_steps):
            raise ValueError(f"{self.baby_steps} baby steps do not split a {self.dimension}-wide "
                             "matrix into whole giant groups")

    @property
    def giant_steps(self) -> int:
        return int(self.dimension) // int(self.baby_steps)

    @property
    def chunk_giants(self) -> int:
        return max(1, int(self.max_plaintext_rows) // int(self.baby_steps))

    @property
    def giant_offset(self) -> int:
        return int(self.baby_steps) * int(self.token_lanes)

    @property
    def baby_offsets(self) -> tuple[int, ...]:
        return tuple(b * int(self.token_lanes) for b in range(int(self.baby_steps)))

    @property
    def anchor_enabled(self) -> bool:
        return int(self.baby_anchor_step) >= 2 and int(self.baby_steps) > int(self.baby_anchor_step)

    @property
    def baby_key_offsets(self) -> tuple[int, ...]:
        """Rotation keys of the baby rotations: the first block's offsets plus
        the anchor step when the babies come in anchored blocks."""
        width = int(self.baby_anchor_step) if self.anchor_enabled else int(self.baby_steps)
        keys = {s * int(self.token_lanes) for s in range(1, width)}
        if self.anchor_enabled:
            keys.add(int(self.baby_anchor_step) * int(self.token_lanes))
        return tuple(sorted(keys))

    @property
    def chunks(self) -> tuple[LinearChunk, ...]:
        per = self.chunk_giants
        return tuple(LinearChunk(i, g0, min(per, self.giant_steps - g0))
                     for i, g0 in enumerate(range(0, self.giant_steps, per)))

    @property
    def cache_key(self) -> tuple[int, ...]:
        return (int(self.dimension), int(self.token_lanes), int(self.baby_steps),
                int(self.max_plaintext_rows))


@dataclass(frozen=True)
class LinearOperatorConfig:
    """Schedule and cache policy of the linear operator (config.py:47-105);
    the defaults are the reference's production schedule for a 4096-wide
    feature-major linear (B = 64, one anchor block, 512-row chunks)."""

    baby_steps: int = 64
    baby_anchor_step: int = 64
    max_plaintext_rows: int = 512
    reuse_baby_rotations: bool = True
    hoist_strategy: str = "normal"
    constant_cache_mode: str = "none"
    raw_weight_policy: str = "device"
    # synchronise after each stage so that apply()'s profile holds device
    # time; False keeps the stream busy across stages and chunks (the
    # profile then holds host time)
    timed_stages: bool = True

    def __post_init__(self) -> None:
        _check_schedule(self.baby_steps, self.baby_anchor_step, self.max_plaintext_rows)
        if str(self.hoist_strategy).lower() not in _HOIST_STRATEGIES:
            raise ValueError(f"unknown hoist strategy {self.hoist_strategy!r} "
                             f"(known: {sorted(_HOIST_STRATEGIES)})")
        if str(self.constant_cache_mode) not in _CACHE_MODES:
            raise ValueError(f"unknown constant cache mode {self.constant_cache_mode!r} "
                             f"(known: {sorted(_CACHE_MODES)})")
        if str(self.raw_weight_policy) not in _RAW_WEIGHT_POLICIES:
            raise ValueError(f"unknown raw weight policy {self.raw_weight_policy!r} "
                             f"(known: {sorted(_RAW_WEIGHT_POLICIES)})")

    def plan(self, *, dimension: int, token_lanes: int) -> LinearPlan:
        return LinearPlan(int(dimension), int(token_lanes), int(self.baby_steps),
                          int(self.baby_anchor_step), int(self.max_plaintext_rows))


def linear_rotations(*, dimension: int, token_lanes: int, slots: int | None = None,
                     include_conjugation: bool = False,
                     operator_config: LinearOperatorConfig | None = None) -> tuple[int, ...]:
    """Every rotation key one linear schedule needs (config.py:276-317): the
    baby keys, the giant key of the Horner chain, and the chunk alignments."""
    cfg = operator_config or LinearOperatorConfig()
    plan = cfg.plan(dimension=dimension, token_lanes=token_lanes)
    keys = set(plan.baby_key_offsets)
    most = max(c.giant_count for c in plan.chunks)
    if most > 1:
        if str(cfg.hoist_strategy).lower() == "ext_double_hoist":
            keys.update(s * plan.giant_offset for s in range(1, most))
        else:
            keys.add(plan.giant_offset)
    keys.update(c.giant_base * plan.giant_offset for c in plan.chunks if c.giant_base)
    if include_conjugation:
        if slots is None:
            raise ValueError("the conjugation key index 4 * slots - 1 needs the slot count")
        keys.add(4 * int(slots) - 1)
    return tuple(sorted(int(k) for k in keys if int(k)))


def _ctx(context):
    return getattr(context, "context", context)


class LinearWeight:
    """A square weight resident on the device, encoded chunk by chunk on
    demand (weight.py:272-366).  The plaintexts of a chunk sit at the inputs'
    level with the level's scale."""

    def __init__(self, weight, *, dtype=np.float64, context=None):
        self.context = _ctx(context) if context is not None else fhe.current_context()
        if isinstance(weight, DeviceTensor):
            self._w = weight
        else:
            w = np.ascontiguousarray(np.asarray(weight, dtype=np.dtype(dtype)))
            if w.ndim != 2 or w.shape[0] != w.shape[1]:
                raise ValueError(f"a linear weight must be square, got {w.shape}.")
            self._w = DeviceTensor(w, context=self.context)
        self.dimension = int(self._w.shape[0])
        self.closed = False

    def plaintext(self, plan: LinearPlan, chunk: LinearChunk, *, limbs: int,
                  operator_config: LinearOperatorConfig | None = None,
                  scale: float | None = None) -> list:
        if self.closed:
            raise RuntimeError("linear weight is closed.")
        if int(plan.dimension) != self.dimension:
            raise ValueError(f"plan dimension={plan.dimension} does not match weight "
                             f"dimension={self.dimension}.")
        cfg = operator_config or LinearOperatorConfig()
        ctx = self.context
        diag = packing.pack_token_lane_bsgs_weight_chunk(
            self._w, slots=ctx.max_slots, dimension=plan.dimension, token_lanes=plan.token_lanes,
            baby_steps=plan.baby_steps, giant_base=chunk.giant_base, giant_count=chunk.giant_count)
        return diag.encode(ctx, limbs=int(limbs),
                           scale=float(scale) if scale else ctx.scale_at(int(limbs)),
                           is_ext=str(cfg.hoist_strategy).lower() != "normal")

    def close(self) -> None:
        if not self.closed:
            self._w.release()
            self.closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _release(values) -> None:
    for v in values or ():
        if v is not None:
            v.release()


class LinearOperator:
    """A reusable BSGS schedule with an operator-local baby cache
    (operator.py:46-436)."""

    def __init__(self, *, context, token_lanes: int, config: LinearOperatorConfig | None = None):
        self.context = _ctx(context)
        self.token_lanes = int(token_lanes)
        if self.token_lanes <= 0:
            raise ValueError(f"a linear operator needs at least one token lane "
                             f"(got {self.token_lanes})")
        self.config = config or LinearOperatorConfig()
        self._babies: dict = {}
        self._hits = self._misses = 0
        self.closed = False

    def plan(self, dimension: int) -> LinearPlan:
        return self.config.plan(dimension=int(dimension), token_lanes=self.token_lanes)

    # -- baby cache ----------------------------------------------------------
    def _key(self, ct, plan: LinearPlan):
        return (id(ct), plan.cache_key + (int(plan.baby_anchor_step),))

    def _ensure_babies(self, inputs, plan: LinearPlan) -> list:
        """The babies of every input: cached ones reused, the missing ones
        computed in one batched call (one key read per baby rotation for the
        batch) and cached when the config reuses them."""
        found, missing = [], []
        for ct in inputs:
            entry = self._babies.get(self._key(ct, plan))
            if entry is not None and entry[0] is ct and entry[1] == int(ct.state.cur_limbs):
                self._hits += 1
                found.append(entry[2])
            else:
                found.append(None)
                missing.append(ct)
        if missing:
            self._misses += len(missing)
            made = fhe.prepare_hoisted_baby_rotations_many(
                missing, plan.baby_offsets, self.context,
                baby_anchor_step=int(plan.baby_anchor_step))
            it = iter(made)
            for n, ct in enumerate(inputs):
                if found[n] is not None:
                    continue
                babies = next(it)
                found[n] = babies
                if self.config.reuse_baby_rotations:
                    key = self._key(ct, plan)
                    old = self._babies.get(key)
                    if old is not None:
                        _release(old[2])
                    self._babies[key] = (ct, int(ct.state.cur_limbs), babies)
        return found

    def release_babies(self, inputs) -> None:
        """Drop the cached babies of these inputs (every plan)."""
        ids = {id(ct) for ct in inputs}
        for key in [k for k, e in self._babies.items() if k[0] in ids and e[0] in inputs]:
            _release(self._babies.pop(key)[2])

    def clear_baby_cache(self) -> None:
        for entry in self._babies.values():
            _release(entry[2])
        self._babies.clear()

    def cache_info(self) -> dict[str, int]:
        return {"baby_entries": len(self._babies), "baby_hits": self._hits,
                "baby_misses": self._misses}

    def prepare_baby_rotations(self, inputs, *, dimension: int) -> dict[str, float]:
        """Fill the baby cache before the plaintexts are prepared."""
        if self.closed:
            raise RuntimeError("linear operator is closed.")
        inputs = tuple(inputs)
        plan = self.plan(dimension)
        if len({int(c.state.cur_limbs) for c in inputs}) > 1:
            raise ValueError("linear inputs must enter at one common level.")
        start = time.perf_counter()
        self._ensure_babies(inputs, plan)
        self.context.synchronize()
        return {"baby_precompute": time.perf_counter() - start}

    # -- application ---------------------------------------------------------
    def apply(self, inputs, weight: LinearWeight, *, output_scale: float | None = None):
        """``W x`` for every input ciphertext, rescaled once; returns the
        outputs and a profile of seconds per stage.  With ``output_scale`` the
        plaintexts are encoded at ``output_scale * q / s_in`` (q the prime the
        rescale drops), so the outputs land exactly on that scale: a
        polynomial ladder that starts there keeps its scales at the primes."""
        if self.closed:
            raise RuntimeError("linear operator is closed.")
        inputs = tuple(inputs)
        stage = {"baby_precompute": 0.0, "pack_encode": 0.0, "online": 0.0, "rescale": 0.0}
        if not inputs:
            return (), stage
        if weight.closed:
            raise RuntimeError("cannot apply a closed linear weight.")
        plan = self.plan(weight.dimension)
        levels = {int(c.state.cur_limbs) for c in inputs}
        if len(levels) != 1:
            raise ValueError("linear inputs must enter at one common level.")
        limbs = levels.pop()
        ctx = self.context
        pt_scale = None
        if output_scale is not None:
            s_in = float(inputs[0].state.scaling_factor)
            if any(abs(float(c.state.scaling_factor) / s_in - 1.0) > 2.0 ** -30 for c in inputs):
                raise ValueError("an exact output scale needs inputs of one scale.")
            pt_scale = float(output_scale) * float(int(ctx.primes()[limbs - 1])) / s_in
        ext = str(self.config.hoist_strategy).lower() != "normal"
        sync = ctx.synchronize if self.config.timed_stages else (lambda: None)
        t0 = time.perf_counter()
        babies = None if ext else self._ensure_babies(inputs, plan)
        sync()
        stage["baby_precompute"] = time.perf_counter() - t0
        acc: list = []
        try:
            for chunk in plan.chunks:
                t0 = time.perf_counter()
                pts = weight.plaintext(plan, chunk, limbs=limbs, operator_config=self.config,
                                       scale=pt_scale)
                sync()
                stage["pack_encode"] += time.perf_counter() - t0
                t0 = time.perf_counter()
                try:
                    if ext:
                        outs = fhe.hoisted_mac_sum_ext_many(
                            list(inputs), plan.baby_offsets, pts, plan.giant_offset,
                            chunk.giant_count, ctx,
                            strategy=str(self.config.hoist_strategy).lower())
                    else:
                        outs = fhe.hoisted_mac_sum_many(babies, pts, plan.giant_offset,
                                                        chunk.giant_count, ctx)
                finally:
                    _release(pts)
                if chunk.giant_base:
                    shifted = fhe.homo_rotate_many(outs, chunk.giant_base * plan.giant_offset, ctx)
                    _release(outs)
                    outs = shifted
                if not acc:
                    acc = outs
                else:
                    summed = fhe.homo_add_many(acc, outs, ctx)
                    _release(acc)
                    _release(outs)
                    acc = summed
                sync()
                stage["online"] += time.perf_counter() - t0
            t0 = time.perf_counter()
            outputs = fhe.rescale_many(acc, ctx)
            sync()
            stage["rescale"] = time.perf_counter() - t0
            return tuple(outputs), stage
        finally:
            _release(acc)
            if not self.config.reuse_baby_rotations and babies is not None:
                for b in babies:
                    _release(b)

    def project(self, inputs, weight, *, dtype=np.float64):
        """apply() with a weight given as an array (uploaded for the call)."""
        t0 = time.perf_counter()
        with LinearWeight(weight, dtype=dtype, context=self.context) as w:
            upload = time.perf_counter() - t0
            outputs, profile = self.apply(inputs, w)
        profile["weight_upload"] = upload
        return outputs, profile

    def close(self) -> None:
        self.clear_baby_cache()
        self.closed = True

    def __enter__(self):
        if self.closed:
            raise RuntimeError("cannot enter a closed linear operator.")
        return self

    def __exit__(self, *exc):
        self.close()


__all__ = ["LinearChunk", "LinearOperator", "LinearOperatorConfig", "LinearPlan", "LinearWeight",
           "linear_rotations"]
