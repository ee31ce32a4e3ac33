"""Frozen MI355X launch plan for the fused attention kernel.

Plays the role of the reference's ``PiperAttentionExecutionPlan`` /
``select_execution_plan`` (``src/piper_kernels/attention/piper_attention/_policy.py:14-96``)
for gfx950: an immutable record chosen from the shape, never autotuned at call time.
``select_plan`` looks the shape up in the frozen table ``mi355x_plans.json`` (written offline
by ``piper_kernels.attention.piper_attention.tune``, the counterpart of the reference's
``benchmarks/tune_piper_attention.py``) and falls back to a heuristic for other shapes;
``select_sage_plan`` does the same for SageAttention2++ with ``mi355x_sage_plans.json`` (the
counterpart of ``sage_attention_2pp/_policy.py`` and ``benchmarks/tune_sage_attention_2pp.py``).
Every plan without a key-range split computes bit-identical results; only the speed differs.
The key-range split plans (``key_parts`` > 1, for grids too small to give every SIMD three waves)
merge partial sums in another order and agree with the others to rounding.
"""

from __future__ import annotations

import json
from dataclasses import asdict, dataclass
from functools import lru_cache
from pathlib import Path

COMPUTE_UNITS = 256  # MI355X
KEY_BLOCK = 64  # keys per streamed tile and per P block (reference.py:16)
QUERIES_PER_WAVE = 32  # one v_mfma_i32_32x32x32_i8 column block
PLAN_TABLE = Path(__file__).with_name("mi355x_plans.json")
SAGE_PLAN_TABLE = Path(__file__).with_name("mi355x_sage_plans.json")

# piper_attention_args.plan bits (include/piper_mi355x.h)
PLAN_FOUR_WAVES = 1
PLAN_CAUSAL_FORWARD = 2
PLAN_NO_XCD_REMAP = 4
PLAN_CAUSAL_INTERLEAVE = 8
PLAN_THREE_WORKGROUPS = 16
PLAN_KEY_PARTS_SHIFT = 5  # bits 5-7: key parts - 1 (PIPER_PLAN_KEY_PARTS)
PLAN_WORK_QUEUE = 256
PLAN_MASK = 511
MAX_KEY_PARTS = 8
WAVE_SLOTS = 3 * 4 * COMPUTE_UNITS  # three waves on each of the 1024 SIMDs


@dataclass(frozen=True)
class MI355XPlan:
    """Launch plan of the fused kernel.

    ``waves``: query waves of 32 queries sharing each K/V tile staged in LDS (8: 256 queries
    per workgroup, one workgroup per CU; 4: 128 queries, two workgroups per CU, each with its own
    LDS ring). ``causal_longest_first``: causal
    grids dispatch the query tiles with the most key blocks first. ``xcd_remap``: consecutive
    workgroups of one head run on one XCD (its L2 then serves the head's K/V tiles).
    ``causal_interleave``: causal, longest first, across the heads of an XCD rather than head
    by head (a shorter tail for short and medium sequences; less L2 reuse for long ones).
    ``three_per_cu`` (4-wave workgroups only): three workgroups per CU, so three waves share each
    SIMD (a 2-stage LDS ring per workgroup and no score look-ahead, to fit 168 VGPRs) instead of
    two.  ``key_parts`` (three per CU, non-causal): the key tiles of each query tile are cut into
    that many ranges, one workgroup each, whose FP32 partial sums a merge kernel combines; for
    grids with too few query waves to give every SIMD three (results equal to rounding).
    ``work_queue`` (three per CU, no split): a persistent grid takes the query tiles from one
    queue per XCC instead of the hardware dispatching one workgroup per tile (bit-identical).
    """

    waves: int = 8
    causal_longest_first: bool = True
    xcd_remap: bool = True
    causal_interleave: bool = False
    three_per_cu: bool = False
    key_parts: int = 1
    work_queue: bool = False

    def __post_init__(self) -> None:
        if self.waves not in (4, 8):
            raise ValueError(f"waves must be 4 or 8, got {self.waves}")
        if self.three_per_cu and self.waves != 4:
            raise ValueError("three workgroups per CU need 4-wave workgroups")
        if not 1 <= self.key_parts <= MAX_KEY_PARTS:
            raise ValueError(f"key_parts must be 1..{MAX_KEY_PARTS}, got {self.key_parts}")
        if self.key_parts > 1 and not self.three_per_cu:
            raise ValueError("the key-range split runs three workgroups per CU")
        if self.work_queue and (not self.three_per_cu or self.key_parts > 1 or not self.xcd_remap):
            raise ValueError("the work-queue plan runs three workgroups per CU, one queue per XCC, without a "
                             "key-range split")

    @property
    def block_m(self) -> int:
        return self.waves * QUERIES_PER_WAVE

    @property
    def plan_id(self) -> int:
        """The ``plan`` field of ``piper_attention_args`` (an OR of PIPER_PLAN_* bits)."""
        return (
            (PLAN_FOUR_WAVES if self.waves == 4 and not self.three_per_cu else 0)
            | (0 if self.causal_longest_first else PLAN_CAUSAL_FORWARD)
            | (0 if self.xcd_remap else PLAN_NO_XCD_REMAP)
            | (PLAN_CAUSAL_INTERLEAVE if self.causal_interleave else 0)
            | (PLAN_THREE_WORKGROUPS if self.three_per_cu else 0)
            | ((self.key_parts - 1) << PLAN_KEY_PARTS_SHIFT)
            | (PLAN_WORK_QUEUE if self.work_queue else 0)
        )

    @classmethod
    def from_id(cls, plan_id: int) -> "MI355XPlan":
        if not 0 <= plan_id <= PLAN_MASK or (plan_id & PLAN_THREE_WORKGROUPS and plan_id & PLAN_FOUR_WAVES):
            raise ValueError(f"unknown plan id {plan_id}")
        three = bool(plan_id & PLAN_THREE_WORKGROUPS)
        return cls(
            waves=4 if plan_id & PLAN_FOUR_WAVES or three else 8,
            causal_longest_first=not plan_id & PLAN_CAUSAL_FORWARD,
            xcd_remap=not plan_id & PLAN_NO_XCD_REMAP,
            causal_interleave=bool(plan_id & PLAN_CAUSAL_INTERLEAVE),
            three_per_cu=three,
            key_parts=((plan_id >> PLAN_KEY_PARTS_SHIFT) & 7) + 1,
            work_queue=bool(plan_id & PLAN_WORK_QUEUE),
        )

    @classmethod
    def all_plans(cls) -> list["MI355XPlan"]:
        """Every distinct plan without a key-range split, by plan id: the plans that compute
        bit-identical results (PIPER_PLAN_THREE_WORKGROUPS implies 4-wave workgroups, so ids that
        also carry PIPER_PLAN_FOUR_WAVES name the same plans and are left out), then the
        work-queue plans."""
        return [cls.from_id(i) for i in range(PLAN_THREE_WORKGROUPS * 2)
                if not (i & PLAN_THREE_WORKGROUPS and i & PLAN_FOUR_WAVES)] + cls.queue_plans()

    @classmethod
    def split_plans(cls) -> list["MI355XPlan"]:
        """The key-range split plans: three workgroups per CU, 2..8 key parts, either workgroup order."""
        return [cls(waves=4, three_per_cu=True, key_parts=k, xcd_remap=x)
                for k in range(2, MAX_KEY_PARTS + 1) for x in (True, False)]

    @classmethod
    def queue_plans(cls) -> list["MI355XPlan"]:
        """The work-queue plans: three workgroups per CU in each causal tile order."""
        return [cls(waves=4, three_per_cu=True, work_queue=True, causal_longest_first=f, causal_interleave=i)
                for f in (True, False) for i in ((False, True) if f else (False,))]

    def workgroups(self, batch: int, heads: int, query_length: int) -> int:
        return batch * heads * (-(-query_length // self.block_m)) * self.key_parts

    def as_dict(self) -> dict:
        return {**asdict(self), "block_m": self.block_m, "block_n": KEY_BLOCK}


def shape_key(batch: int, heads: int, query_length: int, key_length: int, head_dim: int, is_causal: bool) -> tuple:
    """Table key: heads are independent, so only batch * heads matters."""
    return (batch * heads, query_length, key_length, head_dim, bool(is_causal))


def _read_plan_table(path: Path) -> dict:
    """A tuner table: shape key -> plan (empty if the file is absent)."""
    if not path.exists():
        return {}
    table = json.loads(path.read_text())
    plans = {}
    for entry in table.get("entries", []):
        k = entry["key"]
        key = (k["batch_heads"], k["query_length"], k["key_length"], k["head_dim"], bool(k["is_causal"]))
        plans[key] = MI355XPlan(**entry["plan"])
    return plans


@lru_cache(maxsize=1)
def frozen_plans() -> dict:
    """Piper Attention's committed tuner table: shape key -> plan."""
    return _read_plan_table(PLAN_TABLE)


@lru_cache(maxsize=1)
def frozen_sage_plans() -> dict:
    """SageAttention2++'s committed tuner table: shape key -> plan."""
    return _read_plan_table(SAGE_PLAN_TABLE)


def heuristic_plan(batch: int, heads: int, query_length: int) -> MI355XPlan:
    """8-wave workgroups unless that leaves most CUs idle; then 4-wave workgroups (the two-waves-
    per-SIMD plans' choice by grid size)."""
    wide = MI355XPlan(waves=8)
    if wide.workgroups(batch, heads, query_length) >= COMPUTE_UNITS:
        return wide
    return MI355XPlan(waves=4)


def split_parts(batch: int, heads: int, query_length: int, key_length: int) -> int:
    """Key parts for an untuned non-causal shape (1: no split).  A grid whose 128-query tiles
    fall short of one round of three workgroups per CU (768) and whose 256-query tiles leave CUs
    idle splits into 2-4 parts, each of at least two key tiles (c1, 64 tiles: 4 parts, 0.017 vs
    0.029 ms).  A long key range (>= 32768 keys,
    where the partial sums' HBM round trip is small against the work) splits in the 2-4 parts
    that fill the last round best, when that beats the unsplit grid's last round by 10% of a
    round (B1 H1 N131072: 1024 tiles = 1.33 rounds; 3 parts = 4 full rounds, 7.14 vs 7.97 ms).
    At 8192 keys the round trip costs more than the fuller round gains (r1: 3 parts 0.262 vs
    0.254 ms), so mid-length grids stay whole."""
    tiles = batch * heads * (-(-query_length // MI355XPlan(waves=4, three_per_cu=True).block_m))
    key_tiles = -(-key_length // KEY_BLOCK)
    round_slots = 3 * COMPUTE_UNITS
    if tiles < round_slots and MI355XPlan(waves=8).workgroups(batch, heads, query_length) < COMPUTE_UNITS:
        parts = min(4, max(2, round_slots // tiles), key_tiles // 2)
        return parts if parts >= 2 else 1
    if key_length >= 32768:
        def fill(p: int) -> float:
            rounds = tiles * p / round_slots
            return rounds / -(-rounds // 1)
        best = max((2, 3, 4), key=lambda p: (round(fill(p), 6), -p))
        if fill(best) >= fill(1) + 0.1 and key_tiles >= 2 * best:
            return best
    return 1


def piper_heuristic_plan(batch: int, heads: int, query_length: int, is_causal: bool,
                         key_length: int | None = None) -> MI355XPlan:
    """Piper Attention's plan for an untuned shape: three 4-wave workgroups per CU.  With three
    waves per SIMD from three independent workgroups, one wave's MFMA, LDS and barrier waits are
    filled by the other two: measured 7-24% faster than the two-waves-per-SIMD plans at c2-c5.
    Non-causal grids too small or too ragged for whole rounds of three workgroups per CU split
    their key range (``split_parts``).  Otherwise a non-causal grid whose 128-query tiles cannot
    fill three slots per CU, but whose 256-query tiles give every CU one, runs two waves per SIMD
    either way; one 8-wave workgroup per CU is then 1-2% faster (measured at r1, B1 H8 N8192)."""
    three = MI355XPlan(waves=4, three_per_cu=True)
    wide = MI355XPlan(waves=8)
    if not is_causal:
        parts = split_parts(batch, heads, query_length, query_length if key_length is None else key_length)
        if parts > 1:
            return MI355XPlan(waves=4, three_per_cu=True, key_parts=parts)
        if (three.workgroups(batch, heads, query_length) < 3 * COMPUTE_UNITS
                and wide.workgroups(batch, heads, query_length) >= COMPUTE_UNITS):
            return wide
    return three


def sage_plan(batch: int, heads: int, query_length: int) -> MI355XPlan:
    """The SageAttention2++ operator's plan: three 4-wave workgroups per CU on every shape
    (same-box A/B against two per CU: c2 14%, c3 8%, c4 7%, c5 8% faster; two per CU had been
    4-22% faster than one 8-wave workgroup per CU at c2-c5; at r1, where the grid cannot fill
    three slots per CU, three per CU still beat one 8-wave workgroup per CU by 3%)."""
    return MI355XPlan(waves=4, three_per_cu=True)


def select_plan(batch: int, heads: int, query_length: int, key_length: int, head_dim: int, is_causal: bool) -> MI355XPlan:
    """The frozen table's plan for a tuned shape, else Piper Attention's heuristic."""
    plan = frozen_plans().get(shape_key(batch, heads, query_length, key_length, head_dim, is_causal))
    return plan if plan is not None else piper_heuristic_plan(batch, heads, query_length, is_causal, key_length)


def select_sage_plan(batch: int, heads: int, query_length: int, key_length: int, head_dim: int,
                     is_causal: bool) -> MI355XPlan:
    """SageAttention2++'s frozen-table plan for a tuned shape, else ``sage_plan``."""
    plan = frozen_sage_plans().get(shape_key(batch, heads, query_length, key_length, head_dim, is_causal))
    return plan if plan is not None else sage_plan(batch, heads, query_length)
