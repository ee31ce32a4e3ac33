"""Frozen MI355X launch plan for the fused attention kernel.

Plays the role of the reference's ``PiperAttentionExecutionPlan`` /
``select_execution_plan`` (``src/piper_kernels/attention/piper_attention/_policy.py:14-96``)
for gfx950: an immutable record chosen from the shape, never autotuned at call time.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

COMPUTE_UNITS = 256  # MI355X
KEY_BLOCK = 64  # keys per streamed tile and per P block (reference.py:16)
QUERIES_PER_WAVE = 32  # one v_mfma_i32_32x32x32_i8 column block


@dataclass(frozen=True)
class MI355XPlan:
    """Workgroup shape of the fused kernel.

    ``waves`` query waves of 32 queries share each K/V tile staged in LDS (8 waves: 256
    queries per workgroup, one workgroup per CU; 4 waves: 128 queries, two per CU).
    """

    waves: int = 8

    def __post_init__(self) -> None:
        if self.waves not in (4, 8):
            raise ValueError(f"waves must be 4 or 8, got {self.waves}")

    @property
    def block_m(self) -> int:
        return self.waves * QUERIES_PER_WAVE

    @property
    def plan_id(self) -> int:
        """The ``plan`` field of ``piper_attention_args`` (0 = 8 waves, 1 = 4 waves)."""
        return 0 if self.waves == 8 else 1

    def workgroups(self, batch: int, heads: int, query_length: int) -> int:
        return batch * heads * (-(-query_length // self.block_m))

    def as_dict(self) -> dict:
        return {**asdict(self), "block_m": self.block_m, "block_n": KEY_BLOCK}


def select_plan(batch: int, heads: int, query_length: int, key_length: int, head_dim: int, is_causal: bool) -> MI355XPlan:
    """8-wave workgroups unless that leaves most CUs idle; then 4-wave workgroups."""
    wide = MI355XPlan(waves=8)
    if wide.workgroups(batch, heads, query_length) >= COMPUTE_UNITS:
        return wide
    return MI355XPlan(waves=4)
