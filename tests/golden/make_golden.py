"""Write the golden fixtures of tests/golden/ from the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py
Each fixture holds the inputs (as 16-bit patterns), the per-block ("per_warp") prep
outputs -- codes, scales, means -- and the FP32 pre-cast outputs of the oracle for both
Q/K granularities.  The reference package ships no data fixtures; these pin this
repository's oracle (tests/test_golden.py) and are the targets of the GPU parity tests.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path[:0] = [str(REPO), str(REPO / "piper-kernels_amd")]

from oracle import piper_oracle as oracle  # noqa: E402
from piper_kernels.workloads import WORKLOADS, make_inputs  # noqa: E402

CASES = {
    # name: (builder, scale, is_causal)
    "c1_heads01": (lambda: make_inputs(WORKLOADS["c1"], heads=[0, 1]), None, False),
    "ragged65_fp16_d64": (lambda: _randn((1, 2, 65, 64), (1, 2, 65, 64), torch.float16, 51), None, False),
    "rect9x11_bf16_d128": (lambda: _randn((2, 1, 9, 128), (2, 1, 11, 128), torch.bfloat16, 50), 0.2, False),
    "causal193_bf16_d128": (lambda: _randn((1, 2, 193, 128), (1, 2, 193, 128), torch.bfloat16, 54), None, True),
    "causal130_fp16_d64": (lambda: _randn((1, 1, 130, 64), (1, 1, 130, 64), torch.float16, 62), None, True),
    "constv70_fp16_d64": (lambda: _constant_value(), None, False),
}


def _randn(qshape, kshape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(qshape, generator=g).to(dtype)
    k = (torch.randn(kshape, generator=g) + 1.5 * torch.randn(kshape[:2] + (1, kshape[3]), generator=g)).to(dtype)
    v = (torch.randn(kshape, generator=g) + 2.0 * torch.randn(kshape[:2] + (1, kshape[3]), generator=g)).to(dtype)
    return q, k, v


def _constant_value():
    g = torch.Generator().manual_seed(52)
    q = torch.randn((1, 2, 70, 64), generator=g).to(torch.float16)
    k = torch.randn((1, 2, 70, 64), generator=g).to(torch.float16)
    v = torch.randn((1, 2, 1, 64), generator=g).to(torch.float16).expand(1, 2, 70, 64).contiguous()
    return q, k, v


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def build(name: str) -> dict:
    builder, scale, causal = CASES[name]
    q, k, v = builder()
    d = q.shape[-1]
    scale = d**-0.5 if scale is None else scale
    prep = oracle.prepare(q, k, v, causal, "per_warp")
    out_warp = oracle.attention_from_prepared(prep, scale, causal)
    out_thread = oracle.piper_attention_reference(q, k, v, scale, causal, "per_thread")
    return {
        "dtype": np.array(str(q.dtype).removeprefix("torch.")),
        "scale": np.array(scale, dtype=np.float64),
        "is_causal": np.array(causal),
        "query_bits": bits(q),
        "key_bits": bits(k),
        "value_bits": bits(v),
        "query_code": prep["query_code"],
        "query_block_scale": prep["query_block_scale"],
        "key_code": prep["key_code"],
        "key_block_scale": prep["key_block_scale"],
        "key_mean": prep["key_mean"],
        "value_code": prep["value_code"],
        "value_scale": prep["value_scale"],
        "value_mean": prep["value_mean"],
        "output_per_warp": out_warp,
        "output_per_thread": out_thread,
    }


def main() -> None:
    for name in CASES:
        np.savez_compressed(HERE / f"{name}.npz", **build(name))
        print("wrote", name)


if __name__ == "__main__":
    main()
