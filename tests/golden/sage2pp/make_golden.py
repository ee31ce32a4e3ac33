"""Write the SageAttention2++ golden fixtures of tests/golden/sage2pp/ from the CPU oracle.

Run from the repository root:  python tests/golden/sage2pp/make_golden.py
Each fixture holds the inputs (as 16-bit patterns), the prep outputs (K mean, INT8 K codes and
per-block scales, per-channel V scales, FP8 E4M3 V codes) and the FP32 pre-cast outputs of
oracle/sage2pp_oracle.py in both accumulation modes: the reference's FP16 64-key partials and the
FP32 accumulation the MI355X kernel performs.  The reference package ships no data fixtures;
these pin the oracle (tests/test_sage2pp_golden.py) and are targets of the GPU tests.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[2]
sys.path[:0] = [str(REPO)]

from oracle import sage2pp_oracle as oracle  # noqa: E402


def _randn(qshape, kshape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(qshape, generator=g).to(dtype)
    k = (torch.randn(kshape, generator=g) + 1.5 * torch.randn(kshape[:2] + (1, kshape[3]), generator=g)).to(dtype)
    v = (torch.randn(kshape, generator=g) * 1.5 + torch.randn(kshape[:2] + (1, kshape[3]), generator=g)).to(dtype)
    return q, k, v


def _constant_value():
    g = torch.Generator().manual_seed(92)
    q = torch.randn((1, 2, 70, 64), generator=g).to(torch.float16)
    k = torch.randn((1, 2, 70, 64), generator=g).to(torch.float16)
    v = torch.randn((1, 2, 1, 64), generator=g).to(torch.float16).expand(1, 2, 70, 64).contiguous()
    return q, k, v


CASES = {
    # name: (builder, scale, is_causal)
    "ragged65_fp16_d64": (lambda: _randn((1, 2, 65, 64), (1, 2, 65, 64), torch.float16, 91), None, False),
    "rect9x11_bf16_d128": (lambda: _randn((2, 1, 9, 128), (2, 1, 11, 128), torch.bfloat16, 93), 0.2, False),
    "causal193_bf16_d128": (lambda: _randn((1, 2, 193, 128), (1, 2, 193, 128), torch.bfloat16, 94), None, True),
    "constv70_fp16_d64": (_constant_value, None, False),
}


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def build(name: str) -> dict:
    builder, scale, causal = CASES[name]
    q, k, v = builder()
    d = q.shape[-1]
    scale = d**-0.5 if scale is None else scale
    prep = oracle.prepare(q, k, v)
    return {
        "dtype": np.array(str(q.dtype).removeprefix("torch.")),
        "scale": np.array(scale, dtype=np.float64),
        "is_causal": np.array(causal),
        "query_bits": bits(q),
        "key_bits": bits(k),
        "value_bits": bits(v),
        "key_mean": prep["key_mean"],
        "key_code": prep["key_code"],
        "key_block_scale": prep["key_block_scale"],
        "value_scale": prep["value_scale"],
        "value_code": prep["value_code"],
        "output_reference": oracle.attention_from_prepared(prep, scale, causal),
        "output_fp32_accumulation": oracle.attention_from_prepared(prep, scale, causal, accumulate="fp32"),
    }


def main() -> None:
    for name in CASES:
        np.savez_compressed(HERE / f"{name}.npz", **build(name))
        print("wrote", name)


if __name__ == "__main__":
    main()
