"""Seeded synthetic inputs for the benchmark and parity configurations.

Every (batch, head) slice is drawn from its own numpy PCG64 stream, so any subset of
heads can be regenerated bit-identically without materialising the rest.  Inputs are
generated on the CPU in FP32, rounded to the target dtype on the CPU (round to nearest
even), then copied to the device, so a GPU run and a CPU reference see identical bits.
"N(mu, s2)" in the configuration text is read as mean and *variance*.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    heads: int
    query_length: int
    key_length: int
    head_dim: int
    dtype: torch.dtype
    is_causal: bool
    seed: int
    kind: str  # distribution family, see _head()
    description: str

    @property
    def shape(self) -> tuple[int, int, int, int, int]:
        return (self.batch, self.heads, self.query_length, self.key_length, self.head_dim)

    def as_dict(self) -> dict:
        return {
            "workload": self.name,
            "batch": self.batch,
            "heads": self.heads,
            "query_length": self.query_length,
            "key_length": self.key_length,
            "head_dim": self.head_dim,
            "dtype": str(self.dtype).removeprefix("torch."),
            "is_causal": self.is_causal,
            "seed": self.seed,
            "description": self.description,
        }


WORKLOADS: dict[str, Workload] = {
    "c1": Workload("c1", 1, 8, 1024, 1024, 64, torch.float16, False, 1, "kbias",
                   "B1 H8 S1024 D64 fp16 non-causal; QKV~N(0,1), K += per-channel N(0,2)"),
    "c2": Workload("c2", 1, 24, 4096, 4096, 128, torch.float16, False, 2, "kbias_vbias4",
                   "B1 H24 S4096 D128 fp16 non-causal; QK~N(0,1), K += N(0,2) per channel, V~N(0,1)+N(0,4) per feature"),
    "c3": Workload("c3", 1, 24, 16384, 16384, 128, torch.float16, False, 3, "kbias_vbias4",
                   "B1 H24 S16384 D128 fp16 non-causal (headline); distributions as c2"),
    "c4": Workload("c4", 4, 32, 8192, 8192, 128, torch.bfloat16, True, 4, "kbias1",
                   "B4 H32 S8192 D128 bf16 causal; QKV~N(0,1), K += N(0,1) per channel, V uncentred"),
    "c5": Workload("c5", 2, 40, 32768, 32768, 128, torch.float16, False, 5, "student_t",
                   "B2 H40 S32768 D128 fp16 non-causal; QK = 0.5*t(3); heads<20 V constant along S, "
                   "others V~N(0,1)+N(0,8) per feature"),
    # the shape of the reference's only published Piper Attention figures (RTX 5090,
    # benchmarks/README.md:511-523), inputs standard normal as its benchmark draws them
    # (benchmarks/lib/attention.py:99-120)
    "r1": Workload("r1", 1, 8, 8192, 8192, 128, torch.bfloat16, False, 11, "plain",
                   "B1 H8 S8192 D128 bf16 non-causal; QKV~N(0,1) (the reference's published benchmark shape)"),
    # the reference's published long-sequence point (benchmarks/README.md:526): one head of 131072
    "r2": Workload("r2", 1, 1, 131072, 131072, 128, torch.bfloat16, False, 12, "plain",
                   "B1 H1 S131072 D128 bf16 non-causal; QKV~N(0,1) (the reference's published long-sequence shape)"),
}


def _head(w: Workload, b: int, h: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    rng = np.random.default_rng([w.seed, b, h])
    sq, sk, d = w.query_length, w.key_length, w.head_dim
    if w.kind == "student_t":
        q = (0.5 * rng.standard_t(3, size=(sq, d))).astype(np.float32)
        k = (0.5 * rng.standard_t(3, size=(sk, d))).astype(np.float32)
        if h < w.heads // 2:
            v = np.broadcast_to(rng.standard_normal((1, d), dtype=np.float32), (sk, d)).copy()
        else:
            v = rng.standard_normal((sk, d), dtype=np.float32)
            v += np.float32(np.sqrt(8.0)) * rng.standard_normal((1, d), dtype=np.float32)
        return q, k, v
    q = rng.standard_normal((sq, d), dtype=np.float32)
    k = rng.standard_normal((sk, d), dtype=np.float32)
    v = rng.standard_normal((sk, d), dtype=np.float32)
    if w.kind == "plain":
        return q, k, v
    k_bias_std = 1.0 if w.kind == "kbias1" else np.sqrt(2.0)
    k += np.float32(k_bias_std) * rng.standard_normal((1, d), dtype=np.float32)
    if w.kind == "kbias_vbias4":
        v += np.float32(2.0) * rng.standard_normal((1, d), dtype=np.float32)
    return q, k, v


def make_inputs(
    w: Workload,
    device: torch.device | str = "cpu",
    batches: range | list[int] | None = None,
    heads: range | list[int] | None = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Q, K, V of shape [len(batches), len(heads), S, D] in ``w.dtype`` on ``device``."""
    batches = list(range(w.batch)) if batches is None else list(batches)
    heads = list(range(w.heads)) if heads is None else list(heads)
    out = []
    for index in range(3):
        length = w.query_length if index == 0 else w.key_length
        tensor = torch.empty((len(batches), len(heads), length, w.head_dim), dtype=w.dtype)
        out.append(tensor)
    for bi, b in enumerate(batches):
        for hi, h in enumerate(heads):
            for tensor, values in zip(out, _head(w, b, h)):
                tensor[bi, hi] = torch.from_numpy(values).to(w.dtype)
    return tuple(t.to(device) for t in out)  # type: ignore[return-value]
