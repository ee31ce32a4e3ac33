"""bench.py's GPU-side record fields, checked against the CPU oracle on small shapes.

``quality.saturation`` counts the INT8 Q, K and V codes at the quantiser's endpoints (the
reference harness's ``QuantizerSaturation`` fields, benchmarks/lib/quality.py:16-41).  The codes
are bit-exact with the oracle's, so the counts must equal the oracle's counts exactly, over the
valid rows only (padding rows are zero and must not be counted).
"""

from __future__ import annotations

import importlib.util
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from _parity import log
from oracle import piper_oracle as oracle

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


@pytest.mark.parametrize("shape,causal,granularity", [
    ((1, 2, 300, 200, 128), False, "per_thread"),  # ragged: 12 padding query rows, 56 padding keys
    ((2, 1, 129, 129, 64), True, "per_warp"),  # causal: equal lengths
])
def test_saturation_counts_equal_the_oracle_codes(shape, causal, granularity, gfx950_device) -> None:
    b, h, sq, sk, d = shape
    g = torch.Generator().manual_seed(sq + sk)
    q = torch.randn((b, h, sq, d), generator=g).to(torch.float16)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(torch.float16)
    v = (torch.randn((b, h, sk, d), generator=g) * 3).to(torch.float16)
    workload = SimpleNamespace(shape=shape, is_causal=causal)
    log(f"[case] bench saturation {shape} causal={causal} {granularity}")
    got = _bench().saturation_block(q.to(gfx950_device), k.to(gfx950_device), v.to(gfx950_device), d**-0.5,
                                    workload, granularity)
    prep = oracle.prepare(q, k, v, causal, granularity)
    for name, codes in (("query", prep["query_code"][:, :, :sq]), ("key", prep["key_code"][:, :, :sk]),
                        ("value", prep["value_code"][:, :, :sk])):
        low, high = int(np.count_nonzero(codes == -127)), int(np.count_nonzero(codes == 127))
        record = got[name]
        assert (record["minimum_count"], record["maximum_count"]) == (low, high), name
        assert record["total_count"] == codes.size and record["count"] == low + high, name
        assert record["fraction"] == pytest.approx((low + high) / codes.size), name
        # absmax scaling: every block (Q, K) or key row (V) holds at least one endpoint code
        assert low + high > 0, name
