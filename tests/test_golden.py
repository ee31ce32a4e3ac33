"""The committed golden fixtures are reproduced by the oracle (CPU regression pin)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import GOLDEN, load_golden
from oracle import piper_oracle as oracle

FIXTURES = sorted(GOLDEN.glob("*.npz"))


def test_fixtures_exist() -> None:
    assert len(FIXTURES) >= 6


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_oracle_reproduces_fixture(fixture) -> None:
    g = load_golden(fixture)
    prep = oracle.prepare(g["query"], g["key"], g["value"], g["is_causal"], "per_warp")
    for name in ("query_code", "key_code", "value_code"):
        np.testing.assert_array_equal(prep[name], g[name], err_msg=name)
    for name in ("query_block_scale", "key_block_scale", "value_scale", "key_mean", "value_mean"):
        assert np.array_equal(prep[name].view(np.uint32), g[name].view(np.uint32)), name
    out = oracle.attention_from_prepared(prep, g["scale"], g["is_causal"])
    np.testing.assert_allclose(out, g["output_per_warp"], rtol=1e-6, atol=1e-6)
    out_t = oracle.piper_attention_reference(g["query"], g["key"], g["value"], g["scale"], g["is_causal"], "per_thread")
    np.testing.assert_allclose(out_t, g["output_per_thread"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_fixture_means_are_torch_cpu_means(fixture) -> None:
    """The K (and, non-causal, V) means of every fixture are bit for bit what the reference's
    own calls return on CPU: key.float().mean(dim=2) (sage/reference.py:88-89) and
    value.float().mean(dim=2) (reference.py:47-51)."""
    g = load_golden(fixture)
    key = torch.from_numpy(oracle.as_float32(g["key"]))
    assert np.array_equal(key.mean(dim=2).numpy().view(np.uint32), g["key_mean"].view(np.uint32))
    if not g["is_causal"]:
        value = torch.from_numpy(oracle.as_float32(g["value"]))
        assert np.array_equal(value.mean(dim=2).numpy().view(np.uint32), g["value_mean"].view(np.uint32))
