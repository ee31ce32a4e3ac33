"""The committed SageAttention2++ golden fixtures are reproduced by the oracle (CPU regression pin)."""

from __future__ import annotations

import numpy as np
import pytest

from _parity import GOLDEN, load_golden
from oracle import sage2pp_oracle as oracle

FIXTURES = sorted((GOLDEN / "sage2pp").glob("*.npz"))


def test_fixtures_exist() -> None:
    assert len(FIXTURES) >= 4


@pytest.mark.parametrize("fixture", FIXTURES, ids=[p.stem for p in FIXTURES])
def test_oracle_reproduces_fixture(fixture) -> None:
    g = load_golden(fixture)
    prep = oracle.prepare(g["query"], g["key"], g["value"])
    for name in ("key_code", "value_code"):
        np.testing.assert_array_equal(prep[name], g[name], err_msg=name)
    for name in ("key_block_scale", "value_scale", "key_mean"):
        assert np.array_equal(prep[name].view(np.uint32), g[name].view(np.uint32)), name
    for mode, key in (("reference", "output_reference"), ("fp32", "output_fp32_accumulation")):
        out = oracle.attention_from_prepared(prep, g["scale"], g["is_causal"], accumulate=mode)
        np.testing.assert_allclose(out, g[key], rtol=1e-6, atol=1e-6, err_msg=mode)
