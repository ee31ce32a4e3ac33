"""SageAttention2++ host contract (CPU): exports, validation, dispatch, custom op.

Validation cases and messages follow the reference's
tests/attention/sage_attention_2pp/test_dispatch.py:15-110.
"""

from __future__ import annotations

import pytest
import torch

import piper_kernels
from piper_kernels import sage_attention_2pp
from piper_kernels._hip import library as native
from piper_kernels.attention.sage_attention_2pp import dispatch


def _inputs():
    q = torch.randn(1, 2, 16, 64, dtype=torch.float16)
    return q, torch.randn_like(q), torch.randn_like(q)


def test_package_root_exports_sage_attention_2pp() -> None:
    assert piper_kernels.sage_attention_2pp is sage_attention_2pp
    assert "sage_attention_2pp" in piper_kernels.__all__


@pytest.mark.parametrize("dtype", [torch.float32, torch.int8])
def test_rejects_unsupported_dtype(dtype) -> None:
    q = torch.zeros((1, 1, 8, 64), dtype=dtype)
    with pytest.raises(ValueError, match="float16 or bfloat16"):
        sage_attention_2pp(q, q, q)


def test_rejects_mismatched_dtypes() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="share a dtype"):
        sage_attention_2pp(q, k.to(torch.bfloat16), v)


def test_rejects_unsupported_head_dimension() -> None:
    q = torch.randn(1, 1, 8, 32, dtype=torch.float16)
    with pytest.raises(ValueError, match="head dimensions 64 and 128"):
        sage_attention_2pp(q, q, q)


def test_rejects_mismatched_key_value_lengths() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="key/value lengths"):
        sage_attention_2pp(q, k, v[:, :, :-1])


def test_rejects_grouped_query_attention() -> None:
    q = torch.randn(1, 4, 16, 64, dtype=torch.float16)
    k = torch.randn(1, 2, 16, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="equal batch and head dimensions"):
        sage_attention_2pp(q, k, k)


def test_rejects_rectangular_causal_inputs() -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="equal query and key lengths"):
        sage_attention_2pp(q[:, :, :-1], k, v, is_causal=True)


@pytest.mark.parametrize(("query_length", "key_length"), [(0, 8), (8, 0)])
def test_rejects_empty_sequences(query_length, key_length) -> None:
    q = torch.empty((1, 1, query_length, 64), dtype=torch.float16)
    k = torch.empty((1, 1, key_length, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="does not accept empty"):
        sage_attention_2pp(q, k, k)


def test_rejects_noncontiguous_head_dimension() -> None:
    q = torch.randn(1, 1, 8, 128, dtype=torch.float16)[..., ::2]
    with pytest.raises(ValueError, match="head dimension must be contiguous"):
        sage_attention_2pp(q, q, q)


def test_rejects_autograd() -> None:
    q, k, v = _inputs()
    q.requires_grad_(True)
    with pytest.raises(RuntimeError, match="inference-only"):
        sage_attention_2pp(q, k, v)


@pytest.mark.parametrize("scale", [0.0, -1.0, float("inf"), float("nan")])
def test_rejects_invalid_scale(scale) -> None:
    q, k, v = _inputs()
    with pytest.raises(ValueError, match="finite and positive"):
        sage_attention_2pp(q, k, v, scale=scale)


def test_cpu_tensors_fail_loudly_instead_of_falling_back() -> None:
    q, k, v = _inputs()
    with pytest.raises(NotImplementedError, match="gfx950"):
        sage_attention_2pp(q, k, v)


def test_gfx950_dispatch_routes_to_custom_op_with_default_scale(monkeypatch) -> None:
    calls = []
    monkeypatch.setattr(dispatch.AcceleratorTarget, "from_device", classmethod(lambda cls, d: cls("hip", "gfx950")))
    monkeypatch.setattr(dispatch, "load_library", lambda: None)
    monkeypatch.setattr(dispatch, "hip_sage_attention_2pp", lambda q, k, v, s, c: calls.append((s, c)) or q)
    q, k, v = _inputs()
    sage_attention_2pp(q, k, v)
    sage_attention_2pp(q, k, v, scale=0.2, is_causal=True)
    assert calls == [(64**-0.5, False), (0.2, True)]


def test_gfx950_without_library_raises(monkeypatch, tmp_path) -> None:
    monkeypatch.setattr(dispatch.AcceleratorTarget, "from_device", classmethod(lambda cls, d: cls("hip", "gfx950")))
    monkeypatch.setattr(dispatch, "load_library", lambda: native.load_library(tmp_path / "absent.so"))
    monkeypatch.setattr(dispatch, "hip_sage_attention_2pp", lambda *a: pytest.fail("must not run without library"))
    q, k, v = _inputs()
    with pytest.raises(RuntimeError, match="not built"):
        sage_attention_2pp(q, k, v)


def test_custom_op_is_registered_with_reference_schema_and_fake() -> None:
    op = torch.ops.piper_kernels.sage_attention_2pp.default
    assert "Tensor query, Tensor key, Tensor value, float scale, bool is_causal" in str(op._schema)
    q = torch.empty((2, 3, 5, 64), dtype=torch.bfloat16, device="meta").transpose(0, 1)
    out = torch.ops.piper_kernels.sage_attention_2pp(q, q, q, 0.125, False)
    assert out.device.type == "meta" and out.shape == q.shape and out.is_contiguous()
