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


def test_every_native_call_runs_under_the_input_device_guard(monkeypatch) -> None:
    """The SageAttention2++ prep and launch are issued with the inputs' device current, on that
    device's current stream (as the reference's device-guard test, test_dispatch.py:37-96)."""
    from types import SimpleNamespace

    from piper_kernels.attention.sage_attention_2pp import hip

    real = native.load_library()
    guard, calls, streams = [], [], []

    class Guard:
        def __init__(self, device):
            self.device = torch.device(device)

        def __enter__(self):
            guard.append(self.device)

        def __exit__(self, *exc):
            guard.pop()

    class Recorder:
        def sage_prepared_layout(self, shape):
            return real.sage_prepared_layout(shape)

        def sage_prepare(self, args, stream):
            calls.append(("sage_prepare", list(guard), stream, args.flags))

        def sage_attention_forward(self, args, stream):
            calls.append(("sage_attention_forward", list(guard), stream, args.flags))

    def current_stream(device=None):
        streams.append(torch.device(device))
        return SimpleNamespace(cuda_stream=0x5EED)

    monkeypatch.setattr(native, "load_library", lambda *a: Recorder())
    monkeypatch.setattr(torch.cuda, "device", Guard)
    monkeypatch.setattr(torch.cuda, "current_stream", current_stream)
    monkeypatch.setattr(torch.Tensor, "record_stream", lambda self, stream: None)
    q, k, v = _inputs()
    hip._run_sage_attention_2pp(q, k, v, q.shape[-1] ** -0.5, False)
    hip._run_sage_attention_2pp(q, k, v, q.shape[-1] ** -0.5, True, qk_granularity="per_warp")
    hip._run_sage_attention_2pp(q, k, v, q.shape[-1] ** -0.5, False, accumulate="reference")
    assert [c[0] for c in calls] == ["sage_prepare", "sage_attention_forward"] * 3
    assert all(c[1] == [q.device] and c[2] == 0x5EED for c in calls)
    assert set(streams) == {q.device}
    assert calls[0][3] == native.PREPARE_QK_PER_THREAD  # the sage prep never quantises Q
    assert calls[1][3] == native.ATTENTION_QK_PER_THREAD
    assert calls[2][3] == 0 and calls[3][3] == 0
    assert calls[5][3] == native.ATTENTION_QK_PER_THREAD | native.SAGE_FP16_PARTIALS  # the reference's FP16 partials
    with pytest.raises(ValueError, match="accumulate"):
        hip._run_sage_attention_2pp(q, k, v, q.shape[-1] ** -0.5, False, accumulate="fp16")
