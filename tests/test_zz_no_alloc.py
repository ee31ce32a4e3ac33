"""piper_prepare_static (no caller workspace: the prep's workspace lives in the library's static
per-GPU scratch) against piper_prepare, through the C ABI on MI355X: every prepared byte the
header specifies and the attention output equal, on calls in a row, each smaller than the one
before (non-causal single pass, the three-kernel path at D = 64, causal single pass); and a call
on preallocated buffers makes no allocation at all."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import gpu_attention, log, prepared_numpy

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, Sq, Sk, D, dtype, causal): the second is smaller and reuses the scratch the first filled
    (1, 4, 4096, 4096, 128, torch.float16, False),
    (1, 2, 300, 193, 64, torch.bfloat16, False),
    (1, 2, 192, 192, 128, torch.bfloat16, True),
]


def _inputs(case, seed):
    b, h, sq, sk, d, dtype, _ = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, sq, d), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, d), generator=g) + torch.randn((b, h, 1, d), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, d), generator=g) + 2 * torch.randn((b, h, 1, d), generator=g)).to(dtype)
    return q, k, v


def _prepare(q, k, v, d, causal, device, static):
    from piper_kernels.attention.piper_attention.hip import _prepare_piper_attention

    with torch.no_grad():
        prepared = _prepare_piper_attention(
            q.to(device), k.to(device), v.to(device), d**-0.5, causal, static_workspace=static
        )
    torch.cuda.synchronize(device)
    return prepared


def test_static_scratch_prep_equals_workspace_prep(gfx950_device) -> None:
    for i, case in enumerate(CASES):
        b, h, sq, sk, d, dtype, causal = case
        log(f"[case] piper_prepare_static call {i + 1}: {case}")
        q, k, v = _inputs(case, 700 + i)
        static = _prepare(q, k, v, d, causal, gfx950_device, static=True)
        reference = _prepare(q, k, v, d, causal, gfx950_device, static=False)
        got, expected = prepared_numpy(static), prepared_numpy(reference)
        for name, value in expected.items():
            if value is None:
                assert got[name] is None, name
                continue
            a = np.ascontiguousarray(got[name])
            e = np.ascontiguousarray(value)
            assert a.shape == e.shape and a.dtype == e.dtype, name
            assert np.array_equal(a.view(np.uint8), e.view(np.uint8)), f"{name} differs (call {i + 1})"
        out_static = gpu_attention(static, torch.float32)
        out_reference = gpu_attention(reference, torch.float32)
        assert torch.equal(out_static, out_reference), f"attention output differs (call {i + 1})"


def test_static_prep_allocates_nothing(gfx950_device) -> None:
    """A second piper_prepare_static on buffers a first call left: torch's allocator records no
    allocation and no reserved byte more across it, and the outputs repeat bit for bit."""
    from piper_kernels._hip import library as native
    from piper_kernels.attention.piper_attention.hip import _native_input

    case = (1, 2, 1024, 1024, 128, torch.float16, False)
    log(f"[case] piper_prepare_static on preallocated buffers: {case}")
    b, h, sq, sk, d, dtype, causal = case
    q, k, v = (t.to(gfx950_device) for t in _inputs(case, 900))
    first = _prepare(q, k, v, d, causal, gfx950_device, static=True)
    # every buffer the prep writes (the output is the attention kernel's, left uninitialised here)
    saved = {name: value.clone() for name, value in vars(first).items()
             if isinstance(value, torch.Tensor) and name != "output"}
    q, q_arg = _native_input(q)
    k, k_arg = _native_input(k)
    v, v_arg = _native_input(v)
    args = native.PiperPrepareArgs(
        abi_version=native.ABI_VERSION, dtype=native.FLOAT16, is_causal=0, flags=native.PREPARE_QK_PER_THREAD,
        shape=native.PiperShape(b, h, sq, sk, d), query=q_arg, key=k_arg, value=v_arg,
        prepared=first.native_prepared(), workspace=None, workspace_bytes=0,
    )
    lib = native.load_library()
    stream = torch.cuda.current_stream(gfx950_device)
    torch.cuda.synchronize(gfx950_device)
    before = torch.cuda.memory_stats(gfx950_device)
    lib.prepare_static(args, stream.cuda_stream)
    torch.cuda.synchronize(gfx950_device)
    after = torch.cuda.memory_stats(gfx950_device)
    for key in ("allocation.all.allocated", "reserved_bytes.all.allocated", "segment.all.allocated"):
        assert after.get(key, 0) == before.get(key, 0), f"{key}: {before.get(key)} -> {after.get(key)}"
    for name, value in saved.items():
        assert torch.equal(getattr(first, name).view(torch.uint8), value.view(torch.uint8)), f"{name} changed"
