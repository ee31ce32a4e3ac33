"""The single-pass prep's bounded-wait fallback on MI355X, forced from the host.

A chunk of the single pass waits for its batch-head tensor's mean, which the tensor's last chunk
publishes; the wait is bounded, and a chunk whose wait ends computes the mean itself from K/V in
HBM in the same cascade order (csrc/prep.hip, column_mean_from_rows) and is counted in the prep's
status word.  PIPER_PREPARE_SELF_MEAN makes every waiting chunk take that path at once (a wait of
zero polls), so every kernel still runs to its normal end: the codes, scales and means must be
bit-identical to the ordinary prep (and to the oracle, the reference's torch.mean order), and the
status word must count exactly the chunks that waited: (chunks - 1) per centred tensor.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _parity import assert_prep_bit_exact, log, prepared_numpy
from oracle import piper_oracle as oracle
from piper_kernels._hip import library as native

pytestmark = pytest.mark.gpu

CASES = [
    # (B, H, Sq, Sk, dtype, causal); D = 128, the single pass's head size
    (1, 3, 4096, 4096, torch.float16, False),  # 16 chunks
    (2, 2, 1000, 1000, torch.bfloat16, False),  # 4 chunks, the last short (ragged)
    (1, 2, 16384, 16384, torch.float16, False),  # 64 chunks
    (1, 1, 32768, 32768, torch.float16, False),  # 128 chunks: the single pass's longest sequence
    (1, 2, 4096, 4096, torch.bfloat16, True),  # causal: only K is centred and waits
    (1, 1, 100, 100, torch.float16, False),  # one chunk: it is its tensor's last, nothing waits
]


def _inputs(case, seed):
    b, h, sq, sk, dtype, _ = case
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, h, sq, 128), generator=g).to(dtype)
    k = (torch.randn((b, h, sk, 128), generator=g) + 2 * torch.randn((b, h, 1, 128), generator=g)).to(dtype)
    v = (torch.randn((b, h, sk, 128), generator=g) + 4 * torch.randn((b, h, 1, 128), generator=g)).to(dtype)
    return q, k, v


def _prepare(q, k, v, causal, device, flags, static=False):
    from piper_kernels.attention.piper_attention.hip import _prepare_piper_attention

    b, h, sq, d = q.shape
    shape = native.PiperShape(b, h, sq, k.shape[2], d)
    lib = native.load_library()
    workspace = None
    if not static:
        workspace = torch.empty(lib.prepared_layout(shape).workspace_bytes, dtype=torch.uint8, device=device)
    with torch.no_grad():
        # the two-step prep: the single pass's grid also carries the query blocks
        prepared = _prepare_piper_attention(q.to(device), k.to(device), v.to(device), d**-0.5, causal,
                                            workspace=workspace, static_workspace=static, prep_flags=flags)
    stream = torch.cuda.current_stream(device)
    status = lib.prepare_status(shape, None if static else workspace.data_ptr(), stream.cuda_stream)
    return prepared, status


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}x{c[1]}x{c[2]}x{c[3]}-{str(c[4])[6:]}-{'causal' if c[5] else 'full'}")
def test_self_computed_means_are_bit_identical_and_counted(case, gfx950_device) -> None:
    b, h, sq, sk, dtype, causal = case
    chunks = -(-sk // 256)
    log(f"[case] prep fallback {case}: {chunks} chunks per tensor")
    q, k, v = _inputs(case, 4100 + sq)
    normal, normal_status = _prepare(q, k, v, causal, gfx950_device, 0)
    forced, forced_status = _prepare(q, k, v, causal, gfx950_device, native.PREPARE_SELF_MEAN)
    centred = 1 if causal else 2
    expected_count = (chunks - 1) * centred * b * h
    log(f"  status: ordinary {normal_status}, forced {forced_status} (expected {expected_count})")
    assert normal_status == 0
    assert forced_status == expected_count
    got, want = prepared_numpy(forced), prepared_numpy(normal)
    for name, value in want.items():
        if value is None:
            assert got[name] is None, name
            continue
        assert np.array_equal(np.ascontiguousarray(got[name]).view(np.uint8),
                              np.ascontiguousarray(value).view(np.uint8)), f"{name} differs on the fallback path"
    if sk <= 4096:  # the oracle: the reference's torch.mean order and codes
        assert_prep_bit_exact(got, oracle.prepare(q, k, v, causal, "per_thread"), forced.shape, causal)


def test_static_scratch_status_counts_the_forced_fallback(gfx950_device) -> None:
    case = (1, 2, 2048, 2048, torch.float16, False)
    log(f"[case] piper_prepare_static fallback {case}")
    q, k, v = _inputs(case, 77)
    forced, status = _prepare(q, k, v, False, gfx950_device, native.PREPARE_SELF_MEAN, static=True)
    assert status == (8 - 1) * 2 * 2
    normal, status = _prepare(q, k, v, False, gfx950_device, 0, static=True)
    assert status == 0  # each call clears the word it counts in
    got, want = prepared_numpy(forced), prepared_numpy(normal)  # every byte the header specifies
    for name, value in want.items():
        assert np.array_equal(np.ascontiguousarray(got[name]).view(np.uint8),
                              np.ascontiguousarray(value).view(np.uint8)), f"{name} differs on the fallback path"
