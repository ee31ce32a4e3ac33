"""The single-pass prep's progress argument, checked on a model of workgroup dispatch (CPU only).

The single-pass prep (``csrc/prep.hip``, ``prep_single_pass_kernel``) keeps each 256-row chunk of
a batch-head's K or V resident until the tensor's last chunk has arrived.  That terminates without
its bounded wait's fallback only if every tensor's chunks can all be resident at once.  The model
here is the dispatch the kernel relies on:

* workgroup b is dealt to XCC b % X (round-robin over the device's X XCCs);
* each XCC dispatches its workgroups in increasing order into its free slots;
* a chunk holds its slot until every chunk of its tensor has been dispatched, then finishes;
  causal V chunks and the two-step path's Q-block workgroups never wait.

The kernel maps hardware workgroup ids to logical ids with ``xcc_remap(b, n, X)``
(``csrc/common.h``), so that each XCC runs one consecutive range of logical ids, and the host takes
the single pass only when ``single_pass_resident(chunks, cus, xccs)`` holds (``csrc/kernels.h``):
4 * CUs / XCCs >= chunks.  Both are restated below.  The model shows that with the device's own XCC
count every tensor completes in all MI355X partition modes (8, 4, 2 or 1 XCCs of 32 CUs), and
that the earlier remap, which assumed 8 XCCs, leaves tensors unfinished on a 1-XCC device.
"""

from __future__ import annotations

import pytest


def xcc_remap(block: int, blocks: int, xccs: int) -> int:
    """csrc/common.h xcc_remap: hardware block id -> logical id (each XCC a consecutive range)."""
    xcc, local = block % xccs, block // xccs
    base, rem = divmod(blocks, xccs)
    return xcc * base + min(xcc, rem) + local


def single_pass_resident(chunks: int, cus: int, xccs: int) -> bool:
    """csrc/kernels.h single_pass_resident: a tensor's chunks fit in one XCC's slots."""
    return xccs > 0 and cus >= xccs and chunks <= 4 * (cus // xccs)


def simulate(batch_heads: int, chunks: int, xccs: int, slots: int, remap_xccs: int, *, causal: bool = False,
             query_workgroups: int = 0) -> int:
    """Dispatch the single pass's grid on `xccs` XCCs of `slots` workgroup slots each, the kernel
    remapping with `remap_xccs`; returns how many workgroups never finished (0: it terminates)."""
    kv = 2 * batch_heads * chunks
    blocks = kv + query_workgroups
    queues = [[b for b in range(blocks) if b % xccs == x] for x in range(xccs)]
    arrived = [0] * (2 * batch_heads)
    resident: list[list[int]] = [[] for _ in range(xccs)]
    finished = 0

    def waits(logical: int) -> bool:
        if logical >= kv:
            return False  # Q blocks of the two-step path
        tensor = logical // chunks
        return not (causal and tensor % 2 == 1)  # causal V is not centred

    progress = True
    while progress:
        progress = False
        for x in range(xccs):
            while queues[x] and len(resident[x]) < slots:
                logical = xcc_remap(queues[x].pop(0), blocks, remap_xccs)
                if logical < kv:
                    arrived[logical // chunks] += 1
                resident[x].append(logical)
                progress = True
        for x in range(xccs):
            keep = []
            for logical in resident[x]:
                if waits(logical) and arrived[logical // chunks] < chunks:
                    keep.append(logical)
                else:
                    finished += 1
                    progress = True
            resident[x] = keep
    return blocks - finished


def test_remap_is_a_permutation_with_one_range_per_xcc() -> None:
    for xccs in (1, 2, 3, 4, 8):
        for blocks in (1, 7, 64, 3072, 3077):
            logical = [xcc_remap(b, blocks, xccs) for b in range(blocks)]
            assert sorted(logical) == list(range(blocks))
            for x in range(xccs):
                mine = sorted(l for b, l in enumerate(logical) if b % xccs == x)
                assert mine == list(range(mine[0], mine[0] + len(mine))) if mine else True
                # the XCC dispatches its range in order
                assert [l for b, l in enumerate(logical) if b % xccs == x] == mine
    # with 8 XCCs it is the attention kernels' xcd_remap
    blocks = 3072
    assert [xcc_remap(b, blocks, 8) for b in range(16)] == [(b & 7) * (blocks >> 3) + (b >> 3) for b in range(16)]


@pytest.mark.parametrize("xccs", [8, 4, 2, 1])
@pytest.mark.parametrize("batch_heads,chunks", [(24, 64), (128, 32), (80, 64), (7, 64), (3, 17), (1, 1), (33, 63),
                                                (80, 128), (5, 128), (24, 100)])
def test_every_tensor_completes_in_every_partition_mode(xccs, batch_heads, chunks) -> None:
    cus = 32 * xccs  # MI355X: 32 CUs per XCC in every partition mode
    assert single_pass_resident(chunks, cus, xccs)
    slots = 4 * (cus // xccs)
    assert simulate(batch_heads, chunks, xccs, slots, xccs) == 0
    assert simulate(batch_heads, chunks, xccs, slots, xccs, causal=True) == 0
    assert simulate(batch_heads, chunks, xccs, slots, xccs, query_workgroups=50) == 0


def test_the_gate_is_what_keeps_it_terminating() -> None:
    # fewer slots per XCC than a tensor has chunks: the gate refuses, and the model stalls
    assert not single_pass_resident(64, 8 * 8, 8)
    assert simulate(24, 64, 8, 4 * 8, 8) > 0
    # exactly enough slots: accepted and terminates
    assert single_pass_resident(64, 8 * 16, 8)
    assert simulate(24, 64, 8, 64, 8) == 0
    # no XCC count from the runtime: the three-kernel path
    assert not single_pass_resident(16, 256, 0)


def test_a_remap_for_8_xccs_stalls_on_one_xcc() -> None:
    """The remap that assumed 8 XCCs interleaves 8 tensors' chunks on a 1-XCC (CPX) device: more
    chunks must be resident than its 128 slots, so the waits could only end by their bound."""
    assert simulate(24, 64, 1, 128, 8) > 0
    assert simulate(24, 64, 1, 128, 1) == 0
