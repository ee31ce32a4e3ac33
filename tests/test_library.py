"""The C-ABI library on the CPU: it loads, exports what the header declares, and its host-side
validation reports errors.  No call here reaches a kernel launch."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from piper_kernels._hip import library as native

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "piper_mi355x.h"


@pytest.fixture(scope="module")
def lib() -> native.NativeLibrary:
    if not native.library_available():
        pytest.fail("libpiper_mi355x.so is not built; run __graft_entry__.build()")
    return native.load_library()


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|const char\*)\s+(piper_\w+)\s*\(", text, re.MULTILINE))


def test_header_declares_exactly_the_bound_symbols() -> None:
    assert declared_functions() == set(native.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib) -> None:
    missing = [name for name in declared_functions() if not lib.has_symbol(name)]
    assert not missing
    assert lib.abi_version() == native.ABI_VERSION


def test_ctypes_structures_match_the_c_header(tmp_path) -> None:
    structs = {
        "piper_shape": native.PiperShape,
        "piper_tensor": native.PiperTensor,
        "piper_prepared": native.PiperPrepared,
        "piper_layout": native.PiperLayout,
        "piper_prepare_args": native.PiperPrepareArgs,
        "piper_attention_args": native.PiperAttentionArgs,
        "piper_attention_fused_args": native.PiperAttentionFusedArgs,
        "piper_sage_prepared": native.PiperSagePrepared,
        "piper_sage_layout": native.PiperSageLayout,
        "piper_sage_prepare_args": native.PiperSagePrepareArgs,
        "piper_sage_attention_args": native.PiperSageAttentionArgs,
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "piper_mi355x.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} %zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("{cname}.{field} %zu\\n", offsetof({cname}, {field}));')
    lines.append("  return 0; }")
    source = tmp_path / "abi.c"
    source.write_text("\n".join(lines))
    exe = tmp_path / "abi"
    subprocess.run(["gcc", f"-I{REPO / 'include'}", str(source), "-o", str(exe)], check=True)
    expected = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True).stdout.splitlines())
    for cname, cls in structs.items():
        assert int(expected[cname]) == ctypes.sizeof(cls), cname
        for field, _ in cls._fields_:
            assert int(expected[f"{cname}.{field}"]) == getattr(cls, field).offset, f"{cname}.{field}"


def mean_workspace_bytes(batch_heads: int, key_length: int, head_dim: int) -> int:
    """FP32 partials of the K and V means in torch's cascade order: one level-1 sum per chunk of
    L^2 rows (L = 16 rows per block up to 2^19 rows) plus one trailing-rows sum, per column."""
    ceil_log2 = (key_length - 1).bit_length() if key_length > 1 else 0
    block = 1 << max(4, ceil_log2 // 4)
    chunks = -(-key_length // (block * block))
    return 2 * batch_heads * (chunks + 1) * head_dim * 4


def prep_workspace_bytes(batch_heads: int, key_length: int, head_dim: int) -> int:
    """piper_prepare's workspace: the mean partials, then the single-pass prep's sync words: an
    arrival counter per batch-head tensor, the status word and spare words (4 * B * H + 4)."""
    return mean_workspace_bytes(batch_heads, key_length, head_dim) + 4 * (4 * batch_heads + 4)


@pytest.mark.parametrize(
    "shape", [(1, 24, 16384, 16384, 128), (2, 3, 35, 67, 64), (1, 1, 1, 1, 64), (4, 32, 8192, 8192, 128)]
)
def test_prepared_layout_sizes(lib, shape) -> None:
    b, h, sq, sk, d = shape
    layout = lib.prepared_layout(native.PiperShape(*shape))
    sq32, sk64 = -(-sq // 32) * 32, -(-sk // 64) * 64
    assert layout.query_code_bytes == b * h * sq32 * d
    # one scale slot per thread group of the per_thread granularity: 8 per Q block, 4 per K block
    assert layout.query_scale_bytes == b * h * (sq32 // 32) * 8 * 4
    assert layout.key_scale_bytes == b * h * (sk64 // 64) * 4 * 4
    assert layout.value_scale_bytes == b * h * sk64 * 4
    assert layout.mean_bytes == b * h * d * 4
    # one record per 64-key tile, laid out as the attention kernel's LDS stage: K rows of D + 16
    # bytes, V^T rows of 80 bytes, 64 log2 scales, 64 inverse multipliers, D corrections,
    # rounded up to a KiB multiple (the unit of the direct global -> LDS copy)
    raw = 64 * (d + 16) + d * 80 + 256 + 256 + 4 * d
    assert layout.kv_tile_bytes == native.kv_tile_bytes(d) == -(-raw // 1024) * 1024
    assert layout.kv_tile_bytes % 1024 == 0 and layout.kv_tile_bytes - raw < 1024
    assert layout.kv_tiles_bytes == b * h * (sk64 // 64) * layout.kv_tile_bytes
    assert layout.workspace_bytes == prep_workspace_bytes(b * h, sk, d)
    # the status word follows the mean partials and the 2 * B * H arrival counters
    assert layout.workspace_status_offset == mean_workspace_bytes(b * h, sk, d) + 4 * 2 * b * h
    assert layout.workspace_status_offset + 4 <= layout.workspace_bytes


def test_prepare_status_validates_before_touching_the_gpu(lib) -> None:
    with pytest.raises(RuntimeError, match="count is NULL"):
        lib._check(lib._lib.piper_prepare_status(ctypes.byref(native.PiperShape(1, 1, 8, 8, 64)), None, None, None),
                   "piper_prepare_status")
    with pytest.raises(RuntimeError, match="head_dim"):
        lib.prepare_status(native.PiperShape(1, 1, 8, 8, 32), 0x1000, 0)
    with pytest.raises(RuntimeError, match="static scratch"):
        lib.prepare_status(native.PiperShape(2, 64, 32768, 32768, 128), None, 0)


@pytest.mark.parametrize("bad", [(1, 1, 8, 8, 32), (0, 1, 8, 8, 64), (1, 1, 0, 8, 64)])
def test_layout_rejects_bad_shapes(lib, bad) -> None:
    with pytest.raises(RuntimeError, match="piper_prepared_layout failed"):
        lib.prepared_layout(native.PiperShape(*bad))


def test_prepare_validates_before_launching(lib) -> None:
    args = native.PiperPrepareArgs(abi_version=native.ABI_VERSION, dtype=native.FLOAT16, shape=native.PiperShape(1, 1, 8, 8, 64))
    with pytest.raises(RuntimeError, match="query pointer is NULL"):
        lib.prepare(args, 0)
    args.abi_version = 99
    with pytest.raises(RuntimeError, match="ABI version mismatch"):
        lib.prepare(args, 0)
    args.abi_version = native.ABI_VERSION
    args.dtype = native.FLOAT32
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        lib.prepare(args, 0)


def test_prepare_rejects_misaligned_inputs(lib) -> None:
    fake = 0x1000
    args = native.PiperPrepareArgs(
        abi_version=native.ABI_VERSION,
        dtype=native.FLOAT16,
        shape=native.PiperShape(1, 1, 8, 8, 64),
        query=native.PiperTensor(fake + 2, 512, 512, 64),
        key=native.PiperTensor(fake, 512, 512, 64),
        value=native.PiperTensor(fake, 512, 512, 64),
    )
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        lib.prepare(args, 0)


def test_attention_validates_before_launching(lib) -> None:
    args = native.PiperAttentionArgs(
        abi_version=native.ABI_VERSION, output_dtype=native.FLOAT16, shape=native.PiperShape(1, 1, 8, 8, 64), scale=0.0
    )
    with pytest.raises(RuntimeError, match="scale must be finite and positive"):
        lib.attention_forward(args, 0)
    args.scale = 0.125
    args.plan = 512
    with pytest.raises(RuntimeError, match="unknown plan"):
        lib.attention_forward(args, 0)
    # the work-queue plan: three workgroups per CU, no split, with a workspace for its counters
    args.plan = 256
    with pytest.raises(RuntimeError, match="work-queue plan needs PIPER_PLAN_THREE_WORKGROUPS"):
        lib.attention_forward(args, 0)
    args.plan = 16 | 32 | 256
    with pytest.raises(RuntimeError, match="work-queue plan has no key-range split"):
        lib.attention_forward(args, 0)
    args.plan = 16 | 256
    with pytest.raises(RuntimeError, match="work-queue plan needs a workspace of 256 bytes, got 0"):
        lib.attention_forward(args, 0)
    # the key-range split: three workgroups per CU, non-causal, with a workspace
    args.plan = 32
    with pytest.raises(RuntimeError, match="needs PIPER_PLAN_THREE_WORKGROUPS"):
        lib.attention_forward(args, 0)
    args.plan = 16 | 32
    with pytest.raises(RuntimeError, match="workspace of 4224 bytes, got 0"):  # 2 parts x 8 rows x (64 + 2) floats
        lib.attention_forward(args, 0)
    args.workspace, args.workspace_bytes = 0x1008, 1 << 20
    with pytest.raises(RuntimeError, match="workspace must be 16-byte aligned"):
        lib.attention_forward(args, 0)
    args.is_causal = 1
    with pytest.raises(RuntimeError, match="non-causal"):
        lib.attention_forward(args, 0)
    args.is_causal, args.workspace, args.workspace_bytes = 0, None, 0
    args.plan = 0
    args.flags = 2
    with pytest.raises(RuntimeError, match="unknown flags"):
        lib.attention_forward(args, 0)
    args.flags = native.ATTENTION_QK_PER_THREAD
    with pytest.raises(RuntimeError, match="NULL"):
        lib.attention_forward(args, 0)
    args.is_causal = 1
    args.shape = native.PiperShape(1, 1, 8, 9, 64)
    with pytest.raises(RuntimeError, match="equal query and key lengths"):
        lib.attention_forward(args, 0)


def test_prepare_flags(lib) -> None:
    args = native.PiperPrepareArgs(abi_version=native.ABI_VERSION, dtype=native.FLOAT16, shape=native.PiperShape(1, 1, 8, 8, 64))
    for flags in (8, 16, native.PREPARE_SKIP_QUERY | 8):
        args.flags = flags
        with pytest.raises(RuntimeError, match="unknown flags"):
            lib.prepare(args, 0)
    # the per-thread-group granularity is a known flag: validation goes on to the pointers
    args.flags = native.PREPARE_QK_PER_THREAD
    with pytest.raises(RuntimeError, match="query pointer is NULL"):
        lib.prepare(args, 0)
    # skipping the query: its (NULL) pointer is not inspected, the key's is
    args.flags = native.PREPARE_SKIP_QUERY
    with pytest.raises(RuntimeError, match="key pointer is NULL"):
        lib.prepare(args, 0)
    fake = 0x1000
    args.key = native.PiperTensor(fake, 512, 512, 64)
    args.value = native.PiperTensor(fake, 512, 512, 64)
    args.prepared = native.PiperPrepared(None, None, fake, fake, fake, fake, fake)
    args.workspace, args.workspace_bytes = None, 0
    with pytest.raises(RuntimeError, match="workspace"):
        lib.prepare(args, 0)
    args.flags = 0
    args.query = native.PiperTensor(fake, 512, 512, 64)
    with pytest.raises(RuntimeError, match="prepared output pointer is NULL"):
        lib.prepare(args, 0)
    # the self-mean diagnostic is a known flag, alone or with the others
    args.flags = native.PREPARE_SELF_MEAN | native.PREPARE_SKIP_QUERY | native.PREPARE_QK_PER_THREAD
    with pytest.raises(RuntimeError, match="workspace"):
        lib.prepare(args, 0)


def test_prepare_rejects_misaligned_means_and_workspace(lib) -> None:
    """The prep polls the means and counts arrivals in the workspace with 32-bit atomics: a
    key_mean that is not 4-byte aligned and a workspace that is not 16-byte aligned are refused
    on the host (a caller sub-allocating from a byte arena must keep them aligned)."""
    fake = 0x1000
    tensor = native.PiperTensor(fake, 512, 512, 64)
    args = native.PiperPrepareArgs(
        abi_version=native.ABI_VERSION, dtype=native.FLOAT16, flags=native.PREPARE_SKIP_QUERY,
        shape=native.PiperShape(1, 1, 8, 8, 64), key=tensor, value=tensor,
        prepared=native.PiperPrepared(None, None, fake, fake, fake + 2, fake, fake),
        workspace=fake, workspace_bytes=1 << 20,
    )
    with pytest.raises(RuntimeError, match="key_mean must be 4-byte aligned"):
        lib.prepare(args, 0)
    args.prepared = native.PiperPrepared(None, None, fake, fake, fake + 4, fake, fake)
    args.workspace = fake + 8
    with pytest.raises(RuntimeError, match="workspace must be 16-byte aligned"):
        lib.prepare(args, 0)


def test_prepare_static_validates_before_touching_the_gpu(lib) -> None:
    """piper_prepare_static rejects a caller workspace and shapes beyond its static scratch on the
    host, before it looks up the device scratch (so these run without a GPU)."""
    fake = 0x1000
    tensor = native.PiperTensor(fake, 1 << 20, 1 << 20, 128)
    args = native.PiperPrepareArgs(
        abi_version=native.ABI_VERSION,
        dtype=native.FLOAT16,
        flags=native.PREPARE_SKIP_QUERY,
        shape=native.PiperShape(1, 1, 64, 64, 128),
        key=tensor,
        value=tensor,
        prepared=native.PiperPrepared(None, None, fake, fake, fake, fake, fake),
        workspace=fake,
        workspace_bytes=1 << 20,
    )
    with pytest.raises(RuntimeError, match="takes no workspace"):
        lib.prepare_static(args, 0)
    args.workspace, args.workspace_bytes = None, 0
    # 128 batch-heads at Sk = 32768, D = 128 need 2 * 128 * 129 * 128 * 4 bytes: just over 16 MiB
    args.shape = native.PiperShape(2, 64, 32768, 32768, 128)
    assert lib.prepared_layout(args.shape).workspace_bytes > native.STATIC_SCRATCH_BYTES
    with pytest.raises(RuntimeError, match="more than the static 16777216 bytes"):
        lib.prepare_static(args, 0)
    # the largest benchmark workload fits (c5: 80 batch-heads at Sk = 32768)
    assert lib.prepared_layout(native.PiperShape(2, 40, 32768, 32768, 128)).workspace_bytes <= native.STATIC_SCRATCH_BYTES


def test_fused_attention_validates_before_launching(lib) -> None:
    fake = 0x1000
    args = native.PiperAttentionFusedArgs(
        abi_version=native.ABI_VERSION,
        dtype=native.FLOAT32,
        output_dtype=native.FLOAT16,
        shape=native.PiperShape(1, 1, 8, 8, 64),
        scale=0.125,
        query=native.PiperTensor(fake, 512, 512, 64),
        # no query codes or scales: the fused kernel quantises the query itself
        prepared=native.PiperPrepared(None, None, fake, fake, fake, fake, fake),
    )
    with pytest.raises(RuntimeError, match="query dtype"):
        lib.attention_forward_fused(args, 0)
    args.dtype = native.BFLOAT16
    args.query = native.PiperTensor(None, 512, 512, 64)
    with pytest.raises(RuntimeError, match="query pointer is NULL"):
        lib.attention_forward_fused(args, 0)
    args.query = native.PiperTensor(fake + 2, 512, 512, 64)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        lib.attention_forward_fused(args, 0)
    args.query = native.PiperTensor(fake, 512, 512, 64)
    with pytest.raises(RuntimeError, match="output pointer is NULL"):
        lib.attention_forward_fused(args, 0)
    args.plan = 512
    with pytest.raises(RuntimeError, match="unknown plan"):
        lib.attention_forward_fused(args, 0)
    args.plan, args.flags = 0, 4
    with pytest.raises(RuntimeError, match="unknown flags"):
        lib.attention_forward_fused(args, 0)
    args.flags, args.abi_version = native.ATTENTION_QK_PER_THREAD, native.ABI_VERSION + 1
    with pytest.raises(RuntimeError, match="ABI version mismatch"):
        lib.attention_forward_fused(args, 0)


@pytest.mark.parametrize("shape", [(1, 24, 16384, 16384, 128), (2, 3, 35, 67, 64), (1, 1, 1, 1, 64)])
def test_sage_prepared_layout_sizes(lib, shape) -> None:
    b, h, sq, sk, d = shape
    layout = lib.sage_prepared_layout(native.PiperShape(*shape))
    nkb = -(-sk // 64)
    # K rows of D + 16 bytes, FP8 V^T rows of 80 bytes: 19 KiB (D = 128) and 10 KiB (D = 64)
    assert layout.kv_tile_bytes == native.sage_tile_bytes(d) == {128: 19 * 1024, 64: 10 * 1024}[d]
    assert layout.kv_tiles_bytes == b * h * nkb * layout.kv_tile_bytes
    assert layout.key_scale_bytes == b * h * nkb * 4 * 4  # four K thread-group slots per block
    assert layout.mean_bytes == b * h * d * 4
    assert layout.workspace_bytes == mean_workspace_bytes(b * h, sk, d)


def test_sage_prepare_validates_before_launching(lib) -> None:
    fake = 0x1000
    args = native.PiperSagePrepareArgs(abi_version=native.ABI_VERSION, dtype=native.FLOAT32,
                                       shape=native.PiperShape(1, 1, 8, 8, 64))
    with pytest.raises(RuntimeError, match="float16 or bfloat16"):
        lib.sage_prepare(args, 0)
    args.dtype = native.FLOAT16
    args.flags = 1  # PIPER_PREPARE_SKIP_QUERY means nothing to this prep (it never quantises Q)
    with pytest.raises(RuntimeError, match="unknown flags"):
        lib.sage_prepare(args, 0)
    args.flags = native.PREPARE_QK_PER_THREAD
    with pytest.raises(RuntimeError, match="key pointer is NULL"):
        lib.sage_prepare(args, 0)
    args.key = native.PiperTensor(fake, 512, 512, 64)
    args.value = native.PiperTensor(fake + 8, 512, 512, 64)
    with pytest.raises(RuntimeError, match="value must be 16-byte aligned"):
        lib.sage_prepare(args, 0)
    args.value = native.PiperTensor(fake, 512, 512, 64)
    with pytest.raises(RuntimeError, match="prepared output pointer is NULL"):
        lib.sage_prepare(args, 0)
    args.prepared = native.PiperSagePrepared(fake, fake, fake + 4, fake)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        lib.sage_prepare(args, 0)
    args.prepared = native.PiperSagePrepared(fake, fake, fake, fake)
    with pytest.raises(RuntimeError, match="workspace"):
        lib.sage_prepare(args, 0)


def test_sage_attention_validates_before_launching(lib) -> None:
    fake = 0x1000
    args = native.PiperSageAttentionArgs(
        abi_version=native.ABI_VERSION, dtype=native.FLOAT16, output_dtype=native.FLOAT16,
        shape=native.PiperShape(1, 1, 8, 8, 64), scale=0.0,
        query=native.PiperTensor(fake, 512, 512, 64), prepared=native.PiperSagePrepared(fake, fake, fake, fake),
    )
    with pytest.raises(RuntimeError, match="scale must be finite and positive"):
        lib.sage_attention_forward(args, 0)
    args.scale = 0.125
    args.plan = 512
    with pytest.raises(RuntimeError, match="unknown plan"):
        lib.sage_attention_forward(args, 0)
    args.plan = 16 | 32
    with pytest.raises(RuntimeError, match="no key-range split"):
        lib.sage_attention_forward(args, 0)
    args.plan = 16 | 256
    with pytest.raises(RuntimeError, match="no work-queue plan"):
        lib.sage_attention_forward(args, 0)
    args.plan, args.flags = 0, 4
    with pytest.raises(RuntimeError, match="unknown flags"):
        lib.sage_attention_forward(args, 0)
    args.flags = native.ATTENTION_QK_PER_THREAD | native.SAGE_FP16_PARTIALS  # both known
    with pytest.raises(RuntimeError, match="output pointer is NULL"):
        lib.sage_attention_forward(args, 0)
    args.plan = 16  # three workgroups per CU: SageAttention2++'s default plan
    with pytest.raises(RuntimeError, match="output pointer is NULL"):
        lib.sage_attention_forward(args, 0)
    args.is_causal = 1
    args.shape = native.PiperShape(1, 1, 8, 9, 64)
    with pytest.raises(RuntimeError, match="equal query and key lengths"):
        lib.sage_attention_forward(args, 0)
    args.is_causal, args.shape = 0, native.PiperShape(1, 1, 8, 8, 32)
    with pytest.raises(RuntimeError, match="head_dim must be 64 or 128"):
        lib.sage_attention_forward(args, 0)


# ---- the measurement library (libpiper_probe.so, include/piper_probe.h) --------------------
PROBE_HEADER = REPO / "include" / "piper_probe.h"


@pytest.fixture(scope="module")
def probe() -> native.ProbeLibrary:
    return native.load_probe_library()


def test_operator_library_exports_no_probe(lib) -> None:
    """The probes live in their own library: the operator's ABI exports only what its header
    declares (a test and measurement probe is no part of the product)."""
    for name in native.PROBE_EXPORTED_SYMBOLS:
        assert not lib.has_symbol(name), name
    assert "mfma_probe" not in HEADER.read_text()


def test_probe_library_exports_exactly_its_header(probe) -> None:
    text = PROBE_HEADER.read_text()
    declared = set(re.findall(r"^\s*(?:int|const char\*)\s+(piper_\w+)\s*\(", text, re.MULTILINE))
    assert declared == set(native.PROBE_EXPORTED_SYMBOLS)
    assert all(probe.has_symbol(name) for name in declared)


def test_probe_constants_and_structs_match_the_header(tmp_path) -> None:
    source = tmp_path / "probe.c"
    roles = ["IDLE", "MFMA", "FMA", "EXP", "CVT", "MIX", "VALU_MIX", "LDS", "MFMA_FMA", "MIX_VGPR", "CLUSTER", "ADD_LIT",
             "ADD_SGPR", "FMA_SPLIT", "FMA_SAME", "FMAC_SAME", "MAX3", "PERM"]
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "piper_probe.h"', "int main(void) {",
             '  printf("%d %d %d %d %d %d %d %d %d\\n", PIPER_PROBE_ABI_VERSION, PIPER_MFMA_PROBE_I8, PIPER_MFMA_PROBE_F8,'
             ' PIPER_MFMA_PROBE_P_CODES_U8, PIPER_MFMA_PROBE_P_CODES_FP8, PIPER_MFMA_PROBE_P_CODES_U8_SCALED,'
             ' PIPER_MFMA_PROBE_THREADS,'
             ' PIPER_MFMA_PROBE_OPS(PIPER_MFMA_PROBE_I8), PIPER_MFMA_PROBE_OPS(PIPER_MFMA_PROBE_F8));',
             '  printf("%d\\n", PIPER_CLOCK_PROBE_MAX_WORKGROUPS);']
    lines.append('  printf("' + " ".join(["%d"] * (len(roles) + 3)) + '\\n", '
                 + ", ".join(f"PIPER_ISSUE_{r}" for r in roles)
                 + ", PIPER_ISSUE_ROLES, PIPER_ISSUE_MAX_WAVES_PER_SIMD, PIPER_ISSUE_RECORDS_PER_WORKGROUP);")
    for cname, cls in (("piper_issue_record", native.PiperIssueRecord), ("piper_issue_probe_args", native.PiperIssueProbeArgs)):
        lines.append(f'  printf("%zu\\n", sizeof({cname}));')
        for field, _ in cls._fields_:
            lines.append(f'  printf("%zu\\n", offsetof({cname}, {field}));')
    lines.append("  return 0; }")
    source.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "probe"
    subprocess.run(["gcc", f"-I{REPO / 'include'}", str(source), "-o", str(exe)], check=True)
    values = list(map(int, subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()))
    assert values[:9] == [native.PROBE_ABI_VERSION, native.MFMA_PROBE_I8, native.MFMA_PROBE_F8,
                          native.MFMA_PROBE_P_CODES_U8, native.MFMA_PROBE_P_CODES_FP8,
                          native.MFMA_PROBE_P_CODES_U8_SCALED, native.MFMA_PROBE_THREADS,
                          native.MFMA_PROBE_OPS[native.MFMA_PROBE_I8], native.MFMA_PROBE_OPS[native.MFMA_PROBE_F8]]
    assert values[9] == native.CLOCK_PROBE_MAX_WORKGROUPS
    values = values[:9] + values[10:]
    n = len(roles)
    assert values[9:9 + n] == list(range(len(native.ISSUE_ROLES)))
    assert [r.upper() for r in native.ISSUE_ROLES] == roles
    assert values[9 + n:12 + n] == [len(native.ISSUE_ROLES), native.ISSUE_MAX_WAVES_PER_SIMD,
                                    native.ISSUE_RECORDS_PER_WORKGROUP]
    offsets = values[12 + n:]
    expected = []
    for cls in (native.PiperIssueRecord, native.PiperIssueProbeArgs):
        expected.append(ctypes.sizeof(cls))
        expected.extend(getattr(cls, field).offset for field, _ in cls._fields_)
    assert offsets == expected
    # 32x32x32 INT8 and 32x32x64 FP8: two operations per multiply-add
    assert native.MFMA_PROBE_OPS == {native.MFMA_PROBE_I8: 2 * 32 * 32 * 32, native.MFMA_PROBE_F8: 2 * 32 * 32 * 64}


def test_mfma_probe_validates_before_launching(probe) -> None:
    with pytest.raises(RuntimeError, match="unknown MFMA probe kind"):
        probe.mfma_probe(5, 1, 1, 0x1000, 0)
    with pytest.raises(RuntimeError, match="unknown MFMA probe kind"):
        probe.mfma_probe(-1, 1, 1, 0x1000, 0)
    with pytest.raises(RuntimeError, match="workgroups and"):
        probe.mfma_probe(native.MFMA_PROBE_I8, 0, 1, 0x1000, 0)
    with pytest.raises(RuntimeError, match="workgroups and"):
        probe.mfma_probe(native.MFMA_PROBE_F8, 1, 0, 0x1000, 0)
    with pytest.raises(RuntimeError, match="sink must be"):
        probe.mfma_probe(native.MFMA_PROBE_I8, 1, 1, 0, 0)
    with pytest.raises(RuntimeError, match="sink must be"):
        probe.mfma_probe(native.MFMA_PROBE_I8, 1, 1, 0x1002, 0)


def test_issue_probe_validates_before_launching(probe) -> None:
    args = native.PiperIssueProbeArgs(waves_per_simd=0, workgroups=1, cycle_budget=10000, records=0x1000)
    with pytest.raises(RuntimeError, match="waves_per_simd"):
        probe.issue_probe(args, 0)
    args.waves_per_simd = 5
    with pytest.raises(RuntimeError, match="waves_per_simd"):
        probe.issue_probe(args, 0)
    args.waves_per_simd, args.workgroups = 2, 0
    with pytest.raises(RuntimeError, match="workgroups"):
        probe.issue_probe(args, 0)
    args.workgroups, args.cycle_budget = 1, 10
    with pytest.raises(RuntimeError, match="cycle_budget"):
        probe.issue_probe(args, 0)
    args.cycle_budget, args.records = 10000, 0x1004
    with pytest.raises(RuntimeError, match="records"):
        probe.issue_probe(args, 0)
    args.records = 0x1000
    args.roles[1] = len(native.ISSUE_ROLES)
    with pytest.raises(RuntimeError, match="unknown role"):
        probe.issue_probe(args, 0)
    args.roles[0] = native.ISSUE_ROLES.index("mix_vgpr")  # runs in a kernel of its own
    args.roles[1] = native.ISSUE_ROLES.index("fma")
    with pytest.raises(RuntimeError, match="MIX_VGPR"):
        probe.issue_probe(args, 0)


def test_mfma_probe_expected_words() -> None:
    from piper_kernels.measure import mfma_probe_expected

    assert mfma_probe_expected(native.MFMA_PROBE_I8, 4096) == 4096 * 64 * 32
    assert mfma_probe_expected(native.MFMA_PROBE_I8, 1 << 21) == (64 * 32 << 21) % (1 << 32)
    assert mfma_probe_expected(native.MFMA_PROBE_F8, 4096) == 0x4B800000  # 2^24 as FP32
    for kind in (native.MFMA_PROBE_P_CODES_U8, native.MFMA_PROBE_P_CODES_FP8):
        with pytest.raises(ValueError):
            mfma_probe_expected(kind, 1)


def test_probability_codes_rejects_unknown_codes() -> None:
    import torch
    from piper_kernels.measure import probability_codes

    with pytest.raises(ValueError, match="'u8' or 'fp8'"):
        probability_codes([0.5], "int4", torch.device("cpu"))


@pytest.mark.parametrize("shape", [(1, 1, 131072, 131072, 128), (1, 8, 8192, 8192, 128), (2, 3, 35, 67, 64)])
def test_attention_workspace_bytes(lib, shape) -> None:
    """Only the key-range split plans need a workspace: parts x B x H x Sq rows of D numerator
    floats plus (den, mref)."""
    b, h, sq, _, d = shape
    for plan in (0, 1, 16, 31):
        assert lib.attention_workspace_bytes(native.PiperShape(*shape), plan) == 0
    for parts in range(2, 9):
        plan = 16 | ((parts - 1) << 5)
        assert lib.attention_workspace_bytes(native.PiperShape(*shape), plan) == parts * b * h * sq * (d + 2) * 4
    # the work-queue plan: its counters
    assert lib.attention_workspace_bytes(native.PiperShape(*shape), 16 | 256) == 256
    with pytest.raises(RuntimeError, match="unknown plan"):
        lib.attention_workspace_bytes(native.PiperShape(*shape), 512)
