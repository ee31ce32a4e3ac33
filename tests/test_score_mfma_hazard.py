"""The score chains' first MFMA is inline assembly (``score_mfma_first`` in ``csrc/stream.h``):
its accumulator operand is the inline constant 1/(2 pi), which the compiler does not fold when
several MFMAs share the constant.  The compiler's hazard recognizer does not see inside inline
assembly, so the result may only be consumed where the hardware itself interlocks: as the whole
accumulator operand of the next MFMA of its chain.  A copy (``v_mov``, ``v_accvgpr_write``) or
any other VALU read of the result would need wait states nobody inserts.

This test compiles both attention sources to gfx950 assembly, exactly as the build does, and
checks every such MFMA in every instantiation: the first instruction after it that touches its
destination registers must be an MFMA that reads them as its full accumulator operand, with no
branch in between.

The same assembly (and the prep's) also shows each kernel's register spills: the attention loops
run at 168 VGPRs (three 4-wave workgroups per CU), where one value too many goes to scratch memory
and costs a store and a reload with its wait; every product kernel must keep a private segment of
zero bytes.
"""

from __future__ import annotations

import re
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT / "piper-kernels_amd"))

from piper_kernels._hip import build  # noqa: E402

SOURCES = ("attention.hip", "sage2pp.hip")
FIRST_MFMA = "v_mfma_i32_32x32x32_i8"
BIAS_OPERAND = "0.15915494"


def _registers(token: str) -> set[int]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", token)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", token)
    return {int(m.group(1))} if m else set()


def unsafe_first_mfmas(assembly: str) -> tuple[int, list[str]]:
    """(number of first-of-chain score MFMAs, descriptions of the unsafe ones)."""
    lines = assembly.splitlines()
    found, bad = 0, []
    for i, line in enumerate(lines):
        text = line.strip()
        if not (text.startswith(FIRST_MFMA) and BIAS_OPERAND in text):
            continue
        found += 1
        operands = [o.strip() for o in text.split(None, 1)[1].split(",")]
        dst_token, dst = operands[0], _registers(operands[0])
        verdict = "no consumer found"
        for later in lines[i + 1 :]:
            s = later.strip()
            if not s or s.startswith((";", ".")):
                continue
            if s.startswith(("s_cbranch", "s_branch", "s_setpc", "s_endpgm")):
                verdict = f"branch before the consumer: {s}"
                break
            parts = s.split(None, 1)
            if len(parts) < 2:
                continue
            ops = [o.strip() for o in parts[1].split(",")]
            if not any(_registers(o) & dst for o in ops):
                continue
            if (
                parts[0].startswith("v_mfma")
                and len(ops) >= 4
                and ops[3] == dst_token
                and not (_registers(ops[1]) & dst)
                and not (_registers(ops[2]) & dst)
            ):
                verdict = None
            else:
                verdict = f"consumed by: {s}"
            break
        if verdict:
            bad.append(f"{text} -> {verdict}")
    return found, bad


def test_checker_flags_a_copy_of_the_result() -> None:
    good = f"  {FIRST_MFMA} v[0:15], v[16:19], v[20:23], {BIAS_OPERAND}\n  v_mfma_i32_32x32x32_i8 v[0:15], v[24:27], v[28:31], v[0:15]\n"
    copied = f"  {FIRST_MFMA} v[0:15], v[16:19], v[20:23], {BIAS_OPERAND}\n  v_accvgpr_write_b32 a0, v3\n"
    assert unsafe_first_mfmas(good) == (1, [])
    found, bad = unsafe_first_mfmas(copied)
    assert found == 1 and len(bad) == 1 and "v_accvgpr_write_b32" in bad[0]


@pytest.fixture(scope="module")
def assembly(tmp_path_factory) -> dict[str, str]:
    """gfx950 assembly of the attention and prep sources, compiled in parallel as the build does."""
    try:
        compiler = build.hipcc()
    except FileNotFoundError:
        pytest.skip("hipcc not found")
    tmp = tmp_path_factory.mktemp("asm")
    flags = [f for f in build.COMPILE_FLAGS if f != "-fPIC"]
    procs = []
    for source in (*SOURCES, "prep.hip", "probe.hip"):
        out = tmp / (Path(source).stem + ".s")
        cmd = [compiler, *flags, f"-I{build.INCLUDE}", f"-I{build.CSRC}", "--cuda-device-only", "-S",
               str(build.CSRC / source), "-o", str(out)]
        procs.append((source, out, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)))
    texts = {}
    for source, out, proc in procs:
        _, err = proc.communicate(timeout=900)
        assert proc.returncode == 0, f"{source}: {err[-2000:]}"
        texts[source] = out.read_text()
    return texts


def test_every_inline_assembly_score_mfma_feeds_only_its_chain(assembly) -> None:
    total = 0
    for source in SOURCES:
        found, bad = unsafe_first_mfmas(assembly[source])
        assert found > 0, f"{source}: no inline-assembly score MFMA found"
        assert not bad, f"{source}: {len(bad)} unsafe of {found}:\n" + "\n".join(bad[:10])
        total += found
    assert total > 0


def kernel_spills(text: str) -> dict[str, tuple[int, int]]:
    """kernel name -> (private segment bytes, spilled VGPRs), from the code-object metadata."""
    meta = text[text.index("amdhsa.kernels:"):]
    spills = {}
    for m in re.finditer(r"\.name:\s+(\S+)\n(.*?)(?=\n  - |\Z)", meta, re.S):
        body = m.group(2)
        private = re.search(r"\.private_segment_fixed_size:\s+(\d+)", body)
        vgprs = re.search(r"\.vgpr_spill_count:\s+(\d+)", body)
        if private and vgprs:
            spills[m.group(1)] = (int(private.group(1)), int(vgprs.group(1)))
    return spills


def kernel_registers(text: str) -> dict[str, tuple[int, int]]:
    """kernel name -> (VGPRs + AGPRs per lane, largest workgroup), from the code-object metadata."""
    meta = text[text.index("amdhsa.kernels:"):]
    found = {}
    for entry in meta.split("\n  - ")[1:]:
        name = re.search(r"\.name:\s+(\S+)", entry)
        vgprs = re.search(r"\.vgpr_count:\s+(\d+)", entry)
        group = re.search(r"\.max_flat_workgroup_size:\s+(\d+)", entry)
        if name and vgprs and group:
            found[name.group(1)] = (int(vgprs.group(1)), int(group.group(1)))
    return found


def test_every_kernel_fits_its_largest_workgroup(assembly) -> None:
    """A SIMD holds 512 registers per lane; a workgroup of g threads puts ceil(g / 256) of its waves
    on each SIMD, so its kernel may use at most 512 / that many (in granules of 8).  Registers an
    inline-assembly block names explicitly are outside the compiler's budget, and a kernel over it
    builds but cannot be dispatched."""
    for source, text in assembly.items():
        registers = kernel_registers(text)
        assert registers, f"{source}: kernel metadata not found"
        for name, (vgprs, group) in registers.items():
            waves_per_simd = -(-group // 256)
            assert -(-vgprs // 8) * 8 * waves_per_simd <= 512, f"{source}: {name} needs {vgprs} registers at {group} threads"


def test_no_product_kernel_spills_to_scratch(assembly) -> None:
    for source, text in assembly.items():
        if source == "probe.hip":  # the measurement library, not a product kernel
            continue
        spills = kernel_spills(text)
        assert len(spills) > 10, f"{source}: kernel metadata not found"
        bad = {name: v for name, v in spills.items() if v != (0, 0)}
        assert not bad, f"{source}: {len(bad)} kernels use scratch (bytes, VGPRs): {sorted(bad.items())[:5]}"
