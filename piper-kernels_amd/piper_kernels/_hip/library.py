"""ctypes bindings of ``libpiper_mi355x.so`` (the operator's C ABI, ``include/piper_mi355x.h``)
and of ``libpiper_probe.so`` (measurement probes, ``include/piper_probe.h``; loaded only by
bench.py and the tests).

The structures below mirror the header field for field.  torch is imported before the
library is opened: torch ships its own HIP runtime with the same SONAME
(``libamdhip64.so.7``), and the library must bind to that instance so that torch's
stream handles and allocations are valid inside it.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime first; see module docstring)

from .build import LIBRARY_PATH, PROBE_LIBRARY_PATH

ABI_VERSION = 5
QUERY_BLOCK = 32
KEY_BLOCK = 64
QUERY_SCALE_SLOTS = 8  # per 32-row Q block: one per thread group (per-block prep repeats its scale)
KEY_SCALE_SLOTS = 4  # per 64-row K block

FLOAT16 = 0
BFLOAT16 = 1
FLOAT32 = 2

EXPORTED_SYMBOLS = (
    "piper_abi_version",
    "piper_prepared_layout",
    "piper_prepare",
    "piper_prepare_static",
    "piper_prepare_status",
    "piper_attention_forward",
    "piper_attention_forward_fused",
    "piper_attention_workspace_bytes",
    "piper_sage_prepared_layout",
    "piper_sage_prepare",
    "piper_sage_attention_forward",
    "piper_last_error",
)

STATIC_SCRATCH_BYTES = 16 << 20  # PIPER_STATIC_SCRATCH_BYTES: piper_prepare_static's per-GPU scratch
PREPARE_SKIP_QUERY = 1  # piper_prepare_args.flags
PREPARE_QK_PER_THREAD = 2
PREPARE_SELF_MEAN = 4  # diagnostic: waiting single-pass chunks compute the mean themselves (the wait's fallback)
ATTENTION_QK_PER_THREAD = 1  # piper_attention_args.flags / piper_attention_fused_args.flags
SAGE_FP16_PARTIALS = 2  # piper_sage_attention_args.flags: FP16-rounded 64-key partial products

_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p


class PiperShape(ctypes.Structure):
    _fields_ = [
        ("batch", _i64),
        ("heads", _i64),
        ("query_length", _i64),
        ("key_length", _i64),
        ("head_dim", _i64),
    ]


class PiperTensor(ctypes.Structure):
    _fields_ = [("data", _ptr), ("stride_batch", _i64), ("stride_head", _i64), ("stride_seq", _i64)]


class PiperPrepared(ctypes.Structure):
    _fields_ = [
        ("query_code", _ptr),
        ("query_scale", _ptr),
        ("key_scale", _ptr),
        ("value_scale", _ptr),
        ("key_mean", _ptr),
        ("value_mean", _ptr),
        ("kv_tiles", _ptr),
    ]


class PiperLayout(ctypes.Structure):
    _fields_ = [
        ("query_code_bytes", _i64),
        ("query_scale_bytes", _i64),
        ("key_scale_bytes", _i64),
        ("value_scale_bytes", _i64),
        ("mean_bytes", _i64),
        ("kv_tile_bytes", _i64),
        ("kv_tiles_bytes", _i64),
        ("workspace_bytes", _i64),
        ("workspace_status_offset", _i64),
    ]


def kv_k_stride(head_dim: int) -> int:
    """Bytes per K row in a tile record (D codes + 16 bytes of padding)."""
    return head_dim + 16


KV_V_STRIDE = 64 + 16  # bytes per V^T row in a tile record (64 codes + 16 bytes of padding)


def kv_offsets(head_dim: int) -> dict:
    """Byte offsets of the regions of one tile record (PIPER_KV_* in the C header)."""
    v = 64 * kv_k_stride(head_dim)
    log2 = v + head_dim * KV_V_STRIDE
    return {"key": 0, "key_scale": head_dim, "value": v, "log2": log2, "inv": log2 + 256, "corr": log2 + 512}


def kv_tile_bytes(head_dim: int) -> int:
    """Bytes of one 64-key tile record (PIPER_KV_TILE_BYTES in the C header): a KiB multiple."""
    return (kv_offsets(head_dim)["corr"] + 4 * head_dim + 1023) // 1024 * 1024


class PiperPrepareArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("is_causal", _i32),
        ("flags", _i32),
        ("shape", PiperShape),
        ("query", PiperTensor),
        ("key", PiperTensor),
        ("value", PiperTensor),
        ("prepared", PiperPrepared),
        ("workspace", _ptr),
        ("workspace_bytes", _i64),
    ]


class PiperAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("output_dtype", _i32),
        ("is_causal", _i32),
        ("plan", _i32),
        ("shape", PiperShape),
        ("scale", ctypes.c_float),
        ("flags", _i32),
        ("prepared", PiperPrepared),
        ("output", _ptr),
        ("workspace", _ptr),
        ("workspace_bytes", _i64),
    ]


class PiperAttentionFusedArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("output_dtype", _i32),
        ("is_causal", _i32),
        ("plan", _i32),
        ("scale", ctypes.c_float),
        ("flags", _i32),
        ("reserved", _i32),
        ("shape", PiperShape),
        ("query", PiperTensor),
        ("prepared", PiperPrepared),
        ("output", _ptr),
        ("workspace", _ptr),
        ("workspace_bytes", _i64),
    ]


def sage_tile_bytes(head_dim: int) -> int:
    """Bytes of one SageAttention2++ tile record (PIPER_SAGE_TILE_BYTES): K rows, FP8 V^T rows."""
    return (64 * kv_k_stride(head_dim) + head_dim * KV_V_STRIDE + 1023) // 1024 * 1024


class PiperSagePrepared(ctypes.Structure):
    _fields_ = [("key_scale", _ptr), ("key_mean", _ptr), ("value_scale", _ptr), ("kv_tiles", _ptr)]


class PiperSageLayout(ctypes.Structure):
    _fields_ = [
        ("key_scale_bytes", _i64),
        ("mean_bytes", _i64),
        ("kv_tile_bytes", _i64),
        ("kv_tiles_bytes", _i64),
        ("workspace_bytes", _i64),
    ]


class PiperSagePrepareArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("flags", _i32),
        ("reserved", _i32),
        ("shape", PiperShape),
        ("key", PiperTensor),
        ("value", PiperTensor),
        ("prepared", PiperSagePrepared),
        ("workspace", _ptr),
        ("workspace_bytes", _i64),
    ]


class PiperSageAttentionArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", _i32),
        ("dtype", _i32),
        ("output_dtype", _i32),
        ("is_causal", _i32),
        ("plan", _i32),
        ("scale", ctypes.c_float),
        ("flags", _i32),
        ("reserved", _i32),
        ("shape", PiperShape),
        ("query", PiperTensor),
        ("prepared", PiperSagePrepared),
        ("output", _ptr),
    ]


class LibraryUnavailableError(RuntimeError):
    """The gfx950 HIP library is not built or cannot be opened."""


class NativeLibrary:
    """Typed wrapper over the exported C functions; non-zero status raises RuntimeError."""

    def __init__(self, path: Path) -> None:
        self.path = Path(path)
        self._lib = ctypes.CDLL(str(self.path))
        lib = self._lib
        lib.piper_abi_version.argtypes = []
        lib.piper_abi_version.restype = ctypes.c_int
        lib.piper_last_error.argtypes = []
        lib.piper_last_error.restype = ctypes.c_char_p
        lib.piper_prepared_layout.argtypes = [ctypes.POINTER(PiperShape), ctypes.POINTER(PiperLayout)]
        lib.piper_prepared_layout.restype = ctypes.c_int
        lib.piper_prepare.argtypes = [ctypes.POINTER(PiperPrepareArgs), _ptr]
        lib.piper_prepare.restype = ctypes.c_int
        lib.piper_prepare_static.argtypes = [ctypes.POINTER(PiperPrepareArgs), _ptr]
        lib.piper_prepare_static.restype = ctypes.c_int
        lib.piper_prepare_status.argtypes = [ctypes.POINTER(PiperShape), _ptr, ctypes.POINTER(ctypes.c_uint32), _ptr]
        lib.piper_prepare_status.restype = ctypes.c_int
        lib.piper_attention_forward.argtypes = [ctypes.POINTER(PiperAttentionArgs), _ptr]
        lib.piper_attention_forward.restype = ctypes.c_int
        lib.piper_attention_forward_fused.argtypes = [ctypes.POINTER(PiperAttentionFusedArgs), _ptr]
        lib.piper_attention_forward_fused.restype = ctypes.c_int
        lib.piper_attention_workspace_bytes.argtypes = [ctypes.POINTER(PiperShape), _i32, ctypes.POINTER(_i64)]
        lib.piper_attention_workspace_bytes.restype = ctypes.c_int
        lib.piper_sage_prepared_layout.argtypes = [ctypes.POINTER(PiperShape), ctypes.POINTER(PiperSageLayout)]
        lib.piper_sage_prepared_layout.restype = ctypes.c_int
        lib.piper_sage_prepare.argtypes = [ctypes.POINTER(PiperSagePrepareArgs), _ptr]
        lib.piper_sage_prepare.restype = ctypes.c_int
        lib.piper_sage_attention_forward.argtypes = [ctypes.POINTER(PiperSageAttentionArgs), _ptr]
        lib.piper_sage_attention_forward.restype = ctypes.c_int
        version = lib.piper_abi_version()
        if version != ABI_VERSION:
            raise LibraryUnavailableError(
                f"{self.path} has ABI version {version}, this package expects {ABI_VERSION}"
            )

    def has_symbol(self, name: str) -> bool:
        return hasattr(self._lib, name)

    def last_error(self) -> str:
        return (self._lib.piper_last_error() or b"").decode("utf-8", "replace")

    def _check(self, status: int, what: str) -> None:
        if status != 0:
            raise RuntimeError(f"{what} failed (status {status}): {self.last_error()}")

    def abi_version(self) -> int:
        return int(self._lib.piper_abi_version())

    def prepared_layout(self, shape: PiperShape) -> PiperLayout:
        layout = PiperLayout()
        self._check(self._lib.piper_prepared_layout(ctypes.byref(shape), ctypes.byref(layout)), "piper_prepared_layout")
        return layout

    def prepare(self, args: PiperPrepareArgs, stream: int) -> None:
        self._check(self._lib.piper_prepare(ctypes.byref(args), _ptr(stream)), "piper_prepare")

    def prepare_static(self, args: PiperPrepareArgs, stream: int) -> None:
        """piper_prepare with the library's static per-GPU scratch (no workspace in ``args``)."""
        self._check(self._lib.piper_prepare_static(ctypes.byref(args), _ptr(stream)), "piper_prepare_static")

    def prepare_status(self, shape: PiperShape, workspace: int | None, stream: int) -> int:
        """The give-up count of the last prep on ``workspace`` (None: the static scratch of the
        current device): chunks of the single-pass prep whose bounded wait for their tensor's
        mean ended and that computed it themselves.  Synchronises ``stream``."""
        count = ctypes.c_uint32(0)
        self._check(
            self._lib.piper_prepare_status(ctypes.byref(shape), _ptr(workspace), ctypes.byref(count), _ptr(stream)),
            "piper_prepare_status",
        )
        return int(count.value)

    def attention_workspace_bytes(self, shape: PiperShape, plan: int) -> int:
        """Workspace bytes of the attention entry points for ``plan`` (key-range split plans only)."""
        value = _i64(0)
        self._check(self._lib.piper_attention_workspace_bytes(ctypes.byref(shape), plan, ctypes.byref(value)),
                    "piper_attention_workspace_bytes")
        return int(value.value)

    def attention_forward(self, args: PiperAttentionArgs, stream: int) -> None:
        self._check(self._lib.piper_attention_forward(ctypes.byref(args), _ptr(stream)), "piper_attention_forward")

    def attention_forward_fused(self, args: PiperAttentionFusedArgs, stream: int) -> None:
        self._check(
            self._lib.piper_attention_forward_fused(ctypes.byref(args), _ptr(stream)), "piper_attention_forward_fused"
        )

    def sage_prepared_layout(self, shape: PiperShape) -> PiperSageLayout:
        layout = PiperSageLayout()
        self._check(
            self._lib.piper_sage_prepared_layout(ctypes.byref(shape), ctypes.byref(layout)), "piper_sage_prepared_layout"
        )
        return layout

    def sage_prepare(self, args: PiperSagePrepareArgs, stream: int) -> None:
        self._check(self._lib.piper_sage_prepare(ctypes.byref(args), _ptr(stream)), "piper_sage_prepare")

    def sage_attention_forward(self, args: PiperSageAttentionArgs, stream: int) -> None:
        self._check(
            self._lib.piper_sage_attention_forward(ctypes.byref(args), _ptr(stream)), "piper_sage_attention_forward"
        )



_lock = threading.Lock()
_library: NativeLibrary | None = None


def load_library(path: Path | None = None) -> NativeLibrary:
    """Open the in-tree library (once); raise :class:`LibraryUnavailableError` if absent."""
    global _library
    with _lock:
        if path is None and _library is not None:
            return _library
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise LibraryUnavailableError(
                f"{target} is not built; run __graft_entry__.build() or python -m piper_kernels._hip.build"
            )
        try:
            library = NativeLibrary(target)
        except OSError as error:
            raise LibraryUnavailableError(f"cannot open {target}: {error}") from error
        if path is None:
            _library = library
        return library


def library_available() -> bool:
    try:
        load_library()
    except LibraryUnavailableError:
        return False
    return True


# ---------------------------------------------------------------------------------------
# libpiper_probe.so (include/piper_probe.h)
# ---------------------------------------------------------------------------------------
PROBE_ABI_VERSION = 3
PROBE_EXPORTED_SYMBOLS = ("piper_probe_abi_version", "piper_probe_last_error", "piper_mfma_probe", "piper_issue_probe",
                          "piper_clock_probe")

# piper_mfma_probe kinds, workgroup size and operations per MFMA (PIPER_MFMA_PROBE_*)
MFMA_PROBE_I8 = 0
MFMA_PROBE_F8 = 1
MFMA_PROBE_P_CODES_U8 = 2  # Piper Attention's UINT8 probability-code packer on FP32 values from the sink
MFMA_PROBE_P_CODES_FP8 = 3  # SageAttention2++'s FP8 E4M3 probability-code packer, the same way
MFMA_PROBE_P_CODES_U8_SCALED = 4  # Piper Attention's scaled packer: codes of E * c, 64 groups of 4 per workgroup
MFMA_PROBE_THREADS = 512
MFMA_PROBE_OPS = {MFMA_PROBE_I8: 65536, MFMA_PROBE_F8: 131072}

# piper_issue_probe roles (PIPER_ISSUE_*)
ISSUE_ROLES = ("idle", "mfma", "fma", "exp", "cvt", "mix", "valu_mix", "lds", "mfma_fma", "mix_vgpr", "cluster", "add_lit", "add_sgpr",
               "fma_split", "fma_same", "fmac_same", "max3", "perm")
ISSUE_MAX_WAVES_PER_SIMD = 4
ISSUE_RECORDS_PER_WORKGROUP = 16

# piper_clock_probe (PIPER_CLOCK_PROBE_*)
CLOCK_PROBE_MAX_WORKGROUPS = 256


class PiperIssueRecord(ctypes.Structure):
    _fields_ = [
        ("hw_id", ctypes.c_uint32),
        ("xcc_id", ctypes.c_uint32),
        ("role", ctypes.c_uint32),
        ("slot", ctypes.c_uint32),
        ("cycles", ctypes.c_uint64),
        ("rounds", ctypes.c_uint32),
        ("check", ctypes.c_uint32),
    ]


class PiperIssueProbeArgs(ctypes.Structure):
    _fields_ = [
        ("waves_per_simd", _i32),
        ("workgroups", _i32),
        ("roles", _i32 * ISSUE_MAX_WAVES_PER_SIMD),
        ("cycle_budget", _i64),
        ("records", _ptr),
    ]


class ProbeLibrary:
    """Typed wrapper over libpiper_probe.so; non-zero status raises RuntimeError."""

    def __init__(self, path: Path) -> None:
        self.path = Path(path)
        self._lib = ctypes.CDLL(str(self.path))
        lib = self._lib
        lib.piper_probe_abi_version.argtypes = []
        lib.piper_probe_abi_version.restype = ctypes.c_int
        lib.piper_probe_last_error.argtypes = []
        lib.piper_probe_last_error.restype = ctypes.c_char_p
        lib.piper_mfma_probe.argtypes = [_i32, _i32, _i32, _ptr, _ptr]
        lib.piper_mfma_probe.restype = ctypes.c_int
        lib.piper_issue_probe.argtypes = [ctypes.POINTER(PiperIssueProbeArgs), _ptr]
        lib.piper_issue_probe.restype = ctypes.c_int
        lib.piper_clock_probe.argtypes = [_i32, _i64, _ptr, ctypes.POINTER(_i32), _ptr]
        lib.piper_clock_probe.restype = ctypes.c_int
        version = lib.piper_probe_abi_version()
        if version != PROBE_ABI_VERSION:
            raise LibraryUnavailableError(f"{self.path} has ABI version {version}, this package expects {PROBE_ABI_VERSION}")

    def has_symbol(self, name: str) -> bool:
        return hasattr(self._lib, name)

    def last_error(self) -> str:
        return (self._lib.piper_probe_last_error() or b"").decode("utf-8", "replace")

    def _check(self, status: int, what: str) -> None:
        if status != 0:
            raise RuntimeError(f"{what} failed (status {status}): {self.last_error()}")

    def mfma_probe(self, kind: int, workgroups: int, iterations: int, sink: int, stream: int) -> None:
        self._check(self._lib.piper_mfma_probe(kind, workgroups, iterations, _ptr(sink), _ptr(stream)), "piper_mfma_probe")

    def issue_probe(self, args: PiperIssueProbeArgs, stream: int) -> None:
        self._check(self._lib.piper_issue_probe(ctypes.byref(args), _ptr(stream)), "piper_issue_probe")

    def clock_probe(self, workgroups: int, duration_us: int, records: int, stream: int) -> int:
        """Launch the engine-clock probe; returns the wall clock counter's rate in kHz."""
        khz = _i32(0)
        self._check(self._lib.piper_clock_probe(workgroups, duration_us, _ptr(records), ctypes.byref(khz), _ptr(stream)),
                    "piper_clock_probe")
        return khz.value


_probe_library: ProbeLibrary | None = None


def load_probe_library(path: Path | None = None) -> ProbeLibrary:
    """Open the in-tree measurement library (once); raise :class:`LibraryUnavailableError` if absent."""
    global _probe_library
    with _lock:
        if path is None and _probe_library is not None:
            return _probe_library
        target = Path(path) if path is not None else PROBE_LIBRARY_PATH
        if not target.exists():
            raise LibraryUnavailableError(f"{target} is not built; run __graft_entry__.build()")
        try:
            library = ProbeLibrary(target)
        except OSError as error:
            raise LibraryUnavailableError(f"cannot open {target}: {error}") from error
        if path is None:
            _probe_library = library
        return library

