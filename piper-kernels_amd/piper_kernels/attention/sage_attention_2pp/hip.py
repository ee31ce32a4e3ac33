"""MI355X (gfx950) SageAttention2++ backend: prepare / launch over the C ABI, and the custom op.

Mirrors the reference's Triton backend interface
(``src/piper_kernels/attention/sage_attention_2pp/triton.py``): ``_prepare_sage_attention_2pp``
(``:1000-1063``) computes the K/V statistics and quantises K (INT8) and V (FP8 E4M3) into a
:class:`PreparedSageAttention2pp` bundle; ``_launch_sage_attention_2pp`` (``:1066-1102``) runs
only the fused kernel, which quantises the query itself (the reference's fused query
quantisation, ``_prepare_query`` ``:983-997``); ``piper_kernels::sage_attention_2pp`` is
registered with the same schema and fake (``:1136-1155``).  torch allocates every buffer; the C
side only launches kernels on the current stream.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from ..._hip import library as native
from ..piper_attention._plan import MI355XPlan, select_sage_plan

_DTYPE_CODES = {torch.float16: native.FLOAT16, torch.bfloat16: native.BFLOAT16, torch.float32: native.FLOAT32}


@dataclass(frozen=True)
class PreparedSageAttention2pp:
    """Quantised K/V (layouts documented in ``include/piper_mi355x.h``) and the query itself."""

    key_scale: torch.Tensor  # fp32 [B, H, Sk64/64, 4]: per 64-row block and K thread group
    key_mean: torch.Tensor  # fp32 [B, H, D]
    value_scale: torch.Tensor  # fp32 [B, H, D], per channel
    kv_tiles: torch.Tensor  # uint8 [B, H, Sk64/64, sage_tile_bytes(D)]: K rows, FP8 V^T rows
    query: torch.Tensor  # [B, H, Sq, D] input (the kernel quantises it)
    output: torch.Tensor  # [B, H, Sq, D] in the input dtype
    shape: tuple[int, int, int, int, int]  # B, H, Sq, Sk, D
    scale: float
    is_causal: bool
    plan: MI355XPlan
    qk_granularity: str = "per_thread"  # the reference's Q/K scale granularity (sage/reference.py:80-108)

    def native_prepared(self) -> native.PiperSagePrepared:
        return native.PiperSagePrepared(
            self.key_scale.data_ptr(), self.key_mean.data_ptr(), self.value_scale.data_ptr(), self.kv_tiles.data_ptr()
        )

    # views into the tile records (for inspection and tests)
    def key_code(self) -> torch.Tensor:
        """K codes [B, H, Sk64, D] (the stored rows carry 16 bytes of padding)."""
        b, h, _, _, d = self.shape
        stride = native.kv_k_stride(d)
        rows = self.kv_tiles[..., : 64 * stride].reshape(b, h, -1, 64, stride)
        return rows[..., :d].contiguous().view(torch.int8).reshape(b, h, -1, d)

    def value_code(self) -> torch.Tensor:
        """FP8 E4M3 V codes as bytes [B, H, Sk64, D] (stored transposed per tile)."""
        b, h, _, _, d = self.shape
        off = 64 * native.kv_k_stride(d)
        rows = self.kv_tiles[..., off : off + d * native.KV_V_STRIDE].reshape(b, h, -1, d, native.KV_V_STRIDE)
        return rows[..., :64].transpose(-1, -2).contiguous().reshape(b, h, -1, d)


def _native_input(tensor: torch.Tensor) -> tuple[torch.Tensor, native.PiperTensor]:
    """Keep any [B,H,S,D] view whose rows are 16-byte aligned; copy anything else."""
    strides = tensor.stride()[:3]
    if tensor.data_ptr() % 16 != 0 or any(s % 8 != 0 for s in strides):
        tensor = tensor.contiguous()
        strides = tensor.stride()[:3]
    return tensor, native.PiperTensor(tensor.data_ptr(), *strides)


def _prepare_sage_attention_2pp(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
    *,
    plan: MI355XPlan | None = None,
    workspace: torch.Tensor | None = None,
    qk_granularity: str = "per_thread",
) -> PreparedSageAttention2pp:
    """K/V statistics, INT8 K and FP8 V on the GPU (one HIP prep pipeline); allocate the output.

    ``qk_granularity``: ``"per_thread"`` (the default of the reference's portable path,
    ``sage_attention_2pp/reference.py:35``) or ``"per_warp"`` (its grouped SM12x Triton path).
    """
    if qk_granularity not in ("per_warp", "per_thread"):
        raise ValueError(f"unknown Q/K quantization granularity: {qk_granularity}")
    lib = native.load_library()
    batch, heads, sq, d = query.shape
    sk = key.shape[2]
    if plan is None:
        plan = select_sage_plan(batch, heads, sq, sk, d, is_causal)
    shape = native.PiperShape(batch, heads, sq, sk, d)
    layout = lib.sage_prepared_layout(shape)
    device = query.device
    nkb = -(-sk // native.KEY_BLOCK)

    def empty(shape_, dtype):
        return torch.empty(shape_, device=device, dtype=dtype)

    query, _ = _native_input(query)
    prepared = PreparedSageAttention2pp(
        key_scale=empty((batch, heads, nkb, native.KEY_SCALE_SLOTS), torch.float32),
        key_mean=empty((batch, heads, d), torch.float32),
        value_scale=empty((batch, heads, d), torch.float32),
        kv_tiles=empty((batch, heads, nkb, native.sage_tile_bytes(d)), torch.uint8),
        query=query,
        output=empty((batch, heads, sq, d), query.dtype),
        shape=(batch, heads, sq, sk, d),
        scale=float(scale),
        is_causal=bool(is_causal),
        plan=plan,
        qk_granularity=qk_granularity,
    )
    if workspace is None or workspace.numel() < layout.workspace_bytes:
        workspace = empty((max(layout.workspace_bytes, 1),), torch.uint8)
    key, k_arg = _native_input(key)
    value, v_arg = _native_input(value)
    args = native.PiperSagePrepareArgs(
        abi_version=native.ABI_VERSION,
        dtype=_DTYPE_CODES[key.dtype],
        flags=native.PREPARE_QK_PER_THREAD if qk_granularity == "per_thread" else 0,
        shape=shape,
        key=k_arg,
        value=v_arg,
        prepared=prepared.native_prepared(),
        workspace=workspace.data_ptr(),
        workspace_bytes=workspace.numel(),
    )
    with torch.cuda.device(device):
        lib.sage_prepare(args, torch.cuda.current_stream(device).cuda_stream)
    stream = torch.cuda.current_stream(device)
    for tensor in (key, value, workspace):
        tensor.record_stream(stream)
    return prepared


ACCUMULATE_MODES = ("fp32", "reference")


def _launch_sage_attention_2pp(
    prepared: PreparedSageAttention2pp, *, output: torch.Tensor | None = None, accumulate: str = "fp32"
) -> torch.Tensor:
    """Run only the fused kernel (query quantisation in its prologue); ``output`` may be FP32.

    ``accumulate="fp32"`` accumulates every block's FP8 product in the MFMA's FP32 registers;
    ``accumulate="reference"`` rounds each 64-key block's product to FP16 first, the reference's
    arithmetic (``sage_attention_2pp/reference.py:95-98``)."""
    if accumulate not in ACCUMULATE_MODES:
        raise ValueError(f"accumulate must be one of {ACCUMULATE_MODES}, got {accumulate!r}")
    lib = native.load_library()
    batch, heads, sq, sk, d = prepared.shape
    out = prepared.output if output is None else output
    if out.shape != (batch, heads, sq, d) or not out.is_contiguous() or out.dtype not in _DTYPE_CODES:
        raise ValueError("output must be a contiguous [B, H, Sq, D] float16/bfloat16/float32 tensor")
    query = prepared.query
    args = native.PiperSageAttentionArgs(
        abi_version=native.ABI_VERSION,
        dtype=_DTYPE_CODES[query.dtype],
        output_dtype=_DTYPE_CODES[out.dtype],
        is_causal=int(prepared.is_causal),
        plan=prepared.plan.plan_id,
        scale=ctypes.c_float(prepared.scale).value,
        flags=(native.ATTENTION_QK_PER_THREAD if prepared.qk_granularity == "per_thread" else 0)
        | (native.SAGE_FP16_PARTIALS if accumulate == "reference" else 0),
        reserved=0,
        shape=native.PiperShape(batch, heads, sq, sk, d),
        query=native.PiperTensor(query.data_ptr(), *query.stride()[:3]),
        prepared=prepared.native_prepared(),
        output=out.data_ptr(),
    )
    device = out.device
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        lib.sage_attention_forward(args, stream.cuda_stream)
    query.record_stream(stream)
    return out


def _run_sage_attention_2pp(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
    *,
    plan: MI355XPlan | None = None,
    qk_granularity: str = "per_thread",
    accumulate: str = "fp32",
) -> torch.Tensor:
    prepared = _prepare_sage_attention_2pp(query, key, value, scale, is_causal, plan=plan, qk_granularity=qk_granularity)
    return _launch_sage_attention_2pp(prepared, accumulate=accumulate)


@torch.library.custom_op("piper_kernels::sage_attention_2pp", mutates_args=())
def hip_sage_attention_2pp(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
) -> torch.Tensor:
    """SageAttention2++ K/V prep + fused INT8-QK / FP8-PV kernel on MI355X (schema of triton.py:1136-1145)."""
    return _run_sage_attention_2pp(query, key, value, scale, is_causal)


@hip_sage_attention_2pp.register_fake
def _hip_sage_attention_2pp_fake(
    query: torch.Tensor, _key: torch.Tensor, _value: torch.Tensor, _scale: float, _is_causal: bool
) -> torch.Tensor:
    return torch.empty_like(query, memory_format=torch.contiguous_format)
