"""MI355X (gfx950) backend: prepare / launch over the C ABI, and the torch custom op.

Mirrors the reference's Triton backend interface
(``src/piper_kernels/attention/piper_attention/triton.py``): ``_prepare_piper_attention``
(``:772-890``) quantises Q/K/V into a :class:`PreparedPiperAttention` bundle
(``:754-769``), ``_launch_piper_attention`` (``:893-951``) runs only the fused kernel, and
``piper_kernels::piper_attention`` is registered with the same schema and fake
(``:984-1010``).  torch allocates every buffer; the C side only launches kernels on the
current stream and never synchronises.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, replace

import torch

from ..._hip import library as native
from ._plan import MI355XPlan, select_plan

_DTYPE_CODES = {torch.float16: native.FLOAT16, torch.bfloat16: native.BFLOAT16, torch.float32: native.FLOAT32}
ACC_BIAS = 0x4B400000  # integer accumulator bias: bits read as FP32 1.5 * 2^23 + value


@dataclass(frozen=True)
class PreparedPiperAttention:
    """Quantised operands (layouts documented in ``include/piper_mi355x.h``)."""

    query_code: torch.Tensor | None  # int8 [B, H, Sq32, D]; None when the kernel quantises Q
    # fp32 [B, H, Sq32/32, 8]: per 32-row block, the scale of each thread group t (rows t, t+8,
    # t+16, t+24); per_warp repeats the block scale.  None when the kernel quantises Q
    query_scale: torch.Tensor | None
    key_scale: torch.Tensor  # fp32 [B, H, Sk64/64, 4]: per 64-row block and thread group
    value_scale: torch.Tensor  # fp32 [B, H, Sk64]
    key_mean: torch.Tensor  # fp32 [B, H, D]
    value_mean: torch.Tensor  # fp32 [B, H, D]
    kv_tiles: torch.Tensor  # uint8 [B, H, Sk64/64, kv_tile_bytes(D)]: K, V^T, log2 scale, 1/(255 s), 128 colsum
    output: torch.Tensor  # [B, H, Sq, D] in the input dtype
    shape: tuple[int, int, int, int, int]  # B, H, Sq, Sk, D
    scale: float
    is_causal: bool
    plan: MI355XPlan
    query: torch.Tensor | None = None  # [B, H, Sq, D] input, kept for the fused launch
    qk_granularity: str = "per_thread"  # the reference's Q/K scale granularity (sage/reference.py:80-108)

    @property
    def fused_query(self) -> bool:
        """True when the attention kernel quantises the query itself (no query codes here)."""
        return self.query_code is None

    def native_prepared(self) -> native.PiperPrepared:
        return native.PiperPrepared(
            None if self.query_code is None else self.query_code.data_ptr(),
            None if self.query_scale is None else self.query_scale.data_ptr(),
            self.key_scale.data_ptr(),
            self.value_scale.data_ptr(),
            self.key_mean.data_ptr(),
            self.value_mean.data_ptr(),
            self.kv_tiles.data_ptr(),
        )

    # views into the tile records (for inspection and tests)
    def _region(self, name: str, length: int) -> torch.Tensor:
        off = native.kv_offsets(self.shape[4])[name]
        return self.kv_tiles[..., off : off + length]

    def key_code(self) -> torch.Tensor:
        """K codes [B, H, Sk64, D] (the stored rows carry 16 bytes of padding)."""
        b, h, _, _, d = self.shape
        rows = self._region("key", 64 * native.kv_k_stride(d)).reshape(b, h, -1, 64, native.kv_k_stride(d))
        return rows[..., :d].contiguous().view(torch.int8).reshape(b, h, -1, d)

    def key_tile_scale(self) -> torch.Tensor:
        """Copy of each tile's four K scale slots kept in the padding of its first K row:
        [B, H, nkb, 4]."""
        return self._region("key_scale", 4 * native.KEY_SCALE_SLOTS).contiguous().view(torch.float32)

    def value_code_transposed(self) -> torch.Tensor:
        """V codes as stored: [B, H, Sk64/64, D, 64]."""
        b, h, _, _, d = self.shape
        rows = self._region("value", d * native.KV_V_STRIDE).reshape(b, h, -1, d, native.KV_V_STRIDE)
        return rows[..., :64].contiguous().view(torch.int8)

    def value_log2_scale(self) -> torch.Tensor:
        return self._region("log2", 256).contiguous().view(torch.float32).flatten(2)

    def value_inv_multiplier(self) -> torch.Tensor:
        return self._region("inv", 256).contiguous().view(torch.float32).flatten(2)

    def value_correction(self) -> torch.Tensor:
        """128 * column sums of the V codes per tile (the stored words carry a 0x4B400000 bias)."""
        return self._region("corr", 4 * self.shape[4]).contiguous().view(torch.int32) - ACC_BIAS


def _native_input(tensor: torch.Tensor) -> tuple[torch.Tensor, native.PiperTensor]:
    """Keep any [B,H,S,D] view whose rows are 16-byte aligned; copy anything else."""
    strides = tensor.stride()[:3]
    if tensor.data_ptr() % 16 != 0 or any(s % 8 != 0 for s in strides):
        tensor = tensor.contiguous()
        strides = tensor.stride()[:3]
    return tensor, native.PiperTensor(tensor.data_ptr(), *strides)


def _native_shape(batch: int, heads: int, sq: int, sk: int, d: int) -> native.PiperShape:
    return native.PiperShape(batch, heads, sq, sk, d)


def _prepare_piper_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
    *,
    plan: MI355XPlan | None = None,
    workspace: torch.Tensor | None = None,
    quantize_query: bool = True,
    qk_granularity: str = "per_thread",
    static_workspace: bool = False,
    prep_flags: int = 0,
) -> PreparedPiperAttention:
    """Quantise Q/K/V on the GPU (one HIP prep pipeline) and allocate the output.

    With ``quantize_query=False`` only K and V are quantised and the bundle keeps the query
    itself: ``_launch_piper_attention`` then runs the fused entry point, whose kernel
    quantises each query block in its prologue (bit-identical codes and scales).
    ``qk_granularity`` is the reference's ``quantize_query_key`` granularity
    (``sage/reference.py:80-108``): ``"per_thread"`` (the default, as in its portable path --
    ``reference.py:42`` -- which is what the reference runs on MI355X: 8 scales per Q block, 4
    per K block, over interleaved rows) or ``"per_warp"`` (one scale per 32-row Q / 64-row K
    block, its grouped SM12x Triton path).  ``static_workspace=True`` runs ``piper_prepare_static``
    instead: no workspace is allocated, the library's static per-GPU scratch holds the mean
    partials (same outputs; calls overlapping on one GPU race).  ``prep_flags`` adds diagnostic
    ``PIPER_PREPARE_*`` bits (``native.PREPARE_SELF_MEAN``: every waiting single-pass chunk
    computes its tensor's mean itself, the bounded wait's fallback; same outputs).
    """
    if qk_granularity not in ("per_warp", "per_thread"):
        raise ValueError(f"unknown Q/K quantization granularity: {qk_granularity}")
    per_thread = qk_granularity == "per_thread"
    lib = native.load_library()
    batch, heads, sq, d = query.shape
    sk = key.shape[2]
    if plan is None:
        plan = select_plan(batch, heads, sq, sk, d, is_causal)
    shape = _native_shape(batch, heads, sq, sk, d)
    layout = lib.prepared_layout(shape)
    device = query.device
    sq32 = -(-sq // native.QUERY_BLOCK) * native.QUERY_BLOCK
    sk64 = -(-sk // native.KEY_BLOCK) * native.KEY_BLOCK
    nkb = sk64 // native.KEY_BLOCK

    def empty(shape_, dtype):
        return torch.empty(shape_, device=device, dtype=dtype)

    prepared = PreparedPiperAttention(
        query_code=empty((batch, heads, sq32, d), torch.int8) if quantize_query else None,
        query_scale=(
            empty((batch, heads, sq32 // native.QUERY_BLOCK, native.QUERY_SCALE_SLOTS), torch.float32)
            if quantize_query
            else None
        ),
        key_scale=empty((batch, heads, nkb, native.KEY_SCALE_SLOTS), torch.float32),
        value_scale=empty((batch, heads, sk64), torch.float32),
        key_mean=empty((batch, heads, d), torch.float32),
        value_mean=empty((batch, heads, d), torch.float32),
        kv_tiles=empty((batch, heads, nkb, native.kv_tile_bytes(d)), torch.uint8),
        output=empty((batch, heads, sq, d), query.dtype),
        shape=(batch, heads, sq, sk, d),
        scale=float(scale),
        is_causal=bool(is_causal),
        plan=plan,
        qk_granularity=qk_granularity,
    )
    query, q_arg = _native_input(query)
    if not quantize_query:
        prepared = replace(prepared, query=query)
    if static_workspace:
        workspace = None
    elif workspace is None or workspace.numel() < layout.workspace_bytes:
        workspace = empty((max(layout.workspace_bytes, 1),), torch.uint8)
    key, k_arg = _native_input(key)
    value, v_arg = _native_input(value)
    args = native.PiperPrepareArgs(
        abi_version=native.ABI_VERSION,
        dtype=_DTYPE_CODES[query.dtype],
        is_causal=int(bool(is_causal)),
        flags=(0 if quantize_query else native.PREPARE_SKIP_QUERY)
        | (native.PREPARE_QK_PER_THREAD if per_thread else 0)
        | (prep_flags & native.PREPARE_SELF_MEAN),
        shape=shape,
        query=q_arg,
        key=k_arg,
        value=v_arg,
        prepared=prepared.native_prepared(),
        workspace=None if workspace is None else workspace.data_ptr(),
        workspace_bytes=0 if workspace is None else workspace.numel(),
    )
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        if static_workspace:
            lib.prepare_static(args, stream.cuda_stream)
        else:
            lib.prepare(args, stream.cuda_stream)
    # the caching allocator must not recycle inputs or workspace before the stream reaches them
    for tensor in (query, key, value, workspace):
        if tensor is not None:
            tensor.record_stream(stream)
    return prepared


def _launch_piper_attention(
    prepared: PreparedPiperAttention, *, output: torch.Tensor | None = None
) -> torch.Tensor:
    """Run only the fused kernel on prepared operands; ``output`` may be FP32 for tests.

    A bundle prepared with ``quantize_query=False`` goes through
    ``piper_attention_forward_fused`` (query quantisation in the kernel prologue).
    """
    lib = native.load_library()
    batch, heads, sq, sk, d = prepared.shape
    out = prepared.output if output is None else output
    if out.shape != (batch, heads, sq, d) or not out.is_contiguous() or out.dtype not in _DTYPE_CODES:
        raise ValueError("output must be a contiguous [B, H, Sq, D] float16/bfloat16/float32 tensor")
    device = out.device
    flags = native.ATTENTION_QK_PER_THREAD if prepared.qk_granularity == "per_thread" else 0
    # key-range split plans: FP32 partial sums of each key part, merged by the library's kernel;
    # the work-queue plan: its counters
    workspace = None
    if prepared.plan.key_parts > 1 or prepared.plan.work_queue:
        size = lib.attention_workspace_bytes(_native_shape(batch, heads, sq, sk, d), prepared.plan.plan_id)
        workspace = torch.empty(size, dtype=torch.uint8, device=device)
    ws_ptr, ws_bytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel())
    if prepared.fused_query:
        query = prepared.query
        fused = native.PiperAttentionFusedArgs(
            abi_version=native.ABI_VERSION,
            dtype=_DTYPE_CODES[query.dtype],
            output_dtype=_DTYPE_CODES[out.dtype],
            is_causal=int(prepared.is_causal),
            plan=prepared.plan.plan_id,
            scale=ctypes.c_float(prepared.scale).value,
            flags=flags,
            reserved=0,
            shape=_native_shape(batch, heads, sq, sk, d),
            query=native.PiperTensor(query.data_ptr(), *query.stride()[:3]),
            prepared=prepared.native_prepared(),
            output=out.data_ptr(),
            workspace=ws_ptr,
            workspace_bytes=ws_bytes,
        )
        with torch.cuda.device(device):
            stream = torch.cuda.current_stream(device)
            lib.attention_forward_fused(fused, stream.cuda_stream)
        query.record_stream(stream)
        if workspace is not None:
            workspace.record_stream(stream)
        return out
    args = native.PiperAttentionArgs(
        abi_version=native.ABI_VERSION,
        output_dtype=_DTYPE_CODES[out.dtype],
        is_causal=int(prepared.is_causal),
        plan=prepared.plan.plan_id,
        shape=_native_shape(batch, heads, sq, sk, d),
        scale=ctypes.c_float(prepared.scale).value,
        flags=flags,
        prepared=prepared.native_prepared(),
        output=out.data_ptr(),
        workspace=ws_ptr,
        workspace_bytes=ws_bytes,
    )
    with torch.cuda.device(device):
        stream = torch.cuda.current_stream(device)
        lib.attention_forward(args, stream.cuda_stream)
    if workspace is not None:
        workspace.record_stream(stream)
    return out


def _run_piper_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
    *,
    plan: MI355XPlan | None = None,
    fuse_query: bool = True,
    qk_granularity: str = "per_thread",
) -> torch.Tensor:
    """The operator: prep of K and V, then the attention kernel, which quantises the query in
    its prologue (``fuse_query=False``: the prep quantises Q too; the output is the same).
    Q/K scales per thread group by default, the granularity of the reference's portable path."""
    prepared = _prepare_piper_attention(
        query, key, value, scale, is_causal, plan=plan, quantize_query=not fuse_query, qk_granularity=qk_granularity
    )
    return _launch_piper_attention(prepared)


@torch.library.custom_op("piper_kernels::piper_attention", mutates_args=())
def hip_piper_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    scale: float,
    is_causal: bool,
) -> torch.Tensor:
    """Piper Attention K/V prep + fused INT8 kernel (query quantised in its prologue) on MI355X
    (schema of triton.py:984-999)."""
    return _run_piper_attention(query, key, value, scale, is_causal)


@hip_piper_attention.register_fake
def _hip_piper_attention_fake(
    query: torch.Tensor, _key: torch.Tensor, _value: torch.Tensor, _scale: float, _is_causal: bool
) -> torch.Tensor:
    return torch.empty_like(query, memory_format=torch.contiguous_format)
