"""Paged-attention decode on the HIP backend, for torch device tensors.

This is the direct form of the path that simpler submits through its
orchestration function (``examples/a2a3/tensormap_and_ringbuffer/
paged_attention/kernels/orchestration/paged_attention_orch.cpp:77-291``): the
same seven arguments — query, key_cache, value_cache, block_table,
context_lens, out, scale — in the same layouts (``goldens/paged_attention.py
:76-84``), computed by the fused gfx950 decode kernel (plus a small merge kernel) in
``libsimpler_hip.so``.

torch supplies device memory and the current stream only; the arithmetic is
all in the native library, and there is no fallback when it is missing.
"""

from __future__ import annotations

import ctypes
import math
import threading

import torch

from . import _lib
from .task_interface import ArgDirection, ChipCallable, CoreCallable, DataType

NATIVE_CALLABLE_NAME = "simpler_hip_paged_attention_decode"

_OUT_DTYPES = {torch.float32: int(DataType.FLOAT32), torch.bfloat16: int(DataType.BFLOAT16),
               torch.float16: int(DataType.FLOAT16)}
# element formats of query and caches (include/simpler_hip/pa_decode.h SIMPLER_HIP_KV_*):
# bf16, fp8 E4M3FN caches with a bf16 query, fp16
KV_BF16, KV_FP8_E4M3, KV_FP16 = 0, 1, 2
_FP8_DTYPES = (torch.float8_e4m3fn, torch.uint8)
_ERRORS = {
    -1: "invalid argument (shape, dtype, stride or alignment)",
    -2: "unsupported configuration",
    -4: "workspace missing or too small",
    -5: "HIP launch failure",
    -6: "block_table entry outside the KV pool",
    -7: "context_lens entry outside [0, max_blocks_per_seq * block_size] (or, causal, shorter than q_len)",
}


class PagedAttentionError(RuntimeError):
    def __init__(self, rc: int, what: str = "simpler_hip_pa_decode"):
        super().__init__(f"{what} failed with {rc}: {_ERRORS.get(rc, 'error')}")
        self.rc = rc


class _Workspace:
    """Workspace (error word + per-worker partial slots) per (device, stream).

    Launches on one stream run in order, so they may share a buffer; launches
    on different streams get different buffers, so concurrent decodes never
    share partial slots. A buffer only grows (to at least twice its old size),
    and a buffer it replaces is kept alive rather than freed: a HIP graph
    captured earlier holds its address and keeps using it on replay. The
    initialisation is a kernel, not a memset, so a buffer may also be created
    inside a graph capture (the capture then records its zeroing, which runs
    again on every replay). Graphs captured on one stream share that stream's
    buffer: do not replay them concurrently on different streams.
    """

    def __init__(self) -> None:
        self._mu = threading.Lock()
        self._buf: dict[tuple[int, int], torch.Tensor] = {}
        self._retired: list[torch.Tensor] = []

    def get(self, device: torch.device, nbytes: int, stream: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        key = (idx, int(stream or 0))
        with self._mu:
            buf = self._buf.get(key)
            if buf is None or buf.numel() < nbytes:
                size = max(nbytes, 1 << 20, 2 * buf.numel() if buf is not None else 0)
                with torch.cuda.device(idx):
                    raw = torch.empty(size + 256, dtype=torch.uint8, device=torch.device("cuda", idx))
                off = (-raw.data_ptr()) % 256
                new = raw[off : off + size]
                rc = _lib.lib().simpler_hip_pa_decode_workspace_init(new.data_ptr(), new.numel(), stream)
                if rc != 0:
                    raise PagedAttentionError(rc, "simpler_hip_pa_decode_workspace_init")
                if buf is not None:
                    self._retired.append(buf)  # a captured graph may still use it
                self._buf[key] = new
                buf = new
            return buf


_WORKSPACE = _Workspace()


def _check(t: torch.Tensor, name: str, dtype: torch.dtype, ndims: tuple[int, ...]) -> None:
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a device (cuda/HIP) tensor, got {t.device}")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.dim() not in ndims:
        raise ValueError(f"{name} must have {ndims} dims, got shape {tuple(t.shape)}")


def make_args(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    out: torch.Tensor,
    scale: float,
    *,
    causal: bool = False,
    num_workers: int = 0,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> _lib.PaDecodeArgs:
    """Validate torch tensors and fill the C ``SimplerHipPaDecodeArgs``.

    fp8 caches: ``key_cache``/``value_cache`` of dtype ``torch.float8_e4m3fn``
    (or uint8 holding E4M3FN bytes) with ``k_scale``/``v_scale`` fp32
    ``[num_blocks, num_kv_heads]``: element (blk, t, h, d) stands for
    ``float(cache[blk, t, h, d]) * scale[blk, h]``.
    """
    fp8 = key_cache.dtype in _FP8_DTYPES
    fp16 = query.dtype == torch.float16
    kv_dtype = key_cache.dtype if fp8 else (torch.float16 if fp16 else torch.bfloat16)
    if fp8 and fp16:
        raise ValueError("fp8 caches take a bfloat16 query")
    _check(query, "query", torch.float16 if fp16 else torch.bfloat16, (3, 4))
    _check(key_cache, "key_cache", kv_dtype, (4,))
    _check(value_cache, "value_cache", kv_dtype, (4,))
    if fp8:
        if k_scale is None or v_scale is None:
            raise ValueError("fp8 caches need k_scale and v_scale ([num_blocks, num_kv_heads] float32)")
        for name, t in (("k_scale", k_scale), ("v_scale", v_scale)):
            _check(t, name, torch.float32, (2,))
            if not t.is_contiguous() or tuple(t.shape) != (key_cache.shape[0], key_cache.shape[2]):
                raise ValueError(f"{name} must be a contiguous [num_blocks, num_kv_heads] tensor")
    elif k_scale is not None or v_scale is not None:
        raise ValueError("k_scale/v_scale apply to fp8 caches only")
    _check(block_table, "block_table", torch.int32, (2,))
    _check(context_lens, "context_lens", torch.int32, (1,))
    allowed = (torch.float32, torch.float16) if fp16 else (torch.float32, torch.bfloat16)
    if out.dtype not in allowed:
        raise ValueError(f"out must be one of {allowed} for {query.dtype} inputs, got {out.dtype}")
    for name, t in (("query", query), ("block_table", block_table), ("context_lens", context_lens), ("out", out)):
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if key_cache.stride(-1) != 1 or value_cache.stride(-1) != 1:
        raise ValueError("key_cache/value_cache need unit stride in the head dim")
    q4 = query.dim() == 4
    batch = query.shape[0]
    q_len = query.shape[1] if q4 else 1
    hq, dk = query.shape[-2], query.shape[-1]
    nblk, bs, hkv, kd = key_cache.shape
    vnb, vbs, vhkv, dv = value_cache.shape
    if (vnb, vbs, vhkv) != (nblk, bs, hkv) or kd != dk:
        raise ValueError("key_cache/value_cache/query shapes disagree")
    expect_out = (batch, q_len, hq, dv) if q4 else (batch, hq, dv)
    if tuple(out.shape) != expect_out:
        raise ValueError(f"out must have shape {expect_out}, got {tuple(out.shape)}")
    if tuple(block_table.shape[:1]) != (batch,) or tuple(context_lens.shape) != (batch,):
        raise ValueError("block_table/context_lens batch does not match the query")
    a = _lib.PaDecodeArgs()
    a.query = query.data_ptr()
    a.key_cache = key_cache.data_ptr()
    a.value_cache = value_cache.data_ptr()
    a.block_table = block_table.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.out = out.data_ptr()
    a.k_block_stride, a.k_token_stride, a.k_head_stride = key_cache.stride()[:3]
    a.v_block_stride, a.v_token_stride, a.v_head_stride = value_cache.stride()[:3]
    a.batch, a.q_len, a.num_heads, a.num_kv_heads = batch, q_len, hq, hkv
    a.head_dim_k, a.head_dim_v, a.block_size = dk, dv, bs
    a.max_blocks_per_seq, a.num_blocks = block_table.shape[1], nblk
    a.out_dtype = _OUT_DTYPES[out.dtype]
    a.scale = float(scale)
    a.causal = 1 if causal else 0
    a.num_workers = int(num_workers)
    if fp8:
        a.kv_format = KV_FP8_E4M3
        a.k_scale, a.v_scale = k_scale.data_ptr(), v_scale.data_ptr()
    elif fp16:
        a.kv_format = KV_FP16
    return a


PHASE_MAIN, PHASE_MERGE = 1, 2


def launch(args: _lib.PaDecodeArgs, device: torch.device, stream: int | None = None,
           phases: int = PHASE_MAIN | PHASE_MERGE, key_new: torch.Tensor | None = None,
           value_new: torch.Tensor | None = None, prelude: _lib.DecodePreludeArgs | None = None) -> None:
    """Enqueue one decode on ``stream`` (default: torch's current stream).

    ``phases`` selects the main kernel, the merge kernel or both (the default);
    a merge must follow a main launch with the same args. With ``key_new``
    (checked by ``append_tensors``) the decode runs with the fused KV append
    (``simpler_hip_pa_decode_append``, both phases); with ``prelude`` (from
    ``prelude_args``) after the prelude and append
    (``simpler_hip_pa_decode_prelude``, both phases).
    """
    lib = _lib.lib()
    if stream is None:
        stream = torch.cuda.current_stream(device).cuda_stream
    size_of = (lib.simpler_hip_pa_decode_prelude_workspace_size if prelude is not None
               else lib.simpler_hip_pa_decode_workspace_size)
    need = size_of(ctypes.byref(args))
    if need == 0:
        raise PagedAttentionError(-1)
    ws = _WORKSPACE.get(device, need, stream)
    if prelude is not None:
        if phases != PHASE_MAIN | PHASE_MERGE:
            raise ValueError("the prelude entry runs both phases")
        rc = lib.simpler_hip_pa_decode_prelude(ctypes.byref(args), ctypes.byref(prelude), ws.data_ptr(), ws.numel(),
                                               stream)
        if rc != 0:
            raise PagedAttentionError(rc, "simpler_hip_pa_decode_prelude")
        return
    if key_new is not None:
        if phases != PHASE_MAIN | PHASE_MERGE:
            raise ValueError("the fused append runs both phases")
        rc = lib.simpler_hip_pa_decode_append(ctypes.byref(args), key_new.data_ptr(),
                                              value_new.data_ptr() if value_new is not None else None,
                                              ws.data_ptr(), ws.numel(), stream)
        if rc != 0:
            raise PagedAttentionError(rc, "simpler_hip_pa_decode_append")
        return
    if phases == PHASE_MAIN | PHASE_MERGE:
        rc = lib.simpler_hip_pa_decode(ctypes.byref(args), ws.data_ptr(), ws.numel(), stream)
    else:
        rc = lib.simpler_hip_pa_decode_phase(ctypes.byref(args), ws.data_ptr(), ws.numel(), stream, phases)
    if rc != 0:
        raise PagedAttentionError(rc)


def append_tensors(args: _lib.PaDecodeArgs, query: torch.Tensor, key_cache: torch.Tensor,
                   value_cache: torch.Tensor, key_new: torch.Tensor, value_new: torch.Tensor | None) -> None:
    """Check the new tokens of a fused append against decode ``args``:
    ``key_new`` ``[B, q_len, Hkv, Dk]`` (or ``[B, Hkv, Dk]`` for q_len 1) and
    ``value_new`` ``[..., Dv]`` contiguous, of the caches' dtype; ``value_new`` is
    ``None`` exactly when ``value_cache`` is a view of ``key_cache`` (MLA)."""
    kv_dtype = key_cache.dtype
    q_len = args.q_len
    mla = value_cache.data_ptr() == key_cache.data_ptr()
    for name, t, d in (("key_new", key_new, args.head_dim_k), ("value_new", value_new, args.head_dim_v)):
        if t is None:
            if name == "value_new" and mla:
                continue
            raise ValueError(f"{name} is required")
        if name == "value_new" and mla:
            raise ValueError("value_new must be None when value_cache is a view of key_cache (MLA)")
        _check(t, name, kv_dtype, (3, 4))
        shape = (args.batch, q_len, args.num_kv_heads, d) if t.dim() == 4 else (args.batch, args.num_kv_heads, d)
        if t.dim() == 3 and q_len != 1:
            raise ValueError(f"{name} must be [batch, q_len, kv_heads, dim] for q_len > 1")
        if tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous {shape} tensor, got {tuple(t.shape)}")


def paged_attention_decode(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    out: torch.Tensor | None = None,
    scale: float | None = None,
    *,
    causal: bool = False,
    out_dtype: torch.dtype = torch.float32,
    num_workers: int = 0,
    k_scale: torch.Tensor | None = None,
    v_scale: torch.Tensor | None = None,
) -> torch.Tensor:
    """Fused paged-attention decode; returns ``out`` ``[B, (q_len,) Hq, Dv]``.

    ``scale`` defaults to ``1/sqrt(head_dim_k)``. The reference's orchestration
    writes FLOAT32 output (``paged_attention_orch.cpp:130``); BFLOAT16 (bf16
    inputs) or FLOAT16 (fp16 inputs) is also accepted. Query and caches are
    bfloat16, or float16 (the reference's GQA cases). ``value_cache`` may be a
    view of ``key_cache`` (MLA: V = K[..., :Dv], bf16).
    """
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    if out is None:
        shape = (*query.shape[:-1], value_cache.shape[-1])
        out = torch.empty(shape, dtype=out_dtype, device=query.device)
    args = make_args(
        query, key_cache, value_cache, block_table, context_lens, out, scale,
        causal=causal, num_workers=num_workers, k_scale=k_scale, v_scale=v_scale,
    )
    launch(args, query.device)
    return out


def paged_attention_decode_append(
    query: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    key_new: torch.Tensor,
    value_new: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    scale: float | None = None,
    *,
    causal: bool = False,
    out_dtype: torch.dtype = torch.float32,
    num_workers: int = 0,
) -> torch.Tensor:
    """KV-cache append fused into the decode (``simpler_hip_pa_decode_append``).

    The ``q_len`` new tokens of sequence ``b`` are its last positions
    ``context_lens[b] - q_len .. context_lens[b] - 1`` (the lengths count them):
    their K/V (``key_new``/``value_new``, ``[B, q_len, Hkv, D]``) are written to
    the caches at ``block_table[b, p // block_size]``, row ``p % block_size``, and
    the decode attends over them, as ``kv_append`` with that slot mapping
    followed by ``paged_attention_decode`` would. ``value_new`` is ``None`` for
    MLA (V is a prefix of the K row). bf16 or fp16; q_len <= 16.
    """
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    if out is None:
        shape = (*query.shape[:-1], value_cache.shape[-1])
        out = torch.empty(shape, dtype=out_dtype, device=query.device)
    args = make_args(query, key_cache, value_cache, block_table, context_lens, out, scale, causal=causal,
                     num_workers=num_workers)
    append_tensors(args, query, key_cache, value_cache, key_new, value_new)
    launch(args, query.device, key_new=key_new, value_new=value_new)
    return out


def paged_attention_decode_prelude(
    q_proj: torch.Tensor,
    k_proj: torch.Tensor,
    v_proj: torch.Tensor,
    inv_rms: torch.Tensor,
    q_norm_weight: torch.Tensor,
    k_norm_weight: torch.Tensor,
    rope_cos: torch.Tensor,
    rope_sin: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    context_lens: torch.Tensor,
    out: torch.Tensor | None = None,
    scale: float | None = None,
    *,
    eps: float = 1e-6,
    causal: bool = False,
    out_dtype: torch.dtype = torch.float32,
    num_workers: int = 0,
) -> torch.Tensor:
    """Decode prelude, KV append and decode in one call
    (``simpler_hip_pa_decode_prelude``: the prelude's launch, then the decode's two).

    From the fp32 projections ``q_proj`` ``[B, (q_len,) Hq, 128]`` and ``k_proj``
    / ``v_proj`` ``[B, (q_len,) Hkv, 128]``: q and k are RoPE(RMSnorm(proj *
    inv_rms) * weight) at the new tokens' positions ``context_lens[b] - q_len + i``
    (``rope_cos``/``rope_sin`` ``[max_position, 128]``, half-split), v = v_proj *
    inv_rms (``inv_rms`` ``[B]`` or ``[B, q_len]``), all rounded to bf16, as
    ``kv_cache.qk_norm_rope_append`` computes them; the new K/V go into the bf16
    caches and the decode attends over them (see ``paged_attention_decode_append``).
    """
    q4 = q_proj.dim() == 4
    batch, hq, d = q_proj.shape[0], q_proj.shape[-2], q_proj.shape[-1]
    q_len = q_proj.shape[1] if q4 else 1
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if out is None:
        shape = (batch, q_len, hq, value_cache.shape[-1]) if q4 else (batch, hq, value_cache.shape[-1])
        out = torch.empty(shape, dtype=out_dtype, device=q_proj.device)
    args, pre = prelude_args(q_proj, k_proj, v_proj, inv_rms, q_norm_weight, k_norm_weight, rope_cos, rope_sin,
                             key_cache, value_cache, block_table, context_lens, out, scale, eps=eps, causal=causal,
                             num_workers=num_workers)
    launch(args, q_proj.device, prelude=pre)
    return out


def prelude_args(q_proj: torch.Tensor, k_proj: torch.Tensor, v_proj: torch.Tensor, inv_rms: torch.Tensor,
                 q_norm_weight: torch.Tensor, k_norm_weight: torch.Tensor, rope_cos: torch.Tensor,
                 rope_sin: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                 block_table: torch.Tensor, context_lens: torch.Tensor, out: torch.Tensor, scale: float, *,
                 eps: float = 1e-6, causal: bool = False,
                 num_workers: int = 0) -> tuple[_lib.PaDecodeArgs, _lib.DecodePreludeArgs]:
    """The C decode args and prelude args of ``paged_attention_decode_prelude``,
    for repeated ``launch(args, device, prelude=pre)``; checks the tensors."""
    q4 = q_proj.dim() == 4
    q_len = q_proj.shape[1] if q4 else 1
    batch, hq, d = q_proj.shape[0], q_proj.shape[-2], q_proj.shape[-1]
    hkv = key_cache.shape[2]
    kv_shape = (batch, q_len, hkv, d) if q4 else (batch, hkv, d)
    for name, t, shape in (("q_proj", q_proj, tuple(q_proj.shape)), ("k_proj", k_proj, kv_shape),
                           ("v_proj", v_proj, kv_shape)):
        _check(t, name, torch.float32, (3, 4))
        if tuple(t.shape) != shape or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 {shape} tensor, got {tuple(t.shape)}")
    if inv_rms.numel() != batch * q_len or inv_rms.dtype != torch.float32 or not inv_rms.is_contiguous():
        raise ValueError("inv_rms must be a contiguous float32 [batch] or [batch, q_len] tensor")
    for name, t in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        _check(t, name, torch.float32, (1,))
        if tuple(t.shape) != (d,) or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous float32 [{d}] tensor")
    for name, t in (("rope_cos", rope_cos), ("rope_sin", rope_sin)):
        _check(t, name, torch.float32, (2,))
        if t.shape[1] != d or not t.is_contiguous() or t.shape != rope_cos.shape:
            raise ValueError(f"{name} must be a contiguous float32 [max_position, {d}] tensor")
    # the decode args take their query shape from q_proj (the query itself is
    # computed by the prelude; this bf16 view over q_proj's storage is not read)
    query_shape = torch.empty(0, dtype=torch.bfloat16, device=q_proj.device).set_(
        q_proj.untyped_storage(), q_proj.storage_offset() * 2, tuple(q_proj.shape),
        tuple(torch.empty(q_proj.shape, device="meta").stride()))
    args = make_args(query_shape, key_cache, value_cache, block_table, context_lens, out, scale, causal=causal,
                     num_workers=num_workers)
    pre = _lib.DecodePreludeArgs()
    pre.q_proj, pre.k_proj, pre.v_proj = q_proj.data_ptr(), k_proj.data_ptr(), v_proj.data_ptr()
    pre.inv_rms = inv_rms.data_ptr()
    pre.q_norm_weight, pre.k_norm_weight = q_norm_weight.data_ptr(), k_norm_weight.data_ptr()
    pre.rope_cos, pre.rope_sin = rope_cos.data_ptr(), rope_sin.data_ptr()
    pre.max_position = rope_cos.shape[0]
    pre.eps = float(eps)
    return args, pre


def check_errors(device: torch.device | None = None) -> None:
    """Synchronise and raise if a launch on the current stream met an out-of-pool
    block_table entry (rc -6) or a context length it had to clamp (rc -7)."""
    device = device or torch.device("cuda", torch.cuda.current_device())
    stream = torch.cuda.current_stream(device).cuda_stream
    ws = _WORKSPACE.get(device, 1, stream)
    rc = _lib.lib().simpler_hip_pa_decode_check(ws.data_ptr(), ws.numel(), stream)
    if rc != 0:
        raise PagedAttentionError(rc, "paged attention")


def plan(args: _lib.PaDecodeArgs) -> int:
    """Number of workers (work-list slices) a launch with ``args`` uses on the current device.

    A worker is one workgroup for the decode kernel and one slice run by
    ceil(rows / 128) sibling workgroups for the MLA kernel.
    """
    n = ctypes.c_int32()
    rc = _lib.lib().simpler_hip_pa_decode_plan(ctypes.byref(args), ctypes.byref(n))
    if rc != 0:
        raise PagedAttentionError(rc, "simpler_hip_pa_decode_plan")
    return n.value


def kernel_name(args: _lib.PaDecodeArgs) -> str:
    """Name of the main kernel a launch with ``args`` runs ("" if unsupported)."""
    return _lib.lib().simpler_hip_pa_decode_kernel_name(ctypes.byref(args)).decode()


# ---------------------------------------------------------------------------
# Callables accepted by libsimpler_hip.so's simpler_register_callable
# ---------------------------------------------------------------------------

D = ArgDirection
ORCH_SIGNATURE = [D.IN, D.IN, D.IN, D.IN, D.IN, D.OUT]
INCORE_SIGNATURES = {
    0: [D.IN, D.IN, D.OUT],  # QK   aic_qk_matmul
    1: [D.IN, D.OUT, D.OUT, D.OUT],  # SF   aiv_softmax_prepare
    2: [D.IN, D.IN, D.OUT],  # PV   aic_pv_matmul
    3: [D.IN, D.IN, D.IN, D.INOUT, D.INOUT, D.INOUT, D.INOUT],  # UP aiv_online_update
}


def reference_chain_callable(orch_binary: bytes = b"", incore_binaries: dict[int, bytes] | None = None) -> ChipCallable:
    """The reference's paged-attention CALLABLE (test_paged_attention.py:25-61).

    Orchestration ``aicpu_orchestration_entry`` with the QK/SF/PV/UP incores at
    func ids 0..3. The binaries are carried but not executed: the HIP backend
    recognises the chain by its signatures and runs the fused kernel.
    """
    incore_binaries = incore_binaries or {}
    children = [
        (fid, CoreCallable.build(signature=sig, binary=incore_binaries.get(fid, b"")))
        for fid, sig in INCORE_SIGNATURES.items()
    ]
    return ChipCallable.build(
        signature=ORCH_SIGNATURE,
        func_name="aicpu_orchestration_entry",
        binary=orch_binary,
        children=children,
        config_name="aicpu_orchestration_config",
    )


def native_callable() -> ChipCallable:
    """A callable that names the fused decode directly."""
    return ChipCallable.build(signature=ORCH_SIGNATURE, func_name=NATIVE_CALLABLE_NAME, binary=b"", children=[])


# Incore signatures of the grouped split-K ("unroll") chain: QK and PV take a
# third input (tests/st/a2a3/tensormap_and_ringbuffer/paged_attention_unroll/
# test_paged_attention_unroll.py:25-61).
UNROLL_INCORE_SIGNATURES = {
    0: [D.IN, D.IN, D.IN, D.OUT],  # QK   grouped aic_qk_matmul
    1: [D.IN, D.OUT, D.OUT, D.OUT],  # SF   two-pass aiv_softmax_prepare
    2: [D.IN, D.IN, D.IN, D.OUT],  # PV   grouped aic_pv_matmul
    3: [D.IN, D.IN, D.IN, D.INOUT, D.INOUT, D.INOUT, D.INOUT],  # UP
}
# The cooperative AIC/AIV task of spmd_paged_attention: both halves declare the
# shared 9-tensor payload (tests/st/a2a3/tensormap_and_ringbuffer/
# spmd_paged_attention/test_spmd_paged_attention.py:28-54).
SPMD_INCORE_SIGNATURES = {
    0: [D.IN, D.IN, D.IN, D.IN, D.IN, D.INOUT, D.OUT, D.OUT, D.OUT],  # PA_AIC
    1: [D.IN, D.IN, D.IN, D.IN, D.IN, D.INOUT, D.OUT, D.OUT, D.OUT],  # PA_AIV
}

# The high-performance SPMD callable: query, key_cache, value_cache,
# block_table, out, eight workspaces, tiling, null (tests/st/a2a3/
# tensormap_and_ringbuffer/spmd_paged_attention_highperf/
# test_spmd_paged_attention_highperf.py:96-165); both halves of the mix task
# declare the same payload. Lengths and scale travel in the tiling tensor.
HIGHPERF_SIGNATURE = [D.IN, D.IN, D.IN, D.IN, D.OUT] + [D.IN] * 10
HIGHPERF_INCORE_SIGNATURES = {0: HIGHPERF_SIGNATURE, 1: HIGHPERF_SIGNATURE}

# Every paged-attention CALLABLE the reference defines, as (orchestration
# signature, incore signatures, child order by func id). Each registers and
# runs on the fused kernel.
REFERENCE_CALLABLES = {
    # examples/a2a3/tensormap_and_ringbuffer/paged_attention/test_paged_attention.py:25-61
    "paged_attention": (ORCH_SIGNATURE, INCORE_SIGNATURES, [0, 1, 2, 3]),
    # examples/a2a3/tensormap_and_ringbuffer/paged_attention_manual_scope/test_paged_attention_manual_scope.py:25-61
    "paged_attention_manual_scope": (ORCH_SIGNATURE, INCORE_SIGNATURES, [0, 1, 2, 3]),
    # examples/a2a3/tensormap_and_ringbuffer/paged_attention_ringbuffer/test_paged_attention_ringbuffer.py:34-66
    # (children listed as func ids 0, 2, 1, 3)
    "paged_attention_ringbuffer": (ORCH_SIGNATURE, INCORE_SIGNATURES, [0, 2, 1, 3]),
    # tests/st/a2a3/tensormap_and_ringbuffer/batch_paged_attention/test_batch_paged_attention.py:25-61
    "batch_paged_attention": (ORCH_SIGNATURE, INCORE_SIGNATURES, [0, 1, 2, 3]),
    # tests/st/a2a3/tensormap_and_ringbuffer/multi_round_paged_attention/test_multi_round_paged_attention.py:30-66
    "multi_round_paged_attention": (ORCH_SIGNATURE, INCORE_SIGNATURES, [0, 1, 2, 3]),
    # tests/st/a2a3/tensormap_and_ringbuffer/paged_attention_unroll/test_paged_attention_unroll.py:25-61
    "paged_attention_unroll": (ORCH_SIGNATURE, UNROLL_INCORE_SIGNATURES, [0, 1, 2, 3]),
    # examples/a2a3/tensormap_and_ringbuffer/paged_attention_unroll_manual_scope/
    # test_paged_attention_unroll_manual_scope.py:25-61
    "paged_attention_unroll_manual_scope": (ORCH_SIGNATURE, UNROLL_INCORE_SIGNATURES, [0, 1, 2, 3]),
    # tests/st/a2a3/tensormap_and_ringbuffer/paged_attention_unroll_4dims/test_paged_attention_unroll_4dims.py:32-64
    # (query and out as [B, 1, H, D], :120-122)
    "paged_attention_unroll_4dims": (ORCH_SIGNATURE, UNROLL_INCORE_SIGNATURES, [0, 1, 2, 3]),
    # tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention/test_spmd_paged_attention.py:28-54
    "spmd_paged_attention": (ORCH_SIGNATURE, SPMD_INCORE_SIGNATURES, [0, 1]),
    # tests/st/a2a3/tensormap_and_ringbuffer/spmd_paged_attention_highperf/test_spmd_paged_attention_highperf.py:96-165
    "spmd_paged_attention_highperf": (HIGHPERF_SIGNATURE, HIGHPERF_INCORE_SIGNATURES, [0, 1]),
}

_FAMILY_OF_SIGS = {id(INCORE_SIGNATURES): "chain", id(UNROLL_INCORE_SIGNATURES): "unroll",
                   id(SPMD_INCORE_SIGNATURES): "spmd", id(HIGHPERF_INCORE_SIGNATURES): "highperf"}
# The family simpler_hip_callable_family reports for each
REFERENCE_FAMILIES = {name: _FAMILY_OF_SIGS[id(sigs)] for name, (_, sigs, _) in REFERENCE_CALLABLES.items()}
# The callables whose arguments are the 7-argument form (every one but highperf)
SEVEN_ARGUMENT_CALLABLES = sorted(n for n, f in REFERENCE_FAMILIES.items() if f != "highperf")


def reference_callable(name: str, orch_binary: bytes = b"",
                       incore_binaries: dict[int, bytes] | None = None) -> ChipCallable:
    """The reference's CALLABLE ``name`` (a key of ``REFERENCE_CALLABLES``), with
    its signatures and child order. Binaries are carried, not executed."""
    orch_sig, sigs, order = REFERENCE_CALLABLES[name]
    incore_binaries = incore_binaries or {}
    children = [(fid, CoreCallable.build(signature=sigs[fid], binary=incore_binaries.get(fid, b""))) for fid in order]
    return ChipCallable.build(
        signature=orch_sig,
        func_name="aicpu_orchestration_entry",
        binary=orch_binary,
        children=children,
        config_name="aicpu_orchestration_config",
    )
