"""Loader for libsimpler_hip.so (the product's native library).

The library is built in-tree by ``simpler_amd.build`` (or ``__graft_entry__.build``).
There is no fallback: if the library is missing, every entry point raises.

torch is imported first so that the process has exactly one HIP runtime:
torch ships its own ``libamdhip64.so`` (soname ``libamdhip64.so.7``), and the
dynamic linker then binds this library's ``libamdhip64.so.7`` dependency to
that already-loaded copy, so device pointers and streams are shared.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libsimpler_hip.so"

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NativeLibraryMissing(RuntimeError):
    pass


class PaDecodeArgs(ctypes.Structure):
    """Mirror of ``SimplerHipPaDecodeArgs`` (include/simpler_hip/pa_decode.h)."""

    _fields_ = [
        ("query", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p),
        ("value_cache", ctypes.c_void_p),
        ("block_table", ctypes.c_void_p),
        ("context_lens", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("k_block_stride", ctypes.c_int64),
        ("k_token_stride", ctypes.c_int64),
        ("k_head_stride", ctypes.c_int64),
        ("v_block_stride", ctypes.c_int64),
        ("v_token_stride", ctypes.c_int64),
        ("v_head_stride", ctypes.c_int64),
        ("batch", ctypes.c_int32),
        ("q_len", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim_k", ctypes.c_int32),
        ("head_dim_v", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("num_workers", ctypes.c_int32),
        ("kv_format", ctypes.c_int32),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
    ]


class KvAppendArgs(ctypes.Structure):
    """Mirror of ``SimplerHipKvAppendArgs`` (include/simpler_hip/kv_cache.h)."""

    _fields_ = [
        ("key", ctypes.c_void_p),
        ("value", ctypes.c_void_p),
        ("slot_mapping", ctypes.c_void_p),
        ("key_cache", ctypes.c_void_p),
        ("value_cache", ctypes.c_void_p),
        ("error_count", ctypes.c_void_p),
        *[(n, ctypes.c_int64) for n in ("key_token_stride", "key_head_stride", "value_token_stride",
                                         "value_head_stride", "k_block_stride", "k_token_stride", "k_head_stride",
                                         "v_block_stride", "v_token_stride", "v_head_stride")],
        *[(n, ctypes.c_int32) for n in ("num_tokens", "num_kv_heads", "head_dim_k", "head_dim_v", "block_size",
                                         "num_blocks")],
    ]


class QkNormRopeAppendArgs(ctypes.Structure):
    """Mirror of ``SimplerHipQkNormRopeAppendArgs`` (include/simpler_hip/kv_cache.h)."""

    _fields_ = [
        *[(n, ctypes.c_void_p) for n in ("q_proj", "k_proj", "v_proj", "inv_rms", "q_norm_weight", "k_norm_weight",
                                          "rope_cos", "rope_sin", "seq_lens", "slot_mapping", "q_out", "key_cache",
                                          "value_cache", "error_count")],
        *[(n, ctypes.c_int64) for n in ("k_block_stride", "k_token_stride", "k_head_stride", "v_block_stride",
                                         "v_token_stride", "v_head_stride")],
        *[(n, ctypes.c_int32) for n in ("batch", "num_heads", "num_kv_heads", "head_dim", "block_size", "num_blocks",
                                         "max_position")],
        ("eps", ctypes.c_float),
    ]


class DecodePreludeArgs(ctypes.Structure):
    """Mirror of ``SimplerHipDecodePreludeArgs`` (include/simpler_hip/pa_decode.h)."""

    _fields_ = [
        *[(n, ctypes.c_void_p) for n in ("q_proj", "k_proj", "v_proj", "inv_rms", "q_norm_weight", "k_norm_weight",
                                          "rope_cos", "rope_sin")],
        ("max_position", ctypes.c_int32),
        ("eps", ctypes.c_float),
    ]


# Every symbol the public headers declare, with its ctypes signature.
_VP, _SZ, _I32, _U32, _U64, _I = (
    ctypes.c_void_p,
    ctypes.c_size_t,
    ctypes.c_int32,
    ctypes.c_uint32,
    ctypes.c_uint64,
    ctypes.c_int,
)
_ARGS_P = ctypes.POINTER(PaDecodeArgs)
SIGNATURES: dict[str, tuple] = {
    # include/simpler_hip/pa_decode.h
    "simpler_hip_pa_decode_workspace_size": (_SZ, [_ARGS_P]),
    "simpler_hip_pa_decode_workspace_init": (_I, [_VP, _SZ, _VP]),
    "simpler_hip_pa_decode": (_I, [_ARGS_P, _VP, _SZ, _VP]),
    "simpler_hip_pa_decode_phase": (_I, [_ARGS_P, _VP, _SZ, _VP, _I]),
    "simpler_hip_pa_decode_check": (_I, [_VP, _SZ, _VP]),
    "simpler_hip_pa_decode_noalloc": (_I, [_ARGS_P, _VP]),
    "simpler_hip_pa_decode_append": (_I, [_ARGS_P, _VP, _VP, _VP, _SZ, _VP]),
    "simpler_hip_pa_decode_prelude": (_I, [_ARGS_P, ctypes.POINTER(DecodePreludeArgs), _VP, _SZ, _VP]),
    "simpler_hip_pa_decode_prelude_workspace_size": (_SZ, [_ARGS_P]),
    "simpler_hip_pa_decode_kernel_name": (ctypes.c_char_p, [_ARGS_P]),
    "simpler_hip_pa_decode_plan": (_I, [_ARGS_P, ctypes.POINTER(_I32)]),
    # include/simpler_hip/kv_cache.h
    "simpler_hip_kv_append": (_I, [ctypes.POINTER(KvAppendArgs), _VP]),
    "simpler_hip_qk_norm_rope_append": (_I, [ctypes.POINTER(QkNormRopeAppendArgs), _VP]),
    # include/simpler_hip/pto_runtime_c_api.h
    "get_pipeline_contract": (_VP, []),
    "get_runtime_size": (_SZ, []),
    "get_runtime_alignment": (_SZ, []),
    "create_device_context": (_VP, []),
    "destroy_device_context": (None, [_VP]),
    "simpler_init": (_I, [_VP, _I, _VP, _SZ, _VP, _SZ, _VP, _SZ, _VP]),
    "finalize_device": (_I, [_VP]),
    "device_malloc_ctx": (_VP, [_VP, _SZ]),
    "device_free_ctx": (None, [_VP, _VP]),
    "committed_device_memory_ctx": (_SZ, [_VP]),
    "copy_to_device_ctx": (_I, [_VP, _VP, _VP, _SZ]),
    "copy_from_device_ctx": (_I, [_VP, _VP, _VP, _SZ]),
    "simpler_register_callable": (_I, [_VP, _I32, _VP]),
    "simpler_unregister_callable": (_I, [_VP, _I32]),
    "simpler_run": (_I, [_VP, _VP, _I32, _VP, _VP, _VP]),
    "simpler_prepare_run": (_I, [_VP, _VP, _I32, _VP, _VP, _VP]),
    "supports_concurrent_native_prepare_ctx": (_I, [_VP]),
    "simpler_launch_run": (_I, [_VP, _VP]),
    "simpler_poll_run": (_I, [_VP, _VP]),
    "simpler_wait_run": (_I, [_VP, _VP]),
    "simpler_finalize_run": (_I, [_VP, _VP]),
    "get_arena_bank_gm_heap_base_ctx": (_U64, [_VP, _U32]),
    "get_retained_temp_addr_ctx": (_U64, [_VP, _U32]),
    "get_aicpu_dlopen_count": (_SZ, [_VP]),
    "get_host_dlopen_count": (_SZ, [_VP]),
    "get_run_stream_set_create_count": (_SZ, [_VP]),
    "simpler_provision_dma_workspace": (_I, [_VP, _U32, _VP, _U64]),
    "ensure_acl_ready_ctx": (_I, [_VP, _I]),
    "create_comm_stream_ctx": (_VP, [_VP]),
    "destroy_comm_stream_ctx": (_I, [_VP, _VP]),
    "comm_init": (_VP, [_I, _I, _VP, ctypes.c_char_p]),
    "comm_alloc_windows": (_I, [_VP, _SZ, _VP]),
    "comm_get_local_window_base": (_I, [_VP, _VP]),
    "comm_get_window_size": (_I, [_VP, _VP]),
    "comm_derive_context": (_I, [_VP, _VP, _SZ, _U32, _SZ, _SZ, _VP]),
    "comm_alloc_domain_windows": (_I, [_VP, _U64, _VP, _SZ, _U32, _SZ, _VP, _VP]),
    "comm_release_domain_windows": (_I, [_VP, _U64, _SZ, _U32]),
    "comm_global_domain_prepare": (_I, [_U64, _U32, _U32, _SZ, _U32, _VP, _VP]),
    "comm_global_domain_import": (_I, [_U64, _VP, _SZ, _VP]),
    "comm_global_domain_release": (_I, [_U64]),
    "comm_barrier": (_I, [_VP]),
    "comm_destroy": (_I, [_VP]),
    "simpler_hip_context_stream": (_VP, [_VP]),
    "simpler_hip_set_execution": (_I, [_VP, _I32]),
    "simpler_hip_callable_family": (_I, [_VP, _I32]),
    # include/simpler_hip/task_graph.h (tensor arrays are SimplerChipTensor[], passed as void*)
    "simpler_hip_tg_create": (_VP, [_I32, _VP]),
    "simpler_hip_tg_destroy": (None, [_VP]),
    "simpler_hip_tg_bind": (_I, [_VP, _I32, _I32]),
    "simpler_hip_tg_register_kernel": (_I, [_VP, _I32, ctypes.c_char_p, ctypes.c_char_p, _U32, _I32, _U32]),
    "simpler_hip_tg_record_replay": (_I, [_VP, _VP, _U64]),
    "simpler_hip_tg_replay": (_I, [_VP, _VP, _U64]),
    "simpler_hip_tg_scope_begin": (_I, [_VP]),
    "simpler_hip_tg_scope_end": (_I, [_VP]),
    "simpler_hip_tg_submit": (ctypes.c_int64, [_VP, _I32, _VP, ctypes.POINTER(_I32), _I32, ctypes.POINTER(_U64),
                                               _I32, ctypes.POINTER(_U64), _I32, _VP]),
    "simpler_hip_tg_alloc": (ctypes.c_int64, [_VP, _VP, _I32, _VP]),
    "simpler_hip_tg_get_tensor_data": (_I, [_VP, _VP, _U32, ctypes.POINTER(_U32), ctypes.POINTER(_U64)]),
    "simpler_hip_tg_copy_to_host": (_I, [_VP, _VP, _VP, _U64]),
    "simpler_hip_tg_launch": (_I, [_VP]),
    "simpler_hip_tg_wait": (_I, [_VP]),
    "simpler_hip_tg_reset": (_I, [_VP]),
    "simpler_hip_tg_orchestrate_paged_attention": (_I, [_VP, _VP, _U64]),
    "simpler_hip_tg_orchestrate_vector_example": (_I, [_VP, _VP]),
    "simpler_hip_tg_task_count": (ctypes.c_int64, [_VP]),
    "simpler_hip_tg_replay_count": (_U64, [_VP]),
    "simpler_hip_tg_fanin": (_I32, [_VP, ctypes.c_int64, ctypes.POINTER(ctypes.c_int64), _I32]),
    "simpler_hip_tg_arena_bytes": (_U64, [_VP]),
}


def lib() -> ctypes.CDLL:
    """The loaded native library; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m simpler_amd.build` "
                "(the HIP backend has no fallback)"
            )
        import torch  # noqa: F401  — one HIP runtime per process (see module docstring)

        handle = ctypes.CDLL(str(LIB_PATH), mode=os.RTLD_NOW | os.RTLD_LOCAL)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
        return _lib
