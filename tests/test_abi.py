"""CPU checks of the drop-in boundary: byte layouts, exported symbols, host-side logic.

No kernel is launched here (the container has no GPU); everything below runs in
host code of libsimpler_hip.so or in the Python mirror.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from simpler_amd import _lib
from simpler_amd import paged_attention as pa
from simpler_amd.task_interface import (
    ArgDirection,
    CallConfig,
    ChipCallable,
    ChipStorageTaskArgs,
    ChipTensor,
    CoreCallable,
    DataType,
    scalar_to_uint64,
)

ROOT = Path(__file__).resolve().parent.parent


def declared_functions() -> set[str]:
    names = set()
    for hdr in (ROOT / "include").rglob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        for m in re.finditer(r"^[A-Za-z_][\w \*]*?\b([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M):
            if not m.group(0).lstrip().startswith(("typedef", "return", "static")):
                names.add(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert len(names) >= 45, names
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == names


def test_chip_tensor_layout_matches_reference_static_asserts():
    # src/common/task_interface/tensor.h:489-500
    assert ctypes.sizeof(ChipTensor) == 128
    offs = {f[0]: getattr(ChipTensor, f[0]).offset for f in ChipTensor._fields_}
    assert offs["owner_task_id"] == 16 and offs["start_offset"] == 24 and offs["version"] == 32
    assert offs["ndims"] == 36 and offs["dtype"] == 40 and offs["manual_dep"] == 41
    assert offs["is_contiguous"] == 42 and offs["address_space"] == 43 and offs["shapes"] == 44
    assert offs["extent_elem_cache"] == 64 and offs["strides"] == 72


def test_task_args_and_call_config_layout():
    assert ctypes.sizeof(ChipStorageTaskArgs) == 33856
    assert ChipStorageTaskArgs.scalars_.offset == 256 * 128
    assert ChipStorageTaskArgs.tensor_count_.offset == 256 * 128 + 128 * 8
    assert ctypes.sizeof(CallConfig) == 6 * 4 + 12 * 8 + 1024  # call_config.h:146-150
    args = ChipStorageTaskArgs()
    args.add_tensor(ChipTensor.make(0x1000, (2, 3), DataType.FLOAT32))
    args.add_scalar(1.0)
    with pytest.raises(RuntimeError):
        args.add_tensor(ChipTensor.make(0x1000, (2,), DataType.FLOAT32))
    assert args.scalar(0) == 0x3F800000 and args.tensor_count() == 1


def test_chip_tensor_make_fields():
    t = ChipTensor.make(0xABC0, (4, 8, 2, 16), DataType.BFLOAT16, child_memory=True)
    assert t.ndims == 4 and list(t.strides)[:4] == [256, 32, 16, 1]
    assert t.buffer.size == 4 * 8 * 2 * 16 * 2 and t.is_contiguous == 1 and t.address_space == 1
    v = ChipTensor.make(0xABC0, (4, 8, 1, 12), DataType.BFLOAT16, strides=(8 * 16, 16, 16, 1))
    assert v.is_contiguous == 0


def test_scalar_to_uint64_matches_reference_rules():
    assert scalar_to_uint64(1.0) == 0x3F800000
    assert scalar_to_uint64(ctypes.c_float(0.5)) == 0x3F000000
    assert scalar_to_uint64(ctypes.c_double(1.0)) == 0x3FF0000000000000
    assert scalar_to_uint64(-1) == 0xFFFFFFFFFFFFFFFF


def test_callable_byte_layout():
    core = CoreCallable.build(signature=[ArgDirection.IN, ArgDirection.OUT], binary=b"\x01\x02\x03")
    raw = core.buffer
    assert len(raw) == 192 + 3 and raw[192:] == b"\x01\x02\x03"
    assert int.from_bytes(raw[128:132], "little") == 2 and int.from_bytes(raw[132:136], "little") == 3
    chip = pa.reference_chain_callable(orch_binary=b"ORCH")
    raw = chip.buffer
    assert raw[1032:1032 + 25] == b"aicpu_orchestration_entry"
    assert int.from_bytes(raw[9292:9296], "little") == 4  # child_count_
    assert raw[ChipCallable.STORAGE_OFFSET:ChipCallable.STORAGE_OFFSET + 4] == b"ORCH"
    first_child = int.from_bytes(raw[5196:5200], "little")
    assert first_child % 64 == 0 and first_child >= 4


def test_register_recognises_the_reference_pa_callables_only():
    lib = _lib.lib()
    ctx = lib.create_device_context()
    try:
        assert lib.simpler_register_callable(ctx, 0, pa.reference_chain_callable().address()) == 0
        assert lib.simpler_hip_callable_family(ctx, 0) == 0
        assert lib.simpler_register_callable(ctx, 1, pa.native_callable().address()) == 0
        assert lib.simpler_hip_callable_family(ctx, 1) == 3
        other = ChipCallable.build(signature=[ArgDirection.IN], func_name="vector_add", binary=b"",
                                   children=[(0, CoreCallable.build([ArgDirection.IN]))])
        assert lib.simpler_register_callable(ctx, 2, other.address()) == -2
        assert lib.simpler_hip_callable_family(ctx, 2) == -1
        # same orchestration signature but a different incore chain is not the PA chain
        wrong = ChipCallable.build(signature=pa.ORCH_SIGNATURE, func_name="aicpu_orchestration_entry", binary=b"",
                                   children=[(i, CoreCallable.build([ArgDirection.IN])) for i in range(4)])
        assert lib.simpler_register_callable(ctx, 3, wrong.address()) == -2
        assert lib.simpler_register_callable(ctx, 64, pa.native_callable().address()) == -1
    finally:
        lib.destroy_device_context(ctx)


@pytest.mark.parametrize("name", sorted(pa.REFERENCE_CALLABLES))
def test_every_reference_pa_callable_registers_with_its_family(name):
    """Each paged-attention CALLABLE the reference defines (chain, grouped
    "unroll", SPMD mix) registers with 0 and is classified into its family."""
    lib = _lib.lib()
    ctx = lib.create_device_context()
    try:
        assert lib.simpler_register_callable(ctx, 5, pa.reference_callable(name).address()) == 0
        fam = lib.simpler_hip_callable_family(ctx, 5)
        assert {0: "chain", 1: "unroll", 2: "spmd", 4: "highperf"}[fam] == pa.REFERENCE_FAMILIES[name]
    finally:
        lib.destroy_device_context(ctx)


def test_register_rejects_mixed_or_incomplete_families():
    """A chain whose children mix the two families' QK/PV signatures, repeat a
    func id, or miss one is not any reference callable."""
    lib = _lib.lib()
    D = ArgDirection

    def build(children):
        return ChipCallable.build(signature=pa.ORCH_SIGNATURE, func_name="aicpu_orchestration_entry", binary=b"",
                                  children=[(fid, CoreCallable.build(sig)) for fid, sig in children])

    chain, unroll, spmd = pa.INCORE_SIGNATURES, pa.UNROLL_INCORE_SIGNATURES, pa.SPMD_INCORE_SIGNATURES
    bad = [
        [(0, unroll[0]), (1, chain[1]), (2, chain[2]), (3, chain[3])],  # unroll QK with chain PV
        [(0, chain[0]), (1, chain[1]), (1, chain[1]), (3, chain[3])],   # func id 1 twice, 2 missing
        [(0, chain[0]), (1, chain[1]), (2, chain[2])],                  # UP missing
        [(0, spmd[0])],                                                 # half of the SPMD mix
        [(0, spmd[0]), (1, [D.IN] * 9)],                                # wrong AIV payload
    ]
    ctx = lib.create_device_context()
    try:
        for i, children in enumerate(bad):
            assert lib.simpler_register_callable(ctx, i, build(children).address()) == -2, i
    finally:
        lib.destroy_device_context(ctx)


def test_pipeline_contract_and_sizes():
    lib = _lib.lib()
    p = ctypes.cast(lib.get_pipeline_contract(), ctypes.POINTER(ctypes.c_uint32 * 3)).contents
    assert list(p) == [1, 0, 1]  # abi_version, resource_count, pipeline_depth
    assert lib.get_runtime_size() >= 256 and lib.get_runtime_alignment() == 64


def test_unsupported_entry_points_say_so():
    lib = _lib.lib()
    assert lib.comm_init(0, 1, None, b"") is None
    assert lib.comm_barrier(None) == -2
    assert lib.ensure_acl_ready_ctx(None, 0) == -2
    assert lib.simpler_provision_dma_workspace(None, 1, None, 0) == -2
    assert lib.simpler_provision_dma_workspace(None, 0, None, 0) == 0


def _args(**kw) -> _lib.PaDecodeArgs:
    a = _lib.PaDecodeArgs()
    base = dict(query=0x1000, key_cache=0x2000, value_cache=0x3000, block_table=0x4000, context_lens=0x5000,
                out=0x6000, k_block_stride=128 * 8 * 128, k_token_stride=8 * 128, k_head_stride=128,
                v_block_stride=128 * 8 * 128, v_token_stride=8 * 128, v_head_stride=128, batch=32, q_len=1,
                num_heads=32, num_kv_heads=8, head_dim_k=128, head_dim_v=128, block_size=128,
                max_blocks_per_seq=64, num_blocks=1200, out_dtype=6, scale=0.088, causal=0, num_workers=0)
    base.update(kw)
    for k, v in base.items():
        setattr(a, k, v)
    return a


def test_host_validation_rejects_bad_arguments_without_launching():
    lib = _lib.lib()
    good = _args()
    assert lib.simpler_hip_pa_decode_workspace_size(ctypes.byref(good)) > 0
    bad = [
        _args(num_heads=30),  # not a multiple of kv heads
        _args(head_dim_k=100, head_dim_v=100),  # not a multiple of 8
        _args(k_token_stride=0),
        _args(query=0x1001),  # misaligned
        _args(num_workers=-1),
        _args(block_size=0),
    ]
    for a in bad:
        assert lib.simpler_hip_pa_decode(ctypes.byref(a), ctypes.c_void_p(0x100000), 1 << 30, None) == -1
    assert lib.simpler_hip_pa_decode(ctypes.byref(_args(out_dtype=2)), ctypes.c_void_p(0x100000), 1 << 30,
                                     None) == -2
    # unsupported block size (not a multiple of 16)
    assert lib.simpler_hip_pa_decode(ctypes.byref(_args(block_size=48)), ctypes.c_void_p(0x100000), 1 << 30,
                                     None) == -2
    # workspace too small
    assert lib.simpler_hip_pa_decode(ctypes.byref(good), ctypes.c_void_p(0x100000), 16, None) == -4


def _mla_args(**kw) -> _lib.PaDecodeArgs:
    # DeepSeek MLA shape: V = the first 512 dims of the 576-dim latent K (same buffer, same strides)
    base = dict(key_cache=0x2000, value_cache=0x2000, k_block_stride=64 * 576, k_token_stride=576,
                k_head_stride=576, v_block_stride=64 * 576, v_token_stride=576, v_head_stride=576,
                batch=128, num_heads=128, num_kv_heads=1, head_dim_k=576, head_dim_v=512, block_size=64,
                max_blocks_per_seq=128)
    base.update(kw)
    return _args(**base)


def test_mla_dispatch_and_plan():
    lib = _lib.lib()
    name = lambda a: lib.simpler_hip_pa_decode_kernel_name(ctypes.byref(a)).decode()
    assert name(_mla_args()) == "pa_mla_kernel"
    assert name(_mla_args(block_size=32)) == "pa_mla_kernel"
    assert name(_args()) == "pa_decode_kernel"
    # 128 query rows = one 128-row group: 256 slices of one workgroup on a 256-CU device
    assert pa.plan(_mla_args()) == 256
    assert pa.plan(_mla_args(num_heads=192)) == 128  # two row groups per slice
    assert pa.plan(_mla_args(num_heads=16)) == 256
    ws = lambda **kw: lib.simpler_hip_pa_decode_workspace_size(ctypes.byref(_mla_args(**kw)))
    # two partial slots per row tile (8 per slice), 16 rows x 512 fp32 each
    assert ws(num_workers=3) == 256 + 3 * 8 * 2 * 32 * 4 + 3 * 8 * 2 * 16 * 512 * 4
    # V that is not the K prefix (other buffer or strides), or a block size without 32-token steps
    for bad in (_mla_args(value_cache=0x3000), _mla_args(v_token_stride=1152), _mla_args(block_size=16),
                _mla_args(block_size=128)):
        assert lib.simpler_hip_pa_decode(ctypes.byref(bad), ctypes.c_void_p(0x100000), 1 << 30, None) == -2


def test_fused_append_validates_on_the_host():
    lib = _lib.lib()
    k, v = ctypes.c_void_p(0x7000), ctypes.c_void_p(0x8000)

    def call(a, kn, vn, ws_bytes=1 << 30):
        return lib.simpler_hip_pa_decode_append(ctypes.byref(a), kn, vn, ctypes.c_void_p(0x100000), ws_bytes, None)

    assert call(_args(), None, v) == -1  # key_new is required
    assert call(_args(), k, None) == -1  # and value_new for separate caches
    assert call(_args(), ctypes.c_void_p(0x7008), v) == -1  # 16-byte aligned rows
    assert call(_mla_args(), k, v) == -1  # MLA: V is the K prefix, no value_new
    assert call(_args(q_len=17, num_heads=8, causal=1), k, v) == -2  # more than 16 new tokens
    assert call(_args(kv_format=1, k_scale=0x9000, v_scale=0xA000), k, v) == -2  # no fused append for fp8
    assert call(_args(), k, v, ws_bytes=16) == -4  # the decode's workspace rule
    assert call(_mla_args(), k, None, ws_bytes=16) == -4


def test_prelude_entry_validates_on_the_host():
    lib = _lib.lib()

    def pre(**kw):
        p = _lib.DecodePreludeArgs()
        for i, n in enumerate(("q_proj", "k_proj", "v_proj", "inv_rms", "q_norm_weight", "k_norm_weight", "rope_cos",
                               "rope_sin")):
            setattr(p, n, 0x10000 + 0x1000 * i)
        p.max_position, p.eps = 8192, 1e-6
        for k, v in kw.items():
            setattr(p, k, v)
        return p

    def call(a, p, ws_bytes=1 << 30):
        return lib.simpler_hip_pa_decode_prelude(ctypes.byref(a), ctypes.byref(p) if p is not None else None,
                                                 ctypes.c_void_p(0x100000), ws_bytes, None)

    assert call(_args(), None) == -1
    assert call(_args(), pre(k_proj=0)) == -1  # every projection is required
    assert call(_args(), pre(rope_sin=0x20008)) == -1  # 16-byte aligned
    assert call(_args(), pre(max_position=0)) == -1
    assert call(_args(), pre(eps=-1.0)) == -1
    assert call(_args(query=0), pre(), ws_bytes=16) == -4  # the query is not read: only the workspace rule fails
    assert call(_args(head_dim_k=64, head_dim_v=64, k_head_stride=64, v_head_stride=64), pre()) == -2  # 128 only
    assert call(_args(kv_format=1, k_scale=0x9000, v_scale=0xA000), pre()) == -2  # bf16 caches only
    assert call(_args(kv_format=2), pre()) == -2
    assert call(_args(q_len=17, num_heads=8, causal=1), pre()) == -2  # at most 16 new tokens
    assert call(_mla_args(), pre()) == -2


def test_prelude_workspace_holds_the_query_after_the_decode_part():
    lib = _lib.lib()
    size = lambda f, a: getattr(lib, f)(ctypes.byref(a))  # noqa: E731
    for kw in (dict(), dict(q_len=8, causal=1, batch=16), dict(query=0)):
        a = _args(**kw)
        plain = size("simpler_hip_pa_decode_workspace_size", _args(**{**kw, "query": 0x1000}))
        q_rows = a.batch * a.q_len * a.num_heads * 128 * 2  # bf16 query rows
        assert size("simpler_hip_pa_decode_prelude_workspace_size", a) == plain + -(-q_rows // 256) * 256
    # what the prelude does not run on
    for kw in (dict(head_dim_k=64, head_dim_v=64, k_head_stride=64, v_head_stride=64), dict(kv_format=2),
               dict(q_len=17, num_heads=8, causal=1)):
        assert size("simpler_hip_pa_decode_prelude_workspace_size", _args(**kw)) == 0
    assert size("simpler_hip_pa_decode_prelude_workspace_size", _mla_args()) == 0


def test_worker_plan():
    # without a device the launcher assumes an MI355X (256 CUs). 128-dim bf16 heads
    # read K in whole rows through LDS: one worker per SIMD
    assert pa.plan(_args()) == 1024
    # other head dims read K in half lines: two workers per CU
    assert pa.plan(_args(head_dim_k=64, head_dim_v=64, k_head_stride=64, v_head_stride=64)) == 512
    # the default count is rounded down to whole work lists (one per kv head)
    assert pa.plan(_args(num_heads=24, num_kv_heads=6)) == 1020
    assert pa.plan(_args(num_workers=7)) == 7
    ws = lambda **kw: _lib.lib().simpler_hip_pa_decode_workspace_size(ctypes.byref(_args(**kw)))
    # error word, the zero page (16 token strides of 2 KB + 512 B: what one 16-token
    # tile's lane offsets span), two (m, l) and two O partial slots per worker,
    # 256-byte aligned sections
    zero_page = 16 * 2048 + 512
    assert ws(num_workers=7) == 256 + zero_page + 7 * 2 * 32 * 4 + 7 * 2 * 16 * 128 * 4
    assert ws(num_workers=1) == 256 + zero_page + 256 + 2 * 16 * 128 * 4
    # q_len 8 x group 4 = 32 rows = 2 row tiles: with 128-dim heads one wave runs
    # both (three workers per CU), two partial slots per row tile
    assert pa.plan(_args(q_len=8, causal=1)) == 768
    assert ws(q_len=8, causal=1, num_workers=7) == 256 + zero_page + 7 * 2 * 2 * 32 * 4 + 7 * 2 * 2 * 16 * 128 * 4
    # other head dims: a 2-wave workgroup (sibling waves), two per CU
    assert pa.plan(_args(q_len=8, causal=1, head_dim_k=64, head_dim_v=64, k_head_stride=64, v_head_stride=64)) == 512
    # token strides too large for a 1 MB zero page: padding tiles are read as they are
    assert ws(num_workers=7, k_token_stride=1 << 15, v_token_stride=1 << 15, k_block_stride=1 << 22,
              v_block_stride=1 << 22) == 256 + 7 * 2 * 32 * 4 + 7 * 2 * 16 * 128 * 4
    # 25 row tiles: 4-wave workgroups, one per CU, in 7 work lists (row groups)
    assert pa.plan(_args(num_heads=80, num_kv_heads=1, q_len=5, causal=1)) == 252
    # fp8 caches: three single-wave workers per CU, in four work lists
    assert pa.plan(_args(kv_format=1, k_scale=0x7000, v_scale=0x7100)) == 768


def test_work_list_must_fit_32_bit_indices():
    lib = _lib.lib()
    huge = _args(batch=65535, num_heads=32, num_kv_heads=8, max_blocks_per_seq=8192)
    assert lib.simpler_hip_pa_decode(ctypes.byref(huge), ctypes.c_void_p(0x100000), 1 << 40, None) == -2


def test_kv_cache_entry_points_validate_on_the_host():
    lib = _lib.lib()

    def app(**kw):
        a = _lib.KvAppendArgs()
        base = dict(key=0x1000, value=0x2000, slot_mapping=0x3000, key_cache=0x4000, value_cache=0x5000,
                    key_token_stride=8 * 128, key_head_stride=128, value_token_stride=8 * 128, value_head_stride=128,
                    k_block_stride=128 * 8 * 128, k_token_stride=8 * 128, k_head_stride=128,
                    v_block_stride=128 * 8 * 128, v_token_stride=8 * 128, v_head_stride=128, num_tokens=0,
                    num_kv_heads=8, head_dim_k=128, head_dim_v=128, block_size=128, num_blocks=10)
        base.update(kw)
        for k, v in base.items():
            setattr(a, k, v)
        return lib.simpler_hip_kv_append(ctypes.byref(a), None)

    assert app() == 0  # zero tokens: valid, nothing launched
    for bad in (dict(head_dim_k=100), dict(key_cache=0x4008), dict(k_token_stride=4), dict(value=0),
                dict(num_kv_heads=0), dict(head_dim_k=2048)):
        assert app(**bad) == -1, bad
    assert app(value=0, value_cache=0) == 0  # K-only cache (MLA latent)

    def pre(**kw):
        a = _lib.QkNormRopeAppendArgs()
        ptrs = ("q_proj", "k_proj", "v_proj", "inv_rms", "q_norm_weight", "k_norm_weight", "rope_cos", "rope_sin",
                "seq_lens", "slot_mapping", "q_out", "key_cache", "value_cache")
        base = {n: 0x1000 * (i + 1) for i, n in enumerate(ptrs)}
        base.update(k_block_stride=128 * 8 * 128, k_token_stride=8 * 128, k_head_stride=128,
                    v_block_stride=128 * 8 * 128, v_token_stride=8 * 128, v_head_stride=128, batch=0, num_heads=32,
                    num_kv_heads=8, head_dim=128, block_size=128, num_blocks=10, max_position=4096, eps=1e-6)
        base.update(kw)
        for k, v in base.items():
            setattr(a, k, v)
        return lib.simpler_hip_qk_norm_rope_append(ctypes.byref(a), None)

    assert pre() == 0
    for bad in (dict(head_dim=127), dict(q_out=0), dict(max_position=0), dict(eps=-1.0), dict(v_head_stride=0)):
        assert pre(**bad) == -1, bad


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float16", "float8_e4m3fn"])
def test_kv_pools_sit_an_odd_multiple_of_256_bytes_apart(dtype_name):
    import torch

    from simpler_amd.kv_cache import alloc_kv_pools
    from simpler_amd.workloads import make_case

    dtype = getattr(torch, dtype_name)
    for nblk, bs, hkv, dk, dv in ((7, 16, 3, 96, 64), (10, 128, 8, 128, 128), (1, 1, 1, 8, 8)):
        k, v = alloc_kv_pools(nblk, bs, hkv, dk, dtype, "cpu", head_dim_v=dv)
        assert k.shape == (nblk, bs, hkv, dk) and v.shape == (nblk, bs, hkv, dv)
        assert k.is_contiguous() and v.is_contiguous() and k.dtype == v.dtype == dtype
        gap = v.data_ptr() - k.data_ptr()
        assert gap >= k.numel() * k.element_size()  # no overlap
        assert gap % 512 == 256 and gap - k.numel() * k.element_size() < 768
        assert k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()  # one allocation
    case = make_case("cfg1_small")
    pooled = case.to("cpu", kv_pool=True)
    assert torch.equal(pooled.key_cache, case.key_cache) and torch.equal(pooled.value_cache, case.value_cache)
    assert (pooled.value_cache.data_ptr() - pooled.key_cache.data_ptr()) % 512 == 256
