"""simpler's L2 task interface, mirrored for the HIP backend.

Same names, byte layouts and argument meaning as the reference's
``python/simpler/task_interface.py`` and its nanobind module
``_task_interface`` (``python/bindings/task_interface.cpp``), for the part of the
surface an L2 paged-attention workload uses:

* ``DataType``, ``ArgDirection``, ``TensorArgType``, ``AddressSpace`` codes
  (``src/common/task_interface/{data_type.h:47-67, arg_direction.h:22-27,
  tensor.h:43-49}``)
* ``ChipTensor`` (128-byte POD, ``tensor.h:95-113``) with ``ChipTensor.make``
* ``ChipStorageTaskArgs`` (``task_args.h:85-117,185``)
* ``CallConfig`` (packed, ``call_config.h:56-150``)
* ``CoreCallable.build`` / ``ChipCallable.build`` (``callable.h:181-289``)
* ``scalar_to_uint64`` (``python/simpler/task_interface.py:915-937``)
* ``ChipWorker`` (``python/simpler/task_interface.py:1240-1519``) over the
  ``simpler_*`` C API of ``libsimpler_hip.so``

The structures are ``ctypes`` mirrors, so their bytes are what the C API reads.
"""

from __future__ import annotations

import ctypes
import struct
import threading
from enum import IntEnum
from typing import Any, Sequence

MAX_TENSOR_DIMS = 5
CORE_MAX_TENSOR_ARGS = 32
CHIP_MAX_TENSOR_ARGS = 256
CHIP_MAX_SCALAR_ARGS = 128
CALLABLE_ALIGN = 64
CALLABLE_CHILD_ALIGN = 16
CALLABLE_FUNC_NAME_MAX = 64
CHIP_MAX_CHILDREN = 1024
MAX_REGISTERED_CALLABLE_IDS = 64


class DataType(IntEnum):
    FLOAT32 = 0
    FLOAT16 = 1
    INT32 = 2
    INT16 = 3
    INT8 = 4
    UINT8 = 5
    BFLOAT16 = 6
    INT64 = 7
    UINT64 = 8
    UINT16 = 9
    UINT32 = 10
    BOOL = 11
    FP8E4M3FN = 12
    FP8E8M0 = 13
    FP4E2M1 = 14


_ELEM_SIZE = {
    DataType.FLOAT32: 4, DataType.FLOAT16: 2, DataType.INT32: 4, DataType.INT16: 2, DataType.INT8: 1,
    DataType.UINT8: 1, DataType.BFLOAT16: 2, DataType.INT64: 8, DataType.UINT64: 8, DataType.UINT16: 2,
    DataType.UINT32: 4, DataType.BOOL: 1, DataType.FP8E4M3FN: 1, DataType.FP8E8M0: 1, DataType.FP4E2M1: 1,
}


def get_element_size(dtype: DataType) -> int:
    return _ELEM_SIZE[DataType(dtype)]


class ArgDirection(IntEnum):
    SCALAR = 0
    IN = 1
    OUT = 2
    INOUT = 3


class TensorArgType(IntEnum):
    INPUT = 0
    OUTPUT = 1
    INOUT = 2
    OUTPUT_EXISTING = 3
    NO_DEP = 4


class AddressSpace(IntEnum):
    HOST = 0
    DEVICE = 1


class _BufferHandle(ctypes.Structure):
    _fields_ = [("addr", ctypes.c_uint64), ("size", ctypes.c_uint64)]


class ChipTensor(ctypes.Structure):
    """128-byte tensor descriptor (``tensor.h:95-113``)."""

    _fields_ = [
        ("buffer", _BufferHandle),
        ("owner_task_id", ctypes.c_uint64),
        ("start_offset", ctypes.c_uint64),
        ("version", ctypes.c_int32),
        ("ndims", ctypes.c_uint32),
        ("dtype", ctypes.c_uint8),
        ("manual_dep", ctypes.c_uint8),
        ("is_contiguous", ctypes.c_uint8),
        ("address_space", ctypes.c_uint8),
        ("shapes", ctypes.c_uint32 * MAX_TENSOR_DIMS),
        ("extent_elem_cache", ctypes.c_uint64),
        ("strides", ctypes.c_uint32 * MAX_TENSOR_DIMS),
        ("_pad_cl2", ctypes.c_uint8 * 36),
    ]

    @classmethod
    def make(
        cls,
        data: int,
        shapes: Sequence[int],
        dtype: DataType,
        child_memory: bool = False,
        *,
        strides: Sequence[int] | None = None,
    ) -> "ChipTensor":
        """A tensor over existing memory (``make_tensor_external``, ``tensor.h:509-518``).

        ``child_memory=True`` marks ``data`` as a device address (``AddressSpace.DEVICE``),
        which the runtime passes through without staging. ``strides`` (elements)
        default to row-major.
        """
        nd = len(shapes)
        if not 0 < nd <= MAX_TENSOR_DIMS:
            raise ValueError(f"ChipTensor supports 1..{MAX_TENSOR_DIMS} dims, got {nd}")
        if strides is None:
            st, acc = [0] * nd, 1
            for i in range(nd - 1, -1, -1):
                st[i] = acc
                acc *= int(shapes[i])
            strides = st
        if len(strides) != nd or any(int(s) <= 0 for s in strides):
            raise ValueError("strides must be positive, one per dim")
        t = cls()
        total = 1
        for s in shapes:
            total *= int(s)
        last = sum((int(n) - 1) * int(s) for n, s in zip(shapes, strides) if int(n) > 0)
        extent = last + 1 if total else 0
        t.buffer.addr = int(data)
        t.buffer.size = extent * get_element_size(dtype)
        t.owner_task_id = 0xFFFFFFFFFFFFFFFF  # PTO2TaskId::invalid()
        t.start_offset = 0
        t.ndims = nd
        t.dtype = int(dtype)
        t.address_space = int(AddressSpace.DEVICE if child_memory else AddressSpace.HOST)
        for i in range(nd):
            t.shapes[i] = int(shapes[i])
            t.strides[i] = int(strides[i])
        row_major, acc = True, 1
        for i in range(nd - 1, -1, -1):
            if int(shapes[i]) != 1 and int(strides[i]) != acc:
                row_major = False
            acc *= int(shapes[i])
        t.is_contiguous = 1 if row_major else 0
        t.extent_elem_cache = extent
        return t

    def view(self, shapes: Sequence[int], offsets: Sequence[int], manual_dep: bool = False) -> "ChipTensor":
        """Sub-box of this tensor (``ChipTensor::view``, ``tensor.h:283-312``): same buffer and strides,
        ``start_offset`` advanced by ``offsets`` (elements per dim)."""
        nd = self.ndims
        if len(shapes) != nd or len(offsets) != nd:
            raise ValueError(f"view needs {nd} shapes and offsets")
        for i in range(nd):
            if int(shapes[i]) and int(offsets[i]) + int(shapes[i]) > self.shapes[i]:
                raise ValueError(f"view exceeds dim {i}: {offsets[i]} + {shapes[i]} > {self.shapes[i]}")
        t = ChipTensor()
        ctypes.memmove(ctypes.addressof(t), ctypes.addressof(self), ctypes.sizeof(ChipTensor))
        empty = any(int(s) == 0 for s in shapes)
        for i in range(nd):
            if not empty:
                t.start_offset += int(offsets[i]) * int(self.strides[i])
            t.shapes[i] = int(shapes[i])
        t.manual_dep = 1 if manual_dep else 0
        last = sum((int(shapes[i]) - 1) * int(self.strides[i]) for i in range(nd)) if not empty else -1
        t.extent_elem_cache = last + 1
        row_major, acc = True, 1
        for i in range(nd - 1, -1, -1):
            if int(shapes[i]) != 1 and int(self.strides[i]) != acc:
                row_major = False
            acc *= int(shapes[i])
        t.is_contiguous = 1 if (row_major or empty) else 0
        return t

    @property
    def shape(self) -> tuple[int, ...]:
        return tuple(self.shapes[i] for i in range(self.ndims))

    @property
    def data(self) -> int:
        return int(self.buffer.addr)


assert ctypes.sizeof(ChipTensor) == 128
assert ChipTensor.shapes.offset == 44 and ChipTensor.strides.offset == 72 and ChipTensor.address_space.offset == 43


def make_chip_tensor_arg(tensor) -> ChipTensor:
    """ChipTensor over a contiguous torch tensor (``simpler_setup/torch_interop.py:84-119``).

    CPU tensors become HOST tensors (staged by the runtime); device tensors become
    DEVICE tensors (passed through).
    """
    from .torch_interop import torch_dtype_to_datatype

    if not tensor.is_contiguous():
        raise ValueError("make_chip_tensor_arg requires a contiguous tensor; call tensor.contiguous() first")
    dt = torch_dtype_to_datatype(tensor.dtype)
    return ChipTensor.make(tensor.data_ptr(), tuple(int(s) for s in tensor.shape), dt,
                           child_memory=tensor.device.type != "cpu")


class ChipStorageTaskArgs(ctypes.Structure):
    """Fixed L2 argument POD: 256 tensors then 128 u64 scalars (``task_args.h:185``)."""

    _fields_ = [
        ("tensors_", ChipTensor * CHIP_MAX_TENSOR_ARGS),
        ("scalars_", ctypes.c_uint64 * CHIP_MAX_SCALAR_ARGS),
        ("tensor_count_", ctypes.c_int32),
        ("scalar_count_", ctypes.c_int32),
        ("_pad_tail", ctypes.c_uint8 * 56),  # C++ pads to alignof(ChipTensor) = 64
    ]

    def add_tensor(self, t: ChipTensor) -> None:
        if self.scalar_count_ > 0:
            raise RuntimeError("TaskArgs: cannot add tensor after scalar")
        if self.tensor_count_ >= CHIP_MAX_TENSOR_ARGS:
            raise IndexError("TaskArgs: tensor capacity exceeded")
        self.tensors_[self.tensor_count_] = t
        self.tensor_count_ += 1

    def add_scalar(self, s) -> None:
        if self.scalar_count_ >= CHIP_MAX_SCALAR_ARGS:
            raise IndexError("TaskArgs: scalar capacity exceeded")
        self.scalars_[self.scalar_count_] = scalar_to_uint64(s)
        self.scalar_count_ += 1

    def tensor(self, i: int) -> ChipTensor:
        return self.tensors_[i]

    def scalar(self, i: int) -> int:
        return int(self.scalars_[i])

    def tensor_count(self) -> int:
        return int(self.tensor_count_)

    def scalar_count(self) -> int:
        return int(self.scalar_count_)

    def clear(self) -> None:
        self.tensor_count_ = 0
        self.scalar_count_ = 0


assert ctypes.sizeof(ChipStorageTaskArgs) == 33856


class RuntimeEnv(ctypes.Structure):
    _pack_ = 1
    _fields_ = [
        ("ring_task_window", ctypes.c_uint64 * 4),
        ("ring_heap", ctypes.c_uint64 * 4),
        ("ring_dep_pool", ctypes.c_uint64 * 4),
    ]


class CallConfig(ctypes.Structure):
    """Per-run configuration (``call_config.h:111-144``).

    ``aicpu_thread_num`` and ``runtime_env`` are accepted and inert on HIP; the
    diagnostic flags require ``output_prefix`` exactly as in the reference's
    ``CallConfig::validate``.
    """

    _pack_ = 1
    _fields_ = [
        ("aicpu_thread_num", ctypes.c_int32),
        ("enable_chip_swimlane", ctypes.c_int32),
        ("enable_dump_args", ctypes.c_int32),
        ("enable_pmu", ctypes.c_int32),
        ("enable_dep_gen", ctypes.c_int32),
        ("enable_scope_stats", ctypes.c_int32),
        ("runtime_env", RuntimeEnv),
        ("_output_prefix", ctypes.c_char * 1024),
    ]

    @property
    def output_prefix(self) -> str:
        return self._output_prefix.decode()

    @output_prefix.setter
    def output_prefix(self, v: str) -> None:
        b = v.encode()
        if len(b) >= 1024:
            raise ValueError("output_prefix is limited to 1023 bytes")
        self._output_prefix = b

    def diagnostics_any(self) -> bool:
        return any((self.enable_chip_swimlane, self.enable_dump_args, self.enable_pmu, self.enable_dep_gen,
                    self.enable_scope_stats))

    def validate(self) -> None:
        if self.diagnostics_any() and not self.output_prefix:
            raise ValueError(
                "CallConfig: output_prefix must be set whenever any of enable_chip_swimlane / "
                "enable_dump_args / enable_pmu / enable_dep_gen / enable_scope_stats is enabled"
            )
        for arr, name in ((self.runtime_env.ring_task_window, "ring_task_window"),):
            for v in arr:
                if v and (v < 4 or v > 0x7FFFFFFF or v & (v - 1)):
                    raise ValueError(f"RuntimeEnv: {name} must be a power of 2 in [4, INT32_MAX]")
        for v in self.runtime_env.ring_heap:
            if v and v < 1024:
                raise ValueError("RuntimeEnv: ring_heap must be >= 1024 (bytes per ring)")
        for v in self.runtime_env.ring_dep_pool:
            if v and (v < 4 or v > 0x7FFFFFFF):
                raise ValueError("RuntimeEnv: ring_dep_pool must be in [4, INT32_MAX]")


assert ctypes.sizeof(CallConfig) == 6 * 4 + 12 * 8 + 1024


def scalar_to_uint64(value) -> int:
    """Scalar → u64 bits: Python floats as IEEE fp32 bits, ctypes floats by their width."""
    if isinstance(value, bool):
        return int(value)
    if isinstance(value, float):
        return struct.unpack("<I", struct.pack("<f", value))[0]
    if isinstance(value, ctypes._SimpleCData):
        if isinstance(value, ctypes.c_float):
            return ctypes.c_uint32.from_buffer_copy(value).value
        if isinstance(value, ctypes.c_double):
            return ctypes.c_uint64.from_buffer_copy(value).value
        return int(value.value) & 0xFFFFFFFFFFFFFFFF
    return int(value) & 0xFFFFFFFFFFFFFFFF


def _align_up(v: int, a: int) -> int:
    return (v + a - 1) // a * a


class _CallableBlob:
    """Owns a callable's serialized bytes (the layout the C API reads)."""

    def __init__(self, data: bytes):
        self._buf = ctypes.create_string_buffer(bytes(data), len(data))

    @property
    def buffer(self) -> bytes:
        return self._buf.raw

    def address(self) -> int:
        return ctypes.addressof(self._buf)

    def __len__(self) -> int:
        return len(self._buf.raw)


class CoreCallable(_CallableBlob):
    """Leaf callable ``Callable<void, 32, 0>`` (``callable.h:58-95``; factory ``:181-207``)."""

    HEADER = 144
    BINARY_OFFSET = 192  # align_up(144, 64)

    @classmethod
    def build(cls, signature: Sequence[ArgDirection], binary: bytes = b"") -> "CoreCallable":
        sig = [int(s) for s in signature]
        if len(sig) > CORE_MAX_TENSOR_ARGS:
            raise ValueError("make_callable: requested tensor count exceeds supported tensor count 32")
        buf = bytearray(cls.BINARY_OFFSET + len(binary))
        struct.pack_into(f"<{len(sig)}i", buf, 0, *sig)
        struct.pack_into("<iIQ", buf, 128, len(sig), len(binary), 0)
        buf[cls.BINARY_OFFSET :] = binary
        obj = cls(bytes(buf))
        obj.signature = sig
        return obj


class ChipCallable(_CallableBlob):
    """Parent callable ``Callable<CoreCallable, 256, 1024>`` (``callable.h:103-163``; factory ``:213-289``)."""

    STORAGE_OFFSET = 9376  # align_up(9364, 16)

    @classmethod
    def build(
        cls,
        signature: Sequence[ArgDirection],
        func_name: str,
        binary: bytes,
        children: Sequence[tuple[int, CoreCallable]],
        config_name: str = "",
    ) -> "ChipCallable":
        sig = [int(s) for s in signature]
        if len(sig) > CHIP_MAX_TENSOR_ARGS:
            raise ValueError("make_callable: requested tensor count exceeds supported tensor count 256")
        if len(children) > CHIP_MAX_CHILDREN:
            raise ValueError("make_callable: child_count exceeds MaxChildren")
        offset = len(binary)
        offsets = []
        for _, child in children:
            offset = _align_up(offset, CALLABLE_ALIGN)
            offsets.append(offset)
            offset += len(child)
        buf = bytearray(cls.STORAGE_OFFSET + offset)
        struct.pack_into(f"<{len(sig)}i", buf, 0, *sig)
        struct.pack_into("<iI", buf, 1024, len(sig), len(binary))
        name = func_name.encode()[: CALLABLE_FUNC_NAME_MAX - 1]
        buf[1032 : 1032 + len(name)] = name
        struct.pack_into("<I", buf, 1096, len(name))
        for i, ((fid, _), off) in enumerate(zip(children, offsets)):
            struct.pack_into("<i", buf, 1100 + 4 * i, int(fid))
            struct.pack_into("<I", buf, 5196 + 4 * i, off)
        struct.pack_into("<i", buf, 9292, len(children))
        cname = config_name.encode()[: CALLABLE_FUNC_NAME_MAX - 1]
        buf[9296 : 9296 + len(cname)] = cname
        struct.pack_into("<I", buf, 9360, len(cname))
        buf[cls.STORAGE_OFFSET : cls.STORAGE_OFFSET + len(binary)] = binary
        for (_, child), off in zip(children, offsets):
            start = cls.STORAGE_OFFSET + off
            buf[start : start + len(child)] = child.buffer
        obj = cls(bytes(buf))
        obj.signature = sig
        obj.func_name = func_name
        obj.children = list(children)
        return obj


class CallableHandle:
    """Opaque handle returned by ``register_callable`` / ``Worker.register``."""

    def __init__(self, handle_id: int, slot_id: int):
        self._handle_id = handle_id
        self.slot_id = slot_id

    def __repr__(self) -> str:
        return f"CallableHandle(id={self._handle_id}, slot={self.slot_id})"


class ChipWorker:
    """L2 chip worker over ``libsimpler_hip.so`` (reference ``task_interface.py:1240-1519``).

    ``init(device_id, bins=None)``: on HIP there are no AICPU/AICore binaries; a
    ``bins`` object is accepted and ignored. ``register_callable`` returns a handle;
    ``run(handle, args, config)`` executes synchronously. Runtime errors raise
    ``RuntimeError`` with the negative code, as the reference's binding does.
    """

    def __init__(self) -> None:
        from . import _lib

        self._lib = _lib.lib()
        self._ctx = None
        self._device_id = -1
        self._lock = threading.Lock()
        self._slots: dict[int, ChipCallable] = {}
        self._handles: dict[int, int] = {}
        self._next_handle = 0
        size = int(self._lib.get_runtime_size())
        align = int(self._lib.get_runtime_alignment())
        self._runtime_size = size
        self._runtime_raw = ctypes.create_string_buffer(size + align)
        base = ctypes.addressof(self._runtime_raw)
        self._runtime = base + (-base) % align

    # -- lifecycle -------------------------------------------------------------
    def init(self, device_id: int = 0, bins: Any = None, log_level: int | None = None,
             prewarm_config: CallConfig | None = None, enable_sdma: bool = False) -> None:
        del bins, log_level, enable_sdma
        with self._lock:
            if self._ctx is not None:
                raise RuntimeError("ChipWorker is already initialized")
            ctx = self._lib.create_device_context()
            if not ctx:
                raise RuntimeError("create_device_context failed")
            cfg = ctypes.byref(prewarm_config) if prewarm_config is not None else None
            rc = self._lib.simpler_init(ctx, int(device_id), None, 0, None, 0, None, 0, cfg)
            if rc != 0:
                self._lib.destroy_device_context(ctx)
                raise RuntimeError(f"simpler_init(device {device_id}) failed: {rc}")
            self._ctx = ctx
            self._device_id = int(device_id)

    def finalize(self) -> None:
        with self._lock:
            if self._ctx is None:
                return
            self._lib.destroy_device_context(self._ctx)
            self._ctx = None
            self._slots.clear()
            self._handles.clear()

    EXECUTION_MODES = {"fused": 0, "eager": 1, "graph": 2}

    def set_execution(self, mode: str) -> None:
        """How paged-attention callables run from now on (``simpler_hip_set_execution``):
        ``"fused"`` (default) the fused decode kernel; ``"eager"`` / ``"graph"`` the
        reference's QK/SF/PV/UP orchestration on the task-graph backend, launched task by
        task or as one hipGraph."""
        if mode not in self.EXECUTION_MODES:
            raise ValueError(f"execution must be one of {sorted(self.EXECUTION_MODES)}")
        rc = self._lib.simpler_hip_set_execution(self._require(), self.EXECUTION_MODES[mode])
        if rc != 0:
            raise RuntimeError(f"simpler_hip_set_execution failed: {rc}")

    @property
    def initialized(self) -> bool:
        return self._ctx is not None

    @property
    def device_id(self) -> int:
        return self._device_id

    def _require(self):
        if self._ctx is None:
            raise RuntimeError("ChipWorker is not initialized")
        return self._ctx

    # -- callables ---------------------------------------------------------------
    def register_callable(self, callable: ChipCallable) -> CallableHandle:
        ctx = self._require()
        with self._lock:
            slot = next((i for i in range(MAX_REGISTERED_CALLABLE_IDS) if i not in self._slots), None)
            if slot is None:
                raise RuntimeError("callable registry is full (64 ids)")
            rc = self._lib.simpler_register_callable(ctx, slot, callable.address())
            if rc != 0:
                raise RuntimeError(f"simpler_register_callable failed: {rc}")
            self._slots[slot] = callable
            hid = self._next_handle
            self._next_handle += 1
            self._handles[hid] = slot
            return CallableHandle(hid, slot)

    PA_FAMILIES = {0: "chain", 1: "unroll", 2: "spmd", 3: "native", 4: "highperf"}

    def callable_family(self, handle: CallableHandle) -> str | None:
        """Which paged-attention callable family a registration matched
        (``simpler_hip_callable_family``): ``"chain"``, ``"unroll"``, ``"spmd"``,
        ``"native"``, ``"highperf"``, or ``None`` for a callable that is not paged attention."""
        slot = self._handles.get(handle._handle_id)
        if slot is None:
            raise KeyError("unknown callable handle")
        return self.PA_FAMILIES.get(int(self._lib.simpler_hip_callable_family(self._require(), slot)))

    def unregister_callable(self, handle: CallableHandle) -> None:
        ctx = self._require()
        with self._lock:
            slot = self._handles.pop(handle._handle_id, None)
            if slot is None:
                raise KeyError("unknown callable handle")
            if slot not in self._handles.values():
                self._slots.pop(slot, None)
                self._lib.simpler_unregister_callable(ctx, slot)

    def run(self, handle: CallableHandle, args: ChipStorageTaskArgs, config: CallConfig | None = None,
            **kwargs: Any) -> None:
        ctx = self._require()
        cfg = config if config is not None else CallConfig()
        for k, v in kwargs.items():
            setattr(cfg, k, v)
        cfg.validate()
        slot = self._handles.get(handle._handle_id)
        if slot is None:
            raise KeyError("unknown callable handle")
        with self._lock:
            ctypes.memset(self._runtime, 0, self._runtime_size)
            rc = self._lib.simpler_run(ctx, self._runtime, slot, ctypes.addressof(args), ctypes.byref(cfg), None)
        if rc != 0:
            raise RuntimeError(f"simpler_run failed: {rc}")

    # -- device memory -------------------------------------------------------------
    def malloc(self, size: int) -> int:
        p = self._lib.device_malloc_ctx(self._require(), int(size))
        if not p:
            raise MemoryError(f"device_malloc_ctx({size}) failed")
        return int(p)

    def free(self, ptr: int) -> None:
        self._lib.device_free_ctx(self._require(), int(ptr))

    def copy_to(self, dst: int, src: int, size: int) -> None:
        if self._lib.copy_to_device_ctx(self._require(), int(dst), int(src), int(size)) != 0:
            raise RuntimeError("copy_to_device_ctx failed")

    def copy_from(self, dst: int, src: int, size: int) -> None:
        if self._lib.copy_from_device_ctx(self._require(), int(dst), int(src), int(size)) != 0:
            raise RuntimeError("copy_from_device_ctx failed")

    def committed_device_memory(self) -> int:
        return int(self._lib.committed_device_memory_ctx(self._require()))

    def aicpu_dlopen_count(self) -> int:
        return int(self._lib.get_aicpu_dlopen_count(self._require()))

    def host_dlopen_count(self) -> int:
        return int(self._lib.get_host_dlopen_count(self._require()))

    def run_stream_set_create_count(self) -> int:
        return int(self._lib.get_run_stream_set_create_count(self._require()))

    @property
    def pipeline_depth(self) -> int:
        return 1

    def stream(self) -> int:
        """The context's HIP stream (``hipStream_t`` as an int)."""
        return int(self._lib.simpler_hip_context_stream(self._require()) or 0)
