"""Task-graph backend: simpler's orchestration API over ``libsimpler_hip.so``.

An orchestration written against simpler's ``pto_orchestration_api.h`` maps
onto this module name for name (``src/a2a3/runtime/tensormap_and_ringbuffer/
orchestration/pto_orchestration_api.h:120-386``; argument builder
``runtime/pto_types.h:374-398``)::

    reference (C++)                       here (Python)
    TensorCreateInfo(shapes, n, dtype)    TensorCreateInfo(shapes, dtype)
    CoreTaskArgs a; a.add_input(t)        a = CoreTaskArgs(); a.add_input(t)
    a.add_output(ci) / a.add_output(t)    a.add_output(ci) / a.add_output(t)   (OUTPUT / OUTPUT_EXISTING)
    a.add_inout(t); a.add_scalar(x)       a.add_inout(t); a.add_scalar(x)
    rt_submit_aic_task(id, a)             g.rt_submit_aic_task(id, a)
    alloc_tensors(ci, ...)                g.alloc_tensors(ci, ...)
    PTO2_SCOPE() { ... }                  with g.scope(): ...
    get_tensor_data<T>(t, n, idx)         g.get_tensor_data(t, idx, T)
    outs.get_ref(i)                       outs.get_ref(i)

Dependencies are inferred by the native runtime (creator edges, TensorMap
overlap of INPUT/INOUT against earlier INOUT/OUTPUT_EXISTING writers,
explicit dependencies); tasks run as built-in gfx950 incore kernels bound to
func ids with :meth:`TaskGraph.bind`. ``mode="eager"`` launches each task at
submit, ``"graph"`` records a hipGraph launched by :meth:`TaskGraph.launch`,
``"record"`` only computes the DAG (no device needed).
"""

from __future__ import annotations

import contextlib
import ctypes
import os
import struct
from enum import IntEnum
from typing import Iterable, Sequence

from . import _lib
from .task_interface import ChipTensor, DataType, TensorArgType, get_element_size, scalar_to_uint64

TASK_INVALID = 0xFFFFFFFFFFFFFFFF  # PTO2TaskId::invalid()
MAX_TENSOR_ARGS = 32  # CoreTaskArgs capacity (SIMPLER_CORE_MAX_TENSOR_ARGS)
MAX_SCALAR_ARGS = 16


class IncoreKernel(IntEnum):
    """Built-in kernels (``include/simpler_hip/task_graph.h``)."""

    QK_MATMUL = 0
    SOFTMAX_PREPARE = 1
    PV_MATMUL = 2
    ONLINE_UPDATE = 3
    VEC_ADD = 16
    VEC_ADD_SCALAR = 17
    VEC_MUL = 18
    ZERO_FILL = 19


_MODES = {"eager": 0, "graph": 1, "record": 2}


class TaskGraphError(RuntimeError):
    def __init__(self, rc: int, what: str):
        super().__init__(f"{what} failed with {rc}")
        self.rc = rc


def TensorCreateInfo(shapes: Sequence[int], dtype: DataType) -> ChipTensor:  # noqa: N802 — reference name
    """Shape and dtype of a runtime-allocated output (``TensorCreateInfo``)."""
    return ChipTensor.make(0, tuple(int(s) for s in shapes), dtype)


class CoreTaskArgs:
    """Tagged tensors and scalars of one task, in the order the kernel reads them."""

    def __init__(self) -> None:
        self.tensors: list[ChipTensor] = []
        self.tags: list[int] = []
        self.scalars: list[int] = []
        self.deps: list[int] = []

    def _add(self, t: ChipTensor, tag: TensorArgType) -> None:
        if len(self.tensors) >= MAX_TENSOR_ARGS:
            raise ValueError(f"at most {MAX_TENSOR_ARGS} tensors per task")
        self.tensors.append(t)
        self.tags.append(int(tag))

    def add_input(self, *ts: ChipTensor) -> None:
        for t in ts:
            self._add(t, TensorArgType.INPUT)

    def add_output(self, *ts: ChipTensor) -> None:
        """A create info (no buffer) becomes OUTPUT; an existing tensor OUTPUT_EXISTING."""
        for t in ts:
            self._add(t, TensorArgType.OUTPUT if t.buffer.addr == 0 else TensorArgType.OUTPUT_EXISTING)

    def add_inout(self, *ts: ChipTensor) -> None:
        for t in ts:
            self._add(t, TensorArgType.INOUT)

    def add_no_dep(self, *ts: ChipTensor) -> None:
        for t in ts:
            self._add(t, TensorArgType.NO_DEP)

    def add_scalar(self, *vals) -> None:
        for v in vals:
            if len(self.scalars) >= MAX_SCALAR_ARGS:
                raise ValueError(f"at most {MAX_SCALAR_ARGS} scalars per task")
            self.scalars.append(scalar_to_uint64(v))

    def set_dependencies(self, task_ids: Iterable[int]) -> None:
        self.deps = [int(t) for t in task_ids]


class TaskOutputTensors:
    """The runtime-created outputs of a submitted task, in ``add_output`` order."""

    def __init__(self, task_id: int, outputs: list[ChipTensor]):
        self._task_id = task_id
        self._outs = outputs

    def task_id(self) -> int:
        return self._task_id

    def get_ref(self, i: int) -> ChipTensor:
        return self._outs[i]

    def size(self) -> int:
        return len(self._outs)


class TaskGraph:
    """One task graph on the current HIP device (or none, in ``record`` mode)."""

    def __init__(self, mode: str = "eager", stream: int | None = None):
        if mode not in _MODES:
            raise ValueError(f"mode must be one of {sorted(_MODES)}")
        self._lib = _lib.lib()
        if stream is None and mode != "record":
            import torch

            stream = torch.cuda.current_stream().cuda_stream
        self.mode = mode
        self._g = self._lib.simpler_hip_tg_create(_MODES[mode], stream or None)
        if not self._g:
            raise TaskGraphError(-1, "simpler_hip_tg_create")

    # -- lifetime -------------------------------------------------------------
    def close(self) -> None:
        if self._g:
            self._lib.simpler_hip_tg_destroy(self._g)
            self._g = None

    def __enter__(self) -> "TaskGraph":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str) -> int:
        if rc < 0:
            raise TaskGraphError(rc, what)
        return rc

    # -- orchestration API ------------------------------------------------------
    def bind(self, func_id: int, kernel: IncoreKernel) -> None:
        self._check(self._lib.simpler_hip_tg_bind(self._g, int(func_id), int(kernel)), "bind")

    def register_kernel(self, func_id: int, code_object: str | os.PathLike, kernel_name: str, *,
                        block_threads: int = 256, grid_tensor: int = 0, elems_per_workgroup: int = 256) -> None:
        """Bind ``func_id`` to ``extern "C"`` kernel ``kernel_name`` of a gfx950 code
        object (``hipcc --genco``; :func:`simpler_amd.build.build_code_object`). The
        kernel takes one ``SimplerHipKernelArgs`` (``include/simpler_hip/task_graph.h``):
        the task's tensors, then its scalars. Each task launches ``block_threads``
        threads per workgroup and ``ceil(numel(tensor grid_tensor) /
        elems_per_workgroup)`` workgroups (``elems_per_workgroup`` of them when
        ``grid_tensor`` < 0)."""
        rc = self._lib.simpler_hip_tg_register_kernel(self._g, int(func_id), os.fsencode(os.fspath(code_object)),
                                                      kernel_name.encode(), int(block_threads), int(grid_tensor),
                                                      int(elems_per_workgroup))
        self._check(rc, f"register_kernel({kernel_name})")

    def record_replay(self, key: bytes) -> None:
        """GRAPH mode: keep the step submitted since the last reset under ``key``."""
        buf = ctypes.create_string_buffer(bytes(key), max(len(key), 1))
        self._check(self._lib.simpler_hip_tg_record_replay(self._g, buf, len(key)), "record_replay")

    def replay(self, key: bytes) -> bool:
        """GRAPH mode, on a reset graph: restore the step recorded under ``key``
        (True), so that :meth:`launch` runs it without its tasks being submitted
        again; False if ``key`` is not the recorded one."""
        buf = ctypes.create_string_buffer(bytes(key), max(len(key), 1))
        return self._check(self._lib.simpler_hip_tg_replay(self._g, buf, len(key)), "replay") == 1

    def scope_begin(self) -> None:
        self._check(self._lib.simpler_hip_tg_scope_begin(self._g), "scope_begin")

    def scope_end(self) -> None:
        self._check(self._lib.simpler_hip_tg_scope_end(self._g), "scope_end")

    @contextlib.contextmanager
    def scope(self):
        """``PTO2_SCOPE()``: tensors allocated inside are released at the end."""
        self.scope_begin()
        try:
            yield
        finally:
            self.scope_end()

    def submit_task(self, func_id: int, args: CoreTaskArgs) -> TaskOutputTensors:
        n = len(args.tensors)
        arr = (ChipTensor * max(n, 1))(*args.tensors)
        outs = (ChipTensor * max(n, 1))()
        tags = (ctypes.c_int32 * max(n, 1))(*args.tags)
        sc = (ctypes.c_uint64 * max(len(args.scalars), 1))(*args.scalars)
        deps = (ctypes.c_uint64 * max(len(args.deps), 1))(*args.deps)
        tid = self._lib.simpler_hip_tg_submit(self._g, int(func_id), ctypes.addressof(arr), tags, n, sc,
                                              len(args.scalars), deps, len(args.deps), ctypes.addressof(outs))
        self._check(tid, f"submit(func_id={func_id})")
        created = [outs[i] for i in range(n) if args.tags[i] == TensorArgType.OUTPUT]
        return TaskOutputTensors(tid, created)

    def rt_submit_aic_task(self, kernel_id: int, args: CoreTaskArgs) -> TaskOutputTensors:
        return self.submit_task(kernel_id, args)

    def rt_submit_aiv_task(self, kernel_id: int, args: CoreTaskArgs) -> TaskOutputTensors:
        return self.submit_task(kernel_id, args)

    def rt_submit_dummy_task(self, args: CoreTaskArgs) -> TaskOutputTensors:
        return self.submit_task(-1, args)

    def alloc_tensors(self, *create_infos: ChipTensor) -> TaskOutputTensors:
        a = CoreTaskArgs()
        for ci in create_infos:
            a._add(ci, TensorArgType.OUTPUT)
        return self.submit_task(-1, a)

    def get_tensor_data(self, t: ChipTensor, indices: Sequence[int], dtype: str = "raw"):
        """One element (waits for its producers). ``dtype`` "raw" (u64 bits), "int", "float"."""
        idx = (ctypes.c_uint32 * max(len(indices), 1))(*[int(i) for i in indices])
        v = ctypes.c_uint64()
        self._check(self._lib.simpler_hip_tg_get_tensor_data(self._g, ctypes.addressof(t), len(indices), idx,
                                                             ctypes.byref(v)), "get_tensor_data")
        raw = v.value
        if dtype == "raw":
            return raw
        size = get_element_size(DataType(int(t.dtype)))
        if dtype == "int":
            bits = raw & ((1 << (8 * size)) - 1)
            return bits - (1 << (8 * size)) if bits >> (8 * size - 1) else bits
        if dtype == "float":
            if int(t.dtype) == DataType.BFLOAT16:
                return struct.unpack("<f", struct.pack("<I", (raw & 0xFFFF) << 16))[0]
            return struct.unpack("<f", struct.pack("<I", raw & 0xFFFFFFFF))[0]
        raise ValueError("dtype must be raw, int or float")

    def read(self, t: ChipTensor):
        """A tensor's elements as a numpy array (after its producers finish). Dense views only."""
        import numpy as np

        np_dtype = {DataType.FLOAT32: np.float32, DataType.INT32: np.int32, DataType.BFLOAT16: np.uint16,
                    DataType.FLOAT16: np.float16, DataType.UINT8: np.uint8, DataType.INT8: np.int8}[DataType(t.dtype)]
        if not t.is_contiguous:
            raise ValueError("read() needs a dense (row-major) view")
        out = np.empty(t.shape, dtype=np_dtype)
        self._check(self._lib.simpler_hip_tg_copy_to_host(self._g, ctypes.addressof(t), out.ctypes.data,
                                                          out.nbytes), "copy_to_host")
        if DataType(t.dtype) == DataType.BFLOAT16:
            return (out.astype(np.uint32) << 16).view(np.float32)
        return out

    # -- execution --------------------------------------------------------------
    def launch(self) -> None:
        self._check(self._lib.simpler_hip_tg_launch(self._g), "launch")

    def wait(self) -> None:
        self._check(self._lib.simpler_hip_tg_wait(self._g), "wait")

    def reset(self) -> None:
        self._check(self._lib.simpler_hip_tg_reset(self._g), "reset")

    # -- the reference examples' orchestrations (native) -------------------------
    def orchestrate_paged_attention(self, tensors: Sequence[ChipTensor], scale: float) -> None:
        arr = (ChipTensor * 6)(*tensors)
        self._check(self._lib.simpler_hip_tg_orchestrate_paged_attention(self._g, ctypes.addressof(arr),
                                                                          scalar_to_uint64(float(scale))),
                    "orchestrate_paged_attention")

    def orchestrate_vector_example(self, tensors: Sequence[ChipTensor]) -> None:
        arr = (ChipTensor * 3)(*tensors)
        self._check(self._lib.simpler_hip_tg_orchestrate_vector_example(self._g, ctypes.addressof(arr)),
                    "orchestrate_vector_example")

    # -- inspection -------------------------------------------------------------
    @property
    def task_count(self) -> int:
        return int(self._lib.simpler_hip_tg_task_count(self._g))

    @property
    def replay_count(self) -> int:
        """Steps restored by :meth:`replay` (or a native orchestration's own replay)."""
        return int(self._lib.simpler_hip_tg_replay_count(self._g))

    def fanin(self, task: int) -> list[int]:
        cap = 256
        buf = (ctypes.c_int64 * cap)()
        n = self._check(self._lib.simpler_hip_tg_fanin(self._g, int(task), buf, cap), "fanin")
        return [int(buf[i]) for i in range(min(n, cap))]

    @property
    def arena_bytes(self) -> int:
        return int(self._lib.simpler_hip_tg_arena_bytes(self._g))


# The reference vector example's CALLABLE
# (examples/a2a3/tensormap_and_ringbuffer/vector_example/test_vector_example.py:24-49).


def vector_example_callable() -> "ChipCallable":
    """Orchestration [IN, IN, OUT] with kernel_add (0), kernel_add_scalar (1), kernel_mul (2)."""
    from .task_interface import ArgDirection as D, ChipCallable, CoreCallable

    children = [
        (0, CoreCallable.build(signature=[D.IN, D.IN, D.OUT], binary=b"")),
        (1, CoreCallable.build(signature=[D.IN, D.OUT], binary=b"")),
        (2, CoreCallable.build(signature=[D.IN, D.IN, D.OUT], binary=b"")),
    ]
    return ChipCallable.build(signature=[D.IN, D.IN, D.OUT], func_name="aicpu_orchestration_entry", binary=b"",
                              children=children, config_name="aicpu_orchestration_config")
