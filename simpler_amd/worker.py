"""``Worker(level=2)`` — the reference's L2 user API on the HIP backend.

Mirrors the L2 slice of ``python/simpler/worker.py``: ``Worker(level=2, ...)``
(``:4308-4330``), ``init`` (``:7415``), ``register`` (``:6423``), ``run`` /
``submit(...).wait()`` (``:10504-10551``), ``malloc`` / ``free`` / ``copy_to`` /
``copy_from`` (``:10051-10245``) and ``close`` (``:11150``). Levels 3 and above
(multi-chip composition) are not part of this backend and raise.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

from .task_interface import (
    CallableHandle,
    CallConfig,
    ChipCallable,
    ChipStorageTaskArgs,
    ChipTensor,
    ChipWorker,
    DataType,
    TensorArgType,
    make_chip_tensor_arg,
)

PLATFORMS = ("mi355x",)


@dataclass
class Buffer:
    """A device allocation owned by an L2 worker (``Worker.malloc``)."""

    base: int
    size: int
    owner_worker_id: int = 0

    def tensor(self, shapes, dtype: DataType, *, strides=None) -> ChipTensor:
        """Name (a view of) this allocation as a DEVICE task-arg tensor."""
        return ChipTensor.make(self.base, tuple(shapes), DataType(dtype), child_memory=True, strides=strides)


class TaskArgs:
    """Ordered tensors (with tags) then scalars; materialised to ``ChipStorageTaskArgs``.

    Tensors may be ``ChipTensor`` values or contiguous torch tensors (CPU tensors are
    staged by the runtime, device tensors pass through).
    """

    def __init__(self) -> None:
        self._tensors: list[tuple[ChipTensor, TensorArgType]] = []
        self._scalars: list[Any] = []

    def add_tensor(self, t, tag: TensorArgType = TensorArgType.INPUT) -> None:
        if self._scalars:
            raise RuntimeError("TaskArgs: cannot add tensor after scalar")
        if not isinstance(t, ChipTensor):
            t = make_chip_tensor_arg(t)
        self._tensors.append((t, TensorArgType(tag)))

    def add_scalar(self, s) -> None:
        self._scalars.append(s)

    def tensor_count(self) -> int:
        return len(self._tensors)

    def scalar_count(self) -> int:
        return len(self._scalars)

    def materialize(self) -> ChipStorageTaskArgs:
        out = ChipStorageTaskArgs()
        for t, _ in self._tensors:
            out.add_tensor(t)
        for s in self._scalars:
            out.add_scalar(s)
        return out


class RunHandle:
    def __init__(self) -> None:
        self._done = True

    def wait(self) -> None:
        return None

    def done(self) -> bool:
        return self._done


class Worker:
    """Unified worker; only ``level=2`` (one GPU) is provided by this backend."""

    def __init__(self, level: int, **config) -> None:
        if level != 2:
            raise NotImplementedError("the HIP backend provides the L2 (single-device) worker only")
        platform = config.get("platform", "mi355x")
        if platform not in PLATFORMS:
            raise ValueError(f"platform {platform!r} is not served by libsimpler_hip.so (use 'mi355x')")
        self.level = level
        self._config = dict(config)
        self._chip: ChipWorker | None = None

    def init(self) -> "Worker":
        if self._chip is not None:
            raise RuntimeError("Worker is already initialized")
        chip = ChipWorker()
        chip.init(int(self._config.get("device_id", 0)))
        if "execution" in self._config:  # "fused" | "eager" | "graph" (ChipWorker.set_execution)
            chip.set_execution(str(self._config["execution"]))
        self._chip = chip
        return self

    def _require(self) -> ChipWorker:
        if self._chip is None:
            raise RuntimeError("Worker.init() has not been called")
        return self._chip

    @property
    def chip_worker(self) -> ChipWorker:
        return self._require()

    def register(self, target: ChipCallable, *, workers=None) -> CallableHandle:
        del workers
        return self._require().register_callable(target)

    def unregister(self, handle: CallableHandle) -> None:
        self._require().unregister_callable(handle)

    def submit(self, callable: CallableHandle, args=None, config: CallConfig | None = None) -> RunHandle:
        chip = self._require()
        if args is None:
            args = ChipStorageTaskArgs()
        elif isinstance(args, TaskArgs):
            args = args.materialize()
        chip.run(callable, args, config if config is not None else CallConfig())
        return RunHandle()

    def run(self, callable: CallableHandle, args=None, config: CallConfig | None = None) -> None:
        self.submit(callable, args=args, config=config).wait()

    def malloc(self, size: int) -> Buffer:
        return Buffer(self._require().malloc(size), int(size))

    def free(self, handle: Buffer) -> None:
        self._require().free(handle.base)

    @staticmethod
    def _host_ptr(obj, writing: bool) -> tuple[int, int]:
        if hasattr(obj, "data_ptr") and hasattr(obj, "element_size"):
            if obj.device.type != "cpu" or not obj.is_contiguous():
                raise ValueError("host side of a copy must be a contiguous CPU tensor")
            return int(obj.data_ptr()), int(obj.numel() * obj.element_size())
        mv = memoryview(obj)
        if writing and mv.readonly:
            raise ValueError("copy_from needs a writable host buffer")
        c = (ctypes.c_char * mv.nbytes).from_buffer(mv) if not mv.readonly else ctypes.create_string_buffer(
            mv.tobytes(), mv.nbytes)
        return ctypes.addressof(c), mv.nbytes

    def copy_to(self, dst: Buffer, src) -> None:
        ptr, n = self._host_ptr(src, writing=False)
        if n > dst.size:
            raise ValueError("copy_to source is larger than the device buffer")
        self._require().copy_to(dst.base, ptr, n)

    def copy_from(self, dst, src: Buffer) -> None:
        ptr, n = self._host_ptr(dst, writing=True)
        if n > src.size:
            raise ValueError("copy_from destination is larger than the device buffer")
        self._require().copy_from(ptr, src.base, n)

    def close(self) -> None:
        if self._chip is not None:
            self._chip.finalize()
            self._chip = None

    def __enter__(self) -> "Worker":
        return self.init() if self._chip is None else self

    def __exit__(self, *exc) -> None:
        self.close()
