"""simpler_amd — MI355X-native backend for simpler's paged-attention decode path.

The product is ``simpler_amd/lib/libsimpler_hip.so``: simpler's host-runtime C API
(``include/simpler_hip/pto_runtime_c_api.h``) plus the fused decode entry points
(``include/simpler_hip/pa_decode.h``), backed by hand-written gfx950 HIP kernels.
This package is the Python surface over it (ctypes), shaped like the
reference's ``simpler`` package for the L2 path.
"""

from .task_interface import (  # noqa: F401
    AddressSpace,
    ArgDirection,
    CallableHandle,
    CallConfig,
    ChipCallable,
    ChipStorageTaskArgs,
    ChipTensor,
    ChipWorker,
    CoreCallable,
    DataType,
    TensorArgType,
    make_chip_tensor_arg,
    scalar_to_uint64,
)
from .worker import Buffer, TaskArgs, Worker  # noqa: F401

__all__ = [
    "AddressSpace", "ArgDirection", "Buffer", "CallableHandle", "CallConfig", "ChipCallable",
    "ChipStorageTaskArgs", "ChipTensor", "ChipWorker", "CoreCallable", "DataType", "TaskArgs",
    "TensorArgType", "Worker", "make_chip_tensor_arg", "scalar_to_uint64",
]
