/*
 * simpler_hip — byte-exact mirrors of simpler's task-interface PODs.
 *
 * libsimpler_hip.so receives these exactly as simpler's ChipWorker hands them
 * to a host runtime through the C API, so every size and field offset below
 * matches the reference and is pinned by a static assertion:
 *
 *   SimplerChipTensor          <- ChipTensor            src/common/task_interface/tensor.h:95-113,489-500
 *   SimplerChipStorageTaskArgs <- ChipStorageTaskArgs   src/common/task_interface/task_args.h:85-117,185
 *   SimplerCallConfig          <- CallConfig/RuntimeEnv src/common/task_interface/call_config.h:56-150
 *   SimplerCoreCallableHeader  <- CoreCallable          src/common/task_interface/callable.h:58-95,157
 *   SimplerChipCallableHeader  <- ChipCallable          src/common/task_interface/callable.h:103-163
 *   SimplerDataType codes      <- DataType              src/common/task_interface/data_type.h:47-67
 *   SimplerArgDirection codes  <- ArgDirection          src/common/task_interface/arg_direction.h:22-37,54
 *
 * Plain C (C11 or C++11 and later).
 */
#ifndef SIMPLER_HIP_ABI_TYPES_H
#define SIMPLER_HIP_ABI_TYPES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#define SIMPLER_STATIC_ASSERT(c, m) static_assert(c, m)
#define SIMPLER_ALIGNAS(n) alignas(n)
extern "C" {
#else
#define SIMPLER_STATIC_ASSERT(c, m) _Static_assert(c, m)
#define SIMPLER_ALIGNAS(n) _Alignas(n)
#endif

#define SIMPLER_MAX_TENSOR_DIMS 5
#define SIMPLER_CORE_MAX_TENSOR_ARGS 32
#define SIMPLER_CHIP_MAX_TENSOR_ARGS 256
#define SIMPLER_CORE_MAX_SCALAR_ARGS 16
#define SIMPLER_CHIP_MAX_SCALAR_ARGS 128
#define SIMPLER_CALLABLE_ALIGN 64
#define SIMPLER_CALLABLE_CHILD_ALIGN 16
#define SIMPLER_CALLABLE_FUNC_NAME_MAX 64
#define SIMPLER_CHIP_MAX_CHILDREN 1024
#define SIMPLER_RUNTIME_ENV_RING_COUNT 4

typedef enum SimplerDataType {
    SIMPLER_DT_FLOAT32 = 0,
    SIMPLER_DT_FLOAT16 = 1,
    SIMPLER_DT_INT32 = 2,
    SIMPLER_DT_INT16 = 3,
    SIMPLER_DT_INT8 = 4,
    SIMPLER_DT_UINT8 = 5,
    SIMPLER_DT_BFLOAT16 = 6,
    SIMPLER_DT_INT64 = 7,
    SIMPLER_DT_UINT64 = 8,
    SIMPLER_DT_UINT16 = 9,
    SIMPLER_DT_UINT32 = 10,
    SIMPLER_DT_BOOL = 11,
    SIMPLER_DT_FP8E4M3FN = 12,
    SIMPLER_DT_FP8E8M0 = 13,
    SIMPLER_DT_FP4E2M1 = 14,
    SIMPLER_DT_NUM = 15
} SimplerDataType;

typedef enum SimplerArgDirection {
    SIMPLER_ARG_SCALAR = 0,
    SIMPLER_ARG_IN = 1,
    SIMPLER_ARG_OUT = 2,
    SIMPLER_ARG_INOUT = 3
} SimplerArgDirection;

typedef enum SimplerAddressSpace { SIMPLER_ADDR_HOST = 0, SIMPLER_ADDR_DEVICE = 1 } SimplerAddressSpace;

/* Element size of a DataType code (0 for unknown), data_type.h:80-99. */
static inline uint64_t simpler_dtype_size(uint8_t dt) {
    static const uint8_t sz[SIMPLER_DT_NUM] = {4, 2, 4, 2, 1, 1, 2, 8, 8, 2, 4, 1, 1, 1, 1};
    return dt < SIMPLER_DT_NUM ? sz[dt] : 0;
}

typedef struct SimplerBufferHandle {
    uint64_t addr; /* bytes */
    uint64_t size; /* bytes */
} SimplerBufferHandle;

typedef struct SIMPLER_ALIGNAS(64) SimplerChipTensor {
    SimplerBufferHandle buffer;                 /* 0  */
    uint64_t owner_task_id;                     /* 16 */
    uint64_t start_offset;                      /* 24: elements */
    int32_t version;                            /* 32 */
    uint32_t ndims;                             /* 36 */
    uint8_t dtype;                              /* 40: SimplerDataType */
    uint8_t manual_dep;                         /* 41: bool */
    uint8_t is_contiguous;                      /* 42: bool */
    uint8_t address_space;                      /* 43: SimplerAddressSpace */
    uint32_t shapes[SIMPLER_MAX_TENSOR_DIMS];   /* 44 */
    uint64_t extent_elem_cache;                 /* 64 */
    uint32_t strides[SIMPLER_MAX_TENSOR_DIMS];  /* 72: elements, > 0 */
    uint8_t _pad_cl2[36];                       /* 92 */
} SimplerChipTensor;

SIMPLER_STATIC_ASSERT(sizeof(SimplerChipTensor) == 128, "ChipTensor is 128 bytes");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, owner_task_id) == 16, "owner_task_id @16");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, start_offset) == 24, "start_offset @24");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, version) == 32, "version @32");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, ndims) == 36, "ndims @36");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, dtype) == 40, "dtype @40");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, manual_dep) == 41, "manual_dep @41");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, is_contiguous) == 42, "is_contiguous @42");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, address_space) == 43, "address_space @43");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, shapes) == 44, "shapes @44");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, extent_elem_cache) == 64, "extent_elem_cache @64");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipTensor, strides) == 72, "strides @72");

/* TaskArgsTpl<ChipTensor, uint64_t, 256, 128> with an empty tag mixin. */
typedef struct SimplerChipStorageTaskArgs {
    SimplerChipTensor tensors_[SIMPLER_CHIP_MAX_TENSOR_ARGS];
    uint64_t scalars_[SIMPLER_CHIP_MAX_SCALAR_ARGS];
    int32_t tensor_count_;
    int32_t scalar_count_;
} SimplerChipStorageTaskArgs;

SIMPLER_STATIC_ASSERT(offsetof(SimplerChipStorageTaskArgs, scalars_) == 256 * 128, "scalars_ after tensors_");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipStorageTaskArgs, tensor_count_) == 256 * 128 + 128 * 8, "counts");
SIMPLER_STATIC_ASSERT(sizeof(SimplerChipStorageTaskArgs) == 33856, "ChipStorageTaskArgs size");

#pragma pack(push, 1)
typedef struct SimplerRuntimeEnv {
    uint64_t ring_task_window[SIMPLER_RUNTIME_ENV_RING_COUNT];
    uint64_t ring_heap[SIMPLER_RUNTIME_ENV_RING_COUNT];
    uint64_t ring_dep_pool[SIMPLER_RUNTIME_ENV_RING_COUNT];
} SimplerRuntimeEnv;

typedef struct SimplerCallConfig {
    int32_t aicpu_thread_num;
    int32_t enable_chip_swimlane;
    int32_t enable_dump_args;
    int32_t enable_pmu;
    int32_t enable_dep_gen;
    int32_t enable_scope_stats;
    SimplerRuntimeEnv runtime_env;
    char output_prefix[1024];
} SimplerCallConfig;
#pragma pack(pop)

SIMPLER_STATIC_ASSERT(sizeof(SimplerRuntimeEnv) == 12 * 8, "RuntimeEnv wire layout");
SIMPLER_STATIC_ASSERT(sizeof(SimplerCallConfig) == 6 * 4 + 12 * 8 + 1024, "CallConfig wire layout");

/* CoreCallable = Callable<void, 32, 0>: fixed header, binary at the next
 * 64-byte boundary (binary_data_offset). */
typedef struct SimplerCoreCallableHeader {
    int32_t signature_[SIMPLER_CORE_MAX_TENSOR_ARGS];
    int32_t sig_count_;
    uint32_t binary_size_;
    uint64_t resolved_addr_;
} SimplerCoreCallableHeader;

SIMPLER_STATIC_ASSERT(sizeof(SimplerCoreCallableHeader) == 144, "CoreCallable header size");
#define SIMPLER_CORE_CALLABLE_BINARY_OFFSET 192 /* align_up(144, 64) */

/* ChipCallable = Callable<CoreCallable, 256, 1024>: header, then storage_
 * (16-byte aligned) holding the orchestration binary followed by the
 * children at 64-byte aligned offsets (child_offsets_ are storage-relative). */
typedef struct SimplerChipCallableHeader {
    int32_t signature_[SIMPLER_CHIP_MAX_TENSOR_ARGS];
    int32_t sig_count_;
    uint32_t binary_size_;
    char func_name_[SIMPLER_CALLABLE_FUNC_NAME_MAX];
    uint32_t func_name_len_;
    int32_t child_func_ids_[SIMPLER_CHIP_MAX_CHILDREN];
    uint32_t child_offsets_[SIMPLER_CHIP_MAX_CHILDREN];
    int32_t child_count_;
    char config_name_[SIMPLER_CALLABLE_FUNC_NAME_MAX];
    uint32_t config_name_len_;
} SimplerChipCallableHeader;

SIMPLER_STATIC_ASSERT(offsetof(SimplerChipCallableHeader, func_name_) == 1032, "func_name_ @1032");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipCallableHeader, child_func_ids_) == 1100, "child_func_ids_ @1100");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipCallableHeader, child_count_) == 9292, "child_count_ @9292");
SIMPLER_STATIC_ASSERT(offsetof(SimplerChipCallableHeader, config_name_len_) == 9360, "config_name_len_ @9360");
#define SIMPLER_CHIP_CALLABLE_STORAGE_OFFSET 9376 /* align_up(9364, 16) */

#ifdef __cplusplus
}
#endif

#endif /* SIMPLER_HIP_ABI_TYPES_H */
