// Library-internal queries on a task graph (shared by task_graph.cpp and
// orchestrations.cpp); the public surface is include/simpler_hip/task_graph.h.
#pragma once

#include <stdint.h>

#include "simpler_hip/task_graph.h"

namespace simpler_hip {

// SimplerHipTaskGraphMode of `g`.
int32_t tg_mode_of(const SimplerHipTaskGraph *g);

// Nothing submitted, allocated or launched since create / reset.
bool tg_is_fresh(const SimplerHipTaskGraph *g);

// Bring the host copies of n external device tensors up to date with one
// stream synchronisation (get_tensor_data then reads them without another).
int tg_prefetch_host(SimplerHipTaskGraph *g, const SimplerChipTensor *tensors, int n);

}  // namespace simpler_hip
