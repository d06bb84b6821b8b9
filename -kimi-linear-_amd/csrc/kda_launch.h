// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "kda_hip.h"

namespace kda {

// Token-by-token recurrence (kda_recurrent.hip).
bool recurrent_supported(int64_t K, int64_t V);
int recurrent_launch(const kda_fwd_args& a, hipStream_t stream);

// Chunkwise forward (kda_chunkwise.hip).
bool chunkwise_supported(int64_t K, int64_t V);
int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream);

}  // namespace kda
