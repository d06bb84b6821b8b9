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
// Host-side argument checks of the chunkwise contract (gate dtypes, strides).
int chunkwise_check(const kda_fwd_args& a);
// ckpt (nullable): fp32 [B, H, ceil(T/32), K, V], the state before each chunk
int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt = nullptr);

// Chunkwise backward (kda_chunkwise_bwd.hip).
bool chunkwise_bwd_supported(int64_t K, int64_t V);
int64_t chunkwise_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V);
int chunkwise_bwd_launch(const kda_bwd_args& a, hipStream_t stream);
// Device address of the static backward scratch buffer (KDA_BWD_SCRATCH_BYTES)
// on the current device; resolved once per device.  KDA_OK or KDA_ERR_LAUNCH.
int chunkwise_bwd_scratch(void** ptr);

}  // namespace kda
