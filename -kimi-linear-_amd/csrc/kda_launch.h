// Internal launcher declarations shared by the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "kda_hip.h"

namespace kda {

// Token-by-token recurrence (kda_recurrent.hip).
bool recurrent_supported(int64_t K, int64_t V);
// gate (nullable): the fused gate of kda_recurrent_gated_fwd; ckpt (nullable,
// K <= 128): the chunk records of kda_chunkwise_fwd_ckpt, whose fp32 state
// before every 32-token chunk the recurrence stores
int recurrent_launch(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args* gate = nullptr,
                     float* ckpt = nullptr);

// The rest of the fp32 chunk records (kda_ckpt_fp32.hip): R, A, L and N
// of every 32-token chunk from the state the recurrence stored at the
// record's head and the chunk's fp32 q, k, v, g, beta.
int ckpt_fill_fp32_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt);

// Chunkwise forward (kda_chunkwise.hip).
bool chunkwise_supported(int64_t K, int64_t V);
// Host-side argument checks of the chunkwise contract (gate dtypes, strides);
// `gated`: g and beta hold gk and the beta logits.
int chunkwise_check(const kda_fwd_args& a, bool gated = false);
// ckpt (nullable): fp32 [B, H, ceil(T/32), ckpt_record(K, V)], the checkpoints of the
// backward; gate (nullable): the fused gate of kda_chunkwise_gated_fwd (not
// with ckpt)
int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt = nullptr,
                     const kda_gate_args* gate = nullptr);
// The first pass of a split long sequence (kda_chunkwise_long_fwd): per chain
// the state from zero and the transition, state_out [B, H, K, V + K] fp32;
// with cout, also the outputs in fp32: o [B, T, H, V] from the zero state and
// cout [B, T, H, K] those of the transition columns.
bool chunkwise_trans_supported(const kda_fwd_args& a);
int chunkwise_trans_launch(const kda_fwd_args& a, hipStream_t stream, float* cout = nullptr);
// The chunkwise forward with the layer's output epilogue (kda_chunkwise_fused_fwd).
bool chunkwise_fused_supported(const kda_fwd_args& a);
int chunkwise_fused_launch(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args* gate,
                           const kda_out_epilogue& epi);

// Long sequences split into segments (kda_long.hip): workspace bytes for P
// segments, and the three passes (T % P == 0, checked by the caller).
int64_t long_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t P);
int long_launch(const kda_fwd_args& a, int64_t P, void* workspace, hipStream_t stream);

// Chunkwise backward (kda_chunkwise_bwd.hip).
bool chunkwise_bwd_supported(int64_t K, int64_t V);
int64_t chunkwise_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V);
int chunkwise_bwd_launch(const kda_bwd_args& a, hipStream_t stream);
// Device address of the static backward scratch buffer (KDA_BWD_SCRATCH_BYTES)
// on the current device; resolved once per device.  KDA_OK or KDA_ERR_LAUNCH.
int chunkwise_bwd_scratch(void** ptr);

}  // namespace kda
