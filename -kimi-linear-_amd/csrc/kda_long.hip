// Chunkwise KDA forward on long sequences split into segments (gfx950).
//
// kda_chunkwise (kimi_linear/kda.py:58-185) runs each (batch, head) as one
// chain of chunks; with few chains and long T most CUs have nothing to do.
// The state map of a segment of tokens is affine in the state entering it:
//   S_end = Phi S_start + S_loc,
// Phi (K x K) the product of the segment's per-chunk transitions
// Diag(E[31]) - (F * K)^T M (E * K), S_loc the segment's state from zero.  So
// with T split into P segments:
//   1. every (b, h, segment) chain in parallel: S_loc and Phi, the latter as
//      K more state columns that start from the identity and see v = 0
//      (chunkwise_kernel in its TRANS form; no outputs);
//   2. per (b, h), the P segments in order: S_start[p] = S, S <- Phi_p S +
//      S_loc_p (long_combine_kernel, fp32), the last S being the result;
//   3. every chain again in parallel from its true S_start: the outputs.
// Twice the producer work and three times the consumer work of one pass, on
// P times as many chains.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int kCombineCols = 16;   // state columns per combine workgroup

// One workgroup per (b, h, 16 state columns), thread r owning state row r:
// S_start[p] = S; S = Phi_p S + S_loc_p for p = 0 .. P - 1; S_out = S.
// seg: [B P, H, K, V + K] fp32 (columns [0, V) S_loc, [V, V + K) Phi);
// sstart: [B P, H, K, V] fp32; s0 (nullable, any dtype) and sout: [B, H, K, V].
template <int K>
__global__ __launch_bounds__(K) void long_combine_kernel(const float* seg, float* sstart, const void* s0, int s0_dtype,
                                                         void* sout, int sout_dtype, int64_t H, int64_t V, int64_t P) {
    __shared__ float S[K][kCombineCols];
    const int r = threadIdx.x;
    const int nct = static_cast<int>(V / kCombineCols);
    const int64_t bh = blockIdx.x / nct, b = bh / H, h = bh % H;
    const int64_t c0 = static_cast<int64_t>(blockIdx.x % nct) * kCombineCols;
    const int64_t VS = V + K;
    float cur[kCombineCols];
#pragma unroll
    for (int j = 0; j < kCombineCols; ++j)
        cur[j] = s0 ? load_elem(s0, (bh * K + r) * V + c0 + j, s0_dtype) : 0.f;
    for (int64_t p = 0; p < P; ++p) {
        const int64_t bp = b * P + p;
        const float* row = seg + ((bp * H + h) * K + r) * VS;
        float* st = sstart + ((bp * H + h) * K + r) * V + c0;
#pragma unroll
        for (int j = 0; j < kCombineCols; j += 4)
            *reinterpret_cast<float4*>(st + j) = float4{cur[j], cur[j + 1], cur[j + 2], cur[j + 3]};
        __syncthreads();                    // the previous step's reads of S are done
#pragma unroll
        for (int j = 0; j < kCombineCols; ++j) S[r][j] = cur[j];
        __syncthreads();
        float acc[kCombineCols];
#pragma unroll
        for (int j = 0; j < kCombineCols; j += 4) {
            const float4 x = *reinterpret_cast<const float4*>(row + c0 + j);
            acc[j] = x.x; acc[j + 1] = x.y; acc[j + 2] = x.z; acc[j + 3] = x.w;
        }
        for (int k = 0; k < K; k += 4) {
            const float4 t = *reinterpret_cast<const float4*>(row + V + k);     // Phi[r][k .. k + 3]
            const float tk[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int j = 0; j < kCombineCols; ++j) acc[j] = fmaf(tk[u], S[k + u][j], acc[j]);
        }
#pragma unroll
        for (int j = 0; j < kCombineCols; ++j) cur[j] = acc[j];
    }
#pragma unroll
    for (int j = 0; j < kCombineCols; ++j) store_elem(sout, (bh * K + r) * V + c0 + j, sout_dtype, cur[j]);
}

// The [B, T, ...] view of a chain input as a [B P, T / P, ...] view: one
// batch stride serves both when the sequences follow each other in memory
// (or there is one sequence).
bool split_strides(int64_t (&st)[3], int64_t B, int64_t T, int64_t P) {
    if (B > 1 && st[0] != T * st[1]) return false;
    st[0] = (T / P) * st[1];
    return true;
}

}  // namespace

int64_t long_workspace_bytes(int64_t B, int64_t H, int64_t K, int64_t V, int64_t P) {
    return 4 * B * P * H * K * (3 * V + K);
}

int long_launch(const kda_fwd_args& a, int64_t P, void* workspace, hipStream_t stream) {
    const int64_t B = a.B, T = a.T, H = a.H, K = a.K, V = a.V;
    kda_fwd_args s = a;
    s.B = B * P;
    s.T = T / P;
    if (!split_strides(s.q_stride, B, T, P) || !split_strides(s.k_stride, B, T, P) ||
        !split_strides(s.v_stride, B, T, P) || !split_strides(s.g_stride, B, T, P) ||
        !split_strides(s.beta_stride, B, T, P))
        return KDA_ERR_UNSUPPORTED;
    float* seg = static_cast<float*>(workspace);
    float* sstart = seg + B * P * H * K * (V + K);
    float* dummy = sstart + B * P * H * K * V;

    // 1. per chain: the state from zero and the transition
    kda_fwd_args a1 = s;
    a1.state_in = nullptr;
    a1.state_out = seg;
    a1.state_out_dtype = KDA_DTYPE_F32;
    a1.o = nullptr;
    int st = chunkwise_trans_launch(a1, stream);
    if (st != KDA_OK) return st;

    // 2. the segments in order
    const int64_t blocks = B * H * (V / kCombineCols);
    if (K == 64)
        hipLaunchKernelGGL((long_combine_kernel<64>), dim3(static_cast<unsigned>(blocks)), dim3(64), 0, stream, seg,
                           sstart, a.state_in, a.state_in_dtype, a.state_out, a.state_out_dtype, H, V, P);
    else
        hipLaunchKernelGGL((long_combine_kernel<128>), dim3(static_cast<unsigned>(blocks)), dim3(128), 0, stream, seg,
                           sstart, a.state_in, a.state_in_dtype, a.state_out, a.state_out_dtype, H, V, P);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;

    // 3. per chain from its true initial state: the outputs (its final state,
    // the next segment's initial one, is not needed again)
    kda_fwd_args a3 = s;
    a3.state_in = sstart;
    a3.state_in_dtype = KDA_DTYPE_F32;
    a3.state_out = dummy;
    a3.state_out_dtype = KDA_DTYPE_F32;
    return chunkwise_launch(a3, stream);
}

}  // namespace kda
