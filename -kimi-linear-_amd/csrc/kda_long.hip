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
//      S_loc_p (long_combine_kernel, fp32 matrix cores), the last S being the result;
//   3. every chain again in parallel from its true S_start: the outputs.
// Twice the producer work and three times the consumer work of one pass, on
// P times as many chains.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int kCombineCols = 16;   // state columns per combine workgroup
constexpr int kCombineThreads = 256;
constexpr int kCombinePad = 20;    // LDS row of the state strip: conflict-free B-operand reads

// One workgroup of four waves per (b, h, 16 state columns):
// S_start[p] = S; S = Phi_p S + S_loc_p for p = 0 .. P - 1; S_out = S.
// The strip S (K x 16) sits in LDS; wave w computes rows 16 (TPW w + t) ..
// + 15 of Phi_p S on the fp32 matrix cores (v_mfma_f32_16x16x4f32, exact
// products): lane (ln, lg) feeds Phi[r0 + ln][16 U + 4 lg + u] (one 16-byte
// load of the row covers u = 0 .. 3) against S[16 U + 4 lg + u][ln].
// seg: [B P, H, K, V + K] fp32 (columns [0, V) S_loc, [V, V + K) Phi);
// sstart: [B P, H, K, V] fp32; s0 (nullable, any dtype) and sout: [B, H, K, V].
template <int K>
__global__ __launch_bounds__(kCombineThreads) void long_combine_kernel(const float* seg, float* sstart,
                                                                       const void* s0, int s0_dtype, void* sout,
                                                                       int sout_dtype, int64_t B, int64_t H,
                                                                       int64_t V, int64_t P) {
    static_assert(K == 64 || K == 128, "the split path takes K in {64, 128}");
    constexpr int TPW = K / 64;                     // 16-row tiles per wave
    constexpr int EPT = K * kCombineCols / kCombineThreads;   // strip elements per thread
    __shared__ float S[K][kCombinePad];
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int64_t nct = V / kCombineCols;
    // the strips of one head on one XCD (workgroups go to the eight XCDs
    // round robin), so each Phi_p comes from HBM once
    const int64_t g = blockIdx.x, BH = B * H;
    const bool xcd = BH % 8 == 0;
    const int64_t bh = xcd ? (g / 8 / nct) * 8 + g % 8 : g / nct, b = bh / H, h = bh % H;
    const int64_t c0 = (xcd ? (g / 8) % nct : g % nct) * kCombineCols;
    const int64_t VS = V + K;
#pragma unroll
    for (int m = 0; m < EPT; ++m) {
        const int e = t + kCombineThreads * m, r = e / kCombineCols, j = e % kCombineCols;
        S[r][j] = s0 ? load_elem(s0, (bh * K + r) * V + c0 + j, s0_dtype) : 0.f;
    }
    __syncthreads();
    // segment p + 1's Phi rows and S_loc are fetched while segment p is composed
    f4 ph[TPW][K / 16], sl[TPW];
    auto fetch = [&](int64_t p) {
        const float* base = seg + ((b * P + p) * H + h) * K * VS;
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int r0 = 16 * (TPW * w + tt);
#pragma unroll
            for (int j = 0; j < 4; ++j) sl[tt][j] = base[(r0 + 4 * lg + j) * VS + c0 + ln];
#pragma unroll
            for (int U = 0; U < K / 16; ++U)
                ph[tt][U] = *reinterpret_cast<const f4*>(base + (r0 + ln) * VS + V + 16 * U + 4 * lg);
        }
    };
    if (P > 0) fetch(0);
    for (int64_t p = 0; p < P; ++p) {
        const int64_t bp = b * P + p;
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
            const int e = t + kCombineThreads * m, r = e / kCombineCols, j = e % kCombineCols;
            sstart[((bp * H + h) * K + r) * V + c0 + j] = S[r][j];
        }
        f4 acc[TPW];
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            acc[tt] = sl[tt];
#pragma unroll
            for (int U = 0; U < K / 16; ++U)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ph[tt][U][u], S[16 * U + 4 * lg + u][ln], acc[tt],
                                                                   0, 0, 0);
        }
        if (p + 1 < P) fetch(p + 1);
        __syncthreads();                    // every wave's reads of S are done
#pragma unroll
        for (int tt = 0; tt < TPW; ++tt) {
            const int r0 = 16 * (TPW * w + tt);
#pragma unroll
            for (int j = 0; j < 4; ++j) S[r0 + 4 * lg + j][ln] = acc[tt][j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int m = 0; m < EPT; ++m) {
        const int e = t + kCombineThreads * m, r = e / kCombineCols, j = e % kCombineCols;
        store_elem(sout, (bh * K + r) * V + c0 + j, sout_dtype, S[r][j]);
    }
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
    return 4 * B * P * H * K * (2 * V + K);
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
        hipLaunchKernelGGL((long_combine_kernel<64>), dim3(static_cast<unsigned>(blocks)), dim3(kCombineThreads), 0,
                           stream, seg, sstart, a.state_in, a.state_in_dtype, a.state_out, a.state_out_dtype, B, H, V, P);
    else
        hipLaunchKernelGGL((long_combine_kernel<128>), dim3(static_cast<unsigned>(blocks)), dim3(kCombineThreads), 0,
                           stream, seg, sstart, a.state_in, a.state_in_dtype, a.state_out, a.state_out_dtype, B, H, V, P);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;

    // 3. per chain from its true initial state: the outputs only (its final
    // state, the next segment's initial one, is known already: no state_out)
    kda_fwd_args a3 = s;
    a3.state_in = sstart;
    a3.state_in_dtype = KDA_DTYPE_F32;
    a3.state_out = nullptr;
    a3.state_out_dtype = KDA_DTYPE_F32;
    return chunkwise_launch(a3, stream);
}

}  // namespace kda
