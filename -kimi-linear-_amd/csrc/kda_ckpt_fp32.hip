// Exact fp32 checkpoints for the chunkwise backward of fp32 activations.
//
// kda_chunkwise_fwd_ckpt with fp32 q, k, v runs the token recurrence, which
// writes o and the final state in fp32 (the reference's fp32 path is fp32
// throughout, kimi_linear/kda.py:116) and, before every 32-token chunk, stores
// the state at the head of that chunk's record (kda_recurrent.hip, CK).
// ckpt_fill_kernel then fills the rest of each record from that state and the
// chunk's inputs, in fp32 and with the pairwise decays formed directly as the
// reference materialises them (kda.py:150-177), each exp(G_c - G_i) <= 1:
//   G = in-chunk cumulative sum of g,  E = exp(G),  q~ = scale q
//   A[c,i] = sum_k q~[c,k] k[i,k] exp(G[c,k] - G[i,k])   (i <= c, else 0)
//   L[c,i] = sum_k  k[c,k] k[i,k] exp(G[c,k] - G[i,k])   (i <  c, else 0)
//   N = (I + Diag(beta) L)^-1,   R = V - (k * E) S
// -- the quantities the pipelined forward records from its fp16 operands, so
// that the backward's gradients of fp32 inputs start from fp32-exact records.
// One workgroup of 256 threads per (b, h, chunk); rows past T are zero rows
// (q = k = v = g = beta = 0), which the backward treats as padding.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int CT = 32;          // tokens per record
constexpr int NT = 256;         // threads per workgroup
constexpr int VC = NT / 2;      // state columns per pass of the R step

template <int K>
struct __align__(16) FillSmem {
    float q[CT][K + 1];         // q~; then k * E for the R step
    float k[CT][K + 1];
    float G[CT][K + 1];         // g, then its in-chunk cumulative sum
    float A[CT][CT + 1];
    float L[CT][CT + 1];
    float N[CT][CT + 1];
    float beta[CT];
};

template <int K>
__global__ __launch_bounds__(NT) void ckpt_fill_kernel(const kda_fwd_args a, float* ckpt) {
    __shared__ FillSmem<K> sm;
    const int64_t H = a.H, T = a.T, V = a.V;
    const int64_t nck = (T + CT - 1) / CT;
    const int64_t cb = blockIdx.x;                       // (b H + h) nck + n
    const int64_t n = cb % nck, bh = cb / nck, b = bh / H, h = bh % H;
    const int64_t t0 = n * CT;
    const int t = threadIdx.x;
    const float* qp = static_cast<const float*>(a.q);
    const float* kp = static_cast<const float*>(a.k);
    const float* vp = static_cast<const float*>(a.v);
    const float* gp = static_cast<const float*>(a.g);
    const float* bp = static_cast<const float*>(a.beta);

    for (int e = t; e < CT * K; e += NT) {
        const int r = e / K, x = e % K;
        const int64_t tok = t0 + r;
        float qv = 0.f, kv = 0.f, gv = 0.f;
        if (tok < T) {
            qv = qp[b * a.q_stride[0] + tok * a.q_stride[1] + h * a.q_stride[2] + x] * a.scale;
            kv = kp[b * a.k_stride[0] + tok * a.k_stride[1] + h * a.k_stride[2] + x];
            gv = gp[b * a.g_stride[0] + tok * a.g_stride[1] + h * a.g_stride[2] + x];
        }
        sm.q[r][x] = qv;
        sm.k[r][x] = kv;
        sm.G[r][x] = gv;
    }
    if (t < CT) {
        const int64_t tok = t0 + t;
        sm.beta[t] = tok < T ? bp[b * a.beta_stride[0] + tok * a.beta_stride[1] + h * a.beta_stride[2]] : 0.f;
    }
    __syncthreads();
    if (t < K) {
        float run = 0.f;
        for (int r = 0; r < CT; ++r) {
            run += sm.G[r][t];
            sm.G[r][t] = run;
        }
    }
    __syncthreads();

    // A and L: thread t takes column i = t % 32 of rows t / 32 + 8 m
    for (int m = 0; m < CT * CT / NT; ++m) {
        const int i = t % CT, c = t / CT + (NT / CT) * m;
        float sa = 0.f, sl = 0.f;
        if (i <= c) {
            for (int x = 0; x < K; ++x) {
                const float ki = sm.k[i][x] * expf(sm.G[c][x] - sm.G[i][x]);
                sa = fmaf(sm.q[c][x], ki, sa);
                sl = fmaf(sm.k[c][x], ki, sl);
            }
        }
        sm.A[c][i] = sa;
        sm.L[c][i] = i < c ? sl : 0.f;
    }
    __syncthreads();
    // N by columns: N[c][j] = delta_cj - beta_c sum_{j <= i < c} L[c][i] N[i][j];
    // meanwhile the other threads turn q~ into k * E for the R step
    if (t < CT) {
        const int j = t;
        for (int c = 0; c < CT; ++c) {
            float s = 0.f;
            for (int i = j; i < c; ++i) s = fmaf(sm.L[c][i], sm.N[i][j], s);
            sm.N[c][j] = c < j ? 0.f : (c == j ? 1.f : -sm.beta[c] * s);
        }
    }
    for (int e = t; e < CT * K; e += NT) {
        const int r = e / K, x = e % K;
        sm.q[r][x] = sm.k[r][x] * expf(sm.G[r][x]);
    }
    __syncthreads();

    float* rec = ckpt + cb * ckpt_record(K, V);
    float* rr = rec + K * V;                 // R [CT][V]
    float* ra = rec + (K + CT) * V;          // A, L, N [CT][CT] each
    for (int e = t; e < CT * CT; e += NT) {
        const int c = e / CT, i = e % CT;
        ra[e] = sm.A[c][i];
        ra[CT * CT + e] = sm.L[c][i];
        ra[2 * CT * CT + e] = sm.N[c][i];
    }

    // R = V - (k * E) S, VC columns a pass: thread (column t % VC, rows
    // 16 (t / VC) .. + 15)
    const float* S = rec;                    // the state before the chunk, [K][V]
    const int col = t % VC, hf = t / VC;
    for (int64_t c0 = 0; c0 < V; c0 += VC) {
        const int64_t c = c0 + col;
        const bool live = c < V;
        float acc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int64_t tok = t0 + 16 * hf + r;
            acc[r] = live && tok < T ? vp[b * a.v_stride[0] + tok * a.v_stride[1] + h * a.v_stride[2] + c] : 0.f;
        }
        if (live) {
            for (int x = 0; x < K; ++x) {
                const float sv = S[static_cast<int64_t>(x) * V + c];
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] = fmaf(-sm.q[16 * hf + r][x], sv, acc[r]);
            }
#pragma unroll
            for (int r = 0; r < 16; ++r) rr[(16 * hf + r) * V + c] = acc[r];
        }
    }
}

}  // namespace

int ckpt_fill_fp32_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt) {
    const int64_t nck = (a.T + CT - 1) / CT;
    const int64_t blocks = a.B * a.H * nck;
    if (blocks == 0) return KDA_OK;
    if (blocks > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    switch (a.K) {
        case 32: hipLaunchKernelGGL(ckpt_fill_kernel<32>, dim3(static_cast<unsigned>(blocks)), dim3(NT), 0, stream, a, ckpt); break;
        case 64: hipLaunchKernelGGL(ckpt_fill_kernel<64>, dim3(static_cast<unsigned>(blocks)), dim3(NT), 0, stream, a, ckpt); break;
        case 128: hipLaunchKernelGGL(ckpt_fill_kernel<128>, dim3(static_cast<unsigned>(blocks)), dim3(NT), 0, stream, a, ckpt); break;
        default: return KDA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

}  // namespace kda
