// Chunkwise KDA forward for gfx950: fp16 MFMA, fp32 accumulation, fp32 state.
//
// Replaces the body of kda_chunkwise (kimi_linear/kda.py:111-185).  The maths
// is the same UT-transform form (paper Eq. 6-9), evaluated per internal chunk
// of BT = 16 tokens; because the recurrence is chunk-size invariant the
// caller's chunk_size only fixes the T % chunk_size == 0 contract.
//
// Per (b, h) and internal chunk (rows c, i in [0, 16)), with a_t = exp(g_t):
//   E[r]   = prod_{t<=r} a_t              (= exp(gc_r), per channel)
//   L[c,i] = beta_c <k_c, k_i * prod_{t=i+1..c} a_t>,  i < c
//   A[c,i] = scale <q_c, k_i * prod_{t=i+1..c} a_t>,   i <= c
//   M      = (I + L)^-1 Diag(beta),  W = M (E * K),  U = M V
//   P      = U - W S,   O = scale (E * Q) S + A P
//   S     <- Diag(E[15]) S + ((E[15]/E) * K)^T P
//
// Decay factoring without pairwise exponentials.  Every pair i < c inside a
// 16-token chunk has a unique highest differing bit b: c has it set, i has it
// clear, and both lie in the same aligned block of 2^(b+1) rows whose upper
// half starts at ref.  Then
//   prod_{t=i+1..c} a_t = (prod_{t=ref+1..c} a_t) * (prod_{t=i+1..ref} a_t)
// and both factors are <= 1, so per level b one [16 x K] operand X_b holds
// k_r times its factor (query rows: the first product, key rows: the second)
// and L_b = X_b X_b^T is a plain MFMA product; entries outside level b's pairs
// are masked.  Factors only underflow when the true decay is smaller still.
// Level "d" (the diagonal, factor 1) gives A[c,c].
//
// Work split: one workgroup of NW waves per (b, h, 16*NW state columns).  Wave
// w owns state columns [16w, 16w+16) as four-float MFMA accumulator tiles
// (rows 16t + 4*(lane/16) + j, column lane%16) for all K rows, so W S, Q S,
// A P and K^T P need no cross-wave reduction.  The V-independent work
// (operands, L, A, solve, W) is shared by the waves through LDS.
// Operands that are not exact in fp16 (S, P, W, QE, K-hat, A, M) are split
// into fp16 hi + lo and multiplied as hi*hi + hi*lo + lo*hi.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int BT = 16;   // tokens per internal chunk
constexpr int RP = 24;   // padded row (halfs) of the [*][16] operand matrices
constexpr int NLEV = 5;  // operand levels: 0 = diagonal, 1 + b for bit b = 0..3

template <int K, int NW>
struct __align__(16) ChunkSmem {
    static constexpr int VT = 16 * NW;
    static constexpr int KP = K + 16;      // padded row (halfs) of [16][K] operands
    float alpha[BT][K];                    // exp(g)
    float qv[BT][K];                       // q (unscaled)
    float kv[BT][K];
    float beta[BT];
    float elast[K];                        // exp(gc) at the chunk's last row
    float L[BT][BT + 1];                   // beta-scaled strictly-lower L
    _Float16 X[NLEV][BT][KP];              // key-side level operands
    _Float16 Y[NLEV][BT][KP];              // query-side level operands (q * factor)
    _Float16 QE[2][BT][KP];                // q * E, hi/lo
    _Float16 WN[2][BT][KP];                // -W, hi/lo
    _Float16 KET[2][K][RP];                // (k * E)^T, hi/lo
    _Float16 KHT[2][K][RP];                // (k * E[15] / E)^T, hi/lo
    _Float16 VTt[2][VT][RP];               // V^T, hi/lo
    _Float16 AM[2][BT][RP];                // A (scaled), hi/lo
    _Float16 MM[2][BT][RP];                // M, hi/lo
};

__device__ __forceinline__ h4 frag16(const _Float16* base, int stride, int row, int lg) {
    return *reinterpret_cast<const h4*>(base + row * stride + 4 * lg);
}

// 16x16x32 operand fragment: slots 0-3 hold k = 32u + 4lg + j, slots 4-7 hold
// k = 32u + 16 + 4lg + j.  A and B fragments use the same assignment, so the
// product is the full 32-wide dot product whatever slot order the unit uses.
__device__ __forceinline__ h8 frag32(const _Float16* base, int stride, int row, int lg, int u) {
    const _Float16* p = base + row * stride + 32 * u + 4 * lg;
    const h4 lo = *reinterpret_cast<const h4*>(p);
    const h4 hi = *reinterpret_cast<const h4*>(p + 16);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Level b operands of channel c: every row r of the chunk gets k_r times its
// decay factor relative to the upper half-block start ref of its level block.
template <int B, int K, int NW>
__device__ __forceinline__ void level_operands(ChunkSmem<K, NW>& sm, int c) {
    constexpr int Lh = 1 << B;       // half-block size
    constexpr int lev = 1 + B;
#pragma unroll
    for (int s0 = 0; s0 < BT; s0 += 2 * Lh) {
        const int ref = s0 + Lh;
        float f = 1.f;
#pragma unroll
        for (int r = ref; r < s0 + 2 * Lh; ++r) {      // query rows: prod_{ref+1..r}
            if (r > ref) f *= sm.alpha[r][c];
            sm.X[lev][r][c] = static_cast<_Float16>(sm.kv[r][c] * f);
            sm.Y[lev][r][c] = static_cast<_Float16>(sm.qv[r][c] * f);
        }
        f = 1.f;
#pragma unroll
        for (int r = ref - 1; r >= s0; --r) {          // key rows: prod_{r+1..ref}
            f *= sm.alpha[r + 1][c];
            sm.X[lev][r][c] = static_cast<_Float16>(sm.kv[r][c] * f);
            sm.Y[lev][r][c] = static_cast<_Float16>(0.f);
        }
    }
}

template <int K, int NW>
__global__ __launch_bounds__(64 * NW) void chunkwise_kernel(const kda_fwd_args a) {
    using Sm = ChunkSmem<K, NW>;
    constexpr int VT = Sm::VT, KP = Sm::KP, NT = 64 * NW;
    constexpr int KT = K / 16;     // 16-row state tiles
    constexpr int KU = K / 32;     // 32-wide k blocks
    static_assert(K % 32 == 0 && K <= 128, "chunkwise supports K in {32, 64, 128}");
    __shared__ Sm sm;

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nvt = static_cast<int>(V / VT);
    int bid = blockIdx.x;
    const int vt = bid % nvt;
    bid /= nvt;
    const int64_t h = bid % H;
    const int64_t b = bid / H;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int ln = lane & 15, lg = lane >> 4;
    const int64_t v0 = static_cast<int64_t>(vt) * VT;
    const int64_t ncol = v0 + 16 * wave + ln;        // this lane's state / output column
    const float scale = a.scale;
    const bool v_exact = a.qkv_dtype == KDA_DTYPE_F16;

    // ---- initial state, accumulator layout: Sacc[t][j] = S[16t + 4lg + j][ncol]
    const int64_t sbase = (b * H + h) * static_cast<int64_t>(K) * V;
    f4 Sacc[KT];
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = 16 * t + 4 * lg + j;
            Sacc[t][j] = a.state_in ? load_elem(a.state_in, sbase + r * V + ncol, a.state_in_dtype) : 0.f;
        }

    for (int64_t t0 = 0; t0 < T; t0 += BT) {
        // ---- stage the chunk (rows past T are neutral: k = q = v = beta = 0, a = 1)
        for (int idx = tid; idx < BT * K; idx += NT) {
            const int r = idx / K, c = idx % K;
            const int64_t tt = t0 + r;
            float qx = 0.f, kx = 0.f, al = 1.f;
            if (tt < T) {
                qx = load_elem(a.q, b * a.q_stride[0] + tt * a.q_stride[1] + h * a.q_stride[2] + c, a.qkv_dtype);
                kx = load_elem(a.k, b * a.k_stride[0] + tt * a.k_stride[1] + h * a.k_stride[2] + c, a.qkv_dtype);
                al = fast_exp(load_elem(a.g, b * a.g_stride[0] + tt * a.g_stride[1] + h * a.g_stride[2] + c, a.g_dtype));
            }
            sm.qv[r][c] = qx;
            sm.kv[r][c] = kx;
            sm.alpha[r][c] = al;
        }
        for (int idx = tid; idx < BT * VT; idx += NT) {
            const int n = idx % VT, r = idx / VT;
            const int64_t tt = t0 + r;
            float vx = 0.f;
            if (tt < T)
                vx = load_elem(a.v, b * a.v_stride[0] + tt * a.v_stride[1] + h * a.v_stride[2] + v0 + n, a.qkv_dtype);
            split_h(vx, sm.VTt[0][n][r], sm.VTt[1][n][r]);
        }
        if (tid < BT) {
            const int64_t tt = t0 + tid;
            sm.beta[tid] = tt < T ? load_elem(a.beta, b * a.beta_stride[0] + tt * a.beta_stride[1] +
                                                          h * a.beta_stride[2], a.beta_dtype)
                                  : 0.f;
        }
        __syncthreads();

        // ---- per-channel operands: 6 tasks per channel
        for (int idx = tid; idx < 6 * K; idx += NT) {
            const int c = idx % K, task = idx / K;
            switch (task) {
                case 0: {
                    float e = 1.f;
#pragma unroll
                    for (int r = 0; r < BT; ++r) {
                        e *= sm.alpha[r][c];
                        split_h(sm.qv[r][c] * e, sm.QE[0][r][c], sm.QE[1][r][c]);
                        split_h(sm.kv[r][c] * e, sm.KET[0][c][r], sm.KET[1][c][r]);
                    }
                    sm.elast[c] = e;
                    float s = 1.f;
#pragma unroll
                    for (int r = BT - 1; r >= 0; --r) {
                        split_h(sm.kv[r][c] * s, sm.KHT[0][c][r], sm.KHT[1][c][r]);
                        s *= sm.alpha[r][c];
                    }
                    break;
                }
                case 1: level_operands<0>(sm, c); break;
                case 2: level_operands<1>(sm, c); break;
                case 3: level_operands<2>(sm, c); break;
                case 4: level_operands<3>(sm, c); break;
                default: {
#pragma unroll
                    for (int r = 0; r < BT; ++r) {
                        sm.X[0][r][c] = static_cast<_Float16>(sm.kv[r][c]);
                        sm.Y[0][r][c] = static_cast<_Float16>(sm.qv[r][c]);
                    }
                    break;
                }
            }
        }
        __syncthreads();

        // ---- L and A by level: each (c, i) is written by exactly one level
        for (int lev = wave; lev < NLEV; lev += NW) {
            f4 accL = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < KU; ++u) {
                const h8 xf = frag32(&sm.X[lev][0][0], KP, ln, lg, u);
                const h8 yf = frag32(&sm.Y[lev][0][0], KP, ln, lg, u);
                accL = mfma16x16x32(xf, xf, accL);
                accA = mfma16x16x32(yf, xf, accA);
            }
            const int i = ln;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = 4 * lg + j;
                if (lev == 0) {
                    if (i == c) {
                        split_h(accA[j] * scale, sm.AM[0][c][i], sm.AM[1][c][i]);
                    } else if (i > c) {
                        sm.AM[0][c][i] = static_cast<_Float16>(0.f);
                        sm.AM[1][c][i] = static_cast<_Float16>(0.f);
                    }
                } else {
                    const int bb = lev - 1;
                    const bool pair = ((c >> (bb + 1)) == (i >> (bb + 1))) && ((c >> bb) & 1) && !((i >> bb) & 1);
                    if (pair) {
                        sm.L[c][i] = sm.beta[c] * accL[j];
                        split_h(accA[j] * scale, sm.AM[0][c][i], sm.AM[1][c][i]);
                    }
                }
            }
        }
        __syncthreads();

        // ---- M = (I + L)^-1 Diag(beta): forward substitution, one column per lane
        if (tid < BT) {
            const int jc = tid;
            float m[BT];
#pragma unroll
            for (int r = 0; r < BT; ++r) {
                float s = (r == jc) ? 1.f : 0.f;
#pragma unroll
                for (int t = 0; t < r; ++t) s = fmaf(-sm.L[r][t], m[t], s);
                m[r] = s;
            }
            const float bj = sm.beta[jc];
#pragma unroll
            for (int r = 0; r < BT; ++r) split_h(m[r] * bj, sm.MM[0][r][jc], sm.MM[1][r][jc]);
        }
        __syncthreads();

        // ---- W = M (E*K) (shared, written as -W) and U = M V (this wave's columns)
        const h4 mh = frag16(&sm.MM[0][0][0], RP, ln, lg);
        const h4 ml = frag16(&sm.MM[1][0][0], RP, ln, lg);
        for (int tt = wave; tt < KT; tt += NW) {
            const h4 kh = frag16(&sm.KET[0][16 * tt][0], RP, ln, lg);
            const h4 kl = frag16(&sm.KET[1][16 * tt][0], RP, ln, lg);
            f4 w = {0.f, 0.f, 0.f, 0.f};
            w = mfma16x16x16(mh, kh, w);
            w = mfma16x16x16(ml, kh, w);
            w = mfma16x16x16(mh, kl, w);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                split_h(-w[j], sm.WN[0][4 * lg + j][16 * tt + ln], sm.WN[1][4 * lg + j][16 * tt + ln]);
        }
        f4 P = {0.f, 0.f, 0.f, 0.f};
        {
            const h4 vh = frag16(&sm.VTt[0][16 * wave][0], RP, ln, lg);
            P = mfma16x16x16(mh, vh, P);
            P = mfma16x16x16(ml, vh, P);
            if (!v_exact) {
                const h4 vl = frag16(&sm.VTt[1][16 * wave][0], RP, ln, lg);
                P = mfma16x16x16(mh, vl, P);
            }
        }
        __syncthreads();

        // ---- state chain of this wave's 16 columns
        h8 shi[KU], slo[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                _Float16 x0, x1, y0, y1;
                split_h(Sacc[2 * u][j], x0, y0);
                split_h(Sacc[2 * u + 1][j], x1, y1);
                shi[u][j] = x0; slo[u][j] = y0;
                shi[u][4 + j] = x1; slo[u][4 + j] = y1;
            }
        // P = U - W S
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const h8 wh = frag32(&sm.WN[0][0][0], KP, ln, lg, u);
            const h8 wl = frag32(&sm.WN[1][0][0], KP, ln, lg, u);
            P = mfma16x16x32(wh, shi[u], P);
            P = mfma16x16x32(wh, slo[u], P);
            P = mfma16x16x32(wl, shi[u], P);
        }
        // O = scale (Q*E) S + A P
        f4 O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const h8 qh = frag32(&sm.QE[0][0][0], KP, ln, lg, u);
            const h8 ql = frag32(&sm.QE[1][0][0], KP, ln, lg, u);
            O = mfma16x16x32(qh, shi[u], O);
            O = mfma16x16x32(qh, slo[u], O);
            O = mfma16x16x32(ql, shi[u], O);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) O[j] *= scale;
        h4 ph, pl;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            _Float16 x, y;
            split_h(P[j], x, y);
            ph[j] = x; pl[j] = y;
        }
        {
            const h4 ah = frag16(&sm.AM[0][0][0], RP, ln, lg);
            const h4 al = frag16(&sm.AM[1][0][0], RP, ln, lg);
            O = mfma16x16x16(ah, ph, O);
            O = mfma16x16x16(ah, pl, O);
            O = mfma16x16x16(al, ph, O);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t tt = t0 + 4 * lg + j;
            if (tt < T) store_elem(a.o, ((b * T + tt) * H + h) * V + ncol, a.qkv_dtype, O[j]);
        }
        // S <- Diag(E[15]) S + Khat^T P
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const float4 e = *reinterpret_cast<const float4*>(&sm.elast[16 * t + 4 * lg]);
            Sacc[t][0] *= e.x; Sacc[t][1] *= e.y; Sacc[t][2] *= e.z; Sacc[t][3] *= e.w;
            const h4 kh = frag16(&sm.KHT[0][16 * t][0], RP, ln, lg);
            const h4 kl = frag16(&sm.KHT[1][16 * t][0], RP, ln, lg);
            Sacc[t] = mfma16x16x16(kh, ph, Sacc[t]);
            Sacc[t] = mfma16x16x16(kh, pl, Sacc[t]);
            Sacc[t] = mfma16x16x16(kl, ph, Sacc[t]);
        }
        // No barrier needed here: the next chunk's staging writes only alpha,
        // qv, kv, beta and VTt, none of which this phase reads; the barrier
        // after staging orders everything else.
    }

#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t r = 16 * t + 4 * lg + j;
            store_elem(a.state_out, sbase + r * V + ncol, a.state_out_dtype, Sacc[t][j]);
        }
}

template <int K, int NW>
int launch_knw(const kda_fwd_args& a, hipStream_t stream) {
    const int64_t blocks = a.B * a.H * (a.V / (16 * NW));
    hipLaunchKernelGGL((chunkwise_kernel<K, NW>), dim3(static_cast<unsigned>(blocks)), dim3(64 * NW), 0,
                       stream, a);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

template <int K>
int launch_k(const kda_fwd_args& a, hipStream_t stream) {
    if (a.V % 64 == 0) return launch_knw<K, 4>(a, stream);
    if (a.V % 32 == 0) return launch_knw<K, 2>(a, stream);
    return launch_knw<K, 1>(a, stream);
}

}  // namespace

bool chunkwise_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % 16 == 0;
}

int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream) {
    switch (a.K) {
        case 32: return launch_k<32>(a, stream);
        case 64: return launch_k<64>(a, stream);
        case 128: return launch_k<128>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
