// Token-by-token KDA recurrence (decode step) for gfx950.
//
// Replaces the body of kda_recurrent (kimi_linear/kda.py:196-219).  Per token
// the reference makes ~8 elementwise passes over the [K, V] fp32 state; this
// kernel keeps the state of one (batch, head, V-tile) in registers for the
// whole call, so each state element is read from HBM once and written once.
//
// Per token, with a = exp(g), q~ = q * scale (single-pass form of Eq. 1):
//   S' = Diag(a) S,   u = S'^T k,   r = S'^T q~,   d = beta (v - u)
//   S  = S' + k d^T,  o = r + (q~ . k) d            (== S^T q~ after the update)
//
// Work split: one 256-thread workgroup per (b, h, V-tile of VT columns).
// Thread t owns 4 consecutive columns (t % (VT/4)) of rows rg, rg + RG, ...
// with rg = t / (VT/4), so every state row segment is a coalesced 16-byte
// access.  The two K-reductions (u, r) and q~.k go through wave shuffles and
// one LDS exchange per token.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int kRecThreads = 256;

template <int K, int VT>
__global__ __launch_bounds__(kRecThreads) void recurrent_kernel(const kda_fwd_args a) {
    constexpr int CPR = VT / 4;                 // threads per state row
    constexpr int RG = kRecThreads / CPR;       // row groups
    constexpr int RPT = K / RG;                 // rows per thread
    constexpr int NWAVE = kRecThreads / 64;
    static_assert(VT % 4 == 0 && kRecThreads % CPR == 0, "bad V tile");
    static_assert(RPT >= 1 && K % RG == 0, "K must be a multiple of the row-group count");
    static_assert(CPR <= 64, "a state row segment must fit one wave");

    __shared__ float s_q[K], s_k[K], s_a[K];
    __shared__ float s_v[VT];
    __shared__ float s_beta;
    __shared__ float s_red[NWAVE][2 * VT + 1];

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nvt = static_cast<int>(V / VT);
    int bid = blockIdx.x;
    const int vt = bid % nvt;
    bid /= nvt;
    const int64_t h = bid % H;
    const int64_t b = bid / H;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cg = tid % CPR, rg = tid / CPR;
    const int64_t col0 = static_cast<int64_t>(vt) * VT + 4 * cg;

    const int64_t sbase = (b * H + h) * static_cast<int64_t>(K) * V;

    float S[RPT][4];
    const bool vec_in = a.state_in != nullptr && a.state_in_dtype == KDA_DTYPE_F32 &&
                        (reinterpret_cast<uintptr_t>(a.state_in) & 15) == 0;
    if (a.state_in == nullptr) {
#pragma unroll
        for (int j = 0; j < RPT; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) S[j][c] = 0.f;
    } else if (vec_in) {
        const float* sp = static_cast<const float*>(a.state_in);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int64_t r = rg + RG * j;
            const float4 x = *reinterpret_cast<const float4*>(sp + sbase + r * V + col0);
            S[j][0] = x.x; S[j][1] = x.y; S[j][2] = x.z; S[j][3] = x.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int64_t r = rg + RG * j;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                S[j][c] = load_elem(a.state_in, sbase + r * V + col0 + c, a.state_in_dtype);
        }
    }

    const float scale = a.scale;
    for (int64_t t = 0; t < T; ++t) {
        // ---- stage token t: q~, k, exp(g) for all K rows; v for this tile; beta
        if (tid < K) {
            const int64_t iq = b * a.q_stride[0] + t * a.q_stride[1] + h * a.q_stride[2] + tid;
            const int64_t ik = b * a.k_stride[0] + t * a.k_stride[1] + h * a.k_stride[2] + tid;
            const int64_t ig = b * a.g_stride[0] + t * a.g_stride[1] + h * a.g_stride[2] + tid;
            s_q[tid] = load_elem(a.q, iq, a.qkv_dtype) * scale;
            s_k[tid] = load_elem(a.k, ik, a.qkv_dtype);
            s_a[tid] = fast_exp(load_elem(a.g, ig, a.g_dtype));
        }
        if (tid < VT) {
            const int64_t iv = b * a.v_stride[0] + t * a.v_stride[1] + h * a.v_stride[2] +
                               static_cast<int64_t>(vt) * VT + tid;
            s_v[tid] = load_elem(a.v, iv, a.qkv_dtype);
        }
        if (tid == 0) {
            const int64_t ib = b * a.beta_stride[0] + t * a.beta_stride[1] + h * a.beta_stride[2];
            s_beta = load_elem(a.beta, ib, a.beta_dtype);
        }
        __syncthreads();

        // ---- decay, then partial K-reductions over this thread's rows
        float pu[4] = {0.f, 0.f, 0.f, 0.f}, pr[4] = {0.f, 0.f, 0.f, 0.f}, pqk = 0.f;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int r = rg + RG * j;
            const float al = s_a[r], kk = s_k[r], qq = s_q[r];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                S[j][c] *= al;
                pu[c] = fmaf(S[j][c], kk, pu[c]);
                pr[c] = fmaf(S[j][c], qq, pr[c]);
            }
            pqk = fmaf(qq, kk, pqk);
        }
        // lanes that differ only in row group (bits >= log2(CPR)) share columns
#pragma unroll
        for (int off = CPR; off < 64; off <<= 1) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                pu[c] += __shfl_xor(pu[c], off);
                pr[c] += __shfl_xor(pr[c], off);
            }
            pqk += __shfl_xor(pqk, off);
        }
        if (lane < CPR) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                s_red[wave][4 * cg + c] = pu[c];
                s_red[wave][VT + 4 * cg + c] = pr[c];
            }
            if (cg == 0) s_red[wave][2 * VT] = pqk;
        }
        __syncthreads();

        float u[4] = {0.f, 0.f, 0.f, 0.f}, rr[4] = {0.f, 0.f, 0.f, 0.f}, qk = 0.f;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                u[c] += s_red[w][4 * cg + c];
                rr[c] += s_red[w][VT + 4 * cg + c];
            }
            qk += s_red[w][2 * VT];
        }
        const float beta = s_beta;
        float d[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = beta * (s_v[4 * cg + c] - u[c]);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const float kk = s_k[rg + RG * j];
#pragma unroll
            for (int c = 0; c < 4; ++c) S[j][c] = fmaf(kk, d[c], S[j][c]);
        }
        if (rg == 0) {
            const int64_t io = ((b * T + t) * H + h) * V + col0;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                float o = fmaf(qk, d[c], rr[c]);
                if (a.clamp_fp16_out && a.qkv_dtype == KDA_DTYPE_F16) o = clamp_fp16_safe(o);
                store_elem(a.o, io + c, a.qkv_dtype, o);
            }
        }
        __syncthreads();   // the next token's staging overwrites s_* and s_red
    }

    const bool vec_out = a.state_out_dtype == KDA_DTYPE_F32 &&
                         (reinterpret_cast<uintptr_t>(a.state_out) & 15) == 0;
    if (vec_out) {
        float* sp = static_cast<float*>(a.state_out);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int64_t r = rg + RG * j;
            *reinterpret_cast<float4*>(sp + sbase + r * V + col0) =
                make_float4(S[j][0], S[j][1], S[j][2], S[j][3]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int64_t r = rg + RG * j;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                store_elem(a.state_out, sbase + r * V + col0 + c, a.state_out_dtype, S[j][c]);
        }
    }
}

template <int K, int VT>
int launch_k_vt(const kda_fwd_args& a, hipStream_t stream) {
    const int64_t blocks = a.B * a.H * (a.V / VT);
    hipLaunchKernelGGL((recurrent_kernel<K, VT>), dim3(static_cast<unsigned>(blocks)),
                       dim3(kRecThreads), 0, stream, a);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

template <int K>
int launch_k(const kda_fwd_args& a, hipStream_t stream, int vt) {
    switch (vt) {
        case 128: return launch_k_vt<K, 128>(a, stream);
        case 64: return launch_k_vt<K, 64>(a, stream);
        case 32: return launch_k_vt<K, 32>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace

bool recurrent_supported(int64_t K, int64_t V) {
    if (!(K == 32 || K == 64 || K == 128 || K == 256)) return false;
    return V % 32 == 0;
}

int recurrent_launch(const kda_fwd_args& a, hipStream_t stream) {
    // V tile: 64 columns where possible (two workgroups per head at V = 128
    // gives 2048 workgroups at B = 64, H = 16), else 32.
    const int vt = (a.V % 64 == 0) ? 64 : 32;
    switch (a.K) {
        case 32: return launch_k<32>(a, stream, vt);
        case 64: return launch_k<64>(a, stream, vt);
        case 128: return launch_k<128>(a, stream, vt);
        case 256: return launch_k<256>(a, stream, vt);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
