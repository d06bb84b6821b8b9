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
// Work split: one workgroup of NW waves per (b, h, V-tile of 4 CPL NW
// columns); wave w owns 4 CPL columns of the tile for all K rows, lane l the
// four columns 4 (l % CPL) .. +3 of the K CPL / 64 consecutive rows of row
// group l / CPL: a row segment is one 16-byte access.  Both K-reductions
// (u, r) and q~.k are sums over the lanes of one column group, inside the
// wave (DPP row rotations and the permlane swaps of lane bits 4 and 5, all
// on the VALU): no LDS round and no barrier.  q~, k and a of a token are
// staged once per workgroup in LDS.
//
// Gated calls (kda_recurrent_gated_fwd) take the gate's up-projection gk and
// the beta logits instead of g and beta and form, while staging the token,
// a = exp(-exp(A_log) softplus(gk + dt_bias)) and beta = sigmoid(logit) in
// fp32 (kimi_linear/kda.py:452-460).
//
// CK (the checkpointing forward of fp32 activations, kda_chunkwise_fwd_ckpt):
// before every 32-token chunk the state is also stored, in fp32, at the head
// of that chunk's record, so the backward starts from the exact fp32 states
// of this recurrence (kda_ckpt_fp32.hip fills the rest of each record).
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

// VEC: the state is read (unless absent) and written as 16-byte-aligned fp32
// rows with buffer loads/stores; otherwise element by element in any dtype.
// A separate instantiation keeps the generic path's registers out of the
// fast one.
// Sum of x over the 8 lanes that share l & 7 (all-reduce): row_ror:8, then
// the permlane swaps of bits 4 and 5.
__device__ __forceinline__ float lanegroup8_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return x;
}

// Lane l of a wave holds 4 adjacent state columns (column group l % CPL) of
// RPL = K CPL / 64 adjacent rows (row group l / CPL); the K-reductions are
// sums over the lanes of one column group.
template <int K, int NW, int CPL, bool VEC, bool CK = false>
__global__ __launch_bounds__(64 * NW) void recurrent_kernel(const kda_fwd_args a, const kda_gate_args gate,
                                                            float* ckpt) {
    static_assert(CPL == 4 || CPL == 8 || CPL == 16, "column groups per wave");
    constexpr int RPL = K * CPL / 64;           // rows per lane
    constexpr int VT = 4 * CPL * NW;            // columns per workgroup
    static_assert(K % (64 / CPL) == 0 && RPL >= 1, "K must be a multiple of the row groups");
    auto ksum = [](float x) {
        return CPL == 4 ? rowgroup_sum(x) : (CPL == 8 ? lanegroup8_sum(x) : lanegroup4_sum(x));
    };

    __shared__ float s_q[K], s_k[K], s_a[K];

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nvt = static_cast<int>(V / VT);
    int bid = blockIdx.x;
    const int vt = bid % nvt;
    bid /= nvt;
    const int64_t h = bid % H;
    const int64_t b = bid / H;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cg = lane % CPL, rg = lane / CPL;
    const int r0 = RPL * rg;
    const int64_t col0 = static_cast<int64_t>(vt) * VT + 4 * CPL * wave + 4 * cg;
    const int64_t sbase = (b * H + h) * static_cast<int64_t>(K) * V;

    // fp32 state rows go through one buffer descriptor per head: the lane
    // offset is one register and the row offset a scalar
    const uint32_t row_bytes = static_cast<uint32_t>(V) * 4u;
    const uint32_t lane_off = static_cast<uint32_t>(r0) * row_bytes + static_cast<uint32_t>(col0) * 4u;
    // The state is read once per call, and each element's last read comes
    // right before its write: non-temporal loads (nt) keep the read lines from
    // being retained in the caches, which measured 30.7 -> 22.5 us per B=64
    // H=16 d=128 decode step when the state comes from HBM (in place), at a
    // small cost when it sits in the Infinity Cache (20.9 -> 22.2 us).
    constexpr int kLoadNonTemporal = 2;
    // The new state is stored streaming as well (nt with sc1): a decode step
    // over states larger than the Infinity Cache (five rotating 64 MiB sets at
    // B=64 H=16 d=128) measured 24.35 -> 23.30 us per step against plain
    // stores, in place 23.40 -> 23.21 us; one cache-resident set stepped into
    // a fresh tensor pays 23.1 -> 24.1 us.
    constexpr int kStoreStreaming = 2 | 16;
    float S[RPL][4];
    if (a.state_in == nullptr) {
#pragma unroll
        for (int j = 0; j < RPL; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c) S[j][c] = 0.f;
    } else if (VEC) {
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(static_cast<const float*>(a.state_in) + sbase), static_cast<short>(0),
            static_cast<int>(K * row_bytes), 0x00020000);
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(lane_off),
                                                                  static_cast<int>(j * row_bytes), kLoadNonTemporal);
            S[j][0] = __uint_as_float(x[0]); S[j][1] = __uint_as_float(x[1]);
            S[j][2] = __uint_as_float(x[2]); S[j][3] = __uint_as_float(x[3]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < RPL; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                S[j][c] = load_elem(a.state_in, sbase + static_cast<int64_t>(r0 + j) * V + col0 + c,
                                    a.state_in_dtype);
    }

    // channels this thread stages per token, and for a gated call their
    // exp(A_log) and dt_bias, fetched once (beside the state loads)
    constexpr int KPT = (K + 64 * NW - 1) / (64 * NW);
    float gcoef[KPT], gbias[KPT];
    if (gate.a_log) {
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const int i = tid + 64 * NW * j;
            gcoef[j] = i < K ? expf(gate.a_log[h * K + i]) : 0.f;
            gbias[j] = i < K ? gate.dt_bias[h * K + i] * kLog2e : 0.f;
        }
    }
    const float scale = a.scale;
    // CK: the records of this (b, h), one per 32-token chunk
    float* ckh = CK ? ckpt + (b * H + h) * ((T + 31) / 32) * ckpt_record(K, V) : nullptr;
    for (int64_t t = 0; t < T; ++t) {
        if constexpr (CK) {
            if (t % 32 == 0) {
                float* rec = ckh + (t / 32) * ckpt_record(K, V);
#pragma unroll
                for (int j = 0; j < RPL; ++j)
#pragma unroll
                    for (int c = 0; c < 4; ++c) rec[static_cast<int64_t>(r0 + j) * V + col0 + c] = S[j][c];
            }
        }
        // ---- stage token t: q~, k, exp(g) for all K rows; v, beta per lane.
        // Every load is issued before any is decoded.
        const int64_t tq = b * a.q_stride[0] + t * a.q_stride[1] + h * a.q_stride[2];
        const int64_t tk = b * a.k_stride[0] + t * a.k_stride[1] + h * a.k_stride[2];
        const int64_t tg = b * a.g_stride[0] + t * a.g_stride[1] + h * a.g_stride[2];
        const int64_t tv = b * a.v_stride[0] + t * a.v_stride[1] + h * a.v_stride[2] + col0;
        RawElem rv[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) rv[c] = load_raw_elem(a.v, tv + c, a.qkv_dtype);
        const RawElem rb =
            load_raw_elem(a.beta, b * a.beta_stride[0] + t * a.beta_stride[1] + h * a.beta_stride[2], a.beta_dtype);
#pragma unroll
        for (int j = 0; j < KPT; ++j) {
            const int i = tid + 64 * NW * j;
            if (i >= K) break;
            const RawElem rq = load_raw_elem(a.q, tq + i, a.qkv_dtype);
            const RawElem rk = load_raw_elem(a.k, tk + i, a.qkv_dtype);
            const RawElem rg = load_raw_elem(a.g, tg + i, a.g_dtype);
            s_q[i] = decode_elem(rq, a.qkv_dtype) * scale;
            s_k[i] = decode_elem(rk, a.qkv_dtype);
            const float gv = decode_elem(rg, a.g_dtype);
            s_a[i] = gate.a_log ? gate_decay(fmaf(gv, kLog2e, gbias[j]), gcoef[j]) : fast_exp(gv);
        }
        float v[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = decode_elem(rv[c], a.qkv_dtype);
        const float beta = gate.a_log ? sigmoid_f(decode_elem(rb, a.beta_dtype)) : decode_elem(rb, a.beta_dtype);
        __syncthreads();

        // ---- decay, then the lane's partial K-reductions over its rows
        float u[4] = {0.f, 0.f, 0.f, 0.f}, rr[4] = {0.f, 0.f, 0.f, 0.f}, qk = 0.f;
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const float al = s_a[r0 + j], qq = s_q[r0 + j], kk = s_k[r0 + j];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                S[j][c] *= al;
                u[c] = fmaf(S[j][c], kk, u[c]);
                rr[c] = fmaf(S[j][c], qq, rr[c]);
            }
            qk = fmaf(qq, kk, qk);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            u[c] = ksum(u[c]);
            rr[c] = ksum(rr[c]);
        }
        qk = ksum(qk);

        float d[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) d[c] = beta * (v[c] - u[c]);
#pragma unroll
        for (int j = 0; j < RPL; ++j) {
            const float kk = s_k[r0 + j];
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
        if (t + 1 < T) __syncthreads();   // the next token's staging overwrites s_*
    }

    if (VEC) {
        const auto rs = __builtin_amdgcn_make_buffer_rsrc(static_cast<float*>(a.state_out) + sbase,
                                                          static_cast<short>(0), static_cast<int>(K * row_bytes),
                                                          0x00020000);
        typedef unsigned int u4 __attribute__((ext_vector_type(4)));
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            __builtin_amdgcn_raw_buffer_store_b128(
                u4{__float_as_uint(S[j][0]), __float_as_uint(S[j][1]), __float_as_uint(S[j][2]),
                   __float_as_uint(S[j][3])},
                rs, static_cast<int>(lane_off), static_cast<int>(j * row_bytes), kStoreStreaming);
    } else {
#pragma unroll
        for (int j = 0; j < RPL; ++j)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                store_elem(a.state_out, sbase + static_cast<int64_t>(r0 + j) * V + col0 + c, a.state_out_dtype,
                           S[j][c]);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int K, int NW, int CPL>
int launch_k_nw(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args& gate, float* ckpt) {
    const dim3 grid(static_cast<unsigned>(a.B * a.H * (a.V / (4 * CPL * NW)))), block(64 * NW);
    const bool vec = (a.V & 3) == 0 && a.state_out_dtype == KDA_DTYPE_F32 && aligned16(a.state_out) &&
                     (a.state_in == nullptr || (a.state_in_dtype == KDA_DTYPE_F32 && aligned16(a.state_in)));
    if (ckpt != nullptr) {
        if constexpr (K <= 128) {
            hipLaunchKernelGGL((recurrent_kernel<K, NW, CPL, false, true>), grid, block, 0, stream, a, gate, ckpt);
        } else {
            return KDA_ERR_UNSUPPORTED;
        }
    } else if (vec) {
        hipLaunchKernelGGL((recurrent_kernel<K, NW, CPL, true>), grid, block, 0, stream, a, gate, nullptr);
    } else {
        hipLaunchKernelGGL((recurrent_kernel<K, NW, CPL, false>), grid, block, 0, stream, a, gate, nullptr);
    }
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

template <int K>
int launch_k(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args& gate, float* ckpt) {
    // K 128 with V % 64 == 0: one wave of 64 columns (32 rows x 4 columns a
    // lane, 196 VGPRs: the 2048 waves of a B=64 H=16 V=128 step are all
    // resident at once); other K <= 128: one wave of 32 columns (K / 8 rows x
    // 4 columns a lane); K 256: 16 columns a wave (K / 16 rows a lane).
    if constexpr (K == 128) {
        if (a.V % 64 == 0) return launch_k_nw<K, 1, 16>(a, stream, gate, ckpt);
    }
    if constexpr (K <= 128) {
        if (a.V % 32 == 0) return launch_k_nw<K, 1, 8>(a, stream, gate, ckpt);
    }
    if (a.V % 64 == 0) return launch_k_nw<K, 4, 4>(a, stream, gate, ckpt);
    if (a.V % 32 == 0) return launch_k_nw<K, 2, 4>(a, stream, gate, ckpt);
    return launch_k_nw<K, 1, 4>(a, stream, gate, ckpt);
}

}  // namespace

bool recurrent_supported(int64_t K, int64_t V) {
    if (!(K == 32 || K == 64 || K == 128 || K == 256)) return false;
    return V % 16 == 0;
}

int recurrent_launch(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args* gate_p, float* ckpt) {
    const kda_gate_args gate = gate_p ? *gate_p : kda_gate_args{nullptr, nullptr};
    switch (a.K) {
        case 32: return launch_k<32>(a, stream, gate, ckpt);
        case 64: return launch_k<64>(a, stream, gate, ckpt);
        case 128: return launch_k<128>(a, stream, gate, ckpt);
        case 256: return launch_k<256>(a, stream, gate, ckpt);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
