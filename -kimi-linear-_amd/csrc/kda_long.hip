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
// When the first pass fits one round of workgroups (few chains: B P H (V + K)
// / 128 <= the CUs), the third pass is replaced: the first pass also writes
// every state column's outputs in fp32 -- the V columns' (o from a zero
// initial state, oz) and the transition columns' (per token, the row c of
// coefficients of the initial state in the outputs) -- and
//   3'. o[t] = oz[t] + c[t] S_start[p] (long_correct_kernel), rounded once;
// the outputs are linear in the initial state, so this is the same function.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef uint32_t w4 __attribute__((ext_vector_type(4)));
typedef uint32_t w2 __attribute__((ext_vector_type(2)));

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

// Eight values as bf16 pairs: hi = bf16(x), lo = bf16(x - hi), |x - hi - lo|
// <= 2^-18 |x|.
__device__ __forceinline__ void split8_bf16(const float (&v)[8], bf8& hi, bf8& lo) {
    w4 hw, lw;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e], v[2 * e + 1]}, bf2));
        const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xffff0000u);
        hw[e] = hb;
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e] - h0, v[2 * e + 1] - h1}, bf2));
    }
    hi = __builtin_bit_cast(bf8, hw);
    lo = __builtin_bit_cast(bf8, lw);
}

constexpr int kCorrectTokens = 256;   // tokens per correction workgroup

// o[t] = oz[t] + c[t] S_start[p] for the tokens t of segment p (the third
// pass of the few-chain split).  One workgroup of V / 16 waves per (b P + p,
// 256 tokens, h); wave w owns state columns 16 w .. 16 w + 15.  Per 16-token
// step the workgroup stages the step's c rows (16 x K fp32) in LDS as bf16
// pairs, one 16-byte load a thread, the next step's fetched meanwhile; the
// product runs on the bf16 matrix cores as pairs (hi hi + hi lo + lo hi,
// ~2^-16 relative) with fp32 accumulation: the A operand is S_start^T (lane
// (ln, lg): column 16 w + ln, channels 32 u + 8 lg .. + 7, fetched once),
// the B operand c^T (lane (ln, lg): token ln, the same channels, 16-byte LDS
// reads), so the accumulator holds token ln, columns 16 w + 4 lg .. + 3 --
// one 16-byte read of oz and one store of o per lane and step.  A first
// segment that starts from zero (no initial state) takes oz as it is.  Rows
// past the segment's end are outside the descriptors' ranges (read as zero,
// stores dropped).  oz, cf: [B T, H, V] and [B T, H, K] fp32; sstart:
// [B P, H, K, V] fp32; o: [B T, H, V] in the output dtype.
template <int K>
struct CorrectSmem {
    uint16_t hi[2][16][K + 8];
    uint16_t lo[2][16][K + 8];
};
template <int K, typename TO>
__global__ __launch_bounds__(1024) void long_correct_kernel(const float* oz, const float* cf, const float* sstart,
                                                            TO* o, int64_t T, int64_t H, int64_t V, int64_t P,
                                                            int zero_first) {
    __shared__ CorrectSmem<K> sm;
    const int t = threadIdx.x, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int nthr = static_cast<int>(blockDim.x);
    const int w = __builtin_amdgcn_readfirstlane(t >> 6);
    const int64_t Ts = T / P;
    const int64_t nblk = (Ts + kCorrectTokens - 1) / kCorrectTokens;
    int64_t g = blockIdx.x;
    const int64_t h = g % H;
    g /= H;
    const int64_t tb = g % nblk;
    const int64_t bp = g / nblk;                    // b P + p
    const bool none = zero_first && bp % P == 0;    // S_start = 0
    const int64_t c0 = 16 * w;
    const int64_t t0 = tb * kCorrectTokens;
    const int rows = static_cast<int>(Ts - t0 < kCorrectTokens ? Ts - t0 : kCorrectTokens);
    const int64_t row0 = bp * Ts + t0;              // flat token index b T + p Ts + t0
    const int64_t hk = H * K, hv = H * V;
    const auto rc = make_rsrc(cf + row0 * hk + h * K, static_cast<uint32_t>(((rows - 1) * hk + K) * 4));
    const auto rz = make_rsrc(oz + row0 * hv + h * V, static_cast<uint32_t>(((rows - 1) * hv + V) * 4));
    const auto ro = make_rsrc(o + row0 * hv + h * V,
                              static_cast<uint32_t>(((rows - 1) * hv + V) * static_cast<int64_t>(sizeof(TO))));
    auto store_out = [&](const f4& y, int orow) {
        if constexpr (sizeof(TO) == 4) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(w4, y), ro, orow * 4, 0, 0);
        } else {
            w2 p;
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                uint32_t lo16, hi16;
                if constexpr (Elem<TO>::code == KDA_DTYPE_F16) {
                    lo16 = __builtin_bit_cast(uint16_t, static_cast<_Float16>(y[2 * j]));
                    hi16 = __builtin_bit_cast(uint16_t, static_cast<_Float16>(y[2 * j + 1]));
                } else {
                    lo16 = f32_to_bf16_bits(y[2 * j]);
                    hi16 = f32_to_bf16_bits(y[2 * j + 1]);
                }
                p[j] = lo16 | (hi16 << 16);
            }
            __builtin_amdgcn_raw_buffer_store_b64(p, ro, orow * 2, 0, 0);
        }
    };
    if (none) {
        for (int tt = 0; tt < rows; tt += 16) {
            const int orow = static_cast<int>((tt + ln) * hv + c0 + 4 * lg);
            const w4 z = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rz, orow * 4, 0, 0));
            store_out(f4{__uint_as_float(z[0]), __uint_as_float(z[1]), __uint_as_float(z[2]), __uint_as_float(z[3])},
                      orow);
        }
        return;
    }
    bf8 sh[K / 32], sl[K / 32];
    {
        const float* S = sstart + (bp * H + h) * K * V + c0 + ln;
#pragma unroll
        for (int u = 0; u < K / 32; ++u) {
            float v[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = S[(32 * u + 8 * lg + e) * V];
            split8_bf16(v, sh[u], sl[u]);
        }
    }
    // the step's c rows: 16 x K / 4 16-byte pieces, piece i = (row i / (K /
    // 4), channels 4 (i % (K / 4)) ..), at most two a thread
    constexpr int NP = 16 * K / 4;
    w4 fc[2];
    auto fetch = [&](int tt) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int i = t + nthr * m;
            const int r = i / (K / 4), c4 = i % (K / 4);
            // a slot past the step's pieces reads past the range: no memory access
            const int off = i < NP ? static_cast<int>(((tt + r) * hk + 4 * c4) * 4) : 0x7ffffff0;
            fc[m] = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rc, off, 0, 0));
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int i = t + nthr * m;
            if (i < NP) {
                const int r = i / (K / 4), c4 = i % (K / 4);
                w2 hv2, lv2;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const float x0 = __uint_as_float(fc[m][2 * e]), x1 = __uint_as_float(fc[m][2 * e + 1]);
                    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{x0, x1}, bf2));
                    hv2[e] = hb;
                    lv2[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(
                                 f2v{x0 - __uint_as_float(hb << 16), x1 - __uint_as_float(hb & 0xffff0000u)}, bf2));
                }
                *reinterpret_cast<w2*>(&sm.hi[buf][r][4 * c4]) = hv2;
                *reinterpret_cast<w2*>(&sm.lo[buf][r][4 * c4]) = lv2;
            }
        }
    };
    // Every load runs one step ahead of its use: step tt's c rows were
    // fetched during step tt - 16 and staged at its end, step tt's oz
    // during step tt - 16; the rows of step tt + 32 are fetched once step
    // tt + 16's are staged.  (Past the last row the ranges return zeros.)
    auto oz_row = [&](int tt) { return static_cast<int>((tt + ln) * hv + c0 + 4 * lg); };
    fetch(0);
    stage(0);
    w4 z = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rz, oz_row(0) * 4, 0, 0));
    fetch(16);
    {
        // the loop issues its output store after these loads: a store that
        // writes nothing stands in for it, so that the loop is entered with
        // the pattern of outstanding memory operations it repeats
        const auto none_o = make_rsrc(o, 0u);
        __builtin_amdgcn_raw_buffer_store_b32(0u, none_o, 0, 0, 0);
    }
    int buf = 0;
    for (int tt = 0; tt < rows; tt += 16) {
        const w4 zn = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rz, oz_row(tt + 16) * 4, 0, 0));
        __syncthreads();                            // this step's rows are staged
        f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < K / 32; ++u) {
            const bf8 ch = *reinterpret_cast<const bf8*>(&sm.hi[buf][ln][32 * u + 8 * lg]);
            const bf8 cl = *reinterpret_cast<const bf8*>(&sm.lo[buf][ln][32 * u + 8 * lg]);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh[u], ch, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sh[u], cl, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sl[u], ch, acc, 0, 0, 0);
        }
        stage(buf ^ 1);                             // the next step's rows into the other buffer
        fetch(tt + 32);
        f4 y;
#pragma unroll
        for (int j = 0; j < 4; ++j) y[j] = acc[j] + __uint_as_float(z[j]);
        store_out(y, oz_row(tt));
        z = zn;
        buf ^= 1;
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

// The few-chain form: the first pass in one round of 128-column workgroups
// on the current device (and V <= 256: one correction wave per 16 columns).
static bool long_correct_form(int64_t B, int64_t H, int64_t K, int64_t V, int64_t P) {
    if (V > 256) return false;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return (V + K) % 128 == 0 && B * P * H * ((V + K) / 128) <= cus;
}

int64_t long_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t P) {
    // segment states and transitions, initial states; in the few-chain form
    // the fp32 outputs oz and c after them
    return 4 * (B * P * H * K * (2 * V + K) + (long_correct_form(B, H, K, V, P) ? B * T * H * (V + K) : 0));
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
    float* oz = sstart + B * P * H * K * V;
    float* cf = oz + B * T * H * V;
    const bool correct = long_correct_form(B, H, K, V, P);

    // 1. per chain: the state from zero and the transition (and in the
    // few-chain form the fp32 outputs oz and c)
    kda_fwd_args a1 = s;
    a1.state_in = nullptr;
    a1.state_out = seg;
    a1.state_out_dtype = KDA_DTYPE_F32;
    a1.o = correct ? oz : nullptr;
    int st = chunkwise_trans_launch(a1, stream, correct ? cf : nullptr);
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

    if (correct) {
        // 3'. o = oz + c S_start
        const int64_t nblk = (T / P + kCorrectTokens - 1) / kCorrectTokens;
        const dim3 grid(static_cast<unsigned>(B * P * nblk * H)), block(static_cast<unsigned>(4 * V));
        const int zero_first = a.state_in == nullptr ? 1 : 0;
#define KDA_CORRECT(KK, TO)                                                                                    \
    hipLaunchKernelGGL((long_correct_kernel<KK, TO>), grid, block, 0, stream, oz, cf, sstart,                   \
                       static_cast<TO*>(a.o), T, H, V, P, zero_first)
        if (a.qkv_dtype == KDA_DTYPE_F16) {
            if (K == 64) KDA_CORRECT(64, _Float16); else KDA_CORRECT(128, _Float16);
        } else {
            if (K == 64) KDA_CORRECT(64, bf16_t); else KDA_CORRECT(128, bf16_t);
        }
#undef KDA_CORRECT
        return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
    }

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
