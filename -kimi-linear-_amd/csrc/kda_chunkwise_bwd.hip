// Chunkwise KDA backward for gfx950.
//
// Gradient of kda_chunkwise (kimi_linear/kda.py:58-185), whose reference is
// differentiated by autograd (training: scripts/train_musicgpt_fp16.py:519-523).
// The forward is re-evaluated chunk by chunk from the records that
// kda_chunkwise_fwd_ckpt writes: per CT = 32-token chunk, the state before it,
// the chunk's R, A, L and the diagonal blocks of N (below), all of which the
// forward computes anyway; P = M R is formed again from R and N.
//
// Per (b, h) and chunk, rows c, i in [0, CT), channels k, state columns v:
//   G = in-chunk cumulative sum of g,  E = exp(G),  F = exp(G_last - G),
//   eps = exp(G_last),  q~ = scale q
//   A[c,i] = sum_k q~[c,k] k[i,k] exp(G[c,k] - G[i,k])   (i <= c)
//   L[c,i] = sum_k  k[c,k] k[i,k] exp(G[c,k] - G[i,k])   (i <  c)
//   N = (I + Diag(beta) L)^-1,  M = N Diag(beta)
//   R = V - (k*E) S,  P = M R,  O = (q~*E) S + A P,
//   S_end = Diag(eps) S + (k*F)^T P
// and backward, given dO and dS = dL/dS_end:
//   dP = (k*F) dS + A^T dO,  dR = M^T dP,  dV = dR
//   dS_start = Diag(eps) dS + (q~*E)^T dO - (k*E)^T dR
//   d(q~*E) = dO S^T,  d(k*E) = -dR S^T,  d(k*F) = P dS^T,  deps = rowsum(dS * S)
//   dA = tril(dO P^T),  dM = dP R^T
//   dbeta_i += sum_c dM[c,i] N[c,i];  dN = dM Diag(beta);  dX = -N^T dN N^T
//   dbeta_c += sum_{i<c} dX[c,i] L[c,i];  dL = Diag(beta) dX  (strictly lower)
// and the pairwise-decay products of dA and dL give dq~, dk and dG, which
// the reverse in-chunk cumulative sum turns into dg.
//
// Only the chain dS_end -> dP -> dR -> dS_start runs from chunk to chunk;
// everything else is independent per chunk.  Two kernels, one workspace
// between them:
//   1. bwd_state_kernel, one workgroup per (b, h, VA state columns), the chunks
//      in reverse.  First it completes N in the head's chunk records (the
//      forward's solve left the diagonal blocks; the block below them from
//      those and L), then the chain above; it stores each chunk's dS_end, dP
//      and dR and dS_0.  The next chunk's inputs are fetched while the
//      current one is computed.
//   2. bwd_chunk_kernel, one workgroup per (b, h, chunk): writes dv = dR; from
//      S, R (checkpoint), P = M R, dS_end, dP and dR the sums over all state
//      columns (VT at a time) of dA, dM, d(q~E), d(kE), d(kF) and deps, then the chain
//      through the inverse, the pairwise-decay products and the reverse
//      cumulative sum: complete dq, dk, dg and dbeta.
// Rows past T read as zero inputs, which leave the state and every gradient
// of the rows before T unchanged.  q, k, v, dO and dq, dk, dv are in the
// caller's activation dtype (fp32, fp16 or bf16); g, beta, the checkpoints,
// dg, dbeta and the state gradients are fp32.  Products run on the matrix
// cores as bf16 hi/lo pairs (~2^-17 relative each; fp32 accumulation),
// except A and L for 16-bit activations (fp16 operands, the forward's
// precision) and N (fp32 matrix cores).
#include <algorithm>
#include <cstddef>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int CT = 32;          // tokens per chunk = the forward's checkpoint spacing
constexpr int VT = 32;          // state columns per step of bwd_chunk_kernel

// Per (b, h) and chunk (index cb = (b H + h) nck + n): A, L and N (32 x 32)
// from the forward's chunk record (records of ms floats; the forward leaves
// N's block below the diagonal to bwd_state_kernel, which completes it in
// place), and in the workspace dS_end [K][V], dP and dR [CT][V].
struct BwdWs {
    const float* A;
    const float* L;
    float* N;
    float* dS;
    float* dP;
    float* dR;
    int64_t ms;
};

BwdWs ws_layout(void* base, const float* ckpt, int64_t BH, int64_t nck, int64_t K, int64_t V) {
    float* p = static_cast<float*>(base);
    BwdWs w;
    w.A = ckpt + (K + CT) * V;
    w.L = w.A + CT * CT;
    w.N = const_cast<float*>(w.A) + 2 * CT * CT;
    w.ms = ckpt_record(K, V);
    w.dS = p;
    w.dP = w.dS + BH * nck * K * V;
    w.dR = w.dP + BH * nck * CT * V;
    return w;
}

// D += A B for one 16 x 16 tile on the fp32 matrix cores (16x16x4 steps):
// A(r, k) and B(k, c) give the operands; lane (ln, lg) supplies A(ln, 4u + lg)
// and B(4u + lg, ln) and holds D[4 lg + j][ln] in slot j.
template <int KS, typename FA, typename FB>
__device__ __forceinline__ f4 tile_mm(FA fa, FB fb, int ln, int lg, f4 acc) {
#pragma unroll 4
    for (int u = 0; u < KS / 4; ++u)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa(ln, 4 * u + lg), fb(4 * u + lg, ln), acc, 0, 0, 0);
    return acc;
}

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));

// x as a bf16 pair: hi = bf16(x), lo = bf16(x - hi).
__device__ __forceinline__ void split_bf16(float x, uint16_t& hi, uint16_t& lo) {
    const __bf16 h = static_cast<__bf16>(x);
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(x - static_cast<float>(h)));
}

// acc += X Y^T for one 16 x 16 tile over the VT = 32 columns of a step, X and
// Y bf16 pairs (rows of VB elements; xh/xl, yh/yl: row ln of the tile's X and
// Y rows): hi hi + hi lo + lo hi on the bf16 matrix cores
// (v_mfma_f32_16x16x32_bf16; the dropped lo lo term is ~2^-16 relative).
// Lane (ln, lg) supplies columns 8 lg .. 8 lg + 7 of both and holds
// D[4 lg + j][ln] in slot j, the layout of tile_mm.  Only this form runs in
// these accumulator chains.
__device__ __forceinline__ f4 mm_pair(const uint16_t* xh, const uint16_t* xl, const uint16_t* yh,
                                      const uint16_t* yl, int lg, f4 acc) {
    const bf8 ah = *reinterpret_cast<const bf8*>(xh + 8 * lg), al = *reinterpret_cast<const bf8*>(xl + 8 * lg);
    const bf8 bh = *reinterpret_cast<const bf8*>(yh + 8 * lg), bl = *reinterpret_cast<const bf8*>(yl + 8 * lg);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    return acc;
}

// ------------------------------------------------------------------ kernel 1

// The bf16 pair products of mm_pair on fragments held in registers.
__device__ __forceinline__ f4 mfma_pair(const bf8& ah, const bf8& al, const bf8& bh, const bf8& bl, f4 acc) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
    return acc;
}

typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef _Float16 hf2 __attribute__((ext_vector_type(2)));
typedef uint32_t w4 __attribute__((ext_vector_type(4)));
typedef uint32_t w2 __attribute__((ext_vector_type(2)));

// Eight values as bf16 pairs (hi = bf16(x), lo = bf16(x - hi)), two values
// per conversion.
__device__ __forceinline__ void split8(const float (&v)[8], bf8& hi, bf8& lo) {
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

// c + X Y for 16 x 16 fp32 tiles on the fp32 matrix cores (four 16x16x4
// steps): xt holds X^T in accumulator layout (lane (ln, lg) slot u:
// X[ln][4 lg + u]), y holds Y in accumulator layout (slot u: Y[4 lg + u][ln]);
// the result is in accumulator layout.
__device__ __forceinline__ f4 mm_acc(const f4& xt, const f4& y, f4 c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) c = __builtin_amdgcn_mfma_f32_16x16x4f32(xt[u], y[u], c, 0, 0, 0);
    return c;
}

// A value fetched raw (16-bit values in the low half) as fp32.
template <typename TI>
__device__ __forceinline__ float raw_f32(uint32_t w) {
    if constexpr (sizeof(TI) == 4) {
        return __uint_as_float(w);
    } else if constexpr (Elem<TI>::code == KDA_DTYPE_F16) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w)));
    } else {
        return __uint_as_float(w << 16);
    }
}

// N = (I + Diag(beta) L)^-1 of the chunks n = n0, n0 + step, ... of head bh,
// completed in its records: the forward's solve left the diagonal blocks
// N00, N11 there (and zeroed N01); N10 = -N11 X10 N00 with X10 = Diag(beta_1)
// L10 on the fp32 matrix cores, written to the record's N10 block.  One wave,
// eight chunks in flight (their operands fetched together).
__device__ __forceinline__ void complete_n(const kda_bwd_args& a, const BwdWs& ws, int64_t bh, int nck, int n0,
                                           int step, int ln, int lg) {
    const int64_t H = a.H, T = a.T, b = bh / H, h = bh % H;
    constexpr int NF = 8;
    for (int nb = n0; nb < nck; nb += NF * step) {
        f4 xt[NF], n00[NF], n11t[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int n = nb + f * step;
            const bool on = n < nck;
            const int64_t cb = bh * nck + (on ? n : 0);
            const float* L = ws.L + cb * ws.ms;
            const float* N = ws.N + cb * ws.ms;
            const int64_t row1 = static_cast<int64_t>(n) * CT + 16 + ln;
            const float b1 = on && row1 < T ? a.beta[(b * T + row1) * H + h] : 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                xt[f][u] = b1 * L[(16 + ln) * CT + 4 * lg + u];       // X10[ln][4 lg + u]
                n00[f][u] = N[(4 * lg + u) * CT + ln];                // N00[4 lg + u][ln]
                n11t[f][u] = N[(16 + ln) * CT + 16 + 4 * lg + u];     // N11[ln][4 lg + u]
            }
        }
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int n = nb + f * step;
            const f4 y = mm_acc(xt[f], n00[f], f4{0.f, 0.f, 0.f, 0.f});      // X10 N00
            const f4 n10 = mm_acc(n11t[f], y, f4{0.f, 0.f, 0.f, 0.f});       // N11 X10 N00
            if (n < nck) {
                float* N = ws.N + (bh * nck + n) * ws.ms;
#pragma unroll
                for (int j = 0; j < 4; ++j) N[(16 + 4 * lg + j) * CT + ln] = -n10[j];
            }
        }
    }
}

// ------------------------------------------------------------------ kernel 2

// The chain's operands as bf16 hi/lo pairs ([0] hi, [1] lo, as in the chunk
// kernel's column steps), each laid out along its contraction so that every
// MFMA fragment (8 consecutive elements) is one 16-byte read: the transposed
// (q~*E), (k*E), A, N, dO, dP, dR and dS, and k*F as it is.
constexpr int NS = 512;         // threads per workgroup of bwd_state_kernel
constexpr int NWS = NS / 64;    // its waves

// NP: 2 (bf16 pairs) or 1 (fp16 activations: single fp16 operands).
template <int K, int VA, int NP>
struct __align__(16) StateSmem {
    static constexpr int KB = K + 8, TB = CT + 8;
    uint16_t qeT[NP][K][TB];    // (scale q exp(G))^T: [channel][token]
    uint16_t keT[NP][K][TB];    // (k exp(G))^T
    uint16_t kf[NP][CT][KB];    // k exp(G_last - G): [token][channel]
    uint16_t dST[NP][VA][KB];   // dS^T at the chunk end: [column][channel]
    uint16_t dOT[NP][VA][TB];   // dO^T: [column][token]
    uint16_t dPT[NP][VA][TB];
    uint16_t dRT[NP][VA][TB];
    uint16_t AT[NP][CT][TB];    // A^T: [c][c2] = A[c2][c]
    uint16_t NT_[NP][CT][TB];   // N^T
    float tot[NS / K][K];       // per row group, the sum of its g
    float beta[CT];
    float eps[K];
};

// Four values of consecutive rows (a lane's accumulator slots) into a
// transposed bf16 pair row: hi and lo, 8 bytes each.
__device__ __forceinline__ void put4_pair(uint16_t* hi, uint16_t* lo, const f4& x) {
    uint16_t h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) split_bf16(x[j], h[j], l[j]);
    *reinterpret_cast<uint2*>(hi) = uint2{h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16)};
    *reinterpret_cast<uint2*>(lo) = uint2{l[0] | (uint32_t(l[1]) << 16), l[2] | (uint32_t(l[3]) << 16)};
}

// N (2, 4 or 8) values as bf16 pairs into N consecutive hi and lo slots
// (one 4-, 8- or 16-byte write each; two values per conversion).
template <int N>
__device__ __forceinline__ void put_pairs(uint16_t* hi, uint16_t* lo, const float (&v)[N]) {
    static_assert(N == 2 || N == 4 || N == 8, "pair run length");
    uint32_t hw[N / 2], lw[N / 2];
#pragma unroll
    for (int e = 0; e < N / 2; ++e) {
        const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e], v[2 * e + 1]}, bf2));
        const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xffff0000u);
        hw[e] = hb;
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e] - h0, v[2 * e + 1] - h1}, bf2));
    }
    if constexpr (N == 2) {
        *reinterpret_cast<uint32_t*>(hi) = hw[0];
        *reinterpret_cast<uint32_t*>(lo) = lw[0];
    } else if constexpr (N == 4) {
        *reinterpret_cast<w2*>(hi) = w2{hw[0], hw[1]};
        *reinterpret_cast<w2*>(lo) = w2{lw[0], lw[1]};
    } else {
        *reinterpret_cast<w4*>(hi) = w4{hw[0], hw[1], hw[2], hw[3]};
        *reinterpret_cast<w4*>(lo) = w4{lw[0], lw[1], lw[2], lw[3]};
    }
}

// fp16 activations run the chain on single fp16 operands (the [0] arrays
// only, holding fp16 values) and the fp16 matrix cores: the precision of the
// reference's fp16 path, which takes q E, k E, k F, A, M and the state in
// fp16 for its products (kimi_linear/kda.py:163-182) and so differentiates
// them in fp16; dS_end, dP and dR are kept in fp16 for the chunk kernel as
// it is.  Other dtypes keep the bf16 pairs.
template <bool H16>
__device__ __forceinline__ void put4v(uint16_t* hi, uint16_t* lo, const f4& x) {
    if constexpr (H16) {
        uint16_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x[j]));
        *reinterpret_cast<uint2*>(hi) = uint2{h[0] | (uint32_t(h[1]) << 16), h[2] | (uint32_t(h[3]) << 16)};
        (void)lo;
    } else {
        put4_pair(hi, lo, x);
    }
}
template <bool H16, int N>
__device__ __forceinline__ void put_run(uint16_t* hi, uint16_t* lo, const float (&v)[N]) {
    if constexpr (H16) {
        static_assert(N == 2 || N == 4 || N == 8, "run length");
        uint32_t hw[N / 2];
#pragma unroll
        for (int e = 0; e < N / 2; ++e)
            hw[e] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * e]))) |
                    (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * e + 1]))) << 16);
        if constexpr (N == 2) *reinterpret_cast<uint32_t*>(hi) = hw[0];
        else if constexpr (N == 4) *reinterpret_cast<w2*>(hi) = w2{hw[0], hw[1]};
        else *reinterpret_cast<w4*>(hi) = w4{hw[0], hw[1], hw[2], hw[3]};
        (void)lo;
    } else {
        put_pairs(hi, lo, v);
    }
}
// acc += X Y^T over 32 contraction elements (rows xh / yh at the tile's row ln)
template <bool H16>
__device__ __forceinline__ f4 mmv(const uint16_t* xh, const uint16_t* xl, const uint16_t* yh, const uint16_t* yl,
                                 int lg, f4 acc) {
    if constexpr (H16)
        return mfma16x16x32(*reinterpret_cast<const h8*>(xh + 8 * lg), *reinterpret_cast<const h8*>(yh + 8 * lg), acc);
    else
        return mm_pair(xh, xl, yh, yl, lg, acc);
}

// One workgroup per (b, h, VA state columns), the chunks in reverse.  dS, the
// gradient of the state, stays in fp32 accumulators (tile ti = w + 16 m of
// each wave: channels 16 (ti / VTL), columns 16 (ti % VTL)) and is copied as a
// transposed bf16 pair for the next chunk's dP product.  All products on the
// bf16 matrix cores as pairs (mm_pair, ~2^-17 relative per product).
template <int K, int VA, typename TI>
__global__ __launch_bounds__(NS) void bwd_state_kernel(const kda_bwd_args a, const BwdWs ws) {
    constexpr int RPT = CT * K / NS;        // consecutive rows per thread, one channel
    constexpr int DPT = CT * VA / NS;       // dO elements per thread
    constexpr int VTL = VA / 16;            // 16-column tiles
    constexpr int NDP = 2 * VTL;            // tiles of dP and dR (CT x VA)
    constexpr int NTS = (K / 16) * VTL;     // tiles of dS (K x VA)
    constexpr int TPW = (NTS + NWS - 1) / NWS;  // dS tiles per wave
    constexpr int APT = CT * CT / NS;       // elements of A (and of N) per thread
    static_assert(RPT >= 1 && DPT >= 1 && NDP <= NWS, "thread mapping");
    constexpr bool H16 = std::is_same<TI, _Float16>::value;
    constexpr int L1 = H16 ? 0 : 1;         // the lo half of a pair (fp16: unused, aliased to hi)
    __shared__ StateSmem<K, VA, H16 ? 1 : 2> sm;
    const TI* qp = static_cast<const TI*>(a.q);
    const TI* kp = static_cast<const TI*>(a.k);
    const TI* dop = static_cast<const TI*>(a.d_o);

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nva = static_cast<int>(V / VA);
    // Workgroups are dealt to the eight XCDs round robin (g % 8): with B H a
    // multiple of 8, the nva workgroups of one (b, h) share g % 8, hence an
    // XCD and its L2, and read that head's q, k, g from HBM once.
    const int64_t g = blockIdx.x, BH = a.B * H;
    const bool xcd = BH % 8 == 0;
    const int64_t bh = xcd ? (g / 8 / nva) * 8 + g % 8 : g / nva, b = bh / H, h = bh % H;
    const int64_t v0 = (xcd ? (g / 8) % nva : g % nva) * VA;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int x = t % K, rg = t / K;

    // N of every chunk of this head completed in its records (both V-tile
    // workgroups of the head write the same values), before the chain reads it
    complete_n(a, ws, bh, nck, w, NWS, ln, lg);
    __syncthreads();

    // dS at the end of the sequence into the accumulators and its pair copy
    f4 accs[TPW];
#pragma unroll
    for (int m = 0; m < TPW; ++m) {
        const int ti = w + NWS * m;
        if (ti < NTS) {
            const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                accs[m][j] = a.d_state_out ? a.d_state_out[(bh * K + r0 + 4 * lg + j) * V + v0 + c0 + ln] : 0.f;
            put4v<H16>(&sm.dST[0][c0 + ln][r0 + 4 * lg], &sm.dST[L1][c0 + ln][r0 + 4 * lg], accs[m]);
        }
    }

    // Fetched raw through descriptors whose range stops at the chunk's last
    // row before T (rows past T read as zero), one lane offset per tensor and
    // the row in the scalar offset; converted only where staged.  Thread
    // (rg, x): rows RPT rg .. + RPT - 1 of channel x (q, k, g); thread
    // (t % VA, t / VA): rows DPT (t / VA) .. + DPT - 1 of dO column t % VA;
    // thread (t % CT, t / CT): rows APT (t / CT) .. + APT - 1 of A and N
    // column t % CT -- each one contiguous run of the transposed pair arrays.
    constexpr int SZ = sizeof(TI);
    uint32_t pq[RPT], pk[RPT], pg[RPT], pdo[DPT], pa[APT], pn[APT], pb[1] = {0u};
    const uint32_t HK = static_cast<uint32_t>(H * K), HV = static_cast<uint32_t>(H * V);
    const uint32_t lo_x = static_cast<uint32_t>(RPT * rg) * HK + x;
    const int dv_ = t % VA, dc0 = DPT * (t / VA);
    const uint32_t lo_o = static_cast<uint32_t>(dc0) * HV + dv_;
    const int ai = t % CT, ac0 = APT * (t / CT);
    // Every fetch is a buffer load through a descriptor whose range ends at
    // the chunk's last row before T and is empty for n < 0 (the loop fetches
    // chunk -1 after chunk 0: all zeros, nothing read), issued without a
    // branch, from descriptors held in scalar registers.
    auto fetch = [&](int n) {
        const int64_t r0 = static_cast<int64_t>(n < 0 ? 0 : n) * CT;
        const int64_t nrow = n < 0 ? 0 : std::min<int64_t>(CT, T - r0);
        const int64_t base = ((b * T + r0) * H + h) * K;
        const uint32_t span = nrow > 0 ? static_cast<uint32_t>((nrow - 1) * H * K + K) : 0u;
        const auto rq = make_rsrc(qp + base, span * SZ), rk = make_rsrc(kp + base, span * SZ);
        const auto rgc = make_rsrc(a.g + base, span * 4);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const uint32_t so = static_cast<uint32_t>(j) * HK;
            if constexpr (SZ == 2) {
                pq[j] = __builtin_amdgcn_raw_buffer_load_b16(rq, static_cast<int>(2 * lo_x), static_cast<int>(2 * so), 0);
                pk[j] = __builtin_amdgcn_raw_buffer_load_b16(rk, static_cast<int>(2 * lo_x), static_cast<int>(2 * so), 0);
            } else {
                pq[j] = __builtin_amdgcn_raw_buffer_load_b32(rq, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
                pk[j] = __builtin_amdgcn_raw_buffer_load_b32(rk, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
            }
            pg[j] = __builtin_amdgcn_raw_buffer_load_b32(rgc, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
        }
        const auto ro = make_rsrc_uniform(dop + ((b * T + r0) * H + h) * V + v0,
                                  nrow > 0 ? static_cast<uint32_t>(((nrow - 1) * H * V + VA) * SZ) : 0u);
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const uint32_t so = static_cast<uint32_t>(j) * HV * SZ;
            if constexpr (SZ == 2)
                pdo[j] = __builtin_amdgcn_raw_buffer_load_b16(ro, static_cast<int>(2 * lo_o), static_cast<int>(so), 0);
            else
                pdo[j] = __builtin_amdgcn_raw_buffer_load_b32(ro, static_cast<int>(4 * lo_o), static_cast<int>(so), 0);
        }
        const int64_t cn = bh * nck + r0 / CT;
        const auto ra = make_rsrc(ws.A + cn * ws.ms, n < 0 ? 0u : static_cast<uint32_t>(CT * CT * 4));
        const auto rn = make_rsrc(ws.N + cn * ws.ms, n < 0 ? 0u : static_cast<uint32_t>(CT * CT * 4));
#pragma unroll
        for (int j = 0; j < APT; ++j) {
            const int off = ((ac0 + j) * CT + ai) * 4;
            pa[j] = __builtin_amdgcn_raw_buffer_load_b32(ra, off, 0, 0);
            pn[j] = __builtin_amdgcn_raw_buffer_load_b32(rn, off, 0, 0);
        }
        // beta of row t % CT on every thread (threads t < CT stage it)
        const auto rb = make_rsrc(a.beta + (b * T + r0) * H + h, static_cast<uint32_t>(nrow * H * 4));
        pb[0] = __builtin_amdgcn_raw_buffer_load_b32(rb, static_cast<int>((t % CT) * H * 4), 0, 0);
    };
    if (nck > 0) fetch(nck - 1);

    for (int n = nck - 1; n >= 0; --n) {
        const int64_t cb = bh * nck + n;
        // stage chunk n (A^T, N^T, dO^T as pairs, the row groups' g sums); fetch chunk n - 1
        use_here(pq);
        use_here(pk);
        use_here(pg);
        use_here(pdo);
        use_here(pa);
        use_here(pn);
        use_here(pb);
        float cq[RPT], ck[RPT], cg[RPT];
        float run = 0.f;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            run += __uint_as_float(pg[j]);
            cg[j] = run;
            cq[j] = raw_f32<TI>(pq[j]);
            ck[j] = raw_f32<TI>(pk[j]);
        }
        sm.tot[rg][x] = run;
        {
            float va[APT], vn[APT], vo[DPT];
#pragma unroll
            for (int j = 0; j < APT; ++j) {
                va[j] = __uint_as_float(pa[j]);
                vn[j] = __uint_as_float(pn[j]);
            }
#pragma unroll
            for (int j = 0; j < DPT; ++j) vo[j] = raw_f32<TI>(pdo[j]);
            put_run<H16>(&sm.AT[0][ai][ac0], &sm.AT[L1][ai][ac0], va);
            put_run<H16>(&sm.NT_[0][ai][ac0], &sm.NT_[L1][ai][ac0], vn);
            put_run<H16>(&sm.dOT[0][dv_][dc0], &sm.dOT[L1][dv_][dc0], vo);
        }
        if (t < CT) sm.beta[t] = __uint_as_float(pb[0]);
        fetch(n - 1);
        __syncthreads();

        // G, exp(G), exp(G_last - G): the row groups before this thread's and all of them
        {
            float pre = 0.f, last = 0.f;
#pragma unroll
            for (int r = 0; r < NS / K; ++r) {
                const float s = sm.tot[r][x];
                pre += r < rg ? s : 0.f;
                last += s;
            }
            float qe[RPT], ke[RPT];
#pragma unroll
            for (int j = 0; j < RPT; ++j) {
                const int c = RPT * rg + j;
                const float G = pre + cg[j];
                const float E = __expf(G), F = __expf(last - G);
                qe[j] = a.scale * cq[j] * E;
                ke[j] = ck[j] * E;
                if constexpr (H16)
                    sm.kf[0][c][x] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(ck[j] * F));
                else
                    split_bf16(ck[j] * F, sm.kf[0][c][x], sm.kf[L1][c][x]);
            }
            put_run<H16>(&sm.qeT[0][x][RPT * rg], &sm.qeT[L1][x][RPT * rg], qe);
            put_run<H16>(&sm.keT[0][x][RPT * rg], &sm.keT[L1][x][RPT * rg], ke);
            if (rg == 0) sm.eps[x] = __expf(last);
        }
        __syncthreads();

        // dS_end to the workspace; dP = (k*F) dS + A^T dO; dS <- Diag(eps) dS + (q~*E)^T dO
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
                if constexpr (std::is_same<TI, _Float16>::value) {
                    // fp16 activations: dS_end in fp16, accumulator-order tiles
                    // (half_tile_offset), slot j = 64 consecutive halves
                    _Float16* tile = reinterpret_cast<_Float16*>(ws.dS + cb * K * V) +
                                     half_tile_offset(r0, v0 + c0, V) + lane;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        __builtin_nontemporal_store(static_cast<_Float16>(accs[m][j]), tile + 64 * j);
                } else {
                    float* dsn = ws.dS + cb * K * V + v0;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        __builtin_nontemporal_store(accs[m][j],
                                                    &dsn[static_cast<uint32_t>(r0 + 4 * lg + j) * V + c0 + ln]);
                }
            }
        }
        if (w < NDP) {
            const int r0t = 16 * (w / VTL), c0t = 16 * (w % VTL);
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < K / 32; ++u)
                acc = mmv<H16>(&sm.kf[0][r0t + ln][32 * u], &sm.kf[L1][r0t + ln][32 * u], &sm.dST[0][c0t + ln][32 * u],
                              &sm.dST[L1][c0t + ln][32 * u], lg, acc);
            acc = mmv<H16>(sm.AT[0][r0t + ln], sm.AT[L1][r0t + ln], sm.dOT[0][c0t + ln], sm.dOT[L1][c0t + ln], lg, acc);
            if constexpr (std::is_same<TI, _Float16>::value) {
                // fp16 activations: dP and dR in fp16, row-major halves in the
                // first half of their fp32 slots
                _Float16* dpn = reinterpret_cast<_Float16*>(ws.dP + cb * CT * V) + v0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_nontemporal_store(static_cast<_Float16>(acc[j]),
                                                &dpn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln]);
            } else {
                float* dpn = ws.dP + cb * CT * V + v0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_nontemporal_store(acc[j], &dpn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln]);
            }
            put4v<H16>(&sm.dPT[0][c0t + ln][r0t + 4 * lg], &sm.dPT[L1][c0t + ln][r0t + 4 * lg], acc);
        }
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
#pragma unroll
                for (int j = 0; j < 4; ++j) accs[m][j] *= sm.eps[r0 + 4 * lg + j];
                accs[m] = mmv<H16>(sm.qeT[0][r0 + ln], sm.qeT[L1][r0 + ln], sm.dOT[0][c0 + ln], sm.dOT[L1][c0 + ln], lg,
                                  accs[m]);
            }
        }
        __syncthreads();

        // dR = M^T dP = Diag(beta) N^T dP (= dV, which bwd_chunk_kernel writes out)
        if (w < NDP) {
            const int r0t = 16 * (w / VTL), c0t = 16 * (w % VTL);
            f4 acc = mmv<H16>(sm.NT_[0][r0t + ln], sm.NT_[L1][r0t + ln], sm.dPT[0][c0t + ln], sm.dPT[L1][c0t + ln], lg,
                             f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] *= sm.beta[r0t + 4 * lg + j];
            if constexpr (std::is_same<TI, _Float16>::value) {
                _Float16* drn = reinterpret_cast<_Float16*>(ws.dR + cb * CT * V) + v0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_nontemporal_store(static_cast<_Float16>(acc[j]),
                                                &drn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln]);
            } else {
                float* drn = ws.dR + cb * CT * V + v0;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_nontemporal_store(acc[j], &drn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln]);
            }
            put4v<H16>(&sm.dRT[0][c0t + ln][r0t + 4 * lg], &sm.dRT[L1][c0t + ln][r0t + 4 * lg], acc);
        }
        __syncthreads();

        // dS_start = Diag(eps) dS + (q~*E)^T dO - (k*E)^T dR, and its pair copy
        // for the next chunk's dP (read after the next chunk's first barrier)
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
                const f4 kr = mmv<H16>(sm.keT[0][r0 + ln], sm.keT[L1][r0 + ln], sm.dRT[0][c0 + ln], sm.dRT[L1][c0 + ln],
                                      lg, f4{0.f, 0.f, 0.f, 0.f});
                accs[m] -= kr;
                put4v<H16>(&sm.dST[0][c0 + ln][r0 + 4 * lg], &sm.dST[L1][c0 + ln][r0 + 4 * lg], accs[m]);
            }
        }
        // the next chunk's staging writes none of keT, dRT, dST before its
        // first barrier: no barrier here
    }
    if (a.d_state_in) {
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
#pragma unroll
                for (int j = 0; j < 4; ++j) a.d_state_in[(bh * K + r0 + 4 * lg + j) * V + v0 + c0 + ln] = accs[m][j];
            }
        }
    }
}

// ------------------------------------------------------------------ kernel 3

typedef __bf16 bf4 __attribute__((ext_vector_type(4)));

// Four values as bf16 pairs, two values per conversion.
__device__ __forceinline__ void split4(const float (&v)[4], bf4& hi, bf4& lo) {
    w2 hw, lw;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e], v[2 * e + 1]}, bf2));
        const float h0 = __uint_as_float(hb << 16), h1 = __uint_as_float(hb & 0xffff0000u);
        hw[e] = hb;
        lw[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e] - h0, v[2 * e + 1] - h1}, bf2));
    }
    hi = __builtin_bit_cast(bf4, hw);
    lo = __builtin_bit_cast(bf4, lw);
}
__device__ __forceinline__ void split4(const f4& v, bf4& hi, bf4& lo) {
    const float a[4] = {v[0], v[1], v[2], v[3]};
    split4(a, hi, lo);
}

// A B for one 16 x 16 tile over a contraction of 16, bf16 pairs on
// v_mfma_f32_16x16x16_bf16: lane (ln, lg) supplies A[ln][4 lg .. 4 lg + 3]
// and B[4 lg .. 4 lg + 3][ln] and holds D[4 lg + j][ln] in slot j.  Only this
// form runs in these chains.
__device__ __forceinline__ f4 mfma_pair16(const f4& a, const float (&b)[4]) {
    bf4 ah, al, bh, bl;
    split4(a, ah, al);
    split4(b, bh, bl);
    f4 acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bh, f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ah, bl, acc, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(al, bh, acc, 0, 0, 0);
}

// x of lanes ln, ln + 16, ln + 32 and ln + 48 (the four lane groups of the
// lane's column) on every lane, v[l] from lane group l: three permlane swaps
// (VALU; permlane16_swap(u, u) gives u of lanes l & ~16 and l | 16,
// permlane32_swap likewise for bit 5).
__device__ __forceinline__ void lane_groups(float x, float (&v)[4]) {
    const unsigned u = __float_as_uint(x);
    const auto r16 = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    const auto ra = __builtin_amdgcn_permlane32_swap(r16[0], r16[0], false, false);
    const auto rb = __builtin_amdgcn_permlane32_swap(r16[1], r16[1], false, false);
    v[0] = __uint_as_float(ra[0]);
    v[1] = __uint_as_float(rb[0]);
    v[2] = __uint_as_float(ra[1]);
    v[3] = __uint_as_float(rb[1]);
}

// Sum of x over N aligned consecutive lanes (N = 4, 8 or 16), every lane of
// the group gets it: DPP quad permutations, then the half-row and row mirrors.
template <int N>
__device__ __forceinline__ float lanes_sum(float x) {
    static_assert(N == 4 || N == 8 || N == 16, "lane group");
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    if constexpr (N >= 8)
        x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));  // row_half_mirror
    if constexpr (N >= 16)
        x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));  // row_mirror
    return x;
}

// acc += X Y^T over the VT = 32 columns of a step: X a bf16 pair tile in LDS
// (row ln of the tile: xh, xl), Y's fragment in registers (lane (ln, lg):
// row ln, columns 8 lg .. 8 lg + 7, as a pair).
__device__ __forceinline__ f4 mm_pair_r(const uint16_t* xh, const uint16_t* xl, const bf8& yh, const bf8& yl,
                                        int lg, f4 acc) {
    const bf8 ah = *reinterpret_cast<const bf8*>(xh + 8 * lg), al = *reinterpret_cast<const bf8*>(xl + 8 * lg);
    return mfma_pair(ah, al, yh, yl, acc);
}

// The column step's shared tiles, bf16 pairs ([0] hi, [1] lo; x = hi + lo
// with |x - hi - lo| <= 2^-18 |x|), rows of VB elements (80 bytes: every
// MFMA fragment, 8 consecutive columns, is one 16-byte read).
constexpr int VB = VT + 8;
template <int K>
struct __align__(16) ChunkSmem {
    static constexpr int NW = K / 16;
    uint16_t dO[2][CT][VB];
    uint16_t R[2][CT][VB];      // R from the forward's checkpoint
    uint16_t dP[2][CT][VB];
    uint16_t dR[2][CT][VB];
    uint16_t spare[2][CT][VB];  // with the tiles above: the stash after the column steps
    float L[CT][CT + 1];
    float N[CT][CT + 1];
    float dM[CT][CT + 1];       // dM, then dN, then dX
    float Y[CT][CT + 1];        // dN N^T
    // dA (i <= c) and dX (i < c) by rows ([c][i]) and by columns ([i][c]),
    // 16-byte rows for the element step's fragments
    float dAr[CT][CT + 4];
    float dAc[CT][CT + 4];
    float dXr[CT][CT + 4];
    float dXc[CT][CT + 4];
    float red[NW][CT];          // the waves' column sums of dM * N
    float beta[CT];
};

// One workgroup per (b, h, chunk), K / 16 waves; wave w owns channels
// 16 w .. 16 w + 15 for all CT rows (two 16-row element tiles), so the
// state's and its gradient's fragments come straight from HBM into the
// lanes that use them and the per-element step runs in registers.
// Column steps of VT state columns: the CT-row tiles (dO, R, dP, dR) go
// through LDS as bf16 pairs; every product on the bf16 matrix cores as
// pairs.  P = M R (M = N Diag(beta)) enters through R: the column sums take
// X = dO R^T and Z = R dS^T, and M is applied once per chunk afterwards
// (dO P^T = X M^T, P dS^T = M Z) on the fp32 matrix cores.  The next step is fetched (raw, through buffer descriptors whose
// range stops at the chunk's last row before T) while the current one is
// computed.  About 60 KiB of LDS at K = 128: two workgroups share a CU, one
// workgroup's HBM-bound column steps overlapping the other's element step.
template <int K, typename TI>
__global__ __launch_bounds__(4 * K) __attribute__((amdgpu_waves_per_eu(4))) void bwd_chunk_kernel(const kda_bwd_args a, const BwdWs ws) {
    constexpr int NW = K / 16, NTC = 64 * NW;
    constexpr int EPT = CT * VT / NTC;      // tile elements per thread and tensor
    constexpr int MPW = 8 / NW;             // dA / dM tiles per wave
    constexpr int SZ = sizeof(TI);
    static_assert(NTC % VT == 0 && NTC % CT == 0 && EPT >= 1 && MPW >= 1, "thread mapping");
    __shared__ ChunkSmem<K> sm;
    const TI* qp = static_cast<const TI*>(a.q);
    const TI* kp = static_cast<const TI*>(a.k);
    const TI* dop = static_cast<const TI*>(a.d_o);
    TI* dqp = static_cast<TI*>(a.dq);
    TI* dkp = static_cast<TI*>(a.dk);
    TI* dvp = static_cast<TI*>(a.dv);

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const int64_t bh = blockIdx.x / nck, b = bh / H, h = bh % H;
    const int n = static_cast<int>(blockIdx.x % nck);
    const int64_t cb = bh * nck + n;
    const int64_t r0 = static_cast<int64_t>(n) * CT;
    const int nrow = static_cast<int>(std::min<int64_t>(CT, T - r0));     // rows before T
    const int nvt = static_cast<int>(V / VT);
    const float scale = a.scale;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int x = 16 * w + ln;              // the lane's channel

    // ------------------------------------------------------------ loads
    // q, k, g of the lane's rows 16 p + 4 lg + j, channel x: fetched during
    // the last column step, used after the column steps
    uint32_t rq[2][4], rk[2][4], rg[2][4];
    auto fetch_rows = [&]() {
        const int64_t base = ((b * T + r0) * H + h) * K;
        const uint32_t HK = static_cast<uint32_t>(H * K);
        const uint32_t span = static_cast<uint32_t>(nrow - 1) * HK + K;
        const auto dq = make_rsrc(qp + base, span * SZ), dk = make_rsrc(kp + base, span * SZ);
        const auto dg = make_rsrc(a.g + base, span * 4);
        const uint32_t vo = static_cast<uint32_t>(4 * lg) * HK + x;
#pragma unroll
        for (int p = 0; p < 2; ++p)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t so = static_cast<uint32_t>(16 * p + j) * HK;
                if constexpr (SZ == 2) {
                    rq[p][j] = __builtin_amdgcn_raw_buffer_load_b16(dq, static_cast<int>(2 * vo), static_cast<int>(2 * so), 0);
                    rk[p][j] = __builtin_amdgcn_raw_buffer_load_b16(dk, static_cast<int>(2 * vo), static_cast<int>(2 * so), 0);
                } else {
                    rq[p][j] = __builtin_amdgcn_raw_buffer_load_b32(dq, static_cast<int>(4 * vo), static_cast<int>(4 * so), 0);
                    rk[p][j] = __builtin_amdgcn_raw_buffer_load_b32(dk, static_cast<int>(4 * vo), static_cast<int>(4 * so), 0);
                }
                rg[p][j] = __builtin_amdgcn_raw_buffer_load_b32(dg, static_cast<int>(4 * vo), static_cast<int>(4 * so), 0);
            }
    };
    // column-step fetch: the lane's fragments of S (the checkpointed state
    // before the chunk) and dS (the gradient of the state after it), row x,
    // columns v0 + 8 lg .. + 7; the thread's EPT elements of R (checkpoint),
    // dP, dR (workspace) and dO, rows t / VT + (NTC / VT) m, column t % VT
    const auto rck = make_rsrc(a.ckpt + cb * ckpt_record(K, V),
                               static_cast<uint32_t>((K + CT) * V * 4));
    const auto rds = make_rsrc(ws.dS + cb * K * V, static_cast<uint32_t>(K * V * 4));
    const auto rdp = make_rsrc(ws.dP + cb * CT * V, static_cast<uint32_t>(CT * V * 4));
    const auto rdr = make_rsrc(ws.dR + cb * CT * V, static_cast<uint32_t>(CT * V * 4));
    const auto rdo = make_rsrc(dop + ((b * T + r0) * H + h) * V,
                               static_cast<uint32_t>(((nrow - 1) * H + 1) * V * SZ));
    // fp16 activations: S and dS as fp16 in accumulator-order tiles
    // (half_tile_offset): the lane's 8 columns are one 16-byte run, and a
    // 32-column step moves by two tiles (1 KiB)
    constexpr bool HALF = std::is_same<TI, _Float16>::value;
    const uint32_t vo_f = HALF ? static_cast<uint32_t>(2 * half_tile_offset(x, 8 * lg, V))
                               : static_cast<uint32_t>(x * V + 8 * lg) * 4;
    const int tc = t / VT, tv = t % VT;
    const uint32_t vo_t = static_cast<uint32_t>(tc * V + tv) * 4;
    const uint32_t vo_o = static_cast<uint32_t>(tc * H * V + tv) * SZ;
    uint32_t fS[HALF ? 4 : 8], fdS[HALF ? 4 : 8], fR[EPT], fdP[EPT], fdR[EPT], fdO[EPT];
    auto fetch = [&](int vt) {
        const uint32_t v0 = static_cast<uint32_t>(vt) * VT;
        if constexpr (HALF) {
            const int so = static_cast<int>(2 * 256 * 2 * (v0 / 32));
            const w4 s4 = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rck, static_cast<int>(vo_f), so, 0));
            const w4 d4 = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rds, static_cast<int>(vo_f), so, 0));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                fS[e] = s4[e];
                fdS[e] = d4[e];
            }
        } else {
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const w4 s4 = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rck, static_cast<int>(vo_f + 16 * u), static_cast<int>(4 * v0), 0));
                const w4 d4 = __builtin_bit_cast(w4, __builtin_amdgcn_raw_buffer_load_b128(rds, static_cast<int>(vo_f + 16 * u), static_cast<int>(4 * v0), 0));
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    fS[4 * u + e] = s4[e];
                    fdS[4 * u + e] = d4[e];
                }
            }
        }
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
            const uint32_t rowo = static_cast<uint32_t>((NTC / VT) * m) * static_cast<uint32_t>(V);
            if constexpr (HALF) {
                // R, dP, dR in fp16 (row-major halves in the first half of their rows)
                fR[m] = __builtin_amdgcn_raw_buffer_load_b16(rck, static_cast<int>(vo_t / 2), static_cast<int>(4 * K * V + 2 * (rowo + v0)), 0);
                fdP[m] = __builtin_amdgcn_raw_buffer_load_b16(rdp, static_cast<int>(vo_t / 2), static_cast<int>(2 * (rowo + v0)), 0);
                fdR[m] = __builtin_amdgcn_raw_buffer_load_b16(rdr, static_cast<int>(vo_t / 2), static_cast<int>(2 * (rowo + v0)), 0);
            } else {
                fR[m] = __builtin_amdgcn_raw_buffer_load_b32(rck, static_cast<int>(vo_t), static_cast<int>(4 * (K * V + rowo + v0)), 0);
                fdP[m] = __builtin_amdgcn_raw_buffer_load_b32(rdp, static_cast<int>(vo_t), static_cast<int>(4 * (rowo + v0)), 0);
                fdR[m] = __builtin_amdgcn_raw_buffer_load_b32(rdr, static_cast<int>(vo_t), static_cast<int>(4 * (rowo + v0)), 0);
            }
            const uint32_t so = (static_cast<uint32_t>((NTC / VT) * m) * static_cast<uint32_t>(H * V) + v0) * SZ;
            if constexpr (SZ == 2)
                fdO[m] = __builtin_amdgcn_raw_buffer_load_b16(rdo, static_cast<int>(vo_o), static_cast<int>(so), 0);
            else
                fdO[m] = __builtin_amdgcn_raw_buffer_load_b32(rdo, static_cast<int>(vo_o), static_cast<int>(so), 0);
        }
    };
    fetch(0);
    // L, N and beta to LDS (read after the column steps), fetched after the
    // first step's tiles so that both fetches are in flight together
#pragma unroll
    for (int m = 0; m < CT * CT / NTC; ++m) {
        const int e = t + NTC * m;
        sm.L[e / CT][e % CT] = ws.L[cb * ws.ms + e];
        sm.N[e / CT][e % CT] = ws.N[cb * ws.ms + e];
    }
    if (t < CT) sm.beta[t] = t < nrow ? a.beta[(b * T + r0 + t) * H + h] : 0.f;

    // ------------------------------------- sums over the state columns
    // X += dO R^T, dM += dP R^T (MPW tiles a wave), and per element tile p:
    // d(q~E) += dO S^T, d(kE) -= dR S^T (accumulated as + and negated
    // below), Z += R dS^T; deps += rowsum(dS * S).  Then dA = tril(X M^T)
    // and d(kF) = M Z (P = M R).
    f4 accm[MPW];
#pragma unroll
    for (int m = 0; m < MPW; ++m) accm[m] = f4{0.f, 0.f, 0.f, 0.f};
    f4 dqe[2], dke[2], dkf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) dqe[p] = dke[p] = dkf[p] = f4{0.f, 0.f, 0.f, 0.f};
    float deps = 0.f;
    // one column step: stage the fetched tiles, then (after the caller's
    // fetch of what comes next and a barrier) the products
    // fp16 activations: every operand of the column sums (dO, and S, R,
    // dS_end, dP, dR as recorded) is an fp16 value, so each product is one
    // fp16 MFMA, exact with fp32 accumulation; the tiles hold the raw fp16
    // values ([0] only) and the S and dS fragments are used as fetched
    bf8 sh, sl, dsh, dsl;
    h8 sh16, dsh16;
    auto stage = [&](int vt) {
        use_here(fS);
        use_here(fdS);
        use_here(fR);
        use_here(fdP);
        use_here(fdR);
        use_here(fdO);
#pragma unroll
        for (int m = 0; m < EPT; ++m) {
            const int c = tc + (NTC / VT) * m;
            // R, dP, dR: fp16 with fp16 activations, fp32 otherwise
            const float r = HALF ? raw_f32<_Float16>(fR[m]) : __uint_as_float(fR[m]);
            const float dp = HALF ? raw_f32<_Float16>(fdP[m]) : __uint_as_float(fdP[m]);
            const float dr = HALF ? raw_f32<_Float16>(fdR[m]) : __uint_as_float(fdR[m]);
            if constexpr (HALF) {
                sm.R[0][c][tv] = static_cast<uint16_t>(fR[m]);
                sm.dP[0][c][tv] = static_cast<uint16_t>(fdP[m]);
                sm.dR[0][c][tv] = static_cast<uint16_t>(fdR[m]);
                sm.dO[0][c][tv] = static_cast<uint16_t>(fdO[m]);
            } else {
                split_bf16(r, sm.R[0][c][tv], sm.R[1][c][tv]);
                split_bf16(dp, sm.dP[0][c][tv], sm.dP[1][c][tv]);
                split_bf16(dr, sm.dR[0][c][tv], sm.dR[1][c][tv]);
                split_bf16(raw_f32<TI>(fdO[m]), sm.dO[0][c][tv], sm.dO[1][c][tv]);
            }
            if (c < nrow)
                Elem<TI>::st(dvp + ((b * T + r0 + c) * H + h) * V + static_cast<int64_t>(vt) * VT + tv, dr);
        }
        float sv[8], dsv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if constexpr (HALF) {
                sv[e] = raw_f32<_Float16>(fS[e / 2] >> (16 * (e % 2)));
                dsv[e] = raw_f32<_Float16>(fdS[e / 2] >> (16 * (e % 2)));
            } else {
                sv[e] = __uint_as_float(fS[e]);
                dsv[e] = __uint_as_float(fdS[e]);
            }
            deps = fmaf(sv[e], dsv[e], deps);
        }
        if constexpr (HALF) {
            sh16 = __builtin_bit_cast(h8, w4{fS[0], fS[1], fS[2], fS[3]});
            dsh16 = __builtin_bit_cast(h8, w4{fdS[0], fdS[1], fdS[2], fdS[3]});
        } else {
            split8(sv, sh, sl);
            split8(dsv, dsh, dsl);
        }
    };
    auto products = [&]() {
#pragma unroll
        for (int m = 0; m < MPW; ++m) {
            const int tt = w + NW * m, r0t = 16 * ((tt >> 1) & 1), c0t = 16 * (tt & 1);
            const uint16_t (*xa)[CT][VB] = tt < 4 ? sm.dO : sm.dP;
            if constexpr (HALF)
                accm[m] = mfma16x16x32(*reinterpret_cast<const h8*>(&xa[0][r0t + ln][8 * lg]),
                                       *reinterpret_cast<const h8*>(&sm.R[0][c0t + ln][8 * lg]), accm[m]);
            else
                accm[m] = mm_pair(xa[0][r0t + ln], xa[1][r0t + ln], sm.R[0][c0t + ln], sm.R[1][c0t + ln], lg, accm[m]);
        }
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int er = 16 * p + ln;
            if constexpr (HALF) {
                dqe[p] = mfma16x16x32(*reinterpret_cast<const h8*>(&sm.dO[0][er][8 * lg]), sh16, dqe[p]);
                dke[p] = mfma16x16x32(*reinterpret_cast<const h8*>(&sm.dR[0][er][8 * lg]), sh16, dke[p]);
                dkf[p] = mfma16x16x32(*reinterpret_cast<const h8*>(&sm.R[0][er][8 * lg]), dsh16, dkf[p]);
            } else {
                dqe[p] = mm_pair_r(sm.dO[0][er], sm.dO[1][er], sh, sl, lg, dqe[p]);
                dke[p] = mm_pair_r(sm.dR[0][er], sm.dR[1][er], sh, sl, lg, dke[p]);
                dkf[p] = mm_pair_r(sm.R[0][er], sm.R[1][er], dsh, dsl, lg, dkf[p]);
            }
        }
    };
    for (int vt = 0; vt + 1 < nvt; ++vt) {
        stage(vt);
        fetch(vt + 1);
        __syncthreads();
        products();
        __syncthreads();
    }
    // the last step fetches the element step's rows instead
    stage(nvt - 1);
    fetch_rows();
    __syncthreads();
    products();
    __syncthreads();
    // d(kF) = M Z: block p of M times the Z tiles (M lower triangular;
    // xt(p, q) slot u = M[16 p + ln][16 q + 4 lg + u], the A operand of mm_acc)
    {
        auto mt = [&](int p, int q) {
            f4 x;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = 16 * q + 4 * lg + u;
                x[u] = sm.N[16 * p + ln][i] * sm.beta[i];
            }
            return x;
        };
        const f4 z0 = dkf[0];
        dkf[0] = mm_acc(mt(0, 0), z0, f4{0.f, 0.f, 0.f, 0.f});
        dkf[1] = mm_acc(mt(1, 1), dkf[1], mm_acc(mt(1, 0), z0, f4{0.f, 0.f, 0.f, 0.f}));
    }
    // block 0's accumulators wait in the (now free) tile area while block 1's
    // element step runs: slot i of thread t at stash[i * NTC + t]
    float* stash = reinterpret_cast<float*>(&sm.dO[0][0][0]);
    static_assert(12 * NTC * 4 <= 5 * sizeof(sm.dO) && offsetof(ChunkSmem<K>, spare) == 4 * sizeof(sm.dO),
                  "the stash fits the tiles");
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        stash[(0 + j) * NTC + t] = dqe[0][j];
        stash[(4 + j) * NTC + t] = -dke[0][j];
        stash[(8 + j) * NTC + t] = dkf[0][j];
    }
    dke[1] = f4{0.f, 0.f, 0.f, 0.f} - dke[1];
    // deps of channel x: the shares of the four lanes of the channel
    deps = lanegroup4_sum(deps);
    // X (whole) to dXc's area until dA is formed; dM (i <= c)
#pragma unroll
    for (int m = 0; m < MPW; ++m) {
        const int tt = w + NW * m, r0t = 16 * ((tt >> 1) & 1), c0t = 16 * (tt & 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = r0t + 4 * lg + j, i = c0t + ln;
            if (tt < 4)
                sm.dXc[c][i] = accm[m][j];
            else
                sm.dM[c][i] = i <= c ? accm[m][j] : 0.f;
        }
    }
    __syncthreads();
    // N is lower triangular (N01 = 0), dM lower, so of the 16 x 16 tiles of
    // dA = tril(X M^T), Y = dN N^T (dN = dM Diag(beta)) and the strictly lower
    // dX = -N^T Y only the tiles (0,0), (1,0), (1,1) are formed (dX's and
    // dA's (0,1) tiles are zero and never read, Y's is not needed), over
    // the contraction blocks where N is not zero: dA and Y tiles of block
    // column 0 sum over block 0 only, dX tiles of block row 1 over block 1
    // only.  dA and Y (with the column sums of dM * N) share one phase.
    for (int tt = __builtin_amdgcn_readfirstlane(w); tt < 6; tt += NW) {
        // tiles: dA(1,1), Y(1,1), dA(0,0), dA(1,0), Y(0,0), Y(1,0)
        const bool is_da = tt == 0 || tt == 2 || tt == 3;
        const int r0t = tt == 2 || tt == 4 ? 0 : 16, c0t = tt < 2 ? 16 : 0;
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
        if (is_da) {
            // dA = tril(X M^T), M^T[q][i] = N[i][q] beta[q]; X in dXc's area
            auto fx = [&](int r, int q) { return sm.dXc[r0t + r][q]; };
            auto fm = [&](int q, int i) { return sm.N[c0t + i][q] * sm.beta[q]; };
            const f4 acc = c0t ? tile_mm<CT>(fx, fm, ln, lg, zero) : tile_mm<16>(fx, fm, ln, lg, zero);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = r0t + 4 * lg + j, i = c0t + ln;
                const float v = i <= c ? acc[j] : 0.f;
                sm.dAr[c][i] = v;
                sm.dAc[i][c] = v;
            }
        } else {
            // Y = dN N^T with dN[r][m] = dM[r][m] beta[m]
            auto fn = [&](int r, int m) { return sm.dM[r0t + r][m] * sm.beta[m]; };
            auto ft = [&](int m, int i) { return sm.N[c0t + i][m]; };
            const f4 acc = c0t ? tile_mm<CT>(fn, ft, ln, lg, zero) : tile_mm<16>(fn, ft, ln, lg, zero);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.Y[r0t + 4 * lg + j][c0t + ln] = acc[j];
        }
    }

    // ------------------------------- dbeta (M = N Diag(beta))
    // column sums of dM * N: over the thread's entries (one column), the two
    // halves of the wave, then the waves
    {
        float cs = 0.f;
#pragma unroll
        for (int m = 0; m < CT * CT / NTC; ++m) {
            const int e = t + NTC * m, c = e / CT, i = e % CT;
            cs = fmaf(sm.dM[c][i], sm.N[c][i], cs);
        }
        const unsigned u = __float_as_uint(cs);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        cs = __uint_as_float(r[0]) + __uint_as_float(r[1]);
        if (lane < 32) sm.red[w][lane] = cs;
    }
    __syncthreads();
    // dX = -N^T Y, strictly lower (kept in dM and the copies): tiles (0,0)
    // over both blocks, (1,0) and (1,1) over block 1 (N[m][c] = 0 for m < c)
    for (int tt = __builtin_amdgcn_readfirstlane(w); tt < 3; tt += NW) {
        const int r0t = tt ? 16 : 0, c0t = tt == 2 ? 16 : 0;
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
        const f4 acc = tt == 0 ? tile_mm<CT>([&](int r, int m) { return sm.N[m][r]; },
                                             [&](int m, int i) { return sm.Y[m][i]; }, ln, lg, zero)
                               : tile_mm<16>([&](int r, int m) { return sm.N[16 + m][r0t + r]; },
                                             [&](int m, int i) { return sm.Y[16 + m][c0t + i]; }, ln, lg, zero);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = r0t + 4 * lg + j, i = c0t + ln;
            const float v = i < c ? -acc[j] : 0.f;
            sm.dM[c][i] = v;
            sm.dXr[c][i] = v;
            sm.dXc[i][c] = v;
        }
    }
    __syncthreads();
    // dbeta: row sums of dX * L plus the waves' column sums, NTC / CT
    // consecutive lanes a row
    {
        constexpr int TPR = NTC / CT, EPR = CT / TPR;
        static_assert(NW <= TPR, "a lane per wave's column sum");
        const int c = t / TPR, part = t % TPR;
        float s = part < NW ? sm.red[part][c] : 0.f;
#pragma unroll
        for (int e = 0; e < EPR; ++e) {
            const int i = EPR * part + e;
            s = fmaf(sm.dM[c][i], sm.L[c][i], s);
        }
        s = lanes_sum<TPR>(s);
        if (part == 0 && c < nrow) a.dbeta[(b * T + r0 + c) * H + h] = s;
    }

    // ---------------------------- per (row, channel): dq, dk and dg
    // Lane (ln, lg): rows 16 p + 4 lg + j of channel x.  T1 = sum_i dA[c,i]
    // k_i d(c,i); T3 = sum_i dX[c,i] k_i d(c,i) (times beta_c below); T2 =
    // sum_c2 dA[c2,c] q~_c2 d(c2,c); T4 = sum_c2 beta_c2 dX[c2,c] k_c2
    // d(c2,c); d(c,i) = exp(G_c - G_i) for i <= c.  Every decay factor is
    // kept <= 1 by a reference row between the two rows: row 16 across the
    // blocks, the decay levels 3 and 2 within a block (pairs in different
    // 4-row groups: both orientations of a level's pairs in one product),
    // and direct exponentials within the lane's own four rows.
    use_here(rq);
    use_here(rk);
    use_here(rg);
    float qv[2][4], kv[2][4], G[2][4];
    float tot[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
        float run = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            qv[p][j] = raw_f32<TI>(rq[p][j]) * scale;
            kv[p][j] = raw_f32<TI>(rk[p][j]);
            run += __uint_as_float(rg[p][j]);
            G[p][j] = run;
        }
        tot[p] = run;
    }
    {
        // the earlier row groups of the channel (lanes ln + 16 l), block 0 before block 1
        float pre0 = 0.f, pre1 = 0.f, all0 = 0.f, t0v[4], t1v[4];
        lane_groups(tot[0], t0v);
        lane_groups(tot[1], t1v);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            pre0 += l < lg ? t0v[l] : 0.f;
            pre1 += l < lg ? t1v[l] : 0.f;
            all0 += t0v[l];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            G[0][j] += pre0;
            G[1][j] += all0 + pre1;
        }
    }
    float g16, g31;
    {
        float v0[4], v3[4];
        lane_groups(G[1][0], v0);
        lane_groups(G[1][3], v3);
        g16 = v0[0];
        g31 = v3[3];
    }
    asm volatile("" ::: "memory");
    // dg = the reverse in-chunk cumulative sum of dG plus deps * eps plus
    // sum_c d(kF)_c k_c F_c (over the channel's lanes)
    float base;
    {
        float ls = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            ls += stash[(8 + j) * NTC + t] * kv[0][j] * __expf(g31 - G[0][j]);
            ls += dkf[1][j] * kv[1][j] * __expf(g31 - G[1][j]);
        }
        ls = lanegroup4_sum(ls);
        base = deps * __expf(g31) + ls;
    }
    // block 1 first (its rows' dG sums enter block 0's dg)
#pragma unroll
    for (int p = 1; p >= 0; --p) {
        const int o = 16 * p;
        f4 aq, ak, af;          // this block's d(q~E), d(kE), d(kF)
        if (p == 1) {
            aq = dqe[1];
            ak = dke[1];
            af = dkf[1];
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                aq[j] = stash[(0 + j) * NTC + t];
                ak[j] = stash[(4 + j) * NTC + t];
                af[j] = stash[(8 + j) * NTC + t];
            }
        }
        float T1[4], T2[4], T3[4], T4[4], bt[4];
        // across the blocks through row 16: block 1's row side over block 0's
        // rows (T1, T3), block 0's column side over block 1's rows (T2, T4)
        {
            float z[4], z2[4], ex[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (p == 0) {
                    const float e1 = __expf(G[1][e] - g16);
                    z[e] = qv[1][e] * e1;
                    z2[e] = sm.beta[16 + 4 * lg + e] * kv[1][e] * e1;
                    ex[e] = __expf(g16 - G[0][e]);
                } else {
                    ex[e] = __expf(G[1][e] - g16);
                    z[e] = kv[0][e] * __expf(g16 - G[0][e]);
                    z2[e] = z[e];
                }
            }
            const f4 oa = p == 0 ? mfma_pair16(*reinterpret_cast<const f4*>(&sm.dAc[ln][16 + 4 * lg]), z)
                                 : mfma_pair16(*reinterpret_cast<const f4*>(&sm.dAr[16 + ln][4 * lg]), z);
            const f4 om = p == 0 ? mfma_pair16(*reinterpret_cast<const f4*>(&sm.dXc[ln][16 + 4 * lg]), z2)
                                 : mfma_pair16(*reinterpret_cast<const f4*>(&sm.dXr[16 + ln][4 * lg]), z2);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                T1[j] = p == 1 ? ex[j] * oa[j] : 0.f;
                T3[j] = p == 1 ? ex[j] * om[j] : 0.f;
                T2[j] = p == 0 ? ex[j] * oa[j] : 0.f;
                T4[j] = p == 0 ? ex[j] * om[j] : 0.f;
                bt[j] = sm.beta[o + 4 * lg + j];
            }
        }
        // levels 3 (8-row halves, reference row 7) and 2 (4-row halves of
        // each 8-row half, reference row 3 or 11): M Z with M[r][s] =
        // dA[max][min] on the level's pairs, Z[s] = q~_s e_s (upper s) or
        // k_s e_s (lower s), e = exp(-|G - G_ref|); likewise dX with Z'[s] =
        // beta_s k_s e_s or k_s e_s.  The reference rows are row 3 of lanes
        // ln + 16 l.
        float g3v[4];
        lane_groups(G[p][3], g3v);
        const float gref3 = g3v[1];
        const float gref2 = lg & 2 ? g3v[2] : g3v[0];
#pragma unroll
        for (int lev = 2; lev <= 3; ++lev) {
            const bool up = lev == 3 ? lg >= 2 : (lg & 1) != 0;
            const float gref = lev == 3 ? gref3 : gref2;
            float eb[4], z[4], z2[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                eb[j] = __expf(up ? G[p][j] - gref : gref - G[p][j]);
                z[j] = eb[j] * (up ? qv[p][j] : kv[p][j]);
                z2[j] = eb[j] * kv[p][j] * (up ? bt[j] : 1.f);
            }
            const bool pair = lev == 3 ? (ln >> 3) != (lg >> 1)
                                       : (ln >> 3) == (lg >> 1) && ((ln >> 2) & 1) != (lg & 1);
            // row ln after all of columns 4 lg .. 4 lg + 3: dA[ln][s] by rows, else dA[s][ln] by columns
            const bool below = ln > 4 * lg;
            const f4 ma = *reinterpret_cast<const f4*>(below ? &sm.dAr[o + ln][o + 4 * lg] : &sm.dAc[o + ln][o + 4 * lg]);
            const f4 mx = *reinterpret_cast<const f4*>(below ? &sm.dXr[o + ln][o + 4 * lg] : &sm.dXc[o + ln][o + 4 * lg]);
            const f4 zero = {0.f, 0.f, 0.f, 0.f};
            const f4 P = mfma_pair16(pair ? ma : zero, z), P2 = mfma_pair16(pair ? mx : zero, z2);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (up) {
                    T1[j] += eb[j] * P[j];
                    T3[j] += eb[j] * P2[j];
                } else {
                    T2[j] += eb[j] * P[j];
                    T4[j] += eb[j] * P2[j];
                }
            }
        }
        // the lane's own four rows (levels 0 and 1, and the diagonal):
        // pe[z][y] = exp(G_y - G_z), z < y
        float pe[4][4];
#pragma unroll
        for (int y = 1; y < 4; ++y)
#pragma unroll
            for (int z = 0; z < y; ++z) pe[z][y] = __expf(G[p][y] - G[p][z]);
        const int c0 = o + 4 * lg;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + j;
            const f4 arow = *reinterpret_cast<const f4*>(&sm.dAr[c][c0]);    // dA[c][c0 + z]
            const f4 xrow = *reinterpret_cast<const f4*>(&sm.dXr[c][c0]);
            const f4 acol = *reinterpret_cast<const f4*>(&sm.dAc[c][c0]);    // dA[c0 + z][c]
            const f4 xcol = *reinterpret_cast<const f4*>(&sm.dXc[c][c0]);
            T1[j] += arow[j] * kv[p][j];
            T2[j] += arow[j] * qv[p][j];
#pragma unroll
            for (int z = 0; z < 4; ++z) {
                if (z < j) {
                    const float d = pe[z][j] * kv[p][z];
                    T1[j] += arow[z] * d;
                    T3[j] += xrow[z] * d;
                }
                if (z > j) {
                    const float d = pe[j][z];
                    T2[j] += acol[z] * qv[p][z] * d;
                    T4[j] += bt[z] * xcol[z] * kv[p][z] * d;
                }
            }
        }
        // outputs: dq, dk per element; dG per element and its reverse sums
        float dG[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + j;
            const float E = __expf(G[p][j]), F = __expf(g31 - G[p][j]);
            const float t3 = T3[j] * bt[j];
            const float qc = qv[p][j], kc = kv[p][j];
            const float dqt = T1[j] + aq[j] * E;
            const float dk = T2[j] + t3 + T4[j] + ak[j] * E + af[j] * F;
            dG[j] = qc * T1[j] + kc * (t3 - T2[j] - T4[j]) + aq[j] * qc * E + ak[j] * kc * E - af[j] * kc * F;
            if (c < nrow) {
                const int64_t off = ((b * T + r0 + c) * H + h) * K + x;
                Elem<TI>::st(dqp + off, dqt * scale);
                Elem<TI>::st(dkp + off, dk);
            }
        }
        float acc = 0.f, sfx[4];
#pragma unroll
        for (int j = 3; j >= 0; --j) {
            acc += dG[j];
            sfx[j] = acc;
        }
        // the later row groups of the channel in this block, then block 1's
        // rows (for block 0)
        float post = 0.f, all = 0.f, accv[4];
        lane_groups(acc, accv);
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            post += l > lg ? accv[l] : 0.f;
            all += accv[l];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + j;
            if (c < nrow) a.dg[((b * T + r0 + c) * H + h) * K + x] = base + post + sfx[j];
        }
        base += all;
    }
}

// Compute units of the current device.
int cu_count() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    return cus;
}

template <int K, typename TI>
int launch_bwd(const kda_bwd_args& a, hipStream_t stream) {
    const int64_t BH = a.B * a.H;
    const int64_t nck = (a.T + CT - 1) / CT;
    const BwdWs ws = ws_layout(a.workspace, a.ckpt, BH, nck, a.K, a.V);
    // 64 state columns a workgroup, or 32 when that leaves compute units idle
    // and the 32-column workgroups still fit one round (the chain is
    // sequential: more, narrower workgroups shorten it, a second round
    // lengthens it; forward + backward at T=2048 H=16 d=128: B=4 0.80 ms
    // with 32 columns against 0.84 ms, B=6 1.05 ms with 64 against 1.19 ms)
    const int64_t cus = cu_count();
    if (a.V % 64 == 0 && (BH * (a.V / 64) >= cus || BH * (a.V / 32) > cus))
        hipLaunchKernelGGL((bwd_state_kernel<K, 64, TI>), dim3(static_cast<unsigned>(BH * (a.V / 64))), dim3(NS), 0,
                           stream, a, ws);
    else
        hipLaunchKernelGGL((bwd_state_kernel<K, 32, TI>), dim3(static_cast<unsigned>(BH * (a.V / 32))), dim3(NS), 0,
                           stream, a, ws);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    if (nck > 0) {
        hipLaunchKernelGGL((bwd_chunk_kernel<K, TI>), dim3(static_cast<unsigned>(BH * nck)), dim3(4 * K), 0, stream,
                           a, ws);
        if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    }
    return KDA_OK;
}

template <int K>
int launch_bwd_typed(const kda_bwd_args& a, hipStream_t stream) {
    switch (a.io_dtype) {
        case KDA_DTYPE_F32: return launch_bwd<K, float>(a, stream);
        case KDA_DTYPE_F16: return launch_bwd<K, _Float16>(a, stream);
        case KDA_DTYPE_BF16: return launch_bwd<K, bf16_t>(a, stream);
        default: return KDA_ERR_BAD_DTYPE;
    }
}

}  // namespace

bool chunkwise_bwd_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % VT == 0;
}

int64_t chunkwise_bwd_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V) {
    const int64_t nck = (T + CT - 1) / CT;
    return B * H * nck * (K * V + 2 * CT * V) * static_cast<int64_t>(sizeof(float));
}

// Static scratch of kda_chunkwise_bwd_noalloc: the workspace of the
// kernels (N, dS_end, dP, dR) for shapes that fit.  The array's name is
// a host-side stand-in; kernels get the device address hipGetSymbolAddress
// returns for the current device, kept per device.
static __device__ __align__(256) unsigned char scratch[KDA_BWD_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

int chunkwise_bwd_scratch(void** ptr) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KDA_ERR_LAUNCH;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return KDA_ERR_LAUNCH;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *ptr = p;
    return KDA_OK;
}

int chunkwise_bwd_launch(const kda_bwd_args& a, hipStream_t stream) {
    switch (a.K) {
        case 32: return launch_bwd_typed<32>(a, stream);
        case 64: return launch_bwd_typed<64>(a, stream);
        case 128: return launch_bwd_typed<128>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
