// Chunkwise KDA backward for gfx950: fp32 throughout.
//
// Gradient of kda_chunkwise (kimi_linear/kda.py:58-185), whose reference is
// differentiated by autograd (training: scripts/train_musicgpt_fp16.py:519-523).
// The forward is re-evaluated chunk by chunk from the checkpoints that
// kda_chunkwise_fwd_ckpt writes: per CT = 32-token chunk, the state before it
// and the chunk's R and P (below), which the forward computes anyway.
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
// everything else is independent per chunk.  Three kernels, one fp32
// workspace between them:
//   1. bwd_pairs_kernel, one workgroup per (b, h, chunk): A, L and N of every
//      chunk (functions of q, k, g and beta only).
//   2. bwd_state_kernel, one workgroup per (b, h, VA state columns), the chunks
//      in reverse: the chain above; it stores each chunk's dS_end, dP and dR
//      (fp32) and dS_0.  The next chunk's inputs are fetched into registers while
//      the current one is computed.
//   3. bwd_chunk_kernel, one workgroup per (b, h, chunk): writes dv = dR; from
//      S, R, P (checkpoint), dS_end, dP and dR the sums over all state columns
//      (VT at a time) of
//      dA, dM, d(q~E), d(kE), d(kF) and deps, then the chain through the
//      inverse, the pairwise-decay products and the reverse cumulative sum:
//      complete dq, dk, dg and dbeta.
// Rows past T read as zero inputs, which leave the state and every gradient
// of the rows before T unchanged.  q, k, v, dO and dq, dk, dv are in the
// caller's activation dtype (fp32, fp16 or bf16; every product in fp32); g,
// beta, the checkpoints, dg, dbeta and the state gradients are fp32.  The chunk-sized products run on the fp32
// matrix cores (v_mfma_f32_16x16x4f32, no precision loss).
#include <algorithm>
#include <atomic>
#include <mutex>

#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int CT = 32;          // tokens per chunk = the forward's checkpoint spacing
constexpr int VT = 32;          // state columns per step of bwd_chunk_kernel
constexpr int NT = 1024;        // threads per workgroup
static_assert(CT * VT == NT && CT * CT == NT, "one output per thread for the chunk-sized products");

// Workspace, per (b, h) and chunk (index cb = (b H + h) nck + n):
// A, L, N [CT][CT], dS_end [K][V], dP and dR [CT][V], fp32.
struct BwdWs {
    float* A;
    float* L;
    float* N;
    float* dS;
    float* dP;
    float* dR;
};

BwdWs ws_layout(void* base, int64_t BH, int64_t nck, int64_t K, int64_t V) {
    float* p = static_cast<float*>(base);
    const int64_t mat = BH * nck * CT * CT;
    BwdWs w;
    w.A = p;
    w.L = p + mat;
    w.N = p + 2 * mat;
    w.dS = p + 3 * mat;
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

constexpr int NP = 512;         // threads per workgroup of bwd_pairs_kernel

template <int K>
struct __align__(16) PairSmem {
    static constexpr int KP = K + 4;
    float q[CT][KP];            // scale * q
    float k[CT][KP];
    float gc[CT][KP];           // in-chunk cumulative log decay G
    float A[CT][CT + 1];
    float L[CT][CT + 1];
    float N[CT][CT + 1];
    float part[4][2][16][17];   // the waves' shares of A_10 and L_10; first the row groups' g sums
    float Y[16][17];
    float beta[CT];
};

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

// Eight values as fp16, two per conversion.
__device__ __forceinline__ h8 to_h8(const float (&v)[8]) {
    w4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        r[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f2v{v[2 * e], v[2 * e + 1]}, hf2));
    return __builtin_bit_cast(h8, r);
}

__device__ __forceinline__ void lds8(const float* p, float (&v)[8]) {
    const f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        v[e] = a[e];
        v[4 + e] = b[e];
    }
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

// A, L and N of every chunk.  Every decay factor is a product of per-token
// decays between two rows, kept <= 1 by factoring through a reference row
// between them:
//  * diagonal 16-row blocks, by decay level: a pair i < c of a block has a
//    unique highest differing bit lev; both rows sit in the aligned group of
//    2^(lev+1) rows whose lower half ends at ref(c) = ref(i), i <= ref < c,
//    and exp(G_c - G_i) = exp(G_c - G_ref) exp(G_ref - G_i).  Per level, with
//    f_r = exp(-|G_r - G_ref(r)|) for every row r of the block (ref(r): r's
//    reference row at that level, r in either half), the products
//    (q~ f)(k f)^T and (k f)(k f)^T over the channels hold A and L on that
//    level's pairs (c upper, i lower); a row r whose low lev bits are all
//    ones and bit lev clear is its own reference row (f_r = 1), so the
//    diagonal A[r][r] comes from that level's product too, except for the
//    block's row 15, one dot product of its own;
//  * the block below the diagonal, through row 15 (the reference row of
//    every such pair).
// Products on the bf16 matrix cores as hi/lo pairs (~2^-17 relative each).
// N = (I + X)^-1 per diagonal block, X = Diag(beta) L nilpotent:
// (I - X)(I + X^2)(I + X^4)(I + X^8) on the fp32 matrix cores in registers,
// then N10 = -N11 X10 N00.
// Wave w: block w / 4, level w % 4; waves 0 .. K/32 - 1 also one 32-channel
// step of the block below the diagonal.  Persistent: workgroup g takes
// chunks g, g + G, ... (G workgroups) and fetches the next one's inputs into
// registers while the current one is computed.
template <int K, typename TI>
__global__ __launch_bounds__(NP) void bwd_pairs_kernel(const kda_bwd_args a, const BwdWs ws, int64_t nchunks) {
    static_assert(NP % K == 0 && (CT * K) % NP == 0 && NP / K <= 4 * 2 * 16 * 17, "thread mapping");
    static_assert(NP / 64 == 8 && K / 32 <= 4, "wave roles");
    constexpr int RPT = CT * K / NP;        // consecutive rows per thread, one channel
    constexpr bool PAIR = sizeof(TI) == 4;  // fp32 activations: bf16 pairs; 16-bit: fp16 operands
    constexpr float kLog2e = 1.4426950408889634f;
    __shared__ PairSmem<K> sm;
    const TI* qp = static_cast<const TI*>(a.q);
    const TI* kp = static_cast<const TI*>(a.k);
    const int64_t H = a.H, T = a.T;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int kk = t % K, rg = t / K;
    const uint32_t HK = static_cast<uint32_t>(H * K);

    // thread (rg, kk): rows RPT rg .. RPT rg + RPT - 1 of channel kk, fetched
    // raw through descriptors that span the chunk's rows before T (rows past
    // T read as zero) with one lane offset per tensor and the row in the
    // scalar offset
    uint32_t pq[RPT], pk[RPT], pg[RPT], pb[1] = {0u};
    const uint32_t lo_x = static_cast<uint32_t>(RPT * rg) * HK + kk;
    auto fetch = [&](int64_t cb) {
        const int64_t bh = cb / nck, b = bh / H, h = bh % H;
        const int64_t r0 = (cb % nck) * CT;
        const int64_t base = ((b * T + r0) * H + h) * K;
        const uint32_t span = static_cast<uint32_t>((std::min<int64_t>(CT, T - r0) - 1) * H * K + K);
        const auto rq = make_rsrc(qp + base, span * sizeof(TI)), rk = make_rsrc(kp + base, span * sizeof(TI));
        const auto rgc = make_rsrc(a.g + base, span * 4);
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const uint32_t so = static_cast<uint32_t>(j) * HK;
            if constexpr (sizeof(TI) == 2) {
                pq[j] = __builtin_amdgcn_raw_buffer_load_b16(rq, static_cast<int>(2 * lo_x), static_cast<int>(2 * so), 0);
                pk[j] = __builtin_amdgcn_raw_buffer_load_b16(rk, static_cast<int>(2 * lo_x), static_cast<int>(2 * so), 0);
            } else {
                pq[j] = __builtin_amdgcn_raw_buffer_load_b32(rq, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
                pk[j] = __builtin_amdgcn_raw_buffer_load_b32(rk, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
            }
            pg[j] = __builtin_amdgcn_raw_buffer_load_b32(rgc, static_cast<int>(4 * lo_x), static_cast<int>(4 * so), 0);
        }
        if (t < CT) pb[0] = r0 + t < T ? __float_as_uint(a.beta[(b * T + r0 + t) * H + h]) : 0u;
    };
    int64_t cb = blockIdx.x;
    if (cb < nchunks) fetch(cb);
    for (; cb < nchunks; cb += gridDim.x) {
        // stage this chunk (G from per-thread partial sums and the row-group
        // totals); fetch the next one
        use_here(pq);
        use_here(pk);
        use_here(pg);
        use_here(pb);
        float gl[RPT];
        float run = 0.f;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int c = RPT * rg + j;
            sm.q[c][kk] = raw_f32<TI>(pq[j]) * a.scale;
            sm.k[c][kk] = raw_f32<TI>(pk[j]);
            run += __uint_as_float(pg[j]);
            gl[j] = run;
        }
        float* tot = &sm.part[0][0][0][0];
        tot[rg * K + kk] = run;
        if (t < CT) sm.beta[t] = __uint_as_float(pb[0]);
        if (cb + gridDim.x < nchunks) fetch(cb + gridDim.x);
        __syncthreads();
        {
            float pre = 0.f;
#pragma unroll
            for (int r = 0; r < NP / K; ++r) pre += r < rg ? tot[r * K + kk] : 0.f;
#pragma unroll
            for (int j = 0; j < RPT; ++j) sm.gc[RPT * rg + j][kk] = pre + gl[j];
        }
        __syncthreads();

        // diagonal blocks by level; lane (ln, lg) supplies row ln of both
        // operands, channels 32 u + 8 lg .. + 7 of step u, and holds entry
        // (c, i) = (4 lg + j, ln) of the block in slot j
        {
            const int p = w >> 2, lev = w & 3;
            const int r = 16 * p + ln;
            const bool up = (ln >> lev) & 1;
            const int ref = 16 * p + (up ? ((ln >> lev) << lev) - 1 : (ln | ((1 << lev) - 1)));
            // f = exp(G_r - G_ref) (upper rows) or exp(G_ref - G_r) (lower rows)
            const float sg = up ? kLog2e : -kLog2e;
            f4 accA = {0.f, 0.f, 0.f, 0.f}, accL = accA;
            float d15 = 0.f;                    // row 15's diagonal (lanes ln = 15 of level 0)
#pragma unroll 1
            for (int u = 0; u < K / 32; ++u) {
                const int x0 = 32 * u + 8 * lg;
                float qv[8], kv[8], gr[8], gf[8];
                lds8(&sm.q[r][x0], qv);
                lds8(&sm.k[r][x0], kv);
                lds8(&sm.gc[r][x0], gr);
                lds8(&sm.gc[ref][x0], gf);
                if (lev == 0) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) d15 = fmaf(qv[e], kv[e], d15);
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float f = __builtin_amdgcn_exp2f((gr[e] - gf[e]) * sg);
                    qv[e] *= f;
                    kv[e] *= f;
                }
                if constexpr (PAIR) {
                    bf8 qh, ql, kh, kl;
                    split8(qv, qh, ql);
                    split8(kv, kh, kl);
                    accA = mfma_pair(qh, ql, kh, kl, accA);
                    accL = mfma_pair(kh, kl, kh, kl, accL);
                } else {
                    const h8 qh = to_h8(qv), kh = to_h8(kv);
                    accA = mfma16x16x32(qh, kh, accA);
                    accL = mfma16x16x32(kh, kh, accL);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = 4 * lg + j, i = ln;
                const int x = c ^ i;
                // the diagonal entry of level lev: c's low lev bits ones, bit lev clear
                const bool diag = x == 0 && ((c + 1) & ((2 << lev) - 1)) == (1 << lev);
                if ((x >> lev) == 1 || diag) {
                    sm.A[16 * p + c][16 * p + i] = c >= i ? accA[j] : 0.f;
                    sm.L[16 * p + c][16 * p + i] = c > i ? accL[j] : 0.f;
                }
            }
            if (lev == 0) {
                d15 += __shfl_xor(d15, 16);
                d15 += __shfl_xor(d15, 32);
                if (lane == 15) {
                    sm.A[16 * p + 15][16 * p + 15] = d15;
                    sm.L[16 * p + 15][16 * p + 15] = 0.f;
                }
            }
        }
        __syncthreads();

        if (w < 2) {
            // N_pp = (I + X)^-1, X = Diag(beta) L_pp, in accumulator layout
            const int o = 16 * w;
            f4 X, XT;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                X[j] = sm.beta[o + 4 * lg + j] * sm.L[o + 4 * lg + j][o + ln];
                XT[j] = sm.beta[o + ln] * sm.L[o + ln][o + 4 * lg + j];
            }
            const f4 z = {0.f, 0.f, 0.f, 0.f};
            const f4 X2 = mm_acc(XT, X, z), X2T = mm_acc(X, XT, z);
            const f4 X4 = mm_acc(X2T, X2, z), X4T = mm_acc(X2, X2T, z);
            const f4 X8T = mm_acc(X4, X4T, z);
            f4 Q;
#pragma unroll
            for (int j = 0; j < 4; ++j) Q[j] = (4 * lg + j == ln ? 1.f : 0.f) - X[j];
            Q = mm_acc(X2T, Q, Q);
            Q = mm_acc(X4T, Q, Q);
            Q = mm_acc(X8T, Q, Q);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.N[o + 4 * lg + j][o + ln] = Q[j];
        } else if (w >= 4 && w - 4 < K / 32) {
            // the block below the diagonal, one 32-channel step per wave: rows
            // 16 + ln (X) and ln (Y), reference row 15
            const int s4 = w - 4, x0 = 32 * s4 + 8 * lg;
            float q1[8], k1[8], g1[8], k0[8], g0[8], g15[8];
            lds8(&sm.q[16 + ln][x0], q1);
            lds8(&sm.k[16 + ln][x0], k1);
            lds8(&sm.gc[16 + ln][x0], g1);
            lds8(&sm.k[ln][x0], k0);
            lds8(&sm.gc[ln][x0], g0);
            lds8(&sm.gc[15][x0], g15);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float f1 = __builtin_amdgcn_exp2f((g1[e] - g15[e]) * kLog2e);
                q1[e] *= f1;
                k1[e] *= f1;
                k0[e] *= __builtin_amdgcn_exp2f((g15[e] - g0[e]) * kLog2e);
            }
            f4 accA = {0.f, 0.f, 0.f, 0.f}, accL = accA;
            if constexpr (PAIR) {
                bf8 qh, ql, kh, kl, yh, yl;
                split8(q1, qh, ql);
                split8(k1, kh, kl);
                split8(k0, yh, yl);
                accA = mfma_pair(qh, ql, yh, yl, accA);
                accL = mfma_pair(kh, kl, yh, yl, accL);
            } else {
                const h8 qh = to_h8(q1), kh = to_h8(k1), yh = to_h8(k0);
                accA = mfma16x16x32(qh, yh, accA);
                accL = mfma16x16x32(kh, yh, accL);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sm.part[s4][0][4 * lg + j][ln] = accA[j];
                sm.part[s4][1][4 * lg + j][ln] = accL[j];
            }
        }
        __syncthreads();

        if (t < 64) {
            // Y <- X10 N00, X10 = Diag(beta_1) L10 (L10 from the shares); N10 = -N11 Y
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mm<16>(
                [&](int r, int m) {
                    float l = 0.f;
#pragma unroll
                    for (int x = 0; x < K / 32; ++x) l += sm.part[x][1][r][m];
                    return sm.beta[16 + r] * l;
                },
                [&](int m, int i) { return sm.N[m][i]; }, ln, lg, acc);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.Y[4 * lg + j][ln] = acc[j];
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            acc = f4{0.f, 0.f, 0.f, 0.f};
            acc = tile_mm<16>([&](int r, int m) { return sm.N[16 + r][16 + m]; },
                              [&](int m, int i) { return sm.Y[m][i]; }, ln, lg, acc);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.N[16 + 4 * lg + j][ln] = -acc[j];
        } else if (w >= 4) {
            // A_10, L_10 from the shares; zeros above the diagonal blocks
            const int e = t - 256, c = e >> 4, i = e & 15;
            float sa = 0.f, sl = 0.f;
#pragma unroll
            for (int x = 0; x < K / 32; ++x) {
                sa += sm.part[x][0][c][i];
                sl += sm.part[x][1][c][i];
            }
            sm.A[16 + c][i] = sa;
            sm.L[16 + c][i] = sl;
            sm.A[c][16 + i] = 0.f;
            sm.L[c][16 + i] = 0.f;
            sm.N[c][16 + i] = 0.f;
        }
        __syncthreads();
        // the next chunk's staging writes none of A, L, N
        float* ga = ws.A + cb * CT * CT;
        float* gL = ws.L + cb * CT * CT;
        float* gn = ws.N + cb * CT * CT;
#pragma unroll
        for (int j = 0; j < CT * CT / NP; ++j) {
            const int e = t + NP * j;
            ga[e] = sm.A[e / CT][e % CT];
            gL[e] = sm.L[e / CT][e % CT];
            gn[e] = sm.N[e / CT][e % CT];
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

template <int K, int VA>
struct __align__(16) StateSmem {
    static constexpr int KB = K + 8, TB = CT + 8;
    uint16_t qeT[2][K][TB];     // (scale q exp(G))^T: [channel][token]
    uint16_t keT[2][K][TB];     // (k exp(G))^T
    uint16_t kf[2][CT][KB];     // k exp(G_last - G): [token][channel]
    uint16_t dST[2][VA][KB];    // dS^T at the chunk end: [column][channel]
    uint16_t dOT[2][VA][TB];    // dO^T: [column][token]
    uint16_t dPT[2][VA][TB];
    uint16_t dRT[2][VA][TB];
    uint16_t AT[2][CT][TB];     // A^T: [c][c2] = A[c2][c]
    uint16_t NT_[2][CT][TB];    // N^T
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
    __shared__ StateSmem<K, VA> sm;
    const TI* qp = static_cast<const TI*>(a.q);
    const TI* kp = static_cast<const TI*>(a.k);
    const TI* dop = static_cast<const TI*>(a.d_o);

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nva = static_cast<int>(V / VA);
    const int64_t bh = blockIdx.x / nva, b = bh / H, h = bh % H;
    const int64_t v0 = static_cast<int64_t>(blockIdx.x % nva) * VA;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int x = t % K, rg = t / K;

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
            put4_pair(&sm.dST[0][c0 + ln][r0 + 4 * lg], &sm.dST[1][c0 + ln][r0 + 4 * lg], accs[m]);
        }
    }

    // fetched elements stay in the input dtype until they are staged: a
    // conversion next to its load would wait for it
    TI pq[RPT], pk[RPT], pdo[DPT];
    float pg[RPT], pa[APT], pn[APT], pb = 0.f;
    // global addresses as a per-chunk uniform base plus a loop-invariant
    // 32-bit offset per thread (registers for the pipeline, not for addresses)
    const uint32_t HK = static_cast<uint32_t>(H * K), HV = static_cast<uint32_t>(H * V);
    const uint32_t oqk = static_cast<uint32_t>(RPT * rg) * HK + x;
    auto fetch = [&](int n) {
        const int64_t r0 = static_cast<int64_t>(n) * CT;
        const TI* qn = qp + ((b * T + r0) * H + h) * K;
        const TI* kn = kp + ((b * T + r0) * H + h) * K;
        const float* gn = a.g + ((b * T + r0) * H + h) * K;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            pq[j] = pk[j] = TI{};
            pg[j] = 0.f;
            if (r0 + RPT * rg + j < T) {
                const uint32_t o = oqk + j * HK;
                pq[j] = qn[o];
                pk[j] = kn[o];
                pg[j] = gn[o];
            }
        }
        const TI* don = dop + ((b * T + r0) * H + h) * V + v0;
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int e = t + NS * j;
            pdo[j] = r0 + e / VA < T ? don[static_cast<uint32_t>(e / VA) * HV + e % VA] : TI{};
        }
        const int64_t cb = bh * nck + n;
#pragma unroll
        for (int j = 0; j < APT; ++j) {
            pa[j] = ws.A[cb * CT * CT + t + NS * j];
            pn[j] = ws.N[cb * CT * CT + t + NS * j];
        }
        if (t < CT) pb = r0 + t < T ? a.beta[(b * T + r0) * H + h + static_cast<uint32_t>(t) * H] : 0.f;
    };
    if (nck > 0) fetch(nck - 1);

    for (int n = nck - 1; n >= 0; --n) {
        const int64_t cb = bh * nck + n;
        // stage chunk n (A^T, N^T, dO^T as pairs, the row groups' g sums); fetch chunk n - 1
        float cq[RPT], ck[RPT], cg[RPT];
        float run = 0.f;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            run += pg[j];
            cg[j] = run;
            cq[j] = Elem<TI>::ld(&pq[j]);
            ck[j] = Elem<TI>::ld(&pk[j]);
        }
        sm.tot[rg][x] = run;
#pragma unroll
        for (int j = 0; j < APT; ++j) {
            const int e = t + NS * j;
            split_bf16(pa[j], sm.AT[0][e % CT][e / CT], sm.AT[1][e % CT][e / CT]);
            split_bf16(pn[j], sm.NT_[0][e % CT][e / CT], sm.NT_[1][e % CT][e / CT]);
        }
#pragma unroll
        for (int j = 0; j < DPT; ++j) {
            const int e = t + NS * j, c = e / VA, v = e % VA;
            split_bf16(Elem<TI>::ld(&pdo[j]), sm.dOT[0][v][c], sm.dOT[1][v][c]);
        }
        if (t < CT) sm.beta[t] = pb;
        if (n > 0) fetch(n - 1);
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
#pragma unroll
            for (int j = 0; j < RPT; ++j) {
                const int c = RPT * rg + j;
                const float G = pre + cg[j];
                const float E = __expf(G), F = __expf(last - G);
                split_bf16(a.scale * cq[j] * E, sm.qeT[0][x][c], sm.qeT[1][x][c]);
                split_bf16(ck[j] * E, sm.keT[0][x][c], sm.keT[1][x][c]);
                split_bf16(ck[j] * F, sm.kf[0][c][x], sm.kf[1][c][x]);
            }
            if (rg == 0) sm.eps[x] = __expf(last);
        }
        __syncthreads();

        // dS_end to the workspace; dP = (k*F) dS + A^T dO; dS <- Diag(eps) dS + (q~*E)^T dO
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
                float* dsn = ws.dS + cb * K * V + v0;
#pragma unroll
                for (int j = 0; j < 4; ++j) dsn[static_cast<uint32_t>(r0 + 4 * lg + j) * V + c0 + ln] = accs[m][j];
            }
        }
        if (w < NDP) {
            const int r0t = 16 * (w / VTL), c0t = 16 * (w % VTL);
            f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < K / 32; ++u)
                acc = mm_pair(&sm.kf[0][r0t + ln][32 * u], &sm.kf[1][r0t + ln][32 * u], &sm.dST[0][c0t + ln][32 * u],
                              &sm.dST[1][c0t + ln][32 * u], lg, acc);
            acc = mm_pair(sm.AT[0][r0t + ln], sm.AT[1][r0t + ln], sm.dOT[0][c0t + ln], sm.dOT[1][c0t + ln], lg, acc);
            float* dpn = ws.dP + cb * CT * V + v0;
#pragma unroll
            for (int j = 0; j < 4; ++j) dpn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln] = acc[j];
            put4_pair(&sm.dPT[0][c0t + ln][r0t + 4 * lg], &sm.dPT[1][c0t + ln][r0t + 4 * lg], acc);
        }
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
#pragma unroll
                for (int j = 0; j < 4; ++j) accs[m][j] *= sm.eps[r0 + 4 * lg + j];
                accs[m] = mm_pair(sm.qeT[0][r0 + ln], sm.qeT[1][r0 + ln], sm.dOT[0][c0 + ln], sm.dOT[1][c0 + ln], lg,
                                  accs[m]);
            }
        }
        __syncthreads();

        // dR = M^T dP = Diag(beta) N^T dP (= dV, which bwd_chunk_kernel writes out)
        if (w < NDP) {
            const int r0t = 16 * (w / VTL), c0t = 16 * (w % VTL);
            f4 acc = mm_pair(sm.NT_[0][r0t + ln], sm.NT_[1][r0t + ln], sm.dPT[0][c0t + ln], sm.dPT[1][c0t + ln], lg,
                             f4{0.f, 0.f, 0.f, 0.f});
            float* drn = ws.dR + cb * CT * V + v0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[j] *= sm.beta[r0t + 4 * lg + j];
                drn[static_cast<uint32_t>(r0t + 4 * lg + j) * V + c0t + ln] = acc[j];
            }
            put4_pair(&sm.dRT[0][c0t + ln][r0t + 4 * lg], &sm.dRT[1][c0t + ln][r0t + 4 * lg], acc);
        }
        __syncthreads();

        // dS_start = Diag(eps) dS + (q~*E)^T dO - (k*E)^T dR, and its pair copy
        // for the next chunk's dP (read after the next chunk's first barrier)
#pragma unroll
        for (int m = 0; m < TPW; ++m) {
            const int ti = w + NWS * m;
            if (ti < NTS) {
                const int r0 = 16 * (ti / VTL), c0 = 16 * (ti % VTL);
                const f4 kr = mm_pair(sm.keT[0][r0 + ln], sm.keT[1][r0 + ln], sm.dRT[0][c0 + ln], sm.dRT[1][c0 + ln],
                                      lg, f4{0.f, 0.f, 0.f, 0.f});
                accs[m] -= kr;
                put4_pair(&sm.dST[0][c0 + ln][r0 + 4 * lg], &sm.dST[1][c0 + ln][r0 + 4 * lg], accs[m]);
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

// Rows padded to a multiple of 4 floats plus 4: 16-byte vector reads along a
// row, and consecutive rows 4 banks apart.
// The column step's tiles: S and dS (K rows), dO, R, P, dP, dR (CT rows), VT
// columns each.  PAIR (16-bit activations): bf16 pairs, x = hi + lo (hi = x
// rounded to bf16, lo = the rest rounded to bf16: |x - hi - lo| <= 2^-18 |x|),
// rows of VB elements (80 bytes: every MFMA fragment, 8 consecutive columns,
// is one 16-byte read), for the bf16 matrix cores.  Otherwise (fp32
// activations) fp32 rows of VP floats for the fp32 matrix cores, exact
// products.
constexpr int VB = VT + 8;
constexpr int VP = VT + 4;
template <int K, bool PAIR>
struct StepTiles;
template <int K>
struct StepTiles<K, true> {
    uint16_t S[2][K][VB];       // state at the chunk start (checkpoint): hi, lo
    uint16_t dS[2][K][VB];      // gradient of the state at the chunk end
    uint16_t dO[2][CT][VB];
    uint16_t R[2][CT][VB];
    uint16_t P[2][CT][VB];
    uint16_t dP[2][CT][VB];
    uint16_t dR[2][CT][VB];
};
template <int K>
struct StepTiles<K, false> {
    float S[K][VP];
    float dS[K][VP];
    float dO[CT][VP];
    float R[CT][VP];
    float P[CT][VP];
    float dP[CT][VP];
    float dR[CT][VP];
};
template <int K, bool PAIR>
struct __align__(16) ChunkSmem {
    static constexpr int KP = K + 4;
    float q[CT][KP];            // scale * q
    float k[CT][KP];
    float gc[CT][KP];           // in-chunk cumulative log decay G
    float e[CT][KP];            // exp(G); then, per element, dG
    StepTiles<K, PAIR> st;
    float A[CT][CT + 1];        // A (i <= c)
    float L[CT][CT + 1];        // L (i < c)
    float N[CT][CT + 1];        // (I + Diag(beta) L)^-1
    float dA[CT][CT + 1];       // dA (i <= c)
    float dM[CT][CT + 1];       // dM, then dN, then dX
    float Y[CT][CT + 1];        // dN N^T; then, per thread, its rows' share of
                                // sum_c d(k*F)[c] k[c] F[c] (NT floats)
    float beta[CT];
    float dbeta[CT];
    float eps[K];               // exp(G_last)
    float deps[K];              // rowsum(dS * S)
    // the element step's copies of dA and dX live in the dS area when it is
    // large enough (K = 128), here otherwise
    static constexpr int CPY = 4 * CT * (CT + 4);
    static constexpr bool CPY_IN_DS = sizeof(StepTiles<K, PAIR>::dS) / 4 >= CPY;   // floats in the dS area
    float cpy[CPY_IN_DS ? 4 : CPY];
};
static_assert(CT * (CT + 1) >= NT, "the per-thread shares fit Y");

template <int K, typename TI>
__global__ __launch_bounds__(NT) void bwd_chunk_kernel(const kda_bwd_args a, const BwdWs ws) {
    static_assert(NT % K == 0 && (CT * K) % NT == 0, "thread mapping");
    constexpr int RPT = CT * K / NT;        // consecutive rows per thread, one channel
    constexpr int SPT = K * VT / NT;        // state tile elements per thread
    constexpr int TPR = VT / SPT;           // threads per state row
    static_assert(NT / K * K <= CT * (CT + 1), "the row-group sums fit Y");
    constexpr bool PAIR = sizeof(TI) == 2;
    __shared__ ChunkSmem<K, PAIR> sm;
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
    const int nvt = static_cast<int>(V / VT);
    const float scale = a.scale;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;
    const int kk = t % K, rg = t / K;

    // ---------------------------------------------------------------- loads
    // thread (rg, kk): rows RPT rg .. RPT rg + RPT - 1 of channel kk.  The
    // first column step's tiles are fetched right behind these loads.
    float ql[RPT], kl[RPT], gl[RPT];
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int64_t row = static_cast<int64_t>(n) * CT + RPT * rg + j;
        ql[j] = kl[j] = gl[j] = 0.f;
        if (row < T) {
            const int64_t o = ((b * T + row) * H + h) * K + kk;
            ql[j] = Elem<TI>::ld(qp + o) * scale;
            kl[j] = Elem<TI>::ld(kp + o);
            gl[j] = a.g[o];
        }
    }
    const float al = ws.A[cb * CT * CT + t], ll = ws.L[cb * CT * CT + t], nl = ws.N[cb * CT * CT + t];
    float bl = 0.f;
    if (t < CT) {
        const int64_t row = static_cast<int64_t>(n) * CT + t;
        bl = row < T ? a.beta[(b * T + row) * H + h] : 0.f;
    }

    // the checkpoint of chunk cb: the state before it (K rows), then its R
    // and P (CT rows each), V columns
    const float* ck = a.ckpt + cb * static_cast<int64_t>(K + 2 * CT) * V;
    float ps[SPT], pds[SPT], pr = 0.f, pp = 0.f, pdp = 0.f, pdr = 0.f;
    TI pdo{};                               // converted when staged
    const int st_row = t / TPR, st_col = SPT * (t % TPR);
    const int tc = t / VT, tv = t % VT;
    auto fetch = [&](int vt) {
        const int64_t v0 = static_cast<int64_t>(vt) * VT;
#pragma unroll
        for (int j = 0; j < SPT; ++j) {
            ps[j] = ck[st_row * V + v0 + st_col + j];
            pds[j] = ws.dS[(cb * K + st_row) * V + v0 + st_col + j];
        }
        pr = ck[(K + tc) * V + v0 + tv];
        pp = ck[(K + CT + tc) * V + v0 + tv];
        pdp = ws.dP[(cb * CT + tc) * V + v0 + tv];
        pdr = ws.dR[(cb * CT + tc) * V + v0 + tv];
        const int64_t row = static_cast<int64_t>(n) * CT + tc;
        pdo = TI{};
        if (row < T) pdo = dop[((b * T + row) * H + h) * V + v0 + tv];
    };
    fetch(0);

    float run = 0.f;
#pragma unroll
    for (int j = 0; j < RPT; ++j) {
        const int c = RPT * rg + j;
        sm.q[c][kk] = ql[j];
        sm.k[c][kk] = kl[j];
        run += gl[j];
        gl[j] = run;
    }
    float* tot = &sm.Y[0][0];               // [NT / K][K]: per row group, the sum of its g
    tot[rg * K + kk] = run;
    if (t < CT) sm.beta[t] = bl;
    sm.A[t / CT][t % CT] = al;
    sm.L[t / CT][t % CT] = ll;
    sm.N[t / CT][t % CT] = nl;
    __syncthreads();

    // ------------------------------------------- cumulative decays, eps
    {
        float pre = 0.f, last = 0.f;
#pragma unroll
        for (int r = 0; r < NT / K; ++r) {
            const float x = tot[r * K + kk];
            pre += r < rg ? x : 0.f;
            last += x;
        }
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int c = RPT * rg + j;
            sm.gc[c][kk] = pre + gl[j];
            sm.e[c][kk] = __expf(pre + gl[j]);
        }
        if (rg == 0) sm.eps[kk] = __expf(last);
    }

    // ------------------------------------- sums over the state columns
    // per VT-column step (R and P from the forward's checkpoint):
    // dA += dO P^T, dM += dP R^T, d(q~*E) += dO S^T, d(k*E) -= dR S^T,
    // d(k*F) += P dS^T, deps += rowsum(dS * S).  The next step's tiles are
    // fetched into registers while the current one is computed.

    constexpr int KTL = K / 16;
    const bool tw = w < 2 * KTL;
    // element tile of this wave: rows 16 (w / KTL) + 4 lg + j, channel 16 (w % KTL) + ln
    const int ert = 16 * (w / KTL), ekk = 16 * (w % KTL) + ln;
    // CT x CT tile of waves 0-7: rows r0t + 4 lg + j, columns c0t + ln
    const int r0t = 16 * ((w >> 1) & 1), c0t = 16 * (w & 1);
    f4 accm = {0.f, 0.f, 0.f, 0.f};         // dA (waves 0-3), dM (waves 4-7)
    f4 dqe = accm, dke = accm, dkf = accm;
    float deps = 0.f;            // this thread's share of rowsum(dS * S) for row st_row
    for (int vt = 0; vt < nvt; ++vt) {
        auto& tl = sm.st;
#pragma unroll
        for (int j = 0; j < SPT; ++j) deps = fmaf(pds[j], ps[j], deps);
        if constexpr (PAIR) {
#pragma unroll
            for (int j = 0; j < SPT; ++j) {
                split_bf16(ps[j], tl.S[0][st_row][st_col + j], tl.S[1][st_row][st_col + j]);
                split_bf16(pds[j], tl.dS[0][st_row][st_col + j], tl.dS[1][st_row][st_col + j]);
            }
            split_bf16(pr, tl.R[0][tc][tv], tl.R[1][tc][tv]);
            split_bf16(pp, tl.P[0][tc][tv], tl.P[1][tc][tv]);
            split_bf16(Elem<TI>::ld(&pdo), tl.dO[0][tc][tv], tl.dO[1][tc][tv]);
            split_bf16(pdp, tl.dP[0][tc][tv], tl.dP[1][tc][tv]);
            split_bf16(pdr, tl.dR[0][tc][tv], tl.dR[1][tc][tv]);
        } else {
#pragma unroll
            for (int j = 0; j < SPT; ++j) {
                tl.S[st_row][st_col + j] = ps[j];
                tl.dS[st_row][st_col + j] = pds[j];
            }
            tl.R[tc][tv] = pr;
            tl.P[tc][tv] = pp;
            tl.dO[tc][tv] = Elem<TI>::ld(&pdo);
            tl.dP[tc][tv] = pdp;
            tl.dR[tc][tv] = pdr;
        }
        {
            const int64_t row = static_cast<int64_t>(n) * CT + tc;
            if (row < T) Elem<TI>::st(dvp + ((b * T + row) * H + h) * V + static_cast<int64_t>(vt) * VT + tv, pdr);
        }
        if (vt + 1 < nvt) fetch(vt + 1);
        __syncthreads();

        // waves 0-3: dA += dO P^T; waves 4-7: dM += dP R^T; every element wave:
        // d(q~E) += dO S^T, d(kE) -= dR S^T (accumulated as + and negated
        // below), d(kF) += P dS^T
        if constexpr (PAIR) {
            if (w < 8) {
                const uint16_t (*xa)[CT][VB] = w < 4 ? tl.dO : tl.dP;
                const uint16_t (*ya)[CT][VB] = w < 4 ? tl.P : tl.R;
                accm = mm_pair(xa[0][r0t + ln], xa[1][r0t + ln], ya[0][c0t + ln], ya[1][c0t + ln], lg, accm);
            }
            if (tw) {
                const int er = ert + ln, sr = ekk;      // rows of the element tile and of its channels
                dqe = mm_pair(tl.dO[0][er], tl.dO[1][er], tl.S[0][sr], tl.S[1][sr], lg, dqe);
                dke = mm_pair(tl.dR[0][er], tl.dR[1][er], tl.S[0][sr], tl.S[1][sr], lg, dke);
                dkf = mm_pair(tl.P[0][er], tl.P[1][er], tl.dS[0][sr], tl.dS[1][sr], lg, dkf);
            }
        } else {
            if (w < 4)
                accm = tile_mm<VT>([&](int r, int v) { return tl.dO[r0t + r][v]; },
                                   [&](int v, int i) { return tl.P[c0t + i][v]; }, ln, lg, accm);
            else if (w < 8)
                accm = tile_mm<VT>([&](int r, int v) { return tl.dP[r0t + r][v]; },
                                   [&](int v, int i) { return tl.R[c0t + i][v]; }, ln, lg, accm);
            if (tw) {
                dqe = tile_mm<VT>([&](int r, int v) { return tl.dO[ert + r][v]; },
                                  [&](int v, int kc) { return tl.S[ekk - ln + kc][v]; }, ln, lg, dqe);
                dke = tile_mm<VT>([&](int r, int v) { return tl.dR[ert + r][v]; },
                                  [&](int v, int kc) { return tl.S[ekk - ln + kc][v]; }, ln, lg, dke);
                dkf = tile_mm<VT>([&](int r, int v) { return tl.P[ert + r][v]; },
                                  [&](int v, int kc) { return tl.dS[ekk - ln + kc][v]; }, ln, lg, dkf);
            }
        }
        __syncthreads();
    }
    dke = f4{0.f, 0.f, 0.f, 0.f} - dke;
    // deps: the shares of the TPR threads of each state row
#pragma unroll
    for (int m = 1; m < TPR; m <<= 1) deps += __shfl_xor(deps, m);
    // 16-byte-aligned copies for the element step (in the dS area, no longer
    // read, when it is large enough): dA by rows and by columns, dX (the
    // final dM) by rows and by columns
    float* cpy = ChunkSmem<K, PAIR>::CPY_IN_DS ? reinterpret_cast<float*>(&sm.st.dS) : &sm.cpy[0];
    float (*dAr)[CT + 4] = reinterpret_cast<float (*)[CT + 4]>(cpy);
    float (*dAc)[CT + 4] = dAr + CT;
    float (*dXr)[CT + 4] = dAr + 2 * CT;
    float (*dXc)[CT + 4] = dAr + 3 * CT;
    if (w < 8) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = r0t + 4 * lg + j, i = c0t + ln;
            const float x = i <= c ? accm[j] : 0.f;
            if (w < 4) {
                sm.dA[c][i] = x;
                dAr[c][i] = x;
                dAc[i][c] = x;
            } else {
                sm.dM[c][i] = x;
            }
        }
    }
    if (t % TPR == 0) sm.deps[st_row] = deps;
    __syncthreads();

    // ------------------------------- dbeta (M = N Diag(beta)), dN in place
    // column sums of dM * N: over the two rows of each wave, then over the waves
    float* red = reinterpret_cast<float*>(&sm.st.S);   // [NT / 64][CT]; S is no longer read
    {
        const int c = t / CT, i = t % CT;
        const float dm = sm.dM[c][i];
        float p = dm * sm.N[c][i];
        p += __shfl_xor(p, 32);
        if (lane < 32) red[w * CT + i] = p;
        sm.dM[c][i] = dm * sm.beta[i];
    }
    __syncthreads();
    // Y = dN N^T
    if (w < 4) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mm<CT>([&](int r, int m) { return sm.dM[r0t + r][m]; },
                          [&](int m, int i) { return sm.N[c0t + i][m]; }, ln, lg, acc);
#pragma unroll
        for (int j = 0; j < 4; ++j) sm.Y[r0t + 4 * lg + j][c0t + ln] = acc[j];
    }
    __syncthreads();
    // dX = -N^T Y, strictly lower (kept in dM)
    if (w < 4) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = tile_mm<CT>([&](int r, int m) { return sm.N[m][r0t + r]; },
                          [&](int m, int i) { return sm.Y[m][c0t + i]; }, ln, lg, acc);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = r0t + 4 * lg + j, i = c0t + ln;
            const float x = i < c ? -acc[j] : 0.f;
            sm.dM[c][i] = x;
            dXr[c][i] = x;
            dXc[i][c] = x;
        }
    }
    __syncthreads();
    // row sums of dX * L (over the 32 lanes of a row), plus the column sums above
    {
        const int c = t / CT, i = t % CT;
        float p = sm.dM[c][i] * sm.L[c][i];
#pragma unroll
        for (int m = 16; m >= 1; m >>= 1) p += __shfl_xor(p, m);
        if (i == 0) {
            float s = p;
#pragma unroll
            for (int x = 0; x < NT / 64; ++x) s += red[x * CT + c];
            sm.dbeta[c] = s;
        }
    }

    // ---------------------------- per (row, channel): dq, dk and dG
    // Pairs of rows in different 16-row blocks (i < 16 <= c) factor their
    // decay through row 16, exp(G_c - G_i) = exp(G_c - G_16) exp(G_16 - G_i),
    // both <= 1: plain products on the matrix cores whose 16 x 16 output tile
    // is the wave's own element tile (block 1's waves: the row-side sums over
    // block 0; block 0's waves: the column-side sums over block 1).  Within a
    // block, the lane's rows c0 .. c0 + 3 share the decay products through a
    // reference row: for i <= c0, exp(G_c - G_i) = exp(G_c - G_c0) exp(G_c0 - G_i),
    // and for c2 >= c3 = c0 + 3, exp(G_c2 - G_c) = exp(G_c2 - G_c3) exp(G_c3 - G_c),
    // every factor <= 1; the few pairs between the lane's own rows are direct.
    if (tw) {
        auto gcol = [&](int c) { return sm.gc[c][ekk]; };
        auto kcol = [&](int c) { return sm.k[c][ekk]; };
        auto qcol = [&](int c) { return sm.q[c][ekk]; };
        const int c0 = ert + 4 * lg, c3 = c0 + 3;
        const float g0 = gcol(c0), g3 = gcol(c3);
        float t1[4] = {0.f, 0.f, 0.f, 0.f}, t2[4] = {0.f, 0.f, 0.f, 0.f};
        float t3[4] = {0.f, 0.f, 0.f, 0.f}, t4[4] = {0.f, 0.f, 0.f, 0.f};
        // across the blocks, through row 16 (x0: the tile's first channel)
        const int x0 = ekk - ln;
        const float g16 = gcol(16);
        f4 oa = {0.f, 0.f, 0.f, 0.f}, om = oa;
        if (ert == 16) {
            oa = tile_mm<16>([&](int r, int i) { return sm.dA[16 + r][i]; },
                             [&](int i, int x) { return sm.k[i][x0 + x] * __expf(sm.gc[16][x0 + x] - sm.gc[i][x0 + x]); },
                             ln, lg, oa);
            om = tile_mm<16>([&](int r, int i) { return sm.dM[16 + r][i]; },
                             [&](int i, int x) { return sm.k[i][x0 + x] * __expf(sm.gc[16][x0 + x] - sm.gc[i][x0 + x]); },
                             ln, lg, om);
        } else {
            oa = tile_mm<16>([&](int r, int c2) { return sm.dA[16 + c2][r]; },
                             [&](int c2, int x) {
                                 return sm.q[16 + c2][x0 + x] * __expf(sm.gc[16 + c2][x0 + x] - sm.gc[16][x0 + x]);
                             },
                             ln, lg, oa);
            om = tile_mm<16>([&](int r, int c2) { return sm.dM[16 + c2][r]; },
                             [&](int c2, int x) {
                                 return sm.beta[16 + c2] * sm.k[16 + c2][x0 + x] *
                                        __expf(sm.gc[16 + c2][x0 + x] - sm.gc[16][x0 + x]);
                             },
                             ln, lg, om);
        }
        // row side within the block, ert <= i <= c0 (dA and dM vanish above the diagonal)
        for (int i = ert; i <= c0; ++i) {
            const float kh = kcol(i) * __expf(g0 - gcol(i));
            const float4 a4 = *reinterpret_cast<const float4*>(&dAc[i][c0]);
            const float4 m4 = *reinterpret_cast<const float4*>(&dXc[i][c0]);
            t1[0] += a4.x * kh; t1[1] += a4.y * kh; t1[2] += a4.z * kh; t1[3] += a4.w * kh;
            t3[0] += m4.x * kh; t3[1] += m4.y * kh; t3[2] += m4.z * kh; t3[3] += m4.w * kh;
        }
        // column side within the block, c3 <= c2 < ert + 16
        for (int c2 = c3; c2 < ert + 16; ++c2) {
            const float hh = __expf(gcol(c2) - g3);
            const float qh = qcol(c2) * hh, kh = sm.beta[c2] * kcol(c2) * hh;
            const float4 a4 = *reinterpret_cast<const float4*>(&dAr[c2][c0]);
            const float4 m4 = *reinterpret_cast<const float4*>(&dXr[c2][c0]);
            t2[0] += a4.x * qh; t2[1] += a4.y * qh; t2[2] += a4.z * qh; t2[3] += a4.w * qh;
            t4[0] += m4.x * kh; t4[1] += m4.y * kh; t4[2] += m4.z * kh; t4[3] += m4.w * kh;
        }
        float last = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = c0 + j;
            const float gcc = gcol(c);
            const float f0 = __expf(gcc - g0), f3 = __expf(g3 - gcc);
            float T1 = f0 * t1[j], T3 = f0 * t3[j], T2 = f3 * t2[j], T4 = f3 * t4[j];
            if (ert == 16) {
                const float e = __expf(gcc - g16);
                T1 += e * oa[j];
                T3 += e * om[j];
            } else {
                const float e = __expf(g16 - gcc);
                T2 += e * oa[j];
                T4 += e * om[j];
            }
            // the lane's own rows: c0 < i <= c (row side), c <= c2 < c3 (column side)
#pragma unroll
            for (int x = 1; x < 4; ++x) {
                if (x <= j) {
                    const float d = __expf(gcc - gcol(c0 + x)) * kcol(c0 + x);
                    T1 += sm.dA[c][c0 + x] * d;
                    T3 += sm.dM[c][c0 + x] * d;
                }
                if (x - 1 >= j) {
                    const int c2 = c0 + x - 1;
                    const float d = __expf(gcol(c2) - gcc);
                    T2 += sm.dA[c2][c] * qcol(c2) * d;
                    T4 += sm.beta[c2] * sm.dM[c2][c] * kcol(c2) * d;
                }
            }
            T3 *= sm.beta[c];
            const float E = sm.e[c][ekk];
            const float F = __expf(gcol(CT - 1) - gcc);
            const float dqt = T1 + dqe[j] * E;
            const float dk = T2 + T3 + T4 + dke[j] * E + dkf[j] * F;
            const float qc = qcol(c), kc = kcol(c);
            const float dgv = qc * T1 + kc * (T3 - T2 - T4) + dqe[j] * qc * E + dke[j] * kc * E - dkf[j] * kc * F;
            last += dkf[j] * kc * F;
            sm.e[c][ekk] = dgv;   // exp(G) is no longer read: it holds dG from here on
            const int64_t row = static_cast<int64_t>(n) * CT + c;
            if (row < T) {
                const int64_t o = ((b * T + row) * H + h) * K + ekk;
                Elem<TI>::st(dqp + o, dqt * scale);
                Elem<TI>::st(dkp + o, dk);
            }
        }
        (&sm.Y[0][0])[((w / KTL) * 4 + lg) * K + ekk] = last;
    }
    __syncthreads();

    // ------------------------------- dg (reverse in-chunk cumsum), dbeta
    // thread (rg, kk): suffix sums over its rows, then over the later row groups
    {
        float* gtot = reinterpret_cast<float*>(&sm.st.dS);   // [NT / K][K]; dS is no longer read
        float sfx[RPT];
        float acc = 0.f;
#pragma unroll
        for (int j = RPT - 1; j >= 0; --j) {
            acc += sm.e[RPT * rg + j][kk];
            sfx[j] = acc;
        }
        gtot[rg * K + kk] = acc;
        __syncthreads();
        float post = sm.deps[kk] * sm.eps[kk];
#pragma unroll
        for (int x = 0; x < 8; ++x) post += (&sm.Y[0][0])[x * K + kk];
#pragma unroll
        for (int r = 0; r < NT / K; ++r) post += r > rg ? gtot[r * K + kk] : 0.f;
#pragma unroll
        for (int j = 0; j < RPT; ++j) {
            const int64_t row = static_cast<int64_t>(n) * CT + RPT * rg + j;
            if (row < T) a.dg[((b * T + row) * H + h) * K + kk] = post + sfx[j];
        }
    }
    if (t < CT) {
        const int64_t row = static_cast<int64_t>(n) * CT + t;
        if (row < T) a.dbeta[(b * T + row) * H + h] = sm.dbeta[t];
    }
}

// Workgroups of a persistent kernel: as many as are resident at once on the
// current device.
template <typename Kern>
int persistent_grid(Kern kernel, int threads) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || per <= 0) per = 1;
    return cus * per;
}

template <int K, typename TI>
int launch_bwd(const kda_bwd_args& a, hipStream_t stream) {
    const int64_t BH = a.B * a.H;
    const int64_t nck = (a.T + CT - 1) / CT;
    const BwdWs ws = ws_layout(a.workspace, BH, nck, a.K, a.V);
    if (nck > 0) {
        hipLaunchKernelGGL((bwd_pairs_kernel<K, TI>), dim3(static_cast<unsigned>(std::min<int64_t>(BH * nck, persistent_grid(bwd_pairs_kernel<K, TI>, NP)))),
                           dim3(NP), 0, stream, a, ws, BH * nck);
        if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    }
    if (a.V % 64 == 0)
        hipLaunchKernelGGL((bwd_state_kernel<K, 64, TI>), dim3(static_cast<unsigned>(BH * (a.V / 64))), dim3(NS), 0,
                           stream, a, ws);
    else
        hipLaunchKernelGGL((bwd_state_kernel<K, 32, TI>), dim3(static_cast<unsigned>(BH * (a.V / 32))), dim3(NS), 0,
                           stream, a, ws);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    if (nck > 0) {
        hipLaunchKernelGGL((bwd_chunk_kernel<K, TI>), dim3(static_cast<unsigned>(BH * nck)), dim3(NT), 0, stream,
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
    return B * H * nck * (3 * CT * CT + K * V + 2 * CT * V) * static_cast<int64_t>(sizeof(float));
}

// Static scratch of kda_chunkwise_bwd_noalloc: the workspace of the three
// kernels (A, L, N, dS_end, dP, dR) for shapes that fit.  The array's name is
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
