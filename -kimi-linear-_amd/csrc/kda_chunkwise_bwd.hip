// Chunkwise KDA backward for gfx950: fp32 throughout.
//
// Gradient of kda_chunkwise (kimi_linear/kda.py:58-185), whose reference is
// differentiated by autograd (training: scripts/train_musicgpt_fp16.py:519-523).
// The forward is re-evaluated chunk by chunk from the state checkpoints that
// kda_chunkwise_fwd_ckpt writes (the state before every CT = 32-token chunk),
// and the chunks are walked in reverse carrying dS, the gradient of the state
// at the current chunk's end.
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
// Work decomposition: one workgroup of 1024 threads (four waves per SIMD, to
// overlap the LDS latency of the loops) per (b, h, VT = 32 state columns);
// the chunk's q, k, G, E, the state tile S, the gradient tile dS and every
// CT x CT matrix live in LDS.  dq, dk, dg and dbeta are sums over the
// state columns, so each workgroup writes its column tile's share to a
// partial buffer (the caller adds the V / VT shares); dv and dS_0 are exact
// per tile.  Rows past T read as zero inputs, which leave the state and
// every gradient of the rows before T unchanged.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int CT = 32;          // tokens per chunk = the forward's checkpoint spacing
constexpr int VT = 32;          // state columns per workgroup
constexpr int NT = 1024;        // threads per workgroup: one per CT x VT and CT x CT entry
static_assert(CT * VT == NT && CT * CT == NT, "one output per thread for the chunk-sized products");

// Rows padded to a multiple of 4 floats plus 4: 16-byte vector reads along a
// row, and consecutive rows 4 banks apart.
template <int K>
struct __align__(16) BwdSmem {
    static constexpr int KP = K + 4, VP = VT + 4;
    float q[CT][KP];            // scale * q
    float k[CT][KP];
    float gc[CT][KP];           // in-chunk cumulative log decay G
    float e[CT][KP];            // exp(G); then, per element, dG
    float S[K][VP];             // state at the chunk start (checkpoint)
    float dS[K][VP];            // gradient of the state at the chunk end, then at its start
    float v[CT][VP];
    float dO[CT][VP];
    float R[CT][VP];
    float P[CT][VP];
    float dP[CT][VP];
    float dR[CT][VP];
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
};
static_assert(CT * (CT + 1) >= NT, "the per-thread shares fit Y");

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

template <int K>
__global__ __launch_bounds__(NT) void chunkwise_bwd_kernel(const kda_bwd_args a) {
    static_assert(NT % K == 0 && (CT * K) % NT == 0, "thread mapping");
    constexpr int EPT = CT * K / NT;        // (row, channel) elements per thread
    constexpr int SPT = K * VT / NT;        // state tile elements per thread
    __shared__ BwdSmem<K> sm;

    const int64_t H = a.H, T = a.T, V = a.V;
    const int nvt = static_cast<int>(V / VT);
    const int vt = blockIdx.x % nvt;
    const int64_t bh = blockIdx.x / nvt;
    const int64_t b = bh / H, h = bh % H;
    const int64_t v0 = static_cast<int64_t>(vt) * VT;
    const int t0 = threadIdx.x;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const float scale = a.scale;

    constexpr int RSTEP = NT / K;
    // state-tile elements of this thread: SPT adjacent columns of one row
    constexpr int TPR = VT / SPT;           // threads per state row

    // dS <- dL/dS_T
    for (int j = 0; j < SPT; ++j) {
        const int r = t0 / TPR, c = SPT * (t0 % TPR) + j;
        sm.dS[r][c] = a.d_state_out ? a.d_state_out[(bh * K + r) * V + v0 + c] : 0.f;
    }

    for (int n = nck - 1; n >= 0; --n) {
        // The thread index, read afresh per chunk: the many lane-derived LDS
        // addresses are recomputed here instead of being held across the loop.
        int t;
        asm volatile("v_mov_b32 %0, %1" : "=v"(t) : "v"(t0));
        const int w = t >> 6, lane = t & 63, ln = lane & 15, lg = lane >> 4;   // wave, MFMA lane
        // (row, channel) element j of this thread: row t / K + j * (NT / K), channel t % K
        const int kk = t % K;
        const int r0 = t / K;
        auto st_row = [&](int j) { return t / TPR + 0 * j; };
        auto st_col = [&](int j) { return SPT * (t % TPR) + j; };
        // ---------------------------------------------------------------- loads
        for (int j = 0; j < EPT; ++j) {
            const int c = r0 + RSTEP * j;
            const int64_t row = static_cast<int64_t>(n) * CT + c;
            float qv = 0.f, kv = 0.f, gv = 0.f;
            if (row < T) {
                const int64_t o = ((b * T + row) * H + h) * K + kk;
                qv = a.q[o] * scale;
                kv = a.k[o];
                gv = a.g[o];
            }
            sm.q[c][kk] = qv;
            sm.k[c][kk] = kv;
            sm.gc[c][kk] = gv;
        }
        for (int j = 0; j < CT * VT / NT; ++j) {
            const int e = t + NT * j, c = e / VT, vv = e % VT;
            const int64_t row = static_cast<int64_t>(n) * CT + c;
            float x = 0.f, d = 0.f;
            if (row < T) {
                const int64_t o = ((b * T + row) * H + h) * V + v0 + vv;
                x = a.v[o];
                d = a.d_o[o];
            }
            sm.v[c][vv] = x;
            sm.dO[c][vv] = d;
        }
        if (t < CT) {
            const int64_t row = static_cast<int64_t>(n) * CT + t;
            sm.beta[t] = row < T ? a.beta[(b * T + row) * H + h] : 0.f;
            sm.dbeta[t] = 0.f;
        }
        {
            const float* ck = a.ckpt + ((bh * nck + n) * K) * V + v0;
            for (int j = 0; j < SPT; ++j) sm.S[st_row(j)][st_col(j)] = ck[st_row(j) * V + st_col(j)];
        }
        __syncthreads();

        // ------------------------------------------- cumulative decays, eps
        if (t < K) {
            float run = 0.f;
            for (int c = 0; c < CT; ++c) {
                run += sm.gc[c][t];
                sm.gc[c][t] = run;
                sm.e[c][t] = __expf(run);
            }
            sm.eps[t] = __expf(run);
        }
        __syncthreads();

        // Entry (pc, pv) of the CT x VT products and (pc, pv) = (c, i) of the
        // CT x CT ones: thread t.
        const int pc = t / VT, pv = t % VT;

        // ----------------------------------------------------------- A and L
        {
            const int c = pc, i = pv;
            float av = 0.f, lv = 0.f;
            if (i <= c) {
#pragma unroll 2
                for (int x = 0; x < K; x += 4) {
                    const float4 gcv = *reinterpret_cast<const float4*>(&sm.gc[c][x]);
                    const float4 giv = *reinterpret_cast<const float4*>(&sm.gc[i][x]);
                    const float4 kiv = *reinterpret_cast<const float4*>(&sm.k[i][x]);
                    const float4 qcv = *reinterpret_cast<const float4*>(&sm.q[c][x]);
                    const float4 kcv = *reinterpret_cast<const float4*>(&sm.k[c][x]);
                    const float d0 = __expf(gcv.x - giv.x) * kiv.x, d1 = __expf(gcv.y - giv.y) * kiv.y;
                    const float d2 = __expf(gcv.z - giv.z) * kiv.z, d3 = __expf(gcv.w - giv.w) * kiv.w;
                    av += qcv.x * d0 + qcv.y * d1 + qcv.z * d2 + qcv.w * d3;
                    lv += kcv.x * d0 + kcv.y * d1 + kcv.z * d2 + kcv.w * d3;
                }
                if (i == c) lv = 0.f;
            }
            sm.A[c][i] = av;
            sm.L[c][i] = lv;
        }
        __syncthreads();

        // ------------------------------- N = (I + Diag(beta) L)^-1, by columns
        // Blocked: the two 16 x 16 diagonal blocks by forward substitution
        // (lane t of wave 0: column t % 16 of block t / 16, in registers),
        // then N10 = -N11 X10 N00 on the matrix cores, all in wave 0.
        if (t < CT) {
            const int bo = 16 * (t >> 4), jc = t & 15;
            float col[16];
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                float s = 0.f;
#pragma unroll
                for (int m = 0; m < c; ++m) s += sm.L[bo + c][bo + m] * col[m];
                col[c] = c < jc ? 0.f : (c == jc ? 1.f : -sm.beta[bo + c] * s);
            }
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                sm.N[bo + c][bo + jc] = col[c];
                if (bo == 0) sm.N[c][16 + jc] = 0.f;
            }
        }
        if (t < 64) {
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
            __builtin_amdgcn_wave_barrier();
            // Y (free here) <- X10 N00, X10 = Diag(beta_1) L10
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mm<16>([&](int r, int m) { return sm.beta[16 + r] * sm.L[16 + r][m]; },
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
        }
        __syncthreads();

        // The products below run on the fp32 matrix cores, one 16 x 16 output
        // tile per wave: lane (ln, lg) receives rows 4 lg + j, column ln.

        // --------------------------------------- R = V - (k*E) S, dP = (k*F) dS + A^T dO
        if (w < 8) {
            const int rt = (w >> 1) & 1, ct = w & 1, r0t = 16 * rt, c0t = 16 * ct;
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            if (w < 4) {
                acc = tile_mm<K>([&](int r, int x) { return sm.k[r0t + r][x] * sm.e[r0t + r][x]; },
                                 [&](int x, int v) { return sm.S[x][c0t + v]; }, ln, lg, acc);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c = r0t + 4 * lg + j;
                    sm.R[c][c0t + ln] = sm.v[c][c0t + ln] - acc[j];
                }
            } else {
                acc = tile_mm<K>([&](int r, int x) {
                                     return sm.k[r0t + r][x] * __expf(sm.gc[CT - 1][x] - sm.gc[r0t + r][x]);
                                 },
                                 [&](int x, int v) { return sm.dS[x][c0t + v]; }, ln, lg, acc);
                acc = tile_mm<CT>([&](int r, int c2) { return sm.A[c2][r0t + r]; },
                                  [&](int c2, int v) { return sm.dO[c2][c0t + v]; }, ln, lg, acc);
#pragma unroll
                for (int j = 0; j < 4; ++j) sm.dP[r0t + 4 * lg + j][c0t + ln] = acc[j];
            }
        }
        __syncthreads();

        // ------------------------------------------ P = M R, dR = M^T dP = dV
        if (w < 8) {
            const int rt = (w >> 1) & 1, ct = w & 1, r0t = 16 * rt, c0t = 16 * ct;
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            if (w < 4) {
                acc = tile_mm<CT>([&](int r, int i) { return sm.N[r0t + r][i] * sm.beta[i]; },
                                  [&](int i, int v) { return sm.R[i][c0t + v]; }, ln, lg, acc);
#pragma unroll
                for (int j = 0; j < 4; ++j) sm.P[r0t + 4 * lg + j][c0t + ln] = acc[j];
            } else {
                acc = tile_mm<CT>([&](int r, int c2) { return sm.N[c2][r0t + r]; },
                                  [&](int c2, int v) { return sm.dP[c2][c0t + v]; }, ln, lg, acc);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int c = r0t + 4 * lg + j;
                    const float dr = acc[j] * sm.beta[c];
                    sm.dR[c][c0t + ln] = dr;
                    const int64_t row = static_cast<int64_t>(n) * CT + c;
                    if (row < T) a.dv[((b * T + row) * H + h) * V + v0 + c0t + ln] = dr;
                }
            }
        }
        __syncthreads();

        // ------------------------------------------ dA = dO P^T, dM = dP R^T (i <= c)
        if (w < 8) {
            const int rt = (w >> 1) & 1, ct = w & 1, r0t = 16 * rt, c0t = 16 * ct;
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            if (w < 4)
                acc = tile_mm<VT>([&](int r, int v) { return sm.dO[r0t + r][v]; },
                                  [&](int v, int i) { return sm.P[c0t + i][v]; }, ln, lg, acc);
            else
                acc = tile_mm<VT>([&](int r, int v) { return sm.dP[r0t + r][v]; },
                                  [&](int v, int i) { return sm.R[c0t + i][v]; }, ln, lg, acc);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = r0t + 4 * lg + j, i = c0t + ln;
                const float x = i <= c ? acc[j] : 0.f;
                if (w < 4) sm.dA[c][i] = x;
                else sm.dM[c][i] = x;
            }
        }
        __syncthreads();

        // ------------------------------- dbeta (M = N Diag(beta)), dN in place
        if (t < CT) {
            float s = 0.f;
            for (int c = t; c < CT; ++c) s += sm.dM[c][t] * sm.N[c][t];
            sm.dbeta[t] = s;
        }
        __syncthreads();
        sm.dM[t / CT][t % CT] *= sm.beta[t % CT];
        __syncthreads();
        // Y = dN N^T
        if (w < 4) {
            const int r0t = 16 * (w >> 1), c0t = 16 * (w & 1);
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mm<CT>([&](int r, int m) { return sm.dM[r0t + r][m]; },
                              [&](int m, int i) { return sm.N[c0t + i][m]; }, ln, lg, acc);
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.Y[r0t + 4 * lg + j][c0t + ln] = acc[j];
        }
        __syncthreads();
        // dX = -N^T Y, strictly lower (kept in dM)
        if (w < 4) {
            const int r0t = 16 * (w >> 1), c0t = 16 * (w & 1);
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = tile_mm<CT>([&](int r, int m) { return sm.N[m][r0t + r]; },
                              [&](int m, int i) { return sm.Y[m][c0t + i]; }, ln, lg, acc);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = r0t + 4 * lg + j, i = c0t + ln;
                sm.dM[c][i] = i < c ? -acc[j] : 0.f;
            }
        }
        __syncthreads();
        if (t < CT) {
            float s = 0.f;
            for (int i = 0; i < t; ++i) s += sm.dM[t][i] * sm.L[t][i];
            sm.dbeta[t] += s;
        }
        if (t < K) {
            float s = 0.f;
            for (int vv = 0; vv < VT; ++vv) s += sm.dS[t][vv] * sm.S[t][vv];
            sm.deps[t] = s;
        }

        // Per wave, one 16 x 16 tile of the K x VT state gradient and one of
        // the CT x K (row, channel) elements.
        constexpr int KTL = K / 16;
        const bool tw = w < 2 * KTL;
        // ------------------- dS_start = Diag(eps) dS + (q~*E)^T dO - (k*E)^T dR
        f4 dsn = {0.f, 0.f, 0.f, 0.f};
        const int srt = 16 * (w >> 1), sct = 16 * (w & 1);
        // element tile: rows 16 (w / KTL) + 4 lg + j, channel 16 (w % KTL) + ln
        const int ert = 16 * (w / KTL), ekk = 16 * (w % KTL) + ln;
        f4 dqe = {0.f, 0.f, 0.f, 0.f}, dke = dqe, dkf = dqe;
        if (tw) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int x = srt + 4 * lg + j;
                dsn[j] = sm.eps[x] * sm.dS[x][sct + ln];
            }
            dsn = tile_mm<CT>([&](int r, int c) { return sm.q[c][srt + r] * sm.e[c][srt + r]; },
                              [&](int c, int v) { return sm.dO[c][sct + v]; }, ln, lg, dsn);
            dsn = tile_mm<CT>([&](int r, int c) { return -sm.k[c][srt + r] * sm.e[c][srt + r]; },
                              [&](int c, int v) { return sm.dR[c][sct + v]; }, ln, lg, dsn);
            // d(q~*E) = dO S^T, d(k*E) = -dR S^T, d(k*F) = P dS^T
            dqe = tile_mm<VT>([&](int r, int v) { return sm.dO[ert + r][v]; },
                              [&](int v, int kc) { return sm.S[ekk - ln + kc][v]; }, ln, lg, dqe);
            dke = tile_mm<VT>([&](int r, int v) { return -sm.dR[ert + r][v]; },
                              [&](int v, int kc) { return sm.S[ekk - ln + kc][v]; }, ln, lg, dke);
            dkf = tile_mm<VT>([&](int r, int v) { return sm.P[ert + r][v]; },
                              [&](int v, int kc) { return sm.dS[ekk - ln + kc][v]; }, ln, lg, dkf);
        }
        // every read of exp(G) and of the end-of-chunk dS is done: dS takes
        // its new value, and each (row, channel) element's exp(G) becomes dG
        __syncthreads();
        if (tw) {
#pragma unroll
            for (int j = 0; j < 4; ++j) sm.dS[srt + 4 * lg + j][sct + ln] = dsn[j];
        }

        // ---------------------------- per (row, channel): dq, dk and dG
        // The lane's rows c0 .. c0 + 3 share the decay products through a
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
            // row side, i <= c0 (dA and dM vanish above the diagonal)
            for (int i = 0; i <= c0; ++i) {
                const float kh = kcol(i) * __expf(g0 - gcol(i));
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    t1[j] += sm.dA[c0 + j][i] * kh;
                    t3[j] += sm.dM[c0 + j][i] * kh;
                }
            }
            // column side, c2 >= c3
            for (int c2 = c3; c2 < CT; ++c2) {
                const float h = __expf(gcol(c2) - g3);
                const float qh = qcol(c2) * h, kh = sm.beta[c2] * kcol(c2) * h;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    t2[j] += sm.dA[c2][c0 + j] * qh;
                    t4[j] += sm.dM[c2][c0 + j] * kh;
                }
            }
            float last = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = c0 + j;
                const float gcc = gcol(c);
                const float f0 = __expf(gcc - g0), f3 = __expf(g3 - gcc);
                float T1 = f0 * t1[j], T3 = f0 * t3[j], T2 = f3 * t2[j], T4 = f3 * t4[j];
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
                    const int64_t o = ((static_cast<int64_t>(vt) * a.B + b) * T + row) * H * K + h * K + ekk;
                    a.dq_part[o] = dqt * scale;
                    a.dk_part[o] = dk;
                }
            }
            (&sm.Y[0][0])[((w / KTL) * 4 + lg) * K + ekk] = last;
        }
        __syncthreads();

        // ------------------------------- dg (reverse in-chunk cumsum), dbeta
        if (t < K) {
            float run = sm.deps[t] * sm.eps[t];
            for (int x = 0; x < 8; ++x) run += (&sm.Y[0][0])[x * K + t];
            for (int c = CT - 1; c >= 0; --c) {
                run += sm.e[c][t];
                const int64_t row = static_cast<int64_t>(n) * CT + c;
                if (row < T)
                    a.dg_part[((static_cast<int64_t>(vt) * a.B + b) * T + row) * H * K + h * K + t] = run;
            }
        }
        if (t < CT) {
            const int64_t row = static_cast<int64_t>(n) * CT + t;
            if (row < T) a.dbeta_part[((static_cast<int64_t>(vt) * a.B + b) * T + row) * H + h] = sm.dbeta[t];
        }
        __syncthreads();
    }

    if (a.d_state_in) {
        for (int j = 0; j < SPT; ++j) {
            const int r = t0 / TPR, c = SPT * (t0 % TPR) + j;
            a.d_state_in[(bh * K + r) * V + v0 + c] = sm.dS[r][c];
        }
    }
}

template <int K>
int launch_bwd(const kda_bwd_args& a, hipStream_t stream) {
    const int64_t blocks = a.B * a.H * (a.V / VT);
    hipLaunchKernelGGL((chunkwise_bwd_kernel<K>), dim3(static_cast<unsigned>(blocks)), dim3(NT), 0, stream, a);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

}  // namespace

bool chunkwise_bwd_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % VT == 0;
}

int chunkwise_bwd_launch(const kda_bwd_args& a, hipStream_t stream) {
    switch (a.K) {
        case 32: return launch_bwd<32>(a, stream);
        case 64: return launch_bwd<64>(a, stream);
        case 128: return launch_bwd<128>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
