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
// Work decomposition: one workgroup of 256 threads per (b, h, VT = 32 state
// columns); the chunk's q, k, G, E, the state tile S, the gradient tile dS and
// every CT x CT matrix live in LDS.  dq, dk, dg and dbeta are sums over the
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
constexpr int NT = 256;         // threads per workgroup

template <int K>
struct BwdSmem {
    float q[CT][K + 1];         // scale * q
    float k[CT][K + 1];
    float gc[CT][K + 1];        // in-chunk cumulative log decay G
    float e[CT][K + 1];         // exp(G); then, per element, dG
    float S[K][VT + 1];         // state at the chunk start (checkpoint)
    float dS[K][VT + 1];        // gradient of the state at the chunk end, then at its start
    float v[CT][VT + 1];
    float dO[CT][VT + 1];
    float R[CT][VT + 1];
    float P[CT][VT + 1];
    float dP[CT][VT + 1];
    float dR[CT][VT + 1];
    float A[CT][CT + 1];        // A (i <= c)
    float L[CT][CT + 1];        // L (i < c)
    float N[CT][CT + 1];        // (I + Diag(beta) L)^-1
    float dA[CT][CT + 1];       // dA (i <= c)
    float dM[CT][CT + 1];       // dM, then dN
    float Y[CT][CT + 1];        // dN N^T, then dX
    float beta[CT];
    float dbeta[CT];
    float eps[K];               // exp(G_last)
    float deps[K];              // rowsum(dS * S)
    float last[NT / K][K];      // per thread: its rows' share of sum_c d(k*F)[c] k[c] F[c]
};

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
    const int t = threadIdx.x;
    const int nck = static_cast<int>((T + CT - 1) / CT);
    const float scale = a.scale;

    // (row, channel) element j of this thread: row t / K + j * (NT / K), channel t % K
    const int kk = t % K;
    const int r0 = t / K;
    constexpr int RSTEP = NT / K;
    // state-tile element j: row t / (VT / SPT) ... as (k row, v column)
    auto st_row = [&](int j) { return (t + NT * j) / VT; };
    auto st_col = [&](int j) { return (t + NT * j) % VT; };

    // dS <- dL/dS_T
    for (int j = 0; j < SPT; ++j) {
        const int r = st_row(j), c = st_col(j);
        sm.dS[r][c] = a.d_state_out ? a.d_state_out[(bh * K + r) * V + v0 + c] : 0.f;
    }

    for (int n = nck - 1; n >= 0; --n) {
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

        // ----------------------------------------------------------- A and L
        for (int j = 0; j < CT * CT / NT; ++j) {
            const int e = t + NT * j, c = e / CT, i = e % CT;
            float av = 0.f, lv = 0.f;
            if (i <= c) {
                for (int x = 0; x < K; ++x) {
                    const float d = __expf(sm.gc[c][x] - sm.gc[i][x]) * sm.k[i][x];
                    av += sm.q[c][x] * d;
                    lv += sm.k[c][x] * d;
                }
                if (i == c) lv = 0.f;
            }
            sm.A[c][i] = av;
            sm.L[c][i] = lv;
        }
        __syncthreads();

        // ------------------------------- N = (I + Diag(beta) L)^-1, by columns
        if (t < CT) {
            const int jc = t;
            for (int c = 0; c < jc; ++c) sm.N[c][jc] = 0.f;
            sm.N[jc][jc] = 1.f;
            for (int c = jc + 1; c < CT; ++c) {
                float s = 0.f;
                for (int m = jc; m < c; ++m) s += sm.L[c][m] * sm.N[m][jc];
                sm.N[c][jc] = -sm.beta[c] * s;
            }
        }
        __syncthreads();

        // Outputs (c, 4 columns) of the CT x VT products: thread t -> row t / 8.
        const int pc = t / (VT / 4), pv = 4 * (t % (VT / 4));

        // --------------------------------------- R = V - (k*E) S, dP = (k*F) dS + A^T dO
        {
            float rr[4], dp[4];
            for (int u = 0; u < 4; ++u) {
                rr[u] = sm.v[pc][pv + u];
                dp[u] = 0.f;
            }
            for (int x = 0; x < K; ++x) {
                const float ke = sm.k[pc][x] * sm.e[pc][x];
                const float kf = sm.k[pc][x] * __expf(sm.gc[CT - 1][x] - sm.gc[pc][x]);
                for (int u = 0; u < 4; ++u) {
                    rr[u] -= ke * sm.S[x][pv + u];
                    dp[u] += kf * sm.dS[x][pv + u];
                }
            }
            for (int c2 = pc; c2 < CT; ++c2) {
                const float w = sm.A[c2][pc];
                for (int u = 0; u < 4; ++u) dp[u] += w * sm.dO[c2][pv + u];
            }
            for (int u = 0; u < 4; ++u) {
                sm.R[pc][pv + u] = rr[u];
                sm.dP[pc][pv + u] = dp[u];
            }
        }
        __syncthreads();

        // ------------------------------------------ P = M R, dR = M^T dP = dV
        {
            float pp[4] = {0.f, 0.f, 0.f, 0.f}, dr[4] = {0.f, 0.f, 0.f, 0.f};
            for (int i = 0; i <= pc; ++i) {
                const float w = sm.N[pc][i] * sm.beta[i];
                for (int u = 0; u < 4; ++u) pp[u] += w * sm.R[i][pv + u];
            }
            for (int c2 = pc; c2 < CT; ++c2) {
                const float w = sm.N[c2][pc];
                for (int u = 0; u < 4; ++u) dr[u] += w * sm.dP[c2][pv + u];
            }
            const int64_t row = static_cast<int64_t>(n) * CT + pc;
            for (int u = 0; u < 4; ++u) {
                dr[u] *= sm.beta[pc];
                sm.P[pc][pv + u] = pp[u];
                sm.dR[pc][pv + u] = dr[u];
            }
            if (row < T) {
                float* dv = a.dv + ((b * T + row) * H + h) * V + v0 + pv;
                for (int u = 0; u < 4; ++u) dv[u] = dr[u];
            }
        }
        __syncthreads();

        // ------------------------------------------ dA = dO P^T, dM = dP R^T
        for (int j = 0; j < CT * CT / NT; ++j) {
            const int e = t + NT * j, c = e / CT, i = e % CT;
            float da = 0.f, dm = 0.f;
            if (i <= c) {
                for (int vv = 0; vv < VT; ++vv) {
                    da += sm.dO[c][vv] * sm.P[i][vv];
                    dm += sm.dP[c][vv] * sm.R[i][vv];
                }
            }
            sm.dA[c][i] = da;
            sm.dM[c][i] = dm;
        }
        __syncthreads();

        // ------------------------------- dbeta (M = N Diag(beta)), dN in place
        if (t < CT) {
            float s = 0.f;
            for (int c = t; c < CT; ++c) s += sm.dM[c][t] * sm.N[c][t];
            sm.dbeta[t] = s;
        }
        __syncthreads();
        for (int j = 0; j < CT * CT / NT; ++j) {
            const int e = t + NT * j, c = e / CT, i = e % CT;
            sm.dM[c][i] *= sm.beta[i];
        }
        __syncthreads();
        // Y = dN N^T (lower: Y[c,i] = sum_{m <= min(c,i)} dN[c,m] N[i,m])
        for (int j = 0; j < CT * CT / NT; ++j) {
            const int e = t + NT * j, c = e / CT, i = e % CT;
            const int mmax = c < i ? c : i;
            float s = 0.f;
            for (int m = 0; m <= mmax; ++m) s += sm.dM[c][m] * sm.N[i][m];
            sm.Y[c][i] = s;
        }
        __syncthreads();
        // dX[c,i] = -sum_{m >= c} N[m,c] Y[m,i] for i < c (kept in dM)
        for (int j = 0; j < CT * CT / NT; ++j) {
            const int e = t + NT * j, c = e / CT, i = e % CT;
            float s = 0.f;
            if (i < c)
                for (int m = c; m < CT; ++m) s += sm.N[m][c] * sm.Y[m][i];
            sm.dM[c][i] = -s;
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

        // ------------------- dS_start = Diag(eps) dS + (q~*E)^T dO - (k*E)^T dR
        float dsn[SPT];
        for (int j = 0; j < SPT; ++j) {
            const int r = st_row(j), c = st_col(j);
            float s = sm.eps[r] * sm.dS[r][c];
            for (int c2 = 0; c2 < CT; ++c2)
                s += sm.e[c2][r] * (sm.q[c2][r] * sm.dO[c2][c] - sm.k[c2][r] * sm.dR[c2][c]);
            dsn[j] = s;
        }
        __syncthreads();

        // ---------------------------- per (row, channel): dq, dk and dG
        {
            float gcol[CT], kcol[CT], qcol[CT];
            for (int c = 0; c < CT; ++c) {
                gcol[c] = sm.gc[c][kk];
                kcol[c] = sm.k[c][kk];
                qcol[c] = sm.q[c][kk];
            }
            float last = 0.f;
            for (int j = 0; j < EPT; ++j) {
                const int c = r0 + RSTEP * j;
                float dqe = 0.f, dke = 0.f, dkf = 0.f;
                for (int vv = 0; vv < VT; ++vv) {
                    const float s = sm.S[kk][vv];
                    dqe += sm.dO[c][vv] * s;
                    dke -= sm.dR[c][vv] * s;
                    dkf += sm.P[c][vv] * sm.dS[kk][vv];
                }
                float t1 = 0.f, t2 = 0.f, t3 = 0.f, t4 = 0.f;
                const float bc = sm.beta[c];
                for (int i = 0; i <= c; ++i) {
                    const float d = __expf(gcol[c] - gcol[i]) * kcol[i];
                    t1 += sm.dA[c][i] * d;
                    if (i < c) t3 += bc * sm.dM[c][i] * d;
                }
                for (int c2 = c; c2 < CT; ++c2) {
                    const float d = __expf(gcol[c2] - gcol[c]);
                    t2 += sm.dA[c2][c] * qcol[c2] * d;
                    if (c2 > c) t4 += sm.beta[c2] * sm.dM[c2][c] * kcol[c2] * d;
                }
                const float E = sm.e[c][kk];
                const float F = __expf(gcol[CT - 1] - gcol[c]);
                const float dqt = t1 + dqe * E;
                const float dk = t2 + t3 + t4 + dke * E + dkf * F;
                const float dgv = qcol[c] * t1 + kcol[c] * (t3 - t2 - t4) + dqe * qcol[c] * E +
                                  dke * kcol[c] * E - dkf * kcol[c] * F;
                last += dkf * kcol[c] * F;
                sm.e[c][kk] = dgv;   // only this thread reads e[c][kk] from here on
                const int64_t row = static_cast<int64_t>(n) * CT + c;
                if (row < T) {
                    const int64_t o = ((static_cast<int64_t>(vt) * a.B + b) * T + row) * H * K + h * K + kk;
                    a.dq_part[o] = dqt * scale;
                    a.dk_part[o] = dk;
                }
            }
            sm.last[r0][kk] = last;
        }
        __syncthreads();

        // ------------------------- carry, dg (reverse in-chunk cumsum), dbeta
        for (int j = 0; j < SPT; ++j) sm.dS[st_row(j)][st_col(j)] = dsn[j];
        if (t < K) {
            float run = sm.deps[t] * sm.eps[t];
            for (int x = 0; x < NT / K; ++x) run += sm.last[x][t];
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
            const int r = st_row(j), c = st_col(j);
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
