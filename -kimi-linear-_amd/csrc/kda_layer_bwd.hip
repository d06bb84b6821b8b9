// Gradients of the KDA layer's pre- and post-processing (kda_prep_fwd,
// kda_output_fwd), for gfx950.
//
// Training differentiates the whole layer (the reference by autograd through
// _projections and _output, kimi_linear/kda.py:399-470; it trains the layer in
// scripts/train_musicgpt_fp16.py:519-523).  The core has its own backward
// (kda_chunkwise_bwd); these kernels carry the gradients the rest of the way:
//
//   prep_bwd_kernel, one wave per (batch, 64-token tile, tensor, head), lanes
//     across the head's channels as in the forward.  q, k, v: the forward is
//     re-evaluated from the saved projections (conv, SiLU, L2 norm), then
//       ds = rn dy - s rn^3 <s, dy>      (L2 norm; ds = dy / eps when clamped)
//       du = ds sigmoid(u) (1 + u (1 - sigmoid(u)))          (SiLU)
//       dx[t] = sum_j w[j] du[t + cm - j]                     (causal conv)
//     and the tile's shares of dw[j] = sum_t du[t] x[t - cm + j], db = sum du.
//     An 8-token step needs du for cm rows past itself: those are evaluated
//     again by the next step (short steps keep the wave's registers few).  Gates: dgk = dg (-exp(A_log)) sigmoid(z),
//     dbeta_logit = dbeta beta (1 - beta), and the tile's shares of
//     dA_log = sum dg g and ddt_bias = sum dgk.
//   output_bwd_kernel, one wave per (batch, 32-token tile, head):
//       n = o r w, r = rsqrt(mean o^2 + eps), y = n sigmoid(z)
//       dn = dy sigmoid(z),  dz = dy n sigmoid(z) (1 - sigmoid(z))
//       do = r w dn - o r^3 <o, w dn> / V,  and the tile's share of dw = sum dn o r.
//   colsum_kernel: the parameter gradients as sums of the tiles' shares, in
//     tile order (fp32; identical from run to run).
//
// Both are HBM-streaming: every input element is read once per use (plus the
// conv halo), every gradient written once.
#include "kda_common.h"

namespace kda {

namespace {

constexpr int kMaxConvB = 4;      // largest conv_size (as the forward)
constexpr int kStep = 8;          // tokens per step of a prep unit
constexpr int kPrepTile = 64;     // tokens per prep unit
constexpr int kOutStep = 8;       // tokens per step of an output unit
constexpr int kOutTile = 32;      // tokens per output unit

template <typename XT> __device__ __forceinline__ float to_f(XT x);
template <> __device__ __forceinline__ float to_f<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f<_Float16>(_Float16 x) { return static_cast<float>(x); }
template <> __device__ __forceinline__ float to_f<bf16_t>(bf16_t x) { return bf16_bits_to_f32(x.bits); }

template <typename XT> __device__ __forceinline__ XT from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f<_Float16>(float x) { return static_cast<_Float16>(x); }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float x) { return bf16_t{f32_to_bf16_bits(x)}; }

template <typename XT, int CPL>
struct alignas(sizeof(XT) * CPL) Vec {
    XT e[CPL];
};
template <typename XT, int CPL>
__device__ __forceinline__ void vld(const XT* p, float (&x)[CPL]) {
    const Vec<XT, CPL> v = *reinterpret_cast<const Vec<XT, CPL>*>(p);
#pragma unroll
    for (int c = 0; c < CPL; ++c) x[c] = to_f(v.e[c]);
}
template <typename XT, int CPL>
__device__ __forceinline__ void vst(XT* p, const float (&x)[CPL]) {
    Vec<XT, CPL> v;
#pragma unroll
    for (int c = 0; c < CPL; ++c) v.e[c] = from_f<XT>(x[c]);
    *reinterpret_cast<Vec<XT, CPL>*>(p) = v;
}

// Shares of the parameter gradients, one row per unit tile:
// conv i: [rows][D_i * conv_size] weights and [rows][D_i] biases; gates
// [rows][H K] for A_log and for dt_bias.
struct PrepParts {
    float* dw[3];
    float* db[3];
    float* da;
    float* ddt;
    int64_t rows;
};

int64_t prep_rows(int64_t B, int64_t T) { return B * ((T + kPrepTile - 1) / kPrepTile); }

PrepParts prep_parts(void* ws, int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t cs) {
    PrepParts p;
    p.rows = prep_rows(B, T);
    float* f = static_cast<float*>(ws);
    const int64_t D[3] = {H * K, H * K, H * V};
    for (int i = 0; i < 3; ++i) {
        p.dw[i] = f;
        f += p.rows * D[i] * cs;
        p.db[i] = f;
        f += p.rows * D[i];
    }
    p.da = f;
    f += p.rows * H * K;
    p.ddt = f;
    return p;
}

int64_t prep_ws_floats(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t cs) {
    return prep_rows(B, T) * ((2 * H * K + H * V) * (cs + 1) + 2 * H * K);
}

// ---- q, k or v: one head over a 64-token tile ------------------------------
template <typename XT, int CPL>
__device__ void conv_bwd_unit(const kda_prep_bwd_args& a, const PrepParts& pp, int i, int64_t b, int64_t tile,
                              int64_t h, int lane) {
    constexpr int R = kStep + kMaxConvB - 1;   // du rows of a step: its own and cm more
    constexpr int W = R + kMaxConvB - 1;       // x rows those need
    const int64_t Dh = 64 * CPL;
    const int64_t D = a.H * Dh;
    const int64_t ch0 = h * Dh + lane * CPL;
    const int cs = static_cast<int>(a.conv_size), cm = cs - 1;
    const int64_t T = a.T;
    const XT* x = static_cast<const XT*>(a.x[i]) + b * a.x_stride[i][0] + ch0;
    const XT* dy = static_cast<const XT*>(a.dy[i]) + b * T * D + ch0;
    XT* dx = static_cast<XT*>(a.dx[i]) + b * T * D + ch0;

    RawElem rw[kMaxConvB][CPL], rb[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        rb[c] = load_raw_elem(a.conv_b[i] != nullptr ? a.conv_b[i] : a.conv_w[i],
                              a.conv_b[i] != nullptr ? ch0 + c : 0, a.w_dtype);
#pragma unroll
        for (int j = 0; j < kMaxConvB; ++j)
            rw[j][c] = load_raw_elem(a.conv_w[i], j < cs ? (ch0 + c) * cs + j : 0, a.w_dtype);
    }
    float w[kMaxConvB][CPL], bias[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        bias[c] = a.conv_b[i] != nullptr ? decode_elem(rb[c], a.w_dtype) : 0.f;
#pragma unroll
        for (int j = 0; j < kMaxConvB; ++j) w[j][c] = j < cs ? decode_elem(rw[j][c], a.w_dtype) : 0.f;
    }
    // the taps in reverse, wr[j] = w[cm - j]: dx[t] = sum_j wr[j] du[t + j]
    float wr[kMaxConvB][CPL];
#pragma unroll
    for (int jp = 0; jp < kMaxConvB; ++jp)
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float v = 0.f;
#pragma unroll
            for (int j = 0; j < kMaxConvB; ++j) v = j + jp == cm ? w[j][c] : v;
            wr[jp][c] = v;
        }
    const float inv_eps = 1.f / a.l2_eps;

    float dws[kMaxConvB][CPL], dbs[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        dbs[c] = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxConvB; ++j) dws[j][c] = 0.f;
    }
    const int64_t t0 = tile * kPrepTile;
    for (int step = 0; step < kPrepTile / kStep; ++step) {
        const int64_t s0 = t0 + step * kStep;
        if (s0 >= T) break;
        // x row r is token s0 - cm + r, dy and du row r token s0 + r; rows
        // outside [0, T) read a valid row and count as zero
        float xw[W][CPL], dyr[R][CPL];
#pragma unroll
        for (int r = 0; r < W; ++r) {
            const int64_t tok = s0 - cm + r;
            const bool in = tok >= 0 && tok < T;
            vld<XT, CPL>(x + (in ? tok : 0) * a.x_stride[i][1], xw[r]);
            if (!in) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) xw[r][c] = 0.f;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t tok = s0 + r;
            const bool in = tok < T;
            vld<XT, CPL>(dy + (in ? tok : 0) * D, dyr[r]);
            if (!in) {
#pragma unroll
                for (int c = 0; c < CPL; ++c) dyr[r][c] = 0.f;
            }
        }
        float du[R][CPL];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float u[CPL], sg[CPL], s[CPL];
            float ss = 0.f, sd = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                u[c] = bias[c];
#pragma unroll
                for (int j = 0; j < kMaxConvB; ++j)
                    if (j < cs) u[c] = fmaf(w[j][c], xw[r + j][c], u[c]);
                sg[c] = sigmoid_f(u[c]);
                s[c] = u[c] * sg[c];
                ss = fmaf(s[c], s[c], ss);
                sd = fmaf(s[c], dyr[r][c], sd);
            }
            float ds[CPL];
            if (i < 2) {
                // y = s min(rsqrt(sum s^2), 1/eps): a clamped row is s / eps
                const float tot = wave_sum(ss), dot = wave_sum(sd);
                const float rn = rsqrtf(tot);
                const bool clamped = !(rn < inv_eps);
                const float k3 = rn * rn * rn * dot;
#pragma unroll
                for (int c = 0; c < CPL; ++c) ds[c] = clamped ? dyr[r][c] * inv_eps : fmaf(rn, dyr[r][c], -s[c] * k3);
            } else {
#pragma unroll
                for (int c = 0; c < CPL; ++c) ds[c] = dyr[r][c];
            }
            const bool in = s0 + r < T;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const float d = ds[c] * sg[c] * fmaf(u[c], 1.f - sg[c], 1.f);
                du[r][c] = in ? d : 0.f;
            }
        }
        // the step's tokens: dx, and their shares of dw and db
#pragma unroll
        for (int t = 0; t < kStep; ++t) {
            float g[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < kMaxConvB; ++j) acc = fmaf(wr[j][c], du[t + j][c], acc);
                g[c] = acc;
                dbs[c] += du[t][c];
#pragma unroll
                for (int j = 0; j < kMaxConvB; ++j)
                    if (j < cs) dws[j][c] = fmaf(du[t][c], xw[t + j][c], dws[j][c]);
            }
            if (s0 + t < T) vst<XT, CPL>(dx + (s0 + t) * D, g);
        }
    }
    const int64_t row = b * ((T + kPrepTile - 1) / kPrepTile) + tile;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
#pragma unroll
        for (int j = 0; j < kMaxConvB; ++j)
            if (j < cs) pp.dw[i][(row * D + ch0 + c) * cs + j] = dws[j][c];
        if (a.db[i] != nullptr) pp.db[i][row * D + ch0 + c] = dbs[c];
    }
}

// ---- the gates of one head over a 64-token tile ----------------------------
template <typename XT, int CPL>
__device__ void gate_bwd_unit(const kda_prep_bwd_args& a, const PrepParts& pp, int64_t b, int64_t tile, int64_t h,
                              int lane) {
    const int64_t Dh = 64 * CPL;
    const int64_t D = a.H * Dh;
    const int64_t ch0 = h * Dh + lane * CPL;
    const int64_t T = a.T;
    float neg_a[CPL], dtb[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        neg_a[c] = -__expf(load_elem(a.a_log, ch0 + c, a.p_dtype));
        dtb[c] = load_elem(a.dt_bias, ch0 + c, a.p_dtype);
    }
    const XT* gk = static_cast<const XT*>(a.gk) + b * a.gk_stride[0] + ch0;
    const float* dg = a.dg + b * T * D + ch0;
    XT* dgk = static_cast<XT*>(a.dgk) + b * T * D + ch0;
    float sa[CPL], sd[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) sa[c] = sd[c] = 0.f;
    const int64_t t0 = tile * kPrepTile;
    for (int step = 0; step < kPrepTile / kStep; ++step) {
        const int64_t s0 = t0 + step * kStep;
        if (s0 >= T) break;
        float z[kStep][CPL], d[kStep][CPL];
#pragma unroll
        for (int t = 0; t < kStep; ++t) {
            const int64_t tok = s0 + t < T ? s0 + t : s0;
            vld<XT, CPL>(gk + tok * a.gk_stride[1], z[t]);
            vld<float, CPL>(dg + tok * D, d[t]);
        }
#pragma unroll
        for (int t = 0; t < kStep; ++t) {
            if (s0 + t >= T) break;
            float o[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const float zz = z[t][c] + dtb[c];
                // softplus(z) = z above torch's threshold (20), and its
                // derivative 1 there; sigmoid(z) below
                const float sp = softplus(zz);
                const float sl = zz > 20.f ? 1.f : sigmoid_f(zz);
                o[c] = d[t][c] * neg_a[c] * sl;
                sd[c] += o[c];
                sa[c] = fmaf(d[t][c], neg_a[c] * sp, sa[c]);
            }
            vst<XT, CPL>(dgk + (s0 + t) * D, o);
        }
        // beta: lane t of the step takes token s0 + t
        if (lane < kStep && s0 + lane < T) {
            const int64_t tok = s0 + lane;
            const float x = load_elem(a.beta_logit, b * a.beta_stride[0] + tok * a.beta_stride[1] + h, a.x_dtype);
            const float bt = sigmoid_f(x);
            const float g = a.dbeta[(b * T + tok) * a.H + h] * bt * (1.f - bt);
            store_elem(a.dbeta_logit, (b * T + tok) * a.H + h, a.x_dtype, g);
        }
    }
    const int64_t row = b * ((T + kPrepTile - 1) / kPrepTile) + tile;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        pp.da[row * D + ch0 + c] = sa[c];
        pp.ddt[row * D + ch0 + c] = sd[c];
    }
}

// One wave per (batch, tile, part, head); part 0..2 = q, k, v, 3 = the gates.
template <typename XT, int CPLK, int CPLV>
__global__ __launch_bounds__(256) void prep_bwd_kernel(const kda_prep_bwd_args a, const PrepParts pp,
                                                       uint32_t ntiles, uint32_t units, uint32_t nparts) {
    const int lane = threadIdx.x & 63;
    const uint32_t unit = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (unit >= units) return;
    const uint32_t H = static_cast<uint32_t>(a.H);
    uint32_t u = unit;
    const int64_t h = u % H;
    u /= H;
    const int part = static_cast<int>(u % nparts);
    u /= nparts;
    const int64_t tile = u % ntiles;
    const int64_t b = u / ntiles;
    if (part < 2)
        conv_bwd_unit<XT, CPLK>(a, pp, part, b, tile, h, lane);
    else if (part == 2)
        conv_bwd_unit<XT, CPLV>(a, pp, 2, b, tile, h, lane);
    else
        gate_bwd_unit<XT, CPLK>(a, pp, b, tile, h, lane);
}

// ---- output: one wave per (batch, 32-token tile, head) ---------------------
template <typename XT, int CPL>
__global__ __launch_bounds__(256) void output_bwd_kernel(const kda_output_bwd_args a, float* part, uint32_t ntiles,
                                                         uint32_t units) {
    const int lane = threadIdx.x & 63;
    const uint32_t unit = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (unit >= units) return;
    const uint32_t H = static_cast<uint32_t>(a.H);
    const int64_t h = unit % H;
    const uint32_t bt = unit / H;
    const int64_t tile = bt % ntiles, b = bt / ntiles;
    const int64_t V = 64 * CPL, T = a.T;
    const int64_t c0 = lane * CPL;
    const XT* op = static_cast<const XT*>(a.o) + b * a.o_stride[0] + h * a.o_stride[2] + c0;
    const XT* gp = static_cast<const XT*>(a.gate) + b * a.gate_stride[0] + h * V + c0;
    const XT* dyp = static_cast<const XT*>(a.dy) + b * T * a.H * V + h * V + c0;
    XT* dop = static_cast<XT*>(a.d_o) + b * T * a.H * V + h * V + c0;
    XT* dgp = static_cast<XT*>(a.dgate) + b * T * a.H * V + h * V + c0;
    float w[CPL], dws[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        w[c] = load_elem(a.weight, h * V + c0 + c, a.w_dtype);
        dws[c] = 0.f;
    }
    const float inv_v = 1.f / static_cast<float>(V);
    const int64_t t0 = tile * kOutTile;
    for (int step = 0; step < kOutTile / kOutStep; ++step) {
        const int64_t s0 = t0 + step * kOutStep;
        if (s0 >= T) break;
        float o[kOutStep][CPL], z[kOutStep][CPL], d[kOutStep][CPL];
#pragma unroll
        for (int r = 0; r < kOutStep; ++r) {
            const int64_t t = s0 + r < T ? s0 + r : s0;
            vld<XT, CPL>(op + t * a.o_stride[1], o[r]);
            vld<XT, CPL>(gp + t * a.gate_stride[1], z[r]);
            vld<XT, CPL>(dyp + t * a.H * V, d[r]);
        }
#pragma unroll
        for (int r = 0; r < kOutStep; ++r) {
            if (s0 + r >= T) break;
            float ss = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) ss = fmaf(o[r][c], o[r][c], ss);
            const float rs = rsqrtf(wave_sum(ss) * inv_v + a.eps);
            float dn[CPL], dz[CPL], pr = 0.f;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const float sg = sigmoid_f(z[r][c]);
                const float n = to_f(from_f<XT>((o[r][c] * rs) * w[c]));
                dn[c] = d[r][c] * sg;
                dz[c] = d[r][c] * n * sg * (1.f - sg);
                dws[c] = fmaf(dn[c], o[r][c] * rs, dws[c]);
                pr = fmaf(o[r][c], w[c] * dn[c], pr);
            }
            const float k3 = rs * rs * rs * wave_sum(pr) * inv_v;
            float g[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) g[c] = fmaf(rs * w[c], dn[c], -o[r][c] * k3);
            vst<XT, CPL>(dop + (s0 + r) * a.H * V, g);
            vst<XT, CPL>(dgp + (s0 + r) * a.H * V, dz);
        }
    }
#pragma unroll
    for (int c = 0; c < CPL; ++c) part[(b * ntiles + tile) * a.H * V + h * V + c0 + c] = dws[c];
}

// ---- sums of the tiles' shares ---------------------------------------------
struct ColSum {
    const float* src;              // [rows][n]
    float* dst;                    // [n]
    int64_t n;
};
struct ColSums {
    ColSum s[8];
    int64_t rows;
};

__global__ __launch_bounds__(256) void colsum_kernel(const ColSums c) {
    const ColSum d = c.s[blockIdx.y];
    const int64_t k = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (d.src == nullptr || k >= d.n) return;
    // eight independent partial sums keep eight loads in flight; the order of
    // the additions is fixed
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int64_t r = 0;
    for (; r + 8 <= c.rows; r += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u) acc[u] += d.src[(r + u) * d.n + k];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u)
        if (r + u < c.rows) acc[u] += d.src[(r + u) * d.n + k];
    d.dst[k] = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

int launch_colsum(const ColSums& c, int count, hipStream_t stream) {
    int64_t nmax = 0;
    for (int i = 0; i < count; ++i) nmax = c.s[i].n > nmax ? c.s[i].n : nmax;
    if (nmax == 0 || count == 0) return KDA_OK;
    hipLaunchKernelGGL(colsum_kernel, dim3(static_cast<unsigned>((nmax + 255) / 256), static_cast<unsigned>(count)),
                       dim3(256), 0, stream, c);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

bool dtype_ok(int32_t d) { return d == KDA_DTYPE_F32 || d == KDA_DTYPE_F16 || d == KDA_DTYPE_BF16; }
int64_t esize(int32_t d) { return d == KDA_DTYPE_F32 ? 4 : 2; }
bool head_ok(int64_t d) { return d == 64 || d == 128; }
bool aligned(const void* p, int64_t bytes) { return reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(bytes) == 0; }

int validate_prep_bwd(const kda_prep_bwd_args* a) {
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->K <= 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (a->conv_size < 1 || a->conv_size > kMaxConvB) return KDA_ERR_UNSUPPORTED;
    if (!head_ok(a->K) || !head_ok(a->V)) return KDA_ERR_UNSUPPORTED;
    if (!dtype_ok(a->x_dtype) || !dtype_ok(a->w_dtype) || (a->gk && !dtype_ok(a->p_dtype))) return KDA_ERR_BAD_DTYPE;
    if (!(a->l2_eps > 0.f)) return KDA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->H == 0 || a->T == 0) return KDA_OK;
    for (int i = 0; i < 3; ++i) {
        if (!a->x[i] || !a->conv_w[i] || !a->dy[i] || !a->dx[i] || !a->dw[i]) return KDA_ERR_NULL_POINTER;
        const int64_t cpl = (i == 2 ? a->V : a->K) / 64, vb = cpl * esize(a->x_dtype);
        if (!aligned(a->x[i], vb) || a->x_stride[i][0] % cpl || a->x_stride[i][1] % cpl || !aligned(a->dy[i], vb) ||
            !aligned(a->dx[i], vb))
            return KDA_ERR_BAD_SHAPE;
    }
    if (a->gk) {
        if (!a->a_log || !a->dt_bias || !a->beta_logit || !a->dg || !a->dbeta || !a->dgk || !a->dbeta_logit ||
            !a->da_log || !a->ddt_bias)
            return KDA_ERR_NULL_POINTER;
        const int64_t cpl = a->K / 64, vb = cpl * esize(a->x_dtype);
        if (!aligned(a->gk, vb) || a->gk_stride[0] % cpl || a->gk_stride[1] % cpl || !aligned(a->dgk, vb) ||
            !aligned(a->dg, cpl * 4))
            return KDA_ERR_BAD_SHAPE;
    }
    if (!a->workspace) return KDA_ERR_NULL_POINTER;
    if (!aligned(a->workspace, 16)) return KDA_ERR_BAD_SHAPE;
    if (prep_rows(a->B, a->T) * 4 * a->H > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return KDA_OK;
}

int validate_output_bwd(const kda_output_bwd_args* a) {
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (!head_ok(a->V)) return KDA_ERR_UNSUPPORTED;
    if (!dtype_ok(a->x_dtype) || !dtype_ok(a->w_dtype)) return KDA_ERR_BAD_DTYPE;
    if (!(a->eps >= 0.f)) return KDA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->T == 0 || a->H == 0) return KDA_OK;
    if (!a->o || !a->gate || !a->weight || !a->dy || !a->d_o || !a->dgate || !a->dweight || !a->workspace)
        return KDA_ERR_NULL_POINTER;
    const int64_t cpl = a->V / 64, vb = cpl * esize(a->x_dtype);
    if (!aligned(a->o, vb) || a->o_stride[0] % cpl || a->o_stride[1] % cpl || a->o_stride[2] % cpl ||
        !aligned(a->gate, vb) || a->gate_stride[0] % cpl || a->gate_stride[1] % cpl || !aligned(a->dy, vb) ||
        !aligned(a->d_o, vb) || !aligned(a->dgate, vb) || !aligned(a->workspace, 16))
        return KDA_ERR_BAD_SHAPE;
    if (a->B * ((a->T + kOutTile - 1) / kOutTile) * a->H > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return KDA_OK;
}

template <typename XT, int CPLK, int CPLV>
int launch_prep_bwd(const kda_prep_bwd_args& a, hipStream_t stream) {
    const PrepParts pp = prep_parts(a.workspace, a.B, a.T, a.H, a.K, a.V, a.conv_size);
    const uint32_t nparts = a.gk != nullptr ? 4u : 3u;
    const int64_t ntiles = (a.T + kPrepTile - 1) / kPrepTile;
    const int64_t units = a.B * ntiles * nparts * a.H;
    hipLaunchKernelGGL((prep_bwd_kernel<XT, CPLK, CPLV>), dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256), 0,
                       stream, a, pp, static_cast<uint32_t>(ntiles), static_cast<uint32_t>(units), nparts);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    ColSums c{};
    c.rows = pp.rows;
    int n = 0;
    const int64_t D[3] = {a.H * a.K, a.H * a.K, a.H * a.V};
    for (int i = 0; i < 3; ++i) {
        c.s[n++] = ColSum{pp.dw[i], a.dw[i], D[i] * a.conv_size};
        if (a.db[i] != nullptr) c.s[n++] = ColSum{pp.db[i], a.db[i], D[i]};
    }
    if (a.gk != nullptr) {
        c.s[n++] = ColSum{pp.da, a.da_log, a.H * a.K};
        c.s[n++] = ColSum{pp.ddt, a.ddt_bias, a.H * a.K};
    }
    return launch_colsum(c, n, stream);
}

template <typename XT>
int launch_prep_bwd_dims(const kda_prep_bwd_args& a, hipStream_t stream) {
    switch ((a.K / 64) * 10 + a.V / 64) {
        case 11: return launch_prep_bwd<XT, 1, 1>(a, stream);
        case 12: return launch_prep_bwd<XT, 1, 2>(a, stream);
        case 21: return launch_prep_bwd<XT, 2, 1>(a, stream);
        case 22: return launch_prep_bwd<XT, 2, 2>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

template <typename XT>
int launch_output_bwd(const kda_output_bwd_args& a, hipStream_t stream) {
    const int64_t ntiles = (a.T + kOutTile - 1) / kOutTile;
    const int64_t units = a.B * ntiles * a.H;
    float* part = static_cast<float*>(a.workspace);
    const dim3 grid(static_cast<unsigned>((units + 3) / 4)), block(256);
    const uint32_t nt = static_cast<uint32_t>(ntiles), nu = static_cast<uint32_t>(units);
    if (a.V == 64)
        hipLaunchKernelGGL((output_bwd_kernel<XT, 1>), grid, block, 0, stream, a, part, nt, nu);
    else
        hipLaunchKernelGGL((output_bwd_kernel<XT, 2>), grid, block, 0, stream, a, part, nt, nu);
    if (hipGetLastError() != hipSuccess) return KDA_ERR_LAUNCH;
    ColSums c{};
    c.rows = a.B * ntiles;
    c.s[0] = ColSum{part, a.dweight, a.H * a.V};
    return launch_colsum(c, 1, stream);
}

}  // namespace

}  // namespace kda

extern "C" {

size_t kda_prep_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t conv_size) {
    if (B <= 0 || T <= 0 || H <= 0 || K <= 0 || V <= 0 || conv_size < 1) return 0;
    return static_cast<size_t>(kda::prep_ws_floats(B, T, H, K, V, conv_size)) * sizeof(float);
}

int kda_prep_bwd(const kda_prep_bwd_args* args, void* stream) {
    const int st = kda::validate_prep_bwd(args);
    if (st != KDA_OK || args->B == 0 || args->H == 0 || args->T == 0) return st;
    const auto s = static_cast<hipStream_t>(stream);
    switch (args->x_dtype) {
        case KDA_DTYPE_F16: return kda::launch_prep_bwd_dims<_Float16>(*args, s);
        case KDA_DTYPE_BF16: return kda::launch_prep_bwd_dims<kda::bf16_t>(*args, s);
        default: return kda::launch_prep_bwd_dims<float>(*args, s);
    }
}

size_t kda_output_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t V) {
    if (B <= 0 || T <= 0 || H <= 0 || V <= 0) return 0;
    return static_cast<size_t>(B * ((T + kda::kOutTile - 1) / kda::kOutTile) * H * V) * sizeof(float);
}

int kda_output_bwd(const kda_output_bwd_args* args, void* stream) {
    const int st = kda::validate_output_bwd(args);
    if (st != KDA_OK || args->B == 0 || args->T == 0 || args->H == 0) return st;
    const auto s = static_cast<hipStream_t>(stream);
    switch (args->x_dtype) {
        case KDA_DTYPE_F16: return kda::launch_output_bwd<_Float16>(*args, s);
        case KDA_DTYPE_BF16: return kda::launch_output_bwd<kda::bf16_t>(*args, s);
        default: return kda::launch_output_bwd<float>(*args, s);
    }
}

}  // extern "C"
