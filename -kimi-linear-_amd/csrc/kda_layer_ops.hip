// Pre- and post-processing of the KDA layer around the core, for gfx950.
//
// kda_prep_fwd replaces the elementwise part of _projections
// (kimi_linear/kda.py:399-461): per q/k/v channel the causal short
// convolution (kda.py:282-310), SiLU, and for q and k the per-head L2
// normalisation (kda.py:313-325); the forget gate g = -exp(A_log) *
// softplus(gk + dt_bias) and beta = sigmoid(.) (kda.py:452-460).  The
// reference runs these as ~20 separate elementwise kernels with fp16
// round trips between them; here every projection element is read once (plus
// the conv_size - 1 rows of context a token tile needs) and every core input
// is written once, all arithmetic in fp32 and each output rounded once.  A
// call without g and beta outputs skips the gates: the layer hands gk and the
// beta logits to the gated core entry points, whose loaders form them.
//
// kda_output_fwd replaces HeadwiseRMSNorm and the sigmoid output gate of
// _output (kda.py:258-279, 464-470): one read of the core output and of the
// gate projection, one write of the o_proj input.
//
// Both are HBM-streaming kernels: one wave per unit of work (a 16-token tile
// of one head of one tensor, or an 8-token tile of one output head), lanes
// across the head's channels (K / 64 consecutive channels per lane, one
// vector access per row), cross-lane sums on DPP and permlane swaps.  Every
// load of a unit is issued unconditionally before its first use (rows past
// the data re-read a valid row and are masked), so a wave keeps all of its
// rows in flight at once instead of waiting on each.
#include "kda_common.h"

namespace kda {

namespace {

constexpr int kTile = 16;      // tokens per prep unit (a single-token call uses units of one token)
constexpr int kMaxConv = 4;    // largest conv_size

template <typename XT> __device__ __forceinline__ float to_f(XT x);
template <> __device__ __forceinline__ float to_f<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_f<_Float16>(_Float16 x) { return static_cast<float>(x); }
template <> __device__ __forceinline__ float to_f<bf16_t>(bf16_t x) { return bf16_bits_to_f32(x.bits); }

template <typename XT> __device__ __forceinline__ XT from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ _Float16 from_f<_Float16>(float x) { return static_cast<_Float16>(x); }
template <> __device__ __forceinline__ bf16_t from_f<bf16_t>(float x) { return bf16_t{f32_to_bf16_bits(x)}; }

// CPL consecutive elements, accessed as one aligned vector.
template <typename XT, int CPL>
struct alignas(sizeof(XT) * CPL) Pack {
    XT e[CPL];
};

template <typename XT, int CPL>
__device__ __forceinline__ void ld(const XT* p, float (&x)[CPL]) {
    const Pack<XT, CPL> v = *reinterpret_cast<const Pack<XT, CPL>*>(p);
#pragma unroll
    for (int c = 0; c < CPL; ++c) x[c] = to_f(v.e[c]);
}

template <typename XT, int CPL>
__device__ __forceinline__ void st(XT* p, const float (&x)[CPL]) {
    Pack<XT, CPL> v;
#pragma unroll
    for (int c = 0; c < CPL; ++c) v.e[c] = from_f<XT>(x[c]);
    *reinterpret_cast<Pack<XT, CPL>*>(p) = v;
}

// Round to XT and back: the value an XT tensor would hold.
template <typename XT>
__device__ __forceinline__ float round_to(float x) {
    return to_f(from_f<XT>(x));
}



// A small parameter element of a runtime dtype: the load is unconditional
// (a NULL or out-of-range element reads `fallback`'s first word instead and is
// masked), so that every load of a unit is issued before any result is used.
__device__ __forceinline__ RawElem param_load(const void* p, int64_t i, bool valid, const void* fallback,
                                              int dtype) {
    return valid ? load_raw_elem(p, i, dtype) : load_raw_elem(fallback, 0, dtype);
}

// ---- prep: one q, k or v head over a token tile ---------------------------
template <typename XT, int CPL, int TILE>
__device__ __forceinline__ void conv_unit(const kda_prep_args& a, int i, int64_t b, int64_t t0, int64_t h, int lane) {
    constexpr int kRows = TILE + kMaxConv - 1;
    const int64_t Dh = 64 * CPL;
    const int64_t D = a.H * Dh;
    const int64_t ch0 = h * Dh + lane * CPL;
    const int cs = static_cast<int>(a.conv_size), cm = cs - 1;
    const int64_t T = a.T;
    const int n = static_cast<int>((T - t0) < TILE ? (T - t0) : TILE);
    const XT* x = static_cast<const XT*>(a.x[i]) + b * a.x_stride[i][0] + ch0;
    const XT* hist = static_cast<const XT*>(a.hist_in[i]);
    const XT* hrow = hist != nullptr ? hist + b * cm * D + ch0 : x;

    // window row r holds token t0 - cm + r: a token of this call, a cached
    // input (t < 0) or zero.  Every row is loaded unconditionally (rows with
    // no data read token 0 and are masked) so that all loads are in flight
    // together.
    float win[kRows][CPL];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        const int64_t tok = t0 - cm + r;
        const bool in_x = tok >= 0 && tok < T;
        const bool in_h = tok < 0 && hist != nullptr;
        const XT* src = in_x ? x + tok * a.x_stride[i][1] : (in_h ? hrow + (cm + tok) * D : x);
        ld<XT, CPL>(src, win[r]);
        if (!(in_x || in_h)) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) win[r][c] = 0.f;
        }
    }
    RawElem rw[kMaxConv][CPL], rb[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        rb[c] = param_load(a.conv_b[i], ch0 + c, a.conv_b[i] != nullptr, a.conv_w[i], a.w_dtype);
#pragma unroll
        for (int j = 0; j < kMaxConv; ++j)
            rw[j][c] = param_load(a.conv_w[i], (ch0 + c) * cs + j, j < cs, a.conv_w[i], a.w_dtype);
    }
    float w[kMaxConv][CPL], bias[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        bias[c] = a.conv_b[i] != nullptr ? decode_elem(rb[c], a.w_dtype) : 0.f;
#pragma unroll
        for (int j = 0; j < kMaxConv; ++j) w[j][c] = j < cs ? decode_elem(rw[j][c], a.w_dtype) : 0.f;
    }

    XT* out = static_cast<XT*>(i == 0 ? a.q : (i == 1 ? a.k : a.v)) + (b * T + t0) * D + ch0;
    const float inv_eps = 1.f / a.l2_eps;
    // tap j of tile token t reads window row t + j (token t0 + t - cm + j)
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
        float s[CPL];
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            float u = bias[c];
#pragma unroll
            for (int j = 0; j < kMaxConv; ++j)
                if (j < cs) u = fmaf(w[j][c], win[t + j][c], u);
            s[c] = u * sigmoid_f(u);
            ss = fmaf(s[c], s[c], ss);
        }
        if (i < 2) {
            // l2 norm over the head: x * min(rsqrt(sum x^2), 1/eps)
            const float rn = fminf(rsqrtf(wave_sum(ss)), inv_eps);
#pragma unroll
            for (int c = 0; c < CPL; ++c) s[c] *= rn;
        }
        if (t < n) st<XT, CPL>(out + t * D, s);
    }

    // the next call's conv cache: inputs T - cm .. T - 1 = window rows n + r
    if (a.hist_out[i] != nullptr && t0 + n == T) {
        XT* ho = static_cast<XT*>(a.hist_out[i]) + b * cm * D + ch0;
#pragma unroll
        for (int r = 0; r < kMaxConv - 1; ++r) {
            float hv[CPL];
#pragma unroll
            for (int c = 0; c < CPL; ++c) hv[c] = 0.f;
#pragma unroll
            for (int rr = 0; rr < kRows; ++rr)
                if (rr == n + r) {
#pragma unroll
                    for (int c = 0; c < CPL; ++c) hv[c] = win[rr][c];
                }
            if (r < cm) st<XT, CPL>(ho + r * D, hv);
        }
    }
}

// ---- prep: the forget gate of one head over a token tile, and its beta ----
template <typename XT, int CPL, int TILE>
__device__ __forceinline__ void gate_unit(const kda_prep_args& a, int64_t b, int64_t t0, int64_t h, int lane) {
    const int64_t Dh = 64 * CPL;
    const int64_t D = a.H * Dh;
    const int64_t ch0 = h * Dh + lane * CPL;
    const int64_t T = a.T;
    const int n = static_cast<int>((T - t0) < TILE ? (T - t0) : TILE);
    const XT* gk = static_cast<const XT*>(a.gk) + b * a.gk_stride[0] + ch0;

    // every load first (rows past the end re-read the last token)
    float z[TILE][CPL];
#pragma unroll
    for (int t = 0; t < TILE; ++t) ld<XT, CPL>(gk + (t0 + (t < n ? t : n - 1)) * a.gk_stride[1], z[t]);
    const int tl = lane < n ? lane : n - 1;
    const RawElem rlogit =
        load_raw_elem(a.beta_logit, b * a.beta_stride[0] + (t0 + tl) * a.beta_stride[1] + h, a.x_dtype);
    RawElem ra[CPL], rd[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        ra[c] = load_raw_elem(a.a_log, ch0 + c, a.p_dtype);
        rd[c] = load_raw_elem(a.dt_bias, ch0 + c, a.p_dtype);
    }
    float neg_a[CPL], dtb[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        neg_a[c] = -__expf(decode_elem(ra[c], a.p_dtype));
        dtb[c] = decode_elem(rd[c], a.p_dtype);
    }
    float* g = static_cast<float*>(a.g) + (b * T + t0) * D + ch0;
#pragma unroll
    for (int t = 0; t < TILE; ++t) {
        float o[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) o[c] = neg_a[c] * softplus(z[t][c] + dtb[c]);
        if (t < n) st<float, CPL>(g + t * D, o);
    }
    if (lane < n)
        static_cast<float*>(a.beta)[(b * T + t0 + lane) * a.H + h] = sigmoid_f(decode_elem(rlogit, a.x_dtype));
}

// One wave per (batch, tile, part, head), part 0..2 = q, k, v, 3 = gate
// (nparts = 4, or 3 when the call leaves the gates to the core).  The host
// keeps the number of units below 2^31, so the unit index is split with
// 32-bit arithmetic.
template <typename XT, int CPLK, int CPLV, int TILE>
__global__ __launch_bounds__(256) void prep_kernel(const kda_prep_args a, uint32_t ntiles, uint32_t units,
                                                   uint32_t nparts) {
    const int lane = threadIdx.x & 63;
    const uint32_t unit = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (unit >= units) return;
    const uint32_t H = static_cast<uint32_t>(a.H);
    uint32_t u = unit;
    const int64_t h = u % H;
    u /= H;
    const int part = static_cast<int>(u % nparts);
    u /= nparts;
    const int64_t t0 = static_cast<int64_t>(u % ntiles) * TILE;
    const int64_t b = u / ntiles;
    if (part < 2)
        conv_unit<XT, CPLK, TILE>(a, part, b, t0, h, lane);
    else if (part == 2)
        conv_unit<XT, CPLV, TILE>(a, 2, b, t0, h, lane);
    else
        gate_unit<XT, CPLK, TILE>(a, b, t0, h, lane);
}

// ---- output: one wave per (batch, head, tile of kOutRows tokens) -----------
constexpr int kOutRows = 8;

template <typename XT, int CPL>
__global__ __launch_bounds__(256) void output_kernel(const kda_output_args a, uint32_t ntiles, uint32_t units) {
    const int lane = threadIdx.x & 63;
    const uint32_t unit = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (unit >= units) return;
    const uint32_t H = static_cast<uint32_t>(a.H);
    const int64_t h = unit % H;
    const uint32_t bt = unit / H;
    const int64_t t0 = static_cast<int64_t>(bt % ntiles) * kOutRows, b = bt / ntiles;
    const int n = static_cast<int>((a.T - t0) < kOutRows ? (a.T - t0) : kOutRows);
    const int64_t V = 64 * CPL;
    const int64_t c0 = lane * CPL;

    // every load first (rows past the end re-read the last token)
    const XT* op = static_cast<const XT*>(a.o) + b * a.o_stride[0] + h * a.o_stride[2] + c0;
    const XT* gp = static_cast<const XT*>(a.gate) + b * a.gate_stride[0] + h * V + c0;
    float o[kOutRows][CPL], gt[kOutRows][CPL];
#pragma unroll
    for (int r = 0; r < kOutRows; ++r) {
        const int64_t t = t0 + (r < n ? r : n - 1);
        ld<XT, CPL>(op + t * a.o_stride[1], o[r]);
        ld<XT, CPL>(gp + t * a.gate_stride[1], gt[r]);
    }
    RawElem rw[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) rw[c] = load_raw_elem(a.weight, h * V + c0 + c, a.w_dtype);
    float w[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) w[c] = decode_elem(rw[c], a.w_dtype);

    XT* yp = static_cast<XT*>(a.y) + (b * a.T + t0) * a.H * V + h * V + c0;
#pragma unroll
    for (int r = 0; r < kOutRows; ++r) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < CPL; ++c) ss = fmaf(o[r][c], o[r][c], ss);
        const float rstd = rsqrtf(wave_sum(ss) / static_cast<float>(V) + a.eps);
        float y[CPL];
#pragma unroll
        for (int c = 0; c < CPL; ++c) y[c] = round_to<XT>((o[r][c] * rstd) * w[c]) * sigmoid_f(gt[r][c]);
        if (r < n) st<XT, CPL>(yp + r * a.H * V, y);
    }
}

// ---- host side --------------------------------------------------------------
bool dtype_ok(int32_t d) { return d == KDA_DTYPE_F32 || d == KDA_DTYPE_F16 || d == KDA_DTYPE_BF16; }
int64_t esize(int32_t d) { return d == KDA_DTYPE_F32 ? 4 : 2; }
bool head_ok(int64_t d) { return d == 64 || d == 128 || d == 256; }

// A vector access of `cpl` elements needs the pointer and every stride aligned to it.
bool vec_ok(const void* p, const int64_t* strides, int n, int64_t cpl, int32_t dtype) {
    if (reinterpret_cast<uintptr_t>(p) % static_cast<uintptr_t>(cpl * esize(dtype)) != 0) return false;
    for (int i = 0; i < n; ++i)
        if (strides[i] % cpl != 0) return false;
    return true;
}

bool overlap(const void* a, int64_t na, const void* b, int64_t nb) {
    const auto a0 = reinterpret_cast<uintptr_t>(a), b0 = reinterpret_cast<uintptr_t>(b);
    return a0 < b0 + static_cast<uintptr_t>(nb) && b0 < a0 + static_cast<uintptr_t>(na);
}

template <typename XT, int CPLK, int CPLV>
void launch_prep(const kda_prep_args& a, hipStream_t stream) {
    // a single token (the decode step) gets units of one token
    const uint32_t nparts = a.g != nullptr ? 4u : 3u;
    if (a.T == 1) {
        const int64_t units = a.B * nparts * a.H;
        hipLaunchKernelGGL((prep_kernel<XT, CPLK, CPLV, 1>), dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256),
                           0, stream, a, 1u, static_cast<uint32_t>(units), nparts);
        return;
    }
    const int64_t ntiles = (a.T + kTile - 1) / kTile;
    const int64_t units = a.B * ntiles * nparts * a.H;
    hipLaunchKernelGGL((prep_kernel<XT, CPLK, CPLV, kTile>), dim3(static_cast<unsigned>((units + 3) / 4)), dim3(256),
                       0, stream, a, static_cast<uint32_t>(ntiles), static_cast<uint32_t>(units), nparts);
}

template <typename XT>
int launch_prep_dims(const kda_prep_args& a, hipStream_t stream) {
    const int ck = static_cast<int>(a.K / 64), cv = static_cast<int>(a.V / 64);
    switch (ck * 10 + cv) {
        case 11: launch_prep<XT, 1, 1>(a, stream); break;
        case 12: launch_prep<XT, 1, 2>(a, stream); break;
        case 14: launch_prep<XT, 1, 4>(a, stream); break;
        case 21: launch_prep<XT, 2, 1>(a, stream); break;
        case 22: launch_prep<XT, 2, 2>(a, stream); break;
        case 24: launch_prep<XT, 2, 4>(a, stream); break;
        case 41: launch_prep<XT, 4, 1>(a, stream); break;
        case 42: launch_prep<XT, 4, 2>(a, stream); break;
        case 44: launch_prep<XT, 4, 4>(a, stream); break;
        default: return KDA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

template <typename XT>
int launch_output_dims(const kda_output_args& a, hipStream_t stream) {
    const int64_t ntiles = (a.T + kOutRows - 1) / kOutRows;
    const int64_t units = a.B * ntiles * a.H;
    const dim3 grid(static_cast<unsigned>((units + 3) / 4)), block(256);
    const uint32_t nt = static_cast<uint32_t>(ntiles), nu = static_cast<uint32_t>(units);
    switch (a.V) {
        case 64: hipLaunchKernelGGL((output_kernel<XT, 1>), grid, block, 0, stream, a, nt, nu); break;
        case 128: hipLaunchKernelGGL((output_kernel<XT, 2>), grid, block, 0, stream, a, nt, nu); break;
        case 256: hipLaunchKernelGGL((output_kernel<XT, 4>), grid, block, 0, stream, a, nt, nu); break;
        default: return KDA_ERR_UNSUPPORTED;
    }
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

int validate_prep(const kda_prep_args* a) {
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->K <= 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (a->conv_size < 1 || a->conv_size > kMaxConv) return KDA_ERR_UNSUPPORTED;
    if (!head_ok(a->K) || !head_ok(a->V)) return KDA_ERR_UNSUPPORTED;
    if (!dtype_ok(a->x_dtype) || !dtype_ok(a->w_dtype) || !dtype_ok(a->p_dtype)) return KDA_ERR_BAD_DTYPE;
    if (!(a->l2_eps > 0.f)) return KDA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->H == 0) return KDA_OK;
    // no tokens: nothing to compute, and a requested conv cache would need a copy
    if (a->T == 0) {
        for (int i = 0; i < 3; ++i)
            if (a->hist_out[i] != nullptr) return KDA_ERR_BAD_SHAPE;
        return KDA_OK;
    }
    const int64_t cm = a->conv_size - 1;
    for (int i = 0; i < 3; ++i) {
        if (a->x[i] == nullptr || a->conv_w[i] == nullptr) return KDA_ERR_NULL_POINTER;
        const int64_t cpl = (i == 2 ? a->V : a->K) / 64;
        if (!vec_ok(a->x[i], a->x_stride[i], 2, cpl, a->x_dtype)) return KDA_ERR_BAD_SHAPE;
        const int64_t D = a->H * (i == 2 ? a->V : a->K);
        if (a->hist_in[i] && !vec_ok(a->hist_in[i], nullptr, 0, cpl, a->x_dtype)) return KDA_ERR_BAD_SHAPE;
        if (a->hist_out[i]) {
            if (!vec_ok(a->hist_out[i], nullptr, 0, cpl, a->x_dtype)) return KDA_ERR_BAD_SHAPE;
            // in place only when one tile holds every token: the wave that
            // writes the cache is then the one that read it
            const int64_t nb = a->B * cm * D * esize(a->x_dtype);
            if (a->hist_in[i] && overlap(a->hist_in[i], nb, a->hist_out[i], nb) &&
                !(a->hist_in[i] == a->hist_out[i] && a->T <= kTile))
                return KDA_ERR_ALIAS;
        }
    }
    if (!a->q || !a->k || !a->v) return KDA_ERR_NULL_POINTER;
    // g and beta both absent: the gates are left to the core's gated entry points
    const bool gates = a->g != nullptr || a->beta != nullptr;
    if (gates && (!a->gk || !a->a_log || !a->dt_bias || !a->beta_logit || !a->g || !a->beta))
        return KDA_ERR_NULL_POINTER;
    const int64_t ck = a->K / 64, cv = a->V / 64;
    if (!vec_ok(a->q, nullptr, 0, ck, a->x_dtype) || !vec_ok(a->k, nullptr, 0, ck, a->x_dtype) ||
        !vec_ok(a->v, nullptr, 0, cv, a->x_dtype))
        return KDA_ERR_BAD_SHAPE;
    if (gates && (!vec_ok(a->gk, a->gk_stride, 2, ck, a->x_dtype) || !vec_ok(a->g, nullptr, 0, ck, KDA_DTYPE_F32)))
        return KDA_ERR_BAD_SHAPE;
    const int64_t ntiles = (a->T + kTile - 1) / kTile;
    if (a->B * ntiles * 4 * a->H > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return KDA_OK;
}

int validate_output(const kda_output_args* a) {
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (!head_ok(a->V)) return KDA_ERR_UNSUPPORTED;
    if (!dtype_ok(a->x_dtype) || !dtype_ok(a->w_dtype)) return KDA_ERR_BAD_DTYPE;
    if (!(a->eps >= 0.f)) return KDA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->T == 0 || a->H == 0) return KDA_OK;
    if (!a->o || !a->gate || !a->weight || !a->y) return KDA_ERR_NULL_POINTER;
    const int64_t cpl = a->V / 64;
    if (!vec_ok(a->o, a->o_stride, 3, cpl, a->x_dtype) || !vec_ok(a->gate, a->gate_stride, 2, cpl, a->x_dtype) ||
        !vec_ok(a->y, nullptr, 0, cpl, a->x_dtype))
        return KDA_ERR_BAD_SHAPE;
    if (a->B * ((a->T + kOutRows - 1) / kOutRows) * a->H > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return KDA_OK;
}

}  // namespace

}  // namespace kda

extern "C" {

int kda_prep_fwd(const kda_prep_args* args, void* stream) {
    const int st = kda::validate_prep(args);
    if (st != KDA_OK || args->B == 0 || args->H == 0 || args->T == 0) return st;
    const auto s = static_cast<hipStream_t>(stream);
    switch (args->x_dtype) {
        case KDA_DTYPE_F16: return kda::launch_prep_dims<_Float16>(*args, s);
        case KDA_DTYPE_BF16: return kda::launch_prep_dims<kda::bf16_t>(*args, s);
        default: return kda::launch_prep_dims<float>(*args, s);
    }
}

int kda_output_fwd(const kda_output_args* args, void* stream) {
    const int st = kda::validate_output(args);
    if (st != KDA_OK || args->B == 0 || args->T == 0 || args->H == 0) return st;
    const auto s = static_cast<hipStream_t>(stream);
    switch (args->x_dtype) {
        case KDA_DTYPE_F16: return kda::launch_output_dims<_Float16>(*args, s);
        case KDA_DTYPE_BF16: return kda::launch_output_dims<kda::bf16_t>(*args, s);
        default: return kda::launch_output_dims<float>(*args, s);
    }
}

}  // extern "C"
