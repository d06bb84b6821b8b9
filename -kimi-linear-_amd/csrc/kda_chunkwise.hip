// Chunkwise KDA forward for gfx950: fp16 MFMA, fp32 accumulation, fp32 state.
//
// Replaces the body of kda_chunkwise (kimi_linear/kda.py:111-185).  The maths
// is the reference's UT-transform form (paper Eq. 6-9) evaluated per internal
// chunk of BT = 16 tokens; the recurrence is chunk-size invariant, so the
// caller's chunk_size only fixes the T % chunk_size == 0 contract.
//
// Per (b, h) and internal chunk (rows c, i in [0, 16)), with a_t = exp(g_t):
//   E[r]   = prod_{t<=r} a_t              (= exp(gc_r), per channel)
//   L[c,i] = beta_c <k_c, k_i * prod_{t=i+1..c} a_t>,  i < c
//   A[c,i] = scale <q_c, k_i * prod_{t=i+1..c} a_t>,   i <= c
//   M      = (I + L)^-1 Diag(beta)
//   P      = M (V - (E * K) S)           (= U - W S with U = M V, W = M (E * K))
//   O      = scale (E * Q) S + A P
//   S     <- Diag(E[15]) S + ((E[15]/E) * K)^T P
//
// Decay factoring without pairwise exponentials: every pair i < c of a chunk
// has a unique highest differing bit b; c has it set, i clear, and both sit in
// the aligned block of 2^(b+1) rows whose upper half starts at ref.  Then
//   prod_{t=i+1..c} a_t = (prod_{t=ref+1..c} a_t) * (prod_{t=i+1..ref} a_t),
// both factors <= 1, so per level b one [16 x K] operand X_b (row r = k_r times
// its factor) gives L_b = X_b X_b^T as a plain MFMA product, masked to level
// b's pairs.  A factor only underflows when the true decay is smaller still.
// Level "diag" (factor 1) gives A[c, c].
//
// (I + L)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8) for the nilpotent L: four
// 16x16 products and three squarings on MFMA (fp16 hi/lo split operands),
// entirely in registers.  An MFMA accumulator holds X[4g+j][n] in lane n+16g,
// slot j -- the B-operand layout of X and the A-operand layout of X^T -- so a
// chain that keeps X and X^T side by side needs no data movement.
//
// Software pipeline, one workgroup per (b, h, 16*NC state columns):
//   NC consumer waves: wave w owns state columns [16w, 16w+16) for all K rows
//     as MFMA accumulators and runs the sequential chain of chunk n.
//   NP = K/32 producer waves: two lanes per channel (8 rows each) build the
//     operands of chunk n+2 straight from prefetched global loads; producer
//     wave 0 inverts (I + L) of chunk n+1 while the others compute the level
//     products of chunk n+2.
// Each step has two phases separated by workgroup barriers:
//   A: producers: decays + level operands (n+2)
//      | consumers: Z = (E*K) S, O = (E*Q) S, P = M (V - Z)   (n)
//   B: producer 0: (I + L)^-1 (n+1); others: level products (n+2); all
//      producers: E-scaled operands (n+2)
//      | consumers: O += A P, store O, S <- E15 S + Khat^T P   (n)
// Operands that are not exact in fp16 and carry the state (S, P, M and
// V - Z) are split into fp16 hi + lo; the others are single fp16 with fp32
// accumulation.  Operands read through LDS transpose loads are stored
// k-major, so each producer lane stores a channel's 8 rows with one 16-byte
// write.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int BT = 16;    // tokens per internal chunk
constexpr int RP = 24;    // padded row (halfs) of the [*][16] fp16 matrices (48 B rows)
constexpr int LP = 20;    // padded row (floats) of the 16x16 fp32 L
constexpr int NLEV = 5;   // operand levels: 0 = diagonal, 1 + b for bit b = 0..3
constexpr int kXcds = 8;  // accelerator complex dies on MI355X

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Input element access through raw buffer loads.  A chunk's descriptor covers
// exactly its rows before T, so rows past T read as zero -- the neutral
// padding (k = q = v = g = beta = 0) -- with no clamping or masking.  Loaded
// values are held one per 32-bit register and converted only at use, so a
// prefetch load is never followed by a wait.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(nbytes), 0x00020000);
}
__device__ __forceinline__ uint32_t bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(off), 0, 0);
}
__device__ __forceinline__ uint32_t bload32(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(off), 0, 0);
}

template <typename TQ> struct QIn;
template <> struct QIn<_Float16> {
    static __device__ __forceinline__ uint32_t ld(__amdgpu_buffer_rsrc_t r, uint32_t off) { return bload16(r, off); }
    static __device__ __forceinline__ float f(uint32_t r) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(r)));
    }
    static __device__ __forceinline__ h8 oct(const uint32_t (&r)[8]) {   // exact: repack the bits
        h8 x;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(r[i]));
        return x;
    }
};
template <> struct QIn<bf16_t> {
    static __device__ __forceinline__ uint32_t ld(__amdgpu_buffer_rsrc_t r, uint32_t off) { return bload16(r, off); }
    static __device__ __forceinline__ float f(uint32_t r) { return __uint_as_float(r << 16); }
    static __device__ __forceinline__ h8 oct(const uint32_t (&r)[8]) {
        h8 x;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = static_cast<_Float16>(f(r[i]));
        return x;
    }
};
template <> struct QIn<float> {
    static __device__ __forceinline__ uint32_t ld(__amdgpu_buffer_rsrc_t r, uint32_t off) { return bload32(r, off); }
    static __device__ __forceinline__ float f(uint32_t r) { return __uint_as_float(r); }
    static __device__ __forceinline__ h8 oct(const uint32_t (&r)[8]) {
        h8 x;
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = static_cast<_Float16>(f(r[i]));
        return x;
    }
};

// Eight fp32 values rounded to fp16.
__device__ __forceinline__ h8 to_h8(const float (&x)[8]) {
    h8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(x[i]);
    return r;
}

// Operands consumed through LDS transpose reads are stored k-major ([K][16]:
// the 16 chunk rows of one channel are contiguous), so a producer lane writes
// its 8 rows of a channel with one 16-byte store.
template <int K>
struct __align__(16) Smem {
    _Float16 XT[NLEV][K][BT];              // level operands (k * factor), k-major
    _Float16 YT[NLEV][K][BT];              // query-side level operands (q * factor)
    _Float16 QET[3][K][BT];                // q * E                  (chunk % 3)
    _Float16 KET[3][K][BT];                // k * E                  (chunk % 3)
    _Float16 KHT[3][K][RP];                // (k * E15 / E)^T        (chunk % 3)
    _Float16 AM[3][BT][RP];                // scale * A              (chunk % 3)
    _Float16 MH[BT][RP];                   // M hi                   (single)
    _Float16 ML[BT][RP];                   // M lo
    float L[2][BT][LP];                    // beta-scaled L          (chunk % 2)
    float elast[3][K];                     // E[15]                  (chunk % 3)
    float beta[2][BT];                     //                        (chunk % 2)
};

__device__ __forceinline__ h4 frag16(const _Float16* base, int stride, int row, int lg) {
    return *reinterpret_cast<const h4*>(base + row * stride + 4 * lg);
}

typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

// MFMA row fragment from a k-major [K][16] fp16 matrix X^T through the LDS
// transpose read (ds_read_b64_tr_b16): within each 16-lane group, lane 4j+q
// supplies the four rows 4q..4q+3 of channel kbase+j, and lane i receives
// X[i][kbase + 0..3] -- the A-operand fragment of row i, which is also the
// B-operand fragment of column i of X^T.
__device__ __forceinline__ h4 frag16_tr(const _Float16* xt, int kbase, int ln) {
    const _Float16* p = xt + (kbase + (ln >> 2)) * BT + 4 * (ln & 3);
    return __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p)));
}

// 16x16x32 fragment: slots 0-3 hold k = 32u + 4lg + j, slots 4-7 hold
// k = 32u + 16 + 4lg + j.  A and B fragments use the same assignment, so the
// product is the full 32-wide dot product whatever slot order the unit uses;
// it also matches the two state tiles 2u, 2u+1 held by a consumer lane group.
__device__ __forceinline__ h8 frag32_tr(const _Float16* xt, int lg, int ln, int u) {
    const h4 lo = frag16_tr(xt, 32 * u + 4 * lg, ln);
    const h4 hi = frag16_tr(xt, 32 * u + 16 + 4 * lg, ln);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// fp16 lo halves of two fp32 values given their fp16 hi halves: f16(x - hi).
// The compiler forms x - hi with v_fma_mix_f32 (hi read as fp16 in place) and
// packs the pair with one conversion.  (A hand-written v_fma_mixlo/mixhi
// pair on one register is left out: the compiler's hazard pass does not see
// inside inline asm, and that sequence gave run-to-run differences.)
__device__ __forceinline__ h2 split_lo_pair(float x0, float x1, h2 hi) {
    return h2{static_cast<_Float16>(x0 - static_cast<float>(hi[0])),
              static_cast<_Float16>(x1 - static_cast<float>(hi[1]))};
}

// Four fp32 values as fp16 hi + lo (x ~= hi + lo to ~2^-22 relative).
__device__ __forceinline__ void split4(const f4& x, h4& hi, h4& lo) {
    const h2 h01 = h2{static_cast<_Float16>(x[0]), static_cast<_Float16>(x[1])};
    const h2 h23 = h2{static_cast<_Float16>(x[2]), static_cast<_Float16>(x[3])};
    const h2 l01 = split_lo_pair(x[0], x[1], h01);
    const h2 l23 = split_lo_pair(x[2], x[3], h23);
    hi = h4{h01[0], h01[1], h23[0], h23[1]};
    lo = h4{l01[0], l01[1], l23[0], l23[1]};
}

// x of lane (lane ^ 32), through the VALU cross-half swap (no LDS traffic):
// permlane32_swap(x, x) returns {x of lane l-32 in the upper half,
// x of lane l+32 in the lower half} as its two results.
__device__ __forceinline__ float xor32(float x, int lane) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
}

// An fp32 accumulator tile split into fp16 hi + lo operands.
struct Split4 {
    h4 hi, lo;
    __device__ explicit Split4(const f4& x) { split4(x, hi, lo); }
};

// acc(A_layout(a) * B_layout(b)) with both operands split: hi*hi + hi*lo + lo*hi.
__device__ __forceinline__ f4 mm3(const Split4& a, const Split4& b) {
    f4 d = {0.f, 0.f, 0.f, 0.f};
    d = mfma16x16x16(a.hi, b.hi, d);
    d = mfma16x16x16(a.hi, b.lo, d);
    d = mfma16x16x16(a.lo, b.hi, d);
    return d;
}

// Raw per-lane inputs of one chunk for a producer lane (one channel, 8 rows).
struct PrepIn {
    uint32_t g[8], q[8], k[8];
    uint32_t beta;
};

// Prefetched values are converted only where they are used.  Left alone, the
// compiler hoists a conversion (or the packing of two fp16 loads into one
// register) up to the load, which puts a wait for the whole prefetch right
// after it is issued.  An empty volatile asm that "modifies" the registers at
// the point of use keeps every such instruction, and the wait, there.
template <int N>
__device__ __forceinline__ void use_here(uint32_t (&r)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(r[i]));
}
__device__ __forceinline__ void use_here(PrepIn& p) {
    use_here(p.g);
    use_here(p.q);
    use_here(p.k);
    asm volatile("" : "+v"(p.beta));
}

// Accumulator-layout state tiles: S[t][j] = state[16t + 4lg + j][col]; `off`
// is the element offset of (row 4lg, col) and rows are V apart.  All loads
// are issued before any is used.
template <int KT, typename TS>
__device__ __forceinline__ void load_state_t(f4 (&S)[KT], const TS* p, int64_t off, int64_t V) {
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) S[t][j] = Elem<TS>::ld(p + off + (16 * t + j) * V);
}
template <int KT>
__device__ __forceinline__ void load_state(f4 (&S)[KT], const void* p, int dtype, int64_t off, int64_t V) {
    if (p == nullptr) {
#pragma unroll
        for (int t = 0; t < KT; ++t) S[t] = f4{0.f, 0.f, 0.f, 0.f};
    } else if (dtype == KDA_DTYPE_F32) {
        load_state_t<KT>(S, static_cast<const float*>(p), off, V);
    } else if (dtype == KDA_DTYPE_F16) {
        load_state_t<KT>(S, static_cast<const _Float16*>(p), off, V);
    } else {
        load_state_t<KT>(S, static_cast<const bf16_t*>(p), off, V);
    }
}
template <int KT, typename TS>
__device__ __forceinline__ void store_state_t(const f4 (&S)[KT], TS* p, int64_t off, int64_t V) {
#pragma unroll
    for (int t = 0; t < KT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) Elem<TS>::st(p + off + (16 * t + j) * V, S[t][j]);
}
template <int KT>
__device__ __forceinline__ void store_state(const f4 (&S)[KT], void* p, int dtype, int64_t off, int64_t V) {
    if (dtype == KDA_DTYPE_F32) store_state_t<KT>(S, static_cast<float*>(p), off, V);
    else if (dtype == KDA_DTYPE_F16) store_state_t<KT>(S, static_cast<_Float16*>(p), off, V);
    else store_state_t<KT>(S, static_cast<bf16_t*>(p), off, V);
}

template <int K, int NC, typename TQ>
struct Kern {
    static constexpr int KT = K / 16;       // 16-row state tiles
    static constexpr int KU = K / 32;       // 32-wide k blocks
    static constexpr int NP = K / 32;       // producer waves
    static constexpr int NWAVE = NC + NP;
    static constexpr int VT = 16 * NC;

    const kda_fwd_args& a;
    Smem<K>& sm;
    int64_t b, h, T;
    int nch;
    float scale;
    int lane, ln, lg;
    // per-row byte strides and this lane's byte offsets inside a chunk
    uint32_t rs_q, rs_k, rs_g, rs_v, rs_b;
    uint32_t off_q[8], off_k[8], off_g[8], off_v[4], off_b;

    __device__ Kern(const kda_fwd_args& args, Smem<K>& s) : a(args), sm(s) {}

    // Rows of chunk `chunk` that lie before T (1..BT).
    __device__ int rows_in(int chunk) const {
        const int64_t left = T - static_cast<int64_t>(chunk) * BT;
        return left < BT ? static_cast<int>(left) : BT;
    }

    // Buffer descriptor over the rows of one chunk of a [B, T, H, D] view
    // (elements of size es, token stride rs bytes) at (b, t0, h, 0).
    __device__ __amdgpu_buffer_rsrc_t chunk_rsrc(const void* p, const int64_t (&st)[3], int es, uint32_t rs,
                                                 int chunk) const {
        const int64_t e = b * st[0] + static_cast<int64_t>(chunk) * BT * st[1] + h * st[2];
        return make_rsrc(static_cast<const char*>(p) + e * es, static_cast<uint32_t>(rows_in(chunk)) * rs);
    }

    // ------------------------------------------------------------ producers
    __device__ void prep_load(PrepIn& in, int chunk, bool beta_lane) const {
        const auto rq = chunk_rsrc(a.q, a.q_stride, sizeof(TQ), rs_q, chunk);
        const auto rk = chunk_rsrc(a.k, a.k_stride, sizeof(TQ), rs_k, chunk);
        const auto rg = chunk_rsrc(a.g, a.g_stride, 4, rs_g, chunk);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            in.g[i] = bload32(rg, off_g[i]);
            in.q[i] = QIn<TQ>::ld(rq, off_q[i]);
            in.k[i] = QIn<TQ>::ld(rk, off_k[i]);
        }
        if (beta_lane) in.beta = bload32(chunk_rsrc(a.beta, a.beta_stride, 4, rs_b, chunk), off_b);
    }

    // Producer values of one chunk carried from phase A to phase B.
    struct PrepMid {
        h8 qh, kh;                                  // the 8 rows as fp16
        float pre[8], suf[8];
        float emul, kmul;
    };

    // Phase A operands of one chunk for channel c, rows 8*hf .. 8*hf+7: the
    // decays, the level operands X_b, Y_b (k-major, one 16-byte store each)
    // and beta.  Products are packed fp16: factor pairs (fp32 chains rounded
    // once) times the fp16 k / q pairs.
    __device__ void prep_levels(const PrepIn& pin_, PrepMid& mid, int chunk, int c, int hf,
                                bool beta_lane) const {
        PrepIn pin = pin_;
        use_here(pin);
        float al[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) al[i] = fast_exp(__uint_as_float(pin.g[i]));
        mid.qh = QIn<TQ>::oct(pin.q);
        mid.kh = QIn<TQ>::oct(pin.k);
        mid.pre[0] = al[0];                             // prod_{t<=i} within the half
#pragma unroll
        for (int i = 1; i < 8; ++i) mid.pre[i] = mid.pre[i - 1] * al[i];
        mid.suf[7] = 1.f;                               // prod_{t=i+1..7} within the half
#pragma unroll
        for (int i = 6; i >= 0; --i) mid.suf[i] = mid.suf[i + 1] * al[i + 1];
        const float other = xor32(mid.pre[7], lane);    // product over the other half
        const float a8 = xor32(al[0], lane);            // lower half: a of row 8
        const bool up = hf != 0;
        mid.emul = up ? other : 1.f;                    // E = exp(gc): prefix over the chunk
        mid.kmul = up ? 1.f : other;                    // E15 / E: suffix over the chunk
        if (beta_lane) sm.beta[chunk % 2][lane] = __uint_as_float(pin.beta);

        const int r0 = 8 * hf;
        // level factors F_b(row); query-side operands of key rows are never
        // read unmasked, so Y is written for every row with the same factor
        auto store = [&](int lev, h8 x, h8 y) {
            *reinterpret_cast<h8*>(&sm.XT[lev][c][r0]) = x;
            *reinterpret_cast<h8*>(&sm.YT[lev][c][r0]) = y;
        };
        float f[8];
        auto level = [&](int lev) {
            const h8 fh = to_h8(f);
            store(lev, mid.kh * fh, mid.qh * fh);
        };
        // level "diag": factor 1
        store(0, mid.kh, mid.qh);
        // level b = 0: ref = odd rows; key rows even -> a_{i+1}
#pragma unroll
        for (int i = 0; i < 8; i += 2) { f[i] = al[i + 1]; f[i + 1] = 1.f; }
        level(1);
        // level b = 1: ref = 2 mod 4
#pragma unroll
        for (int i = 0; i < 8; i += 4) {
            f[i + 1] = al[i + 2];
            f[i] = al[i + 1] * f[i + 1];
            f[i + 2] = 1.f;
            f[i + 3] = al[i + 3];
        }
        level(2);
        // level b = 2: ref = 4 within the half
        f[3] = al[4]; f[2] = al[3] * f[3]; f[1] = al[2] * f[2]; f[0] = al[1] * f[1];
        f[4] = 1.f; f[5] = al[5]; f[6] = f[5] * al[6]; f[7] = f[6] * al[7];
        level(3);
        // level b = 3: ref = 8; upper half = query rows (prod_{9..r}), lower = key rows
        {
            float q = 1.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (i > 0) q *= al[i];
                f[i] = up ? q : mid.suf[i] * a8;
            }
        }
        level(4);
    }

    // Phase B operands of one chunk: q * E, k * E, k * E15 / E and E15.
    __device__ void prep_e(const PrepMid& mid, int chunk, int c, int hf) const {
        const int b3 = chunk % 3, r0 = 8 * hf;
        float e[8], sf[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            e[i] = mid.pre[i] * mid.emul;
            sf[i] = mid.suf[i] * mid.kmul;
        }
        const h8 eh = to_h8(e), sh = to_h8(sf);
        *reinterpret_cast<h8*>(&sm.QET[b3][c][r0]) = mid.qh * eh;
        *reinterpret_cast<h8*>(&sm.KET[b3][c][r0]) = mid.kh * eh;
        *reinterpret_cast<h8*>(&sm.KHT[b3][c][r0]) = mid.kh * sh;
        if (hf) sm.elast[b3][c] = mid.pre[7] * mid.emul;
    }

    // Level product of one chunk: writes the level's pairs of L and A.
    __device__ void level_mfma(int lev, int chunk) const {
        f4 accL = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const h8 xf = frag32_tr(&sm.XT[lev][0][0], lg, ln, u);
            const h8 yf = frag32_tr(&sm.YT[lev][0][0], lg, ln, u);
            if (lev != 0) accL = mfma16x16x32(xf, xf, accL);
            accA = mfma16x16x32(yf, xf, accA);
        }
        const int i = ln;
        const int lb = chunk % 2, ab = chunk % 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * lg + j;
            if (lev == 0) {
                if (i >= c) {
                    sm.L[lb][c][i] = 0.f;
                    sm.AM[ab][c][i] = static_cast<_Float16>(i == c ? accA[j] * scale : 0.f);
                }
            } else {
                const int bb = lev - 1;
                const bool pair = ((c >> (bb + 1)) == (i >> (bb + 1))) && ((c >> bb) & 1) && !((i >> bb) & 1);
                if (pair) {
                    sm.L[lb][c][i] = sm.beta[lb][c] * accL[j];
                    sm.AM[ab][c][i] = static_cast<_Float16>(accA[j] * scale);
                }
            }
        }
    }

    // M = (I + L)^-1 Diag(beta) of one chunk (one wave), stored as hi/lo
    // A-operand fragments for the consumers.
    __device__ void solve_m(int chunk) const {
        const int lb = chunk % 2;
        f4 Lc, Lt;                                       // acc(L), acc(L^T)
#pragma unroll
        for (int j = 0; j < 4; ++j) Lc[j] = sm.L[lb][4 * lg + j][ln];
        {
            const float4 r = *reinterpret_cast<const float4*>(&sm.L[lb][ln][4 * lg]);
            Lt[0] = r.x; Lt[1] = r.y; Lt[2] = r.z; Lt[3] = r.w;
        }
        const Split4 lc(Lc), lt(Lt);
        const Split4 l2(mm3(lt, lc)), l2t(mm3(lc, lt));  // L^2, (L^2)^T
        const Split4 l4(mm3(l2t, l2)), l4t(mm3(l2, l2t));
        const Split4 l8(mm3(l4t, l4));
        f4 Q;                                            // acc(I - L^T)
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] = (4 * lg + j == ln ? 1.f : 0.f) - Lt[j];
        Q += mm3(l2, Split4(Q));
        Q += mm3(l4, Split4(Q));
        Q += mm3(l8, Split4(Q));                         // acc(Minv^T) = A-layout of Minv
        const float4 bt = *reinterpret_cast<const float4*>(&sm.beta[lb][4 * lg]);
        Q[0] *= bt.x; Q[1] *= bt.y; Q[2] *= bt.z; Q[3] *= bt.w;
        h4 mh, ml;
        split4(Q, mh, ml);
        *reinterpret_cast<h4*>(&sm.MH[ln][4 * lg]) = mh;
        *reinterpret_cast<h4*>(&sm.ML[ln][4 * lg]) = ml;
    }

    // ------------------------------------------------------------ consumers
    __device__ void v_load(uint32_t (&vr)[4], int chunk) const {
        const auto rv = chunk_rsrc(a.v, a.v_stride, sizeof(TQ), rs_v, chunk);
#pragma unroll
        for (int j = 0; j < 4; ++j) vr[j] = QIn<TQ>::ld(rv, off_v[j]);
    }

    __device__ void consumer_a(int chunk, const uint32_t (&vraw_)[4], f4 (&S)[KT], f4& P, f4& O) const {
        uint32_t vraw[4] = {vraw_[0], vraw_[1], vraw_[2], vraw_[3]};
        use_here(vraw);
        float vr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) vr[j] = QIn<TQ>::f(vraw[j]);
        h8 shi[KU], slo[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            h4 h0, l0, h1, l1;
            split4(S[2 * u], h0, l0);
            split4(S[2 * u + 1], h1, l1);
            shi[u] = h8{h0[0], h0[1], h0[2], h0[3], h1[0], h1[1], h1[2], h1[3]};
            slo[u] = h8{l0[0], l0[1], l0[2], l0[3], l1[0], l1[1], l1[2], l1[3]};
        }
        // Z = (k * E) S and O = (q * E) S over the K channels
        const int cb = chunk % 3;
        f4 Z = {0.f, 0.f, 0.f, 0.f};
        O = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const h8 kf = frag32_tr(&sm.KET[cb][0][0], lg, ln, u);
            Z = mfma16x16x32(kf, shi[u], Z);
            Z = mfma16x16x32(kf, slo[u], Z);
            const h8 qf = frag32_tr(&sm.QET[cb][0][0], lg, ln, u);
            O = mfma16x16x32(qf, shi[u], O);
            O = mfma16x16x32(qf, slo[u], O);
        }
        // P = U - W S = M (V - Z)
        f4 R;
#pragma unroll
        for (int j = 0; j < 4; ++j) R[j] = vr[j] - Z[j];
        const Split4 r(R);
        const h4 mh = frag16(&sm.MH[0][0], RP, ln, lg);
        const h4 ml = frag16(&sm.ML[0][0], RP, ln, lg);
        P = f4{0.f, 0.f, 0.f, 0.f};
        P = mfma16x16x16(mh, r.hi, P);
        P = mfma16x16x16(mh, r.lo, P);
        P = mfma16x16x16(ml, r.hi, P);
    }

    __device__ void consumer_b(int chunk, f4 (&S)[KT], const f4& P, f4 O, int64_t col0, uint32_t ocol) const {
        const int cb = chunk % 3;
#pragma unroll
        for (int j = 0; j < 4; ++j) O[j] *= scale;
        h4 ph, pl;
        split4(P, ph, pl);
        const h4 af = frag16(&sm.AM[cb][0][0], RP, ln, lg);
        O = mfma16x16x16(af, ph, O);
        O = mfma16x16x16(af, pl, O);
        // o[b, t, h, col]: wave-uniform chunk base + 32-bit lane offset
        TQ* o = static_cast<TQ*>(a.o) + ((b * T + static_cast<int64_t>(chunk) * BT) * a.H + h) * a.V + col0;
        const uint32_t orow = static_cast<uint32_t>(a.H * a.V);
        const int nrow = rows_in(chunk);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * lg + j < nrow) Elem<TQ>::st(o + (4 * lg + j) * orow + ocol, O[j]);
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const float4 e = *reinterpret_cast<const float4*>(&sm.elast[cb][16 * t + 4 * lg]);
            S[t][0] *= e.x; S[t][1] *= e.y; S[t][2] *= e.z; S[t][3] *= e.w;
            const h4 kf = frag16(&sm.KHT[cb][16 * t][0], RP, ln, lg);
            S[t] = mfma16x16x16(kf, ph, S[t]);
            S[t] = mfma16x16x16(kf, pl, S[t]);
        }
    }
};

template <int K, int NC, typename TQ>
__global__ __launch_bounds__(64 * (NC + K / 32)) void chunkwise_kernel(const kda_fwd_args a) {
    using KN = Kern<K, NC, TQ>;
    constexpr int NP = KN::NP, KT = KN::KT, VT = KN::VT;
    static_assert(K % 32 == 0 && K <= 128, "chunkwise supports K in {32, 64, 128}");
    __shared__ Smem<K> sm;
    KN kn(a, sm);

    const int64_t H = a.H, V = a.V;
    const int nvt = static_cast<int>(V / VT);
    // XCD-aware order: workgroups are dealt round-robin over the 8 XCDs, so
    // renumber them to put consecutive logical workgroups -- the V-tiles of
    // one head, which all read the head's q, k and g -- on one XCD and its L2.
    int bid = blockIdx.x;
    if (gridDim.x % kXcds == 0) bid = (bid % kXcds) * (gridDim.x / kXcds) + bid / kXcds;
    const int vt = bid % nvt;
    bid /= nvt;
    kn.h = bid % H;
    kn.b = bid / H;
    kn.T = a.T;
    kn.nch = static_cast<int>((a.T + BT - 1) / BT);
    kn.scale = a.scale;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    kn.lane = tid & 63;
    kn.ln = kn.lane & 15;
    kn.lg = kn.lane >> 4;
    const int nch = kn.nch;

    const bool consumer = wave < NC;
    // consumer state: S[t][j] = S[16t + 4lg + j][col], col = col0 + ocol
    const int64_t col0 = static_cast<int64_t>(vt) * VT;
    const uint32_t ocol = static_cast<uint32_t>(16 * (consumer ? wave : 0) + kn.ln);
    const int64_t col = col0 + ocol;
    const int64_t sbase = (kn.b * H + kn.h) * static_cast<int64_t>(K) * V;
    // producer lane: channel c, rows 8*hf .. 8*hf+7
    const int pw = wave - NC;
    const int pc = 32 * (consumer ? 0 : pw) + (kn.lane & 31);
    const int phf = kn.lane >> 5;
    const bool beta_lane = !consumer && pw == 0 && kn.lane < BT;
    {
        const uint32_t eq = static_cast<uint32_t>(sizeof(TQ));
        kn.rs_q = static_cast<uint32_t>(a.q_stride[1]) * eq;
        kn.rs_k = static_cast<uint32_t>(a.k_stride[1]) * eq;
        kn.rs_v = static_cast<uint32_t>(a.v_stride[1]) * eq;
        kn.rs_g = static_cast<uint32_t>(a.g_stride[1]) * 4u;
        kn.rs_b = static_cast<uint32_t>(a.beta_stride[1]) * 4u;
        // lane byte offsets inside a chunk; rows past T fall outside the
        // chunk's descriptor and read as zero
        const uint32_t pcol = static_cast<uint32_t>(pc);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t r = static_cast<uint32_t>(8 * phf + i);
            kn.off_q[i] = r * kn.rs_q + pcol * eq;
            kn.off_k[i] = r * kn.rs_k + pcol * eq;
            kn.off_g[i] = r * kn.rs_g + pcol * 4u;
        }
        kn.off_b = static_cast<uint32_t>(kn.lane) * kn.rs_b;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            kn.off_v[j] = static_cast<uint32_t>(4 * kn.lg + j) * kn.rs_v + static_cast<uint32_t>(col) * eq;
    }

    // step sp: producers build chunk sp, producer 0 inverts chunk sp-1,
    // consumers run chunk sp-2.  Each role runs its own loop with the same
    // two barriers per step; register sets alternate with sp's parity and
    // every prefetch is issued unconditionally (chunk index clamped), so the
    // compiler's load accounting stays exact and a wait covers only the chunk
    // being consumed.
    const int nsteps = nch + 2;
    const int last = nch - 1;
    if (consumer) {
        f4 S[KT];
        uint32_t vr0[4], vr1[4];
        load_state<KT>(S, a.state_in, a.state_in_dtype, sbase + (4 * kn.lg) * V + col, V);
        kn.v_load(vr0, 0);
        kn.v_load(vr1, min(1, last));
        f4 P = {0.f, 0.f, 0.f, 0.f}, O = {0.f, 0.f, 0.f, 0.f};
        auto step = [&](int sp, uint32_t (&vr)[4]) {
            const int cc = sp - 2;
            if (cc >= 0) {
                kn.consumer_a(cc, vr, S, P, O);
                kn.v_load(vr, min(cc + 2, last));
            }
            __syncthreads();
            if (cc >= 0) kn.consumer_b(cc, S, P, O, col0, ocol);
            __syncthreads();
        };
        for (int sp = 0; sp < nsteps; sp += 2) {
            step(sp, vr0);
            if (sp + 1 < nsteps) step(sp + 1, vr1);
        }
        store_state<KT>(S, a.state_out, a.state_out_dtype, sbase + (4 * kn.lg) * V + col, V);
    } else {
        PrepIn pin0, pin1;
        kn.prep_load(pin0, 0, beta_lane);
        kn.prep_load(pin1, min(1, last), beta_lane);
        typename KN::PrepMid mid;
        auto step = [&](int sp, PrepIn& pin) {
            const int cp = sp, cs = sp - 1;
            if (cp < nch) {
                kn.prep_levels(pin, mid, cp, pc, phf, beta_lane);
                kn.prep_load(pin, min(cp + 2, last), beta_lane);
            }
            __syncthreads();
            if (pw == 0 && cs >= 0 && cs < nch) kn.solve_m(cs);
            if (cp < nch) {
                if (NP == 1) {
#pragma unroll
                    for (int lev = 0; lev < NLEV; ++lev) kn.level_mfma(lev, cp);
                } else {
#pragma unroll
                    for (int lev = 0; lev < NLEV; ++lev)
                        if (1 + lev % (NP - 1) == pw) kn.level_mfma(lev, cp);
                }
                kn.prep_e(mid, cp, pc, phf);
            }
            __syncthreads();
        };
        for (int sp = 0; sp < nsteps; sp += 2) {
            step(sp, pin0);
            if (sp + 1 < nsteps) step(sp + 1, pin1);
        }
    }
}

template <int K, int NC, typename TQ>
int launch_knq(const kda_fwd_args& a, hipStream_t stream) {
    const int64_t blocks = a.B * a.H * (a.V / (16 * NC));
    hipLaunchKernelGGL((chunkwise_kernel<K, NC, TQ>), dim3(static_cast<unsigned>(blocks)),
                       dim3(64 * (NC + K / 32)), 0, stream, a);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

template <int K, typename TQ>
int launch_kq(const kda_fwd_args& a, hipStream_t stream) {
    if (a.V % 64 == 0) return launch_knq<K, 4, TQ>(a, stream);
    if (a.V % 32 == 0) return launch_knq<K, 2, TQ>(a, stream);
    return launch_knq<K, 1, TQ>(a, stream);
}

template <int K>
int launch_k(const kda_fwd_args& a, hipStream_t stream) {
    switch (a.qkv_dtype) {
        case KDA_DTYPE_F16: return launch_kq<K, _Float16>(a, stream);
        case KDA_DTYPE_BF16: return launch_kq<K, bf16_t>(a, stream);
        case KDA_DTYPE_F32: return launch_kq<K, float>(a, stream);
        default: return KDA_ERR_BAD_DTYPE;
    }
}

}  // namespace

bool chunkwise_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % 16 == 0;
}

int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream) {
    // the pipeline reads gates in fp32 (the wrapper converts other dtypes)
    if (a.g_dtype != KDA_DTYPE_F32 || a.beta_dtype != KDA_DTYPE_F32) return KDA_ERR_BAD_DTYPE;
    // in-chunk offsets are 32-bit byte offsets: 16 token strides + one row must fit
    const int64_t lim = int64_t(1) << 31;
    const int64_t ts[5] = {a.q_stride[1], a.k_stride[1], a.v_stride[1], a.g_stride[1], a.beta_stride[1]};
    for (int64_t st : ts)
        if (st < 0 || (BT + 1) * st * 4 + a.V * 4 >= lim) return KDA_ERR_UNSUPPORTED;
    if ((BT + 1) * a.H * a.V * 4 >= lim) return KDA_ERR_UNSUPPORTED;
    // a chunk's buffer descriptor spans rows_in * token stride bytes, so every
    // token row must be disjoint from the next (stride >= row length)
    if (a.T > 1 && (a.q_stride[1] < a.K || a.k_stride[1] < a.K || a.g_stride[1] < a.K ||
                    a.v_stride[1] < a.V || a.beta_stride[1] < 1))
        return KDA_ERR_UNSUPPORTED;
    switch (a.K) {
        case 32: return launch_k<32>(a, stream);
        case 64: return launch_k<64>(a, stream);
        case 128: return launch_k<128>(a, stream);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
