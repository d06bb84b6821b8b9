// Chunkwise KDA forward for gfx950: fp16 MFMA, fp32 accumulation, fp32 state.
//
// Replaces the body of kda_chunkwise (kimi_linear/kda.py:111-185).  The maths
// is the reference's UT-transform form (paper Eq. 6-9) evaluated per block of
// BT = 16 tokens; the recurrence is chunk-size invariant, so the caller's
// chunk_size only fixes the T % chunk_size == 0 contract.
//
// Per (b, h) and block (rows c, i in [0, 16)), with a_t = exp(g_t):
//   E[r]   = prod_{t<=r} a_t              (= exp(gc_r), per channel)
//   L[c,i] = beta_c <k_c, k_i * prod_{t=i+1..c} a_t>,  i < c
//   A[c,i] = scale <q_c, k_i * prod_{t=i+1..c} a_t>,   i <= c
//   M      = (I + L)^-1 Diag(beta)
//   P      = M (V - (E * K) S)           (= U - W S with U = M V, W = M (E * K))
//   O      = scale (E * Q) S + A P
//   S     <- Diag(E[15]) S + ((E[15]/E) * K)^T P
//
// Decay factoring without pairwise exponentials: every pair i < c of a block
// has a unique highest differing bit b; c has it set, i clear, and both sit in
// the aligned group of 2^(b+1) rows whose upper half starts at ref + 1.  Then
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
// Pipeline, one workgroup per (b, h, 16*NC state columns), in supersteps of
// NB = 4 blocks (64 tokens), each split in two halves by workgroup barriers:
//   NC consumer waves: wave w owns state columns [16w, 16w+16) for all K rows
//     as MFMA accumulators and runs the sequential chain over blocks 0-1 of
//     superstep s in the first half and blocks 2-3 in the second.
//   NB * PW producer waves (PW = 2 for K = 128, else 1): the PW waves of
//     block p build every operand of block NB*(s+1) + p, each over its own
//     channels -- decays, level operands (staged k-major in the slot's own
//     q*E / k*E rows before those receive their final values), partial L
//     and A -- in the first half; in the second the first wave adds the
//     partial sums, writes A and inverts (I + L), the other writes its
//     E-scaled operands.  The next block's loads are issued between levels.
// Operand slots alternate between two sets of NB, so the producers of
// superstep s+1 and the consumers of superstep s never touch the same slot.
// Operands that are not exact in fp16 and carry the state (S, P, M, L and
// V - Z) are split into fp16 hi + lo; the others are single fp16 with fp32
// accumulation.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int BT = 16;          // tokens per block
constexpr int NB = 4;           // blocks per superstep = producer waves
constexpr int NSLOT = 2 * NB;   // operand slots (two supersteps)
constexpr int RP = 24;          // padded row (halfs) of the [16][16] fp16 A-operand matrices
constexpr int LP = 20;          // padded row (floats) of the 16x16 fp32 L
constexpr int kXcds = 8;        // accelerator complex dies on MI355X

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

// Raw buffer loads.  A block's descriptor spans exactly its rows before T;
// the range check covers the whole offset (lane offset + row offset), so
// rows past T read as zero -- the neutral padding (k = q = v = g = beta = 0)
// -- with no clamping or masking.  The row offset is wave-uniform and goes in
// the scalar offset; the lane offset is one register per tensor.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(nbytes), 0x00020000);
}
template <int BYTES> struct BLoad;
template <> struct BLoad<2> {
    static constexpr int W = 1;
    static __device__ __forceinline__ void ld(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b16(r, static_cast<int>(vo), static_cast<int>(so), 0);
    }
};
template <> struct BLoad<4> {
    static constexpr int W = 1;
    static __device__ __forceinline__ void ld(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, static_cast<int>(vo), static_cast<int>(so), 0);
    }
};
template <> struct BLoad<8> {
    static constexpr int W = 2;
    static __device__ __forceinline__ void ld(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(vo), static_cast<int>(so), 0);
        w[0] = x[0];
        w[1] = x[1];
    }
};

// Values are held raw, one load per register set, and converted only where
// they are used.  Left alone, the compiler hoists a conversion (or the
// packing of two fp16 loads into one register) up to the load, which puts a
// wait for the whole prefetch right after it is issued.  An empty volatile
// asm that "modifies" the registers at the point of use keeps every such
// instruction, and the wait, there.
template <int N>
__device__ __forceinline__ void use_here(uint32_t (&r)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i) asm volatile("" : "+v"(r[i]));
}
template <int N, int M>
__device__ __forceinline__ void use_here(uint32_t (&r)[N][M]) {
#pragma unroll
    for (int i = 0; i < N; ++i) use_here(r[i]);
}

// Element type of q, k and v: CH adjacent channels of one token row.
template <typename TQ, int CH>
struct QRow {
    static constexpr int BYTES = CH * static_cast<int>(sizeof(TQ));
    static constexpr int W = BLoad<BYTES>::W;
    // channel j of a raw row
    static __device__ __forceinline__ float val(const uint32_t (&w)[W], int j) {
        if constexpr (sizeof(TQ) == 4) {
            return __uint_as_float(w[j]);
        } else {
            const uint32_t hbits = (w[0] >> (16 * j)) & 0xffffu;
            if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
                return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(hbits)));
            } else {
                return __uint_as_float(hbits << 16);
            }
        }
    }
    // channel j of rows (r0, r1) as an fp16 pair (exact repacking for fp16)
    static __device__ __forceinline__ h2 pair(const uint32_t (&w0)[W], const uint32_t (&w1)[W], int j) {
        if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
            const uint32_t lo = (w0[0] >> (16 * j)) & 0xffffu;
            const uint32_t hi = (w1[0] >> (16 * j)) << 16;
            return __builtin_bit_cast(h2, lo | hi);
        } else {
            return h2{static_cast<_Float16>(val(w0, j)), static_cast<_Float16>(val(w1, j))};
        }
    }
};

// Sixteen fp32 values rounded to fp16, as two h8 (rows 0-7, 8-15).
__device__ __forceinline__ void to_h16(const float (&x)[BT], h8& lo, h8& hi) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo[i] = static_cast<_Float16>(x[i]);
        hi[i] = static_cast<_Float16>(x[8 + i]);
    }
}

// Within one wave, LDS serves requests in issue order, so a wave reads back
// what its own lanes wrote (and reads complete before later overwrites)
// without any barrier; the compiler keeps the order of the possibly
// aliasing LDS accesses.  The per-producer staging areas rely on this.

// Operands of one block, as the consumers read them.  QET and KET are read
// through LDS transpose loads, KHT as A-operand rows of channels; all three
// are k-major ([K][16]: the 16 rows of a channel in one 32-byte line, halves
// swizzled by channel bit 3, see kswz).
template <int K>
struct __align__(16) Slot {
    _Float16 QET[K][BT];                   // q * E
    _Float16 KET[K][BT];                   // k * E
    _Float16 KHT[K][BT];                   // k * E15 / E
    _Float16 AM[BT][RP];                   // scale * A
    _Float16 MH[BT][RP];                   // M hi
    _Float16 ML[BT][RP];                   // M lo
    float elast[K];                        // E[15]
};

// Producer waves per block: for K = 128 two, each with half of the channels
// (one channel per lane); one otherwise.
template <int K>
constexpr int kPW = K == 128 ? 2 : 1;

template <int K>
struct __align__(16) Smem {
    Slot<K> slot[NSLOT];
    // per block: the second producer's partial L and A (lane-major), then
    // the first producer's L for its transpose
    float XCH[NB][2][64][4];
};

__device__ __forceinline__ h4 frag16(const _Float16* base, int stride, int row, int lg) {
    return *reinterpret_cast<const h4*>(base + row * stride + 4 * lg);
}

typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;

// k-major [K][16] fp16 matrices (the 16 rows of a channel in one 32-byte
// line) swap the two 16-byte halves of the line on channels with bit 3 set,
// so the 16-byte writes of 16 consecutive channels (one per lane) cover all
// 64 banks once.  Half h of channel c sits at 8 * (h ^ kswz(c)).
__device__ __forceinline__ int kswz(int c) { return (c >> 3) & 1; }

// Stores the 16 rows of channel c (rows 0-7, 8-15) into a k-major matrix.
__device__ __forceinline__ void store_kmajor(_Float16* xt, int c, const h8& r0_7, const h8& r8_15) {
    const int s = kswz(c) * 8;
    *reinterpret_cast<h8*>(xt + c * BT + s) = r0_7;
    *reinterpret_cast<h8*>(xt + c * BT + (8 - s)) = r8_15;
}

// MFMA row fragment from a k-major [K][16] fp16 matrix X^T through the LDS
// transpose read (ds_read_b64_tr_b16): within each 16-lane group, lane 4j+q
// supplies the four rows 4q..4q+3 of channel kbase+j, and lane i receives
// X[i][kbase + 0..3] -- the A-operand fragment of row i, which is also the
// B-operand fragment of column i of X^T.  kbase is 4lg modulo 16, so the
// channels kbase + j (j < 4) share bit 3 = lg >> 1 and the swizzled column of
// rows 4q..4q+3 is 4 (q ^ 2 (lg >> 1)), a per-lane constant.
__device__ __forceinline__ h4 frag16_tr(const _Float16* xt, int kbase, int ln, int lg) {
    const int q = (ln & 3) ^ ((lg >> 1) * 2);
    const _Float16* p = xt + (kbase + (ln >> 2)) * BT + 4 * q;
    return __builtin_bit_cast(h4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p)));
}

// 16x16x32 fragment: slots 0-3 hold k = 32u + 4lg + j, slots 4-7 hold
// k = 32u + 16 + 4lg + j.  A and B fragments use the same assignment, so the
// product is the full 32-wide dot product whatever slot order the unit uses;
// it also matches the two state tiles 2u, 2u+1 held by a consumer lane group.
__device__ __forceinline__ h8 frag32_tr(const _Float16* xt, int lg, int ln, int u) {
    const h4 lo = frag16_tr(xt, 32 * u + 4 * lg, ln, lg);
    const h4 hi = frag16_tr(xt, 32 * u + 16 + 4 * lg, ln, lg);
    return h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Four fp32 values as fp16 hi + lo, x ~= hi + lo to ~2^-21 relative: hi is x
// truncated to fp16's 11 significant bits (exact in fp16 and in fp32), so
// lo = x - hi is exact in fp32 and is rounded once.  Three VALU operations
// per value, no conversion back from fp16.
__device__ __forceinline__ void split4(const f4& x, h4& hi, h4& lo) {
    float t[4], r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        t[i] = __uint_as_float(__float_as_uint(x[i]) & 0xffffe000u);
        r[i] = x[i] - t[i];
    }
    hi = h4{static_cast<_Float16>(t[0]), static_cast<_Float16>(t[1]), static_cast<_Float16>(t[2]),
            static_cast<_Float16>(t[3])};
    lo = h4{static_cast<_Float16>(r[0]), static_cast<_Float16>(r[1]), static_cast<_Float16>(r[2]),
            static_cast<_Float16>(r[3])};
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
    static constexpr int KT = K / 16;                   // 16-row state tiles
    static constexpr int KU = K / 32;                   // 32-wide k blocks
    static constexpr int PW = kPW<K>;                   // producer waves per block
    static constexpr int KW = K / PW;                   // channels per producer wave
    static constexpr int KUW = KW / 32;                 // 32-wide k blocks per producer wave
    static constexpr int CH = 1;                        // channels per producer lane
    static constexpr int VT = 16 * NC;
    using QR = QRow<TQ, CH>;                            // producer rows of q / k
    using VR = QRow<TQ, 1>;                             // consumer elements of v
    static constexpr int QW = QR::W;

    // One block's raw inputs for a producer lane: channels chan(0..CH-1),
    // rows 0..15, and beta of rows 4lg..4lg+3.
    struct Raw {
        uint32_t q[BT][QW], k[BT][QW];
        uint32_t g[BT][CH];
        uint32_t beta[4];
    };
    // The same block, converted: decays, fp16 q and k (rows 0-7 / 8-15), beta.
    struct Work {
        float al[CH][BT];
        h8 qh[CH][2], kh[CH][2];
        float beta[4];
    };

    const kda_fwd_args& a;
    Smem<K>& sm;
    int64_t b, h, T;
    int nch;
    float scale;
    int lane, ln, lg;
    int hh;                                  // producer: channel part (0 .. PW-1)
    uint32_t rs_q, rs_k, rs_g, rs_v, rs_b;   // token-row strides in bytes
    uint32_t vo_q, vo_k, vo_g, vo_v, vo_b;   // lane byte offsets (v, beta: from row 4lg)

    __device__ Kern(const kda_fwd_args& args, Smem<K>& s) : a(args), sm(s) {}

    // Channel c of this producer lane (lanes 32-63 repeat lanes 0-31 when K = 32).
    __device__ int chan(int c) const { return hh * KW + CH * (KW < 64 ? (lane % KW) : lane) + c; }

    // Rows of block `blk` that lie before T (1..BT).
    __device__ int rows_in(int blk) const {
        const int64_t left = T - static_cast<int64_t>(blk) * BT;
        return left < BT ? static_cast<int>(left) : BT;
    }

    // Descriptor over the rows of one block of a [B, T, H, D] view (elements
    // of es bytes, token stride rs bytes), based at (b, 16 blk, h, 0).
    __device__ __amdgpu_buffer_rsrc_t block_rsrc(const void* p, const int64_t (&st)[3], int es, uint32_t rs,
                                                 int blk) const {
        const int64_t e = b * st[0] + static_cast<int64_t>(blk) * BT * st[1] + h * st[2];
        return make_rsrc(static_cast<const char*>(p) + e * es, static_cast<uint32_t>(rows_in(blk)) * rs);
    }

    // ------------------------------------------------------------ producers
    // Loads of rows [R0, R1) of one block (and beta with the last rows).
    // The loads of the next block are issued in four parts between the
    // levels of the current one, so they never queue up in one burst.
    template <int R0, int R1>
    __device__ void load_rows(Raw& r, int blk) const {
        const auto rq = block_rsrc(a.q, a.q_stride, sizeof(TQ), rs_q, blk);
        const auto rk = block_rsrc(a.k, a.k_stride, sizeof(TQ), rs_k, blk);
        const auto rg = block_rsrc(a.g, a.g_stride, 4, rs_g, blk);
#pragma unroll
        for (int i = R0; i < R1; ++i) {
            BLoad<4 * CH>::ld(r.g[i], rg, vo_g, i * rs_g);
            BLoad<QR::BYTES>::ld(r.q[i], rq, vo_q, i * rs_q);
            BLoad<QR::BYTES>::ld(r.k[i], rk, vo_k, i * rs_k);
        }
        if constexpr (R1 == BT) {
            const auto rb = block_rsrc(a.beta, a.beta_stride, 4, rs_b, blk);
#pragma unroll
            for (int j = 0; j < 4; ++j) BLoad<4>::ld(&r.beta[j], rb, vo_b, j * rs_b);
        }
    }
    __device__ void load_raw(Raw& r, int blk) const { load_rows<0, BT>(r, blk); }

    __device__ void unpack(Raw& r, Work& w) const {
        use_here(r.q);
        use_here(r.k);
        use_here(r.g);
        use_here(r.beta);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
#pragma unroll
            for (int i = 0; i < BT; ++i) w.al[c][i] = fast_exp(__uint_as_float(r.g[i][c]));
#pragma unroll
            for (int p = 0; p < BT / 2; ++p) {
                const h2 qp = QR::pair(r.q[2 * p], r.q[2 * p + 1], c);
                const h2 kp = QR::pair(r.k[2 * p], r.k[2 * p + 1], c);
                w.qh[c][p / 4][2 * (p % 4)] = qp[0];
                w.qh[c][p / 4][2 * (p % 4) + 1] = qp[1];
                w.kh[c][p / 4][2 * (p % 4)] = kp[0];
                w.kh[c][p / 4][2 * (p % 4) + 1] = kp[1];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) w.beta[j] = __uint_as_float(r.beta[j]);
    }

    // Level factors F_b(r), r = 0..15, of one channel: in each aligned group of
    // 2^(b+1) rows, upper-half rows c get prod_{t=ref+1..c} a_t and lower-half
    // rows i get prod_{t=i+1..ref} a_t, ref = the group's last lower row.
    template <int B>
    static __device__ __forceinline__ void level_factors(const float (&al)[BT], float (&f)[BT]) {
        constexpr int S = 2 << B, HALF = 1 << B;
#pragma unroll
        for (int st = 0; st < BT; st += S) {
            float run = al[st + HALF];
            f[st + HALF] = run;
#pragma unroll
            for (int c = st + HALF + 1; c < st + S; ++c) {
                run *= al[c];
                f[c] = run;
            }
            f[st + HALF - 1] = 1.f;
            run = al[st + HALF - 1];
#pragma unroll
            for (int i = st + HALF - 2; i >= st; --i) {
                f[i] = run;
                run *= al[i];
            }
        }
    }

    // Operand level LEV of a block (this wave's channels): X_b = k * F_b and
    // Y_b = q * F_b, stored k-major into a staging pair (xs, ys) whose row 0
    // is this wave's first channel.
    template <int LEV>
    __device__ void stage(const Work& w, _Float16* xs, _Float16* ys) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            h8 x0 = w.kh[c][0], x1 = w.kh[c][1], y0 = w.qh[c][0], y1 = w.qh[c][1];
            if constexpr (LEV > 0) {
                float f[BT];
                level_factors<LEV - 1>(w.al[c], f);
                h8 f0, f1;
                to_h16(f, f0, f1);
                x0 *= f0;
                x1 *= f1;
                y0 *= f0;
                y1 *= f1;
            }
            const int lc = chan(c) - hh * KW;
            store_kmajor(xs, lc, x0, x1);
            store_kmajor(ys, lc, y0, y1);
        }
    }

    // Level LEV's products from its staging pair: L_b = X_b X_b^T and
    // A_b = Y_b X_b^T over this wave's channels, keeping the level's pairs
    // (accumulator layout: row 4lg + j, column ln).
    template <int LEV>
    __device__ void product(const Work& w, const _Float16* xs, const _Float16* ys, f4& Lacc, f4& Aacc) const {
        f4 accL = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KUW; ++u) {
            const h8 xf = frag32_tr(xs, lg, ln, u);
            const h8 yf = frag32_tr(ys, lg, ln, u);
            if constexpr (LEV > 0) accL = mfma16x16x32(xf, xf, accL);
            accA = mfma16x16x32(yf, xf, accA);
        }
        const int i = ln;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * lg + j;
            if constexpr (LEV == 0) {
                if (i == c) Aacc[j] = accA[j];
            } else {
                constexpr int bb = LEV - 1;
                const bool pair = ((c >> (bb + 1)) == (i >> (bb + 1))) && ((c >> bb) & 1) && !((i >> bb) & 1);
                if (pair) {
                    Lacc[j] = w.beta[j] * accL[j];
                    Aacc[j] = accA[j];
                }
            }
        }
    }

    // M = (I + L)^-1 Diag(beta) of one block (producer p), stored as hi/lo
    // A-operand fragments.
    __device__ void solve(const f4& Lc, const float (&beta)[4], Slot<K>& sl, int p) const {
        float* lt = &sm.XCH[p][0][0][0];
#pragma unroll
        for (int j = 0; j < 4; ++j) lt[(4 * lg + j) * LP + ln] = Lc[j];
        f4 Lt;                                           // acc(L^T)
        {
            const float4 r = *reinterpret_cast<const float4*>(lt + ln * LP + 4 * lg);
            Lt[0] = r.x; Lt[1] = r.y; Lt[2] = r.z; Lt[3] = r.w;
        }
        const Split4 lc(Lc), ltt(Lt);
        const Split4 l2(mm3(ltt, lc)), l2t(mm3(lc, ltt));  // L^2, (L^2)^T
        const Split4 l4(mm3(l2t, l2)), l4t(mm3(l2, l2t));
        const Split4 l8(mm3(l4t, l4));
        f4 Q;                                            // acc(I - L^T)
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] = (4 * lg + j == ln ? 1.f : 0.f) - Lt[j];
        Q += mm3(l2, Split4(Q));
        Q += mm3(l4, Split4(Q));
        Q += mm3(l8, Split4(Q));                         // acc(Minv^T) = A-layout of Minv
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] *= beta[j];
        h4 mh, ml;
        split4(Q, mh, ml);
        *reinterpret_cast<h4*>(&sl.MH[ln][4 * lg]) = mh;
        *reinterpret_cast<h4*>(&sl.ML[ln][4 * lg]) = ml;
    }

    // q * E, k * E, k * E15 / E and E15 of one block.
    __device__ void escaled(const Work& w, Slot<K>& sl) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float (&al)[BT] = w.al[c];
            float pre[BT], suf[BT];
            pre[0] = al[0];
#pragma unroll
            for (int i = 1; i < BT; ++i) pre[i] = pre[i - 1] * al[i];
            suf[BT - 1] = 1.f;
#pragma unroll
            for (int i = BT - 2; i >= 0; --i) suf[i] = suf[i + 1] * al[i + 1];
            h8 e0, e1, s0, s1;
            to_h16(pre, e0, e1);
            to_h16(suf, s0, s1);
            const int ch = chan(c);
            store_kmajor(&sl.QET[0][0], ch, w.qh[c][0] * e0, w.qh[c][1] * e1);
            store_kmajor(&sl.KET[0][0], ch, w.kh[c][0] * e0, w.kh[c][1] * e1);
            store_kmajor(&sl.KHT[0][0], ch, w.kh[c][0] * s0, w.kh[c][1] * s1);
            sl.elast[ch] = pre[BT - 1];
        }
    }

    // First half of a superstep: the level products of this wave's channels
    // (partial L and A over them), with the next block's loads issued in
    // between; the first part also writes its E-scaled operands, the second
    // part hands its partial sums to the first.
    __device__ void phase1(Raw& raw, Work& w, f4& Lacc, f4& Aacc, int p, Slot<K>& sl, int next) const {
        unpack(raw, w);
        Lacc = f4{0.f, 0.f, 0.f, 0.f};
        Aacc = f4{0.f, 0.f, 0.f, 0.f};
        // level operands are staged in this part's rows of the slot's QET /
        // KET, which get their final values only after the last level
        _Float16* xs = &sl.QET[hh * KW][0];
        _Float16* ys = &sl.KET[hh * KW][0];
        stage<0>(w, xs, ys);
        product<0>(w, xs, ys, Lacc, Aacc);
        load_rows<0, 4>(raw, next);
        stage<1>(w, xs, ys);
        product<1>(w, xs, ys, Lacc, Aacc);
        load_rows<4, 8>(raw, next);
        stage<2>(w, xs, ys);
        product<2>(w, xs, ys, Lacc, Aacc);
        load_rows<8, 12>(raw, next);
        stage<3>(w, xs, ys);
        product<3>(w, xs, ys, Lacc, Aacc);
        load_rows<12, BT>(raw, next);
        stage<4>(w, xs, ys);
        product<4>(w, xs, ys, Lacc, Aacc);
        if (hh == 0) {
            escaled(w, sl);
        } else {
            *reinterpret_cast<f4*>(&sm.XCH[p][0][lane][0]) = Lacc;
            *reinterpret_cast<f4*>(&sm.XCH[p][1][lane][0]) = Aacc;
        }
    }

    // Second half: the first part completes L and A, writes A and inverts
    // (I + L); the second part writes its E-scaled operands.
    __device__ void phase2(const Work& w, const f4& Lacc, const f4& Aacc, int p, Slot<K>& sl) const {
        if (hh != 0) {
            escaled(w, sl);
            return;
        }
        f4 L = Lacc, A = Aacc;
        if constexpr (PW == 2) {
            L += *reinterpret_cast<const f4*>(&sm.XCH[p][0][lane][0]);
            A += *reinterpret_cast<const f4*>(&sm.XCH[p][1][lane][0]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sl.AM[4 * lg + j][ln] = static_cast<_Float16>(A[j] * scale);
        solve(L, w.beta, sl, p);
    }

    // ------------------------------------------------------------ consumers
    __device__ void v_load(uint32_t (&vr)[4], int blk) const {
        const auto rv = block_rsrc(a.v, a.v_stride, sizeof(TQ), rs_v, blk);
#pragma unroll
        for (int j = 0; j < 4; ++j) BLoad<sizeof(TQ)>::ld(&vr[j], rv, vo_v, j * rs_v);
    }

    // One block of the chain for this wave's 16 state columns.
    __device__ void consume(const Slot<K>& sl, int blk, uint32_t (&vraw)[4], int next, f4 (&S)[KT],
                            int64_t col0, uint32_t ocol) const {
        use_here(vraw);
        float vr[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t w1[1] = {vraw[j]};
            vr[j] = VR::val(w1, 0);
        }
        v_load(vraw, next);
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
        f4 Z = {0.f, 0.f, 0.f, 0.f}, O = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const h8 kf = frag32_tr(&sl.KET[0][0], lg, ln, u);
            Z = mfma16x16x32(kf, shi[u], Z);
            Z = mfma16x16x32(kf, slo[u], Z);
            const h8 qf = frag32_tr(&sl.QET[0][0], lg, ln, u);
            O = mfma16x16x32(qf, shi[u], O);
            O = mfma16x16x32(qf, slo[u], O);
        }
        // P = U - W S = M (V - Z)
        f4 R;
#pragma unroll
        for (int j = 0; j < 4; ++j) R[j] = vr[j] - Z[j];
        const Split4 r(R);
        const h4 mh = frag16(&sl.MH[0][0], RP, ln, lg);
        const h4 ml = frag16(&sl.ML[0][0], RP, ln, lg);
        f4 P = {0.f, 0.f, 0.f, 0.f};
        P = mfma16x16x16(mh, r.hi, P);
        P = mfma16x16x16(mh, r.lo, P);
        P = mfma16x16x16(ml, r.hi, P);
        // O = scale (q * E) S + A P
#pragma unroll
        for (int j = 0; j < 4; ++j) O[j] *= scale;
        h4 ph, pl;
        split4(P, ph, pl);
        const h4 af = frag16(&sl.AM[0][0], RP, ln, lg);
        O = mfma16x16x16(af, ph, O);
        O = mfma16x16x16(af, pl, O);
        // o[b, t, h, col]: wave-uniform block base + 32-bit lane offset
        TQ* o = static_cast<TQ*>(a.o) + ((b * T + static_cast<int64_t>(blk) * BT) * a.H + h) * a.V + col0;
        const uint32_t orow = static_cast<uint32_t>(a.H * a.V);
        const int nrow = rows_in(blk);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * lg + j < nrow) Elem<TQ>::st(o + (4 * lg + j) * orow + ocol, O[j]);
        // S <- E15 S + Khat^T P
        const int kg = lg ^ (((ln >> 3) & 1) * 2);       // KHT halves swapped on channel bit 3
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const float4 e = *reinterpret_cast<const float4*>(&sl.elast[16 * t + 4 * lg]);
            S[t][0] *= e.x; S[t][1] *= e.y; S[t][2] *= e.z; S[t][3] *= e.w;
            const h4 kf = frag16(&sl.KHT[16 * t][0], BT, ln, kg);
            S[t] = mfma16x16x16(kf, ph, S[t]);
            S[t] = mfma16x16x16(kf, pl, S[t]);
        }
    }
};

// Supersteps of NB blocks.  Before superstep s the producers have filled
// slot set s % 2 with the blocks of superstep s; during it they fill the
// other set with superstep s + 1 while the consumers run superstep s; one
// workgroup barrier ends each superstep.  Every wave executes the same
// barriers; every prefetch is issued unconditionally (block index clamped).
template <int K, int NC, typename TQ>
__global__ __launch_bounds__(64 * (NC + NB * kPW<K>)) void chunkwise_kernel(const kda_fwd_args a) {
    using KN = Kern<K, NC, TQ>;
    constexpr int KT = KN::KT, VT = KN::VT;
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
    // wave index as a scalar: block indices and buffer descriptors derived
    // from it stay in SGPRs (no per-lane descriptor loops around the loads)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kn.lane = threadIdx.x & 63;
    kn.ln = kn.lane & 15;
    kn.lg = kn.lane >> 4;
    const int nch = kn.nch;
    const int nss = (nch + NB - 1) / NB;
    const int last = nch - 1;

    const bool consumer = wave < NC;
    // producer wave q = wave - NC builds block q / PW, channel part q % PW
    const int pq = consumer ? 0 : wave - NC;
    kn.hh = pq % KN::PW;
    // consumer state: S[t][j] = S[16t + 4lg + j][col], col = col0 + ocol
    const int64_t col0 = static_cast<int64_t>(vt) * VT;
    const uint32_t ocol = static_cast<uint32_t>(16 * (consumer ? wave : 0) + kn.ln);
    const int64_t col = col0 + ocol;
    const int64_t sbase = (kn.b * H + kn.h) * static_cast<int64_t>(K) * V;
    {
        const uint32_t eq = static_cast<uint32_t>(sizeof(TQ));
        kn.rs_q = static_cast<uint32_t>(a.q_stride[1]) * eq;
        kn.rs_k = static_cast<uint32_t>(a.k_stride[1]) * eq;
        kn.rs_v = static_cast<uint32_t>(a.v_stride[1]) * eq;
        kn.rs_g = static_cast<uint32_t>(a.g_stride[1]) * 4u;
        kn.rs_b = static_cast<uint32_t>(a.beta_stride[1]) * 4u;
        const uint32_t c0 = static_cast<uint32_t>(kn.chan(0));
        kn.vo_q = c0 * eq;
        kn.vo_k = c0 * eq;
        kn.vo_g = c0 * 4u;
        kn.vo_b = static_cast<uint32_t>(4 * kn.lg) * kn.rs_b;
        kn.vo_v = static_cast<uint32_t>(4 * kn.lg) * kn.rs_v + static_cast<uint32_t>(col) * eq;
    }

    if (consumer) {
        f4 S[KT];
        load_state<KT>(S, a.state_in, a.state_in_dtype, sbase + (4 * kn.lg) * V + col, V);
        uint32_t vr[NB][4];
#pragma unroll
        for (int j = 0; j < NB; ++j) kn.v_load(vr[j], min(j, last));
        for (int s = -1; s < nss; ++s) {
            const Slot<K>* set = &sm.slot[(s & 1) * NB];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
#pragma unroll
                for (int j = half * (NB / 2); j < (half + 1) * (NB / 2); ++j) {
                    const int blk = NB * s + j;
                    if (s >= 0 && blk < nch) kn.consume(set[j], blk, vr[j], min(blk + NB, last), S, col0, ocol);
                }
                __syncthreads();
            }
        }
        store_state<KT>(S, a.state_out, a.state_out_dtype, sbase + (4 * kn.lg) * V + col, V);
    } else {
        const int p = pq / KN::PW;
        typename KN::Raw raw;
        typename KN::Work w;
        f4 Lacc, Aacc;
        kn.load_raw(raw, min(p, last));
        for (int s = -1; s < nss; ++s) {
            const int blk = NB * (s + 1) + p;
            Slot<K>& sl = sm.slot[((s + 1) & 1) * NB + p];
            if (blk < nch) kn.phase1(raw, w, Lacc, Aacc, p, sl, min(blk + NB, last));
            __syncthreads();
            if (blk < nch) kn.phase2(w, Lacc, Aacc, p, sl);
            __syncthreads();
        }
    }
}

template <int K, int NC, typename TQ>
int launch_knq(const kda_fwd_args& a, hipStream_t stream) {
    const int64_t blocks = a.B * a.H * (a.V / (16 * NC));
    hipLaunchKernelGGL((chunkwise_kernel<K, NC, TQ>), dim3(static_cast<unsigned>(blocks)),
                       dim3(64 * (NC + NB * kPW<K>)), 0, stream, a);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

// Columns per workgroup: the widest tile (64, 32 or 16 columns) that still
// gives at least one workgroup per CU; 16 when none does (few chains).
template <int K, typename TQ>
int launch_kq(const kda_fwd_args& a, hipStream_t stream) {
    constexpr int64_t kCus = 256;
    const int64_t heads = a.B * a.H;
    if (a.V % 64 == 0 && heads * (a.V / 64) >= kCus) return launch_knq<K, 4, TQ>(a, stream);
    if (a.V % 32 == 0 && heads * (a.V / 32) >= kCus) return launch_knq<K, 2, TQ>(a, stream);
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
