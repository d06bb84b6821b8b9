// Chunkwise KDA forward for gfx950: fp16 MFMA, fp32 accumulation, fp32 state.
//
// Replaces the body of kda_chunkwise (kimi_linear/kda.py:111-185).  The maths
// is the reference's UT-transform form (paper Eq. 6-9) with the state carried
// across chunks of CT = 32 tokens, each made of two blocks of BT = 16 tokens.
// The recurrence is chunk-size invariant, so the caller's chunk_size only
// fixes the T % chunk_size == 0 contract.
//
// Per (b, h) and chunk, with a_t = exp(g_t) per channel, rows c, i of one
// chunk, E[r] = prod_{t <= r} a_t from the chunk start and F = E[31] / E:
//   G[c,i] = <k_c, k_i * prod_{t=i+1..c} a_t>,          i < c
//   A[c,i] = scale <q_c, k_i * prod_{t=i+1..c} a_t>,    i <= c
//   P      = (I + Diag(beta) G)^-1 Diag(beta) (V - (E * K) S)
//   O      = scale (E * Q) S + A P
//   S     <- Diag(E[31]) S + (F * K)^T P
// With blocks 0 and 1 of the chunk, M_bb = (I + Diag(beta_b) G_bb)^-1
// Diag(beta_b) and R_b = V_b - (E * K)_b S, the solve is two block steps:
//   P_0 = M_00 R_0,   P_1 = M_11 (R_1 - G_10 P_0).
//
// Decay factoring without pairwise exponentials.  Diagonal blocks: every
// pair i < c of a block has a unique highest differing bit b; c has it set,
// i clear, and both sit in the aligned group of 2^(b+1) rows whose upper half
// starts at ref + 1.  Then
//   prod_{t=i+1..c} a_t = (prod_{t=ref+1..c} a_t) * (prod_{t=i+1..ref} a_t),
// both factors <= 1, so per level b one [16 x K] operand X_b (row r = k_r
// times its factor) gives G_b = X_b X_b^T as a plain MFMA product, masked to
// level b's pairs.  The diagonal A[c, c] comes from the level whose
// reference row c is (both of its factors are 1); row 15, no level's
// reference row, is one dot product of its own.  Off-diagonal
// block G_10, A_10: the reference row is the last row of block 0, so the
// factors are the block-local decay of row c of block 1 from its block start
// and of row i of block 0 to its block end.  A factor only underflows when
// the true decay is smaller still.
//
// (I + L)^-1 = (I - L)(I + L^2)(I + L^4)(I + L^8) for the nilpotent 16x16
// L = Diag(beta) G_bb: four products and three squarings on MFMA (fp16 hi/lo
// split operands), entirely in registers.  An MFMA accumulator holds
// X[4g+j][n] in lane n+16g, slot j -- the B-operand layout of X and the
// A-operand layout of X^T -- so a chain that keeps X and X^T side by side
// needs no data movement.
//
// Pipeline, one workgroup per (b, h, 16*NC state columns), in supersteps of
// NB = 4 blocks (two chunks), each split in two halves by workgroup barriers:
//   NC consumer waves: wave w owns state columns [16w, 16w+16) for all K rows
//     as MFMA accumulators and runs the chain over chunk 0 of superstep s in
//     the first half and chunk 1 in the second.
//   NB producer waves, one per block: wave p builds every operand of block
//     NB*(s+1) + p.  Lane l holds K/32 adjacent channels of the block's rows
//     8 (l / 32) .. +7, which one 8-byte (fp16) load per row brings in for
//     all K channels of two rows.  First half: decays, the level operands
//     and their products, the operands that need no other block's decay, the
//     block-local operands of the chunk's off-diagonal products, the block
//     decay E[15].  Second half, once the other block's decay is known: the
//     chunk-relative operands, G_10 and A_10 (block 1's wave), A and the
//     inverse of (I + L).  The next block's loads are issued in the first
//     half and land during the rest of the superstep.
// Operand slots alternate between two sets, so the producers of superstep
// s+1 and the consumers of superstep s never touch the same slot.
//
// Operand layouts in LDS.  Row operands (q * E, k * E, the level operands,
// the block-local k * F of block 0) are row-major [16 tokens][K + 8 pad],
// channels permuted by chan_pos so that the eight channels one MFMA lane
// needs (the ones paired with its state rows) are 16 contiguous bytes: a
// producer lane writes a row's channels with one 8-byte store, an MFMA lane
// reads its fragment with one 16-byte load, both free of bank conflicts.
// k * F, which the state update reads by channel, is k-major: one 64-byte
// line per channel holding the chunk's 32 tokens in the order of the
// consumer's P fragments, its 16-byte pieces rotated by channel bits 2-3.
//
// Operands that are not exact in fp16 and carry the state (S, P, M, G_10
// and V - Z) are split into fp16 hi + lo; the others are single fp16 with
// fp32 accumulation.
#include "kda_common.h"
#include "kda_launch.h"

namespace kda {

namespace {

constexpr int BT = 16;          // tokens per block
constexpr int HR = 8;           // rows per producer lane (half a block)
constexpr int CB = 2;           // blocks per chunk (the state advances per chunk)
constexpr int NB = 4;           // blocks per superstep = producer waves
constexpr int NCH = NB / CB;    // chunks per superstep
constexpr int RP = 24;          // padded row (halfs) of the [16][16] fp16 A-operand matrices
constexpr int LP = 20;          // padded row (floats) of the 16x16 fp32 L
constexpr int kXcds = 8;        // accelerator complex dies on MI355X

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

// Raw buffer loads.  A block's descriptor spans exactly its rows before T
// (none for a block past T); the range check covers the whole offset (lane
// offset + row offset), so rows past T read as zero -- the neutral padding
// (k = q = v = g = beta = 0) -- with no clamping or masking.  The row offset
// is wave-uniform and goes in the scalar offset; the lane offset is one
// register per tensor.
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
        const u2 x = __builtin_bit_cast(u2, __builtin_amdgcn_raw_buffer_load_b64(r, static_cast<int>(vo),
                                                                                 static_cast<int>(so), 0));
        w[0] = x[0];
        w[1] = x[1];
    }
};
template <> struct BLoad<16> {
    static constexpr int W = 4;
    static __device__ __forceinline__ void ld(uint32_t* w, __amdgpu_buffer_rsrc_t r, uint32_t vo, uint32_t so) {
        const u4 x = __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(vo),
                                                                                  static_cast<int>(so), 0));
        w[0] = x[0];
        w[1] = x[1];
        w[2] = x[2];
        w[3] = x[3];
    }
};

// Values are held raw, one load per register set, and converted only where
// they are used.  Left alone, the compiler hoists a conversion up to the
// load, which puts a wait for the whole prefetch right after it is issued.
// An empty volatile asm that "modifies" the registers at the point of use
// keeps every such instruction, and the wait, there.
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

// Element j of a raw row of TQ values, as fp16 (exact for fp16 inputs).
template <typename TQ, int W>
__device__ __forceinline__ _Float16 raw_h(const uint32_t (&w)[W], int j) {
    if constexpr (sizeof(TQ) == 4) {
        return static_cast<_Float16>(__uint_as_float(w[j]));
    } else {
        const uint16_t bits = static_cast<uint16_t>(w[j / 2] >> (16 * (j % 2)));
        if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
            return __builtin_bit_cast(_Float16, bits);
        } else {
            return static_cast<_Float16>(__uint_as_float(static_cast<uint32_t>(bits) << 16));
        }
    }
}
// One value of type TQ held raw in the low bits of a word, as fp32.
template <typename TQ>
__device__ __forceinline__ float raw_f(uint32_t w) {
    if constexpr (sizeof(TQ) == 4) {
        return __uint_as_float(w);
    } else if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
        return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xffffu)));
    } else {
        return __uint_as_float(w << 16);
    }
}

__device__ __forceinline__ h8 cat(const h4& a, const h4& b) {
    return h8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Position of channel c inside a row-major operand row.  With c = 32u + 16hi
// + 4g + j, the consumer lane of group g pairs channels 32u + 4g + j and
// 32u + 16 + 4g + j with its state rows; they sit at 32u + 8g + (0..7).
__device__ __forceinline__ int chan_pos(int c) {
    return (c & ~31) | ((c & 12) << 1) | ((c & 16) >> 2) | (c & 3);
}
// 16-byte piece rotation of the k-major k * F lines (channel bits 2-3): the
// 16 channel lines one consumer instruction reads land on 16 distinct bank
// groups.
__device__ __forceinline__ int kh_swz(int c) { return (c >> 2) & 3; }

// Operands of one chunk, as the consumers read them.
template <int K>
struct __align__(16) ChunkOps {
    static constexpr int KR = K + 8;
    _Float16 QE[CB][BT][KR];               // q * E (decay from the chunk start), row-major
    _Float16 KE[CB][BT][KR];               // k * E
    _Float16 KH[K][2 * BT];                // k * F (decay to the chunk end), k-major lines
    _Float16 AM[CB][BT][RP];               // scale * A, diagonal blocks
    _Float16 MH[CB][BT][RP];               // M hi
    _Float16 ML[CB][BT][RP];               // M lo
    _Float16 A10[BT][RP];                  // scale * A, rows of block 1, columns of block 0
    _Float16 GH[BT][RP];                   // -G_10 hi
    _Float16 GL[BT][RP];                   // -G_10 lo
    float echunk[K];                       // decay over the chunk, E[31]
};
// Producer-only exchange of one chunk within a superstep: written in the
// first half, read in the second.
template <int K>
struct __align__(16) Stage {
    _Float16 KH0[BT][K + 8];               // block 0: k * (decay to the block end), row-major
    float e15[CB][K];                      // per block: decay over the block
};
template <int K>
struct __align__(16) Smem {
    ChunkOps<K> set[2][NCH];
    Stage<K> st[NCH];
    float LT[NB][BT][LP];                  // per block: the transposition of L in the solve
};

__device__ __forceinline__ h4 frag16(const _Float16* base, int stride, int row, int lg) {
    return *reinterpret_cast<const h4*>(base + row * stride + 4 * lg);
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

// c + a b with both operands split: (hi + lo)(hi + lo) as two K = 32
// products, [a_hi | a_lo] x [b_hi ; b_hi] + [a_hi | a_lo] x [b_lo ; b_lo]
// (the lo*lo term is below the rounding of the rest and costs nothing).
// cat(a0, a1) x cat(b0, b1) is a0 b0 + a1 b1 for any two pairs of 16x16x16
// fragments: A and B map lane group g, slot s to the same k.
__device__ __forceinline__ f4 mm4(const h4& ahi, const h4& alo, const h4& bhi, const h4& blo, f4 c) {
    const h8 a = cat(ahi, alo);
    c = mfma16x16x32(a, cat(bhi, bhi), c);
    return mfma16x16x32(a, cat(blo, blo), c);
}
__device__ __forceinline__ f4 mm4(const Split4& a, const Split4& b, f4 c = f4{0.f, 0.f, 0.f, 0.f}) {
    return mm4(a.hi, a.lo, b.hi, b.lo, c);
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

// Level whose product supplies entry (row c, column i) of a diagonal block:
// below the diagonal 1 + the highest differing bit; on it the level whose
// reference row c is (1 + the number of trailing ones of c: rows 0, 2, ..
// from level 1, rows 1, 5, .. from level 2, 3 and 11 from level 3, 7 from
// level 4, where both of row c's operands carry the factor 1); 5 for row 15,
// which no level supplies; -1 above the diagonal.
__device__ __forceinline__ int pair_level(int c, int i) {
    if (c < i) return -1;
    if (c == i) return 1 + __builtin_ctz(~static_cast<unsigned>(c));
    return 32 - __builtin_clz(static_cast<unsigned>(c ^ i));
}

template <int K, int NC, typename TQ>
struct Kern {
    static constexpr int KT = K / 16;                   // 16-row state tiles
    static constexpr int KU = K / 32;                   // 32-wide k blocks
    static constexpr int CH = K / 32;                   // channels per producer lane
    static constexpr int KR = K + 8;                    // padded row of a row-major operand
    static constexpr int VT = 16 * NC;
    static constexpr int QB = CH * static_cast<int>(sizeof(TQ));   // bytes of a lane's q / k row
    static constexpr int QW = BLoad<QB>::W;
    static constexpr int GW = BLoad<4 * CH>::W;

    // One block's raw inputs for a producer lane: its CH channels of rows
    // 8hf .. 8hf + 7, and beta of rows 4lg .. 4lg + 3 (for the solve).
    struct Raw {
        uint32_t q[HR][QW], k[HR][QW], g[HR][GW];
        uint32_t beta[4];
    };
    // The same block, converted: decays, fp16 q and k rows (channels in the
    // low CH slots), beta.
    struct Work {
        float al[CH][HR];
        h4 q[HR], k[HR];
        float beta[4];
    };

    const kda_fwd_args& a;
    Smem<K>& sm;
    int64_t b, h, T;
    float scale;
    int lane, ln, lg;
    int hf, cq;                              // producer: row half, channel group (channels CH*cq ..)
    uint32_t rs_q, rs_k, rs_g, rs_v, rs_b;   // token-row strides in bytes
    uint32_t vo_q, vo_k, vo_g, vo_v, vo_b;   // lane byte offsets

    __device__ Kern(const kda_fwd_args& args, Smem<K>& s) : a(args), sm(s) {}

    // Rows of block `blk` that lie before T (0..BT).
    __device__ int rows_in(int blk) const {
        const int64_t left = T - static_cast<int64_t>(blk) * BT;
        return left <= 0 ? 0 : (left < BT ? static_cast<int>(left) : BT);
    }

    // Descriptor over the rows of one block of a [B, T, H, D] view (elements
    // of es bytes, token stride rs bytes), based at (b, 16 blk, h, 0).
    __device__ __amdgpu_buffer_rsrc_t block_rsrc(const void* p, const int64_t (&st)[3], int es, uint32_t rs,
                                                 int blk) const {
        const int64_t e = b * st[0] + static_cast<int64_t>(blk) * BT * st[1] + h * st[2];
        return make_rsrc(static_cast<const char*>(p) + e * es, static_cast<uint32_t>(rows_in(blk)) * rs);
    }

    // ------------------------------------------------------------ producers
    __device__ void load_raw(Raw& r, int blk) const {
        const auto rq = block_rsrc(a.q, a.q_stride, sizeof(TQ), rs_q, blk);
        const auto rk = block_rsrc(a.k, a.k_stride, sizeof(TQ), rs_k, blk);
        const auto rg = block_rsrc(a.g, a.g_stride, 4, rs_g, blk);
        const auto rb = block_rsrc(a.beta, a.beta_stride, 4, rs_b, blk);
#pragma unroll
        for (int i = 0; i < HR; ++i) {
            BLoad<4 * CH>::ld(r.g[i], rg, vo_g, i * rs_g);
            BLoad<QB>::ld(r.q[i], rq, vo_q, i * rs_q);
            BLoad<QB>::ld(r.k[i], rk, vo_k, i * rs_k);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) BLoad<4>::ld(&r.beta[j], rb, vo_b, j * rs_b);
    }

    __device__ void unpack(Raw& r, Work& w) const {
        use_here(r.q);
        use_here(r.k);
        use_here(r.g);
        use_here(r.beta);
#pragma unroll
        for (int i = 0; i < HR; ++i) {
#pragma unroll
            for (int c = 0; c < CH; ++c) w.al[c][i] = fast_exp(__uint_as_float(r.g[i][c]));
            h4 qv = {0, 0, 0, 0}, kv = {0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                qv[c] = raw_h<TQ>(r.q[i], c);
                kv[c] = raw_h<TQ>(r.k[i], c);
            }
            w.q[i] = qv;
            w.k[i] = kv;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) w.beta[j] = __uint_as_float(r.beta[j]);
    }

    // Row r of per-channel values x[c][r], rounded to fp16, as a row vector
    // (channels in the low CH slots).
    static __device__ __forceinline__ h4 rowvec(const float (&x)[CH][HR], int r) {
        h4 v = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = static_cast<_Float16>(x[c][r]);
        return v;
    }

    // One row of a row-major operand: this lane's CH channels.
    __device__ void put_row(_Float16* m, int row, const h4& v) const {
        _Float16* p = m + row * KR + chan_pos(CH * cq);
        if constexpr (CH == 4) {
            *reinterpret_cast<h4*>(p) = v;
        } else if constexpr (CH == 2) {
            *reinterpret_cast<h2*>(p) = h2{v[0], v[1]};
        } else {
            *p = v[0];
        }
    }
    // Rows 4part .. 4part + 3 of this lane's half of block bi into the
    // k-major lines of its channels (one 8-byte piece per channel).
    __device__ void put_kmajor(_Float16 (*kh)[2 * BT], int bi, int part, const h4 (&v)[4]) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int ch = CH * cq + c;
            const h4 piece = {v[0][c], v[1][c], v[2][c], v[3][c]};
            *reinterpret_cast<h4*>(&kh[ch][8 * ((2 * hf + part) ^ kh_swz(ch)) + 4 * bi]) = piece;
        }
    }
    // Row r of x[c][r] * m[c], rounded to fp16, as a row vector.
    static __device__ __forceinline__ h4 rowvec(const float (&x)[CH][HR], const float (&m)[CH], int r) {
        h4 v = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = static_cast<_Float16>(x[c][r] * m[c]);
        return v;
    }

    // Level factors of the half's 8 rows, level B in 0..2 (groups of 2^(B+1)
    // rows inside the half): upper-half rows c get prod_{t=ref+1..c} a_t and
    // lower-half rows i get prod_{t=i+1..ref} a_t, ref = the group's last
    // lower row.
    template <int B>
    static __device__ __forceinline__ void level_factors(const float (&al)[HR], float (&f)[HR]) {
        constexpr int S = 2 << B, HALF = 1 << B;
#pragma unroll
        for (int st = 0; st < HR; st += S) {
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

    // Operand level LEV (1..4) of a block: X_b = k * F_b and Y_b = q * F_b,
    // written row-major into xs / ys, b = LEV - 1.  Y_b is only read in the
    // rows that are the later row of a level-b pair (bit b set, scaled) and
    // in the level's reference rows (the last lower row of each group, factor
    // 1: the diagonal of A); its other rows are not written.  Level 4 pairs
    // the two halves: its factors are the decays from the upper half's start
    // (pl) and to the lower half's end (sl, 1 in the reference row 7); all
    // of its Y rows are written (a lane-dependent choice costs registers).
    template <int LEV>
    __device__ void stage(const Work& w, const float (&pl)[CH][HR], const float (&sl)[CH][HR], _Float16* xs,
                          _Float16* ys) const {
        constexpr int bb = LEV - 1;
        float f[CH][HR];
        if constexpr (LEV <= 3) {
#pragma unroll
            for (int c = 0; c < CH; ++c) level_factors<bb>(w.al[c], f[c]);
        } else {
#pragma unroll
            for (int c = 0; c < CH; ++c)
#pragma unroll
                for (int r = 0; r < HR; ++r) f[c][r] = hf ? pl[c][r] : sl[c][r];
        }
#pragma unroll
        for (int r = 0; r < HR; ++r) {
            const h4 fr = rowvec(f, r);
            put_row(xs, HR * hf + r, w.k[r] * fr);
            if constexpr (LEV <= 3) {
                const bool upper = (r >> bb) & 1, ref = (r & ((2 << bb) - 1)) == (1 << bb) - 1;
                if (upper) put_row(ys, HR * hf + r, w.q[r] * fr);
                else if (ref) put_row(ys, HR * hf + r, w.q[r]);
            } else {
                put_row(ys, HR * hf + r, w.q[r] * fr);
            }
        }
    }

    // A level's staged operands as MFMA fragments (row ln, the 8 channels of
    // lane group lg in each 32-channel block).
    struct Frags {
        h8 x[KU], y[KU];
    };
    __device__ Frags read_frags(const _Float16* xs, const _Float16* ys) const {
        Frags f;
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            f.x[u] = *reinterpret_cast<const h8*>(xs + ln * KR + 32 * u + 8 * lg);
            f.y[u] = *reinterpret_cast<const h8*>(ys + ln * KR + 32 * u + 8 * lg);
        }
        return f;
    }

    // Level LEV's products: G_b = X_b X_b^T and A_b = Y_b X_b^T over all K
    // channels, keeping the entries the level supplies (accumulator layout:
    // row 4lg + j, column ln).
    template <int LEV>
    __device__ void product(const Frags& fr, f4& Gacc, f4& Aacc) const {
        f4 accG = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            accG = mfma16x16x32(fr.x[u], fr.x[u], accG);
            accA = mfma16x16x32(fr.y[u], fr.x[u], accA);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (pair_level(4 * lg + j, ln) == LEV) {
                if (4 * lg + j != ln) Gacc[j] = accG[j];   // G (and L) is strictly lower
                Aacc[j] = accA[j];
            }
        }
    }

    // M = (I + L)^-1 Diag(beta) of one block (wave p, L in accumulator
    // layout), stored as hi/lo A-operand fragments.
    __device__ void solve(const f4& Lc, const float (&beta)[4], _Float16 (*mh)[RP], _Float16 (*ml)[RP], int p) const {
        float* lt = &sm.LT[p][0][0];
#pragma unroll
        for (int j = 0; j < 4; ++j) lt[(4 * lg + j) * LP + ln] = Lc[j];
        f4 Lt;                                           // acc(L^T)
        {
            const float4 r = *reinterpret_cast<const float4*>(lt + ln * LP + 4 * lg);
            Lt[0] = r.x; Lt[1] = r.y; Lt[2] = r.z; Lt[3] = r.w;
        }
        const Split4 lc(Lc), ltt(Lt);
        const Split4 l2(mm4(ltt, lc)), l2t(mm4(lc, ltt));  // L^2, (L^2)^T
        const Split4 l4(mm4(l2t, l2)), l4t(mm4(l2, l2t));
        const Split4 l8(mm4(l4t, l4));
        f4 Q;                                            // acc(I - L^T)
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] = (4 * lg + j == ln ? 1.f : 0.f) - Lt[j];
        Q = mm4(l2, Split4(Q), Q);
        Q = mm4(l4, Split4(Q), Q);
        Q = mm4(l8, Split4(Q), Q);                       // acc(Minv^T) = A-layout of Minv
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] *= beta[j];
        h4 hi, lo;
        split4(Q, hi, lo);
        *reinterpret_cast<h4*>(&mh[ln][4 * lg]) = hi;
        *reinterpret_cast<h4*>(&ml[ln][4 * lg]) = lo;
    }

    // First half of a superstep for block p (bi = p % 2 of chunk cj): the
    // level products (the next block's loads go out after the first two),
    // the decays of the block, and every operand that needs no other block's
    // decay.  `keep` receives, for the second half, the decays to the block
    // end (block 0) or from the block start (block 1).
    __device__ void phase1(Raw& raw, Work& w, f4& Gacc, f4& Aacc, float (&keep)[CH][HR], int p,
                           ChunkOps<K>& co, int next) const {
        const int bi = p % CB, cj = p / CB;
        Stage<K>& st = sm.st[cj];
        unpack(raw, w);
        Gacc = f4{0.f, 0.f, 0.f, 0.f};
        Aacc = f4{0.f, 0.f, 0.f, 0.f};
        // level operands are staged in the block's q * E / k * E rows, which
        // get their final values after the last level
        _Float16* xs = &co.QE[bi][0][0];
        _Float16* ys = &co.KE[bi][0][0];
        float pl[CH][HR], sl[CH][HR];                    // decays from the half's start / to its end
        // Levels are software-pipelined through the one staging pair: LDS
        // serves a wave's requests in order, so level b+1's operands may be
        // written as soon as level b's fragment reads are issued, and their
        // VALU work covers those reads and level b's MFMAs.
        stage<1>(w, pl, sl, xs, ys);
        Frags fr = read_frags(xs, ys);
        stage<2>(w, pl, sl, xs, ys);
        product<1>(fr, Gacc, Aacc);
        load_raw(raw, next);
        fr = read_frags(xs, ys);
        stage<3>(w, pl, sl, xs, ys);
        product<2>(fr, Gacc, Aacc);
        fr = read_frags(xs, ys);
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            pl[c][0] = w.al[c][0];
#pragma unroll
            for (int r = 1; r < HR; ++r) pl[c][r] = pl[c][r - 1] * w.al[c][r];
            sl[c][HR - 1] = 1.f;
#pragma unroll
            for (int r = HR - 2; r >= 0; --r) sl[c][r] = sl[c][r + 1] * w.al[c][r + 1];
        }
        stage<4>(w, pl, sl, xs, ys);
        product<3>(fr, Gacc, Aacc);
        fr = read_frags(xs, ys);
        product<4>(fr, Gacc, Aacc);

        // block decays: the upper half's prefix continues the lower half's,
        // the lower half's suffix continues into the upper half
        float mp[CH], ms[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            // the swap returns this lane's value in one slot and the other
            // half's in the other
            const unsigned u = __float_as_uint(pl[c][HR - 1]);
            const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            const float other = __uint_as_float(sw[0] != u ? sw[0] : sw[1]);
            mp[c] = hf ? other : 1.f;
            ms[c] = hf ? 1.f : other;
            if (hf == 0) st.e15[bi][CH * cq + c] = pl[c][HR - 1] * other;
        }
        // rows are produced and stored one at a time (few registers live)
        if (bi == 0) {
            // block 0: decays from its start are decays from the chunk start
#pragma unroll
            for (int r = 0; r < HR; ++r) {
                const h4 e = rowvec(pl, mp, r), f = rowvec(sl, ms, r);
                put_row(&co.QE[0][0][0], HR * hf + r, w.q[r] * e);
                put_row(&co.KE[0][0][0], HR * hf + r, w.k[r] * e);
                put_row(&st.KH0[0][0], HR * hf + r, w.k[r] * f);
#pragma unroll
                for (int c = 0; c < CH; ++c) keep[c][r] = sl[c][r] * ms[c];
            }
        } else {
            // block 1: decays to its end are decays to the chunk end; its
            // block-local q * E, k * E wait in place for G_10 and A_10
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                h4 fk[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = 4 * part + i;
                    const h4 e = rowvec(pl, mp, r);
                    fk[i] = w.k[r] * rowvec(sl, ms, r);
                    put_row(&co.QE[1][0][0], HR * hf + r, w.q[r] * e);
                    put_row(&co.KE[1][0][0], HR * hf + r, w.k[r] * e);
#pragma unroll
                    for (int c = 0; c < CH; ++c) keep[c][r] = pl[c][r] * mp[c];
                }
                put_kmajor(co.KH, 1, part, fk);
            }
        }
    }

    // Second half: the operands that need the other block's decay (block 0:
    // k * F; block 1: G_10 and A_10 from the block-local operands, then
    // q * E and k * E from the chunk start, and the chunk decay), then A and
    // the inverse of (I + L).
    __device__ void phase2(const Work& w, const f4& Gacc, const f4& Aacc, const float (&keep)[CH][HR], int p,
                           ChunkOps<K>& co) const {
        const int bi = p % CB, cj = p / CB;
        Stage<K>& st = sm.st[cj];
        float d[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) d[c] = st.e15[1 - bi][CH * cq + c];
        if (bi == 0) {
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                h4 fk[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) fk[i] = w.k[4 * part + i] * rowvec(keep, d, 4 * part + i);
                put_kmajor(co.KH, 0, part, fk);
            }
        } else {
            // G_10^T and A_10^T over all K channels: the accumulator holds
            // column ln of block 1 against rows 4lg + j of block 0, the
            // A-operand layout of G_10 and A_10.
            f4 accG = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < KU; ++u) {
                const int o = ln * KR + 32 * u + 8 * lg;
                const h8 hf0 = *reinterpret_cast<const h8*>(&st.KH0[0][0] + o);
                accG = mfma16x16x32(hf0, *reinterpret_cast<const h8*>(&co.KE[1][0][0] + o), accG);
                accA = mfma16x16x32(hf0, *reinterpret_cast<const h8*>(&co.QE[1][0][0] + o), accA);
            }
            h4 gh, gl;
            split4(-accG, gh, gl);
            *reinterpret_cast<h4*>(&co.GH[ln][4 * lg]) = gh;
            *reinterpret_cast<h4*>(&co.GL[ln][4 * lg]) = gl;
            const f4 as = accA * scale;
            *reinterpret_cast<h4*>(&co.A10[ln][4 * lg]) =
                h4{static_cast<_Float16>(as[0]), static_cast<_Float16>(as[1]), static_cast<_Float16>(as[2]),
                   static_cast<_Float16>(as[3])};
#pragma unroll
            for (int r = 0; r < HR; ++r) {
                const h4 e = rowvec(keep, d, r);
                put_row(&co.QE[1][0][0], HR * hf + r, w.q[r] * e);
                put_row(&co.KE[1][0][0], HR * hf + r, w.k[r] * e);
            }
            if (hf == 1) {
                // row 15 of block 1 ends the chunk
#pragma unroll
                for (int c = 0; c < CH; ++c) co.echunk[CH * cq + c] = keep[c][HR - 1] * d[c];
            }
        }
        // A[15][15] = <q_15, k_15>: row 15 is no level's reference row
        f4 A = Aacc;
        {
            float dq = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c)
                dq += static_cast<float>(w.q[HR - 1][c]) * static_cast<float>(w.k[HR - 1][c]);
            dq = wave_sum(hf ? dq : 0.f);
            if (lane == 63) A[3] = dq;
        }
        f4 G = Gacc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            co.AM[bi][4 * lg + j][ln] = static_cast<_Float16>(A[j] * scale);
            G[j] *= w.beta[j];
        }
        solve(G, w.beta, co.MH[bi], co.ML[bi], p);
    }

    // ------------------------------------------------------------ consumers
    __device__ void v_load(uint32_t (&vr)[4], int blk) const {
        const auto rv = block_rsrc(a.v, a.v_stride, sizeof(TQ), rs_v, blk);
#pragma unroll
        for (int j = 0; j < 4; ++j) BLoad<sizeof(TQ)>::ld(&vr[j], rv, vo_v, j * rs_v);
    }

    // Output rows 4lg + j of block blk (rows past T are skipped).
    __device__ void store_o(const f4& O, int blk, int64_t col0, uint32_t ocol) const {
        TQ* o = static_cast<TQ*>(a.o) + ((b * T + static_cast<int64_t>(blk) * BT) * a.H + h) * a.V + col0;
        const uint32_t orow = static_cast<uint32_t>(a.H * a.V);
        const int nrow = rows_in(blk);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (4 * lg + j < nrow) Elem<TQ>::st(o + (4 * lg + j) * orow + ocol, O[j]);
    }

    // One chunk (blocks blk, blk + 1) of the chain for this wave's 16 state
    // columns; the v loads of the same blocks one superstep later are issued
    // into vraw0 / vraw1.  ck (or null): the chunk's checkpoint for the
    // backward, in fp32: rows [0, K) the state before it, [K, K + 32) its
    // R = V - (k * E) S, [K + 32, K + 64) its P.  The stores go out after the
    // v loads, so that waiting for those loads never waits for them.
    __device__ void consume(const ChunkOps<K>& co, int blk, uint32_t (&vraw0)[4], uint32_t (&vraw1)[4],
                            f4 (&S)[KT], int64_t col0, uint32_t ocol, float* ck) const {
        use_here(vraw0);
        use_here(vraw1);
        f4 R0, R1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            R0[j] = raw_f<TQ>(vraw0[j]);
            R1[j] = raw_f<TQ>(vraw1[j]);
        }
        v_load(vraw0, blk + NB);
        v_load(vraw1, blk + 1 + NB);
        const int64_t V = a.V, rc = col0 + ocol;
        if (ck) store_state_t<KT>(S, ck, (4 * lg) * V + rc, V);
        float* rp = ck ? ck + static_cast<int64_t>(K) * V : nullptr;
        h8 shi[KU], slo[KU];
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            h4 h0, l0, h1, l1;
            split4(S[2 * u], h0, l0);
            split4(S[2 * u + 1], h1, l1);
            shi[u] = cat(h0, h1);
            slo[u] = cat(l0, l1);
        }
        // Z_b = (k * E)_b S and O_b = (q * E)_b S over the K channels
        f4 Z0 = {0.f, 0.f, 0.f, 0.f}, Z1 = Z0, O0 = Z0, O1 = Z0;
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int o = ln * KR + 32 * u + 8 * lg;
            const h8 k0 = *reinterpret_cast<const h8*>(&co.KE[0][0][0] + o);
            Z0 = mfma16x16x32(k0, shi[u], Z0);
            Z0 = mfma16x16x32(k0, slo[u], Z0);
            const h8 k1 = *reinterpret_cast<const h8*>(&co.KE[1][0][0] + o);
            Z1 = mfma16x16x32(k1, shi[u], Z1);
            Z1 = mfma16x16x32(k1, slo[u], Z1);
        }
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int o = ln * KR + 32 * u + 8 * lg;
            const h8 q0 = *reinterpret_cast<const h8*>(&co.QE[0][0][0] + o);
            O0 = mfma16x16x32(q0, shi[u], O0);
            O0 = mfma16x16x32(q0, slo[u], O0);
            const h8 q1 = *reinterpret_cast<const h8*>(&co.QE[1][0][0] + o);
            O1 = mfma16x16x32(q1, shi[u], O1);
            O1 = mfma16x16x32(q1, slo[u], O1);
        }
        // P_0 = M_00 (V_0 - Z_0);  P_1 = M_11 (V_1 - Z_1 - G_10 P_0)
        R0 -= Z0;
        R1 -= Z1;
        if (rp) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                rp[(4 * lg + j) * V + rc] = R0[j];
                rp[(16 + 4 * lg + j) * V + rc] = R1[j];
            }
        }
        const Split4 r0(R0);
        const f4 P0 = mm4(frag16(&co.MH[0][0][0], RP, ln, lg), frag16(&co.ML[0][0][0], RP, ln, lg), r0.hi, r0.lo,
                          f4{0.f, 0.f, 0.f, 0.f});
        const Split4 p0(P0);
        R1 = mm4(frag16(&co.GH[0][0], RP, ln, lg), frag16(&co.GL[0][0], RP, ln, lg), p0.hi, p0.lo, R1);
        const Split4 r1(R1);
        const f4 P1 = mm4(frag16(&co.MH[1][0][0], RP, ln, lg), frag16(&co.ML[1][0][0], RP, ln, lg), r1.hi, r1.lo,
                          f4{0.f, 0.f, 0.f, 0.f});
        const Split4 p1(P1);
        if (rp) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                rp[(32 + 4 * lg + j) * V + rc] = P0[j];
                rp[(48 + 4 * lg + j) * V + rc] = P1[j];
            }
        }
        // O = scale (q * E) S + A P
        O0 *= scale;
        O1 *= scale;
        const h4 a00 = frag16(&co.AM[0][0][0], RP, ln, lg);
        O0 = mfma16x16x32(cat(a00, a00), cat(p0.hi, p0.lo), O0);
        const h8 a1 = cat(frag16(&co.A10[0][0], RP, ln, lg), frag16(&co.AM[1][0][0], RP, ln, lg));
        O1 = mfma16x16x32(a1, cat(p0.hi, p1.hi), O1);
        O1 = mfma16x16x32(a1, cat(p0.lo, p1.lo), O1);
        store_o(O0, blk, col0, ocol);
        store_o(O1, blk + 1, col0, ocol);
        // S <- E[31] S + F^T P over both blocks: the k-major line of channel
        // 16t + ln gives tokens 4lg..4lg+3 of block 0 then of block 1, the
        // order of cat(P_0, P_1)
        const h8 ph = cat(p0.hi, p1.hi), pl = cat(p0.lo, p1.lo);
        const int piece = 8 * (lg ^ ((ln >> 2) & 3));
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const float4 e = *reinterpret_cast<const float4*>(&co.echunk[16 * t + 4 * lg]);
            S[t][0] *= e.x; S[t][1] *= e.y; S[t][2] *= e.z; S[t][3] *= e.w;
            const h8 kf = *reinterpret_cast<const h8*>(&co.KH[16 * t + ln][piece]);
            S[t] = mfma16x16x32(kf, ph, S[t]);
            S[t] = mfma16x16x32(kf, pl, S[t]);
        }
    }
};

// Supersteps of NB blocks (NCH chunks).  Before superstep s the producers
// have filled slot set s % 2 with the chunks of superstep s; during it they
// fill the other set with superstep s + 1 while the consumers run superstep
// s; one workgroup barrier ends each half.  Every wave executes the same
// barriers; every prefetch is issued unconditionally (a block past T loads
// zeros).  The chunks cover T rounded up to whole chunks: a padded block
// (all rows past T) is neutral and is built like any other.
template <int K, int NC, typename TQ>
__global__ __launch_bounds__(64 * (NC + NB)) void chunkwise_kernel(const kda_fwd_args a, float* ckpt) {
    using KN = Kern<K, NC, TQ>;
    constexpr int KT = KN::KT, VT = KN::VT, CH = KN::CH;
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
    kn.scale = a.scale;
    // wave index as a scalar: block indices and buffer descriptors derived
    // from it stay in SGPRs (no per-lane descriptor loops around the loads)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    kn.lane = threadIdx.x & 63;
    kn.ln = kn.lane & 15;
    kn.lg = kn.lane >> 4;
    kn.hf = kn.lane >> 5;
    kn.cq = kn.lane & 31;
    const int nch = static_cast<int>((a.T + BT - 1) / BT);
    const int ncc = (nch + CB - 1) / CB;                 // chunks
    const int nblk = CB * ncc;                           // blocks, padded to whole chunks
    const int nss = (ncc + NCH - 1) / NCH;               // supersteps

    const bool consumer = wave < NC;
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
        const uint32_t c0 = static_cast<uint32_t>(CH * kn.cq), r0 = static_cast<uint32_t>(HR * kn.hf);
        kn.vo_q = r0 * kn.rs_q + c0 * eq;
        kn.vo_k = r0 * kn.rs_k + c0 * eq;
        kn.vo_g = r0 * kn.rs_g + c0 * 4u;
        kn.vo_b = static_cast<uint32_t>(4 * kn.lg) * kn.rs_b;
        kn.vo_v = static_cast<uint32_t>(4 * kn.lg) * kn.rs_v + static_cast<uint32_t>(col) * eq;
    }

    if (consumer) {
        f4 S[KT];
        load_state<KT>(S, a.state_in, a.state_in_dtype, sbase + (4 * kn.lg) * V + col, V);
        uint32_t vr[NB][4];
#pragma unroll
        for (int j = 0; j < NB; ++j) kn.v_load(vr[j], j);
        for (int s = -1; s < nss; ++s) {
#pragma unroll
            for (int cj = 0; cj < NCH; ++cj) {
                const int cc = NCH * s + cj;
                if (s >= 0 && cc < ncc) {
                    // the checkpoint of chunk cc, for the backward
                    float* ck = ckpt ? ckpt + ((kn.b * H + kn.h) * ncc + cc) * static_cast<int64_t>(K + 2 * CB * BT) * V
                                     : nullptr;
                    kn.consume(sm.set[s & 1][cj], NB * s + CB * cj, vr[CB * cj], vr[CB * cj + 1], S, col0, ocol, ck);
                }
                __syncthreads();
            }
        }
        store_state<KT>(S, a.state_out, a.state_out_dtype, sbase + (4 * kn.lg) * V + col, V);
    } else {
        const int p = wave - NC;
        typename KN::Raw raw;
        typename KN::Work w;
        f4 Gacc, Aacc;
        float keep[CH][HR];
        kn.load_raw(raw, p);
        for (int s = -1; s < nss; ++s) {
            const int blk = NB * (s + 1) + p;
            ChunkOps<K>& co = sm.set[(s + 1) & 1][p / CB];
            if (blk < nblk) kn.phase1(raw, w, Gacc, Aacc, keep, p, co, blk + NB);
            __syncthreads();
            if (blk < nblk) kn.phase2(w, Gacc, Aacc, keep, p, co);
            __syncthreads();
        }
    }
}

template <int K, int NC, typename TQ>
int launch_knq(const kda_fwd_args& a, hipStream_t stream, float* ckpt) {
    const int64_t blocks = a.B * a.H * (a.V / (16 * NC));
    hipLaunchKernelGGL((chunkwise_kernel<K, NC, TQ>), dim3(static_cast<unsigned>(blocks)), dim3(64 * (NC + NB)), 0,
                       stream, a, ckpt);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

// Columns per workgroup: the widest tile (64, 32 or 16 columns) that still
// gives at least one workgroup per CU; 16 when none does (few chains).
template <int K, typename TQ>
int launch_kq(const kda_fwd_args& a, hipStream_t stream, float* ckpt) {
    constexpr int64_t kCus = 256;
    const int64_t heads = a.B * a.H;
    if (a.V % 64 == 0 && heads * (a.V / 64) >= kCus) return launch_knq<K, 4, TQ>(a, stream, ckpt);
    if (a.V % 32 == 0 && heads * (a.V / 32) >= kCus) return launch_knq<K, 2, TQ>(a, stream, ckpt);
    return launch_knq<K, 1, TQ>(a, stream, ckpt);
}

template <int K>
int launch_k(const kda_fwd_args& a, hipStream_t stream, float* ckpt) {
    switch (a.qkv_dtype) {
        case KDA_DTYPE_F16: return launch_kq<K, _Float16>(a, stream, ckpt);
        case KDA_DTYPE_BF16: return launch_kq<K, bf16_t>(a, stream, ckpt);
        case KDA_DTYPE_F32: return launch_kq<K, float>(a, stream, ckpt);
        default: return KDA_ERR_BAD_DTYPE;
    }
}

}  // namespace

bool chunkwise_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % 16 == 0;
}

int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt) {
    // the pipeline reads gates in fp32 (the wrapper converts other dtypes)
    if (a.g_dtype != KDA_DTYPE_F32 || a.beta_dtype != KDA_DTYPE_F32) return KDA_ERR_BAD_DTYPE;
    // in-block offsets are 32-bit byte offsets: 16 token strides + one row must fit
    const int64_t lim = int64_t(1) << 31;
    const int64_t ts[5] = {a.q_stride[1], a.k_stride[1], a.v_stride[1], a.g_stride[1], a.beta_stride[1]};
    for (int64_t st : ts)
        if (st < 0 || (BT + 1) * st * 4 + a.V * 4 >= lim) return KDA_ERR_UNSUPPORTED;
    if ((BT + 1) * a.H * a.V * 4 >= lim) return KDA_ERR_UNSUPPORTED;
    // a block's buffer descriptor spans rows_in * token stride bytes, so every
    // token row must be disjoint from the next (stride >= row length)
    if (a.T > 1 && (a.q_stride[1] < a.K || a.k_stride[1] < a.K || a.g_stride[1] < a.K ||
                    a.v_stride[1] < a.V || a.beta_stride[1] < 1))
        return KDA_ERR_UNSUPPORTED;
    switch (a.K) {
        case 32: return launch_k<32>(a, stream, ckpt);
        case 64: return launch_k<64>(a, stream, ckpt);
        case 128: return launch_k<128>(a, stream, ckpt);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace kda
