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
// L = Diag(beta) G_bb: products and squarings on the fp32 matrix cores
// (v_mfma_f32_16x16x4f32, no precision loss), entirely in registers.  An MFMA accumulator holds
// X[4g+j][n] in lane n+16g, slot j -- the B-operand layout of X and the
// A-operand layout of X^T -- so a chain that keeps X and X^T side by side
// needs no data movement.
//
// Pipeline, one workgroup per (b, h, 16*NC state columns), in supersteps of
// NB = 4 blocks (two chunks), each split in two halves by workgroup barriers:
//   NC consumer waves: wave w owns state columns [16w, 16w+16) for all K rows
//     as MFMA accumulators and runs the chain over both chunks of superstep s
//     in the first half.  With NC = NB, consumer wave p inverts (I + L) of
//     block p of superstep s+1 in the second half.
//   NB producer waves, one per block: wave p builds every operand of block
//     NB*(s+1) + p.  Lane l holds K/32 adjacent channels of the block's rows
//     8 (l / 32) .. +7, which one 8-byte (fp16) load per row brings in for
//     all K channels of two rows.  First half: decays, the level operands
//     and their products (A to its operand, G to the solve), the operands
//     with decays from the block start, the block-local operands of the
//     chunk's off-diagonal products, the block decay E[15].  Second half,
//     once the other block's decay is known: block 0's k * F to the chunk
//     end, G_10 and A_10 (block 1's wave), the chunk decay (and, with fewer
//     consumer waves than blocks, the inverse of (I + L)).  Block 1's
//     q * E and k * E keep the decay from its own start: the consumers apply
//     block 0's decay to the state instead.  The next block's loads are
//     issued in the first half and land during the rest of the superstep.
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
// Precision: fp32 accumulation everywhere; the state is carried in fp32.
// The solve's results P, M and G_10, which the state update and the chunk's
// outputs take as operands, are split into fp16 hi + lo; S (in Z and O) and
// R = V - Z enter their products as single fp16 operands (rounded once per
// chunk), like q * E, k * E and A.
//
// Range (bf16 activations): the state, V, R and P pass through fp16 operands,
// whose range ends at 65504, while bf16 values reach 3e38.  The chain is
// linear in (V, S), so each consumer wave carries its state scaled by a power
// of two sigma (exact): before a chunk it takes the largest |sigma S| and
// |sigma V| of its columns and, when that passes 2^10 (headroom for Z = (k*E)
// S and P = M R), divides sigma by the power of two that brings it back
// under; outputs, checkpoints and the final state are divided by sigma.  With
// values under 2^10 sigma stays 1 and nothing changes.  fp16 activations keep
// the fp16 range, as the reference's fp16 path does (it casts the state to
// the input dtype for its products, kimi_linear/kda.py:174).
#include <type_traits>

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
// Element j of a raw row of TQ values, as fp32.
template <typename TQ, int W>
__device__ __forceinline__ float raw_ef(const uint32_t (&w)[W], int j) {
    if constexpr (sizeof(TQ) == 4) {
        return __uint_as_float(w[j]);
    } else {
        const uint32_t bits = (w[j / 2] >> (16 * (j % 2))) & 0xffffu;
        if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
            return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
        } else {
            return __uint_as_float(bits << 16);
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

// Four fp32 values rounded to fp16 (round to nearest even).
__device__ __forceinline__ h4 to_h4(const f4& x) {
    return h4{static_cast<_Float16>(x[0]), static_cast<_Float16>(x[1]), static_cast<_Float16>(x[2]),
              static_cast<_Float16>(x[3])};
}

// Position of channel c inside a row-major operand row.  With c = 32u + 16hi
// + 4g + j, the consumer lane of group g pairs channels 32u + 4g + j and
// 32u + 16 + 4g + j with its state rows; they sit at 32u + 8g + (0..7).
__device__ __forceinline__ int chan_pos(int c) {
    return (c & ~31) | ((c & 12) << 1) | ((c & 16) >> 2) | (c & 3);
}
// The k-major k * F lines are 80 bytes apart (64 bytes of data) and their
// 16-byte pieces are rotated by channel bits 4-5: the 16 lines one consumer
// instruction reads start on 16 distinct groups of 4 banks, and the 32 lines
// one producer instruction writes (channels 4 apart) on at most 2 per bank.
constexpr int KHP = 2 * BT + 8;   // halfs per k-major line
__device__ __forceinline__ int kh_swz(int c) { return (c >> 4) & 3; }

// Operands of one chunk, as the consumers read them.
template <int K>
struct __align__(16) ChunkOps {
    static constexpr int KR = K + 8;
    _Float16 QE[CB][BT][KR];               // q * E (decay from the block start), row-major
    _Float16 KE[CB][BT][KR];               // k * E
    _Float16 KH[K][KHP];                   // k * F (decay to the chunk end), k-major lines
    _Float16 AM[CB][BT][RP];               // scale * A, diagonal blocks
    _Float16 MH[CB][BT][RP];               // M hi
    _Float16 ML[CB][BT][RP];               // M lo
    _Float16 A10[BT][RP];                  // scale * A, rows of block 1, columns of block 0
    _Float16 GH[BT][RP];                   // -G_10 hi
    _Float16 GL[BT][RP];                   // -G_10 lo
    float echunk[K];                       // decay over the chunk, E[31]
    float d0[K];                           // decay over block 0, E[15]
};
// Producer-only exchange of one chunk within a superstep: written in the
// first half, read in the second.
template <int K>
struct __align__(16) Stage {
    _Float16 KH0[BT][K + 8];               // block 0: k * (decay to the block end), row-major
    float e15[CB][K];                      // per block: decay over the block
};
constexpr int MAX_NC = 4;        // consumer waves per workgroup (at most)
// Row sums of squares of a chunk's outputs, per consumer wave, for the fused
// output epilogue: [chunk parity][block][row][wave].
template <bool EPI>
struct RowParts {
    float p[2][CB][BT][MAX_NC];
};
template <>
struct RowParts<false> {};
// The solve's inputs per block of a superstep: the level sums G (strictly
// lower, fp32, rows padded to 17 words) and beta, written by the block's
// producer once its level products are done, read by the wave that inverts
// (I + L) after the superstep's middle barrier.
struct __align__(16) SolveIn {
    float g[NB][BT][BT + 1];
    float beta[NB][BT];
};
template <int K, int CG, bool EPI>
struct __align__(16) Smem {
    ChunkOps<K> set[2][NCH];
    Stage<K> st[NCH];
    uint16_t vt[MAX_NC][CB * BT][16];      // per consumer wave: one chunk of v (one column group at a time), 16-bit
    SolveIn sv;
    RowParts<EPI> rows;
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
__host__ __device__ constexpr int pair_level(int c, int i) {
    if (c < i) return -1;
    if (c == i) {
        int t = 0;
        while ((c >> t) & 1) ++t;
        return 1 + t;
    }
    int x = c ^ i, bits = 0;
    while (x) {
        x >>= 1;
        ++bits;
    }
    return bits;
}

// Lane masks of the entries one level supplies, per accumulator slot j:
// lane l = 16 lg + ln holds entry (row 4 lg + j, column ln) of a 16 x 16
// tile.  Kind 0: G, strictly below the diagonal; kind 1: G^T (the mirrored
// entry of the symmetric level product), strictly above; kind 2: A, on or
// below the diagonal.  Constants, so a selection is one v_cndmask with the
// mask in VCC.
constexpr uint64_t level_mask(int lev, int j, int kind) {
    uint64_t m = 0;
    for (int l = 0; l < 64; ++l) {
        const int r = 4 * (l >> 4) + j, c = l & 15;
        const bool on = kind == 0 ? (r != c && pair_level(r, c) == lev)
                        : kind == 1 ? (r != c && pair_level(c, r) == lev)
                                    : pair_level(r, c) == lev;
        if (on) m |= uint64_t{1} << l;
    }
    return m;
}

template <int LEV, int J, int KIND>
constexpr uint64_t kLevelMask = level_mask(LEV, J, KIND);

template <int LEV, int KIND, int J>
__device__ __forceinline__ void take_slot(f4& dst, const f4& src) {
    constexpr uint64_t m = kLevelMask<LEV, J, KIND>;
    if constexpr (m != 0) dst[J] = __builtin_amdgcn_inverse_ballot_w64(m) ? src[J] : dst[J];
}
// dst takes src in the entries level LEV supplies (mask kind KIND).
template <int LEV, int KIND>
__device__ __forceinline__ void take(f4& dst, const f4& src) {
    take_slot<LEV, KIND, 0>(dst, src);
    take_slot<LEV, KIND, 1>(dst, src);
    take_slot<LEV, KIND, 2>(dst, src);
    take_slot<LEV, KIND, 3>(dst, src);
}

// c + X Y for 16 x 16 fp32 tiles on the fp32 matrix cores (four 16x16x4
// steps): xt is the accumulator layout of X^T (lane (ln, lg) slot u holds
// X[ln][4 lg + u], the A operand of step u) and y the accumulator layout of
// Y (slot u holds Y[4 lg + u][ln], the B operand); the result is in
// accumulator layout.  Used only in chains of this one form.
__device__ __forceinline__ f4 mm_f32(const f4& xt, const f4& y, f4 c) {
#pragma unroll
    for (int u = 0; u < 4; ++u) c = __builtin_amdgcn_mfma_f32_16x16x4f32(xt[u], y[u], c, 0, 0, 0);
    return c;
}

// CG: 16-column groups per consumer wave; EPI: the output epilogue (the
// layer's head-wise RMSNorm and sigmoid output gate) on the o tile, which
// needs a head's whole V row in one workgroup (16 NC CG == V).
// TRANS: the first pass of a split long sequence (kda_chunkwise_long_fwd):
// state columns V .. V + K carry the chain's transition -- they start from
// the identity and see v = 0 -- beside the V columns of its own state from
// zero; no o is written, unless TOUT: then the outputs of every state column
// are written in fp32, those of the V columns (the outputs from a zero
// initial state) to o, those of the transition columns (per token, the
// coefficients of the initial state in the outputs) to a second buffer.
template <int K, int NC, typename TQ, bool GATED, int CG = 1, bool EPI = false, bool TRANS = false,
          bool TOUT = false, bool CKPT = false>
struct Kern {
    static constexpr int KT = K / 16;                   // 16-row state tiles
    static constexpr int KU = K / 32;                   // 32-wide k blocks
    static constexpr int CH = K / 32;                   // channels per producer lane
    static constexpr int KR = K + 8;                    // padded row of a row-major operand
    static constexpr int VT = 16 * NC * CG;            // state columns per workgroup
    static constexpr int QB = CH * static_cast<int>(sizeof(TQ));   // bytes of a lane's q / k row
    static constexpr int QW = BLoad<QB>::W;
    // g and beta as loaded: fp32 log decays and rates, or (GATED) the gate's
    // up-projection gk and the beta logits in the dtype of q, k and v
    using TG = typename std::conditional<GATED, TQ, float>::type;
    static constexpr int GB = CH * static_cast<int>(sizeof(TG));   // bytes of a lane's g row
    static constexpr int GW = BLoad<GB>::W;
    static constexpr bool kEarlyDecay = GATED;      // see load_g
    // With one consumer wave per block, consumer wave p inverts (I + L) of
    // block p in the second half of a superstep, where it has no chunk to run;
    // otherwise the block's producer does, at the end of its second half.
    static constexpr bool kConsumerSolve = NC == NB;

    // One block's raw inputs for a producer lane: its CH channels of rows
    // 8hf .. 8hf + 7, and beta of rows 4lg .. 4lg + 3 (for the solve).
    struct Raw {
        uint32_t q[HR][QW], k[HR][QW], g[HR][GW];
        uint32_t beta[4];
        int rows;                            // GATED: rows of the block before T
    };
    // The same block, converted: decays a = exp(g) (GATED: formed from gk,
    // dt_bias and exp(A_log) as in gate_decay), fp16 q and k rows
    // (channels in the low CH slots), beta of rows 4lg .. 4lg + 3.
    struct Work {
        float al[CH][HR];
        h4 q[HR], k[HR];
        float beta[4];
    };
    // The level sums of a block: G (strictly lower), its mirror G^T and A.
    struct Sums {
        f4 G, GT, A;
    };

    const kda_fwd_args& a;
    Smem<K, CG, EPI>& sm;
    int64_t b, h, T;
    float scale;
    int lane, ln, lg;
    int hf, cq;                              // producer: row half, channel group (channels CH*cq ..)
    float gcoef[GATED ? CH : 1], gbias[GATED ? CH : 1];   // GATED: exp(A_log), dt_bias log2(e) of the channels
    uint32_t rs_q, rs_k, rs_g, rs_v, rs_b;   // token-row strides in bytes
    uint32_t vo_q, vo_k, vo_g, vo_v, vo_b;   // lane byte offsets
    // kda_chunkwise_fwd_ckpt: the (b, h)'s chunk records, written by the
    // head's first V-tile workgroup only (null otherwise): per 32-token chunk
    // the state and R ((K + 32) x V) and then A, L and N (32 x 32 each)
    float* ckm = nullptr;
    // The checkpointing kernel with fp16 activations stores the records
    // branch-free (an empty buffer range where there is no record), so the
    // consumers' loop keeps an exact count of its outstanding vector memory
    // operations; the other kernels have no record stores at all.
    static constexpr bool kFlatRec = CKPT && Elem<TQ>::code == KDA_DTYPE_F16;
    float* cout = nullptr;                   // TOUT: the transition columns' outputs [B, T, H, K]
    int nblk = 0;                            // blocks of the real chunks (records exist for these)

    // A, L, N of the chunk holding block blk (row-major 32 x 32, consecutive)
    __device__ float* ck_mats(int blk) const {
        return ckm + static_cast<int64_t>(blk / CB) * ckpt_record(K, a.V) + static_cast<int64_t>(K + CB * BT) * a.V;
    }

    __device__ Kern(const kda_fwd_args& args, Smem<K, CG, EPI>& s) : a(args), sm(s) {}

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
    // Rows G0 .. G1 - 1 of the lane's half of block blk (and beta): issued in
    // small groups between the level products, so that no wave stalls on a
    // burst of vector memory instructions.
    // EARLY: the gate rows are not loaded here but by load_g (a gated call).
    template <int G0, int G1, bool BETA, bool EARLY = kEarlyDecay>
    __device__ void load_rows(Raw& r, int blk) const {
        if constexpr (GATED && !EARLY && G0 == 0) r.rows = rows_in(blk);
        const auto rq = block_rsrc(a.q, a.q_stride, sizeof(TQ), rs_q, blk);
        const auto rk = block_rsrc(a.k, a.k_stride, sizeof(TQ), rs_k, blk);
        const auto rg = block_rsrc(a.g, a.g_stride, sizeof(TG), rs_g, blk);
#pragma unroll
        for (int i = G0; i < G1; ++i) {
            if constexpr (!EARLY) BLoad<GB>::ld(r.g[i], rg, vo_g, i * rs_g);
            BLoad<QB>::ld(r.q[i], rq, vo_q, i * rs_q);
            BLoad<QB>::ld(r.k[i], rk, vo_k, i * rs_k);
        }
        if constexpr (BETA) {
            const auto rb = block_rsrc(a.beta, a.beta_stride, sizeof(TG), rs_b, blk);
#pragma unroll
            for (int j = 0; j < 4; ++j) BLoad<sizeof(TG)>::ld(&r.beta[j], rb, vo_b, j * rs_b);
        }
    }
    __device__ void load_raw(Raw& r, int blk) const { load_rows<0, HR, true, false>(r, blk); }
    // A gated call loads the next block's gate rows at the start of the first
    // half and forms their decays (decays()) once the current block's decays
    // are dead, in the middle of the first half, where the gate's
    // transcendentals fill the level products' latency instead of preceding
    // them.
    __device__ void load_g(Raw& r, int blk) const {
        r.rows = rows_in(blk);
        const auto rg = block_rsrc(a.g, a.g_stride, sizeof(TG), rs_g, blk);
#pragma unroll
        for (int i = 0; i < HR; ++i) BLoad<GB>::ld(r.g[i], rg, vo_g, i * rs_g);
    }
    __device__ void decays(Raw& r, Work& w) const {
        use_here(r.g);
#pragma unroll
        for (int i = 0; i < HR; ++i) {
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                if constexpr (GATED) {
                    // rows past T must stay neutral (a = 1): they read gk = 0,
                    // which the gate would turn into a decay
                    const float a = gate_decay(fmaf(raw_ef<TG>(r.g[i], c), kLog2e, gbias[c]), gcoef[c]);
                    w.al[c][i] = HR * hf + i < r.rows ? a : 1.f;
                } else {
                    w.al[c][i] = fast_exp(__uint_as_float(r.g[i][c]));
                }
            }
        }
    }

    // q, k and beta (and the decays unless kEarlyDecay formed them already).
    __device__ void unpack(Raw& r, Work& w) const {
        use_here(r.q);
        use_here(r.k);
        use_here(r.beta);
        if constexpr (!kEarlyDecay) decays(r, w);
#pragma unroll
        for (int i = 0; i < HR; ++i) {
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
        for (int j = 0; j < 4; ++j) {
            if constexpr (GATED) {
                w.beta[j] = 4 * lg + j < r.rows ? sigmoid_f(raw_f<TG>(r.beta[j])) : 0.f;
            } else {
                w.beta[j] = __uint_as_float(r.beta[j]);
            }
        }
    }

    // Row r of per-channel values x[c][r], rounded to fp16, as a row vector
    // (channels in the low CH slots).
    static __device__ __forceinline__ h4 rowvec(const float (&x)[CH][HR], int r) {
        h4 v = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = static_cast<_Float16>(x[c][r]);
        return v;
    }
    // Per-channel values as a row vector.
    static __device__ __forceinline__ h4 chanvec(const float (&x)[CH]) {
        h4 v = {0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = static_cast<_Float16>(x[c]);
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
    __device__ h4 get_row(const _Float16* m, int row) const {
        const _Float16* p = m + row * KR + chan_pos(CH * cq);
        if constexpr (CH == 4) {
            return *reinterpret_cast<const h4*>(p);
        } else if constexpr (CH == 2) {
            const h2 x = *reinterpret_cast<const h2*>(p);
            return h4{x[0], x[1], 0, 0};
        } else {
            return h4{*p, 0, 0, 0};
        }
    }
    // Rows 4part .. 4part + 3 of this lane's half of block bi into the
    // k-major lines of its channels (one 8-byte piece per channel).
    __device__ void put_kmajor(_Float16 (*kh)[KHP], int bi, int part, const h4 (&v)[4]) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int ch = CH * cq + c;
            const h4 piece = {v[0][c], v[1][c], v[2][c], v[3][c]};
            *reinterpret_cast<h4*>(&kh[ch][8 * ((2 * hf + part) ^ kh_swz(ch)) + 4 * bi]) = piece;
        }
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

    // Operands of level LEV (1..4): X = k * f and Y = q * f row-major into
    // xs / ys.  Rows with the factor 1 (each group's reference row) take k
    // and q as they are.  Y is read only in the rows that are the later row
    // of a level pair and in the reference rows (the diagonal of A); its
    // other rows are left as they are.  Level 4's factors are the in-lane
    // running products (the upper half's prefix products from its start, the
    // lower half's suffix products to its end); it writes every Y row.
    template <int LEV>
    __device__ void stage(const Work& w, const float (&pre)[CH][HR], const float (&suf)[CH][HR], _Float16* xs,
                          _Float16* ys) const {
        constexpr int bb = LEV - 1;
        float f[CH][HR];
        if constexpr (LEV <= 3) {
#pragma unroll
            for (int c = 0; c < CH; ++c) level_factors<bb>(w.al[c], f[c]);
        }
#pragma unroll
        for (int r = 0; r < HR; ++r) {
            if constexpr (LEV <= 3) {
                const bool upper = (r >> bb) & 1, ref = (r & ((2 << bb) - 1)) == (1 << bb) - 1;
                if (ref) {
                    put_row(xs, HR * hf + r, w.k[r]);
                    put_row(ys, HR * hf + r, w.q[r]);
                } else {
                    const h4 fr = rowvec(f, r);
                    put_row(xs, HR * hf + r, w.k[r] * fr);
                    if (upper) put_row(ys, HR * hf + r, w.q[r] * fr);
                }
            } else {
                h4 fr = {0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < CH; ++c) fr[c] = static_cast<_Float16>(hf ? pre[c][r] : suf[c][r]);
                put_row(xs, HR * hf + r, w.k[r] * fr);
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

    // Level LEV's products over all K channels, X X^T (symmetric) and Y X^T,
    // keeping the entries the level supplies: G below the diagonal, its
    // mirror G^T above it, A on and below it.
    template <int LEV>
    __device__ void product(const Frags& fr, Sums& sum) const {
        f4 accG = {0.f, 0.f, 0.f, 0.f}, accA = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            accG = mfma16x16x32(fr.x[u], fr.x[u], accG);
            accA = mfma16x16x32(fr.y[u], fr.x[u], accA);
        }
        take<LEV, 0>(sum.G, accG);
        take<LEV, 1>(sum.GT, accG);
        take<LEV, 2>(sum.A, accA);
    }

    // M = (I + L)^-1 Diag(beta) of one block, L = Diag(beta) G, as hi/lo
    // A-operand fragments.  (I + L)^-T = (I - L^T)(I + (L^2)^T)(I + (L^4)^T)
    // (I + (L^8)^T) (L is nilpotent) on the fp32 matrix cores: a product X Y
    // takes X^T's and Y's accumulator layouts, so the chain keeps powers and
    // their transposes side by side; no data moves between lanes.
    // The inputs are block p's in the solve exchange area (put_solve_in).
    __device__ void solve(int p, int blk, _Float16 (*mh)[RP], _Float16 (*ml)[RP]) const {
        const float (*g)[BT + 1] = sm.sv.g[p];
        const f4 bt = *reinterpret_cast<const f4*>(&sm.sv.beta[p][4 * lg]);   // beta of rows 4lg + j
        const float bc = sm.sv.beta[p][ln];                                   // beta of row ln
        const f4 zero = {0.f, 0.f, 0.f, 0.f};
        f4 L, LT;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            L[j] = g[4 * lg + j][ln] * bt[j];     // row 4lg + j scaled by its beta
            LT[j] = g[ln][4 * lg + j] * bc;       // L^T: column ln of L^T is row ln of L
        }
        const f4 L2 = mm_f32(LT, L, zero), L2T = mm_f32(L, LT, zero);
        const f4 L4 = mm_f32(L2T, L2, zero), L4T = mm_f32(L2, L2T, zero);
        const f4 L8 = mm_f32(L4T, L4, zero);
        f4 Q;
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] = (4 * lg + j == ln ? 1.f : 0.f) - LT[j];
        Q = mm_f32(L2, Q, Q);
        Q = mm_f32(L4, Q, Q);
        Q = mm_f32(L8, Q, Q);                    // acc((I + L)^-T) = A-layout of (I + L)^-1
        if constexpr (kFlatRec) {
            // the backward's N block: N[ln][4 lg + j] = (I + L)^-1
            const bool rec = ckm && blk < nblk;
            const auto rn = make_rsrc(rec ? ck_mats(blk) + 2 * CB * BT * CB * BT : nullptr,
                                      rec ? static_cast<uint32_t>(CB * BT * CB * BT * 4) : 0u);
            const int o = BT * (blk % CB);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Q[j]), rn,
                                                      ((o + ln) * (CB * BT) + o + 4 * lg + j) * 4, 0, 2);
        } else if (CKPT && ckm && blk < nblk) {
            float* n = ck_mats(blk) + 2 * CB * BT * CB * BT;
            const int o = BT * (blk % CB);
#pragma unroll
            for (int j = 0; j < 4; ++j) __builtin_nontemporal_store(Q[j], &n[(o + ln) * (CB * BT) + o + 4 * lg + j]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) Q[j] *= bt[j];
        h4 hi, lo;
        split4(Q, hi, lo);
        *reinterpret_cast<h4*>(&mh[ln][4 * lg]) = hi;
        *reinterpret_cast<h4*>(&ml[ln][4 * lg]) = lo;
    }

    // First half of a superstep for block p (bi = p % 2 of chunk cj): the
    // decays, the level products (with the loads of block `next` between
    // them), and every operand that needs no other block's decay: block 0's
    // q * E, k * E and block-local k * F (staged for G_10, A_10); block 1's
    // block-local q * E and k * E (its operands and those of G_10, A_10) and
    // its k * F into the k-major lines.  The block decay E[15] goes to the
    // stage area (block 0's also to the consumers).
    __device__ void phase1(Raw& raw, Work& w, int p, ChunkOps<K>& co, int next) const {
        const int bi = p % CB, cj = p / CB;
        Stage<K>& st = sm.st[cj];
        unpack(raw, w);
        Sums sum;
        sum.G = f4{0.f, 0.f, 0.f, 0.f};
        sum.GT = sum.G;
        sum.A = sum.G;
        // level operands are staged in the block's q * E / k * E rows, which
        // get their final values after the last level
        _Float16* xs = &co.QE[bi][0][0];
        _Float16* ys = &co.KE[bi][0][0];
        if constexpr (kEarlyDecay) load_g(raw, next);
        // in-lane running products over the half's rows: pre (inclusive, from
        // the half's start) and suf (exclusive, to the half's end)
        float pre[CH][HR], suf[CH][HR];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            pre[c][0] = w.al[c][0];
#pragma unroll
            for (int r = 1; r < HR; ++r) pre[c][r] = pre[c][r - 1] * w.al[c][r];
            suf[c][HR - 1] = 1.f;
#pragma unroll
            for (int r = HR - 2; r >= 0; --r) suf[c][r] = suf[c][r + 1] * w.al[c][r + 1];
        }
        // Levels are software-pipelined through the one staging pair: LDS
        // serves a wave's requests in order, so level b+1's operands may be
        // written as soon as level b's fragment reads are issued.
        stage<1>(w, pre, suf, xs, ys);
        Frags fr = read_frags(xs, ys);
        stage<2>(w, pre, suf, xs, ys);
        product<1>(fr, sum);
        load_rows<0, 2, false>(raw, next);
        fr = read_frags(xs, ys);
        stage<3>(w, pre, suf, xs, ys);
        product<2>(fr, sum);
        load_rows<2, 4, false>(raw, next);
        // the current block's decays are dead: the next block's take their registers
        if constexpr (kEarlyDecay) decays(raw, w);
        fr = read_frags(xs, ys);
        stage<4>(w, pre, suf, xs, ys);
        product<3>(fr, sum);
        load_rows<4, 6, false>(raw, next);
        fr = read_frags(xs, ys);
        product<4>(fr, sum);
        load_rows<6, 8, true>(raw, next);
        // A[15][15] = <q_15, k_15>: row 15 is no level's reference row
        {
            float dq = 0.f;
#pragma unroll
            for (int c = 0; c < CH; ++c)
                dq += static_cast<float>(w.q[HR - 1][c]) * static_cast<float>(w.k[HR - 1][c]);
            dq = wave_sum(hf ? dq : 0.f);
            if (lane == 63) sum.A[3] = dq;
        }
        // the block's sums are complete: A to its operand, G and beta to the
        // solve (and both to the backward's record; block 0 also zeroes the
        // record's blocks above the diagonal)
        if (CKPT && ckm && next - NB < nblk) {
            constexpr int C = CB * BT;
            float* ma = ck_mats(next - NB);
            const int o = BT * bi;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                __builtin_nontemporal_store(sum.A[j] * scale, &ma[(o + 4 * lg + j) * C + o + ln]);
                __builtin_nontemporal_store(sum.G[j], &ma[C * C + (o + 4 * lg + j) * C + o + ln]);
                if (bi == 0) {
                    __builtin_nontemporal_store(0.f, &ma[(4 * lg + j) * C + BT + ln]);
                    __builtin_nontemporal_store(0.f, &ma[C * C + (4 * lg + j) * C + BT + ln]);
                    __builtin_nontemporal_store(0.f, &ma[2 * C * C + (4 * lg + j) * C + BT + ln]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            co.AM[bi][4 * lg + j][ln] = static_cast<_Float16>(sum.A[j] * scale);
            sm.sv.g[p][4 * lg + j][ln] = sum.G[j];
        }
        if (ln == 0) *reinterpret_cast<f4*>(&sm.sv.beta[p][4 * lg]) = f4{w.beta[0], w.beta[1], w.beta[2], w.beta[3]};

        // the other half's total decay; the block decay E[15]
        float other[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            // the swap returns this lane's value in one slot and the other
            // half's in the other
            const unsigned u = __float_as_uint(pre[c][HR - 1]);
            const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
            other[c] = __uint_as_float(sw[0] != u ? sw[0] : sw[1]);
            if (hf == 0) {
                const float e = pre[c][HR - 1] * other[c];
                st.e15[bi][CH * cq + c] = e;
                if (bi == 0) co.d0[CH * cq + c] = e;
            }
        }
        // block-local decays: E (from the block start, inclusive) = pre, times
        // the lower half's total in the upper half; F (to the block end,
        // exclusive) = suf, times the upper half's total in the lower half
        float mE[CH], mF[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            mE[c] = hf ? other[c] : 1.f;
            mF[c] = hf ? 1.f : other[c];
        }
        const h4 hE = chanvec(mE), hF = chanvec(mF);
        // rows are produced and stored one at a time (few registers live)
        if (bi == 0) {
            // block 0: decays from its start are decays from the chunk start
#pragma unroll
            for (int r = 0; r < HR; ++r) {
                const h4 e = rowvec(pre, r) * hE, f = rowvec(suf, r) * hF;
                put_row(&co.QE[0][0][0], HR * hf + r, w.q[r] * e);
                put_row(&co.KE[0][0][0], HR * hf + r, w.k[r] * e);
                put_row(&st.KH0[0][0], HR * hf + r, w.k[r] * f);
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
                    const h4 e = rowvec(pre, r) * hE;
                    fk[i] = w.k[r] * (rowvec(suf, r) * hF);
                    put_row(&co.QE[1][0][0], HR * hf + r, w.q[r] * e);
                    put_row(&co.KE[1][0][0], HR * hf + r, w.k[r] * e);
                }
                put_kmajor(co.KH, 1, part, fk);
            }
        }
    }

    // Second half: the operands that need the other block's decay (block 0:
    // k * F to the chunk end; block 1: G_10 and A_10 from the block-local
    // operands and the chunk decay), and the inverse of (I + L) when no
    // consumer wave takes it.
    __device__ void phase2(int p, int blk, ChunkOps<K>& co) const {
        const int bi = p % CB, cj = p / CB;
        Stage<K>& st = sm.st[cj];
        float d[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) d[c] = st.e15[1 - bi][CH * cq + c];
        const h4 dh = chanvec(d);
        if (bi == 0) {
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                h4 fk[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) fk[i] = get_row(&st.KH0[0][0], HR * hf + 4 * part + i) * dh;
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
            if (CKPT && ckm && blk < nblk) {
                // the backward's A_10 and L_10: slot j holds row 16 + ln, column 4 lg + j
                constexpr int C = CB * BT;
                float* ma = ck_mats(blk);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    __builtin_nontemporal_store(accA[j] * scale, &ma[(BT + ln) * C + 4 * lg + j]);
                    __builtin_nontemporal_store(accG[j], &ma[C * C + (BT + ln) * C + 4 * lg + j]);
                }
            }
            h4 gh, gl;
            split4(-accG, gh, gl);
            *reinterpret_cast<h4*>(&co.GH[ln][4 * lg]) = gh;
            *reinterpret_cast<h4*>(&co.GL[ln][4 * lg]) = gl;
            *reinterpret_cast<h4*>(&co.A10[ln][4 * lg]) = to_h4(accA * scale);
            if (hf == 0) {
#pragma unroll
                for (int c = 0; c < CH; ++c) co.echunk[CH * cq + c] = st.e15[1][CH * cq + c] * d[c];
            }
        }
        if constexpr (!kConsumerSolve) solve(p, blk, co.MH[bi], co.ML[bi]);
    }

    // ------------------------------------------------------------ consumers
    // A consumer wave owns CG groups of 16 state columns, colw + 16 g ..
    // + 15 for group g (lane column ln of each).  The chunk operands read from
    // LDS (q * E, k * E, k * F, M, G_10, A) are shared by the groups.
    //
    // The v values of one chunk for one group: 32 rows x 32 bytes (16-bit
    // inputs: row lane / 2, 8 columns a lane) or 32 x 64 bytes (fp32: rows
    // lane / 4 and 16 + lane / 4, 4 columns a lane), one 16-byte buffer load
    // per lane and row set; rows past T read as zero.
    static constexpr int VW = sizeof(TQ) == 2 ? 4 : 8;
    bool vzero = false;                      // TRANS: this wave's columns read v = 0
    // RANGE (bf16 activations): the wave's power-of-two state scale sigma and 1 / sigma
    static constexpr bool RANGE = Elem<TQ>::code == KDA_DTYPE_BF16;
    mutable float sig = 1.f, isig = 1.f;
    __device__ void v_load(uint32_t (&vr)[VW], int chunk, int grp) const {
        if (TRANS && vzero) {
#pragma unroll
            for (int i = 0; i < VW; ++i) vr[i] = 0u;
            return;
        }
        const int blk = CB * chunk;
        const int64_t e = b * a.v_stride[0] + static_cast<int64_t>(blk) * BT * a.v_stride[1] + h * a.v_stride[2];
        const int left = rows_in(blk) + rows_in(blk + 1);
        const auto rv = make_rsrc(static_cast<const char*>(a.v) + e * static_cast<int64_t>(sizeof(TQ)),
                                  static_cast<uint32_t>(left) * rs_v);
        const uint32_t go = static_cast<uint32_t>(16 * grp * sizeof(TQ));
        uint32_t* w = vr;
        BLoad<16>::ld(w, rv, vo_v, go);
        if constexpr (VW == 8) BLoad<16>::ld(w + 4, rv, vo_v, go + 16 * rs_v);
    }
    // The chunk's v into a group's tile as 16-bit values (fp32 inputs are
    // rounded to fp16 here), then the two blocks' fragments in accumulator
    // layout (rows 4lg + j, column ln) by transposing LDS reads: in each
    // 16-lane group, lane s reads row 4lg + s/4, columns 4 (s % 4) .. + 3,
    // and the read hands lane i, slot j element i % 4 of lane 4j + i / 4.
    __device__ void v_tile(uint32_t (&vr)[VW], uint16_t (*vt)[16], f4& R0, f4& R1) const {
        use_here(vr);
        if constexpr (VW == 4) {
            *reinterpret_cast<u4*>(&vt[lane >> 1][8 * (lane & 1)]) = u4{vr[0], vr[1], vr[2], vr[3]};
        } else {
#pragma unroll
            for (int part = 0; part < 2; ++part) {
                const h4 x = {static_cast<_Float16>(__uint_as_float(vr[4 * part])),
                              static_cast<_Float16>(__uint_as_float(vr[4 * part + 1])),
                              static_cast<_Float16>(__uint_as_float(vr[4 * part + 2])),
                              static_cast<_Float16>(__uint_as_float(vr[4 * part + 3]))};
                *reinterpret_cast<h4*>(&vt[16 * part + (lane >> 2)][4 * (lane & 3)]) = x;
            }
        }
        typedef short s4 __attribute__((ext_vector_type(4)));
        const int s = lane & 15;
#pragma unroll
        for (int bk = 0; bk < CB; ++bk) {
            typedef __attribute__((address_space(3))) s4* lds_s4;
            const s4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4)(&vt[16 * bk + 4 * lg + (s >> 2)][4 * (s & 3)]));
            f4 r;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t bits = static_cast<uint16_t>(x[j]);
                r[j] = Elem<TQ>::code == KDA_DTYPE_BF16 ? __uint_as_float(bits << 16)
                                                        : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
            }
            if (bk == 0) R0 = r;
            else R1 = r;
        }
    }

    // Four values of one output row to o (TQ, [B, T, H, V] contiguous): lane
    // (ln, lg) holds row ln of block blk, columns col + 4lg .. + 3.  A buffer
    // store through a descriptor spanning the block's rows before T: the
    // hardware drops the rows past T, so every lane stores unconditionally.
    // (A branch around the store would hide the number of outstanding vector
    // memory operations from the compiler, which then waits for all of them
    // -- these stores included -- before the next chunk's v tile.)
    __device__ void store_row4(const f4& O, int blk, int64_t col) const {
        const int64_t rs = a.H * a.V;                    // token row stride, elements
        const int64_t e = (b * T + static_cast<int64_t>(blk) * BT) * rs + h * a.V;
        const auto r = make_rsrc(static_cast<TQ*>(a.o) + e,
                                 static_cast<uint32_t>(rows_in(blk) * rs * static_cast<int64_t>(sizeof(TQ))));
        const int vo = static_cast<int>((ln * rs + col + 4 * lg) * static_cast<int64_t>(sizeof(TQ)));
        if constexpr (sizeof(TQ) == 4) {
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, O), r, vo, 0, 0);
        } else if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u2, to_h4(O)), r, vo, 0, 0);
        } else {
            u2 w;
            w[0] = static_cast<uint32_t>(f32_to_bf16_bits(O[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(O[1])) << 16);
            w[1] = static_cast<uint32_t>(f32_to_bf16_bits(O[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(O[3])) << 16);
            __builtin_amdgcn_raw_buffer_store_b64(w, r, vo, 0, 0);
        }
    }

    // A 16-bit output fragment (4 columns) packed two values a word.
    static __device__ __forceinline__ u2 pack4(const f4& O) {
        if constexpr (Elem<TQ>::code == KDA_DTYPE_F16) {
            return __builtin_bit_cast(u2, to_h4(O));
        } else {
            u2 w;
            w[0] = static_cast<uint32_t>(f32_to_bf16_bits(O[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(O[1])) << 16);
            w[1] = static_cast<uint32_t>(f32_to_bf16_bits(O[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(O[3])) << 16);
            return w;
        }
    }
    // Output stores of a chunk, 16-bit TQ: per 16-row tile a lane holds 4
    // adjacent columns (lane group lg: columns 4 lg .. 4 lg + 3) of two
    // fragments x and y (CG = 1: the chunk's two blocks; CG = 2: the wave's two
    // column groups of one block).  One v_permlane16_swap per register trades
    // x of the odd lane groups for y of the even ones, after which lane group
    // lg holds 8 adjacent columns 8 (lg / 2) .. + 7 of x (lg even) or y (lg
    // odd): one 16-byte store instead of two 8-byte ones.
    static constexpr int kOutStores = sizeof(TQ) == 2 ? (CG == 1 ? 1 : CB * CG / 2) : CB * CG;
    __device__ void store_pair(const f4& x, const f4& y, __amdgpu_buffer_rsrc_t r, int vo) const {
        const u2 px = pack4(x), py = pack4(y);
        const auto s0 = __builtin_amdgcn_permlane16_swap(px[0], py[0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(px[1], py[1], false, false);
        __builtin_amdgcn_raw_buffer_store_b128(u4{s0[0], s1[0], s0[1], s1[1]}, r, vo, 0, 0);
    }
    __device__ void store_chunk(const f4 (&O)[CG][CB], int blk, int64_t colw) const {
        static_assert(CG == 1 || CG == 2, "output tiles of one or two column groups");
        if constexpr (sizeof(TQ) == 4) {
#pragma unroll
            for (int g = 0; g < CG; ++g) {
                store_row4(O[g][0], blk, colw + 16 * g);
                store_row4(O[g][1], blk + 1, colw + 16 * g);
            }
        } else {
            const int64_t rs = a.H * a.V;                    // token row stride, elements
            const int64_t e = (b * T + static_cast<int64_t>(blk) * BT) * rs + h * a.V;
            constexpr int64_t es = sizeof(TQ);
            if constexpr (CG == 1) {
                // lane group lg: row ln of block lg % 2, columns 8 (lg / 2) ..
                const auto r = make_rsrc(static_cast<TQ*>(a.o) + e,
                                         static_cast<uint32_t>((rows_in(blk) + rows_in(blk + 1)) * rs * es));
                const int vo = static_cast<int>(((ln + BT * (lg & 1)) * rs + colw + 8 * (lg >> 1)) * es);
                store_pair(O[0][0], O[0][1], r, vo);
            } else {
                // lane group lg: row ln, columns 16 (lg % 2) + 8 (lg / 2) ..
                const int vo = static_cast<int>((ln * rs + colw + 16 * (lg & 1) + 8 * (lg >> 1)) * es);
#pragma unroll
                for (int bk = 0; bk < CB; ++bk) {
                    const auto r = make_rsrc(static_cast<TQ*>(a.o) + e + BT * bk * rs,
                                             static_cast<uint32_t>(rows_in(blk + bk) * rs * es));
                    store_pair(O[0][bk], O[1][bk], r, vo);
                }
            }
        }
    }

    // TOUT: a chunk's outputs in fp32, the V columns' to o ([B, T, H, V]
    // fp32), the transition columns' to cout ([B, T, H, K]); the choice is
    // wave-uniform and taken by selecting the base, not by a branch.
    __device__ void store_fp32_chunk(const f4 (&O)[CG][CB], int blk, int64_t colw) const {
        const bool tr = vzero;
        float* base = tr ? cout : static_cast<float*>(a.o);
        const int64_t W = tr ? K : a.V, col = tr ? colw - a.V : colw;
        const int64_t rs = a.H * W;
        const int64_t e = (b * T + static_cast<int64_t>(blk) * BT) * rs + h * W;
#pragma unroll
        for (int bk = 0; bk < CB; ++bk) {
            const auto r = make_rsrc(base + e + BT * bk * rs, static_cast<uint32_t>(rows_in(blk + bk) * rs * 4));
#pragma unroll
            for (int g = 0; g < CG; ++g)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u4, O[g][bk]), r,
                                                       static_cast<int>((ln * rs + col + 16 * g + 4 * lg) * 4), 0, 0);
        }
    }

    // EPI: a chunk's outputs, rounded to TQ as the reference's o_core is and
    // held as TQ bits (two a word) over one barrier while the other consumer
    // waves' row sums of squares arrive, with the output gate's
    // pre-activations of the same entries.
    struct Pend {
        u2 o[EPI ? CG : 1][CB];
        u2 gt[EPI ? CG : 1][CB];
        int blk;
    };
    // The 16-bit TQ element j of a pair of packed words, as a float.
    static __device__ __forceinline__ float unpack16(const u2& w, int j) {
        const uint32_t bits = (w[j / 2] >> (16 * (j % 2))) & 0xffffu;
        return Elem<TQ>::code == KDA_DTYPE_BF16 ? __uint_as_float(bits << 16)
                                                : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
    }
    // The bits of x (a value of TQ) as a 16-bit element.
    static __device__ __forceinline__ uint32_t bits16(float x) {
        if constexpr (Elem<TQ>::code == KDA_DTYPE_BF16) return f32_to_bf16_bits(x);
        else return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    const void* og = nullptr;                // EPI: the output gate's pre-activations [B, T, H*V]
    int64_t og_s0 = 0, og_s1 = 0;            //      and their (batch, token) strides
    float eps = 0.f;                         //      the norm's epsilon
    float wn[EPI ? CG : 1][4];               //      the norm weight of the lane's columns

    // EPI: the pre-activations of the output gate for the lane's entries of
    // block blk (rows past T read as zero).
    __device__ u2 gate_load(int blk, int64_t col) const {
        const int64_t gs1 = og_s1;
        const int64_t e = b * og_s0 + static_cast<int64_t>(blk) * BT * gs1 + h * a.V + col;
        const auto r = make_rsrc(static_cast<const TQ*>(og) + e,
                                 static_cast<uint32_t>(rows_in(blk) * gs1 * static_cast<int64_t>(sizeof(TQ))));
        uint32_t w[2];
        BLoad<8>::ld(w, r, static_cast<uint32_t>((ln * gs1 + 4 * lg) * static_cast<int64_t>(sizeof(TQ))), 0);
        return u2{w[0], w[1]};
    }

    // EPI, after the barrier that follows a chunk: the head's row norms from
    // every consumer wave's partial sums, then y = TQ(TQ(o rstd w) sigmoid(gate))
    // (kimi_linear/kda.py:273-279, 468), stored in place of o.
    __device__ void finish(const Pend& pd, int64_t colw, int wave) const {
        const float (*parts)[BT][MAX_NC] = sm.rows.p[(pd.blk / CB) & 1];
        const float inv_v = 1.f / static_cast<float>(a.V);
#pragma unroll
        for (int bk = 0; bk < CB; ++bk) {
            const float4 pt = *reinterpret_cast<const float4*>(&parts[bk][ln][0]);
            float tot = pt.x;
            if (NC > 1) tot += pt.y;
            if (NC > 2) tot += pt.z + pt.w;
            const float rstd = rsqrtf(tot * inv_v + eps);
#pragma unroll
            for (int g = 0; g < CG; ++g) {
                f4 y;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float z = unpack16(pd.gt[g][bk], j);
                    const float n = round_elem<TQ>((unpack16(pd.o[g][bk], j) * rstd) * wn[g][j]);
                    y[j] = n * sigmoid_f(z);
                }
                store_row4(y, pd.blk + bk, colw + 16 * g);
            }
        }
        (void)wave;
    }

    // One chunk (blocks blk, blk + 1) of the chain for this wave's CG column
    // groups; the v load of the chunk one superstep later is issued into
    // vraw once its values are in LDS.  ck (or null): the chunk's checkpoint
    // for the backward, in fp32: rows [0, K) the state before it, [K, K + 32)
    // its R = V - (k * E) S.  EPI: the outputs go to
    // pd (and their row sums of squares to LDS) instead of o.
    __device__ void consume(const ChunkOps<K>& co, int blk, uint32_t (&vraw)[CG][VW],
                            uint16_t (*vt)[16], f4 (&S)[CG][KT], int64_t colw, float* ck, Pend& pd,
                            int wave) const {
        f4 R[CG][CB];
#pragma unroll
        for (int g = 0; g < CG; ++g) {
            v_tile(vraw[g], vt, R[g][0], R[g][1]);
            v_load(vraw[g], blk / CB + NCH, g);
        }
        if constexpr (RANGE) {
            // the wave's largest |sigma S| and |V| (R holds V here), then
            // sigma / 2^k when sigma times it passes 2^10
            float ms = 0.f, mv = 0.f;
#pragma unroll
            for (int g = 0; g < CG; ++g) {
#pragma unroll
                for (int t = 0; t < KT; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j) ms = fmaxf(ms, fabsf(S[g][t][j]));
#pragma unroll
                for (int bk = 0; bk < CB; ++bk)
#pragma unroll
                    for (int j = 0; j < 4; ++j) mv = fmaxf(mv, fabsf(R[g][bk][j]));
            }
            const float m = wave_max(fmaxf(ms, mv * sig));
            if (m > kRangeMax) {
                // m = 2^e x 1.f: dividing by 2^(e - 9) leaves it under 2^10
                const int k = static_cast<int>((__float_as_uint(m) >> 23) & 0xffu) - 127 - 9;
                const float f = __uint_as_float(static_cast<uint32_t>(127 - k) << 23);
#pragma unroll
                for (int g = 0; g < CG; ++g)
#pragma unroll
                    for (int t = 0; t < KT; ++t) S[g][t] *= f;
                sig *= f;
                isig = 1.f / sig;
            }
#pragma unroll
            for (int g = 0; g < CG; ++g) {
                R[g][0] *= sig;
                R[g][1] *= sig;
            }
        }
        const int64_t V = a.V;
        if constexpr (kFlatRec) {
            {
                // fp16 in accumulator-order tiles (half_tile_offset): slot j
                // of tile (t, column group) is 64 consecutive halves, the
                // values the products above take as their fp16 state
                // (the tile offsets are wave-uniform: scalar offsets of a
                // buffer store, so no per-tile address is kept in registers)
                const auto rs = make_rsrc(ck, ck ? static_cast<uint32_t>(K * V * 2) : 0u);
                const int lo = 2 * (16 * lg + ln);
#pragma unroll
                for (int g = 0; g < CG; ++g)
#pragma unroll
                    for (int t = 0; t < KT; ++t)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            __builtin_amdgcn_raw_buffer_store_b16(
                                __builtin_bit_cast(uint16_t, static_cast<_Float16>(S[g][t][j])), rs, lo,
                                static_cast<int>(2 * (half_tile_offset(16 * t, colw + 16 * g, V) + 64 * j)), 2);
            }
        } else if (ck) {
            {
#pragma unroll
                for (int g = 0; g < CG; ++g)
#pragma unroll
                    for (int t = 0; t < KT; ++t)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            __builtin_nontemporal_store(RANGE ? S[g][t][j] * isig : S[g][t][j],
                                                        &ck[(4 * lg + 16 * t + j) * V + colw + 16 * g + ln]);
            }
        }
        float* rp = ck ? ck + static_cast<int64_t>(K) * V : nullptr;
        // R rows through one buffer resource: the lane's part of the offset in
        // a vector register, the row and column group's (wave-uniform) part
        // in the scalar offset -- no 64-bit address per store kept in
        // registers.  fp16 activations: R in fp16 (the single fp16 operand the
        // solve below takes), row-major halves in the first half of its rows.
        const auto rr = make_rsrc(rp, rp ? static_cast<uint32_t>(CB * BT * V * 4) : 0u);
        const int rlo = static_cast<int>((4 * lg * V + ln) * 4);
        auto r_store = [&](float x, int row, int g) {
            if constexpr (Elem<TQ>::code == KDA_DTYPE_F16)
                __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, static_cast<_Float16>(x)), rr,
                                                      rlo / 2, static_cast<int>((row * V + colw + 16 * g) * 2), 2);
            else
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), rr, rlo,
                                                      static_cast<int>((row * V + colw + 16 * g) * 4), 2);
        };
        // Z_b = (k * E)_b S; the outputs transposed, O_b^T = S^T (q * E)_b^T:
        // the same fragments as A and B operands the other way round, so that
        // a lane holds four adjacent output columns of one row.  Block 1's
        // operands hold decays from its own start, so its products take
        // Diag(E[15]) S, block 0's decay applied to the state rows.  The state
        // enters as single fp16 operands, rounded once per chunk.
        f4 Z[CG][CB], O[CG][CB];
#pragma unroll
        for (int g = 0; g < CG; ++g)
#pragma unroll
            for (int bk = 0; bk < CB; ++bk) Z[g][bk] = O[g][bk] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < KU; ++u) {
            const int o = ln * KR + 32 * u + 8 * lg;
            const h8 k0 = *reinterpret_cast<const h8*>(&co.KE[0][0][0] + o);
            const h8 k1 = *reinterpret_cast<const h8*>(&co.KE[1][0][0] + o);
            const h8 q0 = *reinterpret_cast<const h8*>(&co.QE[0][0][0] + o);
            const h8 q1 = *reinterpret_cast<const h8*>(&co.QE[1][0][0] + o);
            // block 0's decay on the state rows of tiles 2u and 2u + 1
            const float4 da = *reinterpret_cast<const float4*>(&co.d0[32 * u + 4 * lg]);
            const float4 db = *reinterpret_cast<const float4*>(&co.d0[32 * u + 16 + 4 * lg]);
            const f4 fa = {da.x, da.y, da.z, da.w}, fb = {db.x, db.y, db.z, db.w};
#pragma unroll
            for (int g = 0; g < CG; ++g) {
                const h8 sh = cat(to_h4(S[g][2 * u]), to_h4(S[g][2 * u + 1]));
                const h8 sd = cat(to_h4(S[g][2 * u] * fa), to_h4(S[g][2 * u + 1] * fb));
                Z[g][0] = mfma16x16x32(k0, sh, Z[g][0]);
                Z[g][1] = mfma16x16x32(k1, sd, Z[g][1]);
                O[g][0] = mfma16x16x32(sh, q0, O[g][0]);
                O[g][1] = mfma16x16x32(sd, q1, O[g][1]);
            }
        }
        // P_0 = M_00 (V_0 - Z_0);  P_1 = M_11 (V_1 - Z_1 - G_10 P_0): M (hi + lo)
        // times a single fp16 R is one K = 32 product [M_hi | M_lo] [R ; R]
        const h8 m0 = cat(frag16(&co.MH[0][0][0], RP, ln, lg), frag16(&co.ML[0][0][0], RP, ln, lg));
        const h8 m1 = cat(frag16(&co.MH[1][0][0], RP, ln, lg), frag16(&co.ML[1][0][0], RP, ln, lg));
        const h4 gh = frag16(&co.GH[0][0], RP, ln, lg), gl = frag16(&co.GL[0][0], RP, ln, lg);
        const h4 a00 = frag16(&co.AM[0][0][0], RP, ln, lg);
        const h8 a1 = cat(frag16(&co.A10[0][0], RP, ln, lg), frag16(&co.AM[1][0][0], RP, ln, lg));
        h8 ph[CG], pl[CG];
#pragma unroll
        for (int g = 0; g < CG; ++g) {
            R[g][0] -= Z[g][0];
            R[g][1] -= Z[g][1];
            if (kFlatRec || rp) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    r_store(RANGE ? R[g][0][j] * isig : R[g][0][j], j, g);
                    r_store(RANGE ? R[g][1][j] * isig : R[g][1][j], 16 + j, g);
                }
            }
            const h4 r0 = to_h4(R[g][0]);
            const f4 P0 = mfma16x16x32(m0, cat(r0, r0), f4{0.f, 0.f, 0.f, 0.f});
            const Split4 p0(P0);
            R[g][1] = mm4(gh, gl, p0.hi, p0.lo, R[g][1]);
            const h4 r1 = to_h4(R[g][1]);
            const f4 P1 = mfma16x16x32(m1, cat(r1, r1), f4{0.f, 0.f, 0.f, 0.f});
            const Split4 p1(P1);
            // O^T = scale S^T (q * E)^T + P^T A^T: P^T's A-operand layout is
            // P's accumulator layout, A^T's B-operand layout is A's A-operand
            // layout
            O[g][0] *= scale;
            O[g][1] *= scale;
            O[g][0] = mfma16x16x32(cat(p0.hi, p0.lo), cat(a00, a00), O[g][0]);
            O[g][1] = mfma16x16x32(cat(p0.hi, p1.hi), a1, O[g][1]);
            O[g][1] = mfma16x16x32(cat(p0.lo, p1.lo), a1, O[g][1]);
            if constexpr (RANGE) {
                // both terms came from the sigma-scaled state and R
                O[g][0] *= isig;
                O[g][1] *= isig;
            }
            ph[g] = cat(p0.hi, p1.hi);
            pl[g] = cat(p0.lo, p1.lo);
        }
        if constexpr (EPI) {
            // outputs rounded to TQ (the reference's o_core), their row sums of
            // squares over this wave's columns to LDS, the values held for the
            // norm
            const int par = (blk / CB) & 1;
#pragma unroll
            for (int bk = 0; bk < CB; ++bk) {
                float ss = 0.f;
#pragma unroll
                for (int g = 0; g < CG; ++g) {
                    uint32_t ob[4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float x = round_elem<TQ>(O[g][bk][j]);
                        ob[j] = bits16(x);
                        ss = fmaf(x, x, ss);
                    }
                    pd.o[g][bk] = u2{ob[0] | (ob[1] << 16), ob[2] | (ob[3] << 16)};
                    pd.gt[g][bk] = gate_load(blk + bk, colw + 16 * g);
                }
                ss = lanegroup4_sum(ss);
                if (lg == 0) sm.rows.p[par][bk][ln][wave] = ss;
            }
            pd.blk = blk;
        } else if constexpr (TOUT) {
            store_fp32_chunk(O, blk, colw);
        } else if constexpr (!TRANS) {
            store_chunk(O, blk, colw);
        }
        // S <- E[31] S + F^T P over both blocks: the k-major line of channel
        // 16t + ln gives tokens 4lg..4lg+3 of block 0 then of block 1, the
        // order of cat(P_0, P_1)
#pragma unroll
        for (int t = 0; t < KT; ++t) {
            const int piece = 8 * (lg ^ kh_swz(16 * t + ln));
            const float4 e = *reinterpret_cast<const float4*>(&co.echunk[16 * t + 4 * lg]);
            const h8 kf = *reinterpret_cast<const h8*>(&co.KH[16 * t + ln][piece]);
#pragma unroll
            for (int g = 0; g < CG; ++g) {
                S[g][t][0] *= e.x; S[g][t][1] *= e.y; S[g][t][2] *= e.z; S[g][t][3] *= e.w;
                S[g][t] = mfma16x16x32(kf, ph[g], S[g][t]);
                S[g][t] = mfma16x16x32(kf, pl[g], S[g][t]);
            }
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
// ckpt: CKPT, the chunk records; TOUT, the transition columns' outputs.
template <int K, int NC, typename TQ, bool GATED, int CG = 1, bool EPI = false, bool TRANS = false, bool CKPT = false,
          bool TOUT = false>
__global__ __launch_bounds__(64 * (NC + NB)) void chunkwise_kernel(const kda_fwd_args a, float* ckpt,
                                                                   const kda_gate_args gate,
                                                                   const kda_out_epilogue epi) {
    static_assert(!TOUT || TRANS, "fp32 outputs belong to the transition pass");
    using KN = Kern<K, NC, TQ, GATED, CG, EPI, TRANS, TOUT, CKPT>;
    constexpr int KT = KN::KT, VT = KN::VT, CH = KN::CH;
    static_assert(K % 32 == 0 && K <= 128, "chunkwise supports K in {32, 64, 128}");
    __shared__ Smem<K, CG, EPI> sm;
    KN kn(a, sm);
    if constexpr (EPI) {
        kn.og = epi.gate;
        kn.og_s0 = epi.gate_stride[0];
        kn.og_s1 = epi.gate_stride[1];
        kn.eps = epi.eps;
    }

    const int64_t H = a.H, V = a.V;
    const int64_t VS = V + (TRANS ? K : 0);             // state columns
    const int nvt = static_cast<int>(VS / VT);
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
    kn.nblk = nblk;
    if constexpr (CKPT) {
        if (ckpt != nullptr && vt == 0) kn.ckm = ckpt + (kn.b * H + kn.h) * ncc * ckpt_record(K, V);
    }
    if constexpr (TOUT) kn.cout = ckpt;
    const int nss = (ncc + NCH - 1) / NCH;               // supersteps

    const bool consumer = wave < NC;
    // consumer state: S[g][t][j] = S[16t + 4lg + j][colw + 16g + ln]
    const int64_t col0 = static_cast<int64_t>(vt) * VT;
    const int64_t colw = col0 + 16 * CG * (consumer ? wave : 0);
    const int64_t sbase = (kn.b * H + kn.h) * static_cast<int64_t>(K) * VS;
    {
        const uint32_t eq = static_cast<uint32_t>(sizeof(TQ));
        kn.rs_q = static_cast<uint32_t>(a.q_stride[1]) * eq;
        kn.rs_k = static_cast<uint32_t>(a.k_stride[1]) * eq;
        kn.rs_v = static_cast<uint32_t>(a.v_stride[1]) * eq;
        const uint32_t eg = static_cast<uint32_t>(sizeof(typename KN::TG));
        kn.rs_g = static_cast<uint32_t>(a.g_stride[1]) * eg;
        kn.rs_b = static_cast<uint32_t>(a.beta_stride[1]) * eg;
        const uint32_t c0 = static_cast<uint32_t>(CH * kn.cq), r0 = static_cast<uint32_t>(HR * kn.hf);
        kn.vo_q = r0 * kn.rs_q + c0 * eq;
        kn.vo_k = r0 * kn.rs_k + c0 * eq;
        kn.vo_g = r0 * kn.rs_g + c0 * eg;
        kn.vo_b = static_cast<uint32_t>(4 * kn.lg) * kn.rs_b;
        // v tile loads: 16-bit inputs row lane / 2, columns 8 (lane % 2); fp32
        // row lane / 4, columns 4 (lane % 4), of this wave's 16 columns
        const uint32_t vrow = sizeof(TQ) == 2 ? (kn.lane >> 1) : (kn.lane >> 2);
        const uint32_t vcol = sizeof(TQ) == 2 ? 8 * (kn.lane & 1) : 4 * (kn.lane & 3);
        kn.vo_v = vrow * kn.rs_v + static_cast<uint32_t>(colw + vcol) * eq;
    }

    if (consumer) {
        f4 S[CG][KT];
        if constexpr (TRANS) {
            // the chain's own state from zero; the transition columns from the identity
            kn.vzero = colw >= V;
#pragma unroll
            for (int g = 0; g < CG; ++g)
#pragma unroll
                for (int t = 0; t < KT; ++t)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        S[g][t][j] = kn.vzero && 16 * t + 4 * kn.lg + j == colw - V + 16 * g + kn.ln ? 1.f : 0.f;
        } else {
#pragma unroll
            for (int g = 0; g < CG; ++g)
                load_state<KT>(S[g], a.state_in, a.state_in_dtype, sbase + (4 * kn.lg) * V + colw + 16 * g + kn.ln, V);
        }
        uint32_t vr[NCH][CG][KN::VW];
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
#pragma unroll
            for (int g = 0; g < CG; ++g) kn.v_load(vr[j][g], j, g);
            // a chunk's v loads are followed by its output stores in the loop
            // below: stores that write nothing (an empty buffer range) stand in
            // for them here, so that the loop is entered with the pattern of
            // outstanding vector memory operations it repeats.  The compiler's
            // count at the loop head is then exact; with the entry path's
            // smaller count each chunk's wait for its v tile also waited for
            // the output stores of the chunks before it.
            if constexpr (!EPI && (!CKPT || KN::kFlatRec) && (!TRANS || TOUT)) {
                // (distinct offsets: identical stores would be merged away;
                // flat records: the chunk's state and R stores as well)
                constexpr int ns = TOUT ? CB * CG : KN::kOutStores + (CKPT ? CG * (KN::KT + CB) * 4 : 0);
                const auto none = make_rsrc(a.o, 0u);
#pragma unroll
                for (int i = 0; i < ns; ++i)
                    __builtin_amdgcn_raw_buffer_store_b64(u2{0u, 0u}, none, 0, 8 * (ns * j + i), 0);
            }
            if constexpr (EPI) {
                // a chunk's output-gate loads follow its v loads in the loop
                constexpr int ng = CB * CG;
                const auto none = make_rsrc(a.o, 0u);
#pragma unroll
                for (int i = 0; i < ng; ++i)
                    __builtin_amdgcn_raw_buffer_store_b64(u2{0u, 0u}, none, 0, 8 * (ng * j + i), 0);
            }
        }
        if constexpr (EPI) {
            // and the superstep's output stores (finish) end the loop body
            constexpr int nf = NCH * CB * CG;
            const auto none = make_rsrc(a.o, 0u);
#pragma unroll
            for (int i = 0; i < nf; ++i)
                __builtin_amdgcn_raw_buffer_store_b64(u2{0u, 0u}, none, 0, 8 * (NCH * CB * CG + i), 0);
        }
        uint16_t (*vt)[16] = sm.vt[consumer ? wave : 0];
        typename KN::Pend pd[NCH];
        if constexpr (EPI) {
#pragma unroll
            for (int g = 0; g < CG; ++g)
#pragma unroll
                for (int j = 0; j < 4; ++j) kn.wn[g][j] = epi.weight[kn.h * V + colw + 16 * g + 4 * kn.lg + j];
        }
        // Superstep -1 (the producers build superstep 0): only the solve of
        // block `wave` of superstep 0.  Then per superstep, first half: its
        // chunks one after the other; second half (after the producers'
        // first): the chunks' outputs (EPI: every wave's row sums are in LDS
        // now) and the solve of block `wave` of the next superstep.  Both
        // chunks run in every superstep -- a chunk past T (T / 32 odd) is
        // built by the producers from zero rows and leaves the state as it is,
        // its outputs fall past T and are dropped -- so the loop body has no
        // branch around a chunk: the compiler then counts the outstanding
        // vector memory operations exactly and waits only for the v tile a
        // chunk needs, not for the previous chunk's output stores.
        auto solve_next = [&](int s) {
            if constexpr (KN::kConsumerSolve) {
                const int nb = NB * (s + 1) + wave;
                // flat records: also past the last superstep (its N stores
                // then have an empty range, its M goes to an unused slot), so
                // the loop body has no branch around them
                if ((CKPT && KN::kFlatRec) || s + 1 < nss) {
                    ChunkOps<K>& nx = sm.set[(s + 1) & 1][wave / CB];
                    kn.solve(wave, nb, nx.MH[wave % CB], nx.ML[wave % CB]);
                }
            }
        };
        __syncthreads();
        solve_next(-1);
        __syncthreads();
        for (int s = 0; s < nss; ++s) {
#pragma unroll
            for (int cj = 0; cj < NCH; ++cj) {
                const int cc = NCH * s + cj;
                // the checkpoint of chunk cc, for the backward
                float* ck = CKPT && ckpt && cc < ncc ? ckpt + ((kn.b * H + kn.h) * ncc + cc) * ckpt_record(K, V)
                                                     : nullptr;
                kn.consume(sm.set[s & 1][cj], NB * s + CB * cj, vr[cj], vt, S, colw, ck, pd[cj], wave);
            }
            __syncthreads();
            if constexpr (EPI) {
#pragma unroll
                for (int cj = 0; cj < NCH; ++cj)
                    kn.finish(pd[cj], colw, wave);     // a chunk past T: rows dropped by the store's range
            }
            solve_next(s);
            __syncthreads();
        }
        // a null state_out (the output pass of a split long sequence) keeps no final state
        if (a.state_out != nullptr) {
            if constexpr (KN::RANGE) {
#pragma unroll
                for (int g = 0; g < CG; ++g)
#pragma unroll
                    for (int t = 0; t < KT; ++t) S[g][t] *= kn.isig;
            }
#pragma unroll
            for (int g = 0; g < CG; ++g)
                store_state<KT>(S[g], a.state_out, a.state_out_dtype, sbase + (4 * kn.lg) * VS + colw + 16 * g + kn.ln,
                                VS);
        }
    } else {
        const int p = wave - NC;
        if constexpr (GATED) {
            const int64_t ch = kn.h * K + CH * kn.cq;
#pragma unroll
            for (int c = 0; c < CH; ++c) {
                kn.gcoef[c] = expf(gate.a_log[ch + c]);
                kn.gbias[c] = gate.dt_bias[ch + c] * kLog2e;
            }
        }
        typename KN::Raw raw;
        typename KN::Work w;
        kn.load_raw(raw, p);
        if constexpr (KN::kEarlyDecay) kn.decays(raw, w);
        for (int s = -1; s < nss; ++s) {
            // every block of the supersteps, a padded chunk past T included
            const int blk = NB * (s + 1) + p;
            ChunkOps<K>& co = sm.set[(s + 1) & 1][p / CB];
            if (s + 1 < nss) kn.phase1(raw, w, p, co, blk + NB);
            __syncthreads();
            if (s + 1 < nss) kn.phase2(p, blk, co);
            __syncthreads();
        }
    }
}

template <int K, int NC, typename TQ, bool GATED, int CG = 1, bool EPI = false, bool TRANS = false, bool CKPT = false,
          bool TOUT = false>
int launch_knq(const kda_fwd_args& a, hipStream_t stream, float* ckpt, const kda_gate_args& gate,
               const kda_out_epilogue& epi = kda_out_epilogue{}) {
    const int64_t blocks = a.B * a.H * ((a.V + (TRANS ? K : 0)) / (16 * NC * CG));
    hipLaunchKernelGGL((chunkwise_kernel<K, NC, TQ, GATED, CG, EPI, TRANS, CKPT, TOUT>), dim3(static_cast<unsigned>(blocks)),
                       dim3(64 * (NC + NB)), 0, stream, a, ckpt, gate, epi);
    return hipGetLastError() == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}

// The first pass of a split long sequence: 64-column tiles over the V state
// columns and the K transition columns (128-column tiles when they would
// outnumber the CUs).
template <int K, typename TQ>
int launch_trans(const kda_fwd_args& a, hipStream_t stream, float* cout) {
    const kda_gate_args none{nullptr, nullptr};
    const bool wide = a.B * a.H * ((a.V + K) / 64) > 256 && (a.V + K) % 128 == 0;
    if (cout != nullptr) {
        if (wide) return launch_knq<K, 4, TQ, false, 2, false, true, false, true>(a, stream, cout, none);
        return launch_knq<K, 4, TQ, false, 1, false, true, false, true>(a, stream, cout, none);
    }
    if (wide) return launch_knq<K, 4, TQ, false, 2, false, true>(a, stream, nullptr, none);
    return launch_knq<K, 4, TQ, false, 1, false, true>(a, stream, nullptr, none);
}

// The fused output epilogue: one workgroup per (b, h), 4 consumer waves of
// V / 64 column groups.
template <int K, typename TQ, bool GATED>
int launch_epi(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args& gate, const kda_out_epilogue& epi) {
    if (a.V == 64) return launch_knq<K, 4, TQ, GATED, 1, true>(a, stream, nullptr, gate, epi);
    if (a.V == 128) return launch_knq<K, 4, TQ, GATED, 2, true>(a, stream, nullptr, gate, epi);
    return KDA_ERR_UNSUPPORTED;
}
template <typename TQ, bool GATED>
int launch_epi_k(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args& gate, const kda_out_epilogue& epi) {
    if (a.K == 64) return launch_epi<64, TQ, GATED>(a, stream, gate, epi);
    if (a.K == 128) return launch_epi<128, TQ, GATED>(a, stream, gate, epi);
    return KDA_ERR_UNSUPPORTED;
}

// Columns per workgroup (16, 32, 64 or 128): the fewest rounds of
// workgroups on the 256 CUs, see the cost below.
template <int K, typename TQ, bool GATED>
int launch_kq(const kda_fwd_args& a, hipStream_t stream, float* ckpt, const kda_gate_args& gate) {
    constexpr int64_t kCus = 256;
    const int64_t heads = a.B * a.H;
    // the checkpointing forward is its own instantiation: the record stores
    // cost registers the plain forward does not pay for
    auto go = [&](auto nc, auto cg) {
        constexpr int NC = decltype(nc)::value, CG = decltype(cg)::value;
        if constexpr (!GATED) {
            if (ckpt != nullptr) return launch_knq<K, NC, TQ, GATED, CG, false, false, true>(a, stream, ckpt, gate);
        }
        return launch_knq<K, NC, TQ, GATED, CG>(a, stream, nullptr, gate);
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    // A superstep takes about as long in a 16-, 32- or 64-column workgroup
    // (the producers' chain sets it) and ~10 % longer in a 128-column one
    // (consumer waves of two 16-column groups; 16-bit inputs only, the fp32
    // instantiation serves checkpoints), so the time is about rounds of
    // workgroups x that factor: pick the cheapest (measured at T=2048 H=16
    // d=128, gated, one round against 1.5-2: B=3 178 against 348 us, B=6 182
    // against 350 us; B=16 220 us in 128-column workgroups against 368 us in
    // two rounds of 64-column ones).  On a tie the wider tile wins: the
    // 64-column one's four consumer waves take the inverse of (I + L) off the
    // producers' chain, which fewer consumer waves leave there (B=3 and B=4:
    // 149 against 157-158 us plain, 174 against 180 us gated in 32-column
    // workgroups; B=1 and B=2 equal to 16-column ones).
    const int64_t w1 = a.V % 16 == 0 ? heads * (a.V / 16) : 0;
    const int64_t w2 = a.V % 32 == 0 ? heads * (a.V / 32) : 0;
    const int64_t w4 = a.V % 64 == 0 ? heads * (a.V / 64) : 0;
    const int64_t w8 = sizeof(TQ) == 2 && a.V % 128 == 0 ? heads * (a.V / 128) : 0;
    // cost in tenths of a one-round superstep
    auto cost = [&](int64_t wgs, int64_t tenths) { return ((wgs + kCus - 1) / kCus) * tenths; };
    int best = 1;
    int64_t best_cost = cost(w1, 10);
    if (w2 > 0 && cost(w2, 10) <= best_cost) best = 2, best_cost = cost(w2, 10);
    if (w4 > 0 && cost(w4, 10) <= best_cost) best = 4, best_cost = cost(w4, 10);
    if (w8 > 0 && cost(w8, 11) < best_cost) best = 8, best_cost = cost(w8, 11);
    if constexpr (sizeof(TQ) == 2) {
        if (best == 8) return go(I4{}, I2{});
    }
    if (best == 4) return go(I4{}, I1{});
    if (best == 2) return go(I2{}, I1{});
    return go(I1{}, I1{});
}

template <int K, bool GATED>
int launch_k(const kda_fwd_args& a, hipStream_t stream, float* ckpt, const kda_gate_args& gate) {
    switch (a.qkv_dtype) {
        case KDA_DTYPE_F16: return launch_kq<K, _Float16, GATED>(a, stream, ckpt, gate);
        case KDA_DTYPE_BF16: return launch_kq<K, bf16_t, GATED>(a, stream, ckpt, gate);
        case KDA_DTYPE_F32:
            // fp32 activations take the token recurrence (gated or not), with
            // fp32 checkpoints too (kda_ckpt_fp32.hip): no fp32 pipeline
            return KDA_ERR_BAD_DTYPE;
        default: return KDA_ERR_BAD_DTYPE;
    }
}

template <bool GATED>
int launch_gated(const kda_fwd_args& a, hipStream_t stream, float* ckpt, const kda_gate_args& gate) {
    switch (a.K) {
        case 32: return launch_k<32, GATED>(a, stream, ckpt, gate);
        case 64: return launch_k<64, GATED>(a, stream, ckpt, gate);
        case 128: return launch_k<128, GATED>(a, stream, ckpt, gate);
        default: return KDA_ERR_UNSUPPORTED;
    }
}

}  // namespace

bool chunkwise_supported(int64_t K, int64_t V) {
    return (K == 32 || K == 64 || K == 128) && V % 16 == 0;
}

int chunkwise_check(const kda_fwd_args& a, bool gated) {
    // the pipeline reads gates in fp32 (the wrapper converts other dtypes);
    // a gated call's gk and logits come in the dtype of q, k and v
    if (!gated && (a.g_dtype != KDA_DTYPE_F32 || a.beta_dtype != KDA_DTYPE_F32)) return KDA_ERR_BAD_DTYPE;
    if (gated && a.qkv_dtype != KDA_DTYPE_F32 && (a.g_dtype != a.qkv_dtype || a.beta_dtype != a.qkv_dtype))
        return KDA_ERR_BAD_DTYPE;
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
    return KDA_OK;
}

bool chunkwise_fused_supported(const kda_fwd_args& a) {
    return (a.K == 64 || a.K == 128) && (a.V == 64 || a.V == 128) &&
           (a.qkv_dtype == KDA_DTYPE_F16 || a.qkv_dtype == KDA_DTYPE_BF16);
}

int chunkwise_fused_launch(const kda_fwd_args& a, hipStream_t stream, const kda_gate_args* gate,
                           const kda_out_epilogue& epi) {
    const int st = chunkwise_check(a, gate != nullptr);
    if (st != KDA_OK) return st;
    if (!chunkwise_fused_supported(a)) return KDA_ERR_UNSUPPORTED;
    // the gate rows are read through one descriptor per block: rows may not overlap
    if (epi.gate_stride[1] < a.H * a.V || epi.gate_stride[0] < 0 ||
        (BT + 1) * epi.gate_stride[1] * 2 >= (int64_t(1) << 31))
        return KDA_ERR_UNSUPPORTED;
    const kda_gate_args g = gate ? *gate : kda_gate_args{nullptr, nullptr};
    if (a.qkv_dtype == KDA_DTYPE_F16)
        return gate ? launch_epi_k<_Float16, true>(a, stream, g, epi) : launch_epi_k<_Float16, false>(a, stream, g, epi);
    return gate ? launch_epi_k<bf16_t, true>(a, stream, g, epi) : launch_epi_k<bf16_t, false>(a, stream, g, epi);
}

bool chunkwise_trans_supported(const kda_fwd_args& a) {
    return (a.K == 64 || a.K == 128) && a.V % 64 == 0 &&
           (a.qkv_dtype == KDA_DTYPE_F16 || a.qkv_dtype == KDA_DTYPE_BF16);
}

int chunkwise_trans_launch(const kda_fwd_args& a, hipStream_t stream, float* cout) {
    const int st = chunkwise_check(a, false);
    if (st != KDA_OK) return st;
    if (!chunkwise_trans_supported(a)) return KDA_ERR_UNSUPPORTED;
    if (a.qkv_dtype == KDA_DTYPE_F16)
        return a.K == 64 ? launch_trans<64, _Float16>(a, stream, cout) : launch_trans<128, _Float16>(a, stream, cout);
    return a.K == 64 ? launch_trans<64, bf16_t>(a, stream, cout) : launch_trans<128, bf16_t>(a, stream, cout);
}

int chunkwise_launch(const kda_fwd_args& a, hipStream_t stream, float* ckpt, const kda_gate_args* gate) {
    const int st = chunkwise_check(a, gate != nullptr);
    if (st != KDA_OK) return st;
    if (gate != nullptr) {
        if (ckpt != nullptr) return KDA_ERR_UNSUPPORTED;   // the backward takes g and beta
        return launch_gated<true>(a, stream, nullptr, *gate);
    }
    return launch_gated<false>(a, stream, ckpt, kda_gate_args{nullptr, nullptr});
}

}  // namespace kda
