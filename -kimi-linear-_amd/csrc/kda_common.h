// Shared device helpers for the gfx950 KDA kernels: element loads/stores for
// the three boundary dtypes, fp16 hi/lo operand splitting and MFMA vector types.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kda_hip.h"

namespace kda {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr float kFp16MaxSafe = 60000.0f;   // kimi_linear/fp16.py:97

// ---- scalar element access for a runtime dtype code ----------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float load_elem(const void* p, int64_t i, int dtype) {
    switch (dtype) {
        case KDA_DTYPE_F16: return static_cast<float>(static_cast<const _Float16*>(p)[i]);
        case KDA_DTYPE_BF16: return bf16_bits_to_f32(static_cast<const uint16_t*>(p)[i]);
        default: return static_cast<const float*>(p)[i];
    }
}

// Branch-free element load for a runtime dtype: one 32-bit load of the
// aligned word that holds element i (a 2-byte element sits in its low or high
// half), issued the same way for every dtype so that several such loads are
// in flight together; decode_elem converts it once the data is needed.  The
// word never crosses a 4-byte boundary, so it lies in the element's page.
struct RawElem {
    uint32_t word;
    uint32_t shift;   // 0 or 16 for 2-byte elements
};
__device__ __forceinline__ RawElem load_raw_elem(const void* p, int64_t i, int dtype) {
    const int64_t es = dtype == KDA_DTYPE_F32 ? 4 : 2;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(p) + static_cast<uintptr_t>(i * es);
    RawElem r;
    r.word = *reinterpret_cast<const uint32_t*>(addr & ~static_cast<uintptr_t>(3));
    r.shift = static_cast<uint32_t>(addr & 2) * 8u;
    return r;
}
__device__ __forceinline__ float decode_elem(const RawElem& r, int dtype) {
    if (dtype == KDA_DTYPE_F32) return __uint_as_float(r.word);
    const uint16_t half = static_cast<uint16_t>(r.word >> r.shift);
    if (dtype == KDA_DTYPE_F16) return static_cast<float>(__builtin_bit_cast(_Float16, half));
    return bf16_bits_to_f32(half);
}

__device__ __forceinline__ void store_elem(void* p, int64_t i, int dtype, float x) {
    switch (dtype) {
        case KDA_DTYPE_F16: static_cast<_Float16*>(p)[i] = static_cast<_Float16>(x); break;
        case KDA_DTYPE_BF16: static_cast<uint16_t*>(p)[i] = f32_to_bf16_bits(x); break;
        default: static_cast<float*>(p)[i] = x; break;
    }
}

// ---- compile-time typed access (hot loops) --------------------------------
struct bf16_t { uint16_t bits; };

template <typename T> struct Elem;
template <> struct Elem<float> {
    static __device__ __forceinline__ float ld(const float* p) { return *p; }
    static __device__ __forceinline__ void st(float* p, float x) { *p = x; }
    static constexpr int code = KDA_DTYPE_F32;
};
template <> struct Elem<_Float16> {
    static __device__ __forceinline__ float ld(const _Float16* p) { return static_cast<float>(*p); }
    static __device__ __forceinline__ void st(_Float16* p, float x) { *p = static_cast<_Float16>(x); }
    static constexpr int code = KDA_DTYPE_F16;
};
template <> struct Elem<bf16_t> {
    static __device__ __forceinline__ float ld(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
    static __device__ __forceinline__ void st(bf16_t* p, float x) { p->bits = f32_to_bf16_bits(x); }
    static constexpr int code = KDA_DTYPE_BF16;
};

// x rounded to T and back: the value a T tensor would hold.
template <typename T>
__device__ __forceinline__ float round_elem(float x) {
    if constexpr (Elem<T>::code == KDA_DTYPE_F32) return x;
    else if constexpr (Elem<T>::code == KDA_DTYPE_F16) return static_cast<float>(static_cast<_Float16>(x));
    else return bf16_bits_to_f32(f32_to_bf16_bits(x));
}

// Clamp to +-60000 keeping NaN (the comparisons are false for NaN).
__device__ __forceinline__ float clamp_fp16_safe(float x) {
    return x > kFp16MaxSafe ? kFp16MaxSafe : (x < -kFp16MaxSafe ? -kFp16MaxSafe : x);
}

// exp(x) through the hardware base-2 exponential.
__device__ __forceinline__ float fast_exp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// The layer's forget gate as a decay factor (kimi_linear/kda.py:460):
// a = exp(g), g = -coef softplus(z), coef = exp(A_log), z = gk + dt_bias,
// taken in base 2 from zl = z log2(e) (callers form it as one fma of gk with
// the per-channel log2(e) and dt_bias log2(e)).  With t = 2^-|zl| in (0, 1]:
//   a = 2^(-coef s),   s = softplus(z) log2(e) = max(zl, 0) + log2(1 + t).
// u = 1 + t is rounded; its rounding error t - (u - 1) (exact, as u - 1 is)
// goes back in as the first-order term of log2(1 + t), so s keeps its e^z
// behaviour for z << 0 to about an ulp without a division.  For z > 20,
// t < 2^-28 vanishes against 1 and s = zl: torch's softplus threshold.
constexpr float kLog2e = 1.4426950408889634f;
__device__ __forceinline__ float gate_decay(float zl, float coef) {
    const float t = __builtin_amdgcn_exp2f(-fabsf(zl));
    const float u = 1.f + t;
    const float e = t - (u - 1.f);
    const float s = fmaxf(zl, 0.f) + fmaf(e, kLog2e, __builtin_amdgcn_logf(u));
    return __builtin_amdgcn_exp2f(-coef * s);
}

// beta from its logit (kimi_linear/kda.py:452); the reciprocal to about an ulp.
__device__ __forceinline__ float sigmoid_f(float x) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

// log(1 + x) for x in [0, 1] to about an ulp: with u = 1 + x rounded,
// log(u) x / (u - 1) cancels the rounding of u (u == 1 when x is below half an
// ulp of 1, and then log(1 + x) = x to fp32 precision).
__device__ __forceinline__ float log1p_unit(float x) {
    const float u = 1.f + x;
    return u == 1.f ? x : __logf(u) * (x / (u - 1.f));
}

// softplus with torch's default threshold: z for z > 20, else
// log(1 + e^z) = max(z, 0) + log1p(e^-|z|), which keeps its e^z behaviour for
// z << 0 (log(1 + e^z) in fp32 rounds to 0 below z ~ -17)
__device__ __forceinline__ float softplus(float z) {
    return z > 20.f ? z : fmaxf(z, 0.f) + log1p_unit(__expf(-fabsf(z)));
}

// fp16 hi/lo split: x ~= hi + lo with |x - hi - lo| ~ 2^-22 |x|.
__device__ __forceinline__ void split_h(float x, _Float16& hi, _Float16& lo) {
    hi = static_cast<_Float16>(x);
    lo = static_cast<_Float16>(x - static_cast<float>(hi));
}

// ---- cross-lane sums (VALU only: DPP and permlane swaps) -------------------
// Sum of x over the 16 lanes that share l & 3 (all-reduce, every lane gets it).
__device__ __forceinline__ float rowgroup_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false));  // row_ror:4
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false));  // row_ror:8
    // permlane16_swap(x, x) returns x of lane l & ~16 and of lane l | 16;
    // permlane32_swap likewise for bit 5: the sum of both is the pair sum
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return x;
}

// Sum of x over the 4 lanes that share l & 15 (all-reduce): the permlane
// swaps of bits 4 and 5.
__device__ __forceinline__ float lanegroup4_sum(float x) {
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return x;
}

// Largest x over the whole wave (every lane gets it): the lanes of each
// 16-lane row by DPP rotations, then the permlane swaps of bits 4 and 5.
__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x121, 0xF, 0xF, false)));  // row_ror:1
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x122, 0xF, 0xF, false)));  // row_ror:2
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x124, 0xF, 0xF, false)));  // row_ror:4
    x = fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xF, 0xF, false)));  // row_ror:8
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
        x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    {
        const unsigned u = __float_as_uint(x);
        const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
        x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    }
    return x;
}
// The bf16 chunk pipeline keeps |sigma S| and |sigma V| of a wave at most this
// (a power of two), 64 x under the fp16 operands' 65504.
constexpr float kRangeMax = 1024.f;

// Sum of x over the whole wave (every lane gets it): the four lanes of each
// quad first (quad_perm xor 1, xor 2), then the 16 quads.
__device__ __forceinline__ float wave_sum(float x) {
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    return rowgroup_sum(x);
}

// ---- MFMA wrapper (gfx950) -----------------------------------------------
// 16x16 output tile, f32 accumulate, K = 32.  Lane l holds A row (l % 16) and
// B column (l % 16); lane group g = l / 16 supplies 8 k slots; the
// accumulator holds D[4g + j][l % 16] in slot j.  Only this form is used: an
// MFMA of another form that takes its result as the accumulator right after
// it (or gives it one) reads stale data on gfx950, and the compiler does not
// space such a pair far enough; a chain of one form is forwarded exactly.
__device__ __forceinline__ f4 mfma16x16x32(h8 a, h8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// A raw buffer descriptor over nbytes from base: loads whose offset (lane
// offset + scalar offset) falls past nbytes return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0),
                                             static_cast<int>(nbytes), 0x00020000);
}

// The same descriptor from values the compiler keeps in vector registers
// (64-bit index arithmetic it hoists out of a loop ends up there): a buffer
// instruction needs its descriptor in scalar registers, and a vector-register
// one becomes a loop over the distinct values in the wave, whose control flow
// also makes every later wait on it a wait for all outstanding memory
// operations.  The caller guarantees the values are wave-uniform.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_uniform(const void* base, uint32_t nbytes) {
    const uint64_t u = reinterpret_cast<uint64_t>(base);
    const uint64_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u)));
    const uint64_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(u >> 32)));
    return make_rsrc(reinterpret_cast<const void*>(hi << 32 | lo),
                     static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(nbytes))));
}

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

// Floats of one 32-token chunk's record in kda_chunkwise_fwd_ckpt's output:
// the state before the chunk (K rows) and the chunk's R (32 rows), all V wide,
// then its A, L and N (32 x 32 each, row-major).  The solve's result
// P = N Diag(beta) R is not kept: the backward forms it from R and N.
__host__ __device__ constexpr int64_t ckpt_record(int64_t K, int64_t V) { return (K + 32) * V + 3 * 32 * 32; }

// fp16 activations keep two K x V matrices in fp16: the state at the head of
// each chunk record and the backward's dS_end per chunk.  fp16 is the dtype
// the reference's fp16 path takes the state in for its products
// (kimi_linear/kda.py:174) and the dtype of that cast's gradient.  Each such
// matrix sits in the first half of its fp32 slot, in 16 x 16 tiles in MFMA
// accumulator order: tile (r / 16, c / 16) at (r / 16) (V / 16) + c / 16,
// 256 halves each; inside it, element (r, c) at
// (r % 4) 64 + ((r / 4) % 4) 16 + c % 16.  An accumulator slot j (rows 4lg + j
// of column ln in lane 16lg + ln) is then 64 consecutive halves (one 128-byte
// store), and 8 consecutive columns of one row are 16 contiguous bytes (one
// load of an MFMA fragment).
__host__ __device__ constexpr int64_t half_tile_offset(int64_t r, int64_t c, int64_t V) {
    return ((r / 16) * (V / 16) + c / 16) * 256 + (r % 4) * 64 + ((r / 4) % 4) * 16 + c % 16;
}

}  // namespace kda
