// C ABI of the KDA core: argument validation and dispatch to the gfx950 kernels.
// Declared in include/kda_hip.h.  No C++ exception crosses this boundary and no
// call allocates, frees or synchronises.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kda_hip.h"
#include "kda_launch.h"

namespace {

bool dtype_ok(int32_t d) {
    return d == KDA_DTYPE_F32 || d == KDA_DTYPE_F16 || d == KDA_DTYPE_BF16;
}

int64_t elem_size(int32_t d) { return d == KDA_DTYPE_F32 ? 4 : 2; }

// Checks shared by both entry points.  `in_place_ok`: state_out may be
// state_in itself (same address and dtype), the recurrence's in-place update.
int validate_common(const kda_fwd_args* a, bool in_place_ok) {
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->K <= 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (!dtype_ok(a->qkv_dtype) || !dtype_ok(a->g_dtype) || !dtype_ok(a->beta_dtype) ||
        !dtype_ok(a->state_out_dtype) || (a->state_in && !dtype_ok(a->state_in_dtype)))
        return KDA_ERR_BAD_DTYPE;
    const bool have_heads = a->B > 0 && a->H > 0;
    if (have_heads && a->state_out == nullptr) return KDA_ERR_NULL_POINTER;
    if (have_heads && a->T > 0 &&
        (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->o))
        return KDA_ERR_NULL_POINTER;
    if (have_heads && a->state_in) {
        const int64_t n = a->B * a->H * a->K * a->V;
        const auto in0 = reinterpret_cast<uintptr_t>(a->state_in);
        const auto in1 = in0 + static_cast<uintptr_t>(n * elem_size(a->state_in_dtype));
        const auto out0 = reinterpret_cast<uintptr_t>(a->state_out);
        const auto out1 = out0 + static_cast<uintptr_t>(n * elem_size(a->state_out_dtype));
        const bool same = in0 == out0 && a->state_in_dtype == a->state_out_dtype;
        if (in0 < out1 && out0 < in1 && !(in_place_ok && same)) return KDA_ERR_ALIAS;
    }
    return KDA_OK;
}

// A gated call needs both parameter vectors (when there is work).
int validate_gate(const kda_fwd_args* a, const kda_gate_args* gate) {
    if (gate == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B > 0 && a->H > 0 && a->T > 0 && (gate->a_log == nullptr || gate->dt_bias == nullptr))
        return KDA_ERR_NULL_POINTER;
    return KDA_OK;
}

int recurrent_entry(const kda_fwd_args* args, const kda_gate_args* gate, void* stream) {
    // In place is safe: each workgroup loads its (b, h, column tile) slice of
    // the state before any store to it, and no other workgroup touches it.
    const int st = validate_common(args, true);
    if (st != KDA_OK) return st;
    if (gate) {
        const int gs = validate_gate(args, gate);
        if (gs != KDA_OK) return gs;
    }
    if (args->B == 0 || args->H == 0) return KDA_OK;
    if (!kda::recurrent_supported(args->K, args->V)) return KDA_ERR_UNSUPPORTED;
    if (args->B * args->H * args->V / 32 > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return kda::recurrent_launch(*args, static_cast<hipStream_t>(stream), gate);
}

int chunkwise_entry(const kda_fwd_args* args, float* ckpt, const kda_gate_args* gate, void* stream) {
    const int st = validate_common(args, false);
    if (st != KDA_OK) return st;
    if (gate) {
        const int gs = validate_gate(args, gate);
        if (gs != KDA_OK) return gs;
    }
    if (args->chunk_size <= 0 || args->T % args->chunk_size != 0) return KDA_ERR_BAD_SHAPE;
    if (args->B == 0 || args->H == 0) return KDA_OK;
    if (args->T == 0) {
        // No tokens: the result is the initial state converted to the output
        // dtype (or zeros); the recurrence kernel with an empty token loop does it.
        if (!kda::recurrent_supported(args->K, args->V)) return KDA_ERR_UNSUPPORTED;
        return kda::recurrent_launch(*args, static_cast<hipStream_t>(stream), gate);
    }
    if (!kda::chunkwise_supported(args->K, args->V)) return KDA_ERR_UNSUPPORTED;
    if (args->B * args->H * args->V / 16 > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int chk = kda::chunkwise_check(*args, gate != nullptr);
    if (chk != KDA_OK) return chk;
    if (args->qkv_dtype == KDA_DTYPE_F32) {
        // fp32 activations: the reference computes in fp32 throughout
        // (kimi_linear/kda.py:116), and so does the token recurrence, which
        // gives the same function (the maths is chunk-size invariant) with the
        // state in fp32 registers; the chunk pipeline's operands are fp16.
        // With checkpoints the recurrence also stores the fp32 state before
        // every 32-token chunk and an fp32 kernel fills the rest of each
        // record (R, A, L, N), so the backward starts from exact records.
        if (ckpt) {
            const int st = kda::recurrent_launch(*args, s, gate, ckpt);
            if (st != KDA_OK) return st;
            return kda::ckpt_fill_fp32_launch(*args, s, ckpt);
        }
        return kda::recurrent_launch(*args, s, gate);
    }
    return kda::chunkwise_launch(*args, s, ckpt, gate);
}

}  // namespace

extern "C" {

int kda_recurrent_fwd(const kda_fwd_args* args, void* stream) { return recurrent_entry(args, nullptr, stream); }

int kda_recurrent_gated_fwd(const kda_fwd_args* args, const kda_gate_args* gate, void* stream) {
    if (gate == nullptr) return KDA_ERR_NULL_POINTER;
    return recurrent_entry(args, gate, stream);
}

int kda_chunkwise_fwd(const kda_fwd_args* args, void* stream) { return chunkwise_entry(args, nullptr, nullptr, stream); }

int kda_chunkwise_fwd_ckpt(const kda_fwd_args* args, float* ckpt, void* stream) {
    return chunkwise_entry(args, ckpt, nullptr, stream);
}

int kda_chunkwise_gated_fwd(const kda_fwd_args* args, const kda_gate_args* gate, void* stream) {
    if (gate == nullptr) return KDA_ERR_NULL_POINTER;
    return chunkwise_entry(args, nullptr, gate, stream);
}

size_t kda_chunkwise_long_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t segments) {
    if (B < 0 || T < 0 || H < 0 || K <= 0 || V <= 0 || segments < 1) return 0;
    if (B * H > (int64_t{1} << 31) || K > 4096 || V > 4096 || segments > (int64_t{1} << 20)) return 0;
    return static_cast<size_t>(kda::long_workspace_bytes(B, T, H, K, V, segments));
}

int kda_chunkwise_long_fwd(const kda_fwd_args* args, int64_t segments, void* workspace, void* stream) {
    if (segments == 1) return chunkwise_entry(args, nullptr, nullptr, stream);
    const int st = validate_common(args, false);
    if (st != KDA_OK) return st;
    if (segments < 1) return KDA_ERR_BAD_SHAPE;
    if (args->chunk_size <= 0 || args->T % args->chunk_size != 0 || args->T % segments != 0) return KDA_ERR_BAD_SHAPE;
    if (!kda::chunkwise_trans_supported(*args)) return KDA_ERR_UNSUPPORTED;
    if (args->B == 0 || args->H == 0) return KDA_OK;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (args->T == 0) return kda::recurrent_launch(*args, s);
    if (workspace == nullptr) return KDA_ERR_NULL_POINTER;
    if ((reinterpret_cast<uintptr_t>(workspace) & 15) != 0) return KDA_ERR_BAD_SHAPE;
    if (args->B * segments * args->H * ((args->V + args->K) / 16) > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    const int chk = kda::chunkwise_check(*args);
    if (chk != KDA_OK) return chk;
    return kda::long_launch(*args, segments, workspace, s);
}

int kda_chunkwise_fused_fwd(const kda_fwd_args* args, const kda_gate_args* gate, const kda_out_epilogue* out,
                            void* stream) {
    const int st = validate_common(args, false);
    if (st != KDA_OK) return st;
    if (gate) {
        const int gs = validate_gate(args, gate);
        if (gs != KDA_OK) return gs;
    }
    if (out == nullptr) return KDA_ERR_NULL_POINTER;
    if (args->chunk_size <= 0 || args->T % args->chunk_size != 0) return KDA_ERR_BAD_SHAPE;
    if (!(out->eps >= 0.f)) return KDA_ERR_BAD_SHAPE;
    if (!kda::chunkwise_fused_supported(*args)) return KDA_ERR_UNSUPPORTED;
    if (args->B == 0 || args->H == 0) return KDA_OK;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    // no tokens: no outputs, the state passes through (the recurrence's empty loop)
    if (args->T == 0) return kda::recurrent_launch(*args, s, gate);
    if (out->gate == nullptr || out->weight == nullptr) return KDA_ERR_NULL_POINTER;
    if (args->B * args->H > INT32_MAX) return KDA_ERR_BAD_SHAPE;
    return kda::chunkwise_fused_launch(*args, s, gate, *out);
}

size_t kda_chunkwise_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V) {
    if (B < 0 || T < 0 || H < 0 || K <= 0 || V <= 0) return 0;
    if (T > (int64_t{1} << 40) || B * H > (int64_t{1} << 31) || K > 4096 || V > 4096) return 0;
    return static_cast<size_t>(kda::chunkwise_bwd_workspace_bytes(B, T, H, K, V));
}

}  // extern "C"

namespace {

// Checks shared by both backward entry points; `need_workspace`: the caller
// must supply args->workspace.  KDA_OK with *empty set when nothing is to be
// launched.
int validate_bwd(const kda_bwd_args* a, bool need_workspace, bool* empty) {
    *empty = false;
    if (a == nullptr) return KDA_ERR_NULL_POINTER;
    if (a->B < 0 || a->T < 0 || a->H < 0 || a->K <= 0 || a->V <= 0) return KDA_ERR_BAD_SHAPE;
    if (a->B == 0 || a->H == 0) {
        *empty = true;
        return KDA_OK;
    }
    if (!kda::chunkwise_bwd_supported(a->K, a->V)) return KDA_ERR_UNSUPPORTED;
    if (a->io_dtype != KDA_DTYPE_F32 && a->io_dtype != KDA_DTYPE_F16 && a->io_dtype != KDA_DTYPE_BF16)
        return KDA_ERR_BAD_DTYPE;
    if (a->T > 0 && (!a->q || !a->k || !a->v || !a->g || !a->beta || !a->ckpt || !a->d_o || !a->dq ||
                     !a->dk || !a->dg || !a->dbeta || !a->dv || (need_workspace && !a->workspace)))
        return KDA_ERR_NULL_POINTER;
    // grids: B H ceil(T / 32) and B H V / 32 workgroups
    if (a->B * a->H * ((a->T + 31) / 32) > INT32_MAX || a->B * a->H * (a->V / 32) > INT32_MAX)
        return KDA_ERR_BAD_SHAPE;
    if (a->T == 0 && a->d_state_in == nullptr) *empty = true;
    return KDA_OK;
}

}  // namespace

extern "C" {

int kda_chunkwise_bwd(const kda_bwd_args* a, void* stream) {
    bool empty = false;
    const int st = validate_bwd(a, true, &empty);
    if (st != KDA_OK || empty) return st;
    return kda::chunkwise_bwd_launch(*a, static_cast<hipStream_t>(stream));
}

int kda_chunkwise_bwd_noalloc(const kda_bwd_args* a, void* stream) {
    bool empty = false;
    const int st = validate_bwd(a, false, &empty);
    if (st != KDA_OK || empty) return st;
    if (kda::chunkwise_bwd_workspace_bytes(a->B, a->T, a->H, a->K, a->V) > static_cast<int64_t>(KDA_BWD_SCRATCH_BYTES))
        return KDA_ERR_TOO_LARGE;
    void* scratch = nullptr;
    const int sst = kda::chunkwise_bwd_scratch(&scratch);
    if (sst != KDA_OK) return sst;
    kda_bwd_args b = *a;
    b.workspace = scratch;
    return kda::chunkwise_bwd_launch(b, static_cast<hipStream_t>(stream));
}

const char* kda_status_str(int status) {
    switch (status) {
        case KDA_OK: return "ok";
        case KDA_ERR_NULL_POINTER: return "a required pointer is NULL";
        case KDA_ERR_BAD_SHAPE: return "invalid shape (negative size, T not a multiple of chunk_size, or grid too large)";
        case KDA_ERR_BAD_DTYPE: return "unsupported dtype code";
        case KDA_ERR_UNSUPPORTED: return "no kernel for these head dimensions";
        case KDA_ERR_ALIAS: return "an output overlaps an input (state_out/state_in, or a conv cache written while still read)";
        case KDA_ERR_LAUNCH: return "kernel launch failed (or no current HIP device)";
        case KDA_ERR_TOO_LARGE: return "shape needs more scratch than the static buffer holds (KDA_BWD_SCRATCH_BYTES)";
        default: return "unknown kda_status";
    }
}

int kda_abi_version(void) { return KDA_ABI_VERSION; }

}  // extern "C"
