/*
 * kda_hip.h -- C ABI of the MI355X (gfx950) Kimi Delta Attention core.
 *
 * The reference (Lazy-Hakimi/-kimi-linear-) is pure PyTorch: its hot path is
 * the pair of Python functions
 *
 *   kda_chunkwise(q, k, v, g, beta, initial_state=None, chunk_size=64,
 *                 tile_size=0, state_dtype=None)      kimi_linear/kda.py:58-59
 *   kda_recurrent(q, k, v, g, beta, state=None,
 *                 state_dtype=None)                  kimi_linear/kda.py:188
 *
 * This library replaces their bodies.  A Python wrapper with the same
 * signatures allocates the outputs and calls the entry points below through
 * ctypes; a C/C++ caller fills kda_fwd_args directly.
 *
 * Contract shared by both entry points
 *  - All pointers are device pointers on the current HIP device.
 *  - q, k, g: [B, T, H, K]; v: [B, T, H, V]; beta: [B, T, H].  Each is a
 *    strided view whose last dimension is contiguous; the three strides
 *    (batch, token, head) are given in ELEMENTS.  q, k and v share one dtype.
 *  - state_in (nullable = zeros), state_out: [B, H, K, V] contiguous.
 *  - o: [B, T, H, V] contiguous, in the dtype of v.
 *  - The work is asynchronous and stream-ordered on `stream` (a hipStream_t,
 *    NULL = the legacy default stream).  The library never allocates, frees,
 *    synchronises or copies to the host, so a call may be captured in a
 *    hipGraph.  Inputs are never written.  state_out may not overlap
 *    state_in, except that kda_recurrent_fwd accepts state_out == state_in
 *    (same address and dtype) as an in-place update.
 *  - Returns KDA_OK (0) or a kda_status code; kda_status_str() names it.
 *    Argument errors are detected on the host before any launch.
 */
#ifndef KDA_HIP_H
#define KDA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_ABI_VERSION 14

/* Element types accepted at the boundary. */
typedef enum kda_dtype {
    KDA_DTYPE_F32 = 0,
    KDA_DTYPE_F16 = 1,
    KDA_DTYPE_BF16 = 2
} kda_dtype;

typedef enum kda_status {
    KDA_OK = 0,
    KDA_ERR_NULL_POINTER = 1,      /* a required pointer is NULL                 */
    KDA_ERR_BAD_SHAPE = 2,         /* negative/inconsistent sizes, T % chunk != 0 */
    KDA_ERR_BAD_DTYPE = 3,         /* dtype code outside kda_dtype / o != v dtype */
    KDA_ERR_UNSUPPORTED = 4,       /* head dims this build has no kernel for      */
    KDA_ERR_ALIAS = 5,             /* state_out overlaps state_in (other than an
                                      exact in-place alias for the recurrence)   */
    KDA_ERR_LAUNCH = 6,            /* hipGetLastError() after the launch, or no
                                      current HIP device                         */
    KDA_ERR_TOO_LARGE = 7          /* the shape needs more scratch memory than the
                                      library's static buffer holds               */
} kda_status;

/* One call's arguments.  Plain data: pointers, sizes, strides, codes. */
typedef struct kda_fwd_args {
    int64_t B, T, H, K, V;

    const void* q;                 /* [B,T,H,K] */
    const void* k;                 /* [B,T,H,K] */
    const void* v;                 /* [B,T,H,V] */
    const void* g;                 /* [B,T,H,K] log decay (<= 0) */
    const void* beta;              /* [B,T,H]   delta-rule rate  */
    int64_t q_stride[3];           /* (batch, token, head) strides in elements */
    int64_t k_stride[3];
    int64_t v_stride[3];
    int64_t g_stride[3];
    int64_t beta_stride[3];
    int32_t qkv_dtype;             /* kda_dtype of q, k and v */
    int32_t g_dtype;               /* kda_dtype of g          */
    int32_t beta_dtype;            /* kda_dtype of beta       */

    const void* state_in;          /* [B,H,K,V] contiguous, or NULL for zeros */
    int32_t state_in_dtype;
    void* state_out;               /* [B,H,K,V] contiguous */
    int32_t state_out_dtype;
    void* o;                       /* [B,T,H,V] contiguous, dtype == qkv_dtype */

    float scale;                   /* q multiplier; the reference uses K^-0.5  */
    int32_t clamp_fp16_out;        /* 1: clamp an fp16 o to +-60000 (kda.py:217-218) */
    int64_t chunk_size;            /* chunkwise: T must be a multiple of it (kda.py:109);
                                      it has no other numerical role (the maths is
                                      chunk-size invariant) */
} kda_fwd_args;

/*
 * Chunkwise forward; replaces the body of kda_chunkwise (kimi_linear/kda.py:58-185).
 * o = per-token outputs, state_out = final state.  T may be 0.
 * For T > 0, g and beta must be fp32 (KDA_ERR_BAD_DTYPE otherwise): the
 * reference upcasts both before use (kda.py:119-120).
 */
int kda_chunkwise_fwd(const kda_fwd_args* args, void* stream);

/*
 * Token-by-token recurrence; replaces the body of kda_recurrent
 * (kimi_linear/kda.py:188-219).  Any T >= 0; T == 1 is the decode step.
 * chunk_size is ignored.  state_out == state_in (same address and dtype)
 * updates the state in place: a decode loop over static state buffers then
 * needs no copy of the new state back into its input (the reference copies
 * it back inside its captured graph, kimi_linear/graph_decode.py:257-262).
 */
int kda_recurrent_fwd(const kda_fwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * The KDA layer's gate pre-processing fused into the core's loads
 * (kimi_linear/kda.py:452-460):
 *   g    = -exp(A_log[h, c]) * softplus(gk + dt_bias[h, c])   (softplus(z) = z
 *          for z > 20, torch's default threshold), in fp32
 *   beta = sigmoid(beta_logit), in fp32
 * With these two entry points args->g holds gk, the gate's up-projection
 * output [B,T,H,K], and args->beta the beta logits [B,T,H] (same strides and
 * dtype codes as g and beta otherwise); the kernels form g and beta while
 * they load a token, so neither is ever written to memory: at fp16 the
 * chunkwise call reads 2 bytes of gate per token and channel instead of
 * the 4 of an fp32 g that a separate pre-processing pass wrote before it.
 * Everything else is as in kda_chunkwise_fwd / kda_recurrent_fwd.
 * ------------------------------------------------------------------------- */
typedef struct kda_gate_args {
    const float* a_log;            /* [H, K] contiguous fp32 */
    const float* dt_bias;          /* [H, K] contiguous fp32 */
} kda_gate_args;

/* kda_chunkwise_fwd with the fused gate (replaces the g / beta lines of
 * _projections, kimi_linear/kda.py:452-460, plus kda_chunkwise,
 * kda.py:58-185).  For fp16 / bf16 q, k, v, gk and the logits must be in
 * the same dtype (KDA_ERR_BAD_DTYPE otherwise); fp32 q, k, v run the gated
 * token recurrence, as kda_chunkwise_fwd does, and take any gate dtypes. */
int kda_chunkwise_gated_fwd(const kda_fwd_args* args, const kda_gate_args* gate, void* stream);

/* kda_recurrent_fwd with the fused gate (kimi_linear/kda.py:452-460 plus
 * kda_recurrent, kda.py:188-219); gk and the logits in any dtype.  In place
 * (state_out == state_in) as kda_recurrent_fwd. */
int kda_recurrent_gated_fwd(const kda_fwd_args* args, const kda_gate_args* gate, void* stream);

/* The layer's output epilogue -- HeadwiseRMSNorm and the sigmoid output gate
 * of _output (kimi_linear/kda.py:258-279, 464-470) -- applied by the
 * chunkwise kernel to its output tile before anything is written:
 *   n = TQ(TQ(o) * rsqrt(mean over V of TQ(o)^2 + eps) * weight[h])
 *   y = TQ(n * sigmoid(gate))
 * (TQ: rounded to the dtype of q, k, v, as the reference's o_core and norm
 * output are); args->o receives y, [B, T, H, V] = the o_proj input
 * [B, T, H*V]. */
typedef struct kda_out_epilogue {
    const void* gate;              /* [B, T, H*V] output-gate up-projection, qkv dtype */
    int64_t gate_stride[2];        /* (batch, token) strides in elements; channels contiguous */
    const float* weight;           /* [H, V] contiguous fp32 (the norm weight) */
    float eps;
} kda_out_epilogue;

/* kda_chunkwise_gated_fwd (gate != NULL) or kda_chunkwise_fwd (gate == NULL)
 * with the output epilogue: one workgroup holds a head's whole V row.  q, k, v
 * fp16 or bf16, K in {64, 128}, V in {64, 128} (KDA_ERR_UNSUPPORTED
 * otherwise).  The rest of the layer's forward around the core is
 * kda_prep_fwd before and the o_proj GEMM after. */
int kda_chunkwise_fused_fwd(const kda_fwd_args* args, const kda_gate_args* gate, const kda_out_epilogue* out,
                            void* stream);

/* ---------------------------------------------------------------------------
 * kda_chunkwise_fwd on long sequences with few (batch, head) chains, split
 * into `segments` pieces of T / segments tokens that run in parallel.  The
 * state map of a segment is affine in the state entering it (S_end = Phi
 * S_start + S_loc): a first pass computes every segment's S_loc and Phi
 * (K x K), a short sequential pass composes them (the segments' initial
 * states and the final state, fp32), and a second pass writes the outputs
 * from the true initial states.  When the first pass fits one round of
 * workgroups (B * segments * H * (V + K) / 128 <= the compute units), it also
 * writes the outputs from a zero initial state and, per token, their
 * coefficients of the initial state, and the second pass is o = those
 * outputs + coefficients x initial state.  Same arguments and results as
 * kda_chunkwise_fwd (the same function, rounded differently), for q, k, v
 * fp16 or bf16, K in {64, 128}, V a multiple of 64, T % segments == 0 and,
 * with B > 1, each input's batch stride T times its token stride
 * (KDA_ERR_UNSUPPORTED otherwise).  workspace: device memory of
 * kda_chunkwise_long_workspace_size() bytes, 16-byte aligned, contents on
 * entry irrelevant.  segments == 1 is kda_chunkwise_fwd.
 * ------------------------------------------------------------------------- */
size_t kda_chunkwise_long_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t segments);
int kda_chunkwise_long_fwd(const kda_fwd_args* args, int64_t segments, void* workspace, void* stream);

/* ---------------------------------------------------------------------------
 * Backward of the chunkwise forward.  The reference differentiates
 * kda_chunkwise (kimi_linear/kda.py:58-185) with autograd and trains through
 * it (scripts/train_musicgpt_fp16.py:519-523); these two calls are what a
 * torch.autograd.Function around the HIP forward binds instead.
 * ------------------------------------------------------------------------- */

/* kda_chunkwise_fwd, plus per 32-token chunk a record, in fp32: the state
 * before the chunk and the chunk's R = V - (k * E) S, then its A (scale times
 * the decayed q k^T, i <= c), L (the decayed k k^T, i < c) and N = (I +
 * Diag(beta) L)^-1, of which the forward's solve writes the 16-row diagonal
 * blocks and zeroes the block above them; kda_chunkwise_bwd completes the
 * block below them in place: ckpt is [B, H, ceil(T/32), KDA_CKPT_RECORD(K,
 * V)] contiguous, each record (K + 32) x V (rows [0, K) the state, [K, K + 32)
 * R) followed by three row-major 32 x 32 matrices (the input of
 * kda_chunkwise_bwd, which forms the solve's result P = N Diag(beta) R
 * itself).  Same arguments, errors and results otherwise.  For
 * fp16 / bf16 q, k, v the records come from the chunk pipeline (its fp16
 * operands); for fp32 q, k, v from the fp32 token recurrence (the state) and
 * an fp32 kernel (the rest, with N whole), fp32-exact like the outputs
 * (K in {32, 64, 128}).  With fp16 q, k, v the state is stored in fp16, the
 * dtype the reference's fp16 path casts it to for its products
 * (kimi_linear/kda.py:174), in the first K x V / 2 floats of its rows: 16 x 16
 * tiles, tile (r / 16, c / 16) at (r / 16) (V / 16) + c / 16, 256 halves each,
 * element (r, c) at (r % 4) 64 + ((r / 4) % 4) 16 + c % 16 inside it; and R
 * (the single fp16 operand of the forward's solve) as row-major halves in the
 * first 32 x V / 2 floats of its rows. */
#define KDA_CKPT_RECORD(K, V) (((K) + 32) * (V) + 3 * 32 * 32)
int kda_chunkwise_fwd_ckpt(const kda_fwd_args* args, float* ckpt, void* stream);

/* Every tensor is contiguous in the forward layout: q, k, g, dq, dk, dg
 * [B, T, H, K]; v, d_o, dv [B, T, H, V]; beta, dbeta [B, T, H]; states
 * [B, H, K, V].  q, k, v, d_o, dq, dk and dv are in io_dtype (a kda_dtype);
 * g, beta, ckpt, dg, dbeta and the state gradients are fp32.  workspace: device memory of at least
 * kda_chunkwise_bwd_workspace_size(B, T, H, K, V) bytes, 16-byte aligned (its
 * contents on entry do not matter; calls that share one workspace must not
 * overlap).  K in {32, 64, 128}, V a multiple of 32, any T >= 0. */
typedef struct kda_bwd_args {
    int64_t B, T, H, K, V;
    const void* q;                 /* the forward's inputs (q unscaled)        */
    const void* k;
    const void* v;                 /* not read: R comes from the checkpoint     */
    const float* g;
    const float* beta;
    float* ckpt;                   /* from kda_chunkwise_fwd_ckpt on the same inputs;
                                      the backward completes each record's N in place
                                      (idempotent: a second call writes the same) */
    const void* d_o;               /* dL/do                                      */
    const float* d_state_out;      /* dL/d(final state), or NULL for zeros       */
    void* dq;                      /* [B, T, H, K] */
    void* dk;
    float* dg;
    float* dbeta;                  /* [B, T, H]    */
    void* dv;                      /* [B, T, H, V] */
    float* d_state_in;             /* dL/d(initial state) [B, H, K, V], or NULL   */
    void* workspace;
    float scale;                   /* the forward's q multiplier                  */
    int32_t io_dtype;              /* kda_dtype of q, k, v, d_o, dq, dk, dv       */
} kda_bwd_args;

/* Bytes of workspace kda_chunkwise_bwd needs: per (b, h) and 32-token chunk,
 * (K * V + 2 * 32 * V) floats (with fp16 q, k, v the K x V part,
 * the gradient of the state at the chunk's end, and the two 32 x V parts are
 * kept in fp16 and use half of theirs).  0 for a bad or empty shape. */
size_t kda_chunkwise_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V);

int kda_chunkwise_bwd(const kda_bwd_args* args, void* stream);

/* Bytes of the static device buffer behind kda_chunkwise_bwd_noalloc. */
#define KDA_BWD_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * kda_chunkwise_bwd without a caller workspace and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory -- code under hipGraph capture, tight serving or training
 * loops, harnesses that forbid hipMalloc.  args->workspace is ignored; the
 * two kernels use instead a static device buffer of KDA_BWD_SCRATCH_BYTES
 * that the library holds on every GPU it runs on until the process ends
 * (resolved once per device, on the first call with that device current;
 * `stream` must belong to the current device).  That first call resolves a
 * symbol address, which may load the code object: make it outside graph
 * capture (an eager warm-up call); later calls on the device only launch
 * kernels and may be captured.  Shapes whose
 * kda_chunkwise_bwd_workspace_size() exceeds KDA_BWD_SCRATCH_BYTES return
 * KDA_ERR_TOO_LARGE before any launch.  Every call on one GPU shares that
 * GPU's buffer: calls that overlap on one GPU (two streams, two threads) race
 * and must be serialised by the caller.  Results are identical to
 * kda_chunkwise_bwd's (the same kernels).
 */
int kda_chunkwise_bwd_noalloc(const kda_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Layer pre- and post-processing around the core (the KDA layer,
 * kimi_linear/kda.py:399-470).  Same conventions: device pointers,
 * asynchronous on `stream`, no allocation, KDA_OK or a kda_status code.
 * "x dtype" is the activation dtype (kda_dtype) shared by every activation
 * tensor of one call.
 * ------------------------------------------------------------------------- */

/* Projections -> core inputs, one pass (replaces ShortConv + SiLU + l2norm
 * for q and k, ShortConv + SiLU for v, the forget gate and beta of
 * _projections, kimi_linear/kda.py:399-461, 282-325).  Per token t, head h,
 * channel c of q/k/v (tensor index i = 0, 1, 2):
 *   u[t] = bias[c] + sum_j w[c, j] * x[t - (conv_size - 1) + j]     (causal)
 *   s[t] = u / (1 + exp(-u))                                         (SiLU)
 *   q, k: s * min(rsqrt(sum over the head's K channels of s^2), 1/l2_eps)
 * where x[t < 0] comes from hist_in (the last conv_size - 1 inputs before
 * this call) or is zero.  Gates: g = -exp(a_log) * softplus(gk + dt_bias)
 * (softplus(z) = z for z > 20) and beta = sigmoid(beta_logit), in fp32.
 * hist_out[i] (optional) receives the last conv_size - 1 inputs of
 * [hist_in | x], the conv cache of the next call; it may be hist_in itself
 * only when T <= 16.  g and beta may both be NULL: the gates are then not
 * computed (gk, a_log, dt_bias and beta_logit are not read and may be NULL
 * too), for a caller that hands gk and the logits to the gated core entry
 * points instead. */
typedef struct kda_prep_args {
    int64_t B, T, H, K, V;         /* K, V in {64, 128, 256} */
    int64_t conv_size;             /* 1..4 */
    const void* x[3];              /* q, k, v projections [B, T, H*K] / [B, T, H*V], x dtype */
    int64_t x_stride[3][2];        /* (batch, token) strides in elements; channels contiguous */
    const void* conv_w[3];         /* [D, conv_size] contiguous (nn.Conv1d weight [D, 1, conv_size]) */
    const void* conv_b[3];         /* [D] or NULL */
    int32_t w_dtype;               /* kda_dtype of conv_w and conv_b */
    const void* hist_in[3];        /* [B, conv_size - 1, D] contiguous, x dtype, or NULL (zeros) */
    void* hist_out[3];             /* [B, conv_size - 1, D] contiguous, x dtype, or NULL */
    const void* gk;                /* [B, T, H*K] gate up-projection output, x dtype */
    int64_t gk_stride[2];
    const void* a_log;             /* [H*K] */
    const void* dt_bias;           /* [H*K] */
    int32_t p_dtype;               /* kda_dtype of a_log and dt_bias */
    const void* beta_logit;        /* [B, T, H], x dtype */
    int64_t beta_stride[2];
    void* q;                       /* [B, T, H, K] contiguous, x dtype */
    void* k;                       /* [B, T, H, K] contiguous, x dtype */
    void* v;                       /* [B, T, H, V] contiguous, x dtype */
    void* g;                       /* [B, T, H, K] contiguous fp32 */
    void* beta;                    /* [B, T, H] contiguous fp32 */
    float l2_eps;
    int32_t x_dtype;
} kda_prep_args;

int kda_prep_fwd(const kda_prep_args* args, void* stream);

/* Core output -> o_proj input, one pass (replaces HeadwiseRMSNorm and the
 * sigmoid output gate of _output, kimi_linear/kda.py:258-279, 464-470):
 *   n = o * rsqrt(mean over V of o^2 + eps) * weight[h]   rounded to x dtype
 *   y = n * sigmoid(gate)                                  rounded to x dtype */
typedef struct kda_output_args {
    int64_t B, T, H, V;            /* V in {64, 128, 256} */
    const void* o;                 /* [B, T, H, V], x dtype */
    int64_t o_stride[3];           /* (batch, token, head) strides; V contiguous */
    const void* gate;              /* [B, T, H*V] output-gate up-projection, x dtype */
    int64_t gate_stride[2];        /* (batch, token) strides */
    const void* weight;            /* [H, V] contiguous */
    int32_t w_dtype;
    void* y;                       /* [B, T, H*V] contiguous, x dtype */
    float eps;
    int32_t x_dtype;
} kda_output_args;

int kda_output_fwd(const kda_output_args* args, void* stream);

/* Gradients of kda_prep_fwd, for training through the layer (the reference
 * differentiates _projections, kimi_linear/kda.py:399-461, by autograd;
 * scripts/train_musicgpt_fp16.py:519-523 trains the whole layer).  Given dy,
 * the gradients of the forward's q, k, v outputs, and the forward's inputs
 * (no conv cache: a training call starts from zeros), per tensor i:
 *   dx[i]   [B, T, D]        gradient of the projection x[i]
 *   dw[i]   [D, conv_size]   gradient of the conv weight, fp32
 *   db[i]   [D]              gradient of the conv bias, fp32 (NULL: skipped)
 * through the L2 norm (its 1/l2_eps clamp included), SiLU and the causal
 * convolution; and, when gk is not NULL, through the gates from dg and dbeta
 * (fp32, the gradients of g and beta):
 *   dgk [B, T, H*K] and dbeta_logit [B, T, H] (x dtype), da_log and ddt_bias
 *   [H*K] (fp32).
 * Every sum over tokens runs in fp32 per workgroup tile, then over the tiles
 * in a fixed order (run-to-run identical).  K, V in {64, 128}.  workspace:
 * kda_prep_bwd_workspace_size() bytes of device memory (16-byte aligned); the
 * call allocates nothing. */
typedef struct kda_prep_bwd_args {
    int64_t B, T, H, K, V;         /* K, V in {64, 128} */
    int64_t conv_size;             /* 1..4 */
    const void* x[3];              /* the forward's q, k, v projections [B, T, D], x dtype */
    int64_t x_stride[3][2];        /* (batch, token) strides in elements; channels contiguous */
    const void* conv_w[3];         /* [D, conv_size] contiguous */
    const void* conv_b[3];         /* [D] or NULL */
    int32_t w_dtype;               /* kda_dtype of conv_w and conv_b */
    const void* dy[3];             /* gradients of q, k [B, T, H, K] and v [B, T, H, V], contiguous, x dtype */
    void* dx[3];                   /* [B, T, D] contiguous, x dtype */
    float* dw[3];                  /* [D, conv_size] */
    float* db[3];                  /* [D] or NULL */
    const void* gk;                /* [B, T, H*K] gate up-projection, x dtype, or NULL (no gates) */
    int64_t gk_stride[2];
    const void* a_log;             /* [H*K] */
    const void* dt_bias;           /* [H*K] */
    int32_t p_dtype;               /* kda_dtype of a_log and dt_bias */
    const void* beta_logit;        /* [B, T, H], x dtype */
    int64_t beta_stride[2];
    const float* dg;               /* [B, T, H, K] contiguous */
    const float* dbeta;            /* [B, T, H] contiguous */
    void* dgk;                     /* [B, T, H*K] contiguous, x dtype */
    void* dbeta_logit;             /* [B, T, H] contiguous, x dtype */
    float* da_log;                 /* [H*K] */
    float* ddt_bias;               /* [H*K] */
    float l2_eps;
    int32_t x_dtype;
    void* workspace;
} kda_prep_bwd_args;

size_t kda_prep_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t K, int64_t V, int64_t conv_size);
int kda_prep_bwd(const kda_prep_bwd_args* args, void* stream);

/* Gradients of kda_output_fwd (the reference differentiates HeadwiseRMSNorm
 * and the output gate, kimi_linear/kda.py:258-279, 464-470, by autograd):
 * from dy [B, T, H*V], the gradients of o (d_o [B, T, H, V]) and of the gate
 * (dgate [B, T, H*V]) in x dtype, and of the norm weight (dweight [H*V],
 * fp32; token sums as in kda_prep_bwd).  The rounding of the normalised value
 * to x dtype counts as the identity.  V in {64, 128}. */
typedef struct kda_output_bwd_args {
    int64_t B, T, H, V;            /* V in {64, 128} */
    const void* o;                 /* the forward's o [B, T, H, V], x dtype */
    int64_t o_stride[3];           /* (batch, token, head) strides; V contiguous */
    const void* gate;              /* the forward's gate [B, T, H*V], x dtype */
    int64_t gate_stride[2];
    const void* weight;            /* [H, V] contiguous */
    int32_t w_dtype;
    const void* dy;                /* [B, T, H*V] contiguous, x dtype */
    void* d_o;                     /* [B, T, H, V] contiguous, x dtype */
    void* dgate;                   /* [B, T, H*V] contiguous, x dtype */
    float* dweight;                /* [H*V] */
    float eps;
    int32_t x_dtype;
    void* workspace;               /* kda_output_bwd_workspace_size() bytes */
} kda_output_bwd_args;

size_t kda_output_bwd_workspace_size(int64_t B, int64_t T, int64_t H, int64_t V);
int kda_output_bwd(const kda_output_bwd_args* args, void* stream);

/* Human-readable name of a kda_status code (static storage). */
const char* kda_status_str(int status);

/* KDA_ABI_VERSION of the built library (layout of the argument structs and of
 * the checkpoint records). */
int kda_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KDA_HIP_H */
