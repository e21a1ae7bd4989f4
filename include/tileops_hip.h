/*
 * tileops_hip.h -- C ABI of the MI355X (gfx950) TileOPs forward-operator
 * library, libtileops_hip.so.
 *
 * Every entry point
 *   - takes raw device pointers that the caller allocated (the library never
 *     allocates device memory, except where a workspace is passed in),
 *   - takes element counts / shapes as int64 for contiguous row-major data,
 *   - enqueues its kernels asynchronously on `stream` (a hipStream_t; NULL is
 *     the legacy default stream) and never synchronises the host,
 *   - returns 0 on success, a positive hipError_t code if a launch failed, or
 *     a negative TILEOPS_E* code when an argument is rejected before any launch.
 * tileops_error_string() turns either kind of code into a message.
 *
 * Citations name the reference (Yihuace/tile-ascendnpu-ops) interface each
 * entry point replaces; paths are relative to examples/TileOPs/.
 */
#ifndef TILEOPS_HIP_H
#define TILEOPS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (torch.float32 / float16 / bfloat16). */
enum tileops_dtype {
  TILEOPS_F32 = 0,
  TILEOPS_F16 = 1,
  TILEOPS_BF16 = 2,
};

/* Unary activation / clamp selector for tileops_unary_fwd. */
enum tileops_unary_op {
  TILEOPS_HARDSWISH = 0,
  TILEOPS_HARDSIGMOID = 1,
  TILEOPS_CLAMP = 2,
  TILEOPS_MISH = 3,
};

/* Float predicate selector for tileops_isfp_fwd. */
enum tileops_predicate {
  TILEOPS_ISNAN = 0,
  TILEOPS_ISINF = 1,
  TILEOPS_ISFINITE = 2,
};

/* Flags for tileops_unary_fwd (TILEOPS_CLAMP only). */
#define TILEOPS_CLAMP_HAS_MIN 1
#define TILEOPS_CLAMP_HAS_MAX 2

/* Argument-rejection codes (negative, so they never collide with hipError_t). */
#define TILEOPS_EINVAL (-1)   /* bad dtype, op selector, or flag combination */
#define TILEOPS_ESHAPE (-2)   /* negative / unsupported size */
#define TILEOPS_ENULL (-3)    /* NULL pointer with a non-empty size */
#define TILEOPS_EWORKSPACE (-4) /* workspace missing or too small */

/* Library ABI version (major * 100 + minor). */
int tileops_version(void);

/* Message for a return code of any entry point (static storage). */
const char* tileops_error_string(int code);

/*
 * y[i] = f(x[i]) for i < n, computed in fp32 and rounded once to `dtype`.
 *   TILEOPS_HARDSWISH   x * min(max(x + 3, 0), 6) / 6
 *   TILEOPS_HARDSIGMOID min(max(x + 3, 0), 6) / 6
 *   TILEOPS_CLAMP       min(max(x, lo), hi) with the bounds selected by
 *                       `flags` (TILEOPS_CLAMP_HAS_MIN / _HAS_MAX, at least
 *                       one); a NaN bound yields NaN everywhere.
 *   TILEOPS_MISH        x * tanh(log1p(exp(x)))  (F.mish)
 * NaN inputs propagate.  x and y may alias (in-place).
 * Replaces HardswishFwdKernel.forward
 * (tileops/kernels/elementwise/hardswish/hardswish.py:145-156),
 * HardsigmoidFwdKernel.forward
 * (tileops/kernels/elementwise/hardsigmoid/hardsigmoid.py:147) and
 * ClampScalarFwdKernel.forward
 * (tileops/kernels/elementwise/clamp_scalar/clamp_scalar.py:174-190) and
 * MishFwdKernel.forward (tileops/kernels/elementwise/mish/mish.py).
 */
int tileops_unary_fwd(int op, const void* x, void* y, int64_t n, int dtype,
                      float lo, float hi, int flags, void* stream);

/*
 * y = torch.bitwise_not(x) over `nbytes` bytes of a bool or integer tensor
 * (uint8 / int8 / int16 / int32 / int64): every byte complemented, or, for
 * bool (is_bool != 0, bytes 0 / 1), every byte XOR 1.  x and y may alias.
 * Replaces BitwiseNotFwdKernel.forward
 * (tileops/kernels/elementwise/bitwise_not/bitwise_not.py; op interface
 * tileops/ops/elementwise/bitwise_not.py:33-120).
 */
int tileops_bitwise_not_fwd(const void* x, void* y, int64_t nbytes, int is_bool, void* stream);

/*
 * y = a + alpha * b with broadcasting (torch.add; torch.sub passes -alpha),
 * computed in fp32 and rounded once to `dtype` (F32 / F16 / BF16).  The
 * output is contiguous with `ndim` (<= 8) dimensions `out_shape`; a and b
 * are read at element strides `a_strides` / `b_strides` per output
 * dimension (0 on a broadcast dimension), host arrays of `ndim` entries.
 * Replaces AddFwdKernel.forward / SubFwdKernel.forward
 * (tileops/kernels/elementwise/add, sub; op interfaces
 * tileops/ops/elementwise/add.py:61-155, sub.py), which materialised the
 * broadcast with expand().contiguous() first.
 */
int tileops_add_fwd(const void* a, const void* b, void* y, int ndim, const int64_t* out_shape,
                    const int64_t* a_strides, const int64_t* b_strides, float alpha, int dtype,
                    void* stream);

/*
 * y = lerp(a, b, weight) with broadcasting (torch.lerp): a + w (b - a) for
 * |w| < 0.5, else b - (1 - w)(b - a), each an fp32 fma rounded once to
 * `dtype` (F32 / F16 / BF16).  With `w` NULL the weight is the scalar
 * `weight` (w_strides unused); otherwise the weight tensor `w` (same dtype)
 * is read at `w_strides`.  Output, shapes and strides as tileops_add_fwd.
 * Replaces LerpScalarFwdKernel.forward
 * (tileops/kernels/elementwise/lerp_scalar/lerp_scalar.py:148; op interface
 * tileops/ops/elementwise/lerp_scalar.py:38-157) and
 * LerpTensorFwdKernel.forward
 * (tileops/kernels/elementwise/lerp_tensor/lerp_tensor.py:170; op interface
 * tileops/ops/elementwise/lerp_tensor.py:35-165), which materialised the
 * broadcast with expand().contiguous() first.
 */
int tileops_lerp_fwd(const void* a, const void* b, const void* w, void* y, int ndim,
                     const int64_t* out_shape, const int64_t* a_strides,
                     const int64_t* b_strides, const int64_t* w_strides, float weight, int dtype,
                     void* stream);

/*
 * y[i] = pred(x[i]) as one byte 0/1 (torch.bool storage), i < n.
 * Replaces IsnanFwdKernel.forward (tileops/kernels/elementwise/isnan/isnan.py:142-156),
 * IsinfFwdKernel.forward (tileops/kernels/elementwise/isinf/isinf.py:150) and
 * IsfiniteFwdKernel.forward (tileops/kernels/elementwise/isfinite/isfinite.py:149).
 */
int tileops_isfp_fwd(int pred, const void* x, uint8_t* y, int64_t n, int dtype,
                     void* stream);

/*
 * Fused gated GELU over x[M, 2N] (gate = x[:, :N], value = x[:, N:]):
 *   approx == 0: y = 0.5 * g * (1 + erf(g / sqrt(2))) * v
 *   approx == 1: y = 0.5 * g * (1 + tanh(sqrt(2/pi) * (g + 0.044715 g^3))) * v
 * fp32 math, one rounding to `dtype`; y is [M, N].
 * Replaces GeluAndMulFwdKernel.forward
 * (tileops/kernels/elementwise/gelu_and_mul/gelu_and_mul.py:140-147) and
 * GeluTanhAndMulFwdKernel.forward
 * (tileops/kernels/elementwise/gelu_tanh_and_mul/gelu_tanh_and_mul.py:143).
 */
int tileops_gated_gelu_fwd(int approx, const void* x, void* y, int64_t M, int64_t N,
                           int dtype, void* stream);

/*
 * Per row m < M of N elements:
 *   r_out = round_dtype(x + residual)
 *   y     = round_dtype((r_out - mean) * rsqrt(var + eps) * w + b)
 * with biased variance of the rounded sum, fp32 statistics.  x, residual,
 * y, r_out are `dtype`; w and b are `wdtype` (the same as `dtype`, or
 * TILEOPS_F32).
 * Replaces FusedAddLayerNormKernel.forward
 * (tileops/kernels/norm/fused_add_layer_norm/fused_add_layer_norm.py:131-159).
 */
int tileops_fused_add_layernorm_fwd(const void* x, const void* residual,
                                    const void* w, const void* b, void* y,
                                    void* r_out, int64_t M, int64_t N, float eps,
                                    int dtype, int wdtype, void* stream);

/*
 * y[m] = log(sum_j exp(x[m, j])) over rows of N, fp32 accumulation, rounded
 * to `dtype`.  A row whose maximum is +-inf gives that infinity; NaN
 * propagates.
 * Replaces the npub::logsumexp_fwd custom op called by LogSumExpKernel.forward
 * (tileops/kernels/reduction/logsumexp/logsumexp.py:115-132, 321-336).
 */
int tileops_logsumexp_fwd(const void* x, void* y, int64_t M, int64_t N, int dtype,
                          void* stream);

/*
 * y[m] = index (int64) of the first maximum (is_min == 0) or first minimum
 * (is_min != 0) of row m of N elements; NaN counts as the extreme value, and
 * among equal values the lowest index wins (torch.argmax / argmin).
 * Replaces the npub::argreduce_fwd custom op called by ArgreduceKernel.forward
 * (tileops/kernels/reduction/argmax/argmax.py:67-76, 195-219).
 */
int tileops_argreduce_fwd(const void* x, int64_t* y, int64_t M, int64_t N, int dtype,
                          int is_min, void* stream);

/*
 * Flash attention forward, BSHD layout.
 *   q:    [B, Sq,  H,   D]    k, v: [B, Skv, Hkv, D]   (dtype F16 or BF16)
 *   o:    [B, Sq,  H,   D]    lse:  [B, H, Sq] float32 (log2 domain:
 *                               logsumexp(scale * q k^T, masked) / ln 2)
 * Causal masking is right-aligned: query i sees keys j <= i + (Skv - Sq).
 * H % Hkv == 0 (grouped-query sharing); D must be 64, 96, 128, 192 or 256.
 * softcap > 0 caps the scores, softcap * tanh(scale q.k / softcap), before
 * the mask and the softmax (the lse is then of the capped scores); 0 turns
 * it off; negative, NaN or infinite values are TILEOPS_EINVAL.
 * Replaces the npub::gqa_prefill_fwd_wrapped_kernel custom op called by
 * GQAPrefillFwdKernel.forward
 * (tileops/kernels/attention/multi_head_attention/multi_head_attention.py:77-124, 255-).
 */
int tileops_mha_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                    int64_t B, int64_t Sq, int64_t Skv, int64_t H, int64_t Hkv,
                    int64_t D, int causal, float scale, float softcap, int dtype,
                    void* stream);

/*
 * Chunked gated delta rule (gated DeltaNet) prefill, per (b, h):
 *   S_t = exp(g_t) S_{t-1} + beta_t k_t (v_t - k_t^T exp(g_t) S_{t-1})^T
 *   o_t = scale * q_t^T S_t
 * q, k: [B, T, H, K]  v: [B, T, H, V]  (BF16)   g, beta: [B, T, H] (F32,
 * g is the log-decay)   h0: [B, H, K, V] F32 or NULL (zero state)
 * o: [B, T, H, V] BF16   hT: [B, H, K, V] F32 (final state).
 * K and V must be 128; chunk must be 64.  `ws` is a device workspace of at
 * least tileops_gdn_prefill_workspace_bytes(...) bytes (0 when the sequence
 * runs as one segment; `ws` may then be NULL).
 * No reference kernel exists (GatedDeltaNetPrefillFwdOp was not delivered,
 * MIGRATION_INDEX.md:28); the recurrence follows golden_gdn_sequential
 * (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77) and the chunked
 * form of examples/gdn_prefill/DESIGN.md:6-17.
 */
int tileops_gdn_prefill_fwd(const void* q, const void* k, const void* v,
                            const float* g, const float* beta, const float* h0,
                            void* o, float* hT, int64_t B, int64_t T, int64_t H,
                            int64_t K, int64_t V, int64_t chunk, float scale,
                            int dtype, void* ws, size_t ws_bytes, void* stream);

size_t tileops_gdn_prefill_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t K,
                                           int64_t V, int64_t chunk);

/*
 * tileops_gdn_prefill_fwd with the number of sequence segments chosen by
 * the caller (0: the library's choice, as tileops_gdn_prefill_fwd; 1 .. 16:
 * that many, at most one per chunk).  Segments run in parallel, each with
 * its own state map; the workspace holds the maps
 * (tileops_gdn_prefill_workspace_bytes_ex with the same `segments`).
 * Same interface origin as tileops_gdn_prefill_fwd; the segment count is a
 * scheduling knob of this implementation (the reference's
 * GatedDeltaNetPrefillFwdOp plan names only chunk_size).
 */
int tileops_gdn_prefill_fwd_ex(const void* q, const void* k, const void* v,
                               const float* g, const float* beta, const float* h0,
                               void* o, float* hT, int64_t B, int64_t T, int64_t H,
                               int64_t K, int64_t V, int64_t chunk, float scale,
                               int dtype, int64_t segments, void* ws, size_t ws_bytes,
                               void* stream);

size_t tileops_gdn_prefill_workspace_bytes_ex(int64_t B, int64_t T, int64_t H, int64_t K,
                                              int64_t V, int64_t chunk, int64_t segments);

/*
 * tileops_gdn_prefill_fwd without a workspace argument, for callers that
 * cannot allocate device memory (code under stream capture, serving loops,
 * harnesses that forbid allocation): it allocates nothing and calls no
 * allocating routine.  No counterpart in the reference.  The segment maps
 * live in a 32 MiB device array of the library (one per GPU, held until
 * the process ends): a call uses as many segments N as the array holds
 * (B * H * (2 N - 3) maps of 64 KiB), down to one segment, which needs no
 * array, so every B, T and H is accepted.  Calls that use the array run one
 * after another on the device: each waits for the previous such call's
 * completion event, whatever stream it ran on (once per device, at the
 * first call, the library creates that event and looks up the array's
 * address).  Under stream capture the event is not used, and captured calls
 * on parallel branches of one graph race on the array.  Results equal
 * tileops_gdn_prefill_fwd_ex's with the same segment count bit for bit.
 */
int tileops_gdn_prefill_fwd_noalloc(const void* q, const void* k, const void* v,
                                    const float* g, const float* beta, const float* h0,
                                    void* o, float* hT, int64_t B, int64_t T, int64_t H,
                                    int64_t K, int64_t V, int64_t chunk, float scale,
                                    int dtype, void* stream);

/*
 * Single-token gated linear attention decode, layout BHD, per (b, h):
 *   new_state[dk][dv] = exp(gk[dk]) * state[dk][dv] + k[dk] * v[dv]
 *   o[dv]             = scale * sum_dk q[dk] * new_state[dk][dv]
 * q, k, gk: [B, H, DK]   v, o: [B, H, DV]   state, new_state: [B, H, DK, DV],
 * all of `dtype` (F32, F16 or BF16); fp32 arithmetic, the readout from the
 * unrounded new state.  scale > 0 (the caller resolves its default
 * DK ** -0.5).  DV <= 256, or DV * element size a multiple of 16 with at
 * most 256 such 16-byte groups (TILEOPS_ESHAPE otherwise).
 * Replaces the kernel program GLADecodeKernel.forward runs
 * (tileops/kernels/linear_attention/gla_decode/gla_decode.py:57-66; op
 * interface tileops/ops/linear_attention/gla_decode.py:24-77).
 */
int tileops_gla_decode_fwd(const void* q, const void* k, const void* v, const void* gk,
                           const void* state, void* o, void* new_state, int64_t B, int64_t H,
                           int64_t DK, int64_t DV, float scale, int dtype, void* stream);

/*
 * Single-token gated delta rule (gated DeltaNet) decode, per (b, h):
 *   new_state = exp(g) state + beta k (v - k^T exp(g) state)^T
 *   o         = scale * q^T new_state
 * (one step of the recurrence tileops_gdn_prefill_fwd runs over a sequence,
 * on its state layout).  q, k: [B, H, DK]   v, o: [B, H, DV]  of `dtype`
 * (F32, F16 or BF16)   g, beta: [B, H] F32 (g is the log-decay)
 * state, new_state: [B, H, DK, DV] F32, 16-byte aligned; new_state may be
 * state itself (the step then runs in place).  fp32 arithmetic.  DK a
 * multiple of 32 up to 256, DV a multiple of 32 up to 4096, B * H * DV / 32
 * at most 2^31 - 1 (TILEOPS_ESHAPE otherwise); scale finite.
 * No reference kernel or op exists; the step is one token of
 * golden_gdn_sequential (examples/gdn_prefill/probe/gdn_prefill_probe.py:60-77)
 * and its interface follows GLADecodeOp.forward
 * (tileops/ops/linear_attention/gla_decode.py:24-77) with GDN's g and beta.
 */
int tileops_gdn_decode_fwd(const void* q, const void* k, const void* v, const float* g,
                           const float* beta, const float* state, void* o, float* new_state,
                           int64_t B, int64_t H, int64_t DK, int64_t DV, float scale, int dtype,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEOPS_HIP_H */
