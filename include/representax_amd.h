/*
 * representax_amd: MI355X (gfx950) kernels for representax's quantized-linear
 * path, behind a plain C ABI.
 *
 * Conventions
 *   - Every pointer is a device pointer unless the name says host.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). All work
 *     is enqueued on it; no entry point allocates device memory, and none
 *     synchronizes except the diagnostic rpx_check_device_errors. Scratch
 *     comes from the caller's `workspace`, sized by the matching
 *     *_workspace() query.
 *   - bf16 tensors are passed as their 16-bit patterns; fp8 tensors as uint8
 *     codes in the OCP e4m3fn / e5m2 encodings.
 *   - Matrices are row-major and dense unless strides are given.
 *   - Return value: RPX_OK, or an error code with a message available from
 *     rpx_last_error() (thread local). Invalid arguments are rejected before
 *     anything is launched.
 *
 * The reference (ckgresla/representax) is pure JAX; it has no native FFI. Each
 * entry point below names the reference function whose numerics it replaces;
 * those functions would call it through jax.ffi custom calls.
 */
#ifndef REPRESENTAX_AMD_H_
#define REPRESENTAX_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RPX_ABI_VERSION 1

#define RPX_OK 0
#define RPX_ERR_INVALID 1
#define RPX_ERR_HIP 2
#define RPX_ERR_DEVICE 3 /* a kernel reported a problem (rpx_check_device_errors) */

#define RPX_DTYPE_F32 0
#define RPX_DTYPE_BF16 1

#define RPX_FP8_E4M3FN 0
#define RPX_FP8_E5M2 1

const char* rpx_last_error(void);
int rpx_abi_version(void);

/* ---------------------------------------------------------------------------
 * Kernel-variant overrides ("knobs"), process-wide, for tests that cover every
 * tile shape and for tuning sweeps. No reference counterpart (XLA picks its
 * own kernels). Each knob starts from its environment variable, read once;
 * rpx_set_tuning applies to calls that start after it. Workspace queries
 * follow the knobs too, so a knob must not change between a *_workspace()
 * query and the call it sizes.
 *   RPX_TUNE_INT4_TILE   INT4 fused GEMM tile: 0 planner, 1 256x128, 2 128x128
 *                        (stages by scale footprint), 3 64x128, 7 256x256,
 *                        10 128x128 two stages, 11 128x128 three stages,
 *                        12 256x128 two stages (env RPX_GEMM_TILE)
 *   RPX_TUNE_BF16_TILE   bf16 GEMM tile: 0 planner, 4 256x128, 5 128x128,
 *                        6 64x128, 8 256x256, 9 128x96, 13 256x128 three
 *                        stages; for the input gradient read from the packed
 *                        weight: 14 256x128, 15 128x128, 16 64x128
 *                        (env RPX_GEMM_TILE)
 *   RPX_TUNE_FP8_TILE    fp8 GEMM tile: 0 planner, 1..11 (env RPX_FP8_TILE)
 *   RPX_TUNE_SKINNY_TILE one-launch skinny tile: 0 planner, 1..15; a nonzero
 *                        value also turns the two-launch form off
 *                        (env RPX_SKINNY_TILE)
 *   RPX_TUNE_SKINNY2     two-launch skinny form: -1 planner (M <= 4), 0 never,
 *                        1 for every M <= 16 (env RPX_SKINNY2)
 *   RPX_TUNE_SKINNY2_ONE M <= 4 form: -1 planner (one launch where the rank is a
 *                        multiple of 8 and B 16-byte aligned), 0 two
 *                        launches, 1 one launch (env RPX_SKINNY2_ONE)
 *   RPX_TUNE_SPIN_LIMIT  polls of the skinny kernels' bounded cross-block
 *                        waits (0: the default limit)
 *   RPX_TUNE_GEMM_BAND   row-blocks per band of the bf16, INT4 and fp8 GEMMs'
 *                        tile order: 0 planner, 1 (row-major) .. 64
 *                        (env RPX_GEMM_BAND)
 *   RPX_TUNE_DX_PACKED   INT4 + LoRA input gradient's weight operand: -1
 *                        planner (a bf16 W_b^T written first), 0 the same,
 *                        1 the packed weight dequantized inside the GEMM,
 *                        where the shape allows (env RPX_DX_PACKED)
 *   RPX_TUNE_RANK_BLOCKS workgroups each token-reduction product of the
 *                        LoRA backward (dA, dB) is split for: 0 planner,
 *                        16..8192
 *   RPX_TUNE_RANK_NT_U   128-column steps each wave of the rank-r row kernel
 *                        (h = x A^T, dh = g_a B) keeps in flight: 0 planner,
 *                        4, 8, 16
 *   RPX_TUNE_FP8_SPLITS  fp8 GEMM split-K count: 0 planner, 1..32 where the
 *                        128-deep K slices split into exactly that many
 *                        parts (otherwise the planner's count)
 *   RPX_TUNE_FP8_PAIR    fp8 linear backward's input and weight gradients in
 *                        one launch: -1 planner (where both products' tiles
 *                        allow it), 0 two launches (env RPX_FP8_PAIR)
 * ------------------------------------------------------------------------- */
#define RPX_TUNE_INT4_TILE 0
#define RPX_TUNE_BF16_TILE 1
#define RPX_TUNE_FP8_TILE 2
#define RPX_TUNE_SKINNY_TILE 3
#define RPX_TUNE_SKINNY2 4
#define RPX_TUNE_SKINNY2_ONE 5
#define RPX_TUNE_SPIN_LIMIT 6
#define RPX_TUNE_GEMM_BAND 7
#define RPX_TUNE_DX_PACKED 8
#define RPX_TUNE_RANK_BLOCKS 9
#define RPX_TUNE_RANK_NT_U 10
#define RPX_TUNE_FP8_SPLITS 11
#define RPX_TUNE_FP8_PAIR 12

/* RPX_ERR_INVALID for an unknown knob or value. */
int rpx_set_tuning(int knob, int value);
/* Current value (0 for an unknown knob). */
int rpx_get_tuning(int knob);

/* Kernels with bounded cross-block waits (the one-launch skinny-M forward)
 * raise a bit in a per-device error word when a wait expires; that call's
 * outputs then hold NaN instead of hanging. This takes the current device's
 * word with one atomic exchange (queued on `stream`, after the work already
 * there; a bit raised later by another stream's kernel stays for the next
 * check), synchronizes `stream`, and returns RPX_ERR_DEVICE (with a
 * message naming the kernel) if any bit was set; flags_out (host, may be
 * NULL) receives the bits: 1 = skinny M <= 64 adapter arrivals, 2 = skinny
 * M <= 4 adapter partials. Synchronizes, so it must not be called during graph
 * capture. No reference counterpart (XLA's kernels have no cross-block waits). */
int rpx_check_device_errors(void* stream, uint32_t* flags_out);

/* ---------------------------------------------------------------------------
 * Packed INT4 weights.
 *   packed     uint8 [n, ceil(k/2)]  low nibble = even column, two's
 *                                    complement int4
 *   scale_bits uint16[n, k/group]    bf16 bit patterns
 * group_size <= 0 or == k selects one scale per output row, the reference's
 * scheme; other values must divide k and be even (an extension).
 * ------------------------------------------------------------------------- */

/* Quantize weight [n, k] (f32 or bf16). Replaces _pack_int4_rows,
 * src/representax/models/adapters.py:38-65 (and _bits_from_bfloat16, :30-31). */
int rpx_int4_pack(const void* weight, int dtype, int64_t n, int64_t k, int64_t group_size,
                  uint8_t* packed, uint16_t* scale_bits, void* stream);

/* Dequantize to bf16 bits out [n, k]: bf16(q * s), bit-exact. Replaces
 * _unpack_int4_rows / QuantizedLoRALinear.base_weight,
 * src/representax/models/adapters.py:68-79,141-148. */
int rpx_int4_dequant(const uint8_t* packed, const uint16_t* scale_bits, int64_t n, int64_t k,
                     int64_t group_size, uint16_t* out, void* stream);

/* Merged float32 export weight out [n, k] = f32(W_b) + (B @ A) * scaling with
 * float32 masters lora_a [rank, k], lora_b [n, rank]. Replaces
 * QuantizedLoRALinear.merged_weight, src/representax/models/adapters.py:150-156. */
int rpx_int4_merge(const uint8_t* packed, const uint16_t* scale_bits, const float* lora_a,
                   const float* lora_b, int64_t n, int64_t k, int64_t group_size, int64_t rank,
                   float scaling, float* out, void* stream);

/* ---------------------------------------------------------------------------
 * INT4 base + LoRA linear. `dtype` is the compute dtype of x, the LoRA compute
 * views lora_a [rank, k] / lora_b [n, rank], y, h, grad and dx. `scaling` is
 * alpha / rank; it is rounded to the compute dtype like the reference's weakly
 * typed Python scalar. bias_bits (bf16 bits [n]) may be NULL.
 * Shapes that take the vectorized kernels (bf16, k a multiple of 64, rank <= 64,
 * per-row scales or power-of-two groups >= 32; the backward also needs n a
 * multiple of 64) need x, packed, scale_bits, lora_a and y (backward: grad, x,
 * packed, scale_bits, lora_a, lora_b and dx) 16-byte aligned, as every
 * hipMalloc'd buffer is; the *_workspace() queries size those kernels'
 * scratch from the shape alone, and a misaligned call is rejected with
 * RPX_ERR_INVALID.
 * ------------------------------------------------------------------------- */

size_t rpx_int4lora_forward_workspace(int64_t m, int64_t n, int64_t k, int64_t group_size,
                                      int64_t rank, int dtype);

/* y [m, n] = x W_b^T + ((x A^T) B^T) * scaling (+ bias), h [m, rank] = x A^T,
 * with the reference's rounding points. Replaces QuantizedLoRALinear.__call__,
 * src/representax/models/adapters.py:158-182. */
int rpx_int4lora_forward(const void* x, int dtype, int64_t m, int64_t k, const uint8_t* packed,
                         const uint16_t* scale_bits, int64_t n, int64_t group_size,
                         const uint16_t* bias_bits, const void* lora_a, const void* lora_b,
                         int64_t rank, float scaling, void* y, void* h, void* workspace,
                         size_t workspace_bytes, void* stream);

/* Several INT4 + LoRA projections of one input x (the q / k / v or gate / up
 * projections of a layer), each with its own weight, scales, adapter, bias
 * and outputs. Every projection's y and h are what rpx_int4lora_forward
 * gives for it, within the same numerics (the fused form may split K
 * differently). No single reference function: it replaces consecutive
 * QuantizedLoRALinear.__call__ on one input (adapters.py:158-182), e.g.
 * bert/model.py's query / key / value and qwen3_vl/text.py's gate / up.
 * For bf16 with M <= 4 (the skinny-M regime), one rank and at most 4
 * projections, all of them run in one launch (one pair of launches when
 * the rank is not a multiple of 8) instead of one or two each. Above the skinny sizes, when every projection takes the fused MFMA
 * path and their ranks add up to at most 128 in 16-rank blocks (q / k / v
 * at rank 16 or 32, gate / up at rank 32), one launch forms every h from one pass
 * over x, bit-identical to the per-projection h, and then each projection's
 * GEMM runs. Otherwise they run one after another. */
typedef struct rpx_int4lora_projection {
  const uint8_t* packed;       /* [n, ceil(k/2)] */
  const uint16_t* scale_bits;  /* [n] or [n, k / group_size] */
  int64_t n;
  int64_t group_size;          /* 0 or k: per-row scales */
  const uint16_t* bias_bits;   /* [n] or NULL */
  const void* lora_a;          /* [rank, k], x's dtype */
  const void* lora_b;          /* [n, rank], x's dtype */
  int64_t rank;
  float scaling;
  void* y;                     /* [m, n] */
  void* h;                     /* [m, rank] */
} rpx_int4lora_projection;

/* Sized from the shapes alone: the pointers may be unset. */
size_t rpx_int4lora_forward_multi_workspace(int64_t m, int64_t k, int count,
                                            const rpx_int4lora_projection* projections,
                                            int dtype);
int rpx_int4lora_forward_multi(const void* x, int dtype, int64_t m, int64_t k, int count,
                               const rpx_int4lora_projection* projections, void* workspace,
                               size_t workspace_bytes, void* stream);

/* rpx_int4lora_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc); no counterpart in the reference. Scratch
 * (the skinny-M kernels' split partials) comes from a static device buffer of
 * RPX_STATIC_SCRATCH_BYTES per GPU that the library holds until the process
 * ends; the entry point itself calls no allocator. A call that needs more
 * scratch than that (rpx_int4lora_forward_workspace() above the limit, e.g.
 * the generic path of a large unaligned shape) is rejected with
 * RPX_ERR_INVALID before anything is launched. Every call on a GPU shares that
 * GPU's buffer: calls that overlap on one GPU (different streams) race. */
#define RPX_STATIC_SCRATCH_BYTES (16u << 20)
int rpx_int4lora_forward_static(const void* x, int dtype, int64_t m, int64_t k,
                                const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                                int64_t group_size, const uint16_t* bias_bits, const void* lora_a,
                                const void* lora_b, int64_t rank, float scaling, void* y, void* h,
                                void* stream);

size_t rpx_int4lora_backward_workspace(int64_t m, int64_t n, int64_t k, int64_t group_size,
                                       int64_t rank, int dtype);

/* dx [m, k], d_lora_a f32 [rank, k], d_lora_b f32 [n, rank] from grad [m, n]
 * and the forward's h. Replaces JAX's transpose of
 * src/representax/models/adapters.py:162-181 (the reference has no
 * hand-written VJP for this path). */
int rpx_int4lora_backward(const void* grad, const void* x, int dtype, int64_t m, int64_t k,
                          const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                          int64_t group_size, const void* lora_a, const void* lora_b,
                          int64_t rank, float scaling, const void* h, void* dx, float* d_lora_a,
                          float* d_lora_b, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * INT4 base + LoRA linear without a precision policy, on bf16 activations
 * with the float32 adapter masters: the reference then multiplies bf16 x
 * (bf16 base) -> bf16, but jnp.matmul promotes bf16 x float32 to float32, so
 * h = f32(x A^T), the adapter term and the module output are float32:
 *   y [m, n] f32 = f32(bf16(x W_b^T)) + f32(f32(h B^T) * scaling) (+ f32(bias))
 * with scaling = float32(alpha / rank) (not rounded to bf16). Replaces
 * QuantizedLoRALinear.__call__, src/representax/models/adapters.py:158-182,
 * with compute_parameter returning the masters unchanged
 * (src/representax/precision.py:111-117), as in inference without a
 * precision context (src/representax/inference.py:17-23).
 * ------------------------------------------------------------------------- */

size_t rpx_int4lora_forward_promoted_workspace(int64_t m, int64_t n, int64_t k,
                                               int64_t group_size, int64_t rank);

int rpx_int4lora_forward_promoted(const uint16_t* x, int64_t m, int64_t k, const uint8_t* packed,
                                  const uint16_t* scale_bits, int64_t n, int64_t group_size,
                                  const uint16_t* bias_bits, const float* lora_a,
                                  const float* lora_b, int64_t rank, float scaling, float* y,
                                  float* h, void* workspace, size_t workspace_bytes,
                                  void* stream);

size_t rpx_int4lora_backward_promoted_workspace(int64_t m, int64_t n, int64_t k,
                                                int64_t group_size, int64_t rank);

/* JAX's transpose of the promoted forward, grad [m, n] f32 (the float32
 * output's cotangent): dx [m, k] bf16 = bf16(bf16(bf16(g) W_b) +
 * bf16(f32(dh A))) with dh = f32(f32(g * scaling) B); d_lora_a = f32(dh^T x),
 * d_lora_b = f32(f32(g * scaling)^T h), both float32 (no bf16 rounding).
 * Replaces JAX's transpose of src/representax/models/adapters.py:162-181. */
int rpx_int4lora_backward_promoted(const float* grad, const uint16_t* x, int64_t m, int64_t k,
                                   const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                                   int64_t group_size, const float* lora_a, const float* lora_b,
                                   int64_t rank, float scaling, const float* h, uint16_t* dx,
                                   float* d_lora_a, float* d_lora_b, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Activation epilogues: the FFN steps on either side of an INT4 + LoRA linear,
 * fused into its GEMMs. Activations run in f32 on the bf16 operands and are
 * rounded once; bf16 compute only. All [m, n] operands are dense row-major.
 * ------------------------------------------------------------------------- */

#define RPX_ACT_GELU 1     /* gelu(z) = z (1 + erf(z / sqrt 2)) / 2: activate("gelu"),
                              src/representax/models/components.py:159-160, as in
                              BertMLP, src/representax/models/bert/model.py:249 */
#define RPX_ACT_SILU_MUL 2 /* silu(gate) * z: the Qwen3 MLP's gated product,
                              src/representax/models/qwen3_vl/text.py:202 */
#define RPX_ACT_ADD 3      /* backward only: dz = d + z, the input gradient added to
                              the one accumulated so far for an input several
                              linears share (JAX's cotangent sum of, e.g., the
                              q/k/v projections' input, qwen3_vl/text.py and
                              bert/model.py attention) */

/* The FFN's up projection with its activation: z [m, n] = the linear's output
 * (as rpx_int4lora_forward's y), y [m, n] = gelu(z) (RPX_ACT_GELU) or
 * silu(gate) * z (RPX_ACT_SILU_MUL, gate [m, n] the gate projection's
 * output), h as in rpx_int4lora_forward. Workspace: rpx_int4lora_forward_workspace.
 * Replaces activate(self.input(hidden)) (bert/model.py:249) and
 * jax.nn.silu(self.gate(x)) * self.up(x) (qwen3_vl/text.py:202). */
int rpx_int4lora_forward_act(const void* x, int dtype, int64_t m, int64_t k, const uint8_t* packed,
                             const uint16_t* scale_bits, int64_t n, int64_t group_size,
                             const uint16_t* bias_bits, const void* lora_a, const void* lora_b,
                             int64_t rank, float scaling, int act, const void* gate, void* y,
                             void* z, void* h, void* workspace, size_t workspace_bytes,
                             void* stream);

/* The FFN's down projection backward followed by the activation's backward:
 * x [m, k] is the down projection's input (the activation output), z [m, k]
 * and gate [m, k] the forward's operands of the activation. With d = the
 * down projection's input gradient (rpx_int4lora_backward's dx, rounded):
 *   RPX_ACT_GELU:     dz = d * gelu'(z);
 *   RPX_ACT_SILU_MUL: dz = d * silu(gate) (the up projection's gradient),
 *                     dgate = d * z * silu'(gate) (the gate projection's);
 *   RPX_ACT_ADD:      dz = d + z (z the gradient accumulated so far; dz must
 *                     not alias z).
 * d_lora_a / d_lora_b as in rpx_int4lora_backward; workspace:
 * rpx_int4lora_backward_workspace. Replaces JAX's transpose of the same
 * expressions. */
int rpx_int4lora_backward_act(const void* grad, const void* x, int dtype, int64_t m, int64_t k,
                              const uint8_t* packed, const uint16_t* scale_bits, int64_t n,
                              int64_t group_size, const void* lora_a, const void* lora_b,
                              int64_t rank, float scaling, const void* h, int act, const void* z,
                              const void* gate, void* dz, void* dgate, float* d_lora_a,
                              float* d_lora_b, void* workspace, size_t workspace_bytes,
                              void* stream);

/* ---------------------------------------------------------------------------
 * Dynamically scaled fp8.
 * ------------------------------------------------------------------------- */

size_t rpx_fp8_scale_workspace(int64_t numel);

/* scale_out[0] = max(max|t| / fmax, FLT_MIN) over numel dense elements (NaN
 * propagates). Replaces the scale half of _scaled_quantize,
 * src/representax/precision.py:133-139. */
int rpx_fp8_scale(const void* t, int dtype, int64_t numel, int fmt, float* scale_out,
                  void* workspace, size_t workspace_bytes, void* stream);

/* codes = f8(f32(t) / scale) for the logical matrix t[r * row_stride +
 * c * col_stride] (rows x cols); writes out [rows, cols] and/or out_t
 * [cols, rows] (either may be NULL). Replaces the cast half of
 * _scaled_quantize, src/representax/precision.py:140. */
int rpx_fp8_cast(const void* t, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                 int64_t col_stride, const float* scale, int fmt, uint8_t* out, uint8_t* out_t,
                 void* stream);

size_t rpx_fp8_gemm_workspace(int64_t m, int64_t n, int64_t k);

/* out [m, n] = ((a [m, k] . b [n, k]^T) * scale_a) * scale_b on fp8 codes, f32
 * accumulate. Replaces the dot_general + rescale of _scaled_fp8_dot,
 * src/representax/precision.py:154-170. */
int rpx_fp8_gemm(const uint8_t* a, int fmt_a, const float* scale_a, const uint8_t* b, int fmt_b,
                 const float* scale_b, int64_t m, int64_t n, int64_t k, void* out, int out_dtype,
                 void* workspace, size_t workspace_bytes, void* stream);

size_t rpx_fp8_linear_forward_workspace(int64_t m, int64_t n, int64_t k);

/* out [m, n] = _fp8_linear_dot(left [m, k], right [k, n]) with e4m3 operands;
 * right is addressed through (row_stride, col_stride) so a transposed weight
 * view needs no copy. scales_out[0..1] receive (s_left, s_right). The same
 * pass can also write the backward's operand codes: left_codes [m, k]
 * (row-major, the product's own) and right_codes [k, n] (either may be
 * NULL). m, n, k > 0: an empty operand has no amax, and the reference's max
 * reduction raises on it. Replaces _fp8_linear_dot /
 * _fp8_linear_dot_forward, src/representax/precision.py:173-198 (as used by
 * linear_matmul, :224-239). */
int rpx_fp8_linear_forward(const void* left, int left_dtype, int64_t m, int64_t k,
                           const void* right, int right_dtype, int64_t n, int64_t right_row_stride,
                           int64_t right_col_stride, void* out, int out_dtype, float* scales_out,
                           uint8_t* left_codes, uint8_t* right_codes, void* workspace,
                           size_t workspace_bytes, void* stream);

size_t rpx_fp8_linear_backward_workspace(int64_t m, int64_t n, int64_t k);

/* d_left [m, k] = scaled_dot(g[e5m2], right^T[e4m3]) and d_right =
 * scaled_dot(left^T[e4m3], g[e5m2]) as [k, n], or as [n, k] when
 * d_right_transposed; either output may be NULL to skip it. `scales` are the
 * forward's (s_left, s_right); the operands are re-quantized with them,
 * which reproduces the reference's recomputed amax exactly. m, n, k > 0.
 * Replaces _fp8_linear_dot_backward, src/representax/precision.py:201-218. */
int rpx_fp8_linear_backward(const void* left, int left_dtype, const void* right, int right_dtype,
                            int64_t m, int64_t k, int64_t n, int64_t right_row_stride,
                            int64_t right_col_stride, const void* grad, int grad_dtype,
                            const float* scales, void* d_left, void* d_right,
                            int d_right_transposed, int out_dtype, void* workspace,
                            size_t workspace_bytes, void* stream);

/* The same backward from the operand codes that rpx_fp8_linear_forward
 * saved (left_codes [m, k], right_codes [k, n]); the bf16 operands are not
 * read again. Workspace: rpx_fp8_linear_backward_workspace(m, n, k).
 * Replaces _fp8_linear_dot_backward, src/representax/precision.py:201-218. */
int rpx_fp8_linear_backward_codes(const uint8_t* left_codes, const uint8_t* right_codes,
                                  const float* scales, int64_t m, int64_t k, int64_t n,
                                  const void* grad, int grad_dtype, void* d_left, void* d_right,
                                  int d_right_transposed, int out_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* The two products of that backward from the gradient's codes, for a caller
 * that quantizes the gradient itself (delayed scaling):
 *   d_left [m, k] = ((g . right^T) * s_grad) * s_right, from g_codes [m, n]
 *     (e5m2) and right_codes [k, n] (e4m3);
 *   d_right = ((left^T . g) * s_left) * s_grad, as [k, n] or as [n, k] when
 *     d_right_transposed, from the same g_codes and left_codes [m, k]
 *     (e4m3), both row-major: the kernel reads them along the tokens.
 * Either output may be NULL (then its codes and scale may be too). With both
 * outputs and d_right_transposed, the two products run in one launch where
 * their tile plans allow it (RPX_TUNE_FP8_PAIR), with the same results as
 * two launches. m, n, k > 0. Workspace:
 * rpx_fp8_linear_backward_gemms_workspace(m, n, k).
 * Replaces the two _scaled_fp8_dot calls of _fp8_linear_dot_backward,
 * src/representax/precision.py:201-218. */
int rpx_fp8_linear_backward_gemms(const uint8_t* g_codes, const float* s_grad,
                                  const uint8_t* left_codes, const float* s_left,
                                  const uint8_t* right_codes, const float* s_right, int64_t m,
                                  int64_t k, int64_t n, void* d_left, void* d_right,
                                  int d_right_transposed, int out_dtype, void* workspace,
                                  size_t workspace_bytes, void* stream);

size_t rpx_fp8_linear_backward_gemms_workspace(int64_t m, int64_t n, int64_t k);

/* ---------------------------------------------------------------------------
 * Delayed-scale fp8 state, one entry ("slot") per scaled tensor of a model:
 *   scales       float [n_slots]                 scale used by the casts
 *   fmax         float [n_slots]                 448 (e4m3fn) or 57344 (e5m2)
 *   amax_pending uint32 [n_slots, pending_words] maxima recorded since the
 *                                                last update (zero-initialized)
 *   amax_history uint32 [history_len, n_slots]   per-step maxima, ordered f32
 *                                                bits (zero-initialized)
 *   cursor       int32 [1]                       history row the next update
 *                                                writes
 * The reference's dynamic path (rpx_fp8_linear_*) is unchanged; this is its
 * roadmap item "persistent delayed scales and one coalesced update"
 * (todo.org:1149-1154, docs/precision.md:67-71), which it has not built.
 * ------------------------------------------------------------------------- */

/* Words per slot of amax_pending (a slot's maxima are spread over several
 * cache lines so that a cast's blocks do not queue on one word). */
size_t rpx_fp8_delayed_pending_words(void);

/* codes = f8_sat(f32(t) / scales[slot]) for the logical matrix t (as in
 * rpx_fp8_cast; values beyond the format take its largest finite code, NaN
 * stays NaN), in one pass that also records max|t| into the slot's pending
 * maxima (atomic max, so any number of casts may record into one slot). No
 * reference counterpart: the reference computes every scale from the tensor
 * being cast (_scaled_quantize, src/representax/precision.py:127-140). */
int rpx_fp8_cast_delayed(const void* t, int dtype, int64_t rows, int64_t cols, int64_t row_stride,
                         int64_t col_stride, int fmt, const float* scales,
                         uint32_t* amax_pending, int64_t n_slots, int64_t slot, uint8_t* out,
                         uint8_t* out_t, void* stream);

/* Two such casts of one dtype and format in one launch (an fp8 linear's
 * input and weight). No reference counterpart (see above). */
int rpx_fp8_cast_delayed2(const void* t0, int64_t rows0, int64_t cols0, int64_t row_stride0,
                          int64_t col_stride0, int64_t slot0, uint8_t* out0, uint8_t* out_t0,
                          const void* t1, int64_t rows1, int64_t cols1, int64_t row_stride1,
                          int64_t col_stride1, int64_t slot1, uint8_t* out1, uint8_t* out_t1,
                          int dtype, int fmt, const float* scales, uint32_t* amax_pending,
                          int64_t n_slots, void* stream);

/* The once-per-step update of every slot in one launch: the pending maxima
 * go to history row cursor[0] (and are cleared); scales[s] =
 * max(max_h amax_history[h, s] / fmax[s], FLT_MIN) (NaN if a NaN was
 * recorded) for slots whose history holds a nonzero amax (others keep their
 * scale); cursor[0] advances by one, modulo history_len. No reference
 * counterpart (see above). */
int rpx_fp8_scale_update(float* scales, const float* fmax, uint32_t* amax_pending,
                         uint32_t* amax_history, int32_t* cursor, int64_t n_slots,
                         int64_t history_len, void* stream);

/* Test hook: compares the cast kernels' fp8 encoder (hardware convert in
 * range) with the integer encoder for the f32 bit patterns
 * [first, first + count) and their negations; block_counts[b] /
 * block_first[b] receive each block's mismatch count and lowest mismatching
 * pattern (0xFFFFFFFF if none). No reference counterpart. */
int rpx_fp8_encode_selfcheck(int fmt, uint64_t first, uint64_t count, uint32_t* block_counts,
                             uint32_t* block_first, int64_t blocks, void* stream);

/* Host-side test hook: the device quantizer (divide by scale, round to fp8)
 * run on host memory, so that it can be checked exhaustively on a CPU. No
 * reference counterpart. */
int rpx_host_fp8_quantize(const float* host_in, int64_t n, float scale, int fmt,
                          uint8_t* host_out);

/* ---------------------------------------------------------------------------
 * In-batch multiple-negatives ranking loss, fused (the train-step objective
 * next to the path): replaces `mnr_loss_terms(queries, documents,
 * eye(n_queries, n_documents), scale=scale).loss` with unit weights and
 * every row valid, src/representax/tasks/retrieval/mnr.py:48-52
 * (`_normalize`), :132-158 (`_direction_row_terms`), :338-341 (forward
 * loss). The embeddings (f32 or bf16, dense [n, dim]) are cast to f32 and
 * normalised by max(||row||, 1e-12); logits = scale * cosine; loss = mean
 * over queries of logsumexp_j(logits[i, j]) - logits[i, i].
 * Requires 1 <= n_queries <= n_documents <= 8192, 1 <= dim <= 4096 and a
 * finite scale > 0 (the reference's ValueError).
 * ------------------------------------------------------------------------- */
/* Bytes of the buffer the forward fills and the backward reads (0 for an
 * unsupported shape). */
size_t rpx_mnr_saved_bytes(int64_t n_queries, int64_t n_documents, int64_t dim);

/* *loss (device f32) = the loss; `saved` keeps the normalised rows, norms
 * and softmax rows for the backward. */
int rpx_mnr_forward(const void* queries, const void* documents, int dtype, int64_t n_queries,
                    int64_t n_documents, int64_t dim, float scale, float* loss, void* saved,
                    size_t saved_bytes, void* stream);

/* d_queries / d_documents (dtype as the embeddings) = *grad_loss (device
 * f32) times the gradient of the loss, from the forward's `saved`. */
int rpx_mnr_backward(const float* grad_loss, const void* saved, size_t saved_bytes,
                     int64_t n_queries, int64_t n_documents, int64_t dim, float scale,
                     void* d_queries, void* d_documents, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REPRESENTAX_AMD_H_ */
