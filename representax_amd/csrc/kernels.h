// Kernel launchers shared between translation units.
#pragma once

#include "common.h"

namespace rpx {

// Device error word ----------------------------------------------------------
// One word per device that kernels raise bits in (atomic or) when a bounded
// wait expired; read and cleared by rpx_check_device_errors.
constexpr unsigned int kDevErrSkinnyWait = 1u;     // k_skinny: adapter arrivals
constexpr unsigned int kDevErrSkinnyOneWait = 2u;  // k_skinny_one: adapter partials
// This device's word (nullptr if its address could not be resolved).
unsigned int* device_error_word();

// INT4 -----------------------------------------------------------------------
hipError_t launch_int4_dequant(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                               int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                               int64_t group, hipStream_t stream);
hipError_t launch_int4_dequant_t(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                                 int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                                 int64_t group, int64_t ld_out, hipStream_t stream);
hipError_t launch_int4_pack(const void* weight, int dtype, uint8_t* packed, uint16_t* scales,
                            int64_t n, int64_t k, int64_t packed_cols, int64_t n_groups,
                            int64_t group, hipStream_t stream);
hipError_t launch_int4_merge(const uint8_t* packed, const uint16_t* scales, const float* lora_a,
                             const float* lora_b, float* out, int64_t n, int64_t k,
                             int64_t packed_cols, int64_t n_groups, int64_t group, int64_t rank,
                             float scaling, hipStream_t stream);

// GEMM -----------------------------------------------------------------------
// Low-rank epilogue term added to a GEMM tile:
//   t[m, n] = sum_j C(m, j) * R(n, j)      (fp32 accumulate)
//   y       = bf16(bf16(acc) + bf16(bf16(t) * scale))
//   y       = bf16(y + bias[n])             (when bias != nullptr)
// rank == 0 disables the low-rank term.
struct LowRankEpilogue {
  const uint16_t* rows = nullptr;  // R, indexed by (output column n, j)
  int64_t rows_sn = 0, rows_sj = 0;
  const uint16_t* cols = nullptr;  // C, indexed by (output row m, j)
  int64_t cols_sm = 0, cols_sj = 0;
  int64_t rank = 0;
  float scale = 1.0f;
  const uint16_t* bias = nullptr;  // bf16 bits [N]
  // Activation epilogue (ActMode in act.h) on the rounded output v; the
  // [M, N] operands below share the output's row stride.
  int act = 0;
  const uint16_t* aux = nullptr;   // z (GELU backward) or gate (SiLU-mul)
  const uint16_t* aux2 = nullptr;  // up (SiLU-mul backward)
  uint16_t* pre_out = nullptr;     // v itself (forward modes)
  uint16_t* out2 = nullptr;        // d gate (SiLU-mul backward)
};

// Packed INT4 operand [N, K] (row n holds ceil(K/2) bytes).
struct Int4Operand {
  const uint8_t* packed = nullptr;
  int64_t packed_cols = 0;
  const uint16_t* scales = nullptr;
  int64_t n_groups = 1;
  int64_t group = 0;
};

// y[M, N] = epilogue(A[M, K] . W_b[N, K]^T); A bf16 row-major (lda).
hipError_t launch_gemm_int4(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                            int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                            const LowRankEpilogue& epi, hipStream_t stream);
// y[M, N] = epilogue(A[M, K] . B[N, K]^T) with B[n, k] = W_b[k, n], W packed
// INT4 [K rows, N / 2 bytes] (the INT4 + LoRA input gradient, dx = g . W_b,
// without a bf16 copy of W_b^T). Needs N % 128 == 0, K % 64 == 0, per-row
// or 64-column group scales; int4t_gemm_ok() tells.
bool int4t_gemm_ok(int64_t m, int64_t n, int64_t k, int64_t lda, const void* a,
                   const Int4Operand& w);
hipError_t launch_gemm_int4t(const uint16_t* a, int64_t lda, const Int4Operand& w, int64_t m,
                             int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                             const LowRankEpilogue& epi, hipStream_t stream);
// y[M, N] = epilogue(A[M, K] . B[N, K]^T); A, B bf16 row-major.
hipError_t launch_gemm_bf16(const uint16_t* a, int64_t lda, const uint16_t* b, int64_t ldb,
                            int64_t m, int64_t n, int64_t k, uint16_t* out, int64_t ldc,
                            const LowRankEpilogue& epi, hipStream_t stream);
bool gemm_fast_path_ok(int64_t k, int64_t lda, int64_t ldb_elems, const void* a, const void* b,
                       int64_t ldc, const void* out);

// Skinny-M (M <= 64) INT4 + LoRA forward -------------------------------------
int skinny_tile_count();  // one-launch tile ids are 1 .. skinny_tile_count()
bool skinny_ok(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups, int64_t group);
int64_t skinny_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t rank);
hipError_t launch_skinny_forward(const uint16_t* x, int64_t m, int64_t k, const Int4Operand& w,
                                 int64_t n, const uint16_t* lora_a, const uint16_t* lora_b,
                                 int64_t rank, float scale, const uint16_t* bias, uint16_t* y,
                                 uint16_t* h, float* ws, hipStream_t stream);
// M <= 16 (selected for M <= 4): two launches (weight rows over the whole K
// per block with the adapter's fp32 K-slice partials in the same grid, then
// the LoRA finish), no cross-block exchange.
bool skinny2_ok(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups, int64_t group);
bool skinny2_selected(int64_t m, int64_t n, int64_t k, int64_t rank, int64_t n_groups,
                      int64_t group);
hipError_t launch_skinny2_forward(const uint16_t* x, int64_t m, int64_t k, const Int4Operand& w,
                                  int64_t n, const uint16_t* lora_a, const uint16_t* lora_b,
                                  int64_t rank, float scale, const uint16_t* bias, uint16_t* y,
                                  uint16_t* h, float* ws, hipStream_t stream);
int64_t skinny2_workspace_floats(int64_t m, int64_t n, int64_t k, int64_t rank);
// Several projections of one x (same K and rank) in one pair of launches.
struct Skinny2Projection {
  Int4Operand w;
  int64_t n;
  const uint16_t* lora_a;
  const uint16_t* lora_b;
  int64_t rank;
  float scale;
  const uint16_t* bias;
  uint16_t* y;
  uint16_t* h;
};
bool skinny2_multi_ok(int64_t m, int64_t k, int count, const Skinny2Projection* proj);
int64_t skinny2_multi_workspace_floats(int64_t m, int64_t k, int count,
                                       const Skinny2Projection* proj);
hipError_t launch_skinny2_forward_multi(const uint16_t* x, int64_t m, int64_t k, int count,
                                        const Skinny2Projection* proj, float* ws,
                                        hipStream_t stream);

// Elementwise activation transform (ActMode in act.h) over count dense
// elements: out = f(v, aux, aux2), out2 the second output of the SiLU-mul
// backward. out may alias v.
hipError_t launch_act(int mode, const uint16_t* v, const uint16_t* aux, const uint16_t* aux2,
                      int64_t count, uint16_t* out, uint16_t* out2, hipStream_t stream);

// Rank-r kernels --------------------------------------------------------------
// out[M, r] = bf16(sum_k op(A[m, k]) * R[j, k]); op(a) = bf16(a * a_scale) when
// round_a, else a. R bf16 [r, K] row-major (ldr).
hipError_t launch_rank_nt(const uint16_t* a, int64_t lda, const uint16_t* r_mat, int64_t ldr,
                          int64_t m, int64_t rank, int64_t k, bool round_a, float a_scale,
                          uint16_t* out, int64_t ldo, hipStream_t stream);
// h_i = bf16(A . R_i^T) for several R_i [rank_i, K] (row stride K) of one A
// [M, K] in one launch, h_i [M, rank_i] dense; each h_i has the bits
// launch_rank_nt gives it alone. At most rank_nt_max_blocks() 16-rank blocks
// in all (rank_nt_blocks_of(rank_i) each), else hipErrorInvalidValue.
int rank_nt_blocks_of(int64_t rank);
constexpr int rank_nt_max_blocks() { return 8; }
hipError_t launch_rank_nt_multi(const uint16_t* a, int64_t lda, int64_t m, int64_t k, int count,
                                const uint16_t* const* r_mats, const int64_t* ranks,
                                uint16_t* const* outs, hipStream_t stream);
// out[P, Q] = f32(bf16(sum_m op(X[m, p]) * Y[m, q])); X [M, P] (ldx), Y [M, Q] (ldy)
// bf16 row-major; op as above on X. Uses `partials` (fp32) workspace of
// rank_tn_workspace_floats(...) elements.
int64_t rank_tn_workspace_floats(int64_t m, int64_t p, int64_t q);
hipError_t launch_rank_tn(const uint16_t* x, int64_t ldx, const uint16_t* y, int64_t ldy,
                          int64_t m, int64_t p, int64_t q, bool round_x, float x_scale,
                          float* partials, float* out, hipStream_t stream);
// Two independent products of the form above in one launch (plus one reduce
// launch); each takes its own partials region. x1 == nullptr: first only.
hipError_t launch_rank_tn2(const uint16_t* x0, int64_t ldx0, const uint16_t* y0, int64_t ldy0,
                           int64_t m0, int64_t p0, int64_t q0, bool round_x0, float x_scale0,
                           float* partials0, float* out0, const uint16_t* x1, int64_t ldx1,
                           const uint16_t* y1, int64_t ldy1, int64_t m1, int64_t p1, int64_t q1,
                           bool round_x1, float x_scale1, float* partials1, float* out1,
                           hipStream_t stream);
// B^T [r, N], A^T [K, r] and W_b^T [K, N] (groups that are multiples of 32)
// in one launch; wt == nullptr skips W_b^T.
hipError_t launch_int4lora_bwd_prep(const uint16_t* b, uint16_t* bt, const uint16_t* a,
                                   uint16_t* at, const uint8_t* packed, const uint16_t* scales,
                                   uint16_t* wt, int64_t n, int64_t k, int64_t rank,
                                   int64_t packed_cols, int64_t n_groups, int64_t group,
                                   hipStream_t stream);
hipError_t launch_transpose_bf16(const uint16_t* in, int64_t rows, int64_t cols, int64_t ld_in,
                                 uint16_t* out, int64_t ld_out, hipStream_t stream);
hipError_t launch_fill_f32(float* out, int64_t n, float v, hipStream_t stream);
hipError_t launch_f32_to_bf16(const float* in, uint16_t* out, int64_t n, hipStream_t stream);

// Generic (any shape, any dtype) reference-shaped kernels --------------------
// out[M, N] (fp32) = sum_k A(m, k) * B(n, k) with strided operands.
// a_dtype/b_dtype: kF32 or kBF16; b_int4 replaces B with the packed operand
// W_b, read as B(n, k) = W_b[n, k], or W_b[k, n] when int4_transposed.
hipError_t launch_generic_gemm(const void* a, int a_dtype, int64_t a_sm, int64_t a_sk,
                               const void* b, int b_dtype, int64_t b_sn, int64_t b_sk,
                               const Int4Operand* b_int4, bool int4_transposed, int64_t m,
                               int64_t n, int64_t k, float* out, hipStream_t stream);
hipError_t launch_round_store(const float* in, int64_t n, int dtype, void* out,
                              hipStream_t stream);

// FP8 ------------------------------------------------------------------------
int64_t fp8_amax_partials(int64_t numel);
// Per-block max |t| partials; with scale_out, also the finalized scale.
hipError_t launch_fp8_amax(const void* t, int dtype, int64_t numel, uint32_t* partials,
                           int64_t n_partials, int fmt, float* scale_out, hipStream_t stream);
// codes = f8(t / s) where s is scale[0], or, when partials is given, the
// scale finalized from those amax partials (also written to scale_out).
hipError_t launch_fp8_cast(const void* t, int dtype, int64_t rows, int64_t cols, int64_t s_row,
                           int64_t s_col, const float* scale, const uint32_t* partials,
                           int64_t n_partials, float* scale_out, int fmt, uint8_t* out,
                           uint8_t* out_t, hipStream_t stream);
// Two amax problems (partials only) in one launch.
hipError_t launch_fp8_amax2(const void* t0, int dtype0, int64_t numel0, uint32_t* partials0,
                            int64_t n_partials0, const void* t1, int dtype1, int64_t numel1,
                            uint32_t* partials1, int64_t n_partials1, hipStream_t stream);
// Two casts with scales finalized from their amax partials, one format; one
// launch when both take the row-major tile path with the same input type.
hipError_t launch_fp8_cast2(const void* t0, int dtype0, int64_t rows0, int64_t cols0,
                            int64_t s_row0, int64_t s_col0, const uint32_t* partials0,
                            int64_t n_partials0, float* scale_out0, uint8_t* out0,
                            uint8_t* out_t0, const void* t1, int dtype1, int64_t rows1,
                            int64_t cols1, int64_t s_row1, int64_t s_col1,
                            const uint32_t* partials1, int64_t n_partials1, float* scale_out1,
                            uint8_t* out1, uint8_t* out_t1, int fmt, hipStream_t stream);
// Partials a quantize call needs for a [rows, cols] tensor.
int64_t fp8_quant_partials(int64_t rows, int64_t cols);
// One or two tensors (t1 == nullptr for one), each with its own dynamic
// scale (written to scale_out*): amax, then codes in the requested layouts.
// Row-major inputs of one type take a tile-mapped amax whose blocks touch the
// same tiles, on the same XCDs, as the cast's.
hipError_t launch_fp8_quantize2(const void* t0, int dtype0, int64_t rows0, int64_t cols0,
                                int64_t s_row0, int64_t s_col0, uint32_t* partials0,
                                float* scale_out0, uint8_t* out0, uint8_t* out_t0, const void* t1,
                                int dtype1, int64_t rows1, int64_t cols1, int64_t s_row1,
                                int64_t s_col1, uint32_t* partials1, float* scale_out1,
                                uint8_t* out1, uint8_t* out_t1, int fmt, hipStream_t stream);
hipError_t launch_fp8_gemm(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b,
                           int fmt_b, const float* s_b, int64_t m, int64_t n, int64_t k,
                           void* out, int out_dtype, int64_t ldc, float* split_ws,
                           int64_t split_ws_floats, hipStream_t stream);
int64_t fp8_gemm_workspace_floats(int64_t m, int64_t n, int64_t k);
// The fp8 linear backward's d_left [m, k] = g . right^T and d_right^T [n, k]
// = g^T . left (codes: g [m, n] e5m2, right^T [k, n] and left [m, k] e4m3)
// in one launch, where both plans allow it; *launched says whether it did
// (otherwise nothing was launched).
hipError_t launch_fp8_backward_pair(const uint8_t* g, const uint8_t* right_codes,
                                    const uint8_t* left_codes, const float* s_g,
                                    const float* s_right, const float* s_left, int64_t m,
                                    int64_t k, int64_t n, void* d_left, void* d_right_t,
                                    int out_dtype, float* split_ws, int64_t split_ws_floats,
                                    hipStream_t stream, bool* launched);
// out [m, n] = ((a^T . b) * s_a) * s_b from K-row codes a [k, m] and b [k, n]
// (row strides m and n): k % 128 == 0, m % 16 == 0, n % 16 == 0, 16-byte
// aligned operands; split_ws as fp8_gemm_krows_workspace_floats(m, n, k).
int64_t fp8_gemm_krows_workspace_floats(int64_t m, int64_t n, int64_t k);
hipError_t launch_fp8_gemm_krows(const uint8_t* a, int fmt_a, const float* s_a, const uint8_t* b,
                                 int fmt_b, const float* s_b, int64_t m, int64_t n, int64_t k,
                                 void* out, int out_dtype, int64_t ldc, float* split_ws,
                                 int64_t split_ws_floats, hipStream_t stream);
int fp8_tile_count();  // tile ids are 1 .. fp8_tile_count() - 1 (0: planner)
// Delayed scaling: saturating casts with given scales that also record each
// tensor's amax (atomic max of ordered f32 bits) into its slot's pending
// lanes (fp8_rec_words() words per slot); up to two tensors of one dtype in
// one launch. The per-step update folds the pending maxima into the history
// and recomputes every slot's scale.
struct DelayedCast {
  const void* t;
  int dtype;
  int64_t rows, cols, s_row, s_col;
  const float* scale;
  uint32_t* rec;  // the slot's pending lanes
  uint8_t* out;
  uint8_t* out_t;
};
int64_t fp8_rec_words();
hipError_t launch_fp8_cast_delayed(const DelayedCast& c0, const DelayedCast* c1, int fmt,
                                   hipStream_t stream);
hipError_t launch_fp8_scale_update(float* scales, const float* fmax, uint32_t* pending,
                                   uint32_t* hist, int32_t* cursor, int64_t n_slots,
                                   int64_t hist_len, hipStream_t stream);
hipError_t launch_fp8_encode_selfcheck(int fmt, uint64_t first, uint64_t count, uint32_t* counts,
                                       uint32_t* firsts, int64_t blocks, hipStream_t stream);

// Fused in-batch MNR loss (query i's positive is document i). The forward
// leaves in `saved` (mnr_saved_floats floats) what the backward reads.
constexpr int64_t kMnrMaxDocuments = 8192;
int64_t mnr_saved_floats(int64_t nq, int64_t nd, int64_t dim);
bool mnr_shape_ok(int64_t nq, int64_t nd, int64_t dim);
hipError_t launch_mnr_forward(const void* q, const void* d, int dtype, int64_t nq, int64_t nd,
                              int64_t dim, float scale, float* loss, float* saved,
                              hipStream_t stream);
hipError_t launch_mnr_backward(const float* grad_loss, const float* saved, int64_t nq, int64_t nd,
                               int64_t dim, float scale, void* dq, void* dd, int dtype,
                               hipStream_t stream);

}  // namespace rpx
