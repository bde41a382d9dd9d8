// In-batch multiple-negatives ranking loss, fused: the fp32 casts and row
// normalisation of both embedding sets, the scaled cosine logits, each
// query's log-sum-exp, the mean over queries, and the gradient of all of it
// (src/representax/tasks/retrieval/mnr.py:48-52 `_normalize`, :132-158
// `_direction_row_terms` with query i's positive = document i and unit
// weights, :338-341 the forward loss). Four launches replace the ~30 small
// elementwise, reduction and matmul kernels of the unfused objective.
//
// Every sum runs in a fixed order (per-thread strided partials, then a
// shuffle tree, then the waves in order), so results do not depend on
// scheduling.
#include <hip/hip_runtime.h>

#include <cmath>

#include "common.h"
#include "kernels.h"

namespace rpx {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ float load_elem(const void* p, int dtype, int64_t i) {
  return dtype == kBF16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i])
                        : static_cast<const float*>(p)[i];
}

__device__ __forceinline__ void store_elem(void* p, int dtype, int64_t i, float v) {
  if (dtype == kBF16)
    static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
  else
    static_cast<float*>(p)[i] = v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Block-wide sum, the same value in every thread: wave trees, then the
// waves' partials in wave order.
__device__ __forceinline__ float block_sum(float v, float* sh) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[wave] = v;
  __syncthreads();
  float s = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) s += sh[w];
  return s;
}

__device__ __forceinline__ float block_max(float v, float* sh) {
  v = wave_max(v);
  const int wave = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sh[wave] = v;
  __syncthreads();
  float m = sh[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) m = fmaxf(m, sh[w]);
  return m;
}

// Block r: row r of the queries (r < nq) or row r - nq of the documents,
// cast to f32 and divided by max(||row||, 1e-12) (mnr.py:48-52); the
// unclamped norm is kept for the backward.
__global__ void __launch_bounds__(kThreads)
    k_mnr_normalize(const void* __restrict__ q, const void* __restrict__ d, int dtype, int64_t nq,
                    int64_t dim, float* __restrict__ unit, float* __restrict__ norms) {
  __shared__ float sh[kWaves];
  const int64_t r = blockIdx.x;
  const void* src = r < nq ? q : d;
  const int64_t row = r < nq ? r : r - nq;
  float ss = 0.0f;
  for (int64_t e = threadIdx.x; e < dim; e += kThreads) {
    const float v = load_elem(src, dtype, row * dim + e);
    ss = __builtin_fmaf(v, v, ss);
  }
  const float norm = sqrtf(block_sum(ss, sh));
  const float denom = fmaxf(norm, 1e-12f);
  for (int64_t e = threadIdx.x; e < dim; e += kThreads)
    unit[r * dim + e] = load_elem(src, dtype, row * dim + e) / denom;
  if (threadIdx.x == 0) norms[r] = norm;
}

// Block i (query i): logits l_j = scale * <q_i, d_j> for every document j,
// the log-sum-exp m + log(sum_j exp(l_j - m)), the row loss lse - l_i and
// the softmax row exp(l_j - lse) for the backward.
__global__ void __launch_bounds__(kThreads)
    k_mnr_rows(const float* __restrict__ unit, int64_t nq, int64_t nd, int64_t dim, float scale,
               float* __restrict__ probs, float* __restrict__ row_loss) {
  extern __shared__ float logits[];
  __shared__ float sh[kWaves];
  const int64_t i = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const float* qi = unit + i * dim;
  const float* docs = unit + nq * dim;
  for (int64_t j = wave; j < nd; j += kWaves) {
    const float* dj = docs + j * dim;
    float dot = 0.0f;
    for (int64_t e = lane; e < dim; e += 64) dot = __builtin_fmaf(qi[e], dj[e], dot);
    dot = wave_sum(dot);
    if (lane == 0) logits[j] = dot * scale;
  }
  __syncthreads();
  float m = -INFINITY;
  for (int64_t j = threadIdx.x; j < nd; j += kThreads) m = fmaxf(m, logits[j]);
  m = block_max(m, sh);
  float s = 0.0f;
  for (int64_t j = threadIdx.x; j < nd; j += kThreads) s += expf(logits[j] - m);
  const float lse = m + logf(block_sum(s, sh));
  for (int64_t j = threadIdx.x; j < nd; j += kThreads) probs[i * nd + j] = expf(logits[j] - lse);
  if (threadIdx.x == 0) row_loss[i] = lse - logits[i];
}

// loss = mean over queries of the row losses (mnr.py:338-341, every query
// active).
__global__ void __launch_bounds__(kThreads)
    k_mnr_mean(const float* __restrict__ row_loss, int64_t nq, float* __restrict__ loss) {
  __shared__ float sh[kWaves];
  float s = 0.0f;
  for (int64_t i = threadIdx.x; i < nq; i += kThreads) s += row_loss[i];
  s = block_sum(s, sh);
  if (threadIdx.x == 0) loss[0] = s / static_cast<float>(nq);
}

// Gradient. With c_ij = g * scale * (p_ij - [i == j]) / nq:
//   block i < nq (query i):   du = sum_j c_ij d_j,  over the documents in order;
//   block nq + j (document j): du = sum_i c_ij q_i, over the queries in order;
// then through the normalisation u = v / max(||v||, 1e-12):
//   dv = (du - u <u, du>) / ||v|| when ||v|| > 1e-12, else du / 1e-12.
// Each thread owns the dimensions e = tid, tid + 256, ... (at most kMaxPer).
constexpr int kMaxPer = 16;  // dim <= 4096

__global__ void __launch_bounds__(kThreads)
    k_mnr_grad(const float* __restrict__ unit, const float* __restrict__ norms,
               const float* __restrict__ probs, int64_t nq, int64_t nd, int64_t dim, float scale,
               const float* __restrict__ grad_loss, void* __restrict__ dq, void* __restrict__ dd,
               int dtype) {
  __shared__ float sh[kWaves];
  const int64_t r = blockIdx.x;
  const bool is_q = r < nq;
  const int64_t row = is_q ? r : r - nq;
  const float c0 = grad_loss[0] * scale / static_cast<float>(nq);
  const int64_t others = is_q ? nd : nq;
  const float* other = is_q ? unit + nq * dim : unit;
  float du[kMaxPer];
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) du[t] = 0.0f;
  for (int64_t o = 0; o < others; ++o) {
    const float p = is_q ? probs[row * nd + o] : probs[o * nd + row];
    const float c = c0 * (p - (o == row ? 1.0f : 0.0f));
    const float* v = other + o * dim;
#pragma unroll
    for (int t = 0; t < kMaxPer; ++t) {
      const int64_t e = threadIdx.x + static_cast<int64_t>(t) * kThreads;
      if (e < dim) du[t] = __builtin_fmaf(c, v[e], du[t]);
    }
  }
  const float* u = unit + r * dim;
  float proj = 0.0f;
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) {
    const int64_t e = threadIdx.x + static_cast<int64_t>(t) * kThreads;
    if (e < dim) proj = __builtin_fmaf(u[e], du[t], proj);
  }
  proj = block_sum(proj, sh);
  const float norm = norms[r];
  const bool clamped = !(norm > 1e-12f);
  void* out = is_q ? dq : dd;
#pragma unroll
  for (int t = 0; t < kMaxPer; ++t) {
    const int64_t e = threadIdx.x + static_cast<int64_t>(t) * kThreads;
    if (e >= dim) continue;
    const float g = clamped ? du[t] / 1e-12f : (du[t] - u[e] * proj) / norm;
    store_elem(out, dtype, row * dim + e, g);
  }
}

}  // namespace

int64_t mnr_saved_floats(int64_t nq, int64_t nd, int64_t dim) {
  // unit rows (queries, then documents), norms, softmax rows, row losses
  return (nq + nd) * dim + (nq + nd) + nq * nd + nq;
}

bool mnr_shape_ok(int64_t nq, int64_t nd, int64_t dim) {
  return nq >= 1 && nd >= nq && nd <= kMnrMaxDocuments && dim >= 1 && dim <= kThreads * kMaxPer;
}

hipError_t launch_mnr_forward(const void* q, const void* d, int dtype, int64_t nq, int64_t nd,
                              int64_t dim, float scale, float* loss, float* saved,
                              hipStream_t stream) {
  float* unit = saved;
  float* norms = unit + (nq + nd) * dim;
  float* probs = norms + (nq + nd);
  float* row_loss = probs + nq * nd;
  hipLaunchKernelGGL(k_mnr_normalize, dim3(static_cast<unsigned>(nq + nd)), dim3(kThreads), 0,
                     stream, q, d, dtype, nq, dim, unit, norms);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_mnr_rows, dim3(static_cast<unsigned>(nq)), dim3(kThreads),
                     static_cast<size_t>(nd) * sizeof(float), stream, unit, nq, nd, dim, scale,
                     probs, row_loss);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_mnr_mean, dim3(1), dim3(kThreads), 0, stream, row_loss, nq, loss);
  return hipGetLastError();
}

hipError_t launch_mnr_backward(const float* grad_loss, const float* saved, int64_t nq, int64_t nd,
                               int64_t dim, float scale, void* dq, void* dd, int dtype,
                               hipStream_t stream) {
  const float* unit = saved;
  const float* norms = unit + (nq + nd) * dim;
  const float* probs = norms + (nq + nd);
  hipLaunchKernelGGL(k_mnr_grad, dim3(static_cast<unsigned>(nq + nd)), dim3(kThreads), 0, stream,
                     unit, norms, probs, nq, nd, dim, scale, grad_loss, dq, dd, dtype);
  return hipGetLastError();
}

}  // namespace rpx
