// Elementwise activation transforms for the paths whose GEMM does not carry
// the activation epilogue (skinny-M and generic shapes): the same act.h
// functions, so every path gives the same bits.
#include "act.h"
#include "kernels.h"

namespace rpx {

namespace {

template <int ACT>
__global__ void __launch_bounds__(256) k_act(const uint16_t* v, const uint16_t* aux,
                                             const uint16_t* aux2, int64_t count, uint16_t* out,
                                             uint16_t* out2) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count;
       i += stride) {
    const float a0 = ACT != kActGeluFwd ? bf16_to_f32(aux[i]) : 0.0f;
    const float a1 = ACT == kActSiluMulBwd ? bf16_to_f32(aux2[i]) : 0.0f;
    float r2 = 0.0f;
    const float r = act_apply<ACT>(bf16_to_f32(v[i]), a0, a1, &r2);
    out[i] = f32_to_bf16(r);
    if (ACT == kActSiluMulBwd) out2[i] = f32_to_bf16(r2);
  }
}

}  // namespace

hipError_t launch_act(int mode, const uint16_t* v, const uint16_t* aux, const uint16_t* aux2,
                      int64_t count, uint16_t* out, uint16_t* out2, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  const int64_t want = (count + 255) / 256;
  const unsigned grid = static_cast<unsigned>(want < 4096 ? want : 4096);
  switch (mode) {
    case kActGeluFwd:
      hipLaunchKernelGGL(k_act<kActGeluFwd>, dim3(grid), dim3(256), 0, stream, v, aux, aux2, count,
                         out, out2);
      break;
    case kActSiluMulFwd:
      hipLaunchKernelGGL(k_act<kActSiluMulFwd>, dim3(grid), dim3(256), 0, stream, v, aux, aux2,
                         count, out, out2);
      break;
    case kActGeluBwd:
      hipLaunchKernelGGL(k_act<kActGeluBwd>, dim3(grid), dim3(256), 0, stream, v, aux, aux2, count,
                         out, out2);
      break;
    case kActAddBwd:
      hipLaunchKernelGGL(k_act<kActAddBwd>, dim3(grid), dim3(256), 0, stream, v, aux, aux2, count,
                         out, out2);
      break;
    case kActSiluMulBwd:
      hipLaunchKernelGGL(k_act<kActSiluMulBwd>, dim3(grid), dim3(256), 0, stream, v, aux, aux2,
                         count, out, out2);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace rpx
