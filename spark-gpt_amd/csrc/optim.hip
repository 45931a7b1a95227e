// The Muon momentum stage of spark-gpt's optimizer (gfx950): the consumer of
// the MLP's fp32 weight gradients.  _momentum_stage_kernel
// (train.py:2805-2820) in one HBM pass: for each element,
//   v_new = v + w_v * (g - v)            (torch.lerp, weight < 0.5: w_v = 1 - momentum)
//   u = v_new - (v_new - g) * (1 - w_u)  (torch.lerp, weight >= 0.5: w_u = momentum)
// v updated in place (fp32), u stored as bf16 into the Newton-Schulz staging
// stack.  Both lerps are evaluated as torch's GPU lerp does (fused
// multiply-add, one rounding), so the result is the reference's two-pass
// torch update bit for bit.
#include "common.h"

namespace sfp8 {

// n % 4 == 0; four elements per thread.
__global__ __launch_bounds__(256) void momentum_stage_kernel(const float* __restrict__ g, float* __restrict__ v,
                                                             uint16_t* __restrict__ u, int64_t n, float w_v,
                                                             float w_u1) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  const floatx4 gg = *reinterpret_cast<const floatx4*>(g + i);
  floatx4 vv = *reinterpret_cast<const floatx4*>(v + i);
  uint32_t uu[2];
  momentum4(gg, vv, w_v, w_u1, uu);
  *reinterpret_cast<floatx4*>(v + i) = vv;
  *reinterpret_cast<intx2*>(u + i) = intx2{(int)uu[0], (int)uu[1]};
}

}  // namespace sfp8

using namespace sfp8;

extern "C" {

// w_v = 1 - momentum and w_u = momentum as the reference passes them
// (train.py:2835-2838: Python floats rounded to fp32), w_v < 0.5 <= w_u.
int sfp8_momentum_stage(const float* g, float* v, void* u, int64_t n, float w_v, float w_u, void* stream) {
  if (n > 0 && (!g || !v || !u)) return kErrNullPointer;
  if (n < 0 || n % 4 || !(w_v > -0.5f && w_v < 0.5f) || !(w_u >= 0.5f)) return kErrBadShape;
  if ((((uintptr_t)g) & 15u) || (((uintptr_t)v) & 15u) || (((uintptr_t)u) & 7u)) return kErrBadAlignment;
  if (n == 0) return kOk;
  hipLaunchKernelGGL(momentum_stage_kernel, dim3((unsigned)((n / 4 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     g, v, (uint16_t*)u, n, w_v, 1.0f - w_u);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? kOk : (int)e;
}

}  // extern "C"
