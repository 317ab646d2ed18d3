// Fused elementwise parts of a decode step's transformer layer, for gfx950.
//
// A decode step of a 0.5B-class model at batch 128 is hundreds of small
// kernels; most of them are the pieces of two elementwise chains that
// transformers evaluates op by op:
//   RMSNorm  (modeling_qwen2.Qwen2RMSNorm.forward): x.to(float32), pow(2),
//            mean, + eps, rsqrt, multiply, .to(float16), weight * -- seven
//            launches per norm, two norms per layer;
//   SwiGLU   (modeling_qwen2.Qwen2MLP.forward): silu(gate) then * up.
// Each becomes one launch here, with the same roundings: the norm in fp32,
// rounded to fp16, then the fp16 weight product rounded to fp16; silu in
// fp32 rounded to fp16, then the fp16 product rounded to fp16.
#include <hip/hip_runtime.h>

#include "pa_common.h"

namespace pa {

// One workgroup per row; 256 threads stride over the row.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const f16* __restrict__ x, int64_t xs,
                                                      const f16* __restrict__ w,
                                                      f16* __restrict__ y, int64_t ys, int H,
                                                      float eps) {
  const int64_t r = blockIdx.x;
  const f16* xr = x + r * xs;
  f16* yr = y + r * ys;
  float ss = 0.f;
  for (int i = threadIdx.x; i < H; i += 256) {
    const float v = (float)xr[i];
    ss += v * v;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  // mean as torch's reduction forms it: the sum times 1 / H.
  const float inv = rsqrtf(tot * (1.f / (float)H) + eps);
  for (int i = threadIdx.x; i < H; i += 256) {
    const f16 n = (f16)((float)xr[i] * inv);
    yr[i] = (f16)((float)w[i] * (float)n);
  }
}

// out[r, i] = fp16(fp16(silu(gate[r, i])) * up[r, i]) with gate and up the two
// halves of one row of gu ([rows, 2 * I]: gate first, as a merged gate/up
// projection lays them out).
__global__ __launch_bounds__(256) void silu_mul_kernel(const f16* __restrict__ gu, int64_t gs,
                                                       f16* __restrict__ out, int64_t os, int I,
                                                       int64_t n) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n) return;
  const int64_t r = t / I;
  const int i = (int)(t - r * I);
  const float g = (float)gu[r * gs + i];
  const f16 s = (f16)(g / (1.f + expf(-g)));
  out[r * os + i] = (f16)((float)s * (float)gu[r * gs + I + i]);
}

hipError_t launch_rmsnorm(const f16* x, int64_t xs, const f16* w, f16* y, int64_t ys, int rows,
                          int H, float eps, hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, xs, w, y, ys, H, eps);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const f16* gu, int64_t gs, f16* out, int64_t os, int rows, int I,
                           hipStream_t s) {
  const int64_t n = (int64_t)rows * I;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu, gs,
                     out, os, I, n);
  return hipGetLastError();
}

}  // namespace pa
