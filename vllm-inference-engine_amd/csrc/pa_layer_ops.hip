// Fused elementwise parts of a decode step's transformer layer, for gfx950.
//
// A decode step of a 0.5B-class model at batch 128 is hundreds of small
// kernels; most of them are the pieces of elementwise chains that
// transformers evaluates op by op:
//   residual add + RMSNorm (modeling_qwen2.Qwen2DecoderLayer.forward and
//            Qwen2RMSNorm.forward): residual + x in fp16, then to(float32),
//            pow(2), mean, + eps, rsqrt, multiply, .to(float16), weight * --
//            up to eight launches per norm, two norms per layer;
//   SwiGLU   (modeling_qwen2.Qwen2MLP.forward): silu(gate) then * up;
//   greedy token and margin of the step (paged_attention_integration.py
//            :636-651): arg-max and top-2 of each logits row.
// Each becomes one launch here, with the same roundings: the residual sum
// rounded to fp16, the norm in fp32 rounded to fp16, then the fp16 weight
// product rounded to fp16; silu in fp32 rounded to fp16, then the fp16 product
// rounded to fp16.
#include <hip/hip_runtime.h>

#include "pa_common.h"

namespace pa {

// One workgroup of 256 threads per row; each thread keeps its values of the
// row (at most kNormPer) in registers between the sum of squares and the
// scaling. With `res`, the row is first replaced by fp16(x + res) and that sum
// is also written to `sum`.
constexpr int kNormPer = 8;  // rows up to 256 * 8 = 2048 values take this kernel

__global__ __launch_bounds__(256) void rmsnorm_kernel(const f16* __restrict__ x, int64_t xs,
                                                      const f16* __restrict__ res, int64_t rs,
                                                      f16* __restrict__ sum, int64_t ss_,
                                                      const f16* __restrict__ w,
                                                      f16* __restrict__ y, int64_t ys, int H,
                                                      float eps) {
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const f16* xr = x + r * xs;
  float v[kNormPer];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int i = tid + 256 * k;
    float t = 0.f;
    if (i < H) t = (float)xr[i];
    v[k] = t;
  }
  if (res) {
#pragma unroll
    for (int k = 0; k < kNormPer; ++k) {
      const int i = tid + 256 * k;
      if (i < H) {
        const f16 s = (f16)(v[k] + (float)res[r * rs + i]);
        sum[r * ss_ + i] = s;
        v[k] = (float)s;
      }
    }
  }
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) ss += v[k] * v[k];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  __shared__ float part[4];
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  // mean as torch's reduction forms it: the sum times 1 / H.
  const float inv = rsqrtf(tot * (1.f / (float)H) + eps);
  f16* yr = y + r * ys;
#pragma unroll
  for (int k = 0; k < kNormPer; ++k) {
    const int i = tid + 256 * k;
    if (i < H) {
      const f16 n = (f16)(v[k] * inv);
      yr[i] = (f16)((float)w[i] * (float)n);
    }
  }
}

// Rows longer than 256 * kNormPer: the same arithmetic in two passes over
// the row, the residual sum formed again in the second pass.
__global__ __launch_bounds__(256) void rmsnorm_long_kernel(
    const f16* __restrict__ x, int64_t xs, const f16* __restrict__ res, int64_t rs,
    f16* __restrict__ sum, int64_t ss_, const f16* __restrict__ w, f16* __restrict__ y,
    int64_t ys, int H, float eps) {
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x;
  const f16* xr = x + r * xs;
  auto value = [&](int i) {
    float t = (float)xr[i];
    if (res) t = (float)(f16)(t + (float)res[r * rs + i]);
    return t;
  };
  float ss = 0.f;
  for (int i = tid; i < H; i += 256) {
    const float t = value(i);
    ss += t * t;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  __shared__ float part[4];
  if ((tid & 63) == 0) part[tid >> 6] = ss;
  __syncthreads();
  const float tot = part[0] + part[1] + part[2] + part[3];
  const float inv = rsqrtf(tot * (1.f / (float)H) + eps);
  f16* yr = y + r * ys;
  for (int i = tid; i < H; i += 256) {
    const float t = value(i);
    if (res) sum[r * ss_ + i] = (f16)t;
    const f16 n = (f16)(t * inv);
    yr[i] = (f16)((float)w[i] * (float)n);
  }
}

// out[r, i] = fp16(fp16(silu(gate[r, i])) * up[r, i]) with gate and up the two
// halves of one row of gu ([rows, 2 * I]: gate first, as a merged gate/up
// projection lays them out). Eight values per thread when I allows it.
template <int V>
__global__ __launch_bounds__(256) void silu_mul_kernel(const f16* __restrict__ gu, int64_t gs,
                                                       f16* __restrict__ out, int64_t os, int I,
                                                       int64_t n) {
  const int64_t t = ((int64_t)blockIdx.x * 256 + threadIdx.x) * V;
  if (t >= n) return;
  const int64_t r = t / I;
  const int i = (int)(t - r * I);
  typedef f16 hv __attribute__((ext_vector_type(V)));
  const hv g = *reinterpret_cast<const hv*>(gu + r * gs + i);
  const hv u = *reinterpret_cast<const hv*>(gu + r * gs + I + i);
  hv o;
#pragma unroll
  for (int k = 0; k < V; ++k) {
    const float gf = (float)g[k];
    const f16 s = (f16)(gf / (1.f + expf(-gf)));
    o[k] = (f16)((float)s * (float)u[k]);
  }
  *reinterpret_cast<hv*>(out + r * os + i) = o;
}

// Per row of fp16 logits: the arg-max (first index of the maximum, as
// torch.argmax returns it), the maximum and the second-largest value (the
// top-2 of torch.topk, ties counted twice). One workgroup of 1024 threads per
// row; with VEC, 16-byte loads of eight logits, two in flight per thread.
template <bool VEC>
__global__ __launch_bounds__(1024) void top2_kernel(const f16* __restrict__ logits, int64_t ls,
                                                    int V, int64_t* __restrict__ idx,
                                                    float* __restrict__ top) {
  const int64_t r = blockIdx.x;
  const f16* row = logits + r * ls;
  const int tid = threadIdx.x;
  float m1 = -__builtin_huge_valf(), m2 = -__builtin_huge_valf();
  int i1 = 0x7fffffff;
  auto take = [&](float v, int i) {  // indices reach a thread in increasing order
    if (v > m1) {
      m2 = m1;
      m1 = v;
      i1 = i;
    } else if (v > m2) {
      m2 = v;
    }
  };
  if constexpr (VEC) {
    const int nv = V / 8;
    for (int j = tid; j < nv; j += 2048) {
      const f16x8 a = *reinterpret_cast<const f16x8*>(row + 8 * j);
      const bool two = j + 1024 < nv;
      const f16x8 b = two ? *reinterpret_cast<const f16x8*>(row + 8 * (j + 1024)) : a;
#pragma unroll
      for (int k = 0; k < 8; ++k) take((float)a[k], 8 * j + k);
      if (two) {
#pragma unroll
        for (int k = 0; k < 8; ++k) take((float)b[k], 8 * (j + 1024) + k);
      }
    }
  } else {
    for (int i = tid; i < V; i += 1024) take((float)row[i], i);
  }
  // Combine (m1, i1, m2) across lanes: the larger maximum wins (lower index on
  // ties); the second value is the largest of the other three.
  auto combine = [](float& a1, int& ai, float& a2, float b1, int bi, float b2) {
    if (b1 > a1 || (b1 == a1 && bi < ai)) {
      a2 = fmaxf(a1, b2);
      a1 = b1;
      ai = bi;
    } else {
      a2 = fmaxf(a2, b1);
    }
  };
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float b1 = __shfl_xor(m1, off), b2 = __shfl_xor(m2, off);
    const int bi = __shfl_xor(i1, off);
    combine(m1, i1, m2, b1, bi, b2);
  }
  __shared__ float s1[16], s2[16];
  __shared__ int si[16];
  if ((tid & 63) == 0) {
    s1[tid >> 6] = m1;
    s2[tid >> 6] = m2;
    si[tid >> 6] = i1;
  }
  __syncthreads();
  if (tid == 0) {
    float a1 = s1[0], a2 = s2[0];
    int ai = si[0];
    for (int k = 1; k < 16; ++k) combine(a1, ai, a2, s1[k], si[k], s2[k]);
    idx[r] = ai;
    top[2 * r] = a1;
    top[2 * r + 1] = a2;
  }
}

hipError_t launch_rmsnorm(const f16* x, int64_t xs, const f16* res, int64_t rs, f16* sum,
                          int64_t ss, const f16* w, f16* y, int64_t ys, int rows, int H,
                          float eps, hipStream_t s) {
  if (H <= 256 * kNormPer)
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, xs, res, rs, sum, ss, w, y,
                       ys, H, eps);
  else
    hipLaunchKernelGGL(rmsnorm_long_kernel, dim3(rows), dim3(256), 0, s, x, xs, res, rs, sum, ss,
                       w, y, ys, H, eps);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const f16* gu, int64_t gs, f16* out, int64_t os, int rows, int I,
                           bool vec, hipStream_t s) {
  const int64_t n = (int64_t)rows * I;
  if (vec)
    hipLaunchKernelGGL(silu_mul_kernel<8>, dim3((unsigned)((n / 8 + 255) / 256)), dim3(256), 0, s,
                       gu, gs, out, os, I, n);
  else
    hipLaunchKernelGGL(silu_mul_kernel<1>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, gu,
                       gs, out, os, I, n);
  return hipGetLastError();
}

hipError_t launch_top2(const f16* logits, int64_t ls, int rows, int V, int64_t* idx, float* top,
                       bool vec, hipStream_t s) {
  if (vec)
    hipLaunchKernelGGL(top2_kernel<true>, dim3(rows), dim3(1024), 0, s, logits, ls, V, idx, top);
  else
    hipLaunchKernelGGL(top2_kernel<false>, dim3(rows), dim3(1024), 0, s, logits, ls, V, idx, top);
  return hipGetLastError();
}

}  // namespace pa
