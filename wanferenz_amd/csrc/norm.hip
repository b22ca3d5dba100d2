// RMSNorm and residual add for the decoder-block step around the MoE.
//
// RMSNorm follows wanferenz/model/architecture.py:217-230: fp32 math,
// y = bf16(weight * (x * rsqrt(mean(x^2) + eps))).  One workgroup per token
// row; the row is read once (HBM-bound).
#include "common.h"

namespace wz {

__global__ __launch_bounds__(256) void rmsnorm_kernel(const uint16_t* __restrict__ x,
                                                      const float* __restrict__ w,
                                                      uint16_t* __restrict__ y, int D, float eps) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * D;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < D / 8; c += 256) {
    const v4i v = load16(xr + c * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16lo(uint32_t(v[i])), b = bf16hi(uint32_t(v[i]));
      ss += a * a;
      ss += b * b;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float var = ((part[0] + part[1]) + (part[2] + part[3])) / float(D);
  const float r = 1.0f / sqrtf(var + eps);
  for (int c = threadIdx.x; c < D / 8; c += 256) {
    const v4i v = load16(xr + c * 8);
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = c * 8 + 2 * i;
      const float a = w[d0] * (bf16lo(uint32_t(v[i])) * r);
      const float b = w[d0 + 1] * (bf16hi(uint32_t(v[i])) * r);
      o[i] = uint32_t(f32_to_bf16(a)) | (uint32_t(f32_to_bf16(b)) << 16);
    }
    *reinterpret_cast<v4i*>(y + row * D + c * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
  }
}

__global__ __launch_bounds__(256) void add_bf16_kernel(const uint16_t* __restrict__ a,
                                                       const uint16_t* __restrict__ b,
                                                       uint16_t* __restrict__ out, int64_t n8) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n8) return;
  const v4i va = load16(a + i * 8), vb = load16(b + i * 8);
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float lo = bf16lo(uint32_t(va[j])) + bf16lo(uint32_t(vb[j]));
    const float hi = bf16hi(uint32_t(va[j])) + bf16hi(uint32_t(vb[j]));
    o[j] = uint32_t(f32_to_bf16(lo)) | (uint32_t(f32_to_bf16(hi)) << 16);
  }
  *reinterpret_cast<v4i*>(out + i * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
}

}  // namespace wz

extern "C" int wz_rmsnorm(const void* x_bf16, const float* weight, void* y_bf16, int64_t T, int64_t D,
                          float eps, hipStream_t stream) {
  using namespace wz;
  if (T < 0 || D <= 0 || D % 8) return set_error(WZ_EINVAL, "rmsnorm: D=%lld must be a multiple of 8", (long long)D);
  if (T == 0) return WZ_OK;
  if (!x_bf16 || !weight || !y_bf16) return set_error(WZ_EINVAL, "rmsnorm: null pointer");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(unsigned(T)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(x_bf16), weight, static_cast<uint16_t*>(y_bf16), int(D), eps);
  return check_launch("rmsnorm");
}

extern "C" int wz_add_bf16(const void* a, const void* b, void* out, int64_t n, hipStream_t stream) {
  using namespace wz;
  if (n < 0 || n % 8) return set_error(WZ_EINVAL, "add_bf16: n=%lld must be a multiple of 8", (long long)n);
  if (n == 0) return WZ_OK;
  if (!a || !b || !out) return set_error(WZ_EINVAL, "add_bf16: null pointer");
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(add_bf16_kernel, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint16_t*>(a), static_cast<const uint16_t*>(b), static_cast<uint16_t*>(out), n8);
  return check_launch("add_bf16");
}
