// RMSNorm, residual add and the producer-side FP8 formats of the decoder-block
// step around the MoE.
//
// RMSNorm follows wanferenz/model/architecture.py:217-230: fp32 math,
// y = bf16(weight * (x * rsqrt(mean(x^2) + eps))).  One workgroup per token
// row; the row is read once (HBM-bound).  rmsnorm_quant_kernel fuses the FP8
// act_quant of that output; wire_pack / wire_unpack are the stage-boundary
// FP8 format of serving/chain.py:208-222.
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
      o[i] = f32x2_to_bf16x2(a, b);
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
    o[j] = f32x2_to_bf16x2(lo, hi);
  }
  *reinterpret_cast<v4i*>(out + i * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
}

// RMSNorm fused with the FP8 act_quant of its output (the producer side of an
// FP8 linear): the bf16-rounded normalised row is quantised per 128 columns
// (torch_ops.py:33-49) without a round trip through memory.  Same arithmetic
// as rmsnorm_kernel followed by act_quant_kernel.  The row stays in registers:
// D <= 256 threads x 8 x kRqChunks.  With b, the row is first the residual
// step x + b (fp32 sum rounded once to bf16, add_bf16_kernel's arithmetic),
// which is also written to sum (when given): the block's residual add fused
// into the next norm.
constexpr int kRqChunks = 4;

__global__ __launch_bounds__(256) void rmsnorm_quant_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ b,
                                                            uint16_t* __restrict__ sum,
                                                            const float* __restrict__ w,
                                                            uint8_t* __restrict__ q, void* __restrict__ s,
                                                            int D, float eps, int kind) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * D;
  const bool pow2 = kind != WZ_SCALE_F32;
  v4i v[kRqChunks];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < kRqChunks; ++j) {
    const int c = threadIdx.x + 256 * j;
    v[j] = c < D / 8 ? load16(xr + c * 8) : v4i{0, 0, 0, 0};
    if (b && c < D / 8) {
      const v4i vb = load16(b + row * D + c * 8);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = bf16lo(uint32_t(v[j][i])) + bf16lo(uint32_t(vb[i]));
        const float hi = bf16hi(uint32_t(v[j][i])) + bf16hi(uint32_t(vb[i]));
        v[j][i] = int(f32x2_to_bf16x2(lo, hi));
      }
      if (sum) *reinterpret_cast<v4i*>(sum + row * D + c * 8) = v[j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = bf16lo(uint32_t(v[j][i])), b = bf16hi(uint32_t(v[j][i]));
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
#pragma unroll
  for (int j = 0; j < kRqChunks; ++j) {
    const int c = threadIdx.x + 256 * j;
    if (j * 256 * 8 >= D) break;  // uniform: no thread of the block has this chunk
    const bool valid = c < D / 8;
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int d0 = min(c * 8 + 2 * i, D - 2);
      f[2 * i] = bf16_round(w[d0] * (bf16lo(uint32_t(v[j][i])) * r));
      f[2 * i + 1] = bf16_round(w[d0 + 1] * (bf16hi(uint32_t(v[j][i])) * r));
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = absmax(amax, f[i]);
    amax = wave_absmax_xor(amax, 1);
    amax = wave_absmax_xor(amax, 2);
    amax = wave_absmax_xor(amax, 4);
    amax = wave_absmax_xor(amax, 8);
    const ActScale sc = act_scale(amax, pow2);
    if (valid) {
      const uint32_t lo = pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2),
                                     quant_div(f[2], sc, pow2), quant_div(f[3], sc, pow2));
      const uint32_t hi = pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2),
                                     quant_div(f[6], sc, pow2), quant_div(f[7], sc, pow2));
      *reinterpret_cast<uint2*>(q + row * D + c * 8) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) {
        const int64_t si = row * (D / 128) + c / 16;
        if (kind == WZ_SCALE_UE8M0)
          static_cast<uint8_t*>(s)[si] = uint8_t(sc.e8m0);
        else
          static_cast<float*>(s)[si] = sc.s;
      }
    }
  }
}

// The FP8 wire format of a stage boundary (serving/chain.py:208-222): per row
// scale = bf16(clamp(amax / 448, 1e-8, bf16 max)), q = e4m3(clamp(x / scale,
// +-448)); unpack: bf16(q * scale).  One workgroup per row.
__global__ __launch_bounds__(256) void wire_pack_kernel(const uint16_t* __restrict__ x, uint8_t* __restrict__ q,
                                                        uint16_t* __restrict__ scale, int D) {
  __shared__ float part[4];
  const int64_t row = blockIdx.x;
  const uint16_t* xr = x + row * D;
  float amax = 0.0f;
  for (int c = threadIdx.x; c < D / 8; c += 256) {
    const v4i v = load16(xr + c * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      amax = absmax(absmax(amax, bf16lo(uint32_t(v[i]))), bf16hi(uint32_t(v[i])));
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) amax = wave_absmax_xor(amax, m);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = amax;
  __syncthreads();
  amax = absmax(absmax(part[0], part[1]), absmax(part[2], part[3]));
  const float t = clamp_keep_nan(amax / 448.0f, 1e-8f, 3.3895313892515355e38f);
  const uint16_t sb = f32_to_bf16(t);
  const float sf = bf16_to_f32(sb);
  if (threadIdx.x == 0) scale[row] = sb;
  for (int c = threadIdx.x; c < D / 8; c += 256) {
    const v4i v = load16(xr + c * 8);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = clamp_keep_nan(bf16lo(uint32_t(v[i])) / sf, -kFp8Max, kFp8Max);
      f[2 * i + 1] = clamp_keep_nan(bf16hi(uint32_t(v[i])) / sf, -kFp8Max, kFp8Max);
    }
    *reinterpret_cast<uint2*>(q + row * D + c * 8) =
        make_uint2(pack_fp8x4(f[0], f[1], f[2], f[3]), pack_fp8x4(f[4], f[5], f[6], f[7]));
  }
}

__global__ __launch_bounds__(256) void wire_unpack_kernel(const uint8_t* __restrict__ q,
                                                          const uint16_t* __restrict__ scale,
                                                          uint16_t* __restrict__ y, int D, int64_t n8) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;  // 8 elements
  if (i >= n8) return;
  const int64_t row = (i * 8) / D;
  const float sf = bf16_to_f32(scale[row]);
  const uint2 b = *reinterpret_cast<const uint2*>(q + i * 8);
  // e4m3 -> f32 by the hardware converter (exact), times the scale, RNE to bf16
  const int wx = int(b.x), wy = int(b.y);
  const float f[8] = {__builtin_amdgcn_cvt_f32_fp8(wx, 0), __builtin_amdgcn_cvt_f32_fp8(wx, 1),
                      __builtin_amdgcn_cvt_f32_fp8(wx, 2), __builtin_amdgcn_cvt_f32_fp8(wx, 3),
                      __builtin_amdgcn_cvt_f32_fp8(wy, 0), __builtin_amdgcn_cvt_f32_fp8(wy, 1),
                      __builtin_amdgcn_cvt_f32_fp8(wy, 2), __builtin_amdgcn_cvt_f32_fp8(wy, 3)};
  uint32_t o[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
    o[k] = f32x2_to_bf16x2(f[2 * k] * sf, f[2 * k + 1] * sf);
  *reinterpret_cast<v4i*>(y + i * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
}

}  // namespace wz

extern "C" int wz_rmsnorm_quant(const void* x_bf16, const float* weight, void* q_e4m3, void* s, int64_t T,
                                int64_t D, float eps, int scale_kind, hipStream_t stream) {
  using namespace wz;
  if (T < 0 || D <= 0 || D % 128 || D > 256 * 8 * kRqChunks)
    return set_error(WZ_EINVAL, "rmsnorm_quant: D=%lld must be a multiple of 128 up to %d", (long long)D,
                     256 * 8 * kRqChunks);
  if (scale_kind < WZ_SCALE_F32 || scale_kind > WZ_SCALE_UE8M0_F32)
    return set_error(WZ_EINVAL, "rmsnorm_quant: unknown scale kind %d", scale_kind);
  if (T == 0) return WZ_OK;
  if (!x_bf16 || !weight || !q_e4m3 || !s) return set_error(WZ_EINVAL, "rmsnorm_quant: null pointer");
  WZ_LAUNCH("rmsnorm_quant", stream, rmsnorm_quant_kernel, dim3(unsigned(T)), dim3(256), 0,
            static_cast<const uint16_t*>(x_bf16), nullptr, nullptr, weight, static_cast<uint8_t*>(q_e4m3), s, int(D),
            eps, scale_kind);
  return check_launch("rmsnorm_quant");
}

extern "C" int wz_add_rmsnorm_quant(const void* x_bf16, const void* b_bf16, const float* weight, void* sum_bf16,
                                    void* q_e4m3, void* s, int64_t T, int64_t D, float eps, int scale_kind,
                                    hipStream_t stream) {
  using namespace wz;
  if (T < 0 || D <= 0 || D % 128 || D > 256 * 8 * kRqChunks)
    return set_error(WZ_EINVAL, "add_rmsnorm_quant: D=%lld must be a multiple of 128 up to %d", (long long)D,
                     256 * 8 * kRqChunks);
  if (scale_kind < WZ_SCALE_F32 || scale_kind > WZ_SCALE_UE8M0_F32)
    return set_error(WZ_EINVAL, "add_rmsnorm_quant: unknown scale kind %d", scale_kind);
  if (T == 0) return WZ_OK;
  if (!x_bf16 || !b_bf16 || !weight || !q_e4m3 || !s) return set_error(WZ_EINVAL, "add_rmsnorm_quant: null pointer");
  WZ_LAUNCH("add_rmsnorm_quant", stream, rmsnorm_quant_kernel, dim3(unsigned(T)), dim3(256), 0,
            static_cast<const uint16_t*>(x_bf16), static_cast<const uint16_t*>(b_bf16),
            static_cast<uint16_t*>(sum_bf16), weight, static_cast<uint8_t*>(q_e4m3), s, int(D), eps, scale_kind);
  return check_launch("add_rmsnorm_quant");
}

extern "C" int wz_fp8_wire_pack(const void* x_bf16, void* q_e4m3, void* scale_bf16, int64_t M, int64_t D,
                                hipStream_t stream) {
  using namespace wz;
  if (M < 0 || D <= 0 || D % 8) return set_error(WZ_EINVAL, "fp8_wire_pack: D=%lld must be a multiple of 8", (long long)D);
  if (M == 0) return WZ_OK;
  if (!x_bf16 || !q_e4m3 || !scale_bf16) return set_error(WZ_EINVAL, "fp8_wire_pack: null pointer");
  WZ_LAUNCH("fp8_wire_pack", stream, wire_pack_kernel, dim3(unsigned(M)), dim3(256), 0,
            static_cast<const uint16_t*>(x_bf16), static_cast<uint8_t*>(q_e4m3), static_cast<uint16_t*>(scale_bf16),
            int(D));
  return check_launch("fp8_wire_pack");
}

extern "C" int wz_fp8_wire_unpack(const void* q_e4m3, const void* scale_bf16, void* y_bf16, int64_t M, int64_t D,
                                  hipStream_t stream) {
  using namespace wz;
  if (M < 0 || D <= 0 || D % 8) return set_error(WZ_EINVAL, "fp8_wire_unpack: D=%lld must be a multiple of 8", (long long)D);
  if (M == 0) return WZ_OK;
  if (!q_e4m3 || !scale_bf16 || !y_bf16) return set_error(WZ_EINVAL, "fp8_wire_unpack: null pointer");
  const int64_t n8 = M * D / 8;
  WZ_LAUNCH("fp8_wire_unpack", stream, wire_unpack_kernel, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0,
            static_cast<const uint8_t*>(q_e4m3), static_cast<const uint16_t*>(scale_bf16),
            static_cast<uint16_t*>(y_bf16), int(D), n8);
  return check_launch("fp8_wire_unpack");
}

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
