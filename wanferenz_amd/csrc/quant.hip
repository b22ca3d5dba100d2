// act_quant: per-row, per-128-column dynamic FP8 (e4m3fn) quantisation.
//
// Semantics of wanferenz/kernels/torch_ops.py:33-49 (CPU) and the TileLang
// act_quant_kernel (wanferenz/kernels/reference.py:40-114): amax over each
// 128-block floored at 1e-4; s = amax/448 or its power-of-two ceiling;
// q = e4m3(clamp(x/s, -448, 448)) with round-to-nearest-even.
//
// Layout: one lane owns 8 consecutive bf16 (one 16-byte load); 16 lanes own
// one 128-block, so the block amax is a 4-step xor-shuffle inside a quarter
// wave.  The kernel is HBM-bound (2 B in, 1 B + 4/128 B out per element).
#include "common.h"

namespace wz {

__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x,
                                                        int64_t n8, uint8_t* __restrict__ q,
                                                        void* __restrict__ s, int kind) {
  const int64_t tid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const bool valid = tid < n8;
  v4i w = {0, 0, 0, 0};
  if (valid) w = load16(x + tid * 8);
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16lo(uint32_t(w[i]));
    f[2 * i + 1] = bf16hi(uint32_t(w[i]));
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = absmax(amax, f[i]);
  amax = wave_absmax_xor(amax, 1);
  amax = wave_absmax_xor(amax, 2);
  amax = wave_absmax_xor(amax, 4);
  amax = wave_absmax_xor(amax, 8);
  const bool pow2 = kind != WZ_SCALE_F32;
  const ActScale sc = act_scale(amax, pow2);
  if (!valid) return;
  uint32_t lo = pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2),
                           quant_div(f[2], sc, pow2), quant_div(f[3], sc, pow2));
  uint32_t hi = pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2),
                           quant_div(f[6], sc, pow2), quant_div(f[7], sc, pow2));
  *reinterpret_cast<uint2*>(q + tid * 8) = make_uint2(lo, hi);
  if ((tid & 15) == 0) {
    const int64_t b = tid >> 4;
    if (kind == WZ_SCALE_UE8M0)
      reinterpret_cast<uint8_t*>(s)[b] = uint8_t(sc.e8m0);
    else
      reinterpret_cast<float*>(s)[b] = sc.s;
  }
}

// Stream-ordered act_quant of `rows` rows of K bf16 for the MoE kernels.
int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream) {
  const int64_t n8 = rows * K / 8;
  if (n8 == 0) return WZ_OK;
  WZ_LAUNCH("act_quant", stream, act_quant_kernel, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0,
            static_cast<const uint16_t*>(x), n8, q, s, kind);
  return check_launch("act_quant");
}

}  // namespace wz

extern "C" int wz_act_quant_fp8(const void* x_bf16, int64_t M, int64_t K, void* q_e4m3, void* s,
                                int scale_kind, hipStream_t stream) {
  using namespace wz;
  if (M < 0 || K <= 0 || K % 128)
    return set_error(WZ_EINVAL, "act_quant: K=%lld must be a positive multiple of 128", (long long)K);
  if (scale_kind < WZ_SCALE_F32 || scale_kind > WZ_SCALE_UE8M0_F32)
    return set_error(WZ_EINVAL, "act_quant: unknown scale kind %d", scale_kind);
  if (M == 0) return WZ_OK;
  if (!x_bf16 || !q_e4m3 || !s) return set_error(WZ_EINVAL, "act_quant: null pointer");
  const int64_t n8 = M * K / 8;
  const int64_t blocks = (n8 + 255) / 256;
  WZ_LAUNCH("act_quant", stream, act_quant_kernel, dim3(unsigned(blocks)), dim3(256), 0,
                     static_cast<const uint16_t*>(x_bf16), n8, static_cast<uint8_t*>(q_e4m3), s,
                     scale_kind);
  return check_launch("act_quant");
}
