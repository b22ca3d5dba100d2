// Operand loaders and the scaled-MFMA step shared by the GEMV/GEMM and MoE kernels.
//
// V_MFMA_SCALE_F32_16X16X128_F8F6F4 register layout (one wave, 64 lanes, g = l>>4),
// measured on gfx950 (tests/test_gpu_kernels.py::test_fp4_gemm_k_mapping):
//   A (16 x 128): lane l holds row (l & 15); B (128 x 16): column (l & 15).
//   e2m1 operand: 16 bytes (4 VGPRs) = K-elements [32g, 32g+32), low nibble first.
//   e4m3 operand: 32 bytes (8 VGPRs) = K [16g, 16g+16) in VGPRs 0-3 and
//                 K [64+16g, 64+16g+16) in VGPRs 4-7.
//   D (16 x 16) : lane l holds rows 4g + i, i = 0..3, of column (l & 15).
//   scale_a / scale_b: one e8m0 byte per lane, applied to the MX block
//   K [32g, 32g+32) — so an MXFP4 weight row's per-32 scale rides in the
//   lane that holds that block, and a power-of-two activation scale (one per
//   128, identical in the four lanes of a row) goes straight into the MFMA.
#pragma once

#include "common.h"

namespace wz {

// A operand of one 16x128 K-block: fp8 bytes plus the row's block scale.
struct AOp {
  v8i v;
  int se8;   // e8m0 byte for the MFMA (127 when the scale is applied on the VALU)
  float sf;  // float scale (used only for non-power-of-two activation scales)
};

__device__ __forceinline__ AOp a_zero() {
  AOp a;
  a.v = v8i{0, 0, 0, 0, 0, 0, 0, 0};
  a.se8 = kE8m0One;
  a.sf = 0.0f;
  return a;
}

// Pre-quantised activation row (e4m3 [K]) with its block scales.
// scale_kind: WZ_SCALE_F32 -> float scales; UE8M0 -> e8m0 bytes; UE8M0_F32 -> pow2 floats.
// A operand of K-block kb from a row that exists: no null test, so a batch of
// these loads can be issued together with the weight loads.
__device__ __forceinline__ AOp a_from_fp8_row(const uint8_t* row, const void* srow, int kb, int g,
                                              int scale_kind) {
  AOp a = a_zero();
  const uint8_t* p = row + kb * 128 + g * 16;
  v4i lo = load16(p), hi = load16(p + 64);
  a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  if (scale_kind == WZ_SCALE_UE8M0) {
    a.se8 = reinterpret_cast<const uint8_t*>(srow)[kb];
  } else {
    float s = reinterpret_cast<const float*>(srow)[kb];
    if (scale_kind == WZ_SCALE_UE8M0_F32)
      a.se8 = int((__float_as_uint(s) >> 23) & 0xFFu);
    else
      a.sf = s;
  }
  return a;
}

__device__ __forceinline__ AOp a_from_fp8(const uint8_t* row, const void* srow, int kb, int g,
                                          int scale_kind) {
  AOp a = a_zero();
  if (row == nullptr) return a;
  const uint8_t* p = row + kb * 128 + g * 16;
  v4i lo = load16(p), hi = load16(p + 64);
  a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  if (scale_kind == WZ_SCALE_UE8M0) {
    a.se8 = reinterpret_cast<const uint8_t*>(srow)[kb];
  } else {
    float s = reinterpret_cast<const float*>(srow)[kb];
    if (scale_kind == WZ_SCALE_UE8M0_F32)
      a.se8 = int((__float_as_uint(s) >> 23) & 0xFFu);
    else
      a.sf = s;
  }
  return a;
}

// bf16 activation row with act_quant fused (torch_ops.py:33-49): the four lanes
// that share a row (l, l^16, l^32, l^48) together hold the whole 128-block
// (two 16-element runs each), so the block amax is two xor-shuffles.  Every lane of the
// wave must call this (rows may be null -> zeros).
struct ARaw {
  v4i w[4];
};

// The load half of a_from_bf16: issue it early, quantise (a_quant_bf16) once
// other loads are in flight.
__device__ __forceinline__ ARaw a_load_bf16(const uint16_t* row, int kb, int g) {
  ARaw r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r.w[i] = v4i{0, 0, 0, 0};
  if (row != nullptr) {
    const uint16_t* p = row + kb * 128 + g * 16;
    r.w[0] = load16(p);
    r.w[1] = load16(p + 8);
    r.w[2] = load16(p + 64);
    r.w[3] = load16(p + 72);
  }
  return r;
}

// a_load_bf16 of a row that exists: no null test, so the loads of several
// K-blocks go out back to back.
__device__ __forceinline__ ARaw a_load_bf16_row(const uint16_t* row, int kb, int g) {
  ARaw r;
  const uint16_t* p = row + kb * 128 + g * 16;
  r.w[0] = load16(p);
  r.w[1] = load16(p + 8);
  r.w[2] = load16(p + 64);
  r.w[3] = load16(p + 72);
  return r;
}

__device__ __forceinline__ AOp a_quant_bf16(const ARaw& r, bool pow2) {
  AOp a = a_zero();
  const v4i* w = r.w;
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      amax = absmax(absmax(amax, bf16lo(uint32_t(w[i][j]))), bf16hi(uint32_t(w[i][j])));
  amax = wave_absmax_xor(amax, 16);
  amax = wave_absmax_xor(amax, 32);
  const ActScale sc = act_scale(amax, pow2);
  a.se8 = pow2 ? sc.e8m0 : kE8m0One;
  a.sf = sc.s;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    uint32_t w0 = uint32_t(w[i][0]), w1 = uint32_t(w[i][1]), w2 = uint32_t(w[i][2]),
             w3 = uint32_t(w[i][3]);
    a.v[2 * i] = int(pack_fp8x4(quant_div(bf16lo(w0), sc, pow2), quant_div(bf16hi(w0), sc, pow2),
                                quant_div(bf16lo(w1), sc, pow2), quant_div(bf16hi(w1), sc, pow2)));
    a.v[2 * i + 1] =
        int(pack_fp8x4(quant_div(bf16lo(w2), sc, pow2), quant_div(bf16hi(w2), sc, pow2),
                       quant_div(bf16lo(w3), sc, pow2), quant_div(bf16hi(w3), sc, pow2)));
  }
  return a;
}

__device__ __forceinline__ AOp a_from_bf16(const uint16_t* row, int kb, int g, bool pow2) {
  return a_quant_bf16(a_load_bf16(row, kb, g), pow2);
}

// MXFP4 weight row (packed e2m1 [K/2], e8m0 scales [K/32]) -> B operand of K-block kb.
__device__ __forceinline__ v8i b_fp4(const uint8_t* wrow, int kb, int g) {
  v4i x = load16(wrow + kb * 64 + g * 16);
  return v8i{x[0], x[1], x[2], x[3], 0, 0, 0, 0};
}

__device__ __forceinline__ int b_fp4_scale(const uint8_t* srow, int kb, int g) {
  return srow[kb * 4 + g];
}

// FP8 weight row (e4m3 [K]) -> B operand of K-block kb (same split layout as A).
__device__ __forceinline__ v8i b_fp8(const uint8_t* wrow, int kb, int g) {
  const uint8_t* p = wrow + kb * 128 + g * 16;
  v4i lo = load16(p), hi = load16(p + 64);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// FP8 weight 128x128 block scale -> (e8m0 byte for the MFMA, float for the VALU).
__device__ __forceinline__ void fp8_wscale(const void* ws, int64_t idx, int kind, int& se8,
                                           float& sf) {
  if (kind == WZ_WSCALE_E8M0) {
    se8 = reinterpret_cast<const uint8_t*>(ws)[idx];
    sf = 1.0f;
  } else {
    se8 = kE8m0One;
    sf = reinterpret_cast<const float*>(ws)[idx];
  }
}

// acc += A_blk . B_blk^T * scales.  When both scales are powers of two they
// ride inside the MFMA and the accumulator chains; otherwise the K-block
// partial is formed alone and scaled on the VALU, as the reference GPU
// kernels do per K-block (reference.py:281-285, 558-564).
template <int FA, int FB>
__device__ __forceinline__ void mma_step(v4f& acc, const AOp& a, const v8i& b, int sb_e8,
                                         float sb_f, bool a_pow2, bool b_pow2, int lane) {
  if (a_pow2 && b_pow2) {
    acc = mfma_scaled<FA, FB>(a.v, b, acc, a.se8, sb_e8);
  } else {
    const v4f z = {0.0f, 0.0f, 0.0f, 0.0f};
    v4f p = mfma_scaled<FA, FB>(a.v, b, z, a_pow2 ? a.se8 : kE8m0One, b_pow2 ? sb_e8 : kE8m0One);
    const int rbase = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sa = a_pow2 ? 1.0f : __shfl(a.sf, rbase + i, kWave);
      float sb = b_pow2 ? 1.0f : sb_f;
      acc[i] += p[i] * (sa * sb);
    }
  }
}

}  // namespace wz
