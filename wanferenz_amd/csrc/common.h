// Shared device helpers for the gfx950 (CDNA4) MoE / FP8-linear kernels.
//
// Number formats (OCP MX / OCP FP8): e4m3fn activations and FP8 weights,
// e2m1 (two codes per byte, low nibble = even element) MXFP4 weights with one
// e8m0 scale per 32 K-elements, bf16 activations and outputs.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "wanferenz_amd.h"

namespace wz {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr float kFp8Max = 448.0f;

// MFMA operand formats (cbsz / blgp field values of V_MFMA_SCALE_F32_16X16X128_F8F6F4).
constexpr int kFmtFp8 = 0;
constexpr int kFmtFp4 = 4;
constexpr int kE8m0One = 127;

// ---------------------------------------------------------------- bf16 -------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// float32 -> bfloat16 bits, round to nearest even (NaN stays NaN), by gfx950's
// converter (v_cvt_pk_bf16_f32): one instruction for two values.
typedef float wz_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 wz_bf16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(wz_f32x2{lo, hi}, wz_bf16x2));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return uint16_t(f32x2_to_bf16x2(f, 0.0f)); }

__device__ __forceinline__ float bf16_round(float f) {
  return __uint_as_float(uint32_t(f32_to_bf16(f)) << 16);
}

// ---------------------------------------------------------------- scales -----

// 2^ceil(log2(t)) for a normal positive float t (the ue8m0 activation scale of
// wanferenz/kernels/torch_ops.py:17-21: a power of two keeps its exponent,
// anything else rounds up).  Returns the e8m0 byte (biased exponent).
__device__ __forceinline__ int pow2_ceil_e8m0(float t) {
  uint32_t b = __float_as_uint(t);
  int e = int((b >> 23) & 0xFFu);
  return e + ((b & 0x7FFFFFu) != 0u ? 1 : 0);
}

__device__ __forceinline__ float e8m0_to_f32(int e) { return __uint_as_float(uint32_t(e) << 23); }

// |x| folded into a running block amax the way torch's amax reduces: a NaN
// anywhere makes the result NaN.  The magnitude bits of a float order as
// unsigned integers like the magnitudes themselves, and every NaN sorts above
// +inf, so an integer max of the sign-cleared bits is that reduction.
__device__ __forceinline__ float absmax(float m, float x) {
  return __uint_as_float(max(__float_as_uint(m) & 0x7FFFFFFFu, __float_as_uint(x) & 0x7FFFFFFFu));
}

__device__ __forceinline__ bool is_finite_f32(float x) {
  return (__float_as_uint(x) & 0x7F800000u) != 0x7F800000u;
}

// clamp(x, lo, hi) as torch's clamp: NaN passes through.
__device__ __forceinline__ float clamp_keep_nan(float x, float lo, float hi) {
  return x < lo ? lo : (x > hi ? hi : x);
}

// Activation block scale from the block's amax (torch_ops.py:38-43):
// amax floored at 1e-4, then amax/448 (fp32) or its power-of-two ceiling.
// Non-finite blocks follow the reference's torch arithmetic: the floor keeps
// NaN, the fp32 scale is NaN or inf, and the power-of-two rule gives 1 (frexp
// returns exponent 0 for a non-finite value, torch_ops.py:17-21).
struct ActScale {
  float s;       // the scale the reference stores
  float inv;     // exact reciprocal when pow2 (multiply == divide)
  int e8m0;      // biased exponent byte when pow2, else 127
};

__device__ __forceinline__ ActScale act_scale(float amax, bool pow2) {
  amax = amax < 1e-4f ? 1e-4f : amax;
  float t = amax * (1.0f / 448.0f);
  ActScale r;
  if (pow2) {
    int e = is_finite_f32(t) ? pow2_ceil_e8m0(t) : kE8m0One;
    r.e8m0 = e;
    r.s = e8m0_to_f32(e);
    r.inv = e8m0_to_f32(254 - e);
  } else {
    r.e8m0 = kE8m0One;
    r.s = t;
    r.inv = 0.0f;
  }
  return r;
}

// x / s, clamped to the e4m3 range (torch_ops.py:44; NaN stays NaN).  For a
// power-of-two scale the reciprocal multiply is exact, so it equals the IEEE
// quotient.
__device__ __forceinline__ float quant_div(float x, const ActScale& sc, bool pow2) {
  const float q = pow2 ? x * sc.inv : x / sc.s;
  return clamp_keep_nan(q, -kFp8Max, kFp8Max);
}

// Two floats (already within +-448) -> two e4m3fn bytes, RNE, via the
// hardware converter.  word_sel picks the low or high 16 bits of `old`.
__device__ __forceinline__ uint32_t pack_fp8x4(float a, float b, float c, float d) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true));
}

// act_quant codes of eight values at scale sc, packed e4m3 (quant_div, then
// the converter's RNE).  fast: the clamp to +-448 is left out, which holds for
// power-of-two scales when the block amax is finite: s >= amax / 448 bounds
// |x / s| by 448, up to the rounding of amax / 448, which converts to 448 all
// the same.
__device__ __forceinline__ uint2 quant8(const float (&f)[8], const ActScale& sc, bool pow2, bool fast) {
  if (fast)
    return make_uint2(pack_fp8x4(f[0] * sc.inv, f[1] * sc.inv, f[2] * sc.inv, f[3] * sc.inv),
                      pack_fp8x4(f[4] * sc.inv, f[5] * sc.inv, f[6] * sc.inv, f[7] * sc.inv));
  return make_uint2(pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2), quant_div(f[2], sc, pow2),
                               quant_div(f[3], sc, pow2)),
                    pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2), quant_div(f[6], sc, pow2),
                               quant_div(f[7], sc, pow2)));
}

// the eight bf16 values packed in v, as floats
__device__ __forceinline__ void bf16x8_unpack(const v4i& v, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(uint32_t(v[i]) << 16);
    f[2 * i + 1] = __uint_as_float(uint32_t(v[i]) & 0xFFFF0000u);
  }
}

// ---------------------------------------------------------------- wave ops ---

// whether quant8 may leave out its clamp for every lane of the wave (the
// active lanes' block amaxes): power-of-two scales, every amax finite
__device__ __forceinline__ bool quant_fast(float amax, bool pow2) {
  return pow2 && __ballot((__float_as_uint(amax) & 0x7F800000u) == 0x7F800000u) == 0ull;
}

// Block amax across lanes (see absmax: NaN wins).
__device__ __forceinline__ float wave_absmax_xor(float v, int mask) {
  return absmax(v, __shfl_xor(v, mask, kWave));
}

// absmax over each row of 16 lanes, every lane of the row gets it: DPP moves
// within the row (quad xor 1, quad xor 2, then the half-row and row mirrors,
// which pair each quad with the others), no LDS round trip.  The integer max
// of the sign-cleared bits is absmax's reduction.
__device__ __forceinline__ float row16_absmax(float v) {
  uint32_t m = __float_as_uint(v) & 0x7FFFFFFFu;
  m = max(m, uint32_t(__builtin_amdgcn_mov_dpp(int(m), 0xB1, 0xF, 0xF, false)));   // quad_perm [1,0,3,2]
  m = max(m, uint32_t(__builtin_amdgcn_mov_dpp(int(m), 0x4E, 0xF, 0xF, false)));   // quad_perm [2,3,0,1]
  m = max(m, uint32_t(__builtin_amdgcn_mov_dpp(int(m), 0x141, 0xF, 0xF, false)));  // row_half_mirror
  m = max(m, uint32_t(__builtin_amdgcn_mov_dpp(int(m), 0x140, 0xF, 0xF, false)));  // row_mirror
  return __uint_as_float(m);
}

// absmax of 8 bf16 values (16 bytes), as an f32: the packed 16-bit integer max
// of the sign-cleared bits (absmax's order, NaN above inf), then widened.
__device__ __forceinline__ float bf16x8_absmax(const v4i& w) {
  typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
  auto a = [&](int i) { return __builtin_bit_cast(u16x2, uint32_t(w[i]) & 0x7FFF7FFFu); };
  const u16x2 m = __builtin_elementwise_max(__builtin_elementwise_max(a(0), a(1)),
                                            __builtin_elementwise_max(a(2), a(3)));
  return __uint_as_float(uint32_t(m.x > m.y ? m.x : m.y) << 16);
}

// ---------------------------------------------------------------- MFMA -------

template <int FMT_A, int FMT_B>
__device__ __forceinline__ v4f mfma_scaled(const v8i& a, const v8i& b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, 0, sa, 0, sb);
}
// The same with B's e8m0 scale byte OPB (0..3) of the dword sb: the MFMA
// selects it, no shift or mask on the VALU.
template <int FMT_A, int FMT_B, int OPB>
__device__ __forceinline__ v4f mfma_scaled_bsel(const v8i& a, const v8i& b, v4f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, FMT_A, FMT_B, 0, sa, OPB, sb);
}

// ---------------------------------------------------------------- loads ------

__device__ __forceinline__ v4i load16(const void* p) {
  return *reinterpret_cast<const v4i*>(p);
}

__device__ __forceinline__ v4i load16_nt(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

// One 16-byte-per-lane buffer load straight into LDS at lds_base + 16 * lane.
// Written as asm so the compiler does not treat it as an LDS store it must
// wait for before every LDS read: the kernel waits for it itself (a vmcnt
// wait and a barrier before the rows are read), which lets later loads stay
// in flight meanwhile.
__device__ __forceinline__ void load_lds_16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// The same, 4 bytes per lane, to lds_base + 4 * lane.
__device__ __forceinline__ void load_lds_4(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(lds_base), "v"(voffset), "s"(rsrc)
               : "memory", "m0");
}

// load_lds_16 / load_lds_4 with a wave-uniform byte offset added in the
// instruction's scalar offset operand.
__device__ __forceinline__ void load_lds_16(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voffset,
                                            uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(lds_base), "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}

__device__ __forceinline__ void load_lds_4(__amdgpu_buffer_rsrc_t rsrc, uint32_t lds_base, uint32_t voffset,
                                           uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               :
               : "s"(lds_base), "v"(voffset), "s"(rsrc), "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}

// s_waitcnt immediate that waits for vmcnt <= n only (n < 64; gfx9 encoding:
// vmcnt in bits 3:0 and 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima).
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
// ... vmcnt <= n and lgkmcnt = 0.
constexpr int vmcnt_lgkm0(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4); }
// ... and one that waits for lgkmcnt <= n only (n < 16).
constexpr int lgkmcnt_only(int n) { return 15 | (3 << 14) | (7 << 4) | (n << 8); }

// LDS byte address of a __shared__ object (the m0 operand of load_lds_16).
template <typename X>
__device__ __forceinline__ uint32_t lds_addr(X* p) {
  return uint32_t(uintptr_t((__attribute__((address_space(3))) X*)p));
}

// Workgroups are dispatched to the XCDs round-robin (block b to XCD b % 8),
// each XCD with its own L2.  xcd_runs renumbers the blocks [d0, d0 + n) so
// that each XCD takes runs of 64 consecutive logical blocks (as many as its
// CUs hold at once at two per CU): blocks that share operands, placed next to
// each other in the logical order, then meet in one L2.  Run j goes to XCD
// j % 8; the last, partial round of 8 runs is split contiguously.  A bijection
// on [d0, d0 + n) for any n (checked exhaustively on the CPU), so only
// locality depends on the dispatch order.
__device__ __forceinline__ int xcd_runs(int b, int d0, int n) {
  constexpr int kXcds = 8, kRun = 64;
  const int x = b % kXcds;
  const int fx = d0 + ((x - d0) & (kXcds - 1));  // first routed block on XCD x
  const int k = (b - fx) / kXcds;                // b's place among them
  const int full = n / (kXcds * kRun);           // complete rounds of 8 runs
  if (k < full * kRun) return ((k / kRun) * kXcds + x) * kRun + k % kRun;
  int before = 0;  // blocks of the last round on the XCDs ahead of x
  for (int y = 0; y < x; ++y) {
    const int fy = d0 + ((y - d0) & (kXcds - 1));
    before += (fy < d0 + n ? (d0 + n - fy + kXcds - 1) / kXcds : 0) - full * kRun;
  }
  return full * kXcds * kRun + before + (k - full * kRun);
}


}  // namespace wz

// Error reporting (errors.hip) and optional launch timing (prof.hip).
namespace wz {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
int cu_count();
int prof_pre(hipStream_t s, hipEvent_t* start, hipEvent_t* stop);
void prof_post(int slot, const char* name);
}  // namespace wz

// Launch, timed when profiling is on: WZ_LAUNCH("name", stream, kernel, grid, block, lds, args...).
// A timed launch goes through hipExtLaunchKernelGGL, whose start/stop events take the
// dispatch's own begin and end timestamps (no marker packets around the kernel).
#define WZ_LAUNCH(NAME, STREAM, KERNEL, GRID, BLOCK, LDS, ...)                                  \
  do {                                                                                          \
    hipEvent_t wz_ev_b_ = nullptr, wz_ev_e_ = nullptr;                                          \
    const int wz_prof_slot_ = ::wz::prof_pre(STREAM, &wz_ev_b_, &wz_ev_e_);                      \
    if (wz_prof_slot_ >= 0) {                                                                   \
      hipExtLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, STREAM, wz_ev_b_, wz_ev_e_, 0, __VA_ARGS__); \
      ::wz::prof_post(wz_prof_slot_, NAME);                                                     \
    } else {                                                                                    \
      hipLaunchKernelGGL(KERNEL, GRID, BLOCK, LDS, STREAM, __VA_ARGS__);                        \
    }                                                                                           \
  } while (0)
