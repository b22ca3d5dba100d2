// Load-time relayout of the expert banks into MFMA-ready tiles.
//
// A 16-row x 128-K weight tile is what one V_MFMA_SCALE 16x16x128 consumes
// from one wave: lane l = 16*g + r holds row r, K [32g, 32g+32) (e2m1, 16
// bytes) or K [16g, +16) and [64+16g, +16) (e4m3, 2 x 16 bytes).  Storing the
// tile as 1 KB blocks in lane order makes every weight load instruction of a
// wave read 1 KB contiguous, and a wave's K range a single contiguous stream
// (the row-major reference bank spreads each instruction over 16 rows).
// The e8m0 scales of four consecutive K-blocks are packed into one dword per
// lane (byte j = K-block 4*kg + j), so one 4-byte load serves four MFMAs.
#include "common.h"

namespace wz {

// mode 0: routed w13, 1: routed w2, 2: shared w13 (FP8), 3: shared w2 (FP8)
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ src0,
                                                           const uint8_t* __restrict__ src1,
                                                           uint8_t* __restrict__ dst, int64_t n16,
                                                           int mode, int E, int D, int I) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n16) return;
  const int lane = int(i & 63), r = lane & 15, g = lane >> 4;
  int64_t blk = i >> 6;  // 1 KB block index
  const uint8_t* src;
  if (mode == 0) {
    const int KB = D / 128, FT = I / 16;
    const int m = int(blk & 1);
    blk >>= 1;
    const int kb = int(blk % KB);
    blk /= KB;
    const int ft = int(blk % FT);
    const int64_t e = blk / FT;
    const int64_t row = e * 2 * I + int64_t(m) * I + ft * 16 + r;
    src = src0 + row * (D / 2) + kb * 64 + g * 16;
  } else if (mode == 1) {
    const int KB = I / 128, DT = D / 16;
    const int kb = int(blk % KB);
    blk /= KB;
    const int dt = int(blk % DT);
    const int64_t e = blk / DT;
    const int64_t row = e * D + dt * 16 + r;
    src = src0 + row * (I / 2) + kb * 64 + g * 16;
  } else if (mode == 2) {
    const int KB = D / 128;
    const int h = int(blk & 1);
    blk >>= 1;
    const int m = int(blk & 1);
    blk >>= 1;
    const int kb = int(blk % KB);
    const int ft = int(blk / KB);
    src = (m == 0 ? src0 : src1) + int64_t(ft * 16 + r) * D + kb * 128 + h * 64 + g * 16;
  } else {
    const int KB = I / 128;
    const int h = int(blk & 1);
    blk >>= 1;
    const int kb = int(blk % KB);
    const int dt = int(blk / KB);
    src = src0 + int64_t(dt * 16 + r) * I + kb * 128 + h * 64 + g * 16;
  }
  *reinterpret_cast<v4i*>(dst + i * 16) = load16(src);
}

// mode 0: routed w13 scales [E, 2I, D/32]; 1: routed w2 scales [E, D, I/32]
__global__ __launch_bounds__(256) void pack_scales_kernel(const uint8_t* __restrict__ src,
                                                          uint32_t* __restrict__ dst, int64_t n4,
                                                          int mode, int D, int I) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n4) return;
  const int lane = int(i & 63), r = lane & 15, g = lane >> 4;
  int64_t blk = i >> 6;
  int64_t row;
  int K, KB, kg;
  if (mode == 0) {
    K = D;
    KB = D / 128;
    const int KG = (KB + 3) / 4, FT = I / 16;
    const int m = int(blk & 1);
    blk >>= 1;
    kg = int(blk % KG);
    blk /= KG;
    const int ft = int(blk % FT);
    const int64_t e = blk / FT;
    row = e * 2 * I + int64_t(m) * I + ft * 16 + r;
  } else {
    K = I;
    KB = I / 128;
    const int KG = (KB + 3) / 4, DT = D / 16;
    kg = int(blk % KG);
    blk /= KG;
    const int dt = int(blk % DT);
    const int64_t e = blk / DT;
    row = e * D + dt * 16 + r;
  }
  uint32_t v = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kb = kg * 4 + j;
    if (kb < KB) v |= uint32_t(src[row * (K / 32) + kb * 4 + g]) << (8 * j);
  }
  dst[i] = v;
}

static int64_t packed_bytes(const wz_moe_desc* d, int which) {
  const int64_t E = d->n_experts, D = d->dim, I = d->inter;
  switch (which) {
    case 0: return E * (I / 16) * (D / 128) * 2 * 1024;
    case 1: return E * (I / 16) * ((D / 128 + 3) / 4) * 2 * 256;
    case 2: return E * (D / 16) * (I / 128) * 1024;
    case 3: return E * (D / 16) * ((I / 128 + 3) / 4) * 256;
    case 4: return (I / 16) * (D / 128) * 2 * 2 * 1024;
    case 5: return (D / 16) * (I / 128) * 2 * 1024;
    default: return -1;
  }
}

}  // namespace wz

extern "C" size_t wz_moe_packed_bytes(const wz_moe_desc* d, int which) {
  if (!d) return 0;
  const int64_t b = wz::packed_bytes(d, which);
  return b < 0 ? 0 : size_t(b);
}

namespace wz {

// A dense FP8 weight [N, K] in the shared-expert w2 tile format:
// [N/16][K/128][2 halves][1 KB].
int launch_pack_fp8(const void* w, int64_t N, int64_t K, void* dst, hipStream_t stream) {
  const int64_t n16 = N * K / 16;
  WZ_LAUNCH("fp8_pack", stream, pack_weights_kernel, dim3(unsigned((n16 + 255) / 256)), dim3(256), 0,
            static_cast<const uint8_t*>(w), nullptr, static_cast<uint8_t*>(dst), n16, 3, 1, int(N), int(K));
  return check_launch("fp8_pack");
}

}  // namespace wz

extern "C" int wz_moe_pack(const wz_moe_desc* d, void* w13p, void* w13p_s, void* w2p, void* w2p_s,
                           void* sh13p, void* sh2p, hipStream_t stream) {
  using namespace wz;
  if (!d || !d->w13 || !d->w13_s || !d->w2 || !d->w2_s || !d->sh_w1 || !d->sh_w3 || !d->sh_w2)
    return set_error(WZ_EINVAL, "moe_pack: reference banks missing");
  if (!w13p || !w13p_s || !w2p || !w2p_s || !sh13p || !sh2p)
    return set_error(WZ_EINVAL, "moe_pack: null output");
  if (d->dim % 128 || d->inter % 128) return set_error(WZ_EINVAL, "moe_pack: dims must be multiples of 128");
  const int E = d->n_experts, D = d->dim, I = d->inter;
  struct W {
    const void* a;
    const void* b;
    void* dst;
    int which, mode;
  } ws[] = {{d->w13, nullptr, w13p, 0, 0}, {d->w2, nullptr, w2p, 2, 1},
            {d->sh_w1, d->sh_w3, sh13p, 4, 2}, {d->sh_w2, nullptr, sh2p, 5, 3}};
  for (const W& w : ws) {
    const int64_t n16 = packed_bytes(d, w.which) / 16;
    WZ_LAUNCH("moe_pack", stream, pack_weights_kernel, dim3(unsigned((n16 + 255) / 256)), dim3(256), 0,
              static_cast<const uint8_t*>(w.a), static_cast<const uint8_t*>(w.b), static_cast<uint8_t*>(w.dst),
              n16, w.mode, E, D, I);
    if (int rc = check_launch("moe_pack weights")) return rc;
  }
  struct S {
    const void* src;
    void* dst;
    int which, mode;
  } ss[] = {{d->w13_s, w13p_s, 1, 0}, {d->w2_s, w2p_s, 3, 1}};
  for (const S& s : ss) {
    const int64_t n4 = packed_bytes(d, s.which) / 4;
    WZ_LAUNCH("moe_pack", stream, pack_scales_kernel, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0,
              static_cast<const uint8_t*>(s.src), static_cast<uint32_t*>(s.dst), n4, s.mode, D, I);
    if (int rc = check_launch("moe_pack scales")) return rc;
  }
  return WZ_OK;
}
