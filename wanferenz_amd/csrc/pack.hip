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

// mode 0: routed w13 (src0 = w1 rows, src1 = w3 rows of expert 0, `estride`
// bytes between experts), 1: routed w2, 2: shared w13 (FP8), 3: shared w2 (FP8)
__global__ __launch_bounds__(256) void pack_weights_kernel(const uint8_t* __restrict__ src0,
                                                           const uint8_t* __restrict__ src1,
                                                           uint8_t* __restrict__ dst, int64_t n16,
                                                           int mode, int64_t estride, int D, int I) {
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
    src = (m == 0 ? src0 : src1) + e * estride + int64_t(ft * 16 + r) * (D / 2) + kb * 64 + g * 16;
  } else if (mode == 1) {
    const int KB = I / 128, DT = D / 16;
    const int kb = int(blk % KB);
    blk /= KB;
    const int dt = int(blk % DT);
    const int64_t e = blk / DT;
    src = src0 + e * estride + int64_t(dt * 16 + r) * (I / 2) + kb * 64 + g * 16;
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

// mode 0: routed w13 scales (src0 = w1 rows [I, D/32], src1 = w3 rows, `estride`
// bytes between experts); 1: routed w2 scales [D, I/32] per expert
__global__ __launch_bounds__(256) void pack_scales_kernel(const uint8_t* __restrict__ src0,
                                                          const uint8_t* __restrict__ src1,
                                                          uint32_t* __restrict__ dst, int64_t n4,
                                                          int mode, int64_t estride, int D, int I) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n4) return;
  const int lane = int(i & 63), r = lane & 15, g = lane >> 4;
  int64_t blk = i >> 6;
  const uint8_t* row;
  int KB, kg;
  if (mode == 0) {
    KB = D / 128;
    const int KG = (KB + 3) / 4, FT = I / 16;
    const int m = int(blk & 1);
    blk >>= 1;
    kg = int(blk % KG);
    blk /= KG;
    const int ft = int(blk % FT);
    const int64_t e = blk / FT;
    row = (m == 0 ? src0 : src1) + e * estride + int64_t(ft * 16 + r) * (D / 32);
  } else {
    KB = I / 128;
    const int KG = (KB + 3) / 4, DT = D / 16;
    kg = int(blk % KG);
    blk /= KG;
    const int dt = int(blk % DT);
    const int64_t e = blk / DT;
    row = src0 + e * estride + int64_t(dt * 16 + r) * (I / 32);
  }
  uint32_t v = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kb = kg * 4 + j;
    if (kb < KB) v |= uint32_t(row[kb * 4 + g]) << (8 * j);
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
            static_cast<const uint8_t*>(w), nullptr, static_cast<uint8_t*>(dst), n16, 3, int64_t(0), int(N),
            int(K));
  return check_launch("fp8_pack");
}

static int pack_w(const void* a, const void* b, void* dst, int64_t bytes, int mode, int64_t estride, int D, int I,
                  hipStream_t stream) {
  const int64_t n16 = bytes / 16;
  WZ_LAUNCH("moe_pack", stream, pack_weights_kernel, dim3(unsigned((n16 + 255) / 256)), dim3(256), 0,
            static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), static_cast<uint8_t*>(dst), n16, mode,
            estride, D, I);
  return check_launch("moe_pack weights");
}

static int pack_s(const void* a, const void* b, void* dst, int64_t bytes, int mode, int64_t estride, int D, int I,
                  hipStream_t stream) {
  const int64_t n4 = bytes / 4;
  WZ_LAUNCH("moe_pack", stream, pack_scales_kernel, dim3(unsigned((n4 + 255) / 256)), dim3(256), 0,
            static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), static_cast<uint32_t*>(dst), n4, mode,
            estride, D, I);
  return check_launch("moe_pack scales");
}

static int pack_dims_ok(const wz_moe_desc* d, const char* what) {
  if (d->dim <= 0 || d->inter <= 0 || d->dim % 128 || d->inter % 128 || d->n_experts <= 0)
    return set_error(WZ_EINVAL, "%s: dim=%d, inter=%d must be positive multiples of 128, n_experts=%d > 0", what,
                     d->dim, d->inter, d->n_experts);
  return WZ_OK;
}

}  // namespace wz

extern "C" int wz_moe_pack(const wz_moe_desc* d, void* w13p, void* w13p_s, void* w2p, void* w2p_s,
                           void* sh13p, void* sh2p, hipStream_t stream) {
  using namespace wz;
  if (!d || !d->w13 || !d->w13_s || !d->w2 || !d->w2_s || !d->sh_w1 || !d->sh_w3 || !d->sh_w2)
    return set_error(WZ_EINVAL, "moe_pack: reference banks missing");
  if (!w13p || !w13p_s || !w2p || !w2p_s || !sh13p || !sh2p)
    return set_error(WZ_EINVAL, "moe_pack: null output");
  if (int rc = pack_dims_ok(d, "moe_pack")) return rc;
  const int D = d->dim, I = d->inter;
  const uint8_t* w13 = static_cast<const uint8_t*>(d->w13);
  const uint8_t* w13s = static_cast<const uint8_t*>(d->w13_s);
  const int64_t w1b = int64_t(I) * D / 2, s1b = int64_t(I) * D / 32;
  if (int rc = pack_w(w13, w13 + w1b, w13p, packed_bytes(d, 0), 0, 2 * w1b, D, I, stream)) return rc;
  if (int rc = pack_w(d->w2, nullptr, w2p, packed_bytes(d, 2), 1, w1b, D, I, stream)) return rc;
  if (int rc = pack_w(d->sh_w1, d->sh_w3, sh13p, packed_bytes(d, 4), 2, 0, D, I, stream)) return rc;
  if (int rc = pack_w(d->sh_w2, nullptr, sh2p, packed_bytes(d, 5), 3, 0, D, I, stream)) return rc;
  if (int rc = pack_s(w13s, w13s + s1b, w13p_s, packed_bytes(d, 1), 0, 2 * s1b, D, I, stream)) return rc;
  return pack_s(d->w2_s, nullptr, w2p_s, packed_bytes(d, 3), 1, s1b, D, I, stream);
}

extern "C" int wz_moe_pack_expert(const wz_moe_desc* d, int64_t e, const void* w1, const void* w1_s,
                                  const void* w3, const void* w3_s, const void* w2, const void* w2_s,
                                  hipStream_t stream) {
  using namespace wz;
  if (!d) return set_error(WZ_EINVAL, "moe_pack_expert: null descriptor");
  if (int rc = pack_dims_ok(d, "moe_pack_expert")) return rc;
  if (e < 0 || e >= d->n_experts)
    return set_error(WZ_EINVAL, "moe_pack_expert: expert %lld outside 0..%d", (long long)e, d->n_experts - 1);
  if (!w1 || !w1_s || !w3 || !w3_s || !w2 || !w2_s) return set_error(WZ_EINVAL, "moe_pack_expert: null input");
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s)
    return set_error(WZ_EINVAL, "moe_pack_expert: the descriptor's packed banks are not set");
  const int D = d->dim, I = d->inter;
  const int64_t E = d->n_experts;
  auto slot = [&](const void* bank, int which) {
    return const_cast<uint8_t*>(static_cast<const uint8_t*>(bank)) + packed_bytes(d, which) / E * e;
  };
  if (int rc = pack_w(w1, w3, slot(d->w13p, 0), packed_bytes(d, 0) / E, 0, 0, D, I, stream)) return rc;
  if (int rc = pack_w(w2, nullptr, slot(d->w2p, 2), packed_bytes(d, 2) / E, 1, 0, D, I, stream)) return rc;
  if (int rc = pack_s(w1_s, w3_s, slot(d->w13p_s, 1), packed_bytes(d, 1) / E, 0, 0, D, I, stream)) return rc;
  return pack_s(w2_s, nullptr, slot(d->w2p_s, 3), packed_bytes(d, 3) / E, 1, 0, D, I, stream);
}

extern "C" int wz_moe_pack_shared(const wz_moe_desc* d, const void* sh_w1, const void* sh_w3, const void* sh_w2,
                                  hipStream_t stream) {
  using namespace wz;
  if (!d) return set_error(WZ_EINVAL, "moe_pack_shared: null descriptor");
  if (int rc = pack_dims_ok(d, "moe_pack_shared")) return rc;
  if (!sh_w1 || !sh_w3 || !sh_w2) return set_error(WZ_EINVAL, "moe_pack_shared: null input");
  if (!d->sh13p || !d->sh2p) return set_error(WZ_EINVAL, "moe_pack_shared: the descriptor's packed banks are not set");
  const int D = d->dim, I = d->inter;
  void* sh13p = const_cast<void*>(d->sh13p);
  void* sh2p = const_cast<void*>(d->sh2p);
  if (int rc = pack_w(sh_w1, sh_w3, sh13p, packed_bytes(d, 4), 2, 0, D, I, stream)) return rc;
  return pack_w(sh_w2, nullptr, sh2p, packed_bytes(d, 5), 3, 0, D, I, stream);
}

extern "C" size_t wz_fp4_packed_scale_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || N % 16 || K % 128) return 0;
  return size_t(N / 16) * size_t((K / 128 + 3) / 4) * 256;
}

extern "C" int wz_fp4_pack(const void* w_fp4x2, const void* w_s_e8m0, int64_t N, int64_t K, void* packed,
                           void* packed_s, hipStream_t stream) {
  using namespace wz;
  if (N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp4_pack: N=%lld must be a multiple of 16 and K=%lld of 128", (long long)N,
                     (long long)K);
  if (N > (1 << 30) || K > (1 << 30)) return set_error(WZ_EINVAL, "fp4_pack: dimension too large");
  if (!w_fp4x2 || !w_s_e8m0 || !packed || !packed_s) return set_error(WZ_EINVAL, "fp4_pack: null pointer");
  // the routed w2 relayout of a one-expert bank with D = N rows of K = I
  if (int rc = pack_w(w_fp4x2, nullptr, packed, N * K / 2, 1, 0, int(N), int(K), stream)) return rc;
  return pack_s(w_s_e8m0, nullptr, packed_s, int64_t(wz_fp4_packed_scale_bytes(N, K)), 1, 0, int(N), int(K), stream);
}
