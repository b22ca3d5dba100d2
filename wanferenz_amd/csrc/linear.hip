// FP8 block-scaled linear on packed weights (dense projections, decode and
// prefill widths).
//
// y[M, N] (bf16) = act_quant(x) . W^T, W e4m3 [N, K] with 128x128 block scales
// — linear() on an FP8 weight, architecture.py:121-132 (act_quant +
// fp8_gemm, reference.py:292-311; CPU statement torch_ops.py:93-99).  The
// weight is packed once (wz_fp8_pack) into 16-row x 128-K tiles of 2 x 1 KB
// in lane order, so every weight load instruction of a wave reads 1 KB
// contiguous; the row-major layout spreads each instruction over 16 rows.
//
// M <= 16, K in {1024, 2048, 4096}: fp8_gemv_kernel.  Persistent workgroups of
//   8 waves; wave w owns K-blocks [w NKB, (w+1) NKB) of every 16-column tile.
//   The wave quantises its slice of x once (act_quant fused into the A
//   operand) and keeps it in registers, then the workgroup streams tiles
//   b, b+G, ... with the next tile's weights in flight during the current
//   tile's MFMAs; the eight K partials meet in LDS, summed in wave order.
// Otherwise: act_quant into the caller's workspace, then the dense tile GEMM
//   (launch_dense_fp8: M-tiles of <= 64 rows staged in LDS).
#include "mfma_ops.h"

#include <algorithm>

namespace wz {

int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream);
int launch_pack_fp8(const void* w, int64_t N, int64_t K, void* dst, hipStream_t stream);
int launch_dense_fp8(const uint8_t* wp, const void* w_s, int w_kind, const uint8_t* xq, const float* xs,
                     bool a_pow2, uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream);

constexpr int kGvWaves = 8;
constexpr int kGvThreads = kGvWaves * 64;
constexpr int kGvMaxM = 16;

// K-blocks per wave of the GEMV, 0 when K does not split into 8 x {1, 2, 4}
// (K = 1024, 2048, 4096; wider K would keep more A registers than fit).
static int gemv_nkb(int64_t K) {
  const int64_t kb = K / 128;
  if (K % 1024) return 0;
  const int64_t n = kb / kGvWaves;
  return (n == 1 || n == 2 || n == 4) ? int(n) : 0;
}

template <int NKB>
struct GvBuf {
  v8i w[NKB];
  int se[NKB];
  float sf[NKB];
};

// QA: x is pre-quantised e4m3 [M, K] with block scales xs [M, K/128] of kind
// a_kind (fp8_gemm's a, a_s); otherwise x is bf16 and act_quant is fused.
template <int NKB, bool QA>
__global__ __launch_bounds__(kGvThreads) void fp8_gemv_kernel(const void* __restrict__ x,
                                                              const void* __restrict__ xs, int a_kind,
                                                              const uint8_t* __restrict__ wp,
                                                              const void* __restrict__ w_s, int w_kind,
                                                              uint16_t* __restrict__ y, int M, int N, int K,
                                                              int a_pow2i) {
  __shared__ float red[2][kGvWaves * 4 * kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const bool a_pow2 = a_pow2i != 0, bp = w_kind == WZ_WSCALE_E8M0;
  const int KB = K / 128, kb0 = wave * NKB, items = N / 16, G = gridDim.x;
  const int first = blockIdx.x;
  if (first >= items) return;

  auto fetch = [&](GvBuf<NKB>& b, int item) {
    const uint8_t* t = wp + (int64_t(item) * KB + kb0) * 2048 + lane * 16;
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const v4i lo = load16_nt(t + q * 2048), hi = load16_nt(t + q * 2048 + 1024);
      b.w[q] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int q = 0; q < NKB; ++q) fp8_wscale(w_s, int64_t(item >> 3) * KB + kb0 + q, w_kind, b.se[q], b.sf[q]);
  };

  // this wave's K slice of the (<= 16) token rows, quantised once.  The
  // weights are requested after the quantisation: issuing them first (weights
  // then x, or x then weights with the quantisation in between) measured
  // 0.3-1.3 us slower per launch.
  AOp a[NKB];
  if constexpr (QA) {
    const uint8_t* xrow = nl < M ? static_cast<const uint8_t*>(x) + int64_t(nl) * K : nullptr;
    const void* srow = a_kind == WZ_SCALE_UE8M0
                           ? static_cast<const void*>(static_cast<const uint8_t*>(xs) + int64_t(nl) * KB)
                           : static_cast<const void*>(static_cast<const float*>(xs) + int64_t(nl) * KB);
#pragma unroll
    for (int q = 0; q < NKB; ++q) a[q] = a_from_fp8(xrow, srow, kb0 + q, g, a_kind);
  } else {
    const uint16_t* xrow = nl < M ? static_cast<const uint16_t*>(x) + int64_t(nl) * K : nullptr;
#pragma unroll
    for (int q = 0; q < NKB; ++q) a[q] = a_from_bf16(xrow, kb0 + q, g, a_pow2);
  }
  GvBuf<NKB> b0, b1;
  fetch(b0, first);
  auto process = [&](const GvBuf<NKB>& b, int item, int par) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NKB; ++q) mma_step<kFmtFp8, kFmtFp8>(acc, a[q], b.w[q], b.se[q], b.sf[q], a_pow2, bp, lane);
    float* r = red[par];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[(wave * 4 + i) * kWave + lane] = acc[i];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = r[i * kWave + lane];
#pragma unroll
        for (int w = 1; w < kGvWaves; ++w) v += r[(w * 4 + i) * kWave + lane];
        const int row = g * 4 + i;
        if (row < M) y[int64_t(row) * N + item * 16 + nl] = f32_to_bf16(v);
      }
    }
  };

  int i = first;
  for (; i + 2 * G < items; i += 2 * G) {
    fetch(b1, i + G);
    process(b0, i, 0);
    __builtin_amdgcn_sched_barrier(0);
    fetch(b0, i + 2 * G);
    process(b1, i + G, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (i + G < items) {
    fetch(b1, i + G);
    process(b0, i, 0);
    process(b1, i + G, 1);
  } else {
    process(b0, i, 0);
  }
}

static int gemv_grid(int64_t N, int nkb);

static size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace wz

extern "C" int wz_fp8_pack(const void* w_e4m3, int64_t N, int64_t K, void* packed, hipStream_t stream) {
  using namespace wz;
  if (N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp8_pack: N=%lld must be a multiple of 16 and K=%lld of 128", (long long)N,
                     (long long)K);
  if (!w_e4m3 || !packed) return set_error(WZ_EINVAL, "fp8_pack: null pointer");
  return launch_pack_fp8(w_e4m3, N, K, packed, stream);
}

extern "C" size_t wz_fp8_linear_workspace_bytes(int64_t M, int64_t K) {
  using namespace wz;
  if (M <= 0 || K <= 0) return 0;
  if (M <= kGvMaxM && gemv_nkb(K)) return 0;
  return align256(size_t(M) * size_t(K)) + size_t(M) * size_t(K / 128) * 4;
}

extern "C" int wz_fp8_linear_packed(const void* x_bf16, const void* w_packed, const void* w_s, void* y_bf16,
                                    int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                                    void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp8_linear_packed: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return set_error(WZ_EINVAL, "fp8_linear_packed: dimension too large");
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
      (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
    return set_error(WZ_EINVAL, "fp8_linear_packed: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
  if (M == 0) return WZ_OK;
  if (!x_bf16 || !w_packed || !w_s || !y_bf16) return set_error(WZ_EINVAL, "fp8_linear_packed: null pointer");
  const bool pow2 = act_scale_kind != WZ_SCALE_F32;
  const int nkb = gemv_nkb(K);
  if (M <= kGvMaxM && nkb) {
    const dim3 grid(unsigned(gemv_grid(N, nkb)));
    const uint8_t* w = static_cast<const uint8_t*>(w_packed);
    uint16_t* y = static_cast<uint16_t*>(y_bf16);
#define WZ_GEMV(NKBV)                                                                                   \
  WZ_LAUNCH("fp8_gemv", stream, (fp8_gemv_kernel<NKBV, false>), grid, dim3(kGvThreads), 0, x_bf16,         \
            static_cast<const void*>(nullptr), 0, w, w_s, w_scale_kind, y, int(M), int(N), int(K), pow2 ? 1 : 0)
    switch (nkb) {
      case 1: WZ_GEMV(1); break;
      case 2: WZ_GEMV(2); break;
      default: WZ_GEMV(4); break;
    }
#undef WZ_GEMV
    return check_launch("fp8_gemv");
  }
  const size_t need = wz_fp8_linear_workspace_bytes(M, K);
  if (!ws || ws_bytes < need)
    return set_error(WZ_ESPACE, "fp8_linear_packed: workspace of %zu bytes needed for M=%lld K=%lld, got %zu", need,
                     (long long)M, (long long)K, ws_bytes);
  uint8_t* xq = static_cast<uint8_t*>(ws);
  float* xs = reinterpret_cast<float*>(xq + align256(size_t(M) * size_t(K)));
  const int qkind = pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  if (int rc = launch_act_quant(x_bf16, M, K, xq, xs, qkind, stream)) return rc;
  return launch_dense_fp8(static_cast<const uint8_t*>(w_packed), w_s, w_scale_kind, xq, xs, pow2,
                          static_cast<uint16_t*>(y_bf16), M, N, K, stream);
}

namespace wz {

__global__ void e8m0_to_f32_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = e8m0_to_f32(src[i]);
}

static int gemv_grid(int64_t N, int nkb) {
  // resident workgroups: one per CU at NKB = 4 (193 VGPRs), two below
  const int64_t items = N / 16, per_cu = nkb == 4 ? 1 : 2;
  return int(std::min<int64_t>(items, per_cu * int64_t(cu_count())));
}

}  // namespace wz

extern "C" size_t wz_fp8_gemm_packed_workspace_bytes(int64_t M, int64_t K, int act_scale_kind) {
  using namespace wz;
  if (M <= 0 || K <= 0) return 0;
  if (M <= kGvMaxM && gemv_nkb(K)) return 0;
  return act_scale_kind == WZ_SCALE_UE8M0 ? size_t(M) * size_t(K / 128) * 4 : 0;
}

extern "C" int wz_fp8_gemm_packed(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                                  void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                                  int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp8_gemm_packed: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return set_error(WZ_EINVAL, "fp8_gemm_packed: dimension too large");
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
      (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
    return set_error(WZ_EINVAL, "fp8_gemm_packed: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
  if (M == 0) return WZ_OK;
  if (!a_e4m3 || !a_s || !w_packed || !w_s || !c_bf16) return set_error(WZ_EINVAL, "fp8_gemm_packed: null pointer");
  const bool pow2 = act_scale_kind != WZ_SCALE_F32;
  const int nkb = gemv_nkb(K);
  const uint8_t* w = static_cast<const uint8_t*>(w_packed);
  uint16_t* c = static_cast<uint16_t*>(c_bf16);
  if (M <= kGvMaxM && nkb) {
    const dim3 grid(unsigned(gemv_grid(N, nkb)));
#define WZ_GEMV(NKBV)                                                                                            \
  WZ_LAUNCH("fp8_gemv", stream, (fp8_gemv_kernel<NKBV, true>), grid, dim3(kGvThreads), 0, a_e4m3, a_s,           \
            act_scale_kind, w, w_s, w_scale_kind, c, int(M), int(N), int(K), pow2 ? 1 : 0)
    switch (nkb) {
      case 1: WZ_GEMV(1); break;
      case 2: WZ_GEMV(2); break;
      default: WZ_GEMV(4); break;
    }
#undef WZ_GEMV
    return check_launch("fp8_gemv");
  }
  const float* xs = static_cast<const float*>(a_s);
  if (act_scale_kind == WZ_SCALE_UE8M0) {
    const size_t need = wz_fp8_gemm_packed_workspace_bytes(M, K, act_scale_kind);
    if (!ws || ws_bytes < need)
      return set_error(WZ_ESPACE, "fp8_gemm_packed: workspace of %zu bytes needed for M=%lld K=%lld, got %zu", need,
                       (long long)M, (long long)K, ws_bytes);
    const int64_t n = M * (K / 128);
    WZ_LAUNCH("e8m0_to_f32", stream, e8m0_to_f32_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
              static_cast<const uint8_t*>(a_s), static_cast<float*>(ws), n);
    if (int rc = check_launch("fp8_gemm_packed scales")) return rc;
    xs = static_cast<const float*>(ws);
  }
  return launch_dense_fp8(w, w_s, w_scale_kind, static_cast<const uint8_t*>(a_e4m3), xs, pow2, c, M, N, K, stream);
}
