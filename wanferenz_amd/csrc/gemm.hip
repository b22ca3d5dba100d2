// Block-scaled FP8 / MXFP4 GEMV-GEMM for skinny M (decode widths and up).
//
// C[M,N] (bf16) = sum over 128-wide K-blocks of (A_blk . W_blk^T) * scales
// (wanferenz/kernels/reference.py:235-311 fp8_gemm, :506-591 fp4_gemm; the CPU
// restatement torch_ops.py:93-108).
//
// Decode is bound by streaming W from HBM, so the kernel is shaped around the
// weight stream, not the M dimension:
//   * a workgroup owns 16 output columns (= 16 weight rows) and its four
//     waves split K into four contiguous ranges, so every weight byte is read
//     once, by one lane, in 16-byte loads; partial sums meet in LDS;
//   * each wave batches the loads of UNROLL K-blocks before issuing the MFMAs
//     to keep enough bytes in flight per CU;
//   * tokens ride on the MFMA's M side (16 rows per tile, MT tiles per wave),
//     padded with zero rows, so an M=1..16 GEMV is one V_MFMA_SCALE 16x16x128
//     per 16x128 weight block with no per-byte VALU dequantisation.
#include "mfma_ops.h"

namespace wz {

constexpr int kGemmThreads = 256;

// One workgroup's 16 output columns [n0, n0 + 16) for rows m_base .. m_base + 16 MT.
// kUnroll = K-blocks per load batch (a wave owns about nkb / 4 of them).
template <int WF, bool A_BF16, int MT, int kUnroll>
__device__ __forceinline__ void skinny_body(const void* __restrict__ A, const void* __restrict__ As, int act_kind,
                                            const uint8_t* __restrict__ W, const void* __restrict__ Ws, int w_kind,
                                            uint16_t* __restrict__ C, int M, int N, int K, int m_base, int n0) {
  __shared__ float red[4][MT][kWave][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int nkb = K / 128;
  const int kb0 = (wave * nkb) / 4, kb1 = ((wave + 1) * nkb) / 4;
  const int ldw = WF == kFmtFp4 ? K / 2 : K;
  const uint8_t* wrow = W + int64_t(n0 + nl) * ldw;
  const uint8_t* wsrow = WF == kFmtFp4 ? reinterpret_cast<const uint8_t*>(Ws) + int64_t(n0 + nl) * (K / 32)
                                       : nullptr;
  const bool a_pow2 = act_kind != WZ_SCALE_F32;
  const bool b_pow2 = WF == kFmtFp4 || w_kind == WZ_WSCALE_E8M0;

  v4f acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  for (int kb = kb0; kb < kb1; kb += kUnroll) {
    v8i bb[kUnroll];
    int sbe[kUnroll];
    float sbf[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int k = min(kb + u, kb1 - 1);  // past kb1: a valid re-read whose MFMA is skipped
      if (WF == kFmtFp4) {
        bb[u] = b_fp4(wrow, k, g);
        sbe[u] = b_fp4_scale(wsrow, k, g);
        sbf[u] = 1.0f;
      } else {
        bb[u] = b_fp8(wrow, k, g);
        fp8_wscale(Ws, int64_t(n0 >> 7) * nkb + k, w_kind, sbe[u], sbf[u]);
      }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      const int m = m_base + t * 16 + nl;
      if (A_BF16) {
        const bool live = m < M;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int k = kb + u;
          if (k < kb1) {
            const AOp a = a_from_bf16(live ? reinterpret_cast<const uint16_t*>(A) + int64_t(m) * K : nullptr, k, g,
                                      a_pow2);
            mma_step<kFmtFp8, WF>(acc[t], a, bb[u], sbe[u], sbf[u], a_pow2, b_pow2, lane);
          }
        }
      } else {
        // the tile's A blocks of this batch are all requested before the first
        // MFMA: rows past M read row M - 1 (their outputs are not stored) and
        // K-blocks past kb1 re-read the last one (their MFMAs are skipped)
        const int mr = min(m, M - 1);
        const uint8_t* arow = reinterpret_cast<const uint8_t*>(A) + int64_t(mr) * K;
        const void* asrow = act_kind == WZ_SCALE_UE8M0
                                ? static_cast<const void*>(reinterpret_cast<const uint8_t*>(As) + int64_t(mr) * nkb)
                                : static_cast<const void*>(reinterpret_cast<const float*>(As) + int64_t(mr) * nkb);
        AOp a[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) a[u] = a_from_fp8_row(arow, asrow, min(kb + u, kb1 - 1), g, act_kind);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u)
          if (kb + u < kb1) mma_step<kFmtFp8, WF>(acc[t], a[u], bb[u], sbe[u], sbf[u], a_pow2, b_pow2, lane);
      }
    }
  }

#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[wave][t][lane][i] = acc[t][i];
  __syncthreads();
  // Wave w finishes M-tiles t = w, w+4, ...; partials are summed in wave order.
  for (int t = wave; t < MT; t += 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = red[0][t][lane][i];
      v += red[1][t][lane][i];
      v += red[2][t][lane][i];
      v += red[3][t][lane][i];
      const int m = m_base + t * 16 + g * 4 + i;
      if (m < M) C[int64_t(m) * N + n0 + nl] = f32_to_bf16(v);
    }
  }
}

template <int WF, bool A_BF16, int MT, int U>
__global__ __launch_bounds__(kGemmThreads) void skinny_gemm_kernel(
    const void* __restrict__ A, const void* __restrict__ As, int act_kind,
    const uint8_t* __restrict__ W, const void* __restrict__ Ws, int w_kind,
    uint16_t* __restrict__ C, int M, int N, int K) {
  skinny_body<WF, A_BF16, MT, U>(A, As, act_kind, W, Ws, w_kind, C, M, N, K, blockIdx.y * (16 * MT), blockIdx.x * 16);
}

// K-blocks per load batch for a wave that owns ceil(nkb / 4) of them.
static inline int skinny_unroll(int64_t K) {
  const int64_t per_wave = (K / 128 + 3) / 4;
  return per_wave >= 8 ? 8 : per_wave >= 4 ? 4 : 2;
}

// Row g of A against its own MXFP4 weight W[g] (the per-expert GEMV of the
// banked decode path): blockIdx.y = g, each row one M=1 skinny product.
template <int U>
__global__ __launch_bounds__(kGemmThreads) void grouped_fp4_kernel(const uint8_t* __restrict__ A,
                                                                   const void* __restrict__ As, int act_kind,
                                                                   const uint8_t* __restrict__ W,
                                                                   const uint8_t* __restrict__ Ws,
                                                                   uint16_t* __restrict__ C, int N, int K) {
  const int64_t g = blockIdx.y;
  const int nkb = K / 128;
  const void* as_g = act_kind == WZ_SCALE_UE8M0
                         ? static_cast<const void*>(static_cast<const uint8_t*>(As) + g * nkb)
                         : static_cast<const void*>(static_cast<const float*>(As) + g * nkb);
  skinny_body<kFmtFp4, false, 1, U>(A + g * K, as_g, act_kind, W + g * N * (K / 2), Ws + g * N * (K / 32),
                                 WZ_WSCALE_E8M0, C + g * N, 1, N, K, 0, blockIdx.x * 16);
}

template <int WF, bool A_BF16>
static int launch_skinny(const void* A, const void* As, int act_kind, const void* W, const void* Ws,
                         int w_kind, void* C, int64_t M, int64_t N, int64_t K, hipStream_t stream,
                         const char* what) {
  if (M == 0) return WZ_OK;
  int mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
  const int64_t rows_per_block = 16 * mt;
  dim3 grid(unsigned(N / 16), unsigned((M + rows_per_block - 1) / rows_per_block));
  const uint8_t* w = static_cast<const uint8_t*>(W);
  uint16_t* c = static_cast<uint16_t*>(C);
  const int u = skinny_unroll(K);
#define WZ_SKINNY(MTV, UV)                                                                            \
  WZ_LAUNCH(what, stream, (skinny_gemm_kernel<WF, A_BF16, MTV, UV>), grid, dim3(kGemmThreads), 0, A, As, \
            act_kind, w, Ws, w_kind, c, int(M), int(N), int(K))
#define WZ_SKINNY_U(MTV)            \
  if (u == 8) {                     \
    WZ_SKINNY(MTV, 8);              \
  } else if (u == 4) {              \
    WZ_SKINNY(MTV, 4);              \
  } else {                          \
    WZ_SKINNY(MTV, 2);              \
  }
  switch (mt) {
    case 1: WZ_SKINNY_U(1); break;
    case 2: WZ_SKINNY_U(2); break;
    case 4: WZ_SKINNY_U(4); break;
    default: WZ_SKINNY_U(8); break;
  }
#undef WZ_SKINNY_U
#undef WZ_SKINNY
  return check_launch(what);
}

static int check_dims(const char* what, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N <= 0 || K <= 0)
    return set_error(WZ_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", what, (long long)M,
                     (long long)N, (long long)K);
  if (K % 128)
    return set_error(WZ_EINVAL, "%s: K=%lld must be a multiple of 128", what, (long long)K);
  if (N % 16)
    return set_error(WZ_EINVAL, "%s: N=%lld must be a multiple of 16", what, (long long)N);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return set_error(WZ_EINVAL, "%s: dimension too large", what);
  return WZ_OK;
}

}  // namespace wz

extern "C" int wz_fp8_gemm(const void* a_e4m3, const void* a_s, const void* w_e4m3, const void* w_s,
                           void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                           int w_scale_kind, hipStream_t stream) {
  using namespace wz;
  if (int rc = check_dims("fp8_gemm", M, N, K)) return rc;
  if (act_scale_kind < 0 || act_scale_kind > 2 || (w_scale_kind != 0 && w_scale_kind != 1))
    return set_error(WZ_EINVAL, "fp8_gemm: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
  if (M && (!a_e4m3 || !a_s || !w_e4m3 || !w_s || !c_bf16))
    return set_error(WZ_EINVAL, "fp8_gemm: null pointer");
  return launch_skinny<kFmtFp8, false>(a_e4m3, a_s, act_scale_kind, w_e4m3, w_s, w_scale_kind,
                                       c_bf16, M, N, K, stream, "fp8_gemm");
}

extern "C" int wz_fp8_linear(const void* x_bf16, const void* w_e4m3, const void* w_s, void* y_bf16,
                             int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                             hipStream_t stream) {
  using namespace wz;
  if (int rc = check_dims("fp8_linear", M, N, K)) return rc;
  if (act_scale_kind < 0 || act_scale_kind > 2 || (w_scale_kind != 0 && w_scale_kind != 1))
    return set_error(WZ_EINVAL, "fp8_linear: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
  if (M && (!x_bf16 || !w_e4m3 || !w_s || !y_bf16))
    return set_error(WZ_EINVAL, "fp8_linear: null pointer");
  return launch_skinny<kFmtFp8, true>(x_bf16, nullptr, act_scale_kind, w_e4m3, w_s, w_scale_kind,
                                      y_bf16, M, N, K, stream, "fp8_linear");
}

extern "C" int wz_fp4_gemm(const void* a_e4m3, const void* a_s, const void* w_fp4x2,
                           const void* w_s_e8m0, void* c_bf16, int64_t M, int64_t N, int64_t K,
                           int act_scale_kind, hipStream_t stream) {
  using namespace wz;
  if (int rc = check_dims("fp4_gemm", M, N, K)) return rc;
  if (act_scale_kind < 0 || act_scale_kind > 2)
    return set_error(WZ_EINVAL, "fp4_gemm: bad scale kind %d", act_scale_kind);
  if (M && (!a_e4m3 || !a_s || !w_fp4x2 || !w_s_e8m0 || !c_bf16))
    return set_error(WZ_EINVAL, "fp4_gemm: null pointer");
  return launch_skinny<kFmtFp4, false>(a_e4m3, a_s, act_scale_kind, w_fp4x2, w_s_e8m0,
                                       WZ_WSCALE_E8M0, c_bf16, M, N, K, stream, "fp4_gemm");
}

extern "C" int wz_grouped_fp4_gemm(const void* a_e4m3, const void* a_s, const void* w_fp4x2,
                                   const void* w_s_e8m0, void* c_bf16, int64_t G, int64_t N, int64_t K,
                                   int act_scale_kind, hipStream_t stream) {
  using namespace wz;
  if (int rc = check_dims("grouped_fp4_gemm", G, N, K)) return rc;
  if (G > 65535) return set_error(WZ_EINVAL, "grouped_fp4_gemm: G=%lld rows exceed 65535", (long long)G);
  if (act_scale_kind < 0 || act_scale_kind > 2)
    return set_error(WZ_EINVAL, "grouped_fp4_gemm: bad scale kind %d", act_scale_kind);
  if (G == 0) return WZ_OK;
  if (!a_e4m3 || !a_s || !w_fp4x2 || !w_s_e8m0 || !c_bf16)
    return set_error(WZ_EINVAL, "grouped_fp4_gemm: null pointer");
  const dim3 grid(unsigned(N / 16), unsigned(G));
  const uint8_t* a = static_cast<const uint8_t*>(a_e4m3);
  const uint8_t* w = static_cast<const uint8_t*>(w_fp4x2);
  const uint8_t* ws = static_cast<const uint8_t*>(w_s_e8m0);
  uint16_t* c = static_cast<uint16_t*>(c_bf16);
  const int u = skinny_unroll(K);
  if (u == 8) {
    WZ_LAUNCH("grouped_fp4_gemm", stream, grouped_fp4_kernel<8>, grid, dim3(kGemmThreads), 0, a, a_s, act_scale_kind,
              w, ws, c, int(N), int(K));
  } else if (u == 4) {
    WZ_LAUNCH("grouped_fp4_gemm", stream, grouped_fp4_kernel<4>, grid, dim3(kGemmThreads), 0, a, a_s, act_scale_kind,
              w, ws, c, int(N), int(K));
  } else {
    WZ_LAUNCH("grouped_fp4_gemm", stream, grouped_fp4_kernel<2>, grid, dim3(kGemmThreads), 0, a, a_s, act_scale_kind,
              w, ws, c, int(N), int(K));
  }
  return check_launch("grouped_fp4_gemm");
}
