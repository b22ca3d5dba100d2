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
// M <= 16, K in {1024, 2048, 4096, 8192}: fp8_gemv_kernel.  Persistent
//   workgroups of W waves; wave w owns K-blocks [w NKB, (w+1) NKB) of every
//   16-column tile.  The wave quantises its slice of x once (act_quant fused
//   into the A operand) and keeps it in registers, then the workgroup streams
//   tiles b, b+G, ... through a ring of NB register buffers, so NB tiles'
//   weights are in flight during the current tile's MFMAs; the W K-partials
//   meet in LDS, summed in wave order.
// Otherwise: act_quant into the caller's workspace, then the dense tile GEMM
//   (launch_dense_fp8: M-tiles of <= 64 rows staged in LDS).
#include "mfma_ops.h"

#include <algorithm>

namespace wz {

int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream);
int launch_pack_fp8(const void* w, int64_t N, int64_t K, void* dst, hipStream_t stream);
int launch_dense_fp8(const uint8_t* wp, const void* w_s, int w_kind, const uint8_t* xq, const float* xs,
                     bool a_pow2, uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream);
int launch_dense_fp4(const uint8_t* wp, const uint32_t* wp_s, const uint8_t* xq, const float* xs, bool a_pow2,
                     uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream);
bool tile_gemm_fits(int64_t M, int64_t N, int64_t K);
int launch_tile_gemm(const uint8_t* xq, const float* xs, bool a_pow2, const uint8_t* wp, const void* w_s, int w_kind,
                     const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                     int64_t K, hipStream_t stream);

constexpr int kGvMaxM = 32;

// GEMV shapes: W waves per workgroup, wave w owns K-blocks [w NKB, (w+1) NKB)
// of every 16-column tile, NB tiles in flight per workgroup (a ring of
// register buffers).  K = 128 W NKB.  Each shape keeps about 256 KB of
// weights in flight per CU at the occupancy its registers allow (the layout
// of the MoE w1/w3 stream: few waves, long per-lane K runs).
// (W, NKB, NB, minimum waves per SIMD, XF) per K, the fastest of a sweep of
// 4-, 8- and 16-wave shapes at the V4 and cfg-3 projection widths (T = 1, 8):
// at K >= 4096 sixteen waves halve each wave's share of the fused act_quant,
// which sits in front of the first weight request; at K = 1024 the weight
// requests go out before it.
#ifndef WZ_GV_K1024
#define WZ_GV_K1024 8, 1, 4, 4, true
#endif
#ifndef WZ_GV_K2048
#define WZ_GV_K2048 8, 2, 3, 3, false
#endif
#ifndef WZ_GV_K4096
#define WZ_GV_K4096 16, 2, 2, 4, false
#endif
#ifndef WZ_GV_K8192
#define WZ_GV_K8192 16, 4, 1, 4, false
#endif

static bool gemv_shape_ok(int64_t K) { return K == 1024 || K == 2048 || K == 4096 || K == 8192; }

static bool gemv_serves(bool qa, int64_t M, int64_t N, int64_t K);
static bool gemv_wt_serves(bool norm, int64_t M, int64_t N, int64_t K);
static int gemv_nkb(int64_t K);

// K-blocks per slice of the summation order every FP8 linear path shares (the
// tile GEMM follows it): the K range one GEMV wave owns, or the whole K where
// no GEMV serves it.
int gemv_slice_blocks(int64_t K) { return gemv_shape_ok(K) ? gemv_nkb(K) : int(K / 128); }

// Pre-quantised rows on the M-tiled one-tile GEMV: up to 32 rows where the
// tiles fit the one-tile kernel's range; wider rows and wider N on the tile
// GEMM.
static bool gemv_mt_serves(int64_t M, int64_t N, int64_t K);

template <int NKB>
struct GvBuf {
  v8i w[NKB];
  int se[NKB];
  float sf[NKB];
};

// QA: x is pre-quantised e4m3 [M, K] with block scales xs [M, K/128] of kind
// a_kind (fp8_gemm's a, a_s); otherwise x is bf16 and act_quant is fused.
// RT row tiles of 16 (M <= 16 RT): each weight tile feeds RT MFMAs per K-block.
// Workgroup b takes tiles b, b + G, ... (n_my of them); tile j sits in ring
// slot j % NB, and slot s is refilled with tile j + NB as soon as tile j's
// MFMAs have issued, so NB tiles stay in flight.  The W K-partials of a tile
// meet in LDS and are summed in wave order.  AP2 / BP2: power-of-two
// activation / e8m0 weight scales (compile-time, so the scaled MFMA chains
// without a runtime branch around it).
template <int W, int NKB, int NB, int MINW, bool XF, bool QA, bool AP2, bool BP2, int RT>
__global__ __launch_bounds__(W * 64, MINW) void fp8_gemv_kernel(const void* __restrict__ x, const void* __restrict__ xs,
                                                         int a_kind, const uint8_t* __restrict__ wp,
                                                         const void* __restrict__ w_s, int w_kind,
                                                         const uint16_t* __restrict__ res, uint16_t* __restrict__ y,
                                                         uint16_t* __restrict__ y_hi, int n_split, int M, int N,
                                                         int K, int a_pow2i) {
  __shared__ float red[2][W * 4 * kWave];
  // the wave index is uniform: tile addresses and weight scales stay scalar
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  constexpr bool a_pow2 = AP2, bp = BP2;
  constexpr int wkind = BP2 ? WZ_WSCALE_E8M0 : WZ_WSCALE_F32;
  const int KB = K / 128, kb0 = wave * NKB, items = N / 16, G = gridDim.x;
  const int first = blockIdx.x;
  if (first >= items) return;
  const int n_my = (items - first + G - 1) / G;

  auto fetch = [&](GvBuf<NKB>& b, int j) {
    const int item = first + j * G;
    const uint8_t* t = wp + (int64_t(item) * KB + kb0) * 2048 + lane * 16;
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const v4i lo = load16_nt(t + q * 2048), hi = load16_nt(t + q * 2048 + 1024);
      b.w[q] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int q = 0; q < NKB; ++q) fp8_wscale(w_s, int64_t(item >> 3) * KB + kb0 + q, wkind, b.se[q], b.sf[q]);
  };

  // this wave's K slice of the (<= 16 RT) token rows, quantised once.  XF: the
  // bf16 rows are requested, then the first tile's weights, and the
  // quantisation runs while those are in flight (the x loads, issued first,
  // return first); otherwise the rows are quantised before any weight request.
  AOp a[RT][NKB];
  ARaw xr[RT][QA || !XF ? 1 : NKB];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    const int r = rt * 16 + nl;
    if constexpr (QA) {
      const uint8_t* xrow = r < M ? static_cast<const uint8_t*>(x) + int64_t(r) * K : nullptr;
      const void* srow = a_kind == WZ_SCALE_UE8M0
                             ? static_cast<const void*>(static_cast<const uint8_t*>(xs) + int64_t(r) * KB)
                             : static_cast<const void*>(static_cast<const float*>(xs) + int64_t(r) * KB);
#pragma unroll
      for (int q = 0; q < NKB; ++q) a[rt][q] = a_from_fp8(xrow, srow, kb0 + q, g, a_kind);
    } else {
      const uint16_t* xrow = r < M ? static_cast<const uint16_t*>(x) + int64_t(r) * K : nullptr;
#pragma unroll
      for (int q = 0; q < NKB; ++q) {
        if constexpr (XF)
          xr[rt][q] = a_load_bf16(xrow, kb0 + q, g);
        else
          a[rt][q] = a_from_bf16(xrow, kb0 + q, g, AP2);
      }
    }
  }
  auto quant_x = [&]() {
    if constexpr (!QA && XF) {
#pragma unroll
      for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int q = 0; q < NKB; ++q) a[rt][q] = a_quant_bf16(xr[rt][q], AP2);
    }
  };
  // keeps the weight requests below the quantisation: hoisted above it, they
  // would hold their registers beside the raw rows' and spill
  if constexpr (!QA && !XF) __builtin_amdgcn_sched_barrier(0);

  auto process = [&](const GvBuf<NKB>& b, int j) {
    const int item = first + j * G;
    v4f acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      acc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < NKB; ++q)
        mma_step<kFmtFp8, kFmtFp8>(acc[rt], a[rt][q], b.w[q], b.se[q], b.sf[q], a_pow2, bp, lane);
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      // rounds alternate between the two buffers: a round's writes follow the
      // barrier that wave 0 passes only after reading the previous round
      float* r = red[(j * RT + rt) & 1];
#pragma unroll
      for (int i = 0; i < 4; ++i) r[(wave * 4 + i) * kWave + lane] = acc[rt][i];
      __syncthreads();
      if (wave == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = r[i * kWave + lane];
#pragma unroll
          for (int w = 1; w < W; ++w) v += r[(w * 4 + i) * kWave + lane];
          const int row = rt * 16 + g * 4 + i;
          const int col = item * 16 + nl;
          if (row < M && col < n_split) {
            const int64_t o = int64_t(row) * n_split + col;
            // res: the residual stream, y = x + linear(..): the product rounded
            // to bf16, then the fp32 sum rounded once (a bf16 tensor add)
            y[o] = f32_to_bf16(res ? bf16_round(v) + __uint_as_float(uint32_t(res[o]) << 16) : v);
          } else if (row < M) {
            // columns past n_split: the second of two stacked weights, its own buffer
            y_hi[int64_t(row) * (N - n_split) + (col - n_split)] = f32_to_bf16(v);
          }
        }
      }
    }
  };

  GvBuf<NKB> buf[NB];
  fetch(buf[0], 0);
  quant_x();
  if (n_my < NB) {
    // fewer tiles than ring slots: all of them in flight at once
#pragma unroll
    for (int s = 1; s < NB - 1; ++s)
      if (s < n_my) fetch(buf[s], s);
#pragma unroll
    for (int s = 0; s < NB - 1; ++s)
      if (s < n_my) process(buf[s], s);
    return;
  }
#pragma unroll
  for (int s = 1; s < NB; ++s) fetch(buf[s], s);
  int j = 0;
  // steady state: every refill is a tile of this workgroup
  for (; j + 2 * NB <= n_my; j += NB) {
#pragma unroll
    for (int s = 0; s < NB; ++s) {
      process(buf[s], j + s);
      __builtin_amdgcn_sched_barrier(0);
      fetch(buf[s], j + s + NB);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the last NB .. 2 NB - 1 tiles
#pragma unroll
  for (int s = 0; s < NB; ++s) {
    process(buf[s], j + s);
    if (j + s + NB < n_my) fetch(buf[s], j + s + NB);
  }
#pragma unroll
  for (int s = 0; s < NB; ++s)
    if (j + NB + s < n_my) process(buf[s], j + NB + s);
}

// One 16-column tile per workgroup (grid = N / 16), its K split over W waves
// of NKB K-blocks: the shapes whose tiles fit the chip in about one wave of
// workgroups, where each workgroup's weight share is a single burst and the
// launch is one round trip.  Every load goes out before the first wait: the
// x rows, then the wave's weight K-blocks and their scales; vmcnt counts in
// issue order, so the x rows are waited for while the weights are still in
// flight.
//   QA: x is e4m3 with block scales; each lane loads its A fragments.
//   else: x is bf16 and act_quant runs once per workgroup, densely: sixteen
//   lanes per (row, 128-block) pair, eight elements each, rows < M only
//   (pair 4 (w + j W) + lane / 16 in pass j of wave w, XP passes at most),
//   into LDS as e4m3 rows padded by 16 bytes, which the MFMA A fragments are
//   then read from.  The MFMA lane layout would have every wave quantise all
//   16 row slots of its K-slice, at T = 4 three quarters of them empty.
// The same block amax, scale and rounding as act_quant, and the ring kernel's
// K split, so both kernels give the same bits.  Four waves sum the W
// K-partials of the 16 x 16 tile in wave order.
//   NORM: x is the bf16 input of RMSNorm (fp32 weight nw [K], eps), first the
//   residual step x + xb when xb is given (written to hsum by workgroup 0);
//   the norm output is quantised into LDS as above.  Row r is taken by NWR
//   waves whose thread t = 64 nw + lane holds chunks t + 256 j: the mapping,
//   sequential sum of squares, xor butterfly and partial order of
//   rmsnorm_quant_kernel, so the codes are that kernel's bit for bit.
template <int W, int NKB>
struct GvNorm {
  static constexpr int NJ = (W * NKB + 15) / 16;                               // chunks per thread
  static constexpr int NWR = (W * NKB + 3) / 4 < 4 ? (W * NKB + 3) / 4 : 4;  // waves per row
  static constexpr int ROWS = W / NWR;                                          // rows per launch
};

template <int W, int NKB, int XP, bool QA, bool AP2, bool BP2, bool NORM, int RT>
__global__ __launch_bounds__(W * 64) void fp8_gemv1_kernel(const void* __restrict__ x, const void* __restrict__ xs,
                                                           int a_kind, const uint8_t* __restrict__ wp,
                                                           const void* __restrict__ w_s,
                                                           const uint16_t* __restrict__ res, uint16_t* __restrict__ y,
                                                           uint16_t* __restrict__ y_hi, int n_split, int M, int N,
                                                           int K, const float* __restrict__ nw, float eps,
                                                           const uint16_t* __restrict__ xb,
                                                           uint16_t* __restrict__ hsum, int n_mt) {
  static_assert(W >= 4, "the epilogue uses four waves");
  static_assert(!(NORM && QA), "the norm path starts from bf16 rows");
  static_assert(!(NORM && RT > 1), "the norm path serves up to 16 rows");
  static_assert(QA || RT <= 2, "the bf16 paths serve up to 32 rows");
  using NP = GvNorm<W, NKB>;
  __shared__ float part[NORM ? NP::ROWS : 1][4];
  // !QA: e4m3 rows [M][K + 16], then (e8m0, scale) per pair; afterwards (and
  // always with QA) the W K-partials of the RT 16 x 16 tiles, [RT][W][4][64]
  extern __shared__ __align__(16) uint8_t gv_lds[];
  float* red = reinterpret_cast<float*>(gv_lds);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int KB = K / 128, kb0 = wave * NKB;
  // QA with n_mt > 1: workgroup b takes (tile, M-tile of 16 RT rows) t =
  // xcd_runs(b), so the M-tiles of one weight tile run on one XCD together and
  // read its tiles from that L2; otherwise tile b over rows 0 ..
  int item = blockIdx.x, m0 = 0;
  if (QA && n_mt > 1) {
    const int t = xcd_runs(int(blockIdx.x), 0, (N / 16) * n_mt);
    item = t / n_mt;
    m0 = (t - item * n_mt) * 16 * RT;
  }
  const int ldk = K + 16;

  AOp a[RT][NKB];
  uint4 xr[QA || NORM ? 1 : XP];
  v4i nv[NORM ? NP::NJ : 1], nbv[NORM ? NP::NJ : 1], nwv[NORM ? NP::NJ : 1][2];
  const int P = M * KB;
  if constexpr (QA) {
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      const int r = m0 + rt * 16 + nl, xrow = r < M ? r : M - 1;  // rows past M repeat row M - 1; dropped
      const uint8_t* row = static_cast<const uint8_t*>(x) + int64_t(xrow) * K;
      const void* srow = a_kind == WZ_SCALE_UE8M0
                             ? static_cast<const void*>(static_cast<const uint8_t*>(xs) + int64_t(xrow) * KB)
                             : static_cast<const void*>(static_cast<const float*>(xs) + int64_t(xrow) * KB);
#pragma unroll
      for (int q = 0; q < NKB; ++q) a[rt][q] = a_from_fp8_row(row, srow, kb0 + q, g, a_kind);
    }
  } else if constexpr (NORM) {
    const int nr = wave / NP::NWR, rr = nr < M ? nr : M - 1, t = (wave % NP::NWR) * 64 + lane;
#pragma unroll
    for (int j = 0; j < NP::NJ; ++j) {
      const int64_t o = int64_t(rr) * K + (t + 256 * j) * 8;
      nv[j] = load16(static_cast<const uint16_t*>(x) + o);
      nbv[j] = load16((xb ? xb : static_cast<const uint16_t*>(x)) + o);  // unconditional: see below
      nwv[j][0] = load16(nw + (t + 256 * j) * 8);
      nwv[j][1] = load16(nw + (t + 256 * j) * 8 + 4);
    }
  } else {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      int pr = 4 * (wave + j * W) + g;
      pr = pr < P ? pr : P - 1;
      const int r = pr / KB, kb = pr - r * KB;
      xr[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + int64_t(r) * K + kb * 128 + nl * 8);
    }
  }
  // the residual of this wave's first epilogue element, requested with the x
  // rows: read in the epilogue it was a round trip after the reduction.  The
  // load has no branch around it (clamped indices; without a residual it reads
  // y's same element, unused): behind one, its use was moved into the branch
  // and waited for every x load there, before the weights were requested
  uint16_t res0;
  {
    const int row = min(m0 + ((wave >> 2) % RT) * 16 + g * 4 + (wave & 3), M - 1);
    const int col = min(item * 16 + nl, n_split - 1);
    res0 = (res ? res : y)[int64_t(row) * n_split + col];
  }
  __builtin_amdgcn_sched_barrier(0);

  v8i w[NKB];
  int se[NKB];
  float sf[NKB];
  const uint8_t* t = wp + (int64_t(item) * KB + kb0) * 2048 + lane * 16;
#pragma unroll
  for (int q = 0; q < NKB; ++q) {
    const v4i lo = load16_nt(t + q * 2048), hi = load16_nt(t + q * 2048 + 1024);
    w[q] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
#pragma unroll
  for (int q = 0; q < NKB; ++q)
    fp8_wscale(w_s, int64_t(item >> 3) * KB + kb0 + q, BP2 ? WZ_WSCALE_E8M0 : WZ_WSCALE_F32, se[q], sf[q]);
  __builtin_amdgcn_sched_barrier(0);

  if constexpr (NORM) {
    uint8_t* xq = gv_lds;
    int2* xsc = reinterpret_cast<int2*>(gv_lds + M * ldk);
    const int nr = wave / NP::NWR, nwi = wave % NP::NWR, t = nwi * 64 + lane;
    // the addend's loads stay ahead of the weight loads: used only under the
    // branch below, they would otherwise be sunk into it, behind the weights
#pragma unroll
    for (int j = 0; j < NP::NJ; ++j) asm volatile("" ::"v"(nbv[j]));
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NP::NJ; ++j) {
      if (xb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16lo(uint32_t(nv[j][i])) + bf16lo(uint32_t(nbv[j][i]));
          const float hi = bf16hi(uint32_t(nv[j][i])) + bf16hi(uint32_t(nbv[j][i]));
          nv[j][i] = int(f32x2_to_bf16x2(lo, hi));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0 = bf16lo(uint32_t(nv[j][i])), b0 = bf16hi(uint32_t(nv[j][i]));
        ss += a0 * a0;
        ss += b0 * b0;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
    if (lane == 0) part[nr][nwi] = ss;
    __syncthreads();
    {
      const float* pp = part[nr];
      const float p2 = NP::NWR > 2 ? pp[2] : 0.0f, p3 = NP::NWR > 3 ? pp[3] : 0.0f;
      const float var = ((pp[0] + pp[1]) + (p2 + p3)) / float(K);
      const float rs = 1.0f / sqrtf(var + eps);
#pragma unroll
      for (int j = 0; j < NP::NJ; ++j) {
        const int c = t + 256 * j;
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float w0 = __int_as_float(nwv[j][i >> 1][(i & 1) * 2]);
          const float w1 = __int_as_float(nwv[j][i >> 1][(i & 1) * 2 + 1]);
          f[2 * i] = bf16_round(w0 * (bf16lo(uint32_t(nv[j][i])) * rs));
          f[2 * i + 1] = bf16_round(w1 * (bf16hi(uint32_t(nv[j][i])) * rs));
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = absmax(amax, f[i]);
        amax = row16_absmax(amax);
        const ActScale sc = act_scale(amax, AP2);
        const uint2 qv = quant8(f, sc, AP2, quant_fast(amax, AP2));
        const uint32_t q0 = qv.x, q1 = qv.y;
        if (nr < M) {
          *reinterpret_cast<uint2*>(xq + nr * ldk + c * 8) = make_uint2(q0, q1);
          if ((lane & 15) == 0) xsc[nr * KB + c / 16] = make_int2(AP2 ? sc.e8m0 : kE8m0One, __float_as_int(sc.s));
        }
      }
    }
  }
  if constexpr (NORM || !QA) {
    uint8_t* xq = gv_lds;
    int2* xsc = reinterpret_cast<int2*>(gv_lds + M * ldk);
    if constexpr (!NORM) {
    // each lane's amax of its eight elements, for every pass: the x loads
    // are used here, ahead of the passes' branches, so none of them is sunk
    // into a branch behind the weight loads (its wait would drain those)
    float lmax[XP];
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const float m = bf16x8_absmax(v4i{int(xr[j].x), int(xr[j].y), int(xr[j].z), int(xr[j].w)});
      asm volatile("" ::"v"(m));  // an unconditional use: the load stays here
      lmax[j] = m;
    }
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int pr = 4 * (wave + j * W) + g;
      if (4 * (wave + j * W) < P) {  // wave-uniform: the pass holds a pair
        const float amax = row16_absmax(lmax[j]);
        const ActScale sc = act_scale(amax, AP2);
        float f[8];
        bf16x8_unpack(v4i{int(xr[j].x), int(xr[j].y), int(xr[j].z), int(xr[j].w)}, f);
        const uint2 qv = quant8(f, sc, AP2, quant_fast(amax, AP2));
        const uint32_t q0 = qv.x, q1 = qv.y;
        if (pr < P) {
          const int r = pr / KB, kb = pr - r * KB;
          *reinterpret_cast<uint2*>(xq + r * ldk + kb * 128 + nl * 8) = make_uint2(q0, q1);
          if (nl == 0) xsc[pr] = make_int2(AP2 ? sc.e8m0 : kE8m0One, __float_as_int(sc.s));
        }
      }
    }
    }
    __syncthreads();
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
      for (int q = 0; q < NKB; ++q) {
        const int r = rt * 16 + nl;
        a[rt][q] = a_zero();
        if (r < M) {
          const uint8_t* pa = xq + r * ldk + (kb0 + q) * 128 + g * 16;
          const uint4 lo = *reinterpret_cast<const uint4*>(pa), hi = *reinterpret_cast<const uint4*>(pa + 64);
          a[rt][q].v = v8i{int(lo.x), int(lo.y), int(lo.z), int(lo.w), int(hi.x), int(hi.y), int(hi.z), int(hi.w)};
          const int2 s2 = xsc[r * KB + kb0 + q];
          a[rt][q].se8 = s2.x;
          a[rt][q].sf = __int_as_float(s2.y);
        }
      }
  }
  v4f acc[RT];
#pragma unroll
  for (int rt = 0; rt < RT; ++rt) {
    acc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < NKB; ++q) mma_step<kFmtFp8, kFmtFp8>(acc[rt], a[rt][q], w[q], se[q], sf[q], AP2, BP2, lane);
  }
  // the partials go where the x rows were: every wave has its A fragments
  if constexpr (NORM || !QA) __syncthreads();
#pragma unroll
  for (int rt = 0; rt < RT; ++rt)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((rt * W + wave) * 4 + i) * kWave + lane] = acc[rt][i];
  __syncthreads();
  // (row tile, row of the four a lane holds) pairs, one per wave: wave order sums
  for (int pi = wave; pi < 4 * RT; pi += W) {
    const int rt = pi >> 2, i = pi & 3, row = m0 + rt * 16 + g * 4 + i;
    const float* rr = red + rt * W * 4 * kWave;
    if (row < M) {
      float v = rr[i * kWave + lane];
#pragma unroll
      for (int ww = 1; ww < W; ++ww) v += rr[(ww * 4 + i) * kWave + lane];
      const int col = item * 16 + nl;
      if (col < n_split) {
        const int64_t o = int64_t(row) * n_split + col;
        const uint16_t rv = res ? (pi == wave ? res0 : res[o]) : 0;
        y[o] = f32_to_bf16(res ? bf16_round(v) + __uint_as_float(uint32_t(rv) << 16) : v);
      } else {
        y_hi[int64_t(row) * (N - n_split) + (col - n_split)] = f32_to_bf16(v);
      }
    }
  }
  if constexpr (NORM) {
    // the residual step's sum, by workgroup 0, last: stores count in vmcnt, so
    // issued earlier they would make the quantisation's waits cover the weights
    const int nr = wave / NP::NWR, t = (wave % NP::NWR) * 64 + lane;
    if (xb && hsum && blockIdx.x == 0 && nr < M) {
#pragma unroll
      for (int j = 0; j < NP::NJ; ++j) *reinterpret_cast<v4i*>(hsum + int64_t(nr) * K + (t + 256 * j) * 8) = nv[j];
    }
  }
}

// Wave-tile GEMV, K = 128 KB (compile time), M <= 16 RT: one 16-column tile per
// WAVE over the whole K, W tiles per workgroup (RT row tiles of 16: each
// weight K-block feeds RT MFMAs; the norm path serves one).  The workgroup quantises the
// x rows into LDS once for its W tiles, exactly as fp8_gemv1_kernel does (the
// dense bf16 passes, or with NORM the RMSNorm of x (+ b) in
// rmsnorm_quant_kernel's thread mapping), and no partial crosses waves: a wave
// computes the K slices of SL K-blocks (the K range one wave of the split
// kernels owns) each from zero and folds them in K order, which is the split
// kernels' wave-order sum, so every output has their bits.  Each wave requests
// its tile's weights before the prologue.  Where a tile holds few bytes (K =
// 1024: 16 KB) the split kernels spend a prologue and a cross-wave sum with a
// barrier on every tile; here one prologue serves W tiles and the steady state
// has no barrier.
template <int W, int KB, int SL, int XP, bool AP2, bool BP2, bool NORM, int RT>
__global__ __launch_bounds__(W * 64, RT > 1 ? 2 : 3) void fp8_gemv_wt_kernel(const void* __restrict__ x,
                                                             const uint8_t* __restrict__ wp,
                                                             const void* __restrict__ w_s,
                                                             const uint16_t* __restrict__ res,
                                                             uint16_t* __restrict__ y, uint16_t* __restrict__ y_hi,
                                                             int n_split, int M, int N, const float* __restrict__ nw,
                                                             float eps, const uint16_t* __restrict__ xb,
                                                             uint16_t* __restrict__ hsum) {
  static_assert(KB % SL == 0, "the slices cover K");
  static_assert(!(NORM && RT > 1), "the norm path serves up to 16 rows");
  constexpr int K = KB * 128, ldk = K + 16;
  // the norm's thread mapping: NWR waves (64 NWR threads) per row, thread t
  // holding the 8-element chunks t + 256 j (GvNorm's, with W NKB = KB)
  constexpr int NJ = (KB + 15) / 16, NWR = (KB + 3) / 4 < 4 ? (KB + 3) / 4 : 4, NROWS = W / NWR;
  __shared__ float part[NORM ? NROWS : 1][4];
  extern __shared__ __align__(16) uint8_t gv_lds[];
  uint8_t* xq = gv_lds;
  int2* xsc = reinterpret_cast<int2*>(gv_lds + M * ldk);
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int tiles = N / 16, item = int(blockIdx.x) * W + wave, it = item < tiles ? item : tiles - 1;
  const int P = M * KB;

  // ---- x: the loads of the prologue (fp8_gemv1_kernel's) ----
  uint4 xr[NORM ? 1 : XP];
  v4i nv[NORM ? NJ : 1], nbv[NORM ? NJ : 1], nwv[NORM ? NJ : 1][2];
  if constexpr (NORM) {
    const int nr = wave / NWR, rr = nr < M ? nr : M - 1, t = (wave % NWR) * 64 + lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t o = int64_t(rr) * K + (t + 256 * j) * 8;
      nv[j] = load16(static_cast<const uint16_t*>(x) + o);
      nbv[j] = load16((xb ? xb : static_cast<const uint16_t*>(x)) + o);
      nwv[j][0] = load16(nw + (t + 256 * j) * 8);
      nwv[j][1] = load16(nw + (t + 256 * j) * 8 + 4);
    }
  } else {
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      int pr = 4 * (wave + j * W) + g;
      pr = pr < P ? pr : P - 1;
      const int r = pr / KB, kb = pr - r * KB;
      xr[j] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(x) + int64_t(r) * K + kb * 128 + nl * 8);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- this wave's tile: every K-block and its block scale ----
  v8i w[KB];
  int se[KB];
  float sf[KB];
  {
    const uint8_t* t = wp + int64_t(it) * KB * 2048 + lane * 16;
#pragma unroll
    for (int q = 0; q < KB; ++q) {
      const v4i lo = load16_nt(t + q * 2048), hi = load16_nt(t + q * 2048 + 1024);
      w[q] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int q = 0; q < KB; ++q)
      fp8_wscale(w_s, int64_t(it >> 3) * KB + q, BP2 ? WZ_WSCALE_E8M0 : WZ_WSCALE_F32, se[q], sf[q]);
  }
  __builtin_amdgcn_sched_barrier(0);

  // ---- the quantised rows into LDS (the arithmetic of fp8_gemv1_kernel) ----
  if constexpr (NORM) {
    const int nr = wave / NWR, nwi = wave % NWR, t = nwi * 64 + lane;
#pragma unroll
    for (int j = 0; j < NJ; ++j) asm volatile("" ::"v"(nbv[j]));
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      if (xb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float lo = bf16lo(uint32_t(nv[j][i])) + bf16lo(uint32_t(nbv[j][i]));
          const float hi = bf16hi(uint32_t(nv[j][i])) + bf16hi(uint32_t(nbv[j][i]));
          nv[j][i] = int(f32x2_to_bf16x2(lo, hi));
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a0 = bf16lo(uint32_t(nv[j][i])), b0 = bf16hi(uint32_t(nv[j][i]));
        ss += a0 * a0;
        ss += b0 * b0;
      }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
    if (lane == 0 && nr < NROWS) part[nr][nwi] = ss;
    __syncthreads();
    if (nr < NROWS) {
      const float* pp = part[nr];
      const float p2 = NWR > 2 ? pp[2] : 0.0f, p3 = NWR > 3 ? pp[3] : 0.0f;
      const float var = ((pp[0] + pp[1]) + (p2 + p3)) / float(K);
      const float rs = 1.0f / sqrtf(var + eps);
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int c = t + 256 * j;
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float w0 = __int_as_float(nwv[j][i >> 1][(i & 1) * 2]);
          const float w1 = __int_as_float(nwv[j][i >> 1][(i & 1) * 2 + 1]);
          f[2 * i] = bf16_round(w0 * (bf16lo(uint32_t(nv[j][i])) * rs));
          f[2 * i + 1] = bf16_round(w1 * (bf16hi(uint32_t(nv[j][i])) * rs));
        }
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = absmax(amax, f[i]);
        amax = row16_absmax(amax);
        const ActScale sc = act_scale(amax, AP2);
        const uint2 qv = quant8(f, sc, AP2, quant_fast(amax, AP2));
        const uint32_t q0 = qv.x, q1 = qv.y;
        if (nr < M && c < K / 8) {
          *reinterpret_cast<uint2*>(xq + nr * ldk + c * 8) = make_uint2(q0, q1);
          if ((lane & 15) == 0) xsc[nr * KB + c / 16] = make_int2(AP2 ? sc.e8m0 : kE8m0One, __float_as_int(sc.s));
        }
      }
    }
  } else {
    float lmax[XP];
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const float m = bf16x8_absmax(v4i{int(xr[j].x), int(xr[j].y), int(xr[j].z), int(xr[j].w)});
      asm volatile("" ::"v"(m));
      lmax[j] = m;
    }
#pragma unroll
    for (int j = 0; j < XP; ++j) {
      const int pr = 4 * (wave + j * W) + g;
      if (4 * (wave + j * W) < P) {
        const float amax = row16_absmax(lmax[j]);
        const ActScale sc = act_scale(amax, AP2);
        float f[8];
        bf16x8_unpack(v4i{int(xr[j].x), int(xr[j].y), int(xr[j].z), int(xr[j].w)}, f);
        const uint2 qv = quant8(f, sc, AP2, quant_fast(amax, AP2));
        const uint32_t q0 = qv.x, q1 = qv.y;
        if (pr < P) {
          const int r = pr / KB, kb = pr - r * KB;
          *reinterpret_cast<uint2*>(xq + r * ldk + kb * 128 + nl * 8) = make_uint2(q0, q1);
          if (nl == 0) xsc[pr] = make_int2(AP2 ? sc.e8m0 : kE8m0One, __float_as_int(sc.s));
        }
      }
    }
  }
  __syncthreads();

  // ---- the tile: K slices from zero, folded in K order ----
  v4f tot[RT];
#pragma unroll
  for (int s = 0; s < KB / SL; ++s) {
    v4f acc[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) acc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < SL; ++q) {
      const int kb = s * SL + q;
#pragma unroll
      for (int rt = 0; rt < RT; ++rt) {
        const int r = rt * 16 + nl;
        AOp a = a_zero();
        if (r < M) {
          const uint8_t* pa = xq + r * ldk + kb * 128 + g * 16;
          const uint4 lo = *reinterpret_cast<const uint4*>(pa), hi = *reinterpret_cast<const uint4*>(pa + 64);
          a.v = v8i{int(lo.x), int(lo.y), int(lo.z), int(lo.w), int(hi.x), int(hi.y), int(hi.z), int(hi.w)};
          const int2 s2 = xsc[r * KB + kb];
          a.se8 = s2.x;
          a.sf = __int_as_float(s2.y);
        }
        mma_step<kFmtFp8, kFmtFp8>(acc[rt], a, w[kb], se[kb], sf[kb], AP2, BP2, lane);
      }
    }
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
      if (s == 0) {
        tot[rt] = acc[rt];
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) tot[rt][i] += acc[rt][i];
      }
    }
  }
  if (item < tiles) {
#pragma unroll
    for (int ri = 0; ri < 4 * RT; ++ri) {
      const int rt = ri >> 2, i = ri & 3;
      const int row = rt * 16 + g * 4 + i;
      if (row < M) {
        const float v = tot[rt][i];
        const int col = item * 16 + nl;
        if (col < n_split) {
          const int64_t o = int64_t(row) * n_split + col;
          y[o] = f32_to_bf16(res ? bf16_round(v) + __uint_as_float(uint32_t(res[o]) << 16) : v);
        } else {
          y_hi[int64_t(row) * (N - n_split) + (col - n_split)] = f32_to_bf16(v);
        }
      }
    }
  }
  if constexpr (NORM) {
    // the residual step's sum, by workgroup 0, last (as fp8_gemv1_kernel)
    const int nr = wave / NWR, t = (wave % NWR) * 64 + lane;
    if (xb && hsum && blockIdx.x == 0 && nr < M && nr < NROWS) {
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        if (t + 256 * j < K / 8) *reinterpret_cast<v4i*>(hsum + int64_t(nr) * K + (t + 256 * j) * 8) = nv[j];
    }
  }
}

// dynamic LDS of the one-tile kernel's bf16 path: e4m3 rows + per-pair scales
static size_t gemv1_lds_bytes(int64_t M, int64_t K) { return size_t(M) * size_t(K + 16) + size_t(M) * size_t(K / 128) * 8; }
// ... and in total: that region, then the K-partials of RT row tiles in its place
static size_t gemv1_dyn_bytes(bool qa, int64_t M, int64_t K, int W, int RT) {
  const size_t red = size_t(RT) * size_t(W) * 4 * kWave * 4;
  return qa ? red : std::max(gemv1_lds_bytes(M, K), red);
}

// LDS a workgroup may hold on gfx950 (160 KB); dynamic LDS past 64 KB is
// requested per kernel once (hipFuncAttributeMaxDynamicSharedMemorySize).
constexpr size_t kLdsMax = 160 * 1024;
template <typename F>
static int allow_lds(F* kernel, size_t bytes, int& granted) {
  if (bytes <= 64 * 1024 || int(bytes) <= granted) return 0;
  if (hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                          int(bytes)) != hipSuccess)
    return set_error(WZ_ELAUNCH, "fp8 gemv: %zu bytes of LDS refused", bytes);
  granted = int(bytes);
  return 0;
}

template <int W, int NKB, int NB, int MINW, bool XF, bool QA>
static int launch_gemv(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                       uint16_t* y, int64_t M, int64_t N, int64_t K, bool pow2, hipStream_t stream);

static int gemv_dispatch(bool qa, const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s,
                         int w_kind, const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M,
                         int64_t N, int64_t K, bool pow2, hipStream_t stream);
static int gemv_mt_dispatch(const void* xq, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                            const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                            int64_t K, bool pow2, hipStream_t stream);

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

// No workspace where the GEMV serves every N (M <= 16); otherwise the act_quant
// of x for the tile GEMM (M <= 32 may still run the GEMV, depending on N).
extern "C" size_t wz_fp8_linear_workspace_bytes(int64_t M, int64_t K) {
  using namespace wz;
  if (M <= 0 || K <= 0) return 0;
  if (M <= 16 && gemv_shape_ok(K)) return 0;
  return align256(size_t(M) * size_t(K)) + size_t(M) * size_t(K / 128) * 4;
}

namespace wz {

// The residual operand of the *_add entry points: y = residual + linear(..),
// fused into the GEMV's epilogue; on the tile-GEMM path a bf16 add follows.
static int add_residual(const uint16_t* res, uint16_t* y, int64_t M, int64_t N, int rc, hipStream_t stream) {
  if (rc || !res) return rc;
  return wz_add_bf16(res, y, y, M * N, stream);
}

static int overlap(const void* a, const void* b, size_t bytes) {
  const char *pa = static_cast<const char*>(a), *pb = static_cast<const char*>(b);
  return pa < pb + bytes && pb < pa + bytes;
}

static int linear_packed(const char* name, const void* x_bf16, const void* w_packed, const void* w_s,
                         const uint16_t* res, void* y_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                         int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream) {
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp8_linear_packed: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return set_error(WZ_EINVAL, "fp8_linear_packed: dimension too large");
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
      (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
    return set_error(WZ_EINVAL, "fp8_linear_packed: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
  if (M == 0) return WZ_OK;
  if (!x_bf16 || !w_packed || !w_s || !y_bf16) return set_error(WZ_EINVAL, "%s: null pointer", name);
  if (res && overlap(res, y_bf16, size_t(M) * size_t(N) * 2))
    return set_error(WZ_EINVAL, "%s: the residual and the output overlap", name);
  const bool pow2 = act_scale_kind != WZ_SCALE_F32;
  uint16_t* y = static_cast<uint16_t*>(y_bf16);
  if (gemv_serves(false, M, N, K))
    return gemv_dispatch(false, x_bf16, nullptr, 0, static_cast<const uint8_t*>(w_packed), w_s, w_scale_kind, res, y,
                         nullptr, N, M, N, K, pow2, stream);
  const size_t need = wz_fp8_linear_workspace_bytes(M, K);
  if (!ws || ws_bytes < need)
    return set_error(WZ_ESPACE, "%s: workspace of %zu bytes needed for M=%lld K=%lld, got %zu", name, need,
                     (long long)M, (long long)K, ws_bytes);
  uint8_t* xq = static_cast<uint8_t*>(ws);
  float* xs = reinterpret_cast<float*>(xq + align256(size_t(M) * size_t(K)));
  const int qkind = pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  if (int rc = launch_act_quant(x_bf16, M, K, xq, xs, qkind, stream)) return rc;
  const uint8_t* wp = static_cast<const uint8_t*>(w_packed);
  if (gemv_mt_serves(M, N, K))
    return gemv_mt_dispatch(xq, xs, qkind, wp, w_s, w_scale_kind, res, y, nullptr, N, M, N, K, pow2, stream);
  if (tile_gemm_fits(M, N, K))
    return launch_tile_gemm(xq, xs, pow2, wp, w_s, w_scale_kind, res, y, nullptr, N, M, N, K, stream);
  return add_residual(res, y, M, N, launch_dense_fp8(wp, w_s, w_scale_kind, xq, xs, pow2, y, M, N, K, stream),
                      stream);
}

}  // namespace wz

extern "C" int wz_fp8_linear_packed(const void* x_bf16, const void* w_packed, const void* w_s, void* y_bf16,
                                    int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                                    void* ws, size_t ws_bytes, hipStream_t stream) {
  return wz::linear_packed("fp8_linear_packed", x_bf16, w_packed, w_s, nullptr, y_bf16, M, N, K, act_scale_kind,
                           w_scale_kind, ws, ws_bytes, stream);
}

extern "C" int wz_fp8_linear_packed_add(const void* x_bf16, const void* w_packed, const void* w_s,
                                        const void* residual_bf16, void* y_bf16, int64_t M, int64_t N, int64_t K,
                                        int act_scale_kind, int w_scale_kind, void* ws, size_t ws_bytes,
                                        hipStream_t stream) {
  if (!residual_bf16) return wz::set_error(WZ_EINVAL, "fp8_linear_packed_add: null residual");
  return wz::linear_packed("fp8_linear_packed_add", x_bf16, w_packed, w_s,
                           static_cast<const uint16_t*>(residual_bf16), y_bf16, M, N, K, act_scale_kind,
                           w_scale_kind, ws, ws_bytes, stream);
}

namespace wz {

__global__ void e8m0_to_f32_kernel(const uint8_t* __restrict__ src, float* __restrict__ dst, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) dst[i] = e8m0_to_f32(src[i]);
}

// Resident workgroups per CU of one GEMV instantiation (its registers and
// LDS decide), asked once.  The grid is that many per CU, or one per tile.
template <int W, int NKB, int NB, int MINW, bool XF, bool QA, bool AP2, bool BP2, int RT>
static int launch_gemv_k(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                         const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                         int64_t K, hipStream_t stream) {
  static const int per_cu = [] {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fp8_gemv_kernel<W, NKB, NB, MINW, XF, QA, AP2, BP2, RT>,
                                                     W * 64, 0) != hipSuccess ||
        n < 1)
      n = 1;
    return n;
  }();
  const dim3 grid(unsigned(std::min<int64_t>(N / 16, int64_t(per_cu) * cu_count())));
  WZ_LAUNCH("fp8_gemv", stream, (fp8_gemv_kernel<W, NKB, NB, MINW, XF, QA, AP2, BP2, RT>), grid, dim3(W * 64), 0, x,
            xs, a_kind, w, w_s, w_kind, res, y, y_hi, int(n_split), int(M), int(N), int(K), AP2 ? 1 : 0);
  return check_launch("fp8_gemv");
}

template <int W, int NKB, int NB, int MINW, bool XF, bool QA, int RT>
static int launch_gemv_rt(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                          const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                          int64_t K, bool pow2, hipStream_t stream) {
  const bool bp = w_kind == WZ_WSCALE_E8M0;
#define WZ_GVK(AP, BP) \
  launch_gemv_k<W, NKB, NB, MINW, XF, QA, AP, BP, RT>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, stream)
  if (pow2) return bp ? WZ_GVK(true, true) : WZ_GVK(true, false);
  return bp ? WZ_GVK(false, true) : WZ_GVK(false, false);
#undef WZ_GVK
}

// M <= 16 (one row tile): a second row tile's x slice and the ring do not
// fit the registers of sixteen waves, so wider M goes to the tile GEMM
template <int W, int NKB, int NB, int MINW, bool XF, bool QA>
static int launch_gemv(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                       const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                       int64_t K, bool pow2, hipStream_t stream) {
  return launch_gemv_rt<W, NKB, NB, MINW, XF, QA, 1>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K,
                                                      pow2, stream);
}

template <int W, int NKB, int XP, bool QA, int RT>
static int launch_gemv1_rt(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                           const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                           int64_t K, bool pow2, hipStream_t stream) {
  const dim3 grid(unsigned(N / 16)), block(W * 64);
  const bool bp = w_kind == WZ_WSCALE_E8M0;
  const size_t lds = gemv1_dyn_bytes(QA, M, K, W, RT);
#define WZ_GV1(AP, BP)                                                                                        \
  do {                                                                                                          \
    static int granted = 0;                                                                                     \
    if (int rc = allow_lds(fp8_gemv1_kernel<W, NKB, XP, QA, AP, BP, false, RT>, lds, granted)) return rc;          \
    WZ_LAUNCH("fp8_gemv1", stream, (fp8_gemv1_kernel<W, NKB, XP, QA, AP, BP, false, RT>), grid, block, lds, x, xs,  \
              a_kind, w, w_s, res, y, y_hi, int(n_split), int(M), int(N), int(K), nullptr, 0.0f, nullptr, nullptr, 1); \
  } while (0)
  if (pow2) {
    if (bp) WZ_GV1(true, true); else WZ_GV1(true, false);
  } else {
    if (bp) WZ_GV1(false, true); else WZ_GV1(false, false);
  }
#undef WZ_GV1
  return check_launch("fp8_gemv1");
}

template <int W, int NKB, int XP, bool QA>
static int launch_gemv1(const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                        const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                        int64_t K, bool pow2, hipStream_t stream) {
  if (M <= 16)
    return launch_gemv1_rt<W, NKB, XP, QA, 1>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2,
                                              stream);
  return launch_gemv1_rt<W, NKB, XP, QA, 2>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2,
                                            stream);
}

// Pre-quantised rows past the GEMV's 16 on the one-tile kernel, M-tiled: a
// workgroup per (16-column tile, 16 RT rows), every load of its K range issued
// at once, the same K split and wave-order sum as the GEMV (so the same bits).
template <int W, int NKB, int RT>
static int launch_gemv_mt(const void* xq, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                          const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                          int64_t K, bool pow2, hipStream_t stream) {
  const int n_mt = int((M + 16 * RT - 1) / (16 * RT));
  const dim3 grid(unsigned((N / 16) * n_mt)), block(W * 64);
  const bool bp = w_kind == WZ_WSCALE_E8M0;
  const size_t lds = gemv1_dyn_bytes(true, M, K, W, RT);
#define WZ_GVM(AP, BP)                                                                                        \
  do {                                                                                                          \
    static int granted = 0;                                                                                     \
    if (int rc = allow_lds(fp8_gemv1_kernel<W, NKB, 1, true, AP, BP, false, RT>, lds, granted)) return rc;         \
    WZ_LAUNCH("fp8_gemv_mt", stream, (fp8_gemv1_kernel<W, NKB, 1, true, AP, BP, false, RT>), grid, block, lds, xq,   \
              xs, a_kind, w, w_s, res, y, y_hi, int(n_split), int(M), int(N), int(K), nullptr, 0.0f, nullptr,     \
              nullptr, n_mt);                                                                                   \
  } while (0)
  if (pow2) {
    if (bp) WZ_GVM(true, true); else WZ_GVM(true, false);
  } else {
    if (bp) WZ_GVM(false, true); else WZ_GVM(false, false);
  }
#undef WZ_GVM
  return check_launch("fp8_gemv_mt");
}

// GEMV shape per K for the one-tile kernel: (W, NKB) as the ring kernel's, so
// both split K the same way and give the same bits.  It serves N / 16 tiles up
// to WZ_GV1_MAX_TILES; above that the ring kernel's persistent workgroups
// (x quantised once per workgroup, several tiles streamed) are faster.
#ifndef WZ_GV1_MAX_TILES
#define WZ_GV1_MAX_TILES 512
#endif
#ifndef WZ_GV1_K1024
#define WZ_GV1_K1024 8, 1, 8
#endif
#ifndef WZ_GV1_K2048
#define WZ_GV1_K2048 8, 2, 8
#endif
#ifndef WZ_GV1_K4096
#define WZ_GV1_K4096 16, 2, 8
#endif
#ifndef WZ_GV1_K8192
#define WZ_GV1_K8192 16, 4, 8
#endif

template <int W, int NKB, int NB, int MINW, bool XF>
constexpr int ring_nkb() { return NKB; }
template <int W, int NKB, int XP>
constexpr int one_nkb() { return NKB; }
template <int W, int NKB, int XP>
constexpr int one_w() { return W; }
template <int W, int NKB, int XP>
constexpr int one_xp() { return XP; }
// the one-tile and ring kernels split K alike at every K, so they give the same bits
static_assert(ring_nkb<WZ_GV_K1024>() == one_nkb<WZ_GV1_K1024>() && ring_nkb<WZ_GV_K2048>() == one_nkb<WZ_GV1_K2048>() &&
                  ring_nkb<WZ_GV_K4096>() == one_nkb<WZ_GV1_K4096>() && ring_nkb<WZ_GV_K8192>() == one_nkb<WZ_GV1_K8192>(),
              "GEMV kernels must share the K split");

static int gemv_nkb(int64_t K) {
  switch (K) {
    case 1024: return ring_nkb<WZ_GV_K1024>();
    case 2048: return ring_nkb<WZ_GV_K2048>();
    case 4096: return ring_nkb<WZ_GV_K4096>();
    default: return ring_nkb<WZ_GV_K8192>();
  }
}

static bool gemv_mt_serves(int64_t M, int64_t N, int64_t K) {
  return gemv_shape_ok(K) && M <= kGvMaxM && N / 16 <= WZ_GV1_MAX_TILES;
}

// Whether a GEMV kernel serves (M, N, K) from x as given: every M <= 16; M <= 32
// on the one-tile kernel with two row tiles, where its tiles fit one launch and,
// for bf16 x, the quantised rows fit its passes and LDS.  The rest quantises x
// first and runs the M-tiled one-tile kernel.
static bool gemv_serves(bool qa, int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || !gemv_shape_ok(K)) return false;
  if (M <= 16) return true;
  if (!qa && gemv_wt_serves(false, M, N, K)) return true;
  if (M > kGvMaxM || N / 16 > WZ_GV1_MAX_TILES) return false;
  if (qa) return true;
  int W = 0, XP = 0;
  switch (K) {
    case 1024: W = one_w<WZ_GV1_K1024>(); XP = one_xp<WZ_GV1_K1024>(); break;
    case 2048: W = one_w<WZ_GV1_K2048>(); XP = one_xp<WZ_GV1_K2048>(); break;
    case 4096: W = one_w<WZ_GV1_K4096>(); XP = one_xp<WZ_GV1_K4096>(); break;
    default: W = one_w<WZ_GV1_K8192>(); XP = one_xp<WZ_GV1_K8192>(); break;
  }
  return M * (K / 128) <= 4 * W * XP && gemv1_dyn_bytes(false, M, K, W, 2) + 64 <= kLdsMax;
}

// Row tiles per workgroup of the M-tiled kernel at each K (registers: RT x
// NKB A fragments beside the weights).
#ifndef WZ_GVM_K1024
#define WZ_GVM_K1024 4
#endif
#ifndef WZ_GVM_K2048
#define WZ_GVM_K2048 4
#endif
#ifndef WZ_GVM_K4096
#define WZ_GVM_K4096 4
#endif
#ifndef WZ_GVM_K8192
#define WZ_GVM_K8192 2
#endif

static int gemv_mt_dispatch(const void* xq, const void* xs, int a_kind, const uint8_t* w, const void* w_s, int w_kind,
                            const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                            int64_t K, bool pow2, hipStream_t stream) {
#define WZ_MT_(W_, NKB_, XP_, RT_)                                                                          \
  return launch_gemv_mt<W_, NKB_, RT_>(xq, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, \
                                       stream)
#define WZ_MT(...) WZ_MT_(__VA_ARGS__)
  switch (K) {
    case 1024: WZ_MT(WZ_GV1_K1024, WZ_GVM_K1024);
    case 2048: WZ_MT(WZ_GV1_K2048, WZ_GVM_K2048);
    case 4096: WZ_MT(WZ_GV1_K4096, WZ_GVM_K4096);
    case 8192: WZ_MT(WZ_GV1_K8192, WZ_GVM_K8192);
    default: return set_error(WZ_EINVAL, "fp8 gemv: no shape for K=%lld", (long long)K);
  }
#undef WZ_MT
#undef WZ_MT_
}

// The wave-tile GEMV (fp8_gemv_wt_kernel) at K = 1024 from WZ_GVWT_MIN_TILES
// tiles up, where the split kernels pay a prologue and a cross-wave sum on
// every 16-KB tile; its slices are the split kernels' (one_nkb), so all give
// the same bits.  Twelve waves (three per SIMD at its ~150 registers) fill a
// CU.  32768 x 1024 (2048 tiles) T = 1 / 4 / 8: 8.4 / 10.1 / 10.4 -> 7.6 /
// 8.3 / 8.7 us; the stage's 40960-row q projection pair with its norm fused
// (2560 tiles): the decode stage 1255 -> 1211 us per step.  Below ~1000 tiles
// its few workgroups lose: 4096 x 1024 2.9 -> 5.3 us, 8192 x 1024 3.8 -> 5.5 us.
#ifndef WZ_GVWT_MIN_TILES
#define WZ_GVWT_MIN_TILES 2048
#endif
#ifndef WZ_GVWT_W
#define WZ_GVWT_W 12
#endif
constexpr int kWtW = WZ_GVWT_W;
// rows of the fused norm: two waves per row at K = 1024, and no more than the
// split kernel serves (wz_fp8_norm_linear_max_rows), so every N has one limit
constexpr int kWtNormRows = kWtW / 2 < GvNorm<one_w<WZ_GV1_K1024>(), one_nkb<WZ_GV1_K1024>()>::ROWS
                                ? kWtW / 2
                                : GvNorm<one_w<WZ_GV1_K1024>(), one_nkb<WZ_GV1_K1024>()>::ROWS;

static bool gemv_wt_serves(bool norm, int64_t M, int64_t N, int64_t K) {
  return K == 1024 && M >= 1 && M <= (norm ? kWtNormRows : 32) && N / 16 >= WZ_GVWT_MIN_TILES;
}

template <bool NORM>
static int launch_gemv_wt(const void* x, const uint16_t* b, const float* nw, float eps, uint16_t* hsum,
                          const uint8_t* w, const void* w_s, int w_kind, const uint16_t* res, uint16_t* y,
                          uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N, bool pow2, hipStream_t stream) {
  constexpr int W = kWtW, KB = 8, SL = one_nkb<WZ_GV1_K1024>();
  // rows 17..32: two row tiles on eight waves (two per SIMD: the second row
  // tile's fragments and sums did not fit the registers of three)
  constexpr int W2 = 8;
  const int wv = M <= 16 ? W : W2;
  const dim3 grid(unsigned((N / 16 + wv - 1) / wv)), block(wv * 64);
  const size_t lds = size_t(M) * (1024 + 16) + size_t(M) * KB * 8;
  const bool bp = w_kind == WZ_WSCALE_E8M0;
  // passes of four (row, K-block) pairs per wave
  const int xp = M * KB <= 4 * wv ? 1 : M * KB <= 8 * wv ? 2 : M * KB <= 16 * wv ? 4 : 8;
  if (M > 32 || (NORM && M > 16) || M * KB > 4 * wv * 8)
    return set_error(WZ_EINVAL, "fp8 gemv (wave tile): M=%lld outside its rows", (long long)M);
#define WZ_WT(W_, XP_, AP, BP, RT_)                                                                                \
  WZ_LAUNCH("fp8_gemv_wt", stream, (fp8_gemv_wt_kernel<W_, KB, SL, XP_, AP, BP, NORM, RT_>), grid, block, lds, x, \
            w, w_s, res, y, y_hi, int(n_split), int(M), int(N), nw, eps, b, hsum)
#define WZ_WTK(W_, XP_, RT_)                                 \
  do {                                                       \
    if (pow2) {                                              \
      if (bp) WZ_WT(W_, XP_, true, true, RT_);               \
      else WZ_WT(W_, XP_, true, false, RT_);                 \
    } else {                                                 \
      if (bp) WZ_WT(W_, XP_, false, true, RT_);              \
      else WZ_WT(W_, XP_, false, false, RT_);                \
    }                                                        \
  } while (0)
  if constexpr (NORM) {
    WZ_WTK(W, 1, 1);
  } else {
    if (M > 16)
      WZ_WTK(W2, 8, 2);
    else if (xp == 1)
      WZ_WTK(W, 1, 1);
    else if (xp == 2)
      WZ_WTK(W, 2, 1);
    else
      WZ_WTK(W, 4, 1);
  }
#undef WZ_WTK
#undef WZ_WT
  return check_launch("fp8_gemv_wt");
}

static int gemv_dispatch(bool qa, const void* x, const void* xs, int a_kind, const uint8_t* w, const void* w_s,
                         int w_kind, const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M,
                         int64_t N, int64_t K, bool pow2, hipStream_t stream) {
  // the bf16 path quantises M x K / 128 pairs in passes of four per wave, the
  // fewest of 1, 2, 4, 8, 16 passes that cover them (at most the third value
  // of each WZ_GV1_K*), and holds them in LDS
  if (!qa && gemv_wt_serves(false, M, N, K))
    return launch_gemv_wt<false>(x, nullptr, nullptr, 0.0f, nullptr, w, w_s, w_kind, res, y, y_hi, n_split, M, N,
                                 pow2, stream);
  const int rt = M <= 16 ? 1 : 2;
  auto fits1 = [&](int W_, int XP_) {
    return M * (K / 128) <= 4 * W_ * XP_ && gemv1_dyn_bytes(false, M, K, W_, rt) + 64 <= kLdsMax;
  };
  if (N / 16 <= WZ_GV1_MAX_TILES) {
#define WZ_G1_(W_, NKB_, XP_)                                                                                 \
  if (qa) return launch_gemv1<W_, NKB_, 1, true>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream); \
  if (fits1(W_, 1)) return launch_gemv1<W_, NKB_, 1, false>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream); \
  if (XP_ >= 2 && fits1(W_, 2)) return launch_gemv1<W_, NKB_, (XP_ >= 2 ? 2 : 1), false>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream); \
  if (XP_ >= 4 && fits1(W_, 4)) return launch_gemv1<W_, NKB_, (XP_ >= 4 ? 4 : 1), false>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream); \
  if (XP_ >= 8 && fits1(W_, 8)) return launch_gemv1<W_, NKB_, (XP_ >= 8 ? 8 : 1), false>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream); \
  break
#define WZ_G1(...) WZ_G1_(__VA_ARGS__)
    switch (K) {
      case 1024: WZ_G1(WZ_GV1_K1024);
      case 2048: WZ_G1(WZ_GV1_K2048);
      case 4096: WZ_G1(WZ_GV1_K4096);
      case 8192: WZ_G1(WZ_GV1_K8192);
      default: break;
    }
#undef WZ_G1
#undef WZ_G1_
  }
  if (M > 16) return set_error(WZ_EINVAL, "fp8 gemv: M=%lld rows need the one-tile kernel", (long long)M);
#define WZ_GV(...)                                                                                          \
  return qa ? launch_gemv<__VA_ARGS__, true>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream)          \
            : launch_gemv<__VA_ARGS__, false>(x, xs, a_kind, w, w_s, w_kind, res, y, y_hi, n_split, M, N, K, pow2, stream)
  switch (K) {
    case 1024: WZ_GV(WZ_GV_K1024);
    case 2048: WZ_GV(WZ_GV_K2048);
    case 4096: WZ_GV(WZ_GV_K4096);
    case 8192: WZ_GV(WZ_GV_K8192);
    default: return set_error(WZ_EINVAL, "fp8 gemv: no shape for K=%lld", (long long)K);
  }
#undef WZ_GV
}

}  // namespace wz

extern "C" size_t wz_fp8_gemm_packed_workspace_bytes(int64_t M, int64_t K, int act_scale_kind) {
  using namespace wz;
  if (M <= 0 || K <= 0) return 0;
  if (M <= 16 && gemv_shape_ok(K)) return 0;  // the GEMV kernels read e8m0 scales as they are
  return act_scale_kind == WZ_SCALE_UE8M0 ? size_t(M) * size_t(K / 128) * 4 : 0;
}

namespace wz {

// y_hi / n_split: two stacked weights, the columns from n_split on to their own
// buffer (nullptr / N: one weight).
static int gemm_packed(const char* name, const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                       const uint16_t* res, void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                       int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream, uint16_t* y_hi = nullptr,
                       int64_t n_split = -1) {
  if (n_split < 0) n_split = N;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld", name, (long long)M, (long long)N, (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30)) return set_error(WZ_EINVAL, "%s: dimension too large", name);
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
      (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
    return set_error(WZ_EINVAL, "%s: bad scale kinds %d/%d", name, act_scale_kind, w_scale_kind);
  if (M == 0) return WZ_OK;
  if (!a_e4m3 || !a_s || !w_packed || !w_s || !c_bf16) return set_error(WZ_EINVAL, "%s: null pointer", name);
  if (res && overlap(res, c_bf16, size_t(M) * size_t(N) * 2))
    return set_error(WZ_EINVAL, "%s: the residual and the output overlap", name);
  const bool pow2 = act_scale_kind != WZ_SCALE_F32;
  const uint8_t* w = static_cast<const uint8_t*>(w_packed);
  uint16_t* c = static_cast<uint16_t*>(c_bf16);
  if (gemv_serves(true, M, N, K))
    return gemv_dispatch(true, a_e4m3, a_s, act_scale_kind, w, w_s, w_scale_kind, res, c, y_hi, n_split, M, N, K,
                         pow2, stream);
  if (gemv_mt_serves(M, N, K))
    return gemv_mt_dispatch(a_e4m3, a_s, act_scale_kind, w, w_s, w_scale_kind, res, c, y_hi, n_split, M, N, K, pow2,
                            stream);
  const bool tile = tile_gemm_fits(M, N, K);
  if (y_hi && !tile) return set_error(WZ_EINVAL, "%s: a split output outside the tile GEMM's range", name);
  const float* xs = static_cast<const float*>(a_s);
  if (act_scale_kind == WZ_SCALE_UE8M0) {
    const size_t need = wz_fp8_gemm_packed_workspace_bytes(M, K, act_scale_kind);
    if (!ws || ws_bytes < need)
      return set_error(WZ_ESPACE, "%s: workspace of %zu bytes needed for M=%lld K=%lld, got %zu", name, need,
                       (long long)M, (long long)K, ws_bytes);
    const int64_t n = M * (K / 128);
    WZ_LAUNCH("e8m0_to_f32", stream, e8m0_to_f32_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
              static_cast<const uint8_t*>(a_s), static_cast<float*>(ws), n);
    if (int rc = check_launch("fp8_gemm_packed scales")) return rc;
    xs = static_cast<const float*>(ws);
  }
  const uint8_t* xq = static_cast<const uint8_t*>(a_e4m3);
  if (tile) return launch_tile_gemm(xq, xs, pow2, w, w_s, w_scale_kind, res, c, y_hi, n_split, M, N, K, stream);
  return add_residual(res, c, M, N, launch_dense_fp8(w, w_s, w_scale_kind, xq, xs, pow2, c, M, N, K, stream),
                      stream);
}

}  // namespace wz

extern "C" int wz_fp8_gemm_packed(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                                  void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                                  int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream) {
  return wz::gemm_packed("fp8_gemm_packed", a_e4m3, a_s, w_packed, w_s, nullptr, c_bf16, M, N, K, act_scale_kind,
                         w_scale_kind, ws, ws_bytes, stream);
}

extern "C" int wz_fp8_gemm_packed_add(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                                      const void* residual_bf16, void* c_bf16, int64_t M, int64_t N, int64_t K,
                                      int act_scale_kind, int w_scale_kind, void* ws, size_t ws_bytes,
                                      hipStream_t stream) {
  if (!residual_bf16) return wz::set_error(WZ_EINVAL, "fp8_gemm_packed_add: null residual");
  return wz::gemm_packed("fp8_gemm_packed_add", a_e4m3, a_s, w_packed, w_s,
                         static_cast<const uint16_t*>(residual_bf16), c_bf16, M, N, K, act_scale_kind, w_scale_kind,
                         ws, ws_bytes, stream);
}

extern "C" int wz_fp8_gemm_packed_pair(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                                       void* c0_bf16, int64_t N0, void* c1_bf16, int64_t M, int64_t N, int64_t K,
                                       int act_scale_kind, int w_scale_kind, void* ws, size_t ws_bytes,
                                       hipStream_t stream) {
  using namespace wz;
  if (N0 <= 0 || N0 >= N || N0 % 128)
    return set_error(WZ_EINVAL, "fp8_gemm_packed_pair: split N0=%lld must be a multiple of 128 inside N=%lld",
                     (long long)N0, (long long)N);
  if (!c1_bf16) return set_error(WZ_EINVAL, "fp8_gemm_packed_pair: null pointer");
  if (M > 0 && gemv_serves(true, M, N, K) && N % 16 == 0 && K % 128 == 0 && N <= (1 << 30) && K <= (1 << 30)) {
    if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
        (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
      return set_error(WZ_EINVAL, "fp8_gemm_packed_pair: bad scale kinds %d/%d", act_scale_kind, w_scale_kind);
    if (!a_e4m3 || !a_s || !w_packed || !w_s || !c0_bf16) return set_error(WZ_EINVAL, "fp8_gemm_packed_pair: null pointer");
    return gemv_dispatch(true, a_e4m3, a_s, act_scale_kind, static_cast<const uint8_t*>(w_packed), w_s, w_scale_kind,
                         nullptr, static_cast<uint16_t*>(c0_bf16), static_cast<uint16_t*>(c1_bf16), N0, M, N, K,
                         act_scale_kind != WZ_SCALE_F32, stream);
  }
  if (gemv_mt_serves(M, N, K) || tile_gemm_fits(M, N, K))
    // the M-tiled GEMV and the tile GEMM write the columns past N0 to the second buffer
    return gemm_packed("fp8_gemm_packed_pair", a_e4m3, a_s, w_packed, w_s, nullptr, c0_bf16, M, N, K, act_scale_kind,
                       w_scale_kind, ws, ws_bytes, stream, static_cast<uint16_t*>(c1_bf16), N0);
  // outside both: the two weights one after the other (the packed tiles of
  // rows N0.. and their block-scale rows start where the first weight's end)
  if (int rc = gemm_packed("fp8_gemm_packed_pair", a_e4m3, a_s, w_packed, w_s, nullptr, c0_bf16, M, N0, K,
                           act_scale_kind, w_scale_kind, ws, ws_bytes, stream))
    return rc;
  const size_t sbytes = w_scale_kind == WZ_WSCALE_E8M0 ? 1 : 4;
  return gemm_packed("fp8_gemm_packed_pair", a_e4m3, a_s, static_cast<const uint8_t*>(w_packed) + size_t(N0) * K,
                     static_cast<const uint8_t*>(w_s) + size_t(N0 / 128) * size_t((K + 127) / 128) * sbytes,
                     nullptr, c1_bf16, M, N - N0, K, act_scale_kind, w_scale_kind, ws, ws_bytes, stream);
}

extern "C" size_t wz_fp4_gemm_packed_workspace_bytes(int64_t M, int64_t K, int act_scale_kind) {
  if (M <= 0 || K <= 0) return 0;
  return act_scale_kind == WZ_SCALE_UE8M0 ? size_t(M) * size_t(K / 128) * 4 : 0;
}

extern "C" int wz_fp4_gemm_packed(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_packed_s,
                                  void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind, void* ws,
                                  size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (M < 0 || N <= 0 || K <= 0 || N % 16 || K % 128)
    return set_error(WZ_EINVAL, "fp4_gemm_packed: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N,
                     (long long)K);
  if (M > (1 << 30) || N > (1 << 30) || K > (1 << 30))
    return set_error(WZ_EINVAL, "fp4_gemm_packed: dimension too large");
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32)
    return set_error(WZ_EINVAL, "fp4_gemm_packed: unknown activation scale kind %d", act_scale_kind);
  if (M == 0) return WZ_OK;
  if (!a_e4m3 || !a_s || !w_packed || !w_packed_s || !c_bf16) return set_error(WZ_EINVAL, "fp4_gemm_packed: null pointer");
  const float* xs = static_cast<const float*>(a_s);
  if (act_scale_kind == WZ_SCALE_UE8M0) {
    const size_t need = wz_fp4_gemm_packed_workspace_bytes(M, K, act_scale_kind);
    if (!ws || ws_bytes < need)
      return set_error(WZ_ESPACE, "fp4_gemm_packed: workspace of %zu bytes needed for M=%lld K=%lld, got %zu", need,
                       (long long)M, (long long)K, ws_bytes);
    const int64_t n = M * (K / 128);
    WZ_LAUNCH("e8m0_to_f32", stream, e8m0_to_f32_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0,
              static_cast<const uint8_t*>(a_s), static_cast<float*>(ws), n);
    if (int rc = check_launch("fp4_gemm_packed scales")) return rc;
    xs = static_cast<const float*>(ws);
  }
  return launch_dense_fp4(static_cast<const uint8_t*>(w_packed), static_cast<const uint32_t*>(w_packed_s),
                          static_cast<const uint8_t*>(a_e4m3), xs, act_scale_kind != WZ_SCALE_F32,
                          static_cast<uint16_t*>(c_bf16), M, N, K, stream);
}

namespace wz {

// RMSNorm (+ the residual step) fused into the one-tile GEMV's x path.
template <int W, int NKB>
static int launch_norm_gemv1(const void* x, const uint16_t* b, const float* nw, float eps, uint16_t* hsum,
                             const uint8_t* w, const void* w_s, int w_kind, uint16_t* y, uint16_t* y_hi,
                             int64_t n_split, int64_t M, int64_t N, int64_t K, bool pow2, hipStream_t stream) {
  if (M > GvNorm<W, NKB>::ROWS)
    return set_error(WZ_EINVAL, "fp8_norm_linear_packed: M=%lld rows exceed the %d the fused norm serves at K=%lld",
                     (long long)M, GvNorm<W, NKB>::ROWS, (long long)K);
  const dim3 grid(unsigned(N / 16)), block(W * 64);
  const size_t lds = gemv1_dyn_bytes(false, M, K, W, 1);
  const bool bp = w_kind == WZ_WSCALE_E8M0;
#define WZ_NG1(AP, BP)                                                                                          \
  do {                                                                                                          \
    static int granted = 0;                                                                                     \
    if (int rc = allow_lds(fp8_gemv1_kernel<W, NKB, 1, false, AP, BP, true, 1>, lds, granted)) return rc;             \
    WZ_LAUNCH("fp8_norm_gemv1", stream, (fp8_gemv1_kernel<W, NKB, 1, false, AP, BP, true, 1>), grid, block, lds, x, nullptr, 0, \
              w, w_s, nullptr, y, y_hi, int(n_split), int(M), int(N), int(K), nw, eps, b, hsum, 1);            \
  } while (0)
  if (pow2) {
    if (bp) WZ_NG1(true, true); else WZ_NG1(true, false);
  } else {
    if (bp) WZ_NG1(false, true); else WZ_NG1(false, false);
  }
#undef WZ_NG1
  return check_launch("fp8_norm_gemv1");
}

template <int W, int NKB, int XP>
static int norm_rows(int) { return GvNorm<W, NKB>::ROWS; }

}  // namespace wz

extern "C" int wz_fp8_norm_linear_max_rows(int64_t K) {
  using namespace wz;
#define WZ_NR(...) return norm_rows<__VA_ARGS__>(0)
  switch (K) {
    case 1024: WZ_NR(WZ_GV1_K1024);
    case 2048: WZ_NR(WZ_GV1_K2048);
    case 4096: WZ_NR(WZ_GV1_K4096);
    case 8192: WZ_NR(WZ_GV1_K8192);
    default: return 0;
  }
#undef WZ_NR
}

extern "C" int wz_fp8_norm_linear_packed_pair(const void* x_bf16, const void* b_bf16, const float* norm_weight,
                                              float eps, void* sum_bf16, const void* w_packed, const void* w_s,
                                              void* c0_bf16, int64_t N0, void* c1_bf16, int64_t M, int64_t N,
                                              int64_t K, int act_scale_kind, int w_scale_kind, hipStream_t stream) {
  using namespace wz;
  const char* name = "fp8_norm_linear_packed_pair";
  if (M < 0 || N <= 0 || N % 16 || N > (1 << 30) || !gemv_shape_ok(K))
    return set_error(WZ_EINVAL, "%s: bad shape M=%lld N=%lld K=%lld (K in 1024, 2048, 4096, 8192)", name,
                     (long long)M, (long long)N, (long long)K);
  if (c1_bf16 ? (N0 <= 0 || N0 >= N || N0 % 128) : N0 != N)
    return set_error(WZ_EINVAL, "%s: split N0=%lld must be a multiple of 128 inside N=%lld (N0 = N without c1)",
                     name, (long long)N0, (long long)N);
  if (act_scale_kind < WZ_SCALE_F32 || act_scale_kind > WZ_SCALE_UE8M0_F32 ||
      (w_scale_kind != WZ_WSCALE_F32 && w_scale_kind != WZ_WSCALE_E8M0))
    return set_error(WZ_EINVAL, "%s: bad scale kinds %d/%d", name, act_scale_kind, w_scale_kind);
  if (sum_bf16 && !b_bf16) return set_error(WZ_EINVAL, "%s: a sum output needs the addend b", name);
  if (M == 0) return WZ_OK;
  if (!x_bf16 || !norm_weight || !w_packed || !w_s || !c0_bf16) return set_error(WZ_EINVAL, "%s: null pointer", name);
  // workgroup 0 writes the sum while the others read x and b; every workgroup
  // writes its outputs while others may still read x, b
  const size_t xbytes = size_t(M) * size_t(K) * 2;
  const size_t y0bytes = size_t(M) * size_t(N0) * 2, y1bytes = size_t(M) * size_t(N - N0) * 2;
  auto meets = [](const void* a, size_t na, const void* b, size_t nb) {
    const char *pa = static_cast<const char*>(a), *pb = static_cast<const char*>(b);
    return pa < pb + nb && pb < pa + na;
  };
  const void* ins[2] = {x_bf16, b_bf16};
  for (const void* in : ins) {
    if (!in) continue;
    if ((sum_bf16 && meets(sum_bf16, xbytes, in, xbytes)) || meets(c0_bf16, y0bytes, in, xbytes) ||
        (c1_bf16 && meets(c1_bf16, y1bytes, in, xbytes)))
      return set_error(WZ_EINVAL, "%s: an output overlaps an input", name);
  }
  const uint8_t* w = static_cast<const uint8_t*>(w_packed);
  const uint16_t* b = static_cast<const uint16_t*>(b_bf16);
  uint16_t *y0 = static_cast<uint16_t*>(c0_bf16), *y1 = static_cast<uint16_t*>(c1_bf16),
           *hs = static_cast<uint16_t*>(sum_bf16);
  const bool pow2 = act_scale_kind != WZ_SCALE_F32;
  if (gemv_wt_serves(true, M, N, K))
    return launch_gemv_wt<true>(x_bf16, b, norm_weight, eps, hs, w, w_s, w_scale_kind, nullptr, y0, y1, N0, M, N, pow2,
                                stream);
#define WZ_NL_(W_, NKB_, XP_)                                                                                  \
  return launch_norm_gemv1<W_, NKB_>(x_bf16, b, norm_weight, eps, hs, w, w_s, w_scale_kind, y0, y1, N0, M, N, K, \
                                     pow2, stream)
#define WZ_NL(...) WZ_NL_(__VA_ARGS__)
  switch (K) {
    case 1024: WZ_NL(WZ_GV1_K1024);
    case 2048: WZ_NL(WZ_GV1_K2048);
    case 4096: WZ_NL(WZ_GV1_K4096);
    default: WZ_NL(WZ_GV1_K8192);
  }
#undef WZ_NL
#undef WZ_NL_
}
