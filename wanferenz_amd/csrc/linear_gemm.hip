// FP8 block-scaled GEMM on packed weights, for the rows the GEMV does not serve
// (M > 16 where a second row tile would not fit the GEMV's registers, and every
// M > 32): y[M, N] (bf16) = dequant(xq) . dequant(W)^T — fp8_gemm,
// reference.py:292-311 (CPU statement torch_ops.py:93-99), on the weight tiles
// wz_fp8_pack writes ([N/16][K/128][2][1 KB] in MFMA lane order).
//
// Batch invariance.  The reference enables its decode GEMV only where it is
// bit-equal to its GEMM at every M up to 32 (fp8_vector.py:235-252), so a
// token's projection does not depend on how many tokens share the call.  Here
// the GEMV fixes the order: K is cut into slices of NKB K-blocks (the K-range
// one GEMV wave owns: 1024 -> 1, 2048 -> 2, 4096 -> 2, 8192 -> 4), each slice
// accumulates from zero through the MFMA chain (or, for float scales, one
// scaled partial per K-block added on the VALU), and the slices are summed in
// order, the first one taken as it is.  This kernel walks K in order and does
// exactly that with a slice accumulator and a running total, so every output
// element has the bits the GEMV gives it, whatever M is.
//
// Tiles.  A workgroup of four waves (2 x 2) owns BM x BN outputs; a wave owns
// RT x CT tiles of 16 x 16.  Each K-block's A rows (BM x 128 e4m3, 16-byte
// chunks XOR-swizzled by row) and weight tiles (BN / 16 x 2 KB) are brought into
// LDS by 16-byte buffer loads that write LDS directly, in stages of KS
// K-blocks, S stages ahead through S + 1 buffers; every wave issues the same
// number of them per stage, so a fixed vmcnt wait and one barrier per stage
// cover it.  Within a K-block a wave reads all its fragments, then issues its
// RT x CT MFMAs back to back into separate accumulators, then does the VALU
// work (float scales, the slice sums).  The activation block scales and the
// weight block scales of the whole K range sit in LDS from the start.  No load
// in the loop has a register destination, so the compiler inserts no memory
// waits there.  Workgroups are renumbered with
// xcd_runs so the M-tiles of one N-block (which read the same weight tiles)
// run on one XCD, one after the other in its L2.
#include "mfma_ops.h"

#include <algorithm>

namespace wz {

template <int RT_, int CT_, int S_, int KS_>
struct TileCfg {
  static constexpr int WM = 2, WN = 2;                 // waves along M and N
  static constexpr int RT = RT_, CT = CT_;             // 16 x 16 tiles per wave
  static constexpr int S = S_, KS = KS_;               // stages in flight; K-blocks per stage
  static constexpr int BM = 16 * RT * WM, BN = 16 * CT * WN;
  static constexpr int NBUF = S + 1;
  static constexpr int STEP = (BM + BN) * 128;        // bytes of one K-block: A rows, then weight tiles
  static constexpr int STAGE = KS * STEP;
  static constexpr int LA = BM / 32, LB = BN / 32;    // 1-KB loads per wave per K-block
  static constexpr int LW = KS * (LA + LB);           // ... per stage
  static_assert(LA >= 1 && LB >= 1, "every wave takes a share of both operands");
  static_assert((S - 1) * LW < 64, "the stage wait is a vmcnt immediate");
  static_assert(CT * 16 <= 128, "a wave's columns share one weight-scale block");
};

// slot of the 16-byte chunk q of A row r: q ^ gemm_swz(r), so the 16 rows of an
// A-operand read (one chunk each) fall in distinct banks
__device__ __forceinline__ int gemm_swz(int row) { return (row >> 1) & 7; }

// Activation block scales kept in LDS for the whole K range: power-of-two
// scales as their exponent bytes (what the MFMA takes), float scales as floats.
template <bool AP2>
struct AScaleT {
  using T = float;
};
template <>
struct AScaleT<true> {
  using T = uint8_t;
};

template <class C, bool AP2, bool BP2>
__global__ __launch_bounds__(256, 1) void fp8_tile_gemm_kernel(const uint8_t* __restrict__ xq,
                                                               const float* __restrict__ xs,
                                                               const uint8_t* __restrict__ wp,
                                                               const void* __restrict__ w_s,
                                                               const uint16_t* __restrict__ res,
                                                               uint16_t* __restrict__ y, uint16_t* __restrict__ y_hi,
                                                               int n_split, int M, int N, int K, int slice, int n_mt,
                                                               int n_nb) {
  using AS = typename AScaleT<AP2>::T;
  constexpr bool CH = AP2 && BP2;  // both scales ride in the MFMA: the slice chains through it
  extern __shared__ __align__(1024) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int wm = wave / C::WN, wn = wave % C::WN;
  const int KB = K / 128, NT = N / 16, NSB = (N + 127) / 128;
  const int t = xcd_runs(int(blockIdx.x), 0, n_mt * n_nb);
  const int mt = t % n_mt, nb = t / n_mt;
  const int m0 = mt * C::BM, n0 = nb * C::BN;
  float* const ws_l = reinterpret_cast<float*>(lds + C::NBUF * C::STAGE);   // [KB]
  AS* const as_l = reinterpret_cast<AS*>(ws_l + KB);                        // [BM][KB]

  // this wave's direct loads of a K-block: A blocks wave*LA + j (rows 8i .. 8i+7,
  // lane l: row 8i + l/8, slot l%8 holding chunk slot ^ swz(row)), weight
  // blocks wave*LB + j (tile b/2, half b%2; lane l: 16 bytes at 16 l)
  const __amdgpu_buffer_rsrc_t a_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(xq), short(0),
                                                                        M * K, 0x00020000);
  const __amdgpu_buffer_rsrc_t b_rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wp), short(0),
                                                                        N * K, 0x00020000);
  uint32_t avo[C::LA], bvo[C::LB];
#pragma unroll
  for (int j = 0; j < C::LA; ++j) {
    const int i = wave * C::LA + j, row = 8 * i + (lane >> 3), slot = lane & 7;
    const int src = min(m0 + row, M - 1);  // rows past M repeat the last; their outputs are dropped
    avo[j] = uint32_t(src) * uint32_t(K) + uint32_t((slot ^ gemm_swz(row)) << 4);
  }
#pragma unroll
  for (int j = 0; j < C::LB; ++j) {
    const int b = wave * C::LB + j;
    const int nt = min(n0 / 16 + (b >> 1), NT - 1);  // tiles past N repeat the last; dropped
    bvo[j] = uint32_t(nt) * uint32_t(KB) * 2048u + uint32_t(b & 1) * 1024u + uint32_t(lane) * 16u;
  }
  const uint32_t lds0 = lds_addr(lds);
  // stage q holds K-blocks q KS .. q KS + KS - 1 (past the end: the last, unread)
  auto issue = [&](int q) {
    const uint32_t buf = lds0 + uint32_t(q % C::NBUF) * C::STAGE;
#pragma unroll
    for (int u = 0; u < C::KS; ++u) {
      const int kb = min(q * C::KS + u, KB - 1);
      const uint32_t sb = buf + u * C::STEP;
#pragma unroll
      for (int j = 0; j < C::LA; ++j)
        load_lds_16(a_rs, __builtin_amdgcn_readfirstlane(sb + (wave * C::LA + j) * 1024), avo[j],
                    uint32_t(kb) * 128u);
#pragma unroll
      for (int j = 0; j < C::LB; ++j)
        load_lds_16(b_rs, __builtin_amdgcn_readfirstlane(sb + C::BM * 128 + (wave * C::LB + j) * 1024), bvo[j],
                    uint32_t(kb) * 2048u);
    }
  };

  // the first S stages, then the scales with ordinary loads: the compiler's
  // wait for those drains the stages as well, one round trip for both
  const int NQ = (KB + C::KS - 1) / C::KS;
#pragma unroll
  for (int q = 0; q < C::S; ++q) issue(q);
  for (int i = tid; i < C::BM * KB; i += 256) {
    const int r = i / KB, kb = i - r * KB;
    const float v = xs[int64_t(min(m0 + r, M - 1)) * KB + kb];
    if constexpr (AP2)
      as_l[i] = uint8_t((__float_as_uint(v) >> 23) & 0xFFu);
    else
      as_l[i] = v;
  }
  for (int kb = tid; kb < KB; kb += 256) {
    const int64_t si = int64_t(min(n0 / 128, NSB - 1)) * KB + kb;
    ws_l[kb] = BP2 ? e8m0_to_f32(static_cast<const uint8_t*>(w_s)[si]) : static_cast<const float*>(w_s)[si];
  }
  __syncthreads();

  const v4f zero = {0.f, 0.f, 0.f, 0.f};
  v4f sac[C::RT][C::CT], tot[C::RT][C::CT];
#pragma unroll
  for (int r = 0; r < C::RT; ++r)
#pragma unroll
    for (int c = 0; c < C::CT; ++c) sac[r][c] = tot[r][c] = zero;
  const int arow0 = wm * 16 * C::RT;  // first A row of this wave in the tile
  int sj = 0;                         // position of the K-block in its slice

  for (int q = 0; q < NQ; ++q) {
    // this stage's loads have landed: S - 1 stages of this wave's loads follow them
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"((C::S - 1) * C::LW) : "memory");
    const uint8_t* buf = lds + (q % C::NBUF) * C::STAGE;
#pragma unroll
    for (int u = 0; u < C::KS; ++u) {
      const int kb = q * C::KS + u;
      if (C::KS > 1 && kb >= KB) break;  // a ragged last stage
      const uint8_t* st = buf + u * C::STEP;
      // every fragment of the K-block first, then the MFMAs back to back
      v8i av[C::RT], bv[C::CT];
      int ase[C::RT];
#pragma unroll
      for (int c = 0; c < C::CT; ++c) {
        const uint8_t* p = st + C::BM * 128 + ((wn * C::CT + c) * 2) * 1024 + lane * 16;
        const v4i lo = *reinterpret_cast<const v4i*>(p), hi = *reinterpret_cast<const v4i*>(p + 1024);
        bv[c] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
      for (int r = 0; r < C::RT; ++r) {
        const int row = arow0 + r * 16 + nl, sw = gemm_swz(row);
        const uint8_t* pa = st + row * 128;
        const v4i lo = *reinterpret_cast<const v4i*>(pa + ((g ^ sw) << 4));
        const v4i hi = *reinterpret_cast<const v4i*>(pa + (((g + 4) ^ sw) << 4));
        av[r] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        if constexpr (AP2) ase[r] = int(as_l[row * KB + kb]);
      }
      const float wsf = ws_l[kb];
      const int wse = int((__float_as_uint(wsf) >> 23) & 0xFFu);
      const bool first = sj == 0;
      sj = sj + 1 == slice ? 0 : sj + 1;
      const bool last = sj == 0 || kb + 1 == KB, first_slice = kb < slice;
      v4f p[C::RT][C::CT];
#pragma unroll
      for (int r = 0; r < C::RT; ++r)
#pragma unroll
        for (int c = 0; c < C::CT; ++c) {
          if constexpr (CH)
            p[r][c] = mfma_scaled<kFmtFp8, kFmtFp8>(av[r], bv[c], first ? zero : sac[r][c], ase[r], wse);
          else
            p[r][c] = mfma_scaled<kFmtFp8, kFmtFp8>(av[r], bv[c], zero, AP2 ? ase[r] : kE8m0One,
                                                    BP2 ? wse : kE8m0One);
        }
#pragma unroll
      for (int r = 0; r < C::RT; ++r) {
        if constexpr (CH) {
#pragma unroll
          for (int c = 0; c < C::CT; ++c) sac[r][c] = p[r][c];
        } else {
          // the GEMV's per-K-block form (mma_step): the partial scaled on the VALU,
          // (activation scale x weight scale) first, then one multiply-add
          float sa[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            sa[i] = AP2 ? 1.0f : float(as_l[(arow0 + r * 16 + g * 4 + i) * KB + kb]);
          const float sb = BP2 ? 1.0f : wsf;
#pragma unroll
          for (int c = 0; c < C::CT; ++c) {
            v4f a = first ? zero : sac[r][c];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] += p[r][c][i] * (sa[i] * sb);
            sac[r][c] = a;
          }
        }
      }
      if (last) {
#pragma unroll
        for (int r = 0; r < C::RT; ++r)
#pragma unroll
          for (int c = 0; c < C::CT; ++c) tot[r][c] = first_slice ? sac[r][c] : tot[r][c] + sac[r][c];
      }
    }
    issue(q + C::S);
  }
  // the trailing loads write LDS: drained before the workgroup ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

#pragma unroll
  for (int r = 0; r < C::RT; ++r)
#pragma unroll
    for (int c = 0; c < C::CT; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = m0 + arow0 + r * 16 + g * 4 + i, col = n0 + (wn * C::CT + c) * 16 + nl;
        if (row >= M || col >= N) continue;
        const float v = tot[r][c][i];
        if (col < n_split) {
          const int64_t o = int64_t(row) * n_split + col;
          // the residual stream: the product rounded to bf16, then one fp32 add
          y[o] = f32_to_bf16(res ? bf16_round(v) + __uint_as_float(uint32_t(res[o]) << 16) : v);
        } else {
          y_hi[int64_t(row) * (N - n_split) + (col - n_split)] = f32_to_bf16(v);
        }
      }
}

// Tile shapes, largest first: 128 x 128 (RT 4, CT 4; one K-block a stage,
// three in flight), 64 x 128 (RT 2, CT 4; two K-blocks a stage, two stages in
// flight), 32 x 64 and 32 x 32 (four K-blocks a stage; two and three stages).
// The largest with at least one workgroup per CU is taken, else the one with
// the most workgroups.  Float activation scales hold four bytes per (row,
// K-block) in LDS, so their 64 x 128 tile takes one K-block a stage and their
// 128 x 128 tile serves K up to 6144.
using Tile128 = TileCfg<4, 4, 3, 1>;
using Tile64 = TileCfg<2, 4, 2, 2>;
using Tile64f = TileCfg<2, 4, 4, 1>;
using Tile32w = TileCfg<1, 2, 2, 4>;
using Tile32 = TileCfg<1, 1, 3, 4>;

template <class C>
static size_t tile_lds(int64_t K, bool a_pow2) {
  return size_t(C::NBUF) * C::STAGE + size_t(K / 128) * 4 + size_t(C::BM) * size_t(K / 128) * (a_pow2 ? 1 : 4);
}

template <class C>
static int64_t tile_blocks(int64_t M, int64_t N) {
  return ((M + C::BM - 1) / C::BM) * ((N + C::BN - 1) / C::BN);
}

template <class C, bool AP2, bool BP2>
static int launch_tile(const uint8_t* xq, const float* xs, const uint8_t* wp, const void* w_s, const uint16_t* res,
                       uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N, int64_t K, int slice,
                       hipStream_t stream) {
  const size_t lds = tile_lds<C>(K, AP2);
  static int granted = 0;
  if (int(lds) > granted) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(fp8_tile_gemm_kernel<C, AP2, BP2>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)) != hipSuccess)
      return set_error(WZ_ELAUNCH, "fp8 tile gemm: %zu bytes of LDS refused", lds);
    granted = int(lds);
  }
  const int n_mt = int((M + C::BM - 1) / C::BM), n_nb = int((N + C::BN - 1) / C::BN);
  WZ_LAUNCH("fp8_tile_gemm", stream, (fp8_tile_gemm_kernel<C, AP2, BP2>), dim3(unsigned(n_mt * n_nb)), dim3(256), lds,
            xq, xs, wp, w_s, res, y, y_hi, int(n_split), int(M), int(N), int(K), slice, n_mt, n_nb);
  return check_launch("fp8_tile_gemm");
}

template <class C>
static int launch_tile_kinds(const uint8_t* xq, const float* xs, bool a_pow2, const uint8_t* wp, const void* w_s,
                             int w_kind, const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M,
                             int64_t N, int64_t K, int slice, hipStream_t stream) {
  const bool bp = w_kind == WZ_WSCALE_E8M0;
#define WZ_TK(AP, BP) launch_tile<C, AP, BP>(xq, xs, wp, w_s, res, y, y_hi, n_split, M, N, K, slice, stream)
  if (a_pow2) return bp ? WZ_TK(true, true) : WZ_TK(true, false);
  return bp ? WZ_TK(false, true) : WZ_TK(false, false);
#undef WZ_TK
}

// K-blocks per slice of the canonical summation order (the GEMV's per-wave K
// range at the K it serves; one slice elsewhere).
int gemv_slice_blocks(int64_t K);

// Whether the tile GEMM serves these dimensions (operand sizes addressable by
// 32-bit buffer offsets, the K range's scales within the LDS budget).
bool tile_gemm_fits(int64_t M, int64_t N, int64_t K) {
  constexpr size_t kLds = 160 * 1024;
  return M * K < (int64_t(1) << 31) && N * K < (int64_t(1) << 31) && K % 128 == 0 && N % 16 == 0 &&
         tile_lds<Tile64>(K, true) <= kLds && tile_lds<Tile64f>(K, false) <= kLds &&
         tile_lds<Tile32w>(K, false) <= kLds && tile_lds<Tile32>(K, false) <= kLds;
}

int launch_tile_gemm(const uint8_t* xq, const float* xs, bool a_pow2, const uint8_t* wp, const void* w_s, int w_kind,
                     const uint16_t* res, uint16_t* y, uint16_t* y_hi, int64_t n_split, int64_t M, int64_t N,
                     int64_t K, hipStream_t stream) {
  if (!tile_gemm_fits(M, N, K))
    return set_error(WZ_EINVAL, "fp8 tile gemm: M=%lld N=%lld K=%lld outside its range", (long long)M, (long long)N,
                     (long long)K);
  const int slice = gemv_slice_blocks(K);
  const int64_t cus = cu_count();
#define WZ_TL(C) launch_tile_kinds<C>(xq, xs, a_pow2, wp, w_s, w_kind, res, y, y_hi, n_split, M, N, K, slice, stream)
  if (M > 64 && tile_blocks<Tile128>(M, N) >= cus && tile_lds<Tile128>(K, a_pow2) <= 160 * 1024)
    return WZ_TL(Tile128);
  if (M > 32 && tile_blocks<Tile64>(M, N) >= cus) return a_pow2 ? WZ_TL(Tile64) : WZ_TL(Tile64f);
  if (tile_blocks<Tile32w>(M, N) >= cus) return WZ_TL(Tile32w);
  return WZ_TL(Tile32);
#undef WZ_TL
}

}  // namespace wz
