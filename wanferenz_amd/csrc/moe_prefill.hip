// MoE prefill path (T > 16 tokens): expert-grouped MFMA GEMMs over the
// canonical (expert, token, slot) pair order produced by the routing kernels.
//
//   (the routing's perm_kernel also cuts each active expert's pair rows into
//   M-tiles of 64 rows)
//   xquant    act_quant(x) once for all experts (quant.hip).
//   w13       per (M-tile, 64 intermediate features): the gathered 128 fp8
//             activation rows of one 128-wide K-block are staged in LDS; each
//             of the 4 waves streams the packed 16x128 w1 and w3 tiles of its
//             16 features once and runs them against the 8 row tiles
//             (V_MFMA_SCALE_F32_16X16X128_F8F6F4, e4m3 x e2m1); SwiGLU with
//             clamp and the routing weight fused, bf16 h in pair order.  The
//             FP8 shared expert is the same kernel over the token rows.
//   hquant    act_quant of h (pairs) and of the shared rows.
//   w2        per (M-tile, 64 output columns): contiguous h rows of the tile
//             staged per K-block, packed w2 tiles streamed, bf16 out rows.
//   combine   (moe.hip) per token: routed rows in ascending expert id, then
//             the shared row, fp32 sum, bf16.
//
// Semantics: Expert.forward / MoE.forward of wanferenz/model/architecture.py
// (w1/w3 outputs rounded to bf16, clamp, silu(g)*u*weight -> bf16 -> w2).
#include "moe_common.h"

namespace wz {

constexpr int kPM = kPrefillTileRows;  // pair rows per M-tile (64: the tile bodies then fit two
                                       // workgroups per CU, twice the weight bytes in flight)
constexpr int kPThreads = 256;    // 4 waves
// 16-column weight tiles per wave of a tile-GEMM mode: 0 (routed w1/w3) 4, two
// feature tiles x {w1, w3}; 1 and 3 (FP8 shared tiles, twice the bytes) 2;
// 2 (routed w2) 2; 4 (a dense MXFP4 linear) 4.  Each A operand read from LDS
// feeds NTW MFMAs, and the LDS reads of A bound the dense GEMM: at M = 2048
// four tiles per wave took w1|w3 62.7 -> 55.2 us and w2 44.1 -> 40.9 us.  The
// routed w2 keeps two: with the wider N-blocks a skewed T = 2048 batch has
// half the workgroups and its w2 took 291 -> 301 us.
constexpr int ntw_of(int mode) { return (mode == 0 || mode == 4) ? 4 : 2; }

// ------------------------------------------------------------------- gate ---
//
// Prefill routing must pick exactly the experts the exact fp32 logits pick
// (the reference evaluates the gate as one fp32 GEMM; the oracle and the
// decode path use the correctly rounded dot product).  Two passes:
//
//  gate_mfma   approximate logits a~[t,e] with V_MFMA_F32_16X16X16_BF16: each
//              64-wide K chunk is summed by four MFMAs from zero and added to
//              an fp64 accumulator, so |a~ - a| <= 65 * 2^-23 * S + (fp64
//              terms), S = sum_d |x_d w_d|, whatever order or rounding mode
//              the MFMA uses inside a chunk (bf16 x bf16 products are exact
//              in fp32).  S itself comes from the same MFMA on |x|, |w|.
//  topk_refine one wave per token: key bounds [b~ - G, b~ + G] from the logit
//              bound through the score function's slope (sigmoid <= 1/4,
//              sqrt(softplus) <= 0.61); theta = k-th largest lower bound; every
//              expert whose upper bound reaches theta is a candidate (the
//              exact top-k is among them); candidates get the exact fp64 dot,
//              exact keys pick the top-k (ties -> lower index) and the
//              weights come from exact scores.  Hash-routed layers take the
//              table's experts and compute only their exact scores.
// Softmax gates need every logit exactly (the denominator) and use the
// fp64 gate of moe.hip.

typedef short v4s __attribute__((ext_vector_type(4)));

constexpr int kGateChunk = 64;  // K elements summed in fp32 (four MFMAs from zero) per fp64 add

__device__ __forceinline__ v4s v4s_lo(v4i a) {
  return v4s{short(a[0] & 0xFFFF), short(uint32_t(a[0]) >> 16), short(a[1] & 0xFFFF), short(uint32_t(a[1]) >> 16)};
}
__device__ __forceinline__ v4s v4s_hi(v4i a) {
  return v4s{short(a[2] & 0xFFFF), short(uint32_t(a[2]) >> 16), short(a[3] & 0xFFFF), short(uint32_t(a[3]) >> 16)};
}
__device__ __forceinline__ v4i abs_bf16x8(v4i a) {
  return v4i{a[0] & 0x7FFF7FFF, a[1] & 0x7FFF7FFF, a[2] & 0x7FFF7FFF, a[3] & 0x7FFF7FFF};
}

// One workgroup: 32 tokens x 64 experts in four waves; wave w computes every
// (16-token, 16-expert) tile of the block over K quarter w, so each token and
// weight fragment is loaded once per workgroup (waves that split the experts
// instead loaded every token fragment four times and took 48-51 us at
// T = 2048, bound by L1 accesses).  Each 64-wide K chunk is summed from zero
// by four MFMAs and added into the quarter's fp64 accumulator; the quarters
// meet in LDS in quarter order.
constexpr int kGateQ = 4;  // K quarters, one per wave
__global__ __launch_bounds__(64 * kGateQ) void gate_mfma_kernel(const uint16_t* __restrict__ x,
                                                               const uint16_t* __restrict__ W,
                                                               float* __restrict__ approx,
                                                               float* __restrict__ absdot, int T, int E, int D) {
  __shared__ double red[kGateQ - 1][4][2][4][64];  // quarters 1.., expert tile, token tile, i, lane
  __shared__ float reds[kGateQ - 1][4][2][4][64];
  const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int egs = (E + 63) / 64;
  const int tg = blockIdx.x / egs, eg = blockIdx.x % egs;
  const int nl = lane & 15, g = lane >> 4;
  // clamped rows: every load is unconditional; rows past T / E are never stored
  const uint16_t* wr[4];
#pragma unroll
  for (int et = 0; et < 4; ++et) wr[et] = W + int64_t(min(eg * 64 + et * 16 + nl, E - 1)) * D;
  const uint16_t* xr0 = x + int64_t(min(tg * 32 + nl, T - 1)) * D;
  const uint16_t* xr1 = x + int64_t(min(tg * 32 + 16 + nl, T - 1)) * D;
  const int nch = D / kGateChunk, c0 = (q * nch) / kGateQ, c1 = ((q + 1) * nch) / kGateQ;
  double acc[4][2][4];
  v4f sabs[4][2];
  const v4f z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int et = 0; et < 4; ++et)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      sabs[et][m] = z;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[et][m][i] = 0.0;
    }
#pragma unroll 2
  for (int ch = c0; ch < c1; ++ch) {
    const int k0 = ch * kGateChunk;
    v4i a0[2], a1[2], b[4][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      a0[h] = load16(xr0 + k0 + 32 * h + 8 * g);
      a1[h] = load16(xr1 + k0 + 32 * h + 8 * g);
#pragma unroll
      for (int et = 0; et < 4; ++et) b[et][h] = load16(wr[et] + k0 + 32 * h + 8 * g);
    }
    v4i a0a[2], a1a[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      a0a[h] = abs_bf16x8(a0[h]);
      a1a[h] = abs_bf16x8(a1[h]);
    }
#pragma unroll
    for (int et = 0; et < 4; ++et) {
      v4f p0 = z, p1 = z;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        p0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(a0[h]), v4s_lo(b[et][h]), p0, 0, 0, 0);
        p0 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(a0[h]), v4s_hi(b[et][h]), p0, 0, 0, 0);
        p1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(a1[h]), v4s_lo(b[et][h]), p1, 0, 0, 0);
        p1 = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(a1[h]), v4s_hi(b[et][h]), p1, 0, 0, 0);
        const v4i ba = abs_bf16x8(b[et][h]);
        sabs[et][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(a0a[h]), v4s_lo(ba), sabs[et][0], 0, 0, 0);
        sabs[et][0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(a0a[h]), v4s_hi(ba), sabs[et][0], 0, 0, 0);
        sabs[et][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(a1a[h]), v4s_lo(ba), sabs[et][1], 0, 0, 0);
        sabs[et][1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(a1a[h]), v4s_hi(ba), sabs[et][1], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[et][0][i] += double(p0[i]);
        acc[et][1][i] += double(p1[i]);
      }
    }
  }
  if (q > 0) {
#pragma unroll
    for (int et = 0; et < 4; ++et)
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          red[q - 1][et][m][i][lane] = acc[et][m][i];
          reds[q - 1][et][m][i][lane] = sabs[et][m][i];
        }
  }
  __syncthreads();
  if (q > 0) return;
#pragma unroll
  for (int et = 0; et < 4; ++et) {
    const int ex = eg * 64 + et * 16 + nl;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        double v = acc[et][m][i];
        float sv = sabs[et][m][i];
#pragma unroll
        for (int qq = 0; qq < kGateQ - 1; ++qq) {
          v += red[qq][et][m][i][lane];
          sv += reds[qq][et][m][i][lane];
        }
        const int t = tg * 32 + m * 16 + g * 4 + i;
        if (t < T && ex < E) {
          approx[int64_t(t) * E + ex] = float(v);
          absdot[int64_t(t) * E + ex] = sv;
        }
      }
  }
}

// Small T: one workgroup per 16 tokens x 16 experts, the four waves split K
// (32-wide chunks; its error stays within the 64-chunk bound used below).
__global__ __launch_bounds__(256) void gate_mfma_ksplit_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ W,
                                                        float* __restrict__ approx, float* __restrict__ absdot,
                                                        int T, int E, int D) {
  __shared__ double red[3][64][4];
  __shared__ float reds[3][64][4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int etiles = (E + 15) / 16;
  const int tt = blockIdx.x / etiles, et = blockIdx.x % etiles;
  const int nl = lane & 15, g = lane >> 4;
  const int tok = tt * 16 + nl, ex = et * 16 + nl;
  const uint16_t* xr = tok < T ? x + int64_t(tok) * D : nullptr;
  const uint16_t* wr = ex < E ? W + int64_t(ex) * D : nullptr;
  const int nsteps = D / 32, s0 = (wave * nsteps) / 4, s1 = ((wave + 1) * nsteps) / 4;
  double acc[4] = {0.0, 0.0, 0.0, 0.0};
  v4f sabs = {0.f, 0.f, 0.f, 0.f};
  const v4f z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
  for (int st = s0; st < s1; ++st) {
    const int k0 = st * 32;
    const v4i a = xr ? load16(xr + k0 + 8 * g) : v4i{0, 0, 0, 0};
    const v4i b = wr ? load16(wr + k0 + 8 * g) : v4i{0, 0, 0, 0};
    v4f p = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(a), v4s_lo(b), z, 0, 0, 0);
    p = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(a), v4s_hi(b), p, 0, 0, 0);
    const v4i aa = abs_bf16x8(a), ba = abs_bf16x8(b);
    sabs = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_lo(aa), v4s_lo(ba), sabs, 0, 0, 0);
    sabs = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(v4s_hi(aa), v4s_hi(ba), sabs, 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += double(p[i]);
  }
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      red[wave - 1][lane][i] = acc[i];
      reds[wave - 1][lane][i] = sabs[i];
    }
  }
  __syncthreads();
  if (wave > 0) return;
  const int e = et * 16 + nl;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const double v = acc[i] + red[0][lane][i] + red[1][lane][i] + red[2][lane][i];
    const float sv = sabs[i] + reds[0][lane][i] + reds[1][lane][i] + reds[2][lane][i];
    const int t = tt * 16 + g * 4 + i;
    if (t < T && e < E) {
      approx[int64_t(t) * E + e] = float(v);
      absdot[int64_t(t) * E + e] = sv;
    }
  }
}

// Exact logit of (token row, expert row w): fp32-exact products summed in fp64
// across the wave (the arithmetic of gate_dot_kernel in moe.hip).  xv holds
// the token row's first kXC * 512 elements (8 per lane per chunk); all weight
// loads of a chunk group are issued before the products.
constexpr int kXC = 8;

// acc + this lane's products of one chunk group, in chunk, word, half order.
// The empty asm after each chunk keeps the compiler from converting every
// product of the group to fp64 ahead of the sum (64 doubles in registers).
__device__ __forceinline__ double exact_dot_lane(const v4i (&xb)[kXC], const v4i (&wv)[kXC], double acc) {
#pragma unroll
  for (int c = 0; c < kXC; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      acc += double(bf16lo(uint32_t(xb[c][j])) * bf16lo(uint32_t(wv[c][j])));
      acc += double(bf16hi(uint32_t(xb[c][j])) * bf16hi(uint32_t(wv[c][j])));
    }
    asm volatile("" : "+v"(acc));
  }
  return acc;
}

__device__ __forceinline__ float wave_sum_f64(double acc) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, kWave);
  return float(acc);
}

// Exact logits of the token row against NW weight rows w[0..NW-1]: every
// row's loads of a chunk group are issued before any product, so NW rows cost
// one memory round trip per chunk group.
template <int NW>
__device__ __forceinline__ void exact_logits(const v4i (&xv)[kXC], const uint16_t* __restrict__ xrow,
                                             const uint16_t* const (&w)[NW], int D, int lane, float (&out)[NW]) {
  double acc[NW];
#pragma unroll
  for (int n = 0; n < NW; ++n) acc[n] = 0.0;
  {  // the first chunk group: the token row is in xv already
    v4i wv[NW][kXC];
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int off = (lane + 64 * c) * 8;
#pragma unroll
      for (int n = 0; n < NW; ++n) wv[n][c] = off < D ? load16(w[n] + off) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int n = 0; n < NW; ++n) acc[n] = exact_dot_lane(xv, wv[n], acc[n]);
  }
  for (int base = kXC * 512; base < D; base += kXC * 512) {
    v4i wv[NW][kXC], xb[kXC];
#pragma unroll
    for (int c = 0; c < kXC; ++c) {
      const int off = base + (lane + 64 * c) * 8;
#pragma unroll
      for (int n = 0; n < NW; ++n) wv[n][c] = off < D ? load16(w[n] + off) : v4i{0, 0, 0, 0};
      xb[c] = off < D ? load16(xrow + off) : v4i{0, 0, 0, 0};
    }
#pragma unroll
    for (int n = 0; n < NW; ++n) acc[n] = exact_dot_lane(xb, wv[n], acc[n]);
  }
#pragma unroll
  for (int n = 0; n < NW; ++n) out[n] = wave_sum_f64(acc[n]);
}

constexpr float kChunkErr = float(kGateChunk + 1) / 8388608.0f;  // (chunk + 1) * 2^-23
constexpr int kRefineWaves = 4;

// G waves per token (4: one token per workgroup, for small batches; 1: four
// tokens per workgroup, whose waves then keep more tokens in flight at large
// T).  The waves of a token derive the same candidate set from the MFMA
// logits' bounds (each computes a share of the bounds, met in LDS); the
// candidates' exact logits are shared out over them (candidate r of the set,
// in expert order, to wave r % G, two rows per round trip) and meet in LDS,
// where the token's first wave picks the top-k.  kRSlots: 64-expert slots per
// lane (E <= 64 kRSlots).
template <int kRSlots, int G>
__global__ __launch_bounds__(kRefineWaves * 64, 2) void topk_refine_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ W, const float* __restrict__ approx,
    const float* __restrict__ absdot, const float* __restrict__ bias, const int32_t* __restrict__ tid2eid,
    const int64_t* __restrict__ input_ids, int64_t vocab, int T, int E, int D, int k, int score_func,
    float route_scale, float* __restrict__ weights, int32_t* __restrict__ idx) {
  constexpr int NG = kRefineWaves / G;  // tokens per workgroup
  __shared__ float s_sx[NG][kMaxExperts];  // exact score of a candidate (hash: of table slot j)
  __shared__ float s_kx[NG][kMaxExperts];  // its selection key; -inf: not a candidate
  __shared__ float s_lo[NG][kMaxExperts], s_hi[NG][kMaxExperts];  // key bounds (-inf past E)
  __shared__ int s_list[kRefineWaves][kMaxExperts / G];            // each wave's candidates
  __shared__ int s_hash[NG][17];  // hash: the table's experts (k <= 16); [16]: poison flag
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave / G, gw = wave % G;
  const int t0 = blockIdx.x * NG + grp;
  const bool live = t0 < T;
  const int t = min(t0, T - 1);  // a spare wave works on the last token and stores nothing
  const uint16_t* xr = x + int64_t(t) * D;
  v4i xv[kXC];
#pragma unroll
  for (int c = 0; c < kXC; ++c) {
    const int off = (lane + 64 * c) * 8;
    xv[c] = off < D ? load16(xr + off) : v4i{0, 0, 0, 0};
  }
  for (int e = gw * 64 + lane; e < E; e += G * 64) {
    s_kx[grp][e] = -INFINITY;
    s_sx[grp][e] = 0.0f;
  }
  int my_sel = 0;
  float mine = 0.0f;    // exact score of the lane's slot (lane < k)
  bool poison = false;  // hash id or table entry out of range: NaN weights, in-range reads
  if (tid2eid != nullptr) {
    if (gw == 0) {  // the k table slots, one per lane
      int64_t id = input_ids[t];
      const bool bad_id = id < 0 || id >= vocab;
      id = bad_id ? 0 : id;
      bool bad_e = false;
      if (lane < k) {
        const int e = tid2eid[id * k + lane];
        bad_e = e < 0 || e >= E;
        s_hash[grp][lane] = bad_e ? 0 : e;
      }
      const bool any_bad = bad_id || __ballot(bad_e) != 0ull;
      if (lane == 0) s_hash[grp][16] = any_bad ? 1 : 0;
    }
    __syncthreads();
    for (int j = gw; j < k; j += G) {
      const uint16_t* const w1[1] = {W + int64_t(s_hash[grp][j]) * D};
      float lg[1];
      exact_logits<1>(xv, xr, w1, D, lane, lg);
      if (lane == 0) s_sx[grp][j] = score_of(lg[0], score_func);
    }
    __syncthreads();
    if (gw != 0 || !live) return;
    poison = s_hash[grp][16] != 0;
    if (lane < k) {
      my_sel = s_hash[grp][lane];
      mine = s_sx[grp][lane];
    }
  } else {
    // key bounds, slot i by the token's wave i % G
    const float L = score_func == WZ_SCORE_SIGMOID ? 0.25f : 0.61f;
#pragma unroll
    for (int i = gw; i < kRSlots; i += G) {
      const int e = lane + 64 * i;
      float l = -INFINITY, h = -INFINITY;
      if (e < E) {
        const float a = approx[int64_t(t) * E + e];
        const float S = absdot[int64_t(t) * E + e] * 1.001f;
        const float f = score_of(a, score_func);
        const float key = bias ? f + bias[e] : f;
        const float Gb = L * (kChunkErr * S + 2.4e-7f * fabsf(a)) + 4.8e-7f * (fabsf(f) + fabsf(key)) + 1e-30f;
        l = key - Gb;
        h = key + Gb;
      }
      s_lo[grp][e] = l;
      s_hi[grp][e] = h;
    }
    __syncthreads();  // bounds in LDS, s_kx cleared
    float lo[kRSlots], hi[kRSlots];
#pragma unroll
    for (int i = 0; i < kRSlots; ++i) {
      lo[i] = s_lo[grp][lane + 64 * i];
      hi[i] = s_hi[grp][lane + 64 * i];
    }
    // theta = k-th largest lower bound
    unsigned taken = 0u;
    float theta = -INFINITY;
    for (int j = 0; j < k; ++j) {
      Cand best = {-INFINITY, 0x7FFFFFFF};
#pragma unroll
      for (int i = 0; i < kRSlots; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((taken >> i) & 1u)) best = cand_better(best, Cand{lo[i], e});
      }
      best = wave_argmax_dpp(best);
      theta = best.v;
      if ((best.i & 63) == lane) taken |= 1u << (best.i >> 6);
    }
    // this wave's share of the candidates (upper bound reaches theta): the
    // set in expert order, candidate r to wave r % G, listed in LDS
    int r = 0;  // candidates in the slots so far
#pragma unroll
    for (int i = 0; i < kRSlots; ++i) {
      const bool c = lane + 64 * i < E && hi[i] >= theta;
      const unsigned long long m = __ballot(c);
      const int R = r + __popcll(m & ((1ull << lane) - 1ull));  // this lane's candidate's rank
      if (c && R % G == gw) s_list[wave][R / G] = lane + 64 * i;
      r += __popcll(m);
    }
    const int n = (r - gw + G - 1) / G;  // ranks = gw (mod G) below r
    // exact keys, two candidates per round trip (an odd last one is computed
    // twice and stored once)
#pragma unroll 1
    for (int q = 0; q < n; q += 2) {
      const int e0 = s_list[wave][q], e1 = s_list[wave][min(q + 1, n - 1)];
      const uint16_t* const w2[2] = {W + int64_t(e0) * D, W + int64_t(e1) * D};
      float lg[2];
      exact_logits<2>(xv, xr, w2, D, lane, lg);
      if (lane == 0) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int e = h ? e1 : e0;
          const float sc = score_of(lg[h], score_func);
          s_sx[grp][e] = sc;
          s_kx[grp][e] = bias ? sc + bias[e] : sc;
        }
      }
    }
    __syncthreads();
    if (gw != 0 || !live) return;
    float sx[kRSlots], kx[kRSlots];
#pragma unroll
    for (int i = 0; i < kRSlots; ++i) {
      const int e = lane + 64 * i;
      sx[i] = e < E ? s_sx[grp][e] : 0.0f;
      kx[i] = e < E ? s_kx[grp][e] : -INFINITY;
    }
    // top-k of the exact keys (ties -> lower index)
    taken = 0u;
    for (int j = 0; j < k; ++j) {
      Cand best = {-INFINITY, 0x7FFFFFFF};
#pragma unroll
      for (int i = 0; i < kRSlots; ++i) {
        const int e = lane + 64 * i;
        if (e < E && !((taken >> i) & 1u) && kx[i] != -INFINITY) best = cand_better(best, Cand{kx[i], e});
      }
      best = wave_argmax_dpp(best);
      const int bi = clampi(best.i, 0, E - 1);
      float sv = 0.0f;
#pragma unroll
      for (int i = 0; i < kRSlots; ++i) {
        const float v = __shfl(sx[i], bi & 63, kWave);
        if ((bi >> 6) == i) sv = v;
      }
      if (lane == j) {
        my_sel = bi;
        mine = sv;
      }
      if ((bi & 63) == lane) taken |= 1u << (bi >> 6);
    }
  }
  float tot = 0.0f;
  for (int j = 0; j < k; ++j) tot += __shfl(mine, j, kWave);  // slot order, fp32
  const float v = poison ? __builtin_nanf("") : mine / tot * route_scale;
  if (lane < k) {
    weights[int64_t(t) * k + lane] = v;
    idx[int64_t(t) * k + lane] = my_sel;
  }
}

int launch_prefill_gate(const wz_moe_desc* d, const MoeWs& w, const void* x, const int64_t* input_ids, int64_t T,
                        hipStream_t stream) {
  const int E = d->n_experts, D = d->dim;
  const uint16_t* xb = static_cast<const uint16_t*>(x);
  const uint16_t* gw = static_cast<const uint16_t*>(d->gate_w);
  if (!d->tid2eid) {
    // the 32 x 64 tiles need T >= 1024 to give every CU a workgroup; below,
    // the 16 x 16 tiles with K split over the waves
    if (T < 1024) {
      const int64_t tiles = ((T + 15) / 16) * ((E + 15) / 16);
      WZ_LAUNCH("moe_gate", stream, gate_mfma_ksplit_kernel, dim3(unsigned(tiles)), dim3(256), 0, xb, gw, w.scores,
                w.biased, int(T), E, D);
      if (int rc = check_launch("moe gate")) return rc;
    } else {
      const int64_t tiles = ((T + 31) / 32) * ((E + 63) / 64);
      WZ_LAUNCH("moe_gate", stream, gate_mfma_kernel, dim3(unsigned(tiles)), dim3(64 * kGateQ), 0, xb, gw,
                w.scores, w.biased, int(T), E, D);
      if (int rc = check_launch("moe gate")) return rc;
    }
  }
  const float* gb = d->tid2eid ? nullptr : d->gate_bias;
  // one token per workgroup below 1024 tokens (T = 128 / 512: route 48.6 /
  // 59.7 -> 36.9 / 48.2 us), four per workgroup above (more tokens in flight)
  const bool wide = T < 1024;
  const unsigned grid = unsigned(wide ? T : (T + kRefineWaves - 1) / kRefineWaves);
#define WZ_TOPK(KS, G)                                                                                     \
  WZ_LAUNCH("moe_topk", stream, (topk_refine_kernel<KS, G>), dim3(grid), dim3(kRefineWaves * 64), 0, xb, gw, \
            w.scores, w.biased, gb, d->tid2eid, input_ids, d->vocab, int(T), E, D, d->topk, d->score_func,     \
            d->route_scale, w.weights, w.idx)
  if (E <= 256) {
    if (wide)
      WZ_TOPK(4, kRefineWaves);
    else
      WZ_TOPK(4, 1);
  } else {
    if (wide)
      WZ_TOPK(kMaxExperts / 64, kRefineWaves);
    else
      WZ_TOPK(kMaxExperts / 64, 1);
  }
#undef WZ_TOPK
  return check_launch("moe topk");
}

// ------------------------------------------------------------ tile GEMMs ---

struct TileRows {
  int row0, nrows, e;
  bool keep;  // other M-tiles read the same weight tiles: keep them in L2
};

// Tile of the grid: routed tiles come from the M-tile table; dense tiles
// (the shared expert) are consecutive 128-row blocks of the T tokens.
__device__ __forceinline__ bool tile_of(const MoeWs& ws, int mt, bool dense, int T, int P, int E, TileRows& tr) {
  if (dense) {
    tr.row0 = mt * kPM;
    tr.nrows = min(kPM, T - tr.row0);
    tr.e = 0;
    tr.keep = T > kPM;
    return tr.nrows > 0;
  }
  if (mt >= ws.n_mt[0]) return false;
  const int u = clampi(ws.mt_u[mt], 0, E - 1);
  tr.e = clampi(ws.active[u], 0, E - 1);
  tr.keep = ws.act_cnt[u] > kPM;
  tr.row0 = clampi(ws.mt_row0[mt], 0, P);
  tr.nrows = clampi(ws.mt_n[mt], 0, min(kPM, P - tr.row0));
  return tr.nrows > 0;
}

// A K-step in LDS: 64 rows of 128 bytes, the 16-byte chunk q of row r at slot
// q ^ a_swz(r), so the 16 rows an A operand read touches (one chunk each) fall
// in distinct banks; the rows' scales at as_s[(r / 16) * 64 + r % 16].
__device__ __forceinline__ int a_swz(int row) { return (row >> 1) & 7; }

// The K pipeline's four A buffers (rows and their scales), each its own LDS
// array: the direct loads into them are the compiler's own buffer-to-LDS
// builtin, so it counts them among the outstanding loads and, the arrays being
// distinct objects, waits before a read of one buffer only for the loads into
// that one.  K-step kb lives in buffer kb % 4 (the K loop is unrolled by four,
// so every index is a constant).
constexpr int kNBuf = 4;
struct StageBufs {
  uint8_t* a[kNBuf];
  float* s[kNBuf];
};
typedef __attribute__((address_space(3))) void lds_void;
// declares the four buffers (distinct LDS arrays) and a StageBufs L over them
#define WZ_STAGE_BUFS(L)                                                                          \
  __shared__ __align__(1024) uint8_t L##_a0[kPM * 128], L##_a1[kPM * 128], L##_a2[kPM * 128],      \
      L##_a3[kPM * 128];                                                                          \
  __shared__ __align__(16) float L##_s0[256], L##_s1[256], L##_s2[256], L##_s3[256];               \
  const StageBufs L = {{L##_a0, L##_a1, L##_a2, L##_a3}, {L##_s0, L##_s1, L##_s2, L##_s3}}

__device__ __forceinline__ AOp a_from_lds(const uint8_t* a_s, const float* as_s, int row, int g, bool pow2) {
  AOp a;
  const uint8_t* p = a_s + row * 128;
  const int sw = a_swz(row);
  const v4i lo = *reinterpret_cast<const v4i*>(p + ((g ^ sw) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(p + (((g + 4) ^ sw) << 4));
  a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  const float s = as_s[(row >> 4) * 64 + (row & 15)];
  a.sf = s;
  a.se8 = pow2 ? int((__float_as_uint(s) >> 23) & 0xFFu) : kE8m0One;
  return a;
}

// B operands of one K-block for the NT weight tiles a wave owns (fp4: lo only).
// The MXFP4 scale stays the raw packed dword until the MFMA needs its byte:
// extracting it at fetch time would make the fetch wait for its own loads.
template <int NT>
struct BTiles {
  v4i lo[NT], hi[NT];
  uint32_t sw[NT];  // fp4: packed e8m0 dword (byte kb & 3); fp8: the e8m0 byte
  float f[NT];
};

// Expert-grouped tile GEMM over one M-tile (<= 64 rows) and one N-block.
//   MODE 0: routed w1/w3 (packed MXFP4) over gathered x rows -> SwiGLU -> h
//   MODE 1: shared w1/w3 (packed FP8) over token rows        -> SwiGLU -> sh_h
//   MODE 2: routed w2 (packed MXFP4) over h rows             -> out2
//   MODE 3: shared w2 (packed FP8) over shared h rows        -> sh_out
//   MODE 4: a dense MXFP4 linear (w2's tile format, one "expert") over rows
//           in order                                         -> sh_out
// A wave owns NTW weight tiles of 16 output columns (routed w13: 4, i.e. 2
// feature tiles x {w1, w3}; routed w2: 2 column tiles; shared FP8 tiles are
// twice the bytes, so 2), and one A operand read from LDS feeds NTW MFMAs.
// The K loop is software-pipelined three K-steps deep: while step kb
// computes, the B tiles (registers) and the A rows (LDS, direct buffer loads
// that need no registers) of steps kb+1 .. kb+3 are in flight; A goes through
// the four StageBufs buffers and B through four register sets, with one
// barrier per step.
//
// CHAIN: activation and weight scales are both powers of two, so they ride in
// the MFMA's e8m0 scale operands and the accumulators chain over K; otherwise
// each K-block partial is scaled on the VALU (mma_step).  KEEP: the weight
// tiles are read by other M-tiles too (an expert with more than one M-tile,
// the shared expert over several), so they are loaded as ordinary cached
// loads; otherwise non-temporal, as a single-use stream that should not evict
// the activation rows the N-blocks of an M-tile share.
template <int MODE, bool CHAIN, int NM, bool KEEP>
__device__ __forceinline__ void gemm_tile_body(const wz_moe_desc& d, const MoeWs& ws, int T, const TileRows& tr,
                                               int nt, const StageBufs& L, float (*am_s)[kPM]) {
  // DENSE: FP8 weights (the shared expert, an FP8 linear); DROWS: rows in
  // token order (no M-tile table)
  constexpr bool W13 = MODE < 2, DENSE = MODE == 1 || MODE == 3, DROWS = DENSE || MODE == 4;
  constexpr int WF = DENSE ? kFmtFp8 : kFmtFp4;
  // weight tiles per wave: routed w1/w3 4 (2 feature tiles x {w1, w3}); routed
  // w2 2 (4 spilled registers at two workgroups per CU and measured 7 % slower);
  // FP8 shared tiles, twice the bytes, 2
  constexpr int NTW = ntw_of(MODE);
  // vector loads every K-step issues for certain: NTW weight tiles (fp4: a
  // tile and its scale dword; FP8: two halves, the block scale possibly a
  // scalar load) and the three direct A loads
  constexpr int kStepLoads = 2 * NTW + 3;
  constexpr int CPW = W13 ? NTW / 2 : NTW;    // 16-column output tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, k = d.topk, P = T * k;
  const int K = W13 ? D : I, KB = K / 128, KG = (KB + 3) / 4;
  const int NCT = (W13 ? I : D) / 16;  // 16-column tiles of the output
  const bool a_pow2 = CHAIN || d.act_scale_kind != WZ_SCALE_F32;
  const bool bp = CHAIN || !DENSE || d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int row0 = tr.row0, nrows = tr.nrows, e = tr.e;
  const int ct0 = (nt * 4 + wave) * CPW;  // first column tile of this wave

  // weight tile j of this wave: column tile ct(j), w1/w3 selector which(j).
  // Every load of the K loop is unconditional (tiles past the last column
  // re-read the last one; rows past nrows re-read the last row), so the
  // compiler can count outstanding loads exactly and keep the prefetches in
  // flight across the barriers; only the epilogue looks at validity.
  int ct[NTW], cl[NTW], which[NTW];
  bool jv[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    ct[j] = W13 ? ct0 + (j >> 1) : ct0 + j;
    cl[j] = min(ct[j], NCT - 1);
    which[j] = W13 ? (j & 1) : 0;
    jv[j] = ct[j] < NCT;
  }

  // A staging: wave w brings rows 16w .. 16w + 15 of a K-step into LDS with
  // two 1-KB direct loads (lane l: row 16w + 8i + l / 8, slot l % 8, which
  // holds the row's chunk (l % 8) ^ a_swz(row)) and their scales with one
  // 4-byte load (lane l: row 16w + l % 16).  Rows past nrows repeat the last
  // row (their outputs are dropped).  A wave whose 16 rows are all past nrows
  // issues its loads against an empty buffer range: they return without
  // touching memory, and every wave issues the same loads (no branch).
  auto src_of = [&](int r) {
    const int rr = min(r, nrows - 1);
    if (MODE == 0) return clampi(ws.perm_token[row0 + rr], 0, T - 1);
    if (MODE == 3) return P + row0 + rr;
    return row0 + rr;
  };
  const bool a_rows = 16 * wave < nrows;
  uint32_t avo[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 16 * wave + 8 * i + (lane >> 3);
    avo[i] = uint32_t(src_of(row)) * uint32_t(K) + uint32_t(((lane & 7) ^ a_swz(row)) << 4);
  }
  const uint32_t svo = uint32_t(src_of(16 * wave + (lane & 15))) * uint32_t(KB) * 4u;
  const int64_t a_nrows = W13 ? T : P + T;  // rows of xq / hq
  const __amdgpu_buffer_rsrc_t a_rs = __builtin_amdgcn_make_buffer_rsrc(
      W13 ? ws.xq : ws.hq, short(0), a_rows ? int(a_nrows * K) : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t s_rs = __builtin_amdgcn_make_buffer_rsrc(
      W13 ? ws.xs : ws.hs, short(0), a_rows ? int(a_nrows * KB * 4) : 0, 0x00020000);
  // K-step kb into buffer buf (a constant wherever it is called)
  auto a_issue = [&](int kb, int buf) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_rs, (lds_void*)(L.a[buf] + (2 * wave + i) * 1024), 16, int(avo[i]),
                                               kb * 128, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(s_rs, (lds_void*)(L.s[buf] + wave * 64), 4, int(svo), kb * 4, 0, 0);
  };

  auto wload = [](const uint8_t* p) { return KEEP ? load16(p) : load16_nt(p); };
  auto b_fetch = [&](BTiles<NTW>& b, int kb) {
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      if (MODE == 0) {
        const int64_t t = int64_t(e) * NCT + cl[j];
        const uint8_t* w = static_cast<const uint8_t*>(d.w13p) + ((t * KB + kb) * 2 + which[j]) * 1024;
        b.lo[j] = wload(w + lane * 16);
        const uint32_t* sw = static_cast<const uint32_t*>(d.w13p_s) + ((t * KG + (kb >> 2)) * 2 + which[j]) * 64;
        b.sw[j] = sw[lane];
        b.f[j] = 1.0f;
      } else if (MODE == 2 || MODE == 4) {
        const int64_t t = int64_t(e) * NCT + cl[j];
        const uint8_t* w = static_cast<const uint8_t*>(d.w2p) + (t * KB + kb) * 1024;
        b.lo[j] = wload(w + lane * 16);
        const uint32_t* sw = static_cast<const uint32_t*>(d.w2p_s) + (t * KG + (kb >> 2)) * 64;
        b.sw[j] = sw[lane];
        b.f[j] = 1.0f;
      } else {
        const uint8_t* w;
        const void* s;
        if (MODE == 1) {
          w = static_cast<const uint8_t*>(d.sh13p) + ((int64_t(cl[j]) * KB + kb) * 2 + which[j]) * 2048;
          s = which[j] ? d.sh_w3_s : d.sh_w1_s;
        } else {
          w = static_cast<const uint8_t*>(d.sh2p) + (int64_t(cl[j]) * KB + kb) * 2048;
          s = d.sh_w2_s;
        }
        b.lo[j] = wload(w + lane * 16);
        b.hi[j] = wload(w + 1024 + lane * 16);
        const int64_t si = int64_t(cl[j] >> 3) * KB + kb;
        if (CHAIN) {
          b.sw[j] = static_cast<const uint8_t*>(s)[si];
          b.f[j] = 1.0f;
        } else {
          int se8;
          fp8_wscale(s, si, d.shared_w_scale_kind, se8, b.f[j]);
          b.sw[j] = uint32_t(se8);
        }
      }
    }
  };

  // routed w1/w3: the routing weight of each of this lane's output rows,
  // requested now so the epilogue does not wait on three dependent loads
  float wts[NM][4];
#pragma unroll
  for (int m = 0; m < NM; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      wts[m][i] = 0.0f;
      if (MODE == 0) {
        const int p = row0 + min(m * 16 + g * 4 + i, nrows - 1);
        wts[m][i] = ws.weights[int64_t(clampi(ws.perm_token[p], 0, T - 1)) * k + clampi(ws.perm_slot[p], 0, k - 1)];
      }
    }
  v4f acc[NTW][NM];
#pragma unroll
  for (int j = 0; j < NTW; ++j)
#pragma unroll
    for (int m = 0; m < NM; ++m) acc[j][m] = v4f{0.f, 0.f, 0.f, 0.f};

  // K-step kb from buffer / register set buf = kb % 4
  // (fp4 weights: the scale is byte buf of the packed dword, which the chained
  // MFMA selects itself)
  auto compute = [&](int buf, const BTiles<NTW>& b) {
    int e8[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) e8[j] = DENSE || CHAIN ? int(b.sw[j]) : int((b.sw[j] >> (8 * buf)) & 0xFFu);
    const int bsel = DENSE ? 0 : buf;
#pragma unroll
    for (int m = 0; m < NM; ++m) {
      const AOp a = a_from_lds(L.a[buf], L.s[buf], m * 16 + nl, g, CHAIN || a_pow2);
#pragma unroll
      for (int j = 0; j < NTW; ++j) {
        const v8i bv = DENSE ? v8i{b.lo[j][0], b.lo[j][1], b.lo[j][2], b.lo[j][3], b.hi[j][0], b.hi[j][1],
                                   b.hi[j][2], b.hi[j][3]}
                             : v8i{b.lo[j][0], b.lo[j][1], b.lo[j][2], b.lo[j][3], 0, 0, 0, 0};
        if (CHAIN) {
          if (bsel == 0)
            acc[j][m] = mfma_scaled_bsel<kFmtFp8, WF, 0>(a.v, bv, acc[j][m], a.se8, e8[j]);
          else if (bsel == 1)
            acc[j][m] = mfma_scaled_bsel<kFmtFp8, WF, 1>(a.v, bv, acc[j][m], a.se8, e8[j]);
          else if (bsel == 2)
            acc[j][m] = mfma_scaled_bsel<kFmtFp8, WF, 2>(a.v, bv, acc[j][m], a.se8, e8[j]);
          else
            acc[j][m] = mfma_scaled_bsel<kFmtFp8, WF, 3>(a.v, bv, acc[j][m], a.se8, e8[j]);
        } else
          mma_step<kFmtFp8, WF>(acc[j][m], a, bv, e8[j], b.f[j], a_pow2, bp, lane);
      }
    }
  };

  // Step kb (set / buffer i = kb % 4): wait until at most the loads of the
  // (up to two) later K-steps already requested are outstanding -- loads
  // complete in order, so B(kb) and this wave's rows of A(kb) have landed --
  // then a barrier (every wave's rows of A(kb) are in LDS, and every wave has
  // finished step kb - 1, whose buffer and register set are free), request
  // K-step kb + 3 into them, and compute step kb.  The wait is the explicit
  // one: the compiler's own waits for B(kb) and A(kb) come after the barrier.
  // kStepLoads is a lower bound of each step's loads, so the count never
  // lets one of step kb's loads still be outstanding.
  // (lgkmcnt(0) too: this wave's LDS reads of step kb - 1 have returned
  // before any wave may overwrite that buffer)
  auto step_wait = [&](int ahead) {  // ahead: later K-steps requested (0..2)
    __builtin_amdgcn_sched_barrier(0);
    if (ahead >= 2)
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(2 * kStepLoads));
    else if (ahead == 1)
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(kStepLoads));
    else
      __builtin_amdgcn_s_waitcnt(vmcnt_lgkm0(0));
    asm volatile("s_barrier" : : : "memory");
  };
  // the first three steps' loads, unconditionally (K-steps past the end
  // repeat the last one; nothing reads them): a load behind a branch would
  // leave the compiler unsure how many loads follow B(0) at the loop head, and
  // it would drain them all there.  The fence after each step's loads keeps
  // the compiler from merging the repeated fp4 scale-dword loads of steps 0..2
  // (one dword holds four K-blocks' scales): every step then issues its
  // kStepLoads, as the explicit waits count, and the loop head sees the same
  // outstanding loads on entry as from the loop's own end.
  BTiles<NTW> bt[kNBuf];
#pragma unroll
  for (int j = 0; j < kNBuf - 1; ++j) {
    b_fetch(bt[j], min(j, KB - 1));
    a_issue(min(j, KB - 1), j);
    asm volatile("" : : : "memory");
  }
  int kb = 0;
  // steady state: every step refills (its K-step + 3 is in range)
  for (; kb + 7 <= KB; kb += kNBuf) {
#pragma unroll
    for (int i = 0; i < kNBuf; ++i) {
      step_wait(2);
      b_fetch(bt[(i + 3) & 3], kb + i + 3);
      a_issue(kb + i + 3, (i + 3) & 3);
      __builtin_amdgcn_sched_barrier(0);
      compute(i, bt[i]);
    }
  }
  // last K-steps (kb is a multiple of four)
  for (; kb < KB; kb += kNBuf) {
#pragma unroll
    for (int i = 0; i < kNBuf; ++i) {
      const int s = kb + i;
      if (s >= KB) break;
      step_wait(min(KB - 1 - s, 2));
      if (s + 3 < KB) {
        b_fetch(bt[(i + 3) & 3], s + 3);
        a_issue(s + 3, (i + 3) & 3);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(i, bt[i]);
    }
  }

  // epilogue
  if (W13) {
    // h = SwiGLU (the routed rows times their routing weight), rounded to
    // bf16 as the expert's intermediate is (architecture.py:739-741)
    float hb[CPW][NM][4];
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      const int f = ct[2 * q] * 16 + nl;
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m * 16 + g * 4 + i;
          hb[q][m][i] = 0.0f;
          if (jv[2 * q] && r < nrows) {
            float gv = bf16_round(acc[2 * q][m][i]), uv = bf16_round(acc[2 * q + 1][m][i]);
            if (d.swiglu_limit > 0.0f) {
              uv = clamp_keep_nan(uv, -d.swiglu_limit, d.swiglu_limit);
              gv = gv > d.swiglu_limit ? d.swiglu_limit : gv;
            }
            const float hv = silu_f32(gv) * uv;
            if (DENSE) {
              ws.sh_h[int64_t(row0 + r) * I + f] = f32_to_bf16(hv);
            } else {
              hb[q][m][i] = bf16_round(wts[m][i] * hv);
            }
          }
        }
    }
    if (!DENSE) {
      // act_quant of the routed h rows (torch_ops.py:33-49, the arithmetic of
      // act_quant_kernel): this workgroup's 128 features [128 nt, +128) are
      // exactly one quantisation block, so a row's amax is this lane's two
      // features, then its 16 lanes, then the 4 waves through LDS; codes go
      // to hq and the block scale to hs (no bf16 h and no hquant launch).
      float am[NM][4];
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float v = 0.0f;
#pragma unroll
          for (int q = 0; q < CPW; ++q) v = absmax(v, hb[q][m][i]);
          v = wave_absmax_xor(v, 1);
          v = wave_absmax_xor(v, 2);
          v = wave_absmax_xor(v, 4);
          v = wave_absmax_xor(v, 8);
          am[m][i] = v;
          if (nl == 0) am_s[wave][m * 16 + g * 4 + i] = v;
        }
      __syncthreads();
      const int KBh = I / 128;
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m * 16 + g * 4 + i;
          float amax = am[m][i];
#pragma unroll
          for (int w = 0; w < 4; ++w) amax = absmax(amax, am_s[w][r]);
          const ActScale sc = act_scale(amax, a_pow2);
          if (r < nrows) {
            const int64_t p = row0 + r;
#pragma unroll
            for (int q = 0; q < CPW; ++q) {
              if (!jv[2 * q]) continue;
              const uint32_t b = uint32_t(__builtin_amdgcn_cvt_pk_fp8_f32(quant_div(hb[q][m][i], sc, a_pow2), 0.0f, 0, false));
              ws.hq[p * I + ct[2 * q] * 16 + nl] = uint8_t(b & 0xFFu);
            }
            if (wave == 0 && nl == 0) ws.hs[p * KBh + nt] = sc.s;
          }
        }
    }
  } else {
    uint16_t* out = DROWS ? ws.sh_out : ws.out2;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      if (!jv[j]) continue;
      const int c = ct[j] * 16 + nl;
#pragma unroll
      for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m * 16 + g * 4 + i;
          if (r < nrows) out[int64_t(row0 + r) * D + c] = f32_to_bf16(acc[j][m][i]);
        }
    }
  }
}

// Tile dispatch on its height: the body is compiled for 1, 2 or 4 row
// tiles of 16, so its MFMA loops carry no row branches.
template <int MODE, bool CHAIN>
__device__ __forceinline__ void gemm_tile(const wz_moe_desc& d, const MoeWs& ws, int T, int mt, int nt,
                                          const StageBufs& L, float (*am_s)[kPM]) {
  TileRows tr;
  if (!tile_of(ws, mt, MODE == 1 || MODE == 3 || MODE == 4, T, T * d.topk, d.n_experts, tr)) return;
  static_assert(kPM == 64, "tile heights up to 4 row tiles");
  if (tr.keep) {
    if (tr.nrows <= 16)
      gemm_tile_body<MODE, CHAIN, 1, true>(d, ws, T, tr, nt, L, am_s);
    else if (tr.nrows <= 32)
      gemm_tile_body<MODE, CHAIN, 2, true>(d, ws, T, tr, nt, L, am_s);
    else
      gemm_tile_body<MODE, CHAIN, 4, true>(d, ws, T, tr, nt, L, am_s);
  } else {
    if (tr.nrows <= 16)
      gemm_tile_body<MODE, CHAIN, 1, false>(d, ws, T, tr, nt, L, am_s);
    else if (tr.nrows <= 32)
      gemm_tile_body<MODE, CHAIN, 2, false>(d, ws, T, tr, nt, L, am_s);
    else
      gemm_tile_body<MODE, CHAIN, 4, false>(d, ws, T, tr, nt, L, am_s);
  }
}

// The routed blocks [d0, d0 + n) run through xcd_runs (common.h): each XCD takes
// runs of 64 consecutive (M-tile, N-block) pairs, so an M-tile's N-blocks share
// its gathered activation rows in one L2 and the M-tiles of a group read the same
// weight tiles there; the many runs of a hot expert spread over every XCD (one
// XCD had held all 368 blocks of the hottest expert of a T = 2048 batch and
// ended 25 % after the first).

// (M-tile, N-block) of routed block r, r < n_mt * nblk: groups of gm M-tiles
// take their N-blocks in parts of gn.  A window of consecutive blocks (the
// workgroups resident on one XCD, 64) then covers gm M-tiles x (64 / gm)
// N-blocks: an N-block's weight tiles come from beyond L2 once per gm M-tiles
// and an M-tile's rows once per nblk / gn parts.  gm = 1, gn = nblk is M-tile
// major (an M-tile's rows fetched once; right when experts hold one or two
// M-tiles); gm = gn = 8 suits hot experts with many M-tiles (their weights came
// once per 4 M-tiles in M-tile-major order).  A bijection on [0, n_mt * nblk):
// the last group holds n_mt % gm M-tiles and the last part nblk % gn N-blocks.
__device__ __forceinline__ void tile_order(int r, int n_mt, int nblk, int gm, int gn, int& mt, int& nt) {
  const int full = n_mt / gm, per = gm * nblk;
  const int q = r / per, rr = r % per;
  const int h = q < full ? gm : n_mt - full * gm;  // M-tiles in this group
  // only the last part can be narrower, so part p starts at p * gn * h
  const int part = rr / (gn * h), i = rr % (gn * h);
  mt = q * gm + i % h;
  nt = part * gn + i / h;
}

// One launch serves the shared expert's dense tiles (block ids first, so the
// few long-running shared tiles start early) and the routed experts' M-tiles.
// W13 selects w1/w3 + SwiGLU or w2; CR / CS: scale chaining of routed / shared.
template <bool W13, bool CR, bool CS>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2))) void prefill_gemm_kernel(
    wz_moe_desc d, MoeWs ws, int T, int nblk, int nblk_dense, int dense_blocks, int gm, int gn) {
  WZ_STAGE_BUFS(L);
  __shared__ float am_s[4][kPM];  // w1/w3 epilogue: each wave's row amax of its features
  const int b = blockIdx.x;
  if (b < dense_blocks) {
    gemm_tile<W13 ? 1 : 3, CS>(d, ws, T, b / nblk_dense, b % nblk_dense, L, am_s);
  } else {
    const int n = ws.n_mt[0] * nblk;  // routed blocks with work
    if (b - dense_blocks >= n) return;
    const int r = xcd_runs(b, dense_blocks, n);
    int mt, nt;
    tile_order(r, ws.n_mt[0], nblk, gm, gn, mt, nt);
    gemm_tile<W13 ? 0 : 2, CR>(d, ws, T, mt, nt, L, am_s);
  }
}

// A dense MXFP4 linear in tiles: block b = (M-tile b / nblk, N-block b % nblk).
// CHAIN: power-of-two activation scales (they ride in the MFMA with the e8m0
// weight scales).
template <bool CHAIN>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2))) void dense_fp4_kernel(
    wz_moe_desc d, MoeWs ws, int M, int nblk) {
  WZ_STAGE_BUFS(L);
  __shared__ float am_s[4][kPM];
  gemm_tile<4, CHAIN>(d, ws, M, int(blockIdx.x) / nblk, int(blockIdx.x) % nblk, L, am_s);
}

int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream);

// M-tiles a grid must cover: sum over experts of ceil(c/128) <= P/128 + active experts.
static inline int64_t prefill_mt_max(int64_t P, int E) { return P / kPM + (P < E ? P : E) + 1; }

// only < 0: every expert stage; otherwise the one stage WZ_STAGE_* (profiling replays).
int launch_prefill_experts(const wz_moe_desc* d, const MoeWs& w, const void* x, int64_t T, hipStream_t stream,
                           int only) {
  const int E = d->n_experts, k = d->topk, D = d->dim, I = d->inter;
  const int64_t P = T * k;
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe prefill: packed banks missing (call wz_moe_pack)");
  const int qkind = d->act_scale_kind == WZ_SCALE_F32 ? WZ_SCALE_F32 : WZ_SCALE_UE8M0_F32;
  const int64_t mt_max = prefill_mt_max(P, E), mt_dense = (T + kPM - 1) / kPM;
  if (only < 0 || only == WZ_STAGE_ROUTE) {
    if (int rc = launch_act_quant(x, T, D, w.xq, w.xs, qkind, stream)) return rc;
  }
  // column tiles of 16 per WG: routed w1/w3 4 waves x 2 feature tiles, routed w2
  // and the shared tiles 4 waves x 2
  const int nb13 = (I / 16 + 7) / 8, nb13d = (I / 16 + 3) / 4;
  const int nb2 = (D / 16 + 4 * ntw_of(2) - 1) / (4 * ntw_of(2)), nb2d = (D / 16 + 7) / 8;
  const bool cr = d->act_scale_kind != WZ_SCALE_F32;
  const bool cs = cr && d->shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int Ti = int(T), dn13 = int(mt_dense * nb13d), dn2 = int(mt_dense * nb2d);
  const dim3 blk(kPThreads), g13(unsigned(dn13 + mt_max * nb13)), g2(unsigned(dn2 + mt_max * nb2));
  // routed block order (tile_order): 8 M-tiles x 8 N-blocks per group at T >= 1024,
  // where skewed batches give hot experts many M-tiles (T = 2048, calibrated skew:
  // 1327 -> 1250 us per layer); M-tile major below (T = 128: 341 vs 367 us)
  const bool grouped = T >= 1024;
  const int gm = grouped ? 8 : 1, gn13 = grouped ? 8 : nb13, gn2 = grouped ? 8 : nb2;
  if (only < 0 || only == WZ_STAGE_W13) {
    if (cr && cs) {
      WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, true, true>), g13, blk, 0, *d, w, Ti, nb13, nb13d, dn13, gm, gn13);
    } else if (cr) {
      WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, true, false>), g13, blk, 0, *d, w, Ti, nb13, nb13d, dn13, gm, gn13);
    } else {
      WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, false, false>), g13, blk, 0, *d, w, Ti, nb13, nb13d,
                dn13, gm, gn13);
    }
    if (int rc = check_launch("moe w13")) return rc;
  }
  // the routed h rows are quantised in the w1/w3 epilogue; the shared rows here
  if (only < 0 || only == WZ_STAGE_HQUANT) {
    if (int rc = launch_act_quant(w.sh_h, T, I, w.hq + P * I, w.hs + P * (I / 128), qkind, stream)) return rc;
  }
  if (only < 0 || only == WZ_STAGE_W2) {
    if (cr && cs) {
      WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, true, true>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2, gm, gn2);
    } else if (cr) {
      WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, true, false>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2, gm, gn2);
    } else {
      WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, false, false>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2, gm, gn2);
    }
    if (int rc = check_launch("moe w2")) return rc;
  }
  return WZ_OK;
}

// Dense FP8 GEMM y[M, N] (bf16) = xq[M, K] . W^T for a linear whose weight is
// in the packed tile format (launch_pack_fp8): the shared-expert w2 tile path
// (MODE 3) with the linear's dimensions, M-tiles of up to 64 rows staged in
// LDS, 8 column tiles per workgroup.
int launch_dense_fp8(const uint8_t* wp, const void* w_s, int w_kind, const uint8_t* xq, const float* xs,
                     bool a_pow2, uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  wz_moe_desc d = {};
  d.dim = int(N);
  d.inter = int(K);
  d.n_experts = 1;
  d.topk = 0;
  d.act_scale_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  d.shared_w_scale_kind = w_kind;
  d.sh2p = wp;
  d.sh_w2_s = w_s;
  MoeWs w = {};
  w.hq = const_cast<uint8_t*>(xq);
  w.hs = const_cast<float*>(xs);
  w.sh_out = y;
  if (M * K >= (int64_t(1) << 31)) return set_error(WZ_EINVAL, "fp8_linear: M * K must be below 2^31");
  const int nb2d = int((N / 16 + 7) / 8);
  const int dense = int((M + kPM - 1) / kPM) * nb2d;
  const bool cs = a_pow2 && w_kind == WZ_WSCALE_E8M0;
  const dim3 grid{unsigned(dense)}, blk{unsigned(kPThreads)};
  if (cs) {
    WZ_LAUNCH("fp8_linear", stream, (prefill_gemm_kernel<false, true, true>), grid, blk, 0, d, w, int(M), 1, nb2d,
              dense, 1, 1);
  } else if (a_pow2) {
    WZ_LAUNCH("fp8_linear", stream, (prefill_gemm_kernel<false, true, false>), grid, blk, 0, d, w, int(M), 1, nb2d,
              dense, 1, 1);
  } else {
    WZ_LAUNCH("fp8_linear", stream, (prefill_gemm_kernel<false, false, false>), grid, blk, 0, d, w, int(M), 1,
              nb2d, dense, 1, 1);
  }
  return check_launch("fp8_linear dense");
}

// Dense MXFP4 GEMM y[M, N] (bf16) = xq[M, K] . W^T for a weight packed by
// wz_fp4_pack (the routed w2 tile format of one expert: 16-row x 128-K tiles of
// e2m1, [N/16][K/128][1 KB], and its e8m0 scales packed four K-blocks to a
// dword, [N/16][ceil(K/512)][64]); M-tiles of up to 64 rows staged in LDS,
// 8 column tiles per workgroup.
int launch_dense_fp4(const uint8_t* wp, const uint32_t* wp_s, const uint8_t* xq, const float* xs, bool a_pow2,
                     uint16_t* y, int64_t M, int64_t N, int64_t K, hipStream_t stream) {
  if (M * K >= (int64_t(1) << 31)) return set_error(WZ_EINVAL, "fp4_gemm_packed: M * K must be below 2^31");
  wz_moe_desc d = {};
  d.dim = int(N);
  d.inter = int(K);
  d.n_experts = 1;
  d.topk = 0;
  d.act_scale_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  d.w2p = wp;
  d.w2p_s = wp_s;
  MoeWs w = {};
  w.hq = const_cast<uint8_t*>(xq);
  w.hs = const_cast<float*>(xs);
  w.sh_out = y;
  const int nblk = int((N / 16 + 4 * ntw_of(4) - 1) / (4 * ntw_of(4)));
  const int blocks = int((M + kPM - 1) / kPM) * nblk;
  const dim3 grid{unsigned(blocks)}, blk{unsigned(kPThreads)};
  if (a_pow2) {
    WZ_LAUNCH("fp4_gemm_packed", stream, dense_fp4_kernel<true>, grid, blk, 0, d, w, int(M), nblk);
  } else {
    WZ_LAUNCH("fp4_gemm_packed", stream, dense_fp4_kernel<false>, grid, blk, 0, d, w, int(M), nblk);
  }
  return check_launch("fp4_gemm_packed");
}

}  // namespace wz
