// MoE prefill path (T > 16 tokens): expert-grouped MFMA GEMMs over the
// canonical (expert, token, slot) pair order produced by the routing kernels.
//
//   mtile     each active expert's pair rows cut into tiles of 128 rows.
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

constexpr int kPM = 128;          // pair rows per M-tile
constexpr int kPThreads = 256;    // 4 waves, 16 features (or columns) each
constexpr int kARow = 144;        // LDS row stride of the staged A tile (bytes)

// ----------------------------------------------------------- M-tile table ---

// One workgroup: cut each active expert's pair rows into tiles of kPM.
__global__ __launch_bounds__(1024) void mtile_kernel(MoeWs ws, int E, int P, int mt_cap) {
  __shared__ int wsum[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_act = min(ws.n_active[0], E);
  const int c = tid < n_act ? clampi(ws.act_cnt[tid], 0, P) : 0;
  const int nt = (c + kPM - 1) / kPM;
  int inc = nt;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  int base = 0;
  for (int w = 0; w < wave; ++w) base += wsum[w];
  const int first = base + inc - nt;
  const int row0 = tid < n_act ? ws.act_off[tid] : 0;
  for (int i = 0; i < nt && first + i < mt_cap; ++i) {
    ws.mt_u[first + i] = tid;
    ws.mt_row0[first + i] = row0 + i * kPM;
    ws.mt_n[first + i] = min(kPM, c - i * kPM);
  }
  if (tid == 1023) ws.n_mt[0] = min(base + inc, mt_cap);
}

// ------------------------------------------------------------ tile GEMMs ---

struct TileRows {
  int row0, nrows, e;
};

// Tile of the grid: routed tiles come from the M-tile table; dense tiles
// (the shared expert) are consecutive 128-row blocks of the T tokens.
__device__ __forceinline__ bool tile_of(const MoeWs& ws, int mt, bool dense, int T, int P, int E, TileRows& tr) {
  if (dense) {
    tr.row0 = mt * kPM;
    tr.nrows = min(kPM, T - tr.row0);
    tr.e = 0;
    return tr.nrows > 0;
  }
  if (mt >= ws.n_mt[0]) return false;
  const int u = clampi(ws.mt_u[mt], 0, E - 1);
  tr.e = clampi(ws.active[u], 0, E - 1);
  tr.row0 = clampi(ws.mt_row0[mt], 0, P);
  tr.nrows = clampi(ws.mt_n[mt], 0, min(kPM, P - tr.row0));
  return tr.nrows > 0;
}

// Stage one 128-row x 128-K fp8 A tile (+ its block scales) into LDS.
// src_row(r) gives the source row of tile row r (or -1 for a zero row).
template <typename RowFn>
__device__ __forceinline__ void stage_a(uint8_t* a_s, float* as_s, const uint8_t* A, const float* As, int K, int kb,
                                        int nrows, RowFn src_row) {
  const int tid = threadIdx.x;
  const int r = tid >> 1, h = tid & 1;
  const int sr = r < nrows ? src_row(r) : -1;
  v4i v[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
  if (sr >= 0) {
    const uint8_t* p = A + int64_t(sr) * K + kb * 128 + h * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = load16(p + 16 * i);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(a_s + r * kARow + h * 64 + 16 * i) = v[i];
  if (h == 0) as_s[r] = sr >= 0 ? As[int64_t(sr) * (K / 128) + kb] : 1.0f;
}

__device__ __forceinline__ AOp a_from_lds(const uint8_t* a_s, const float* as_s, int row, int g, bool pow2) {
  AOp a;
  const uint8_t* p = a_s + row * kARow + g * 16;
  const v4i lo = *reinterpret_cast<const v4i*>(p), hi = *reinterpret_cast<const v4i*>(p + 64);
  a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  const float s = as_s[row];
  a.sf = s;
  a.se8 = pow2 ? int((__float_as_uint(s) >> 23) & 0xFFu) : kE8m0One;
  return a;
}

// w1/w3 + SwiGLU.  WF = kFmtFp4: routed experts (packed MXFP4 bank);
// WF = kFmtFp8: the shared expert over the T token rows (DENSE).
template <int WF>
__global__ __launch_bounds__(kPThreads) void prefill_w13_kernel(wz_moe_desc d, MoeWs ws, int T) {
  __shared__ __align__(16) uint8_t a_s[kPM * kARow];
  __shared__ float as_s[kPM];
  constexpr bool DENSE = WF == kFmtFp8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts, k = d.topk, P = T * k;
  const int KB = D / 128, KG = (KB + 3) / 4, FT = I / 16, NT = I / 64;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int mt = blockIdx.x / NT, nt = blockIdx.x % NT;
  TileRows tr;
  if (!tile_of(ws, mt, DENSE, T, P, E, tr)) return;
  const int ft = nt * 4 + wave, f0 = ft * 16;
  v4f acc[2][8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[0][m] = acc[1][m] = v4f{0.f, 0.f, 0.f, 0.f};
  const uint8_t* wt;
  const uint32_t* st = nullptr;
  if (DENSE) {
    wt = static_cast<const uint8_t*>(d.sh13p) + int64_t(ft) * KB * 4096;
  } else {
    wt = static_cast<const uint8_t*>(d.w13p) + (int64_t(tr.e) * FT + ft) * KB * 2048;
    st = static_cast<const uint32_t*>(d.w13p_s) + (int64_t(tr.e) * FT + ft) * KG * 2 * 64 + lane;
  }
  const bool bp = !DENSE || d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int64_t sbase = int64_t(f0 >> 7) * KB;
  const int32_t* ptok = ws.perm_token;
  const int row0 = tr.row0;
  for (int kb = 0; kb < KB; ++kb) {
    __syncthreads();
    stage_a(a_s, as_s, ws.xq, ws.xs, D, kb, tr.nrows,
            [&](int r) { return DENSE ? row0 + r : clampi(ptok[row0 + r], 0, T - 1); });
    v8i b1, b3;
    int e1, e3;
    float f1 = 1.0f, f3 = 1.0f;
    if (DENSE) {
      const uint8_t* tp = wt + int64_t(kb) * 4096;
      const v4i l1 = load16_nt(tp + lane * 16), h1 = load16_nt(tp + 1024 + lane * 16);
      const v4i l3 = load16_nt(tp + 2048 + lane * 16), h3 = load16_nt(tp + 3072 + lane * 16);
      b1 = v8i{l1[0], l1[1], l1[2], l1[3], h1[0], h1[1], h1[2], h1[3]};
      b3 = v8i{l3[0], l3[1], l3[2], l3[3], h3[0], h3[1], h3[2], h3[3]};
      fp8_wscale(d.sh_w1_s, sbase + kb, d.shared_w_scale_kind, e1, f1);
      fp8_wscale(d.sh_w3_s, sbase + kb, d.shared_w_scale_kind, e3, f3);
    } else {
      const uint8_t* tp = wt + int64_t(kb) * 2048;
      const v4i x1 = load16_nt(tp + lane * 16), x3 = load16_nt(tp + 1024 + lane * 16);
      b1 = v8i{x1[0], x1[1], x1[2], x1[3], 0, 0, 0, 0};
      b3 = v8i{x3[0], x3[1], x3[2], x3[3], 0, 0, 0, 0};
      const int kg = kb >> 2, sh = 8 * (kb & 3);
      e1 = int((st[(kg * 2 + 0) * 64] >> sh) & 0xFFu);
      e3 = int((st[(kg * 2 + 1) * 64] >> sh) & 0xFFu);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m * 16 < tr.nrows) {
        const AOp a = a_from_lds(a_s, as_s, m * 16 + nl, g, a_pow2);
        mma_step<kFmtFp8, WF>(acc[0][m], a, b1, e1, f1, a_pow2, bp, lane);
        mma_step<kFmtFp8, WF>(acc[1][m], a, b3, e3, f3, a_pow2, bp, lane);
      }
    }
  }
  // epilogue: SwiGLU (+ routing weight) -> bf16 h
#pragma unroll
  for (int m = 0; m < 8; ++m) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m * 16 + g * 4 + i;
      if (r < tr.nrows) {
        float gs = acc[0][m][i], us = acc[1][m][i];
        float gv = bf16_round(gs), uv = bf16_round(us);
        if (d.swiglu_limit > 0.0f) {
          uv = fminf(fmaxf(uv, -d.swiglu_limit), d.swiglu_limit);
          gv = fminf(gv, d.swiglu_limit);
        }
        const float hv = silu_f32(gv) * uv;
        if (DENSE) {
          ws.sh_h[int64_t(row0 + r) * I + f0 + nl] = f32_to_bf16(hv);
        } else {
          const int p = row0 + r;
          const float wt_ = ws.weights[int64_t(clampi(ptok[p], 0, T - 1)) * k + clampi(ws.perm_slot[p], 0, k - 1)];
          ws.h[int64_t(p) * I + f0 + nl] = f32_to_bf16(wt_ * hv);
        }
      }
    }
  }
}

// w2: A rows are contiguous hq rows (pairs of the tile, or shared rows P + t).
template <int WF>
__global__ __launch_bounds__(kPThreads) void prefill_w2_kernel(wz_moe_desc d, MoeWs ws, int T) {
  __shared__ __align__(16) uint8_t a_s[kPM * kARow];
  __shared__ float as_s[kPM];
  constexpr bool DENSE = WF == kFmtFp8;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts, k = d.topk, P = T * k;
  const int KB = I / 128, KG = (KB + 3) / 4, DT = D / 16, NT = D / 64;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int mt = blockIdx.x / NT, nt = blockIdx.x % NT;
  TileRows tr;
  if (!tile_of(ws, mt, DENSE, T, P, E, tr)) return;
  const int dt = nt * 4 + wave, n0 = dt * 16;
  v4f acc[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) acc[m] = v4f{0.f, 0.f, 0.f, 0.f};
  const uint8_t* wt;
  const uint32_t* st = nullptr;
  if (DENSE) {
    wt = static_cast<const uint8_t*>(d.sh2p) + int64_t(dt) * KB * 2048;
  } else {
    wt = static_cast<const uint8_t*>(d.w2p) + (int64_t(tr.e) * DT + dt) * KB * 1024;
    st = static_cast<const uint32_t*>(d.w2p_s) + (int64_t(tr.e) * DT + dt) * KG * 64 + lane;
  }
  const bool bp = !DENSE || d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int64_t sbase = int64_t(n0 >> 7) * KB;
  const int arow0 = DENSE ? P + tr.row0 : tr.row0;
  for (int kb = 0; kb < KB; ++kb) {
    __syncthreads();
    stage_a(a_s, as_s, ws.hq, ws.hs, I, kb, tr.nrows, [&](int r) { return arow0 + r; });
    v8i b;
    int es;
    float fs = 1.0f;
    if (DENSE) {
      const uint8_t* tp = wt + int64_t(kb) * 2048;
      const v4i lo = load16_nt(tp + lane * 16), hi = load16_nt(tp + 1024 + lane * 16);
      b = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      fp8_wscale(d.sh_w2_s, sbase + kb, d.shared_w_scale_kind, es, fs);
    } else {
      const v4i x = load16_nt(wt + int64_t(kb) * 1024 + lane * 16);
      b = v8i{x[0], x[1], x[2], x[3], 0, 0, 0, 0};
      es = int((st[(kb >> 2) * 64] >> (8 * (kb & 3))) & 0xFFu);
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m * 16 < tr.nrows) {
        const AOp a = a_from_lds(a_s, as_s, m * 16 + nl, g, a_pow2);
        mma_step<kFmtFp8, WF>(acc[m], a, b, es, fs, a_pow2, bp, lane);
      }
    }
  }
#pragma unroll
  for (int m = 0; m < 8; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = m * 16 + g * 4 + i;
      if (r < tr.nrows) {
        if (DENSE)
          ws.sh_out[int64_t(tr.row0 + r) * D + n0 + nl] = f32_to_bf16(acc[m][i]);
        else
          ws.out2[int64_t(tr.row0 + r) * D + n0 + nl] = f32_to_bf16(acc[m][i]);
      }
    }
}

int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream);

// M-tiles a grid must cover: sum over experts of ceil(c/128) <= P/128 + active experts.
static inline int64_t prefill_mt_max(int64_t P, int E) { return P / kPM + (P < E ? P : E) + 1; }

int launch_prefill_experts(const wz_moe_desc* d, const MoeWs& w, const void* x, int64_t T, hipStream_t stream) {
  const int E = d->n_experts, k = d->topk, D = d->dim, I = d->inter;
  const int64_t P = T * k;
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe prefill: packed banks missing (call wz_moe_pack)");
  if (D % 64 || I % 64) return set_error(WZ_EINVAL, "moe prefill: dim and inter must be multiples of 64");
  const int qkind = d->act_scale_kind == WZ_SCALE_F32 ? WZ_SCALE_F32 : WZ_SCALE_UE8M0_F32;
  const int64_t mt_max = prefill_mt_max(P, E), mt_dense = (T + kPM - 1) / kPM;
  WZ_LAUNCH("moe_mtile", stream, mtile_kernel, dim3(1), dim3(1024), 0, w, E, int(P), int(mt_max));
  if (int rc = check_launch("moe mtile")) return rc;
  if (int rc = launch_act_quant(x, T, D, w.xq, w.xs, qkind, stream)) return rc;
  WZ_LAUNCH("moe_w13", stream, prefill_w13_kernel<kFmtFp4>, dim3(unsigned(mt_max * (I / 64))), dim3(kPThreads), 0,
            *d, w, int(T));
  if (int rc = check_launch("moe w13")) return rc;
  WZ_LAUNCH("moe_sh13", stream, prefill_w13_kernel<kFmtFp8>, dim3(unsigned(mt_dense * (I / 64))), dim3(kPThreads),
            0, *d, w, int(T));
  if (int rc = check_launch("moe sh13")) return rc;
  if (int rc = launch_act_quant(w.h, P, I, w.hq, w.hs, qkind, stream)) return rc;
  if (int rc = launch_act_quant(w.sh_h, T, I, w.hq + P * I, w.hs + P * (I / 128), qkind, stream)) return rc;
  WZ_LAUNCH("moe_w2", stream, prefill_w2_kernel<kFmtFp4>, dim3(unsigned(mt_max * (D / 64))), dim3(kPThreads), 0, *d,
            w, int(T));
  if (int rc = check_launch("moe w2")) return rc;
  WZ_LAUNCH("moe_sh2", stream, prefill_w2_kernel<kFmtFp8>, dim3(unsigned(mt_dense * (D / 64))), dim3(kPThreads), 0,
            *d, w, int(T));
  return check_launch("moe sh2");
}

}  // namespace wz
