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
constexpr int kPThreads = 256;    // 4 waves
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

// B operands of one K-block for the NT weight tiles a wave owns (fp4: lo only).
// The MXFP4 scale stays the raw packed dword until the MFMA needs its byte:
// extracting it at fetch time would make the fetch wait for its own loads.
template <int NT>
struct BTiles {
  v4i lo[NT], hi[NT];
  uint32_t sw[NT];  // fp4: packed e8m0 dword (byte kb & 3); fp8: the e8m0 byte
  float f[NT];
};

// Expert-grouped tile GEMM over one M-tile (<= 128 rows) and one N-block.
//   MODE 0: routed w1/w3 (packed MXFP4) over gathered x rows -> SwiGLU -> h
//   MODE 1: shared w1/w3 (packed FP8) over token rows        -> SwiGLU -> sh_h
//   MODE 2: routed w2 (packed MXFP4) over h rows             -> out2
//   MODE 3: shared w2 (packed FP8) over shared h rows        -> sh_out
// A wave owns NTW weight tiles of 16 output columns (routed: 4, i.e. w13: 2
// feature tiles x {w1, w3}, w2: 4 column tiles; shared FP8 tiles are twice
// the bytes, so 2), and one A operand read from LDS feeds NTW MFMAs.
// The K loop is software-pipelined: the A block of K-step kb+1 is fetched to
// registers and the B tiles of kb+2 are in flight while kb computes; A goes
// through two LDS buffers with one barrier per K-step.
//
// CHAIN: activation and weight scales are both powers of two, so they ride in
// the MFMA's e8m0 scale operands and the accumulators chain over K; otherwise
// each K-block partial is scaled on the VALU (mma_step).
template <int MODE, bool CHAIN>
__device__ __forceinline__ void gemm_tile(const wz_moe_desc& d, const MoeWs& ws, int T, int mt, int nt,
                                          uint8_t (*a_s)[kPM * kARow], float (*as_s)[kPM]) {
  constexpr bool W13 = MODE < 2, DENSE = (MODE & 1) != 0;
  constexpr int WF = DENSE ? kFmtFp8 : kFmtFp4;
  constexpr int NTW = DENSE ? 2 : 4;          // weight tiles per wave
  constexpr int CPW = W13 ? NTW / 2 : NTW;    // 16-column output tiles per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts, k = d.topk, P = T * k;
  const int K = W13 ? D : I, KB = K / 128, KG = (KB + 3) / 4;
  const int NCT = (W13 ? I : D) / 16;  // 16-column tiles of the output
  const bool a_pow2 = CHAIN || d.act_scale_kind != WZ_SCALE_F32;
  const bool bp = CHAIN || !DENSE || d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  TileRows tr;
  if (!tile_of(ws, mt, DENSE, T, P, E, tr)) return;
  const int row0 = tr.row0, nrows = tr.nrows, e = tr.e;
  const int ct0 = (nt * 4 + wave) * CPW;  // first column tile of this wave

  // weight tile j of this wave: column tile ct(j), w1/w3 selector which(j)
  int ct[NTW], which[NTW];
  bool jv[NTW];
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    ct[j] = W13 ? ct0 + (j >> 1) : ct0 + j;
    which[j] = W13 ? (j & 1) : 0;
    jv[j] = ct[j] < NCT;
  }

  // A staging: thread -> (row, half of the 128-byte K-block)
  const int sr = tid >> 1, sh = tid & 1;
  const uint8_t* arow = nullptr;
  const float* asrow = nullptr;
  if (sr < nrows) {
    int src;
    if (MODE == 0) src = clampi(ws.perm_token[row0 + sr], 0, T - 1);
    else if (MODE == 1) src = row0 + sr;
    else if (MODE == 2) src = row0 + sr;
    else src = P + row0 + sr;
    const uint8_t* A = W13 ? ws.xq : ws.hq;
    const float* As = W13 ? ws.xs : ws.hs;
    arow = A + int64_t(src) * K + sh * 64;
    asrow = As + int64_t(src) * KB;
  }
  v4i av[4];
  float asv = 1.0f;
  auto a_fetch = [&](int kb) {
    if (arow) {
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = load16(arow + kb * 128 + 16 * i);
      asv = asrow[kb];
    }
  };
  auto a_put = [&](int buf) {
    if (arow) {
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<v4i*>(&a_s[buf][sr * kARow + sh * 64 + 16 * i]) = av[i];
      if (sh == 0) as_s[buf][sr] = asv;
    }
  };

  auto b_fetch = [&](BTiles<NTW>& b, int kb) {
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      if (!jv[j]) continue;
      if (MODE == 0) {
        const int64_t t = int64_t(e) * NCT + ct[j];
        const uint8_t* w = static_cast<const uint8_t*>(d.w13p) + ((t * KB + kb) * 2 + which[j]) * 1024;
        b.lo[j] = load16_nt(w + lane * 16);
        const uint32_t* sw = static_cast<const uint32_t*>(d.w13p_s) + ((t * KG + (kb >> 2)) * 2 + which[j]) * 64;
        b.sw[j] = sw[lane];
        b.f[j] = 1.0f;
      } else if (MODE == 2) {
        const int64_t t = int64_t(e) * NCT + ct[j];
        const uint8_t* w = static_cast<const uint8_t*>(d.w2p) + (t * KB + kb) * 1024;
        b.lo[j] = load16_nt(w + lane * 16);
        const uint32_t* sw = static_cast<const uint32_t*>(d.w2p_s) + (t * KG + (kb >> 2)) * 64;
        b.sw[j] = sw[lane];
        b.f[j] = 1.0f;
      } else {
        const uint8_t* w;
        const void* s;
        if (MODE == 1) {
          w = static_cast<const uint8_t*>(d.sh13p) + ((int64_t(ct[j]) * KB + kb) * 2 + which[j]) * 2048;
          s = which[j] ? d.sh_w3_s : d.sh_w1_s;
        } else {
          w = static_cast<const uint8_t*>(d.sh2p) + (int64_t(ct[j]) * KB + kb) * 2048;
          s = d.sh_w2_s;
        }
        b.lo[j] = load16_nt(w + lane * 16);
        b.hi[j] = load16_nt(w + 1024 + lane * 16);
        int se8;
        fp8_wscale(s, int64_t(ct[j] >> 3) * KB + kb, d.shared_w_scale_kind, se8, b.f[j]);
        b.sw[j] = uint32_t(se8);
      }
    }
  };

  v4f acc[NTW][8];
#pragma unroll
  for (int j = 0; j < NTW; ++j)
#pragma unroll
    for (int m = 0; m < 8; ++m) acc[j][m] = v4f{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int buf, const BTiles<NTW>& b, int kb) {
    int e8[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) e8[j] = DENSE ? int(b.sw[j]) : int((b.sw[j] >> (8 * (kb & 3))) & 0xFFu);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      if (m * 16 < nrows) {
        const AOp a = a_from_lds(a_s[buf], as_s[buf], m * 16 + nl, g, CHAIN || a_pow2);
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          if (!jv[j]) continue;
          const v8i bv = DENSE ? v8i{b.lo[j][0], b.lo[j][1], b.lo[j][2], b.lo[j][3], b.hi[j][0], b.hi[j][1],
                                     b.hi[j][2], b.hi[j][3]}
                               : v8i{b.lo[j][0], b.lo[j][1], b.lo[j][2], b.lo[j][3], 0, 0, 0, 0};
          if (CHAIN)
            acc[j][m] = mfma_scaled<kFmtFp8, WF>(a.v, bv, acc[j][m], a.se8, e8[j]);
          else
            mma_step<kFmtFp8, WF>(acc[j][m], a, bv, e8[j], b.f[j], a_pow2, bp, lane);
        }
      }
    }
  };

  BTiles<NTW> b0, b1;
  a_fetch(0);
  b_fetch(b0, 0);
  a_put(0);
  if (KB > 1) {
    a_fetch(1);
    b_fetch(b1, 1);
  }
  __syncthreads();
  for (int kb = 0; kb < KB; kb += 2) {
    compute(0, b0, kb);
    if (kb + 1 < KB) a_put(1);
    if (kb + 2 < KB) {
      a_fetch(kb + 2);
      b_fetch(b0, kb + 2);
    }
    __syncthreads();
    if (kb + 1 >= KB) break;
    compute(1, b1, kb + 1);
    if (kb + 2 < KB) a_put(0);
    if (kb + 3 < KB) {
      a_fetch(kb + 3);
      b_fetch(b1, kb + 3);
    }
    __syncthreads();
  }

  // epilogue
  if (W13) {
#pragma unroll
    for (int q = 0; q < CPW; ++q) {
      if (!jv[2 * q]) continue;
      const int f = ct[2 * q] * 16 + nl;
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m * 16 + g * 4 + i;
          if (r < nrows) {
            float gv = bf16_round(acc[2 * q][m][i]), uv = bf16_round(acc[2 * q + 1][m][i]);
            if (d.swiglu_limit > 0.0f) {
              uv = fminf(fmaxf(uv, -d.swiglu_limit), d.swiglu_limit);
              gv = fminf(gv, d.swiglu_limit);
            }
            const float hv = silu_f32(gv) * uv;
            if (DENSE) {
              ws.sh_h[int64_t(row0 + r) * I + f] = f32_to_bf16(hv);
            } else {
              const int p = row0 + r;
              const float wt =
                  ws.weights[int64_t(clampi(ws.perm_token[p], 0, T - 1)) * k + clampi(ws.perm_slot[p], 0, k - 1)];
              ws.h[int64_t(p) * I + f] = f32_to_bf16(wt * hv);
            }
          }
        }
    }
  } else {
    uint16_t* out = DENSE ? ws.sh_out : ws.out2;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      if (!jv[j]) continue;
      const int c = ct[j] * 16 + nl;
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = m * 16 + g * 4 + i;
          if (r < nrows) out[int64_t(row0 + r) * D + c] = f32_to_bf16(acc[j][m][i]);
        }
    }
  }
}

// One launch serves the shared expert's dense tiles (block ids first, so the
// few long-running shared tiles start early) and the routed experts' M-tiles.
// W13 selects w1/w3 + SwiGLU or w2; CR / CS: scale chaining of routed / shared.
template <bool W13, bool CR, bool CS>
__global__ __launch_bounds__(kPThreads) __attribute__((amdgpu_waves_per_eu(2))) void prefill_gemm_kernel(
    wz_moe_desc d, MoeWs ws, int T, int nblk, int nblk_dense, int dense_blocks) {
  __shared__ __align__(16) uint8_t a_s[2][kPM * kARow];
  __shared__ float as_s[2][kPM];
  const int b = blockIdx.x;
  if (b < dense_blocks)
    gemm_tile<W13 ? 1 : 3, CS>(d, ws, T, b / nblk_dense, b % nblk_dense, a_s, as_s);
  else
    gemm_tile<W13 ? 0 : 2, CR>(d, ws, T, (b - dense_blocks) / nblk, (b - dense_blocks) % nblk, a_s, as_s);
}

int launch_act_quant(const void* x, int64_t rows, int64_t K, uint8_t* q, void* s, int kind, hipStream_t stream);

// M-tiles a grid must cover: sum over experts of ceil(c/128) <= P/128 + active experts.
static inline int64_t prefill_mt_max(int64_t P, int E) { return P / kPM + (P < E ? P : E) + 1; }

int launch_prefill_experts(const wz_moe_desc* d, const MoeWs& w, const void* x, int64_t T, hipStream_t stream) {
  const int E = d->n_experts, k = d->topk, D = d->dim, I = d->inter;
  const int64_t P = T * k;
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe prefill: packed banks missing (call wz_moe_pack)");
  const int qkind = d->act_scale_kind == WZ_SCALE_F32 ? WZ_SCALE_F32 : WZ_SCALE_UE8M0_F32;
  const int64_t mt_max = prefill_mt_max(P, E), mt_dense = (T + kPM - 1) / kPM;
  WZ_LAUNCH("moe_mtile", stream, mtile_kernel, dim3(1), dim3(1024), 0, w, E, int(P), int(mt_max));
  if (int rc = check_launch("moe mtile")) return rc;
  if (int rc = launch_act_quant(x, T, D, w.xq, w.xs, qkind, stream)) return rc;
  // column tiles of 16 per WG: routed 4 waves x 4 weight tiles, shared 4 x 2
  const int nb13 = (I / 16 + 7) / 8, nb13d = (I / 16 + 3) / 4;
  const int nb2 = (D / 16 + 15) / 16, nb2d = (D / 16 + 7) / 8;
  const bool cr = d->act_scale_kind != WZ_SCALE_F32;
  const bool cs = cr && d->shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int Ti = int(T), dn13 = int(mt_dense * nb13d), dn2 = int(mt_dense * nb2d);
  const dim3 blk(kPThreads), g13(unsigned(dn13 + mt_max * nb13)), g2(unsigned(dn2 + mt_max * nb2));
  if (cr && cs) {
    WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, true, true>), g13, blk, 0, *d, w, Ti, nb13, nb13d, dn13);
  } else if (cr) {
    WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, true, false>), g13, blk, 0, *d, w, Ti, nb13, nb13d, dn13);
  } else {
    WZ_LAUNCH("moe_w13", stream, (prefill_gemm_kernel<true, false, false>), g13, blk, 0, *d, w, Ti, nb13, nb13d, dn13);
  }
  if (int rc = check_launch("moe w13")) return rc;
  if (int rc = launch_act_quant(w.h, P, I, w.hq, w.hs, qkind, stream)) return rc;
  if (int rc = launch_act_quant(w.sh_h, T, I, w.hq + P * I, w.hs + P * (I / 128), qkind, stream)) return rc;
  if (cr && cs) {
    WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, true, true>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2);
  } else if (cr) {
    WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, true, false>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2);
  } else {
    WZ_LAUNCH("moe_w2", stream, (prefill_gemm_kernel<false, false, false>), g2, blk, 0, *d, w, Ti, nb2, nb2d, dn2);
  }
  return check_launch("moe w2");
}

}  // namespace wz
