// MoE decode path (T <= 16 tokens: the decode step and the DSpark verify widths).
//
// Four stream-ordered launches, no host sync, no allocation (graph-capturable):
//
//   route   WG per 4 experts: gate logits x.W^T (exact bf16 products, fp64
//           sums); the last gate WG to arrive (agent-scope counter) does score
//           function + bias + top-k + renormalise for every token, the
//           canonical (expert, token, slot) permutation, the active-expert
//           list and per-token combine lists.  T more WGs quantise x
//           (act_quant, one token each).
//   w13     per (expert, 16 intermediate features), routed MXFP4 experts and
//           the FP8 shared expert alike: w1 and w3 rows streamed once, A =
//           act_quant(x) rows of the expert's tokens, SwiGLU + clamp (+ the
//           routing weight), bf16 h.
//   hquant  act_quant of every h row (routed pairs and shared rows).
//   w2      one WG per 16 output columns; each wave computes one expert's
//           [rows x 16] tile over the full K (MXFP4 w2, or FP8 for the shared
//           expert) into LDS, then the WG sums each token's experts in
//           ascending id, adds the shared expert and writes bf16 y
//           (architecture.py:781-794, fp4_grouped.py:318-324) — the combine
//           never leaves the workgroup.
//
// Weight tiles are consumed with 16-byte loads, the loads of up to eight
// 128-wide K-blocks issued before the first MFMA, non-temporal (read once).
#include "moe_common.h"

namespace wz {

constexpr int kDecThreads = 256;

__device__ __forceinline__ v8i b_fp4_nt(const uint8_t* wrow, int kb, int g) {
  v4i x = load16_nt(wrow + kb * 64 + g * 16);
  return v8i{x[0], x[1], x[2], x[3], 0, 0, 0, 0};
}

__device__ __forceinline__ v8i b_fp8_nt(const uint8_t* wrow, int kb, int g) {
  const uint8_t* p = wrow + kb * 128 + g * 16;
  v4i lo = load16_nt(p), hi = load16_nt(p + 64);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Accumulate NB weight matrices (rows of this lane: wrow[m]) against one
// 16-row A tile over K-blocks [kb0, kb1).  WF: weight format.  A is either
// pre-quantised e4m3 (arow/asrow, float scales) or bf16 with act_quant fused.
template <int NB, int WF, bool A_BF16, int B>
__device__ __forceinline__ void tile_accum(v4f (&acc)[NB], const uint8_t* const (&wrow)[NB],
                                           const uint8_t* const (&srow)[NB], const void* const (&ws8)[NB],
                                           const int64_t (&ws8_base)[NB], int ws8_kind,
                                           const void* arow, const float* asrow, bool a_pow2,
                                           int kb0, int kb1, int g, int lane) {
  const bool b_pow2 = WF == kFmtFp4 || ws8_kind == WZ_WSCALE_E8M0;
  const int a_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  for (int kb = kb0; kb < kb1; kb += B) {
    v8i w[NB][B];
    int se[NB][B];
    float sf[NB][B];
#pragma unroll
    for (int q = 0; q < B; ++q) {
      const int kk = kb + q;
      if (kk < kb1) {
#pragma unroll
        for (int m = 0; m < NB; ++m) {
          if (WF == kFmtFp4) {
            w[m][q] = b_fp4_nt(wrow[m], kk, g);
            se[m][q] = b_fp4_scale(srow[m], kk, g);
            sf[m][q] = 1.0f;
          } else {
            w[m][q] = b_fp8_nt(wrow[m], kk, g);
            fp8_wscale(ws8[m], ws8_base[m] + kk, ws8_kind, se[m][q], sf[m][q]);
          }
        }
      }
    }
#pragma unroll
    for (int q = 0; q < B; ++q) {
      const int kk = kb + q;
      if (kk < kb1) {
        const AOp a = A_BF16 ? a_from_bf16(static_cast<const uint16_t*>(arow), kk, g, a_pow2)
                             : a_from_fp8(static_cast<const uint8_t*>(arow), asrow, kk, g, a_kind);
#pragma unroll
        for (int m = 0; m < NB; ++m)
          mma_step<kFmtFp8, WF>(acc[m], a, w[m][q], se[m][q], sf[m][q], a_pow2, b_pow2, lane);
      }
    }
  }
}

// Cross-wave K reduction through LDS: returns, in every wave, the sum of the
// four waves' accumulators (summed in wave order) for matrix m.
template <int NB>
__device__ __forceinline__ void reduce_waves(v4f (&acc)[NB], float* red, int wave, int lane) {
#pragma unroll
  for (int m = 0; m < NB; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * NB + m) * 4 + i) * kWave + lane] = acc[m][i];
  __syncthreads();
#pragma unroll
  for (int m = 0; m < NB; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = red[((0 * NB + m) * 4 + i) * kWave + lane];
      v += red[((1 * NB + m) * 4 + i) * kWave + lane];
      v += red[((2 * NB + m) * 4 + i) * kWave + lane];
      v += red[((3 * NB + m) * 4 + i) * kWave + lane];
      acc[m][i] = v;
    }
}

// SwiGLU with clamp (Expert.forward, architecture.py:733-739) on bf16-rounded
// linear outputs.
__device__ __forceinline__ float swiglu(float gs, float us, float limit) {
  float gv = bf16_round(gs), uv = bf16_round(us);
  if (limit > 0.0f) {
    uv = fminf(fmaxf(uv, -limit), limit);
    gv = fminf(gv, limit);
  }
  return silu_f32(gv) * uv;
}

// ------------------------------------------------------------------ route ---

__device__ void route_last(const wz_moe_desc& d, const MoeWs& ws, const int64_t* ids, int T) {
  __shared__ int s_idx[kDecodeMaxT * 16];
  __shared__ int cnt[kMaxExperts];
  __shared__ int base[kMaxExperts];
  __shared__ int wc[4][kMaxExperts];
  const int E = d.n_experts, k = d.topk, P = T * k;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kSlots = kMaxExperts / 64;
  // top-k per token, one wave per token
  for (int t = wave; t < T; t += 4) {
    const float* a = ws.scores + int64_t(t) * E;
    float s[kSlots], b[kSlots];
    double mx = -1e300, sum = 0.0;
    if (d.score_func == WZ_SCORE_SOFTMAX) {
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (lane + 64 * i < E) mx = fmax(mx, double(a[lane + 64 * i]));
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) mx = fmax(mx, __shfl_xor(mx, m, kWave));
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (lane + 64 * i < E) sum += exp(double(a[lane + 64 * i]) - mx);
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, kWave);
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int e = lane + 64 * i;
      float v = -INFINITY;
      if (e < E) {
        v = d.score_func == WZ_SCORE_SOFTMAX ? float(exp(double(a[e]) - mx) / sum)
                                             : score_of(a[e], d.score_func);
      }
      s[i] = v;
      b[i] = (e < E && d.tid2eid == nullptr && d.gate_bias != nullptr) ? v + d.gate_bias[e] : v;
    }
    int my_sel = 0;
    if (d.tid2eid != nullptr) {
      int64_t id = ids[t];
      id = id < 0 ? 0 : (id >= d.vocab ? d.vocab - 1 : id);
      if (lane < k) {
        const int e = d.tid2eid[id * k + lane];
        my_sel = e < 0 ? 0 : (e >= E ? E - 1 : e);
      }
    } else {
      unsigned taken = 0u;
      for (int j = 0; j < k; ++j) {
        Cand best = {-INFINITY, 0x7FFFFFFF};
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
          const int e = lane + 64 * i;
          if (e < E && !((taken >> i) & 1u)) best = cand_better(best, Cand{b[i], e});
        }
        best = wave_argmax(best);
        if (lane == j) my_sel = best.i;
        if ((best.i & 63) == lane) taken |= 1u << (best.i >> 6);
      }
    }
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const float v = __shfl(s[i], my_sel & 63, kWave);
      if ((my_sel >> 6) == i) mine = v;
    }
    float tot = 0.0f;
    for (int j = 0; j < k; ++j) tot += __shfl(mine, j, kWave);
    float v = mine;
    if (d.score_func != WZ_SCORE_SOFTMAX) v = v / tot;
    v = v * d.route_scale;
    if (lane < k) {
      ws.weights[t * k + lane] = v;
      ws.idx[t * k + lane] = my_sel;
      s_idx[t * k + lane] = my_sel;
    }
  }
  for (int e = tid; e < kMaxExperts; e += kDecThreads) cnt[e] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += kDecThreads) atomicAdd(&cnt[s_idx[p]], 1);
  __syncthreads();
  // exclusive scan of counts and of (count > 0) over E <= 512 experts, 2 per thread
  {
    const int e0 = 2 * tid, e1 = 2 * tid + 1;
    const int c0 = e0 < E ? cnt[e0] : 0, c1 = e1 < E ? cnt[e1] : 0;
    int v = c0 + c1;
    int f = (c0 > 0) + (c1 > 0);
    int vi = v, fi = f;
#pragma unroll
    for (int dd = 1; dd < 64; dd <<= 1) {
      const int ov = __shfl_up(vi, dd, kWave), of = __shfl_up(fi, dd, kWave);
      if (lane >= dd) {
        vi += ov;
        fi += of;
      }
    }
    if (lane == 63) {
      wc[0][wave] = vi;
      wc[1][wave] = fi;
    }
    __syncthreads();
    int vb = 0, fb = 0;
    for (int w = 0; w < wave; ++w) {
      vb += wc[0][w];
      fb += wc[1][w];
    }
    const int ex0 = vb + vi - v, fx0 = fb + fi - f;
    if (e0 < E) {
      base[e0] = ex0;
      ws.offsets[e0] = ex0;
      if (c0 > 0) {
        ws.active[fx0] = e0;
        ws.act_off[fx0] = ex0;
        ws.act_cnt[fx0] = c0;
      }
    }
    if (e1 < E) {
      base[e1] = ex0 + c0;
      ws.offsets[e1] = ex0 + c0;
      if (c1 > 0) {
        const int u = fx0 + (c0 > 0);
        ws.active[u] = e1;
        ws.act_off[u] = ex0 + c0;
        ws.act_cnt[u] = c1;
      }
    }
    if (tid == kDecThreads - 1) {
      ws.offsets[E] = vb + vi;
      ws.n_active[0] = fb + fi;
    }
  }
  __syncthreads();
  // stable placement of the P <= 256 pairs (one pass)
  {
    int nbits = 1;
    while ((1 << nbits) < E) ++nbits;
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int p = tid;
    const bool valid = p < P;
    const int e = valid ? s_idx[p] : 0;
    unsigned long long mask = __ballot(valid);
    if (!valid) mask = ~mask;
    for (int bit = 0; bit < nbits; ++bit) {
      const bool on = (e >> bit) & 1;
      const unsigned long long m = __ballot(on);
      mask &= on ? m : ~m;
    }
    const int rank = __popcll(mask & lt);
    const bool leader = (mask & lt) == 0ull;
    for (int i = tid; i < 4 * kMaxExperts; i += kDecThreads) (&wc[0][0])[i] = 0;
    __syncthreads();
    if (valid && leader) wc[wave][e] = __popcll(mask);
    __syncthreads();
    if (valid) {
      int before = 0;
      for (int w = 0; w < wave; ++w) before += wc[w][e];
      const int q = base[e] + before + rank;
      ws.perm_token[q] = p / k;
      ws.perm_slot[q] = p % k;
      ws.pos[p] = q;
      s_idx[p] = q | (e << 16);  // position and expert, for the combine lists
    }
  }
  __syncthreads();
  // per-token combine list: positions ascending (== experts ascending), one per expert
  if (tid < T) {
    int ps[16];
    for (int j = 0; j < k; ++j) ps[j] = s_idx[tid * k + j];
    for (int i = 1; i < k; ++i) {
      const int v = ps[i];
      int j = i - 1;
      while (j >= 0 && (ps[j] & 0xFFFF) > (v & 0xFFFF)) {
        ps[j + 1] = ps[j];
        --j;
      }
      ps[j + 1] = v;
    }
    int n = 0, prev_e = -1;
    for (int j = 0; j < k; ++j) {
      const int e = ps[j] >> 16;
      if (e == prev_e) {
        ws.tok_pos[tid * k + n - 1] = ps[j] & 0xFFFF;  // repeated expert: keep the last slot
        continue;
      }
      prev_e = e;
      ws.tok_pos[tid * k + n] = ps[j] & 0xFFFF;
      ++n;
    }
    ws.tok_n[tid] = n;
  }
}

__device__ void quant_row(const MoeWs& ws, const uint16_t* x, int t, int D, bool pow2) {
  // act_quant of one token row (torch_ops.py:33-49): 8 elements per lane,
  // 16 lanes per 128-block.
  for (int c0 = 0; c0 < D; c0 += kDecThreads * 8) {
    const int c = c0 + threadIdx.x * 8;
    const bool valid = c < D;
    v4i w = {0, 0, 0, 0};
    if (valid) w = load16(x + int64_t(t) * D + c);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16lo(uint32_t(w[i]));
      f[2 * i + 1] = bf16hi(uint32_t(w[i]));
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = wave_max_xor(amax, 1);
    amax = wave_max_xor(amax, 2);
    amax = wave_max_xor(amax, 4);
    amax = wave_max_xor(amax, 8);
    const ActScale sc = act_scale(amax, pow2);
    if (valid) {
      const uint32_t lo = pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2),
                                     quant_div(f[2], sc, pow2), quant_div(f[3], sc, pow2));
      const uint32_t hi = pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2),
                                     quant_div(f[6], sc, pow2), quant_div(f[7], sc, pow2));
      *reinterpret_cast<uint2*>(ws.xq + int64_t(t) * D + c) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) ws.xs[int64_t(t) * (D / 128) + c / 128] = sc.s;
    }
  }
}

__global__ __launch_bounds__(kDecThreads) void route_decode_kernel(wz_moe_desc d, MoeWs ws,
                                                                   const uint16_t* __restrict__ x,
                                                                   const int64_t* __restrict__ ids,
                                                                   int T, int n_gate) {
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts;
  int b = blockIdx.x;
  if (b < n_gate) {
    // ---- gate logits: one expert per wave, all T tokens ----
    const int e = b * 4 + wave;
    if (e < E) {
      const uint16_t* wr = static_cast<const uint16_t*>(d.gate_w) + int64_t(e) * D;
      const int nc = D / 8;
      double acc[kDecodeMaxT];
#pragma unroll
      for (int t = 0; t < kDecodeMaxT; ++t) acc[t] = 0.0;
      for (int c0 = 0; c0 < nc; c0 += 64 * 8) {
        v4i wv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int c = c0 + lane + 64 * i;
          wv[i] = c < nc ? load16(wr + c * 8) : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int t = 0; t < kDecodeMaxT; ++t) {
          if (t < T) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int c = c0 + lane + 64 * i;
              if (c < nc) {
                const v4i xv = load16(x + int64_t(t) * D + c * 8);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                  acc[t] += double(bf16lo(uint32_t(xv[j])) * bf16lo(uint32_t(wv[i][j])));
                  acc[t] += double(bf16hi(uint32_t(xv[j])) * bf16hi(uint32_t(wv[i][j])));
                }
              }
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < kDecodeMaxT; ++t) {
        if (t < T) {
          double v = acc[t];
#pragma unroll
          for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
          if (lane == 0) ws.scores[int64_t(t) * E + e] = float(v);
        }
      }
    }
    release_agent();
    __syncthreads();
    if (tid == 0) s_last = arrive_last(&ws.counters[0], uint32_t(n_gate)) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    acquire_agent();
    route_last(d, ws, ids, T);
    return;
  }
  b -= n_gate;
  quant_row(ws, x, b, D, d.act_scale_kind != WZ_SCALE_F32);
}

// -------------------------------------------------------------------- w13 ---

__global__ __launch_bounds__(kDecThreads) void w13_decode_kernel(wz_moe_desc d, MoeWs ws, int T,
                                                                 int n_sh) {
  __shared__ float red[4 * 2 * 4 * kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, k = d.topk;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int nkb = D / 128;
  const int kb0 = (wave * nkb) / 4, kb1 = ((wave + 1) * nkb) / 4;
  const int ftiles = I / 16;
  int b = blockIdx.x;
  const bool shared = b < n_sh;
  int f0, row0, nrows;
  const uint8_t* wrow[2];
  const uint8_t* srow[2] = {nullptr, nullptr};
  const void* ws8[2] = {nullptr, nullptr};
  int64_t sb[2] = {0, 0};
  if (shared) {
    f0 = b * 16;
    row0 = 0;
    nrows = T;
    wrow[0] = static_cast<const uint8_t*>(d.sh_w1) + int64_t(f0 + nl) * D;
    wrow[1] = static_cast<const uint8_t*>(d.sh_w3) + int64_t(f0 + nl) * D;
    ws8[0] = d.sh_w1_s;
    ws8[1] = d.sh_w3_s;
    sb[0] = sb[1] = int64_t(f0 >> 7) * nkb;
  } else {
    b -= n_sh;
    const int u = b / ftiles;
    f0 = (b % ftiles) * 16;
    if (u >= ws.n_active[0]) return;
    const int e = ws.active[u];
    row0 = ws.act_off[u];
    nrows = ws.act_cnt[u];
    const int64_t ebase = int64_t(e) * 2 * I;
    const uint8_t* w13 = static_cast<const uint8_t*>(d.w13);
    const uint8_t* w13s = static_cast<const uint8_t*>(d.w13_s);
    wrow[0] = w13 + (ebase + f0 + nl) * (D / 2);
    wrow[1] = w13 + (ebase + I + f0 + nl) * (D / 2);
    srow[0] = w13s + (ebase + f0 + nl) * (D / 32);
    srow[1] = w13s + (ebase + I + f0 + nl) * (D / 32);
  }
  for (int r0 = 0; r0 < nrows; r0 += 16) {
    // this lane's A row (token) and, for the epilogue, the routing weight of its output rows
    const int r = r0 + nl;
    const int tok = r < nrows ? (shared ? r : ws.perm_token[row0 + r]) : -1;
    float wt[4] = {1.f, 1.f, 1.f, 1.f};
    if (!shared && wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = r0 + g * 4 + i;
        if (rr < nrows) {
          const int p = row0 + rr;
          wt[i] = ws.weights[ws.perm_token[p] * k + ws.perm_slot[p]];
        }
      }
    }
    const uint8_t* arow = tok >= 0 ? ws.xq + int64_t(tok) * D : nullptr;
    const float* asrow = tok >= 0 ? ws.xs + int64_t(tok) * (D / 128) : nullptr;
    v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    if (shared)
      tile_accum<2, kFmtFp8, false, 4>(acc, wrow, srow, ws8, sb, d.shared_w_scale_kind, arow, asrow, a_pow2,
                                       kb0, kb1, g, lane);
    else
      tile_accum<2, kFmtFp4, false, 8>(acc, wrow, srow, ws8, sb, 0, arow, asrow, a_pow2, kb0, kb1, g, lane);
    reduce_waves<2>(acc, red, wave, lane);
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = r0 + g * 4 + i;
        if (rr < nrows) {
          const float hv = swiglu(acc[0][i], acc[1][i], d.swiglu_limit);
          if (shared)
            ws.sh_h[int64_t(rr) * I + f0 + nl] = f32_to_bf16(hv);
          else
            ws.h[int64_t(row0 + rr) * I + f0 + nl] = f32_to_bf16(wt[i] * hv);
        }
      }
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------- hquant ---

// act_quant of one h row per WG: rows [0, P) are routed pairs (h), [P, P+T)
// the shared expert's rows (sh_h).
__global__ __launch_bounds__(kDecThreads) void hquant_kernel(MoeWs ws, int P, int I, bool pow2) {
  const int row = blockIdx.x;
  const uint16_t* src = row < P ? ws.h + int64_t(row) * I : ws.sh_h + int64_t(row - P) * I;
  for (int c0 = 0; c0 < I; c0 += kDecThreads * 8) {
    const int c = c0 + threadIdx.x * 8;
    const bool valid = c < I;
    v4i w = {0, 0, 0, 0};
    if (valid) w = load16(src + c);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16lo(uint32_t(w[i]));
      f[2 * i + 1] = bf16hi(uint32_t(w[i]));
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(f[i]));
    amax = wave_max_xor(amax, 1);
    amax = wave_max_xor(amax, 2);
    amax = wave_max_xor(amax, 4);
    amax = wave_max_xor(amax, 8);
    const ActScale sc = act_scale(amax, pow2);
    if (valid) {
      const uint32_t lo = pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2),
                                     quant_div(f[2], sc, pow2), quant_div(f[3], sc, pow2));
      const uint32_t hi = pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2),
                                     quant_div(f[6], sc, pow2), quant_div(f[7], sc, pow2));
      *reinterpret_cast<uint2*>(ws.hq + int64_t(row) * I + c) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) ws.hs[int64_t(row) * (I / 128) + c / 128] = sc.s;
    }
  }
}

// --------------------------------------------------------------------- w2 ---

constexpr int kW2Waves = 16;
constexpr int kW2Threads = kW2Waves * 64;

__global__ __launch_bounds__(kW2Threads) void w2_combine_kernel(wz_moe_desc d, MoeWs ws, int T,
                                                                uint16_t* __restrict__ y) {
  __shared__ float out_s[kDecodeMaxT * 16][16];   // routed pair rows (permuted order) x 16 columns
  __shared__ float sh_s[kDecodeMaxT][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, k = d.topk;
  const int P = T * k;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int n0 = blockIdx.x * 16;
  const int nkb = I / 128;
  const int n_act = ws.n_active[0];
  for (int job = wave; job <= n_act; job += kW2Waves) {
    const bool shared = job == n_act;
    int row0, nrows;
    const uint8_t* wrow[1];
    const uint8_t* srow[1] = {nullptr};
    const void* ws8[1] = {nullptr};
    int64_t sb[1] = {0};
    if (shared) {
      row0 = P;  // shared rows follow the pairs in hq
      nrows = T;
      wrow[0] = static_cast<const uint8_t*>(d.sh_w2) + int64_t(n0 + nl) * I;
      ws8[0] = d.sh_w2_s;
      sb[0] = int64_t(n0 >> 7) * nkb;
    } else {
      const int e = ws.active[job];
      row0 = ws.act_off[job];
      nrows = ws.act_cnt[job];
      const int64_t ebase = int64_t(e) * D;
      wrow[0] = static_cast<const uint8_t*>(d.w2) + (ebase + n0 + nl) * (I / 2);
      srow[0] = static_cast<const uint8_t*>(d.w2_s) + (ebase + n0 + nl) * (I / 32);
    }
    for (int r0 = 0; r0 < nrows; r0 += 16) {
      const int r = r0 + nl;
      const uint8_t* arow = r < nrows ? ws.hq + int64_t(row0 + r) * I : nullptr;
      const float* asrow = r < nrows ? ws.hs + int64_t(row0 + r) * (I / 128) : nullptr;
      v4f acc[1] = {{0.f, 0.f, 0.f, 0.f}};
      if (shared)
        tile_accum<1, kFmtFp8, false, 4>(acc, wrow, srow, ws8, sb, d.shared_w_scale_kind, arow, asrow, a_pow2,
                                         0, nkb, g, lane);
      else
        tile_accum<1, kFmtFp4, false, 8>(acc, wrow, srow, ws8, sb, 0, arow, asrow, a_pow2, 0, nkb, g, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rr = r0 + g * 4 + i;
        if (rr < nrows) {
          const float v = bf16_round(acc[0][i]);  // each linear's output is bf16 (architecture.py:741)
          if (shared)
            sh_s[rr][nl] = v;
          else
            out_s[row0 + rr][nl] = v;
        }
      }
    }
  }
  __syncthreads();
  if (tid < 16 * T) {
    const int t = tid >> 4, col = tid & 15;
    const int n = ws.tok_n[t];
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc += out_s[ws.tok_pos[t * k + j]][col];
    acc += sh_s[t][col];
    y[int64_t(t) * D + n0 + col] = f32_to_bf16(acc);
  }
}

int launch_decode(const wz_moe_desc* d, const MoeWs& w, const void* x, const int64_t* ids, int64_t T,
                  void* y, hipStream_t stream) {
  const int E = d->n_experts, k = d->topk, D = d->dim, I = d->inter;
  const int n_gate = (E + 3) / 4;
  const int64_t P = T * k;
  const int u_max = int(P < E ? P : E);
  if (P > kDecodeMaxT * 16) return set_error(WZ_EINVAL, "moe decode: T*topk=%lld exceeds %d", (long long)P,
                                             kDecodeMaxT * 16);
  WZ_LAUNCH("moe_route", stream, route_decode_kernel, dim3(unsigned(n_gate + T)), dim3(kDecThreads), 0, *d, w,
            static_cast<const uint16_t*>(x), ids, int(T), n_gate);
  if (int rc = check_launch("moe route")) return rc;
  WZ_LAUNCH("moe_w13", stream, w13_decode_kernel, dim3(unsigned(I / 16 + u_max * (I / 16))), dim3(kDecThreads),
            0, *d, w, int(T), I / 16);
  if (int rc = check_launch("moe w13")) return rc;
  WZ_LAUNCH("moe_hquant", stream, hquant_kernel, dim3(unsigned(P + T)), dim3(kDecThreads), 0, w, int(P), I,
            d->act_scale_kind != WZ_SCALE_F32);
  if (int rc = check_launch("moe hquant")) return rc;
  WZ_LAUNCH("moe_w2", stream, w2_combine_kernel, dim3(unsigned(D / 16)), dim3(kW2Threads), 0, *d, w, int(T),
            static_cast<uint16_t*>(y));
  return check_launch("moe w2");
}

}  // namespace wz
