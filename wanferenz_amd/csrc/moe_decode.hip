// MoE decode path (T <= 16 tokens: the decode step and the DSpark verify widths).
//
// Three stream-ordered launches while w2's LDS image fits (at the V4 shape
// T <= 8), four or five otherwise; no host sync, no allocation
// (graph-capturable):
//
//   route   gate WGs: each expert's logits x.W^T for all T tokens (exact bf16
//           products, fp64 sums), its K range split over 1-8 waves; each gate
//           thread applies the score function and the bias for one (expert,
//           token).  The last gate WG to arrive (agent-scope counter) does
//           top-k + renormalise for every token (Gate.forward,
//           architecture.py:696-718), one wave per token, and one wave
//           builds the active-expert list, the (expert, token) -> pair-row
//           map and the per-token combine lists.  In the same launch T WGs
//           quantise x (act_quant) and the rest stream the shared expert's
//           w1 / w3, which needs no routing.
//   w13     per (active expert, 16 intermediate features): MXFP4 w1 and w3
//           tiles streamed once, SwiGLU + clamp + routing weight, bf16 h;
//           the shared expert's w1 / w3 ran in the route launch.
//   hquant  act_quant of the h rows that are routed, and of the shared rows
//           (only when w2_lds_kernel does not serve: that kernel quantises h
//           into LDS itself).
//   w2      one WG per 16 output columns (w2_lds_kernel): the WG copies the
//           e4m3 h rows of every routed pair and the shared rows into LDS,
//           then each wave computes one expert's 16-column tile over the full
//           K (MXFP4, or FP8 for the shared expert's K halves) with the next
//           job's tiles streaming into the registers it frees, and the WG
//           sums each token's experts in ascending id, adds the shared expert
//           and writes bf16 y (architecture.py:781-794, fp4_grouped.py:318-324).
//
// Tokens ride on the MFMA's 16-row side: the A operand of every expert is
// the whole (<= 16 token) batch, row t = token t, and only the rows of the
// tokens routed to that expert are kept.  So a workgroup needs one table
// lookup (its expert id) before its weight stream starts, and no per-lane
// token gather.  Weights come from the packed banks (pack.hip): every load
// instruction reads 1 KB contiguous, non-temporal (read once).
#include <algorithm>
#include <type_traits>

#include "moe_common.h"

namespace wz {

constexpr int kDecThreads = 256;
constexpr int kRouteWaves = 8;                  // waves of a route-launch workgroup
constexpr int kRouteThreads_ = kRouteWaves * 64;

__device__ __forceinline__ v8i pk_fp4(const uint8_t* tile, int lane) {
  const v4i x = load16_nt(tile + lane * 16);
  return v8i{x[0], x[1], x[2], x[3], 0, 0, 0, 0};
}

__device__ __forceinline__ v8i pk_fp8(const uint8_t* tile, int lane) {
  const v4i lo = load16_nt(tile + lane * 16), hi = load16_nt(tile + 1024 + lane * 16);
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Cross-wave K reduction through LDS (partials summed in wave order).
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

// SwiGLU with clamp (Expert.forward, architecture.py:733-739) on the
// bf16-rounded outputs of w1 and w3.
__device__ __forceinline__ float swiglu(float gs, float us, float limit) {
  float gv = bf16_round(gs), uv = bf16_round(us);
  if (limit > 0.0f) {
    uv = clamp_keep_nan(uv, -limit, limit);
    gv = gv > limit ? limit : gv;
  }
  return silu_f32(gv) * uv;
}

// ------------------------------------------------------------------ route ---

constexpr int kMaxDecPairs = kDecodeMaxT * 16;
constexpr int kMaxUT = kDecodeMaxT * kMaxDecPairs;

// KS: 64-expert slots per lane (E <= 64 KS); 4 serve V4's 256 experts.
// GEN: the softmax and hash-table routes are compiled in; without it (a
// top-k gate with another score function, the V4 case) the code this one
// workgroup runs, fetched cold once per launch, is that much shorter.
struct RouteLds {
  unsigned long long s_mask[kMaxExperts / 64];  // selected experts
  int s_e[kMaxDecPairs];
  float s_w[kMaxDecPairs];
  int s_umap[kMaxUT];
  float s_uwt[kMaxUT];
};

template <int KS, bool GEN>
__device__ __forceinline__ void route_last(const wz_moe_desc& d, const MoeWs& ws, const int64_t* ids, int T, int u_max,
                           RouteLds& L) {
  int* s_e = L.s_e;
  float* s_w = L.s_w;
  int* s_umap = L.s_umap;
  float* s_uwt = L.s_uwt;
  const int E = d.n_experts, k = d.topk, P = T * k, UT = u_max * T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  constexpr int kSlots = KS;
  // ---- top-k, one wave per token.  The gate waves already wrote each
  // expert's score (softmax: its logit; the whole row is needed here).
  // (Loops in this single-workgroup phase stay rolled: it runs once per
  // launch, so its code is fetched cold and code size is its latency.) ----
#pragma unroll 1
  for (int t = wave; t < T; t += kRouteWaves) {
    float sv[kSlots];
    uint32_t key[kSlots];
    float raw[kSlots], rawb[kSlots];
    const bool smax = GEN && d.score_func == WZ_SCORE_SOFTMAX;
    // the selection key: the score plus the gate bias (a constant input, so
    // read here beside the scores rather than published with them), the fp32
    // add the reference's `scores + bias` makes
    const bool addb = d.score_func != WZ_SCORE_SOFTMAX && d.tid2eid == nullptr && d.gate_bias != nullptr;
    float bv[kSlots];
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int e = lane + 64 * i;
      bv[i] = (addb && e < E) ? d.gate_bias[e] : 0.0f;
      raw[i] = e < E ? load_agent(ws.scores + int64_t(t) * E + e) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) rawb[i] = addb ? raw[i] + bv[i] : raw[i];
    double mx = -1e300, sum = 0.0;
    if (smax) {
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (lane + 64 * i < E) mx = fmax(mx, double(raw[i]));
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) mx = fmax(mx, __shfl_xor(mx, m, kWave));
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (lane + 64 * i < E) sum += exp(double(raw[i]) - mx);
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, kWave);
    }
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int e = lane + 64 * i;
      sv[i] = 0.0f;
      key[i] = 0u;
      if (e < E) {
        if (smax) {
          sv[i] = float(exp(double(raw[i]) - mx) / sum);
          key[i] = f32_key((d.tid2eid == nullptr && d.gate_bias != nullptr) ? sv[i] + d.gate_bias[e] : sv[i]);
        } else {
          sv[i] = raw[i];
          key[i] = f32_key(rawb[i]);
        }
      }
    }
    int my_sel = 0;
    float mine = 0.0f;    // lane j < k: the score of the token's j-th expert
    float tot = 0.0f;     // the k scores summed in slot order (fp32)
    bool poison = false;  // hash id or table entry out of range: NaN weights, in-range reads
    if (GEN && d.tid2eid != nullptr) {
      int64_t id = ids[t];
      const bool bad_id = id < 0 || id >= d.vocab;
      id = bad_id ? 0 : id;
      bool bad_e = false;
      if (lane < k) {
        const int e = d.tid2eid[id * k + lane];
        bad_e = e < 0 || e >= E;
        my_sel = bad_e ? 0 : e;
      }
      poison = bad_id || __ballot(bad_e) != 0ull;
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const float v = __shfl(sv[i], my_sel & 63, kWave);
        if ((my_sel >> 6) == i) mine = v;
      }
      for (int j = 0; j < k; ++j) tot += __shfl(mine, j, kWave);
    } else {
      // The lane's experts sorted by key, best first.  Adjacent swaps on a
      // strictly larger key keep equal keys in slot order, i.e. ascending id;
      // slots past E hold key 0 and come last in slot order, so they sort
      // behind every valid expert and `live` counts the valid ones left.
      uint32_t hk[kSlots];
      int hs[kSlots];
      float hv[kSlots];
      int live = 0;
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        hk[i] = key[i];
        hs[i] = i;
        hv[i] = sv[i];
        live += lane + 64 * i < E ? 1 : 0;
      }
#pragma unroll
      for (int a = 0; a < kSlots - 1; ++a)
#pragma unroll
        for (int i = 0; i + 1 < kSlots - a; ++i)
          if (hk[i + 1] > hk[i]) {
            const uint32_t tk = hk[i];
            const int ts = hs[i];
            const float tv = hv[i];
            hk[i] = hk[i + 1];
            hs[i] = hs[i + 1];
            hv[i] = hv[i + 1];
            hk[i + 1] = tk;
            hs[i + 1] = ts;
            hv[i + 1] = tv;
          }
      // k rounds: the wave max of the lanes' heads, the winner pops its head.
      // Vector instructions only (selects, no branch on a lane condition), so
      // the round never waits for a vector result in the scalar unit: with a
      // ballot and a readlane per round it took ~0.33 us a round at T = 1.
#pragma unroll 1
      for (int j = 0; j < k; ++j) {
        const uint32_t m = wave_max_all_u32(live > 0 ? hk[0] : 0u);
        const bool cand = live > 0 && hk[0] == m;
        // equal keys: the lowest expert id wins (torch.topk keeps the earlier index)
        const int we = int(wave_min_all_u32(cand ? uint32_t(lane + 64 * hs[0]) : 0xFFFFFFFFu));
        const int wl = __builtin_amdgcn_readfirstlane(we) & 63;
        const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(hv[0]), wl));
        tot += wv;
        const bool mine_j = lane == j;
        my_sel = mine_j ? we : my_sel;
        mine = mine_j ? wv : mine;
        const bool pop = lane == wl;
#pragma unroll
        for (int i = 0; i + 1 < kSlots; ++i) {
          hk[i] = pop ? hk[i + 1] : hk[i];
          hs[i] = pop ? hs[i + 1] : hs[i];
          hv[i] = pop ? hv[i + 1] : hv[i];
        }
        hk[kSlots - 1] = pop ? 0u : hk[kSlots - 1];
        live -= pop ? 1 : 0;
      }
    }
    float v = mine;
    if (d.score_func != WZ_SCORE_SOFTMAX) v = v / tot;
    v = v * d.route_scale;
    if (poison) v = __builtin_nanf("");
    if (lane < k) {
      ws.weights[t * k + lane] = v;
      ws.idx[t * k + lane] = my_sel;
      s_e[t * k + lane] = my_sel;
      s_w[t * k + lane] = v;
    }
  }
  // ---- the tables, by wave 0 alone (its LDS accesses are in program order,
  // so no barrier separates the steps).  What the later launches read: the
  // active-expert list, umap / uwt (active expert u, token t) -> the pair row
  // and its weight, and the per-token combine lists.  A routed (expert, token)
  // is stored at the row of its pair p = t k + j (the token's last slot with
  // that expert, architecture.py:790 index_put semantics): any row < P unique
  // to the (expert, token) serves, so no canonical permutation is needed
  // here.  The active index of an expert is the count of selected experts
  // below it, from a presence mask; a token's combine order (ascending expert
  // id) compares its own k experts.  All of it is vector work with no loop
  // over the pairs: this phase is one wave's dependent instruction chain, and
  // the earlier count / scan / placement version took 3.3 us at T = 1, a
  // loop over the pairs 2.6 us at T = 1 and 4.5 us at T = 4. ----
  __syncthreads();  // the token waves' s_e / s_w
  if (wave != 0) return;
  unsigned long long* s_mask = L.s_mask;
  if (lane < KS) s_mask[lane] = 0ull;
  for (int p = lane; p < P; p += kWave) {
    const int e = s_e[p];
    atomicOr(&s_mask[e >> 6], 1ull << (e & 63));
  }
  unsigned long long mw[KS];
  int n_act = 0;
#pragma unroll
  for (int w = 0; w < KS; ++w) {
    mw[w] = s_mask[w];
    n_act += __popcll(mw[w]);
  }
  if (lane == 0) ws.n_active[0] = n_act;
  for (int i = lane; i < UT; i += kWave) s_umap[i] = -1;
  for (int p = lane; p < P; p += kWave) {
    const int e = s_e[p], t = p / k, j = p - t * k;
    int uc = 0;  // active index of e
#pragma unroll
    for (int w = 0; w < KS; ++w) {
      const int ew = e >> 6;
      const unsigned long long below = w < ew ? mw[w] : (w == ew ? mw[w] & ((1ull << (e & 63)) - 1ull) : 0ull);
      uc += __popcll(below);
    }
    ws.active[uc] = e;  // every pair of the expert stores the same id
    // the token's experts (reads past its k clamp to its last one, and are
    // masked out of the counts)
    int te[16];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) te[jj] = s_e[t * k + min(jj, k - 1)];
    bool last = true;
    int rank = 0, n = 0;
    if (GEN) {
      // a hash table can repeat an expert within a token: only its last slot counts
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) {
        bool lj = jj < k;
#pragma unroll
        for (int j2 = jj + 1; j2 < 16; ++j2) lj = lj && !(j2 < k && te[j2] == te[jj]);
        if (jj > j && jj < k && te[jj] == e) last = false;
        n += lj ? 1 : 0;
        rank += (lj && te[jj] < e) ? 1 : 0;
      }
    } else {
      // top-k never repeats an expert within a token
      n = k;
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) rank += (jj < k && te[jj] < e) ? 1 : 0;
    }
    if (last) {
      s_umap[uc * T + t] = p;
      s_uwt[uc * T + t] = s_w[p];
      ws.tok_pos[t * k + rank] = p;
      if (rank == 0) ws.tok_n[t] = n;
    }
  }
  for (int i = lane; i < UT; i += kWave) {
    ws.umap[i] = s_umap[i];
    ws.uwt[i] = s_uwt[i];
  }
}

// The token rows as a route-launch workgroup (512 threads) reads them, in
// rmsnorm_kernel's thread mapping: thread (h, t) holds chunks t + 256 j
// (8 bf16 each) of rows 2 p + h, the rows of pass p < kPass present when
// 2 p < T (a row 2 p + 1 = T repeats row T - 1 and is not used).  D <= kNormMaxD.
//
// The ffn RMSNorm folded into the route launch (route_decode_kernel<KS, true>,
// wz_moe_forward_norm): x is then the block's hidden state h, and each
// workgroup forms 1 / sqrt(mean(h^2) + eps) of every row in rmsnorm_kernel's
// arithmetic (the chunks summed in order, the wave butterfly, the four wave
// partials as (p0 + p1) + (p2 + p3)) and the MoE input bf16(w (h r)) element by
// element, so the codes and logits equal those of the unfused launches.
constexpr int kRowCh = kNormMaxD / 2048;  // chunks per thread and row
struct NormLds {
  float rs[kDecodeMaxT];
  float part[kDecodeMaxT][4];
};

template <int kPass>
__device__ __forceinline__ void load_rows(v4i (&hv)[kPass][kRowCh], const uint16_t* __restrict__ x, int T, int D) {
  const int half = threadIdx.x >> 8, vt = threadIdx.x & 255, nch = D / 8;
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (2 * p < T) {
      const uint16_t* xr = x + int64_t(min(2 * p + half, T - 1)) * D;
#pragma unroll
      for (int j = 0; j < kRowCh; ++j) hv[p][j] = load16(xr + min(vt + 256 * j, nch - 1) * 8);
    }
}

// the norm weight of the thread's chunks
__device__ __forceinline__ void load_norm_w(float4 (&nwv)[kRowCh][2], const float* __restrict__ nw, int D) {
  const int vt = threadIdx.x & 255, nch = D / 8;
#pragma unroll
  for (int j = 0; j < kRowCh; ++j) {
    const float* w = nw + min(vt + 256 * j, nch - 1) * 8;
    nwv[j][0] = *reinterpret_cast<const float4*>(w);
    nwv[j][1] = *reinterpret_cast<const float4*>(w + 4);
  }
}

// bf16(w (h r)) of the 8 elements packed in v (rmsnorm_kernel's value)
__device__ __forceinline__ v4i norm_chunk(const v4i& v, const float4 (&w)[2], float r) {
  const float wf[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
  v4i o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float a = wf[2 * i] * (bf16lo(uint32_t(v[i])) * r);
    const float b = wf[2 * i + 1] * (bf16hi(uint32_t(v[i])) * r);
    o[i] = int(f32x2_to_bf16x2(a, b));
  }
  return o;
}

// Every row's norm factor from the loaded rows, then the rows normalised in place.
template <int kPass>
__device__ __forceinline__ void norm_rows(v4i (&hv)[kPass][kRowCh], const float4 (&nwv)[kRowCh][2], float eps,
                                          int T, int D, NormLds& L) {
  const int tid = threadIdx.x, lane = tid & 63, half = tid >> 8, vt = tid & 255, nch = D / 8;
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (2 * p < T) {
      float ss = 0.0f;
#pragma unroll
      for (int j = 0; j < kRowCh; ++j)
        if (vt + 256 * j < nch) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float a = bf16lo(uint32_t(hv[p][j][i])), c = bf16hi(uint32_t(hv[p][j][i]));
            ss += a * a;
            ss += c * c;
          }
        }
#pragma unroll
      for (int m = 32; m >= 1; m >>= 1) ss += __shfl_xor(ss, m, kWave);
      if (lane == 0 && 2 * p + half < T) L.part[2 * p + half][vt >> 6] = ss;
    }
  __syncthreads();
  if (tid < T) {
    const float* pp = L.part[tid];
    const float var = ((pp[0] + pp[1]) + (pp[2] + pp[3])) / float(D);
    L.rs[tid] = 1.0f / sqrtf(var + eps);
  }
  __syncthreads();
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (2 * p < T) {
      const float r = L.rs[min(2 * p + half, T - 1)];
#pragma unroll
      for (int j = 0; j < kRowCh; ++j) hv[p][j] = norm_chunk(hv[p][j], nwv[j], r);
    }
}

__device__ __forceinline__ void quant_row(uint8_t* __restrict__ q, float* __restrict__ s, const uint16_t* __restrict__ x,
                          int K, bool pow2) {
  // act_quant of one row (torch_ops.py:33-49): 8 elements per lane, 16 lanes per 128-block.
  for (int c0 = 0; c0 < K; c0 += int(blockDim.x) * 8) {
    const int c = c0 + threadIdx.x * 8;
    const bool valid = c < K;
    v4i w = {0, 0, 0, 0};
    if (valid) w = load16(x + c);
    float f[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = bf16lo(uint32_t(w[i]));
      f[2 * i + 1] = bf16hi(uint32_t(w[i]));
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = absmax(amax, f[i]);
    amax = wave_absmax_xor(amax, 1);
    amax = wave_absmax_xor(amax, 2);
    amax = wave_absmax_xor(amax, 4);
    amax = wave_absmax_xor(amax, 8);
    const ActScale sc = act_scale(amax, pow2);
    if (valid) {
      const uint32_t lo = pack_fp8x4(quant_div(f[0], sc, pow2), quant_div(f[1], sc, pow2),
                                     quant_div(f[2], sc, pow2), quant_div(f[3], sc, pow2));
      const uint32_t hi = pack_fp8x4(quant_div(f[4], sc, pow2), quant_div(f[5], sc, pow2),
                                     quant_div(f[6], sc, pow2), quant_div(f[7], sc, pow2));
      *reinterpret_cast<uint2*>(q + c) = make_uint2(lo, hi);
      if ((threadIdx.x & 15) == 0) s[c / 128] = sc.s;
    }
  }
}

// Shared expert w1 / w3 for features 16 b .. 16 b + 15 with act_quant(x) fused
// into the A-operand load (this runs in the route launch, before xq exists);
// the waves split K and meet in LDS.  AP2: power-of-two activation scales;
// WP2: e8m0 weight block scales (both fix the loads at compile time).  Every
// load of a wave's K range (token rows, weight tiles, their scales) is issued
// before the first wait: token rows past T read row T - 1 (their outputs are
// not stored) and K-blocks past the range re-read its last one (not added).
// With the loads behind guards the compiler waited on each K-block in turn,
// and these items, not the routing, ended the launch (T = 1: 16.9 us against
// 14.4 us for the routing).
template <bool AP2, bool WP2>
__device__ __forceinline__ void w13_shared_item_bf16(const wz_moe_desc& d, const MoeWs& ws,
                                                     const uint16_t* __restrict__ x, int T, int b, float* red) {
  constexpr int kQ = 4;  // K-blocks per batch (D = 4096: the wave's whole range)
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter;
  const int KB = D / 128;
  const int kb0 = (wave * KB) / kRouteWaves, kb1 = ((wave + 1) * KB) / kRouteWaves;
  const uint16_t* xrow = x + int64_t(min(nl, T - 1)) * D;
  const int f0 = b * 16;
  const uint8_t* tiles = static_cast<const uint8_t*>(d.sh13p) + int64_t(b) * KB * 4096;
  const int wkind = WP2 ? WZ_WSCALE_E8M0 : WZ_WSCALE_F32;
  const int64_t sbase = int64_t(f0 >> 7) * KB;
  v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  for (int kb = kb0; kb < kb1; kb += kQ) {
    v8i w[2][kQ];
    int se[2][kQ];
    float sf[2][kQ];
    ARaw xr[kQ];  // x first: its quantisation then overlaps the weight loads
#pragma unroll
    for (int q = 0; q < kQ; ++q) xr[q] = a_load_bf16(xrow, min(kb + q, kb1 - 1), g);
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int kk = min(kb + q, kb1 - 1);
      w[0][q] = pk_fp8(tiles + int64_t(kk) * 4096, lane);
      w[1][q] = pk_fp8(tiles + int64_t(kk) * 4096 + 2048, lane);
      fp8_wscale(d.sh_w1_s, sbase + kk, wkind, se[0][q], sf[0][q]);
      fp8_wscale(d.sh_w3_s, sbase + kk, wkind, se[1][q], sf[1][q]);
    }
#pragma unroll
    for (int q = 0; q < kQ; ++q)
      if (kb + q < kb1) {
        const AOp a = a_quant_bf16(xr[q], AP2);
        mma_step<kFmtFp8, kFmtFp8>(acc[0], a, w[0][q], se[0][q], sf[0][q], AP2, WP2, lane);
        mma_step<kFmtFp8, kFmtFp8>(acc[1], a, w[1][q], se[1][q], sf[1][q], AP2, WP2, lane);
      }
  }
  // red: [kRouteWaves][2][4][64] floats; partials summed in wave order
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * 2 + m) * 4 + i) * kWave + lane] = acc[m][i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float gs = red[((0 * 2 + 0) * 4 + i) * kWave + lane], us = red[((0 * 2 + 1) * 4 + i) * kWave + lane];
#pragma unroll
      for (int w = 1; w < kRouteWaves; ++w) {
        gs += red[((w * 2 + 0) * 4 + i) * kWave + lane];
        us += red[((w * 2 + 1) * 4 + i) * kWave + lane];
      }
      const int t = g * 4 + i;
      if (t < T) ws.sh_h[int64_t(t) * I + f0 + nl] = f32_to_bf16(swiglu(gs, us, d.swiglu_limit));
    }
  }
}

// Shared expert w1 / w3 for features 16 b .. 16 b + 15, the token rows staged
// in LDS (D <= kNormMaxD): the workgroup loads the T rows once (load_rows),
// (NORM) normalises them (norm_rows), act_quant-s them into LDS, 16 lanes per
// (row, 128-block) as quant_row does, so the codes equal the unfused path's,
// and only then requests its weight tiles: the gate workgroups' loads, which
// the routing waits on, reach HBM first.  Each wave reads its A operands from
// LDS (rows past T repeat row T - 1; their outputs are not stored).  Item
// b < T also writes token row b's codes and block scales to xq / xs for the
// w1 / w3 launch.  Quantising each wave's K range in the MFMA layout instead
// covered all 16 row slots (three quarters empty at T = 4) in every wave, and
// with the norm folded in that cost the launch 5 us.
struct ItemLds {
  uint8_t xq[kDecodeMaxT][kNormMaxD + 16];  // e4m3 rows, padded against bank conflicts
  float xs[kDecodeMaxT][kNormMaxD / 128];   // their block scales
};
// a route-launch workgroup's token rows: a shared item's codes, or a gate
// block's bf16 rows (T <= kNormMaxT)
union RowLds {
  ItemLds il;
  uint16_t xn[kNormMaxT][kNormMaxD];
};
template <bool AP2, bool WP2, bool NORM>
__device__ __forceinline__ void w13_shared_item_lds(const wz_moe_desc& d, const MoeWs& ws,
                                                    const uint16_t* __restrict__ x, const float* __restrict__ nw,
                                                    float eps, int T, int b, float* red, NormLds& NL, ItemLds& IL) {
  constexpr int kQ = 4, kPass = (NORM ? kNormMaxT : kDecodeMaxT) / 2;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4, half = tid >> 8, vt = tid & 255;
  const int D = d.dim, I = d.inter, KB = D / 128, nch = D / 8;
  const int kb0 = (wave * KB) / kRouteWaves, kb1 = ((wave + 1) * KB) / kRouteWaves;
  const int f0 = b * 16;
  const uint8_t* tiles = static_cast<const uint8_t*>(d.sh13p) + int64_t(b) * KB * 4096;
  const int wkind = WP2 ? WZ_WSCALE_E8M0 : WZ_WSCALE_F32;
  const int64_t sbase = int64_t(f0 >> 7) * KB;
  v4i hv[kPass][kRowCh];
  load_rows<kPass>(hv, x, T, D);
  if constexpr (NORM) {
    float4 nwv[kRowCh][2];
    load_norm_w(nwv, nw, D);
    norm_rows<kPass>(hv, nwv, eps, T, D, NL);
  }
  // ---- act_quant of the rows into LDS (quant_row's arithmetic) ----
#pragma unroll
  for (int p = 0; p < kPass; ++p)
    if (2 * p < T) {
      const int row = 2 * p + half;
#pragma unroll
      for (int j = 0; j < kRowCh; ++j)
        if (256 * j < nch) {  // uniform: the 16-lane groups of a chunk range are whole
          const int c = vt + 256 * j, col = min(c, nch - 1) * 8;
          const float amax = row16_absmax(bf16x8_absmax(hv[p][j]));
          const ActScale sc = act_scale(amax, AP2);
          float f[8];
          bf16x8_unpack(hv[p][j], f);
          const uint2 qv = quant8(f, sc, AP2, quant_fast(amax, AP2));
          if (row < T && c < nch) {
            *reinterpret_cast<uint2*>(&IL.xq[row][col]) = qv;
            if ((tid & 15) == 0) IL.xs[row][col / 128] = sc.s;
          }
        }
    }
  __syncthreads();
  v8i w[2][kQ];
  int se[2][kQ];
  float sf[2][kQ];
  // The first fetch runs before the K loop, also for a wave whose K range is
  // empty (KB < kRouteWaves, D < 1024): its K-blocks are clamped into [0, KB)
  // (kb1 - 1 alone is -1 for wave 0 there, 4 KB before the bank) and never used.
  auto fetch = [&](int kb) {
#pragma unroll
    for (int q = 0; q < kQ; ++q) {
      const int kk = min(kb + q, max(kb1 - 1, 0));
      w[0][q] = pk_fp8(tiles + int64_t(kk) * 4096, lane);
      w[1][q] = pk_fp8(tiles + int64_t(kk) * 4096 + 2048, lane);
      fp8_wscale(d.sh_w1_s, sbase + kk, wkind, se[0][q], sf[0][q]);
      fp8_wscale(d.sh_w3_s, sbase + kk, wkind, se[1][q], sf[1][q]);
    }
  };
  fetch(kb0);
  // ---- item b < T: token row b's codes and scales for the w1 / w3 launch ----
  if (b < T) {
    for (int c = tid; c < nch; c += kRouteThreads_)
      *reinterpret_cast<uint2*>(ws.xq + int64_t(b) * D + c * 8) = *reinterpret_cast<const uint2*>(&IL.xq[b][c * 8]);
    if (tid < KB) ws.xs[int64_t(b) * KB + tid] = IL.xs[b][tid];
  }
  // ---- the K loop, A from LDS ----
  const int arow = min(nl, T - 1);
  v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  for (int kb = kb0; kb < kb1; kb += kQ) {
    if (kb != kb0) fetch(kb);
#pragma unroll
    for (int q = 0; q < kQ; ++q)
      if (kb + q < kb1) {
        AOp a = a_zero();
        const uint8_t* pa = &IL.xq[arow][(kb + q) * 128 + g * 16];
        const v4i lo = *reinterpret_cast<const v4i*>(pa), hi = *reinterpret_cast<const v4i*>(pa + 64);
        a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        const float sc = IL.xs[arow][kb + q];
        a.sf = sc;
        a.se8 = AP2 ? int((__float_as_uint(sc) >> 23) & 0xFFu) : kE8m0One;
        mma_step<kFmtFp8, kFmtFp8>(acc[0], a, w[0][q], se[0][q], sf[0][q], AP2, WP2, lane);
        mma_step<kFmtFp8, kFmtFp8>(acc[1], a, w[1][q], se[1][q], sf[1][q], AP2, WP2, lane);
      }
  }
  // red: [kRouteWaves][2][4][64] floats; partials summed in wave order
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[((wave * 2 + m) * 4 + i) * kWave + lane] = acc[m][i];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float gs = red[((0 * 2 + 0) * 4 + i) * kWave + lane], us = red[((0 * 2 + 1) * 4 + i) * kWave + lane];
#pragma unroll
      for (int w2 = 1; w2 < kRouteWaves; ++w2) {
        gs += red[((w2 * 2 + 0) * 4 + i) * kWave + lane];
        us += red[((w2 * 2 + 1) * 4 + i) * kWave + lane];
      }
      const int t = g * 4 + i;
      if (t < T) ws.sh_h[int64_t(t) * I + f0 + nl] = f32_to_bf16(swiglu(gs, us, d.swiglu_limit));
    }
  }
}

// Blocks [0, n_gate): gate waves.  An expert's logits for all T tokens are
// split over `split` consecutive waves of one block (a K range each, fp64
// partials summed in wave order), so the gate's fp64 work spreads over
// n_gate = E * split / 8 CUs; then the last block to arrive routes.  The
// rest: the shared expert's w1 / w3 items, one per block (its waves split K),
// which do not depend on the routing and so stream while it runs; item b < T
// then writes act_quant of token row b.  NORM: x is the hidden state h and the MoE input
// is its RMSNorm with weight nw (route_norm_prologue), formed where it is read.
template <int KS, bool NORM>
__global__ __launch_bounds__(kRouteThreads_) void route_decode_kernel(wz_moe_desc d, MoeWs ws,
                                                                   const uint16_t* __restrict__ x,
                                                                   const int64_t* __restrict__ ids, int T,
                                                                   int n_gate, int split, int u_max,
                                                                   const float* __restrict__ nw, float eps) {
  __shared__ NormLds nls;
  __shared__ __align__(16) RowLds rows;
  __shared__ int s_last;
  __shared__ double part[kRouteWaves][kDecodeMaxT];
  // 16 KB: a gate block's per-lane partials (double [8][4][64]) or a shared
  // item's cross-wave sums (float [8][2][4][64])
  __shared__ __align__(16) float rbuf[kRouteWaves * 2 * 4 * kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int D = d.dim, E = d.n_experts;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  int b = blockIdx.x;
  if (b < n_gate) {
    // ---- partial gate logits: expert e, 16-byte chunks [c0, c1) of D ----
    const int task = b * kRouteWaves + wave;
    const int e = task / split, sp = task % split;
    const int nc = D / 8, c0 = (sp * nc) / split, c1 = ((sp + 1) * nc) / split;
    // the (expert, token) this thread finishes below
    const int epb = kRouteWaves / split;
    const int fin_e = b * epb + tid / max(T, 1);
    const bool fin = tid < epb * T && fin_e < E;
    double acc[kDecodeMaxT];
#pragma unroll
    for (int t = 0; t < kDecodeMaxT; ++t) acc[t] = 0.0;
    const uint16_t* wr = static_cast<const uint16_t*>(d.gate_w) + int64_t(min(e, E - 1)) * D;
    // T <= kNormMaxT (D <= kNormMaxD): the rows are staged in LDS once for the
    // block's waves (read in load_rows' mapping; NORM: normalised there), then
    // the first weight chunks are requested: the staging waits on the rows (and
    // the norm weight) alone
    const bool staged = NORM || (T <= kNormMaxT && D <= kNormMaxD);
    v4i hv[kNormMaxT / 2][kRowCh];
    float4 nwv[kRowCh][2];
    if (staged) load_rows<kNormMaxT / 2>(hv, x, T, D);
    if constexpr (NORM) load_norm_w(nwv, nw, D);
    __builtin_amdgcn_sched_barrier(0);
    v4i wv0[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = c0 + lane + 64 * i;
      wv0[i] = (e < E && c < c1) ? load16(wr + c * 8) : v4i{0, 0, 0, 0};
    }
    __builtin_amdgcn_sched_barrier(0);
    if (staged) {
      if constexpr (NORM) norm_rows<kNormMaxT / 2>(hv, nwv, eps, T, D, nls);
      const int half = tid >> 8, vt = tid & 255, nch = D / 8;
#pragma unroll
      for (int p = 0; p < kNormMaxT / 2; ++p)
        if (2 * p < T) {
          const int row = 2 * p + half;
#pragma unroll
          for (int j = 0; j < kRowCh; ++j) {
            const int c = vt + 256 * j;
            if (row < T && c < nch) *reinterpret_cast<v4i*>(&rows.xn[row][c * 8]) = hv[p][j];
          }
        }
      __syncthreads();
    }
    if (e < E && c0 < c1) {
#pragma unroll 1
      for (int cb = c0; cb < c1; cb += 64 * 2) {
        // two 16-byte chunks per lane; a chunk past c1 gets w = 0 and a clamped,
        // valid x address, so every load below is unconditional
        v4i wv[2];
        int cx[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = cb + lane + 64 * i;
          if (cb == c0)
            wv[i] = wv0[i];
          else
            wv[i] = c < c1 ? load16(wr + c * 8) : v4i{0, 0, 0, 0};
          cx[i] = min(c, c1 - 1);
        }
        // tokens in groups of 8: a group's x chunks are all requested before any
        // is used (one round trip per group; token indices past T are clamped)
#pragma unroll
        for (int tg = 0; tg < kDecodeMaxT; tg += 8) {
          if (tg < T) {
            v4i xv[8][2];
            if (staged) {
#pragma unroll
              for (int j = 0; j < 8; ++j)
                if (tg + j < T) {
#pragma unroll
                  for (int i = 0; i < 2; ++i) xv[j][i] = *reinterpret_cast<const v4i*>(&rows.xn[tg + j][cx[i] * 8]);
                }
            } else {
#pragma unroll
              for (int j = 0; j < 8; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i) xv[j][i] = load16(x + int64_t(min(tg + j, T - 1)) * D + cx[i] * 8);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (tg + j < T) {
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                  for (int q = 0; q < 4; ++q) {
                    acc[tg + j] += double(bf16lo(uint32_t(xv[j][i][q])) * bf16lo(uint32_t(wv[i][q])));
                    acc[tg + j] += double(bf16hi(uint32_t(xv[j][i][q])) * bf16hi(uint32_t(wv[i][q])));
                  }
              }
          }
        }
      }
    }
    // ---- each token's sum over the wave's 64 lanes, 4 tokens at a time: the
    // lanes' partials go through this wave's LDS rows, then 16 lanes per token
    // each add 4 of them and 4 shuffle levels finish (fixed order) ----
    double(*gsum)[4][kWave] = reinterpret_cast<double(*)[4][kWave]>(rbuf);
#pragma unroll
    for (int t0 = 0; t0 < kDecodeMaxT; t0 += 4) {
      if (t0 < T) {
#pragma unroll
        for (int c = 0; c < 4; ++c) gsum[wave][c][lane] = acc[t0 + c];
        const int c = lane >> 4, j = lane & 15;
        double v = gsum[wave][c][4 * j];
        v += gsum[wave][c][4 * j + 1];
        v += gsum[wave][c][4 * j + 2];
        v += gsum[wave][c][4 * j + 3];
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
        if (j == 0 && t0 + c < T) part[wave][t0 + c] = v;
      }
    }
    __syncthreads();
    // ---- one thread per (expert of this block, token): partials in wave
    // order, then the score function and the bias (the selection key) ----
    if (fin) {
      const int es = tid / T, t = tid % T, e2 = fin_e;
      double v = 0.0;
      for (int s2 = 0; s2 < split; ++s2) v += part[es * split + s2][t];
      const int64_t o = int64_t(t) * E + e2;
      const float logit = float(v);
      store_agent(ws.scores + o, d.score_func == WZ_SCORE_SOFTMAX ? logit : score_of(logit, d.score_func));
    }
    vm_drain();  // this wave's score stores are performed before the arrival below
    __syncthreads();
    if (tid == 0) s_last = arrive_last(&ws.counters[0], uint32_t(n_gate)) ? 1 : 0;
    __syncthreads();
    if (!s_last) return;
    // reads the scores with load_agent
    __shared__ RouteLds rl;
    if (d.score_func != WZ_SCORE_SOFTMAX && d.tid2eid == nullptr)
      route_last<KS, false>(d, ws, ids, T, u_max, rl);
    else
      route_last<KS, true>(d, ws, ids, T, u_max, rl);
    return;
  }
  b -= n_gate;
  const bool wp2 = d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  if (D <= kNormMaxD) {
    // the token rows staged in LDS once for the item (and normalised: NORM)
#define WZ_ITEM(AP, WP) w13_shared_item_lds<AP, WP, NORM>(d, ws, x, nw, eps, T, b, rbuf, nls, rows.il)
    if (a_pow2 && wp2)
      WZ_ITEM(true, true);
    else if (a_pow2)
      WZ_ITEM(true, false);
    else if (wp2)
      WZ_ITEM(false, true);
    else
      WZ_ITEM(false, false);
#undef WZ_ITEM
    return;
  }
  // wider rows (never NORM: the launch refuses it): act_quant in the MFMA layout
  if (a_pow2 && wp2)
    w13_shared_item_bf16<true, true>(d, ws, x, T, b, rbuf);
  else if (a_pow2)
    w13_shared_item_bf16<true, false>(d, ws, x, T, b, rbuf);
  else if (wp2)
    w13_shared_item_bf16<false, true>(d, ws, x, T, b, rbuf);
  else
    w13_shared_item_bf16<false, false>(d, ws, x, T, b, rbuf);
  // item b < T also quantises token row b (the w1 / w3 launch's A operand), so
  // the launch is n_gate + I / 16 workgroups: one per CU at V4 (with separate
  // act_quant workgroups, T of them waited for a second round)
  if (b < T)
    quant_row(ws.xq + int64_t(b) * D, ws.xs + int64_t(b) * (D / 128), x + int64_t(b) * D, D, a_pow2);
}

// -------------------------------------------------------------------- w13 ---

__global__ __launch_bounds__(kDecThreads) void w13_decode_kernel(wz_moe_desc d, MoeWs ws, int T, int u_max) {
  __shared__ float red[4 * 2 * 4 * kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int a_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  const int KB = D / 128, KG = (KB + 3) / 4, FT = I / 16;
  const int kb0 = (wave * KB) / 4, kb1 = ((wave + 1) * KB) / 4;
  // A operand: the token batch, row t = token t (act_quant(x) from the route kernel)
  const uint8_t* arow = nl < T ? ws.xq + int64_t(nl) * D : nullptr;
  const float* asrow = nl < T ? ws.xs + int64_t(nl) * (D / 128) : nullptr;
  v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const int b = blockIdx.x;
  // ---- routed expert: MXFP4 w1 / w3 for features ft*16 .. +15 ----
  const int u = b / FT, ft = b % FT;
  if (u >= min(ws.n_active[0], u_max)) return;
  const int e = clampi(ws.active[u], 0, d.n_experts - 1);
  const int64_t tile0 = (int64_t(e) * FT + ft) * KB;  // first K-block of (e, ft)
  const uint8_t* wt = static_cast<const uint8_t*>(d.w13p) + tile0 * 2048;
  const uint32_t* st = static_cast<const uint32_t*>(d.w13p_s) + (int64_t(e) * FT + ft) * KG * 2 * 64 + lane;
  // epilogue data for this lane's output rows (token 4g + i), fetched early
  int qrow[4];
  float wrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = g * 4 + i;
    qrow[i] = t < T ? ws.umap[u * T + t] : -1;
    wrow[i] = t < T ? ws.uwt[u * T + t] : 0.0f;
  }
  for (int kb = kb0; kb < kb1; kb += 8) {
    v8i w[2][8];
    uint32_t s1[3], s3[3];
#pragma unroll
    for (int q = 0; q < 3; ++q) {
      const int kg = (kb >> 2) + q;
      s1[q] = kg < KG ? st[(kg * 2 + 0) * 64] : 0u;
      s3[q] = kg < KG ? st[(kg * 2 + 1) * 64] : 0u;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q)
      if (kb + q < kb1) {
        w[0][q] = pk_fp4(wt + int64_t(kb + q) * 2048, lane);
        w[1][q] = pk_fp4(wt + int64_t(kb + q) * 2048 + 1024, lane);
      }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int kk = kb + q;
      if (kk < kb1) {
        const AOp a = a_from_fp8(arow, asrow, kk, g, a_kind);
        const int sh = 8 * (kk & 3), qi = (kk >> 2) - (kb >> 2);
        const int e1 = int((s1[qi] >> sh) & 0xFFu), e3 = int((s3[qi] >> sh) & 0xFFu);
        mma_step<kFmtFp8, kFmtFp4>(acc[0], a, w[0][q], e1, 1.0f, a_pow2, true, lane);
        mma_step<kFmtFp8, kFmtFp4>(acc[1], a, w[1][q], e3, 1.0f, a_pow2, true, lane);
      }
    }
  }
  reduce_waves<2>(acc, red, wave, lane);
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (qrow[i] >= 0 && qrow[i] < T * d.topk)
        ws.h[int64_t(qrow[i]) * I + ft * 16 + nl] = f32_to_bf16(wrow[i] * swiglu(acc[0][i], acc[1][i], d.swiglu_limit));
    }
  }
}

// ----------------------------------------------------------------- hquant ---

// hq row r < u_max*T: (active expert u, token t), quantised from h's pair row
// umap[r] only when routed; row u_max*T + t: the shared expert's row t.
// Routed experts' w1/w3 for the decode batch on persistent workgroups.
//
// Work item = (active expert u, 16 intermediate features ft): 64 KB of packed
// MXFP4 tiles.  Items are numbered u * FT + ft, so a run of consecutive items
// is one contiguous stretch of the packed bank; workgroup b takes items b,
// b + G, b + 2G, ... of the N = n_active * FT items (grid stride), so the
// resident workgroups always stream one contiguous window of the bank.  Per item the four
// waves split K (at most 8 K-blocks each) and meet in LDS; while an item's
// MFMAs, reduction and epilogue run, the next item's tiles are in flight (two
// register buffers, steady-state loads unconditional so the counted waits
// stay exact).  The A operand (the token batch's e4m3 rows for this wave's
// K-blocks) is loaded once and kept in registers for every item; its block
// scales must be powers of two (they ride in the MFMA), the other scale kinds
// take w13_decode_kernel.

template <int NKB>
struct W13Buf {
  v4i w1[NKB], w3[NKB];
  uint32_t s1[2], s3[2];  // packed e8m0 dwords (4 K-blocks each)
  int q[4];               // epilogue: pair rows of this lane's four token rows (-1: unrouted)
  float wt[4];            //           and their routing weights
  int u, ft;
};

// NKB = K-blocks per wave = D / 512 (compile-time, so no load is conditional).
template <int NKB>
__global__ __launch_bounds__(kDecThreads) void w13_stream_kernel(wz_moe_desc d, MoeWs ws, int T, int u_max) {
  __shared__ float red[2][4 * 2 * 4 * kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts;
  const int a_kind = WZ_SCALE_UE8M0_F32;  // power-of-two scales (host-checked)
  const int KB = 4 * NKB, KG = (KB + 3) / 4, FT = I / 16;
  const int kb0 = wave * NKB;
  // active-expert ids in LDS, so a tile address never waits on a global load
  // (all u_max entries, read together with n_active: one round trip)
  __shared__ int s_act[kMaxExperts];
  const int n_act = min(ws.n_active[0], u_max);
  for (int j = tid; j < u_max; j += kDecThreads) s_act[j] = clampi(ws.active[j], 0, E - 1);
  __syncthreads();
  const int N = n_act * FT;
  // grid-stride over items: at any moment the resident workgroups read one
  // contiguous window of the bank (G consecutive items)
  const int G = gridDim.x;
  const int i0 = blockIdx.x;
  if (i0 >= N) return;
  const int kg0 = kb0 >> 2;
  v8i av[NKB];  // the A operand (this wave's K-blocks), loaded after the first tiles
  int ae[NKB];

  auto fetch = [&](W13Buf<NKB>& b, int item) {
    b.u = item / FT;
    b.ft = item % FT;
    const int e = s_act[b.u];
    const int64_t tile = int64_t(e) * FT + b.ft;
    const uint8_t* wt = static_cast<const uint8_t*>(d.w13p) + (tile * KB + kb0) * 2048 + lane * 16;
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      b.w1[q] = load16_nt(wt + q * 2048);
      b.w3[q] = load16_nt(wt + q * 2048 + 1024);
    }
    const uint32_t* st = static_cast<const uint32_t*>(d.w13p_s) + tile * KG * 2 * 64 + lane;
#pragma unroll
    for (int q = 0; q < (NKB + 3) / 4; ++q) {
      const int kg = min(kg0 + q, KG - 1);
      b.s1[q] = st[(kg * 2 + 0) * 64];
      b.s3[q] = st[(kg * 2 + 1) * 64];
    }
    // the epilogue's row map travels with the tiles: loaded inside process it
    // would be issued after the next item's tiles and its wait would include them
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = min(g * 4 + i, T - 1);
      b.q[i] = ws.umap[b.u * T + t];
      b.wt[i] = ws.uwt[b.u * T + t];
    }
  };

  auto process = [&](const W13Buf<NKB>& b, int par) {
    v4f acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const int kk = kb0 + q, qi = (kk >> 2) - kg0, sh = 8 * (kk & 3);
      const int e1 = int(((qi ? b.s1[1] : b.s1[0]) >> sh) & 0xFFu);
      const int e3 = int(((qi ? b.s3[1] : b.s3[0]) >> sh) & 0xFFu);
      const v8i w1 = v8i{b.w1[q][0], b.w1[q][1], b.w1[q][2], b.w1[q][3], 0, 0, 0, 0};
      const v8i w3 = v8i{b.w3[q][0], b.w3[q][1], b.w3[q][2], b.w3[q][3], 0, 0, 0, 0};
      acc[0] = mfma_scaled<kFmtFp8, kFmtFp4>(av[q], w1, acc[0], ae[q], e1);
      acc[1] = mfma_scaled<kFmtFp8, kFmtFp4>(av[q], w3, acc[1], ae[q], e3);
    }
    float* r = red[par];
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) r[((wave * 2 + m) * 4 + i) * kWave + lane] = acc[m][i];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float gs = r[((0 * 2 + 0) * 4 + i) * kWave + lane], us = r[((0 * 2 + 1) * 4 + i) * kWave + lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
          gs += r[((w * 2 + 0) * 4 + i) * kWave + lane];
          us += r[((w * 2 + 1) * 4 + i) * kWave + lane];
        }
        const int t = g * 4 + i;
        if (t < T && b.q[i] >= 0 && b.q[i] < T * d.topk)
          ws.h[int64_t(b.q[i]) * I + b.ft * 16 + nl] = f32_to_bf16(b.wt[i] * swiglu(gs, us, d.swiglu_limit));
      }
    }
  };

  W13Buf<NKB> b0, b1;
  fetch(b0, i0);
  // the A operand after the first item's tiles: token rows past T read row
  // T - 1 (their outputs are dropped), so its loads go out as one batch
  {
    const uint8_t* arow = ws.xq + int64_t(min(nl, T - 1)) * D;
    const float* asrow = ws.xs + int64_t(min(nl, T - 1)) * (D / 128);
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const AOp a = a_from_fp8_row(arow, asrow, kb0 + q, g, a_kind);
      av[q] = a.v;
      ae[q] = a.se8;
    }
  }
  int i = i0;
  // steady state: the next item's fetch is always valid
  for (; i + 2 * G < N; i += 2 * G) {
    fetch(b1, i + G);
    process(b0, 0);
    __builtin_amdgcn_sched_barrier(0);
    fetch(b0, i + 2 * G);
    process(b1, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  // last one or two items
  if (i + G < N) {
    fetch(b1, i + G);
    process(b0, 0);
    process(b1, 1);
  } else {
    process(b0, 0);
  }
}

__global__ __launch_bounds__(kDecThreads) void hquant_kernel(MoeWs ws, int T, int k, int I, int u_max, bool pow2) {
  const int r = blockIdx.x, UT = u_max * T;
  const uint16_t* src;
  if (r < UT) {
    const int q = ws.umap[r];  // h holds the (expert, token) row at its pair row
    if (r / T >= min(ws.n_active[0], u_max) || q < 0 || q >= T * k) return;
    src = ws.h + int64_t(q) * I;
  } else {
    src = ws.sh_h + int64_t(r - UT) * I;
  }
  quant_row(ws.hq + int64_t(r) * I, ws.hs + int64_t(r) * (I / 128), src, I, pow2);
}

// --------------------------------------------------------------------- w2 ---

constexpr int kW2Waves = 16;
constexpr int kW2Threads = kW2Waves * 64;

// One workgroup per 16 output columns; jobs go to waves round-robin: the
// shared expert (FP8, twice the bytes of a routed expert per column) as two K
// halves first, then every active routed expert over the full K.  Every load
// of a batch (weight tiles, their scales, the batch's A blocks) is issued
// before the first wait: token rows past T read row T - 1 (their MFMA output
// rows are dropped) and K-blocks past the end re-read the last one (their
// MFMAs are skipped), so no load sits behind a branch.  Each job's 16-column
// result for the batch's token rows lands in LDS; the workgroup then sums each
// token's experts in ascending id, adds the shared expert and writes bf16 y.
__global__ __launch_bounds__(kW2Threads) void w2_combine_kernel(wz_moe_desc d, MoeWs ws, int T, int u_max,
                                                                uint16_t* __restrict__ y) {
  constexpr int kShParts = 2;
  __shared__ float out_s[kMaxDecPairs][16];  // routed pair (its pair row) x 16 columns
  __shared__ float sh_s[kShParts][kDecodeMaxT][16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, k = d.topk;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int a_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  const int dt = blockIdx.x, n0 = dt * 16;
  const int KB = I / 128, KG = (KB + 3) / 4, DT = D / 16, UT = u_max * T;
  const int P = T * k;
  const int n_act = min(ws.n_active[0], u_max);
  const int nrow = min(nl, T - 1);
  for (int job = wave; job < kShParts + n_act; job += kW2Waves) {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (job < kShParts) {
      const uint8_t* arow = ws.hq + int64_t(UT + nrow) * I;
      const float* asrow = ws.hs + int64_t(UT + nrow) * (I / 128);
      const uint8_t* tiles = static_cast<const uint8_t*>(d.sh2p) + int64_t(dt) * KB * 2048;
      const bool bp = d.shared_w_scale_kind == WZ_WSCALE_E8M0;
      const int64_t sbase = int64_t(n0 >> 7) * KB;
      const int kb0 = job * KB / kShParts, kb1 = (job + 1) * KB / kShParts;
      for (int kb = kb0; kb < kb1; kb += 4) {
        v8i w[4];
        int se[4];
        float sf[4];
        AOp a[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int kk = min(kb + q, kb1 - 1);
          w[q] = pk_fp8(tiles + int64_t(kk) * 2048, lane);
          fp8_wscale(d.sh_w2_s, sbase + kk, d.shared_w_scale_kind, se[q], sf[q]);
          a[q] = a_from_fp8_row(arow, asrow, kk, g, a_kind);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (kb + q < kb1) mma_step<kFmtFp8, kFmtFp8>(acc, a[q], w[q], se[q], sf[q], a_pow2, bp, lane);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g * 4 + i < T) sh_s[job][g * 4 + i][nl] = acc[i];
    } else {
      const int u = job - kShParts;
      const uint8_t* arow = ws.hq + int64_t(u * T + nrow) * I;
      const float* asrow = ws.hs + int64_t(u * T + nrow) * (I / 128);
      const int e = clampi(ws.active[u], 0, d.n_experts - 1);
      const uint8_t* wt = static_cast<const uint8_t*>(d.w2p) + (int64_t(e) * DT + dt) * KB * 1024 + lane * 16;
      const uint32_t* st = static_cast<const uint32_t*>(d.w2p_s) + (int64_t(e) * DT + dt) * KG * 64 + lane;
      int qrow[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) qrow[i] = g * 4 + i < T ? ws.umap[u * T + g * 4 + i] : -1;
      for (int kb = 0; kb < KB; kb += 4) {  // one scale dword per batch of 4 K-blocks
        v4i w[4];
        AOp a[4];
        const uint32_t sc = st[(kb >> 2) * 64];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int kk = min(kb + q, KB - 1);
          w[q] = load16_nt(wt + int64_t(kk) * 1024);
          a[q] = a_from_fp8_row(arow, asrow, kk, g, a_kind);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (kb + q < KB) {
            const int es = int((sc >> (8 * q)) & 0xFFu);
            const v8i wb = v8i{w[q][0], w[q][1], w[q][2], w[q][3], 0, 0, 0, 0};
            mma_step<kFmtFp8, kFmtFp4>(acc, a[q], wb, es, 1.0f, a_pow2, true, lane);
          }
      }
      // each linear's output is bf16 (architecture.py:741)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (qrow[i] >= 0 && qrow[i] < P) out_s[qrow[i]][nl] = bf16_round(acc[i]);
    }
  }
  __syncthreads();
  if (tid < 16 * T) {
    const int t = tid >> 4, col = tid & 15;
    const int n = clampi(ws.tok_n[t], 0, k);
    float acc = 0.0f;
    for (int j = 0; j < n; ++j) acc += out_s[clampi(ws.tok_pos[t * k + j], 0, P - 1)][col];
    acc += bf16_round(sh_s[0][t][col] + sh_s[1][t][col]);
    y[int64_t(t) * D + n0 + col] = f32_to_bf16(acc);
  }
}

// ------------------------------------------------- w2 (A rows in LDS) ---
//
// One workgroup per 16 output columns, with the A operand read from LDS.
//
// * The shared expert (FP8) is split over the 16 waves by K-block (wave w:
//   K-block w, 2 KB of tiles and its scale).  Nothing about it depends on the
//   routing, so its loads go out before any routed tile's and stream while the
//   image is built; its partials meet in K order in the combine.
// * The workgroup copies into LDS, act_quant-ed (torch_ops.py:33-49), every
//   e4m3 h row it can need: one per routed (expert, token) pair, at its pair
//   row q < P, then the T shared rows.
// * The routed experts are the jobs: wave w takes active experts w, w + 16,
//   ... over the full K (MXFP4).  A wave's registers hold only weight tiles:
//   the NS = I / 128 one-KB tile slots of its job are in flight at once, and
//   while it computes job j the tiles of job j + 16 are requested slot by slot
//   into the registers just consumed.
// * Every load instruction runs in every wave, as a buffer load whose range
//   is empty where there is nothing to read (a wave with no job or no next
//   job, h chunks past the image): such a lane reads zeros without a memory
//   request.  Counted waits (s_waitcnt vmcnt) then stay exact; with the loads
//   behind branches the compiler waited for a whole batch of tiles before the
//   first h chunk could be quantised, and clamped re-reads of one address
//   piled onto one channel.
// * Request order: the routing tables, the image's h chunks (NQ per thread,
//   the host's smallest choice that holds the image in one pass, else 8 with
//   the next pass requested ahead), the shared expert's K-block, then the
//   first job's scales and its first tile slots.  The image is quantised while
//   those are in flight; the rest of the first job's tiles follow the barrier.
//   Loads return in issue order and a CU serves a bounded number at once, so
//   the chunks queued behind a batch of tiles had waited for the batch (with
//   the tiles first the image was ready at 10 / 14 us at T = 1 / 4); in this
//   order it waits on the h read alone, which the tile stream still slows
//   (ready at about 7.6 / 9 us).
constexpr int kW2LdsBytes = 152 * 1024;

// LDS bytes of w2_lds_kernel: A rows, their scales, umap, active ids and
// first pair rows, the per-token combine lists, the pair outputs and the
// shared expert's per-wave K-block partials.
__host__ __device__ inline int64_t w2_lds_bytes(int64_t T, int64_t k, int64_t I, int64_t u_max) {
  const int64_t P = T * k, R = P + T, KB = I / 128;
  return ((R * I + 1023) & ~int64_t(1023)) + ((R * KB * 4 + 255) & ~int64_t(255)) +
         4 * (u_max * T + 2 * u_max + P + T + P * 16 + kW2Waves * T * 16);
}

// POW2: activation scales are powers of two (they ride in the MFMA).  NQ: h
// chunks per thread and pass of the image (2, 4 or 8; the host picks the
// smallest that holds the image in one pass, else 8).  PF: more than one pass,
// the next pass's chunks requested before the current pass is quantised.
// The registers the image does not take hold the first job's early tiles.
template <int NS, bool POW2, int NQ, bool PF>
__global__ __launch_bounds__(kW2Threads) void w2_lds_kernel(wz_moe_desc d, MoeWs ws, int T, int u_max,
                                                            uint16_t* __restrict__ y) {
  __shared__ __align__(1024) uint8_t smem[kW2LdsBytes];
  constexpr int KB = NS, I = NS * 128, KG = (KB + 3) / 4;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, k = d.topk, E = d.n_experts;
  const int dt = blockIdx.x, n0 = dt * 16, DT = D / 16;
  const int P = T * k, R = P + T, UT = u_max * T;
  const int a_bytes = (R * I + 1023) & ~1023, as_bytes = (R * KB * 4 + 255) & ~255;
  float* as_s = reinterpret_cast<float*>(smem + a_bytes);           // [R][KB] scales of the A rows
  int* um_s = reinterpret_cast<int*>(smem + a_bytes + as_bytes);    // [UT] umap
  int* act_s = um_s + UT;                                   // [u_max] active expert ids
  int* uf_s = act_s + u_max;                                // [u_max] first routed pair of expert u
  int* tp_s = uf_s + u_max;                                 // [P] tok_pos
  int* tn_s = tp_s + P;                                     // [T] tok_n
  float* out_s = reinterpret_cast<float*>(tn_s + T);        // [P][16] routed pair outputs
  float* sh_s = out_s + P * 16;                             // [16 waves][T][16] shared K-block partials

  // Order of requests: the routing tables, the h rows of the image (two passes'
  // worth), the shared expert's K-block, the first job's scales and its first
  // kPre tile slots; the rest of its tiles once the image is in LDS.  Loads
  // complete in issue order and every CU serves a bounded number of them at
  // once, so a load requested behind a batch of tiles waits for the batch.

  // Buffer loads: a lane whose offset is past num_records reads zeros and
  // makes no memory request, so every thread issues every load with no lane
  // re-reading another's address.
  auto rs_of = [](const void* p, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), short(0), bytes, 0x00020000);
  };
  auto bload_i32 = [&](__amdgpu_buffer_rsrc_t r) {
    return __builtin_bit_cast(int, __builtin_amdgcn_raw_buffer_load_b32(r, tid * 4, 0, 0));
  };
  // ---- the routing tables: one load per thread and table (the host keeps
  // u_max * T within one load per thread) ----
  const int um_v = bload_i32(rs_of(ws.umap, UT * 4));
  const int act_v = bload_i32(rs_of(ws.active, u_max * 4));
  const int tp_v = bload_i32(rs_of(ws.tok_pos, P * 4));
  const int tn_v = bload_i32(rs_of(ws.tok_n, T * 4));
  const int nact_v = ws.n_active[0];

  // ---- A rows: act_quant (torch_ops.py:33-49, the arithmetic of quant_row)
  // of the bf16 h rows, into LDS as e4m3 codes and block scales.  The image is
  // h's first R rows: row q < P is pair row q (the w1/w3 launch stores a
  // routed (expert, token) at its pair row; a row no pair owns holds stale
  // values and is never read as an operand), rows P .. P + T - 1 the shared
  // rows (sh_h).  A 16-lane group takes one 128-block (8 elements per lane),
  // kQ chunks per thread and pass; the next pass's chunks are requested before
  // the current pass is quantised.  Chunks past the image are out of the
  // buffer's range: zeros, no request, not stored. ----
  constexpr int CPR = I / 8;  // 16-byte chunks per row
  constexpr int kQ = NQ;
  const int nch = R * CPR;
  const __amdgpu_buffer_rsrc_t h_rs = rs_of(ws.h, nch * 16);
  // chunk c_base + tid; the whole offset in the lane's offset register (the
  // range check covers that one, not the scalar offset)
  auto h_chunk = [&](int c_base) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(h_rs, (c_base + tid) * 16, 0, 0));
  };
  // Chunks wholly past the image are skipped (a wave-uniform test).  In a
  // wave whose blocks are all finite the clamp to +-448 is left out: with a
  // power-of-two scale s >= amax / 448, |x / s| <= 448 already.
  auto quant_pass = [&](int c0, const v4i (&hv)[kQ]) {
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
      const int cb = c0 + i * kW2Threads;
      if (cb >= nch) continue;
      const int c = cb + tid;
      const float amax = row16_absmax(bf16x8_absmax(hv[i]));
      const ActScale sc = act_scale(amax, POW2);
      float f[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        f[2 * q] = bf16lo(uint32_t(hv[i][q]));
        f[2 * q + 1] = bf16hi(uint32_t(hv[i][q]));
      }
      uint32_t lo, hi;
      if (POW2 && __ballot(!is_finite_f32(amax)) == 0ull) {
        lo = pack_fp8x4(f[0] * sc.inv, f[1] * sc.inv, f[2] * sc.inv, f[3] * sc.inv);
        hi = pack_fp8x4(f[4] * sc.inv, f[5] * sc.inv, f[6] * sc.inv, f[7] * sc.inv);
      } else {
        lo = pack_fp8x4(quant_div(f[0], sc, POW2), quant_div(f[1], sc, POW2), quant_div(f[2], sc, POW2),
                        quant_div(f[3], sc, POW2));
        hi = pack_fp8x4(quant_div(f[4], sc, POW2), quant_div(f[5], sc, POW2), quant_div(f[6], sc, POW2),
                        quant_div(f[7], sc, POW2));
      }
      if (c < nch) {
        const int row = c / CPR, off = (c % CPR) * 8;
        *reinterpret_cast<uint2*>(smem + row * I + off) = make_uint2(lo, hi);
        if ((lane & 15) == 0) as_s[row * KB + off / 128] = sc.s;
      }
    }
  };
  v4i hv[kQ], hn[PF ? kQ : 1];
#pragma unroll
  for (int i = 0; i < kQ; ++i) hv[i] = h_chunk(i * kW2Threads);
  if constexpr (PF) {
#pragma unroll
    for (int i = 0; i < kQ; ++i) hn[i] = h_chunk((kQ + i) * kW2Threads);
  }

  // ---- the shared expert's K-block of this wave: tiles and block scale.
  // Waves past KB re-read K-block KB - 1 and skip its MFMA.  Both scale kinds'
  // loads are issued (the unused one reads the array's first element) and
  // selected, so no load sits behind a branch. ----
  const int kb_s = min(wave, KB - 1);
  const uint8_t* sh_tile = static_cast<const uint8_t*>(d.sh2p) + (int64_t(dt) * KB + kb_s) * 2048 + lane * 16;
  const v4i sw0 = load16_nt(sh_tile), sw1 = load16_nt(sh_tile + 1024);
  const int sidx = (n0 >> 7) * KB + kb_s;
  const bool sh_e8 = d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  const uint8_t sh_b = static_cast<const uint8_t*>(d.sh_w2_s)[sh_e8 ? sidx : 0];
  const float sh_f = static_cast<const float*>(d.sh_w2_s)[sh_e8 ? 0 : sidx];
  __builtin_amdgcn_sched_barrier(0);

  // ---- routed job u: buffer resources over expert e's tiles and scales,
  // empty (num_records 0: the loads return zeros without a memory request)
  // when there is no such job, so a wave with no job issues the same
  // instructions ----
  auto tiles_rs = [&](int e, bool ok) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(static_cast<const uint8_t*>(d.w2p) + (int64_t(e) * DT + dt) * KB * 1024), short(0),
        ok ? KB * 1024 : 0, 0x00020000);
  };
  auto scales_rs = [&](int e, bool ok) {
    return __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(static_cast<const uint32_t*>(d.w2p_s) + (int64_t(e) * DT + dt) * KG * 64), short(0),
        ok ? KG * 256 : 0, 0x00020000);
  };
  // 16 bytes per lane, non-temporal (read once)
  auto bload16 = [&](__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(r, lane * 16, off, 2));
  };
  auto bload4 = [&](__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_raw_buffer_load_b32(r, lane * 4, off, 0));
  };
  // ---- the first job (active expert `wave`): its id read here (one
  // wave-uniform word), its scales and first kPre tile slots requested before
  // the image is quantised; the rest after ----
  const int n_act = min(nact_v, u_max);
  constexpr int kPre = PF ? (NS < 2 ? NS : 2) : NQ <= 2 ? NS : NQ <= 4 ? (NS < 12 ? NS : 12) : (NS < 8 ? NS : 8);
  v4i w[NS];
  uint32_t sc[KG];
  const bool ok0 = wave < n_act;
  const int e0 = __builtin_amdgcn_readfirstlane(clampi(ws.active[min(wave, u_max - 1)], 0, E - 1));
  const __amdgpu_buffer_rsrc_t t_rs0 = tiles_rs(e0, ok0), s_rs0 = scales_rs(e0, ok0);
#pragma unroll
  for (int c = 0; c < KG; ++c) sc[c] = bload4(s_rs0, c * 256);
#pragma unroll
  for (int s = 0; s < kPre; ++s) w[s] = bload16(t_rs0, s * 1024);
  __builtin_amdgcn_sched_barrier(0);

  // ---- the tables into LDS ----
  if (tid < UT) um_s[tid] = um_v;
  if (tid < u_max) {
    act_s[tid] = clampi(act_v, 0, E - 1);
    uf_s[tid] = P;
  }
  if (tid < P) tp_s[tid] = clampi(tp_v, 0, P - 1);
  if (tid < T) tn_s[tid] = clampi(tn_v, 0, k);
  // ---- the image, pass by pass ----
  quant_pass(0, hv);  // out of the loop, so its waits cover its own chunks alone
  for (int c0 = kQ * kW2Threads; c0 < nch; c0 += kQ * kW2Threads) {
    if constexpr (PF) {
#pragma unroll
      for (int i = 0; i < kQ; ++i) hv[i] = hn[i];
#pragma unroll
      for (int i = 0; i < kQ; ++i) hn[i] = h_chunk(c0 + (kQ + i) * kW2Threads);
    } else {
#pragma unroll
      for (int i = 0; i < kQ; ++i) hv[i] = h_chunk(c0 + i * kW2Threads);
    }
    quant_pass(c0, hv);
  }
  // Bare barriers: __syncthreads' fence would wait for the shared tiles.
  __builtin_amdgcn_s_waitcnt(lgkmcnt_only(0));
  asm volatile("s_barrier" : : : "memory");
  // the first routed pair row of each expert
  if (tid < UT && um_v >= 0 && um_v < P) atomicMin(&uf_s[tid / T], um_v);
  __builtin_amdgcn_s_waitcnt(lgkmcnt_only(0));
  asm volatile("s_barrier" : : : "memory");

#pragma unroll
  for (int s = kPre; s < NS; ++s) w[s] = bload16(t_rs0, s * 1024);

  // A operand of K-block kk from LDS row `row`
  auto a_lds = [&](int row, int kk) {
    AOp a = a_zero();
    const uint8_t* p = smem + row * I + kk * 128 + g * 16;
    const v4i lo = *reinterpret_cast<const v4i*>(p), hi = *reinterpret_cast<const v4i*>(p + 64);
    a.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    const float s = as_s[row * KB + kk];
    if constexpr (POW2)
      a.se8 = int((__float_as_uint(s) >> 23) & 0xFFu);
    else
      a.sf = s;
    return a;
  };

  const int trow = min(nl, T - 1);
  // ---- the shared expert's K-block (FP8: one MFMA over its two slots) ----
  {
    v4f acc = {0.f, 0.f, 0.f, 0.f};
    if (wave < KB) {
      const AOp a = a_lds(P + trow, kb_s);
      const v8i wb = v8i{sw0[0], sw0[1], sw0[2], sw0[3], sw1[0], sw1[1], sw1[2], sw1[3]};
      mma_step<kFmtFp8, kFmtFp8>(acc, a, wb, sh_e8 ? int(sh_b) : kE8m0One, sh_e8 ? 1.0f : sh_f, POW2, sh_e8, lane);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (g * 4 + i < T) sh_s[(wave * T + g * 4 + i) * 16 + nl] = acc[i];
  }

  // Keeps slot s's MFMA ahead of the load that refills slot s: without it the
  // MFMAs (pure) sink to the end of the job and every old tile stays live.
  auto pin = [](v4f& acc) { asm volatile("" : "+v"(acc) : : "memory"); };
  // routed job u (expert u, full K); requests job u + 16's scales and tiles,
  // slot s right after slot s's MFMA
  for (int u = wave; u < n_act; u += kW2Waves) {
    const int q = um_s[u * T + trow], qf = uf_s[u];
    // a token not routed to u reads u's first routed row (its output row is
    // dropped below), so the wave reads few distinct LDS rows
    const int lrow = (q >= 0 && q < P) ? q : (qf < P ? qf : P + trow);
    const int un = u + kW2Waves;
    const int en = __builtin_amdgcn_readfirstlane(act_s[un < n_act ? un : 0]);
    const __amdgpu_buffer_rsrc_t t_rs = tiles_rs(en, un < n_act), s_rs = scales_rs(en, un < n_act);
    uint32_t scn[KG];
#pragma unroll
    for (int c = 0; c < KG; ++c) scn[c] = bload4(s_rs, c * 256);
    v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const AOp a = a_lds(lrow, s);
      const int es = int((sc[s >> 2] >> (8 * (s & 3))) & 0xFFu);
      const v8i wb = v8i{w[s][0], w[s][1], w[s][2], w[s][3], 0, 0, 0, 0};
      mma_step<kFmtFp8, kFmtFp4>(acc, a, wb, es, 1.0f, POW2, true, lane);
      pin(acc);
      w[s] = bload16(t_rs, s * 1024);
    }
#pragma unroll
    for (int c = 0; c < KG; ++c) sc[c] = scn[c];
    // each linear's output is bf16 (architecture.py:741)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = g * 4 + i;
      const int qo = t < T ? um_s[u * T + t] : -1;
      if (qo >= 0 && qo < P) out_s[qo * 16 + nl] = bf16_round(acc[i]);
    }
  }
  __syncthreads();
  if (tid < 16 * T) {
    const int t = tid >> 4, col = tid & 15;
    const int n = tn_s[t];
    float acc = 0.0f;
    for (int jj = 0; jj < n; ++jj) acc += out_s[tp_s[t * k + jj] * 16 + col];
    // the shared expert: its K-blocks' partials in K order, one bf16 output
    float sh = 0.0f;
    for (int w2 = 0; w2 < min(KB, kW2Waves); ++w2) sh += sh_s[(w2 * T + t) * 16 + col];
    acc += bf16_round(sh);
    y[int64_t(t) * D + n0 + col] = f32_to_bf16(acc);
  }
}

// ------------------------------------------------------- w2 (streamed) ---
//
// Routed experts' w2 on persistent workgroups, then combine_decode.
// Work item = (active expert u, 64 output columns): four 16-column tiles over
// the full K = I, 64 KB of packed MXFP4, contiguous in the packed bank.  A
// workgroup takes a contiguous run of items, so consecutive items share the
// expert and its A operand (the expert's e4m3 h rows for this wave's quarter
// of K) stays in registers until the expert changes.  Each wave computes its
// K quarter of all four tiles; the quarters meet in LDS; the bf16 expert
// output goes to its pair row out2[q].  The next item's tiles are in flight
// while the current one computes.  The shared expert's 64-column groups
// (FP8) are the first D/64 workgroups and write sh_out.
template <int NKB>
struct W2Buf {
  v4i w[4][NKB];
  uint32_t s[4];  // packed e8m0 dword of each column tile (this wave's K quarter)
  int q[4];       // pair rows of this lane's four token rows (-1: unrouted), fetched with the tiles
  int u, g64;
};

__device__ __forceinline__ void w2_shared_group(const wz_moe_desc& d, const MoeWs& ws, int T, int u_max,
                                                int grp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, KB = I / 128;
  const bool a_pow2 = d.act_scale_kind != WZ_SCALE_F32;
  const int a_kind = a_pow2 ? WZ_SCALE_UE8M0_F32 : WZ_SCALE_F32;
  const bool bp = d.shared_w_scale_kind == WZ_WSCALE_E8M0;
  const int UT = u_max * T;
  // rows past T read row T - 1 (their outputs are not stored), so every load of
  // a batch is issued before the first wait
  const int nrow = min(nl, T - 1);
  const uint8_t* arow = ws.hq + int64_t(UT + nrow) * I;
  const float* asrow = ws.hs + int64_t(UT + nrow) * (I / 128);
  const int dt = grp * 4 + wave, n0 = dt * 16;  // wave w: column tile 4 grp + w, full K
  const uint8_t* tiles = static_cast<const uint8_t*>(d.sh2p) + int64_t(dt) * KB * 2048;
  const int64_t sbase = int64_t(n0 >> 7) * KB;
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  for (int kb = 0; kb < KB; kb += 4) {
    v8i w[4];
    int se[4];
    float sf[4];
    AOp a[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int kk = min(kb + q, KB - 1);
      w[q] = pk_fp8(tiles + int64_t(kk) * 2048, lane);
      fp8_wscale(d.sh_w2_s, sbase + kk, d.shared_w_scale_kind, se[q], sf[q]);
      a[q] = a_from_fp8_row(arow, asrow, kk, g, a_kind);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (kb + q < KB) mma_step<kFmtFp8, kFmtFp8>(acc, a[q], w[q], se[q], sf[q], a_pow2, bp, lane);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = g * 4 + i;
    if (t < T) ws.sh_out[int64_t(t) * D + n0 + nl] = f32_to_bf16(acc[i]);
  }
}

// NKB = K-blocks per wave = I / 512 (compile time: no conditional loads).
template <int NKB>
__global__ __launch_bounds__(kDecThreads) void w2_stream_kernel(wz_moe_desc d, MoeWs ws, int T, int u_max) {
  __shared__ float red[2][4 * 4 * 4 * kWave];
  __shared__ int s_act[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int D = d.dim, I = d.inter, E = d.n_experts, P = T * d.topk;
  const int KB = 4 * NKB, KG = (KB + 3) / 4, DT = D / 16, NG = D / 64;
  const int kb0 = wave * NKB, kg0 = kb0 >> 2;
  if (int(blockIdx.x) < NG) {
    w2_shared_group(d, ws, T, u_max, blockIdx.x);
    return;
  }
  const int n_act = min(ws.n_active[0], u_max);
  const int N = n_act * NG;
  const int G = gridDim.x - NG, b = blockIdx.x - NG;
  const int i0 = int((int64_t(b) * N) / G), i1 = int((int64_t(b + 1) * N) / G);
  if (i0 >= i1) return;
  for (int j = tid; j < n_act; j += kDecThreads) s_act[j] = clampi(ws.active[j], 0, E - 1);
  __syncthreads();

  auto fetch = [&](W2Buf<NKB>& bf, int item) {
    bf.u = item / NG;
    bf.g64 = item % NG;
    const int e = s_act[bf.u];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int64_t tile = int64_t(e) * DT + bf.g64 * 4 + c;
      const uint8_t* wt = static_cast<const uint8_t*>(d.w2p) + (tile * KB + kb0) * 1024 + lane * 16;
#pragma unroll
      for (int q = 0; q < NKB; ++q) bf.w[c][q] = load16_nt(wt + q * 1024);
      bf.s[c] = static_cast<const uint32_t*>(d.w2p_s)[(tile * KG + kg0) * 64 + lane];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) bf.q[i] = ws.umap[bf.u * T + min(g * 4 + i, T - 1)];
  };

  v8i av[NKB];
  int ae[NKB];
  int cur_u = -1;
  auto load_a = [&](int u) {  // rows past T read row T - 1 (their outputs are not stored)
    const int nrow = min(nl, T - 1);
    const uint8_t* arow = ws.hq + int64_t(u * T + nrow) * I;
    const float* asrow = ws.hs + int64_t(u * T + nrow) * (I / 128);
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const AOp a = a_from_fp8_row(arow, asrow, kb0 + q, g, WZ_SCALE_UE8M0_F32);
      av[q] = a.v;
      ae[q] = a.se8;
    }
    cur_u = u;
  };

  auto process = [&](const W2Buf<NKB>& bf, int par) {
    if (bf.u != cur_u) load_a(bf.u);
    v4f acc[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int q = 0; q < NKB; ++q) {
      const int sh = 8 * ((kb0 + q) & 3);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const v8i w = v8i{bf.w[c][q][0], bf.w[c][q][1], bf.w[c][q][2], bf.w[c][q][3], 0, 0, 0, 0};
        acc[c] = mfma_scaled<kFmtFp8, kFmtFp4>(av[q], w, acc[c], ae[q], int((bf.s[c] >> sh) & 0xFFu));
      }
    }
    float* r = red[par];
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int i = 0; i < 4; ++i) r[((wave * 4 + c) * 4 + i) * kWave + lane] = acc[c][i];
    __syncthreads();
    // wave c finishes column tile c: K quarters summed in wave order, bf16 to the pair row
    const int c = wave;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int t = g * 4 + i;
      const int q = t < T ? bf.q[i] : -1;
      float v = r[((0 * 4 + c) * 4 + i) * kWave + lane];
#pragma unroll
      for (int w = 1; w < 4; ++w) v += r[((w * 4 + c) * 4 + i) * kWave + lane];
      if (q >= 0 && q < P) ws.out2[int64_t(q) * D + (bf.g64 * 4 + c) * 16 + nl] = f32_to_bf16(v);
    }
  };

  W2Buf<NKB> b0, b1;
  fetch(b0, i0);
  int i = i0;
  for (; i + 2 < i1; i += 2) {
    fetch(b1, i + 1);
    process(b0, 0);
    __builtin_amdgcn_sched_barrier(0);
    fetch(b0, i + 2);
    process(b1, 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  if (i + 1 < i1) {
    fetch(b1, i + 1);
    process(b0, 0);
    process(b1, 1);
  } else {
    process(b0, 0);
  }
}

// y[t] = bf16(sum over the token's distinct experts, ascending id, of out2 rows
// + the shared row); tok_pos / tok_n come from the decode routing.
__global__ __launch_bounds__(256) void combine_decode_kernel(MoeWs ws, int T, int k, int D,
                                                             uint16_t* __restrict__ y) {
  const int i = blockIdx.x * 256 + threadIdx.x;  // one 8-column chunk of one token
  const int t = i / (D / 8), c = i % (D / 8);
  if (t >= T) return;
  const int P = T * k;
  const int n = clampi(ws.tok_n[t], 0, k);
  // every row is requested before the first sum: slots past n re-read the
  // token's first row and are not added
  v4i v[kDecodeMaxT];
#pragma unroll
  for (int j = 0; j < kDecodeMaxT; ++j)
    if (j < k) v[j] = load16(ws.out2 + int64_t(clampi(ws.tok_pos[t * k + (j < n ? j : 0)], 0, P - 1)) * D + c * 8);
  const v4i sv = load16(ws.sh_out + int64_t(t) * D + c * 8);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < kDecodeMaxT; ++j)
    if (j < n) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        acc[2 * m] += bf16lo(uint32_t(v[j][m]));
        acc[2 * m + 1] += bf16hi(uint32_t(v[j][m]));
      }
    }
  uint32_t o[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    o[m] = uint32_t(f32_to_bf16(acc[2 * m] + bf16lo(uint32_t(sv[m])))) |
           (uint32_t(f32_to_bf16(acc[2 * m + 1] + bf16hi(uint32_t(sv[m])))) << 16);
  *reinterpret_cast<v4i*>(y + int64_t(t) * D + c * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
}

// only < 0: the whole layer; otherwise the one stage WZ_STAGE_* (profiling replays).
// nw: x is the hidden state and the MoE input its RMSNorm (weight nw, eps),
// computed inside the route launch (D <= kNormMaxD, T <= kNormMaxT).
int launch_decode(const wz_moe_desc* d, const MoeWs& w, const void* x, const int64_t* ids, int64_t T,
                  void* y, hipStream_t stream, int only, const float* nw, float eps) {
  const int E = d->n_experts, k = d->topk, D = d->dim, I = d->inter;
  // K-split of the gate: the largest of 8, 4, 2, 1 waves per expert that keeps
  // the gate within 128 workgroups (of 8 waves)
  int split = 8;
  while (split > 1 && int64_t(E) * split > 128 * kRouteWaves) split >>= 1;
  const int n_gate = int((int64_t(E) * split + kRouteWaves - 1) / kRouteWaves);
  const int64_t P = T * k;
  const int u_max = int(P < E ? P : E);
  if (P > kMaxDecPairs) return set_error(WZ_EINVAL, "moe decode: T*topk=%lld exceeds %d", (long long)P, kMaxDecPairs);
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe decode: packed banks missing (wz_moe_pack)");
  if (only < 0 || only == WZ_STAGE_ROUTE) {
    // top-k lanes walk E / 64 slots: 4 for up to 256 experts, else 8
    if (T > I / 16) return set_error(WZ_EINVAL, "moe decode: T=%lld exceeds the %d shared items", (long long)T, I / 16);
    const dim3 rgrid{unsigned(n_gate + I / 16)};
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    if (nw && (D > kNormMaxD || T > kNormMaxT))
      return set_error(WZ_EINVAL, "moe decode: the fused norm serves D <= %d and T <= %d (D=%d, T=%lld)",
                       kNormMaxD, kNormMaxT, D, (long long)T);
#define WZ_RK(KS, NORM)                                                                                       \
  WZ_LAUNCH("moe_route", stream, (route_decode_kernel<KS, NORM>), rgrid, dim3(kRouteThreads_), 0, *d, w, xb, ids, \
            int(T), n_gate, split, u_max, nw, eps)
    if (E <= 256) {
      if (nw) WZ_RK(4, true); else WZ_RK(4, false);
    } else {
      if (nw) WZ_RK(8, true); else WZ_RK(8, false);
    }
#undef WZ_RK
    if (int rc = check_launch("moe route")) return rc;
  }
  if (only < 0 || only == WZ_STAGE_W13) {
    const int nkb = D / 512;
    if (D % 512 == 0 && (nkb == 1 || nkb == 2 || nkb == 4 || nkb == 8) && d->act_scale_kind != WZ_SCALE_F32) {
      // routed WGs: two per CU (measured 0.5-2 us faster than one per CU at T = 1..4);
      // the shared expert's w1 / w3 ran in the route launch
      const int64_t items = int64_t(u_max) * (I / 16), cus = cu_count();
      const dim3 grid(unsigned(std::min<int64_t>(items, 2 * cus)));
      if (nkb == 8) {
        WZ_LAUNCH("moe_w13", stream, w13_stream_kernel<8>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      } else if (nkb == 4) {
        WZ_LAUNCH("moe_w13", stream, w13_stream_kernel<4>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      } else if (nkb == 2) {
        WZ_LAUNCH("moe_w13", stream, w13_stream_kernel<2>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      } else {
        WZ_LAUNCH("moe_w13", stream, w13_stream_kernel<1>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      }
    } else {
      WZ_LAUNCH("moe_w13", stream, w13_decode_kernel, dim3(unsigned(u_max * (I / 16))), dim3(kDecThreads), 0,
                *d, w, int(T), u_max);
    }
    if (int rc = check_launch("moe w13")) return rc;
  }
  // w2_lds_kernel wherever its LDS image fits (V4: T <= 8; 21.5 / 35.4 us at
  // T = 4 / 8 against 25.1 us for w2_combine_kernel and 41.9 us for the
  // streamed w2 plus its combine launch).  Otherwise the streamed pair at
  // T >= 6 and w2_combine_kernel below.  w2_lds_kernel quantises h itself.
  const int nkb2 = I / 512, kb2 = I / 128;
  // K-blocks of 2 .. 16 (16 only with power-of-two activation scales: the
  // float-scale variant spills there), the LDS image fits, the (expert, token)
  // map takes one load per thread, and the shared expert's w2 scale array
  // holds at least one 4-byte word (both kinds' first elements are read)
  const bool p2 = d->act_scale_kind != WZ_SCALE_F32;
  const bool w2l = I % 128 == 0 && (kb2 == 2 || kb2 == 4 || kb2 == 8 || (kb2 == 16 && p2)) &&
                   w2_lds_bytes(T, k, I, u_max) <= kW2LdsBytes && int64_t(u_max) * T <= kW2Threads &&
                   (D / 128) * kb2 >= 4;
  if (!w2l && (only < 0 || only == WZ_STAGE_HQUANT)) {
    WZ_LAUNCH("moe_hquant", stream, hquant_kernel, dim3(unsigned(u_max * T + T)), dim3(kDecThreads), 0, w, int(T),
              k, I, u_max, d->act_scale_kind != WZ_SCALE_F32);
    if (int rc = check_launch("moe hquant")) return rc;
  }
  const bool w2s = !w2l && T >= 6 && I % 512 == 0 && (nkb2 == 1 || nkb2 == 2 || nkb2 == 4) && D % 64 == 0 &&
                   d->act_scale_kind != WZ_SCALE_F32;
  if (only < 0 || only == WZ_STAGE_W2) {
    if (w2l) {
      const dim3 grid{unsigned(D / 16)};
      uint16_t* yo = static_cast<uint16_t*>(y);
      const int64_t cpt = (int64_t(T) * (k + 1) * (I / 8) + kW2Threads - 1) / kW2Threads;  // h chunks per thread
#define WZ_W2L_P(NS, P2, NQ, PF) \
  WZ_LAUNCH("moe_w2", stream, (w2_lds_kernel<NS, P2, NQ, PF>), grid, dim3(kW2Threads), 0, *d, w, int(T), u_max, yo)
#define WZ_W2L(NS)                    \
  do {                                \
    if (p2)                           \
      WZ_W2L_P(NS, true, 8, false);   \
    else                              \
      WZ_W2L_P(NS, false, 8, false);  \
  } while (0)
      if (kb2 == 16) {
        if (cpt <= 2)
          WZ_W2L_P(16, true, 2, false);
        else if (cpt <= 4)
          WZ_W2L_P(16, true, 4, false);
        else if (cpt <= 8)
          WZ_W2L_P(16, true, 8, false);
        else
          WZ_W2L_P(16, true, 8, true);
      } else if (kb2 == 8) {
        WZ_W2L(8);
      } else if (kb2 == 4) {
        WZ_W2L(4);
      } else {
        WZ_W2L(2);
      }
#undef WZ_W2L
#undef WZ_W2L_P
    } else if (w2s) {
      const int64_t items = int64_t(u_max) * (D / 64), cus = cu_count();
      const dim3 grid(unsigned(D / 64 + std::min<int64_t>(items, std::max<int64_t>(cus, std::min<int64_t>(2 * cus, items / 8)))));
      if (nkb2 == 4) {
        WZ_LAUNCH("moe_w2", stream, w2_stream_kernel<4>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      } else if (nkb2 == 2) {
        WZ_LAUNCH("moe_w2", stream, w2_stream_kernel<2>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      } else {
        WZ_LAUNCH("moe_w2", stream, w2_stream_kernel<1>, grid, dim3(kDecThreads), 0, *d, w, int(T), u_max);
      }
    } else {
      WZ_LAUNCH("moe_w2", stream, w2_combine_kernel, dim3(unsigned(D / 16)), dim3(kW2Threads), 0, *d, w, int(T),
                u_max, static_cast<uint16_t*>(y));
    }
    if (int rc = check_launch("moe w2")) return rc;
  }
  if (w2s && (only < 0 || only == WZ_STAGE_COMBINE)) {
    const int64_t n = T * (D / 8);
    WZ_LAUNCH("moe_combine", stream, combine_decode_kernel, dim3(unsigned((n + 255) / 256)), dim3(256), 0, w,
              int(T), k, D, static_cast<uint16_t*>(y));
    if (int rc = check_launch("moe combine")) return rc;
  }
  return WZ_OK;
}

}  // namespace wz
