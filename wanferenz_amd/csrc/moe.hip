// MoE layer: gate scoring + top-k routing, canonical permutation, MXFP4 routed
// experts (w1/w3 SwiGLU, then w2), FP8 shared expert, weighted combine.
//
// Semantics: MoE.forward / Gate.forward / Expert.forward of
// wanferenz/model/architecture.py:696-794, with the canonical pair order of
// wanferenz/kernels/expert_batch.py:24-37 (experts ascending, then token,
// then slot) and the combine of fp4_grouped.py:318-324 (fp32 sum of the
// routed bf16 outputs in ascending expert id, then the shared expert, then
// bf16).  A token that lists an expert twice (hash-routed layers) receives it
// once (architecture.py:790 is a non-accumulating index_put).
//
// The layer runs as a fixed sequence of stream-ordered launches with no host
// synchronisation and no allocation, so a step can be captured in a HIP
// graph.  Grids are sized from T on the host; blocks beyond the device-side
// number of active experts return at once.  T <= 16 runs the decode kernels
// (moe_decode.hip); larger T runs the routing below and the expert-grouped
// GEMMs of moe_prefill.hip.
//
//   gate_dot   scores[T,E] = x . W^T, exact bf16 products summed in fp64, one
//              wave per (expert, 8 tokens): reads the bf16 gate once.
//   topk       one wave per token: score function, +bias, top-k (ties -> lower
//              index), renormalise, x route_scale; hash layers read tid2eid.
//   perm       one workgroup: expert counts, offsets, active-expert list and
//              the stable (expert, token, slot) permutation via wave ballots.
//   combine    y[t] = bf16(sum_{experts asc} out[t,e] + shared[t]).
#include "moe_common.h"

#include <mutex>

namespace wz {

// ------------------------------------------------------------------ gate ----

// scores[t, e] = fp32(sum_d x[t,d] * W[e,d]).  bf16 x bf16 is exact in fp32;
// the fp64 running sums make the result the correctly rounded dot product
// except in vanishingly rare cases, so the GPU and the oracle agree on the
// fp32 scores that decide the top-k.
__global__ __launch_bounds__(256) void gate_dot_kernel(const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ W,
                                                       float* __restrict__ scores, int T, int E,
                                                       int D) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave;
  const int t0 = blockIdx.y * kGateTok;
  if (e >= E) return;
  double acc[kGateTok];
#pragma unroll
  for (int i = 0; i < kGateTok; ++i) acc[i] = 0.0;
  const int nc = D / 8;
  for (int c = lane; c < nc; c += 64) {
    const v4i wv = load16(W + int64_t(e) * D + c * 8);
    float wf[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      wf[2 * j] = bf16lo(uint32_t(wv[j]));
      wf[2 * j + 1] = bf16hi(uint32_t(wv[j]));
    }
#pragma unroll
    for (int i = 0; i < kGateTok; ++i) {
      if (t0 + i < T) {
        const v4i xv = load16(x + int64_t(t0 + i) * D + c * 8);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          acc[i] += double(bf16lo(uint32_t(xv[j])) * wf[2 * j]);
          acc[i] += double(bf16hi(uint32_t(xv[j])) * wf[2 * j + 1]);
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < kGateTok; ++i) {
    double v = acc[i];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    if (lane == 0 && t0 + i < T) scores[int64_t(t0 + i) * E + e] = float(v);
  }
}

// ------------------------------------------------------------------ top-k ---

constexpr int kSlots = kMaxExperts / 64;

__global__ __launch_bounds__(256) void topk_kernel(const float* __restrict__ scores,
                                                   const float* __restrict__ bias,
                                                   const int32_t* __restrict__ tid2eid,
                                                   const int64_t* __restrict__ input_ids,
                                                   int64_t vocab, int T, int E, int k,
                                                   int score_func, float route_scale,
                                                   float* __restrict__ weights,
                                                   int32_t* __restrict__ idx) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  if (t >= T) return;
  const float* a = scores + int64_t(t) * E;
  float s[kSlots], b[kSlots];
  double mx = -1e300, sum = 0.0;
  if (score_func == WZ_SCORE_SOFTMAX) {
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int e = lane + 64 * i;
      if (e < E) mx = fmax(mx, double(a[e]));
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) mx = fmax(mx, __shfl_xor(mx, m, kWave));
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int e = lane + 64 * i;
      if (e < E) sum += exp(double(a[e]) - mx);
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, kWave);
  }
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const int e = lane + 64 * i;
    float v = -INFINITY;
    if (e < E) {
      const float ae = a[e];
      if (score_func == WZ_SCORE_SOFTMAX)
        v = float(exp(double(ae) - mx) / sum);
      else if (score_func == WZ_SCORE_SIGMOID)
        v = float(1.0 / (1.0 + exp(-double(ae))));
      else
        v = float(sqrt(double(softplus_f32(ae))));
    }
    s[i] = v;
    b[i] = (e < E && bias != nullptr) ? v + bias[e] : v;
  }
  // lane j < k ends up holding the j-th selected expert
  int my_sel = 0;
  bool poison = false;  // hash id or table entry out of range: NaN weights, in-range reads
  if (tid2eid != nullptr) {
    int64_t id = input_ids[t];
    const bool bad_id = id < 0 || id >= vocab;
    id = bad_id ? 0 : id;
    bool bad_e = false;
    if (lane < k) {
      const int e = tid2eid[id * k + lane];
      bad_e = e < 0 || e >= E;
      my_sel = bad_e ? 0 : e;
    }
    poison = bad_id || __ballot(bad_e) != 0ull;
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
  // weights = original scores gathered at the selected experts (architecture.py:714-717)
  float mine = 0.0f;
#pragma unroll
  for (int i = 0; i < kSlots; ++i) {
    const float v = __shfl(s[i], my_sel & 63, kWave);
    if ((my_sel >> 6) == i) mine = v;
  }
  float tot = 0.0f;
  for (int j = 0; j < k; ++j) tot += __shfl(mine, j, kWave);  // slot order, fp32
  float v = mine;
  if (score_func != WZ_SCORE_SOFTMAX) v = v / tot;
  v = v * route_scale;
  if (poison) v = __builtin_nanf("");
  if (lane < k) {
    weights[int64_t(t) * k + lane] = v;
    idx[int64_t(t) * k + lane] = my_sel;
  }
}

// ------------------------------------------------------------ permutation ---

__device__ __forceinline__ int block_excl_scan(int v, int* wsum, int& total) {
  // exclusive scan over the 1024 threads of the block
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    int o = __shfl_up(inc, d, kWave);
    if (lane >= d) inc += o;
  }
  if (lane == 63) wsum[wave] = inc;
  __syncthreads();
  if (threadIdx.x < 64) {
    int x = threadIdx.x < (kRouteThreads / 64) ? wsum[threadIdx.x] : 0;
    int xi = x;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      int o = __shfl_up(xi, d, kWave);
      if (threadIdx.x >= d) xi += o;
    }
    wsum[32 + threadIdx.x] = xi - x;  // exclusive prefix of wave totals
    if (threadIdx.x == 63) wsum[31] = xi;
  }
  __syncthreads();
  total = wsum[31];
  int r = inc - v + wsum[32 + wave];
  __syncthreads();
  return r;
}

// The permutation's tables from each expert's pair count c (thread e of the
// block holds expert e; E <= 1024 = block size): offsets and the active-expert
// list (offsets, counts), and the M-tile table of the prefill GEMMs (each
// active expert's pair rows cut into tiles of kPrefillTileRows, in active
// order).  Returns the expert's first slot.
__device__ int perm_tables(int c, int E, int32_t* __restrict__ offsets, int32_t* __restrict__ active,
                           int32_t* __restrict__ act_off, int32_t* __restrict__ act_cnt,
                           int32_t* __restrict__ n_active, int32_t* __restrict__ mt_u,
                           int32_t* __restrict__ mt_row0, int32_t* __restrict__ mt_n, int32_t* __restrict__ n_mt,
                           int mt_cap, int* wsum) {
  const int tid = threadIdx.x;
  int total;
  const int ex = block_excl_scan(c, wsum, total);
  const int flag = c > 0 ? 1 : 0;
  int nact;
  const int u = block_excl_scan(flag, wsum, nact);
  if (tid < E) {
    offsets[tid] = ex;
    if (flag) {
      active[u] = tid;
      act_off[u] = ex;
      act_cnt[u] = c;
    }
  }
  if (tid == 0) {
    offsets[E] = total;
    n_active[0] = nact;
  }
  const int ntile = flag ? (c + kPrefillTileRows - 1) / kPrefillTileRows : 0;
  int ntiles;
  const int mt0 = block_excl_scan(ntile, wsum, ntiles);
  for (int i = 0; i < ntile && mt0 + i < mt_cap; ++i) {
    mt_u[mt0 + i] = u;
    mt_row0[mt0 + i] = ex + i * kPrefillTileRows;
    mt_n[mt0 + i] = min(kPrefillTileRows, c - i * kPrefillTileRows);
  }
  if (tid == 0) n_mt[0] = min(ntiles, mt_cap);
  return ex;
}

// Rank of each lane's expert e among the lanes below it with the same expert
// (a match over e's nbits bits by ballots), and whether the lane is the lowest
// with it; with the invalid lanes as one group of their own.
__device__ __forceinline__ int wave_match_rank(int e, bool valid, int nbits, bool& leader,
                                               unsigned long long& group) {
  const int lane = threadIdx.x & 63;
  const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  unsigned long long mask = __ballot(valid);
  if (!valid) mask = ~mask;
  for (int bit = 0; bit < nbits; ++bit) {
    const bool on = (e >> bit) & 1;
    const unsigned long long m = __ballot(on);
    mask &= on ? m : ~m;
  }
  leader = (mask & lt) == 0ull;
  group = mask;
  return __popcll(mask & lt);
}

// P > 1024 pairs, in two launches (one workgroup walked every pair in turn:
// 21 us at T = 2048).  perm_count_kernel: workgroup b counts the experts of
// pairs [1024 b, 1024 (b + 1)) and publishes the counts (agent-scope stores,
// drained, then the arrival count); the last to arrive sums them per expert in
// workgroup order, writes the tables (perm_tables) and each workgroup's first
// slot per expert.  perm_place_kernel: workgroup b places its pairs, a pair's
// slot its workgroup's first slot for the expert plus the pairs of that
// expert in the earlier waves and lanes: the pairs of an expert in pair order,
// perm_kernel's placement.
__global__ __launch_bounds__(kRouteThreads) void perm_count_kernel(
    const int32_t* __restrict__ idx, int T, int E, int k, int32_t* __restrict__ cnt, int32_t* __restrict__ base,
    uint32_t* __restrict__ counter, int32_t* __restrict__ offsets, int32_t* __restrict__ active,
    int32_t* __restrict__ act_off, int32_t* __restrict__ act_cnt, int32_t* __restrict__ n_active,
    int32_t* __restrict__ mt_u, int32_t* __restrict__ mt_row0, int32_t* __restrict__ mt_n,
    int32_t* __restrict__ n_mt, int mt_cap) {
  constexpr int kMaxBlocks = kMaxPairs / kRouteThreads;
  __shared__ int hist[kMaxExperts];
  __shared__ int wsum[128];
  __shared__ int s_last;
  const int tid = threadIdx.x, b = blockIdx.x, nb = gridDim.x, P = T * k;
  for (int e = tid; e < E; e += kRouteThreads) hist[e] = 0;
  __syncthreads();
  const int p = b * kRouteThreads + tid;
  if (p < P) atomicAdd(&hist[clampi(idx[p], 0, E - 1)], 1);
  __syncthreads();
  for (int e = tid; e < E; e += kRouteThreads) store_agent_i(cnt + int64_t(b) * E + e, hist[e]);
  vm_drain();  // this thread's counts are performed before the arrival below
  __syncthreads();
  if (tid == 0) s_last = arrive_last(counter, uint32_t(nb)) ? 1 : 0;
  __syncthreads();
  if (!s_last) return;
  int v[kMaxBlocks];
#pragma unroll
  for (int bb = 0; bb < kMaxBlocks; ++bb)
    v[bb] = (tid < E && bb < nb) ? load_agent_i(cnt + int64_t(bb) * E + tid) : 0;
  int c = 0;
#pragma unroll
  for (int bb = 0; bb < kMaxBlocks; ++bb) c += v[bb];
  const int ex = perm_tables(c, E, offsets, active, act_off, act_cnt, n_active, mt_u, mt_row0, mt_n, n_mt, mt_cap,
                             wsum);
  if (tid < E) {
    int run = ex;
#pragma unroll
    for (int bb = 0; bb < kMaxBlocks; ++bb)
      if (bb < nb) {
        base[int64_t(bb) * E + tid] = run;
        run += v[bb];
      }
  }
}

__global__ __launch_bounds__(kRouteThreads) void perm_place_kernel(const int32_t* __restrict__ idx, int T, int E,
                                                                   int k, const int32_t* __restrict__ base,
                                                                   int32_t* __restrict__ perm_token,
                                                                   int32_t* __restrict__ perm_slot,
                                                                   int32_t* __restrict__ pos) {
  constexpr int kW = kRouteThreads / 64;
  __shared__ int wcnt[kW][kMaxExperts];  // pairs of expert e in wave w, then their first slot
  const int tid = threadIdx.x, wave = tid >> 6, b = blockIdx.x, P = T * k;
  for (int i = tid; i < kW * kMaxExperts; i += kRouteThreads) (&wcnt[0][0])[i] = 0;
  const int p = b * kRouteThreads + tid;
  const bool valid = p < P;
  const int e = valid ? clampi(idx[p], 0, E - 1) : 0;
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  bool leader;
  unsigned long long group;
  const int rank = wave_match_rank(e, valid, nbits, leader, group);
  __syncthreads();
  if (valid && leader) wcnt[wave][e] = __popcll(group);
  __syncthreads();
  if (tid < E) {
    int run = base[int64_t(b) * E + tid];
    for (int w = 0; w < kW; ++w) {
      const int n = wcnt[w][tid];
      wcnt[w][tid] = run;
      run += n;
    }
  }
  __syncthreads();
  if (valid) {
    const int q = wcnt[wave][e] + rank;
    perm_token[q] = p / k;
    perm_slot[q] = p % k;
    pos[p] = q;
  }
}

__global__ __launch_bounds__(kRouteThreads) void perm_kernel(const int32_t* __restrict__ idx, int T,
                                                             int E, int k, int32_t* __restrict__ offsets,
                                                             int32_t* __restrict__ active,
                                                             int32_t* __restrict__ act_off,
                                                             int32_t* __restrict__ act_cnt,
                                                             int32_t* __restrict__ n_active,
                                                             int32_t* __restrict__ perm_token,
                                                             int32_t* __restrict__ perm_slot,
                                                             int32_t* __restrict__ pos, int32_t* __restrict__ mt_u,
                                                             int32_t* __restrict__ mt_row0,
                                                             int32_t* __restrict__ mt_n, int32_t* __restrict__ n_mt,
                                                             int mt_cap) {
  constexpr int kW = kRouteThreads / 64;  // waves
  __shared__ int wcnt[kW][kMaxExperts];   // pairs of expert e in wave w's chunk, then their first slot
  __shared__ int wsum[128];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int P = T * k;
  // wave w owns pairs [w C, (w + 1) C): its chunk in 64-pair rounds, so the
  // placement below needs no barrier per round
  const int C = (P + kW * 64 - 1) / (kW * 64) * 64;
  const int p0 = wave * C, p1 = min(P, p0 + C);
  for (int i = tid; i < kW * kMaxExperts; i += kRouteThreads) (&wcnt[0][0])[i] = 0;
  __syncthreads();
  for (int p = p0 + lane; p < p1; p += 64) atomicAdd(&wcnt[wave][clampi(idx[p], 0, E - 1)], 1);
  __syncthreads();
  // per expert: its count, then each wave's first slot (expert base + the
  // pairs of the waves before it)
  int c = 0;
  if (tid < E)
    for (int w = 0; w < kW; ++w) c += wcnt[w][tid];
  const int ex = perm_tables(c, E, offsets, active, act_off, act_cnt, n_active, mt_u, mt_row0, mt_n, n_mt, mt_cap,
                             wsum);
  if (tid < E) {
    int run = ex;
    for (int w = 0; w < kW; ++w) {
      const int n = wcnt[w][tid];
      wcnt[w][tid] = run;
      run += n;
    }
  }
  __syncthreads();
  // stable placement: a pair's slot is its wave's next slot for its expert
  // plus its rank among the round's lanes with the same expert
  int nbits = 1;
  while ((1 << nbits) < E) ++nbits;
  for (int c0 = p0; c0 < p1; c0 += 64) {
    const int p = c0 + lane;
    const bool valid = p < p1;
    const int e = valid ? clampi(idx[p], 0, E - 1) : 0;
    bool leader;
    unsigned long long mask;
    const int rank = wave_match_rank(e, valid, nbits, leader, mask);
    if (valid) {
      const int q = wcnt[wave][e] + rank;
      perm_token[q] = p / k;
      perm_slot[q] = p % k;
      pos[p] = q;
    }
    // every lane has read its slot base (program order within the wave)
    if (valid && leader) wcnt[wave][e] += __popcll(mask);
  }
}

// --------------------------------------------------------------- combine ----

// One workgroup per (token, 2048 columns).  The token's slots are ordered by
// their permuted position (= ascending expert id) by every wave alike: the
// positions and experts are the same across the workgroup, so each wave reads
// them once and a fixed exchange network sorts them in scalar registers (no
// shuffle, LDS or barrier in front of the row loads).  A repeated expert of a hash-routed token
// counts once, by its last slot (the row a decode step computes;
// architecture.py:790 index_put keeps the last write): a row is skipped when
// the next in position order has the same expert.  Each thread requests its 8
// columns of all KMAX rows at once (rows past k repeat the first one and are
// not added) and sums them in that order, then adds the shared expert's row.
template <int KMAX>
__global__ __launch_bounds__(256) void combine_kernel(const MoeWs ws, int k, int D, uint16_t* __restrict__ y) {
  const int t = blockIdx.y;
  const int c = blockIdx.x * 256 + threadIdx.x;  // 8-column chunk
  const int P = gridDim.y * k;
  // lane j < k reads slot j (one vector load per array, one wait), then each
  // slot is read out of its lane into a scalar register
  const int lane = threadIdx.x & 63, jl = lane < k ? lane : 0;
  const int pl = clampi(ws.pos[int64_t(t) * k + jl], 0, P - 1);
  const int el = ws.idx[int64_t(t) * k + jl];
  int ps[KMAX], es[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    ps[j] = j < k ? __builtin_amdgcn_readlane(pl, j) : 0x7FFFFFFF;
    es[j] = j < k ? __builtin_amdgcn_readlane(el, j) : -1;
  }
#pragma unroll
  for (int a = 0; a < KMAX - 1; ++a)
#pragma unroll
    for (int i = 0; i + 1 < KMAX - a; ++i)
      if (ps[i] > ps[i + 1]) {
        const int tp = ps[i], te = es[i];
        ps[i] = ps[i + 1];
        es[i] = es[i + 1];
        ps[i + 1] = tp;
        es[i + 1] = te;
      }
  if (c * 8 >= D) return;
  v4i v[KMAX];
#pragma unroll
  for (int r = 0; r < KMAX; ++r) v[r] = load16(ws.out2 + int64_t(r < k ? ps[r] : ps[0]) * D + c * 8);
  const v4i sv = load16(ws.sh_out + int64_t(t) * D + c * 8);
  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
  for (int r = 0; r < KMAX; ++r) {
    const bool use = r < k && !(r + 1 < k && es[r + 1] == es[r]);
    if (use) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += bf16lo(uint32_t(v[r][i]));
        acc[2 * i + 1] += bf16hi(uint32_t(v[r][i]));
      }
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = acc[2 * i] + bf16lo(uint32_t(sv[i]));
    const float hi = acc[2 * i + 1] + bf16hi(uint32_t(sv[i]));
    o[i] = f32x2_to_bf16x2(lo, hi);
  }
  *reinterpret_cast<v4i*>(y + int64_t(t) * D + c * 8) = v4i{int(o[0]), int(o[1]), int(o[2]), int(o[3])};
}

int launch_combine(const MoeWs& w, int64_t T, int k, int D, void* y, hipStream_t stream) {
  const dim3 grid(unsigned((D / 8 + 255) / 256), unsigned(T));
  if (k <= 8) {
    WZ_LAUNCH("moe_combine", stream, combine_kernel<8>, grid, dim3(256), 0, w, k, D, static_cast<uint16_t*>(y));
  } else {
    WZ_LAUNCH("moe_combine", stream, combine_kernel<16>, grid, dim3(256), 0, w, k, D, static_cast<uint16_t*>(y));
  }
  return check_launch("moe combine");
}

__global__ void export_routing_kernel(const MoeWs ws, int P, float* __restrict__ w_out,
                                      int64_t* __restrict__ i_out) {
  const int p = blockIdx.x * blockDim.x + threadIdx.x;
  if (p >= P) return;
  if (w_out) w_out[p] = ws.weights[p];
  if (i_out) i_out[p] = ws.idx[p];
}

// ------------------------------------------------------------------ host ----

int launch_decode(const wz_moe_desc* d, const MoeWs& w, const void* x, const int64_t* ids, int64_t T,
                  void* y, hipStream_t stream, int only, const float* nw = nullptr, float eps = 0.0f);
int launch_prefill_experts(const wz_moe_desc* d, const MoeWs& w, const void* x, int64_t T, hipStream_t stream,
                           int only);
int launch_prefill_gate(const wz_moe_desc* d, const MoeWs& w, const void* x, const int64_t* input_ids, int64_t T,
                        hipStream_t stream);

// Tokens per call of the kernel sequence: the routed pairs of one call (T * k)
// fit the kMaxPairs-row tables.  wz_moe_forward serves larger T as successive
// chunks of this many tokens on the same workspace (the layer is token-local).
static int64_t chunk_tokens(const wz_moe_desc* d) { return kMaxPairs / d->topk; }

static int validate(const wz_moe_desc* d, int64_t T, const void* ws, size_t ws_bytes,
                    const char* what, bool chunked = false) {
  if (!d) return set_error(WZ_EINVAL, "%s: null descriptor", what);
  if (d->dim <= 0 || d->dim % 128 || d->inter <= 0 || d->inter % 128)
    return set_error(WZ_EINVAL, "%s: dim=%d and inter=%d must be positive multiples of 128", what,
                     d->dim, d->inter);
  if (d->n_experts <= 0 || d->n_experts > kMaxExperts)
    return set_error(WZ_EINVAL, "%s: n_experts=%d outside 1..%d", what, d->n_experts, kMaxExperts);
  if (d->topk <= 0 || d->topk > 16 || d->topk > d->n_experts)
    return set_error(WZ_EINVAL, "%s: topk=%d outside 1..min(16, n_experts)", what, d->topk);
  if (T < 0 || T > (int64_t(1) << 40) || (!chunked && T * d->topk > kMaxPairs))
    return set_error(WZ_EINVAL, "%s: T=%lld x topk=%d exceeds %d routed pairs", what, (long long)T,
                     d->topk, kMaxPairs);
  if (d->score_func < 0 || d->score_func > 2)
    return set_error(WZ_EINVAL, "%s: unknown score_func %d", what, d->score_func);
  if (d->act_scale_kind < 0 || d->act_scale_kind > 2)
    return set_error(WZ_EINVAL, "%s: unknown act_scale_kind %d", what, d->act_scale_kind);
  if (!d->gate_w) return set_error(WZ_EINVAL, "%s: gate weight missing", what);
  if (d->tid2eid && d->vocab <= 0) return set_error(WZ_EINVAL, "%s: tid2eid without vocab", what);
  if (!d->tid2eid && !d->gate_bias && d->score_func == WZ_SCORE_SQRTSOFTPLUS) {
    // a score-routed layer without bias is legal (bias optional), nothing to check
  }
  if (T == 0) return WZ_OK;  // nothing to do: no workspace needed
  if (!ws) return set_error(WZ_EINVAL, "%s: null workspace", what);
  const size_t need = wz_moe_workspace_bytes(d, T);
  if (ws_bytes < need)
    return set_error(WZ_ESPACE, "%s: workspace %zu bytes < %zu needed for T=%lld", what, ws_bytes,
                     need, (long long)T);
  return WZ_OK;
}

static int launch_routing(const wz_moe_desc* d, const MoeWs& w, const void* x,
                          const int64_t* input_ids, int64_t T, hipStream_t stream) {
  const int E = d->n_experts, k = d->topk, D = d->dim;
  if (d->tid2eid && !input_ids) return set_error(WZ_EINVAL, "moe: hash-routed layer needs input_ids");
  if (T > kDecodeMaxT && d->score_func != WZ_SCORE_SOFTMAX) {
    // MFMA gate + exact refinement at the top-k boundary (moe_prefill.hip)
    if (int rc = launch_prefill_gate(d, w, x, input_ids, T, stream)) return rc;
  } else {
    WZ_LAUNCH("moe_gate", stream, gate_dot_kernel, dim3((E + 3) / 4, unsigned((T + kGateTok - 1) / kGateTok)),
              dim3(256), 0, static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(d->gate_w), w.scores,
              int(T), E, D);
    if (int rc = check_launch("moe gate")) return rc;
    WZ_LAUNCH("moe_topk", stream, topk_kernel, dim3(unsigned((T + 3) / 4)), dim3(256), 0, w.scores,
              d->tid2eid ? nullptr : d->gate_bias, d->tid2eid, input_ids, d->vocab, int(T), E, k, d->score_func,
              d->route_scale, w.weights, w.idx);
    if (int rc = check_launch("moe topk")) return rc;
  }
  const int64_t P = T * k, mt_cap = P / kPrefillTileRows + (P < E ? P : E) + 1;
  if (P <= kRouteThreads) {
    WZ_LAUNCH("moe_perm", stream, perm_kernel, dim3(1), dim3(kRouteThreads), 0, w.idx, int(T), E, k, w.offsets,
              w.active, w.act_off, w.act_cnt, w.n_active, w.perm_token, w.perm_slot, w.pos, w.mt_u, w.mt_row0,
              w.mt_n, w.n_mt, int(mt_cap));
    return check_launch("moe perm");
  }
  // the gate scores are spent once the top-k is chosen: their [T, E] floats hold
  // the per-workgroup counts and first slots ([nb, E] each; P > 1024 makes T >= 64)
  const int nb = int((P + kRouteThreads - 1) / kRouteThreads);
  if (int64_t(2) * nb * E > T * E || nb > kMaxPairs / kRouteThreads)
    return set_error(WZ_EINVAL, "moe perm: %d count blocks do not fit the score buffer (T=%lld)", nb, (long long)T);
  int32_t* cnt = reinterpret_cast<int32_t*>(w.scores);
  int32_t* base = cnt + int64_t(nb) * E;
  WZ_LAUNCH("moe_perm", stream, perm_count_kernel, dim3(unsigned(nb)), dim3(kRouteThreads), 0, w.idx, int(T), E, k,
            cnt, base, &w.counters[kCounterWords - 1], w.offsets, w.active, w.act_off, w.act_cnt, w.n_active,
            w.mt_u, w.mt_row0, w.mt_n, w.n_mt, int(mt_cap));
  if (int rc = check_launch("moe perm count")) return rc;
  WZ_LAUNCH("moe_perm", stream, perm_place_kernel, dim3(unsigned(nb)), dim3(kRouteThreads), 0, w.idx, int(T), E, k,
            base, w.perm_token, w.perm_slot, w.pos);
  return check_launch("moe perm place");
}

}  // namespace wz

extern "C" size_t wz_moe_workspace_bytes(const wz_moe_desc* d, int64_t T) {
  if (!d || T < 0 || d->topk <= 0) return 0;
  if (T > wz::chunk_tokens(d)) T = wz::chunk_tokens(d);
  const size_t big = wz::moe_ws_layout(d, T, nullptr).bytes;
  const size_t dec = wz::moe_ws_layout(d, T < wz::kDecodeMaxT ? T : wz::kDecodeMaxT, nullptr).bytes;
  return big > dec ? big : dec;
}

__global__ void zero_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

extern "C" int wz_moe_workspace_init(void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (!ws || ws_bytes < sizeof(uint32_t) * kCounterWords)
    return set_error(WZ_ESPACE, "moe_workspace_init: workspace smaller than the %zu-byte counter block",
                     sizeof(uint32_t) * kCounterWords);
  WZ_LAUNCH("moe_ws_init", stream, zero_words_kernel, dim3(kCounterWords / 256), dim3(256), 0,
            static_cast<uint32_t*>(ws), kCounterWords);
  return check_launch("moe_workspace_init");
}

extern "C" int wz_moe_route(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids,
                            int64_t T, float* weights, int64_t* indices, int32_t* offsets,
                            int32_t* perm_token, int32_t* perm_slot, void* ws, size_t ws_bytes,
                            hipStream_t stream) {
  using namespace wz;
  if (int rc = validate(d, T, ws, ws_bytes, "moe_route")) return rc;
  if (T == 0) return WZ_OK;
  const MoeWs w = moe_ws_layout(d, T, static_cast<uint8_t*>(ws));
  if (int rc = launch_routing(d, w, x_bf16, input_ids, T, stream)) return rc;
  const int P = int(T * d->topk);
  WZ_LAUNCH("moe_export", stream, export_routing_kernel, dim3((P + 255) / 256), dim3(256), 0, w, P, weights,
                     indices);
  if (int rc = check_launch("moe_route export")) return rc;
  if (offsets && hipMemcpyAsync(offsets, w.offsets, sizeof(int32_t) * (d->n_experts + 1),
                                hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return set_error(WZ_ELAUNCH, "moe_route: offsets copy failed");
  if (perm_token && hipMemcpyAsync(perm_token, w.perm_token, sizeof(int32_t) * P,
                                   hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return set_error(WZ_ELAUNCH, "moe_route: perm copy failed");
  if (perm_slot && hipMemcpyAsync(perm_slot, w.perm_slot, sizeof(int32_t) * P,
                                  hipMemcpyDeviceToDevice, stream) != hipSuccess)
    return set_error(WZ_ELAUNCH, "moe_route: perm copy failed");
  return WZ_OK;
}

namespace wz {

static int forward_chunk(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T, void* y_bf16,
                         float* weights_out, int64_t* indices_out, void* ws, hipStream_t stream) {
  const MoeWs w = moe_ws_layout(d, T, static_cast<uint8_t*>(ws));
  const int k = d->topk, D = d->dim;
  const int64_t P = T * k;
  if (T <= kDecodeMaxT) {
    if (int rc = launch_decode(d, w, x_bf16, input_ids, T, y_bf16, stream, -1)) return rc;
  } else {
    if (int rc = launch_routing(d, w, x_bf16, input_ids, T, stream)) return rc;
    if (int rc = launch_prefill_experts(d, w, x_bf16, T, stream, -1)) return rc;
    if (int rc = launch_combine(w, T, k, D, y_bf16, stream)) return rc;
  }
  if (weights_out || indices_out) {
    WZ_LAUNCH("moe_export", stream, export_routing_kernel, dim3(unsigned((P + 255) / 256)), dim3(256), 0, w,
              int(P), weights_out, indices_out);
    if (int rc = check_launch("moe export")) return rc;
  }
  return WZ_OK;
}

}  // namespace wz

extern "C" int wz_moe_forward(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids,
                              int64_t T, void* y_bf16, float* weights_out, int64_t* indices_out,
                              void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (int rc = validate(d, T, ws, ws_bytes, "moe_forward", true)) return rc;
  if (T == 0) return WZ_OK;
  if (!x_bf16 || !y_bf16) return set_error(WZ_EINVAL, "moe_forward: null x or y");
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe_forward: packed expert banks missing (build them with wz_moe_pack)");
  if (!d->sh_w1_s || !d->sh_w3_s || !d->sh_w2_s)
    return set_error(WZ_EINVAL, "moe_forward: shared-expert block scales missing");
  if (d->tid2eid && !input_ids) return set_error(WZ_EINVAL, "moe: hash-routed layer needs input_ids");
  const int64_t C = chunk_tokens(d), k = d->topk, D = d->dim;
  for (int64_t t0 = 0; t0 < T; t0 += C) {
    const int64_t n = T - t0 < C ? T - t0 : C;
    if (int rc = forward_chunk(d, static_cast<const uint16_t*>(x_bf16) + t0 * D, input_ids ? input_ids + t0 : nullptr,
                               n, static_cast<uint16_t*>(y_bf16) + t0 * D, weights_out ? weights_out + t0 * k : nullptr,
                               indices_out ? indices_out + t0 * k : nullptr, ws, stream))
      return rc;
  }
  return WZ_OK;
}

extern "C" int wz_moe_forward_norm(const wz_moe_desc* d, const void* h_bf16, const float* norm_weight, float eps,
                                   const int64_t* input_ids, int64_t T, void* y_bf16, float* weights_out,
                                   int64_t* indices_out, void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (int rc = validate(d, T, ws, ws_bytes, "moe_forward_norm", true)) return rc;
  if (T == 0) return WZ_OK;
  if (T > kNormMaxT)
    return set_error(WZ_EINVAL, "moe_forward_norm: the fused norm serves T <= %d (T=%lld); run the norm, then "
                     "wz_moe_forward", kNormMaxT, (long long)T);
  if (!h_bf16 || !y_bf16 || !norm_weight) return set_error(WZ_EINVAL, "moe_forward_norm: null h, y or norm weight");
  if (!d->w13p || !d->w13p_s || !d->w2p || !d->w2p_s || !d->sh13p || !d->sh2p)
    return set_error(WZ_EINVAL, "moe_forward_norm: packed expert banks missing (build them with wz_moe_pack)");
  if (!d->sh_w1_s || !d->sh_w3_s || !d->sh_w2_s)
    return set_error(WZ_EINVAL, "moe_forward_norm: shared-expert block scales missing");
  if (d->tid2eid && !input_ids) return set_error(WZ_EINVAL, "moe: hash-routed layer needs input_ids");
  const MoeWs w = moe_ws_layout(d, T, static_cast<uint8_t*>(ws));
  if (int rc = launch_decode(d, w, h_bf16, input_ids, T, y_bf16, stream, -1, norm_weight, eps)) return rc;
  if (weights_out || indices_out) {
    const int P = int(T * d->topk);
    WZ_LAUNCH("moe_export", stream, export_routing_kernel, dim3(unsigned((P + 255) / 256)), dim3(256), 0, w, P,
              weights_out, indices_out);
    return check_launch("moe_forward_norm export");
  }
  return WZ_OK;
}

extern "C" int wz_moe_replay_stage(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T,
                                   int stage, void* y_bf16, void* ws, size_t ws_bytes, hipStream_t stream) {
  using namespace wz;
  if (int rc = validate(d, T, ws, ws_bytes, "moe_replay_stage")) return rc;
  if (stage < WZ_STAGE_ROUTE || stage > WZ_STAGE_COMBINE)
    return set_error(WZ_EINVAL, "moe_replay_stage: unknown stage %d", stage);
  if (T == 0) return WZ_OK;
  if (!x_bf16 || !y_bf16) return set_error(WZ_EINVAL, "moe_replay_stage: null x or y");
  const MoeWs w = moe_ws_layout(d, T, static_cast<uint8_t*>(ws));
  if (T <= kDecodeMaxT) return launch_decode(d, w, x_bf16, input_ids, T, y_bf16, stream, stage);
  if (stage == WZ_STAGE_ROUTE) {
    if (int rc = launch_routing(d, w, x_bf16, input_ids, T, stream)) return rc;
  }
  if (stage == WZ_STAGE_COMBINE) return launch_combine(w, T, d->topk, d->dim, y_bf16, stream);
  return launch_prefill_experts(d, w, x_bf16, T, stream, stage);
}

// ------------------------------------------------------- no-allocation entry ----
//
// wz_moe_forward with the workspace in a file-scope device array instead of a
// caller-provided buffer, for callers that cannot allocate.  Each GPU the
// library runs on holds its own copy of `scratch` until the process ends.  A
// device address is taken once per device with hipGetSymbolAddress and used
// for every kernel argument; host code never passes the array's name itself.

namespace wz {

static __device__ __align__(256) uint8_t scratch[WZ_MOE_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static void* g_scratch_ptr[kMaxDevices];
static std::once_flag g_scratch_once[kMaxDevices];
static int g_scratch_rc[kMaxDevices];

// The device address of this device's scratch array (nullptr on failure, with the error set).
static uint8_t* scratch_for_current_device(const char* what) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error(WZ_EINVAL, "%s: no current device (or device index >= %d)", what, kMaxDevices);
    return nullptr;
  }
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    g_scratch_rc[dev] = int(e);
    g_scratch_ptr[dev] = e == hipSuccess ? p : nullptr;
  });
  if (!g_scratch_ptr[dev]) {
    set_error(WZ_ELAUNCH, "%s: hipGetSymbolAddress of the scratch array failed on device %d (hip error %d)", what,
              dev, g_scratch_rc[dev]);
    return nullptr;
  }
  return static_cast<uint8_t*>(g_scratch_ptr[dev]);
}

}  // namespace wz

extern "C" int wz_moe_forward_noalloc(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids,
                                      int64_t T, void* y_bf16, float* weights_out, int64_t* indices_out,
                                      hipStream_t stream) {
  using namespace wz;
  if (!d) return set_error(WZ_EINVAL, "moe_forward_noalloc: null descriptor");
  if (d->topk <= 0 || d->topk > 16) return set_error(WZ_EINVAL, "moe_forward_noalloc: topk=%d outside 1..16", d->topk);
  if (T < 0) return set_error(WZ_EINVAL, "moe_forward_noalloc: T=%lld < 0", (long long)T);
  if (T == 0) return WZ_OK;
  const size_t need = wz_moe_workspace_bytes(d, T);
  if (need > size_t(WZ_MOE_NOALLOC_SCRATCH_BYTES))
    return set_error(WZ_ESPACE,
                     "moe_forward_noalloc: this layer at T=%lld needs %zu bytes of scratch, more than the %d "
                     "the library holds per device; call wz_moe_forward with a workspace instead",
                     (long long)T, need, WZ_MOE_NOALLOC_SCRATCH_BYTES);
  uint8_t* ws = scratch_for_current_device("moe_forward_noalloc");
  if (!ws) return WZ_ELAUNCH;
  // the arrival counters must start at zero: clear them on every call (a fill
  // kernel, so the call stays capturable without a memset node)
  WZ_LAUNCH("moe_ws_init", stream, zero_words_kernel, dim3(kCounterWords / 256), dim3(256), 0,
            reinterpret_cast<uint32_t*>(ws), kCounterWords);
  if (int rc = check_launch("moe_forward_noalloc counters")) return rc;
  return wz_moe_forward(d, x_bf16, input_ids, T, y_bf16, weights_out, indices_out, ws,
                        size_t(WZ_MOE_NOALLOC_SCRATCH_BYTES), stream);
}
