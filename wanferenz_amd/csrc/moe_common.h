// Workspace layout and helpers shared by the MoE kernels (moe.hip, moe_decode.hip).
#pragma once

#include "mfma_ops.h"

namespace wz {

constexpr int kRouteThreads = 1024;
constexpr int kMaxExperts = 512;
constexpr int kMaxPairs = 16384;
constexpr int kGateTok = 8;
constexpr int kDecodeMaxT = 16;       // tokens served by the decode kernels
constexpr int kNormMaxT = 8;          // rows the decode route launch normalises itself (fused ffn norm)
constexpr int kNormMaxD = 4096;       // and their width
constexpr int kPrefillTileRows = 64;  // pair rows per M-tile of the prefill / dense GEMMs
constexpr int kCounterWords = 4096;   // arrival counters at the start of the workspace

// Scratch of one MoE layer call, carved from the caller's workspace.  The
// arrival counters sit at offset 0 so wz_moe_workspace_init can zero them
// without knowing T; every kernel that bumps a counter resets it to zero.
struct MoeWs {
  uint32_t* counters;  // [kCounterWords]: [0] route, [1 + d_tile] combine, [kCounterWords - 1] permutation
  float* scores;       // [T, E] gate logits (general path) / scores (decode path)
  float* biased;       // [T, E] decode: scores + bias (the selection key); prefill: sum |x||w| (gate error bound)
  float* weights;      // [T, k]
  int32_t* idx;        // [T, k]
  int32_t* offsets;    // [E + 1]
  int32_t* active;     // [E] active expert ids, ascending
  int32_t* act_off;    // [E] first pair of active expert u
  int32_t* act_cnt;    // [E] pairs of active expert u
  int32_t* n_active;   // [1]
  int32_t* perm_token; // [P]
  int32_t* perm_slot;  // [P]
  int32_t* pos;        // [P] permuted position of pair t*k + j
  int32_t* tok_pos;    // [T, k] a token's positions, ascending, one per distinct expert
  int32_t* tok_n;      // [T]
  int32_t* umap;       // [U_max, T] decode: permuted position of (active expert u, token t), -1 if unrouted
  float* uwt;          // [U_max, T] decode: its routing weight
  uint8_t* xq;         // [T, D] e4m3 act_quant(x)
  float* xs;           // [T, D/128] its block scales
  uint8_t* hq;         // decode: [U_max*T + T, I] e4m3 act_quant(h) (rows (u, t), then shared t)
  float* hs;           // [U_max*T + T, I/128]
  uint16_t* h;         // [P, I] bf16 (a routed (expert, token) at its pair row), then sh_h
  int32_t* mt_u;       // prefill M-tile table: active expert of tile
  int32_t* mt_row0;    //   first pair row of tile
  int32_t* mt_n;       //   rows in tile (<= 128)
  int32_t* n_mt;       //   number of tiles
  uint16_t* sh_h;      // [T, I] bf16, = h + P * I
  uint16_t* out2;      // [P, D] bf16
  uint16_t* sh_out;    // [T, D] bf16
  size_t bytes;
};

static inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

static inline MoeWs moe_ws_layout(const wz_moe_desc* d, int64_t T, uint8_t* base) {
  const int64_t E = d->n_experts, k = d->topk, P = T * k, D = d->dim, I = d->inter;
  const int64_t UT = T <= kDecodeMaxT ? (P < E ? P : E) * T : 0;  // decode tables only
  size_t off = 0;
  MoeWs w;
  auto take = [&](size_t bytes) {
    uint8_t* p = base ? base + off : nullptr;
    off += align256(bytes);
    return p;
  };
  w.counters = reinterpret_cast<uint32_t*>(take(sizeof(uint32_t) * kCounterWords));
  w.scores = reinterpret_cast<float*>(take(sizeof(float) * T * E));
  w.biased = reinterpret_cast<float*>(take(sizeof(float) * T * E));
  w.weights = reinterpret_cast<float*>(take(sizeof(float) * P));
  w.idx = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * P));
  w.offsets = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * (E + 1)));
  w.active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  w.act_off = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  w.act_cnt = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * E));
  w.n_active = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 64));
  w.perm_token = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * P));
  w.perm_slot = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * P));
  w.pos = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * P));
  w.tok_pos = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * P));
  w.tok_n = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * T));
  w.umap = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * UT));
  w.uwt = reinterpret_cast<float*>(take(sizeof(float) * UT));
  w.xq = take(size_t(T) * D);
  w.xs = reinterpret_cast<float*>(take(sizeof(float) * T * (D / 128)));
  const int64_t HQ = (T <= kDecodeMaxT ? UT : P) + T;  // decode rows (u, t) / prefill pairs, then shared rows
  w.hq = take(size_t(HQ) * I);
  w.hs = reinterpret_cast<float*>(take(sizeof(float) * HQ * (I / 128)));
  const int64_t MT = P / kPrefillTileRows + (P < E ? P : E) + 1;  // M-tiles of pair rows (prefill)
  w.mt_u = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * MT));
  w.mt_row0 = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * MT));
  w.mt_n = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * MT));
  w.n_mt = reinterpret_cast<int32_t*>(take(sizeof(int32_t) * 64));
  // h: P pair rows, then the T shared rows (sh_h), one contiguous image
  w.h = reinterpret_cast<uint16_t*>(take(2 * size_t(P + T) * I));
  w.sh_h = w.h ? w.h + size_t(P) * I : nullptr;
  w.out2 = reinterpret_cast<uint16_t*>(take(2 * size_t(P) * D));
  w.sh_out = reinterpret_cast<uint16_t*>(take(2 * size_t(T) * D));
  w.bytes = off;
  return w;
}

// Routing tables live in device memory and are produced by an earlier kernel;
// every consumer clamps what it reads so that no table value can address
// outside the weight banks, the workspace or LDS.
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + expf(-g)); }

// torch F.softplus(beta=1, threshold=20) evaluated in fp64, rounded to fp32
__device__ __forceinline__ float softplus_f32(float a) {
  if (a > 20.0f) return a;
  return float(log1p(exp(double(a))));
}

// Routing score of one raw gate logit (Gate.forward, architecture.py:700-705);
// softmax is handled by the caller (it needs the row max and sum).
__device__ __forceinline__ float score_of(float a, int score_func) {
  if (score_func == WZ_SCORE_SIGMOID) return float(1.0 / (1.0 + exp(-double(a))));
  return float(sqrt(double(softplus_f32(a))));
}

struct Cand {
  float v;
  int i;
};

// larger value wins; equal values -> lower expert index (stable descending order)
__device__ __forceinline__ Cand cand_better(Cand a, Cand b) {
  if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
  return a;
}

__device__ __forceinline__ Cand wave_argmax(Cand c) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) {
    Cand o;
    o.v = __shfl_xor(c.v, m, kWave);
    o.i = __shfl_xor(c.i, m, kWave);
    c = cand_better(c, o);
  }
  return c;
}

// Order-preserving map float -> uint32 (larger float -> larger key; -inf lowest).
__device__ __forceinline__ uint32_t f32_key(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Wave-wide max of a uint32 through DPP row ops (no LDS round trips): quad
// swaps and row mirrors give every lane its row's max, row_bcast15/31 fold
// the four rows into lane 63, readlane broadcasts it.  The masked-off rows of
// the broadcasts read `old` = 0, the identity of an unsigned max, which lets
// the compiler fold each move into its v_max_u32_dpp (one instruction a step
// instead of two).
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, true)));   // quad_perm 1,0,3,2
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, true)));   // quad_perm 2,3,0,1
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x141, 0xF, 0xF, true)));  // row_half_mirror
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x140, 0xF, 0xF, true)));  // row_mirror
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x142, 0xA, 0xF, false)));  // row_bcast:15
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x143, 0xC, 0xF, false)));  // row_bcast:31
  return uint32_t(__builtin_amdgcn_readlane(int(v), 63));
}

__device__ __forceinline__ uint32_t dpp_min_u32(uint32_t v) { return ~dpp_max_u32(~v); }

// Wave-wide max of a uint32 left in every lane, in vector instructions only:
// DPP steps give every lane its row's max, then the gfx950 row and half swaps
// (v_permlane16_swap, v_permlane32_swap) exchange rows and halves.  With no
// readlane, ballot or scalar step the chain never waits for a vector result
// to reach the scalar unit, which in a lone wave costs more than the steps.
__device__ __forceinline__ uint32_t wave_max_all_u32(uint32_t v) {
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, true)));   // quad_perm 1,0,3,2
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, true)));   // quad_perm 2,3,0,1
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x141, 0xF, 0xF, true)));  // row_half_mirror
  v = max(v, uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x140, 0xF, 0xF, true)));  // row_mirror
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);  // rows 0 <-> 1, 2 <-> 3
  v = max(uint32_t(r[0]), uint32_t(r[1]));
  const auto h = __builtin_amdgcn_permlane32_swap(v, v, false, false);  // lanes 0-31 <-> 32-63
  return max(uint32_t(h[0]), uint32_t(h[1]));
}

__device__ __forceinline__ uint32_t wave_min_all_u32(uint32_t v) { return ~wave_max_all_u32(~v); }

// wave_argmax's winner in every lane with no LDS round trip, for a full wave
// and non-negative indices.  With no NaN value in the wave, cand_better is a
// total order (value, with -0 == +0, then the lower index), so the winner is
// the lane with the largest order-preserving key of its value (zeros keyed
// alike) and, among the lanes holding that key, the lowest index: two
// all-lane DPP maxima, the second over the complemented indices.  The value
// returned is the key's float (+0 for a zero winner).  A NaN anywhere in the
// wave takes the shuffle butterfly, unchanged.
__device__ __forceinline__ Cand wave_argmax_dpp(Cand c) {
  if (__ballot(c.v != c.v) != 0ull) return wave_argmax(c);
  const uint32_t key = c.v == 0.0f ? 0x80000000u : f32_key(c.v);
  const uint32_t km = wave_max_all_u32(key);
  const uint32_t im = wave_max_all_u32(key == km ? ~uint32_t(c.i) : 0u);
  Cand r;
  r.v = __uint_as_float((km & 0x80000000u) ? (km & 0x7FFFFFFFu) : ~km);
  r.i = int(~im);
  return r;
}

// Agent-scope arrival counter: returns true in the last of `n` arrivals and
// resets the counter for the next launch.
__device__ __forceinline__ bool arrive_last(uint32_t* ctr, uint32_t n) {
  const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (old == n - 1) {
    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  }
  return false;
}

// Publication of the routing scores from the gate workgroups to the last
// arrival (route_decode_kernel).  The producers store with agent-scope relaxed
// atomics (store_agent), drain their vector-memory counter (vm_drain), meet at
// a barrier, and one thread adds to the counter; the last arrival reads with
// agent-scope relaxed atomics (load_agent).  What makes this sufficient is how
// gfx950 performs agent-scope atomics: a relaxed agent-scope load or store is
// issued with the sc1 bit, which makes it act at the device coherence point
// (the store writes through this XCD's L2, the load does not hit a stale L2
// copy); s_waitcnt 0 returns only once the store has been acknowledged there;
// and the agent-scope add is performed at that same point after the barrier.
// An agent-scope release fence is the same wait plus an L2 writeback that only
// non-atomic stores need, and the acquire an L2 invalidate that only
// non-atomic loads need.  Written as a release/acquire add instead (the form
// the HIP memory model guarantees), every gate workgroup's release writes back
// its XCD's L2: measured +5 us per route launch at T = 1..4.
__device__ __forceinline__ void store_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent_i(int32_t* p, int32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int32_t load_agent_i(const int32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void vm_drain() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace wz
