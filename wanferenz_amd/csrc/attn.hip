// Sparse attention over gathered KV rows (decode and chunked prefill).
//
// o[b, s, h, :] = sum_j p_j kv[b, idx_j, :] / (sum_j p_j + exp(sink[h] - m)),
// p_j = exp(q[b, s, h, :] . kv[b, idx_j, :] * scale - m) over the valid
// (idx >= 0) entries of topk_idxs[b, s, :], m the running maximum — the
// blockwise online softmax of wanferenz/kernels/torch_ops.py:114-146 (CPU)
// and reference.py:314-418 (GPU), one KV row shared by all heads (K = V).
// With no valid index in the first block of 64 the reference's
// exp(-inf - -inf) turns its sums into NaN for good, and so does this code.
#include "common.h"

namespace wz {

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

constexpr int kAttnBlock = 64;     // indices per block (the reference's SPARSE_ATTN_BLOCK)
constexpr int kAttnIdxCap = 2048;  // indices one workgroup covers (32 blocks)
constexpr int kAttnMaxSplit = 64;  // workgroups one query's blocks are split over
constexpr float kLazyMax = 8.0f;   // the running max moves when a block exceeds it by more

__device__ __forceinline__ v4f mfma_bf16_32(v8s_t a, v8s_t b, v4f c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf_t, a), __builtin_bit_cast(v8bf_t, b), c, 0,
                                                 0, 0);
}

// Floats of one (query, 64 heads, split) partial: m[64], l[64], O[64][D].
__host__ __device__ constexpr int64_t attn_part_floats(int d) { return 128 + 64 * int64_t(d); }

// LDS image of one block of 64 KV rows, row-major, no padding.  The 16-byte
// chunks of row r sit XOR-swizzled (chunk c at slot c ^ swz(r)), so that both
// read patterns are free of bank conflicts: 16 rows reading one chunk (the K
// operand of S^T) land on 16 distinct 4-bank groups, and 8 rows reading two
// adjacent chunks (the transpose reads of V) on 16 distinct groups as well.
template <int D>
struct KsLayout {
  static constexpr int RB = 2 * D;             // bytes per row
  static constexpr int RPI = 1024 / RB;        // rows per 1 KB load
  static constexpr int NG = kAttnBlock / RPI;  // loads per block
  static constexpr int BYTES = kAttnBlock * RB;
  static __device__ __forceinline__ int swz(int row) { return ((row & 7) << 1) ^ ((row >> 3) & 1); }
  // byte address of element `col` (a multiple of 4) of `row`
  static __device__ __forceinline__ int at(int row, int col) {
    return row * RB + (((col >> 3) ^ swz(row)) << 4) + ((col & 7) << 1);
  }
};

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return f32x2_to_bf16x2(a, b);
}

// Two floats -> packed bf16 pair with the hardware converter (round to nearest
// even, as f32_to_bf16; a NaN stays a NaN).
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// One workgroup per (query, 64 heads, range of 64-index blocks), 4 waves;
// wave w owns heads 64 hq + 16w .. +16 (a wave whose head group is past H only
// helps load).  Per block:
//   * the 64 gathered KV rows sit in LDS row-major ([row][d], padded); they
//     were loaded while the previous block was computed (double buffer);
//   * S^T[64 rows, 16 heads] = K Q^T with V_MFMA_F32_16X16X32_BF16, K from
//     LDS, the wave's Q fragments in registers for the launch.  The transposed
//     product leaves lane (head n, group g) holding rows 16rt + 4g + i, which
//     is the A-operand layout of P in P V once two row tiles are paired
//     (k slots 0-3: rows 32kc + 4g + i, slots 4-7: rows 32kc + 16 + 4g + i):
//     P never leaves registers and the softmax needs no other wave;
//   * P = exp(S - m) in bf16 (the GPU reference also multiplies a bf16 P,
//     reference.py:404-405), with m moved only when a block's maximum exceeds
//     it by more than kLazyMax (P <= e^8; the final division by the sum taken
//     with the same m makes the result independent of m);
//   * O[16 heads, D] += P V, the V operand read from the row-major rows with
//     the LDS transpose read (ds_read_b64_tr_b16: in each 16-lane group, lane
//     i addressing row base + (i >> 2), column c0 + 4(i & 3) makes lane j
//     receive rows base..base+3 of column c0 + j).
// A workgroup that covers every block normalises (sink term included) and
// stores bf16; for few queries the blocks are split over workgroups that
// store (m, l, O) partials and sparse_attn_combine_kernel merges them.
template <int D, bool SPLIT>
__global__ __launch_bounds__(256, 1) void sparse_attn_kernel(const uint16_t* __restrict__ q,
                                                            const uint16_t* __restrict__ kv,
                                                            const float* __restrict__ sink,
                                                            const int32_t* __restrict__ idx,
                                                            uint16_t* __restrict__ o, float* __restrict__ part, int S,
                                                            int H, int N, int topk, int bps, int nsplit,
                                                            float scale) {
  using L = KsLayout<D>;
  constexpr int KC = D / 32;  // 32-wide d chunks of S
  constexpr int NT = D / 16;  // 16-column tiles of O
  static_assert(L::NG % 4 == 0, "a block's loads must split evenly over the 4 waves");
  static_assert(L::RB / 16 >= 16, "the swizzle permutes 16 chunks of a row");
  __shared__ __align__(16) uint8_t ksb[2][L::BYTES];
  __shared__ int s_idx[kAttnIdxCap];
  __shared__ int s_any;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nl = lane & 15, g = lane >> 4;
  const int HQ = (H + 63) / 64;
  const int c = blockIdx.x % nsplit, qh = blockIdx.x / nsplit;
  const int hq = qh % HQ, bs = qh / HQ, b = bs / S;
  const int nblk = (topk + kAttnBlock - 1) / kAttnBlock;
  const int blk0 = c * bps, blk1 = min(blk0 + bps, nblk);
  const int nb = blk1 - blk0;  // >= 1: the host never launches an empty split
  const int hg0 = hq * 64 + 16 * wave;
  const bool active = hg0 < H;  // H % 16 == 0: the whole head group exists

  // Q fragments first (they do not wait for the indices; B operand of S^T): lane (head nl, group g) holds d 32cc + 8g .. +8
  v8s_t qb[KC];
  const uint16_t* qrow = q + (int64_t(bs) * H + (active ? hg0 : 0) + nl) * D;
#pragma unroll
  for (int cc = 0; cc < KC; ++cc) qb[cc] = *reinterpret_cast<const v8s_t*>(qrow + 32 * cc + 8 * g);

  const int32_t* ib = idx + int64_t(bs) * topk + int64_t(blk0) * kAttnBlock;
  if (tid == 0) s_any = 0;
  for (int j = tid; j < nb * kAttnBlock; j += 256) {
    const int v = blk0 * kAttnBlock + j < topk ? ib[j] : -1;
    s_idx[j] = (v >= 0 && v < N) ? v : -1;
  }
  __syncthreads();
  if (blk0 == 0 && tid < kAttnBlock && s_idx[tid] >= 0) s_any = 1;

  // rows of block t -> ksb[t & 1]; an unused index reads past the end of the
  // buffer, which returns zeros (the reference zero-fills those rows)
  const __amdgpu_buffer_rsrc_t kv_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(kv + int64_t(b) * N * D), short(0), int(int64_t(N) * L::RB), 0x00020000);
  const uint32_t ks_lds = uint32_t(uintptr_t((__attribute__((address_space(3))) uint8_t*)&ksb[0][0]));
  // Load gi of a block fills rows gi * RPI .. +RPI; lane i writes slot i & (RB/16 - 1)
  // of row gi * RPI + i / (RB/16), so it fetches that row's chunk slot ^ swz(row).
  auto issue = [&](int t) {
    const int rin = lane / (L::RB / 16), slot = lane % (L::RB / 16);
    int ri[L::NG / 4];  // every row index first: the asm loads below order memory accesses
#pragma unroll
    for (int j = 0; j < L::NG / 4; ++j) ri[j] = s_idx[t * kAttnBlock + (j * 4 + wave) * L::RPI + rin];
#pragma unroll
    for (int j = 0; j < L::NG / 4; ++j) {
      const int gi = j * 4 + wave, row = gi * L::RPI + rin;
      const uint32_t vo = ri[j] < 0 ? 0x80000000u : uint32_t(ri[j]) * L::RB + ((slot ^ L::swz(row)) << 4);
      load_lds_16(kv_rsrc, __builtin_amdgcn_readfirstlane(ks_lds + (t & 1) * L::BYTES + gi * 1024), vo);
    }
  };
  issue(0);

  v4f acc[NT];  // acc[nt][i] = O[head 4g + i][16nt + nl]
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) acc[nt] = v4f{0.f, 0.f, 0.f, 0.f};
  float m_use = -INFINITY, l_run = 0.0f;  // head nl: running max, this lane's share of the sum

  for (int t = 0; t < nb; ++t) {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's loads of block t have landed
    __syncthreads();                // ... and every wave's; block t - 1's buffer is free
    if (t + 1 < nb) issue(t + 1);
    const uint8_t* ks = ksb[t & 1];
    const uint64_t vmask = __ballot(s_idx[t * kAttnBlock + lane] >= 0);
    if (!active) continue;

    // ---- S^T[rows, 16 heads]: sacc[rt][i] = S[row 16rt + 4g + i][head nl] ----
    // K fragments are read two d chunks ahead of their MFMAs (three buffers)
    v4f sacc[4];
#pragma unroll
    for (int rt = 0; rt < 4; ++rt) sacc[rt] = v4f{0.f, 0.f, 0.f, 0.f};
    v8s_t kf[3][4];
    auto kload = [&](int cc, v8s_t* dst) {
#pragma unroll
      for (int rt = 0; rt < 4; ++rt)
        dst[rt] = *reinterpret_cast<const v8s_t*>(ks + L::at(16 * rt + nl, 32 * cc + 8 * g));
    };
    kload(0, kf[0]);
    kload(1, kf[1]);
#pragma unroll
    for (int cc = 0; cc < KC; ++cc) {
      if (cc + 2 < KC) kload(cc + 2, kf[(cc + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);  // keep the reads two chunks ahead of their use
#pragma unroll
      for (int rt = 0; rt < 4; ++rt) sacc[rt] = mfma_bf16_32(kf[cc % 3][rt], qb[cc], sacc[rt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int rt = 0; rt < 4; ++rt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * rt + 4 * g + i;
        sacc[rt][i] = (vmask >> row) & 1 ? sacc[rt][i] * scale : -INFINITY;
        bmax = fmaxf(bmax, sacc[rt][i]);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, kWave));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, kWave));
    const bool bump = bmax > m_use + kLazyMax;
    if (__ballot(bump)) {
      const float m_new = bump ? bmax : m_use;
      const bool fresh = m_use == -INFINITY;  // nothing accumulated yet for this head
      const float resc = !bump ? 1.0f : (fresh ? 0.0f : __expf(m_use - m_new));
      l_run *= resc;
      m_use = m_new;
      // O[h, :] *= resc(h) on the matrix core, so the accumulators stay where the
      // P V products keep them: O += A_i B_i (V_MFMA_F32_16X16X4_F32, k = lane
      // group g) with B_i[g][n] = O[4g + i][n] (component i of each lane) and
      // A_i[m][g] = resc(m) - 1 where m = 4g + i, else 0; step i only changes
      // rows = i (mod 4), which later steps do not read.  Skipped while every
      // bumped head is fresh (its accumulators are still zero).
      if (__ballot(bump && !fresh)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float ai = nl == 4 * g + i ? resc - 1.0f : 0.0f;
#pragma unroll
          for (int nt = 0; nt < NT; ++nt)
            acc[nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(ai, acc[nt][i], acc[nt], 0, 0, 0);
        }
      }
    }
    v8s_t pa[2];
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      float pv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pv[i] = sacc[2 * kc][i] == -INFINITY ? 0.0f : __expf(sacc[2 * kc][i] - m_use);
        pv[4 + i] = sacc[2 * kc + 1][i] == -INFINITY ? 0.0f : __expf(sacc[2 * kc + 1][i] - m_use);
        l_run += pv[i] + pv[4 + i];
      }
      const uint4 u = make_uint4(cvt_bf16x2(pv[0], pv[1]), cvt_bf16x2(pv[2], pv[3]), cvt_bf16x2(pv[4], pv[5]),
                                 cvt_bf16x2(pv[6], pv[7]));
      pa[kc] = __builtin_bit_cast(v8s_t, u);
    }

    // ---- O[16 heads, D] += P[16 heads, 64 rows] V[64 rows, D] ----
    // V fragments are read two column tiles ahead of their MFMAs (three buffers)
    v8s_t vf[3][2];
    auto vload = [&](int nt, v8s_t* dst) {
      const int col = 16 * nt + 4 * (nl & 3);
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const int row = 32 * kc + 4 * g + (nl >> 2);
        const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t*)(ks + L::at(row, col)));
        const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t*)(ks + L::at(row + 16, col)));
        dst[kc] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      }
    };
    vload(0, vf[0]);
    vload(1, vf[1]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (nt + 2 < NT) vload(nt + 2, vf[(nt + 2) % 3]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) acc[nt] = mfma_bf16_32(pa[kc], vf[nt % 3][kc], acc[nt]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if (!active) return;

  l_run += __shfl_xor(l_run, 16, kWave);
  l_run += __shfl_xor(l_run, 32, kWave);
  const bool poisoned = blk0 == 0 && s_any == 0;
  if (!SPLIT) {
    // normalise by the sum (sink term included): one reciprocal per head, then
    // products (within 1 fp32 ulp of the quotient, before the bf16 rounding)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hd = hg0 + 4 * g + i;
      const float lh = __shfl(l_run, 4 * g + i, kWave), mh = __shfl(m_use, 4 * g + i, kWave);
      const float inv = poisoned ? __builtin_nanf("") : 1.0f / (lh + __expf(sink[hd] - mh));
      uint16_t* orow = o + (int64_t(bs) * H + hd) * D;
#pragma unroll
      for (int nt = 0; nt < NT; nt += 2) {
        const uint32_t pr = cvt_bf16x2(acc[nt][i] * inv, acc[nt + 1][i] * inv);
        orow[16 * nt + nl] = uint16_t(pr & 0xFFFFu);
        orow[16 * nt + 16 + nl] = uint16_t(pr >> 16);
      }
    }
  } else {
    float* pp = part + int64_t(blockIdx.x) * attn_part_floats(D);
    if (g == 0) {
      pp[16 * wave + nl] = m_use;
      pp[64 + 16 * wave + nl] = poisoned ? __builtin_nanf("") : l_run;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float* orow = pp + 128 + int64_t(16 * wave + 4 * g + i) * D;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) orow[16 * nt + nl] = acc[nt][i];
    }
  }
}

// Merge the (m, l, O) partials of 4 heads of one (query, 64 heads):
// o = sum_c e^(m_c - M) O_c / (sum_c e^(m_c - M) l_c + e^(sink - M)), M = max_c m_c.
// Every partial's (m, l) is loaded at once, then the O partials in batches of
// 16 splits, so each phase costs one memory round trip.
template <int D>
__global__ __launch_bounds__(256) void sparse_attn_combine_kernel(const float* __restrict__ part,
                                                                  const float* __restrict__ sink,
                                                                  uint16_t* __restrict__ o, int H, int nsplit) {
  constexpr int64_t PF = attn_part_floats(D);
  constexpr int kBatch = 16;
  __shared__ float s_m[4][kAttnMaxSplit], s_l[4][kAttnMaxSplit];
  __shared__ float wts[4][kAttnMaxSplit];
  __shared__ float inv[4];
  const int tid = threadIdx.x, HQ = (H + 63) / 64;
  const int k = blockIdx.x & 15, qh = blockIdx.x >> 4;
  const int hq = qh % HQ, bs = qh / HQ;
  const int hl0 = 4 * k;
  if (hq * 64 + hl0 >= H) return;  // heads come in groups of 16 (whole workgroup)
  const float* pb = part + int64_t(qh) * nsplit * PF;
  for (int j = tid; j < 4 * nsplit; j += 256) {
    const int h4 = j & 3, cs = j >> 2;
    s_m[h4][cs] = pb[cs * PF + hl0 + h4];
    s_l[h4][cs] = pb[cs * PF + 64 + hl0 + h4];
  }
  __syncthreads();
  if (tid < 4) {
    float M = -INFINITY;
    for (int cs = 0; cs < nsplit; ++cs) M = fmaxf(M, s_m[tid][cs]);
    float den = __expf(sink[hq * 64 + hl0 + tid] - M);
    for (int cs = 0; cs < nsplit; ++cs) {
      const float w = __expf(s_m[tid][cs] - M);
      wts[tid][cs] = w;
      den += w * s_l[tid][cs];
    }
    inv[tid] = 1.0f / den;
  }
  __syncthreads();
  for (int e = tid * 4; e < 4 * D; e += 256 * 4) {
    const int h4 = e / D, d = e % D;
    const float* src = pb + 128 + int64_t(hl0 + h4) * D + d;
    float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int c0 = 0; c0 < nsplit; c0 += kBatch) {
      float4 v[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        v[u] = c0 + u < nsplit ? *reinterpret_cast<const float4*>(src + (c0 + u) * PF) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const float w = c0 + u < nsplit ? wts[h4][c0 + u] : 0.0f;
        a.x += w * v[u].x;
        a.y += w * v[u].y;
        a.z += w * v[u].z;
        a.w += w * v[u].w;
      }
    }
    const float s = inv[h4];
    uint16_t* orow = o + (int64_t(bs) * H + hq * 64 + hl0 + h4) * D + d;
    *reinterpret_cast<uint2*>(orow) = make_uint2(pack_bf16x2(a.x * s, a.y * s), pack_bf16x2(a.z * s, a.w * s));
  }
}

// Split of one query's blocks over workgroups: enough workgroups for the chip
// (about 512) when there are few queries, at most kAttnIdxCap indices each.
struct AttnSplit {
  int nsplit, bps;
};

static inline AttnSplit attn_split(int64_t units, int64_t topk) {
  const int nblk = int((topk + kAttnBlock - 1) / kAttnBlock);
  const int cap_bps = kAttnIdxCap / kAttnBlock;
  int want = int(units >= 512 ? 1 : (512 + units - 1) / units);
  want = std::min(std::min(want, nblk), kAttnMaxSplit);
  int bps = (nblk + want - 1) / want;
  if (bps > cap_bps) bps = cap_bps;
  const int nsplit = (nblk + bps - 1) / bps;
  return {nsplit, bps};
}

template <int D>
static int launch_attn(const uint16_t* q, const uint16_t* kv, const float* sink, const int32_t* idx, uint16_t* o,
                       float* part, int64_t units, int S, int H, int N, int topk, AttnSplit sp, float scale,
                       hipStream_t stream) {
  if (sp.nsplit == 1) {
    WZ_LAUNCH("sparse_attn", stream, (sparse_attn_kernel<D, false>), dim3{unsigned(units)}, dim3(256), 0, q, kv,
              sink, idx, o, part, S, H, N, topk, sp.bps, 1, scale);
    return check_launch("sparse_attn");
  }
  WZ_LAUNCH("sparse_attn", stream, (sparse_attn_kernel<D, true>), dim3{unsigned(units * sp.nsplit)}, dim3(256), 0, q,
            kv, sink, idx, o, part, S, H, N, topk, sp.bps, sp.nsplit, scale);
  if (int rc = check_launch("sparse_attn")) return rc;
  WZ_LAUNCH("sparse_attn_combine", stream, sparse_attn_combine_kernel<D>, dim3{unsigned(units * 16)}, dim3(256), 0,
            part, sink, o, H, sp.nsplit);
  return check_launch("sparse_attn_combine");
}

}  // namespace wz

extern "C" int64_t wz_sparse_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int64_t topk) {
  using namespace wz;
  if (B <= 0 || S <= 0 || H <= 0 || topk <= 0 || H % 16) return 0;
  const int64_t units = B * S * ((H + 63) / 64);
  const AttnSplit sp = attn_split(units, topk);
  if (sp.nsplit <= 1) return 0;
  return units * sp.nsplit * attn_part_floats(int(D)) * int64_t(sizeof(float));
}

extern "C" int wz_sparse_attn(const void* q_bf16, const void* kv_bf16, const float* attn_sink,
                              const int32_t* topk_idxs, void* o_bf16, int64_t B, int64_t S, int64_t H, int64_t D,
                              int64_t N, int64_t topk, float softmax_scale, void* workspace, int64_t workspace_bytes,
                              hipStream_t stream) {
  using namespace wz;
  if (B < 0 || S < 0 || H <= 0 || N <= 0 || topk <= 0 || H % 16)
    return set_error(WZ_EINVAL, "sparse_attn: bad shape B=%lld S=%lld H=%lld (multiple of 16) N=%lld topk=%lld",
                     (long long)B, (long long)S, (long long)H, (long long)N, (long long)topk);
  if (D != 128 && D != 256 && D != 512)
    return set_error(WZ_EINVAL, "sparse_attn: head dim %lld (128, 256 or 512 are built)", (long long)D);
  if (B * S == 0) return WZ_OK;
  if (!q_bf16 || !kv_bf16 || !attn_sink || !topk_idxs || !o_bf16)
    return set_error(WZ_EINVAL, "sparse_attn: null pointer");
  if ((reinterpret_cast<uintptr_t>(q_bf16) | reinterpret_cast<uintptr_t>(kv_bf16) |
       reinterpret_cast<uintptr_t>(o_bf16) | reinterpret_cast<uintptr_t>(workspace)) & 15)
    return set_error(WZ_EINVAL, "sparse_attn: q, kv, o and the workspace must be 16-byte aligned");
  if (N * D * 2 > 0x7FFFFFFFLL)
    return set_error(WZ_EINVAL, "sparse_attn: a KV cache of %lld rows x %lld exceeds 2 GiB per sequence",
                     (long long)N, (long long)D);
  const int64_t units = B * S * ((H + 63) / 64);
  AttnSplit sp = attn_split(units, topk);
  if (sp.nsplit > kAttnMaxSplit)
    return set_error(WZ_EINVAL, "sparse_attn: topk %lld exceeds %d blocks of %d", (long long)topk,
                     kAttnMaxSplit * (kAttnIdxCap / kAttnBlock), kAttnBlock);
  const int64_t need = wz_sparse_attn_workspace_bytes(B, S, H, D, topk);
  if (sp.nsplit > 1 && (!workspace || workspace_bytes < need)) {
    if (workspace)
      return set_error(WZ_EINVAL, "sparse_attn: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
                       (long long)need);
    // no workspace: one workgroup per (query, 64 heads) over every block
    if (topk > kAttnIdxCap)
      return set_error(WZ_EINVAL, "sparse_attn: topk %lld > %d needs a workspace (wz_sparse_attn_workspace_bytes)",
                       (long long)topk, kAttnIdxCap);
    sp = AttnSplit{1, int((topk + kAttnBlock - 1) / kAttnBlock)};
  }
  const uint16_t* q = static_cast<const uint16_t*>(q_bf16);
  const uint16_t* kv = static_cast<const uint16_t*>(kv_bf16);
  uint16_t* o = static_cast<uint16_t*>(o_bf16);
  float* part = static_cast<float*>(workspace);
  if (D == 512)
    return launch_attn<512>(q, kv, attn_sink, topk_idxs, o, part, units, int(S), int(H), int(N), int(topk), sp,
                            softmax_scale, stream);
  if (D == 256)
    return launch_attn<256>(q, kv, attn_sink, topk_idxs, o, part, units, int(S), int(H), int(N), int(topk), sp,
                            softmax_scale, stream);
  return launch_attn<128>(q, kv, attn_sink, topk_idxs, o, part, units, int(S), int(H), int(N), int(topk), sp,
                          softmax_scale, stream);
}
