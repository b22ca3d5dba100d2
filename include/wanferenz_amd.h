/* wanferenz_amd — C ABI of the MI355X (gfx950) MoE + FP8-linear hot path.
 *
 * One shared library, libwanferenz_amd.so, replaces the kernel layer the
 * reference model calls (wanferenz/kernels/reference.py, its CPU twin
 * wanferenz/kernels/torch_ops.py, and the MoE dispatch patches in
 * wanferenz/kernels/{fp4_grouped,fp8_vector,expert_dispatch,expert_batch}.py).
 *
 * Conventions
 *   - Every entry point returns 0 on success and a negative code on error;
 *     wz_last_error() returns a thread-local message for the last failure.
 *   - All tensor arguments are device pointers to dense row-major storage.
 *   - Work is enqueued on the given stream.  No entry point allocates device
 *     memory, synchronises the host or reads device data back, so every call
 *     can be captured in a HIP graph.  Scratch memory comes in as `ws`.
 *   - Formats: bf16 activations/outputs; e4m3fn FP8 (OCP); e2m1 MXFP4 packed
 *     two per byte, low nibble = even element; e8m0 scales (2^(b-127)).
 */
#ifndef WANFERENZ_AMD_H
#define WANFERENZ_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes. */
#define WZ_OK 0
#define WZ_EINVAL (-1)   /* bad shape / argument */
#define WZ_ELAUNCH (-2)  /* HIP launch failure */
#define WZ_ESPACE (-3)   /* workspace too small */

/* Activation scale kinds (act_quant's scale_fmt / scale_dtype pair,
 * wanferenz/kernels/torch_ops.py:33-49, partition.py:128-134). */
#define WZ_SCALE_F32 0        /* s = amax/448, stored float32 (scale_fmt=None)       */
#define WZ_SCALE_UE8M0 1      /* s = 2^ceil(log2(amax/448)), stored as e8m0 bytes    */
#define WZ_SCALE_UE8M0_F32 2  /* same power-of-two s, stored as float32              */

/* Weight block-scale storage for FP8 weights (128x128 blocks). */
#define WZ_WSCALE_F32 0
#define WZ_WSCALE_E8M0 1

/* Gate score functions (ModelArgs.score_func, architecture.py:57). */
#define WZ_SCORE_SOFTMAX 0
#define WZ_SCORE_SIGMOID 1
#define WZ_SCORE_SQRTSOFTPLUS 2

const char* wz_last_error(void);

/* Library / device properties. */
int wz_device_info(int* cu_count, int* xcd_count);

/* act_quant: per-row, per-128-column dynamic FP8 quantisation.
 * Replaces act_quant(x, block_size=128, scale_fmt, scale_dtype) —
 * wanferenz/kernels/reference.py:117-146 (TileLang) / torch_ops.py:33-49 (CPU).
 * x_bf16 [M, K] -> q_e4m3 [M, K], s [M, K/128] (float32 or e8m0 per scale_kind). */
int wz_act_quant_fp8(const void* x_bf16, int64_t M, int64_t K, void* q_e4m3, void* s,
                     int scale_kind, hipStream_t stream);

/* fp8_gemm: C[M,N] bf16 = (a * a_s) @ (w * w_s)^T, K-blocks of 128.
 * Replaces fp8_gemm(a, a_s, b, b_s, scale_dtype) — reference.py:292-311 / torch_ops.py:93-99,
 * and the decode retile _fp8_gemm_fast — fp8_vector.py:289-297.
 * a_e4m3 [M,K], a_s [M,K/128] (act_scale_kind), w_e4m3 [N,K],
 * w_s [ceil(N/128), ceil(K/128)] (w_scale_kind). */
int wz_fp8_gemm(const void* a_e4m3, const void* a_s, const void* w_e4m3, const void* w_s,
                void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                int w_scale_kind, hipStream_t stream);

/* fp8 linear with act_quant fused into the GEMM prologue: y = linear(x, w) for an
 * FP8 weight — architecture.py:121-132 (act_quant + fp8_gemm). */
int wz_fp8_linear(const void* x_bf16, const void* w_e4m3, const void* w_s, void* y_bf16,
                  int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                  hipStream_t stream);

/* FP8 linear on a packed weight.  wz_fp8_pack relays W e4m3 [N, K] (N % 16 == 0,
 * K % 128 == 0) once into MFMA-ready 16-row x 128-K tiles, [N/16][K/128][2][1 KB]
 * (N*K bytes), the load-time relayout the reference does for its FP8 decode GEMV
 * (fp8_vector.py:316-351 _lay_shared).  wz_fp8_linear_packed then computes
 * y[M,N] bf16 = linear(x, w) with act_quant fused — architecture.py:121-132
 * (act_quant + fp8_gemm, reference.py:117-146, 292-311); w_s [ceil(N/128), K/128]
 * float32 or e8m0 (w_scale_kind); act_scale_kind selects the activation scale rule
 * (WZ_SCALE_F32: amax/448, otherwise the power-of-two ue8m0 rule).  M <= 16 with
 * K in {1024, 2048, 4096, 8192} needs no workspace; otherwise ws must hold
 * wz_fp8_linear_workspace_bytes(M, K) bytes (the quantised x). */
int wz_fp8_pack(const void* w_e4m3, int64_t N, int64_t K, void* packed, hipStream_t stream);
size_t wz_fp8_linear_workspace_bytes(int64_t M, int64_t K);
int wz_fp8_linear_packed(const void* x_bf16, const void* w_packed, const void* w_s, void* y_bf16,
                         int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                         void* ws, size_t ws_bytes, hipStream_t stream);

/* fp8_gemm on a packed weight (wz_fp8_pack): the same product as wz_fp8_gemm from
 * pre-quantised activations a_e4m3 [M, K] with a_s [M, K/128] (act_scale_kind) —
 * fp8_gemm(a, a_s, b, b_s), reference.py:292-311, served the way the reference's
 * decode retile serves it (_fp8_gemm_fast, fp8_vector.py:289-297): M <= 16 with
 * K in {1024, 2048, 4096, 8192} runs the GEMV, otherwise the dense tile GEMM.  ws must
 * hold wz_fp8_gemm_packed_workspace_bytes(M, K, act_scale_kind) bytes (nonzero
 * only for e8m0 activation scales outside the GEMV). */
size_t wz_fp8_gemm_packed_workspace_bytes(int64_t M, int64_t K, int act_scale_kind);
int wz_fp8_gemm_packed(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                       void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                       void* ws, size_t ws_bytes, hipStream_t stream);

/* The two entries above with the decoder block's residual step fused into the
 * producer: y = residual + linear(..), the product rounded to bf16 and the fp32
 * sum rounded once, as the bf16 tensor add x + attn(x) of Block.forward
 * (architecture.py:853-874).  No counterpart in the reference's kernel set (its
 * add is a separate torch op); for a decode stage that keeps the residual
 * stream out of an extra pass.  residual [M, N] bf16 must not overlap y; the
 * workspace rules are those of the entry without the residual. */
int wz_fp8_linear_packed_add(const void* x_bf16, const void* w_packed, const void* w_s, const void* residual_bf16,
                             void* y_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind, int w_scale_kind,
                             void* ws, size_t ws_bytes, hipStream_t stream);
int wz_fp8_gemm_packed_add(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                           const void* residual_bf16, void* c_bf16, int64_t M, int64_t N, int64_t K,
                           int act_scale_kind, int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream);

/* Two FP8 projections of the same quantised input in one launch, as the
 * decoder block has them (wq_a and wkv on the normed hidden state, wq_b and the
 * indexer's wq_b on the normed query latent, architecture.py:611-672): the
 * weights stacked row-wise [W0; W1] (N = N0 + N1 rows, N0 % 128 == 0) and packed
 * once (wz_fp8_pack), w_s their stacked block scales; c0 [M, N0] and c1 [M, N1]
 * receive fp8_gemm(a, a_s, W0, s0) and fp8_gemm(a, a_s, W1, s1).  No counterpart
 * in the reference's kernel set (two launches there).  Workspace rules of
 * wz_fp8_gemm_packed. */
int wz_fp8_gemm_packed_pair(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_s,
                            void* c0_bf16, int64_t N0, void* c1_bf16, int64_t M, int64_t N, int64_t K,
                            int act_scale_kind, int w_scale_kind, void* ws, size_t ws_bytes, hipStream_t stream);

/* fp4_gemm: C[M,N] bf16 = (a * a_s) @ (e2m1(w) * w_s)^T, weight scale e8m0 per 32 K.
 * Replaces fp4_gemm(a, a_s, b, b_s, scale_dtype) — reference.py:572-591 / torch_ops.py:102-108.
 * a_e4m3 [M,K], a_s [M,K/128], w_fp4x2 [N,K/2], w_s_e8m0 [N,K/32]. */
int wz_fp4_gemm(const void* a_e4m3, const void* a_s, const void* w_fp4x2, const void* w_s_e8m0,
                void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                hipStream_t stream);

/* fp4_gemm on a packed weight, for row counts past decode (the M = 2048 product of
 * one prefill expert): the same product as wz_fp4_gemm — reference.py:572-591 /
 * torch_ops.py:102-108 — served by the tile GEMM of the MoE prefill instead of the
 * row-major skinny kernel.  wz_fp4_pack relays w_fp4x2 [N, K/2] and w_s_e8m0
 * [N, K/32] once (N % 16 == 0, K % 128 == 0) into the 16-row x 128-K tile format
 * of the expert banks: packed N*K/2 bytes, packed_s wz_fp4_packed_scale_bytes(N, K)
 * bytes — the relayout fp4_grouped._relayout_moe does for its bank, for one
 * weight (fp4_grouped.py:142-188).  ws must hold
 * wz_fp4_gemm_packed_workspace_bytes(M, K, act_scale_kind) bytes (nonzero only
 * for e8m0 activation scales). */
size_t wz_fp4_packed_scale_bytes(int64_t N, int64_t K);
int wz_fp4_pack(const void* w_fp4x2, const void* w_s_e8m0, int64_t N, int64_t K, void* packed, void* packed_s,
                hipStream_t stream);
size_t wz_fp4_gemm_packed_workspace_bytes(int64_t M, int64_t K, int act_scale_kind);
int wz_fp4_gemm_packed(const void* a_e4m3, const void* a_s, const void* w_packed, const void* w_packed_s,
                       void* c_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind, void* ws,
                       size_t ws_bytes, hipStream_t stream);

/* Grouped MXFP4 GEMM — grouped_fp4_gemm(a, a_s, w, w_s, scale_dtype),
 * fp4_grouped.py:96-128: row g of a against its own weight, C[g, :] =
 * dequant(a[g]) @ (e2m1(w[g]) * w_s[g])^T, i.e. fp4_gemm of one row per expert
 * (the reference's CPU path loops fp4_gemm the same way, :112-121).
 * a [G, K] e4m3 + a_s [G, K/128] (act_scale_kind as wz_fp4_gemm), w [G, N, K/2]
 * e2m1x2 + w_s [G, N, K/32] e8m0 -> c [G, N] bf16; N % 16 == 0, K % 128 == 0. */
int wz_grouped_fp4_gemm(const void* a_e4m3, const void* a_s, const void* w_fp4x2, const void* w_s_e8m0,
                        void* c_bf16, int64_t G, int64_t N, int64_t K, int act_scale_kind,
                        hipStream_t stream);

/* One MoE layer (Gate + routed MXFP4 experts + FP8 shared expert + combine).
 * Mirrors MoE.forward — architecture.py:744-794, Gate.forward :696-718, Expert.forward :729-741,
 * on the expert-bank layout of fp4_grouped._relayout_moe (fp4_grouped.py:142-188). */
typedef struct wz_moe_desc {
  int32_t dim;            /* D */
  int32_t inter;          /* I (moe_inter_dim) */
  int32_t n_experts;      /* E */
  int32_t topk;           /* k (n_activated_experts) */
  int32_t score_func;     /* WZ_SCORE_* */
  int32_t act_scale_kind; /* WZ_SCALE_* (module scale_fmt) */
  int32_t shared_w_scale_kind; /* WZ_WSCALE_* of the shared expert's FP8 weights */
  float route_scale;
  float swiglu_limit;     /* <= 0: no clamp */
  int64_t vocab;          /* rows of tid2eid (hash layers) */
  const void* gate_w;     /* bf16 [E, D] */
  const float* gate_bias; /* fp32 [E]; NULL for hash-routed layers */
  const int32_t* tid2eid; /* int32 [vocab, k] for hash-routed layers, else NULL */
  /* Reference-layout weights: read only by wz_moe_pack; wz_moe_forward and
   * wz_moe_route accept NULL for these seven (w13, w13_s, w2, w2_s, sh_w1, sh_w3,
   * sh_w2), so a caller that packs expert by expert never holds them. */
  const void* w13;        /* fp4x2 [E, 2I, D/2]: rows [0,I) = w1, [I,2I) = w3 */
  const void* w13_s;      /* e8m0  [E, 2I, D/32] */
  const void* w2;         /* fp4x2 [E, D, I/2] */
  const void* w2_s;       /* e8m0  [E, D, I/32] */
  const void* sh_w1;      /* e4m3 [I, D] */
  const void* sh_w1_s;    /* [I/128, D/128]; the three shared scales are always required */
  const void* sh_w3;      /* e4m3 [I, D] */
  const void* sh_w3_s;
  const void* sh_w2;      /* e4m3 [D, I] */
  const void* sh_w2_s;    /* [D/128, I/128] */
  /* Packed banks (wz_moe_pack): MFMA-ready 16-row x 128-K tiles stored as 1 KB blocks in
   * lane order, so each weight load instruction of a wave reads 1 KB contiguous.  The
   * expert kernels of wz_moe_forward read only these; NULL -> wz_moe_forward fails. */
  const void* w13p;       /* [E][I/16][D/128][2 (w1,w3)][1024] */
  const void* w13p_s;     /* [E][I/16][ceil(D/512)][2][64 x 4]: 4 K-blocks of e8m0 per lane */
  const void* w2p;        /* [E][D/16][I/128][1024] */
  const void* w2p_s;      /* [E][D/16][ceil(I/512)][64 x 4] */
  const void* sh13p;      /* [I/16][D/128][2 (w1,w3)][2 halves][1024] */
  const void* sh2p;       /* [D/16][I/128][2 halves][1024] */
} wz_moe_desc;

/* Bytes of each packed bank (which: 0 w13p, 1 w13p_s, 2 w2p, 3 w2p_s, 4 sh13p, 5 sh2p). */
size_t wz_moe_packed_bytes(const wz_moe_desc* d, int which);

/* Build the packed banks from the reference-layout pointers of d (a one-time
 * load-step relayout, the role of fp4_grouped._relayout_moe, fp4_grouped.py:142-188).
 * Outputs are the six buffers of wz_moe_packed_bytes; d itself is not modified. */
int wz_moe_pack(const wz_moe_desc* d, void* w13p, void* w13p_s, void* w2p, void* w2p_s, void* sh13p,
                void* sh2p, hipStream_t stream);

/* Pack one routed expert straight from its own tensors into slot e of the packed
 * banks that d points at (d->w13p, w13p_s, w2p, w2p_s must be set; the other
 * pointers of d are not read): w1, w3 e2m1x2 [I, D/2] with e8m0 scales [I, D/32],
 * w2 e2m1x2 [D, I/2] with e8m0 [D, I/32].  Loading expert by expert this way
 * never materialises the reference-layout bank: the packed banks are the only
 * copy, the role of _relayout_moe(preserve=False) — fp4_grouped.py:142-188,
 * serving/partition.py:398-405, where the checkpoint is loaded into the bank. */
int wz_moe_pack_expert(const wz_moe_desc* d, int64_t e, const void* w1, const void* w1_s, const void* w3,
                       const void* w3_s, const void* w2, const void* w2_s, hipStream_t stream);

/* Pack the shared expert's FP8 weights (sh_w1, sh_w3 e4m3 [I, D], sh_w2 [D, I])
 * into d->sh13p and d->sh2p — the shared w1|w3 bank of fp8_vector._lay_shared
 * (fp8_vector.py:316-351) in the MFMA tile format. */
int wz_moe_pack_shared(const wz_moe_desc* d, const void* sh_w1, const void* sh_w3, const void* sh_w2,
                       hipStream_t stream);

/* Bytes of scratch that serve every wz_moe_forward / wz_moe_route call of 1..T
 * tokens (the decode tables of T <= 16 can outgrow a small prefill's needs).
 * T is capped at the chunk that wz_moe_forward runs at once (16384 / k tokens),
 * so the workspace of a long prompt stays that of one chunk. */
size_t wz_moe_workspace_bytes(const wz_moe_desc* d, int64_t T);

/* Zero the parts of a fresh workspace that must start at zero (arrival
 * counters).  Call once after allocating ws; the kernels leave them at zero. */
int wz_moe_workspace_init(void* ws, size_t ws_bytes, hipStream_t stream);

/* Full layer: x_bf16 [T, D], input_ids int64 [T] (read only by hash layers) -> y_bf16 [T, D].
 * Optional routing outputs (may be NULL): weights fp32 [T,k], indices int64 [T,k].
 * Any T: the tokens run in successive chunks of 16384 / k on one workspace
 * (MoE.forward takes any number of tokens, architecture.py:777-794).  A hash id
 * outside [0, vocab), or a tid2eid entry outside [0, E), gives that token NaN
 * routing weights and a NaN output row (the reference's tid2eid[input_ids]
 * raises); reads stay in bounds. */
int wz_moe_forward(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T,
                   void* y_bf16, float* weights_out, int64_t* indices_out, void* ws,
                   size_t ws_bytes, hipStream_t stream);

/* The block's ffn RMSNorm and the layer in one call: y_bf16 = MoE(RMSNorm(h_bf16)),
 * x = self.ffn_norm(x); x = self.ffn(x, input_ids) of Block.forward
 * (architecture.py:871-872); the norm is wz_rmsnorm's (RMSNorm.forward,
 * architecture.py:225-230: fp32 mean of squares, times 1 / sqrt(mean + eps),
 * times the fp32 weight, rounded to bf16).  norm_weight fp32 [D], D <= 4096.  Decode widths only,
 * 1 <= T <= 8 (the norm runs inside the routing launch, whose workgroups each
 * normalise the rows they read); other T: run the norm, then wz_moe_forward.
 * Bit-for-bit the output of the norm followed by wz_moe_forward. */
int wz_moe_forward_norm(const wz_moe_desc* d, const void* h_bf16, const float* norm_weight, float eps,
                        const int64_t* input_ids, int64_t T, void* y_bf16, float* weights_out,
                        int64_t* indices_out, void* ws, size_t ws_bytes, hipStream_t stream);

/* wz_moe_forward without a caller workspace: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The scratch is a device array
 * inside the library, WZ_MOE_NOALLOC_SCRATCH_BYTES (16 MiB) per GPU, held until the
 * process ends: enough for a V4-shape layer (D 4096, I 2048, 256 experts, top-6) up
 * to T = 156 tokens, and for any T where wz_moe_workspace_bytes(d, T) fits.  A larger
 * call fails with WZ_ESPACE and launches nothing.  The function allocates nothing;
 * its arrival counters are cleared by a fill kernel at the start of every call.
 * All calls on one GPU share its scratch array: calls that overlap on one GPU
 * (concurrent streams, or host threads) race and must be serialised by the caller. */
#define WZ_MOE_NOALLOC_SCRATCH_BYTES (16 << 20)
int wz_moe_forward_noalloc(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T,
                           void* y_bf16, float* weights_out, int64_t* indices_out, hipStream_t stream);

/* Profiling replay: re-launch one kernel stage of the preceding wz_moe_forward call
 * made with the same d, x, T, y and ws (the workspace still holds that call's
 * routing tables and intermediates), so a stage can be timed on its own or
 * captured alone in a graph.  Stages: WZ_STAGE_ROUTE (gate + top-k + permutation;
 * prefill also its M-tiles and act_quant(x)), WZ_STAGE_W13 (w1|w3 + SwiGLU, routed
 * and shared), WZ_STAGE_HQUANT (act_quant of h), WZ_STAGE_W2 (w2), WZ_STAGE_COMBINE
 * (the weighted combine into y; a no-op where a decode shape fuses it into w2).
 * No counterpart in the reference (its benchmarks time whole calls). */
#define WZ_STAGE_ROUTE 0
#define WZ_STAGE_W13 1
#define WZ_STAGE_HQUANT 2
#define WZ_STAGE_W2 3
#define WZ_STAGE_COMBINE 4
int wz_moe_replay_stage(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T,
                        int stage, void* y_bf16, void* ws, size_t ws_bytes, hipStream_t stream);

/* Routing only (Gate.forward + the canonical permutation of expert_batch.py:24-37):
 * weights fp32 [T,k], indices int64 [T,k], offsets int32 [E+1],
 * perm_token int32 [T*k], perm_slot int32 [T*k]; T * k <= 16384. */
int wz_moe_route(const wz_moe_desc* d, const void* x_bf16, const int64_t* input_ids, int64_t T,
                 float* weights, int64_t* indices, int32_t* offsets, int32_t* perm_token,
                 int32_t* perm_slot, void* ws, size_t ws_bytes, hipStream_t stream);

/* RMSNorm (architecture.py:217-230): y = bf16(w * x * rsqrt(mean(x^2) + eps)), fp32 math;
 * x_bf16 [T, D], weight fp32 [D]. */
int wz_rmsnorm(const void* x_bf16, const float* weight, void* y_bf16, int64_t T, int64_t D,
               float eps, hipStream_t stream);

/* bf16 elementwise add (residual): out = bf16(float(a) + float(b)). */
int wz_add_bf16(const void* a, const void* b, void* out, int64_t n, hipStream_t stream);

/* RMSNorm fused with the FP8 act_quant of its output — RMSNorm.forward
 * (architecture.py:217-230) followed by act_quant (reference.py:117-146,
 * torch_ops.py:33-49) as the producer of an FP8 linear's input, without the
 * bf16 row in memory.  x [T, D] bf16 (D % 128 == 0, D <= 8192), weight fp32 [D]
 * -> q e4m3 [T, D], s [T, D/128] (scale_kind as wz_act_quant_fp8). */
int wz_rmsnorm_quant(const void* x_bf16, const float* weight, void* q_e4m3, void* s, int64_t T,
                     int64_t D, float eps, int scale_kind, hipStream_t stream);

/* The residual step of the decoder block (h = x + b, Block.forward
 * architecture.py:853-874, a bf16 tensor add) fused with the next RMSNorm and
 * its act_quant (wz_rmsnorm_quant): sum_bf16 (optional, may be null) receives
 * h, q / s the FP8 input of the next linear.  No counterpart in the reference's
 * kernel set (three torch ops there). */
int wz_add_rmsnorm_quant(const void* x_bf16, const void* b_bf16, const float* weight, void* sum_bf16,
                         void* q_e4m3, void* s, int64_t T, int64_t D, float eps, int scale_kind, hipStream_t stream);

/* The decoder block's norm and the FP8 projections it feeds in one launch:
 * c0 / c1 = the two linears of wz_fp8_gemm_packed_pair on act_quant(RMSNorm(h))
 * (architecture.py:217-230, reference.py:117-146; the attention side's
 * attn_norm -> wq_a / wkv and q_norm -> wq_b / indexer wq_b,
 * architecture.py:611-672, 853-874), where h = x, or h = x + b (the residual
 * step, a bf16 add) when b_bf16 is given; sum_bf16 (optional, needs b)
 * receives h.  x, b [M, K] bf16, norm_weight fp32 [K], K in {1024, 2048, 4096,
 * 8192}; c1 null means one linear (N0 = N).  The codes the linears read are
 * those of wz_add_rmsnorm_quant / wz_rmsnorm_quant bit for bit.  M is limited
 * to wz_fp8_norm_linear_max_rows(K) (4 at K = 1024, 4096, 8192; 2 at 2048);
 * larger M raises WZ_EINVAL (run the unfused ops).  Outputs must not overlap
 * the inputs.  No counterpart in the reference's kernel set. */
int wz_fp8_norm_linear_packed_pair(const void* x_bf16, const void* b_bf16, const float* norm_weight, float eps,
                                   void* sum_bf16, const void* w_packed, const void* w_s, void* c0_bf16,
                                   int64_t N0, void* c1_bf16, int64_t M, int64_t N, int64_t K, int act_scale_kind,
                                   int w_scale_kind, hipStream_t stream);

/* Rows wz_fp8_norm_linear_packed_pair serves at K (0: K unsupported). */
int wz_fp8_norm_linear_max_rows(int64_t K);

/* Sparse attention over gathered KV rows — sparse_attn(q, kv, attn_sink, topk_idxs,
 * softmax_scale), torch_ops.py:114-146 / reference.py:314-418: blockwise online
 * softmax with a per-head sink logit in the denominator, K = V = kv (one KV head).
 * q [B, S, H, D] bf16 (H % 16 == 0, D in {128, 256, 512}), kv [B, N, D] bf16,
 * attn_sink [H] fp32, topk_idxs [B, S, topk] int32 (-1 or >= N: unused) ->
 * o [B, S, H, D] bf16; q, kv, o 16-byte aligned.  A query whose first 64 indices
 * are all unused gets NaN, as in the reference.  With H % 64 == 0 and few queries
 * the 64-index blocks of a query are split over workgroups whose partial results
 * go to `workspace` (wz_sparse_attn_workspace_bytes; 0 = no split at this shape):
 * pass NULL to compute every query in one workgroup instead (topk <= 2048). */
int64_t wz_sparse_attn_workspace_bytes(int64_t B, int64_t S, int64_t H, int64_t D, int64_t topk);
int wz_sparse_attn(const void* q_bf16, const void* kv_bf16, const float* attn_sink,
                   const int32_t* topk_idxs, void* o_bf16, int64_t B, int64_t S, int64_t H,
                   int64_t D, int64_t N, int64_t topk, float softmax_scale, void* workspace,
                   int64_t workspace_bytes, hipStream_t stream);

/* The FP8 wire format of a pipeline-stage boundary — _pack_t / _unpack_t
 * (serving/chain.py:208-222): per row scale = bf16(clamp(amax/448, 1e-8, bf16 max)),
 * q = e4m3(clamp(x/scale, +-448)); unpack y = bf16(q * scale).  x, y [M, D] bf16,
 * q [M, D] e4m3, scale [M] bf16. */
int wz_fp8_wire_pack(const void* x_bf16, void* q_e4m3, void* scale_bf16, int64_t M, int64_t D,
                     hipStream_t stream);
int wz_fp8_wire_unpack(const void* q_e4m3, const void* scale_bf16, void* y_bf16, int64_t M, int64_t D,
                       hipStream_t stream);

/* Synthetic-input generator (no reference counterpart: fills benchmark and test inputs
 * with the portable counter-based hash of wanferenz_amd/synth.py).
 * mode 0: u8 = low byte of draw; 1: e8m0 = lo + draw % (hi-lo+1);
 * 2: e4m3 = low byte with NaN codes zeroed; 3: f32 = lo + (draw>>41)*2^-23*(hi-lo). */
int wz_synth_fill(void* dst, int64_t n, uint64_t key, int64_t start, int mode, double lo,
                  double hi, hipStream_t stream);

/* Live kernel timing (no reference counterpart; used by bench.py): while enabled,
 * every launch of this library made outside graph capture is bracketed by two
 * HIP events on its stream.  wz_prof_end() disables and returns the number of
 * recorded launches; wz_prof_get(i) synchronises launch i and returns its name
 * and elapsed milliseconds. */
int wz_prof_begin(int max_launches);
int wz_prof_end(void);
int wz_prof_get(int i, const char** name, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* WANFERENZ_AMD_H */
