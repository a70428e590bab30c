/*
 * cgdr_wy.h -- C ABI of the MI355X (gfx950) WY producer: the inputs w, u and g of
 * ChunkGatedDeltaRuleFwdH from keys, values, beta and the per-token log-decay.
 *
 * Per sequence, value head h (key head h / (H/Hg)) and chunk of L <= 64 tokens:
 *
 *     g_i  = a_0 + ... + a_i                          chunk-local cumsum of the log-decay a
 *     A_ij = beta_i (k_i . k_j) e^{g_i - g_j}         j < i
 *     T    = (I + A)^{-1}
 *     w    = T diag(beta e^g) k,   u = T diag(beta) v
 *
 * Reference interfaces replaced (paths relative to the reference's
 * ChunkGatedDeltaRuleFwdH_problem_290_template/):
 *   - the WY part of the full operator's fp32 golden,
 *     ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:102-124
 *     (k_beta, v_beta, chunk cumsum of g, decay mask, the forward-substitution loop,
 *     value = attn @ v_beta, k_cumdecay = attn @ (k_beta e^g));
 *   - its device stage 1, class Stage1 in
 *     ref/chunk_gated_delta_rule/op_kernel/arch22/chunk_gated_delta_rule_stage1.h:69-924,
 *     and the bf16 variant stage1_opt of
 *     ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py:14-93.
 * The reference exposes these only inside the full operator's ACLNN API
 * (ref/chunk_gated_delta_rule/op_host/op_api/aclnn_chunk_gated_delta_rule.cpp:125-226).
 *
 * Precision: g in fp32 (sequential sum), k k^T accumulated in fp32, T in fp32, the scaled T
 * rounded to bf16 as the operand of the final products, w and u stored in in_dtype.
 * Conventions are those of cgdr_fwd_h.h.
 */
#ifndef CGDR_WY_H_
#define CGDR_WY_H_

#include "cgdr_fwd_h.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Token-major (FLA) shapes: k [B,T,Hg,K], v [B,T,H,V], beta [B,T,H], g [B,T,H]
 * -> w [B,T,H,K], u [B,T,H,V], g_cumsum [B,T,H]. */
typedef struct cgdr_wy_args {
  const void* k;                /* required, in_dtype                                          */
  const void* v;                /* required, in_dtype                                          */
  const void* beta;             /* required, beta_dtype                                        */
  const float* g;               /* nullable: per-token log-decay (no decay when NULL)          */
  const int64_t* cu_seqlens;    /* nullable: fixed-length batch; else N+1 offsets, B == 1      */
  const int64_t* chunk_indices; /* nullable: NT rows of (sequence, chunk); derived when NULL   */
  void* w;                      /* required, in_dtype                                          */
  void* u;                      /* required, in_dtype                                          */
  float* g_cumsum;              /* nullable: chunk-local cumsum of g (FwdH's g input), fp32    */

  int64_t B, T, H, Hg, K, V, N, NT, chunk_size;
  int32_t in_dtype;             /* only CGDR_BF16 is built                                     */
  int32_t beta_dtype;           /* CGDR_BF16 or CGDR_F32                                        */

  /* element strides (b, t, head) of each tensor */
  int64_t stride_k[3];
  int64_t stride_v[3];
  int64_t stride_beta[3];
  int64_t stride_g[3];
  int64_t stride_w[3];
  int64_t stride_u[3];
  int64_t stride_g_cumsum[3];
} cgdr_wy_args;

/* Validate and enqueue on `stream`.  Needs no workspace. */
cgdr_status cgdr_wy_launch(const cgdr_wy_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CGDR_WY_H_ */
