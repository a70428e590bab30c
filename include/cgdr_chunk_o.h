/*
 * cgdr_chunk_o.h -- C ABI of the MI355X (gfx950) chunk-output operator, the consumer of
 * ChunkGatedDeltaRuleFwdH's h and v_new.
 *
 * For every batch row b, value head h (key head h / (H/Hg)) and token i of chunk c:
 *
 *     o[i] = scale * ( e^{g_i} q_i . h[c]  +  sum_{j <= i, j in chunk c} (q_i . k_j) e^{g_i - g_j} v_new[j] )
 *
 * with g the chunk-local cumulative log-decay (the FwdH gate input).  Chunks are
 * independent: the state h[c] entering each chunk comes from cgdr_fwd_h_launch.
 *
 * Reference interfaces replaced (paths relative to the reference's
 * ChunkGatedDeltaRuleFwdH_problem_290_template/):
 *   - the per-chunk output of the full operator's fp32 golden,
 *     ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:136-142
 *     (core_attn_out = attn_inter + attn @ v_new; query scaled at :99-100, decay mask :116);
 *   - its device stages: attn_inter = (scale e^{g} q) S in
 *     ref/chunk_gated_delta_rule/op_kernel/arch22/chunk_gated_delta_rule_stage2.h:170 and the
 *     masked (scale q k^T e^{g_i - g_j}) v_new product of
 *     ref/chunk_gated_delta_rule/op_kernel/arch22/chunk_gated_delta_rule_stage3.h:131-180.
 * The reference exposes these only inside the full operator's ACLNN API
 * (ref/chunk_gated_delta_rule/op_host/op_api/aclnn_chunk_gated_delta_rule.cpp:125-226); this
 * entry point takes FwdH's outputs directly.
 *
 * Conventions are those of cgdr_fwd_h.h: device pointers, element strides of the outer
 * dimensions (token-major and head-major layouts both expressed by strides), status codes
 * and cgdr_last_error(), no allocation, no synchronisation, stream-ordered, deterministic.
 */
#ifndef CGDR_CHUNK_O_H_
#define CGDR_CHUNK_O_H_

#include "cgdr_fwd_h.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Arguments of one chunk-output call.  Token-major (FLA) shapes:
 * q, k [B,T,Hg,K], v_new [B,T,H,V], h [B,NT,H,K,V], g [B,T,H] -> o [B,T,H,V]. */
typedef struct cgdr_chunk_o_args {
  const void* q;                /* required, in_dtype                                          */
  const void* k;                /* required, in_dtype                                          */
  const void* v_new;            /* required, in_dtype (FwdH v_new)                             */
  const void* h;                /* required, in_dtype (FwdH h: state entering every chunk)     */
  const float* g;               /* nullable: no gating                                         */
  const int64_t* cu_seqlens;    /* nullable: fixed-length batch; else N+1 offsets, B == 1      */
  const int64_t* chunk_indices; /* nullable: NT rows of (sequence, chunk); derived on the
                                   device from cu_seqlens when NULL                           */
  void* o;                      /* required, in_dtype                                          */

  int64_t B, T, H, Hg, K, V;    /* batch, tokens, value heads, key heads, head dims            */
  int64_t N;                    /* sequences: B, or len(cu_seqlens) - 1                        */
  int64_t NT;                   /* chunks per batch row: ceil(T/64), or sum ceil(L_n/64)       */
  int64_t chunk_size;           /* must be 64                                                  */
  float scale;                  /* multiplies q (the reference's default is K^-0.5)            */
  int32_t in_dtype;             /* cgdr_dtype of q, k, v_new, h, o; only CGDR_BF16 is built    */

  /* element strides of the outer dimensions */
  int64_t stride_q[3];          /* (b, t, key head)                                            */
  int64_t stride_k[3];          /* (b, t, key head)                                            */
  int64_t stride_v[3];          /* (b, t, head) of v_new                                       */
  int64_t stride_h[3];          /* (b, chunk, head); each K x V block contiguous               */
  int64_t stride_g[3];          /* (b, t, head)                                                */
  int64_t stride_o[3];          /* (b, t, head)                                                */
} cgdr_chunk_o_args;

/* Validate and enqueue on `stream` (a hipStream_t, or NULL for the default stream).  Needs
 * no workspace.  Tokens of o outside every sequence (varlen gaps) are left untouched. */
cgdr_status cgdr_chunk_o_launch(const cgdr_chunk_o_args* args, void* stream);

/* Grid of the launch for `args` (host only): value columns per workgroup and workgroups. */
cgdr_status cgdr_chunk_o_get_plan(const cgdr_chunk_o_args* args, int32_t* v_tile, int64_t* workgroups);

#ifdef __cplusplus
}
#endif

#endif /* CGDR_CHUNK_O_H_ */
