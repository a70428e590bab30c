/*
 * cgdr_fwd_h.h -- C ABI of the MI355X (gfx950) ChunkGatedDeltaRuleFwdH operator.
 *
 * The operator runs the chunked gated delta-rule state recurrence.  For every
 * sequence n, value head h (key head h / (H/Hg)) and chunk c of up to 64 tokens:
 *
 *     h[c]      = S                                   (state entering the chunk)
 *     Vn        = U_c - W_c S                         ([L,V] = [L,V] - [L,K][K,V])
 *     v_new[c]  = Vn                                  (un-gated)
 *     S         = exp(g_last) S + K_c^T (exp(g_last - g_c) (.) Vn)
 *     final[n]  = S after the last chunk
 *
 * Reference interfaces replaced (paths relative to the reference's
 * ChunkGatedDeltaRuleFwdH_problem_290_template/):
 *   - Triton wrapper chunk_gated_delta_rule_fwd_h(k, w, u, g, initial_state,
 *     chunk_size, save_new_value, cu_seqlens, chunk_indices, chunk_offsets)
 *     -> (h, v_new, final_state)                       docs/problem.txt:436-500
 *   - ACLNN two-phase API generated from code/op_host/chunk_gated_delta_rule_fwd_h_def.cpp:8-78,
 *     as called in code/examples/test_aclnn_chunk_gated_delta_rule_fwd_h.cpp:299-325:
 *       aclnnChunkGatedDeltaRuleFwdHGetWorkspaceSize(...)   -> cgdr_fwd_h_workspace_size
 *       aclnnChunkGatedDeltaRuleFwdH(ws, size, exec, stream) -> cgdr_fwd_h_launch
 *   - host shape/dtype validation InferShapeChunkGatedDeltaRuleFwdH
 *     (code/op_host/chunk_gated_delta_rule_fwd_h_infershape.cpp:135-298) and the
 *     tiling function (code/op_host/chunk_gated_delta_rule_fwd_h_tiling.cpp:152-261),
 *     both folded into the validation done by every entry point below.
 *
 * Conventions
 *   - All tensor pointers are device pointers (HBM) except where a function says "host".
 *   - Element strides are given per tensor for its outer dimensions; the innermost
 *     dimension (K or V) and, for state tensors, the whole K x V block are contiguous.
 *     Token-major (FLA: w [B,T,H,K]) and head-major (contest run(): w [B,H,T,K]) layouts
 *     are both expressed by strides, with no copies.
 *   - No entry point allocates device memory, synchronises or keeps global state;
 *     cgdr_fwd_h_launch enqueues on the caller's HIP stream and returns.  Results are
 *     deterministic (no atomics, fixed reduction order).
 *   - Errors are returned as cgdr_status; cgdr_last_error() gives a message for the
 *     calling thread's most recent failure (the role of OP_LOGE in the reference).
 */
#ifndef CGDR_FWD_H_H_
#define CGDR_FWD_H_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CGDR_ABI_VERSION 4
#define CGDR_CHUNK_SIZE 64

/* Status codes.  The reference's aclnnStatus values for the same conditions are
 * ACLNN_ERR_PARAM_NULLPTR=161001, ACLNN_ERR_PARAM_INVALID=161002 and
 * ACLNN_ERR_INNER_TILING_ERROR=561002 (ref/chunk_gated_delta_rule/docs/aclnnChunkGatedDeltaRule.md:240-250). */
typedef enum cgdr_status {
  CGDR_OK = 0,
  CGDR_ERR_NULLPTR = 1,     /* a required pointer is null                         */
  CGDR_ERR_INVALID = 2,     /* shapes / strides / sizes are inconsistent          */
  CGDR_ERR_UNSUPPORTED = 3, /* valid request the library does not implement         */
  CGDR_ERR_LAUNCH = 4       /* the HIP runtime rejected the launch                 */
} cgdr_status;

typedef enum cgdr_dtype {
  CGDR_BF16 = 0,
  CGDR_F32 = 1
} cgdr_dtype;

/* Rounding model of the recurrence (cgdr_fwd_h_args.numerics).
 *   CGDR_NUMERICS_DEFAULT: bf16 inputs follow the Triton kernel (docs/problem.txt:330-432):
 *     fp32 state, bf16(S) and bf16(gated v_new) as GEMM operands; fp32 inputs are exact fp32.
 *   CGDR_NUMERICS_CONTEST: bf16 inputs only; the contest reference run() /
 *     run_reference (docs/problem.txt:81-167, code/tests/golden/generate_golden.py:350-440):
 *     bf16 state, bf16 GEMM outputs, saturating fp16 casts and nan_to_num after each GEMM,
 *     on the same pipelined kernel (a fast pass with plain fp16 roundings, then the casts
 *     again for the heads where one could matter; same results). */
typedef enum cgdr_numerics {
  CGDR_NUMERICS_DEFAULT = 0,
  CGDR_NUMERICS_CONTEST = 1
} cgdr_numerics;

/* Optional overrides of the launch plan (cgdr_fwd_h_args.tuning; NULL = the library's plan).
 * Every field has a "library's choice" value, so a zero-initialised struct with helpers,
 * prefetch and helper_lead set to -1 changes nothing.  Results never depend on these fields
 * (outputs are bit-identical for every V-tile, depth, load-wave count and helper setting);
 * they exist for tests, benchmarks and devices the library has not been tuned on.  There is
 * no counterpart in the reference: its tiling function picks one plan per shape. */
typedef struct cgdr_fwd_h_tuning {
  int32_t v_tile;        /* 0: library's choice; else 16, 32 or 64 value columns per task    */
  int32_t helpers;       /* -1: library's choice; 0: off; 1: on when tasks + helpers fit     */
  int32_t load_waves;    /* 0: library's choice; else 1, 2 or 4 (bf16 kernel)                 */
  int32_t stages;        /* 0: library's choice; else 2, 3 or 4 LDS stages (bf16 kernel)      */
  int32_t prefetch;      /* -1: library's choice; L2 touch distance in chunks without helpers */
  int32_t helper_lead;   /* -1: library's choice; chunks a helper runs ahead of its task       */
  int32_t helper_waves;  /* 0: library's choice; waves per helper workgroup                   */
  int32_t cu_count;      /* 0: the current device's compute units; else plan for this count  */
  int32_t xcd_count;     /* 0: the current device's XCDs (accelerator complex dies)          */
  int32_t row_split;     /* 0: library's choice; 1: one compute wave per 16 value columns; 2: two,
                            each with half of the state rows (bf16: K of 64 or 128); 4: four
                            (fp32 inputs, K of 64 or 128; bf16 takes 2)                       */
} cgdr_fwd_h_tuning;

/* Layout of each head's block in initial_state and final_state (h is always K x V). */
typedef enum cgdr_state_layout {
  CGDR_STATE_KV = 0,  /* K x V, rows of V: the Triton wrapper's [N,H,K,V] (docs/problem.txt:441-446) */
  CGDR_STATE_VK = 1   /* V x K, rows of K: the full operator's [N,Nv,Dv,Dk]
                         (ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_benchmark.py:101,184;
                         ref/chunk_gated_delta_rule/tests/assets/impl/golden.py:113-115) */
} cgdr_state_layout;

/* Arguments of one FwdH call.  Field meaning follows the Triton wrapper
 * (docs/problem.txt:436-472): k [B,T,Hg,K], w [B,T,H,K], u [B,T,H,V], g [B,T,H],
 * initial_state [N,H,K,V] -> h [B,NT,H,K,V], v_new [B,T,H,V], final_state [N,H,K,V]. */
typedef struct cgdr_fwd_h_args {
  const void* k;                /* required, in_dtype                                     */
  const void* w;                /* required, in_dtype                                     */
  const void* u;                /* required, in_dtype                                     */
  const float* g;               /* nullable: no gating (docs/problem.txt:400-402)         */
  const void* initial_state;    /* nullable: zero initial state; h0_dtype                 */
  const int64_t* cu_seqlens;    /* nullable: fixed-length batch; else N+1 offsets, B == 1 */
  const int64_t* chunk_offsets; /* nullable: derived on the device from cu_seqlens        */
  void* h;                      /* required, in_dtype, state entering every chunk         */
  void* v_new;                  /* nullable (save_new_value=False), in_dtype              */
  void* final_state;            /* nullable (output_final_state=False), final_dtype       */

  int64_t B, T, H, Hg, K, V;    /* batch, tokens, value heads, key heads, head dims       */
  int64_t N;                    /* sequences: B, or len(cu_seqlens) - 1                   */
  int64_t NT;                   /* chunks per batch row: ceil(T/64), or sum ceil(L_n/64)  */
  int64_t chunk_size;           /* must be 64 (code/op_host/chunk_gated_delta_rule_fwd_h_def.cpp:72-74) */

  int32_t in_dtype;             /* cgdr_dtype of k, w, u, h, v_new                        */
  int32_t h0_dtype;             /* cgdr_dtype of initial_state                            */
  int32_t final_dtype;          /* cgdr_dtype of final_state                              */
  int32_t numerics;             /* cgdr_numerics (0 = CGDR_NUMERICS_DEFAULT)              */

  /* element strides of the outer dimensions */
  int64_t stride_k[3];          /* (b, t, key head)                                        */
  int64_t stride_w[3];          /* (b, t, head)                                            */
  int64_t stride_u[3];          /* (b, t, head)                                            */
  int64_t stride_g[3];          /* (b, t, head)                                            */
  int64_t stride_h[3];          /* (b, chunk, head); each K x V block contiguous           */
  int64_t stride_v[3];          /* (b, t, head) of v_new                                   */
  int64_t stride_h0[2];         /* (n, head); each K x V block contiguous                  */
  int64_t stride_final[2];      /* (n, head); each K x V block contiguous                  */

  const cgdr_fwd_h_tuning* tuning; /* nullable (host memory): plan overrides, see above    */
  int32_t state_layout;         /* cgdr_state_layout of initial_state and final_state     */
  int32_t reserved;             /* must be 0                                              */
} cgdr_fwd_h_args;

/* Phase 1 (host only, no device access): validate the arguments and report the
 * workspace the launch needs: B*H*T*4 bytes rounded up to 256 (a head-major copy of g) when
 * g is given with a token stride other than 1, plus 128 bytes per task (progress counters)
 * when the plan uses helper workgroups, plus N*H*4 bytes (one flag per sequence and head)
 * with CGDR_NUMERICS_CONTEST; 0 when none applies.
 * Replaces aclnnChunkGatedDeltaRuleFwdHGetWorkspaceSize. */
cgdr_status cgdr_fwd_h_workspace_size(const cgdr_fwd_h_args* args, size_t* workspace_bytes);

/* Phase 2: validate again and enqueue the operator on `stream` (a hipStream_t, or
 * NULL for the default stream).  `workspace` (16-byte aligned device memory of at least
 * the phase-1 size; NULL when that size is 0) must not be in use by another launch until
 * this one has completed on `stream`.
 * Replaces aclnnChunkGatedDeltaRuleFwdH(workspace, size, executor, stream) and the
 * kernel launch of the Triton wrapper (docs/problem.txt:475-499). */
cgdr_status cgdr_fwd_h_launch(const cgdr_fwd_h_args* args, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Phase 2 without a workspace and without allocating.  No counterpart in the reference: for
 * callers that cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The same kernels as cgdr_fwd_h_launch, with the
 * workspace in a static device array of CGDR_NO_ALLOC_SCRATCH_BYTES (16 MiB) that each GPU
 * holds until the process ends; a call whose phase-1 workspace size exceeds it (a token-major
 * g needs B*H*T*4 bytes) returns CGDR_ERR_UNSUPPORTED.  It calls no hipMalloc/hipFree; the
 * first call on a device looks up the array's address there.  Every call on one GPU shares
 * that GPU's array: calls whose executions overlap on one GPU (other streams, or the same
 * stream from several host threads without ordering) race on it. */
#define CGDR_NO_ALLOC_SCRATCH_BYTES ((size_t)16 << 20)
cgdr_status cgdr_fwd_h_launch_no_alloc(const cgdr_fwd_h_args* args, void* stream);

/* Launch plan chosen for `args` (host only): the kernel variant and its grid.
 * Exposed for tests and benchmarks; the reference's counterpart is the tiling data
 * written by ChunkGatedDeltaRuleFwdHTilingFunc (code/op_host/chunk_gated_delta_rule_fwd_h_tiling.cpp:152-261). */
typedef struct cgdr_fwd_h_plan {
  int32_t kernel;       /* 0: bf16 MFMA pipeline, 1: fp32 MFMA kernel, 2: contest numerics */
  int32_t v_tile;       /* value columns per workgroup                               */
  int32_t compute_waves;/* 64-lane waves doing MFMA work per workgroup               */
  int32_t total_waves;  /* waves per workgroup (compute + load/store)                */
  int32_t stages;       /* LDS pipeline depth in chunks                              */
  int32_t lds_bytes;    /* LDS per workgroup                                          */
  int64_t workgroups;   /* grid size                                                  */
  int32_t helpers;      /* 1: one L2-prefetch helper workgroup beside every task        */
  int32_t load_waves;   /* DMA waves per task workgroup (bf16 kernel)                   */
  int32_t cu_count;     /* compute units the plan was made for                          */
  int32_t xcd_count;    /* XCDs the plan was made for                                   */
  int32_t row_split;    /* compute waves per 16 value columns (2, 4: state rows split)     */
} cgdr_fwd_h_plan;

cgdr_status cgdr_fwd_h_get_plan(const cgdr_fwd_h_args* args, cgdr_fwd_h_plan* plan);

/* Host helpers mirroring prepare_chunk_offsets / prepare_chunk_indices
 * (docs/problem.txt:251-270).  All pointers are host memory.
 * cu_seqlens has n_seq + 1 entries, starts at 0 and is non-decreasing.
 *   chunk_offsets_out: n_seq + 1 entries.
 *   chunk_indices_out: 2 * NT entries (rows of (sequence, chunk)); may be NULL, in which
 *   case only *nt_out is produced. */
cgdr_status cgdr_prepare_chunk_offsets(const int64_t* cu_seqlens, int64_t n_seq, int64_t chunk_size,
                                       int64_t* chunk_offsets_out);
cgdr_status cgdr_prepare_chunk_indices(const int64_t* cu_seqlens, int64_t n_seq, int64_t chunk_size,
                                       int64_t* chunk_indices_out, int64_t capacity_rows,
                                       int64_t* nt_out);

const char* cgdr_status_string(cgdr_status status);
const char* cgdr_last_error(void);
int cgdr_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CGDR_FWD_H_H_ */
