// cgdr_fwd_h.hip -- C ABI of the gfx950 ChunkGatedDeltaRuleFwdH operator (include/cgdr_fwd_h.h).
//
// Host side: argument validation (the role of InferShapeChunkGatedDeltaRuleFwdH,
// code/op_host/chunk_gated_delta_rule_fwd_h_infershape.cpp:135-298 of the reference, without
// its Ascend-only limits B=1, K==V and N<=4), the launch plan (the role of the tiling function,
// code/op_host/chunk_gated_delta_rule_fwd_h_tiling.cpp:152-261) and the kernel launch.  The
// kernels of each key dimension are instantiated in cgdr_fwd_h_k{32,64,128,256}.hip.
#include "../../include/cgdr_fwd_h.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <mutex>

#include "cgdr_fwd_h_dispatch.h"
#include "cgdr_host.h"
#include "cgdr_kernels.h"

namespace {

using cgdr_fwd::Plan;
using cgdr_host::fail;

constexpr int64_t kMaxHeadDim = 256;     // docs/problem.txt:466 (Triton wrapper assert K <= 256)
constexpr int64_t kMaxValueDim = 1024;   // V-tiling lifts the reference's K == V <= 256
constexpr int64_t kMaxTasks = 1 << 30;
constexpr int kDefaultCUs = 256;         // MI355X, when no device can be queried
constexpr int kDefaultXCDs = 8;
constexpr int64_t kHelperMinChunks = 96;  // shorter sequences run faster without helper workgroups

// Shape, stride and pointer checks shared by every entry point.
cgdr_status validate(const cgdr_fwd_h_args* a) {
  if (a == nullptr) return fail(CGDR_ERR_NULLPTR, "args is NULL");
  if (a->k == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input k is missing");
  if (a->w == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input w is missing");
  if (a->u == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input u is missing");
  if (a->h == nullptr) return fail(CGDR_ERR_NULLPTR, "Required output h is missing");
  if (a->chunk_size != CGDR_CHUNK_SIZE)
    return fail(CGDR_ERR_UNSUPPORTED, "chunk_size must be %d, but got %lld", CGDR_CHUNK_SIZE,
                (long long)a->chunk_size);
  if (a->in_dtype != CGDR_BF16 && a->in_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "in_dtype %d is not a cgdr_dtype", a->in_dtype);
  if (a->initial_state != nullptr && a->h0_dtype != CGDR_BF16 && a->h0_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "h0_dtype %d is not a cgdr_dtype", a->h0_dtype);
  if (a->final_state != nullptr && a->final_dtype != CGDR_BF16 && a->final_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "final_dtype %d is not a cgdr_dtype", a->final_dtype);
  if (a->numerics != CGDR_NUMERICS_DEFAULT && a->numerics != CGDR_NUMERICS_CONTEST)
    return fail(CGDR_ERR_INVALID, "numerics %d is not a cgdr_numerics", a->numerics);
  if (a->numerics == CGDR_NUMERICS_CONTEST && a->in_dtype != CGDR_BF16)
    return fail(CGDR_ERR_UNSUPPORTED, "contest numerics are defined for bf16 inputs only");
  if (a->state_layout != CGDR_STATE_KV && a->state_layout != CGDR_STATE_VK)
    return fail(CGDR_ERR_INVALID, "state_layout %d is not a cgdr_state_layout", a->state_layout);
  if (a->reserved != 0) return fail(CGDR_ERR_INVALID, "reserved must be 0");
  if (a->B < 1) return fail(CGDR_ERR_INVALID, "B must be >= 1, but got %lld", (long long)a->B);
  if (a->T < 1) return fail(CGDR_ERR_INVALID, "T must be >= 1, but got %lld", (long long)a->T);
  if (a->H < 1 || a->Hg < 1)
    return fail(CGDR_ERR_INVALID, "H/Hg are out of range: H=%lld, Hg=%lld", (long long)a->H, (long long)a->Hg);
  if (a->H % a->Hg != 0)
    return fail(CGDR_ERR_INVALID, "H must be divisible by Hg: H=%lld, Hg=%lld", (long long)a->H, (long long)a->Hg);
  if (a->K < 1 || a->K > kMaxHeadDim)
    return fail(CGDR_ERR_INVALID, "K must be in [1, %lld], but got %lld", (long long)kMaxHeadDim, (long long)a->K);
  if (a->V < 1 || a->V > kMaxValueDim)
    return fail(CGDR_ERR_INVALID, "V must be in [1, %lld], but got %lld", (long long)kMaxValueDim, (long long)a->V);

  const int64_t nt_fixed = (a->T + CGDR_CHUNK_SIZE - 1) / CGDR_CHUNK_SIZE;
  if (a->cu_seqlens == nullptr) {
    if (a->chunk_offsets != nullptr)
      return fail(CGDR_ERR_INVALID, "chunk_offsets given without cu_seqlens");
    if (a->N != a->B)
      return fail(CGDR_ERR_INVALID, "N must equal B without cu_seqlens: N=%lld, B=%lld", (long long)a->N, (long long)a->B);
    if (a->NT != nt_fixed)
      return fail(CGDR_ERR_INVALID, "NT must be ceil(T/64)=%lld, but got %lld", (long long)nt_fixed, (long long)a->NT);
  } else {
    if (a->B != 1) return fail(CGDR_ERR_INVALID, "B must be 1 with cu_seqlens, but got %lld", (long long)a->B);
    if (a->N < 1) return fail(CGDR_ERR_INVALID, "N must be >= 1 with cu_seqlens, but got %lld", (long long)a->N);
    if (a->N > a->T)
      return fail(CGDR_ERR_INVALID, "The number of non-empty sequences cannot exceed T");
    // code/op_host/chunk_gated_delta_rule_fwd_h_infershape.cpp:257-275
    const int64_t lo = nt_fixed, hi = nt_fixed + a->N - 1;
    if (a->NT < lo || a->NT > hi)
      return fail(CGDR_ERR_INVALID, "NT=%lld is impossible for T=%lld and N=%lld; expected range [%lld, %lld]",
                  (long long)a->NT, (long long)a->T, (long long)a->N, (long long)lo, (long long)hi);
  }

  // Strides: inner dims contiguous by contract; outer strides must be positive and large enough
  // that rows do not overlap within one tensor.
  const int64_t* sk = a->stride_k;
  const int64_t* sw = a->stride_w;
  const int64_t* su = a->stride_u;
  const int64_t* sh = a->stride_h;
  struct { const char* name; const int64_t* s; int64_t inner; bool present; } st3[] = {
      {"k", sk, a->K, true}, {"w", sw, a->K, true}, {"u", su, a->V, true},
      {"g", a->stride_g, 1, a->g != nullptr}, {"v_new", a->stride_v, a->V, a->v_new != nullptr},
  };
  for (auto& e : st3) {
    if (!e.present) continue;
    if (e.s[1] < 1 || e.s[2] < 1 || e.s[0] < 0)
      return fail(CGDR_ERR_INVALID, "%s has non-positive strides (%lld, %lld, %lld)", e.name,
                  (long long)e.s[0], (long long)e.s[1], (long long)e.s[2]);
  }
  if (sh[0] < 0 || sh[1] < a->K * a->V || sh[2] < a->K * a->V)
    return fail(CGDR_ERR_INVALID, "h strides must keep K x V blocks apart");
  if (a->initial_state != nullptr && (a->stride_h0[0] < 0 || a->stride_h0[1] < a->K * a->V))
    return fail(CGDR_ERR_INVALID, "initial_state strides must keep K x V blocks apart");
  if (a->final_state != nullptr && (a->stride_final[0] < 0 || a->stride_final[1] < a->K * a->V))
    return fail(CGDR_ERR_INVALID, "final_state strides must keep K x V blocks apart");
  return CGDR_OK;
}

int bf16_max_stages(int64_t K, int ncw, int nlw, int rs);

bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

// Compute units and XCDs of the calling thread's current device (tuning overrides first; the
// MI355X figures when no device answers, e.g. when planning on a host without a GPU).
// The counts are queried once per device and kept (they cannot change while the process runs;
// every call plans twice, for its workspace size and for its launch).
constexpr int kTopoDevices = 64;
std::atomic<int> g_topo_cus[kTopoDevices], g_topo_xcds[kTopoDevices];

void topology(const cgdr_fwd_h_tuning* tu, int* cus, int* xcds) {
  *cus = kDefaultCUs;
  *xcds = kDefaultXCDs;
  int dev = 0, c = 0, x = 0;
  if (hipGetDevice(&dev) == hipSuccess) {
    const bool cached = dev >= 0 && dev < kTopoDevices;
    if (cached) {
      c = g_topo_cus[dev].load(std::memory_order_relaxed);
      x = g_topo_xcds[dev].load(std::memory_order_relaxed);
    }
    if (c <= 0 || x <= 0) {
      int v = 0;
      if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) c = v;
      if (hipDeviceGetAttribute(&v, hipDeviceAttributeNumberOfXccs, dev) == hipSuccess && v > 0) x = v;
      (void)hipGetLastError();   // a failed query is not the caller's error
      if (cached && c > 0 && x > 0) {
        g_topo_cus[dev].store(c, std::memory_order_relaxed);
        g_topo_xcds[dev].store(x, std::memory_order_relaxed);
      }
    }
  } else {
    (void)hipGetLastError();   // no device on this host (planning only): not the caller's error
  }
  if (c > 0) *cus = c;
  if (x > 0) *xcds = x;
  if (tu != nullptr && tu->cu_count > 0) *cus = tu->cu_count;
  if (tu != nullptr && tu->xcd_count > 0) *xcds = tu->xcd_count;
}

cgdr_status check_tuning(const cgdr_fwd_h_tuning* tu) {
  if (tu == nullptr) return CGDR_OK;
  if (tu->v_tile != 0 && tu->v_tile != 16 && tu->v_tile != 32 && tu->v_tile != 64)
    return fail(CGDR_ERR_INVALID, "tuning.v_tile must be 0, 16, 32 or 64, got %d", tu->v_tile);
  if (tu->helpers < -1 || tu->helpers > 1) return fail(CGDR_ERR_INVALID, "tuning.helpers must be -1, 0 or 1");
  if (tu->load_waves != 0 && tu->load_waves != 1 && tu->load_waves != 2 && tu->load_waves != 4)
    return fail(CGDR_ERR_INVALID, "tuning.load_waves must be 0, 1, 2 or 4, got %d", tu->load_waves);
  if (tu->stages != 0 && (tu->stages < 2 || tu->stages > 4))
    return fail(CGDR_ERR_INVALID, "tuning.stages must be 0, 2, 3 or 4, got %d", tu->stages);
  if (tu->prefetch < -1 || tu->prefetch > 64) return fail(CGDR_ERR_INVALID, "tuning.prefetch must be in [-1, 64]");
  if (tu->helper_lead < -1) return fail(CGDR_ERR_INVALID, "tuning.helper_lead must be >= -1");
  if (tu->helper_waves < 0 || tu->helper_waves > 16) return fail(CGDR_ERR_INVALID, "tuning.helper_waves must be in [0, 16]");
  if (tu->cu_count < 0 || tu->xcd_count < 0) return fail(CGDR_ERR_INVALID, "tuning.cu_count/xcd_count must be >= 0");
  if (tu->row_split < 0 || tu->row_split > 4 || tu->row_split == 3)
    return fail(CGDR_ERR_INVALID, "tuning.row_split must be 0, 1, 2 or 4");
  return CGDR_OK;
}

// The key dim the kernels are instantiated for: K rounded up to 32, 64, 128 or 256 (MFMA
// contraction slices of 32 and the LDS swizzles); the tiles' columns and the state's rows
// past K are zero padding.
int kernel_kd(int64_t K) { return K <= 32 ? 32 : K <= 64 ? 64 : K <= 128 ? 128 : 256; }

// Kernel variant and grid.  The kernels need K a multiple of 16 (whole 16-row state tiles; the
// reference accepts any K = V in [32, 256], _infershape.cpp:35-36,214-223), V a multiple of
// 16, 16-byte aligned rows of k/w/u (direct-to-LDS loads, and the fp32 kernel's vector loads,
// move 16 bytes per lane) and 8-byte aligned rows of h/v_new.
cgdr_status make_plan(const cgdr_fwd_h_args* a, Plan* pl) {
  cgdr_status st = validate(a);
  if (st != CGDR_OK) return st;
  const cgdr_fwd_h_tuning* tu = a->tuning;
  st = check_tuning(tu);
  if (st != CGDR_OK) return st;
  const int64_t K = a->K, V = a->V;
  const int es = a->in_dtype == CGDR_BF16 ? 2 : 4;
  if (K < 32 || K % 16 != 0)
    return fail(CGDR_ERR_UNSUPPORTED, "K=%lld is not supported (must be at least 32)", (long long)K);
  const int kd = kernel_kd(K);
  if (V % 16 != 0) return fail(CGDR_ERR_UNSUPPORTED, "V=%lld is not a multiple of 16", (long long)V);
  const int row_align = 16;   // bf16: direct-to-LDS loads; fp32: 16-byte vector loads
  const void* ptrs[] = {a->k, a->w, a->u};
  const int64_t* strides[] = {a->stride_k, a->stride_w, a->stride_u};
  for (int i = 0; i < 3; ++i) {
    if (!aligned(ptrs[i], row_align))
      return fail(CGDR_ERR_UNSUPPORTED, "k/w/u base pointers must be %d-byte aligned", row_align);
    for (int d = 0; d < 3; ++d)
      if ((strides[i][d] * es) % row_align != 0)
        return fail(CGDR_ERR_UNSUPPORTED, "k/w/u strides must be multiples of %d bytes", row_align);
  }
  for (int i = 0; i < 3; ++i)
    if (strides[i][1] * es * 64 >= ((int64_t)1 << 31))
      return fail(CGDR_ERR_UNSUPPORTED, "k/w/u token strides must keep 64 rows within 2 GiB");
  if (!aligned(a->h, 8) || (a->v_new != nullptr && !aligned(a->v_new, 8)))
    return fail(CGDR_ERR_UNSUPPORTED, "h and v_new must be 8-byte aligned");
  for (int d = 0; d < 3; ++d) {
    if ((a->stride_h[d] * es) % 8 != 0 || (a->v_new != nullptr && (a->stride_v[d] * es) % 8 != 0))
      return fail(CGDR_ERR_UNSUPPORTED, "h and v_new strides must be multiples of 8 bytes");
  }

  int cus, xcds;
  topology(tu, &cus, &xcds);
  pl->cus = cus;
  pl->xcds = xcds;
  int ncw;
  const int64_t pairs = a->N * a->H;
  // Helper mode (bf16 only): 32-column V-tiles, and one L2-prefetch workgroup beside every
  // task, when tasks and helpers together fit the device at one workgroup per CU (all
  // resident at once) and the tasks split evenly over the XCDs.
  const int helpers_req = tu != nullptr ? tu->helpers : -1;
  const bool helper_shape = a->in_dtype == CGDR_BF16 && kd <= 128 && V % 32 == 0 &&
                            (pairs * (V / 32)) % xcds == 0 && 2 * pairs * (V / 32) <= cus;
  // Helpers pay only on long sequences: at B=1, H=32, K=V=128 they measured 64.7 vs 54.7 us
  // (16-column tiles, no helpers) at 64 chunks per sequence and 112 vs 143 us at 128.  A packed
  // batch is judged by its mean sequence length.
  const int64_t seq_chunks = a->cu_seqlens != nullptr ? a->NT / (a->N > 0 ? a->N : 1) : a->NT;
  const bool use_helpers = helper_shape && helpers_req != 0 && (helpers_req == 1 || seq_chunks >= kHelperMinChunks);
  const int forced = tu != nullptr ? tu->v_tile : 0;
  if (forced != 0) {
    ncw = forced / 16;
  } else if (use_helpers) {
    ncw = 2;
  } else if (a->in_dtype == CGDR_F32) {
    // fp32: all four waves of a task compute at every tile width (the row split, K up to 128;
    // at K = 256 the waves of one tile's 16-column blocks), so a task's time per chunk grows with
    // its width while wider tiles read W and K fewer times.  Pick the width with the least
    // (rounds of the device) x (time of one round relative to 16 columns), the latter measured
    // with one task per CU: K = 128, 32 chunks: 109 / 177 / 245 us at 16 / 32 / 64 columns;
    // K = 256: 587 / 665 / 716 us.  At B=4, T=4096, H=32, K=V=128 (1,024 / 512 / 256 tasks, 4 / 2
    // / 1 rounds) this picks 64 columns: 581 us against 906 / 786 us at 16 / 32 columns.
    static const double cost_rs[3] = {1.0, 1.62, 2.25}, cost_256[3] = {1.0, 1.13, 1.22};
    const double* cost = kd <= 128 ? cost_rs : cost_256;
    ncw = 1;
    double best = 0.0;
    for (int i = 0, w = 1; w <= 4; ++i, w *= 2) {
      if (V % (16 * w) != 0) break;
      const int64_t tasks = pairs * (V / (16 * w));
      const double t = (double)((tasks + cus - 1) / cus) * cost[i];
      if (w == 1 || t < best) best = t, ncw = w;
    }
  } else {
    // Enough workgroups to cover the CUs first, then wider V-tiles (fewer K/W re-reads).
    ncw = 1;
    if (pairs * (V / 32) >= 2 * cus && V % 32 == 0) ncw = 2;
    // The bf16 kernel runs one task workgroup per CU, and every task walks its whole sequence:
    // when 16-column tiles would need more than one round of the device, 32-column tiles need
    // half the rounds.  Measured at B=4, T=8192, H=8, K=128, V=256 (512 vs 256 tasks): 297 us
    // with 16 columns, 198 us with 32.
    if (a->in_dtype == CGDR_BF16 && V % 32 == 0 && pairs * (V / 16) > cus) ncw = 2;
  }
  if (V % (16 * ncw) != 0) ncw = 1;
  pl->rs = 1;
  if (a->in_dtype == CGDR_F32) {
    pl->kernel = 1;
    pl->ncw = ncw;
    pl->nlw = 0;
    pl->stages = 1;
    pl->threads = cgdr::F32Layout<32, 1>::THREADS;   // four waves at every key dim
    // Row split: all four waves compute (wave (j, r) holds state rows KD/RSF r .. of column block
    // j), where the staging buffers fit (K up to 128) and each wave keeps whole 16-row tiles.
    int rs = tu != nullptr ? tu->row_split : 0;
    const int kt = kd / 16;
    const int full = 4 / ncw;                      // 4, 2 or 1 row groups per column block
    int best = (kd <= 128) ? (kt % full == 0 ? full : (kt % 2 == 0 && full >= 2 ? 2 : 1)) : 1;
    if (rs == 0 || rs > best || (rs != 1 && rs != 2 && rs != 4)) rs = best;
    if (rs > 1 && kt % rs != 0) rs = 1;
    pl->rs = rs;
  } else {
    // bf16: the pipelined kernel, with the contest rounding model when asked for
    pl->kernel = a->numerics == CGDR_NUMERICS_CONTEST ? 2 : 0;
    if (kd == 256) ncw = 1;   // K=256 state and tiles leave LDS room for one compute wave only
    pl->ncw = ncw;
    int nlw = tu != nullptr ? tu->load_waves : 0;
    // With helper workgroups the task's loads are L2 hits and one load wave keeps up; at most
    // 8 waves per workgroup (two per SIMD), so that no wave is squeezed below 256 VGPRs.
    // K = 256: one load wave (two push the kernel past 256 VGPRs into scratch spills).
    // 32-column tiles without helpers: one load wave (with the L2 touches 2 chunks ahead,
    // below) measured 925 us against 1,020 us with two, for 16 packed sequences of lengths
    // U[64, 8192] at H=32, K=V=128.
    if (nlw == 0) nlw = (use_helpers || kd == 256 || ncw == 2) ? 1 : 2;
    if (pl->kernel == 2 && nlw == 4) nlw = 2;   // contest instantiations: 1 or 2 load waves
    if (kd == 256) nlw = 1;
    // Row split (two compute waves per 16 columns, each with half of the state rows): for the
    // contest numerics, whose per-element casts make the compute waves the bound.  It needs
    // an even number of 32-row state blocks (K of 64 or 128 here) and at most 8 waves.
    // Default numerics: 16-column tiles without helpers (one short chain per CU) split too.
    // Measured by events, row split 1 vs 2: B=2, T=2048, H=16, K=V=128, h0: 40.2 vs 37.3 us;
    // B=2, T=4096: 62.4 vs 58.2; B=1, T=4096, H=32: 60.4 vs 58.3; B=4, T=1024, H=16: 32.6 vs
    // 30.6.  With helpers it is slower (B=1, T=8192, H=32: 115.3 vs 125.2 us), and at 32 columns
    // without helpers no faster (16 packed sequences of U[64, 8192], H=32: 891-895 vs 897 us).
    int rs = tu != nullptr ? tu->row_split : 0;
    if (rs == 0) rs = (pl->kernel == 2 || (!use_helpers && ncw == 1)) ? 2 : 1;
    if (rs == 4) rs = 2;   // the bf16 kernels split the rows two ways at most
    if (rs == 2 && !(kd == 64 || kd == 128) ) rs = 1;
    if (rs == 2 && ncw > 2) rs = 1;
    while (nlw > 1 && (rs + 1) * ncw + nlw + 1 > 8) nlw /= 2;
    if (rs == 2 && bf16_max_stages(K, ncw, nlw, 2) == 0) rs = 1;
    pl->rs = rs;
    pl->nlw = nlw;
    int stages = tu != nullptr ? tu->stages : 0;
    // deepest ring that fits the LDS and the vmcnt range
    const int max_stages = bf16_max_stages(K, ncw, nlw, rs);
    if (stages < 2 || stages > max_stages) stages = max_stages;
    pl->stages = stages;
    pl->threads = 64 * (rs * ncw + nlw + ncw + 1);   // compute, load, store (one per 16 columns), gate
  }
  pl->tasks = a->N * a->H * (V / (16 * ncw));
  if (pl->tasks > kMaxTasks) return fail(CGDR_ERR_UNSUPPORTED, "too many tasks (%lld)", (long long)pl->tasks);
  // Helper workgroups (one per task, on the task's XCD) when the doubled grid still fits the
  // device at one workgroup per CU, so that tasks and helpers are all resident together.
  pl->helpers = 0;
  // (a progress value holds up to 2^24 - 1 chunks)
  if (pl->kernel != 1 && pl->tasks % xcds == 0 && 2 * pl->tasks <= cus && helpers_req != 0 &&
      (use_helpers || helpers_req == 1) && a->NT < (1 << 24))
    pl->helpers = 1;
  return CGDR_OK;
}

cgdr::FwdHParams to_params(const cgdr_fwd_h_args* a, const Plan& pl) {
  cgdr::FwdHParams p;
  memset(&p, 0, sizeof(p));
  p.k = a->k; p.w = a->w; p.u = a->u; p.g = a->g; p.h0 = a->initial_state;
  p.cu_seqlens = a->cu_seqlens; p.chunk_offsets = a->chunk_offsets;
  p.h = a->h; p.v_new = a->v_new; p.final_state = a->final_state;
  p.T = a->T; p.H = a->H; p.Hg = a->Hg; p.V = a->V; p.N = a->N; p.NT = a->NT;
  p.sk_b = a->stride_k[0]; p.sk_t = a->stride_k[1]; p.sk_h = a->stride_k[2];
  p.sw_b = a->stride_w[0]; p.sw_t = a->stride_w[1]; p.sw_h = a->stride_w[2];
  p.su_b = a->stride_u[0]; p.su_t = a->stride_u[1]; p.su_h = a->stride_u[2];
  p.sg_b = a->stride_g[0]; p.sg_t = a->stride_g[1]; p.sg_h = a->stride_g[2];
  p.sh_b = a->stride_h[0]; p.sh_c = a->stride_h[1]; p.sh_h = a->stride_h[2];
  p.sv_b = a->stride_v[0]; p.sv_t = a->stride_v[1]; p.sv_h = a->stride_v[2];
  p.sh0_n = a->stride_h0[0]; p.sh0_h = a->stride_h0[1];
  p.sf_n = a->stride_final[0]; p.sf_h = a->stride_final[1];
  p.n_vtiles = (int)(a->V / (16 * pl.ncw));
  p.n_tasks = (int)pl.tasks;
  p.head_ratio = (int)(a->H / a->Hg);
  p.h0_f32 = a->h0_dtype == CGDR_F32;
  p.final_f32 = a->final_dtype == CGDR_F32;
  p.has_g = a->g != nullptr;
  const cgdr_fwd_h_tuning* tu = a->tuning;
  // L2 touch distance of store wave 0 without helpers: 2 chunks for 32-column tiles (one load
  // wave; measured 925 us at 2, 937 at 3, 975 at 4 for the packed batch above), 4 for 16
  p.prefetch = (tu != nullptr && tu->prefetch >= 0) ? tu->prefetch : (pl.ncw == 2 ? 2 : 4);
  p.helpers = pl.helpers;
  p.helper_lead = (tu != nullptr && tu->helper_lead >= 0) ? tu->helper_lead : 4;
  {
    const int hw = (tu != nullptr && tu->helper_waves > 0) ? tu->helper_waves : 4;
    const int max_hw = pl.threads / 64;
    p.helper_waves = hw > max_hw ? max_hw : hw;
  }
  p.n_xcd = pl.xcds;
  p.K = (int32_t)a->K;
  p.state_vk = a->state_layout == CGDR_STATE_VK;
  p.progress = nullptr;
  {
    // 16-byte stores of 4 fp32 value columns need 16-byte aligned rows of h and v_new
    auto mult4 = [](const int64_t* st) { return st[0] % 4 == 0 && st[1] % 4 == 0 && st[2] % 4 == 0; };
    p.vec_out = a->in_dtype == CGDR_F32 && a->V % 4 == 0 && aligned(a->h, 16) && mult4(a->stride_h) &&
                (a->v_new == nullptr || (aligned(a->v_new, 16) && mult4(a->stride_v)));
  }
  return p;
}

// Compile-time layout facts of the bf16 kernel instantiation a plan selects.
template <int KD, typename F>
auto with_bf16_config(const Plan& pl, F f) {
  auto by_rs = [&](auto rs) {
    constexpr int RS = decltype(rs)::value;
    auto by_nlw = [&](auto ncw) {
      constexpr int NCW = decltype(ncw)::value;
      auto by_stages = [&](auto nlw) {
        constexpr int NLW = decltype(nlw)::value;
        if (pl.stages == 4) return f(cgdr::Bf16Layout<KD, NCW, NLW, 4, RS>{});
        if (pl.stages == 3) return f(cgdr::Bf16Layout<KD, NCW, NLW, 3, RS>{});
        return f(cgdr::Bf16Layout<KD, NCW, NLW, 2, RS>{});
      };
      if (pl.nlw == 1) return by_stages(std::integral_constant<int, 1>{});
      if (pl.nlw == 4) return by_stages(std::integral_constant<int, 4>{});
      return by_stages(std::integral_constant<int, 2>{});
    };
    if (pl.ncw == 4) return by_nlw(std::integral_constant<int, 4>{});
    if (pl.ncw == 2) return by_nlw(std::integral_constant<int, 2>{});
    return by_nlw(std::integral_constant<int, 1>{});
  };
  if (pl.rs == 2) return by_rs(std::integral_constant<int, 2>{});
  return by_rs(std::integral_constant<int, 1>{});
}

int bf16_max_stages(int64_t K, int ncw, int nlw, int rs) {
  auto pick = [&](auto kd) -> int {
    constexpr int KD = decltype(kd)::value;
    auto by_ncw = [&](auto c) -> int {
      constexpr int NCW = decltype(c)::value;
      if (rs == 2) {
        if (nlw == 1) return cgdr::bf16_max_stages<KD, NCW, 1, 2>();
        if (nlw == 4) return cgdr::bf16_max_stages<KD, NCW, 4, 2>();
        return cgdr::bf16_max_stages<KD, NCW, 2, 2>();
      }
      if (nlw == 1) return cgdr::bf16_max_stages<KD, NCW, 1>();
      if (nlw == 4) return cgdr::bf16_max_stages<KD, NCW, 4>();
      return cgdr::bf16_max_stages<KD, NCW, 2>();
    };
    if (ncw == 4) return by_ncw(std::integral_constant<int, 4>{});
    if (ncw == 2) return by_ncw(std::integral_constant<int, 2>{});
    return by_ncw(std::integral_constant<int, 1>{});
  };
  switch (kernel_kd(K)) {
    case 32: return pick(std::integral_constant<int, 32>{});
    case 64: return pick(std::integral_constant<int, 64>{});
    case 128: return pick(std::integral_constant<int, 128>{});
    default: return pick(std::integral_constant<int, 256>{});
  }
}

int lds_bytes_of(const Plan& pl, int64_t K) {
  if (pl.kernel == 1) {
    auto f32 = [&](auto kd) -> int {
      constexpr int KD = decltype(kd)::value;
      auto by_rs = [&](auto c) -> int {
        constexpr int NCW = decltype(c)::value;
        if (pl.rs == 4) return cgdr::F32Layout<KD, NCW, 4>::LDS_BYTES;
        if (pl.rs == 2) return cgdr::F32Layout<KD, NCW, 2>::LDS_BYTES;
        return cgdr::F32Layout<KD, NCW, 1>::LDS_BYTES;
      };
      return pl.ncw == 1 ? by_rs(std::integral_constant<int, 1>{})
                         : pl.ncw == 2 ? by_rs(std::integral_constant<int, 2>{}) : by_rs(std::integral_constant<int, 4>{});
    };
    switch (kernel_kd(K)) {
      case 32: return f32(std::integral_constant<int, 32>{});
      case 64: return f32(std::integral_constant<int, 64>{});
      case 128: return f32(std::integral_constant<int, 128>{});
      default: return f32(std::integral_constant<int, 256>{});
    }
  }
  // bf16: the layout of the instantiated kernel
  auto lds = [](auto layout) -> int { return decltype(layout)::LDS_BYTES; };
  switch (kernel_kd(K)) {
    case 32: return with_bf16_config<32>(pl, lds);
    case 64: return with_bf16_config<64>(pl, lds);
    case 128: return with_bf16_config<128>(pl, lds);
    default: return with_bf16_config<256>(pl, lds);
  }
}

// Workspace: the head-major copy of g, needed when g's token stride is not 1 (the kernels
// read one chunk's g row of one head as one contiguous 256-byte row), then, with helper
// workgroups, one int32 progress counter per task, then, for contest numerics, one int32 flag
// per (sequence, head).
size_t g_relayout_bytes(const cgdr_fwd_h_args* a) {
  if (a->g == nullptr || a->stride_g[1] == 1) return 0;
  return ((size_t)a->B * (size_t)a->H * (size_t)a->T * sizeof(float) + 255) & ~(size_t)255;
}

size_t progress_ints(const Plan& pl) { return pl.helpers ? (size_t)pl.tasks * cgdr::kProgressStride : 0; }
size_t redo_ints(const cgdr_fwd_h_args* a, const Plan& pl) { return pl.kernel == 2 ? (size_t)(a->N * a->H) : 0; }

size_t workspace_bytes_of(const cgdr_fwd_h_args* a, const Plan& pl) {
  return g_relayout_bytes(a) + (progress_ints(pl) + redo_ints(a, pl)) * sizeof(int32_t);
}

hipError_t launch_g_relayout(const cgdr_fwd_h_args* a, float* gt, hipStream_t s) {
  const dim3 grid((unsigned)((a->T + 63) / 64), (unsigned)((a->H + 63) / 64), (unsigned)a->B);
  hipLaunchKernelGGL(cgdr::cgdr_g_head_major_kernel, grid, dim3(256), 0, s, a->g, gt, a->T, a->H,
                     a->stride_g[0], a->stride_g[1], a->stride_g[2]);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// K or V not a multiple of 16 (the reference accepts any K = V in [32, 256]): the call runs on
// dense copies padded to multiples of 16 in the workspace.  k, w, u and the initial state are
// copied in with zeros in the padding, the kernels run on the padded shapes (exact: zero key
// columns and value columns contribute nothing, and the padding rows of the state stay zero),
// and h, v_new and the final state are copied out.  Rows of k/w/u whose length is not a
// multiple of 8 elements are not 16-byte aligned, which the direct-to-LDS loads need.

bool needs_repack(const cgdr_fwd_h_args* a) { return a != nullptr && (a->K % 16 != 0 || a->V % 16 != 0); }

struct Repack {
  cgdr_fwd_h_args pa;   // the padded call; its buffer pointers are offsets from the workspace
  size_t off_k, off_w, off_u, off_h0, off_h, off_v, off_f, bytes;
};

int64_t round16(int64_t x) { return (x + 15) / 16 * 16; }
size_t round256(size_t x) { return (x + 255) & ~(size_t)255; }
int elem_bytes(int32_t dtype) { return dtype == CGDR_BF16 ? 2 : 4; }

// The padded call, with buffers at workspace offsets from `base` (16-byte aligned).
Repack make_repack(const cgdr_fwd_h_args* a, char* base) {
  Repack r;
  r.pa = *a;
  cgdr_fwd_h_args& p = r.pa;
  const int64_t B = a->B, T = a->T, H = a->H, Hg = a->Hg, N = a->N, NT = a->NT;
  const int64_t Kp = round16(a->K), Vp = round16(a->V);
  const size_t es = elem_bytes(a->in_dtype);
  size_t off = 0;
  auto take = [&](size_t bytes) { const size_t o = off; off += round256(bytes); return o; };
  r.off_k = take((size_t)(B * T * Hg * Kp) * es);
  r.off_w = take((size_t)(B * T * H * Kp) * es);
  r.off_u = take((size_t)(B * T * H * Vp) * es);
  r.off_h0 = a->initial_state ? take((size_t)(N * H * Kp * Vp) * elem_bytes(a->h0_dtype)) : 0;
  r.off_h = take((size_t)(B * NT * H * Kp * Vp) * es);
  r.off_v = a->v_new ? take((size_t)(B * T * H * Vp) * es) : 0;
  r.off_f = a->final_state ? take((size_t)(N * H * Kp * Vp) * elem_bytes(a->final_dtype)) : 0;
  r.bytes = off;
  p.K = Kp;
  p.V = Vp;
  p.k = base + r.off_k;
  p.w = base + r.off_w;
  p.u = base + r.off_u;
  p.initial_state = a->initial_state ? base + r.off_h0 : nullptr;
  p.h = base + r.off_h;
  p.v_new = a->v_new ? base + r.off_v : nullptr;
  p.final_state = a->final_state ? base + r.off_f : nullptr;
  const int64_t sk[3] = {T * Hg * Kp, Hg * Kp, Kp}, sw[3] = {T * H * Kp, H * Kp, Kp};
  const int64_t su[3] = {T * H * Vp, H * Vp, Vp}, sh[3] = {NT * H * Kp * Vp, H * Kp * Vp, Kp * Vp};
  const int64_t s0[2] = {H * Kp * Vp, Kp * Vp};
  memcpy(p.stride_k, sk, sizeof sk);
  memcpy(p.stride_w, sw, sizeof sw);
  memcpy(p.stride_u, su, sizeof su);
  memcpy(p.stride_v, su, sizeof su);
  memcpy(p.stride_h, sh, sizeof sh);
  memcpy(p.stride_h0, s0, sizeof s0);
  memcpy(p.stride_final, s0, sizeof s0);
  return r;
}

// Copies between a strided tensor of rows (row (i0, i1, i2, r) at i0*s0 + i1*s1 + i2*s2 + r*s3,
// C contiguous elements) and a dense one of n0 x n1 x n2 x Rp rows of Cp elements.  Into the
// dense side, rows r >= R and columns c >= C are zero; out of it, only r < R, c < C are written.
struct RowSet {
  int64_t n0, n1, n2, R, Rp, C, Cp;
  int64_t s0, s1, s2, s3;
};

template <typename E>
__global__ void __launch_bounds__(256) cgdr_repack_kernel(const E* __restrict__ src, E* __restrict__ dst,
                                                          RowSet rs, int to_dense) {
  const int64_t total = rs.n0 * rs.n1 * rs.n2 * rs.Rp * rs.Cp;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (int64_t)gridDim.x * 256) {
    int64_t q = i;
    const int64_t c = q % rs.Cp;
    q /= rs.Cp;
    const int64_t r = q % rs.Rp;
    q /= rs.Rp;
    const int64_t i2 = q % rs.n2;
    q /= rs.n2;
    const int64_t i1 = q % rs.n1;
    const int64_t i0 = q / rs.n1;
    const bool real = r < rs.R && c < rs.C;
    const int64_t strided = i0 * rs.s0 + i1 * rs.s1 + i2 * rs.s2 + r * rs.s3 + c;
    if (to_dense) dst[i] = real ? src[strided] : E(0);
    else if (real) dst[strided] = src[i];
  }
}

hipError_t repack(const void* src, void* dst, int esize, const RowSet& rs, bool to_dense, hipStream_t s) {
  const int64_t total = rs.n0 * rs.n1 * rs.n2 * rs.Rp * rs.Cp;
  if (total == 0) return hipSuccess;
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 1 << 16);
  if (esize == 2)
    hipLaunchKernelGGL(cgdr_repack_kernel<uint16_t>, dim3(grid), dim3(256), 0, s, (const uint16_t*)src,
                       (uint16_t*)dst, rs, (int)to_dense);
  else
    hipLaunchKernelGGL(cgdr_repack_kernel<uint32_t>, dim3(grid), dim3(256), 0, s, (const uint32_t*)src,
                       (uint32_t*)dst, rs, (int)to_dense);
  return hipGetLastError();
}

// A fake, aligned workspace base for sizing the padded call on the host.
char* const kSizingBase = (char*)(uintptr_t)(1u << 20);

// The padded call of a repacked one, validated, with its plan.
cgdr_status plan_repack(const cgdr_fwd_h_args* a, char* base, Repack* r, Plan* pl) {
  cgdr_status st = validate(a);
  if (st != CGDR_OK) return st;
  if (a->K < 32) return fail(CGDR_ERR_UNSUPPORTED, "K=%lld is not supported (must be at least 32)", (long long)a->K);
  *r = make_repack(a, base);
  return make_plan(&r->pa, pl);
}

// Workspace bytes of any call (the padded copies first when repacked).
cgdr_status workspace_need(const cgdr_fwd_h_args* a, size_t* need) {
  Plan pl;
  if (needs_repack(a)) {
    Repack r;
    cgdr_status st = plan_repack(a, kSizingBase, &r, &pl);
    if (st != CGDR_OK) return st;
    *need = r.bytes + workspace_bytes_of(&r.pa, pl);
    return CGDR_OK;
  }
  cgdr_status st = make_plan(a, &pl);
  if (st != CGDR_OK) return st;
  *need = workspace_bytes_of(a, pl);
  return CGDR_OK;
}

// Scratch of cgdr_fwd_h_launch_no_alloc: a file-scope device array that every GPU the library
// runs on holds (its own copy, at its own address) until the process ends.  Host code never
// passes the array's name to a kernel or a copy: its device address is looked up once per
// device with hipGetSymbolAddress (scratch_address below) and that pointer is used instead.
constexpr size_t kNoAllocScratchBytes = CGDR_NO_ALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on `device`, looked up on the first call for that device with
// that device current (the caller's current device is restored afterwards).
cgdr_status scratch_address(int device, void** out) {
  if (device < 0 || device >= kMaxDevices)
    return fail(CGDR_ERR_UNSUPPORTED, "device %d is beyond the %d devices the static scratch serves", device,
                kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[device] == nullptr) {
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (cur != device && (e = hipSetDevice(device)) != hipSuccess)
      return fail(CGDR_ERR_LAUNCH, "hipSetDevice(%d) failed: %s", device, hipGetErrorString(e));
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (cur != device) (void)hipSetDevice(cur);
    if (e != hipSuccess || ptr == nullptr)
      return fail(CGDR_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", device,
                  hipGetErrorString(e));
    g_scratch_ptr[device] = ptr;
  }
  *out = g_scratch_ptr[device];
  return CGDR_OK;
}

}  // namespace

extern "C" {

int cgdr_abi_version(void) { return CGDR_ABI_VERSION; }

const char* cgdr_last_error(void) { return cgdr_host::last_error; }

const char* cgdr_status_string(cgdr_status status) {
  switch (status) {
    case CGDR_OK: return "CGDR_OK";
    case CGDR_ERR_NULLPTR: return "CGDR_ERR_NULLPTR";
    case CGDR_ERR_INVALID: return "CGDR_ERR_INVALID";
    case CGDR_ERR_UNSUPPORTED: return "CGDR_ERR_UNSUPPORTED";
    case CGDR_ERR_LAUNCH: return "CGDR_ERR_LAUNCH";
  }
  return "CGDR_ERR_UNKNOWN";
}

cgdr_status cgdr_fwd_h_workspace_size(const cgdr_fwd_h_args* args, size_t* workspace_bytes) {
  if (workspace_bytes == nullptr) return fail(CGDR_ERR_NULLPTR, "workspace_bytes is NULL");
  return workspace_need(args, workspace_bytes);
}

cgdr_status cgdr_fwd_h_get_plan(const cgdr_fwd_h_args* args, cgdr_fwd_h_plan* plan) {
  if (plan == nullptr) return fail(CGDR_ERR_NULLPTR, "plan is NULL");
  Plan pl;
  Repack r;
  const bool rp = needs_repack(args);
  cgdr_status st = rp ? plan_repack(args, kSizingBase, &r, &pl) : make_plan(args, &pl);
  if (st != CGDR_OK) return st;
  if (rp) args = &r.pa;   // the plan of the padded call
  plan->kernel = pl.kernel;
  plan->v_tile = 16 * pl.ncw;
  plan->compute_waves = pl.ncw * pl.rs;
  plan->total_waves = pl.threads / 64;
  plan->stages = pl.stages;
  plan->lds_bytes = lds_bytes_of(pl, args->K);
  plan->workgroups = pl.helpers ? 2 * pl.tasks : pl.tasks;
  plan->helpers = pl.helpers;
  plan->load_waves = pl.nlw;
  plan->cu_count = pl.cus;
  plan->xcd_count = pl.xcds;
  plan->row_split = pl.rs;
  return CGDR_OK;
}

cgdr_status cgdr_fwd_h_launch(const cgdr_fwd_h_args* args, void* workspace, size_t workspace_bytes, void* stream) {
  if (needs_repack(args)) {
    size_t need = 0;
    cgdr_status st = workspace_need(args, &need);
    if (st != CGDR_OK) return st;
    if (workspace == nullptr || workspace_bytes < need)
      return fail(CGDR_ERR_INVALID, "workspace of %zu bytes required (got %zu)", need,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    if (!aligned(workspace, 16)) return fail(CGDR_ERR_INVALID, "workspace must be 16-byte aligned");
    Repack r;
    Plan pl;
    st = plan_repack(args, (char*)workspace, &r, &pl);
    if (st != CGDR_OK) return st;
    const cgdr_fwd_h_args* a = args;
    const cgdr_fwd_h_args& p = r.pa;
    const int es = elem_bytes(a->in_dtype);
    hipStream_t s = (hipStream_t)stream;
    // state blocks: rows x columns of K x V (rows of V) or V x K (rows of K)
    const bool vk = a->state_layout == CGDR_STATE_VK;
    const int64_t sr = vk ? a->V : a->K, srp = vk ? p.V : p.K, sc = vk ? a->K : a->V, scp = vk ? p.K : p.V;
    const RowSet k_rows{a->B, a->T, a->Hg, 1, 1, a->K, p.K, a->stride_k[0], a->stride_k[1], a->stride_k[2], 0};
    const RowSet w_rows{a->B, a->T, a->H, 1, 1, a->K, p.K, a->stride_w[0], a->stride_w[1], a->stride_w[2], 0};
    const RowSet u_rows{a->B, a->T, a->H, 1, 1, a->V, p.V, a->stride_u[0], a->stride_u[1], a->stride_u[2], 0};
    const RowSet v_rows{a->B, a->T, a->H, 1, 1, a->V, p.V, a->stride_v[0], a->stride_v[1], a->stride_v[2], 0};
    const RowSet h_rows{a->B, a->NT, a->H, a->K, p.K, a->V, p.V, a->stride_h[0], a->stride_h[1], a->stride_h[2], a->V};
    const RowSet h0_rows{a->N, a->H, 1, sr, srp, sc, scp, a->stride_h0[0], a->stride_h0[1], 0, sc};
    const RowSet f_rows{a->N, a->H, 1, sr, srp, sc, scp, a->stride_final[0], a->stride_final[1], 0, sc};
    hipError_t e = repack(a->k, (void*)p.k, es, k_rows, true, s);
    if (e == hipSuccess) e = repack(a->w, (void*)p.w, es, w_rows, true, s);
    if (e == hipSuccess) e = repack(a->u, (void*)p.u, es, u_rows, true, s);
    if (e == hipSuccess && a->initial_state)
      e = repack(a->initial_state, (void*)p.initial_state, elem_bytes(a->h0_dtype), h0_rows, true, s);
    if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "repack launch failed: %s", hipGetErrorString(e));
    st = cgdr_fwd_h_launch(&p, (char*)workspace + r.bytes, workspace_bytes - r.bytes, stream);
    if (st != CGDR_OK) return st;
    e = repack(p.h, a->h, es, h_rows, false, s);
    if (e == hipSuccess && a->v_new) e = repack(p.v_new, a->v_new, es, v_rows, false, s);
    if (e == hipSuccess && a->final_state)
      e = repack(p.final_state, a->final_state, elem_bytes(a->final_dtype), f_rows, false, s);
    if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "repack launch failed: %s", hipGetErrorString(e));
    return CGDR_OK;
  }
  Plan pl;
  cgdr_status st = make_plan(args, &pl);
  if (st != CGDR_OK) return st;
  cgdr::FwdHParams p = to_params(args, pl);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  const size_t need = workspace_bytes_of(args, pl);
  if (need > 0) {
    if (workspace == nullptr || workspace_bytes < need)
      return fail(CGDR_ERR_INVALID, "workspace of %zu bytes required (got %zu)", need,
                  workspace == nullptr ? (size_t)0 : workspace_bytes);
    if (!aligned(workspace, 16)) return fail(CGDR_ERR_INVALID, "workspace must be 16-byte aligned");
  }
  const size_t g_bytes = g_relayout_bytes(args);
  if (g_bytes > 0) {
    e = launch_g_relayout(args, (float*)workspace, s);
    if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "g relayout launch failed: %s", hipGetErrorString(e));
    p.g = (const float*)workspace;
    p.sg_b = args->H * args->T;
    p.sg_t = 1;
    p.sg_h = args->T;
  }
  // The helpers' progress counters and the contest flags hold this launch's epoch instead of
  // being cleared before it (no reset launch): a value left by another launch reads as no
  // progress, or as an unflagged head.
  int32_t* counters = (int32_t*)((char*)workspace + g_bytes);
  if (pl.helpers || pl.kernel == 2) {
    static std::atomic<uint32_t> launches{0};
    p.epoch = 1 + (int32_t)(launches.fetch_add(1, std::memory_order_relaxed) % 255u);
  }
  if (pl.helpers) p.progress = counters;
  if (pl.kernel == 2) p.redo = counters + progress_ints(pl);
  switch (kernel_kd(args->K)) {
    case 32: e = cgdr_fwd::launch_kd<32>(p, pl, s); break;
    case 64: e = cgdr_fwd::launch_kd<64>(p, pl, s); break;
    case 128: e = cgdr_fwd::launch_kd<128>(p, pl, s); break;
    default: e = cgdr_fwd::launch_kd<256>(p, pl, s); break;
  }
  if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "kernel launch failed: %s", hipGetErrorString(e));
  return CGDR_OK;
}

cgdr_status cgdr_prepare_chunk_offsets(const int64_t* cu_seqlens, int64_t n_seq, int64_t chunk_size,
                                       int64_t* chunk_offsets_out) {
  if (cu_seqlens == nullptr || chunk_offsets_out == nullptr)
    return fail(CGDR_ERR_NULLPTR, "cu_seqlens and chunk_offsets_out are required");
  if (n_seq < 0 || chunk_size < 1) return fail(CGDR_ERR_INVALID, "n_seq must be >= 0 and chunk_size >= 1");
  if (n_seq >= 0 && cu_seqlens[0] != 0) return fail(CGDR_ERR_INVALID, "cu_seqlens must start at zero");
  chunk_offsets_out[0] = 0;
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t len = cu_seqlens[i + 1] - cu_seqlens[i];
    if (len < 0) return fail(CGDR_ERR_INVALID, "cu_seqlens must be non-decreasing (entry %lld)", (long long)(i + 1));
    chunk_offsets_out[i + 1] = chunk_offsets_out[i] + (len + chunk_size - 1) / chunk_size;
  }
  return CGDR_OK;
}

cgdr_status cgdr_prepare_chunk_indices(const int64_t* cu_seqlens, int64_t n_seq, int64_t chunk_size,
                                       int64_t* chunk_indices_out, int64_t capacity_rows, int64_t* nt_out) {
  if (cu_seqlens == nullptr || nt_out == nullptr) return fail(CGDR_ERR_NULLPTR, "cu_seqlens and nt_out are required");
  if (n_seq < 0 || chunk_size < 1) return fail(CGDR_ERR_INVALID, "n_seq must be >= 0 and chunk_size >= 1");
  if (cu_seqlens[0] != 0) return fail(CGDR_ERR_INVALID, "cu_seqlens must start at zero");
  int64_t rows = 0;
  for (int64_t i = 0; i < n_seq; ++i) {
    const int64_t len = cu_seqlens[i + 1] - cu_seqlens[i];
    if (len < 0) return fail(CGDR_ERR_INVALID, "cu_seqlens must be non-decreasing (entry %lld)", (long long)(i + 1));
    const int64_t nc = (len + chunk_size - 1) / chunk_size;
    for (int64_t c = 0; c < nc; ++c, ++rows) {
      if (chunk_indices_out != nullptr) {
        if (rows >= capacity_rows) return fail(CGDR_ERR_INVALID, "chunk_indices_out holds fewer than NT rows");
        chunk_indices_out[2 * rows] = i;
        chunk_indices_out[2 * rows + 1] = c;
      }
    }
  }
  *nt_out = rows;
  return CGDR_OK;
}

cgdr_status cgdr_fwd_h_launch_no_alloc(const cgdr_fwd_h_args* args, void* stream) {
  size_t need = 0;
  cgdr_status st = workspace_need(args, &need);
  if (st != CGDR_OK) return st;
  if (need > kNoAllocScratchBytes)
    return fail(CGDR_ERR_UNSUPPORTED,
                "this call needs %zu bytes of scratch; cgdr_fwd_h_launch_no_alloc holds %zu (pass g with token "
                "stride 1, or call cgdr_fwd_h_launch with a workspace)",
                need, kNoAllocScratchBytes);
  if (need == 0) return cgdr_fwd_h_launch(args, nullptr, 0, stream);
  int device = -1;
  hipError_t e = stream != nullptr ? hipStreamGetDevice((hipStream_t)stream, &device) : hipGetDevice(&device);
  if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "cannot find the stream's device: %s", hipGetErrorString(e));
  void* ws = nullptr;
  st = scratch_address(device, &ws);
  if (st != CGDR_OK) return st;
  return cgdr_fwd_h_launch(args, ws, kNoAllocScratchBytes, stream);
}

}  // extern "C"
