// cgdr_chunk_o.hip -- C ABI of the gfx950 chunk-output operator (include/cgdr_chunk_o.h).
//
// Host side: argument validation, the choice of the V-tile, and the launch of one workgroup
// per (batch row, chunk, value head, V-tile).  The reference computes this output inside its
// full operator (stage 2 attn_inter + stage 3 masked product,
// ref/chunk_gated_delta_rule/op_kernel/arch22/chunk_gated_delta_rule_stage3.h:102-129 splits
// Nv x chunks over cores the same way).
#include "../../include/cgdr_chunk_o.h"

#include <hip/hip_runtime.h>

#include <cstring>

#include "cgdr_chunk_o_kernel.h"
#include "cgdr_host.h"

namespace {

using cgdr_host::fail;

constexpr int64_t kMaxValueDim = 1024;
constexpr int64_t kMaxUnits = (int64_t(1) << 31) - 1;

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// V-tile: 128 value columns when V allows it (and K <= 128, which keeps the LDS of one
// workgroup at 48 KiB so three fit a CU), else 64, else 32.
int pick_vtile(const cgdr_chunk_o_args* a) {
  if (a->V % 128 == 0 && a->K <= 128) return 128;
  if (a->V % 64 == 0) return 64;
  if (a->V % 32 == 0) return 32;
  return 0;
}

cgdr_status validate(const cgdr_chunk_o_args* a, int* vt_out) {
  if (a == nullptr) return fail(CGDR_ERR_NULLPTR, "args is NULL");
  if (a->q == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input q is missing");
  if (a->k == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input k is missing");
  if (a->v_new == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input v_new is missing");
  if (a->h == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input h is missing");
  if (a->o == nullptr) return fail(CGDR_ERR_NULLPTR, "Required output o is missing");
  if (a->chunk_size != CGDR_CHUNK_SIZE)
    return fail(CGDR_ERR_UNSUPPORTED, "chunk_size must be %d, but got %lld", CGDR_CHUNK_SIZE, (long long)a->chunk_size);
  if (a->in_dtype != CGDR_BF16 && a->in_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "in_dtype %d is not a cgdr_dtype", a->in_dtype);
  if (a->in_dtype != CGDR_BF16) return fail(CGDR_ERR_UNSUPPORTED, "chunk output is built for bf16 inputs only");
  if (a->B < 1) return fail(CGDR_ERR_INVALID, "B must be >= 1, but got %lld", (long long)a->B);
  if (a->T < 1) return fail(CGDR_ERR_INVALID, "T must be >= 1, but got %lld", (long long)a->T);
  if (a->H < 1 || a->Hg < 1 || a->H % a->Hg != 0)
    return fail(CGDR_ERR_INVALID, "H must be a positive multiple of Hg: H=%lld, Hg=%lld", (long long)a->H,
                (long long)a->Hg);
  if (a->K != 32 && a->K != 64 && a->K != 128 && a->K != 256)
    return fail(CGDR_ERR_UNSUPPORTED, "K must be 32, 64, 128 or 256, but got %lld", (long long)a->K);
  if (a->V < 1 || a->V > kMaxValueDim)
    return fail(CGDR_ERR_INVALID, "V must be in [1, %lld], but got %lld", (long long)kMaxValueDim, (long long)a->V);
  const int vt = pick_vtile(a);
  if (vt == 0) return fail(CGDR_ERR_UNSUPPORTED, "V must be a multiple of 32, but got %lld", (long long)a->V);
  if (!(a->scale == a->scale)) return fail(CGDR_ERR_INVALID, "scale is NaN");

  const int64_t nt_fixed = (a->T + CGDR_CHUNK_SIZE - 1) / CGDR_CHUNK_SIZE;
  if (a->cu_seqlens == nullptr) {
    if (a->chunk_indices != nullptr) return fail(CGDR_ERR_INVALID, "chunk_indices given without cu_seqlens");
    if (a->N != a->B)
      return fail(CGDR_ERR_INVALID, "N must equal B without cu_seqlens: N=%lld, B=%lld", (long long)a->N, (long long)a->B);
    if (a->NT != nt_fixed)
      return fail(CGDR_ERR_INVALID, "NT must be ceil(T/64)=%lld, but got %lld", (long long)nt_fixed, (long long)a->NT);
  } else {
    if (a->B != 1) return fail(CGDR_ERR_INVALID, "B must be 1 with cu_seqlens, but got %lld", (long long)a->B);
    if (a->N < 1 || a->N > a->T)
      return fail(CGDR_ERR_INVALID, "N must be in [1, T] with cu_seqlens, but got %lld", (long long)a->N);
    const int64_t lo = nt_fixed, hi = nt_fixed + a->N - 1;
    if (a->NT < lo || a->NT > hi)
      return fail(CGDR_ERR_INVALID, "NT=%lld is impossible for T=%lld and N=%lld; expected range [%lld, %lld]",
                  (long long)a->NT, (long long)a->T, (long long)a->N, (long long)lo, (long long)hi);
  }
  const int64_t units = a->B * a->NT * a->H * (a->V / vt);
  if (units > kMaxUnits) return fail(CGDR_ERR_UNSUPPORTED, "%lld workgroups exceed one launch", (long long)units);

  // 16-byte rows: q/k/o rows are moved with 16-byte loads and stores, h/v_new rows by
  // 16-byte direct-to-LDS pieces.
  struct { const char* name; const void* ptr; const int64_t* s; bool present; } t3[] = {
      {"q", a->q, a->stride_q, true}, {"k", a->k, a->stride_k, true}, {"v_new", a->v_new, a->stride_v, true},
      {"o", a->o, a->stride_o, true}, {"g", a->g, a->stride_g, a->g != nullptr},
  };
  for (auto& t : t3) {
    if (!t.present) continue;
    if (t.s[0] < 0 || t.s[1] < 1 || t.s[2] < 1)
      return fail(CGDR_ERR_INVALID, "%s has non-positive strides (%lld, %lld, %lld)", t.name, (long long)t.s[0],
                  (long long)t.s[1], (long long)t.s[2]);
    if (t.ptr == a->g) continue;
    if (!aligned16(t.ptr) || (t.s[0] % 8) || (t.s[1] % 8) || (t.s[2] % 8))
      return fail(CGDR_ERR_UNSUPPORTED, "%s rows must be 16-byte aligned (pointer and strides multiples of 8 elements)",
                  t.name);
  }
  if (64 * a->stride_v[1] * 2 >= (int64_t(1) << 31))
    return fail(CGDR_ERR_UNSUPPORTED, "64 rows of v_new span 2 GiB or more");
  const int64_t* sh = a->stride_h;
  if (sh[0] < 0 || sh[1] < a->K * a->V || sh[2] < a->K * a->V)
    return fail(CGDR_ERR_INVALID, "h strides must keep K x V blocks apart");
  if (!aligned16(a->h) || (sh[0] % 8) || (sh[1] % 8) || (sh[2] % 8) || (a->V % 8))
    return fail(CGDR_ERR_UNSUPPORTED, "h blocks must be 16-byte aligned");
  *vt_out = vt;
  return CGDR_OK;
}

cgdr::ChunkOParams to_params(const cgdr_chunk_o_args* a, int vt) {
  cgdr::ChunkOParams p;
  memset(&p, 0, sizeof(p));
  p.q = a->q; p.k = a->k; p.v = a->v_new; p.h = a->h; p.g = a->g;
  p.cu_seqlens = a->cu_seqlens; p.chunk_indices = a->chunk_indices; p.o = a->o;
  p.T = a->T; p.NT = a->NT; p.V = a->V;
  p.H = (int32_t)a->H; p.Hg = (int32_t)a->Hg; p.N = (int32_t)a->N; p.n_vtiles = (int32_t)(a->V / vt);
  p.scale = a->scale;
  p.n_xcd = cgdr_host::device_xcds();
  p.sq_b = a->stride_q[0]; p.sq_t = a->stride_q[1]; p.sq_h = a->stride_q[2];
  p.sk_b = a->stride_k[0]; p.sk_t = a->stride_k[1]; p.sk_h = a->stride_k[2];
  p.sv_b = a->stride_v[0]; p.sv_t = a->stride_v[1]; p.sv_h = a->stride_v[2];
  p.sh_b = a->stride_h[0]; p.sh_c = a->stride_h[1]; p.sh_h = a->stride_h[2];
  p.sg_b = a->stride_g[0]; p.sg_t = a->stride_g[1]; p.sg_h = a->stride_g[2];
  p.so_b = a->stride_o[0]; p.so_t = a->stride_o[1]; p.so_h = a->stride_o[2];
  return p;
}

template <int KD, int VT>
hipError_t launch(const cgdr::ChunkOParams& p, int64_t units, hipStream_t s) {
  hipLaunchKernelGGL((cgdr::cgdr_chunk_o_bf16_kernel<KD, VT>), dim3((unsigned)units), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int KD>
hipError_t dispatch_vt(const cgdr::ChunkOParams& p, int vt, int64_t units, hipStream_t s) {
  switch (vt) {
    case 128:
      if constexpr (KD <= 128) return launch<KD, 128>(p, units, s);
      return hipErrorInvalidValue;
    case 64: return launch<KD, 64>(p, units, s);
    default: return launch<KD, 32>(p, units, s);
  }
}

}  // namespace

extern "C" {

cgdr_status cgdr_chunk_o_get_plan(const cgdr_chunk_o_args* args, int32_t* v_tile, int64_t* workgroups) {
  if (v_tile == nullptr || workgroups == nullptr) return fail(CGDR_ERR_NULLPTR, "v_tile and workgroups are required");
  int vt = 0;
  cgdr_status st = validate(args, &vt);
  if (st != CGDR_OK) return st;
  *v_tile = vt;
  *workgroups = args->B * args->NT * args->H * (args->V / vt);
  return CGDR_OK;
}

cgdr_status cgdr_chunk_o_launch(const cgdr_chunk_o_args* args, void* stream) {
  int vt = 0;
  cgdr_status st = validate(args, &vt);
  if (st != CGDR_OK) return st;
  const cgdr::ChunkOParams p = to_params(args, vt);
  const int64_t units = args->B * args->NT * args->H * (args->V / vt);
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (args->K) {
    case 32: e = dispatch_vt<32>(p, vt, units, s); break;
    case 64: e = dispatch_vt<64>(p, vt, units, s); break;
    case 128: e = dispatch_vt<128>(p, vt, units, s); break;
    default: e = dispatch_vt<256>(p, vt, units, s); break;
  }
  if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "chunk output launch failed: %s", hipGetErrorString(e));
  return CGDR_OK;
}

}  // extern "C"
