// cgdr_wy.hip -- C ABI of the gfx950 WY producer (include/cgdr_wy.h): validation and the
// launch of one workgroup per (batch row, chunk, value head).  The reference's stage 1 splits
// chunk groups over cores (ref/chunk_gated_delta_rule/op_host/chunk_gated_delta_rule_tiling.cpp:122).
#include "../../include/cgdr_wy.h"

#include <hip/hip_runtime.h>

#include <cstring>

#include "cgdr_host.h"
#include "cgdr_wy_kernel.h"

namespace {

using cgdr_host::fail;

constexpr int64_t kMaxUnits = (int64_t(1) << 31) - 1;

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }
bool dim_ok(int64_t d) { return d == 32 || d == 64 || d == 128 || d == 256; }

cgdr_status validate(const cgdr_wy_args* a) {
  if (a == nullptr) return fail(CGDR_ERR_NULLPTR, "args is NULL");
  if (a->k == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input k is missing");
  if (a->v == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input v is missing");
  if (a->beta == nullptr) return fail(CGDR_ERR_NULLPTR, "Required input beta is missing");
  if (a->w == nullptr) return fail(CGDR_ERR_NULLPTR, "Required output w is missing");
  if (a->u == nullptr) return fail(CGDR_ERR_NULLPTR, "Required output u is missing");
  if (a->chunk_size != CGDR_CHUNK_SIZE)
    return fail(CGDR_ERR_UNSUPPORTED, "chunk_size must be %d, but got %lld", CGDR_CHUNK_SIZE, (long long)a->chunk_size);
  if (a->in_dtype != CGDR_BF16 && a->in_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "in_dtype %d is not a cgdr_dtype", a->in_dtype);
  if (a->in_dtype != CGDR_BF16) return fail(CGDR_ERR_UNSUPPORTED, "the WY producer is built for bf16 inputs only");
  if (a->beta_dtype != CGDR_BF16 && a->beta_dtype != CGDR_F32)
    return fail(CGDR_ERR_INVALID, "beta_dtype %d is not a cgdr_dtype", a->beta_dtype);
  if (a->B < 1) return fail(CGDR_ERR_INVALID, "B must be >= 1, but got %lld", (long long)a->B);
  if (a->T < 1) return fail(CGDR_ERR_INVALID, "T must be >= 1, but got %lld", (long long)a->T);
  if (a->H < 1 || a->Hg < 1 || a->H % a->Hg != 0)
    return fail(CGDR_ERR_INVALID, "H must be a positive multiple of Hg: H=%lld, Hg=%lld", (long long)a->H,
                (long long)a->Hg);
  if (!dim_ok(a->K)) return fail(CGDR_ERR_UNSUPPORTED, "K must be 32, 64, 128 or 256, but got %lld", (long long)a->K);
  if (!dim_ok(a->V)) return fail(CGDR_ERR_UNSUPPORTED, "V must be 32, 64, 128 or 256, but got %lld", (long long)a->V);

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
  if (a->B * a->NT * a->H > kMaxUnits) return fail(CGDR_ERR_UNSUPPORTED, "too many workgroups for one launch");

  struct { const char* name; const void* ptr; const int64_t* s; bool rows16; } t3[] = {
      {"k", a->k, a->stride_k, true},        {"v", a->v, a->stride_v, true},
      {"w", a->w, a->stride_w, true},        {"u", a->u, a->stride_u, true},
      {"beta", a->beta, a->stride_beta, false}, {"g", a->g, a->stride_g, false},
      {"g_cumsum", a->g_cumsum, a->stride_g_cumsum, false},
  };
  for (auto& t : t3) {
    if (t.ptr == nullptr) continue;
    if (t.s[0] < 0 || t.s[1] < 1 || t.s[2] < 1)
      return fail(CGDR_ERR_INVALID, "%s has non-positive strides (%lld, %lld, %lld)", t.name, (long long)t.s[0],
                  (long long)t.s[1], (long long)t.s[2]);
    if (t.rows16 && (!aligned16(t.ptr) || (t.s[0] % 8) || (t.s[1] % 8) || (t.s[2] % 8)))
      return fail(CGDR_ERR_UNSUPPORTED, "%s rows must be 16-byte aligned (pointer and strides multiples of 8 elements)",
                  t.name);
  }
  if (64 * a->stride_k[1] * 2 >= (int64_t(1) << 31) || 64 * a->stride_v[1] * 2 >= (int64_t(1) << 31))
    return fail(CGDR_ERR_UNSUPPORTED, "64 rows of k or v span 2 GiB or more");
  return CGDR_OK;
}

template <int KD, int VD>
hipError_t launch(const cgdr::WyParams& p, int64_t units, hipStream_t s) {
  hipLaunchKernelGGL((cgdr::cgdr_wy_bf16_kernel<KD, VD>), dim3((unsigned)units), dim3(256), 0, s, p);
  return hipGetLastError();
}

template <int KD>
hipError_t dispatch_v(const cgdr::WyParams& p, int64_t V, int64_t units, hipStream_t s) {
  switch (V) {
    case 32: return launch<KD, 32>(p, units, s);
    case 64: return launch<KD, 64>(p, units, s);
    case 128: return launch<KD, 128>(p, units, s);
    default: return launch<KD, 256>(p, units, s);
  }
}

}  // namespace

extern "C" cgdr_status cgdr_wy_launch(const cgdr_wy_args* a, void* stream) {
  cgdr_status st = validate(a);
  if (st != CGDR_OK) return st;
  cgdr::WyParams p;
  memset(&p, 0, sizeof(p));
  p.k = a->k; p.v = a->v; p.beta = a->beta; p.g = a->g;
  p.cu_seqlens = a->cu_seqlens; p.chunk_indices = a->chunk_indices;
  p.w = a->w; p.u = a->u; p.gc = a->g_cumsum;
  p.T = a->T; p.NT = a->NT;
  p.H = (int32_t)a->H; p.Hg = (int32_t)a->Hg; p.N = (int32_t)a->N; p.beta_f32 = a->beta_dtype == CGDR_F32;
  p.n_xcd = cgdr_host::device_xcds();
  p.sk_b = a->stride_k[0]; p.sk_t = a->stride_k[1]; p.sk_h = a->stride_k[2];
  p.sv_b = a->stride_v[0]; p.sv_t = a->stride_v[1]; p.sv_h = a->stride_v[2];
  p.sb_b = a->stride_beta[0]; p.sb_t = a->stride_beta[1]; p.sb_h = a->stride_beta[2];
  p.sg_b = a->stride_g[0]; p.sg_t = a->stride_g[1]; p.sg_h = a->stride_g[2];
  p.sw_b = a->stride_w[0]; p.sw_t = a->stride_w[1]; p.sw_h = a->stride_w[2];
  p.su_b = a->stride_u[0]; p.su_t = a->stride_u[1]; p.su_h = a->stride_u[2];
  p.sc_b = a->stride_g_cumsum[0]; p.sc_t = a->stride_g_cumsum[1]; p.sc_h = a->stride_g_cumsum[2];
  const int64_t units = a->B * a->NT * a->H;
  hipStream_t s = (hipStream_t)stream;
  hipError_t e;
  switch (a->K) {
    case 32: e = dispatch_v<32>(p, a->V, units, s); break;
    case 64: e = dispatch_v<64>(p, a->V, units, s); break;
    case 128: e = dispatch_v<128>(p, a->V, units, s); break;
    default: e = dispatch_v<256>(p, a->V, units, s); break;
  }
  if (e != hipSuccess) return fail(CGDR_ERR_LAUNCH, "WY launch failed: %s", hipGetErrorString(e));
  return CGDR_OK;
}
