// cgdr_kernels.h -- gfx950 device code of the ChunkGatedDeltaRuleFwdH operator.
//
// One workgroup owns one task (sequence n, value head h, V-tile of 16*NCW columns) and
// walks the chunks of its sequence in order.  The K x Vt fp32 state never leaves the
// VGPRs of the compute waves.  Per chunk (docs/problem.txt:353-422 of the reference):
//
//   MM1  Vn = U - W bf16(S)             [64 x K] x [K x 16] per compute wave, bf16 MFMA
//   v_new = bf16(Vn)                     (staged through LDS, stored by the store wave)
//   Vd   = bf16(Vn * exp(g_last - g))    (safe_exp, docs/problem.txt:272-274)
//   MM2  S = exp(g_last) S + K^T Vd      [K x 64] x [64 x 16] per compute wave
//   h[c] = bf16(S entering the chunk)    (staged through LDS, stored by the store wave)
//
// Operand orientation is chosen so that neither the state nor Vd needs a layout change
// between the two MFMAs: the MM2 accumulator (S) is directly the MM1 B operand after a
// bf16 conversion, and the MM1 accumulator (Vn) is directly the MM2 B operand.  This
// works because the row order inside an MFMA tile is free: MM2 tile kt row i holds
// k = pi(kt, i) and MM1 tile tt row i holds token sigma(tt, i) with
//     pi(2kb + hh, 4g + r)    = 32 kb + 8 g + 4 hh + r
//     sigma(2tb + hh, 4g + r) = 32 tb + 8 g + 4 hh + r
// so lane group g of two adjacent tiles holds 8 consecutive k (or tokens), which is the
// 8-element contraction slice the v_mfma_f32_16x16x32_bf16 B operand wants.
//
// Roles inside a workgroup (wave index; the waves of a workgroup are dealt to the CU's four
// SIMDs in order, so waves w and w+4 share one):
//   0 .. NCWT-1  compute waves (NCWT = RS * NCW): 16 value columns each, or with RS = 2 two
//               waves per 16 columns, each holding half of the state rows; no global memory
//               traffic in the loop
//   NCWT .. NCWT+NSW-1  store waves (NSW = NCW): h snapshot and v_new of chunk c-1 from LDS
//               staging to HBM, store instructions shared round-robin; without helper
//               workgroups, store wave 0 also touches chunk c+prefetch into L2
//   NCWT+NSW .. NCWT+NSW+NLW-1  load waves: direct-to-LDS DMA of the W, K, U tiles of chunk
//               c+STAGES-1 (shared round-robin)
//   NCWT+NSW+NLW gate wave: loads the raw g rows (two chunks ahead, into registers) and
//               writes the gate factors of chunk c+1 into LDS
// With two compute waves the order puts the store waves on SIMDs of their own and the light
// load and gate waves beside the compute waves (measured: 13 % faster than the store waves
// beside the compute waves).
// One s_barrier per chunk hands stages over; no wave waits on another wave's memory
// counters, and no wave mixes VMEM loads and stores (which would force vmcnt(0)).
//
// CONTEST = true runs the numerics of the contest reference run() (docs/problem.txt:81-167;
// code/tests/golden/generate_golden.py:350-440), "O2", on the same pipeline:
//   state S in bf16;  ws = bf16(W S);  v16 = f16sat(f16sat(u) - nan_to_num(fp16(ws)))
//   v_new = bf16(v16);  vd = bf16(f16sat(v16 * f16sat(exp(g_last - g))))
//   hd = f16sat(f16sat(S) * fp16(exp(fp16(g_last))));  up = nan_to_num(fp16(bf16(K^T vd)))
//   S = bf16(bf16(hd) + bf16(up))
// where f16sat is the reference's cast_to_float16 (round to fp16, finite overflow saturates to
// +-65504, inf and NaN pass through).  The operands are bf16, so the MFMA products are the bf16
// GEMMs' products, accumulated in fp32 and rounded once to bf16: MM1 starts from zero instead of
// U, and MM2 accumulates K^T vd alone, combined with the decayed state after it.  Contest
// numerics take two launches: a fast pass (NUM = 1) with plain fp16 roundings in place of the
// saturating casts and nan_to_num, where the store waves (h snapshots, v_new), the gate wave
// (gates, decay) and the compute waves (final state, once) flag the (sequence, head) whose
// values leave the range where the two agree; then a full pass (NUM = 2) with the casts, whose
// workgroups return at once for unflagged heads.  So the result is the full pass's everywhere.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "cgdr_schedule.h"

namespace cgdr {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

constexpr int kChunk = 64;

// Kernel arguments (one kernarg block).  Strides are in elements.
struct FwdHParams {
  const void* k;
  const void* w;
  const void* u;
  const float* g;
  const void* h0;
  const int64_t* cu_seqlens;
  const int64_t* chunk_offsets;
  void* h;
  void* v_new;
  void* final_state;
  int64_t T, H, Hg, V, N, NT;
  int64_t sk_b, sk_t, sk_h;
  int64_t sw_b, sw_t, sw_h;
  int64_t su_b, su_t, su_h;
  int64_t sg_b, sg_t, sg_h;
  int64_t sh_b, sh_c, sh_h;
  int64_t sv_b, sv_t, sv_h;
  int64_t sh0_n, sh0_h;
  int64_t sf_n, sf_h;
  int32_t n_vtiles;     // V / Vt
  int32_t n_tasks;      // N * H * n_vtiles
  int32_t head_ratio;   // H / Hg
  int32_t h0_f32;       // initial_state dtype is fp32 (else bf16)
  int32_t final_f32;    // final_state dtype is fp32 (else bf16)
  int32_t has_g;
  int32_t prefetch;     // L2 prefetch distance in chunks (0: off)
  int32_t helpers;      // 1: one L2-prefetch workgroup per task (grid = 2 * n_tasks)
  int32_t helper_lead;  // chunks a helper runs ahead of its task's load waves
  int32_t helper_waves; // waves per helper workgroup issuing touches
  int32_t n_xcd;        // XCDs workgroups are dealt to round-robin (blockIdx % n_xcd)
  int32_t K;            // key dim, a multiple of 16 up to the kernel's KD: columns K..KD-1 of
                        // the K and W tiles and rows K..KD-1 of the state are zero padding
  int32_t state_vk;     // initial and final state blocks are V x K (rows of K), else K x V
  int32_t epoch;        // this launch's tag (1..255): the top byte of a helper's progress value,
                        // and the value of a contest flag this launch raised
  int32_t* progress;    // helpers: chunk iterations completed per task, one 128-byte line per
                        // task (kProgressStride ints; epoch-tagged, not cleared)
  int32_t* redo;        // contest: one flag per (sequence, head); a head is flagged when its flag
                        // holds this launch's epoch (flags are not cleared between launches)
  int32_t vec_out;      // fp32 kernel: h and v_new take 16-byte stores of 4 value columns (aligned
                        // pointers, strides and V multiples of 4 elements)
};

constexpr int kProgressStride = 32;

// Scalar load that bypasses the scalar cache (reads L2): a helper workgroup polls its task's
// progress counter with it, so the poll never waits behind the helper's own outstanding
// vector loads (those are counted by vmcnt, this by lgkmcnt).
__device__ __forceinline__ int poll_l2(const int* addr) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(addr) : "memory");
  return v;
}

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] at [15:14]).
__device__ __forceinline__ constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | (7 << 4) | ((lgkm & 15) << 8) | (((vm >> 4) & 3) << 14);
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0)); }
template <int VM>
__device__ __forceinline__ void wait_vm() { __builtin_amdgcn_s_waitcnt(waitcnt_imm(VM, 15)); }

// Workgroup barrier without the implied release/acquire fences of __syncthreads(): the
// fences would make every wave drain its memory counters (vmcnt(0)), which would stall
// the load wave's prefetches.  Each role waits for exactly what it hands over before
// arriving.  The asm statements keep the compiler from moving memory operations across.
__device__ __forceinline__ void block_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Direct-to-LDS DMA: each lane moves 16 (or 4) bytes from sbase + voff to LDS address
// lds_addr + 16 * lane (4 * lane).  Written as asm so the compiler's waitcnt insertion does
// not track it; callers wait with explicit s_waitcnt vmcnt.  M0 holds the LDS address.
__device__ __forceinline__ void dma_b128(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds_addr) : "memory", "m0");
}
// 4 bytes per lane from a per-lane 64-bit address (used to touch lines into L2).
__device__ __forceinline__ void dma_b32_addr(const void* addr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :: "v"(addr), "s"(lds_addr) : "memory", "m0");
}
__device__ __forceinline__ void dma_b32(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :: "v"(voff), "s"(sbase), "s"(lds_addr) : "memory", "m0");
}

__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
  bf16x2 v;
  v[0] = (__bf16)lo;
  v[1] = (__bf16)hi;
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ float bf16_lo(unsigned x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(unsigned x) { return __uint_as_float(x & 0xffff0000u); }

__device__ __forceinline__ float safe_exp(float x) { return x <= 0.f ? expf(x) : 0.f; }

// cast_to_float16 (code/tests/golden/generate_golden.py:285-290), returned as its fp32 value
__device__ __forceinline__ float f16_sat(float x) {
  float r = (float)(_Float16)x;
  if (__builtin_isfinite(x)) r = fminf(fmaxf(r, -65504.f), 65504.f);
  return r;
}
// torch.nan_to_num(x.to(float16), nan=0, posinf=inf, neginf=-inf)
__device__ __forceinline__ float f16_nan_to_num(float x) {
  const float r = (float)(_Float16)x;
  return r != r ? 0.f : r;
}
__device__ __forceinline__ float bf16_rnd(float x) { return (float)(__bf16)x; }
__device__ __forceinline__ float f16_rnd(float x) { return (float)(_Float16)x; }

// Pairs of fp16 values for the contest fast pass (v_cvt_pk_f16_f32, v_pk_add_f16 and
// v_pk_mul_f16, all round-to-nearest-even).  A sum or product of two fp16 values rounded once
// to fp16 equals the reference's float32 operation followed by a cast to fp16: a product of two
// fp16 significands is exact in float32, and a float32 sum rounded again to fp16 is a double
// rounding with 24 >= 2 * 11 + 2 bits, which never changes the result.
typedef __attribute__((ext_vector_type(2))) _Float16 h16x2;
typedef __attribute__((ext_vector_type(2))) float f32x2;
__device__ __forceinline__ h16x2 to_h16x2(float lo, float hi) {
  return __builtin_convertvector((f32x2){lo, hi}, h16x2);
}
__device__ __forceinline__ h16x2 bf16x2_to_h16x2(unsigned w) { return to_h16x2(bf16_lo(w), bf16_hi(w)); }
// A word as an fp16 pair.  Takes the word by value: __builtin_bit_cast applied directly to an
// element of an ext_vector_type (v[j]) reads element 0 whatever j is (found with this kernel's
// gate factors), so vector elements are copied out first.
__device__ __forceinline__ h16x2 as_h16x2(unsigned w) { return __builtin_bit_cast(h16x2, w); }
__device__ __forceinline__ unsigned h16x2_to_bf16x2(h16x2 x) {
  const f32x2 f = __builtin_convertvector(x, f32x2);
  return pack_bf16x2(f[0], f[1]);
}
// The value unchanged, but opaque to the optimizer: it keeps a packed bf16 pair as one word
// (one v_cvt_pk_bf16_f32 and two unpacks), instead of re-deriving each half with a rounding of
// its own, and it pins a value computed in one phase of the chunk to that phase.
__device__ __forceinline__ unsigned opaque(unsigned x) {
  asm volatile("" : "+v"(x));
  return x;
}
__device__ __forceinline__ float opaque_f(float x) {
  asm volatile("" : "+v"(x));
  return x;
}
// c + the fp16 value in the low (high) half of h, in float32 (v_fma_mix_f32 with a factor of 1:
// one rounding, i.e. the float32 sum; it reads the fp16 operand without a conversion).
__device__ __forceinline__ float add_f16lo(h16x2 h, float c) {
  float d;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(c));
  return d;
}
__device__ __forceinline__ float add_f16hi(h16x2 h, float c) {
  float d;
  asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(h), "v"(c));
  return d;
}
// Contest fast pass, state decay of one pair of the bf16 state (packed): bf16(fp16(fp16(S) a16))
// as two floats, pinned to the phase that computes them.
__device__ __forceinline__ void contest_decay_pair(unsigned sp, h16x2 a16, float& hd0, float& hd1) {
  const f32x2 f = __builtin_convertvector(to_h16x2(bf16_lo(sp), bf16_hi(sp)) * a16, f32x2);
  const unsigned hw = opaque(pack_bf16x2(f[0], f[1]));
  hd0 = opaque_f(bf16_lo(hw));
  hd1 = opaque_f(bf16_hi(hw));
}
// Contest fast pass, state combine of one pair: bf16(hd + up), packed, with up = bf16(fp16(bf16(x)))
// of the MFMA sums x.  The fp16 value of a bf16 has at most 8 significant bits, so it is already
// up; the float32 sum is rounded once to bf16 (as the reference's bf16 addition does).
__device__ __forceinline__ unsigned contest_combine_pair(float x0, float x1, float hd0, float hd1) {
  const unsigned b = opaque(pack_bf16x2(x0, x1));
  const h16x2 up = to_h16x2(bf16_lo(b), bf16_hi(b));
  return opaque(pack_bf16x2(add_f16lo(up, hd0), add_f16hi(up, hd1)));
}

// Running maximum of |x| over the two bf16 of a word, per half, in one instruction: the bit
// patterns are read as fp16 and v_pk_maximum3_f16 takes max(acc, x, -x).  Magnitude bit patterns
// order like the values they encode in either format, and the patterns at or above 0x7c00
// (bf16 values from 2^121 up, infinities and NaNs) are fp16 infinities and NaNs, which this
// maximum propagates, so they end up above any finite threshold too.
__device__ __forceinline__ unsigned pk_absmax_bf16(unsigned acc, unsigned w) {
  asm("v_pk_maximum3_f16 %0, %0, %1, %1 neg_lo:[0,0,1] neg_hi:[0,0,1]" : "+v"(acc) : "v"(w));
  return acc;
}

// ---------------------------------------------------------------------------------------------
// Swizzles of 16-byte pieces inside LDS tiles (P = pieces per row).  Each is chosen so that the
// 16 lanes of one MFMA lane group hit 16 distinct 16-byte bank groups of the 256-byte bank row.

// W tile [64 tokens][K]: read by ds_read_b128, lanes i of a group read rows sigma(tt, i).
template <int P>
__device__ __forceinline__ int swz_w(int r) {
  if constexpr (P == 4) return (r >> 3) & 3;
  else if constexpr (P == 8) return ((r >> 1) & 1) | (((r >> 3) & 3) << 1);
  else return (r & 3) | (((r >> 3) & 3) << 2);
}
// K tile [64 tokens][K]: read by ds_read_b64_tr_b16, lanes 4e+q read row R0+e, piece 4kb+q.
template <int P>
__device__ __forceinline__ int swz_k(int r) {
  if constexpr (P == 4) return 0;
  else if constexpr (P == 8) return 4 * ((r >> 1) & 1);
  else return 4 * (r & 3);
}
// State staging [Vt rows = value columns][K]: written by ds_write_b128 from lanes n = 0..15.
template <int P>
__device__ __forceinline__ int swz_s(int v) {
  if constexpr (P == 4) return (v >> 2) & 3;
  else if constexpr (P == 8) return (v >> 1) & 7;
  else return v & 15;
}
// v_new staging [Vt rows][64 tokens] (8 pieces per row).
__device__ __forceinline__ int swz_v(int v) { return (v >> 1) & 7; }

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Task decoding shared by both kernels.  Workgroups are dealt to the XCDs round-robin
// (blockIdx % n_xcd), so consecutive task ids are remapped onto one XCD: the V-tiles of a
// head, and the heads sharing a key head, then share that XCD's L2 for their K and W reads.
// Compile-time loop: f(std::integral_constant<int, I>) for I in [I0, N).
template <int I0, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I0 < N) {
    f(std::integral_constant<int, I0>{});
    static_for<I0 + 1, N>(f);
  }
}

struct Task {
  int n, head, vtile;
  int64_t bos, len, boh;   // token offset, length, first chunk index of the sequence
  int b;                   // batch row (fixed-length mode) or 0
  int nc;                  // chunks this task walks (clamped so every write stays in bounds)
};

__device__ __forceinline__ int xcd_remap(int bid, int nblocks, int nx) {
  const int q = nblocks / nx, r = nblocks - q * nx;
  const int xcd = bid % nx, local = bid / nx;
  return (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + local;
}

__device__ __forceinline__ Task decode_task(const FwdHParams& p, int task_id) {
  Task t;
  t.vtile = task_id % p.n_vtiles;
  const int nh = task_id / p.n_vtiles;
  t.head = nh % (int)p.H;
  t.n = nh / (int)p.H;
  if (p.cu_seqlens != nullptr) {
    int64_t bos = p.cu_seqlens[t.n], eos = p.cu_seqlens[t.n + 1];
    bos = bos < 0 ? 0 : (bos > p.T ? p.T : bos);
    eos = eos < bos ? bos : (eos > p.T ? p.T : eos);
    int64_t boh;
    if (p.chunk_offsets != nullptr) {
      boh = p.chunk_offsets[t.n];
    } else {
      boh = 0;
      for (int m = 0; m < t.n; ++m) {
        int64_t l = p.cu_seqlens[m + 1] - p.cu_seqlens[m];
        boh += l > 0 ? (l + kChunk - 1) / kChunk : 0;
      }
    }
    t.b = 0;
    t.bos = bos;
    t.len = eos - bos;
    t.boh = boh;
  } else {
    t.b = t.n;
    t.bos = 0;
    t.len = p.T;
    t.boh = 0;
  }
  int64_t nc = (t.len + kChunk - 1) / kChunk;
  if (t.boh < 0 || t.boh >= p.NT) nc = 0;
  else if (t.boh + nc > p.NT) nc = p.NT - t.boh;
  t.nc = (int)nc;
  return t;
}

// Dispatch order of a packed variable-length batch.  Task ids are sequence-major
// ((n * H + head) * n_vtiles + vtile), and xcd_remap hands every XCD a contiguous range of
// dispatch indices, so in that order an XCD would receive whole sequences and the XCD with
// the longest ones would set the kernel's time.  With cu_seqlens and H % n_xcd == 0 a
// dispatch index is read instead as (XCD block, sequence rank, head within the block,
// V-tile): every XCD gets H/n_xcd heads of every sequence (equal work), a head's V-tiles and
// the heads sharing a key head stay on one XCD, and within an XCD longer sequences are
// dispatched first
// (ranked by length, longest first, ties by index, when N <= 64; natural order above that).
// Fixed-length batches keep the identity order.  Every lane of the calling wave must be active.
__device__ __forceinline__ int order_task(const FwdHParams& p, int d) {
  if (p.cu_seqlens == nullptr || ((int)p.H % p.n_xcd) != 0) return d;
  const int N = (int)p.N;
  const sched::VarlenSlot s = sched::varlen_slot(d, p.n_tasks, (int)p.H, p.n_vtiles, p.n_xcd);
  int n = s.rank;
  if (N <= 64) {
    // lane m < N holds sequence m's rank; they are a permutation of 0 .. N-1, so exactly one
    // lane matches
    const int lane = threadIdx.x & 63;
    const int rank = lane < N ? sched::seq_rank(p.cu_seqlens, N, lane) : -1;
    const unsigned long long hit = __ballot(rank == s.rank);
    if (hit != 0ull) n = __ffsll(hit) - 1;
  }
  return (n * (int)p.H + s.head) * p.n_vtiles + s.vtile;
}

// =============================================================================================
// bf16 pipeline kernel.
//   KD      key dim (32, 64, 128, 256)
//   NCW     compute waves; Vt = 16 * NCW
//   NLW     load waves (1, 2 or 4)
//   STAGES  LDS ring depth (chunks in flight: STAGES - 1 ahead of the compute waves)
//   RS      compute waves per 16 value columns: 1, or 2 with the state rows split between them
// =============================================================================================
template <int KD, int NCW, int NLW, int STAGES, int RS = 1>
struct Bf16Layout {
  static constexpr int VT = 16 * NCW;
  static constexpr int NCWT = RS * NCW;            // compute waves
  static constexpr int P = KD / 8;                 // 16-byte pieces per K row
  static constexpr int W_OFF = 0;
  static constexpr int K_OFF = 128 * KD;
  static constexpr int U_OFF = 256 * KD;
  static constexpr int G_OFF = 256 * KD + 128 * VT;            // gamma[64], a
  static constexpr int STAGE_BYTES = ((G_OFF + 260) + 255) / 256 * 256;
  static constexpr int SS_BUFS = RS == 1 ? 2 : 3;
  static constexpr int SS_OFF = STAGES * STAGE_BYTES;          // state staging, SS_BUFS buffers
  static constexpr int SS_BYTES = VT * KD * 2;
  static constexpr int SV_OFF = SS_OFF + SS_BUFS * SS_BYTES;   // v_new staging, 2 buffers
  static constexpr int SV_BYTES = VT * kChunk * 2;
  static constexpr int XV_OFF = SV_OFF + 2 * SV_BYTES;         // row split: Vd exchange, 1 KiB a wave
  static constexpr int XV_BYTES = RS == 1 ? 0 : NCWT * 1024;
  static constexpr int XF_OFF = XV_OFF + XV_BYTES;             // row split: exchange flags
  static constexpr int XF_BYTES = RS == 1 ? 0 : 256;
  static constexpr int TRASH_OFF = XF_OFF + XF_BYTES;          // L2-prefetch landing area
  static constexpr int LDS_BYTES = TRASH_OFF + 256;
  static constexpr int NSW = NCW;                              // store waves
  static constexpr int THREADS = 64 * (NCWT + NLW + NSW + 1);
  static constexpr int DMA_W = 128 * KD / 1024;               // DMA instructions per tile
  static constexpr int DMA_U = (128 * VT + 1023) / 1024;
  static constexpr int DMA_TILES = 2 * DMA_W + DMA_U;         // per chunk, over all load waves
  // DMA instructions load wave lw issues per full chunk: tile instruction i goes to wave
  // i % NLW.
  template <int LW>
  static constexpr int dma_per_chunk() {
    return DMA_TILES / NLW + (LW < DMA_TILES % NLW ? 1 : 0);
  }
};

// A configuration is valid when its LDS fits one gfx950 workgroup (160 KiB) and the prefetch
// depth D = STAGES - 1 can be awaited with vmcnt (<= 63 outstanding VMEM instructions per
// wave; load wave 0 carries the most per chunk).  The row split needs an even number of
// 32-row state blocks (KD >= 64) and at most 8 waves (two per SIMD).
template <int KD, int NCW, int NLW, int STAGES, int RS = 1>
constexpr bool bf16_config_ok() {
  using L = Bf16Layout<KD, NCW, NLW, STAGES, RS>;
  constexpr int per_chunk = L::template dma_per_chunk<0>();
  constexpr bool rs_ok = RS == 1 || (RS == 2 && (KD / 32) % 2 == 0 && L::THREADS <= 512);
  return rs_ok && STAGES >= 2 && L::LDS_BYTES <= 160 * 1024 && (STAGES - 2) * per_chunk <= 63;
}
template <int KD, int NCW, int NLW, int RS = 1>
constexpr int bf16_max_stages() {
  return bf16_config_ok<KD, NCW, NLW, 4, RS>() ? 4 : bf16_config_ok<KD, NCW, NLW, 3, RS>() ? 3
                                                                                          : bf16_config_ok<KD, NCW, NLW, 2, RS>() ? 2 : 0;
}

// NUM: 0 default numerics; 1 contest, fast pass (plain fp16 roundings, flags the heads where a
// saturating cast or nan_to_num could matter); 2 contest, full pass (the saturating casts, only
// for flagged heads).
template <int KD, int NCW, int NLW, int STAGES, int NUM = 0, int RS = 1>
__global__ void __launch_bounds__(64 * (RS * NCW + NLW + NCW + 1))
cgdr_fwd_h_bf16_kernel(const FwdHParams p) {
  constexpr bool CONTEST = NUM != 0, FULL = NUM == 2;
  using L = Bf16Layout<KD, NCW, NLW, STAGES, RS>;
  constexpr int NCWT = L::NCWT;
  constexpr int VT = L::VT, P = L::P;
  constexpr int KT = KD / 16;   // MM2 output tiles (rows of S)
  constexpr int KB = KD / 32;   // MM1 contraction blocks
  __shared__ __attribute__((aligned(1024))) char smem[L::LDS_BYTES];
  static_assert(L::LDS_BYTES <= 160 * 1024, "LDS budget of one gfx950 workgroup exceeded");

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform per wave
  const int lane = threadIdx.x & 63;
  const int slot = xcd_remap(blockIdx.x, gridDim.x, p.n_xcd);
  // With helpers the grid is 2 * n_tasks (n_tasks a multiple of n_xcd): every XCD holds m
  // tasks followed by their m helpers, so a helper and its task share that XCD's L2.
  int task_id = slot;
  bool helper = false;
  if (p.helpers) {
    const int m = p.n_tasks / p.n_xcd;
    const int x = slot / (2 * m), i = slot - x * 2 * m;
    helper = i >= m;
    task_id = x * m + (helper ? i - m : i);
  }
  if (task_id >= p.n_tasks) return;   // uniform per workgroup
  const Task tk = decode_task(p, order_task(p, task_id));
  if constexpr (FULL)
    if (p.redo[(int64_t)tk.n * p.H + tk.head] != p.epoch) return;   // uniform: the fast pass was exact
  const int NC = tk.nc;
  const int vbase = tk.vtile * VT;
  const int hk = tk.head / p.head_ratio;
  const bool has_g = p.g != nullptr;

  // Gate factors of chunk c into stage st from its raw g row (one wave; gv = g of token
  // `lane` of the chunk): gamma_t = safe_exp(g_last - g_t) for t < len, 0 for padded rows,
  // and a = exp(g_last) in slot 64.  No gating: gamma = 1, a = 1.
  bool gbad = false;   // contest fast pass, gate wave: a gate above 1 or NaN
  auto gates = [&](int c, int st, float gv) {
    const int64_t rem = tk.len - (int64_t)c * kChunk;
    const int len = rem < kChunk ? (int)rem : kChunk;
    float* gdst = (float*)(smem + st * L::STAGE_BYTES + L::G_OFF);
    float gamma, a;
    if (has_g) {
      const float glast = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(gv), len - 1));
      if constexpr (CONTEST) {
        // fp16 gate of every token and fp16 exp of the fp16 g_last (generate_golden.py:409-416)
        gamma = lane < len ? f16_sat(expf(glast - gv)) : 0.f;
        a = (float)(_Float16)expf(f16_sat(glast));
        gbad |= !(gamma <= 1.f) || !(a <= 1.f);   // the fast pass is exact for gates in [0, 1]
      } else {
        gamma = lane < len ? safe_exp(glast - gv) : 0.f;
        a = expf(glast);
      }
    } else {
      gamma = lane < len ? 1.f : 0.f;
      a = 1.f;
    }
    if constexpr (NUM == 1) ((_Float16*)gdst)[lane] = (_Float16)gamma;   // fp16-valued: exact
    else gdst[lane] = gamma;
    if (lane == 0) gdst[64] = a;
  };

  // L2 touch of chunk j: the head's K, W and U rows of the chunk are touched one `seg`-byte
  // segment per lane (a 4-byte DMA into a scratch LDS area; nothing waits on it until exit),
  // the segments shared round-robin among the head's V-tile tasks, so that the load waves'
  // DMAs of that chunk hit L2 rather than HBM.  Per-lane segment addresses are fixed here; a
  // chunk only adds t0 * row stride.  Used by store wave 0 when there are no helper
  // workgroups, touching a few chunks ahead of the load waves.
  constexpr int PF_INSTR = 4;
  const char* lptr[PF_INSTR];
  int64_t lstride[PF_INSTR];
  int npf = 0;
  const uint32_t trash = (uint32_t)(uintptr_t)((lds_char*)smem) + L::TRASH_OFF;
  auto l2_touch_setup = [&]() {
    const int nvt = p.n_vtiles;
    const int kb = 2 * p.K, vb = (int)(2 * p.V);   // row bytes, multiples of 32
    const int seg = (kb % 128 == 0 && vb % 128 == 0) ? 128 : ((kb % 64 == 0 && vb % 64 == 0) ? 64 : 32);
    const int segk = kb / seg, segv = vb / seg;
    const int segs = 64 * (2 * segk + segv);
    const char* kpf = (const char*)((const __bf16*)p.k + tk.b * p.sk_b + (int64_t)hk * p.sk_h);
    const char* wpf = (const char*)((const __bf16*)p.w + tk.b * p.sw_b + (int64_t)tk.head * p.sw_h);
    const char* upf = (const char*)((const __bf16*)p.u + tk.b * p.su_b + (int64_t)tk.head * p.su_h);
#pragma unroll
    for (int m = 0; m < PF_INSTR; ++m) {
      int i = tk.vtile + nvt * (64 * m + lane);
      i = i < segs ? i : segs - 1;
      if (i < 64 * segk) {
        lstride[m] = p.sk_t * 2; lptr[m] = kpf + (i / segk) * lstride[m] + (int64_t)seg * (i % segk);
      } else if (i < 128 * segk) {
        i -= 64 * segk;
        lstride[m] = p.sw_t * 2; lptr[m] = wpf + (i / segk) * lstride[m] + (int64_t)seg * (i % segk);
      } else {
        i -= 128 * segk;
        lstride[m] = p.su_t * 2; lptr[m] = upf + (i / segv) * lstride[m] + (int64_t)seg * (i % segv);
      }
    }
    npf = (segs / nvt + 63) / 64 < PF_INSTR ? (segs / nvt + 63) / 64 : PF_INSTR;
  };
  auto l2_touch = [&](int j) {
    const int64_t t0 = tk.bos + (int64_t)j * kChunk;
#pragma unroll
    for (int m = 0; m < PF_INSTR; ++m)
      if (m < npf) dma_b32_addr(lptr[m] + t0 * lstride[m], trash);
  };

  if (helper) {
    // ------------------------------------------------------------------ helper workgroup
    // Takes the task's HBM misses on this CU, so that the task's own CU only sees L2 hits
    // (an HBM miss holds up every later load of the CU that issued it).  One wave touches
    // chunks up to `helper_lead` chunks beyond the task's load waves, pacing itself on the
    // task's progress counter.  Nothing waits on a helper; a helper gives up after a bounded
    // number of idle polls, so it always exits.
    const int hwaves = p.helper_waves;
    if (wave >= hwaves) return;
    // Helper waves take chunks round-robin (wave w: chunks w+1, w+1+hwaves, ...).
    // Helper v of the head's n_vtiles covers rows [v R, (v+1) R), R = 64 / n_vtiles, of the
    // chunk's K, W and U rows (whole rows: every V-tile's U), with 16-byte-per-lane DMAs over
    // contiguous rows into a 1 KiB scratch area; helper 0 also touches the chunk's g row.
    const int nvt = p.n_vtiles;
    const int R = 64 / nvt;
    const int r0 = tk.vtile * R;
    const char* hk_base = (const char*)((const __bf16*)p.k + tk.b * p.sk_b + (int64_t)hk * p.sk_h);
    const char* hw_base = (const char*)((const __bf16*)p.w + tk.b * p.sw_b + (int64_t)tk.head * p.sw_h);
    const char* hu_base = (const char*)((const __bf16*)p.u + tk.b * p.su_b + (int64_t)tk.head * p.su_h);
    const char* hg_base = has_g ? (const char*)(p.g + tk.b * p.sg_b + (int64_t)tk.head * p.sg_h) : nullptr;
    const int64_t hk_st = p.sk_t * 2, hw_st = p.sw_t * 2, hu_st = p.su_t * 2, hg_st = p.sg_t * 4;
    const uint32_t hscratch = (uint32_t)(uintptr_t)((lds_char*)smem);
    auto touch_rows = [&](const char* base, int64_t stride, int row_bytes) {
      const int lpr = row_bytes / 16;           // lanes per row
      const int rpi = 64 / lpr;                 // rows per instruction
      const int lrow = lane / lpr, lcol = lane % lpr;
      for (int r = r0; r < r0 + R; r += rpi) {
        const int row = r + lrow;
        if (row < r0 + R)
          dma_b128(base, (uint32_t)(row * stride) + 16u * (uint32_t)lcol, hscratch);
      }
    };
    auto helper_touch = [&](int j) {
      const int64_t t0 = tk.bos + (int64_t)j * kChunk;
      touch_rows(hk_base + t0 * hk_st, hk_st, 2 * p.K);
      touch_rows(hw_base + t0 * hw_st, hw_st, 2 * p.K);
      touch_rows(hu_base + t0 * hu_st, hu_st, (int)(2 * p.V));
      if (hg_base != nullptr && tk.vtile == 0) dma_b32(hg_base + t0 * hg_st, (uint32_t)(lane * hg_st), hscratch);
    };
    constexpr int D = STAGES - 1;
    const int* prog_addr = p.progress + task_id * kProgressStride;
    // A progress value is (epoch << 24) | chunks done; a value left by an earlier launch (other
    // tag) or never written reads as 0.  The counters are not cleared before a launch.
    auto progress_of = [&](int v) -> int {
      return ((unsigned)v >> 24) == (unsigned)p.epoch ? (v & 0xffffff) : 0;
    };
    int issued = 1 + wave;   // chunk 0 is loaded before the task's first barrier
    int idle = 0;
    const int max_idle = 8 * NC + 4096;
    while (issued < NC) {
      const int done = progress_of(poll_l2(prog_addr));
      // Chunks below done + D are already in the task's own loads (a helper that starts late,
      // e.g. on a device shared with other work, skips them instead of touching them again).
      const int lo = done + D;
      if (issued < lo) issued += (lo - issued + hwaves - 1) / hwaves * hwaves;
      int target = done + D + p.helper_lead;
      target = target < NC ? target : NC;
      if (issued < target) {
        for (; issued < target; issued += hwaves)
          if (tk.len - (int64_t)issued * kChunk >= kChunk) helper_touch(issued);
        idle = 0;
      } else {
        if (++idle > max_idle) break;
        __builtin_amdgcn_s_sleep(16);
      }
    }
    wait_vm<0>();   // the touches write this workgroup's LDS: drain them before exit
    return;
  }

  if (wave < NCWT) {
   if constexpr (RS == 2) {
    // ------------------------------------------------------------------ compute waves, rows split
    // Wave (j, r) = (wave % NCW, wave / NCW) owns value columns 16 j .. 16 j + 15 of the tile and the
    // state rows of MM2 tiles kt = KT/2 r .. KT/2 r + KT/2 - 1 (k = KD/2 r .. KD/2 r + KD/2 - 1).
    // MM1 for token block tb = r takes the whole bf16(-S) of its columns, its own rows and its
    // partner's, from the staging buffer the store waves read for the h snapshot (three buffers:
    // bf16(-S) of chunk c+1 is staged at the end of chunk c; the contest fast pass stages +S, as
    // its MM1 starts from zero and the epilogue subtracts).  MM2 of its rows needs Vd of both
    // token blocks, so the two partners swap Vd through LDS once per chunk (1 KiB each, with a
    // flag).  Each wave reads half of the W and K^T operands and does half of the MFMA and VALU
    // work of a wave that owns all rows; every accumulation chain runs in the same order
    // (MM1: U, then k-blocks 0, 1, ...; MM2: a S, then token block 0, then 1), so the results
    // are bit-identical to that layout.
    constexpr int KTH = KT / 2, KBH = KB / 2;
    // (with two column blocks the partners sit on SIMDs 0 and 2, or 1 and 3, so each pair shares
    // its SIMDs with one store wave and with the load or the gate wave)
    const int j = wave % NCW, r = wave / NCW;
    const int g = lane >> 4, n = lane & 15;
    const int e = n >> 2, q = n & 3;
    const int vcol = vbase + 16 * j + n;         // value column owned by this lane
    const int vrow = 16 * j + n;                 // its row in the staging buffers
    // state element (i, rr) of this wave: own tile kt = KTH r + i, k row krow(i, rr)
    auto krow_of = [&](int i, int rr) { return 32 * (KBH * r + (i >> 1)) + 8 * g + 4 * (i & 1) + rr; };
    f32x4 S[KTH];
    if (p.h0 != nullptr) {
      const int64_t base = (int64_t)tk.n * p.sh0_n + (int64_t)tk.head * p.sh0_h;
#pragma unroll
      for (int i = 0; i < KTH; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int krow = krow_of(i, rr);
          const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
          S[i][rr] = krow >= p.K ? 0.f
                     : p.h0_f32 ? ((const float*)p.h0)[off]
                                : bf16_lo(((const unsigned short*)p.h0)[off]);
          if constexpr (CONTEST) S[i][rr] = bf16_rnd(S[i][rr]);   // the state is bf16
        }
    } else {
#pragma unroll
      for (int i = 0; i < KTH; ++i) S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // contest fast pass: the bf16 state kept as packed pairs between chunks (S holds only the
    // MFMA sums of a chunk)
    unsigned Sp[NUM == 1 ? KTH : 1][2];
    if constexpr (NUM == 1)
#pragma unroll
      for (int i = 0; i < KTH; ++i)
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) Sp[i][rr] = pack_bf16x2(S[i][2 * rr], S[i][2 * rr + 1]);
    // byte offsets of the staged pieces (vrow, k-block kb) of bf16(-S): all k-blocks (MM1
    // operands), and this wave's own ones (where it stages its rows)
    int soff[KB], sown[KBH];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) soff[kb] = (vrow * P + ((4 * kb + g) ^ swz_s<P>(vrow))) * 16;
#pragma unroll
    for (int ib = 0; ib < KBH; ++ib) sown[ib] = (vrow * P + ((4 * (KBH * r + ib) + g) ^ swz_s<P>(vrow))) * 16;
    // K^T operand pieces of own k-block ib: the swizzle of row 32 tb + 8 g + 4 half + e depends
    // only on the row's two low bits, which are e's
    int kofs[KBH];
#pragma unroll
    for (int ib = 0; ib < KBH; ++ib) kofs[ib] = ((4 * (KBH * r + ib) + q) ^ swz_k<P>(8 * g + e)) * 16;
    auto stage_state = [&](int buf) {
      char* ss = smem + L::SS_OFF + buf * L::SS_BYTES;
#pragma unroll
      for (int ib = 0; ib < KBH; ++ib) {
        u32x4 w;
        if constexpr (NUM == 1) {
          w = u32x4{Sp[2 * ib][0], Sp[2 * ib][1], Sp[2 * ib + 1][0], Sp[2 * ib + 1][1]};   // +S
        } else {
          w[0] = pack_bf16x2(-S[2 * ib][0], -S[2 * ib][1]);
          w[1] = pack_bf16x2(-S[2 * ib][2], -S[2 * ib][3]);
          w[2] = pack_bf16x2(-S[2 * ib + 1][0], -S[2 * ib + 1][1]);
          w[3] = pack_bf16x2(-S[2 * ib + 1][2], -S[2 * ib + 1][3]);
        }
        *(u32x4*)(ss + sown[ib]) = w;
      }
    };
    char* const xme = smem + L::XV_OFF + ((2 * j + r) * 64 + lane) * 16;
    const char* const xpa = smem + L::XV_OFF + ((2 * j + (r ^ 1)) * 64 + lane) * 16;
    typedef __attribute__((address_space(3))) int lds_int;
    volatile lds_int* const fme = (volatile lds_int*)((lds_char*)smem + L::XF_OFF) + 2 * j + r;
    volatile lds_int* const fpa = (volatile lds_int*)((lds_char*)smem + L::XF_OFF) + 2 * j + (r ^ 1);
    if (lane == 0) *fme = 0;
    stage_state(0);
    block_barrier();   // P: stage 0 ready, bf16(-S_0) staged, flags cleared

    // One chunk per loop iteration, with the stage and staging parity computed at run time:
    // unrolled over the stage cycle (every LDS address an immediate offset) this path measured
    // 3 % slower (507 vs 491 us, contest numerics), its loop body then being six times larger.
    auto chunk_step = [&](const int c) {
      const int st = c % STAGES;
      const int par = c & 1;
      const char* sbase = smem + st * L::STAGE_BYTES;
      const lds_char* stage = (const lds_char*)sbase;
      const float* gam = (const float*)(sbase + L::G_OFF);
      const char* ssr = smem + L::SS_OFF + (c % 3) * L::SS_BYTES;   // bf16(-S_c)

      // Phase 1: the LDS reads of MM1 and the epilogue (token block r): a, gamma, U, W, bf16(-S).
      const float a = gam[64];
      // gamma of tokens 32 r + 8 g + 4 hh + (0..3); the contest fast pass has them as fp16 pairs
      f32x4 gm[NUM == 1 ? 1 : 2];
      u32x4 g16;
      if constexpr (NUM == 1) {
        g16 = *(const u32x4*)((const char*)gam + 2 * (32 * r + 8 * g));
      } else {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) gm[hh] = *(const f32x4*)(gam + 32 * r + 8 * g + 4 * hh);
      }
      u32x2 uraw[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int t0 = 32 * r + 8 * g + 4 * hh;
        const lds_char* up = stage + L::U_OFF + ((t0 + e) * VT + 16 * j + 4 * q) * 2;
        uraw[hh] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)up));
      }
      u32x4 wop[2][KB];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const int row = 32 * r + 8 * e + 4 * hh + q;
        const u32x4* wrow = (const u32x4*)(sbase + L::W_OFF) + row * P;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) wop[hh][kb] = wrow[(4 * kb + g) ^ swz_w<P>(row)];
      }
      u32x4 Sw[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) Sw[kb] = *(const u32x4*)(ssr + soff[kb]);
      f32x4 acc[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
        acc[hh] = CONTEST ? f32x4{0.f, 0.f, 0.f, 0.f}
                          : f32x4{bf16_lo(uraw[hh][0]), bf16_hi(uraw[hh][0]), bf16_lo(uraw[hh][1]), bf16_hi(uraw[hh][1])};
      __builtin_amdgcn_sched_barrier(0);

      // Phase 2: MM1 of token block r (two chains, k-block major), the decay of own rows and the
      // K^T reads of token block 0 between the MFMAs.
      auto read_kop = [&](int tb, u32x4* kop) {
#pragma unroll
        for (int i = 0; i < KTH; ++i) {
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int row = 32 * tb + 8 * g + 4 * half + e;
            const lds_char* kp = stage + L::K_OFF + row * P * 16 + kofs[i >> 1] + 8 * (i & 1);
            const u32x2 kw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)kp));
            kop[i][2 * half] = kw[0];
            kop[i][2 * half + 1] = kw[1];
          }
        }
      };
      u32x4 kop0[KTH], kop1[KTH];
      unsigned hdp[FULL ? KTH : 1][2];
      float hdf[NUM == 1 ? KTH : 1][4];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
          acc[hh] = mfma_bf16(__builtin_bit_cast(bf16x8, wop[hh][kb]), __builtin_bit_cast(bf16x8, Sw[kb]), acc[hh]);
#pragma unroll
      for (int i = 0; i < KTH; ++i) {
        if constexpr (FULL) {
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
            hdp[i][rr] = pack_bf16x2(f16_sat(f16_sat(S[i][2 * rr]) * a), f16_sat(f16_sat(S[i][2 * rr + 1]) * a));
          S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else if constexpr (CONTEST) {
          const h16x2 a16 = to_h16x2(a, a);
#pragma unroll
          for (int rr = 0; rr < 2; ++rr) contest_decay_pair(Sp[i][rr], a16, hdf[i][2 * rr], hdf[i][2 * rr + 1]);
          S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
          S[i] = S[i] * a;
        }
      }
      read_kop(0, kop0);
#pragma unroll
      for (int i = 0; i < 2 * KB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, (KTH + 2 * KB - 1) / (2 * KB), 0);   // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, (2 * KTH + 2 * KB - 1) / (2 * KB), 0);   // DS read
      }
      __builtin_amdgcn_sched_barrier(0);

      // Phase 3: epilogue of token block r (v_new staging, Vd), Vd to the partner.
      u32x4 pv, pd;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int hh = jj >> 1, rr = 2 * (jj & 1);
        const float v0 = acc[hh][rr], v1 = acc[hh][rr + 1];
        if constexpr (CONTEST) {
          const u32x2 ur = uraw[hh];
          const float u0 = rr == 0 ? bf16_lo(ur[0]) : bf16_lo(ur[1]);
          const float u1 = rr == 0 ? bf16_hi(ur[0]) : bf16_hi(ur[1]);
          if constexpr (FULL) {
            const float x0 = f16_sat(f16_sat(u0) - f16_nan_to_num(-bf16_rnd(v0)));
            const float x1 = f16_sat(f16_sat(u1) - f16_nan_to_num(-bf16_rnd(v1)));
            pv[jj] = pack_bf16x2(x0, x1);
            pd[jj] = pack_bf16x2(f16_sat(x0 * gm[hh][rr]), f16_sat(x1 * gm[hh][rr + 1]));
          } else {
            // acc = +W S (the fast pass stages +S): v16 = fp16(u) + fp16(bf16(-acc)); v16 is
            // staged as fp16
            const h16x2 x16 = to_h16x2(u0, u1) + bf16x2_to_h16x2(pack_bf16x2(-v0, -v1));
            pv[jj] = __builtin_bit_cast(unsigned, x16);
            pd[jj] = h16x2_to_bf16x2(x16 * as_h16x2(g16[jj]));
          }
        } else {
          pv[jj] = pack_bf16x2(v0, v1);
          pd[jj] = pack_bf16x2(v0 * gm[hh][rr], v1 * gm[hh][rr + 1]);
        }
      }
      {
        u32x4* sv = (u32x4*)(smem + L::SV_OFF + par * L::SV_BYTES);
        sv[vrow * 8 + ((4 * r + g) ^ swz_v(vrow))] = pv;
      }
      *(u32x4*)xme = pd;
      // the Vd write has landed before the flag is raised (LDS ops of a wave complete in order,
      // and lgkmcnt(0) waits for them)
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane == 0) *fme = c + 1;
      read_kop(1, kop1);
      // The partner raises its flag to c + 1 once its Vd of chunk c is in LDS.  It cannot be a
      // chunk ahead: it writes chunk c+1's Vd and flag only after barrier B_c, which this wave
      // reaches after reading.  The bound on the polls only guarantees an exit.
      auto partner_vd = [&]() -> bf16x8 {
        for (int it = 0; it < (1 << 20); ++it)
          if (__builtin_amdgcn_readfirstlane(*fpa) >= c + 1) break;
        asm volatile("" ::: "memory");
        return __builtin_bit_cast(bf16x8, *(const u32x4*)xpa);
      };

      // Phase 4: MM2 of own rows, token block 0 then 1 (the order of the one-wave layout).
      bf16x8 Vd1;
      if (r == 0) {
        const bf16x8 Vd0 = __builtin_bit_cast(bf16x8, pd);
#pragma unroll
        for (int i = 0; i < KTH; ++i) S[i] = mfma_bf16(__builtin_bit_cast(bf16x8, kop0[i]), Vd0, S[i]);
        Vd1 = partner_vd();
      } else {
        const bf16x8 Vd0 = partner_vd();
#pragma unroll
        for (int i = 0; i < KTH; ++i) S[i] = mfma_bf16(__builtin_bit_cast(bf16x8, kop0[i]), Vd0, S[i]);
        Vd1 = __builtin_bit_cast(bf16x8, pd);
      }
#pragma unroll
      for (int i = 0; i < KTH; ++i) S[i] = mfma_bf16(__builtin_bit_cast(bf16x8, kop1[i]), Vd1, S[i]);
      if constexpr (CONTEST) {
#pragma unroll
        for (int i = 0; i < KTH; ++i) {
          if constexpr (FULL) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const unsigned hw = hdp[i][rr >> 1];
              const float hd = (rr & 1) ? bf16_hi(hw) : bf16_lo(hw);
              S[i][rr] = bf16_rnd(hd + bf16_rnd(f16_nan_to_num(bf16_rnd(S[i][rr]))));
            }
          } else {
#pragma unroll
            for (int rr = 0; rr < 2; ++rr)
              Sp[i][rr] = contest_combine_pair(S[i][2 * rr], S[i][2 * rr + 1], hdf[i][2 * rr], hdf[i][2 * rr + 1]);
          }
        }
      }
      stage_state((c + 1) % 3);   // bf16(-S_{c+1}): MM1 of chunk c+1 and the h snapshot
      wait_lgkm0();
      block_barrier();   // B_c
    };
    for (int c = 0; c < NC; ++c) chunk_step(c);

    if constexpr (NUM == 1) {
#pragma unroll
      for (int i = 0; i < KTH; ++i)
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          S[i][2 * rr] = bf16_lo(Sp[i][rr]);
          S[i][2 * rr + 1] = bf16_hi(Sp[i][rr]);
        }
      bool bad = false;
#pragma unroll
      for (int i = 0; i < KTH; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) bad |= S[i][rr] != S[i][rr];
      if (__any(bad) && lane == 0) p.redo[(int64_t)tk.n * p.H + tk.head] = p.epoch;
    }
    if (p.final_state != nullptr) {
      const int64_t base = (int64_t)tk.n * p.sf_n + (int64_t)tk.head * p.sf_h;
#pragma unroll
      for (int i = 0; i < KTH; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int krow = krow_of(i, rr);
          const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
          if (krow >= p.K) continue;
          if (p.final_f32) ((float*)p.final_state)[off] = S[i][rr];
          else ((__bf16*)p.final_state)[off] = (__bf16)S[i][rr];
        }
    }
   } else {
    // ------------------------------------------------------------------ compute wave
    const int g = lane >> 4, n = lane & 15;
    const int vcol = vbase + 16 * wave + n;      // value column owned by this lane
    f32x4 S[KT];

    if (p.h0 != nullptr) {
      const int64_t base = (int64_t)tk.n * p.sh0_n + (int64_t)tk.head * p.sh0_h;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
          const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
          S[kt][r] = krow >= p.K ? 0.f
                     : p.h0_f32 ? ((const float*)p.h0)[off]
                                : bf16_lo(((const unsigned short*)p.h0)[off]);
          if constexpr (CONTEST) S[kt][r] = bf16_rnd(S[kt][r]);   // the state is bf16
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) S[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // contest fast pass: the bf16 state kept as packed pairs between chunks
    unsigned Sp[NUM == 1 ? KT : 1][2];
    if constexpr (NUM == 1)
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 2; ++r) Sp[kt][r] = pack_bf16x2(S[kt][2 * r], S[kt][2 * r + 1]);
    block_barrier();   // P: stage 0 ready

    // One chunk; the stage (c % STAGES) and the staging buffer (c % 2) are template constants,
    // so every LDS address below is a fixed offset from a per-lane base (the chunk loop is
    // unrolled over a whole cycle of both).
    auto chunk_step = [&](const int c, auto st_tag, auto par_tag) {
      constexpr int st = decltype(st_tag)::value;
      constexpr int par = decltype(par_tag)::value;
      const char* sbase = smem + st * L::STAGE_BYTES;
      const lds_char* stage = (const lds_char*)sbase;
      const float* gam = (const float*)(sbase + L::G_OFF);
      const int e = n >> 2, q = n & 3;

      // Phase 1: every LDS read MM1 and the epilogue need (a, gamma, U, W operands) is issued
      // up front, so their latency hides under the bf16 conversion and the first MFMAs.
      const float a = gam[64];
      f32x4 gm[2][NUM == 1 ? 1 : 2];  // gamma of tokens 32 tb + 8 g + 4 hh + (0..3)
      u32x4 g16[2];                   // the contest fast pass has them as fp16 pairs
#pragma unroll
      for (int tb = 0; tb < 2; ++tb) {
        if constexpr (NUM == 1) {
          g16[tb] = *(const u32x4*)((const char*)gam + 2 * (32 * tb + 8 * g));
        } else {
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) gm[tb][hh] = *(const f32x4*)(gam + 32 * tb + 8 * g + 4 * hh);
        }
      }
      // U rows sigma(tt, 4g + r), column 16*wave + n, by a transposed read: source lane 4e+q
      // addresses row t0+e, columns 16*wave + 4q .. +3.
      u32x2 uraw[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int t0 = 32 * (tt >> 1) + 8 * g + 4 * (tt & 1);
        const lds_char* up = stage + L::U_OFF + ((t0 + e) * VT + 16 * wave + 4 * q) * 2;
        uraw[tt] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)up));
      }
      // W operands: tile tt row i = n holds token sigma(tt, n); contraction slice 8g..8g+7 of
      // k-block kb is LDS piece 4kb + g of that row.
      u32x4 wop[4][KB];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const int row = 32 * (tt >> 1) + 8 * e + 4 * (tt & 1) + q;
        const u32x4* wrow = (const u32x4*)(sbase + L::W_OFF) + row * P;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) wop[tt][kb] = wrow[(4 * kb + g) ^ swz_w<P>(row)];
      }
      // bf16(-S): the MM1 B operands (so MM1 accumulates U - W S onto U) and the h snapshot,
      // staged sign-flipped (the store wave flips it back).  The contest fast pass uses +S: its
      // MM1 starts from zero and the epilogue subtracts, so nothing is flipped there.
      u32x4 Sw[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if constexpr (NUM == 1) {
          Sw[kb] = u32x4{Sp[2 * kb][0], Sp[2 * kb][1], Sp[2 * kb + 1][0], Sp[2 * kb + 1][1]};   // +S
        } else {
          Sw[kb][0] = pack_bf16x2(-S[2 * kb][0], -S[2 * kb][1]);
          Sw[kb][1] = pack_bf16x2(-S[2 * kb][2], -S[2 * kb][3]);
          Sw[kb][2] = pack_bf16x2(-S[2 * kb + 1][0], -S[2 * kb + 1][1]);
          Sw[kb][3] = pack_bf16x2(-S[2 * kb + 1][2], -S[2 * kb + 1][3]);
        }
      }
      {
        u32x4* ss = (u32x4*)(smem + L::SS_OFF + par * L::SS_BYTES);
        const int vrow = 16 * wave + n;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) ss[vrow * P + ((4 * kb + g) ^ swz_s<P>(vrow))] = Sw[kb];
      }
      f32x4 acc[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
        acc[tt] = CONTEST ? f32x4{0.f, 0.f, 0.f, 0.f}   // W S is its own bf16 GEMM
                          : f32x4{bf16_lo(uraw[tt][0]), bf16_hi(uraw[tt][0]), bf16_lo(uraw[tt][1]), bf16_hi(uraw[tt][1])};
      __builtin_amdgcn_sched_barrier(0);

      // Phase 2: MM1 acc[tt] = U_tt + W_tt bf16(-S), four independent chains issued k-block
      // major, with the state decay S *= a on the VALU and the token-block-0 K^T operand reads
      // (two transposed reads each: lane (g, i) gets K[32tb + 8g + 4half + (0..3)][pi(kt, i)])
      // slotted between the MFMAs.
      auto read_kop = [&](int tb, u32x4* kop) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const int kb = kt >> 1, hh = kt & 1;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int row = 32 * tb + 8 * g + 4 * half + e;
            const int piece = (4 * kb + q) ^ swz_k<P>(row);
            const lds_char* kp = stage + L::K_OFF + (row * P + piece) * 16 + 8 * hh;
            const u32x2 kw = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)kp));
            kop[kt][2 * half] = kw[0];
            kop[kt][2 * half + 1] = kw[1];
          }
        }
      };
      u32x4 kop0[KT], kop1[KT];
      unsigned hdp[FULL ? KT : 1][2];      // contest, full pass: bf16(hd) pairs of the decayed state
      float hdf[NUM == 1 ? KT : 1][4];     // contest, fast pass: bf16(hd) as floats
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
          acc[tt] = mfma_bf16(__builtin_bit_cast(bf16x8, wop[tt][kb]), __builtin_bit_cast(bf16x8, Sw[kb]), acc[tt]);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        if constexpr (FULL) {
          // hd = f16sat(f16sat(S) a), kept as bf16(hd); S becomes the K^T Vd accumulator
#pragma unroll
          for (int r = 0; r < 2; ++r)
            hdp[kt][r] = pack_bf16x2(f16_sat(f16_sat(S[kt][2 * r]) * a), f16_sat(f16_sat(S[kt][2 * r + 1]) * a));
          S[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else if constexpr (CONTEST) {
          // fast pass: plain fp16 roundings (exact while |S| <= 65504 and 0 <= a <= 1), as
          // packed fp16 products of fp16(S) and the fp16 decay a
          const h16x2 a16 = to_h16x2(a, a);
#pragma unroll
          for (int r = 0; r < 2; ++r) contest_decay_pair(Sp[kt][r], a16, hdf[kt][2 * r], hdf[kt][2 * r + 1]);
          S[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else {
          S[kt] = S[kt] * a;
        }
      }
      read_kop(0, kop0);
#pragma unroll
      for (int i = 0; i < 4 * KB; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, (2 * KT + 4 * KB - 1) / (4 * KB), 0);   // VALU
        __builtin_amdgcn_sched_group_barrier(0x100, (4 * KT + 4 * KB - 1) / (4 * KB), 0);   // DS read
      }
      __builtin_amdgcn_sched_barrier(0);

      // Phase 3: epilogue of token block 0 (v_new staging, Vd = bf16(Vn * gamma)).
      u32x4* sv = (u32x4*)(smem + L::SV_OFF + par * L::SV_BYTES);
      const int vrow = 16 * wave + n;
      // Contest: the saturating casts in the full pass; plain fp16 roundings in the fast pass,
      // which give the same values while v16 = fp16(u - ws) is finite (a NaN or infinite ws, or
      // a u beyond the fp16 range, makes it inf or NaN) and the gates are at most 1.
      auto epilogue = [&](int tb) -> bf16x8 {
        u32x4 pv, pd;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int hh = j >> 1, r = 2 * (j & 1);
          const float v0 = acc[2 * tb + hh][r], v1 = acc[2 * tb + hh][r + 1];
          if constexpr (CONTEST) {
            // acc = -W S: ws = nan_to_num(fp16(bf16(W S))), v16 = f16sat(f16sat(u) - ws)
            const u32x2 ur = uraw[2 * tb + hh];
            const float u0 = r == 0 ? bf16_lo(ur[0]) : bf16_lo(ur[1]);
            const float u1 = r == 0 ? bf16_hi(ur[0]) : bf16_hi(ur[1]);
            if constexpr (FULL) {
              const float x0 = f16_sat(f16_sat(u0) - f16_nan_to_num(-bf16_rnd(v0)));
              const float x1 = f16_sat(f16_sat(u1) - f16_nan_to_num(-bf16_rnd(v1)));
              pv[j] = pack_bf16x2(x0, x1);
              pd[j] = pack_bf16x2(f16_sat(x0 * gm[tb][hh][r]), f16_sat(x1 * gm[tb][hh][r + 1]));
            } else {
              // v16 = fp16(u) - fp16(bf16(W S)) = fp16(u) + fp16(bf16(-acc)), acc = +W S (the fast
              // pass stages +S; the negation is a source modifier of the bf16 conversion); v16 is
              // staged as fp16 and rounded to bf16 by the store waves
              const h16x2 x16 = to_h16x2(u0, u1) + bf16x2_to_h16x2(pack_bf16x2(-v0, -v1));
              pv[j] = __builtin_bit_cast(unsigned, x16);
              pd[j] = h16x2_to_bf16x2(x16 * as_h16x2(g16[tb][j]));
            }
          } else {
            pv[j] = pack_bf16x2(v0, v1);
            pd[j] = pack_bf16x2(v0 * gm[tb][hh][r], v1 * gm[tb][hh][r + 1]);
          }
        }
        sv[vrow * 8 + ((4 * tb + g) ^ swz_v(vrow))] = pv;
        return __builtin_bit_cast(bf16x8, pd);
      };
      const bf16x8 Vd0 = epilogue(0);
      __builtin_amdgcn_sched_barrier(0);

      // Phase 4: MM2 of token block 0, with the block-1 K^T reads and epilogue slotted in.
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) S[kt] = mfma_bf16(__builtin_bit_cast(bf16x8, kop0[kt]), Vd0, S[kt]);
      read_kop(1, kop1);
      const bf16x8 Vd1 = epilogue(1);
#pragma unroll
      for (int i = 0; i < KT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // 1 MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);   // DS read
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
      }
      __builtin_amdgcn_sched_barrier(0);

      // Phase 5: MM2 of token block 1.
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) S[kt] = mfma_bf16(__builtin_bit_cast(bf16x8, kop1[kt]), Vd1, S[kt]);
      if constexpr (CONTEST) {
        // S = bf16(bf16(hd) + bf16(nan_to_num(fp16(bf16(K^T Vd))))).  nan_to_num changes only a
        // NaN, which the fast pass leaves in the new state (seen in the next h snapshot, or in
        // the final state below).
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          if constexpr (FULL) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const unsigned hw = hdp[kt][r >> 1];
              const float hd = (r & 1) ? bf16_hi(hw) : bf16_lo(hw);
              S[kt][r] = bf16_rnd(hd + bf16_rnd(f16_nan_to_num(bf16_rnd(S[kt][r]))));
            }
          } else {
#pragma unroll
            for (int r = 0; r < 2; ++r)
              Sp[kt][r] = contest_combine_pair(S[kt][2 * r], S[kt][2 * r + 1], hdf[kt][2 * r], hdf[kt][2 * r + 1]);
          }
        }
      }
      wait_lgkm0();
      block_barrier();   // B_c
    };
    constexpr int UNROLL = (STAGES % 2 == 0) ? STAGES : 2 * STAGES;
    for (int c0 = 0; c0 < NC; c0 += UNROLL) {
      static_for<0, UNROLL>([&](auto i) {
        constexpr int I = decltype(i)::value;
        if (c0 + I < NC)
          chunk_step(c0 + I, std::integral_constant<int, I % STAGES>{}, std::integral_constant<int, I % 2>{});
      });
    }

    if constexpr (NUM == 1) {
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          S[kt][2 * r] = bf16_lo(Sp[kt][r]);
          S[kt][2 * r + 1] = bf16_hi(Sp[kt][r]);
        }
      bool bad = false;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) bad |= S[kt][r] != S[kt][r];
      if (__any(bad) && lane == 0) p.redo[(int64_t)tk.n * p.H + tk.head] = p.epoch;
    }
    if (p.final_state != nullptr) {
      const int64_t base = (int64_t)tk.n * p.sf_n + (int64_t)tk.head * p.sf_h;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
          const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
          if (krow >= p.K) continue;
          if (p.final_f32) ((float*)p.final_state)[off] = S[kt][r];
          else ((__bf16*)p.final_state)[off] = (__bf16)S[kt][r];
        }
    }
   }
  } else if (wave >= NCWT + L::NSW && wave < NCWT + L::NSW + NLW) {
    // ------------------------------------------------------------------ load waves
    // The tile DMAs of a chunk are dealt round-robin over the NLW load waves (instruction
    // i goes to wave i % NLW), so each wave's vmcnt covers only its share and more loads are
    // in flight per CU.  The g rows are not theirs: the gate wave loads them into registers.
    const int lw = wave - NCWT - L::NSW;
    const __bf16* kbase = (const __bf16*)p.k + tk.b * p.sk_b + (int64_t)hk * p.sk_h;
    const __bf16* wbase = (const __bf16*)p.w + tk.b * p.sw_b + (int64_t)tk.head * p.sw_h;
    const __bf16* ubase = (const __bf16*)p.u + tk.b * p.su_b + (int64_t)tk.head * p.su_h + vbase;

    // Per-lane byte offsets (within a chunk) of the 16-byte pieces each DMA instruction moves,
    // hoisted out of the chunk loop: instruction m, lane -> LDS piece 64m + lane = (row r,
    // slot s), filled from global piece (r, s ^ swizzle(r)).  With one scalar base per tile
    // and chunk, every DMA is saddr + voffset (the host guarantees 64 rows span < 2 GiB).
    constexpr int RPI = 64 / P;                 // rows per DMA instruction
    constexpr int PU = VT / 8;                  // U pieces per row
    const int lrow = lane / P, lcol = lane % P;
    const int64_t stw = p.sw_t * 2, stk = p.sk_t * 2, stu = p.su_t * 2;   // row strides in bytes
    // A key dim K below KD: the pieces at or past K/8 of a row are padding.  Their lanes load
    // piece 0 of the row instead (in bounds, same cache line as a real piece), and once the
    // chunk has landed the load wave overwrites those LDS slots with zeros (zero_padding).
    const int kp = p.K / 8;
    const bool padded = kp < P;
    uint32_t woff[L::DMA_W], koff[L::DMA_W], uoff[L::DMA_U];
#pragma unroll
    for (int m = 0; m < L::DMA_W; ++m) {
      const int r = m * RPI + lrow;
      const int gw = lcol ^ swz_w<P>(r), gk = lcol ^ swz_k<P>(r);
      woff[m] = (uint32_t)(r * stw) + 16u * (uint32_t)(gw < kp ? gw : 0);
      koff[m] = (uint32_t)(r * stk) + 16u * (uint32_t)(gk < kp ? gk : 0);
    }
#pragma unroll
    for (int m = 0; m < L::DMA_U; ++m) {
      const int qd = 64 * m + lane;
      uoff[m] = (uint32_t)((qd / PU) * stu) + 16u * (uint32_t)(qd % PU);
    }
    const char* wsrc = (const char*)wbase;
    const char* ksrc = (const char*)kbase;
    const char* usrc = (const char*)ubase;
    const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_char*)smem);

    // One load wave's schedule; LW is its index (compile-time, selects its DMA share).
    auto run_loader = [&](auto lw_tag) {
      constexpr int LW = decltype(lw_tag)::value;
      // Issue this wave's share of the W, K, U tiles of chunk c into stage st.  Every load is a direct-to-LDS DMA written as
      // inline asm: the compiler then tracks none of them, and the explicit in-order vmcnt
      // waits below are the only waits (its own tracking cannot express more than 63
      // outstanding loads and would drain the whole pipeline instead).  A partial (last) chunk takes a masked path: rows at or
      // past the sequence end are zero-filled in LDS instead of loaded (the masked loads with
      // other=0 of the reference kernel).
      auto issue = [&](int c, int st) {
        const int64_t t0 = tk.bos + (int64_t)c * kChunk;
        const int64_t rem = tk.len - (int64_t)c * kChunk;
        const int len = rem < kChunk ? (int)rem : kChunk;
        const uint32_t lbase = lds0 + (uint32_t)(st * L::STAGE_BYTES);
        char* sbase = smem + st * L::STAGE_BYTES;
        const char* wchunk = wsrc + t0 * stw;
        const char* kchunk = ksrc + t0 * stk;
        const char* uchunk = usrc + t0 * stu;
        if (len == kChunk) {
#pragma unroll
          for (int m = 0; m < L::DMA_W; ++m)
            if ((m % NLW) == LW) dma_b128(wchunk, woff[m], lbase + L::W_OFF + 1024 * m);
#pragma unroll
          for (int m = 0; m < L::DMA_W; ++m)
            if (((L::DMA_W + m) % NLW) == LW) dma_b128(kchunk, koff[m], lbase + L::K_OFF + 1024 * m);
#pragma unroll
          for (int m = 0; m < L::DMA_U; ++m)
            if (((2 * L::DMA_W + m) % NLW) == LW) dma_b128(uchunk, uoff[m], lbase + L::U_OFF + 1024 * m);
        } else {
#pragma unroll
          for (int m = 0; m < L::DMA_W; ++m) {
            if ((m % NLW) != LW) continue;
            if (m * RPI + lrow < len) dma_b128(wchunk, woff[m], lbase + L::W_OFF + 1024 * m);
            else *(u32x4*)(sbase + L::W_OFF + 1024 * m + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int m = 0; m < L::DMA_W; ++m) {
            if (((L::DMA_W + m) % NLW) != LW) continue;
            if (m * RPI + lrow < len) dma_b128(kchunk, koff[m], lbase + L::K_OFF + 1024 * m);
            else *(u32x4*)(sbase + L::K_OFF + 1024 * m + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
          }
#pragma unroll
          for (int m = 0; m < L::DMA_U; ++m) {
            if (((2 * L::DMA_W + m) % NLW) != LW) continue;
            if ((64 * m + lane) / PU < len) dma_b128(uchunk, uoff[m], lbase + L::U_OFF + 1024 * m);
            else *(u32x4*)(sbase + L::U_OFF + 1024 * m + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
          }
        }
      };

      // Zero this wave's padding slots of the W and K tiles in stage st, once its DMAs of the
      // chunk there have landed (each wave zeroes the slots of its own DMA instructions).
      auto zero_padding = [&](int st) {
        if (!padded) return;
        char* sbase = smem + st * L::STAGE_BYTES;
#pragma unroll
        for (int m = 0; m < L::DMA_W; ++m) {
          const int r = m * RPI + lrow;
          if ((m % NLW) == LW && (lcol ^ swz_w<P>(r)) >= kp)
            *(u32x4*)(sbase + L::W_OFF + 1024 * m + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
          if (((L::DMA_W + m) % NLW) == LW && (lcol ^ swz_k<P>(r)) >= kp)
            *(u32x4*)(sbase + L::K_OFF + 1024 * m + 16 * lane) = u32x4{0u, 0u, 0u, 0u};
        }
      };

      // Schedule.  D = STAGES - 1 chunks are in flight ahead of the compute waves.  Each loop
      // iteration first issues chunk c+D (into the stage the last barrier freed), then waits
      // for chunk c+1.  vmcnt completes loads in order, so that wait is "at most D-1 full
      // chunk groups outstanding" while only full groups follow chunk c+1, and vmcnt(0) once
      // the (possibly shorter) last group of the sequence is among them (cgdr_schedule.h).
      constexpr int D = STAGES - 1;
      constexpr int PER_CHUNK = L::template dma_per_chunk<LW>();
      static_assert(D >= 1, "at least one chunk of prefetch");
      static_assert((D - 1) * PER_CHUNK <= 63, "prefetch depth exceeds the vmcnt range");
      constexpr int STEADY_VM = (D - 1) * PER_CHUNK;

      // Prologue: chunks 0 .. D-1 issued; chunk 0 landed here.
      if (NC > 0) {
        for (int j = 0; j < D && j < NC; ++j) issue(j, j);
        if (sched::prologue_allowance(D, NC) > 0) wait_vm<STEADY_VM>();
        else wait_vm<0>();
        zero_padding(0);
      }
      wait_lgkm0();
      block_barrier();   // P

      for (int c = 0; c < NC; ++c) {
        if (c + D < NC) issue(c + D, (c + D) % STAGES);
        if (c + 1 < NC) {
          if (sched::loop_allowance(c, D, NC) > 0) wait_vm<STEADY_VM>();
          else wait_vm<0>();
          zero_padding((c + 1) % STAGES);
        }
        wait_lgkm0();      // zero-fill writes of a partial chunk and of padding
        block_barrier();   // B_c
      }
    };
    if constexpr (NLW == 1) {
      run_loader(std::integral_constant<int, 0>{});
    } else if constexpr (NLW == 2) {
      if (lw == 0) run_loader(std::integral_constant<int, 0>{});
      else run_loader(std::integral_constant<int, 1>{});
    } else {
      static_assert(NLW == 4, "1, 2 or 4 load waves");
      if (lw == 0) run_loader(std::integral_constant<int, 0>{});
      else if (lw == 1) run_loader(std::integral_constant<int, 1>{});
      else if (lw == 2) run_loader(std::integral_constant<int, 2>{});
      else run_loader(std::integral_constant<int, 3>{});
    }
  } else if (wave >= NCWT && wave < NCWT + L::NSW) {
    // ------------------------------------------------------------------ store waves
    // h snapshot and v_new of a chunk, from the LDS staging buffers: each 16-lane block takes
    // units of (16 rows x 8 value columns); two transposed reads give a lane 8 consecutive
    // value columns of one row, stored as one 16-byte write.
    const int sw = wave - NCWT;   // this store wave takes store instructions m % NSW == sw
    const int blk = lane >> 4, i = lane & 15;
    const int e = i >> 2, q = i & 3;
    __bf16* hbase = (__bf16*)p.h + tk.b * p.sh_b + (int64_t)tk.head * p.sh_h + vbase;
    __bf16* vbase_ptr = p.v_new == nullptr ? nullptr
                       : (__bf16*)p.v_new + tk.b * p.sv_b + (int64_t)tk.head * p.sv_h + vbase;
    // contest fast pass: largest |h| and |v_new| seen.  The fast pass is exact while every state
    // entering a chunk (the h snapshot, bf16 = S) is within +-65504 and every v_new is finite;
    // both hold when no bf16 exceeds 65280 (0x477f): the next bf16 is 65536.
    unsigned amax = 0;

    // One chunk's stores; SW (this store wave's index, a compile-time constant) selects its
    // share: h instruction m when m % NSW == SW, v_new instruction m when (MH + m) % NSW == SW.
    // All of the share's LDS reads are issued first and awaited once, then the stores.
    auto store_chunk = [&](int c, auto sw_tag) {
      constexpr int SW = decltype(sw_tag)::value;
      constexpr int UNITS_H = (KD / 16) * (VT / 8), MH = UNITS_H / 4;   // 16-byte row stores of h
      constexpr int UNITS_V = 4 * (VT / 8), MV = UNITS_V / 4;           // and of v_new
      const int len = (int)((tk.len - (int64_t)c * kChunk) < kChunk ? (tk.len - (int64_t)c * kChunk) : kChunk);
      const char* ss = smem + L::SS_OFF + (RS == 1 ? (c & 1) : c % 3) * L::SS_BYTES;
      const char* sv = smem + L::SV_OFF + (c & 1) * L::SV_BYTES;
      const bool with_v = vbase_ptr != nullptr || NUM == 1;
      u32x2 hx[MH][2], vx[MV][2];
#pragma unroll
      for (int m = 0; m < MH; ++m) {
        if (m % L::NSW != SW) continue;
        const int unit = 4 * m + blk;
        const int k0 = 16 * (unit / (VT / 8)), v0 = 8 * (unit % (VT / 8));
        const int kk = k0 + 4 * q;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const int vrow = v0 + 4 * half + e;
          const int piece = (kk >> 3) ^ swz_s<P>(vrow);
          const lds_char* sp = (const lds_char*)ss + (vrow * P + piece) * 16 + 8 * ((kk >> 2) & 1);
          hx[m][half] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)sp));
        }
      }
      if (with_v) {
#pragma unroll
        for (int m = 0; m < MV; ++m) {
          if ((MH + m) % L::NSW != SW) continue;
          const int unit = 4 * m + blk;
          const int t0 = 16 * (unit / (VT / 8)), v0 = 8 * (unit % (VT / 8));
          const int tt = t0 + 4 * q;
#pragma unroll
          for (int half = 0; half < 2; ++half) {
            const int vrow = v0 + 4 * half + e;
            const int piece = (tt >> 3) ^ swz_v(vrow);
            const lds_char* sp = (const lds_char*)sv + (vrow * 8 + piece) * 16 + 8 * ((tt >> 2) & 1);
            vx[m][half] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)sp));
          }
        }
      }
      __bf16* hdst = hbase + (tk.boh + c) * p.sh_c;
#pragma unroll
      for (int m = 0; m < MH; ++m) {
        if (m % L::NSW != SW) continue;
        const int unit = 4 * m + blk;
        const int k0 = 16 * (unit / (VT / 8)), v0 = 8 * (unit % (VT / 8));
        u32x4 hv;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          // staged as bf16(-S), or as bf16(+S) by the contest fast pass
          hv[2 * half] = NUM == 1 ? hx[m][half][0] : hx[m][half][0] ^ 0x80008000u;
          hv[2 * half + 1] = NUM == 1 ? hx[m][half][1] : hx[m][half][1] ^ 0x80008000u;
          if constexpr (NUM == 1) amax = pk_absmax_bf16(pk_absmax_bf16(amax, hx[m][half][0]), hx[m][half][1]);
        }
        if (k0 < p.K) *(u32x4*)(hdst + (int64_t)(k0 + i) * p.V + v0) = hv;   // rows >= K: padding
      }
      if (with_v) {
        __bf16* vdst = vbase_ptr == nullptr ? nullptr : vbase_ptr + (tk.bos + (int64_t)c * kChunk) * p.sv_t;
#pragma unroll
        for (int m = 0; m < MV; ++m) {
          if ((MH + m) % L::NSW != SW) continue;
          const int unit = 4 * m + blk;
          const int t0 = 16 * (unit / (VT / 8)), v0 = 8 * (unit % (VT / 8));
          u32x4 vv = {vx[m][0][0], vx[m][0][1], vx[m][1][0], vx[m][1][1]};
          if constexpr (NUM == 1) {
            // the fast pass stages v16 as fp16 pairs: v_new = bf16(v16)
            const unsigned w0 = vx[m][0][0], w1 = vx[m][0][1], w2 = vx[m][1][0], w3 = vx[m][1][1];
            vv = u32x4{h16x2_to_bf16x2(as_h16x2(w0)), h16x2_to_bf16x2(as_h16x2(w1)),
                       h16x2_to_bf16x2(as_h16x2(w2)), h16x2_to_bf16x2(as_h16x2(w3))};
          }
          if (t0 + i < len) {
            if (vbase_ptr != nullptr) *(u32x4*)(vdst + (int64_t)(t0 + i) * p.sv_t + v0) = vv;
            if constexpr (NUM == 1)
              amax = pk_absmax_bf16(pk_absmax_bf16(pk_absmax_bf16(pk_absmax_bf16(amax, vv[0]), vv[1]), vv[2]), vv[3]);
          }
        }
      }
    };

    // Without helper workgroups, store wave 0 also touches chunk c+prefetch into L2
    // (l2_touch) at the start of iteration c.  Nothing waits on those touches until exit.
    const int pf = p.prefetch;
    const bool touching = sw == 0 && pf > 0 && !p.helpers;
    auto prefetch = [&](int j) {
      if (!touching || j >= NC || tk.len - (int64_t)j * kChunk < kChunk) return;
      l2_touch(j);
    };
    if (touching) l2_touch_setup();
    for (int j = 1; j < pf; ++j) prefetch(j);
    block_barrier();   // P
    auto run_stores = [&](auto sw_tag) {
      constexpr int SW = decltype(sw_tag)::value;
      for (int c = 0; c < NC; ++c) {
        prefetch(c + pf);
        if (c >= 1) store_chunk(c - 1, sw_tag);
        wait_lgkm0();
        block_barrier();   // B_c
        if (SW == 0 && p.helpers && lane == 0)
          __hip_atomic_store(p.progress + task_id * kProgressStride,
                             (int)(((unsigned)p.epoch << 24) | (unsigned)(c + 1)), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
      if (NC > 0) store_chunk(NC - 1, sw_tag);
    };
    if (sw == 0) run_stores(std::integral_constant<int, 0>{});
    else if constexpr (L::NSW >= 2) {
      if (sw == 1) run_stores(std::integral_constant<int, 1>{});
      else if constexpr (L::NSW == 4) {
        if (sw == 2) run_stores(std::integral_constant<int, 2>{});
        else run_stores(std::integral_constant<int, 3>{});
      }
    }
    if (touching) wait_vm<0>();   // the touches write this workgroup's LDS: drain them
    if constexpr (NUM == 1)
      if (__any((amax & 0x7fffu) > 0x477fu || ((amax >> 16) & 0x7fffu) > 0x477fu) && lane == 0)
        p.redo[(int64_t)tk.n * p.H + tk.head] = p.epoch;
  } else if (wave == NCWT + L::NSW + NLW) {
    // ------------------------------------------------------------------ gate wave
    // Loads the raw g rows itself, with ordinary loads into registers two chunks ahead, and
    // turns them into the gate factors of chunk c+1 during iteration c (read by the compute
    // waves after barrier B_c).  The row of chunk c+2 is issued before the factors of chunk
    // c+1 are computed, so the only wait is for a load issued one iteration earlier.  Rows
    // past the sequence end repeat its last row.  (Keeping the g rows out of the load waves'
    // DMA stream matters: a 256-byte row in that stream cost as much as a quarter of a tile.)
    const float* gsrc = has_g ? p.g + tk.b * p.sg_b + (int64_t)tk.head * p.sg_h : nullptr;
    auto graw = [&](int j) -> float {
      if (gsrc == nullptr || j >= NC) return 0.f;
      const int64_t rem = tk.len - (int64_t)j * kChunk;
      const int len = rem < kChunk ? (int)rem : kChunk;
      return gsrc[(tk.bos + (int64_t)j * kChunk + (lane < len ? lane : len - 1)) * p.sg_t];
    };
    float g_next = graw(1);
    if (NC > 0) gates(0, 0, graw(0));
    wait_lgkm0();
    block_barrier();   // P
    for (int c = 0; c < NC; ++c) {
      const float g_after = graw(c + 2);
      if (c + 1 < NC) gates(c + 1, (c + 1) % STAGES, g_next);
      g_next = g_after;
      wait_lgkm0();
      block_barrier();   // B_c
    }
    if constexpr (NUM == 1)
      if (__any(gbad) && lane == 0) p.redo[(int64_t)tk.n * p.H + tk.head] = p.epoch;
  }
}

// =============================================================================================
// g relayout: [B, T, H] (any strides) -> head-major [B, H, T] in the workspace, so that the
// g row of one chunk of one head is 256 contiguous bytes (4 cache lines) instead of 64 rows of
// a token-major array (64 cache lines per chunk and workgroup).  One 64-token x 64-head tile
// per workgroup, transposed through LDS: reads coalesced along heads, writes along tokens.
// (static: each translation unit that includes this header gets its own copy)
static __global__ void __launch_bounds__(256)
cgdr_g_head_major_kernel(const float* __restrict__ g, float* __restrict__ gt, int64_t T, int64_t H,
                         int64_t sg_b, int64_t sg_t, int64_t sg_h) {
  __shared__ float tile[64][65];
  const int64_t t0 = (int64_t)blockIdx.x * 64, h0 = (int64_t)blockIdx.y * 64, b = blockIdx.z;
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int tt = i >> 6, hh = i & 63;
    if (t0 + tt < T && h0 + hh < H) tile[tt][hh] = g[b * sg_b + (t0 + tt) * sg_t + (h0 + hh) * sg_h];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 64 * 64; i += 256) {
    const int hh = i >> 6, tt = i & 63;
    if (t0 + tt < T && h0 + hh < H) gt[(b * H + h0 + hh) * T + t0 + tt] = tile[tt][hh];
  }
}

// =============================================================================================
// fp32 kernel (fp32 k/w/u/h/v_new): same task decomposition and the same tile orderings
// (pi, sigma) with v_mfma_f32_16x16x4_f32, whose operands are one element per lane, so no
// transposed reads are needed.  Four waves per workgroup; all four load chunk c+1 into
// registers (16-byte loads) while chunk c is computed, and store it to LDS after the chunk's
// barrier.  It is the exact-arithmetic path (fp32 products, fp32 accumulation).
// RSF = 1: waves 0 .. NCW-1 compute, one per 16 value columns.  RSF > 1 (NCW * RSF <= 4): wave
// (j, r) = (wave % NCW, wave / NCW) holds state rows KD/RSF r .. KD/RSF (r+1) - 1 of column
// block j and runs MM1 for token tiles 4/RSF r .. 4/RSF (r+1) - 1; the full state of a column
// block reaches MM1 through an fp32 staging buffer, and Vd of all 64 tokens reaches MM2 through
// another, with one more barrier per chunk.  Every accumulation chain keeps its order (MM1:
// k-blocks in order; MM2: a S, then token tiles in order), so the results are the RSF = 1
// results bit for bit.
// =============================================================================================

template <int KD, int NCW, int RSF = 1>
struct F32Layout {
  static constexpr int VT = 16 * NCW;
  static constexpr int WP = KD + 4;     // padded row pitch (floats)
  static constexpr int W_OFF = 0;
  static constexpr int K_OFF = 64 * WP * 4;
  static constexpr int U_OFF = 2 * 64 * WP * 4;
  static constexpr int G_OFF = U_OFF + 64 * (VT + 4) * 4;
  static constexpr int SSP = KD + 4;    // row split: state staging [VT columns][KD], padded
  static constexpr int SS_OFF = G_OFF + 80 * 4;
  static constexpr int SS_BYTES = RSF > 1 ? VT * SSP * 4 : 0;
  static constexpr int VDP = 64 + 4;    // row split: Vd staging [VT columns][64 tokens], padded
  static constexpr int VD_OFF = SS_OFF + SS_BYTES;
  static constexpr int VD_BYTES = RSF > 1 ? VT * VDP * 4 : 0;
  static constexpr int LDS_BYTES = VD_OFF + VD_BYTES;
  static constexpr int THREADS = 256;                 // four waves load; NCW of them compute
  static constexpr int PW = 64 * KD / 4 / THREADS;    // 16-byte pieces per thread of the W (and K) tile
  static constexpr int PU = 64 * VT / 4 / THREADS;    // ... of the U tile
};

// The fp32 row split needs whole 16-row state tiles per wave and at most four compute waves,
// and its staging buffers must fit beside the tiles (K up to 128).
template <int KD, int NCW, int RSF>
constexpr bool f32_config_ok() {
  return RSF == 1 || (NCW * RSF <= 4 && (KD / 16) % RSF == 0 && KD <= 128 &&
                      F32Layout<KD, NCW, RSF>::LDS_BYTES <= 160 * 1024);
}

template <int KD, int NCW, int RSF = 1>
__global__ void __launch_bounds__(256)
cgdr_fwd_h_f32_kernel(const FwdHParams p) {
  using L = F32Layout<KD, NCW, RSF>;
  static_assert(f32_config_ok<KD, NCW, RSF>(), "fp32 row split configuration");
  constexpr int VT = L::VT, WP = L::WP, UP = VT + 4;
  constexpr int KT = KD / 16;
  constexpr int KTR = KT / RSF;         // own state tiles
  constexpr int TPW = 4 / RSF;          // own MM1 token tiles (RSF > 1)
  constexpr int SSP = L::SSP, VDP = L::VDP;
  __shared__ __attribute__((aligned(16))) float smem[L::LDS_BYTES / 4];
  float* Ws = smem + L::W_OFF / 4;
  float* Ks = smem + L::K_OFF / 4;
  float* Us = smem + L::U_OFF / 4;
  float* Gs = smem + L::G_OFF / 4;
  float* SSs = smem + L::SS_OFF / 4;
  float* VDs = smem + L::VD_OFF / 4;

  // wave index as a uniform value, so that the role branches below are scalar branches (every
  // barrier of the chunk loop stands outside them and is reached by every wave, idle ones too)
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int task_id = xcd_remap(blockIdx.x, gridDim.x, p.n_xcd);
  if (task_id >= p.n_tasks) return;
  const Task tk = decode_task(p, order_task(p, task_id));
  const int vbase = tk.vtile * VT;
  const int hk = tk.head / p.head_ratio;
  const int g = lane >> 4, n = lane & 15;
  const int cj = wave % NCW, rgrp = wave / NCW;   // column block, row group (RSF = 1: 0)
  const int vcol = vbase + 16 * cj + n;
  const int kt0 = KTR * rgrp;                   // first own state tile
  // float offsets of the lane's 4-row slice of state tile kt (state staging) and of the 4-token
  // slice of token tile tt (Vd staging)
  auto ss_at = [&](int kt) { return (16 * cj + n) * SSP + 32 * (kt >> 1) + 8 * g + 4 * (kt & 1); };
  auto vd_at = [&](int tt) { return (16 * cj + n) * VDP + 32 * (tt >> 1) + 8 * g + 4 * (tt & 1); };

  using E = float;   // element type of k/w/u/h/v_new
  const E* kb_ = (const E*)p.k + tk.b * p.sk_b + (int64_t)hk * p.sk_h;
  const E* wb_ = (const E*)p.w + tk.b * p.sw_b + (int64_t)tk.head * p.sw_h;
  const E* ub_ = (const E*)p.u + tk.b * p.su_b + (int64_t)tk.head * p.su_h + vbase;
  const float* gb_ = p.g == nullptr ? nullptr : p.g + tk.b * p.sg_b + (int64_t)tk.head * p.sg_h;
  E* hb_ = (E*)p.h + tk.b * p.sh_b + (int64_t)tk.head * p.sh_h;
  E* vb_ = p.v_new == nullptr ? nullptr : (E*)p.v_new + tk.b * p.sv_b + (int64_t)tk.head * p.sv_h;

  const bool computes = wave < NCW * RSF;   // uniform per wave
  f32x4 S[KTR];                             // own state tiles kt0 .. kt0 + KTR - 1
  if (computes && p.h0 != nullptr) {
    const int64_t base = (int64_t)tk.n * p.sh0_n + (int64_t)tk.head * p.sh0_h;
#pragma unroll
    for (int i = 0; i < KTR; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kt = kt0 + i;
        const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
        const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
        S[i][r] = krow >= p.K ? 0.f
                  : p.h0_f32 ? ((const float*)p.h0)[off] : bf16_lo(((const unsigned short*)p.h0)[off]);
      }
  } else {
#pragma unroll
    for (int i = 0; i < KTR; ++i) S[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if constexpr (RSF > 1)   // the state entering chunk 0, for MM1 (read after the first barrier)
    if (computes)
#pragma unroll
      for (int i = 0; i < KTR; ++i) *(f32x4*)(SSs + ss_at(kt0 + i)) = S[i];

  // Chunk c's tiles in registers: thread i holds 16-byte pieces i, i + 256, ... of each tile
  // (rows past the sequence end and key columns past K read as zero), and wave 0 the g row.
  const int tid = threadIdx.x;
  f32x4 rw[L::PW], rk[L::PW], ru[L::PU];
  float rg = 0.f;
  auto chunk_len = [&](int c) {
    const int64_t rem = tk.len - (int64_t)c * kChunk;
    return rem < kChunk ? (int)rem : kChunk;
  };
  auto fetch = [&](int c) {
    const int64_t t0 = tk.bos + (int64_t)c * kChunk;
    const int len = chunk_len(c);
#pragma unroll
    for (int i = 0; i < L::PW; ++i) {
      const int q = tid + L::THREADS * i, r = q / (KD / 4), c4 = 4 * (q % (KD / 4));
      const bool ok = r < len && c4 < p.K;
      rw[i] = ok ? *(const f32x4*)(wb_ + (t0 + r) * p.sw_t + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
      rk[i] = ok ? *(const f32x4*)(kb_ + (t0 + r) * p.sk_t + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < L::PU; ++i) {
      const int q = tid + L::THREADS * i, r = q / (VT / 4), c4 = 4 * (q % (VT / 4));
      ru[i] = r < len ? *(const f32x4*)(ub_ + (t0 + r) * p.su_t + c4) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    if (tid < 64) rg = (gb_ != nullptr && tid < len) ? gb_[(t0 + tid) * p.sg_t] : 0.f;
  };
  // K = 256: the tiles of the next chunk and the state do not fit the registers together, so
  // each chunk is loaded after its barrier instead of during the previous chunk
  constexpr bool PREFETCH = KD <= 128;
  if (PREFETCH && tk.nc > 0) fetch(0);

  for (int c = 0; c < tk.nc; ++c) {
    const int64_t t0 = tk.bos + (int64_t)c * kChunk;
    const int len = chunk_len(c);
    __syncthreads();   // the previous chunk's reads of the tiles are done
    if constexpr (!PREFETCH) fetch(c);
#pragma unroll
    for (int i = 0; i < L::PW; ++i) {
      const int q = tid + L::THREADS * i, r = q / (KD / 4), c4 = 4 * (q % (KD / 4));
      *(f32x4*)(Ws + r * WP + c4) = rw[i];
      *(f32x4*)(Ks + r * WP + c4) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < L::PU; ++i) {
      const int q = tid + L::THREADS * i, r = q / (VT / 4), c4 = 4 * (q % (VT / 4));
      *(f32x4*)(Us + r * UP + c4) = ru[i];
    }
    if (threadIdx.x < 64) {
      const int t = threadIdx.x;
      const float gv = rg;
      float gamma = t < len ? 1.f : 0.f, a = 1.f;
      if (gb_ != nullptr) {
        const float glast = __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(gv), len - 1));
        gamma = t < len ? safe_exp(glast - gv) : 0.f;
        a = expf(glast);
      }
      Gs[t] = gamma;
      if (t == 0) Gs[64] = a;
    }
    __syncthreads();
    if (PREFETCH && c + 1 < tk.nc) fetch(c + 1);   // in flight while chunk c is computed
    if constexpr (RSF == 1) {
      if (!computes) continue;
      // h snapshot (exact)
      {
        E* hdst = hb_ + (tk.boh + c) * p.sh_c;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
            if (krow < p.K) hdst[(int64_t)krow * p.V + vcol] = (E)S[kt][r];
          }
      }
      // MM1: acc[tt] = W S   (contraction slot g of step (kt, r) is k = pi(kt, 4g + r))
      f32x4 acc[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int row = 32 * (tt >> 1) + 8 * (n >> 2) + 4 * (tt & 1) + (n & 3);
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
          const int kcol = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1);
          const f32x4 wv = *(const f32x4*)(Ws + row * WP + kcol);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[tt] = mfma_f32(wv[r], S[kt][r], acc[tt]);
        }
      }
      // Epilogue
      const float a = Gs[64];
      f32x4 Vd[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 32 * (tt >> 1) + 8 * g + 4 * (tt & 1) + r;
          const float vn = Us[t * UP + 16 * cj + n] - acc[tt][r];
          if (vb_ != nullptr && t < len) vb_[(t0 + t) * p.sv_t + vcol] = vn;
          Vd[tt][r] = vn * Gs[t];
        }
      // MM2: S = a S + K^T Vd  (contraction slot g of step (tt, r) is token sigma(tt, 4g + r))
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        f32x4 up = S[kt] * a;
        const int krow = 32 * (kt >> 1) + 8 * (n >> 2) + 4 * (kt & 1) + (n & 3);
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 32 * (tt >> 1) + 8 * g + 4 * (tt & 1) + r;
            up = mfma_f32(Ks[t * WP + krow], Vd[tt][r], up);
          }
        S[kt] = up;
      }
    } else {
      // vec: h and v_new leave as 16-byte row pieces written by all 256 threads (the h snapshot
      // from the state staging buffer, v_new from the U tile, which the epilogue overwrites
      // with it); else each compute wave stores its own elements
      const bool vec = p.vec_out != 0;
      E* hdst = hb_ + (tk.boh + c) * p.sh_c;
      float a = 0.f;
      if (computes) {
        a = Gs[64];
        if (!vec) {   // h snapshot (exact), own rows
#pragma unroll
          for (int i = 0; i < KTR; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int kt = kt0 + i;
              const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
              if (krow < p.K) hdst[(int64_t)krow * p.V + vcol] = (E)S[i][r];
            }
        }
        // MM1 of own token tiles, the whole state of the column block from the staging buffer
#pragma unroll
        for (int q = 0; q < TPW; ++q) {
          const int tt = TPW * rgrp + q;
          f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
          const int row = 32 * (tt >> 1) + 8 * (n >> 2) + 4 * (tt & 1) + (n & 3);
#pragma unroll
          for (int kt = 0; kt < KT; ++kt) {
            const int kcol = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1);
            const f32x4 wv = *(const f32x4*)(Ws + row * WP + kcol);
            const f32x4 sv = *(const f32x4*)(SSs + ss_at(kt));
#pragma unroll
            for (int r = 0; r < 4; ++r) acc = mfma_f32(wv[r], sv[r], acc);
          }
          // epilogue: v_new, and Vd to the staging buffer.  Each U element is read, and with vec
          // overwritten by v_new, by this lane alone.
          f32x4 vd;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int t = 32 * (tt >> 1) + 8 * g + 4 * (tt & 1) + r;
            float* up_ = Us + t * UP + 16 * cj + n;
            const float vn = *up_ - acc[r];
            if (vec) *up_ = vn;
            else if (vb_ != nullptr && t < len) vb_[(t0 + t) * p.sv_t + vcol] = vn;
            vd[r] = vn * Gs[t];
          }
          *(f32x4*)(VDs + vd_at(tt)) = vd;
        }
      }
      if (vec) {
        // h snapshot of chunk c = the state entering it, all of it in the staging buffer since
        // the previous chunk's MM2 (rewritten only after the next barrier): thread i stores 4
        // columns of row i / (VT / 4), then of the rows 256 / (VT / 4) further down
        constexpr int HP = KD * VT / 4;   // 16-byte pieces of the K x Vt block
#pragma unroll
        for (int i = 0; i < (HP + 255) / 256; ++i) {
          const int q = threadIdx.x + 256 * i, row = q / (VT / 4), c4 = 4 * (q % (VT / 4));
          if (q < HP && row < p.K) {
            f32x4 hv;
#pragma unroll
            for (int j = 0; j < 4; ++j) hv[j] = SSs[(c4 + j) * SSP + row];
            *(f32x4*)(hdst + (int64_t)row * p.V + vbase + c4) = hv;
          }
        }
      }
      __syncthreads();   // Vd and v_new of all tokens staged; every read of the staged state done
      if (computes) {
        // MM2 of own rows: S = a S + K^T Vd, token tiles in order
#pragma unroll
        for (int i = 0; i < KTR; ++i) {
          const int kt = kt0 + i;
          f32x4 up = S[i] * a;
          const int krow = 32 * (kt >> 1) + 8 * (n >> 2) + 4 * (kt & 1) + (n & 3);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const f32x4 vdv = *(const f32x4*)(VDs + vd_at(tt));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int t = 32 * (tt >> 1) + 8 * g + 4 * (tt & 1) + r;
              up = mfma_f32(Ks[t * WP + krow], vdv[r], up);
            }
          }
          S[i] = up;
          *(f32x4*)(SSs + ss_at(kt)) = up;   // the state entering chunk c+1 (read after the next barrier)
        }
      }
      if (vec && vb_ != nullptr) {
        // v_new rows from the U tile (rewritten only after the next chunk's first barrier)
        constexpr int VP = 64 * VT / 4;
#pragma unroll
        for (int i = 0; i < (VP + 255) / 256; ++i) {
          const int q = threadIdx.x + 256 * i, t = q / (VT / 4), c4 = 4 * (q % (VT / 4));
          if (q < VP && t < len) *(f32x4*)(vb_ + (t0 + t) * p.sv_t + vbase + c4) = *(const f32x4*)(Us + t * UP + c4);
        }
      }
    }
  }
  if (computes && p.final_state != nullptr) {
    const int64_t base = (int64_t)tk.n * p.sf_n + (int64_t)tk.head * p.sf_h;
#pragma unroll
    for (int i = 0; i < KTR; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int kt = kt0 + i;
        const int krow = 32 * (kt >> 1) + 8 * g + 4 * (kt & 1) + r;
        const int64_t off = base + (p.state_vk ? (int64_t)vcol * p.K + krow : (int64_t)krow * p.V + vcol);
        if (krow >= p.K) continue;
        if (p.final_f32) ((float*)p.final_state)[off] = S[i][r];
        else ((__bf16*)p.final_state)[off] = (__bf16)S[i][r];
      }
  }
}

}  // namespace cgdr
