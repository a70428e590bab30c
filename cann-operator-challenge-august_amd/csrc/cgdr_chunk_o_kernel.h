// cgdr_chunk_o_kernel.h -- gfx950 device code of the chunk-output operator.
//
// One workgroup (4 waves) owns one unit (batch row, chunk, value head, V-tile of VT columns);
// units are independent.  Per unit, with L <= 64 tokens, i, j in [0, L):
//
//   A'   = bf16( scale (q_i . k_j) e^{g_i - g_j} )  for j <= i, else 0      [64 x 64]
//   o_i  = bf16( scale e^{g_i} (q_i . h_c) + sum_j A'_ij v_new_j )           [64 x VT]
//
// (ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:136-142 of the
// reference; stage2.h:170 attn_inter and stage3.h:131-180 the masked product.)
//
// All three products are computed transposed, so that no operand needs a layout change:
//   A^T  = k q^T      A operand k rows (contiguous), B operand q rows (contiguous)
//   O^T  = h^T q^T    A operand h^T by ds_read_b64_tr_b16 from the h tile in LDS
//   O^T += v^T A'^T   A operand v_new^T by ds_read_b64_tr_b16, B operand A'^T from registers
// Wave w owns tokens i = 16w .. 16w+15 (the MFMA column index n = lane % 16).  In the A^T
// tiles the row order is free: tile x of token pair jp holds row 4G + r <-> token
// j = 32 jp + 8 G + 4 x + r, so lane group G of the two tiles holds 8 consecutive tokens for
// its column, which is the contraction slice the v_mfma_f32_16x16x32_bf16 B operand wants.
// The same ordering of the value columns (tile x of column pair p: row 4G + r <-> column
// 32 p + 8 G + 4 x + r) leaves every lane with 8 consecutive o columns of one token: o is
// written with one 16-byte store per lane and column pair, straight from the accumulators.
//
// Data movement: q and k rows go straight to VGPRs (16-byte loads), the h tile [K][VT] and the
// v_new tile [64][VT] by direct-to-LDS DMA (16-byte pieces XOR-swizzled per row), g through a
// per-wave LDS row.  Rows past the chunk end are zero-filled, never read.
#pragma once

#include "cgdr_chunk_common.h"

namespace cgdr {

struct ChunkOParams {
  const void* q;
  const void* k;
  const void* v;
  const void* h;
  const float* g;
  const int64_t* cu_seqlens;
  const int64_t* chunk_indices;
  void* o;
  int64_t T, NT, V;
  int32_t H, Hg, N, n_vtiles;
  float scale;
  int32_t n_xcd;       // XCDs workgroups are dealt to round-robin
  int64_t sq_b, sq_t, sq_h;
  int64_t sk_b, sk_t, sk_h;
  int64_t sv_b, sv_t, sv_h;
  int64_t sh_b, sh_c, sh_h;
  int64_t sg_b, sg_t, sg_h;
  int64_t so_b, so_t, so_h;
};

template <int KD, int VT>
struct ChunkOLayout {
  static constexpr int PV = VT / 8;                  // 16-byte pieces per h / v_new tile row
  static constexpr int H_OFF = 0;                    // h tile [KD][VT] bf16
  static constexpr int V_OFF = KD * VT * 2;          // v_new tile [64][VT] bf16
  static constexpr int G_OFF = V_OFF + 64 * VT * 2;  // per-wave g rows, 4 x 64 fp32
  static constexpr int LDS_BYTES = G_OFF + 4 * 256;
  static constexpr int RPD = 64 / PV;                // tile rows per DMA instruction
  static constexpr int DMA_H = KD / RPD;
  static constexpr int DMA_V = 64 / RPD;
};

template <int KD, int VT>
__global__ void __launch_bounds__(256) cgdr_chunk_o_bf16_kernel(const ChunkOParams p) {
  using L = ChunkOLayout<KD, VT>;
  constexpr int KS = KD / 32;   // contraction steps over K
  constexpr int NP = VT / 32;   // value-column tile pairs
  constexpr int PV = L::PV;
  __shared__ __attribute__((aligned(1024))) char smem[L::LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, G = lane >> 4;
  const int e = n >> 2, qd = n & 3;

  // unit -> (b, chunk, head, vtile); consecutive units share an XCD (V-tiles and the heads of
  // one key head reuse q and k from that XCD's L2)
  int64_t unit = xcd_remap(blockIdx.x, gridDim.x, p.n_xcd);
  const int vtile = (int)(unit % p.n_vtiles);
  unit /= p.n_vtiles;
  const int head = (int)(unit % p.H);
  unit /= p.H;
  const int64_t chunk = unit % p.NT;
  const int b = (int)(unit / p.NT);
  const ChunkRange cr = chunk_range(p.T, p.N, p.cu_seqlens, p.chunk_indices, chunk);
  const int len = __builtin_amdgcn_readfirstlane(cr.len);
  if (len == 0) return;   // uniform over the workgroup
  const int64_t start = cr.start;
  const int kh = head / (p.H / p.Hg);

  const __bf16* qb = (const __bf16*)p.q + b * p.sq_b + start * p.sq_t + kh * p.sq_h;
  const __bf16* kb = (const __bf16*)p.k + b * p.sk_b + start * p.sk_t + kh * p.sk_h;
  const char* vb = (const char*)((const __bf16*)p.v + b * p.sv_b + start * p.sv_t + head * p.sv_h + vtile * VT);
  const char* hb = (const char*)((const __bf16*)p.h + b * p.sh_b + chunk * p.sh_c + head * p.sh_h + vtile * VT);
  __bf16* ob = (__bf16*)p.o + b * p.so_b + start * p.so_t + head * p.so_h + vtile * VT;

  // ---- direct-to-LDS DMA of the h and v_new tiles: instruction m, lane -> LDS piece
  // 64 m + lane = (row r, slot s), filled from global piece (r, s ^ swz_k(r)); instructions
  // are dealt to the waves round-robin.  v_new rows past the chunk end are zero-filled.
  const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_char*)smem);
  {
    const int lrow = lane / PV, lcol = lane % PV;
    const int64_t hrow = p.V * 2, vrow = p.sv_t * 2;
#pragma unroll
    for (int m = 0; m < L::DMA_H; ++m) {
      if (m % 4 != wave) continue;
      const int r = m * L::RPD + lrow;
      dma_b128(hb, (uint32_t)(r * hrow) + 16u * (uint32_t)(lcol ^ swz_k<PV>(r)), lds0 + L::H_OFF + 1024u * m);
    }
#pragma unroll
    for (int m = 0; m < L::DMA_V; ++m) {
      if ((L::DMA_H + m) % 4 != wave) continue;
      const int r = m * L::RPD + lrow;
      if (r < len)
        dma_b128(vb, (uint32_t)(r * vrow) + 16u * (uint32_t)(lcol ^ swz_k<PV>(r)), lds0 + L::V_OFF + 1024u * m);
      else
        *(u32x4*)(smem + L::V_OFF + 1024 * m + 16 * lane) = u32x4{0, 0, 0, 0};
    }
  }

  // ---- q rows of this wave's tokens, k rows of the token pairs it needs, g row
  const int i_tok = 16 * wave + n;
  const int njp = (wave >> 1) + 1;   // token pairs j < 16 wave + 16
  const u32x4 zero4 = {0, 0, 0, 0};
  u32x4 qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qf[ks] = i_tok < len ? *(const u32x4*)(qb + i_tok * p.sq_t + 32 * ks + 8 * G) : zero4;
  u32x4 kf[2][2][KS];
#pragma unroll
  for (int jp = 0; jp < 2; ++jp)
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const int j = 32 * jp + 8 * e + 4 * x + qd;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        kf[jp][x][ks] = (jp < njp && j < len) ? *(const u32x4*)(kb + j * p.sk_t + 32 * ks + 8 * G) : zero4;
    }
  float* grow = (float*)(smem + L::G_OFF + 256 * wave);
  {
    float gv = 0.f;
    if (p.g != nullptr && lane < len) gv = p.g[b * p.sg_b + (start + lane) * p.sg_t + head * p.sg_h];
    grow[lane] = gv;
  }

  wait_vm<0>();
  wait_lgkm0();
  block_barrier();
  if (16 * wave >= len) return;   // no token of this wave is in the chunk

  // ---- A^T = k q^T, then the masked, decayed, scaled bf16 A'^T operands
  const float g_i = grow[i_tok];
  u32x4 ap[2];
#pragma unroll
  for (int jp = 0; jp < 2; ++jp) {
    if (jp >= njp) continue;
    f32x4 at[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      at[x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        at[x] = mfma_bf16(__builtin_bit_cast(bf16x8, kf[jp][x][ks]), __builtin_bit_cast(bf16x8, qf[ks]), at[x]);
    }
    float a[8];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      const f32x4 gj = *(const f32x4*)(grow + 32 * jp + 8 * G + 4 * x);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 32 * jp + 8 * G + 4 * x + r;
        a[4 * x + r] = j <= i_tok ? p.scale * at[x][r] * expf(g_i - gj[r]) : 0.f;
      }
    }
    ap[jp] = u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]), pack_bf16x2(a[6], a[7])};
  }

  // ---- O^T = h^T q^T (two transposed reads per operand: lane (G, n) gets
  // T[32 s + 8 G + 4 half + (0..3)][column 32 p + 8 (n / 4) + 4 x + n % 4])
  auto tr_op = [&](int off, int rbase, int pp, int x) {
    return tr_operand<PV>((const lds_char*)smem + off, rbase, pp, x, G, e, qd);
  };
  f32x4 acc[NP][2];
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      acc[pp][x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        acc[pp][x] = mfma_bf16(__builtin_bit_cast(bf16x8, tr_op(L::H_OFF, 32 * ks, pp, x)),
                               __builtin_bit_cast(bf16x8, qf[ks]), acc[pp][x]);
    }
  const float f = p.scale * expf(g_i);
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int x = 0; x < 2; ++x) acc[pp][x] = acc[pp][x] * f;

  // ---- O^T += v_new^T A'^T, then 16-byte stores of o[i][32 p + 8 G .. +7]
#pragma unroll
  for (int pp = 0; pp < NP; ++pp)
#pragma unroll
    for (int x = 0; x < 2; ++x)
#pragma unroll
      for (int jp = 0; jp < 2; ++jp) {
        if (jp >= njp) continue;
        acc[pp][x] = mfma_bf16(__builtin_bit_cast(bf16x8, tr_op(L::V_OFF, 32 * jp, pp, x)),
                               __builtin_bit_cast(bf16x8, ap[jp]), acc[pp][x]);
      }
  if (i_tok < len) {
    __bf16* orow = ob + i_tok * p.so_t + 8 * G;
#pragma unroll
    for (int pp = 0; pp < NP; ++pp) {
      const u32x4 v = {pack_bf16x2(acc[pp][0][0], acc[pp][0][1]), pack_bf16x2(acc[pp][0][2], acc[pp][0][3]),
                       pack_bf16x2(acc[pp][1][0], acc[pp][1][1]), pack_bf16x2(acc[pp][1][2], acc[pp][1][3])};
      *(u32x4*)(orow + 32 * pp) = v;
    }
  }
}

}  // namespace cgdr
