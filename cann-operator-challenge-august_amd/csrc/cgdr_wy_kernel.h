// cgdr_wy_kernel.h -- gfx950 device code of the WY producer of FwdH's w, u and g.
//
// One workgroup (4 waves) owns one unit (batch row, chunk, value head).  With L <= 64 tokens,
// per-token log-decay a, beta and keys k (key head of the value head), values v:
//
//   g_i  = a_0 + ... + a_i                                   (chunk-local cumsum, sequential)
//   A_ij = beta_i (k_i . k_j) e^{g_i - g_j}  for j < i, else 0
//   T    = (I + A)^{-1}                                      (unit lower triangular, fp32)
//   w    = bf16( bf16(T diag(beta e^g)) k ),  u = bf16( bf16(T diag(beta)) v )
//
// (ref/chunk_gated_delta_rule/tests/pytest/chunk_gated_delta_rule_golden.py:102-124 of the
// reference, and its device stage 1, op_kernel/arch22/chunk_gated_delta_rule_stage1.h.)
//
// Phases, separated by workgroup barriers:
//   0  DMA of the k tile into LDS by waves 0-2; wave 3 forms g (each lane sums a_0..a_i in order, which is
//      the sequential cumsum bit for bit), beta e^g and beta.  Then each wave touches its share
//      of this unit's v rows into L2.
//   1  S = k k^T with bf16 MFMA (wave w: columns i = 16w..16w+15, operands read from the k tile),
//      A written to LDS in fp32
//   2  T: each wave inverts its own 16x16 diagonal block by forward substitution right after
//      writing its row block of A (lane = column; each solved row updates the partial sums of all
//      later rows at once, so the dependent chain is 16 steps); after one barrier, wave j computes
//      column block j, T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj for i = j+1 .. 3 in order, with fp32
//      MFMA 16x16x4 and no further barrier.  The contraction slot of lane group G at step kk is
//      4 G + kk, so a C-layout result is directly the B operand of the next product.  A and T
//      share one fp32 matrix M: A_ij = M[i][j] below the diagonal, T is stored transposed,
//      T_ij = M[j][i] on and above it (T's upper triangle is zero).
//   3  w^T = k^T T'^T and u^T = v^T T''^T with bf16 MFMA: the A operands are transposed reads of
//      the k / v tiles, the B operands rows of T scaled per column and rounded to bf16; each lane
//      ends with 8 consecutive columns of one token, written with 16-byte stores.  The B operands
//      go to registers first; the v tile then takes M's place in LDS (its DMA runs while w is
//      computed), so a workgroup needs k, M and g only: 34,816 B at K = V = 128.
#pragma once

#include "cgdr_chunk_common.h"

namespace cgdr {

struct WyParams {
  const void* k;
  const void* v;
  const void* beta;
  const float* g;
  const int64_t* cu_seqlens;
  const int64_t* chunk_indices;
  void* w;
  void* u;
  float* gc;
  int64_t T, NT;
  int32_t H, Hg, N, beta_f32;
  int32_t n_xcd, reserved;   // XCDs workgroups are dealt to round-robin
  int64_t sk_b, sk_t, sk_h;
  int64_t sv_b, sv_t, sv_h;
  int64_t sb_b, sb_t, sb_h;
  int64_t sg_b, sg_t, sg_h;
  int64_t sw_b, sw_t, sw_h;
  int64_t su_b, su_t, su_h;
  int64_t sc_b, sc_t, sc_h;
};

template <int KD, int VD>
struct WyLayout {
  static constexpr int PK = KD / 8, PV = VD / 8;   // 16-byte pieces per k / v tile row
  static constexpr int MS = 68;                    // fp32 row stride of A and T (conflict-free columns)
  static constexpr int K_OFF = 0;                  // k tile [64][KD] bf16
  static constexpr int M_OFF = 64 * KD * 2;        // A (strictly lower) and T^T (upper), fp32
  static constexpr int V_OFF = M_OFF;              // v tile [64][VD] bf16, once T is in registers
  static constexpr int MV_BYTES = 64 * MS * 4 > 64 * VD * 2 ? 64 * MS * 4 : 64 * VD * 2;
  static constexpr int G_OFF = M_OFF + MV_BYTES;   // g [64], beta e^g [64], beta [64], a [64]
  static constexpr int LDS_BYTES = G_OFF + 4 * 256;
  static constexpr int RPDK = 64 / PK, RPDV = 64 / PV;
  static constexpr int DMA_K = 64 / RPDK, DMA_V = 64 / RPDV;
};

template <int KD, int VD>
__global__ void __launch_bounds__(256) cgdr_wy_bf16_kernel(const WyParams p) {
  using L = WyLayout<KD, VD>;
  constexpr int KS = KD / 32;
  constexpr int MS = L::MS;
  __shared__ __attribute__((aligned(1024))) char smem[L::LDS_BYTES];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, G = lane >> 4;
  const int e = n >> 2, qd = n & 3;

  // unit -> (b, chunk, head); consecutive units (the heads of one key head) share an XCD
  int64_t unit = xcd_remap(blockIdx.x, gridDim.x, p.n_xcd);
  const int head = (int)(unit % p.H);
  unit /= p.H;
  const int64_t chunk = unit % p.NT;
  const int b = (int)(unit / p.NT);
  const ChunkRange cr = chunk_range(p.T, p.N, p.cu_seqlens, p.chunk_indices, chunk);
  const int len = __builtin_amdgcn_readfirstlane(cr.len);
  if (len == 0) return;   // uniform over the workgroup
  const int64_t start = cr.start;
  const int kh = head / (p.H / p.Hg);

  const __bf16* kb = (const __bf16*)p.k + b * p.sk_b + start * p.sk_t + kh * p.sk_h;
  const __bf16* vb = (const __bf16*)p.v + b * p.sv_b + start * p.sv_t + head * p.sv_h;
  __bf16* wb = (__bf16*)p.w + b * p.sw_b + start * p.sw_t + head * p.sw_h;
  __bf16* ub = (__bf16*)p.u + b * p.su_b + start * p.su_t + head * p.su_h;

  // ---- phase 0: k tile (rows past the chunk end zero-filled), by waves 0-2; the v tile
  // follows in phase 3.  Wave 3 meanwhile loads beta and the log-decays and forms g, so that
  // its waits on those loads do not also wait for DMAs of its own (vmcnt counts both).  A full
  // chunk issues its DMAs in one uniform branch, without a per-lane condition around each.
  const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_char*)smem);
  {
    const int64_t krow = p.sk_t * 2;
    if (len == 64) {
#pragma unroll
      for (int m = 0; m < L::DMA_K; ++m) {
        if (m % 3 != wave) continue;
        const int r = m * L::RPDK + lane / L::PK, c = lane % L::PK;
        dma_b128(kb, (uint32_t)(r * krow) + 16u * (uint32_t)(c ^ swz_k<L::PK>(r)), lds0 + L::K_OFF + 1024u * m);
      }
    } else {
#pragma unroll
      for (int m = 0; m < L::DMA_K; ++m) {
        if (m % 3 != wave) continue;
        const int r = m * L::RPDK + lane / L::PK, c = lane % L::PK;
        if (r < len)
          dma_b128(kb, (uint32_t)(r * krow) + 16u * (uint32_t)(c ^ swz_k<L::PK>(r)), lds0 + L::K_OFF + 1024u * m);
        else
          *(u32x4*)(smem + L::K_OFF + 1024 * m + 16 * lane) = u32x4{0, 0, 0, 0};
      }
    }
  }
  float* GA = (float*)(smem + L::G_OFF);
  if (wave == 3) {
    float bt = 0.f, at = 0.f;
    if (lane < len) {
      const int64_t ob = b * p.sb_b + (start + lane) * p.sb_t + head * p.sb_h;
      bt = p.beta_f32 ? ((const float*)p.beta)[ob] : (float)((const __bf16*)p.beta)[ob];
      if (p.g != nullptr) at = p.g[b * p.sg_b + (start + lane) * p.sg_t + head * p.sg_h];
    }
    GA[192 + lane] = at;
    wait_lgkm0();
    // g_lane = ((a_0 + a_1) + a_2) + ... + a_lane, the order of a sequential cumsum
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 64; j += 4) {
      const f32x4 a4 = *(const f32x4*)(GA + 192 + j);
#pragma unroll
      for (int r = 0; r < 4; ++r)
        if (j + r <= lane) s += a4[r];
    }
    GA[lane] = s;
    GA[64 + lane] = bt * expf(s);
    GA[128 + lane] = bt;
    if (p.gc != nullptr && lane < len) p.gc[b * p.sc_b + (start + lane) * p.sc_t + head * p.sc_h] = s;
  }
  wait_vm<0>();
  wait_lgkm0();
  block_barrier();

  // ---- L2 prefetch of this unit's v rows, which phase 3 loads into LDS: one 4-byte
  // direct-to-LDS load per 128-byte line, landing in the a[] slot of the g area (not read after
  // phase 0); each wave drains its own before the barrier ahead of phase 3.
  {
    constexpr int LK = KD >= 64 ? KD / 64 : 1, LV = VD >= 64 ? VD / 64 : 1;   // lines per row
    const uint32_t trash = lds0 + L::G_OFF + 768u;
#pragma unroll
    for (int m = 0; m < LV; ++m) {
      if ((LK + m) % 4 != wave) continue;
      const int t = 64 * m + lane, r = t / LV;
      if (r < len) dma_b32_addr((const char*)vb + r * p.sv_t * 2 + 128 * (t % LV), trash);
    }
  }

  // ---- phase 1: A_ij = beta_i S_ij e^{g_i - g_j} (j < i) by 16x16 tiles (row block rb, column
  // block t <= rb); for tile (rb, t) lane holds S[16t + 4G + r][16rb + n].  Operands are k rows
  // from the tile: row j, contraction slice 32 ks + 8 G .. +7 (one piece).  The ten tiles are
  // dealt 3, 3, 2, 2: wave w computes its diagonal tile (w, w), then (2,0) (1,0) (2,1) (3,2)
  // for w = 0..3, then (3,0) (3,1) for w = 0, 1.
  float* M = (float*)(smem + L::M_OFF);
  const int i = 16 * wave + n;
  const lds_char* ktile = (const lds_char*)smem + L::K_OFF;
  auto krow = [&](int j, int ks) {
    return __builtin_bit_cast(bf16x8, *(const u32x4*)(ktile + (j * L::PK + ((4 * ks + G) ^ swz_k<L::PK>(j))) * 16));
  };
  auto a_tile = [&](int rb, int t) {
    const int ii = 16 * rb + n;
    const float gi = GA[ii], bi = GA[128 + ii];
    bf16x8 kc[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kc[ks] = krow(ii, ks);
    f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) c = mfma_bf16(krow(16 * t + n, ks), kc[ks], c);
    const f32x4 gj = *(const f32x4*)(GA + 16 * t + 4 * G);
    f32x4 a;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 16 * t + 4 * G + r;
      a[r] = j < ii ? bi * c[r] * expf(gi - gj[r]) : 0.f;
    }
    *(f32x4*)(M + ii * MS + 16 * t + 4 * G) = a;
  };
  a_tile(wave, wave);
  a_tile(wave == 0 ? 2 : wave, wave == 0 ? 0 : wave - 1);
  if (wave < 2) a_tile(3, wave);
  wait_lgkm0();

  // T_rc (r >= c) lives at M[c][r]; entries above T's diagonal read as zero
  auto tval = [&](int r, int c) { return r >= c ? M[c * MS + r] : 0.f; };

  // ---- phase 2a: this wave's diagonal block T_ww = (I + A_ww)^{-1}, right after it wrote
  // A_ww (its own LDS writes are visible to its later reads without a barrier).  Lane c < 16
  // solves column c; acc[r] collects 1_{r=c} - sum_{j<r} A_rj T_jc in the order j = 0, ..., r-1.
  if (G == 0) {
    const int c = n, o = 16 * wave;
    float acc[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = r == c ? 1.f : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
#pragma unroll
      for (int r2 = r + 1; r2 < 16; ++r2) acc[r2] -= M[(o + r2) * MS + o + r] * acc[r];
    }
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (r >= c) M[(o + c) * MS + o + r] = acc[r];
  }
  wait_lgkm0();
  block_barrier();

  // ---- phase 2b: off-diagonal blocks by column block: wave j computes T_ij for i = j+1 .. 3 in
  // order, T_ij = -T_ii sum_{k=j}^{i-1} A_ik T_kj.  Every A block and diagonal T block is in LDS
  // after the barrier above, and the T_kj (k > j) it needs are its own earlier results, kept in
  // registers (their C layout is the B operand layout), so no further barrier is needed and no
  // LDS write stands between two steps: the blocks are written to LDS once all are done.
  // acc += A[xr.., xc..] B, with B a 16x16 block of T in C layout
  auto mm = [&](f32x4 acc, int xr, int xc, const f32x4& B) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma_f32(M[(xr + n) * MS + xc + 4 * G + kk], B[kk], acc);
    return acc;
  };
  // -(T_{tr,tr} Y), Y held in C layout
  auto finish = [&](const f32x4& Y, int tr) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) acc = mfma_f32(tval(tr + n, tr + 4 * G + kk), Y[kk], acc);
    return -acc;
  };
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  const int cw = 16 * wave;
  f32x4 tb[4];   // T_{kb, wave}: the diagonal block from LDS, then this wave's results
  const f32x4 diag = {tval(cw + 4 * G, cw + n), tval(cw + 4 * G + 1, cw + n), tval(cw + 4 * G + 2, cw + n),
                      tval(cw + 4 * G + 3, cw + n)};
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) tb[kb] = kb == wave ? diag : z4;
#pragma unroll
  for (int ib = 1; ib < 4; ++ib) {
    if (ib <= wave) continue;
    f32x4 y = z4;
#pragma unroll
    for (int kb = 0; kb < 3; ++kb)
      if (kb >= wave && kb < ib) y = mm(y, 16 * ib, 16 * kb, tb[kb]);
    tb[ib] = finish(y, 16 * ib);
  }
#pragma unroll
  for (int ib = 1; ib < 4; ++ib) {
    if (ib <= wave) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) M[(cw + n) * MS + 16 * ib + 4 * G + r] = tb[ib][r];
  }
  wait_lgkm0();
  wait_vm<0>();   // the prefetch loads (issued two phases ago) have landed
  block_barrier();

  // ---- phase 3: w^T = k^T T'^T, u^T = v^T T''^T.  The B operands (rows of T scaled per column,
  // bf16) go to registers first, so that the v tile can take the A/T matrix's place: its DMA
  // (rows mostly in L2 by now) runs while w is computed.  The work comes in units of 32 output
  // columns of [w | u] per token block, NPP units per block; a unit of token block tb costs
  // 2 njp MFMAs (contraction j <= i: njp = 1 for blocks 0 and 1, 2 for blocks 2 and 3).  Wave w
  // takes token block w; when Q = NPP / 4 units are all w columns, waves 2 and 3 leave units
  // 0 .. Q-1 of their blocks to waves 0 and 1 (wave w takes them for block 3 - w), so every wave
  // does 1.5 NPP units' worth of MFMAs.
  constexpr int NPW = KD / 32, NPP = (KD + VD) / 32;
  constexpr int Q = (NPP % 4 == 0 && NPP / 4 <= NPW) ? NPP / 4 : 0;
  const bool active = 16 * wave < len;   // wave-uniform; idle waves still share the DMA and barriers
  const int njp = (wave >> 1) + 1;
  const int ufirst = wave >= 2 ? Q : 0;  // first unit this wave takes of its own block
  const int i2 = 16 * (3 - wave) + n;    // waves 0, 1: token of the second block
  const bool has2 = Q > 0 && wave < 2 && 16 * (3 - wave) < len;
  // B operands of token ti: bw[jp] (w, columns scaled by beta e^g), bu[jp] (u, by beta)
  auto bops = [&](int ti, int nj, u32x4* bwx, u32x4* bux) {
#pragma unroll
    for (int jp = 0; jp < 2; ++jp) {
      if (jp >= nj) continue;
      const int j0 = 32 * jp + 8 * G;
      float tw[8], tu[8];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x4 sg = *(const f32x4*)(GA + 64 + j0 + 4 * h);
        const f32x4 sb = *(const f32x4*)(GA + 128 + j0 + 4 * h);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float t = tval(ti, j0 + 4 * h + r);
          tw[4 * h + r] = t * sg[r];
          tu[4 * h + r] = t * sb[r];
        }
      }
      bwx[jp] = u32x4{pack_bf16x2(tw[0], tw[1]), pack_bf16x2(tw[2], tw[3]), pack_bf16x2(tw[4], tw[5]), pack_bf16x2(tw[6], tw[7])};
      if (bux != nullptr)
        bux[jp] = u32x4{pack_bf16x2(tu[0], tu[1]), pack_bf16x2(tu[2], tu[3]), pack_bf16x2(tu[4], tu[5]), pack_bf16x2(tu[6], tu[7])};
    }
  };
  u32x4 bw[2], bu[2], bw2[2];
  if (active) bops(i, njp, bw, bu);
  if (has2) bops(i2, 2, bw2, nullptr);
  wait_lgkm0();
  block_barrier();   // every wave is done with A/T

  {
    const int64_t vrow = p.sv_t * 2;
    if (len == 64) {   // a full chunk: one uniform branch, no per-lane condition per DMA
#pragma unroll
      for (int m = 0; m < L::DMA_V; ++m) {
        if ((L::DMA_K + m) % 4 != wave) continue;
        const int r = m * L::RPDV + lane / L::PV, c = lane % L::PV;
        dma_b128(vb, (uint32_t)(r * vrow) + 16u * (uint32_t)(c ^ swz_k<L::PV>(r)), lds0 + L::V_OFF + 1024u * m);
      }
    } else {
#pragma unroll
      for (int m = 0; m < L::DMA_V; ++m) {
        if ((L::DMA_K + m) % 4 != wave) continue;
        const int r = m * L::RPDV + lane / L::PV, c = lane % L::PV;
        if (r < len)
          dma_b128(vb, (uint32_t)(r * vrow) + 16u * (uint32_t)(c ^ swz_k<L::PV>(r)), lds0 + L::V_OFF + 1024u * m);
        else
          *(u32x4*)(smem + L::V_OFF + 1024 * m + 16 * lane) = u32x4{0, 0, 0, 0};
      }
    }
  }
  // One unit: columns 32 pp + 8 G .. +7 of the lane's token, bf16-packed
  auto wu_unit = [&](const lds_char* tile, auto pv_tag, int pp, int nj, const u32x4* b) -> u32x4 {
    constexpr int PX = decltype(pv_tag)::value;
    f32x4 acc[2];
#pragma unroll
    for (int x = 0; x < 2; ++x) {
      acc[x] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jp = 0; jp < 2; ++jp)
        if (jp < nj)
          acc[x] = mfma_bf16(__builtin_bit_cast(bf16x8, tr_operand<PX>(tile, 32 * jp, pp, x, G, e, qd)),
                             __builtin_bit_cast(bf16x8, b[jp]), acc[x]);
    }
    return u32x4{pack_bf16x2(acc[0][0], acc[0][1]), pack_bf16x2(acc[0][2], acc[0][3]),
                 pack_bf16x2(acc[1][0], acc[1][1]), pack_bf16x2(acc[1][2], acc[1][3])};
  };
  using PKT = std::integral_constant<int, L::PK>;
  using PVT = std::integral_constant<int, L::PV>;
  u32x4 wpk[NPW], wpk2[Q > 0 ? Q : 1];   // w results, held until the v tile lands
  if (active) {
#pragma unroll
    for (int pp = 0; pp < NPW; ++pp)
      if (pp >= ufirst) wpk[pp] = wu_unit(ktile, PKT{}, pp, njp, bw);
  }
  if (has2) {
#pragma unroll
    for (int q = 0; q < Q; ++q) wpk2[q] = wu_unit(ktile, PKT{}, q, 2, bw2);
  }
  wait_vm<0>();
  wait_lgkm0();
  block_barrier();   // v tile in LDS
  if (has2 && i2 < len) {
#pragma unroll
    for (int q = 0; q < Q; ++q) *(u32x4*)(wb + i2 * p.sw_t + 32 * q + 8 * G) = wpk2[q];
  }
  if (!active) return;

  const lds_char* vtile = (const lds_char*)smem + L::V_OFF;
  const bool store = i < len;
  if (store) {
#pragma unroll
    for (int pp = 0; pp < NPW; ++pp)
      if (pp >= ufirst) *(u32x4*)(wb + i * p.sw_t + 32 * pp + 8 * G) = wpk[pp];
  }
#pragma unroll
  for (int pp = 0; pp < VD / 32; ++pp) {
    const u32x4 r = wu_unit(vtile, PVT{}, pp, njp, bu);
    if (store) *(u32x4*)(ub + i * p.su_t + 32 * pp + 8 * G) = r;
  }
}

}  // namespace cgdr
