// cgdr_chunk_common.h -- device helpers shared by the per-chunk kernels (chunk output, WY).
#pragma once

#include "cgdr_kernels.h"

namespace cgdr {

// Token range of one global chunk: start token and length (0 when the chunk maps to no
// tokens; malformed metadata never leads to an access outside [0, T)).  Fixed length: chunk c
// of every batch row covers [64 c, min(64 c + 64, T)).  Varlen (B == 1): the chunk's
// (sequence, chunk-in-sequence) row comes from chunk_indices when given (the reference's
// prepare_chunk_indices, docs/problem.txt:251-261), else from a scan of cu_seqlens with the
// per-sequence chunk counts ceil(L_n / 64) (docs/problem.txt:263-270).
struct ChunkRange {
  int64_t start;
  int len;
};

__device__ __forceinline__ ChunkRange chunk_range(int64_t T, int N, const int64_t* cu_seqlens,
                                                  const int64_t* chunk_indices, int64_t chunk) {
  ChunkRange r{0, 0};
  int64_t start, end;
  if (cu_seqlens == nullptr) {
    start = chunk * kChunk;
    end = T;
  } else {
    int64_t n, cc;
    if (chunk_indices != nullptr) {
      n = chunk_indices[2 * chunk];
      cc = chunk_indices[2 * chunk + 1];
      if (n < 0 || n >= N || cc < 0) return r;
    } else {
      int64_t boh = 0;
      for (n = 0; n < N; ++n) {
        const int64_t l = cu_seqlens[n + 1] - cu_seqlens[n];
        const int64_t nc = l > 0 ? (l + kChunk - 1) / kChunk : 0;
        if (chunk < boh + nc) break;
        boh += nc;
      }
      if (n == N) return r;
      cc = chunk - boh;
    }
    start = cu_seqlens[n] + cc * kChunk;
    end = cu_seqlens[n + 1];
  }
  if (start < 0 || start >= T) return r;
  if (end > T) end = T;
  const int64_t len = end - start;
  r.start = start;
  r.len = len <= 0 ? 0 : (len > kChunk ? kChunk : (int)len);
  return r;
}

// MFMA 16x16x32 bf16 operand of a transposed tile: the LDS tile holds rows = contraction index
// (tokens or K) and columns = operand rows, bf16, PV 16-byte pieces per row, XOR-swizzled with
// swz_k<PV>.  Returns for lane (group G, n = 4 e + qd) the 8 contraction elements
// rbase + 8 G + (0..7) of operand row 32 pp + 8 e + 4 x + qd (two ds_read_b64_tr_b16: source
// lane 4 e + qd addresses row rbase + 8 G + 4 half + e, columns 32 pp + 8 qd + 4 x .. +3).
template <int PV>
__device__ __forceinline__ u32x4 tr_operand(const lds_char* tile, int rbase, int pp, int x, int G, int e, int qd) {
  u32x4 op;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int row = rbase + 8 * G + 4 * half + e;
    const int piece = (4 * pp + qd) ^ swz_k<PV>(row);
    const lds_char* a = tile + (row * PV + piece) * 16 + 8 * x;
    const u32x2 w = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)a));
    op[2 * half] = w[0];
    op[2 * half + 1] = w[1];
  }
  return op;
}

}  // namespace cgdr
