// Weight-stationary row tiles for the HBM-bound projection / epilogue kernels.
//
// A workgroup of 4 waves owns a tile of 64 pair rows at a time (persistent
// over many tiles).  The 256 threads stage the tile's rows through a fused
// LayerNorm into LDS (4 threads per row, C/4 channels each, fp32 statistics,
// two-pass), then every wave reads K32 fragments of all 64 rows from LDS and
// multiplies them with the slice of the weight matrix it keeps in registers
// for the whole kernel.  Weight bytes are fetched once per workgroup instead
// of once per 16 rows, so the kernels stream z and their outputs at HBM rate.
#pragma once

#include "common.hpp"

namespace odde {

constexpr int kTileRows = 64;

// LDS row stride (elements) for a tile of C channels: +16 bytes breaks the
// bank aliasing of power-of-two rows for 16-byte fragment reads.
template <typename CT, int C>
struct TileLD {
  static constexpr int value = C + 16 / (int)sizeof(CT);
};

// Stage 64 rows x C channels, LayerNorm'd, into `lds` (row stride TileLD).
// row_ptr(r) gives row r's first element (or nullptr for an invalid row,
// which is staged as zeros).  All 256 threads participate; the caller
// synchronises afterwards.
template <typename ZT, typename CT, int C, typename RowPtr>
__device__ __forceinline__ void stage_ln_tile(RowPtr row_ptr, const float* __restrict__ ln_w,
                                              const float* __restrict__ ln_b, float eps, CT* lds) {
  constexpr int Q = C / 4;  // channels per thread
  constexpr int LD = TileLD<CT, C>::value;
  const int t = threadIdx.x;
  const int r = t >> 2, quarter = t & 3;
  const ZT* p = row_ptr(r);
  float x[Q];
  if (p) {
#pragma unroll
    for (int e = 0; e < Q; e += 8) load8(p + quarter * Q + e, x + e);
  } else {
#pragma unroll
    for (int e = 0; e < Q; ++e) x[e] = 0.f;
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < Q; ++e) s += x[e];
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  const float mean = s * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < Q; ++e) {
    const float d = x[e] - mean;
    q += d * d;
  }
  q += __shfl_xor(q, 1, 64);
  q += __shfl_xor(q, 2, 64);
  const float rstd = rsqrtf(q * (1.0f / C) + eps);
  CT* dst = lds + r * LD + quarter * Q;
#pragma unroll
  for (int e = 0; e < Q; e += 4) {
    float w[4], b[4];
    load4(ln_w + quarter * Q + e, w);
    load4(ln_b + quarter * Q + e, b);
    float y[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) y[k] = p ? (x[e + k] - mean) * rstd * w[k] + b[k] : 0.f;
    store4(dst + e, y[0], y[1], y[2], y[3]);
  }
}

// K32 fragments of tile row (rb*16 + lane%16), all C/32 contraction steps.
template <typename CT, int C>
__device__ __forceinline__ void tile_frags(const CT* lds, int rb, Frag<CT> (&f)[C / 32]) {
  constexpr int LD = TileLD<CT, C>::value;
  const int g = lane_id() >> 4, r16 = lane_id() & 15;
  const CT* row = lds + (rb * 16 + r16) * LD + 8 * g;
#pragma unroll
  for (int t = 0; t < C / 32; ++t) f[t].load(row + 32 * t);
}

// Weight fragments kept in registers: NB column blocks of 16 output rows of
// W[out][K] starting at output o0 (rows >= n_out are zero).
template <typename CT, int NB, int KS>
__device__ __forceinline__ void load_w_slice(const CT* __restrict__ w, int ld, int o0, int n_out,
                                             Frag<CT> (&f)[NB][KS]) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int t = 0; t < KS; ++t) load_w_frag(w, ld, o0 + 16 * b, n_out, t, f[b][t]);
}

}  // namespace odde
