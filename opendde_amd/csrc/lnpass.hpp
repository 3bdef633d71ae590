// LayerNorm passes that feed the wide-channel GEMM kernels (gemm.hpp) with
// normalised bf16 rows: the A operand of an NT GEMM is then a plain
// row-major [rows][C] matrix that the mainloop streams into LDS by direct
// loads.  Statistics are f32, two-pass, over the C channels of a row.
#pragma once

#include "common.hpp"

namespace odde {

// out[m][:] = LN(z[x][y][:]) for m = x * R + y, x < X, y < R, where
// z[x][y][c] = z + x * s0 + y * s1 + c; rows with x >= n or y >= n (padding)
// are written as zeros.  16 lanes per row, C / 16 contiguous channels per
// lane (16-byte loads and stores); grid-stride over rows.
template <typename ZT, int C>
__global__ __launch_bounds__(256) void ln_view_bf16_kernel(const ZT* __restrict__ z, int64_t s0,
                                                           int64_t s1, int n, int X, int R,
                                                           const float* __restrict__ ln_w,
                                                           const float* __restrict__ ln_b,
                                                           float eps, bf16* __restrict__ out) {
  constexpr int E = C / 16;                      // channels per lane
  constexpr int LV = E * (int)sizeof(ZT) / 16;   // 16-byte loads per lane
  constexpr int SV = E * 2 / 16;                 // 16-byte stores per lane
  static_assert(E % 8 == 0, "C a multiple of 128");
  const int sub = threadIdx.x & 15;
  const int64_t rows = (int64_t)X * R;
  const int64_t r0 = (int64_t(blockIdx.x) * 256 + threadIdx.x) >> 4;
  const int64_t nr = (int64_t(gridDim.x) * 256) >> 4;
  float lw[E], lb[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    lw[e] = ln_w[sub * E + e];
    lb[e] = ln_b[sub * E + e];
  }
  for (int64_t r = r0; r < rows; r += nr) {  // uniform over the 16 lanes of a row
    const int x = (int)(r / R), y = (int)(r % R);
    const bool valid = x < n && y < n;
    float v[E];
    if (valid) {
      const ZT* src = z + (int64_t)x * s0 + (int64_t)y * s1 + sub * E;
#pragma unroll
      for (int k = 0; k < LV; ++k) {
        const f32x4 c = reinterpret_cast<const f32x4*>(src)[k];
        if constexpr (sizeof(ZT) == 4) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v[4 * k + e] = c[e];
        } else {
          const bf16x8 h = __builtin_bit_cast(bf16x8, c);
#pragma unroll
          for (int e = 0; e < 8; ++e) v[8 * k + e] = (float)h[e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = 0.f;
    }
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) s += v[e];
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o, 64);
    const float mean = s * (1.0f / C);
    float q = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float d = v[e] - mean;
      q += d * d;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) q += __shfl_xor(q, o, 64);
    const float rstd = rsqrtf(q * (1.0f / C) + eps);
    bf16* dst = out + r * C + sub * E;
#pragma unroll
    for (int k = 0; k < SV; ++k) {
      bf16x8 h;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = 8 * k + e;
        h[e] = (bf16)(valid ? (v[c] - mean) * rstd * lw[c] + lb[c] : 0.f);
      }
      reinterpret_cast<bf16x8*>(dst)[k] = h;
    }
  }
}

// out[x * np + y][:] = LN(P[:][x][y]) for the channel-major P[CH][np][np]
// (bf16): a workgroup transposes the 64-column block P[:, x, y0..y0+63]
// through LDS, then normalises its 64 rows in two passes of 32, 8 threads
// per row: thread part p owns the 16-byte chunks p, p + 8, ... of the row, so
// one store instruction writes 8 whole 128-byte lines.  Grid (np / 64, np).
// Columns with x >= n or y >= n are written as zeros.  P is read once and the
// rows are written once: both with the streaming policy.
// In the transposed tile, row y keeps channel c at column
// c ^ (8 * ((y >> 3) & 7)) (8-channel groups permuted by y / 8): the lanes of
// one transposing store cover 8 channels at 8 rows y0 + 8k + e, which then
// fall on distinct bank groups instead of one.
template <int CH>
__global__ __launch_bounds__(256) void ln_transpose_bf16_kernel(const bf16* __restrict__ P, int np,
                                                                int n,
                                                                const float* __restrict__ ln_w,
                                                                const float* __restrict__ ln_b,
                                                                float eps, bf16* __restrict__ out) {
  constexpr int LD = CH + 8;     // LDS row stride (elements) of the transposed tile
  constexpr int CPT = CH / 64;   // 16-byte chunks per thread in the LayerNorm pass
  static_assert(CH % 64 == 0, "the column permutation stays within 64-channel groups");
  __shared__ __attribute__((aligned(16))) bf16 t[64 * LD];
  const int x = blockIdx.y, y0 = blockIdx.x * 64;
  const bf16* src = P + (size_t)x * np + y0;
  // unit u: channels 4 (u >> 3) .. + 3 at columns 8 (u & 7) .. + 7, four
  // 16-byte loads (eight lanes read a channel's whole 128-byte line),
  // transposed in registers into eight 8-byte LDS stores (one per column).
  // Channel c of column yy sits at c ^ (8 (yy >> 3)): 4-channel groups stay
  // contiguous under the swizzle.
  constexpr int NU = CH * 2;                 // units
  constexpr int UPT = (NU + 255) / 256;      // units per thread
  uint32_t ld[UPT][4][4];                    // [unit][channel][column pair]
#pragma unroll
  for (int k = 0; k < UPT; ++k) {  // all loads in flight before the first LDS store
    const int u = threadIdx.x + 256 * k, c4 = (u >> 3) * 4, yy = (u & 7) * 8;
    if (NU % 256 == 0 || u < NU) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x4 v =
            load_stream(reinterpret_cast<const f32x4*>(src + (size_t)(c4 + i) * np * np + yy));
#pragma unroll
        for (int e = 0; e < 4; ++e) ld[k][i][e] = __float_as_uint(v[e]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < UPT; ++k) {
    const int u = threadIdx.x + 256 * k, c4 = (u >> 3) * 4, yy = (u & 7) * 8;
    if (!(NU % 256 == 0 || u < NU)) continue;
    const int cs = c4 ^ (8 * ((yy >> 3) & 7));
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      // columns yy + 2p (low halves) and yy + 2p + 1 (high halves) of the
      // four channels: byte permutes pair channel i with i + 1
      const uint32_t lo01 = __builtin_amdgcn_perm(ld[k][1][p], ld[k][0][p], 0x05040100u);
      const uint32_t lo23 = __builtin_amdgcn_perm(ld[k][3][p], ld[k][2][p], 0x05040100u);
      const uint32_t hi01 = __builtin_amdgcn_perm(ld[k][1][p], ld[k][0][p], 0x07060302u);
      const uint32_t hi23 = __builtin_amdgcn_perm(ld[k][3][p], ld[k][2][p], 0x07060302u);
      *reinterpret_cast<uint2*>(t + (yy + 2 * p) * LD + cs) = make_uint2(lo01, lo23);
      *reinterpret_cast<uint2*>(t + (yy + 2 * p + 1) * LD + cs) = make_uint2(hi01, hi23);
    }
  }
  __syncthreads();
  const int part = threadIdx.x & 7;
#pragma unroll
  for (int pass = 0; pass < 2; ++pass) {
    const int yl = 32 * pass + (threadIdx.x >> 3);
    const int y = y0 + yl;
    const bool valid = x < n && y < n;
    const bf16* row = t + yl * LD;
    const int sw = 8 * ((yl >> 3) & 7);
    float v[CPT][8];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const bf16x8 h = *reinterpret_cast<const bf16x8*>(row + ((8 * (8 * k + part)) ^ sw));
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v[k][e] = (float)h[e];
        s += v[k][e];
      }
    }
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    s += __shfl_xor(s, 4, 64);
    const float mean = s * (1.0f / CH);
    float q = 0.f;
#pragma unroll
    for (int k = 0; k < CPT; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[k][e] - mean;
        q += d * d;
      }
    q += __shfl_xor(q, 1, 64);
    q += __shfl_xor(q, 2, 64);
    q += __shfl_xor(q, 4, 64);
    const float rstd = rsqrtf(q * (1.0f / CH) + eps);
    bf16* dst = out + ((size_t)x * np + y) * CH;
#pragma unroll
    for (int k = 0; k < CPT; ++k) {
      const int c0 = 8 * (8 * k + part);  // LayerNorm parameters as 16-byte vectors
      float lw[8], lb[8];
      load4(ln_w + c0, lw);
      load4(ln_w + c0 + 4, lw + 4);
      load4(ln_b + c0, lb);
      load4(ln_b + c0 + 4, lb + 4);
      bf16x8 h;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        h[e] = (bf16)(valid ? (v[k][e] - mean) * rstd * lw[e] + lb[e] : 0.f);
      store_stream(reinterpret_cast<bf16x8*>(dst + c0), h);
    }
  }
}

}  // namespace odde
