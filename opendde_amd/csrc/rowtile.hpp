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

#include <type_traits>

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

// ---------------------------------------------------------------------------
// Raw tile staging by direct global->LDS loads (global_load_lds_dwordx4): the
// next tile's rows stream into LDS while the current tile is computed, with
// no staging registers.  Each wave instruction writes 64 lanes x 16 bytes =
// one contiguous KiB of LDS (lane l at +16*l), so the LDS layout is chosen
// through the source each lane fetches: slot s of row r holds the row's
// 16-byte chunk s ^ (r & 7).  The LayerNorm pass (4 threads per row, each
// reading its quarter chunk by chunk) then hits 16 distinct 16-byte bank
// groups per instruction.
// ---------------------------------------------------------------------------
template <typename ZT, int C>
struct RawTile {
  static constexpr int ROW_BYTES = C * (int)sizeof(ZT);
  static constexpr int BYTES = kTileRows * ROW_BYTES;
  static constexpr int CHUNKS = ROW_BYTES / 16;            // 16-byte chunks per row
  static constexpr int ROWS_PER_OP = 64 / CHUNKS;          // rows per wave instruction
  static constexpr int OPS_PER_WAVE = kTileRows / ROWS_PER_OP / 4;
  static_assert(CHUNKS >= 8 && 64 % CHUNKS == 0, "row must be 8..64 chunks of 16 bytes");
  static_assert(kTileRows % (4 * ROWS_PER_OP) == 0, "tile rows per wave");
};

// Issue the tile's loads.  Tile row r is row min(r0 + r, n - 1) of a view
// whose row 0 starts at `base` with rows `s1` elements apart (rows past the
// end re-read the last real row; raw_tile_ln masks them).  Completion is
// awaited by raw_tile_wait().  kPolicy is the loads' cache policy (kStream for
// a tile the kernel reads once).
//
// Wave w loads tile rows [w R, (w + 1) R), R = kTileRows / 4, one op of
// ROWS_PER_OP rows at a time.  Where all of them exist the addresses are
// affine in the op: the lane's row pointer is formed once and each op adds a
// uniform step; the row swizzle (r & 7) repeats every 8 / ROWS_PER_OP ops,
// so that many lane pointers (chunk offset folded in) cover every op.
template <typename ZT, int C, int kPolicy = 0>
__device__ __forceinline__ void raw_tile_issue(const ZT* base, int64_t s1, int r0, int n,
                                               unsigned char* raw) {
  using T = RawTile<ZT, C>;
  constexpr int RPO = T::ROWS_PER_OP, OPS = T::OPS_PER_WAVE;
  constexpr int P = RPO >= 8 ? 1 : 8 / RPO;  // ops per period of the row swizzle
  static_assert(OPS % P == 0 && (OPS * RPO) % 8 == 0, "swizzle period");
  const int w = __builtin_amdgcn_readfirstlane(wave_id());
  int l = lane_id();
  // the lane offsets below are recomputed per call (a few VALU) rather than
  // hoisted out of the caller's tile loop and kept in registers, which the
  // weight-stationary kernels cannot spare
  asm volatile("" : "+v"(l));
  const int rl = l / T::CHUNKS, cl = l % T::CHUNKS;
  const int first = w * OPS * RPO;  // a multiple of 8: r & 7 = (op * RPO + rl) & 7
  unsigned char* dst = raw + w * OPS * 1024;
  if (r0 + first + OPS * RPO <= n) {
    // buffer loads based at the wave's first row: per lane one 32-bit offset
    // per swizzle phase (row rl, chunk), per op a uniform row step; the
    // wave's rows span less than 4 GiB
    const ZT* wbase = base + (int64_t)(r0 + first) * s1;
    const uint32_t rowb = (uint32_t)((int64_t)rl * s1 * (int64_t)sizeof(ZT));
    const uint32_t step = (uint32_t)((int64_t)RPO * s1 * (int64_t)sizeof(ZT));  // bytes per op
    uint32_t lo[P];
#pragma unroll
    for (int k = 0; k < P; ++k) lo[k] = rowb + (cl ^ ((k * RPO + rl) & 7)) * 16;
#pragma unroll
    for (int op = 0; op < OPS; ++op)
      buffer_load_lds16<kPolicy>(wbase, 0xffffffffu, dst + op * 1024, lo[op % P], op * step);
  } else {
#pragma unroll 1
    for (int op = 0; op < OPS; ++op) {  // one address live at a time
      const int r = first + op * RPO + rl;
      const int chunk = cl ^ (r & 7);
      const unsigned char* src =
          reinterpret_cast<const unsigned char*>(base + (int64_t)min(r0 + r, n - 1) * s1) +
          chunk * 16;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(dst + op * 1024), 16, 0, kPolicy);
    }
  }
}

// All of this workgroup's tile loads have landed in LDS.
__device__ __forceinline__ void raw_tile_wait() {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
}

// LayerNorm of the raw tile into `lds` (row stride TileLD), as stage_ln_tile;
// rows with !valid(r) become zeros.  With `lds_lo` (bf16 only) the rounding
// remainder y - bf16(y) goes there too, so that hi + lo carries y to about
// 16 significant bits (two MFMAs, hi and lo against one weight fragment, then
// replace one bf16 rounding of the activation).  The caller synchronises
// afterwards.
template <typename ZT, typename CT, int C, typename Valid>
__device__ __forceinline__ void raw_tile_ln(const unsigned char* raw, Valid valid,
                                            const float* __restrict__ ln_w,
                                            const float* __restrict__ ln_b, float eps, CT* lds,
                                            CT* lds_lo = nullptr) {
  using T = RawTile<ZT, C>;
  constexpr int Q = C / 4;                        // channels per thread
  constexpr int EPC = 16 / (int)sizeof(ZT);       // elements per chunk
  constexpr int NCH = Q / EPC;                    // chunks per thread
  constexpr int LD = TileLD<CT, C>::value;
  const int t = threadIdx.x;
  const int r = t >> 2, quarter = t & 3;
  const bool ok = valid(r);
  const unsigned char* row = raw + r * T::ROW_BYTES;
  float x[Q];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int chunk = quarter * NCH + k;
    const ZT* src = reinterpret_cast<const ZT*>(row + ((chunk ^ (r & 7)) * 16));
    if constexpr (sizeof(ZT) == 4) {
      load4(src, x + k * EPC);
    } else {
      load8(src, x + k * EPC);
    }
  }
  if (!ok) {
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
    for (int k = 0; k < 4; ++k) y[k] = ok ? (x[e + k] - mean) * rstd * w[k] + b[k] : 0.f;
    store4(dst + e, y[0], y[1], y[2], y[3]);
    if constexpr (sizeof(CT) == 2) {
      if (lds_lo) {
        float lo[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) lo[k] = y[k] - round_to<CT>(y[k]);
        store4(lds_lo + r * LD + quarter * Q + e, lo[0], lo[1], lo[2], lo[3]);
      }
    }
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
template <typename WT, typename FT, int NB, int KS>
__device__ __forceinline__ void load_w_slice(const WT* __restrict__ w, int ld, int o0, int n_out,
                                             Frag<FT> (&f)[NB][KS]) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int t = 0; t < KS; ++t) load_w_frag(w, ld, o0 + 16 * b, n_out, t, f[b][t]);
}
// The same as fp16 fragments of scale * w (load_w_frag_scaled).
template <int NB, int KS>
__device__ __forceinline__ void load_w_slice_scaled(const bf16* __restrict__ w, int ld, int o0,
                                                    int n_out, float scale,
                                                    Frag<f16> (&f)[NB][KS]) {
#pragma unroll
  for (int b = 0; b < NB; ++b)
#pragma unroll
    for (int t = 0; t < KS; ++t) load_w_frag_scaled(w, ld, o0 + 16 * b, n_out, t, scale, f[b][t]);
}

// Output rows of a row-tile kernel: lane (g, r16) holds, for its row, NB
// blocks of 4 consecutive outputs r[cb] (float[4] or f32x4) at channels
// c_base + 16 cb + 4 g.
// With fp32 rows and NB even, blocks 2L and 2L + 1 are slots g and 4 + g of
// one 128-byte line, stored with the streaming policy as whole lines together
// with the row of lane r16 ^ 1 (store_line_pair; `partner_row`, and ok /
// partner_ok, say which rows exist).  Otherwise the blocks are stored one by
// one.  Every lane of the wave must be active.
template <typename ZT, int NB, typename Block>
__device__ __forceinline__ void store_row_blocks(ZT* row, ZT* partner_row, int c_base,
                                                 const Block (&r)[NB], bool ok, bool partner_ok) {
  const int g = lane_id() >> 4;
  if constexpr (std::is_same<ZT, float>::value && NB % 2 == 0) {
#pragma unroll
    for (int L = 0; L < NB / 2; ++L) {
      const f32x4 lo = {r[2 * L][0], r[2 * L][1], r[2 * L][2], r[2 * L][3]};
      const f32x4 hi = {r[2 * L + 1][0], r[2 * L + 1][1], r[2 * L + 1][2], r[2 * L + 1][3]};
      store_line_pair(reinterpret_cast<f32x4*>(row + c_base + 32 * L),
                      reinterpret_cast<f32x4*>(partner_row + c_base + 32 * L), g, lo, hi, ok,
                      partner_ok);
    }
  } else {
    if (!ok) return;
#pragma unroll
    for (int cb = 0; cb < NB; ++cb)
      store4(row + c_base + 16 * cb + 4 * g, r[cb][0], r[cb][1], r[cb][2], r[cb][3]);
  }
}

}  // namespace odde
