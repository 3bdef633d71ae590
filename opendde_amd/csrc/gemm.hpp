// NT GEMM mainloop shared by the triangle contraction and the wide-channel
// (C >= 256) projection / output kernels:
//   acc = A[x0 .. x0+TX) . B[y0 .. y0+TY)^T   (A: [rows][K], B: [rows][K], bf16)
// on a workgroup of 8 waves (WX along x, 8/WX along y; each wave owns a
// (TX/WX) x (TY/WY) block as MX x MY 16x16 fragments).
//
// K advances in stages of 32 staged by direct global -> LDS loads
// (global_load_lds_dwordx4) into NS buffers: stage s+NS-1 streams in while
// stage s is multiplied.  One fence-free barrier per stage suffices: each
// wave first waits for its own loads of stage s (vmcnt) and its own LDS reads
// of stage s-1 (lgkmcnt), and the buffer refilled at stage s was last read at
// stage s-1.  LDS rows are 64 bytes (4 chunks of 16); slot t of row r holds
// chunk t ^ ((r >> 1) & 3), which spreads the K32 fragment reads of 16
// consecutive rows over all banks.  Every load issued is consumed before the
// mainloop returns (no load is in flight afterwards).
//
// Orientation (the accumulator layout, see common.hpp):
//   kPairCols = true : acc[i][j] column (lane % 16) is A row
//                      x0 + wx*TX/WX + 16 i + lane%16, its 4 values are B rows
//                      y0 + wy*TY/WY + 16 j + 4 (lane/16) + e;
//   kPairCols = false: the transpose: column = B row y0 + .. + 16 j + lane%16,
//                      values = A rows x0 + .. + 16 i + 4 (lane/16) + e.
#pragma once

#include "common.hpp"

namespace odde {

constexpr int kCk = 32;  // k per stage

__device__ __forceinline__ int ct_swz(int row, int chunk) { return chunk ^ ((row >> 1) & 3); }

template <int TX, int TY, int WX>
struct GemmShape {
  static constexpr int WY = 8 / WX;
  static constexpr int MX = TX / WX / 16, MY = TY / WY / 16;  // fragments per wave
  static constexpr int OPS_A = TX / 16 / 8, OPS_B = TY / 16 / 8;  // 1 KiB loads per wave
  static constexpr int OPS = OPS_A + OPS_B;
  static constexpr int STAGE_ELEMS = (TX + TY) * kCk;             // bf16 per stage
  static_assert(TX % (16 * 8) == 0 && TY % (16 * 8) == 0, "16-row blocks per wave");
};

// arow(r) / brow(r): pointer to element k = 0 of the tile's A row r
// (r < TX) / B row r (r < TY), each readable for K elements; K a multiple
// of 32 and at least 32 * (NS - 1).  sm holds NS stages of STAGE_ELEMS.
template <int TX, int TY, int WX, int NS, bool kPairCols, typename ARow, typename BRow>
__device__ __forceinline__ void gemm_nt_mainloop(
    ARow arow, BRow brow, int K, bf16* sm,
    f32x4 (&acc)[GemmShape<TX, TY, WX>::MX][GemmShape<TX, TY, WX>::MY]) {
  using S = GemmShape<TX, TY, WX>;
  constexpr int MX = S::MX, MY = S::MY, OPS_A = S::OPS_A, OPS_B = S::OPS_B, OPS = S::OPS;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % WX, wy = w / WX;

  // 1 KiB (16 rows of 64 bytes) per wave instruction; wave w loads A blocks
  // w*OPS_A.. and B blocks w*OPS_B..; source pointers are fixed per lane, only
  // k advances.
  const bf16* src0[OPS];
#pragma unroll
  for (int op = 0; op < OPS; ++op) {
    const bool isb = op >= OPS_A;
    const int blk = isb ? w * OPS_B + (op - OPS_A) : w * OPS_A + op;
    const int row = blk * 16 + (l >> 2);
    src0[op] = (isb ? brow(row) : arow(row)) + ct_swz(row, l & 3) * 8;
  }
  auto issue = [&](int st) {
    const int k0 = st * kCk;
    bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
#pragma unroll
    for (int op = 0; op < OPS; ++op) {
      const bool isb = op >= OPS_A;
      const int blk = isb ? w * OPS_B + (op - OPS_A) : w * OPS_A + op;
      const bf16* src = src0[op] + k0;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(base + (isb ? TX * kCk : 0) + blk * 512),
          16, 0, 0);
    }
  };

#pragma unroll
  for (int i = 0; i < MX; ++i)
#pragma unroll
    for (int j = 0; j < MY; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fragment offsets: the swizzle depends on r16 only (rows step by 16)
  const int fsw = ct_swz(r16, g) * 8;
  const int aoff = (wx * (TX / WX) + r16) * kCk + fsw;
  const int boff = TX * kCk + (wy * (TY / S::WY) + r16) * kCk + fsw;

  const int nst = K / kCk;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st) issue(st);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st landed (up to NS-2 later stages in flight)
    const int ahead = min(nst - 1 - st, NS - 2);
    if (ahead >= 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * OPS) : "memory");
    } else if (ahead == 1) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(OPS) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // own reads of stage st-1 done
    barrier_nofence();
    if (st + NS - 1 < nst) issue(st + NS - 1);
    const bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
    Frag<bf16> af[MX], bfr[MY];
#pragma unroll
    for (int j = 0; j < MY; ++j) bfr[j].load(base + boff + j * 16 * kCk);
#pragma unroll
    for (int i = 0; i < MX; ++i) af[i].load(base + aoff + i * 16 * kCk);
#pragma unroll
    for (int i = 0; i < MX; ++i)
#pragma unroll
      for (int j = 0; j < MY; ++j) {
        if constexpr (kPairCols) {
          mma(acc[i][j], bfr[j], af[i]);
        } else {
          mma(acc[i][j], af[i], bfr[j]);
        }
      }
  }
  // the stage buffers may be refilled by the caller's next mainloop
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
}

}  // namespace odde
