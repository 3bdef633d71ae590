// NT GEMM mainloop shared by the triangle contraction and the wide-channel
// (C >= 256) projection / output kernels:
//   acc = A[x0 .. x0+TX) . B[y0 .. y0+TY)^T   (A: [rows][K], B: [rows][K], bf16)
// on a workgroup of 8 waves (WX along x, 8/WX along y; each wave owns a
// (TX/WX) x (TY/WY) block as MX x MY 16x16 fragments).
//
// K advances in stages of KC (32 or 64) staged by direct global -> LDS loads
// (global_load_lds_dwordx4) into NS buffers: stage s+NS-1 streams in while
// stage s is multiplied.  One fence-free barrier per stage suffices: each
// wave first waits for its own loads of stage s (vmcnt) and its own LDS reads
// of stage s-1 (lgkmcnt), and the buffer refilled at stage s was last read at
// stage s-1.  An LDS row holds the KC elements of one A or B row (KC/8
// chunks of 16 bytes); its slot t holds chunk t ^ f(row) with
// f = (row >> 1) & 3 for KC = 32 and f = row & 7 for KC = 64, which keeps the
// fragment reads of 8 consecutive rows on distinct bank groups.  Every load
// issued is consumed before the mainloop returns (no load is in flight
// afterwards).
//
// KC = 64 reads whole 128-byte lines of every row per stage: a direct load
// that covers 16 rows x 64 bytes moves half as many bytes per cycle from L2
// as one covering 8 rows x 128 bytes.
//
// Orientation (the accumulator layout, see common.hpp):
//   kPairCols = true : acc[i][j] column (lane % 16) is A row
//                      x0 + wx*TX/WX + 16 i + lane%16, its 4 values are B rows
//                      y0 + wy*TY/WY + 16 j + 4 (lane/16) + e;
//   kPairCols = false: the transpose: column = B row y0 + .. + 16 j + lane%16,
//                      values = A rows x0 + .. + 16 i + 4 (lane/16) + e.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace odde {

constexpr int kCk = 32;  // default k per stage

// LDS slot of chunk `chunk` of row `row` (an involution: also the chunk held
// by a slot)
template <int KC>
__device__ __forceinline__ int gemm_swz(int row, int chunk) {
  if constexpr (KC == 32) {
    return chunk ^ ((row >> 1) & 3);
  } else {
    return chunk ^ (row & 7);
  }
}
__device__ __forceinline__ int ct_swz(int row, int chunk) { return gemm_swz<32>(row, chunk); }

template <int TX, int TY, int WX, int KC = kCk>
struct GemmShape {
  static_assert(KC == 32 || KC == 64, "32 or 64 k per stage");
  static constexpr int WY = 8 / WX;
  static constexpr int MX = TX / WX / 16, MY = TY / WY / 16;  // fragments per wave
  static constexpr int CPR = KC / 8;                          // 16-byte chunks per row
  static constexpr int RPO = 64 / CPR;                        // rows per 1 KiB load
  static constexpr int OPS_A = TX / RPO / 8, OPS_B = TY / RPO / 8;  // 1 KiB loads per wave
  static constexpr int OPS = OPS_A + OPS_B;
  static constexpr int STAGE_ELEMS = (TX + TY) * KC;          // bf16 per stage
  static_assert(TX % (16 * 8) == 0 && TY % (16 * 8) == 0, "16-row blocks per wave");
};

// arow(r) / brow(r): pointer to element k = 0 of the tile's A row r
// (r < TX) / B row r (r < TY), each readable for K elements; K a positive
// multiple of KC.  sm holds NS stages of STAGE_ELEMS.
template <int TX, int TY, int WX, int NS, bool kPairCols, int KC = kCk, typename ARow,
          typename BRow>
__device__ __forceinline__ void gemm_nt_mainloop(
    ARow arow, BRow brow, int K, bf16* sm,
    f32x4 (&acc)[GemmShape<TX, TY, WX, KC>::MX][GemmShape<TX, TY, WX, KC>::MY]) {
  using S = GemmShape<TX, TY, WX, KC>;
  static_assert(NS >= 2 && NS <= 4, "2 to 4 stage buffers");
  constexpr int MX = S::MX, MY = S::MY, OPS_A = S::OPS_A, OPS_B = S::OPS_B, OPS = S::OPS;
  constexpr int CPR = S::CPR, RPO = S::RPO;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % WX, wy = w / WX;

  // 1 KiB (RPO rows of KC elements) per wave instruction; wave w loads A
  // blocks w*OPS_A.. and B blocks w*OPS_B..; lane l fills slot l % CPR of row
  // l / CPR of the block.  Source pointers are fixed per lane, only k advances.
  const bf16* src0[OPS];
#pragma unroll
  for (int op = 0; op < OPS; ++op) {
    const bool isb = op >= OPS_A;
    const int blk = isb ? w * OPS_B + (op - OPS_A) : w * OPS_A + op;
    const int row = blk * RPO + l / CPR;
    src0[op] = (isb ? brow(row) : arow(row)) + gemm_swz<KC>(row, l % CPR) * 8;
  }
  auto issue = [&](int st) {
    const int k0 = st * KC;
    bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
#pragma unroll
    for (int op = 0; op < OPS; ++op) {
      const bool isb = op >= OPS_A;
      const int blk = isb ? w * OPS_B + (op - OPS_A) : w * OPS_A + op;
      const bf16* src = src0[op] + k0;
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(base + (isb ? TX * KC : 0) + blk * 512),
          16, 0, 0);
    }
  };

#pragma unroll
  for (int i = 0; i < MX; ++i)
#pragma unroll
    for (int j = 0; j < MY; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fragment rows: the swizzle depends on r16 only (rows step by 16)
  const int arow0 = (wx * (TX / WX) + r16) * KC;
  const int brow0 = TX * KC + (wy * (TY / S::WY) + r16) * KC;

  const int nst = K / KC;
#pragma unroll
  for (int st = 0; st < NS - 1; ++st)
    if (st < nst) issue(st);
  for (int st = 0; st < nst; ++st) {
    // this wave's loads of stage st landed (up to NS-2 later stages in flight)
    const int later = min(nst - 1 - st, NS - 2);
    if (later >= 2) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * OPS) : "memory");
    } else if (later == 1) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(OPS) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // own reads of stage st-1 done
    barrier_nofence();
    if (st + NS - 1 < nst) issue(st + NS - 1);
    const bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
    // all fragments of the stage are requested before the first multiply
    constexpr int KSUB = KC / 32;
    Frag<bf16> fa[KSUB][MX], fb[KSUB][MY];
#pragma unroll
    for (int kk = 0; kk < KSUB; ++kk) {
      const int fsw = gemm_swz<KC>(r16, 4 * kk + g) * 8;
#pragma unroll
      for (int j = 0; j < MY; ++j) fb[kk][j].load(base + brow0 + j * 16 * KC + fsw);
#pragma unroll
      for (int i = 0; i < MX; ++i) fa[kk][i].load(base + arow0 + i * 16 * KC + fsw);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KSUB; ++kk)
#pragma unroll
      for (int i = 0; i < MX; ++i)
#pragma unroll
        for (int j = 0; j < MY; ++j) {
          if constexpr (kPairCols) {
            mma(acc[i][j], fb[kk][j], fa[kk][i]);
          } else {
            mma(acc[i][j], fa[kk][i], fb[kk][j]);
          }
        }
  }
  // the stage buffers may be refilled by the caller's next mainloop
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
}

// Software-pipelined form for KC = 64 and two stage buffers (whole 128-byte
// lines per row and stage), used where one workgroup of 8 waves owns the CU
// (the triangle contraction): the two K32 halves of stage s are multiplied in
// turn; the fragments of half 1 are read under half 0's MFMAs, and those of
// stage s+1's half 0 under half 1's.  The one barrier per stage sits between
// the halves, when every wave holds all of stage s in registers: it frees
// buffer s % 2 for stage s+2 and publishes stage s+1.
// General form: `nst` stages of 64 k, and koff(is_b, st) the element offset
// of stage st within a row of A (is_b false) or B (a uniform value), so the k
// walk may revisit or skip parts of a row (the three-part fp32 contraction
// walks [hi | hi | lo] of A against [hi | lo | hi] of B).
//
// With kBuf the direct loads go through buffer resources based at bufs.a /
// bufs.b (uniform pointers; every A row pointer arow(r) lies within
// bufs.a_bytes of bufs.a, likewise for B): each lane keeps one 32-bit byte
// offset per load, the k advance is the uniform offset and the LDS
// destinations are uniform, so a stage's loads issue no vector instructions
// (the 64-bit form spends a 64-bit add, a v_readfirstlane for M0 and an
// offset add per load).
struct GemmBufs {
  const bf16* a = nullptr;
  uint32_t a_bytes = 0;
  const bf16* b = nullptr;
  uint32_t b_bytes = 0;
};
template <int TX, int TY, int WX, bool kPairCols, bool kBuf = false, typename ARow, typename BRow,
          typename KOff>
__device__ __forceinline__ void gemm_nt_mainloop_pipe64_k(
    ARow arow, BRow brow, int nst, KOff koff, bf16* sm,
    f32x4 (&acc)[GemmShape<TX, TY, WX, 64>::MX][GemmShape<TX, TY, WX, 64>::MY],
    GemmBufs bufs = GemmBufs{}) {
  constexpr int KC = 64, NS = 2;
  using S = GemmShape<TX, TY, WX, KC>;
  constexpr int MX = S::MX, MY = S::MY, OPS_A = S::OPS_A, OPS = S::OPS;
  constexpr int CPR = S::CPR, RPO = S::RPO;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % WX, wy = w / WX;
  const int wu = __builtin_amdgcn_readfirstlane(w);

  const bf16* src0[kBuf ? 1 : OPS];
  uint32_t voff[kBuf ? OPS : 1];
#pragma unroll
  for (int op = 0; op < OPS; ++op) {
    const bool isb = op >= OPS_A;
    const int blk = isb ? w * S::OPS_B + (op - OPS_A) : w * OPS_A + op;
    const int row = blk * RPO + l / CPR;
    const bf16* src = (isb ? brow(row) : arow(row)) + gemm_swz<KC>(row, l % CPR) * 8;
    if constexpr (kBuf)
      voff[op] = (uint32_t)((src - (isb ? bufs.b : bufs.a)) * (int64_t)sizeof(bf16));
    else
      src0[op] = src;
  }
  auto issue = [&](int st) {
    bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
#pragma unroll
    for (int op = 0; op < OPS; ++op) {
      const bool isb = op >= OPS_A;
      const int blk = isb ? wu * S::OPS_B + (op - OPS_A) : wu * OPS_A + op;
      bf16* dst = base + (isb ? TX * KC : 0) + blk * 512;
      if constexpr (kBuf) {
        buffer_load_lds16(isb ? bufs.b : bufs.a, isb ? bufs.b_bytes : bufs.a_bytes, dst, voff[op],
                          (uint32_t)koff(isb, st) * (uint32_t)sizeof(bf16));
      } else {
        __builtin_amdgcn_global_load_lds(
            (const __attribute__((address_space(1))) void*)(src0[op] + koff(isb, st)),
            (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
      }
    }
  };

#pragma unroll
  for (int i = 0; i < MX; ++i)
#pragma unroll
    for (int j = 0; j < MY; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int arow0 = (wx * (TX / WX) + r16) * KC;
  const int brow0 = TX * KC + (wy * (TY / S::WY) + r16) * KC;
  const int fsw0 = gemm_swz<KC>(r16, g) * 8, fsw1 = gemm_swz<KC>(r16, 4 + g) * 8;
  Frag<bf16> fa[2][MX], fb[2][MY];
  auto read_half = [&](auto set_c, int st, int fsw) {
    constexpr int set = decltype(set_c)::value;
    const bf16* base = sm + (st % NS) * S::STAGE_ELEMS;
#pragma unroll
    for (int j = 0; j < MY; ++j) fb[set][j].load(base + brow0 + j * 16 * KC + fsw);
#pragma unroll
    for (int i = 0; i < MX; ++i) fa[set][i].load(base + arow0 + i * 16 * KC + fsw);
  };
  auto mult = [&](auto set_c) {
    constexpr int set = decltype(set_c)::value;
#pragma unroll
    for (int i = 0; i < MX; ++i)
#pragma unroll
      for (int j = 0; j < MY; ++j) {
        if constexpr (kPairCols) {
          mma(acc[i][j], fb[set][j], fa[set][i]);
        } else {
          mma(acc[i][j], fa[set][i], fb[set][j]);
        }
      }
    // one LDS read after each MFMA pair (reads requested just before)
#pragma unroll
    for (int k = 0; k < MX + MY; ++k) {
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MX * MY - 2 * (MX + MY), 0);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  issue(0);
  if (nst > 1) {
    issue(1);
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(OPS) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  barrier_nofence();
  read_half(I0{}, 0, fsw0);
  for (int st = 0; st < nst; ++st) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // half 0 of stage st in registers
    read_half(I1{}, st, fsw1);
    mult(I0{});
    // the wait below is ordered only against memory operations: keep the
    // half's last MFMAs ahead of it, so they run while its reads land
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // all of stage st in registers
    if (st + 1 < nst) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads of stage st+1
      barrier_nofence();  // every wave's; buffer st % 2 is free
      if (st + 2 < nst) issue(st + 2);
    }
    // stage st+1's half 0 (after the last stage: an unused re-read)
    read_half(I0{}, st + 1, fsw0);
    mult(I1{});
  }
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
}

// K contiguous per row: stage st at k = 64 st.
template <int TX, int TY, int WX, bool kPairCols, typename ARow, typename BRow>
__device__ __forceinline__ void gemm_nt_mainloop_pipe64(
    ARow arow, BRow brow, int K, bf16* sm,
    f32x4 (&acc)[GemmShape<TX, TY, WX, 64>::MX][GemmShape<TX, TY, WX, 64>::MY]) {
  gemm_nt_mainloop_pipe64_k<TX, TY, WX, kPairCols>(
      arow, brow, K / 64, [](bool, int st) { return st * 64; }, sm, acc);
}

}  // namespace odde
