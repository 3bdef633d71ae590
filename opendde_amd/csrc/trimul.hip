// Triangle multiplicative update (outgoing / incoming) for gfx950.
//
// Three kernels, stream ordered:
//   1. trimul_proj     — LN_in + the four gated projections per pair row,
//                        a = mask*sigmoid(x Wag^T)*(x Wap^T) (b likewise),
//                        written channel-major as A[c][x][k], B[c][y][k] so
//                        that the contraction is one NT GEMM per channel.
//                        Incoming reads z through swapped strides, which
//                        writes a[k,i] at A[c][i][k]: no transposed copy.
//   2. trimul_contract — P[c][x][y] = sum_k A[c][x][k] B[c][y][k]: a batched
//                        NT GEMM on MFMA, 128x128 tiles, LDS-staged K blocks,
//                        XCD-aware tile order (all tiles of one channel on
//                        one XCD so A_c and B_c stay in that XCD's L2).
//   3. trimul_out      — per pair row: LN_out over the channel-major P
//                        (transposed through LDS), W_z, times
//                        sigmoid(W_g LN_in(z)) recomputed from z (which is
//                        read for the residual anyway), plus the residual.
//
// Workspace (CT = compute type, Np = N rounded up to 128):
//   A, B, P : [Ch][Np][Np]
#include <string.h>

#include "common.hpp"
#include "gemm.hpp"
#include "lnpass.hpp"
#include "rowtile.hpp"
#include "runtime.hpp"

namespace odde {

// ---------------------------------------------------------------------------
// 1. projection
// ---------------------------------------------------------------------------
template <typename ZT, typename CT>
struct TrimulProjArgs {
  const ZT* z;
  int64_t z_s0, z_s1;
  const float* mask;
  int64_t m_s0, m_s1;
  const float* ln_w;
  const float* ln_b;
  const CT* wp;  // [2Ch][C]  a_p rows then b_p rows
  const CT* wg;  // [2Ch][C]  a_g rows then b_g rows
  CT* A;
  CT* B;
  int n, np, ch;
  float eps;
};

// Wave w of a workgroup owns pair rows (x, y0 + 16 w .. + 15) for kRB
// consecutive first indices x: every weight fragment it reads from L2 serves
// kRB row blocks (the fp32 form, whose weights are too large to hold, is
// bound by those reads).  kX3 (f32 compute, ODDE_F32X3): A and B are written
// as bf16 rows of 2 Np, [hi | lo] with hi = bf16(a) and lo = bf16(a - hi),
// for the three-part contraction.  kX3Mul (f32 compute, ODDE_F32X3): the
// projections' products in three bf16 parts (rows split once after the
// LayerNorm, weight fragments as they are read).  blockIdx.z of gridDim.z
// takes channels [z Ch / Z, (z + 1) Ch / Z) (small grids).  kStage (f32
// data): the four weight row blocks of each 16-channel block (fp32 rows, or
// the three-part split rows: the same bytes) are staged in LDS, double-
// buffered, and shared by the workgroup's 4 waves, so a weight byte fetched
// from L2 serves 64 kRB rows instead of 16 kRB.
template <typename ZT, typename CT, int kC, int kRB = 1, bool kX3 = false, bool kX3Mul = false,
          bool kStage = false>
__global__ __launch_bounds__(256) void trimul_proj_kernel(TrimulProjArgs<ZT, CT> a) {
  constexpr int C = kC * 32;
  using MF = MulFrag<CT, kX3Mul>;
  static_assert(!kStage || sizeof(CT) == 4, "staging: f32 weights");
  constexpr int WL = C + 4;                     // staged row stride (floats)
  constexpr int CHUNK = 4 * 16 * WL;            // a_p, a_g, b_p, b_g rows of one block
  constexpr int PT = 4 * 16 * C / 4;            // 16-byte pieces per chunk
  constexpr int PPT = (PT + 255) / 256;
  __shared__ __attribute__((aligned(16))) float wsm[kStage ? 2 * CHUNK : 4];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int y0 = blockIdx.x * 64 + w * 16;
  const int yl = y0 + r16;
  // mask for the four rows y0+4g .. +3 this lane writes
  const int yb = y0 + 4 * g;
  MF xf[kRB][kC];
  float mk[kRB][4];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int x_ = blockIdx.y * kRB + rb;  // first index of the (strided) view
    const bool valid = x_ < a.n && yl < a.n;
    const ZT* rowp =
        a.z + (int64_t)(valid ? x_ : 0) * a.z_s0 + (int64_t)(valid ? yl : 0) * a.z_s1;
    {
      Frag<CT> xt[kC];
      ln_rows_to_frags<ZT, CT, C>(rowp, valid, a.ln_w, a.ln_b, a.eps, xt);
#pragma unroll
      for (int t = 0; t < kC; ++t) to_mul(xt[t], xf[rb][t]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int y = yb + r;
      mk[rb][r] = (x_ < a.n && y < a.n)
                      ? (a.mask ? a.mask[(int64_t)x_ * a.m_s0 + (int64_t)y * a.m_s1] : 1.0f)
                      : 0.f;
    }
  }
  const int ch = a.ch, np = a.np;
  const int cb_per = (ch / 16) / (int)gridDim.z;
  const int cb_lo = (int)blockIdx.z * cb_per, cb_hi = cb_lo + cb_per;
  // staging: piece q of block cb is matrix m = q / (4 C) (a_p, a_g, b_p,
  // b_g), row r, 16-byte column piece c4
  f32x4 wreg[kStage ? PPT : 1];
  auto wload = [&](int cb) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      if (PT % 256 == 0 || q < PT) {
        const int m = q / (4 * C), u = q % (4 * C), r = u / (C / 4), c4 = u % (C / 4);
        const CT* src = (m & 1) ? a.wg : a.wp;
        wreg[k] = *reinterpret_cast<const f32x4*>(src + (size_t)((m >> 1) * ch + cb * 16 + r) * C +
                                                  4 * c4);
      }
    }
  };
  auto wstore = [&](int buf) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      if (PT % 256 == 0 || q < PT) {
        const int m = q / (4 * C), u = q % (4 * C), r = u / (C / 4), c4 = u % (C / 4);
        *reinterpret_cast<f32x4*>(&wsm[buf * CHUNK + (m * 16 + r) * WL + 4 * c4]) = wreg[k];
      }
    }
  };
  if constexpr (kStage) {
    wload(cb_lo);
    wstore(0);
    if (cb_lo + 1 < cb_hi) wload(cb_lo + 1);
    __syncthreads();
  }
  for (int cb = cb_lo; cb < cb_hi; ++cb) {
    f32x4 ap[kRB], ag[kRB], bp[kRB], bg[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) ap[rb] = ag[rb] = bp[rb] = bg[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* wsb = wsm + ((cb - cb_lo) & 1) * CHUNK + r16 * WL;
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      if constexpr (kStage) staged_w_frag(wsb, C, t, f);
      else load_w_frag(a.wp, C, cb * 16, 2 * ch, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ap[rb], xf[rb][t], f);
      if constexpr (kStage) staged_w_frag(wsb + 16 * WL, C, t, f);
      else load_w_frag(a.wg, C, cb * 16, 2 * ch, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ag[rb], xf[rb][t], f);
      if constexpr (kStage) staged_w_frag(wsb + 32 * WL, C, t, f);
      else load_w_frag(a.wp, C, ch + cb * 16, 2 * ch, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(bp[rb], xf[rb][t], f);
      if constexpr (kStage) staged_w_frag(wsb + 48 * WL, C, t, f);
      else load_w_frag(a.wg, C, ch + cb * 16, 2 * ch, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(bg[rb], xf[rb][t], f);
    }
    const int c = cb * 16 + r16;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int x_ = blockIdx.y * kRB + rb;
      float va[4], vb[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        va[r] = mk[rb][r] * sigmoidf_(ag[rb][r]) * ap[rb][r];
        vb[r] = mk[rb][r] * sigmoidf_(bg[rb][r]) * bp[rb][r];
      }
      if constexpr (kX3) {
        const size_t off = ((size_t)c * np + x_) * 2 * np + yb;
        bf16x4 ha, la, hb, lb;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          ha[r] = (bf16)va[r];
          la[r] = (bf16)(va[r] - (float)ha[r]);
          hb[r] = (bf16)vb[r];
          lb[r] = (bf16)(vb[r] - (float)hb[r]);
        }
        bf16* A16 = reinterpret_cast<bf16*>(a.A) + off;
        bf16* B16 = reinterpret_cast<bf16*>(a.B) + off;
        *reinterpret_cast<bf16x4*>(A16) = ha;
        *reinterpret_cast<bf16x4*>(A16 + np) = la;
        *reinterpret_cast<bf16x4*>(B16) = hb;
        *reinterpret_cast<bf16x4*>(B16 + np) = lb;
      } else {
        const size_t off = ((size_t)c * np + x_) * np + yb;
        store4(a.A + off, va[0], va[1], va[2], va[3]);
        store4(a.B + off, vb[0], vb[1], vb[2], vb[3]);
      }
    }
    if constexpr (kStage) {
      // buffer (cb + 1 - cb_lo) & 1 was last read in block cb - 1, before
      // the barrier that ended it
      if (cb + 1 < cb_hi) {
        wstore((cb + 1 - cb_lo) & 1);
        if (cb + 2 < cb_hi) wload(cb + 2);
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// 2. contraction: batched NT GEMM, P_c = A_c B_c^T
// ---------------------------------------------------------------------------
template <typename CT>
struct ContractArgs {
  const CT* A;
  const CT* B;
  CT* P;
  int np, ch;
};

template <typename CT> struct ContractCfg;
template <> struct ContractCfg<bf16> { static constexpr int BK = 64; static constexpr int PAD = 8; };
template <> struct ContractCfg<float> { static constexpr int BK = 32; static constexpr int PAD = 4; };

template <typename CT>
__global__ __launch_bounds__(256) void trimul_contract_kernel(ContractArgs<CT> a) {
  constexpr int BK = ContractCfg<CT>::BK;
  constexpr int LD = BK + ContractCfg<CT>::PAD;
  constexpr int VEC = 16 / sizeof(CT);            // elements per 16-byte chunk
  constexpr int CHUNKS = 128 * BK / VEC;          // chunks per operand tile
  __shared__ __attribute__((aligned(16))) CT As[128 * LD];
  __shared__ __attribute__((aligned(16))) CT Bs[128 * LD];

  const int T = a.np / 128;
  const int tiles = T * T;
  // XCD-aware order: workgroup ids are dealt round-robin over 8 XCDs; give
  // every tile of one channel to the same XCD when the channel count allows.
  int bid = blockIdx.x, c, tile;
  if ((a.ch & 7) == 0) {
    const int xcd = bid & 7, local = bid >> 3;
    c = (local / tiles) * 8 + xcd;
    tile = local % tiles;
  } else {
    c = bid / tiles;
    tile = bid % tiles;
  }
  const int x0 = (tile / T) * 128, y0 = (tile % T) * 128;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wm = w >> 1, wn = w & 1;
  const size_t plane = (size_t)a.np * a.np;
  const CT* Ab = a.A + c * plane + (size_t)x0 * a.np;
  const CT* Bb = a.B + c * plane + (size_t)y0 * a.np;

  f32x4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int k0 = 0; k0 < a.np; k0 += BK) {
#pragma unroll
    for (int it = 0; it < CHUNKS / 256; ++it) {
      const int ci = threadIdx.x + it * 256;
      const int r = ci / (BK / VEC), cc = (ci % (BK / VEC)) * VEC;
      *reinterpret_cast<f32x4*>(&As[r * LD + cc]) =
          *reinterpret_cast<const f32x4*>(Ab + (size_t)r * a.np + k0 + cc);
      *reinterpret_cast<f32x4*>(&Bs[r * LD + cc]) =
          *reinterpret_cast<const f32x4*>(Bb + (size_t)r * a.np + k0 + cc);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; kk += 32) {
      Frag<CT> af[4], bfr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        af[i].load(&As[(wm * 64 + i * 16 + r16) * LD + kk + 8 * g]);
        bfr[i].load(&Bs[(wn * 64 + i * 16 + r16) * LD + kk + 8 * g]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) mma(acc[i][j], bfr[j], af[i]);
    }
    __syncthreads();
  }
  // acc[i][j]: column = row x (x0 + 64wm + 16i + r16), rows y = y0 + 64wn + 16j + 4g + r
  CT* Pb = a.P + c * plane;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int xx = x0 + wm * 64 + i * 16 + r16;
      const int yy = y0 + wn * 64 + j * 16 + 4 * g;
      store4(Pb + (size_t)xx * a.np + yy, acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
    }
}

// Large-tile form (bf16, Np a multiple of 256): TX x TY tiles per workgroup
// of 8 waves, the shared NT mainloop (gemm.hpp) over k = 0..Np.
template <int TX, int TY, int WX, int NS, int KC, bool kPipe = false>
__global__ __launch_bounds__(512) void trimul_contract_big_kernel(ContractArgs<bf16> a) {
  using S = GemmShape<TX, TY, WX, KC>;
  static_assert(!kPipe || (KC == 64 && NS == 2), "the pipelined mainloop: two 64-k stages");
  __shared__ __attribute__((aligned(16))) bf16 sm[NS * S::STAGE_ELEMS];
  const int TXn = a.np / TX, TYn = a.np / TY;
  const int tiles = TXn * TYn;
  int bid = blockIdx.x, c, tile;
  if ((a.ch & 7) == 0) {  // all tiles of a channel on one XCD
    const int xcd = bid & 7, local = bid >> 3;
    c = (local / tiles) * 8 + xcd;
    tile = local % tiles;
  } else {
    c = bid / tiles;
    tile = bid % tiles;
  }
  const int x0 = (tile / TYn) * TX, y0 = (tile % TYn) * TY;
  const size_t plane = (size_t)a.np * a.np;
  f32x4 acc[S::MX][S::MY];
  const bf16* Ab = a.A + c * plane + (size_t)x0 * a.np;
  const bf16* Bb = a.B + c * plane + (size_t)y0 * a.np;
  // B row r of the tile (staged in LDS row r) is column y0 + perm(r): within
  // each 32 rows, row block 2p + b, MFMA row m is column 8 (m >> 2) + 4 b +
  // (m & 3), so a lane's results of row blocks 2p and 2p + 1 are 8
  // consecutive columns (one 16-byte store)
  auto arow = [&](int r) { return Ab + (size_t)r * a.np; };
  auto brow = [&](int r) {
    const int m = r & 15;
    return Bb + (size_t)((r & ~31) + 8 * (m >> 2) + 4 * ((r >> 4) & 1) + (m & 3)) * a.np;
  };
  if constexpr (kPipe) {
    // buffer-resource loads based at the tile's first A and B rows
    GemmBufs bufs;
    bufs.a = Ab;
    bufs.a_bytes = (uint32_t)((size_t)TX * a.np * sizeof(bf16));
    bufs.b = Bb;
    bufs.b_bytes = (uint32_t)((size_t)TY * a.np * sizeof(bf16));
    gemm_nt_mainloop_pipe64_k<TX, TY, WX, true, true>(
        arow, brow, a.np / 64, [](bool, int st) { return st * 64; }, sm, acc, bufs);
  } else
    gemm_nt_mainloop<TX, TY, WX, NS, true, KC>(arow, brow, a.np, sm, acc);
  // acc[i][j]: column = row x (x0 + wx*TX/WX + 16i + r16); rows = columns
  // y0 + wy*TY/WY + 16 (j & ~1) + 8g + 4 (j & 1) + r
  // Row blocks j, j + 1 give a lane 8 consecutive columns (slot g of a 64-
  // column, 128-byte line of its row), row blocks j + 2, j + 3 slot 4 + g of
  // the same line; lanes r16 and r16 ^ 1 (rows xx, xx ^ 1) complete each
  // other's lines, stored whole with the streaming policy (store_line_pair).
  static_assert(S::MY % 4 == 0 && (TY / S::WY) % 64 == 0, "row blocks form whole lines");
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % WX, wy = w / WX;
  bf16* Pb = a.P + c * plane;
#pragma unroll
  for (int i = 0; i < S::MX; ++i)
#pragma unroll
    for (int j = 0; j < S::MY; j += 4) {
      const int xx = x0 + wx * (TX / WX) + i * 16 + r16;
      const int y = y0 + wy * (TY / S::WY) + j * 16;
      bf16x8 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = (bf16)acc[i][j][e];
        lo[4 + e] = (bf16)acc[i][j + 1][e];
        hi[e] = (bf16)acc[i][j + 2][e];
        hi[4 + e] = (bf16)acc[i][j + 3][e];
      }
      store_line_pair(reinterpret_cast<bf16x8*>(Pb + (size_t)xx * a.np + y),
                      reinterpret_cast<bf16x8*>(Pb + (size_t)(xx ^ 1) * a.np + y), g, lo, hi);
    }
}

// Np >= 768: 256 x 256 tiles staged 64 k at a time (whole 128-byte lines of
// each row; 128 KiB of LDS, one workgroup per CU), software-pipelined, each
// wave a 64 x 128 block; Np = 512: 256 x 128 tiles staged 32 k at a time
// (two workgroups per CU), which keeps more workgroups per channel.  Chosen
// by measurement on MI355X (N = 1024: the pipelined loop 0.311 / 0.281 ms
// outgoing / incoming against 0.317 / 0.290 ms for the plain one; deeper
// 32-k staging, with or without a k-blocked operand layout, was slower;
// N = 768: 0.138 against 0.152 ms for the 256 x 128 form).
// ODDE_CONTRACT_TILE=256x256 or 256x128 overrides the choice by Np (tuning).
inline int contract_tile_override() {
  static const int v = [] {
    const char* e = getenv("ODDE_CONTRACT_TILE");
    if (!e) return 0;
    if (strcmp(e, "256x256") == 0) return 1;
    if (strcmp(e, "256x128") == 0) return 2;
    return 0;
  }();
  return v;
}

inline void launch_contract_big(const ContractArgs<bf16>& k, int np, int ch, hipStream_t st) {
  const int ov = contract_tile_override();
  // 256 x 256 from Np = 768 up (N = 768: 0.152 -> 0.138 ms against 256 x 128)
  if (ov == 1 || (ov == 0 && np >= 768)) {
    const int tiles = (np / 256) * (np / 256);
    hipLaunchKernelGGL((trimul_contract_big_kernel<256, 256, 4, 2, 64, true>), dim3(tiles * ch),
                       dim3(512), 0, st, k);
  } else {
    const int tiles = (np / 256) * (np / 128);
    hipLaunchKernelGGL((trimul_contract_big_kernel<256, 128, 4, 3, 32>), dim3(tiles * ch), dim3(512),
                       0, st, k);
  }
}

// Three-part fp32 contraction (ODDE_F32X3): A and B rows of 2 Np bf16,
// [hi | lo]; P = A_hi B_hi^T + A_hi B_lo^T + A_lo B_hi^T as one NT GEMM over
// k = 3 Np, whose walk visits hi, hi, lo of each A row against hi, lo, hi of
// each B row (256 x 256 tiles, the pipelined 64-k mainloop); P in fp32.
__global__ __launch_bounds__(512) void trimul_contract_x3_kernel(ContractArgs<bf16> a, float* P) {
  constexpr int TX = 256, TY = 256, WX = 4;
  using S = GemmShape<TX, TY, WX, 64>;
  __shared__ __attribute__((aligned(16))) bf16 sm[2 * S::STAGE_ELEMS];
  const int TXn = a.np / TX, TYn = a.np / TY;
  const int tiles = TXn * TYn;
  int bid = blockIdx.x, c, tile;
  if ((a.ch & 7) == 0) {  // all tiles of a channel on one XCD
    const int xcd = bid & 7, local = bid >> 3;
    c = (local / tiles) * 8 + xcd;
    tile = local % tiles;
  } else {
    c = bid / tiles;
    tile = bid % tiles;
  }
  const int x0 = (tile / TYn) * TX, y0 = (tile % TYn) * TY;
  const int ld = 2 * a.np;
  const size_t plane = (size_t)a.np * ld;
  f32x4 acc[S::MX][S::MY];
  const bf16* Ab = a.A + c * plane + (size_t)x0 * ld;
  const bf16* Bb = a.B + c * plane + (size_t)y0 * ld;
  // B rows staged in the paired-row order of trimul_contract_big_kernel
  auto arow = [&](int r) { return Ab + (size_t)r * ld; };
  auto brow = [&](int r) {
    const int m = r & 15;
    return Bb + (size_t)((r & ~31) + 8 * (m >> 2) + 4 * ((r >> 4) & 1) + (m & 3)) * ld;
  };
  const int nst0 = a.np / 64;
  auto koff = [nst0](bool isb, int st) {
    const int seg = st / nst0, k = st - seg * nst0;
    return (k + ((isb ? seg == 1 : seg == 2) ? nst0 : 0)) * 64;
  };
  GemmBufs bufs;
  bufs.a = Ab;
  bufs.a_bytes = (uint32_t)((size_t)TX * ld * sizeof(bf16));
  bufs.b = Bb;
  bufs.b_bytes = (uint32_t)((size_t)TY * ld * sizeof(bf16));
  gemm_nt_mainloop_pipe64_k<TX, TY, WX, true, true>(arow, brow, 3 * nst0, koff, sm, acc, bufs);
  // lane: row xx, columns y + 8g .. + 7 (row blocks j, j + 1) and
  // y + 32 + 8g .. + 7 (row blocks j + 2, j + 3)
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % WX, wy = w / WX;
  float* Pb = P + (size_t)c * a.np * a.np;
#pragma unroll
  for (int i = 0; i < S::MX; ++i)
#pragma unroll
    for (int j = 0; j < S::MY; j += 4) {
      const int xx = x0 + wx * (TX / WX) + i * 16 + r16;
      float* row = Pb + (size_t)xx * a.np + y0 + wy * (TY / S::WY) + j * 16;
      store4(row + 8 * g, acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]);
      store4(row + 8 * g + 4, acc[i][j + 1][0], acc[i][j + 1][1], acc[i][j + 1][2],
             acc[i][j + 1][3]);
      store4(row + 32 + 8 * g, acc[i][j + 2][0], acc[i][j + 2][1], acc[i][j + 2][2],
             acc[i][j + 2][3]);
      store4(row + 32 + 8 * g + 4, acc[i][j + 3][0], acc[i][j + 3][1], acc[i][j + 3][2],
             acc[i][j + 3][3]);
    }
}

// ---------------------------------------------------------------------------
// 3. LN_out + W_z, gate, residual
// ---------------------------------------------------------------------------
template <typename ZT, typename CT>
struct TrimulOutArgs {
  const CT* P;  // [Ch][Np][Np]
  const ZT* z;
  int64_t z_s0, z_s1;
  ZT* out;
  int64_t o_s0, o_s1;
  const float* ln_in_w;
  const float* ln_in_b;
  const float* ln_out_w;
  const float* ln_out_b;
  const CT* wz;  // [C][Ch] (the weight-stationary kernel: W_z diag(ln_out_w))
  const CT* wg;  // [C][C]
  const float* wz_sum;   // weight-stationary kernel: row sums of wz
  const float* wz_bias;  // weight-stationary kernel: W_z ln_out_b
  int n, np, c;
  int add;
  float eps;
};

// LN_out folded into the output projection (weight-stationary kernel):
// W'[o][k] = bf16(W_z[o][k] ln_out_w[k]) (from the f32 W_z when given, one
// rounding), s[o] = sum_k W'[o][k] (the values the MFMA multiplies),
// c[o] = sum_k ln_out_b[k] W_z[o][k].  One workgroup per output row, sums in
// a fixed order.
__global__ __launch_bounds__(256) void trimul_fold_ln_out_kernel(const float* __restrict__ wz32,
                                                                 const bf16* __restrict__ wz16,
                                                                 const float* __restrict__ lw,
                                                                 const float* __restrict__ lb,
                                                                 int ch, bf16* __restrict__ wf,
                                                                 float* __restrict__ s,
                                                                 float* __restrict__ c) {
  __shared__ float red[2][256];
  const int o = blockIdx.x, t = threadIdx.x;
  float ss = 0.f, cc = 0.f;
  for (int k = t; k < ch; k += 256) {
    const size_t i = (size_t)o * ch + k;
    const float wv = wz32 ? wz32[i] : (float)wz16[i];
    const bf16 f = (bf16)(wv * lw[k]);
    wf[i] = f;
    ss += (float)f;
    cc += lb[k] * wv;
  }
  red[0][t] = ss;
  red[1][t] = cc;
  __syncthreads();
  for (int h = 128; h > 0; h >>= 1) {
    if (t < h) {
      red[0][t] += red[0][t + h];
      red[1][t] += red[1][t + h];
    }
    __syncthreads();
  }
  if (t == 0) {
    s[o] = red[0][0];
    c[o] = red[1][0];
  }
}

// kX3Mul (f32 compute, ODDE_F32X3): products in three bf16 parts.
// kRB consecutive first indices x per workgroup: every W_z and W_g fragment
// a wave reads from L2 serves kRB row blocks (the fp32 form reads its
// weights per fragment).  blockIdx.z of gridDim.z takes output channels
// [z C / Z, (z + 1) C / Z) (small grids).
template <typename ZT, typename CT, int kC, int kCh, bool kX3Mul = false, int kRB = 1>
__global__ __launch_bounds__(256) void trimul_out_kernel(TrimulOutArgs<ZT, CT> a) {
  constexpr int C = kC * 32, CH = kCh * 32;
  using MF = MulFrag<CT, kX3Mul>;
  constexpr int LD = CH + 16 / sizeof(CT);   // row stride of the transposed tile
  __shared__ __attribute__((aligned(16))) CT pt[kRB][64 * LD];

  const int x0 = blockIdx.y * kRB;
  const int y0 = blockIdx.x * 64;
  // stage P[:, x, y0:y0+64] transposed to pt[rb][y][c] (rows x past n read
  // row n - 1, which exists, and are never stored)
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    constexpr int VEC = 16 / sizeof(CT);
    constexpr int PER_C = 64 / VEC;              // 16-byte chunks per channel row
    const CT* src = a.P + (size_t)min(x0 + rb, a.n - 1) * a.np + y0;
    for (int ci = threadIdx.x; ci < CH * PER_C; ci += 256) {
      const int c = ci / PER_C, yy = (ci % PER_C) * VEC;
      CT v[VEC];
      *reinterpret_cast<f32x4*>(v) =
          *reinterpret_cast<const f32x4*>(src + (size_t)c * a.np * a.np + yy);
#pragma unroll
      for (int e = 0; e < VEC; ++e) pt[rb][(yy + e) * LD + c] = v[e];
    }
  }
  __syncthreads();

  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int yl = y0 + w * 16 + r16;
  MF xp[kRB][kCh], xz[kRB][kC];
  bool valid[kRB];
  const ZT* zrow[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int x_ = x0 + rb;
    valid[rb] = x_ < a.n && yl < a.n;
    zrow[rb] = a.z + (int64_t)(valid[rb] ? x_ : 0) * a.z_s0 + (int64_t)(valid[rb] ? yl : 0) * a.z_s1;
    Frag<CT> tp[kCh], tz[kC];
    ln_rows_to_frags<CT, CT, CH>(&pt[rb][(w * 16 + r16) * LD], true, a.ln_out_w, a.ln_out_b, a.eps,
                                 tp);
    ln_rows_to_frags<ZT, CT, C>(zrow[rb], valid[rb], a.ln_in_w, a.ln_in_b, a.eps, tz);
#pragma unroll
    for (int t = 0; t < kCh; ++t) to_mul(tp[t], xp[rb][t]);
#pragma unroll
    for (int t = 0; t < kC; ++t) to_mul(tz[t], xz[rb][t]);
  }

  const int cb_per = (C / 16) / (int)gridDim.z;
  for (int cb = (int)blockIdx.z * cb_per; cb < ((int)blockIdx.z + 1) * cb_per; ++cb) {
    f32x4 ay[kRB], agt[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) ay[rb] = agt[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kCh; ++t) {
      MF f;
      load_w_frag(a.wz, CH, cb * 16, C, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ay[rb], f, xp[rb][t]);
    }
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      load_w_frag(a.wg, C, cb * 16, C, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(agt[rb], f, xz[rb][t]);
    }
    const int c0 = cb * 16 + 4 * g;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      if (!valid[rb]) continue;
      float base[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.add) load4(zrow[rb] + c0, base);
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = base[e] + ay[rb][e] * sigmoidf_(agt[rb][e]);
      store4(a.out + (int64_t)(x0 + rb) * a.o_s0 + (int64_t)yl * a.o_s1 + c0, r[0], r[1], r[2],
             r[3]);
    }
  }
}

// f32 data with W_z and W_g staged in LDS (fp32 rows, or with kX3Mul the
// three-part split rows: the same bytes), 16 output channels at a time,
// shared by the workgroup's 4 waves: every weight byte fetched from L2
// serves the workgroup's 64 rows instead of one wave's 16.  Chunks are
// double-buffered (the next one waits in registers while the current one is
// multiplied), one barrier per chunk.  One first index x per workgroup, as
// trimul_out_kernel; the arithmetic per output is the same.
template <typename ZT, int kC, int kCh, bool kX3Mul = false>
__global__ __launch_bounds__(256) void trimul_out_f32s_kernel(TrimulOutArgs<ZT, float> a) {
  using MF = MulFrag<float, kX3Mul>;
  constexpr int C = kC * 32, CH = kCh * 32, NCB = C / 16;
  constexpr int LD = CH + 4;                    // row stride of the transposed P tile
  constexpr int WLZ = CH + 4, WLG = C + 4;      // staged W_z / W_g row strides (floats)
  constexpr int WCH = 16 * WLZ + 16 * WLG;      // floats per chunk buffer
  constexpr int PZ = 16 * CH / 4, PT = PZ + 16 * C / 4;  // 16-byte pieces per chunk
  constexpr int PPT = (PT + 255) / 256;         // pieces per thread
  __shared__ __attribute__((aligned(16))) float pt[64 * LD];
  __shared__ __attribute__((aligned(16))) float wsm[2][WCH];

  const int x_ = blockIdx.y;
  const int y0 = blockIdx.x * 64;
  f32x4 wreg[PPT];
  auto wload = [&](int cb) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      if (q < PZ) {
        const int r = q / (CH / 4), c4 = q % (CH / 4);
        wreg[k] = *reinterpret_cast<const f32x4*>(a.wz + (size_t)(cb * 16 + r) * CH + 4 * c4);
      } else if (q < PT) {
        const int u = q - PZ, r = u / (C / 4), c4 = u % (C / 4);
        wreg[k] = *reinterpret_cast<const f32x4*>(a.wg + (size_t)(cb * 16 + r) * C + 4 * c4);
      }
    }
  };
  auto wstore = [&](int buf) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      if (q < PZ) {
        const int r = q / (CH / 4), c4 = q % (CH / 4);
        *reinterpret_cast<f32x4*>(&wsm[buf][r * WLZ + 4 * c4]) = wreg[k];
      } else if (q < PT) {
        const int u = q - PZ, r = u / (C / 4), c4 = u % (C / 4);
        *reinterpret_cast<f32x4*>(&wsm[buf][16 * WLZ + r * WLG + 4 * c4]) = wreg[k];
      }
    }
  };
  wload(0);
  // stage P[:, x, y0:y0+64] transposed to pt[y][c]
  {
    constexpr int PER_C = 16;                   // 16-byte chunks per channel row
    const float* src = a.P + (size_t)x_ * a.np + y0;
    for (int ci = threadIdx.x; ci < CH * PER_C; ci += 256) {
      const int c = ci / PER_C, yy = (ci % PER_C) * 4;
      const f32x4 v = *reinterpret_cast<const f32x4*>(src + (size_t)c * a.np * a.np + yy);
#pragma unroll
      for (int e = 0; e < 4; ++e) pt[(yy + e) * LD + c] = v[e];
    }
  }
  wstore(0);
  if (NCB > 1) wload(1);
  __syncthreads();  // pt and chunk 0 staged

  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int yl = y0 + w * 16 + r16;
  const bool valid = x_ < a.n && yl < a.n;
  MF xp[kCh], xz[kC];
  const ZT* zrow = a.z + (int64_t)(valid ? x_ : 0) * a.z_s0 + (int64_t)(valid ? yl : 0) * a.z_s1;
  {
    Frag<float> tp[kCh], tz[kC];
    ln_rows_to_frags<float, float, CH>(&pt[(w * 16 + r16) * LD], true, a.ln_out_w, a.ln_out_b,
                                       a.eps, tp);
    ln_rows_to_frags<ZT, float, C>(zrow, valid, a.ln_in_w, a.ln_in_b, a.eps, tz);
#pragma unroll
    for (int t = 0; t < kCh; ++t) to_mul(tp[t], xp[t]);
#pragma unroll
    for (int t = 0; t < kC; ++t) to_mul(tz[t], xz[t]);
  }

  for (int cb = 0; cb < NCB; ++cb) {
    const float* wz_s = wsm[cb & 1] + r16 * WLZ;
    const float* wg_s = wsm[cb & 1] + 16 * WLZ + r16 * WLG;
    f32x4 ay = {0.f, 0.f, 0.f, 0.f}, agt = ay;
#pragma unroll
    for (int t = 0; t < kCh; ++t) {
      MF f;
      staged_w_frag(wz_s, CH, t, f);
      mma(ay, f, xp[t]);
    }
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      staged_w_frag(wg_s, C, t, f);
      mma(agt, f, xz[t]);
    }
    if (valid) {
      const int c0 = cb * 16 + 4 * g;
      float base[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.add) load4(zrow + c0, base);
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = base[e] + ay[e] * sigmoidf_(agt[e]);
      store4(a.out + (int64_t)x_ * a.o_s0 + (int64_t)yl * a.o_s1 + c0, r[0], r[1], r[2], r[3]);
    }
    // buffer (cb + 1) & 1 was last read in chunk cb - 1, before the barrier
    // that ended it
    if (cb + 1 < NCB) {
      wstore((cb + 1) & 1);
      if (cb + 2 < NCB) wload(cb + 2);
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// weight-stationary forms (per-wave weight slices in registers, LN'd row
// tiles staged once in LDS, persistent over 64-row tiles)
// ---------------------------------------------------------------------------

// Projection: wave w holds the gate and value rows of a (w < 2) or b (w >= 2)
// for channels [(w & 1) * Ch/2, (w & 1 + 1) * Ch/2).
template <typename ZT, typename CT, int kC, int kCH>
__global__ __launch_bounds__(256, 2) void trimul_proj_ws_kernel(TrimulProjArgs<ZT, CT> a,
                                                                int ntiles) {
  constexpr int C = kC * 32, CH = kCH * 32, NB = kCH;  // NB blocks of 16 = Ch/2 channels
  // bf16 arithmetic multiplies in fp16 here: LN(z) rounded to fp16 (11
  // mantissa bits against bf16's 8, well inside fp16's range) times the bf16
  // weights, which fp16 holds exactly; same MFMA rate, fp32 accumulation
  using XT = typename std::conditional<sizeof(CT) == 2, f16, CT>::type;
  __shared__ __attribute__((aligned(16))) XT xs[kTileRows * TileLD<XT, C>::value];
  __shared__ __attribute__((aligned(16))) unsigned char raw[RawTile<ZT, C>::BYTES];
  __shared__ float mk_s[kTileRows];
  __shared__ float lnp[2 * C];  // LayerNorm weight, bias
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  for (int t = threadIdx.x; t < C; t += 256) {
    lnp[t] = a.ln_w[t];
    lnp[C + t] = a.ln_b[t];
  }
  const int which = w >> 1, half = w & 1;
  const int o0 = which * CH + half * (CH / 2);
  // with fp16 operands the gate weights carry -log2(e), so the gate's
  // accumulator feeds exp2 directly (sigmoid_nl2e)
  constexpr bool kFold = std::is_same<XT, f16>::value;
  Frag<XT> wpf[NB][kC], wgf[NB][kC];
  load_w_slice(a.wp, C, o0, 2 * CH, wpf);
  if constexpr (kFold) load_w_slice_scaled(a.wg, C, o0, 2 * CH, kNegLog2e, wgf);
  else load_w_slice(a.wg, C, o0, 2 * CH, wgf);
  CT* dst = which ? a.B : a.A;
  const int np = a.np, n = a.n, tiles_per_row = np / kTileRows;
  // the next tile's z rows stream into LDS while a tile is computed; rows
  // outside n x n read a real row and are masked in the LN pass
  auto issue = [&](int tl) {
    const int tx = min(tl / tiles_per_row, n - 1), ty0 = (tl % tiles_per_row) * kTileRows;
    raw_tile_issue<ZT, C, kStream>(a.z + (int64_t)tx * a.z_s0, a.z_s1, ty0, n, raw);
  };
  // wave 0 loads the next tile's mask values (lane = column) with its z rows
  float mnext = 0.f;
  auto mfetch = [&](int tl) {
    const int tx = tl / tiles_per_row, y = (tl % tiles_per_row) * kTileRows + l;
    if (w == 0)
      mnext = (tx < n && y < n)
                  ? (a.mask ? a.mask[(int64_t)tx * a.m_s0 + (int64_t)y * a.m_s1] : 1.0f)
                  : 0.f;
  };
  if ((int)blockIdx.x < ntiles) {
    issue(blockIdx.x);
    mfetch(blockIdx.x);
  }
  raw_tile_wait();
  // Per tile: LN the raw tile, start the next tile's loads, compute, then wait
  // for this wave's loads and only then issue the tile's stores (kept in
  // registers until then), so a wave never waits for its own stores to drain:
  // they complete while the next tile is normalised and computed.  The
  // closing barrier makes the next raw tile complete for every wave and
  // releases xs / mk_s.
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int x = tile / tiles_per_row;
    const int y0 = (tile % tiles_per_row) * kTileRows;
    const float mcur = mnext;
    raw_tile_ln<ZT, XT, C>(raw, [&](int r) { return x < n && y0 + r < n; }, lnp, lnp + C,
                           a.eps, xs);
    if (w == 0) mk_s[l] = mcur;
    lds_barrier();  // xs and mk_s ready; raw consumed
    if (tile + (int)gridDim.x < ntiles) {
      issue(tile + gridDim.x);  // raw is free again
      mfetch(tile + gridDim.x);
    }
    // Row block rb covers tile rows 32 (rb >> 1) + 8 (m >> 2) + 4 (rb & 1) + (m & 3)
    // for MFMA row m, so a lane's outputs of row blocks 2p and 2p + 1 are the
    // 8 consecutive rows 32 p + 8 g .. + 7 of one channel: one 16-byte store.
    bf16x4 ov[kTileRows / 16][NB];
#pragma unroll
    for (int rb = 0; rb < kTileRows / 16; ++rb) {
      const int rbase = 32 * (rb >> 1) + 4 * (rb & 1);
      Frag<XT> xf[kC];
      {
        constexpr int LD = TileLD<XT, C>::value;
        const int off = (rbase + 8 * (r16 >> 2) + (r16 & 3)) * LD + 8 * g;
#pragma unroll
        for (int t = 0; t < kC; ++t) xf[t].load(xs + off + 32 * t);
      }
      float mk[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) mk[e] = mk_s[rbase + 8 * g + e];
#pragma unroll
      for (int cb = 0; cb < NB; ++cb) {
        f32x4 ap = {0.f, 0.f, 0.f, 0.f}, ag = ap;
#pragma unroll
        for (int t = 0; t < kC; ++t) {
          mma(ap, xf[t], wpf[cb][t]);
          mma(ag, xf[t], wgf[cb][t]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
          ov[rb][cb][e] =
              (bf16)(mk[e] * (kFold ? sigmoid_nl2e(ag[e]) : sigmoidf_(ag[e])) * ap[e]);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // next raw tile (own part) landed
    // a lane holds rows y0 + 8 g .. + 7 (row blocks 0, 1) and y0 + 32 + 8 g ..
    // + 7 (row blocks 2, 3) of channel c: slots g and 4 + g of the channel's
    // 128-byte line of this tile; lanes r16 and r16 ^ 1 (channels c, c ^ 1)
    // complete each other's lines
    static_assert(kTileRows == 64, "one 128-byte line of bf16 per channel and tile");
#pragma unroll
    for (int cb = 0; cb < NB; ++cb) {
      const int c = half * (CH / 2) + cb * 16 + r16;
      bf16x8 lo, hi;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        lo[e] = ov[0][cb][e];
        lo[4 + e] = ov[1][cb][e];
        hi[e] = ov[2][cb][e];
        hi[4 + e] = ov[3][cb][e];
      }
      store_line_pair(reinterpret_cast<bf16x8*>(dst + ((size_t)c * np + x) * np + y0),
                      reinterpret_cast<bf16x8*>(dst + ((size_t)(c ^ 1) * np + x) * np + y0), g, lo,
                      hi);
    }
    lds_barrier();  // every wave's part of the next raw tile landed; xs, mk_s free
  }
}

// Epilogue: wave w produces output channels [w*C/4, (w+1)*C/4): W' and W_g
// slices in registers; P (staged transposed from its channel-major planes,
// as stored) and LN_in(z) tiles in LDS.  LN_out is folded into the weights
// (a.wz = W' = W_z diag(ln_out_w) in bf16, a.wz_sum = row sums of W',
// a.wz_bias = W_z ln_out_b):  LN_out(p) W_z^T = rstd (p W'^T - mean s) + c,
// with the row statistics of p from LDS, so p enters the MFMA without being
// rounded again after the normalisation.
template <typename ZT, typename CT, int kC, int kCH>
__global__ __launch_bounds__(256, 2) void trimul_out_ws_kernel(TrimulOutArgs<ZT, CT> a, int ntiles) {
  constexpr int C = kC * 32, CH = kCH * 32, NBO = C / 64;
  constexpr int LDP = TileLD<CT, CH>::value;
  __shared__ __attribute__((aligned(16))) CT xp[kTileRows * LDP];
  // the gate multiplies in fp16 with bf16 arithmetic (LN_in(z) rounded to
  // fp16, the weights carrying -log2(e); see the projection)
  using GT = typename std::conditional<sizeof(CT) == 2, f16, CT>::type;
  constexpr bool kFold = std::is_same<GT, f16>::value;
  __shared__ __attribute__((aligned(16))) GT xz[kTileRows * TileLD<GT, C>::value];
  __shared__ __attribute__((aligned(16))) unsigned char raw[RawTile<ZT, C>::BYTES];
  __shared__ __attribute__((aligned(16))) float lnp[4 * C];  // LN_in weight, bias; s; c
  __shared__ float pst[2 * kTileRows];                      // LN_out mean, rstd per row
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  for (int t = threadIdx.x; t < C; t += 256) {
    lnp[t] = a.ln_in_w[t];
    lnp[C + t] = a.ln_in_b[t];
    lnp[2 * C + t] = a.wz_sum[t];
    lnp[3 * C + t] = a.wz_bias[t];
  }
  Frag<CT> wzf[NBO][kCH];
  Frag<GT> wgf[NBO][kC];
  load_w_slice(a.wz, CH, w * (C / 4), C, wzf);
  if constexpr (kFold) load_w_slice_scaled(a.wg, C, w * (C / 4), C, kNegLog2e, wgf);
  else load_w_slice(a.wg, C, w * (C / 4), C, wgf);
  const int np = a.np, n = a.n, tiles_per_row = np / kTileRows;
  auto issue = [&](int tl) {  // the next tile's z rows (for LN_in), as in the projection
    const int tx = tl / tiles_per_row, ty0 = (tl % tiles_per_row) * kTileRows;
    raw_tile_issue<ZT, C, kStream>(a.z + (int64_t)tx * a.z_s0, a.z_s1, ty0, n, raw);
  };
  // P[:, x, y0:y0+64] of the next tile is loaded into registers while the
  // current tile is computed, then written transposed to xp[y][c]: thread t
  // holds channels PCH*(t/8) .. +PCH-1 at rows 8*(t%8) .. +7 and writes
  // them as eight PCH-channel row pieces.
  static_assert(sizeof(CT) == 2 && kTileRows == 64, "bf16 P, 64-row tiles");
  constexpr int PCH = CH / 32;  // channels per thread (16-byte loads of 8 rows each)
  f32x4 ppre[PCH];
  const int pcg = threadIdx.x >> 3, pyb = threadIdx.x & 7;
  auto pfetch = [&](int tl) {
    const int tx = tl / tiles_per_row, ty0 = (tl % tiles_per_row) * kTileRows;
    const CT* src = a.P + (size_t)tx * np + ty0 + 8 * pyb;
#pragma unroll
    for (int k = 0; k < PCH; ++k)
      ppre[k] = load_stream(reinterpret_cast<const f32x4*>(src + (size_t)(PCH * pcg + k) * np * np));
  };
  if ((int)blockIdx.x < ntiles) {
    issue(blockIdx.x);
    pfetch(blockIdx.x);
  }
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int x = tile / tiles_per_row;
    const int y0 = (tile % tiles_per_row) * kTileRows;
    {
      CT v[PCH][8];
#pragma unroll
      for (int k = 0; k < PCH; ++k) *reinterpret_cast<f32x4*>(v[k]) = ppre[k];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        CT rowv[PCH];
#pragma unroll
        for (int k = 0; k < PCH; ++k) rowv[k] = v[k][e];
        CT* dst = xp + (8 * pyb + e) * LDP + PCH * pcg;
        if constexpr (PCH == 4) {
          *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(rowv);
        } else {
          *reinterpret_cast<unsigned*>(dst) = *reinterpret_cast<const unsigned*>(rowv);
        }
      }
    }
    raw_tile_wait();  // z rows landed; every wave is done with the previous tile
    raw_tile_ln<ZT, GT, C>(raw, [&](int r) { return y0 + r < n; }, lnp, lnp + C, a.eps, xz);
    {  // LN_out statistics of each staged P row (the row itself stays as stored)
      constexpr int Q = CH / 4;
      const int r = threadIdx.x >> 2, quarter = threadIdx.x & 3;
      const CT* row = xp + r * LDP + quarter * Q;
      float v[Q];
#pragma unroll
      for (int e = 0; e < Q; e += 8) load8(row + e, v + e);
      float sm = 0.f;
#pragma unroll
      for (int e = 0; e < Q; ++e) sm += v[e];
      sm += __shfl_xor(sm, 1, 64);
      sm += __shfl_xor(sm, 2, 64);
      const float mean = sm * (1.0f / CH);
      float q = 0.f;
#pragma unroll
      for (int e = 0; e < Q; ++e) q += (v[e] - mean) * (v[e] - mean);
      q += __shfl_xor(q, 1, 64);
      q += __shfl_xor(q, 2, 64);
      if (quarter == 0) {
        pst[r] = mean;
        pst[kTileRows + r] = rsqrtf(q * (1.0f / CH) + a.eps);
      }
    }
    // residual z values of this lane's outputs, taken from the raw tile before
    // the next tile's rows overwrite it (row r, 16-byte chunk c in slot c ^ (r & 7))
    float res[kTileRows / 16][NBO][4];
#pragma unroll
    for (int rb = 0; rb < kTileRows / 16; ++rb)
#pragma unroll
      for (int cb = 0; cb < NBO; ++cb) {
        const int r = rb * 16 + r16;
        const int c0 = w * (C / 4) + cb * 16 + 4 * g;
        constexpr int EPC = 16 / (int)sizeof(ZT);
        const ZT* rowp = reinterpret_cast<const ZT*>(raw + r * RawTile<ZT, C>::ROW_BYTES);
        const int chunk = c0 / EPC;
        const ZT* src = rowp + ((chunk ^ (r & 7)) * EPC) + (c0 % EPC);
        if (a.add) {
          load4(src, res[rb][cb]);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) res[rb][cb][e] = 0.f;
        }
      }
    lds_barrier();  // xp and xz ready; raw consumed
    if (tile + (int)gridDim.x < ntiles) {
      issue(tile + gridDim.x);  // raw is free again
      pfetch(tile + gridDim.x);
    }
#pragma unroll
    for (int rb = 0; rb < kTileRows / 16; ++rb) {
      Frag<CT> pf[kCH];
      Frag<GT> zf[kC];
      tile_frags<CT, CH>(xp, rb, pf);
      tile_frags<GT, C>(xz, rb, zf);
      const int yr = y0 + rb * 16 + r16;
      const float pmean = pst[rb * 16 + r16], prstd = pst[kTileRows + rb * 16 + r16];
      float r[NBO][4];
#pragma unroll
      for (int cb = 0; cb < NBO; ++cb) {
        f32x4 ay = {0.f, 0.f, 0.f, 0.f}, ag = ay;
#pragma unroll
        for (int t = 0; t < kCH; ++t) mma(ay, wzf[cb][t], pf[t]);
#pragma unroll
        for (int t = 0; t < kC; ++t) mma(ag, wgf[cb][t], zf[t]);
        const int c0 = w * (C / 4) + cb * 16 + 4 * g;
        float sw[4], cw[4];
        load4(lnp + 2 * C + c0, sw);
        load4(lnp + 3 * C + c0, cw);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float y = prstd * (ay[e] - pmean * sw[e]) + cw[e];
          r[cb][e] = res[rb][cb][e] + y * (kFold ? sigmoid_nl2e(ag[e]) : sigmoidf_(ag[e]));
        }
      }
      ZT* orow = a.out + (int64_t)x * a.o_s0;
      store_row_blocks<ZT>(orow + (int64_t)yr * a.o_s1, orow + (int64_t)(yr ^ 1) * a.o_s1,
                           w * (C / 4), r, yr < n, (yr ^ 1) < n);
    }
    lds_barrier();  // xp and xz are rewritten for the next tile
  }
}

// ---------------------------------------------------------------------------
// 4. wide channels (bf16; C or Ch of 256 and more): LayerNorm passes
//    (lnpass.hpp) into bf16 rows, then NT GEMMs on the shared mainloop
//    (gemm.hpp) with the gating / residual epilogues.  Rows are the pairs of
//    the padded grid, m = x * Np + y (Np^2 rows, a multiple of 2048).
// ---------------------------------------------------------------------------
constexpr int kWTX = 256, kWTY = 128, kWWX = 4, kWNS = 3, kWKC = 32;
using WideShape = GemmShape<kWTX, kWTY, kWWX, kWKC>;

// Linear workgroup id -> (row tile, column tile) such that all column tiles
// of a row tile run on one XCD (workgroups are dealt to the 8 XCDs
// round-robin), so the tile's A rows are fetched into one L2.  The row tile
// count must be a multiple of 8.
__device__ __forceinline__ void wide_tile_map(int L, int ncol, int& rt, int& ct) {
  const int xcd = L & 7, s = L >> 3;
  rt = xcd + 8 * (s / ncol);
  ct = s % ncol;
}

struct TrimulWideProjArgs {
  const bf16* zn;   // [Np^2][C] LN_in rows in the projection's view order
  const bf16* wp;   // [2*Ch][C] (a_p rows, then b_p rows)
  const bf16* wg;   // [2*Ch][C]
  const float* mask;
  int64_t m_s0, m_s1;
  bf16* A;          // [Ch][Np][Np]
  bf16* B;
  int n, np, c, ch;
};

// Output rows of the GEMM are the 4*Ch projections interleaved in 16-row
// blocks [a_p | a_g | a_p | a_g ... | b_p | b_g ...] (read in place through
// the row functor, no copy), so a wave's fragments j (value) and j + 1
// (gate) hold the same 16 channels.  Accumulator: one channel, four pairs
// per lane per row block; two row blocks give 8 consecutive pairs -> 16-byte
// stores into the channel-major planes.
__global__ __launch_bounds__(512) void trimul_proj_wide_kernel(TrimulWideProjArgs a, int ncol) {
  __shared__ __attribute__((aligned(16))) bf16 sm[kWNS * WideShape::STAGE_ELEMS];
  int rt, ct;
  wide_tile_map(blockIdx.x, ncol, rt, ct);
  const int64_t x0 = (int64_t)rt * kWTX;
  const int y0 = ct * kWTY;
  const int C = a.c, CH = a.ch, np = a.np;
  f32x4 acc[WideShape::MX][WideShape::MY];
  // Tile row r (staged in LDS row r) is pair x0 + wide_pair_perm(r): within
  // each 32 rows, row block 2p + b, MFMA row m is pair 8 (m >> 2) + 4 b +
  // (m & 3), so a lane's results of row blocks 2p and 2p + 1 are 8
  // consecutive pairs of one channel (one 16-byte store).
  auto wide_pair_perm = [](int r) {
    const int m = r & 15;
    return (r & ~31) + 8 * (m >> 2) + 4 * ((r >> 4) & 1) + (m & 3);
  };
  gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, false, kWKC>(
      [&](int r) { return a.zn + (x0 + wide_pair_perm(r)) * C; },
      [&](int r) {
        const int R = y0 + r, side = R / (2 * CH), within = R % (2 * CH), t = within & 31;
        const int chan = side * CH + (within >> 5) * 16 + (t & 15);
        return (t < 16 ? a.wp : a.wg) + (size_t)chan * C;
      },
      C, sm, acc);
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kWWX, wy = w / kWWX;
  // The wave's 64 pairs lie in one row x (np is a multiple of 64): row blocks
  // 0, 1 give a lane pairs y + 8g .. + 7 (slot g of the channel's 128-byte
  // line of this row), row blocks 2, 3 the pairs 32 further (slot 4 + g);
  // lanes r16 and r16 ^ 1 (channels chan, chan ^ 1) complete each other's
  // lines, stored whole with the streaming policy (store_line_pair).
  static_assert(WideShape::MX == 4 && kWTX / kWWX == 64, "one 64-pair line per channel and wave");
  const int64_t mw = x0 + wx * (kWTX / kWWX);
  const int x = (int)(mw / np), yw = (int)(mw % np);
  float mk[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int y = yw + 32 * hh + 8 * g + e;
      mk[hh][e] = (x < a.n && y < a.n)
                      ? (a.mask ? a.mask[(int64_t)x * a.m_s0 + (int64_t)y * a.m_s1] : 1.0f)
                      : 0.f;
    }
#pragma unroll
  for (int j = 0; j < WideShape::MY; j += 2) {
    const int R = y0 + wy * (kWTY / WideShape::WY) + 16 * j;  // first row of the value block
    const int side = R / (2 * CH), chan = ((R % (2 * CH)) >> 5) * 16 + r16;
    bf16x8 v[2];
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 2 * hh;
        v[hh][e] = (bf16)(mk[hh][e] * sigmoidf_(acc[i][j + 1][e]) * acc[i][j][e]);
        v[hh][4 + e] = (bf16)(mk[hh][4 + e] * sigmoidf_(acc[i + 1][j + 1][e]) * acc[i + 1][j][e]);
      }
    bf16* dst = side ? a.B : a.A;
    store_line_pair(reinterpret_cast<bf16x8*>(dst + ((size_t)chan * np + x) * np + yw),
                    reinterpret_cast<bf16x8*>(dst + ((size_t)(chan ^ 1) * np + x) * np + yw), g,
                    v[0], v[1]);
  }
}

template <typename ZT>
struct TrimulWideOutArgs {
  const bf16* pn;   // [Np^2][Ch] LN_out(P) rows, natural order
  const bf16* zn;   // [Np^2][C] LN_in(z) rows in the projection's view order
  const bf16* wz;   // [C][Ch]
  const bf16* wg;   // [C][C]
  const ZT* z;
  int64_t z_s0, z_s1;
  ZT* out;
  int64_t o_s0, o_s1;
  int n, np, c, ch, add, zn_transposed;
};

// out[x][y][c] = (add ? z : 0) + sigmoid(LN_in(z) W_g^T) * (LN_out(P) W_z^T):
// two NT GEMMs over the same tile (K = Ch, then K = C), then the epilogue.
// Accumulator: one pair, four consecutive channels per lane.
template <typename ZT>
__global__ __launch_bounds__(512) void trimul_out_wide_kernel(TrimulWideOutArgs<ZT> a, int ncol) {
  __shared__ __attribute__((aligned(16))) bf16 sm[kWNS * WideShape::STAGE_ELEMS];
  int rt, ct;
  wide_tile_map(blockIdx.x, ncol, rt, ct);
  const int64_t x0 = (int64_t)rt * kWTX;
  const int y0 = ct * kWTY;
  const int C = a.c, CH = a.ch, np = a.np;
  f32x4 accy[WideShape::MX][WideShape::MY], accg[WideShape::MX][WideShape::MY];
  gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, true, kWKC>(
      [&](int r) { return a.pn + (x0 + r) * CH; },
      [&](int r) { return a.wz + (size_t)(y0 + r) * CH; }, CH, sm, accy);
  gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, true, kWKC>(
      [&](int r) {
        const int64_t m = x0 + r;  // the incoming form's z rows were normalised transposed
        const int64_t zr = a.zn_transposed ? (m % np) * np + m / np : m;
        return a.zn + zr * C;
      },
      [&](int r) { return a.wg + (size_t)(y0 + r) * C; }, C, sm, accg);
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kWWX, wy = w / kWWX;
#pragma unroll
  for (int i = 0; i < WideShape::MX; ++i) {
    const int64_t m = x0 + wx * (kWTX / kWWX) + 16 * i + r16;
    const int x = (int)(m / np), y = (int)(m % np);  // np is even: lane r16 ^ 1 has y ^ 1
    const bool ok = x < a.n && y < a.n, pok = x < a.n && (y ^ 1) < a.n;
    float r[WideShape::MY][4];
#pragma unroll
    for (int j = 0; j < WideShape::MY; ++j) {
      const int c0 = y0 + wy * (kWTY / WideShape::WY) + 16 * j + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[j][e] = 0.f;
      if (a.add && ok) load4(a.z + (int64_t)x * a.z_s0 + (int64_t)y * a.z_s1 + c0, r[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) r[j][e] += sigmoidf_(accg[i][j][e]) * accy[i][j][e];
    }
    ZT* orow = a.out + (int64_t)x * a.o_s0;
    store_row_blocks<ZT>(orow + (int64_t)y * a.o_s1, orow + (int64_t)(y ^ 1) * a.o_s1,
                         y0 + wy * (kWTY / WideShape::WY), r, ok, pok);
  }
}

}  // namespace odde

// ===========================================================================
// host side
// ===========================================================================
using namespace odde;

namespace {

// Wide-channel path: bf16 compute, C in {128, 256, 384} and C or Ch of 256
// and more (the weight slices of the register-resident kernels no longer fit).
bool trimul_wide(int c, int ch, int dt) {
  return dt == ODDE_BF16 && (c == 128 || c == 256 || c == 384) && (c >= 256 || ch >= 256);
}

// Shapes of the weight-stationary (register-resident weight slices) kernels:
// bf16 compute with (C, Ch) in {(128, 128), (64, 64), (64, 128)}.
bool trimul_ws_shape(int c, int ch, int dt) {
  return dt == ODDE_BF16 && ((c == 128 && ch == 128) || (c == 64 && (ch == 64 || ch == 128)));
}

struct TrimulWs {
  void* A; void* B; void* P; void* zn;
  bf16* wfold; float* wsum; float* wbias;  // LN_out folded into W_z (ws shapes)
  // ODDE_F32X3: W_p, W_g of the input ([2 Ch][C] each), W_z ([C][Ch]) and
  // W_g of the output ([C][C]) split once per call into bf16 hi | lo rows
  char* wsplit;
  uint64_t bytes;
};

TrimulWs carve_trimul(void* base, uint64_t size, int n, int c, int ch, int dt) {
  const int np = round_up(n, 128);
  const uint64_t plane = (uint64_t)ch * np * np * dtype_size(dt);
  Carver cv(base, size);
  TrimulWs w;
  w.A = cv.take<char>(plane);
  w.B = cv.take<char>(plane);
  w.P = cv.take<char>(plane);
  // the wide path's LN_in(z) rows (its LN_out(P) rows reuse A after the
  // contraction)
  w.zn = trimul_wide(c, ch, dt) ? cv.take<char>((uint64_t)np * np * c * 2) : nullptr;
  const bool fold = trimul_ws_shape(c, ch, dt);
  w.wfold = fold ? cv.take<bf16>((uint64_t)c * ch) : nullptr;
  w.wsum = fold ? cv.take<float>(c) : nullptr;
  w.wbias = fold ? cv.take<float>(c) : nullptr;
  w.wsplit =
      dt == ODDE_F32X3 ? cv.take<char>(((uint64_t)4 * ch * c + (uint64_t)c * ch + (uint64_t)c * c) * 4)
                       : nullptr;
  w.bytes = (cv.used + 255) & ~uint64_t(255);
  return w;
}

template <typename ZT>
int run_trimul_wide(const odde_trimul_args* a, const TrimulWs& ws, hipStream_t st) {
  const int n = a->n, C = a->c, ch = a->c_hidden, np = round_up(n, 128);
  const bool outgoing = a->outgoing != 0;
  const int64_t vs0 = outgoing ? a->z_s0 : a->z_s1, vs1 = outgoing ? a->z_s1 : a->z_s0;
  const int64_t rows = (int64_t)np * np;             // a multiple of 16384
  const int row_tiles = (int)(rows / kWTX);          // a multiple of 8
  bf16* zn = static_cast<bf16*>(ws.zn);
  {
    LaunchScope ls(ODDE_K_TRIMUL_PROJ, st);
    const int lg = (int)std::min<int64_t>(rows / 16, 4096);
    const ZT* z = static_cast<const ZT*>(a->z);
    if (C == 128)
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 128>), dim3(lg), dim3(256), 0, st, z, vs0, vs1, n,
                         np, np, a->norm_in_weight, a->norm_in_bias, a->eps, zn);
    else if (C == 256)
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 256>), dim3(lg), dim3(256), 0, st, z, vs0, vs1, n,
                         np, np, a->norm_in_weight, a->norm_in_bias, a->eps, zn);
    else
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 384>), dim3(lg), dim3(256), 0, st, z, vs0, vs1, n,
                         np, np, a->norm_in_weight, a->norm_in_bias, a->eps, zn);
    TrimulWideProjArgs p;
    p.zn = zn;
    p.wp = static_cast<const bf16*>(a->p_in_weight);
    p.wg = static_cast<const bf16*>(a->g_in_weight);
    p.mask = a->mask;
    p.m_s0 = outgoing ? a->mask_s0 : a->mask_s1;
    p.m_s1 = outgoing ? a->mask_s1 : a->mask_s0;
    p.A = static_cast<bf16*>(ws.A);
    p.B = static_cast<bf16*>(ws.B);
    p.n = n; p.np = np; p.c = C; p.ch = ch;
    const int ncol = 4 * ch / kWTY;
    hipLaunchKernelGGL(trimul_proj_wide_kernel, dim3(row_tiles * ncol), dim3(512), 0, st, p, ncol);
    int rc = check_launch("trimul_proj (wide)");
    if (rc) return rc;
  }
  ContractArgs<bf16> k;
  k.A = static_cast<bf16*>(ws.A); k.B = static_cast<bf16*>(ws.B); k.P = static_cast<bf16*>(ws.P);
  k.np = np; k.ch = ch;
  {
    LaunchScope ls(ODDE_K_TRIMUL_CONTRACT, st);
    if (np % 256 == 0) {
      launch_contract_big(k, np, ch, st);
    } else {
      const int tiles = (np / 128) * (np / 128);
      hipLaunchKernelGGL((trimul_contract_kernel<bf16>), dim3(tiles * ch), dim3(256), 0, st, k);
    }
    int rc = check_launch("trimul_contract");
    if (rc) return rc;
  }
  {
    LaunchScope ls(ODDE_K_TRIMUL_OUT, st);
    bf16* pn = static_cast<bf16*>(ws.A);  // A is dead after the contraction
    const dim3 tg(np / 64, np);
    switch (ch) {
      case 64: hipLaunchKernelGGL((ln_transpose_bf16_kernel<64>), tg, dim3(256), 0, st, k.P, np, n,
                                  a->norm_out_weight, a->norm_out_bias, a->eps, pn); break;
      case 128: hipLaunchKernelGGL((ln_transpose_bf16_kernel<128>), tg, dim3(256), 0, st, k.P, np,
                                   n, a->norm_out_weight, a->norm_out_bias, a->eps, pn); break;
      case 256: hipLaunchKernelGGL((ln_transpose_bf16_kernel<256>), tg, dim3(256), 0, st, k.P, np,
                                   n, a->norm_out_weight, a->norm_out_bias, a->eps, pn); break;
      case 384: hipLaunchKernelGGL((ln_transpose_bf16_kernel<384>), tg, dim3(256), 0, st, k.P, np,
                                   n, a->norm_out_weight, a->norm_out_bias, a->eps, pn); break;
      default: return set_error(ODDE_EUNSUPPORTED, "trimul: unsupported c_hidden");
    }
    TrimulWideOutArgs<ZT> o;
    o.pn = pn; o.zn = zn;
    o.wz = static_cast<const bf16*>(a->p_out_weight);
    o.wg = static_cast<const bf16*>(a->g_out_weight);
    o.z = static_cast<const ZT*>(a->z); o.z_s0 = a->z_s0; o.z_s1 = a->z_s1;
    o.out = static_cast<ZT*>(a->out); o.o_s0 = a->out_s0; o.o_s1 = a->out_s1;
    o.n = n; o.np = np; o.c = C; o.ch = ch; o.add = a->add_residual;
    o.zn_transposed = outgoing ? 0 : 1;
    const int ncol = C / kWTY;
    hipLaunchKernelGGL((trimul_out_wide_kernel<ZT>), dim3(row_tiles * ncol), dim3(512), 0, st, o,
                       ncol);
    return check_launch("trimul_out (wide)");
  }
}

int kdim(int c) {
  switch (c) {
    case 64: return 2;
    case 128: return 4;
    case 256: return 8;
    case 384: return 12;
    default: return 0;
  }
}

int check_trimul(const odde_trimul_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "trimul: null args");
  if (a->struct_size != sizeof(odde_trimul_args))
    return set_error(ODDE_EINVAL, "trimul: struct_size mismatch (ABI version skew)");
  if (a->n <= 0 || a->c <= 0 || a->c_hidden <= 0)
    return set_error(ODDE_EINVAL, "trimul: n, c and c_hidden must be positive");
  if (a->batch < 0) return set_error(ODDE_EINVAL, "trimul: batch must be >= 0");
  if (!kdim(a->c) || !kdim(a->c_hidden))
    return set_error(ODDE_EUNSUPPORTED, "trimul: c and c_hidden must be 64, 128, 256 or 384");
  if (!valid_dtype(a->z_dtype) ||
      !(valid_dtype(a->compute_dtype) || a->compute_dtype == ODDE_F32X3))
    return set_error(ODDE_EINVAL, "trimul: bad dtype");
  if (a->z_dtype == ODDE_BF16 && a->compute_dtype != ODDE_BF16)
    return set_error(ODDE_EUNSUPPORTED, "trimul: bf16 storage with f32 compute");
  return ODDE_OK;
}

// ODDE_TRIMUL_PROJ_F32_PLAIN=1: the fp32 projection without staged weights
// (tuning).  ODDE_TRIMUL_PROJ_SRB: row blocks per wave of the staged form.
inline bool trimul_proj_f32_plain() {
  static const bool v = [] {
    const char* e = getenv("ODDE_TRIMUL_PROJ_F32_PLAIN");
    return e && atoi(e) != 0;
  }();
  return v;
}
constexpr int kSRB = 2;
// kX3Out: A and B as [hi | lo] bf16 rows (the three-part contraction);
// kX3Mul: the projections' products in three bf16 parts (f32 compute)
template <typename ZT, typename CT, int kC, bool kX3Out = false, bool kX3Mul = false>
void launch_tp(const TrimulProjArgs<ZT, CT>& p, hipStream_t st) {
  // fp32 weights are read from L2 per fragment: more row blocks per wave as
  // registers allow (4 up to C = 128, 2 at C = 256), once the grid stays
  // large enough (np >= 256: np^2 / 256 workgroups and more)
  constexpr int kRB = sizeof(CT) != 4 ? 1 : kC <= 4 ? 4 : kC <= 8 ? 2 : 1;
  if constexpr (sizeof(CT) == 4 && kC <= 4) {
    // f32 data from Np = 256: the weights staged in LDS (kSRB row blocks
    // per wave)
    if (p.np >= 256 && !trimul_proj_f32_plain()) {
      dim3 grid(p.np / 64, p.np / kSRB);
      hipLaunchKernelGGL((trimul_proj_kernel<ZT, CT, kC, kSRB, kX3Out, kX3Mul, true>), grid,
                         dim3(256), 0, st, p);
      return;
    }
  }
  if (kX3Out || (kRB > 1 && p.np >= 256)) {
    dim3 grid(p.np / 64, p.np / kRB, proj_split((int64_t)(p.np / 64) * (p.np / kRB), p.ch / 16));
    hipLaunchKernelGGL((trimul_proj_kernel<ZT, CT, kC, kRB, kX3Out, kX3Mul>), grid, dim3(256), 0,
                       st, p);
    return;
  }
  dim3 grid(p.np / 64, p.np, proj_split((int64_t)(p.np / 64) * p.np, p.ch / 16));
  hipLaunchKernelGGL((trimul_proj_kernel<ZT, CT, kC, 1, false, kX3Mul>), grid, dim3(256), 0, st, p);
}
template <typename ZT, int kC>
void launch_tp_f32(const TrimulProjArgs<ZT, float>& p, bool x3out, bool x3mul, hipStream_t st) {
  if (x3out) launch_tp<ZT, float, kC, true, true>(p, st);
  else if (x3mul) launch_tp<ZT, float, kC, false, true>(p, st);
  else launch_tp<ZT, float, kC>(p, st);
}

// Weight-stationary launches where the per-wave weight slices fit in
// registers (bf16, C and Ch in {64, 128}); false otherwise.
template <typename ZT, typename CT, int kC, int kCH>
void launch_tp_ws_t(const TrimulProjArgs<ZT, CT>& p, hipStream_t st) {
  const int ntiles = p.np * (p.np / kTileRows);
  static const int resident =
      resident_grid(reinterpret_cast<const void*>(&trimul_proj_ws_kernel<ZT, CT, kC, kCH>), 256);
  hipLaunchKernelGGL((trimul_proj_ws_kernel<ZT, CT, kC, kCH>), dim3(min(ntiles, resident)),
                     dim3(256), 0, st, p, ntiles);
}
template <typename ZT, typename CT>
bool launch_tp_ws(const TrimulProjArgs<ZT, CT>& p, int C, int ch, hipStream_t st) {
  if constexpr (sizeof(CT) != 2) {
    return false;
  } else {
  if (C == 128 && ch == 128) { launch_tp_ws_t<ZT, CT, 4, 4>(p, st); return true; }
  if (C == 64 && ch == 64) { launch_tp_ws_t<ZT, CT, 2, 2>(p, st); return true; }
  if (C == 64 && ch == 128) { launch_tp_ws_t<ZT, CT, 2, 4>(p, st); return true; }
    return false;
  }
}
template <typename ZT, typename CT, int kC, int kCH>
void launch_to_ws_t(const TrimulOutArgs<ZT, CT>& p, hipStream_t st) {
  const int ntiles = p.n * (p.np / kTileRows);
  static const int resident =
      resident_grid(reinterpret_cast<const void*>(&trimul_out_ws_kernel<ZT, CT, kC, kCH>), 256);
  hipLaunchKernelGGL((trimul_out_ws_kernel<ZT, CT, kC, kCH>), dim3(min(ntiles, resident)),
                     dim3(256), 0, st, p, ntiles);
}
template <typename ZT, typename CT>
bool launch_to_ws(const TrimulOutArgs<ZT, CT>& p, int C, int ch, hipStream_t st) {
  if constexpr (sizeof(CT) != 2) {
    return false;
  } else {
  if (C == 128 && ch == 128) { launch_to_ws_t<ZT, CT, 4, 4>(p, st); return true; }
  if (C == 64 && ch == 64) { launch_to_ws_t<ZT, CT, 2, 2>(p, st); return true; }
  if (C == 64 && ch == 128) { launch_to_ws_t<ZT, CT, 2, 4>(p, st); return true; }
    return false;
  }
}

// ODDE_TRIMUL_OUT_F32_PLAIN=1: the fp32 output kernel without staged
// weights (tuning).
inline bool trimul_out_f32_plain() {
  static const bool v = [] {
    const char* e = getenv("ODDE_TRIMUL_OUT_F32_PLAIN");
    return e && atoi(e) != 0;
  }();
  return v;
}
template <typename ZT, typename CT, int kC, int kCh, bool kX3Mul, int kRB>
void launch_to_rb(const TrimulOutArgs<ZT, CT>& p, hipStream_t st) {
  // every workgroup reads all channels of its z rows (LN_in for the gate):
  // with out overlapping z, a channel split would let one split overwrite
  // rows another still reads, so the in-place form keeps one workgroup per
  // row block
  const int64_t ext = (int64_t)(p.n - 1) * (p.z_s0 + p.z_s1) + kC * 32;
  const int64_t oext = (int64_t)(p.n - 1) * (p.o_s0 + p.o_s1) + kC * 32;
  const bool overlap = p.out < p.z + ext && p.z < p.out + oext;
  const int rows = (p.n + kRB - 1) / kRB;
  dim3 grid(p.np / 64, rows, overlap ? 1 : proj_split((int64_t)(p.np / 64) * rows, kC * 2));
  hipLaunchKernelGGL((trimul_out_kernel<ZT, CT, kC, kCh, kX3Mul, kRB>), grid, dim3(256), 0, st, p);
}
template <typename ZT, typename CT, int kC, int kCh>
void launch_to(const TrimulOutArgs<ZT, CT>& p, bool x3, hipStream_t st) {
  if constexpr (sizeof(CT) == 4) {
    if (x3) {
      // three-part products: the weights staged in LDS from N = 256 (C =
      // Ch = 128 at N = 1024: 1.24 -> 1.17 ms with two first indices per
      // workgroup sharing each L2 fragment read, which the staged form
      // replaces)
      if constexpr (kC <= 4 && kCh <= 4) {
        if (p.n >= 256 && !trimul_out_f32_plain()) {
          hipLaunchKernelGGL((trimul_out_f32s_kernel<ZT, kC, kCh, true>), dim3(p.np / 64, p.n),
                             dim3(256), 0, st, p);
          return;
        }
        if (p.n >= 256) {
          launch_to_rb<ZT, CT, kC, kCh, true, 2>(p, st);
          return;
        }
      }
      launch_to_rb<ZT, CT, kC, kCh, true, 1>(p, st);
      return;
    }
  }
  if constexpr (sizeof(CT) == 4 && kC <= 4 && kCh <= 4) {
    // true fp32 products from N = 256: weights staged in LDS (the grid no
    // longer needs an output-channel split)
    if (p.n >= 256 && !trimul_out_f32_plain()) {
      hipLaunchKernelGGL((trimul_out_f32s_kernel<ZT, kC, kCh>), dim3(p.np / 64, p.n), dim3(256), 0,
                         st, p);
      return;
    }
  }
  launch_to_rb<ZT, CT, kC, kCh, false, 1>(p, st);
}

template <typename ZT, typename CT, int kC>
bool dispatch_to(const TrimulOutArgs<ZT, CT>& p, int ch, bool x3, hipStream_t st) {
  switch (ch) {
    case 64: launch_to<ZT, CT, kC, 2>(p, x3, st); return true;
    case 128: launch_to<ZT, CT, kC, 4>(p, x3, st); return true;
    case 256: launch_to<ZT, CT, kC, 8>(p, x3, st); return true;
    case 384: launch_to<ZT, CT, kC, 12>(p, x3, st); return true;
    default: return false;
  }
}

template <typename ZT, typename CT>
int run_trimul(const odde_trimul_args* a, hipStream_t st) {
  const int n = a->n, C = a->c, ch = a->c_hidden;
  const int np = round_up(n, 128);
  TrimulWs ws = carve_trimul(a->workspace, a->workspace_bytes, n, C, ch, a->compute_dtype);
  if constexpr (sizeof(CT) == 2) {
    if (trimul_wide(C, ch, a->compute_dtype)) return run_trimul_wide<ZT>(a, ws, st);
  }
  const bool out = a->outgoing != 0;

  TrimulProjArgs<ZT, CT> p;
  p.z = static_cast<const ZT*>(a->z);
  // incoming: a[k,i] lands at A[c][i][k] by reading the view transposed
  p.z_s0 = out ? a->z_s0 : a->z_s1;
  p.z_s1 = out ? a->z_s1 : a->z_s0;
  p.mask = a->mask;
  p.m_s0 = out ? a->mask_s0 : a->mask_s1;
  p.m_s1 = out ? a->mask_s1 : a->mask_s0;
  p.ln_w = a->norm_in_weight; p.ln_b = a->norm_in_bias;
  p.wp = static_cast<const CT*>(a->p_in_weight);
  p.wg = static_cast<const CT*>(a->g_in_weight);
  p.A = static_cast<CT*>(ws.A); p.B = static_cast<CT*>(ws.B);
  p.n = n; p.np = np; p.ch = ch; p.eps = a->eps;
  // the three-part fp32 form: the projections' and the output's products
  // always, the contraction where its tiles fit (Np a multiple of 256;
  // otherwise true fp32 products)
  const bool x3mul = sizeof(CT) == 4 && a->compute_dtype == ODDE_F32X3;
  const bool x3 = x3mul && np % 256 == 0;
  const CT* w_z = static_cast<const CT*>(a->p_out_weight);
  const CT* w_go = static_cast<const CT*>(a->g_out_weight);
  if (x3mul) {
    // the weights as bf16 hi | lo rows, split once for this call
    char* d = ws.wsplit;
    launch_split_x3(a->p_in_weight, 2 * ch, C, d, false, st);
    p.wp = reinterpret_cast<const CT*>(d);
    d += (size_t)2 * ch * C * 4;
    launch_split_x3(a->g_in_weight, 2 * ch, C, d, false, st);
    p.wg = reinterpret_cast<const CT*>(d);
    d += (size_t)2 * ch * C * 4;
    launch_split_x3(a->p_out_weight, C, ch, d, false, st);
    w_z = reinterpret_cast<const CT*>(d);
    d += (size_t)C * ch * 4;
    launch_split_x3(a->g_out_weight, C, C, d, false, st);
    w_go = reinterpret_cast<const CT*>(d);
  }
  {
    LaunchScope ls(ODDE_K_TRIMUL_PROJ, st);
    if constexpr (sizeof(CT) == 4) {
      switch (C) {
        case 64: launch_tp_f32<ZT, 2>(p, x3, x3mul, st); break;
        case 128: launch_tp_f32<ZT, 4>(p, x3, x3mul, st); break;
        case 256: launch_tp_f32<ZT, 8>(p, x3, x3mul, st); break;
        case 384: launch_tp_f32<ZT, 12>(p, x3, x3mul, st); break;
      }
    } else if (!launch_tp_ws<ZT, CT>(p, C, ch, st)) {
      switch (C) {
        case 64: launch_tp<ZT, CT, 2>(p, st); break;
        case 128: launch_tp<ZT, CT, 4>(p, st); break;
        case 256: launch_tp<ZT, CT, 8>(p, st); break;
        case 384: launch_tp<ZT, CT, 12>(p, st); break;
      }
    }
    int rc = check_launch("trimul_proj");
    if (rc) return rc;
  }

  ContractArgs<CT> k;
  k.A = p.A; k.B = p.B; k.P = static_cast<CT*>(ws.P); k.np = np; k.ch = ch;
  {
    LaunchScope ls(ODDE_K_TRIMUL_CONTRACT, st);
    if (x3) {
      ContractArgs<bf16> kb;
      kb.A = static_cast<const bf16*>(ws.A); kb.B = static_cast<const bf16*>(ws.B);
      kb.P = nullptr; kb.np = np; kb.ch = ch;
      const int tiles = (np / 256) * (np / 256);
      hipLaunchKernelGGL(trimul_contract_x3_kernel, dim3(tiles * ch), dim3(512), 0, st, kb,
                         static_cast<float*>(ws.P));
    } else if constexpr (sizeof(CT) == 2) {
      if (np % 256 == 0) {
        launch_contract_big(k, np, ch, st);
      } else {
        const int tiles = (np / 128) * (np / 128);
        hipLaunchKernelGGL((trimul_contract_kernel<CT>), dim3(tiles * ch), dim3(256), 0, st, k);
      }
    } else {
      const int tiles = (np / 128) * (np / 128);
      hipLaunchKernelGGL((trimul_contract_kernel<CT>), dim3(tiles * ch), dim3(256), 0, st, k);
    }
    int rc = check_launch("trimul_contract");
    if (rc) return rc;
  }

  TrimulOutArgs<ZT, CT> o;
  o.P = k.P;
  o.z = static_cast<const ZT*>(a->z); o.z_s0 = a->z_s0; o.z_s1 = a->z_s1;
  o.out = static_cast<ZT*>(a->out); o.o_s0 = a->out_s0; o.o_s1 = a->out_s1;
  o.ln_in_w = a->norm_in_weight; o.ln_in_b = a->norm_in_bias;
  o.ln_out_w = a->norm_out_weight; o.ln_out_b = a->norm_out_bias;
  o.wz = w_z;
  o.wg = w_go;
  o.wz_sum = o.wz_bias = nullptr;
  o.n = n; o.np = np; o.c = C; o.add = a->add_residual; o.eps = a->eps;
  {
    LaunchScope ls(ODDE_K_TRIMUL_OUT, st);
    if constexpr (sizeof(CT) == 2) {
      if (trimul_ws_shape(C, ch, a->compute_dtype)) {
        hipLaunchKernelGGL(trimul_fold_ln_out_kernel, dim3(C), dim3(256), 0, st,
                           a->p_out_weight_f32, static_cast<const bf16*>(a->p_out_weight),
                           a->norm_out_weight, a->norm_out_bias, ch, ws.wfold, ws.wsum,
                           ws.wbias);
        o.wz = ws.wfold;
        o.wz_sum = ws.wsum;
        o.wz_bias = ws.wbias;
      }
    }
    bool ok = launch_to_ws<ZT, CT>(o, C, ch, st);
    if (!ok) switch (C) {
      case 64: ok = dispatch_to<ZT, CT, 2>(o, ch, x3mul, st); break;
      case 128: ok = dispatch_to<ZT, CT, 4>(o, ch, x3mul, st); break;
      case 256: ok = dispatch_to<ZT, CT, 8>(o, ch, x3mul, st); break;
      case 384: ok = dispatch_to<ZT, CT, 12>(o, ch, x3mul, st); break;
    }
    if (!ok) return set_error(ODDE_EUNSUPPORTED, "trimul: unsupported c/c_hidden");
    return check_launch("trimul_out");
  }
}

}  // namespace

extern "C" {

int odde_trimul_workspace_bytes(const odde_trimul_args* a, uint64_t* bytes) {
  int rc = check_trimul(a);
  if (rc) return rc;
  if (!bytes) return set_error(ODDE_EINVAL, "trimul: null bytes");
  *bytes = carve_trimul(nullptr, 0, a->n, a->c, a->c_hidden, a->compute_dtype).bytes;
  return ODDE_OK;
}

int odde_trimul_fwd(const odde_trimul_args* a, void* stream) {
  int rc = check_trimul(a);
  if (rc) return rc;
  if (!a->z || !a->out || !a->norm_in_weight || !a->norm_in_bias || !a->norm_out_weight ||
      !a->norm_out_bias || !a->p_in_weight || !a->g_in_weight || !a->p_out_weight ||
      !a->g_out_weight)
    return set_error(ODDE_EINVAL, "trimul: null tensor pointer");
  const uint64_t need = carve_trimul(nullptr, 0, a->n, a->c, a->c_hidden, a->compute_dtype).bytes;
  if (!a->workspace || a->workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(a->workspace) & 255))
    return set_error(ODDE_EWORKSPACE, "trimul: workspace missing, too small or not 256-byte aligned");
  const int zes = dtype_size(a->z_dtype);
  const int nb = a->batch > 1 ? a->batch : 1;
  const int64_t sb = nb > 1 ? (a->z_sb | a->out_sb) : 0;
  if ((reinterpret_cast<uintptr_t>(a->z) | reinterpret_cast<uintptr_t>(a->out)) & 15 ||
      ((a->z_s0 | a->z_s1 | a->out_s0 | a->out_s1 | sb) * zes) & 15)
    return set_error(ODDE_EINVAL, "trimul: z/out rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // The views of a batch run in order on the stream and share the workspace.
  odde_trimul_args e = *a;
  for (int b = 0; b < nb; ++b) {
    e.z = static_cast<const char*>(a->z) + (int64_t)b * a->z_sb * zes;
    e.out = static_cast<char*>(a->out) + (int64_t)b * a->out_sb * zes;
    e.mask = a->mask ? a->mask + (int64_t)b * a->mask_sb : nullptr;
    if (a->z_dtype == ODDE_F32 && a->compute_dtype != ODDE_BF16) rc = run_trimul<float, float>(&e, st);
    else if (a->z_dtype == ODDE_F32) rc = run_trimul<float, bf16>(&e, st);
    else rc = run_trimul<bf16, bf16>(&e, st);
    if (rc) return rc;
  }
  return ODDE_OK;
}

}  // extern "C"
