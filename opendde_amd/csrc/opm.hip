// OuterProductMean (the MSA -> pair update) on gfx950.
//
// Replaces OuterProductMean._forward / _opm (opendde/model/triangular/
// layers.py:525-616):
//   y = LN(m[s, i]);  a[s, i] = mask[s, i] * W_1 y;  b[s, i] = mask[s, i] * W_2 y
//   out[i, j, z] = (sum_{c1, c2} W_out[z][c1 * 32 + c2] sum_s a[s, i, c1] b[s, j, c2]
//                   + b_out[z]) / (sum_s mask[s, i] mask[s, j] + eps)
// with c_hidden = 32, in two kernels:
//
// 1. opm_proj: one workgroup per (64 MSA rows s, residue i).  LayerNorm and
//    the two projections on MFMA, then the 64 x 64 result goes through LDS so
//    that a and b are stored transposed, s innermost: At[i * 32 + c][s],
//    Bt[j * 32 + c][s] (bf16, rows padded to Sp = S rounded up to 64 with
//    zeros).  The mask is stored transposed as bf16 maskT[i][s] when given,
//    and opm_norm forms norm[i][j] = sum_s maskT[i][s] maskT[j][s] + eps on
//    the same GEMM mainloop (exact for 0/1 masks).
// 2. opm_outer: one workgroup per (8 residues i) x (8 residues j): the NT
//    GEMM mainloop (gemm.hpp) over k = s gives the 256 x 256 block of
//    outer products (64 residue pairs, each a 32 x 32 block); the block is
//    rounded to bf16 into LDS as P[pair][c1 * 32 + c2] (the reference rounds
//    the outer product to bf16 before linear_out under autocast), then
//    out[pair][z] = P W_out^T on MFMA with W_out fragments from global
//    memory, + b_out, / norm, rounded to bf16 (the update's dtype), plus the
//    residual when asked.
#include "common.hpp"
#include "gemm.hpp"
#include "runtime.hpp"

namespace odde {

constexpr int kOpmC = 32;     // c_hidden
constexpr int kOpmSB = 64;    // MSA rows per projection workgroup (and the S padding)
constexpr int kOpmPP = kOpmC * kOpmC + 8;  // LDS pitch of one pair's block (bf16)

// Outer-product workgroup tile: TI residues i x TJ residues j (GEMM rows
// 32 TI x 32 TJ), WX waves along i, NS stages of KC MSA rows.
template <int TI_, int TJ_, int WX_, int NS_, int KC_>
struct OpmTile {
  static constexpr int TI = TI_, TJ = TJ_, WX = WX_, NS = NS_, KC = KC_;
  static constexpr int PAIRS = TI * TJ;
  using Shape = GemmShape<TI * kOpmC, TJ * kOpmC, WX, KC>;
  static constexpr int MAIN_BYTES = NS * Shape::STAGE_ELEMS * 2;
  static constexpr int EPI_BYTES = PAIRS * kOpmPP * 2;
  static constexpr int LDS_BYTES = MAIN_BYTES > EPI_BYTES ? MAIN_BYTES : EPI_BYTES;
  static constexpr int PT = PAIRS / 16;  // 16-pair tiles of the projection
};
// 256 x 256 GEMM tiles staged 64 MSA rows at a time (whole 128-byte lines),
// one workgroup per CU; the 64 pairs' blocks reuse the stage buffers.
using OpmTileBig = OpmTile<8, 8, 2, 2, 64>;
// 256 x 128 GEMM tiles staged 32 MSA rows at a time, two workgroups per CU.
using OpmTileSmall = OpmTile<8, 4, 4, 3, 32>;
using OpmTileUsed = OpmTileBig;  // measured 3.20 vs 3.69 ms at S=1280, N=1024

struct OpmProjArgs {
  const void* m;
  const float* mask;  // [S][N] or null
  const float* ln_w;
  const float* ln_b;
  const bf16* w12;    // [64][c_m]: W_1 rows then W_2 rows
  bf16* at;           // [Np * 32][Sp]
  bf16* bt;
  bf16* maskt;        // [Np][Sp] or null
  int S, N, Sp;
  float eps;
};

// grid (Sp / 64, Np), 256 threads: wave w takes MSA rows s0 + 16 w .. + 15
// of residue i.
template <typename MT, int CM>
__global__ __launch_bounds__(256) void opm_proj_kernel(OpmProjArgs a) {
  constexpr int kC = CM / 32;
  constexpr int LDT = kOpmSB + 8;  // LDS pitch of the transposed tile
  __shared__ __attribute__((aligned(16))) bf16 t[2 * kOpmC * LDT];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int s0 = blockIdx.x * kOpmSB, i = blockIdx.y;
  const int s = s0 + 16 * w + r16;
  const bool valid = s < a.S && i < a.N;
  const MT* row = static_cast<const MT*>(a.m) + ((size_t)(valid ? s : 0) * a.N + (valid ? i : 0)) * CM;
  Frag<bf16> xf[kC];
  ln_rows_to_frags<MT, bf16, CM>(row, valid, a.ln_w, a.ln_b, a.eps, xf);
  // this lane's four rows in the accumulator layout: s0 + 16 w + 4 g + r
  float mk[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int sr = s0 + 16 * w + 4 * g + r;
    mk[r] = (sr < a.S && i < a.N) ? (a.mask ? a.mask[(size_t)sr * a.N + i] : 1.f) : 0.f;
  }
#pragma unroll
  for (int ot = 0; ot < 4; ++ot) {  // outputs 16 ot .. 16 ot + 15 (a: 0..31, b: 32..63)
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < kC; ++kt) {
      Frag<bf16> wf;
      load_w_frag(a.w12, CM, 16 * ot, 64, kt, wf);
      mma(acc, xf[kt], wf);  // D[row = MSA row 4g + r][col = output l % 16]
    }
    const int o = 16 * ot + r16;
    bf16x4 v;
#pragma unroll
    for (int r = 0; r < 4; ++r) v[r] = (bf16)(acc[r] * mk[r]);
    *reinterpret_cast<bf16x4*>(&t[o * LDT + 16 * w + 4 * g]) = v;
  }
  if (a.maskt && threadIdx.x < kOpmSB) {
    const int sr = s0 + threadIdx.x;
    a.maskt[(size_t)i * a.Sp + sr] =
        (bf16)((sr < a.S && i < a.N) ? (a.mask ? a.mask[(size_t)sr * a.N + i] : 1.f) : 0.f);
  }
  __syncthreads();
  // 64 output rows of 64 MSA rows (128 bytes each): 512 chunks of 16 bytes
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int ci = threadIdx.x + 256 * k, o = ci >> 3, ch = ci & 7;
    bf16* dst = (o < kOpmC ? a.at + ((size_t)i * kOpmC + o) * a.Sp
                           : a.bt + ((size_t)i * kOpmC + o - kOpmC) * a.Sp) + s0 + 8 * ch;
    *reinterpret_cast<bf16x8*>(dst) = *reinterpret_cast<const bf16x8*>(&t[o * LDT + 8 * ch]);
  }
}

// norm[i][j] = sum_s maskT[i][s] maskT[j][s] + eps over 128 x 128 tiles
// (grid (Np / 128)^2, 512 threads).
__global__ __launch_bounds__(512) void opm_norm_kernel(const bf16* __restrict__ maskt, int Np, int Sp,
                                                       float eps, float* __restrict__ norm) {
  using S = GemmShape<128, 128, 2>;
  __shared__ __attribute__((aligned(16))) bf16 sm[3 * S::STAGE_ELEMS];
  const int nt = Np / 128, ti = blockIdx.x / nt, tj = blockIdx.x % nt;
  const bf16* A = maskt + (size_t)ti * 128 * Sp;
  const bf16* B = maskt + (size_t)tj * 128 * Sp;
  f32x4 acc[S::MX][S::MY];
  gemm_nt_mainloop<128, 128, 2, 3, true>([&](int r) { return A + (size_t)r * Sp; },
                                         [&](int r) { return B + (size_t)r * Sp; }, Sp, sm, acc);
  // acc[mi][mj]: column (lane % 16) = row i, values = 4 consecutive j
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % 2, wy = w / 2;
#pragma unroll
  for (int mi = 0; mi < S::MX; ++mi)
#pragma unroll
    for (int mj = 0; mj < S::MY; ++mj) {
      const int i = ti * 128 + wx * 64 + 16 * mi + r16;
      const int j = tj * 128 + wy * 32 + 16 * mj + 4 * g;
      store4(norm + (size_t)i * Np + j, acc[mi][mj][0] + eps, acc[mi][mj][1] + eps,
             acc[mi][mj][2] + eps, acc[mi][mj][3] + eps);
    }
}

struct OpmOuterArgs {
  const bf16* at;
  const bf16* bt;
  const float* norm;   // [Np][Np] or null (all ones: norm = S + eps)
  const bf16* w_out;   // [c_z][1024]
  const float* b_out;  // [c_z] or null
  void* out;           // [N][N][c_z]
  int S, N, Np, Sp, add;
  float eps;
};

// Workgroup -> (i block, j block).  Workgroups are dealt to the 8 XCDs
// round-robin; each XCD takes bands of 8 x 8 tiles at a time, so the rows of
// A and B that a band's workgroups share are fetched into one L2.
__device__ __forceinline__ void opm_tile_map(int L, int nti, int ntj, int& ti, int& tj) {
  const int nbands = (nti / 8) * (ntj / 8);
  if ((nti & 7) || (ntj & 7) || (nbands & 7)) {
    ti = L / ntj;
    tj = L % ntj;
    return;
  }
  const int xcd = L & 7, local = L >> 3;
  const int band = (local >> 6) * 8 + xcd, w = local & 63;
  const int bpr = ntj / 8;  // bands per band-row
  ti = (band / bpr) * 8 + (w >> 3);
  tj = (band % bpr) * 8 + (w & 7);
}

template <typename OT, int CZ, typename TL>
__global__ __launch_bounds__(512) void opm_outer_kernel(OpmOuterArgs a) {
  using S = typename TL::Shape;
  constexpr int TI = TL::TI, TJ = TL::TJ, PAIRS = TL::PAIRS;
  constexpr int RI = S::MX / 2, RJ = S::MY / 2;  // residues per wave along i, j
  // projection split over the 8 waves: WZ along the CZ / 16 z tiles, WP along
  // the PT 16-pair tiles
  constexpr int ZT = CZ / 16, PT = TL::PT;
  constexpr int WZ = ZT < 8 ? ZT : 8, WP = 8 / WZ;
  constexpr int NU = ZT / WZ, NV = PT / WP;
  static_assert(ZT % WZ == 0 && PT % WP == 0 && 8 % WZ == 0, "projection tiles split evenly");
  __shared__ __attribute__((aligned(16))) bf16 sm[TL::LDS_BYTES / 2];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  int ti, tj;
  opm_tile_map(blockIdx.x, a.Np / TI, a.Np / TJ, ti, tj);
  const bf16* A = a.at + (size_t)ti * TI * kOpmC * a.Sp;
  const bf16* B = a.bt + (size_t)tj * TJ * kOpmC * a.Sp;
  f32x4 acc[S::MX][S::MY];
  gemm_nt_mainloop<TI * kOpmC, TJ * kOpmC, TL::WX, TL::NS, true, TL::KC>(
      [&](int r) { return A + (size_t)r * a.Sp; }, [&](int r) { return B + (size_t)r * a.Sp; },
      a.Sp, sm, acc);
  // acc[mi][mj]: column (lane % 16) = A row 32 RI wx + 16 mi + r16 (residue
  // RI wx + mi / 2, c1 = 16 (mi % 2) + r16); values e = B rows
  // 32 RJ wy + 16 mj + 4 g + e (residue RJ wy + mj / 2, c2 = 16 (mj % 2) + 4 g + e)
  const int wx = w % TL::WX, wy = w / TL::WX;
  bf16* P = sm;
#pragma unroll
  for (int mi = 0; mi < S::MX; ++mi)
#pragma unroll
    for (int mj = 0; mj < S::MY; ++mj) {
      const int pair = (RI * wx + mi / 2) * TJ + RJ * wy + mj / 2;
      const int c1 = 16 * (mi & 1) + r16, c2 = 16 * (mj & 1) + 4 * g;
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[mi][mj][e];
      *reinterpret_cast<bf16x4*>(&P[pair * kOpmPP + c1 * kOpmC + c2]) = v;
    }
  __syncthreads();
  // out[pair][z] = sum_k P[pair][k] W_out[z][k]: WZ waves along z, WP
  // along pairs; wave w takes z tiles w % WZ + WZ u and pair tiles
  // w / WZ + WP v, so each W_out fragment read from memory serves NV pair
  // tiles (with c_z >= 128 every W_out row is read once per workgroup)
  const int zw = w % WZ, pw = w / WZ;
  f32x4 acc2[NU][NV];
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int v = 0; v < NV; ++v) acc2[u][v] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16* wrow[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u)
    wrow[u] = a.w_out + (size_t)(16 * (zw + WZ * u) + r16) * (kOpmC * kOpmC) + 8 * g;
#pragma unroll 8
  for (int ks = 0; ks < kOpmC; ++ks) {
    Frag<bf16> wf[NU], pf[NV];
#pragma unroll
    for (int u = 0; u < NU; ++u) wf[u].load(wrow[u] + ks * kOpmC);
#pragma unroll
    for (int v = 0; v < NV; ++v)
      pf[v].load(P + (16 * (pw + WP * v) + r16) * kOpmPP + 8 * g + ks * kOpmC);
#pragma unroll
    for (int u = 0; u < NU; ++u)
#pragma unroll
      for (int v = 0; v < NV; ++v) mma(acc2[u][v], wf[u], pf[v]);  // D[z 4g + r][pair l % 16]
  }
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int pair = 16 * (pw + WP * v) + r16;
    const int i = ti * TI + pair / TJ, j = tj * TJ + pair % TJ;
    if (i >= a.N || j >= a.N) continue;
    const float inv = 1.0f / (a.norm ? a.norm[(size_t)i * a.Np + j] : (float)a.S + a.eps);
    OT* dst = static_cast<OT*>(a.out) + ((size_t)i * a.N + j) * CZ;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int z0 = 16 * (zw + WZ * u) + 4 * g;
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float bo = a.b_out ? a.b_out[z0 + r] : 0.f;
        o[r] = round_to<bf16>((acc2[u][v][r] + bo) * inv);
      }
      if (a.add) {
        float zr[4];
        load4(dst + z0, zr);
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] += zr[r];
      }
      store4(dst + z0, o[0], o[1], o[2], o[3]);
    }
  }
}

namespace {

int opm_np(int n) { return round_up(n, 128); }
int opm_sp(int s) { return round_up(s, kOpmSB); }

uint64_t opm_ws_bytes(const odde_opm_args* a) {
  const uint64_t np = opm_np(a->n_res), sp = opm_sp(a->n_seq);
  Carver c(nullptr, 0);
  c.take<bf16>(np * kOpmC * sp);
  c.take<bf16>(np * kOpmC * sp);
  if (a->mask) {
    c.take<bf16>(np * sp);
    c.take<float>(np * np);
  }
  return c.used;
}

template <typename MT, typename OT>
int run_opm(const odde_opm_args* a, hipStream_t st) {
  const int S = a->n_seq, N = a->n_res, Np = opm_np(N), Sp = opm_sp(S);
  Carver c(a->workspace, a->workspace_bytes);
  bf16* at = c.take<bf16>((uint64_t)Np * kOpmC * Sp);
  bf16* bt = c.take<bf16>((uint64_t)Np * kOpmC * Sp);
  bf16* maskt = a->mask ? c.take<bf16>((uint64_t)Np * Sp) : nullptr;
  float* norm = a->mask ? c.take<float>((uint64_t)Np * Np) : nullptr;
  LaunchScope ls(ODDE_K_OPM, st);
  if (S > 0) {  // with no MSA rows the outer products are empty: update = b_out / eps
    OpmProjArgs p;
    p.m = a->m; p.mask = a->mask; p.ln_w = a->ln_w; p.ln_b = a->ln_b;
    p.w12 = static_cast<const bf16*>(a->w_12);
    p.at = at; p.bt = bt; p.maskt = maskt;
    p.S = S; p.N = N; p.Sp = Sp; p.eps = a->ln_eps;
    dim3 grid(Sp / kOpmSB, Np);
    switch (a->c_m) {
      case 32: hipLaunchKernelGGL((opm_proj_kernel<MT, 32>), grid, dim3(256), 0, st, p); break;
      case 64: hipLaunchKernelGGL((opm_proj_kernel<MT, 64>), grid, dim3(256), 0, st, p); break;
      case 128: hipLaunchKernelGGL((opm_proj_kernel<MT, 128>), grid, dim3(256), 0, st, p); break;
      default: return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: c_m in {32, 64, 128}");
    }
    int rc = check_launch("opm_proj");
    if (rc) return rc;
  }
  if (norm) {
    const int nt = Np / 128;
    hipLaunchKernelGGL(opm_norm_kernel, dim3(nt * nt), dim3(512), 0, st, maskt, Np, Sp, a->eps,
                       norm);
    int rc = check_launch("opm_norm");
    if (rc) return rc;
  }
  OpmOuterArgs q;
  q.at = at; q.bt = bt; q.norm = norm;
  q.w_out = static_cast<const bf16*>(a->w_out);
  q.b_out = a->b_out;
  q.out = a->out;
  q.S = S; q.N = N; q.Np = Np; q.Sp = Sp; q.add = a->add_residual; q.eps = a->eps;
  using TL = OpmTileUsed;
  const unsigned tiles = (unsigned)(Np / TL::TI) * (unsigned)(Np / TL::TJ);
  switch (a->c_z) {
    case 64: hipLaunchKernelGGL((opm_outer_kernel<OT, 64, TL>), dim3(tiles), dim3(512), 0, st, q); break;
    case 128: hipLaunchKernelGGL((opm_outer_kernel<OT, 128, TL>), dim3(tiles), dim3(512), 0, st, q); break;
    case 256: hipLaunchKernelGGL((opm_outer_kernel<OT, 256, TL>), dim3(tiles), dim3(512), 0, st, q); break;
    case 384: hipLaunchKernelGGL((opm_outer_kernel<OT, 384, TL>), dim3(tiles), dim3(512), 0, st, q); break;
    default: return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: c_z in {64, 128, 256, 384}");
  }
  return check_launch("opm_outer");
}

int opm_check(const odde_opm_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "outer_product_mean: null args");
  if (a->struct_size != sizeof(odde_opm_args))
    return set_error(ODDE_EINVAL, "outer_product_mean: struct_size mismatch (ABI version skew)");
  if (a->n_seq < 0 || a->n_res < 0 || a->c_m <= 0 || a->c_hidden <= 0 || a->c_z <= 0)
    return set_error(ODDE_EINVAL, "outer_product_mean: bad sizes");
  if (a->c_hidden != kOpmC)
    return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: c_hidden must be 32");
  if (a->c_m != 32 && a->c_m != 64 && a->c_m != 128)
    return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: c_m in {32, 64, 128}");
  if (a->c_z != 64 && a->c_z != 128 && a->c_z != 256 && a->c_z != 384)
    return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: c_z in {64, 128, 256, 384}");
  if ((int64_t)opm_np(a->n_res) * kOpmC * opm_sp(a->n_seq) >= (int64_t(1) << 31) ||
      (int64_t)a->n_seq * a->n_res >= (int64_t(1) << 31))
    return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: at most 2^31 elements per operand");
  return ODDE_OK;
}

}  // namespace
}  // namespace odde

using namespace odde;

extern "C" {

int odde_opm_workspace_bytes(const odde_opm_args* a, uint64_t* bytes) {
  if (!bytes) return set_error(ODDE_EINVAL, "outer_product_mean: null argument");
  int rc = opm_check(a);
  if (rc) return rc;
  *bytes = opm_ws_bytes(a);
  return ODDE_OK;
}

int odde_opm_fwd(const odde_opm_args* a, void* stream) {
  int rc = opm_check(a);
  if (rc) return rc;
  if (!valid_dtype(a->m_dtype) || !valid_dtype(a->out_dtype) || !valid_dtype(a->compute_dtype))
    return set_error(ODDE_EINVAL, "outer_product_mean: bad dtype");
  if (a->compute_dtype != ODDE_BF16)
    return set_error(ODDE_EUNSUPPORTED, "outer_product_mean: the kernels compute in bf16");
  if ((!a->m && a->n_seq > 0) || !a->out || !a->ln_w || !a->ln_b || !a->w_12 || !a->w_out)
    return set_error(ODDE_EINVAL, "outer_product_mean: null tensor pointer");
  if ((reinterpret_cast<uintptr_t>(a->m) | reinterpret_cast<uintptr_t>(a->out) |
       reinterpret_cast<uintptr_t>(a->ln_w) | reinterpret_cast<uintptr_t>(a->ln_b) |
       reinterpret_cast<uintptr_t>(a->w_12) | reinterpret_cast<uintptr_t>(a->w_out)) & 15)
    return set_error(ODDE_EINVAL, "outer_product_mean: tensors must be 16-byte aligned");
  if (a->n_res == 0) return ODDE_OK;
  const uint64_t need = opm_ws_bytes(a);
  if (!a->workspace || a->workspace_bytes < need)
    return set_error(ODDE_EWORKSPACE, "outer_product_mean: workspace too small");
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255)
    return set_error(ODDE_EWORKSPACE, "outer_product_mean: workspace must be 256-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->m_dtype == ODDE_F32) {
    return a->out_dtype == ODDE_F32 ? run_opm<float, float>(a, st) : run_opm<float, bf16>(a, st);
  }
  return a->out_dtype == ODDE_F32 ? run_opm<bf16, float>(a, st) : run_opm<bf16, bf16>(a, st);
}

}  // extern "C"
