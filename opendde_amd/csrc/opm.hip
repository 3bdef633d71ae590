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
//    zeros).  The mask is stored transposed as f32 maskT[i][s] when given.
// 2. opm_outer: one workgroup per (8 residues i) x (4 residues j): the NT
//    GEMM mainloop (gemm.hpp) over k = s gives the 256 x 128 block of
//    outer products (32 residue pairs, each a 32 x 32 block); the block is
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
constexpr int kOpmTI = 8;     // residues i per outer workgroup (256 GEMM rows)
constexpr int kOpmTJ = 4;     // residues j per outer workgroup (128 GEMM rows)
constexpr int kOpmNS = 3;     // mainloop stages
constexpr int kOpmPairs = kOpmTI * kOpmTJ;
constexpr int kOpmPP = kOpmC * kOpmC + 8;  // LDS pitch of one pair's block (bf16)
using OpmShape = GemmShape<kOpmTI * kOpmC, kOpmTJ * kOpmC, 4>;

struct OpmProjArgs {
  const void* m;
  const float* mask;  // [S][N] or null
  const float* ln_w;
  const float* ln_b;
  const bf16* w12;    // [64][c_m]: W_1 rows then W_2 rows
  bf16* at;           // [Np * 32][Sp]
  bf16* bt;
  float* maskt;       // [Np][Sp] or null
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
        (sr < a.S && i < a.N) ? (a.mask ? a.mask[(size_t)sr * a.N + i] : 1.f) : 0.f;
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

struct OpmOuterArgs {
  const bf16* at;
  const bf16* bt;
  const float* maskt;  // [Np][Sp] or null (all ones: norm = S + eps)
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

template <typename OT, int CZ>
__global__ __launch_bounds__(512) void opm_outer_kernel(OpmOuterArgs a) {
  static_assert(kOpmPairs * kOpmPP * 2 + kOpmPairs * 4 <= kOpmNS * OpmShape::STAGE_ELEMS * 2,
                "the pair blocks and norms fit in the mainloop's LDS");
  constexpr int NU = CZ / 64;  // 16-wide z tiles per wave
  __shared__ __attribute__((aligned(16))) bf16 sm[kOpmNS * OpmShape::STAGE_ELEMS];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  int ti, tj;
  opm_tile_map(blockIdx.x, a.Np / kOpmTI, a.Np / kOpmTJ, ti, tj);
  const bf16* A = a.at + (size_t)ti * kOpmTI * kOpmC * a.Sp;
  const bf16* B = a.bt + (size_t)tj * kOpmTJ * kOpmC * a.Sp;
  f32x4 acc[OpmShape::MX][OpmShape::MY];
  gemm_nt_mainloop<kOpmTI * kOpmC, kOpmTJ * kOpmC, 4, kOpmNS, true>(
      [&](int r) { return A + (size_t)r * a.Sp; }, [&](int r) { return B + (size_t)r * a.Sp; },
      a.Sp, sm, acc);
  // acc[mi][mj]: column (lane % 16) = A row 64 wx + 16 mi + r16 (residue
  // 2 wx + mi / 2, c1 = 16 (mi % 2) + r16); values e = B rows
  // 64 wy + 16 mj + 4 g + e (residue 2 wy + mj / 2, c2 = 16 (mj % 2) + 4 g + e)
  const int wx = w & 3, wy = w >> 2;
  bf16* P = sm;
  float* normv = reinterpret_cast<float*>(sm + kOpmPairs * kOpmPP);
#pragma unroll
  for (int mi = 0; mi < OpmShape::MX; ++mi)
#pragma unroll
    for (int mj = 0; mj < OpmShape::MY; ++mj) {
      const int pair = (2 * wx + mi / 2) * kOpmTJ + 2 * wy + mj / 2;
      const int c1 = 16 * (mi & 1) + r16, c2 = 16 * (mj & 1) + 4 * g;
      bf16x4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (bf16)acc[mi][mj][e];
      *reinterpret_cast<bf16x4*>(&P[pair * kOpmPP + c1 * kOpmC + c2]) = v;
    }
  // norm[pair] = sum_s maskT[i][s] maskT[j][s] + eps: 16 lanes per pair
  {
    const int pair = threadIdx.x >> 4, part = threadIdx.x & 15;
    const int i = ti * kOpmTI + pair / kOpmTJ, j = tj * kOpmTJ + pair % kOpmTJ;
    float sum = 0.f;
    if (a.maskt) {
      const float* mi_ = a.maskt + (size_t)i * a.Sp;
      const float* mj_ = a.maskt + (size_t)j * a.Sp;
      for (int s = part; s < a.S; s += 16) sum += mi_[s] * mj_[s];
    } else if (part == 0) {
      sum = (float)a.S;
    }
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if (part == 0) normv[pair] = sum + a.eps;
  }
  __syncthreads();
  // out[pair][z] = sum_k P[pair][k] W_out[z][k]: wave w takes pairs
  // 16 (w & 1) .. + 15 and z tiles (w >> 1) + 4 u
  const int pt = w & 1;
  f32x4 acc2[NU];
#pragma unroll
  for (int u = 0; u < NU; ++u) acc2[u] = f32x4{0.f, 0.f, 0.f, 0.f};
  const bf16* prow = P + (16 * pt + r16) * kOpmPP + 8 * g;
#pragma unroll 4
  for (int ks = 0; ks < kOpmC; ++ks) {
    Frag<bf16> pf;
    pf.load(prow + ks * kOpmC);
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      Frag<bf16> wf;
      wf.load(a.w_out + (size_t)(16 * ((w >> 1) + 4 * u) + r16) * (kOpmC * kOpmC) + ks * kOpmC + 8 * g);
      mma(acc2[u], wf, pf);  // D[row = z 4g + r][col = pair l % 16]
    }
  }
  const int pair = 16 * pt + r16;
  const int i = ti * kOpmTI + pair / kOpmTJ, j = tj * kOpmTJ + pair % kOpmTJ;
  if (i >= a.N || j >= a.N) return;
  const float inv = 1.0f / normv[pair];
  OT* dst = static_cast<OT*>(a.out) + ((size_t)i * a.N + j) * CZ;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int z0 = 16 * ((w >> 1) + 4 * u) + 4 * g;
    float v[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float bo = a.b_out ? a.b_out[z0 + r] : 0.f;
      v[r] = round_to<bf16>((acc2[u][r] + bo) * inv);
    }
    if (a.add) {
      float zr[4];
      load4(dst + z0, zr);
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += zr[r];
    }
    store4(dst + z0, v[0], v[1], v[2], v[3]);
  }
}

namespace {

int opm_np(int n) { return round_up(n, 64); }
int opm_sp(int s) { return round_up(s, kOpmSB); }

uint64_t opm_ws_bytes(const odde_opm_args* a) {
  const uint64_t np = opm_np(a->n_res), sp = opm_sp(a->n_seq);
  Carver c(nullptr, 0);
  c.take<bf16>(np * kOpmC * sp);
  c.take<bf16>(np * kOpmC * sp);
  if (a->mask) c.take<float>(np * sp);
  return c.used;
}

template <typename MT, typename OT>
int run_opm(const odde_opm_args* a, hipStream_t st) {
  const int S = a->n_seq, N = a->n_res, Np = opm_np(N), Sp = opm_sp(S);
  Carver c(a->workspace, a->workspace_bytes);
  bf16* at = c.take<bf16>((uint64_t)Np * kOpmC * Sp);
  bf16* bt = c.take<bf16>((uint64_t)Np * kOpmC * Sp);
  float* maskt = a->mask ? c.take<float>((uint64_t)Np * Sp) : nullptr;
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
  OpmOuterArgs q;
  q.at = at; q.bt = bt; q.maskt = maskt;
  q.w_out = static_cast<const bf16*>(a->w_out);
  q.b_out = a->b_out;
  q.out = a->out;
  q.S = S; q.N = N; q.Np = Np; q.Sp = Sp; q.add = a->add_residual; q.eps = a->eps;
  const unsigned tiles = (unsigned)(Np / kOpmTI) * (unsigned)(Np / kOpmTJ);
  switch (a->c_z) {
    case 64: hipLaunchKernelGGL((opm_outer_kernel<OT, 64>), dim3(tiles), dim3(512), 0, st, q); break;
    case 128: hipLaunchKernelGGL((opm_outer_kernel<OT, 128>), dim3(tiles), dim3(512), 0, st, q); break;
    case 256: hipLaunchKernelGGL((opm_outer_kernel<OT, 256>), dim3(tiles), dim3(512), 0, st, q); break;
    case 384: hipLaunchKernelGGL((opm_outer_kernel<OT, 384>), dim3(tiles), dim3(512), 0, st, q); break;
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
