// Triangle attention (starting node over a strided pair view) for gfx950.
//
// Kernels, stream ordered:
//   0. triatt_prep   — per pair row: does it keep any key?  Initialises the
//                      per-row flags and the bound accumulators.
//   1. triatt_proj   — LayerNorm + one pass of bias-free projections per pair
//                      row: q (pre-scaled by log2(e)/sqrt(D)), k, v (zeroed on
//                      masked keys of rows that keep some key), sigmoid(g),
//                      the triangle bias (pre-scaled by log2(e)), the additive
//                      mask row and per-key keep flags, plus max |k| per
//                      (row, head) and max bias per (head, query).
//   2a. triatt_core_fast — flash attention without a running max: with
//                      s = q.k + bias (log2 units) bounded above by
//                      |q| max|k| + max bias, p = exp2(s) cannot overflow
//                      when that bound is small; masked keys drop out because
//                      their v rows are zero and the row sum is
//                      sum_k keep[k] p[k].  The only per-logit vector work
//                      is one exp2, half a convert and half a dot2.  Rows
//                      whose bound is too large, whose row sum underflows, or
//                      that keep no key at all are flagged for 2b.
//   2b. triatt_core_exact — online softmax with a running max and the exact
//                      additive mask (inf*(mask-1)); runs only for flagged
//                      rows (others exit at once).  A fully masked row gets a
//                      uniform softmax, i.e. the mean of v, as in the
//                      reference's float32 arithmetic.
//   3. triatt_out    — o W_o^T on MFMA plus the residual add, written through
//                      the (possibly transposed) output strides; on the
//                      weight-stationary path (bf16, C and H*32 of 64 or 128)
//                      it also computes the gate from the z rows it stages.
// The N x N x N logits never touch memory.
//
// Workspace layouts (CT = compute type, Jp = N rounded up to 64, I = rows):
//   q, k, gate : [I][H][Jp][32]           (no gate plane on the weight-stationary path)
//   v          : [I][H][Jp/32][2][64][8]  MFMA-ready V^T fragments: per block
//                of 32 keys, channel half db, lane (m + 16*g) with channel
//                d = 8 (m >> 2) + 4 db + (m & 3), slot e holds key 4g+e (e<4)
//                or 16+4g+(e-4) (e>=4)
//   keep       : [I][Jp/32][4][8]          the same key-slot order, 1 = kept
//   bias       : [Bb][H][Jp][Jp] f32       log2e-scaled tri bias (Bb batches)
//   mb         : [I][Jp] f32               log2e-scaled additive mask, -inf pads
//   mflag      : [I][Jp/32]                block holds a masked or padded key
//   kmax       : [I][H]   (f32 bits)       max over keys of |k|
//   bmax       : [Bb][H][Jp] (ordered int) max over keys of the bias row
//   rowflag    : [I]                       row needs the exact path
//   anykeep    : [I]                       row keeps at least one key
//   o          : [I][Jp][H*32]             attention output (gated off the
//                                           weight-stationary path)
#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

#include "common.hpp"
#include "gemm.hpp"
#include "lnpass.hpp"
#include "rowtile.hpp"
#include "runtime.hpp"

namespace odde {

// order-preserving float <-> int keys for atomicMax on signed values
__device__ __forceinline__ int fkey(float f) {
  const int b = __float_as_int(f);
  return b >= 0 ? b : b ^ 0x7fffffff;
}
__device__ __forceinline__ float fkey_inv(int k) { return __int_as_float(k >= 0 ? k : k ^ 0x7fffffff); }

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
  return v;
}
__device__ __forceinline__ float lanes16_max(float v) {
#pragma unroll
  for (int s = 1; s < 16; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
  return v;
}

__device__ __forceinline__ size_t vperm_offset(int row, int h, int heads, int jp, int j, int d) {
  const int kb = j >> 5, jj = j & 31;
  const int half = jj >> 4, gp = (jj & 15) >> 2, e = 4 * half + (jj & 3);
  // channel d = 8 (dl >> 2) + 4 db + (dl & 3): the PV accumulator row m of
  // channel half db is channel 8 (m >> 2) + 4 db + (m & 3), so a lane's two
  // halves hold 8 consecutive channels of its query (one 16-byte store)
  const int db = (d >> 2) & 1, dl = 4 * (d >> 3) + (d & 3);
  return (((((size_t)row * heads + h) * (jp >> 5) + kb) * 2 + db) * 64 + dl + 16 * gp) * 8 + e;
}
// slot (g, e) of a 32-key block -> key offset within the block
__device__ __forceinline__ int slot_key(int g, int e) { return e < 4 ? 4 * g + e : 16 + 4 * g + (e - 4); }
// key offset within a 32-key block -> index g*8+e of its slot
__device__ __forceinline__ int key_slot(int jj) {
  const int half = jj >> 4, gp = (jj & 15) >> 2;
  return gp * 8 + 4 * half + (jj & 3);
}

constexpr float kFastBound = 100.0f;      // log2 units; exp2 overflows past 128
constexpr float kUnderflowSum = 1e-30f;   // row sums below this go to the exact path

// ---------------------------------------------------------------------------
// 0. per-row preparation (module path): one workgroup per row
// ---------------------------------------------------------------------------
struct PrepArgs {
  const float* mask;
  int64_t m_s0, m_s1;
  int* anykeep;
  int* rowflag;
  unsigned* kmax;
  int* bmax;
  int n, jp, heads;
};

__global__ __launch_bounds__(256) void triatt_prep_kernel(PrepArgs a) {
  const int i = blockIdx.x;
  int keep = 0;
  for (int k = threadIdx.x; k < a.n; k += 256)
    keep |= a.mask ? a.mask[(int64_t)i * a.m_s0 + (int64_t)k * a.m_s1] == 1.0f : 1;
  keep = __syncthreads_or(keep);
  if (threadIdx.x == 0) {
    a.anykeep[i] = keep;
    a.rowflag[i] = !keep;
  }
  if (threadIdx.x < a.heads) {
    a.kmax[i * a.heads + threadIdx.x] = 0u;
    a.bmax[threadIdx.x * a.jp + i] = fkey(-INFINITY);
  }
}

// ---------------------------------------------------------------------------
// 1. projection
// ---------------------------------------------------------------------------
template <typename ZT, typename CT>
struct TriattProjArgs {
  const ZT* z;
  int64_t z_s0, z_s1;
  const float* mask;
  int64_t m_s0, m_s1;
  const float* ln_w;
  const float* ln_b;
  const CT* wb;  // [H][C]
  const CT* wq;  // [HD][C]
  const CT* wk;
  const CT* wv;
  const CT* wg;
  CT* q;
  CT* k;
  CT* v;
  CT* gate;
  CT* keep;
  float* bias;
  float* mb;
  int* mflag;
  unsigned* kmax;
  int* bmax;
  const int* anykeep;
  int n, jp, heads;
  float q_scale;   // log2(e) / sqrt(D)
  float mask_inf;  // inf * log2(e)
  float eps;
};

// Wave w of a workgroup owns pair rows (i, j0 + 16 w .. + 15) for kRB
// consecutive rows i: every weight fragment it reads from L2 serves kRB row
// blocks (the fp32 form, whose weights are too large to hold, is bound by
// those reads).  Rows i at or past n are skipped (workgroup-uniform).
// blockIdx.z of gridDim.z takes heads [z H / Z, (z + 1) H / Z) of q, k, v
// and the gate (small grids); z = 0 also writes the mask outputs and the
// triangle bias.
// kX3Mul (f32 compute, ODDE_F32X3): products in three bf16 parts.
// kStage (f32 data, one split): the weight rows of each 16-channel block --
// W_q, W_k, W_g, then W_v, then the H bias rows -- are staged in LDS
// (fp32 rows, or the three-part split rows: the same bytes), double-
// buffered, and shared by the workgroup's 4 waves.
template <typename ZT, typename CT, int kC, int kRB = 1, bool kX3Mul = false, bool kStage = false>
__global__ __launch_bounds__(256) void triatt_proj_kernel(TriattProjArgs<ZT, CT> a) {
  constexpr int C = kC * 32;
  using MF = MulFrag<CT, kX3Mul>;
  static_assert(!kStage || sizeof(CT) == 4, "staging: f32 weights");
  constexpr int WL = C + 4;                     // staged row stride (floats)
  constexpr int CHUNK = 3 * 16 * WL;            // three 16-row slots
  constexpr int PT = 3 * 16 * C / 4;            // 16-byte pieces per chunk
  constexpr int PPT = (PT + 255) / 256;
  __shared__ __attribute__((aligned(16))) float wsm[kStage ? 2 * CHUNK : 4];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int j0 = blockIdx.x * 64 + w * 16;
  const int jl = j0 + r16;
  const int i0 = blockIdx.y * kRB;
  const int H = a.heads, HD = H * 32, jp = a.jp;
  const bool lead = blockIdx.z == 0;
  const int ob_per = (HD / 16) / (int)gridDim.z;  // whole heads: two blocks each
  const int ob_lo = (int)blockIdx.z * ob_per, ob_hi = ob_lo + ob_per;
  MF x[kRB][kC];
  // staged chunks: ci < NOB: W_q, W_k, W_g rows 16 ci ..; NOB <= ci < 2 NOB:
  // W_v rows 16 (ci - NOB) .. in slot 0; ci = 2 NOB: the bias rows (< H,
  // zeros above) in slot 0.  Piece q of a chunk: slot q / (4 C), row r,
  // 16-byte column piece c4.
  const int NOB = HD / 16, NCHK = 2 * NOB + 1;
  f32x4 wreg[kStage ? PPT : 1];
  auto wload = [&](int ci) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      const int sl = q / (4 * C), u = q % (4 * C), r = u / (C / 4), c4 = u % (C / 4);
      const CT* src = nullptr;
      if (ci < NOB) src = (sl == 0 ? a.wq : sl == 1 ? a.wk : a.wg) + (size_t)(ci * 16 + r) * C;
      else if (sl == 0 && ci < 2 * NOB) src = a.wv + (size_t)((ci - NOB) * 16 + r) * C;
      else if (sl == 0 && r < H) src = a.wb + (size_t)r * C;
      wreg[k] = (PT % 256 == 0 || q < PT) && src ? *reinterpret_cast<const f32x4*>(src + 4 * c4)
                                                 : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto wstore = [&](int buf) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k;
      const int sl = q / (4 * C), u = q % (4 * C), r = u / (C / 4), c4 = u % (C / 4);
      if (PT % 256 == 0 || q < PT)
        *reinterpret_cast<f32x4*>(&wsm[buf * CHUNK + (sl * 16 + r) * WL + 4 * c4]) = wreg[k];
    }
  };
  // after chunk `cur` is multiplied: stage chunk cur + 1 (its buffer was
  // last read in chunk cur - 1, before the barrier that ended it), request
  // chunk cur + 2, and make chunk cur + 1 visible
  int cur = 0;
  auto advance = [&]() {
    if (cur + 1 < NCHK) {
      wstore((cur + 1) & 1);
      if (cur + 2 < NCHK) wload(cur + 2);
    }
    __syncthreads();
    ++cur;
  };
  auto wslot = [&](int sl) { return wsm + (cur & 1) * CHUNK + (sl * 16 + r16) * WL; };

  // mask rows: additive form for the exact core, keep flags for the fast one
  __shared__ float keep_s[kRB][64];
  __shared__ int wmasked[kRB][4];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int i = i0 + rb;
    const bool live = i < a.n;
    const bool valid = live && jl < a.n;
    const ZT* rowp = a.z + (int64_t)(live ? i : 0) * a.z_s0 + (int64_t)(valid ? jl : 0) * a.z_s1;
    {
      Frag<CT> xt[kC];
      ln_rows_to_frags<ZT, CT, C>(rowp, valid, a.ln_w, a.ln_b, a.eps, xt);
#pragma unroll
      for (int t = 0; t < kC; ++t) to_mul(xt[t], x[rb][t]);
    }
    float mv = -INFINITY, kp = 0.f;
    if (valid) {
      const float m = a.mask ? a.mask[(int64_t)i * a.m_s0 + (int64_t)jl * a.m_s1] : 1.0f;
      mv = (m - 1.0f) * a.mask_inf;
      kp = m == 1.0f ? 1.f : 0.f;
    }
    if (g == 0) {
      if (live && lead) a.mb[(size_t)i * jp + jl] = mv;
      keep_s[rb][w * 16 + r16] = kp;
    }
    const bool any_masked = __any(mv != 0.f);
    if (l == 0) wmasked[rb][w] = any_masked ? 1 : 0;
  }
  __syncthreads();
  bool zero_v[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const int i = i0 + rb;
    zero_v[rb] = false;
    if (i >= a.n) continue;
    if (lead && threadIdx.x < 2) {
      const int b = threadIdx.x;  // 32-key block b of this 64-key tile = waves 2b, 2b+1
      a.mflag[(size_t)i * (jp >> 5) + blockIdx.x * 2 + b] = wmasked[rb][2 * b] | wmasked[rb][2 * b + 1];
    }
    if (lead && threadIdx.x < 64) {
      const int t = threadIdx.x, kb = t >> 5, s = t & 31;
      a.keep[((size_t)i * (jp >> 5) + blockIdx.x * 2 + kb) * 32 + s] =
          from_f32<CT>(keep_s[rb][kb * 32 + slot_key(s >> 3, s & 7)]);
    }
    zero_v[rb] = a.anykeep[i] != 0;
  }

  if constexpr (kStage) {
    wload(0);
    wstore(0);
    wload(1);
    __syncthreads();
  }
  // q, k, gate: product W x^T -> lane holds pair row jl, channels o..o+3.
  float ss[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) ss[rb] = 0.f;
  for (int ob = ob_lo; ob < ob_hi; ++ob) {
    f32x4 aq[kRB], ak[kRB], ag[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) aq[rb] = ak[rb] = ag[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      if constexpr (kStage) staged_w_frag(wslot(0), C, t, f);
      else load_w_frag(a.wq, C, ob * 16, HD, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(aq[rb], f, x[rb][t]);
      if constexpr (kStage) staged_w_frag(wslot(1), C, t, f);
      else load_w_frag(a.wk, C, ob * 16, HD, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ak[rb], f, x[rb][t]);
      if constexpr (kStage) staged_w_frag(wslot(2), C, t, f);
      else load_w_frag(a.wg, C, ob * 16, HD, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ag[rb], f, x[rb][t]);
    }
    const int o = ob * 16 + 4 * g;
    const int h = o >> 5, d = o & 31;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int i = i0 + rb;
      if (i >= a.n) continue;
      const size_t off = (((size_t)i * H + h) * jp + jl) * 32 + d;
      const float s = a.q_scale;
      store4(a.q + off, aq[rb][0] * s, aq[rb][1] * s, aq[rb][2] * s, aq[rb][3] * s);
      store4(a.k + off, ak[rb][0], ak[rb][1], ak[rb][2], ak[rb][3]);
      store4(a.gate + off, sigmoidf_(ag[rb][0]), sigmoidf_(ag[rb][1]), sigmoidf_(ag[rb][2]),
             sigmoidf_(ag[rb][3]));
      ss[rb] += ak[rb][0] * ak[rb][0] + ak[rb][1] * ak[rb][1] + ak[rb][2] * ak[rb][2] +
                ak[rb][3] * ak[rb][3];
      if (ob & 1) {  // the 32 channels of head ob/2 are complete
        const float nrm = lanes16_max(sqrtf(group_sum_fast(ss[rb])));
        if (l == 0) atomicMax(&a.kmax[i * H + (ob >> 1)], __float_as_uint(nrm));
        ss[rb] = 0.f;
      }
    }
    if constexpr (kStage) advance();
  }

  // v: product x W^T -> lane holds channel o, pair rows j0+4g .. +3.
  const int jb = j0 + 4 * g;
  float vk[kRB][4];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int e = 0; e < 4; ++e) vk[rb][e] = zero_v[rb] ? keep_s[rb][w * 16 + 4 * g + e] : 1.f;
  for (int ob = ob_lo; ob < ob_hi; ++ob) {
    f32x4 av[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) av[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      if constexpr (kStage) staged_w_frag(wslot(0), C, t, f);
      else load_w_frag(a.wv, C, ob * 16, HD, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(av[rb], x[rb][t], f);
    }
    const int o = ob * 16 + r16;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int i = i0 + rb;
      if (i >= a.n) continue;
      store4(a.v + vperm_offset(i, o >> 5, H, jp, jb, o & 31), av[rb][0] * vk[rb][0],
             av[rb][1] * vk[rb][1], av[rb][2] * vk[rb][2], av[rb][3] * vk[rb][3]);
    }
    if constexpr (kStage) advance();
  }

  // triangle bias: channel h = r16 (< H), rows jb..jb+3 -> bias[h][i][jb..]
  if (lead) {
    f32x4 ab[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) ab[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      MF f;
      if constexpr (kStage) staged_w_frag(wslot(0), C, t, f);
      else load_w_frag(a.wb, C, 0, H, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(ab[rb], x[rb][t], f);
    }
    const float s = kLog2e;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int i = i0 + rb;
      if (i >= a.n) continue;
      const float bm =
          group_max_fast(fmaxf(fmaxf(ab[rb][0], ab[rb][1]), fmaxf(ab[rb][2], ab[rb][3])) * s);
      if (r16 < H) {
        store4(a.bias + ((size_t)r16 * jp + i) * jp + jb, ab[rb][0] * s, ab[rb][1] * s,
               ab[rb][2] * s, ab[rb][3] * s);
        if (g == 0) atomicMax(&a.bmax[r16 * jp + i], fkey(bm));
      }
    }
  }
}

// Weight-stationary form of the projection (used when each wave's weight
// slice fits in registers, e.g. C = H*D = 128 in bf16): wave 0 holds W_q (and
// the tri-bias rows), wave 1 W_k, wave 2 W_v (the gate is computed by the
// output kernel, triatt_out_ws_kernel); the workgroup loops over 64-row tiles
// (i, j0..j0+63), staging LN(z) once in LDS per tile.  The next tile's z rows
// stream into LDS (direct loads) while a tile is computed.
template <typename ZT, typename CT, int kC, int kHD>
__global__ __launch_bounds__(256, 2) void triatt_proj_ws_kernel(TriattProjArgs<ZT, CT> a,
                                                                int ntiles) {
  constexpr int C = kC * 32, HD = kHD * 32, NB = HD / 16;
  __shared__ __attribute__((aligned(16))) CT xs[kTileRows * TileLD<CT, C>::value];
  __shared__ __attribute__((aligned(16))) unsigned char raw[RawTile<ZT, C>::BYTES];
  __shared__ float keep_s[kTileRows];
  __shared__ float lnp[2 * C];  // LayerNorm weight, bias
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int H = a.heads, jp = a.jp, n = a.n;
  for (int t = threadIdx.x; t < C; t += 256) {
    lnp[t] = a.ln_w[t];
    lnp[C + t] = a.ln_b[t];
  }
  // wave 3 only helps stage the tile: the gate is computed in the output kernel
  const CT* W = w == 0 ? a.wq : w == 1 ? a.wk : a.wv;
  Frag<CT> wf[NB][kC];
  load_w_slice(W, C, 0, HD, wf);
  Frag<CT> wbf[kC];
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    if (w == 0) load_w_frag(a.wb, C, 0, H, t, wbf[t]);
    else wbf[t].zero();
  }
  const int tiles_per_row = jp / kTileRows;
  // rows past n read row n-1 (always present) and are masked in the LN pass
  auto issue = [&](int tl) {
    const int ti = tl / tiles_per_row, tj0 = (tl % tiles_per_row) * kTileRows;
    raw_tile_issue<ZT, C, kStream>(a.z + (int64_t)ti * a.z_s0, a.z_s1, tj0, n, raw);
  };
  // the next tile's mask value (wave 0, lane = key) and row flag are loaded
  // with its z rows, so no global load latency sits inside a tile
  float mnext = 1.f;
  int aknext = 0;
  auto mfetch = [&](int tl) {
    const int ti = tl / tiles_per_row, j = (tl % tiles_per_row) * kTileRows + l;
    if (w == 0 && a.mask && j < n) mnext = a.mask[(int64_t)ti * a.m_s0 + (int64_t)j * a.m_s1];
    aknext = a.anykeep[ti];
  };
  if ((int)blockIdx.x < ntiles) {
    issue(blockIdx.x);
    mfetch(blockIdx.x);
  }
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int i = tile / tiles_per_row;
    const int j0 = (tile % tiles_per_row) * kTileRows;
    const float mcur = mnext;
    const bool zero_v = aknext != 0;
    raw_tile_wait();  // also: every wave is done with the previous tile's xs
    raw_tile_ln<ZT, CT, C>(raw, [&](int r) { return j0 + r < n; }, lnp, lnp + C, a.eps, xs);
    if (w == 0) {  // mask row of the tile's 64 keys (lane l = key j0 + l)
      const int j = j0 + l;
      float mv = -INFINITY, kp = 0.f;
      if (j < n) {
        const float m = mcur;
        mv = (m - 1.0f) * a.mask_inf;
        kp = m == 1.0f ? 1.f : 0.f;
      }
      a.mb[(size_t)i * jp + j] = mv;
      keep_s[l] = kp;
      const uint64_t bal = __ballot(mv != 0.f);
      if (l < 2)
        a.mflag[(size_t)i * (jp >> 5) + (j0 >> 5) + l] =
            ((l == 0 ? bal : bal >> 32) & 0xffffffffull) != 0;
    }
    lds_barrier();  // xs and keep_s ready; raw consumed
    if (tile + (int)gridDim.x < ntiles) {
      issue(tile + gridDim.x);  // raw is free again
      mfetch(tile + gridDim.x);
    }
    if (threadIdx.x < kTileRows) {
      const int t = threadIdx.x, kb = t >> 5, sl = t & 31;
      a.keep[((size_t)i * (jp >> 5) + (j0 >> 5) + kb) * 32 + sl] =
          from_f32<CT>(keep_s[kb * 32 + slot_key(sl >> 3, sl & 7)]);
    }
    float knm[kHD];
#pragma unroll
    for (int h = 0; h < kHD; ++h) knm[h] = 0.f;
    float bmx = -INFINITY;
#pragma unroll
    for (int rb = 0; rb < kTileRows / 16; ++rb) {
      if (w == 3) break;
      Frag<CT> xf[kC];
      tile_frags<CT, C>(xs, rb, xf);
      if (w == 2) {  // v: x W^T -> lane holds channel o, rows jb..jb+3
        const int jb = j0 + rb * 16 + 4 * g;
        float vk[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) vk[e] = zero_v ? keep_s[rb * 16 + 4 * g + e] : 1.f;
#pragma unroll
        for (int ob = 0; ob < NB; ++ob) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < kC; ++t) mma(acc, xf[t], wf[ob][t]);
          const int o = ob * 16 + r16;
          store4(a.v + vperm_offset(i, o >> 5, H, jp, jb, o & 31), acc[0] * vk[0],
                 acc[1] * vk[1], acc[2] * vk[2], acc[3] * vk[3]);
        }
      } else {  // q / k: W x^T -> lane holds row jr, channels o..o+3
        const int jr = j0 + rb * 16 + r16;
        float ss = 0.f;
#pragma unroll
        for (int ob = 0; ob < NB; ++ob) {
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < kC; ++t) mma(acc, wf[ob][t], xf[t]);
          const int o = ob * 16 + 4 * g;
          const size_t off = (((size_t)i * H + (o >> 5)) * jp + jr) * 32 + (o & 31);
          if (w == 0) {
            const float sc = a.q_scale;
            store4(a.q + off, acc[0] * sc, acc[1] * sc, acc[2] * sc, acc[3] * sc);
          } else {
            store4(a.k + off, acc[0], acc[1], acc[2], acc[3]);
            ss += acc[0] * acc[0] + acc[1] * acc[1] + acc[2] * acc[2] + acc[3] * acc[3];
            if (ob & 1) {
              knm[ob >> 1] = fmaxf(knm[ob >> 1], sqrtf(group_sum_fast(ss)));
              ss = 0.f;
            }
          }
        }
        if (w == 0) {  // tri bias: lane h = r16, rows jb..jb+3
          f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int t = 0; t < kC; ++t) mma(acc, xf[t], wbf[t]);
          const float sc = kLog2e;
          const int jb = j0 + rb * 16 + 4 * g;
          if (r16 < H)
            store4(a.bias + ((size_t)r16 * jp + i) * jp + jb, acc[0] * sc, acc[1] * sc,
                   acc[2] * sc, acc[3] * sc);
          bmx = fmaxf(bmx, fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3])) * sc);
        }
      }
    }
    if (w == 1) {
#pragma unroll
      for (int h = 0; h < kHD; ++h) {
        const float v = lanes16_max(knm[h]);
        if (l == 0 && h < H) atomicMax(&a.kmax[i * H + h], __float_as_uint(v));
      }
    }
    if (w == 0) {
      const float bm = group_max_fast(bmx);
      if (g == 0 && r16 < H) atomicMax(&a.bmax[r16 * jp + i], fkey(bm));
    }
    // xs and keep_s are rewritten only after the barrier in raw_tile_wait()
  }
}

// Projection for H*32 = 128 with the 384 q, k, v output channels split evenly
// over the four waves, 96 each (whole heads): wave 0 q heads 0-2 (and the
// tri-bias rows), wave 1 q head 3 and k heads 0-1, wave 2 k heads 2-3 and v
// head 0, wave 3 v heads 1-3 (with the gate computed by the output kernel,
// the three-matrix split of triatt_proj_ws_kernel leaves a wave idle).  Each
// wave keeps its 6 x kC weight fragments in registers.  A wave's results
// stay in registers until its part of the next tile's z rows has landed and
// are stored only then, so no wave waits for its own stores: they drain
// while the next tile is normalised and multiplied.
// Keeps a value packed where it is formed (the 4 x bf16 results are held
// until after a wait; left to the scheduler, their f32 sources stay live).
__device__ __forceinline__ void pin(bf16x4& v) { asm volatile("" : "+v"(v)); }

template <int W, typename ZT, typename CT, int kC>
__device__ __forceinline__ void proj_ws4_role(const TriattProjArgs<ZT, CT>& a, const CT* xs,
                                              const float* keep_s, const Frag<CT> (&wf)[6][kC],
                                              const Frag<CT> (&wbf)[kC], int i, int j0,
                                              bool zero_v) {
  constexpr int RB = kTileRows / 16, H = 4;
  const int l = lane_id(), g = l >> 4, r16 = l & 15;
  const int jp = a.jp;
  bf16x4 out[RB][6];
  f32x4 bo[RB];
  float knm[H], ss = 0.f, bmx = -INFINITY;
#pragma unroll
  for (int h = 0; h < H; ++h) knm[h] = 0.f;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    Frag<CT> xf[kC];
    tile_frags<CT, 32 * kC>(xs, rb, xf);
#pragma unroll
    for (int ob = 0; ob < 6; ++ob) {
      constexpr int base = 96 * W;
      const int gc = base + 16 * ob, mat = gc >> 7, ch = gc & 127;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (mat == 2) {  // v: x W^T -> lane holds channel ch + r16, rows 4g..4g+3
#pragma unroll
        for (int t = 0; t < kC; ++t) mma(acc, xf[t], wf[ob][t]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          out[rb][ob][e] = (bf16)(acc[e] * (zero_v ? keep_s[rb * 16 + 4 * g + e] : 1.f));
        pin(out[rb][ob]);
      } else {  // q, k: W x^T -> lane holds row r16, channels ch + 4g..4g+3
#pragma unroll
        for (int t = 0; t < kC; ++t) mma(acc, wf[ob][t], xf[t]);
        const float sc = mat == 0 ? a.q_scale : 1.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) out[rb][ob][e] = (bf16)(acc[e] * sc);
        pin(out[rb][ob]);
        if (mat == 1) {
          ss += acc[0] * acc[0] + acc[1] * acc[1] + acc[2] * acc[2] + acc[3] * acc[3];
          if (ch & 16) {  // the 32 channels of k head ch / 32 are complete
            knm[ch >> 5] = fmaxf(knm[ch >> 5], sqrtf(group_sum_fast(ss)));
            ss = 0.f;
          }
        }
      }
    }
    if (W == 0) {  // tri bias: lane h = r16, rows 4g..4g+3
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < kC; ++t) mma(acc, xf[t], wbf[t]);
#pragma unroll
      for (int e = 0; e < 4; ++e) bo[rb][e] = acc[e] * kLog2e;
      bmx = fmaxf(bmx, fmaxf(fmaxf(bo[rb][0], bo[rb][1]), fmaxf(bo[rb][2], bo[rb][3])));
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of the next tile landed
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int ob = 0; ob < 6; ++ob) {
      const int gc = 96 * W + 16 * ob, mat = gc >> 7, ch = gc & 127;
      bf16x8 v8;
      if (mat == 2) {
        // keys 4g..4g+3 of row block rb and the same keys + 16 of row block
        // rb + 1 fill one 16-byte slot group of the V fragment layout
        if (rb & 1) continue;
        const int o = ch + r16;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v8[e] = out[rb][ob][e];
          v8[4 + e] = out[rb + 1][ob][e];
        }
        store_stream(reinterpret_cast<bf16x8*>(a.v + vperm_offset(i, o >> 5, H, jp, j0 + rb * 16 + 4 * g,
                                                                  o & 31)), v8);
      } else {
        if (ch & 16) continue;  // stored with the head's first block
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v8[e] = out[rb][ob][e];
          v8[4 + e] = out[rb][ob + 1][e];
        }
        store_stream(reinterpret_cast<bf16x8*>((mat ? a.k : a.q) +
                                               (((size_t)i * H + (ch >> 5)) * jp + j0 + rb * 16 + r16) * 32 +
                                               8 * g), v8);
      }
    }
    if (W == 0 && r16 < H)
      *reinterpret_cast<f32x4*>(a.bias + ((size_t)r16 * jp + i) * jp + j0 + rb * 16 + 4 * g) =
          bo[rb];  // half lines: the default policy (the core re-reads the bias through L2)
  }
  if (W == 1 || W == 2) {
#pragma unroll
    for (int h = 0; h < H; ++h) {
      const int kh0 = W == 1 ? 0 : 2;  // this wave's k heads: kh0, kh0 + 1
      if (h < kh0 || h > kh0 + 1) continue;
      const float v = lanes16_max(knm[h]);
      if (l == 0) atomicMax(&a.kmax[i * H + h], __float_as_uint(v));
    }
  }
  if (W == 0) {
    const float bm = group_max_fast(bmx);
    if (g == 0 && r16 < H) atomicMax(&a.bmax[r16 * jp + i], fkey(bm));
  }
}

template <typename ZT, typename CT, int kC>
__global__ __launch_bounds__(256, 2) void triatt_proj_ws4_kernel(TriattProjArgs<ZT, CT> a,
                                                                 int ntiles) {
  constexpr int C = kC * 32, HD = 128;
  static_assert(sizeof(CT) == 2, "bf16 compute");
  __shared__ __attribute__((aligned(16))) CT xs[kTileRows * TileLD<CT, C>::value];
  __shared__ __attribute__((aligned(16))) unsigned char raw[RawTile<ZT, C>::BYTES];
  __shared__ float keep_s[kTileRows];
  __shared__ float lnp[2 * C];  // LayerNorm weight, bias
  const int w = wave_id(), l = lane_id();
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int jp = a.jp, n = a.n;
  for (int t = threadIdx.x; t < C; t += 256) {
    lnp[t] = a.ln_w[t];
    lnp[C + t] = a.ln_b[t];
  }
  // q, k: output block ob of a head (the head's 32 channels in two blocks)
  // computes channels 8 (m >> 2) + 4 (ob & 1) + (m & 3) for MFMA row m, so a
  // lane's results of the two blocks are 8 consecutive channels (one 16-byte
  // store); v keeps the natural order (its lanes hold channels)
  Frag<CT> wf[6][kC];
  {
    const int r16 = l & 15, g = l >> 4;
#pragma unroll
    for (int ob = 0; ob < 6; ++ob) {
      const int gc = 96 * wu + 16 * ob, mat = gc >> 7, ch = gc & 127;
      const CT* W = mat == 0 ? a.wq : mat == 1 ? a.wk : a.wv;
      const int row = mat == 2 ? ch + r16
                               : (ch & ~31) + 8 * (r16 >> 2) + 4 * ((ch >> 4) & 1) + (r16 & 3);
#pragma unroll
      for (int t = 0; t < kC; ++t) wf[ob][t].load(W + (size_t)row * C + 32 * t + 8 * g);
    }
  }
  Frag<CT> wbf[kC];
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    if (wu == 0) load_w_frag(a.wb, C, 0, a.heads, t, wbf[t]);
    else wbf[t].zero();
  }
  const int tiles_per_row = jp / kTileRows;
  auto issue = [&](int tl) {
    const int ti = tl / tiles_per_row, tj0 = (tl % tiles_per_row) * kTileRows;
    raw_tile_issue<ZT, C, kStream>(a.z + (int64_t)ti * a.z_s0, a.z_s1, tj0, n, raw);
  };
  // the next tile's mask value (wave 0, lane = key) and row flag are loaded
  // with its z rows
  float mnext = 1.f;
  int aknext = 0;
  auto mfetch = [&](int tl) {
    const int ti = tl / tiles_per_row, j = (tl % tiles_per_row) * kTileRows + l;
    if (w == 0 && a.mask && j < n) mnext = a.mask[(int64_t)ti * a.m_s0 + (int64_t)j * a.m_s1];
    aknext = a.anykeep[ti];
  };
  if ((int)blockIdx.x < ntiles) {
    issue(blockIdx.x);
    mfetch(blockIdx.x);
  }
  raw_tile_wait();
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int i = tile / tiles_per_row;
    const int j0 = (tile % tiles_per_row) * kTileRows;
    const float mcur = mnext;
    const bool zero_v = aknext != 0;
    raw_tile_ln<ZT, CT, C>(raw, [&](int r) { return j0 + r < n; }, lnp, lnp + C, a.eps, xs);
    if (w == 0) {  // mask row of the tile's 64 keys (lane l = key j0 + l)
      const int j = j0 + l;
      float mv = -INFINITY, kp = 0.f;
      if (j < n) {
        mv = (mcur - 1.0f) * a.mask_inf;
        kp = mcur == 1.0f ? 1.f : 0.f;
      }
      a.mb[(size_t)i * jp + j] = mv;
      keep_s[l] = kp;
      const uint64_t bal = __ballot(mv != 0.f);
      if (l < 2)
        a.mflag[(size_t)i * (jp >> 5) + (j0 >> 5) + l] =
            ((l == 0 ? bal : bal >> 32) & 0xffffffffull) != 0;
    }
    lds_barrier();  // xs and keep_s ready; raw consumed
    if (tile + (int)gridDim.x < ntiles) {
      issue(tile + gridDim.x);  // raw is free again
      mfetch(tile + gridDim.x);
    }
    if (threadIdx.x < kTileRows) {
      const int t = threadIdx.x, kb = t >> 5, sl = t & 31;
      a.keep[((size_t)i * (jp >> 5) + (j0 >> 5) + kb) * 32 + sl] =
          from_f32<CT>(keep_s[kb * 32 + slot_key(sl >> 3, sl & 7)]);
    }
    switch (wu) {
      case 0: proj_ws4_role<0>(a, xs, keep_s, wf, wbf, i, j0, zero_v); break;
      case 1: proj_ws4_role<1>(a, xs, keep_s, wf, wbf, i, j0, zero_v); break;
      case 2: proj_ws4_role<2>(a, xs, keep_s, wf, wbf, i, j0, zero_v); break;
      default: proj_ws4_role<3>(a, xs, keep_s, wf, wbf, i, j0, zero_v); break;
    }
    lds_barrier();  // every wave's part of the next raw tile landed; xs, keep_s free
  }
}

// ---------------------------------------------------------------------------
// 2. flash cores
// ---------------------------------------------------------------------------
template <typename CT>
struct TriattCoreArgs {
  const CT* q;
  const CT* k;
  const CT* v;
  const CT* keep;
  const float* bias;  // [Bb][H][Jp][Jp] f32, log2e-scaled
  const float* mb;    // [rows][Jp] f32, log2e-scaled additive mask, -inf on pads
  const int* mflag;   // [rows][Jp/32] nonzero if that key block needs the mask
  const unsigned* kmax;
  const int* bmax;
  int* rowflag;
  const int* anykeep; // [rows] row keeps at least one key
  const CT* gate;     // may be null
  CT* out;
  int64_t o_row, o_h, o_j;  // element strides of out[row][h][q][d]
  int rows, heads, n, jp, rows_per_bias;
  int out16;  // bf16 out with every (row, h, q) start 16-byte aligned
  // f32 data, products on the bf16 MFMA in three parts (ODDE_F32X3)
  int x3 = 0;
};

// Row sums of the probabilities: bf16 pairs through v_dot2 (the same rounded
// values the PV product consumes), f32 by fused multiply-adds.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float psum8(const Frag<bf16>& p, const Frag<bf16>& wgt, float acc) {
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    bf16x2_t pr = {p.v[e], p.v[e + 1]};
    bf16x2_t wr = {wgt.v[e], wgt.v[e + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(pr, wr, acc, false);
  }
  return acc;
}
__device__ __forceinline__ float psum8(const Frag<float>& p, const Frag<float>& wgt, float acc) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = fmaf(p.get(e), wgt.get(e), acc);
  return acc;
}
__device__ __forceinline__ Frag<bf16> ones_frag(bf16) {
  Frag<bf16> f;
  for (int e = 0; e < 8; ++e) f.v[e] = (bf16)1.0f;
  return f;
}
__device__ __forceinline__ Frag<float> ones_frag(float) {
  Frag<float> f;
  f.lo = f32x4{1.f, 1.f, 1.f, 1.f};
  f.hi = f.lo;
  return f;
}

// Epilogue shared by both cores: 1/l, sigmoid gate, store.  The lane's
// output address is formed once; rows and query blocks step it by uniform
// (scalar) offsets, so no per-store 64-bit multiplies run on the VALU.
template <typename CT, int R, int QB>
__device__ __forceinline__ void core_store(const TriattCoreArgs<CT>& a, int row0, int h, int q0,
                                           f32x4 (&o)[R][2][QB], const float (&inv)[R][QB]) {
  const int g = lane_id() >> 4, r16 = lane_id() & 15;
  CT* const base = a.out + (int64_t)row0 * a.o_row + (int64_t)h * a.o_h +
                   (int64_t)(q0 + r16) * a.o_j + 8 * g;
  const CT* const gbase =
      a.gate ? a.gate + (((size_t)row0 * a.heads + h) * a.jp + q0 + r16) * 32 + 8 * g : nullptr;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int row = row0 + r;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qq = q0 + 16 * qb + r16;
      if (row >= a.rows || qq >= a.n) continue;
      // lane (g, r16) holds channels 8g .. 8g + 7 of query qq: half db gives
      // 8g + 4db + e (the V fragment channel order)
      float ov[8];
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[4 * db + e] = o[r][db][qb][e] * inv[r][qb];
      if (a.gate) {
        const CT* gp = gbase + ((size_t)r * a.heads * a.jp + 16 * qb) * 32;
        float gv[8];
        load4(gp, gv);
        load4(gp + 4, gv + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) ov[e] *= gv[e];
      }
      CT* dst = base + (int64_t)r * a.o_row + (int64_t)(16 * qb) * a.o_j;
      if constexpr (sizeof(CT) == 2) {
        if (a.out16) {
          bf16x8 v8;
#pragma unroll
          for (int e = 0; e < 8; ++e) v8[e] = (bf16)ov[e];
          store_stream(reinterpret_cast<bf16x8*>(dst), v8);
          continue;
        }
      }
      store4(dst, ov[0], ov[1], ov[2], ov[3]);
      store4(dst + 4, ov[4], ov[5], ov[6], ov[7]);
    }
  }
}

// LDS staging of one 32-key block for a workgroup: K and V blocks of its
// R_WG rows, their keep flags, and the f32 bias tile of its Q_WG queries.
// 16-byte chunks are placed so that fragment reads are bank-conflict free:
// a K key row's chunks are xor-swizzled by (key / 4) % 4 (bf16), a bias row's
// eight chunks by q % 8.
template <typename CT, int R_WG, int Q_WG>
struct CoreStage {
  static constexpr int VEC = 16 / sizeof(CT);        // elements per chunk
  static constexpr int KCH = 32 / VEC;               // chunks per key row (4 bf16, 8 f32)
  static constexpr int K_CHUNKS = R_WG * 32 * KCH;   // K (and V) chunks per stage
  static constexpr int KP_CHUNKS = R_WG * KCH;       // keep chunks (32 flags per row)
  static constexpr int B_CHUNKS = Q_WG * 8;          // bias chunks (32 f32 per query)
  static constexpr int TOTAL = 2 * K_CHUNKS + KP_CHUNKS + B_CHUNKS;
  f32x4 k[K_CHUNKS];
  f32x4 v[K_CHUNKS];
  f32x4 kp[KP_CHUNKS];
  f32x4 b[B_CHUNKS];
};

__device__ __forceinline__ int kswz(int key, int chunk, int kch) {
  return kch == 4 ? (chunk ^ ((key >> 2) & 3)) : chunk;
}

// One workgroup = RG x QS waves over R_WG = RG*R rows and Q_WG = QS*16*QB
// queries of one head.  Per 32-key block the workgroup stages K, V, keep and
// the bias tile in LDS once (double buffered: the loads of block t+1 are in
// flight while block t is computed), so each byte fetched from L2 feeds R_WG
// rows x Q_WG queries.  The staging goes straight from global memory into LDS
// (buffer loads with the LDS flag): each lane's byte offsets into K, V, keep
// and the bias are fixed for the whole kernel and the block advance is a
// uniform scalar offset, so staging costs no registers, no LDS writes by the
// waves and no per-block vector address arithmetic.  Wave (rg, qs) owns rows
// rg*R.. and queries qs*16*QB..: S^T = K Q^T on MFMA with the accumulator
// initialised from the bias fragment (shared by its R rows), p = exp2(s), row
// sums sum_k keep[k] p[k] (bf16: one more MFMA per query block with the keep
// flags as the A operand, so the sum is over the same rounded p the PV product
// consumes; f32: fused multiply-adds), O^T += V^T P^T on MFMA.
// Workgroups are dealt to the 8 XCDs round-robin by linear id.  Map the
// linear id L to (query block x, group) so that the nx query blocks of one
// group (a set of rows of one head) run back to back on one XCD: that
// group's K and V rows are then fetched into one L2 and reused from there,
// instead of being fetched into every XCD's L2.  A plain row-major order is
// used when the group count is not a multiple of 8.
__device__ __forceinline__ void xcd_group_map(int L, int nx, int ngroups, int& x, int& grp) {
  if (ngroups & 7) {
    x = L % nx;
    grp = L / nx;
    return;
  }
  const int xcd = L & 7, s = L >> 3;
  grp = xcd + 8 * (s / nx);
  x = s % nx;
}

template <typename CT, int R, int QB, int RG, int QS, bool kX3 = false>
__global__ __launch_bounds__(64 * RG * QS) void triatt_core_fast_kernel(TriattCoreArgs<CT> a, int nx,
                                                                        int ny) {
  static_assert(!kX3 || sizeof(CT) == 4, "the three-part form takes f32 data");
  constexpr int NW = RG * QS;
  constexpr int R_WG = RG * R, Q_WG = QS * 16 * QB;
  typedef CoreStage<CT, R_WG, Q_WG> Stage;
  constexpr int VEC = Stage::VEC, KCH = Stage::KCH;
  constexpr bool kMfmaSum = sizeof(CT) == 2;
  // direct-load instructions (64 lanes x 16 bytes) per region, dealt to the
  // waves round-robin
  constexpr int NKI = Stage::K_CHUNKS / 64, NBI = Stage::B_CHUNKS / 64;
  constexpr int KPW = (NKI + NW - 1) / NW, BPW = (NBI + NW - 1) / NW;
  static_assert(Stage::K_CHUNKS % 64 == 0 && Stage::B_CHUNKS % 64 == 0, "whole instructions");
  static_assert(Stage::KP_CHUNKS <= 64, "keep flags of a block in one instruction");
  __shared__ Stage st[2];

  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int rg = w / QS, qs = w % QS;
  int bx, grp;
  xcd_group_map(blockIdx.x, nx, ny * a.heads, bx, grp);
  const int h = grp / ny;
  const int jp = a.jp, n = a.n;
  const int wg_row0 = (grp % ny) * R_WG;
  const int wg_q0 = bx * Q_WG;
  const int row0 = wg_row0 + rg * R;
  const int q0 = wg_q0 + qs * 16 * QB;
  const int bb = min(wg_row0, a.rows - 1) / a.rows_per_bias;
  const float* B = a.bias + ((size_t)bb * a.heads + h) * jp * jp;

  // ---- staging plan: raw buffers based at the workgroup's first row ----
  const int base_row = min(wg_row0, a.rows - 1);
  const size_t row_elems = (size_t)a.heads * jp * 32;
  const CT* kbase = a.k + (size_t)base_row * row_elems;
  const CT* vbase = a.v + (size_t)base_row * row_elems;
  const CT* kpbase = a.keep + (size_t)base_row * jp;
  const uint32_t kv_bytes = clamp_bytes((uint64_t)(a.rows - base_row) * row_elems * sizeof(CT));
  const uint32_t kp_bytes = clamp_bytes((uint64_t)(a.rows - base_row) * jp * sizeof(CT));
  const uint32_t b_bytes = clamp_bytes((uint64_t)jp * jp * sizeof(float));
  uint32_t ok[KPW], ov[KPW], ob[BPW], okp = 0;
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const int p = (wu + j * NW) * 64 + l;  // chunk position in the K (V) region
    const int rr = min(p / (32 * KCH), R_WG - 1), key = (p / KCH) % 32;
    const int ch = kswz(key, p % KCH, KCH);  // an involution: the source chunk
    const int lrow = min(wg_row0 + rr, a.rows - 1) - base_row;
    const size_t rh = (size_t)lrow * a.heads + h;
    ok[j] = (uint32_t)(((rh * jp + key) * 32 + ch * VEC) * sizeof(CT));
    ov[j] = (uint32_t)((rh * jp * 32 + (p % (32 * KCH)) * VEC) * sizeof(CT));
  }
#pragma unroll
  for (int j = 0; j < BPW; ++j) {
    const int p = (wu + j * NW) * 64 + l;
    const int qq = p >> 3, ch = (p & 7) ^ (qq & 7);
    const int qrow = min(min(wg_q0 + qq, n - 1), jp - 1);
    ob[j] = (uint32_t)(((size_t)qrow * jp + ch * 4) * sizeof(float));
  }
  if (l < Stage::KP_CHUNKS) {
    const int rr = l / KCH, ch = l % KCH;
    const int lrow = min(wg_row0 + rr, a.rows - 1) - base_row;
    okp = (uint32_t)(((size_t)lrow * jp + ch * VEC) * sizeof(CT));
  }
  // loads of key block t into stage buffer `buf`
  auto issue = [&](int t, int buf) {
    Stage& S = st[buf];
    const uint32_t skv = (uint32_t)t * 32 * 32 * sizeof(CT);
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
      const int i = wu + j * NW;
      // (always true when the instructions divide evenly over the waves:
      // then no branch is emitted)
      if (NKI % NW == 0 || i < NKI) {
        buffer_load_lds16(kbase, kv_bytes, S.k + i * 64, ok[j], skv);
        buffer_load_lds16(vbase, kv_bytes, S.v + i * 64, ov[j], skv);
      }
    }
#pragma unroll
    for (int j = 0; j < BPW; ++j) {
      const int i = wu + j * NW;
      if (NBI % NW == 0 || i < NBI)
        buffer_load_lds16(B, b_bytes, S.b + i * 64, ob[j], (uint32_t)t * 32 * sizeof(float));
    }
    if (wu == NW - 1 && l < Stage::KP_CHUNKS)
      buffer_load_lds16(kpbase, kp_bytes, S.kp, okp, (uint32_t)t * 32 * sizeof(CT));
  };

  // ---- per-wave state ----
  // (every flag is loaded, without short-circuit branches, so that no load
  // waits for another before the first key block is requested)
  int rr[R], rf[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rr[r] = min(row0 + r, a.rows - 1);
    rf[r] = a.rowflag[rr[r]];
  }
  // q fragments, then the first key block's staging, so that the two
  // latencies overlap; the overflow bound is checked while the stage lands
  Frag<CT> qf[R][QB];
  float bqv[QB], kmv[R];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int qq = min(q0 + 16 * qb + r16, jp - 1);
    bqv[qb] = fkey_inv(a.bmax[((size_t)bb * a.heads + h) * jp + min(qq, n - 1)]);
#pragma unroll
    for (int r = 0; r < R; ++r)
      qf[r][qb].load(a.q + (((size_t)rr[r] * a.heads + h) * jp + qq) * 32 + 8 * g);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) kmv[r] = __uint_as_float(a.kmax[(size_t)rr[r] * a.heads + h]);
  issue(0, 0);
  bool skip = true;
#pragma unroll
  for (int r = 0; r < R; ++r) skip &= (row0 + r >= a.rows) | (rf[r] != 0);
  bool over = false;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float q2 = 0.f;
      for (int e = 0; e < 8; ++e) q2 += qf[r][qb].get(e) * qf[r][qb].get(e);
      over = over || (sqrtf(group_sum_fast(q2)) * kmv[r] + bqv[qb] > kFastBound);
    }
  if (__any(over) && !skip) {
    if (l < R && row0 + l < a.rows) a.rowflag[row0 + l] = 1;
    skip = true;
  }
  // the same for every lane of the wave (its rows and their flags): made
  // provably uniform so that `if (!skip)` is a scalar branch, not an exec mask
  skip = __builtin_amdgcn_readfirstlane((int)skip) != 0;
  // three-part form: q as bf16 pairs, once
  Frag<bf16> qh[kX3 ? R : 1][QB], ql[kX3 ? R : 1][QB];
  if constexpr (kX3) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        if constexpr (sizeof(CT) == 4) split_x3(qf[r][qb], qh[r][qb], ql[r][qb]);
  }

  f32x4 o[R][2][QB];
  float lsum[R][QB];
  f32x4 lacc[kMfmaSum ? R : 1][QB];  // bf16: row sums on the MFMA
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      o[r][0][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
      o[r][1][qb] = o[r][0][qb];
      lsum[r][qb] = 0.f;
      if constexpr (kMfmaSum) lacc[r][qb] = o[r][0][qb];
    }

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  // Two key blocks per trip with the stage buffer a compile-time constant, so
  // every LDS fragment address is a lane base plus an immediate offset and
  // the direct loads' LDS destinations are constants (no per-block address
  // arithmetic); nblk is even because jp is a multiple of 64.
  const int nblk = jp >> 5;
  auto block = [&](auto buf_c, int t) {
    constexpr int kBuf = decltype(buf_c)::value;
    // buffer kBuf ^ 1 was last read in the previous block, which every wave
    // has left (barrier at its end)
    if (t + 1 < nblk) issue(t + 1, kBuf ^ 1);
    if (!skip) {
      const Stage& S = st[kBuf];
      const CT* Ks = reinterpret_cast<const CT*>(S.k);
      const CT* Vs = reinterpret_cast<const CT*>(S.v);
      const CT* KPs = reinterpret_cast<const CT*>(S.kp);
      const float* Bs = reinterpret_cast<const float*>(S.b);
      f32x4 bfr[2][QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int ql = qs * 16 * QB + 16 * qb + r16;  // query row within the tile
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          bfr[kb][qb] = *reinterpret_cast<const f32x4*>(Bs + (ql * 8 + ((4 * kb + g) ^ (ql & 7))) * 4);
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int lr = rg * R + r;  // row within the workgroup
        Frag<CT> kf[2], vf[2], kpf;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const int key = 16 * kb + r16;
          if constexpr (KCH == 4) {
            kf[kb].load(Ks + ((lr * 32 + key) * KCH + kswz(key, g, KCH)) * VEC);
          } else {
            kf[kb].load(Ks + (lr * 32 + key) * 32 + 8 * g);
          }
          vf[kb].load(Vs + ((size_t)lr * 1024 + (kb * 64 + l) * 8));
        }
        kpf.load(KPs + lr * 32 + 8 * g);
        f32x4 s[2][QB];
        // raised issue priority while this wave issues QK^T: with two waves
        // per SIMD, its MFMAs go ahead of the other wave's exponentials
        __builtin_amdgcn_s_setprio(1);
        if constexpr (kX3) {
          Frag<bf16> kh[2], kl[2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb) split_x3(kf[kb], kh[kb], kl[kb]);
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              s[kb][qb] = bfr[kb][qb];
              mma_x3(s[kb][qb], kh[kb], kl[kb], qh[r][qb], ql[r][qb]);
            }
        } else {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              s[kb][qb] = bfr[kb][qb];
              mma(s[kb][qb], kf[kb], qf[r][qb]);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        Frag<CT> pf[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) pf[qb].set(4 * kb + e, __builtin_amdgcn_exp2f(s[kb][qb][e]));
          if constexpr (!kMfmaSum) lsum[r][qb] = psum8(pf[qb], kpf, lsum[r][qb]);
        }
        if constexpr (kX3) {
          Frag<bf16> vh[2], vl[2];
#pragma unroll
          for (int db = 0; db < 2; ++db) split_x3(vf[db], vh[db], vl[db]);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) {
            Frag<bf16> ph, pl;
            split_x3(pf[qb], ph, pl);
#pragma unroll
            for (int db = 0; db < 2; ++db) mma_x3(o[r][db][qb], vh[db], vl[db], ph, pl);
          }
        } else {
#pragma unroll
          for (int db = 0; db < 2; ++db)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) mma(o[r][db][qb], vf[db], pf[qb]);
        }
        if constexpr (kMfmaSum) {
          // lane (g, r16) ends with the sum for query r16 in every slot
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) mma(lacc[r][qb], kpf, pf[qb]);
        }
      }
    }
    // this wave's loads of block t + 1 have landed; the barrier makes every
    // wave's visible and ends all reads of buffer kBuf
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  };
  for (int t = 0; t < nblk; t += 2) {
    block(std::integral_constant<int, 0>{}, t);
    block(std::integral_constant<int, 1>{}, t + 1);
  }
  if (skip) return;

  // A row whose sum underflows (or that keeps no key) goes to the exact core;
  // flagged one row at a time, as the exact core recomputes whole rows.
  float inv[R][QB];
  int under = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    bool ur = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      float lt;
      if constexpr (kMfmaSum) lt = lacc[r][qb][0];
      else lt = group_sum_fast(lsum[r][qb]);
      ur = ur || !(lt >= kUnderflowSum);
      inv[r][qb] = __builtin_amdgcn_rcpf(lt);  // lt >= kUnderflowSum here, else flagged
    }
    if (__any(ur)) under |= 1 << r;
  }
  if (under && l < R && row0 + l < a.rows && ((under >> l) & 1)) a.rowflag[row0 + l] = 1;
  if (q0 >= jp) return;
  core_store<CT, R, QB>(a, row0, h, q0, o, inv);
}

// Exact online softmax (running max, additive mask as in the reference), run
// for the rows the fast core flagged; every other wave exits at once.
template <typename CT, int R, int QB>
__global__ __launch_bounds__(256) void triatt_core_exact_kernel(TriattCoreArgs<CT> a) {
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int row0 = (blockIdx.y * 4 + w) * R;
  if (row0 >= a.rows) return;
  int rr[R];
  bool any_flagged = false;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    rr[r] = __builtin_amdgcn_readfirstlane(min(row0 + r, a.rows - 1));
    any_flagged = any_flagged || (row0 + r < a.rows && a.rowflag[rr[r]] != 0);
  }
  if (!any_flagged) return;
  const int h = blockIdx.z;
  const int jp = a.jp, n = a.n;
  const float* B = a.bias + ((size_t)(row0 / a.rows_per_bias) * a.heads + h) * jp * jp;

  // Rows that keep no key: every logit carries the same -inf*log2e term, which
  // absorbs q.k + bias in f32, so the softmax is uniform over the n keys and
  // the output is mean_k v (the reference's f32 result for such rows),
  // computed once and written to every query.
  bool all_masked = true;
#pragma unroll
  for (int r = 0; r < R; ++r)
    all_masked = all_masked && (row0 + r >= a.rows || a.anykeep[rr[r]] == 0);
  if (all_masked) {
    f32x4 o[R][2][QB];
    float inv[R][QB];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const CT* Vr = a.v + ((size_t)rr[r] * a.heads + h) * jp * 32;
      float sum[2] = {0.f, 0.f};
      // eight key blocks' loads in flight at a time (walking the blocks one
      // by one costs one load latency each); keys >= n are selected out
      for (int k0 = 0; k0 < jp; k0 += 8 * 32) {
        Frag<CT> vf[8][2];  // lane: channel half db, row r16; keys k0 + 32u + slot_key(g, e)
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (k0 + 32 * u < jp)
#pragma unroll
            for (int db = 0; db < 2; ++db)
              vf[u][db].load(Vr + (size_t)((k0 >> 5) + u) * 1024 + (db * 64 + l) * 8);
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (k0 + 32 * u < jp)
#pragma unroll
            for (int db = 0; db < 2; ++db)
#pragma unroll
              for (int e = 0; e < 8; ++e)
                sum[db] += k0 + 32 * u + slot_key(g, e) < n ? vf[u][db].get(e) : 0.f;
      }
#pragma unroll
      for (int db = 0; db < 2; ++db) {
        sum[db] = group_sum_fast(sum[db]);  // every lane with this r16: channel 16*db + r16
      }
      // accumulator layout: lane (g, r16) holds channels 16*db + 4g + e of query r16
#pragma unroll
      for (int db = 0; db < 2; ++db)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float t = __shfl(sum[db], 4 * g + e, 64);
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) o[r][db][qb][e] = t;
        }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) inv[r][qb] = 1.0f / (float)n;
    }
    for (int q0 = blockIdx.x * (16 * QB); q0 < jp; q0 += gridDim.x * (16 * QB))
      core_store<CT, R, QB>(a, row0, h, q0, o, inv);
    return;
  }

  // query blocks of the row, gridDim.x apart
  for (int q0 = blockIdx.x * (16 * QB); q0 < jp; q0 += gridDim.x * (16 * QB)) {

    const CT* Qp[R];
    const CT* Kp[R];
    const CT* Vp[R];
    const float* MBp[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const size_t rh = (size_t)rr[r] * a.heads + h;
      Qp[r] = a.q + rh * jp * 32;
      Kp[r] = a.k + rh * jp * 32;
      Vp[r] = a.v + rh * jp * 32;
      MBp[r] = a.mb + (size_t)rr[r] * jp;
    }
    Frag<CT> qf[R][QB];
    const float* brow[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int qq = q0 + 16 * qb + r16;
      brow[qb] = B + (size_t)min(qq, n - 1) * jp + 4 * g;
#pragma unroll
      for (int r = 0; r < R; ++r) qf[r][qb].load(Qp[r] + (size_t)qq * 32 + 8 * g);
    }
    const Frag<CT> ones = ones_frag(CT());

    f32x4 o[R][2][QB];
    float m[R][QB], lsum[R][QB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        o[r][0][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
        o[r][1][qb] = o[r][0][qb];
        m[r][qb] = -1e30f;
        lsum[r][qb] = 0.f;
      }

    for (int k0 = 0; k0 < jp; k0 += 32) {
      f32x4 bfr[2][QB];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          bfr[kb][qb] = *reinterpret_cast<const f32x4*>(brow[qb] + k0 + 16 * kb);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        Frag<CT> kf[2], vf[2];
        f32x4 mbv[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          kf[kb].load(Kp[r] + (size_t)(k0 + 16 * kb + r16) * 32 + 8 * g);
          vf[kb].load(Vp[r] + (size_t)(k0 >> 5) * 1024 + (kb * 64 + l) * 8);
          mbv[kb] = *reinterpret_cast<const f32x4*>(MBp[r] + k0 + 16 * kb + 4 * g);
        }
        f32x4 s[2][QB];
        if (a.mflag[(size_t)rr[r] * (jp >> 5) + (k0 >> 5)]) {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              s[kb][qb] = bfr[kb][qb] + mbv[kb];
              mma(s[kb][qb], kf[kb], qf[r][qb]);
            }
        } else {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
              s[kb][qb] = bfr[kb][qb];
              mma(s[kb][qb], kf[kb], qf[r][qb]);
            }
        }
        Frag<CT> pf[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          float mx = fmaxf(fmaxf(fmaxf(s[0][qb][0], s[0][qb][1]), fmaxf(s[0][qb][2], s[0][qb][3])),
                           fmaxf(fmaxf(s[1][qb][0], s[1][qb][1]), fmaxf(s[1][qb][2], s[1][qb][3])));
          mx = group_max_fast(mx);
          if (__any(mx > m[r][qb])) {
            const float mnew = fmaxf(m[r][qb], mx);
            const float sc = __builtin_amdgcn_exp2f(m[r][qb] - mnew);
            m[r][qb] = mnew;
            lsum[r][qb] *= sc;
            o[r][0][qb] *= sc;
            o[r][1][qb] *= sc;
          }
          const float mm = m[r][qb];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e) pf[qb].set(4 * kb + e, __builtin_amdgcn_exp2f(s[kb][qb][e] - mm));
          lsum[r][qb] = psum8(pf[qb], ones, lsum[r][qb]);
        }
#pragma unroll
        for (int db = 0; db < 2; ++db)
#pragma unroll
          for (int qb = 0; qb < QB; ++qb) mma(o[r][db][qb], vf[db], pf[qb]);
      }
    }
    float inv[R][QB];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) inv[r][qb] = 1.0f / group_sum_fast(lsum[r][qb]);
    core_store<CT, R, QB>(a, row0, h, q0, o, inv);
  }
}

// ---------------------------------------------------------------------------
// 3. output projection + residual
// ---------------------------------------------------------------------------
template <typename ZT, typename CT>
struct TriattOutArgs {
  const CT* o;  // [I][Jp][HD]
  const CT* wo; // [C][HD]
  const ZT* res;  // z: the residual, and the gate's input where the gate is fused here
  int64_t r_s0, r_s1;
  ZT* out;
  int64_t o_s0, o_s1;
  int n, jp, c;
  int add;
  // gate fused into the output kernel (weight-stationary path)
  const CT* wg;  // [HD][C]
  const float* ln_w;
  const float* ln_b;
  float eps;
};

// kRB consecutive rows i per workgroup: every weight fragment a wave reads
// from L2 serves kRB row blocks (the fp32 form reads W_o per fragment).
// blockIdx.z of gridDim.z takes output channels [z C / Z, (z + 1) C / Z)
// (small grids).  kStage (f32 data): W_o rows of each 16-channel block
// (fp32 rows, or the three-part split rows: the same bytes) staged in LDS,
// double-buffered, shared by the workgroup's 4 waves.
template <typename ZT, typename CT, int kHD, bool kX3Mul = false, int kRB = 1, bool kStage = false>
__global__ __launch_bounds__(256) void triatt_out_kernel(TriattOutArgs<ZT, CT> a) {
  constexpr int HD = kHD * 32;
  using MF = MulFrag<CT, kX3Mul>;
  static_assert(!kStage || sizeof(CT) == 4, "staging: f32 weights");
  constexpr int WL = HD + 4;                    // staged row stride (floats)
  constexpr int CHUNK = 16 * WL;
  constexpr int PT = 16 * HD / 4;               // 16-byte pieces per chunk
  constexpr int PPT = (PT + 255) / 256;
  __shared__ __attribute__((aligned(16))) float wsm[kStage ? 2 * CHUNK : 4];
  const int i0 = blockIdx.y * kRB;
  const int w = wave_id(), g = lane_id() >> 4, r16 = lane_id() & 15;
  const int jl = blockIdx.x * 64 + w * 16 + r16;
  MF x[kRB][kHD];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
    const bool valid = i0 + rb < a.n && jl < a.n;
    const CT* orow = a.o + ((size_t)(valid ? i0 + rb : 0) * a.jp + jl) * HD;
#pragma unroll
    for (int t = 0; t < kHD; ++t) {
      if (valid) x[rb][t].load(orow + 32 * t + 8 * g);
      else x[rb][t].zero();
    }
  }
  const int cb_per = (a.c / 16) / (int)gridDim.z;
  const int cb_lo = (int)blockIdx.z * cb_per, cb_hi = cb_lo + cb_per;
  f32x4 wreg[kStage ? PPT : 1];
  auto wload = [&](int cb) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k, r = q / (HD / 4), c4 = q % (HD / 4);
      if (PT % 256 == 0 || q < PT)
        wreg[k] = *reinterpret_cast<const f32x4*>(a.wo + (size_t)(cb * 16 + r) * HD + 4 * c4);
    }
  };
  auto wstore = [&](int buf) {
#pragma unroll
    for (int k = 0; k < PPT; ++k) {
      const int q = (int)threadIdx.x + 256 * k, r = q / (HD / 4), c4 = q % (HD / 4);
      if (PT % 256 == 0 || q < PT)
        *reinterpret_cast<f32x4*>(&wsm[buf * CHUNK + r * WL + 4 * c4]) = wreg[k];
    }
  };
  if constexpr (kStage) {
    wload(cb_lo);
    wstore(0);
    if (cb_lo + 1 < cb_hi) wload(cb_lo + 1);
    __syncthreads();
  }
  for (int cb = cb_lo; cb < cb_hi; ++cb) {
    f32x4 acc[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) acc[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float* wrow = wsm + ((cb - cb_lo) & 1) * CHUNK + (lane_id() & 15) * WL;
#pragma unroll
    for (int t = 0; t < kHD; ++t) {
      MF f;
      if constexpr (kStage) staged_w_frag(wrow, HD, t, f);
      else load_w_frag(a.wo, HD, cb * 16, a.c, t, f);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) mma(acc[rb], f, x[rb][t]);
    }
    const int c0 = cb * 16 + 4 * g;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int i = i0 + rb;
      if (i >= a.n || jl >= a.n) continue;
      float base[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.add) load4(a.res + (int64_t)i * a.r_s0 + (int64_t)jl * a.r_s1 + c0, base);
      store4(a.out + (int64_t)i * a.o_s0 + (int64_t)jl * a.o_s1 + c0, base[0] + acc[rb][0],
             base[1] + acc[rb][1], base[2] + acc[rb][2], base[3] + acc[rb][3]);
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

// Weight-stationary output projection with the gate fused in.  Per 64-row
// tile (i, j0..j0+63) the z rows stream into LDS (direct loads, one tile
// ahead) and are LayerNorm'd there; wave w computes gate channels
// [w*HD/4, (w+1)*HD/4) of g = sigmoid(LN(z) W_g^T) with its W_g rows held in
// registers and scales its columns of the o tile (staged in LDS) by them;
// then wave w projects output channels [w*C/4, (w+1)*C/4) of the gated tile
// with its W_o rows held in registers and adds the residual, read from the
// staged z rows.  Gating here rather than in the flash core saves the gate
// tensor's write and read in HBM.
template <typename ZT, typename CT, int kHD, int kC>
__global__ __launch_bounds__(256, 2) void triatt_out_ws_kernel(TriattOutArgs<ZT, CT> a, int ntiles) {
  constexpr int HD = kHD * 32, C = kC * 32, NBO = C / 64, NBG = HD / 64, RB = kTileRows / 16;
  constexpr int LD = TileLD<CT, HD>::value;
  constexpr int VEC = 16 / sizeof(CT), PER_ROW = HD / VEC;
  constexpr int OCH = kTileRows * PER_ROW / 256;  // 16-byte chunks of o per thread
  constexpr int EPC = 16 / (int)sizeof(ZT);       // z elements per 16-byte chunk
  using Raw = RawTile<ZT, C>;
  static_assert(kTileRows * PER_ROW % 256 == 0, "o tile chunks");
  static_assert(sizeof(CT) == 2, "gate scaling in LDS takes 4 x 16-bit o values");
  __shared__ __attribute__((aligned(16))) CT xo[kTileRows * LD];
  // the gate multiplies in fp16 (LN(z) rounded to fp16, 11 significant bits;
  // the bf16 weights carry -log2(e) in fp16, so the gate's accumulator feeds
  // exp2 directly)
  __shared__ __attribute__((aligned(16))) f16 xs[kTileRows * TileLD<f16, C>::value];
  __shared__ __attribute__((aligned(16))) unsigned char raw[Raw::BYTES];
  __shared__ float lnp[2 * C];  // LayerNorm weight, bias
  const int w = wave_id(), g = lane_id() >> 4, r16 = lane_id() & 15;
  for (int t = threadIdx.x; t < C; t += 256) {
    lnp[t] = a.ln_w[t];
    lnp[C + t] = a.ln_b[t];
  }
  Frag<CT> wof[NBO][kHD];
  load_w_slice(a.wo, HD, w * (C / 4), C, wof);
  Frag<f16> wgf[NBG][kC];
  load_w_slice_scaled(a.wg, C, w * (HD / 4), HD, kNegLog2e, wgf);
  const int jp = a.jp, n = a.n, tiles_per_row = jp / kTileRows;

  // The next tile's z rows (into LDS) and o rows (into registers) are loaded
  // while the current tile is computed; rows past n read row n-1 (always
  // present), are LayerNorm'd as zeros and never stored.
  f32x4 opre[OCH];
  auto fetch = [&](int tl) {
    const int ti = tl / tiles_per_row, tj0 = (tl % tiles_per_row) * kTileRows;
    raw_tile_issue<ZT, C, kStream>(a.res + (int64_t)ti * a.r_s0, a.r_s1, tj0, n, raw);
    const CT* src = a.o + ((size_t)ti * jp + tj0) * HD;
#pragma unroll
    for (int k = 0; k < OCH; ++k) {
      const int ci = threadIdx.x + k * 256, r = ci / PER_ROW, cc = (ci % PER_ROW) * VEC;
      opre[k] = load_stream(reinterpret_cast<const f32x4*>(src + (size_t)r * HD + cc));
    }
  };
  if ((int)blockIdx.x < ntiles) fetch(blockIdx.x);
  for (int tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int i = tile / tiles_per_row;
    const int j0 = (tile % tiles_per_row) * kTileRows;
    raw_tile_wait();  // also: every wave is done with the previous tile's xs and xo
#pragma unroll
    for (int k = 0; k < OCH; ++k) {
      const int ci = threadIdx.x + k * 256, r = ci / PER_ROW, cc = (ci % PER_ROW) * VEC;
      *reinterpret_cast<f32x4*>(xo + r * LD + cc) = opre[k];
    }
    raw_tile_ln<ZT, f16, C>(raw, [&](int r) { return j0 + r < n; }, lnp, lnp + C, a.eps, xs);
    // this lane's residual values: rows rb*16 + r16, channels c0..c0+3
    float res[RB][NBO][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int r = rb * 16 + r16;
#pragma unroll
      for (int cb = 0; cb < NBO; ++cb) {
        const int c0 = w * (C / 4) + cb * 16 + 4 * g;
        const ZT* p = reinterpret_cast<const ZT*>(raw + r * Raw::ROW_BYTES +
                                                  (((c0 / EPC) ^ (r & 7)) * 16)) + c0 % EPC;
#pragma unroll
        for (int e = 0; e < 4; ++e) res[rb][cb][e] = a.add ? to_f32(p[e]) : 0.f;
      }
    }
    lds_barrier();  // xs and xo ready; raw consumed
    if (tile + (int)gridDim.x < ntiles) fetch(tile + gridDim.x);
    // gate: lane holds row rb*16 + r16, gate channels o..o+3 of its slice
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      Frag<f16> xf[kC];
      tile_frags<f16, C>(xs, rb, xf);
#pragma unroll
      for (int gb = 0; gb < NBG; ++gb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < kC; ++t) mma(acc, wgf[gb][t], xf[t]);
        const int o = w * (HD / 4) + gb * 16 + 4 * g;
        bf16x4* p = reinterpret_cast<bf16x4*>(xo + (rb * 16 + r16) * LD + o);
        bf16x4 ov = *p;
#pragma unroll
        for (int e = 0; e < 4; ++e) ov[e] = (bf16)((float)ov[e] * sigmoid_nl2e(acc[e]));
        *p = ov;
      }
    }
    lds_barrier();  // the gated o tile is complete
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      Frag<CT> xf[kHD];
      tile_frags<CT, HD>(xo, rb, xf);
      const int jr = j0 + rb * 16 + r16;
      float r[NBO][4];
#pragma unroll
      for (int cb = 0; cb < NBO; ++cb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < kHD; ++t) mma(acc, wof[cb][t], xf[t]);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[cb][e] = res[rb][cb][e] + acc[e];
      }
      ZT* orow = a.out + (int64_t)i * a.o_s0;
      store_row_blocks<ZT>(orow + (int64_t)jr * a.o_s1, orow + (int64_t)(jr ^ 1) * a.o_s1,
                           w * (C / 4), r, jr < n, (jr ^ 1) < n);
    }
    // xs and xo are rewritten only after the barrier in raw_tile_wait()
  }
}

// ---------------------------------------------------------------------------
// 4. core-only slot: strided q/k/v/bias/mask -> core layouts
// ---------------------------------------------------------------------------
template <typename CT>
struct RelayoutArgs {
  const CT* q; int64_t q_sb, q_si, q_sh, q_sj;
  const CT* k; int64_t k_sb, k_si, k_sh, k_sj;
  const CT* v; int64_t v_sb, v_si, v_sh, v_sj;
  const float* bias; int64_t b_sb, b_sh, b_sq, b_sk;
  const uint8_t* mask; int64_t m_sb, m_si, m_sk;
  CT* wq; CT* wk; CT* wv; CT* wkeep; float* wbias; float* wmb;
  int* anykeep; int* rowflag; unsigned* kmax; int* bmax;
  int batch, rows, heads, n, jp;
  float q_scale, mask_inf;
};

// One workgroup per flattened row r = b*I + i: keep test and initialisation.
template <typename CT>
__global__ __launch_bounds__(256) void triatt_slot_prep_kernel(RelayoutArgs<CT> a) {
  const int r = blockIdx.x;
  const int b = r / a.rows, i = r % a.rows;
  int keep = 0;
  for (int k = threadIdx.x; k < a.n; k += 256)
    keep |= a.mask ? a.mask[b * a.m_sb + i * a.m_si + (int64_t)k * a.m_sk] != 0 : 1;
  keep = __syncthreads_or(keep);
  if (threadIdx.x == 0) {
    a.anykeep[r] = keep;
    a.rowflag[r] = !keep;
  }
  if (threadIdx.x < a.heads) a.kmax[r * a.heads + threadIdx.x] = 0u;
}

// One thread per (row r, head h, key j): 32 channels of q, k, v; max |k| per
// (row, head) via one atomic per wave (a wave holds 64 keys of one (r, h));
// threads with h == 0 also write the mask row and keep flags.
template <typename CT>
__global__ __launch_bounds__(256) void triatt_relayout_kernel(RelayoutArgs<CT> a) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.batch * a.rows * a.heads * a.jp;
  if (tid >= total) return;  // jp % 64 == 0: whole waves exit together
  const int j = (int)(tid % a.jp);
  const int h = (int)((tid / a.jp) % a.heads);
  const int64_t r = tid / ((int64_t)a.jp * a.heads);
  const int b = (int)(r / a.rows), i = (int)(r % a.rows);
  const bool valid = j < a.n;
  const bool keep = valid && (a.mask ? a.mask[b * a.m_sb + i * a.m_si + (int64_t)j * a.m_sk] != 0 : true);
  const float vmul = (a.anykeep[r] && !keep) ? 0.f : 1.f;
  const size_t off = (((size_t)r * a.heads + h) * a.jp + j) * 32;
  const CT* qs = a.q + b * a.q_sb + i * a.q_si + h * a.q_sh + (int64_t)(valid ? j : 0) * a.q_sj;
  const CT* ks = a.k + b * a.k_sb + i * a.k_si + h * a.k_sh + (int64_t)(valid ? j : 0) * a.k_sj;
  const CT* vs = a.v + b * a.v_sb + i * a.v_si + h * a.v_sh + (int64_t)(valid ? j : 0) * a.v_sj;
  float k2 = 0.f;
  for (int d = 0; d < 32; ++d) {
    const float qv = valid ? to_f32(qs[d]) * a.q_scale : 0.f;
    const float kv = valid ? to_f32(ks[d]) : 0.f;
    const float vv = valid ? to_f32(vs[d]) * vmul : 0.f;
    k2 += kv * kv;
    a.wq[off + d] = from_f32<CT>(qv);
    a.wk[off + d] = from_f32<CT>(kv);
    a.wv[vperm_offset((int)r, h, a.heads, a.jp, j, d)] = from_f32<CT>(vv);
  }
  const float km = wave_max(sqrtf(k2));
  if (lane_id() == 0) atomicMax(&a.kmax[r * a.heads + h], __float_as_uint(km));
  if (h == 0) {
    a.wmb[(size_t)r * a.jp + j] = valid ? (keep ? 0.f : -a.mask_inf) : -INFINITY;
    a.wkeep[(size_t)r * a.jp + (j & ~31) + key_slot(j & 31)] = from_f32<CT>(keep ? 1.f : 0.f);
  }
}

// One thread per (bias batch b, head h, query q, key k): bias * log2(e) into
// [B][H][Jp][Jp], zero outside the n x n block.
template <typename CT>
__global__ __launch_bounds__(256) void triatt_bias_relayout_kernel(RelayoutArgs<CT> a) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.batch * a.heads * a.jp * a.jp;
  if (tid >= total) return;
  const int k = (int)(tid % a.jp);
  const int q = (int)((tid / a.jp) % a.jp);
  const int64_t bh = tid / ((int64_t)a.jp * a.jp);
  const int h = (int)(bh % a.heads), b = (int)(bh / a.heads);
  float bv = 0.f;
  if (q < a.n && k < a.n)
    bv = a.bias[b * a.b_sb + h * a.b_sh + (int64_t)q * a.b_sq + (int64_t)k * a.b_sk] * kLog2e;
  a.wbias[tid] = bv;
}

// Max of each relaid bias row over its n keys (one thread per (b, h, q)).
__global__ __launch_bounds__(256) void triatt_bmax_fold_kernel(const float* wbias, int* bmax,
                                                               int bh_count, int n, int jp) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= (int64_t)bh_count * jp) return;
  const int q = (int)(tid % jp);
  const float* row = wbias + tid * jp;
  float m = -INFINITY;
  if (q < n)
    for (int k = 0; k < n; ++k) m = fmaxf(m, row[k]);
  bmax[tid] = fkey(m);
}

// One thread per (row, 32-key block): flag blocks whose additive mask row has
// any nonzero entry (masked or padded keys).
__global__ __launch_bounds__(256) void triatt_mflag_kernel(const float* mb, int* mflag, int rows,
                                                           int jp) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int nb = jp >> 5;
  if (tid >= (int64_t)rows * nb) return;
  const float* p = mb + (tid / nb) * jp + (tid % nb) * 32;
  int any = 0;
  for (int e = 0; e < 32; ++e) any |= p[e] != 0.f;
  mflag[tid] = any;
}

// ---------------------------------------------------------------------------
// 5. wide channels (bf16; C or H*32 of 256 and more): a LayerNorm pass into
//    bf16 rows (lnpass.hpp), then NT GEMMs on the shared mainloop
//    (gemm.hpp).  Rows are the pairs m = i * Jp + j, padded to a multiple of
//    2048 (rows past n * Jp are never stored).
// ---------------------------------------------------------------------------
constexpr int kWTX = 256, kWTY = 128, kWWX = 4, kWNS = 3, kWKC = 32;
using WideShape = GemmShape<kWTX, kWTY, kWWX, kWKC>;

__device__ __forceinline__ void wide_tile_map(int L, int ncol, int& rt, int& ct) {
  const int xcd = L & 7, s = L >> 3;  // all column tiles of a row tile on one XCD
  rt = xcd + 8 * (s / ncol);
  ct = s % ncol;
}

// Mask outputs (mb, mflag, keep) and the triangle bias of 64 pairs (i, j0..)
// from the normalised rows, as in the register projection kernel: a
// workgroup of 4 waves, 16 pairs per wave.
template <typename ZT, int kC>
__global__ __launch_bounds__(256) void triatt_bias_mask_wide_kernel(TriattProjArgs<ZT, bf16> a,
                                                                    const bf16* zn) {
  constexpr int C = kC * 32;
  const int i = blockIdx.y;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int H = a.heads, jp = a.jp;
  const int j0 = blockIdx.x * 64 + w * 16;
  const int jl = j0 + r16;
  const bool valid = jl < a.n;
  Frag<bf16> x[kC];
  const bf16* row = zn + ((size_t)i * jp + jl) * C + 8 * g;
#pragma unroll
  for (int t = 0; t < kC; ++t) x[t].load(row + 32 * t);

  __shared__ float keep_s[64];
  __shared__ int wmasked[4];
  float mv = -INFINITY, kp = 0.f;
  if (valid) {
    const float m = a.mask ? a.mask[(int64_t)i * a.m_s0 + (int64_t)jl * a.m_s1] : 1.0f;
    mv = (m - 1.0f) * a.mask_inf;
    kp = m == 1.0f ? 1.f : 0.f;
  }
  if (g == 0) {
    a.mb[(size_t)i * jp + jl] = mv;
    keep_s[w * 16 + r16] = kp;
  }
  const bool any_masked = __any(mv != 0.f);
  if (l == 0) wmasked[w] = any_masked ? 1 : 0;
  __syncthreads();
  if (threadIdx.x < 2) {
    const int b = threadIdx.x;  // 32-key block b of this 64-key tile = waves 2b, 2b+1
    a.mflag[(size_t)i * (jp >> 5) + blockIdx.x * 2 + b] = wmasked[2 * b] | wmasked[2 * b + 1];
  }
  if (threadIdx.x < 64) {
    const int t = threadIdx.x, kb = t >> 5, s = t & 31;
    a.keep[((size_t)i * (jp >> 5) + blockIdx.x * 2 + kb) * 32 + s] =
        (bf16)keep_s[kb * 32 + slot_key(s >> 3, s & 7)];
  }
  // triangle bias: channel h = r16 (< H), rows j0+4g .. +3 -> bias[h][i][..]
  f32x4 ab = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    Frag<bf16> f;
    load_w_frag(a.wb, C, 0, H, t, f);
    mma(ab, x[t], f);
  }
  const float sc = kLog2e;
  const int jb = j0 + 4 * g;
  const float bm = group_max_fast(fmaxf(fmaxf(ab[0], ab[1]), fmaxf(ab[2], ab[3])) * sc);
  if (r16 < H) {
    store4(a.bias + ((size_t)r16 * jp + i) * jp + jb, ab[0] * sc, ab[1] * sc, ab[2] * sc,
           ab[3] * sc);
    if (g == 0) atomicMax(&a.bmax[r16 * jp + i], fkey(bm));
  }
}

// q, k, v, gate as one NT GEMM of the normalised rows with the weight rows
// [W_q | W_k | W_v | W_g] (H*32 each, a multiple of the 128-row column tile,
// so a tile is one of the four).  q, k, gate: one pair and four consecutive
// channels per lane (8-byte stores into [I][H][Jp][32]); v: one channel and
// four consecutive pairs per lane (8-byte stores into the fragment-ordered
// V layout), zeroed on masked keys of rows that keep a key.  k also yields
// the per-(row, head) maximum key norm for the fast core's bound.
template <typename ZT>
__global__ __launch_bounds__(512) void triatt_qkvg_wide_kernel(TriattProjArgs<ZT, bf16> a,
                                                               const bf16* zn, int C, int ncol) {
  __shared__ __attribute__((aligned(16))) bf16 sm[kWNS * WideShape::STAGE_ELEMS];
  int rt, ct;
  wide_tile_map(blockIdx.x, ncol, rt, ct);
  const int H = a.heads, HD = H * 32, jp = a.jp, n = a.n;
  const int64_t x0 = (int64_t)rt * kWTX;
  const int per = HD / kWTY, type = ct / per, o0 = (ct % per) * kWTY;
  const bf16* W = type == 0 ? a.wq : type == 1 ? a.wk : type == 2 ? a.wv : a.wg;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kWWX, wy = w / kWWX;
  auto arow = [&](int r) { return zn + (x0 + r) * C; };
  auto brow = [&](int r) { return W + (size_t)(o0 + r) * C; };
  // q, k, gate: within each 32 weight rows (one head), row block 2p + b, MFMA
  // row m is channel 8 (m >> 2) + 4 b + (m & 3), so a lane's results of the
  // head's two row blocks are 8 consecutive channels (one 16-byte store)
  auto brow_perm = [&](int r) {
    const int m = r & 15;
    return W + (size_t)(o0 + (r & ~31) + 8 * (m >> 2) + 4 * ((r >> 4) & 1) + (m & 3)) * C;
  };
  f32x4 acc[WideShape::MX][WideShape::MY];
  static_assert(WideShape::MX % 2 == 0 && WideShape::MY % 2 == 0, "row blocks pair up");
  if (type == 2) {  // v: channel-per-lane orientation
    gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, false, kWKC>(arow, brow, C, sm, acc);
    // row blocks i and i + 1 hold keys 4g..4g+3 and the same keys + 16 of a
    // 32-key block: one 16-byte slot group of the V layout
#pragma unroll
    for (int i = 0; i < WideShape::MX; i += 2) {
      const int64_t m = x0 + wx * (kWTX / kWWX) + 16 * i + 4 * g;  // pairs m .. m+3, m+16 ..
      const int row = (int)(m / jp), jj = (int)(m % jp);
      if (row >= n) continue;
      float vk[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
      if (a.anykeep[row] != 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int key = jj + (e & 3) + 16 * (e >> 2);
          const float mv = key < n ? (a.mask ? a.mask[(int64_t)row * a.m_s0 +
                                                      (int64_t)key * a.m_s1]
                                             : 1.0f)
                                   : 0.f;
          vk[e] = mv == 1.0f ? 1.f : 0.f;
        }
      }
#pragma unroll
      for (int j = 0; j < WideShape::MY; ++j) {
        const int o = o0 + wy * (kWTY / WideShape::WY) + 16 * j + r16;
        bf16x8 v8;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v8[e] = (bf16)(acc[i][j][e] * vk[e]);
          v8[4 + e] = (bf16)(acc[i + 1][j][e] * vk[4 + e]);
        }
        *reinterpret_cast<bf16x8*>(a.v + vperm_offset(row, o >> 5, H, jp, jj, o & 31)) = v8;
      }
    }
    return;
  }
  gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, true, kWKC>(arow, brow_perm, C, sm, acc);
  // the wave's 64 pairs lie in one row (Jp and the offsets are multiples of 64)
  const int64_t mw = x0 + wx * (kWTX / kWWX);
  const int row = (int)(mw / jp);
  if (row >= n) return;
  const int ob = o0 + wy * (kWTY / WideShape::WY);  // the wave's 64 channels = heads ob/32, +1
  float knm[2] = {0.f, 0.f};
#pragma unroll
  for (int i = 0; i < WideShape::MX; ++i) {
    const int jj = (int)((mw + 16 * i + r16) % jp);
    float ss[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < WideShape::MY; j += 2) {
      const int o = ob + 16 * j + 8 * g;  // 8 channels: block j gives o..o+3, j + 1 o+4..o+7
      const size_t off = (((size_t)row * H + (o >> 5)) * jp + jj) * 32 + (o & 31);
      float v[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = acc[i][j][e];
        v[4 + e] = acc[i][j + 1][e];
      }
      bf16x8 v8;
      if (type == 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v8[e] = (bf16)(v[e] * a.q_scale);
        store_stream(reinterpret_cast<bf16x8*>(a.q + off), v8);
      } else if (type == 1) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          v8[e] = (bf16)v[e];
          ss[j >> 1] += v[e] * v[e];
        }
        store_stream(reinterpret_cast<bf16x8*>(a.k + off), v8);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v8[e] = (bf16)sigmoidf_(v[e]);
        store_stream(reinterpret_cast<bf16x8*>(a.gate + off), v8);
      }
    }
    if (type == 1) {
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) knm[hh] = fmaxf(knm[hh], sqrtf(group_sum_fast(ss[hh])));
    }
  }
  if (type == 1) {
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const float v = lanes16_max(knm[hh]);
      if (l == 0) atomicMax(&a.kmax[row * H + (ob >> 5) + hh], __float_as_uint(v));
    }
  }
}

// out[i][j][c] = (add ? res : 0) + o W_o^T: NT GEMM of the gated attention
// rows o [I*Jp][H*32] with W_o [C][H*32]; one pair and four consecutive
// channels per lane.
template <typename ZT>
__global__ __launch_bounds__(512) void triatt_out_wide_kernel(TriattOutArgs<ZT, bf16> a, int HD,
                                                              int ncol) {
  __shared__ __attribute__((aligned(16))) bf16 sm[kWNS * WideShape::STAGE_ELEMS];
  int rt, ct;
  wide_tile_map(blockIdx.x, ncol, rt, ct);
  const int64_t x0 = (int64_t)rt * kWTX;
  const int y0 = ct * kWTY;
  f32x4 acc[WideShape::MX][WideShape::MY];
  gemm_nt_mainloop<kWTX, kWTY, kWWX, kWNS, true, kWKC>(
      [&](int r) { return a.o + (x0 + r) * HD; },
      [&](int r) { return a.wo + (size_t)(y0 + r) * HD; }, HD, sm, acc);
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kWWX, wy = w / kWWX;
#pragma unroll
  for (int i = 0; i < WideShape::MX; ++i) {
    const int64_t m = x0 + wx * (kWTX / kWWX) + 16 * i + r16;
    const int row = (int)(m / a.jp), jj = (int)(m % a.jp);  // jp is even: lane r16 ^ 1 has jj ^ 1
    const bool ok = row < a.n && jj < a.n, pok = row < a.n && (jj ^ 1) < a.n;
    float r[WideShape::MY][4];
#pragma unroll
    for (int j = 0; j < WideShape::MY; ++j) {
      const int c0 = y0 + wy * (kWTY / WideShape::WY) + 16 * j + 4 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) r[j][e] = 0.f;
      if (a.add && ok) load4(a.res + (int64_t)row * a.r_s0 + (int64_t)jj * a.r_s1 + c0, r[j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) r[j][e] += acc[i][j][e];
    }
    ZT* orow = a.out + (int64_t)row * a.o_s0;
    store_row_blocks<ZT>(orow + (int64_t)jj * a.o_s1, orow + (int64_t)(jj ^ 1) * a.o_s1,
                         y0 + wy * (kWTY / WideShape::WY), r, ok, pok);
  }
}

}  // namespace odde

// ===========================================================================
// host side
// ===========================================================================
using namespace odde;

namespace {

struct CoreBufs {
  void* q; void* k; void* v; void* keep; float* bias; float* mb; int* mflag;
  unsigned* kmax; int* bmax; int* rowflag; int* anykeep;
};

// Workspace common to both entry points; `bias_batches` bias planes.
void carve_core_bufs(Carver& c, CoreBufs& w, int rows, int heads, int jp, int bias_batches,
                     int dt) {
  const uint64_t es = dtype_size(dt);
  const uint64_t per = (uint64_t)rows * heads * jp * 32;
  w.q = c.take<char>(per * es);
  w.k = c.take<char>(per * es);
  w.v = c.take<char>(per * es);
  w.keep = c.take<char>((uint64_t)rows * jp * es);
  w.bias = c.take<float>((uint64_t)bias_batches * heads * jp * jp);
  w.mb = c.take<float>((uint64_t)rows * jp);
  w.mflag = c.take<int>((uint64_t)rows * (jp / 32));
  w.kmax = c.take<unsigned>((uint64_t)rows * heads);
  w.bmax = c.take<int>((uint64_t)bias_batches * heads * jp);
  w.rowflag = c.take<int>((uint64_t)rows);
  w.anykeep = c.take<int>((uint64_t)rows);
}

// Wide-channel path: bf16 compute, C and H*32 in {128, 256, 384}, one of them
// 256 or more (the weight slices of the register-resident kernels no longer
// fit).
bool triatt_wide(int c, int heads, int dt) {
  const int hd = heads * 32;
  return dt == ODDE_BF16 && (c == 128 || c == 256 || c == 384) &&
         (hd == 128 || hd == 256 || hd == 384) && (c >= 256 || hd >= 256);
}
// The weight-stationary projection / output pair, with the gate fused into the
// output kernel: bf16 compute where C and H*32 are 64 or 128 (each wave's
// weight slices fit in registers).  Disjoint from the wide path.
bool triatt_ws(int c, int heads, int dt) {
  const int hd = heads * 32;
  return dt == ODDE_BF16 && (c == 64 || c == 128) && (hd == 64 || hd == 128);
}
// rows of the wide path's GEMMs: the n * Jp pairs padded to whole groups of
// 8 row tiles
int64_t triatt_wide_rows(int n) { return (int64_t)round_up(n * round_up(n, 64), 2048); }

// wsplit (ODDE_F32X3): W_q, W_k, W_v, W_g ([HD][C] each), W_b ([H][C]) and
// W_o ([C][HD]) split once per call into bf16 hi | lo rows
struct TriattWs { CoreBufs c; void* gate; void* o; void* zn; char* wsplit; uint64_t bytes; };

TriattWs carve_triatt(void* base, uint64_t size, int n, int heads, int cz, int dt) {
  const int jp = round_up(n, 64);
  const bool wide = triatt_wide(cz, heads, dt);
  const uint64_t per = (uint64_t)n * heads * jp * 32 * dtype_size(dt);
  Carver c(base, size);
  TriattWs w;
  carve_core_bufs(c, w.c, n, heads, jp, 1, dt);
  w.gate = triatt_ws(cz, heads, dt) ? nullptr : c.take<char>(per);
  // the wide path reads o as GEMM rows, whole 256-row tiles
  w.o = c.take<char>(wide ? (uint64_t)triatt_wide_rows(n) * heads * 32 * 2 : per);
  w.zn = wide ? c.take<char>((uint64_t)triatt_wide_rows(n) * cz * 2) : nullptr;
  const uint64_t hd = (uint64_t)heads * 32;
  w.wsplit = dt == ODDE_F32X3 ? c.take<char>((5 * hd + heads) * cz * 4) : nullptr;
  w.bytes = (c.used + 255) & ~uint64_t(255);
  return w;
}

int check_triatt(const odde_triatt_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "triatt: null args");
  if (a->struct_size != sizeof(odde_triatt_args))
    return set_error(ODDE_EINVAL, "triatt: struct_size mismatch (ABI version skew)");
  if (a->n <= 0 || a->c <= 0 || a->heads <= 0)
    return set_error(ODDE_EINVAL, "triatt: n, c and heads must be positive");
  if (a->batch < 0) return set_error(ODDE_EINVAL, "triatt: batch must be >= 0");
  if (a->head_dim != 32) return set_error(ODDE_EUNSUPPORTED, "triatt: head_dim must be 32");
  if (a->heads > 16) return set_error(ODDE_EUNSUPPORTED, "triatt: at most 16 heads");
  if (!valid_dtype(a->z_dtype) ||
      !(valid_dtype(a->compute_dtype) || a->compute_dtype == ODDE_F32X3))
    return set_error(ODDE_EINVAL, "triatt: bad dtype");
  if (a->z_dtype == ODDE_BF16 && a->compute_dtype != ODDE_BF16)
    return set_error(ODDE_EUNSUPPORTED, "triatt: bf16 storage with f32 compute");
  return ODDE_OK;
}

// ODDE_TRIATT_PROJ_F32_PLAIN=1: the fp32 projection without staged weights
// (tuning).
inline bool triatt_proj_f32_plain() {
  static const bool v = [] {
    const char* e = getenv("ODDE_TRIATT_PROJ_F32_PLAIN");
    return e && atoi(e) != 0;
  }();
  return v;
}
template <typename ZT, typename CT, int kC, bool kX3Mul = false>
void launch_proj(const TriattProjArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  // fp32 weights are read from L2 per fragment: more rows i per wave as
  // registers allow (4 up to C = 128, 2 at C = 256), once the grid stays
  // large enough (n >= 256)
  constexpr int kRB = sizeof(CT) != 4 ? 1 : kC <= 8 ? 2 : 1;
  if constexpr (sizeof(CT) == 4 && kC <= 4) {
    // f32 data from n = 256: the weights staged in LDS
    if (n >= 256 && !triatt_proj_f32_plain()) {
      dim3 grid(jp / 64, (n + 1) / 2);
      hipLaunchKernelGGL((triatt_proj_kernel<ZT, CT, kC, 2, kX3Mul, true>), grid, dim3(256), 0, st,
                         p);
      return;
    }
  }
  if (kRB > 1 && n >= 256) {
    const int rows = (n + kRB - 1) / kRB;
    dim3 grid(jp / 64, rows, proj_split((int64_t)(jp / 64) * rows, p.heads));
    hipLaunchKernelGGL((triatt_proj_kernel<ZT, CT, kC, kRB, kX3Mul>), grid, dim3(256), 0, st, p);
    return;
  }
  dim3 grid(jp / 64, n, proj_split((int64_t)(jp / 64) * n, p.heads));
  hipLaunchKernelGGL((triatt_proj_kernel<ZT, CT, kC, 1, kX3Mul>), grid, dim3(256), 0, st, p);
}
// f32 compute: true fp32 products, or three bf16 parts (x3)
template <typename ZT, typename CT, int kC>
void launch_proj_ct(const TriattProjArgs<ZT, CT>& p, int n, int jp, bool x3, hipStream_t st) {
  if constexpr (sizeof(CT) == 4) {
    if (x3) {
      launch_proj<ZT, CT, kC, true>(p, n, jp, st);
      return;
    }
  }
  launch_proj<ZT, CT, kC>(p, n, jp, st);
}

// Persistent weight-stationary projection where the per-wave weight slice
// fits in registers (bf16: (HD/16)*(C/32) <= 32 fragments); false otherwise.
template <typename ZT, typename CT, int kC, int kHD>
void launch_proj_ws_t(const TriattProjArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  const int ntiles = n * (jp / kTileRows);
  static const int resident =
      resident_grid(reinterpret_cast<const void*>(&triatt_proj_ws_kernel<ZT, CT, kC, kHD>), 256);
  hipLaunchKernelGGL((triatt_proj_ws_kernel<ZT, CT, kC, kHD>), dim3(min(ntiles, resident)),
                     dim3(256), 0, st, p, ntiles);
}

// H*32 = 128: the q, k, v channels split over all four waves.
template <typename ZT, typename CT, int kC>
void launch_proj_ws4_t(const TriattProjArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  const int ntiles = n * (jp / kTileRows);
  static const int resident =
      resident_grid(reinterpret_cast<const void*>(&triatt_proj_ws4_kernel<ZT, CT, kC>), 256);
  hipLaunchKernelGGL((triatt_proj_ws4_kernel<ZT, CT, kC>), dim3(min(ntiles, resident)), dim3(256),
                     0, st, p, ntiles);
}

template <typename ZT, typename CT>
bool launch_proj_ws(const TriattProjArgs<ZT, CT>& p, int C, int HD, int n, int jp, hipStream_t st) {
  if constexpr (sizeof(CT) != 2) {
    return false;
  } else {
  if (C == 128 && HD == 128) { launch_proj_ws4_t<ZT, CT, 4>(p, n, jp, st); return true; }
  if (C == 64 && HD == 64) { launch_proj_ws_t<ZT, CT, 2, 2>(p, n, jp, st); return true; }
  if (C == 128 && HD == 64) { launch_proj_ws_t<ZT, CT, 4, 2>(p, n, jp, st); return true; }
  if (C == 64 && HD == 128) { launch_proj_ws4_t<ZT, CT, 2>(p, n, jp, st); return true; }
    return false;
  }
}

template <typename ZT, typename CT, int kHD, int kC>
void launch_out_ws_t(const TriattOutArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  const int ntiles = n * (jp / kTileRows);
  static const int resident =
      resident_grid(reinterpret_cast<const void*>(&triatt_out_ws_kernel<ZT, CT, kHD, kC>), 256);
  hipLaunchKernelGGL((triatt_out_ws_kernel<ZT, CT, kHD, kC>), dim3(min(ntiles, resident)),
                     dim3(256), 0, st, p, ntiles);
}
template <typename ZT, typename CT>
bool launch_out_ws(const TriattOutArgs<ZT, CT>& p, int HD, int C, int n, int jp, hipStream_t st) {
  if constexpr (sizeof(CT) != 2) {
    return false;
  } else {
  if (HD == 128 && C == 128) { launch_out_ws_t<ZT, CT, 4, 4>(p, n, jp, st); return true; }
  if (HD == 64 && C == 64) { launch_out_ws_t<ZT, CT, 2, 2>(p, n, jp, st); return true; }
  if (HD == 64 && C == 128) { launch_out_ws_t<ZT, CT, 2, 4>(p, n, jp, st); return true; }
  if (HD == 128 && C == 64) { launch_out_ws_t<ZT, CT, 4, 2>(p, n, jp, st); return true; }
    return false;
  }
}

// ODDE_TRIATT_OUT_F32_PLAIN=1: the fp32 output kernel without staged
// weights (tuning).
inline bool triatt_out_f32_plain() {
  static const bool v = [] {
    const char* e = getenv("ODDE_TRIATT_OUT_F32_PLAIN");
    return e && atoi(e) != 0;
  }();
  return v;
}
template <typename ZT, typename CT, int kHD>
void launch_out(const TriattOutArgs<ZT, CT>& p, int n, int jp, bool x3, hipStream_t st) {
  // fp32: W_o is read from L2 per fragment, so 4 rows i per workgroup up to
  // HD = 128 (2 up to 256) once the grid stays large (n >= 256)
  constexpr int kRB = sizeof(CT) != 4 ? 1 : kHD <= 4 ? 4 : kHD <= 8 ? 2 : 1;
  if constexpr (kRB > 1) {
    if (n >= 256) {
      const int rows = (n + kRB - 1) / kRB;
      if (kHD <= 4 && !triatt_out_f32_plain()) {
        // f32 data: W_o staged in LDS (one split)
        dim3 grid(jp / 64, rows);
        if (x3)
          hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD, true, kRB, true>), grid, dim3(256), 0,
                             st, p);
        else
          hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD, false, kRB, true>), grid, dim3(256), 0,
                             st, p);
        return;
      }
      dim3 grid(jp / 64, rows, proj_split((int64_t)(jp / 64) * rows, p.c / 16));
      if (x3)
        hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD, true, kRB>), grid, dim3(256), 0, st, p);
      else
        hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD, false, kRB>), grid, dim3(256), 0, st, p);
      return;
    }
  }
  dim3 grid(jp / 64, n, proj_split((int64_t)(jp / 64) * n, p.c / 16));
  if constexpr (sizeof(CT) == 4) {
    if (x3) {
      hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD, true>), grid, dim3(256), 0, st, p);
      return;
    }
  }
  hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD>), grid, dim3(256), 0, st, p);
}

// Core tiling: waves own R rows x 16*QB queries; a workgroup of RG x QS
// waves shares its staged K/V (R_WG = RG*R rows) and bias (Q_WG = QS*16*QB
// queries).  The default was chosen by measurement on MI355X;
// ODDE_TRIATT_TILE="R,QB,RG,QS" selects another instantiation.
struct CoreTile { int r, qb, rg, qs; };

CoreTile core_tile(int rows_per_bias, int batches, bool f32, int jp, int rows, int heads) {
  // f32 fragments are twice as wide: the bf16 tile would spill
  static CoreTile env = [] {
    CoreTile d{0, 0, 0, 0};
    if (const char* e = getenv("ODDE_TRIATT_TILE")) {
      int r = 0, qb = 0, rg = 0, qs = 0;
      if (sscanf(e, "%d,%d,%d,%d", &r, &qb, &rg, &qs) == 4) d = CoreTile{r, qb, rg, qs};
    }
    return d;
  }();
  CoreTile t = env.r ? env : (f32 ? CoreTile{2, 2, 2, 4} : CoreTile{2, 4, 2, 2});
  // bf16 at small sizes: with fewer than 2048 workgroups of 4 rows x 128
  // queries the last round of workgroups leaves most CUs idle; 4 rows x 64
  // queries doubles the count (3 workgroups per CU).  N = 384: 0.089 ->
  // 0.080 ms; from N = 512 up the default is as fast or faster.
  if (!env.r && !f32 && (int64_t)(jp / 128) * ((rows + 3) / 4) * heads < 2048)
    t = CoreTile{2, 2, 2, 2};
  // all rows of a workgroup share one bias batch
  if (batches > 1 && rows_per_bias % (t.r * t.rg) != 0) return CoreTile{1, t.qb, 1, t.qs};
  return t;
}

template <typename CT, int R, int QB, int RG, int QS>
void launch_core_t(const TriattCoreArgs<CT>& p, hipStream_t st) {
  constexpr int R_WG = R * RG, Q_WG = 16 * QB * QS;
  const int nx = (p.jp + Q_WG - 1) / Q_WG, ny = (p.rows + R_WG - 1) / R_WG;
  bool done = false;
  if constexpr (sizeof(CT) == 4 && QB == 2 && QS == 4 && ((R == 2 && RG == 2) || (R == 1 && RG == 1))) {
    // the three-part form at the f32 default tiles (whole and batched)
    if (p.x3) {
      hipLaunchKernelGGL((triatt_core_fast_kernel<CT, R, QB, RG, QS, true>),
                         dim3((unsigned)(nx * ny * p.heads)), dim3(64 * RG * QS), 0, st, p, nx, ny);
      done = true;
    }
  }
  if (!done)
    hipLaunchKernelGGL((triatt_core_fast_kernel<CT, R, QB, RG, QS>),
                       dim3((unsigned)(nx * ny * p.heads)), dim3(64 * RG * QS), 0, st, p, nx, ny);
  // the exact core keeps a modest tile; each wave loops over up to 8 query
  // blocks of one row (it does work only for rows the fast core flagged)
  dim3 grid2((p.jp + 255) / 256, (p.rows + 3) / 4, p.heads);
  hipLaunchKernelGGL((triatt_core_exact_kernel<CT, 1, 2>), grid2, dim3(256), 0, st, p);
}

template <typename CT>
int launch_core(const TriattCoreArgs<CT>& p0, int batches, hipStream_t st) {
  TriattCoreArgs<CT> p = p0;
  p.out16 = sizeof(CT) == 2 && (reinterpret_cast<uintptr_t>(p.out) & 15) == 0 &&
            ((p.o_row | p.o_h | p.o_j) & 7) == 0;
  const CoreTile t = core_tile(p.rows_per_bias, batches, sizeof(CT) == 4, p.jp, p.rows, p.heads);
  LaunchScope ls(ODDE_K_TRIATT_CORE, st);
#define ODDE_TILE(R, QB, RG, QS)                                              \
  else if (t.r == R && t.qb == QB && t.rg == RG && t.qs == QS)                \
    launch_core_t<CT, R, QB, RG, QS>(p, st);
  if (false) {}
  ODDE_TILE(2, 4, 2, 4)
  ODDE_TILE(2, 4, 2, 2)
  ODDE_TILE(2, 2, 2, 4)
  ODDE_TILE(2, 4, 1, 4)
  ODDE_TILE(1, 4, 4, 2)
  ODDE_TILE(2, 2, 4, 2)
  ODDE_TILE(1, 4, 1, 4)
  ODDE_TILE(1, 4, 1, 1)
  ODDE_TILE(1, 2, 1, 4)
  ODDE_TILE(1, 2, 1, 1)
  ODDE_TILE(2, 2, 2, 2)
  ODDE_TILE(2, 2, 1, 4)
  ODDE_TILE(1, 4, 2, 2)
  else return set_error(ODDE_EINVAL, "ODDE_TRIATT_TILE: unsupported R,QB,RG,QS");
#undef ODDE_TILE
  return check_launch("triatt_core");
}

template <typename CT>
void fill_core_args(TriattCoreArgs<CT>& c, const CoreBufs& b) {
  c.q = static_cast<const CT*>(b.q);
  c.k = static_cast<const CT*>(b.k);
  c.v = static_cast<const CT*>(b.v);
  c.keep = static_cast<const CT*>(b.keep);
  c.bias = b.bias; c.mb = b.mb; c.mflag = b.mflag; c.kmax = b.kmax; c.bmax = b.bmax;
  c.rowflag = b.rowflag; c.anykeep = b.anykeep;
}

// Wide-channel projection: LayerNorm pass into bf16 rows, mask outputs and
// triangle bias, then q, k, v, gate as one NT GEMM.
template <typename ZT>
int run_triatt_proj_wide(const TriattProjArgs<ZT, bf16>& p, const odde_triatt_args* a, bf16* zn,
                         hipStream_t st) {
  const int n = p.n, jp = p.jp, C = a->c, HD = p.heads * 32;
  const int64_t rows = (int64_t)n * jp;
  const int lg = (int)std::min<int64_t>((rows + 15) / 16, 4096);
  switch (C) {
    case 128:
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 128>), dim3(lg), dim3(256), 0, st, p.z, p.z_s0,
                         p.z_s1, n, n, jp, p.ln_w, p.ln_b, p.eps, zn);
      hipLaunchKernelGGL((triatt_bias_mask_wide_kernel<ZT, 4>), dim3(jp / 64, n), dim3(256), 0,
                         st, p, zn);
      break;
    case 256:
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 256>), dim3(lg), dim3(256), 0, st, p.z, p.z_s0,
                         p.z_s1, n, n, jp, p.ln_w, p.ln_b, p.eps, zn);
      hipLaunchKernelGGL((triatt_bias_mask_wide_kernel<ZT, 8>), dim3(jp / 64, n), dim3(256), 0,
                         st, p, zn);
      break;
    case 384:
      hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 384>), dim3(lg), dim3(256), 0, st, p.z, p.z_s0,
                         p.z_s1, n, n, jp, p.ln_w, p.ln_b, p.eps, zn);
      hipLaunchKernelGGL((triatt_bias_mask_wide_kernel<ZT, 12>), dim3(jp / 64, n), dim3(256), 0,
                         st, p, zn);
      break;
    default: return set_error(ODDE_EUNSUPPORTED, "triatt: c must be 128, 256 or 384 here");
  }
  const int row_tiles = (int)(triatt_wide_rows(n) / kWTX), ncol = 4 * HD / kWTY;
  hipLaunchKernelGGL((triatt_qkvg_wide_kernel<ZT>), dim3(row_tiles * ncol), dim3(512), 0, st, p,
                     zn, C, ncol);
  return ODDE_OK;
}

template <typename ZT, typename CT>
int run_triatt(const odde_triatt_args* a, hipStream_t st) {
  const int n = a->n, H = a->heads, C = a->c, HD = H * 32;
  const int jp = round_up(n, 64);
  TriattWs ws = carve_triatt(a->workspace, a->workspace_bytes, n, H, C, a->compute_dtype);
  bool wide = false;
  if constexpr (sizeof(CT) == 2) wide = triatt_wide(C, H, a->compute_dtype);
  const bool ws_path = triatt_ws(C, H, a->compute_dtype);
  // f32 data with reduced-precision products allowed: every product of the
  // module in three bf16 parts
  const bool x3 = sizeof(CT) == 4 && a->compute_dtype == ODDE_F32X3;

  TriattProjArgs<ZT, CT> p;
  p.z = static_cast<const ZT*>(a->z);
  p.z_s0 = a->z_s0; p.z_s1 = a->z_s1;
  p.mask = a->mask; p.m_s0 = a->mask_s0; p.m_s1 = a->mask_s1;
  p.ln_w = a->ln_w; p.ln_b = a->ln_b;
  p.wb = static_cast<const CT*>(a->w_bias);
  p.wq = static_cast<const CT*>(a->w_q);
  p.wk = static_cast<const CT*>(a->w_k);
  p.wv = static_cast<const CT*>(a->w_v);
  p.wg = static_cast<const CT*>(a->w_g);
  p.q = static_cast<CT*>(ws.c.q); p.k = static_cast<CT*>(ws.c.k); p.v = static_cast<CT*>(ws.c.v);
  p.gate = static_cast<CT*>(ws.gate); p.keep = static_cast<CT*>(ws.c.keep);
  const CT* w_o = static_cast<const CT*>(a->w_o);
  if (x3) {
    // the weights as bf16 hi | lo rows, split once for this call
    const int HDw = H * 32;
    char* d = ws.wsplit;
    const void* src[5] = {a->w_q, a->w_k, a->w_v, a->w_g, a->w_bias};
    const CT** dstp[5] = {&p.wq, &p.wk, &p.wv, &p.wg, &p.wb};
    for (int m = 0; m < 5; ++m) {
      const int rows = m < 4 ? HDw : H;
      launch_split_x3(src[m], rows, C, d, false, st);
      *dstp[m] = reinterpret_cast<const CT*>(d);
      d += (size_t)rows * C * 4;
    }
    launch_split_x3(a->w_o, C, HDw, d, false, st);
    w_o = reinterpret_cast<const CT*>(d);
  }
  p.bias = ws.c.bias; p.mb = ws.c.mb; p.mflag = ws.c.mflag; p.kmax = ws.c.kmax;
  p.bmax = ws.c.bmax; p.anykeep = ws.c.anykeep;
  p.n = n; p.jp = jp; p.heads = H;
  p.q_scale = kLog2e / sqrtf((float)a->head_dim);
  p.mask_inf = a->inf * kLog2e;
  p.eps = a->eps;
  {
    LaunchScope ls(ODDE_K_TRIATT_PROJ, st);
    PrepArgs pa{a->mask, a->mask_s0, a->mask_s1, ws.c.anykeep, ws.c.rowflag, ws.c.kmax,
                ws.c.bmax, n, jp, H};
    hipLaunchKernelGGL(triatt_prep_kernel, dim3(n), dim3(256), 0, st, pa);
    if constexpr (sizeof(CT) == 2) {
      if (wide) {
        int rc = run_triatt_proj_wide<ZT>(p, a, static_cast<bf16*>(ws.zn), st);
        if (rc) return rc;
      }
    }
    if (ws_path) {
      if (!launch_proj_ws<ZT, CT>(p, C, HD, n, jp, st))
        return set_error(ODDE_EUNSUPPORTED, "triatt: no weight-stationary projection for this shape");
    } else if (!wide) {
      switch (C) {
        case 64: launch_proj_ct<ZT, CT, 2>(p, n, jp, x3, st); break;
        case 128: launch_proj_ct<ZT, CT, 4>(p, n, jp, x3, st); break;
        case 256: launch_proj_ct<ZT, CT, 8>(p, n, jp, x3, st); break;
        case 384: launch_proj_ct<ZT, CT, 12>(p, n, jp, x3, st); break;
        default: return set_error(ODDE_EUNSUPPORTED, "triatt: c must be 64, 128, 256 or 384");
      }
    }
    int rc = check_launch("triatt_proj");
    if (rc) return rc;
  }

  TriattCoreArgs<CT> c;
  fill_core_args(c, ws.c);
  c.x3 = x3;
  c.gate = ws_path ? nullptr : static_cast<const CT*>(ws.gate);  // else gated in triatt_out_ws
  c.out = static_cast<CT*>(ws.o);
  c.o_row = (int64_t)jp * HD; c.o_h = 32; c.o_j = HD;
  c.rows = n; c.heads = H; c.n = n; c.jp = jp; c.rows_per_bias = n;
  int rc = launch_core<CT>(c, 1, st);
  if (rc) return rc;

  TriattOutArgs<ZT, CT> o;
  o.o = static_cast<const CT*>(ws.o);
  o.wo = w_o;
  o.res = static_cast<const ZT*>(a->z); o.r_s0 = a->z_s0; o.r_s1 = a->z_s1;
  o.out = static_cast<ZT*>(a->out); o.o_s0 = a->out_s0; o.o_s1 = a->out_s1;
  o.n = n; o.jp = jp; o.c = C; o.add = a->add_residual;
  o.wg = static_cast<const CT*>(a->w_g); o.ln_w = a->ln_w; o.ln_b = a->ln_b; o.eps = a->eps;
  {
    LaunchScope ls(ODDE_K_TRIATT_OUT, st);
    if constexpr (sizeof(CT) == 2) {
      if (wide) {
        const int row_tiles = (int)(triatt_wide_rows(n) / kWTX), ncol = C / kWTY;
        hipLaunchKernelGGL((triatt_out_wide_kernel<ZT>), dim3(row_tiles * ncol), dim3(512), 0, st,
                           o, HD, ncol);
        return check_launch("triatt_out (wide)");
      }
    }
    if (ws_path) {
      if (!launch_out_ws<ZT, CT>(o, HD, C, n, jp, st))
        return set_error(ODDE_EUNSUPPORTED, "triatt: no weight-stationary output for this shape");
      return check_launch("triatt_out");
    }
    switch (HD) {
      case 64: launch_out<ZT, CT, 2>(o, n, jp, x3, st); break;
      case 128: launch_out<ZT, CT, 4>(o, n, jp, x3, st); break;
      case 256: launch_out<ZT, CT, 8>(o, n, jp, x3, st); break;
      case 384: launch_out<ZT, CT, 12>(o, n, jp, x3, st); break;
      default: return set_error(ODDE_EUNSUPPORTED, "triatt: heads*32 must be 64, 128, 256 or 384");
    }
    return check_launch("triatt_out");
  }
}

}  // namespace

extern "C" {

int odde_triatt_workspace_bytes(const odde_triatt_args* a, uint64_t* bytes) {
  int rc = check_triatt(a);
  if (rc) return rc;
  if (!bytes) return set_error(ODDE_EINVAL, "triatt: null bytes");
  *bytes = carve_triatt(nullptr, 0, a->n, a->heads, a->c, a->compute_dtype).bytes;
  return ODDE_OK;
}

int odde_triatt_fwd(const odde_triatt_args* a, void* stream) {
  int rc = check_triatt(a);
  if (rc) return rc;
  if (!a->z || !a->out || !a->ln_w || !a->ln_b || !a->w_bias || !a->w_q || !a->w_k ||
      !a->w_v || !a->w_g || !a->w_o)
    return set_error(ODDE_EINVAL, "triatt: null tensor pointer");
  const uint64_t need = carve_triatt(nullptr, 0, a->n, a->heads, a->c, a->compute_dtype).bytes;
  if (!a->workspace || a->workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(a->workspace) & 255))
    return set_error(ODDE_EWORKSPACE, "triatt: workspace missing, too small or not 256-byte aligned");
  const int zes = dtype_size(a->z_dtype);
  const int nb = a->batch > 1 ? a->batch : 1;
  const int64_t sb = nb > 1 ? (a->z_sb | a->out_sb) : 0;
  if ((reinterpret_cast<uintptr_t>(a->z) | reinterpret_cast<uintptr_t>(a->out)) & 15 ||
      ((a->z_s0 | a->z_s1 | a->out_s0 | a->out_s1 | sb) * zes) & 15)
    return set_error(ODDE_EINVAL, "triatt: z/out rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // The views of a batch run in order on the stream and share the workspace.
  odde_triatt_args e = *a;
  for (int b = 0; b < nb; ++b) {
    e.z = static_cast<const char*>(a->z) + (int64_t)b * a->z_sb * zes;
    e.out = static_cast<char*>(a->out) + (int64_t)b * a->out_sb * zes;
    e.mask = a->mask ? a->mask + (int64_t)b * a->mask_sb : nullptr;
    if (a->z_dtype == ODDE_F32 && a->compute_dtype != ODDE_BF16) rc = run_triatt<float, float>(&e, st);
    else if (a->z_dtype == ODDE_F32) rc = run_triatt<float, bf16>(&e, st);
    else rc = run_triatt<bf16, bf16>(&e, st);
    if (rc) return rc;
  }
  return ODDE_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// core-only slot
// ---------------------------------------------------------------------------
namespace {

struct CoreWs { CoreBufs c; uint64_t bytes; };

CoreWs carve_core(void* base, uint64_t size, const odde_triatt_core_args* a) {
  const int jp = round_up(a->n, 64);
  Carver c(base, size);
  CoreWs w;
  carve_core_bufs(c, w.c, a->batch * a->rows, a->heads, jp, a->batch, a->dtype);
  w.bytes = (c.used + 255) & ~uint64_t(255);
  return w;
}

int check_core(const odde_triatt_core_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "triatt_core: null args");
  if (a->struct_size != sizeof(odde_triatt_core_args))
    return set_error(ODDE_EINVAL, "triatt_core: struct_size mismatch (ABI version skew)");
  if (a->batch <= 0 || a->rows <= 0 || a->heads <= 0 || a->n <= 0)
    return set_error(ODDE_EINVAL, "triatt_core: sizes must be positive");
  if (a->head_dim != 32) return set_error(ODDE_EUNSUPPORTED, "triatt_core: head_dim must be 32");
  if (a->heads > 256) return set_error(ODDE_EUNSUPPORTED, "triatt_core: at most 256 heads");
  if (!valid_dtype(a->dtype)) return set_error(ODDE_EINVAL, "triatt_core: bad dtype");
  return ODDE_OK;
}

template <typename CT>
int run_core(const odde_triatt_core_args* a, hipStream_t st) {
  const int jp = round_up(a->n, 64);
  CoreWs ws = carve_core(a->workspace, a->workspace_bytes, a);
  const int rows = a->batch * a->rows;
  RelayoutArgs<CT> r;
  r.q = static_cast<const CT*>(a->q); r.q_sb = a->q_sb; r.q_si = a->q_si; r.q_sh = a->q_sh; r.q_sj = a->q_sj;
  r.k = static_cast<const CT*>(a->k); r.k_sb = a->k_sb; r.k_si = a->k_si; r.k_sh = a->k_sh; r.k_sj = a->k_sj;
  r.v = static_cast<const CT*>(a->v); r.v_sb = a->v_sb; r.v_si = a->v_si; r.v_sh = a->v_sh; r.v_sj = a->v_sj;
  r.bias = a->bias; r.b_sb = a->b_sb; r.b_sh = a->b_sh; r.b_sq = a->b_sq; r.b_sk = a->b_sk;
  r.mask = a->mask; r.m_sb = a->m_sb; r.m_si = a->m_si; r.m_sk = a->m_sk;
  r.wq = static_cast<CT*>(ws.c.q); r.wk = static_cast<CT*>(ws.c.k); r.wv = static_cast<CT*>(ws.c.v);
  r.wkeep = static_cast<CT*>(ws.c.keep);
  r.wbias = ws.c.bias; r.wmb = ws.c.mb;
  r.anykeep = ws.c.anykeep; r.rowflag = ws.c.rowflag; r.kmax = ws.c.kmax; r.bmax = ws.c.bmax;
  r.batch = a->batch; r.rows = a->rows; r.heads = a->heads; r.n = a->n; r.jp = jp;
  r.q_scale = a->scale * kLog2e;
  r.mask_inf = a->inf_value * kLog2e;
  {
    const int64_t total = (int64_t)rows * a->heads * jp;
    const int64_t total_b = (int64_t)a->batch * a->heads * jp * jp;
    const int64_t nbh = (int64_t)a->batch * a->heads * jp;
    const int64_t nflag = (int64_t)rows * (jp / 32);
    LaunchScope ls(ODDE_K_TRIATT_RELAYOUT, st);
    hipLaunchKernelGGL((triatt_slot_prep_kernel<CT>), dim3(rows), dim3(256), 0, st, r);
    hipLaunchKernelGGL((triatt_relayout_kernel<CT>), dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, st, r);
    hipLaunchKernelGGL((triatt_bias_relayout_kernel<CT>),
                       dim3((unsigned)((total_b + 255) / 256)), dim3(256), 0, st, r);
    hipLaunchKernelGGL(triatt_bmax_fold_kernel, dim3((unsigned)((nbh + 255) / 256)), dim3(256),
                       0, st, ws.c.bias, ws.c.bmax, a->batch * a->heads, a->n, jp);
    hipLaunchKernelGGL(triatt_mflag_kernel, dim3((unsigned)((nflag + 255) / 256)), dim3(256), 0,
                       st, ws.c.mb, ws.c.mflag, rows, jp);
    int rc = check_launch("triatt_relayout");
    if (rc) return rc;
  }
  TriattCoreArgs<CT> c;
  fill_core_args(c, ws.c);
  c.gate = nullptr;
  c.out = static_cast<CT*>(a->out);
  c.o_row = a->o_si;  // rows are (b, i): o_sb == rows * o_si is checked by the caller
  c.o_h = a->o_sh; c.o_j = a->o_sj;
  c.rows = rows; c.heads = a->heads; c.n = a->n; c.jp = jp;
  c.rows_per_bias = a->rows;
  return launch_core<CT>(c, a->batch, st);
}

}  // namespace

extern "C" {

int odde_triatt_core_workspace_bytes(const odde_triatt_core_args* a, uint64_t* bytes) {
  int rc = check_core(a);
  if (rc) return rc;
  if (!bytes) return set_error(ODDE_EINVAL, "triatt_core: null bytes");
  *bytes = carve_core(nullptr, 0, a).bytes;
  return ODDE_OK;
}

int odde_triatt_core_fwd(const odde_triatt_core_args* a, void* stream) {
  int rc = check_core(a);
  if (rc) return rc;
  if (!a->q || !a->k || !a->v || !a->bias || !a->out)
    return set_error(ODDE_EINVAL, "triatt_core: null tensor pointer");
  if (a->o_sb != (int64_t)a->rows * a->o_si)
    return set_error(ODDE_EUNSUPPORTED, "triatt_core: out must have o_sb == rows * o_si");
  const int es = dtype_size(a->dtype);
  if ((reinterpret_cast<uintptr_t>(a->out) & 15) || ((a->o_si | a->o_sh | a->o_sj) * es) & 15)
    return set_error(ODDE_EINVAL, "triatt_core: out rows must be 16-byte aligned");
  const uint64_t need = carve_core(nullptr, 0, a).bytes;
  if (!a->workspace || a->workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(a->workspace) & 255))
    return set_error(ODDE_EWORKSPACE, "triatt_core: workspace missing, too small or misaligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == ODDE_F32) return run_core<float>(a, st);
  return run_core<bf16>(a, st);
}

}  // extern "C"
