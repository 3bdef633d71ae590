// Fused pair/single Transition (SwiGLU) for gfx950:
//   y = LN(x);  h = silu(y W_a^T) * (y W_b^T);  out = (add ? x : 0) + h W_o^T
// with hidden = NF * C.  One workgroup (4 waves) owns 128 rows at a time
// (persistent); every wave keeps its 32 rows' LN fragments and 32 x C output
// accumulators in registers while the hidden dimension is walked in chunks
// of 32: the chunk's W_a / W_b rows and W_o columns are staged in LDS once
// per workgroup, GEMM1 (W x^T orientation) leaves each lane with hidden units
// {4g..4g+3, 16+4g..16+4g+3} of its row -- exactly the eight contraction slots
// of a K32 B-operand fragment -- so silu(a)*b feeds GEMM2 straight from
// registers (W_o fragments are read with the same slot order).  The hidden
// activations never touch memory.
#include <algorithm>

#include "common.hpp"
#include "gemm.hpp"
#include "lnpass.hpp"
#include "rowtile.hpp"
#include "runtime.hpp"

namespace odde {

template <typename ZT, typename CT>
struct TransitionArgs {
  const ZT* x;
  ZT* out;
  const float* ln_w;
  const float* ln_b;
  const CT* wa;  // [NF*C][C]
  const CT* wb;  // [NF*C][C]
  const CT* wo;  // [C][NF*C]
  int64_t rows;
  int add;
  float eps;
  // optional 16-head projection of LN'(out) (null pb_out = off)
  const float* pb_ln_w;
  const float* pb_ln_b;  // may be null
  const CT* pb_w;        // [16][C]
  float* pb_out;         // [16][rows]
  float pb_eps;
  const float* pb_zero;  // C zeros (stand-in for a null pb_ln_b)
  // fp32 form with the hidden dimension split over gridDim.y workgroups:
  // partial outputs [splits][rows][C] (null: one split, full epilogue)
  float* part = nullptr;
};

constexpr int kTrRows = 128;  // rows per workgroup tile
constexpr int kTrHid = 32;    // hidden units per chunk

// Pair-bias projection of the rows just written (AttentionPairBias's
// linear_nobias_z(layernorm_z(z)) over the updated z): the wave's 16 rows sit
// in the output accumulators, lane (g, r16) holding channels cb*16 + 4g + e of
// row r16.  LayerNorm statistics come from a reduction over the four lanes of
// a row; the normalised row feeds an MFMA as the B operand in that same
// channel order (K32 block t = channel blocks 2t, 2t+1), with W rows read in
// the matching order, giving heads 4g + e of row r16 per lane.
template <typename ZT, typename CT, int kC>
__device__ __forceinline__ void pair_bias_epilogue(const TransitionArgs<ZT, CT>& a,
                                                   const f32x4 (&zacc)[kC * 2], int64_t row,
                                                   bool valid, const float* pb_ln_w,
                                                   const float* pb_ln_b, const CT* pb_w) {
  constexpr int C = kC * 32, NCB = C / 16;
  int l = lane_id();
  asm volatile("" : "+v"(l));  // lane addresses recomputed per call, not kept live by callers
  const int g = l >> 4, r16 = l & 15;
  float zv[NCB][4];
  float s = 0.f;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      zv[cb][e] = round_to<ZT>(zacc[cb][e]);  // the value as stored
      s += zv[cb][e];
    }
  const float mean = group_sum_fast(s) * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float d = zv[cb][e] - mean;
      q += d * d;
    }
  const float rstd = rsqrtf(group_sum_fast(q) * (1.0f / C) + a.pb_eps);
  f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    float lw[8], lb[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, wv[8];
    load4(pb_ln_w + 32 * t + 4 * g, lw);
    load4(pb_ln_w + 32 * t + 16 + 4 * g, lw + 4);
    if (pb_ln_b) {
      load4(pb_ln_b + 32 * t + 4 * g, lb);
      load4(pb_ln_b + 32 * t + 16 + 4 * g, lb + 4);
    }
    load4(pb_w + r16 * C + 32 * t + 4 * g, wv);
    load4(pb_w + r16 * C + 32 * t + 16 + 4 * g, wv + 4);
    Frag<CT> yf, wf;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = zv[2 * t + (e >> 2)][e & 3];
      yf.set(e, (z - mean) * rstd * lw[e] + lb[e]);
      wf.set(e, wv[e]);
    }
    mma(pacc, wf, yf);
  }
  if (valid) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a.pb_out[(size_t)(4 * g + e) * a.rows + row] = pacc[e];
  }
}

template <typename ZT, typename CT, int kC, int NF>
__global__ __launch_bounds__(256, 2) void transition_kernel(TransitionArgs<ZT, CT> a,
                                                            int64_t ntiles) {
  constexpr int C = kC * 32, HID = NF * C, NCB = C / 16;
  constexpr int LDX = TileLD<CT, C>::value;          // x tile / W_a, W_b chunk rows
  constexpr int LDO = kTrHid + 16 / (int)sizeof(CT); // W_o chunk rows
  __shared__ __attribute__((aligned(16))) CT xs[kTrRows * LDX];
  __shared__ __attribute__((aligned(16))) CT wab[2 * kTrHid * LDX];
  __shared__ __attribute__((aligned(16))) CT wos[C * LDO];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  constexpr int VEC = 16 / sizeof(CT);

  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t r0 = tile * kTrRows;
#pragma unroll
    for (int half = 0; half < 2; ++half)
      stage_ln_tile<ZT, CT, C>(
          [&](int r) -> const ZT* {
            const int64_t row = r0 + half * 64 + r;
            return row < a.rows ? a.x + row * C : nullptr;
          },
          a.ln_w, a.ln_b, a.eps, xs + half * 64 * LDX);
    __syncthreads();
    Frag<CT> xf[2][kC];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) tile_frags<CT, C>(xs, 2 * w + rb, xf[rb]);
    f32x4 acc[2][NCB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int h0 = 0; h0 < HID; h0 += kTrHid) {
      __syncthreads();  // previous chunk's weights fully consumed
      // W_a, W_b rows h0..h0+31 (C each) and W_o columns h0..h0+31 (C rows)
      for (int ci = threadIdx.x; ci < 2 * kTrHid * (C / VEC); ci += 256) {
        const int m = ci / (kTrHid * (C / VEC)), rem = ci % (kTrHid * (C / VEC));
        const int r = rem / (C / VEC), cc = (rem % (C / VEC)) * VEC;
        const CT* src = (m ? a.wb : a.wa) + (size_t)(h0 + r) * C + cc;
        *reinterpret_cast<f32x4*>(wab + (m * kTrHid + r) * LDX + cc) =
            *reinterpret_cast<const f32x4*>(src);
      }
      for (int ci = threadIdx.x; ci < C * (kTrHid / VEC); ci += 256) {
        const int r = ci / (kTrHid / VEC), cc = (ci % (kTrHid / VEC)) * VEC;
        *reinterpret_cast<f32x4*>(wos + r * LDO + cc) =
            *reinterpret_cast<const f32x4*>(a.wo + (size_t)r * HID + h0 + cc);
      }
      __syncthreads();
      // weight fragments of this chunk (shared by the wave's two row blocks)
      Frag<CT> fa[2][kC], fb[2][kC];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb)
#pragma unroll
        for (int t = 0; t < kC; ++t) {
          fa[hb][t].load(wab + (hb * 16 + r16) * LDX + 32 * t + 8 * g);
          fb[hb][t].load(wab + (kTrHid + hb * 16 + r16) * LDX + 32 * t + 8 * g);
        }
      Frag<CT> fo[NCB];  // W_o[c][h0 + slot]: hidden 4g..4g+3 and 16+4g..16+4g+3
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const CT* row = wos + (cb * 16 + r16) * LDO;
        float v[8];
        load4(row + 4 * g, v);
        load4(row + 16 + 4 * g, v + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) fo[cb].set(e, v[e]);
      }
#pragma unroll
      for (int rb = 0; rb < 2; ++rb) {
        Frag<CT> hf;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
#pragma unroll
          for (int t = 0; t < kC; ++t) {
            mma(sa, fa[hb][t], xf[rb][t]);
            mma(sb, fb[hb][t], xf[rb][t]);
          }
          // lane: row (2w+rb)*16 + r16, hidden h0 + 16*hb + 4g + e
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float av = sa[e];
            hf.set(4 * hb + e, siluf_(av) * sb[e]);
          }
        }
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) mma(acc[rb][cb], fo[cb], hf);
      }
    }
    // epilogue: lane holds row (2w+rb)*16 + r16, channels cb*16 + 4g + e
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
      const int64_t row = r0 + (2 * w + rb) * 16 + r16;
      const bool valid = row < a.rows;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const int c0 = cb * 16 + 4 * g;
        float base[4] = {0.f, 0.f, 0.f, 0.f};
        if (valid && a.add) load4(a.x + row * C + c0, base);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[rb][cb][e] += base[e];
        if (valid) store4(a.out + row * C + c0, acc[rb][cb][0], acc[rb][cb][1], acc[rb][cb][2],
                          acc[rb][cb][3]);
      }
      if (a.pb_out)
        pair_bias_epilogue<ZT, CT, kC>(a, acc[rb], row, valid, a.pb_ln_w, a.pb_ln_b, a.pb_w);
    }
    __syncthreads();  // xs reused by the next tile
  }
}

// Pipelined form for C = 128, n = 4 (the pair transition).  Two workgroups
// of 4 waves per CU; a workgroup owns 64 kRB rows at a time, wave w rows
// 16 kRB w .. (kRB 16-row blocks): every weight fragment read from LDS serves
// kRB row blocks.  The rows never go through LDS: each wave loads its rows'
// K32 fragment slots straight into registers and applies the LayerNorm there
// (the four lanes of a row reduce by shuffles).  The hidden dimension is
// walked in chunks of 32 whose W_a / W_b rows and W_o columns (24 KiB) stream
// into three LDS stages by direct global -> LDS loads, two chunks ahead,
// continuing across row tiles (every tile walks the same chunks).
// Residual: GEMM2's output rows are permuted so that a lane's accumulators
// hold exactly the channels of the K32 fragment slots it loads for the
// LayerNorm (block cb of row r16 holds channels 32 (cb >> 1) + 8 g + 4 (cb & 1)
// + 0..3; the W_o fragment row of lane r16 in block cb is channel
// 32 (cb >> 1) + 8 (r16 >> 2) + 4 (cb & 1) + (r16 & 3)), so the rows loaded
// for the LayerNorm become the accumulators' initial values: x is read from
// memory once and the epilogue has no residual to load or add.  At a tile
// boundary each row block in turn stores (a lane's 8 consecutive channels,
// whole lines together with the neighbouring row's lanes), forms the pair
// bias (if asked) from the stored values and loads its rows of the next tile
// into the registers just stored; so the loads of one workgroup overlap its
// own epilogue and the other workgroup's MFMA work.
// LDS layouts (bf16 elements): W_a, W_b chunk rows of 128 (16 slots of 16
// bytes; slot t of row r holds chunk t ^ (r & 15)); W_o chunk rows of 32
// (4 slots; slot t of channel row c holds chunk t ^ ((c >> 3) & 3): the 16
// rows of a fragment read, channels 8j + i + const for i, j = 0..3, then
// cover 16 distinct (row position, slot) pairs of a 256-byte bank period,
// free of bank conflicts).
// The gate's exponent scale rides on the data: the LayerNorm output is
// multiplied by -log2(e) (folded into its weight and bias), so GEMM1 yields
// a'' = -log2(e) a and b'' = -log2(e) b; then
// silu(a) b = (ln 2)^2 a'' b'' / (1 + 2^a'') = a'' b'' / (log2(e)^2 (1 + 2^a'')),
// the denominator one FMA, as 1 + 2^a'' was one add.  This removes one
// multiply per hidden unit from the gate and the output scale from the
// epilogue.
constexpr float kLog2eSq = 2.08136898100560782f;  // log2(e)^2 = 1 / (ln 2)^2
constexpr int kRB = 3;                   // 16-row blocks per wave
constexpr int kTpRows = 64 * kRB;
constexpr int kTpStages = 3;
constexpr int kTpChunkElems = 3 * 4096;  // W_a, W_b: 32 x 128; W_o: 128 x 32
constexpr int kTpOps = 6;                // 1 KiB direct loads per wave per chunk

// The pair bias of one 16-row block of the pipelined C = 128 form, from the
// rows as stored: LN(z) @ W^T for 16 heads with the LayerNorm weight folded
// into W' = W diag(ln_w) (bf16, in LDS in fragment order: 16 bytes per lane
// and step) and its bias into b = W ln_b, so pb = rstd (W' (z - mean)) + b.
// The MFMA's K slots follow the accumulator layout of z: slot e of step t is
// channel 32t + 8g + e.
template <typename ZT>
__device__ __forceinline__ void pair_bias_folded(const TransitionArgs<ZT, bf16>& a,
                                                 const f32x4 (&zacc)[8], int64_t row, bool valid,
                                                 const bf16* pbwf, const float* pbb) {
  constexpr int C = 128, NCB = 8;
  int l = lane_id();
  asm volatile("" : "+v"(l));  // lane addresses recomputed per call, not kept live by callers
  const int g = l >> 4;
  float d[NCB][4];
  float s = 0.f;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d[cb][e] = round_to<ZT>(zacc[cb][e]);  // the value as stored
      s += d[cb][e];
    }
  const float mean = group_sum_fast(s) * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      d[cb][e] -= mean;
      q += d[cb][e] * d[cb][e];
    }
  const float rstd = rsqrtf(group_sum_fast(q) * (1.0f / C) + a.pb_eps);
  f32x4 pacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    Frag<bf16> wf, yf;
    wf.load(pbwf + (t * 64 + l) * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) yf.set(e, d[2 * t + (e >> 2)][e & 3]);
    mma(pacc, wf, yf);
  }
  float bb[4];
  load4(pbb + 4 * g, bb);
  if (valid) {
#pragma unroll
    for (int e = 0; e < 4; ++e) a.pb_out[(size_t)(4 * g + e) * a.rows + row] = pacc[e] * rstd + bb[e];
  }
}

// A lane's K32 fragment slots of one C = 128 row (channels 32t + 8g .. +7 for
// t = 0..3) held as raw 16-byte chunks until they are normalised.
template <typename ZT>
struct RowSlots {
  static constexpr int PER_T = 8 * (int)sizeof(ZT) / 16;  // chunks per K32 block
  f32x4 c[4 * PER_T];
  __device__ __forceinline__ void load(const ZT* row, int g) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int k = 0; k < PER_T; ++k)
        c[t * PER_T + k] =
            *reinterpret_cast<const f32x4*>(row + 32 * t + 8 * g + k * (16 / (int)sizeof(ZT)));
  }
  __device__ __forceinline__ void get(int t, float (&x)[8]) const {
    if constexpr (sizeof(ZT) == 4) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        x[e] = c[2 * t][e];
        x[4 + e] = c[2 * t + 1][e];
      }
    } else {
      const bf16x8 v = __builtin_bit_cast(bf16x8, c[t]);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
    }
  }
};

// One output row of the pipelined form from its accumulators: lane (g, r16)
// holds channels 32t + 8g .. +7 in blocks 2t, 2t + 1.  fp32 rows go out as
// whole 128-byte lines (line t) together with the row of lane r16 ^ 1.
template <typename ZT>
__device__ __forceinline__ void store_rows_pipe(ZT* row, ZT* partner_row, const f32x4 (&r)[8],
                                                bool ok, bool partner_ok) {
  const int g = lane_id() >> 4;
  if constexpr (sizeof(ZT) == 4) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      store_line_pair_at(reinterpret_cast<f32x4*>(row + 32 * t),
                         reinterpret_cast<f32x4*>(partner_row + 32 * t), 2 * g, 2 * g + 1,
                         r[2 * t], r[2 * t + 1], ok, partner_ok);
  } else {
    if (!ok) return;
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
      store4(row + 32 * (cb >> 1) + 8 * g + 4 * (cb & 1), r[cb][0], r[cb][1], r[cb][2], r[cb][3]);
  }
}

// kAdd / kPb: the residual add and the pair-bias epilogue, fixed per
// instantiation so that each form's epilogue is straight-line code
template <typename ZT, bool kAdd, bool kPb>
__global__ __launch_bounds__(256, 2) void transition_pipe_kernel(TransitionArgs<ZT, bf16> a,
                                                                 int64_t ntiles) {
  constexpr int C = 128, kC = 4, HID = 512, NCB = C / 16, NCHUNK = HID / kTrHid;
  __shared__ __attribute__((aligned(16))) bf16 ws[kTpStages][kTpChunkElems];
  // parameters read every tile, kept in LDS: LN weight, bias; and for the
  // pair-bias epilogue the folded 16 x C projection (fragment order) and
  // its 16 biases
  __shared__ __attribute__((aligned(16))) float lnp[2 * C];
  __shared__ __attribute__((aligned(16))) bf16 pbwf[16 * C];
  __shared__ __attribute__((aligned(16))) float pbb[16 + 64];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  for (int t = threadIdx.x; t < C; t += 256) {
    // the LayerNorm output carries the factor -log2(e) (see the gate below)
    lnp[t] = a.ln_w[t] * kNegLog2e;
    lnp[C + t] = a.ln_b[t] * kNegLog2e;
  }
  if (kPb) {
    // thread (w, g, r16) forms fragment slot set (t = w, g) of head r16:
    // W'[r16][c] = W[r16][c] ln_w[c] for c = 32w + 8g + e,
    // and its part of b[r16] = sum_c W[r16][c] ln_b[c]; the parts are summed
    // over g by lane swaps and over w in a fixed order
    Frag<bf16> wf;
    float part = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int c = 32 * w + 8 * g + e;
      const float wv = (float)a.pb_w[r16 * C + c];
      wf.set(e, wv * a.pb_ln_w[c]);
      if (a.pb_ln_b) part += wv * a.pb_ln_b[c];
    }
    *reinterpret_cast<bf16x8*>(pbwf + threadIdx.x * 8) = wf.v;
    part = group_sum_fast(part);
    if (g == 0) pbb[16 + 16 * w + r16] = part;
    __syncthreads();
    if (threadIdx.x < 16)
      pbb[threadIdx.x] = ((pbb[16 + threadIdx.x] + pbb[32 + threadIdx.x]) + pbb[48 + threadIdx.x]) +
                         pbb[64 + threadIdx.x];
  }
  __syncthreads();  // lnp / pbwf / pbb are read before the first chunk barrier

  // this workgroup's tiles and chunk loads (only loads that will be consumed
  // are issued, so none is in flight when the workgroup ends)
  const int my_tiles =
      blockIdx.x < ntiles ? (int)((ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x) : 0;
  if (my_tiles == 0) return;
  const int Q = my_tiles * NCHUNK;
  // A chunk is 24 blocks of 1 KiB (8 per region: W_a, W_b, W_o); wave w's op
  // `op` loads block bi = 4 (op & 1) + w of region op >> 1, so the region is
  // known at compile time and the lane's part of the source offset depends
  // only on op & 1: W_a / W_b block bi holds rows 4 bi + (l >> 4), whose
  // 16-byte chunks are swizzled by key(row) = (4 (row >> 3) + (row & 3)) & 15
  // = 8 (op & 1) + 4 (w >> 1) + (l >> 4) (the 16 rows one GEMM1 fragment read
  // touches, 8 (m >> 2) + 4 hb + (m & 3), have the distinct keys m); W_o
  // block bi holds channels c = 16 bi + (l >> 2), swizzled by
  // (c >> 3) & 3 = (2 w + (l >> 5)) & 3.
  const int wu = __builtin_amdgcn_readfirstlane(w);
  int lane_ab[2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
    lane_ab[p] = (l >> 4) * C + ((l & 15) ^ (8 * p + 4 * (w >> 1) + (l >> 4))) * 8;
  const int lane_o = (l >> 2) * HID + ((l & 3) ^ ((2 * w + (l >> 5)) & 3)) * 8;
  auto issue = [&](int q) {
    const int h0 = (q % NCHUNK) * kTrHid;
    bf16* base = ws[q % kTpStages];
#pragma unroll
    for (int op = 0; op < kTpOps; ++op) {
      const int region = op >> 1, bi = 4 * (op & 1) + wu;
      const bf16* src = region == 2 ? a.wo + bi * 16 * HID + h0 + lane_o
                                    : (region ? a.wb : a.wa) + (h0 + bi * 4) * C + lane_ab[op & 1];
      __builtin_amdgcn_global_load_lds(
          (const __attribute__((address_space(1))) void*)src,
          (__attribute__((address_space(3))) void*)(base + region * 4096 + bi * 512), 16, 0, 0);
    }
  };
  issue(0);
  if (Q > 1) issue(1);

  auto row_of = [&](int64_t tile, int rb) -> int64_t {
    return tile * kTpRows + (kRB * w + rb) * 16 + r16;
  };
  RowSlots<ZT> xr[kRB];  // the rows of the tile about to start
  // per-lane row addresses are recomputed at each use (an opaque lane id)
  // rather than hoisted out of the tile loop, where they would be spilled
  auto lane_g = [&]() {
    int ll = lane_id();
    asm volatile("" : "+v"(ll));
    return ll >> 4;
  };
  auto load_rows = [&](int64_t tile) {
    const int gg = lane_g();
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int64_t row = min(row_of(tile, rb), a.rows - 1);  // pad rows read a real row
      xr[rb].load(a.x + row * C, gg);
    }
  };
  load_rows(blockIdx.x);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // GEMM1's output row m of half hb is hidden unit 8 (m >> 2) + 4 hb + (m & 3)
  // of the chunk: the W_a / W_b fragment row a lane reads (staged row `row`,
  // whose chunks are swizzled by key(row) = r16).  A lane's accumulator rows
  // 4g..4g+3 of the two halves are then the consecutive hidden units
  // 8g..8g+7, so GEMM2's W_o fragment is one 16-byte read.
  int sa_off[2];
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) sa_off[hb] = (8 * (r16 >> 2) + 4 * hb + (r16 & 3)) * C;
  const int so_sw = (r16 >> 2) & 3;
  const int so_ch = 8 * (r16 >> 2) + (r16 & 3);
  const float* ln_w = lnp;
  const float* ln_b = lnp + C;
  int q = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    // LayerNorm of the wave's rows (already in registers) into B fragments:
    // the statistics of every row block, then the normalisation one K32 step
    // at a time over the row blocks, so that a step's parameters (16
    // registers) are read once and die with it.  The rows themselves then
    // become the accumulators' initial values (the residual), in the
    // accumulator layout (block cb = slots 2t + k: channels 32t + 8g + 4k +
    // 0..3).
    Frag<bf16> xf[kRB][kC];
    float mean[kRB], rstd[kRB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      float x[kC][8];
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < kC; ++t) {
        xr[rb].get(t, x[t]);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[t][e];
      }
      mean[rb] = group_sum_fast(s) * (1.0f / C);
      float v = 0.f;
#pragma unroll
      for (int t = 0; t < kC; ++t)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = x[t][e] - mean[rb];
          v += d * d;
        }
      rstd[rb] = rsqrtf(group_sum_fast(v) * (1.0f / C) + a.eps);
    }
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      float lw[8], lb[8];
      load4(ln_w + 32 * t + 8 * g, lw);
      load4(ln_w + 32 * t + 8 * g + 4, lw + 4);
      load4(ln_b + 32 * t + 8 * g, lb);
      load4(ln_b + 32 * t + 8 * g + 4, lb + 4);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        // (x - mean) rstd lw + lb as x (rstd lw) + (lb - mean rstd lw), so that
        // no x - mean is kept from the variance pass (the rows stay live as
        // the residual; 32 more live values per row block would spill)
        const bool valid = row_of(tile, rb) < a.rows;
        float x[8];
        xr[rb].get(t, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float sc = rstd[rb] * lw[e];
          xf[rb][t].set(e, valid ? fmaf(x[e], sc, fmaf(-mean[rb], sc, lb[e])) : 0.f);
        }
      }
    }
    f32x4 acc[kRB][NCB];
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        if (!kAdd) {
          acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        } else if constexpr (sizeof(ZT) == 4) {
          acc[rb][cb] = xr[rb].c[cb];
        } else {
          const bf16x8 xv = __builtin_bit_cast(bf16x8, xr[rb].c[cb >> 1]);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][cb][e] = (float)xv[4 * (cb & 1) + e];
        }
      }

    for (int hc = 0; hc < NCHUNK; ++hc, ++q) {
      // This wave's loads of chunk q have landed: the loads of a tile's
      // chunks 0 and 1 (issued during the previous tile's last two chunks, or
      // before the first tile) were awaited at the tile boundary; from
      // hc == 2 on, only the loads of chunk q + 1 (kTpOps of them) were
      // issued after chunk q's.
      if (hc < 2) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      } else if (q + 1 < Q) {
        asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      }
      static_assert(kTpOps == 6, "the vmcnt above counts one chunk's loads");
      barrier_nofence();
      if (q + 2 < Q) issue(q + 2);
      const bf16* wa = ws[q % kTpStages];
      const bf16* wb = wa + 4096;
      const bf16* wo = wa + 8192;
      // GEMM1 per 16 hidden units (hb): each gate / value fragment pair of
      // hb serves both row blocks; silu(a) * b lands in slots 4hb..4hb+3 of
      // each row block's hidden fragment
      Frag<bf16> hf[kRB];
      // W_a / W_b fragments of step s = 4 hb + t, double buffered: step s + 1's
      // LDS reads are in flight while step s multiplies
      Frag<bf16> fa[2], fb[2];
      auto load_ab = [&](int s, int buf) {
        const int off = sa_off[s >> 2] + ((4 * (s & 3) + g) ^ r16) * 8;
        fa[buf].load(wa + off);
        fb[buf].load(wb + off);
      };
      load_ab(0, 0);
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        // raised issue priority while this wave feeds the matrix pipe, so
        // that with two waves per SIMD the MFMAs of one overlap the other's
        // gate arithmetic instead of queueing behind it
        __builtin_amdgcn_s_setprio(1);
        f32x4 sa[kRB], sb[kRB];
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) sa[rb] = sb[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < kC; ++t) {
          const int s = 4 * hb + t, buf = s & 1;
          if (s + 1 < 2 * kC) load_ab(s + 1, buf ^ 1);
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int rb = 0; rb < kRB; ++rb) {
            mma(sa[rb], fa[buf], xf[rb][t]);
            mma(sb[rb], fb[buf], xf[rb][t]);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            hf[rb].set(4 * hb + e,
                       (sa[rb][e] * sb[rb][e]) *
                           __builtin_amdgcn_rcpf(fmaf(__builtin_amdgcn_exp2f(sa[rb][e]),
                                                      kLog2eSq, kLog2eSq)));
      }
      // GEMM2: W_o[c][h0 + 8g .. + 7] fragments (staged chunk g, swizzled by
      // (c >> 3) & 3 = (r16 >> 2) & 3), one 16-channel block at a time, all
      // row blocks; fragment row r16 of block cb is channel
      // 32 (cb >> 1) + 8 (r16 >> 2) + 4 (cb & 1) + (r16 & 3)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        Frag<bf16> fo;
        fo.load(wo + (32 * (cb >> 1) + 4 * (cb & 1) + so_ch) * kTrHid + (g ^ so_sw) * 8);
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) mma(acc[rb][cb], fo, hf[rb]);
      }
    }
    // tile boundary.  The loads of the next tile's first two chunks (issued
    // during this tile's last two chunks) are the only vector memory
    // operations in flight: complete them here, before any row load, since
    // the next tile's first chunks only wait on lgkmcnt and the barrier.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // Then one row block at a time: store, form the pair bias from the stored
    // values, and load the block's rows of the next tile into the registers
    // just stored (their latency covered by the remaining blocks' epilogues).
    const int64_t next = tile + gridDim.x;
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb) {
      const int64_t row = row_of(tile, rb);
      const bool valid = row < a.rows;
      store_rows_pipe<ZT>(a.out + row * C, a.out + (row ^ 1) * C, acc[rb], valid,
                          (row ^ 1) < a.rows);
      if (kPb)
        pair_bias_folded<ZT>(a, acc[rb], row, valid, pbwf, pbb);
      {
        // after the last tile this reads row rows - 1 again, unused
        const int64_t nrow = min(row_of(next, rb), a.rows - 1);  // pad rows read a real row
        xr[rb].load(a.x + nrow * C, lane_g());
      }
    }
  }
  // the last tile's unused row loads complete before the wave ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// fp32 arithmetic (true fp32 products on v_mfma_f32_16x16x4_f32), any C in
// {64, 128, 256, 384}, n = 4.  A workgroup of 4 waves owns 16 rows at a time;
// every wave LayerNorms the 16 rows into K32 fragments (registers) and takes
// every fourth hidden chunk (wave w: chunks w, w + 4, ...), keeping a partial
// 16 x C output in registers.  Waves 1..3 hand their partials to wave 0
// through LDS, which sums them in a fixed order (deterministic), adds the
// residual, stores, and forms the pair bias from the stored values.  Weight
// fragments come straight from global memory: the whole weight set (12 C^2
// floats, <= 7 MB) stays resident in L2 and the rows of a workgroup read it
// once.  Splitting the hidden dimension over the waves keeps short row counts
// (the single track's N rows) spread over 4x more waves than a row split.
// For short row counts the hidden chunks are also split over gridDim.y
// workgroups (a.part set): each writes its partial 16 x C output to
// a.part[blockIdx.y], and transition_f32_reduce_kernel adds the partials in
// split order and the residual.
// kX3 (ODDE_F32X3): the products in three bf16 parts (rows and hidden
// activations split once, weight fragments as they are read).
template <typename ZT, int kC, bool kX3 = false>
__global__ __launch_bounds__(256) void transition_f32_kernel(TransitionArgs<ZT, float> a,
                                                             int64_t nblk) {
  constexpr int C = kC * 32, HID = 4 * C, NCB = C / 16, NCHUNK = HID / kTrHid;
  static_assert(NCHUNK % 4 == 0, "hidden chunks split evenly over the 4 waves");
  using MF = MulFrag<float, kX3>;
  __shared__ f32x4 part[3][NCB][64];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  for (int64_t b = blockIdx.x; b < nblk; b += gridDim.x) {
    const int64_t row = b * 16 + r16;
    const bool valid = row < a.rows;
    MF xf[kC];
    {
      Frag<float> xt[kC];
      ln_rows_to_frags<ZT, float, C>(a.x + (valid ? row : 0) * C, valid, a.ln_w, a.ln_b, a.eps,
                                     xt);
#pragma unroll
      for (int t = 0; t < kC; ++t) to_mul(xt[t], xf[t]);
    }
    f32x4 acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int per = NCHUNK / (int)gridDim.y;  // hidden chunks of this split
    for (int hc = (int)blockIdx.y * per + w; hc < ((int)blockIdx.y + 1) * per; hc += 4) {
      const int h0 = hc * kTrHid;
      // GEMM1 (W x^T orientation): lane (g, r16) ends with hidden units
      // h0 + 16 hb + 4g + e of row r16 -- slot 4 hb + e of a B fragment
      Frag<float> hf;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
#pragma unroll
        for (int t = 0; t < kC; ++t) {
          MF fa, fb;
          load_w_frag(a.wa, C, h0 + 16 * hb, HID, t, fa);
          load_w_frag(a.wb, C, h0 + 16 * hb, HID, t, fb);
          mma(sa, fa, xf[t]);
          mma(sb, fb, xf[t]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) hf.set(4 * hb + e, siluf_(sa[e]) * sb[e]);
      }
      MF hm;
      to_mul(hf, hm);
      // GEMM2: W_o[c][h0 + slot] with the same slot -> hidden map (three-part:
      // W_o split with its hidden units permuted within blocks of 32, so the
      // slots of lane group g are 8 consecutive units of the hi and lo rows)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        MF fm;
        if constexpr (kX3) {
          const bf16* w16 = reinterpret_cast<const bf16*>(a.wo) +
                            (size_t)(cb * 16 + r16) * 2 * HID + h0 + 8 * g;
          fm.hi.load(w16);
          fm.lo.load(w16 + HID);
        } else {
          const float* wrow = a.wo + (size_t)(cb * 16 + r16) * HID + h0;
          fm.lo = *reinterpret_cast<const f32x4*>(wrow + 4 * g);
          fm.hi = *reinterpret_cast<const f32x4*>(wrow + 16 + 4 * g);
        }
        mma(acc[cb], fm, hm);
      }
    }
    if (w) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) part[w - 1][cb][l] = acc[cb];
    }
    __syncthreads();
    if (w == 0 && a.part) {
      // this split's partial: lane holds row r16, channels cb*16 + 4g + e
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[cb] += part[k][cb][l];
        if (valid)
          *reinterpret_cast<f32x4*>(a.part + ((size_t)blockIdx.y * a.rows + row) * C + cb * 16 +
                                    4 * g) = acc[cb];
      }
    } else if (w == 0) {
      // lane holds row r16, channels cb*16 + 4g + e
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[cb] += part[k][cb][l];
        const int c0 = cb * 16 + 4 * g;
        float base[4] = {0.f, 0.f, 0.f, 0.f};
        if (valid && a.add) load4(a.x + row * C + c0, base);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[cb][e] += base[e];
        if (valid) store4(a.out + row * C + c0, acc[cb][0], acc[cb][1], acc[cb][2], acc[cb][3]);
      }
      if (a.pb_out)
        pair_bias_epilogue<ZT, float, kC>(a, acc, row, valid, a.pb_ln_w, a.pb_ln_b, a.pb_w);
    }
    __syncthreads();  // part is reused by the next row block
  }
}

// out = (add ? x : 0) + sum over splits of part[split] (split order), f32x4
// per thread over rows x C.
template <typename ZT>
__global__ __launch_bounds__(256) void transition_f32_reduce_kernel(TransitionArgs<ZT, float> a,
                                                                    int splits, int c) {
  const int64_t n4 = a.rows * c / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
    f32x4 v = a.add ? reinterpret_cast<const f32x4*>(a.x)[i] : f32x4{0.f, 0.f, 0.f, 0.f};
    for (int y = 0; y < splits; ++y) v += reinterpret_cast<const f32x4*>(a.part)[y * n4 + i];
    reinterpret_cast<f32x4*>(a.out)[i] = v;
  }
}

// fp32 arithmetic, pipelined form for C in {64, 128}, n = 4 (the pair
// transition in fp32 arithmetic).  Wave w of a workgroup of kW waves owns 16
// rows of a 16 kW-row tile (persistent over tiles), LayerNorms them into K32
// fragments in registers and walks the whole hidden dimension in chunks of
// 32; the chunk's W_a / W_b rows and W_o columns (fp32, 384 C bytes) stream
// into two LDS stages by direct global -> LDS loads, one chunk ahead, shared
// by every wave of the workgroup.  Against the unstaged fp32 form (16 rows
// per workgroup, weight fragments straight from L2) a weight byte fetched
// from L2 serves 16 kW rows instead of 16.  GEMM1 runs in W x^T orientation:
// lane (g, r16) ends with hidden units h0 + 16 hb + 4g + e of its row, slot
// 4 hb + e of GEMM2's B fragment.  LDS layouts (16-byte chunks): W_a / W_b
// chunk rows of C / 4 chunks, W_o rows (one per channel) of 8 chunks; chunk
// position p of row r holds chunk p ^ (r & 7), so the 8 rows that a group of
// 8 lanes reads at one chunk index land on 8 distinct 16-byte bank groups.
template <int kC>
struct TfStage {
  static constexpr int C = kC * 32;
  f32x4 wa[kTrHid * C / 4];  // [32 hidden][C / 4 chunks]
  f32x4 wb[kTrHid * C / 4];
  f32x4 wo[C * 8];           // [C][8 chunks of 4 hidden]
};

// kX3 (ODDE_F32X3): the products in three bf16 parts (rows and hidden
// activations split once, weight fragments as they are read from LDS).
template <typename ZT, int kC, int kW, bool kX3 = false>
__global__ __launch_bounds__(64 * kW) void transition_f32_pipe_kernel(TransitionArgs<ZT, float> a,
                                                                      int64_t ntiles) {
  constexpr int C = kC * 32, HID = 4 * C, NCB = C / 16, NCHUNK = HID / kTrHid;
  using MF = MulFrag<float, kX3>;
  constexpr int CPR = C / 4;                 // 16-byte chunks per W_a / W_b row
  constexpr int NAB = kTrHid * CPR / 64;     // direct loads per W_a (W_b) chunk
  constexpr int NO = C * 8 / 64;             // direct loads per W_o chunk
  constexpr int NOPS = 2 * NAB + NO;
  static_assert(NOPS % kW == 0, "every wave issues the same number of direct loads");
  __shared__ TfStage<kC> st[2];
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wu = __builtin_amdgcn_readfirstlane(w);

  // this workgroup's tiles; only loads that will be consumed are issued
  const int my_tiles =
      blockIdx.x < ntiles ? (int)((ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x) : 0;
  if (my_tiles == 0) return;
  const int Q = my_tiles * NCHUNK;
  // chunk q of the workgroup's sequence into stage q & 1: wave w issues ops
  // w, w + kW, ...; op < 2 NAB is 1 KiB of W_a (W_b) rows (lane l: row
  // (64 i + l) / CPR, position (64 i + l) % CPR), the rest 1 KiB of W_o
  // (lane l: channel 8 i + (l >> 3), position l & 7)
  auto issue = [&](int q) {
    const int h0 = (q % NCHUNK) * kTrHid;
    TfStage<kC>& S = st[q & 1];
#pragma unroll
    for (int j = 0; j < NOPS / kW; ++j) {
      const int op = wu + j * kW;
      const float* src;
      f32x4* dst;
      if (op < 2 * NAB) {
        const int m = op / NAB, i = op % NAB;
        const int idx = 64 * i + l, rr = idx / CPR, pos = idx % CPR;
        src = (m ? a.wb : a.wa) + (size_t)(h0 + rr) * C + (pos ^ (rr & 7)) * 4;
        dst = (m ? S.wb : S.wa) + 64 * i;
      } else {
        const int i = op - 2 * NAB;
        const int c = 8 * i + (l >> 3), sp = (l & 7) ^ (c & 7);
        // three-part: W_o rows of 2 HID bf16 (hi | lo, the same bytes per
        // row as f32); a chunk's 32 hidden units are 4 chunks of hi (sp < 4)
        // and 4 of lo
        if constexpr (kX3)
          src = a.wo + (size_t)c * HID + (sp < 4 ? h0 / 2 + sp * 4 : HID / 2 + h0 / 2 + (sp - 4) * 4);
        else
          src = a.wo + (size_t)c * HID + h0 + sp * 4;
        dst = S.wo + 64 * i;
      }
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)dst, 16, 0, 0);
    }
  };
  issue(0);

  const int key = r16 & 7;  // the swizzle key of every fragment row this lane reads
  int q = 0;
  for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
    const int64_t row = tile * (16 * kW) + 16 * w + r16;
    const bool valid = row < a.rows;
    MF xf[kC];
    {
      Frag<float> xt[kC];
      ln_rows_to_frags<ZT, float, C>(a.x + (valid ? row : 0) * C, valid, a.ln_w, a.ln_b, a.eps,
                                     xt);
#pragma unroll
      for (int t = 0; t < kC; ++t) to_mul(xt[t], xf[t]);
    }
    f32x4 acc[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int hc = 0; hc < NCHUNK; ++hc, ++q) {
      // this wave's loads of chunk q (its only vector memory operations in
      // flight) have landed and its reads of chunk q - 1 are done; the
      // barrier publishes chunk q and frees stage (q + 1) & 1 for chunk q + 1
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      barrier_nofence();
      if (q + 1 < Q) issue(q + 1);
      const TfStage<kC>& S = st[q & 1];
      Frag<float> hf;
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
        const int rr = 16 * hb + r16;
#pragma unroll
        for (int t = 0; t < kC; ++t) {
          MF ma, mb;
          if constexpr (kX3) {
            // rows of C / 8 hi chunks, then C / 8 lo chunks
            ma.hi.v = as_bf16x8(S.wa[rr * CPR + ((4 * t + g) ^ key)]);
            ma.lo.v = as_bf16x8(S.wa[rr * CPR + ((C / 8 + 4 * t + g) ^ key)]);
            mb.hi.v = as_bf16x8(S.wb[rr * CPR + ((4 * t + g) ^ key)]);
            mb.lo.v = as_bf16x8(S.wb[rr * CPR + ((C / 8 + 4 * t + g) ^ key)]);
          } else {
            ma.lo = S.wa[rr * CPR + ((8 * t + 2 * g) ^ key)];
            ma.hi = S.wa[rr * CPR + ((8 * t + 2 * g + 1) ^ key)];
            mb.lo = S.wb[rr * CPR + ((8 * t + 2 * g) ^ key)];
            mb.hi = S.wb[rr * CPR + ((8 * t + 2 * g + 1) ^ key)];
          }
          mma(sa, ma, xf[t]);
          mma(sb, mb, xf[t]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) hf.set(4 * hb + e, siluf_(sa[e]) * sb[e]);
      }
      MF hm;
      to_mul(hf, hm);
      // GEMM2: W_o[c][h0 + 4g .. + 3] and [h0 + 16 + 4g .. + 3] (chunks g, 4 + g)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const int c = 16 * cb + r16;
        MF mo;
        if constexpr (kX3) {
          // hi chunk g and lo chunk g: hidden units 4g .. 4g+3, 16+4g .. +3
          mo.hi.v = as_bf16x8(S.wo[c * 8 + (g ^ key)]);
          mo.lo.v = as_bf16x8(S.wo[c * 8 + ((4 + g) ^ key)]);
        } else {
          mo.lo = S.wo[c * 8 + (g ^ key)];
          mo.hi = S.wo[c * 8 + ((4 + g) ^ key)];
        }
        mma(acc[cb], mo, hm);
      }
    }
    // epilogue: lane holds row r16 of the wave, channels 16 cb + 4g + e
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int c0 = cb * 16 + 4 * g;
      float base[4] = {0.f, 0.f, 0.f, 0.f};
      if (valid && a.add) load4(a.x + row * C + c0, base);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[cb][e] += base[e];
      if (valid) store4(a.out + row * C + c0, acc[cb][0], acc[cb][1], acc[cb][2], acc[cb][3]);
    }
    if (a.pb_out)
      pair_bias_epilogue<ZT, float, kC>(a, acc, row, valid, a.pb_ln_w, a.pb_ln_b, a.pb_w);
  }
  // the last chunk's loads were all consumed; nothing is in flight
}

// Wide form (C = 384): a LayerNorm pass into bf16 rows, then two NT GEMMs on
// the shared mainloop (gemm.hpp) with the hidden activations in the
// workspace:  h = silu(y W_a^T) * (y W_b^T)  ([Mp][4C] bf16), then
// out = (add ? x : 0) + h W_o^T.  GEMM1 reads W_a / W_b rows interleaved in
// 16-row blocks, so a wave's fragments j (gate) and j + 1 (value) hold the
// same 16 hidden units.  Rows are padded to whole groups of 8 row tiles;
// rows past `rows` are never stored.
__global__ void fill_zero_kernel(float* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0.f;
}

// Pair-bias projection of the rows as written (the fused kernels do this in
// their epilogue): 16 rows per wave, each lane loads its K32 fragment slots of
// a row, LayerNorm statistics over the four lanes of the row, then 16 heads
// by MFMA against pb_w; pb_out[h][r] = sum_c LN'(out[r])[c] pb_w[h][c].
template <typename ZT, int kC>
__global__ __launch_bounds__(256) void transition_pair_bias_kernel(TransitionArgs<ZT, bf16> a) {
  constexpr int C = kC * 32;
  const int l = lane_id(), g = l >> 4, r16 = l & 15;
  const int64_t nblk = (a.rows + 15) / 16;
  Frag<bf16> wf[kC];
#pragma unroll
  for (int t = 0; t < kC; ++t) load_w_frag(a.pb_w, C, 0, 16, t, wf[t]);
  for (int64_t b = int64_t(blockIdx.x) * 4 + wave_id(); b < nblk; b += int64_t(gridDim.x) * 4) {
    const int64_t row = b * 16 + r16;
    const bool valid = row < a.rows;
    Frag<bf16> yf[kC];
    ln_rows_to_frags<ZT, bf16, C>(a.out + (valid ? row : 0) * C, valid, a.pb_ln_w,
                                  a.pb_ln_b ? a.pb_ln_b : a.pb_zero, a.pb_eps, yf);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) mma(acc, wf[t], yf[t]);
    if (valid) {
#pragma unroll
      for (int e = 0; e < 4; ++e) a.pb_out[(size_t)(4 * g + e) * a.rows + row] = acc[e];
    }
  }
}

constexpr int kTwTX = 256, kTwTY = 128, kTwWX = 4, kTwNS = 3, kTwKC = 32;
using TwShape = GemmShape<kTwTX, kTwTY, kTwWX, kTwKC>;

__device__ __forceinline__ void tw_tile_map(int L, int ncol, int& rt, int& ct) {
  const int xcd = L & 7, s = L >> 3;  // all column tiles of a row tile on one XCD
  rt = xcd + 8 * (s / ncol);
  ct = s % ncol;
}

template <int TX, int TY = kTwTY, int KC = kTwKC>
__global__ __launch_bounds__(512) void transition_wide_gate_kernel(const bf16* __restrict__ yn,
                                                                   const bf16* __restrict__ wa,
                                                                   const bf16* __restrict__ wb,
                                                                   bf16* __restrict__ h, int C,
                                                                   int ncol) {
  using TwShape = GemmShape<TX, TY, kTwWX, KC>;
  constexpr int NS = KC == 64 ? 2 : kTwNS;
  __shared__ __attribute__((aligned(16))) bf16 sm[NS * TwShape::STAGE_ELEMS];
  int rt, ct;
  tw_tile_map(blockIdx.x, ncol, rt, ct);
  const int64_t x0 = (int64_t)rt * TX;
  const int y0 = ct * TY, HID = 4 * C;
  f32x4 acc[TwShape::MX][TwShape::MY];
  auto arow = [&](int r) { return yn + (x0 + r) * C; };
  // Columns come in 32-wide groups q = R >> 5: 16 of W_a then the same 16
  // hidden units of W_b.  With 256-wide tiles (a wave's 128 columns = 64
  // hidden units, one 128-byte line of h per row) group q's column n is
  // hidden unit 64 (q >> 2) + 32 ((q >> 1) & 1) + 8 (n >> 2) + 4 (q & 1) +
  // (n & 3), so that a lane's groups 2k and 2k + 1 are 8 consecutive units;
  // otherwise 16 (q) + n.
  constexpr bool kLines = TY == 256;
  auto brow = [&](int r) {
    const int R = y0 + r, t = R & 31, q = R >> 5, nn = t & 15;
    const int hid = kLines ? 64 * (q >> 2) + 32 * ((q >> 1) & 1) + 8 * (nn >> 2) + 4 * (q & 1) +
                                 (nn & 3)
                           : q * 16 + nn;
    return (t < 16 ? wa : wb) + (size_t)hid * C;
  };
  if constexpr (KC == 64)
    gemm_nt_mainloop_pipe64<TX, TY, kTwWX, true>(arow, brow, C, sm, acc);
  else
    gemm_nt_mainloop<TX, TY, kTwWX, NS, true, KC>(arow, brow, C, sm, acc);
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kTwWX, wy = w / kTwWX;
#pragma unroll
  for (int i = 0; i < TwShape::MX; ++i) {
    const int64_t m = x0 + wx * (TX / kTwWX) + 16 * i + r16;
    if constexpr (kLines) {
      // hidden units 64 (2 ct + wy) + 8g .. + 7 (slot g of row m's line) from
      // groups 0, 1 of the wave, the same + 32 (slot 4 + g) from groups 2, 3;
      // rows m and m ^ 1 (lanes r16, r16 ^ 1) complete each other's lines
      static_assert(TwShape::MY == 8, "four column groups per wave");
      bf16x8 v[2];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * hh;
          v[hh][e] = (bf16)(siluf_(acc[i][j][e]) * acc[i][j + 1][e]);
          v[hh][4 + e] = (bf16)(siluf_(acc[i][j + 2][e]) * acc[i][j + 3][e]);
        }
      const int hb = (y0 + wy * (TY / TwShape::WY)) / 2;  // the wave's first hidden unit
      store_line_pair(reinterpret_cast<bf16x8*>(h + m * HID + hb),
                      reinterpret_cast<bf16x8*>(h + (m ^ 1) * HID + hb), g, v[0], v[1]);
    } else {
#pragma unroll
      for (int j = 0; j < TwShape::MY; j += 2) {
        const int hid = ((y0 + wy * (TY / TwShape::WY) + 16 * j) >> 5) * 16 + 4 * g;
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(siluf_(acc[i][j][e]) * acc[i][j + 1][e]);
        *reinterpret_cast<bf16x4*>(h + m * HID + hid) = v;
      }
    }
  }
}

// kSplit > 1: workgroup column ks of the grid (blockIdx.y) takes hidden
// units [ks HID / kSplit, (ks + 1) HID / kSplit) and writes its fp32 partial
// sums to part[ks][m][c] (rows of the padded tile range); the residual is
// added by transition_wide_reduce_kernel, which sums the partials in order.
template <typename ZT, int TX, int kSplit>
__global__ __launch_bounds__(512) void transition_wide_out_kernel(const bf16* __restrict__ h,
                                                                  const bf16* __restrict__ wo,
                                                                  const ZT* x, ZT* out,
                                                                  float* __restrict__ part,
                                                                  int64_t rows, int64_t mp,
                                                                  int C, int add, int ncol) {
  using TwShape = GemmShape<TX, kTwTY, kTwWX, kTwKC>;
  __shared__ __attribute__((aligned(16))) bf16 sm[kTwNS * TwShape::STAGE_ELEMS];
  int rt, ct;
  tw_tile_map(blockIdx.x, ncol, rt, ct);
  const int64_t x0 = (int64_t)rt * TX;
  const int y0 = ct * kTwTY, HID = 4 * C, KS = HID / kSplit, k0 = (int)blockIdx.y * KS;
  f32x4 acc[TwShape::MX][TwShape::MY];
  gemm_nt_mainloop<TX, kTwTY, kTwWX, kTwNS, true, kTwKC>(
      [&](int r) { return h + (x0 + r) * HID + k0; },
      [&](int r) { return wo + (size_t)(y0 + r) * HID + k0; }, KS, sm, acc);
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int wx = w % kTwWX, wy = w / kTwWX;
#pragma unroll
  for (int i = 0; i < TwShape::MX; ++i) {
    const int64_t m = x0 + wx * (TX / kTwWX) + 16 * i + r16;
    if constexpr (kSplit > 1) {
      if (m >= rows) continue;
#pragma unroll
      for (int j = 0; j < TwShape::MY; ++j) {
        const int c0 = y0 + wy * (kTwTY / TwShape::WY) + 16 * j + 4 * g;
        store4(part + ((int64_t)blockIdx.y * mp + m) * C + c0, acc[i][j][0], acc[i][j][1],
               acc[i][j][2], acc[i][j][3]);
      }
    } else {
      // rows m and m ^ 1 (lanes r16, r16 ^ 1) complete each other's lines
      const bool ok = m < rows, pok = (m ^ 1) < rows;
      float r[TwShape::MY][4];
#pragma unroll
      for (int j = 0; j < TwShape::MY; ++j) {
        const int c0 = y0 + wy * (kTwTY / TwShape::WY) + 16 * j + 4 * g;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[j][e] = 0.f;
        if (add && ok) load4(x + m * C + c0, r[j]);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[j][e] += acc[i][j][e];
      }
      store_row_blocks<ZT>(out + m * C, out + (m ^ 1) * C, y0 + wy * (kTwTY / TwShape::WY), r,
                           ok, pok);
    }
  }
}

// out = (add ? x : 0) + sum over ks of part[ks] (in ks order: deterministic),
// four channels per thread.
template <typename ZT, int kSplit>
__global__ __launch_bounds__(256) void transition_wide_reduce_kernel(const float* __restrict__ part,
                                                                     const ZT* x, ZT* out,
                                                                     int64_t rows, int64_t mp,
                                                                     int C, int add) {
  const int64_t n4 = rows * C / 4;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * 256) {
    float r[4] = {0.f, 0.f, 0.f, 0.f};
    if (add) load4(x + 4 * i, r);
#pragma unroll
    for (int ks = 0; ks < kSplit; ++ks) {
      const f32x4 p = *reinterpret_cast<const f32x4*>(part + ks * mp * C + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] += p[e];
    }
    store4(out + 4 * i, r[0], r[1], r[2], r[3]);
  }
}

}  // namespace odde

using namespace odde;

namespace {

template <typename ZT, typename CT, int kC, int NF>
void launch_tr(const TransitionArgs<ZT, CT>& p, hipStream_t st) {
  const int64_t ntiles = (p.rows + kTrRows - 1) / kTrRows;
  const int grid = (int)std::min<int64_t>(ntiles, 2 * 256);
  hipLaunchKernelGGL((transition_kernel<ZT, CT, kC, NF>), dim3(grid), dim3(256), 0, st, p, ntiles);
}

bool transition_wide(int c, int nf, int dt) { return dt == ODDE_BF16 && c == 384 && nf == 4; }
// Up to kTwSmallRows rows (the single track) the GEMMs take 128-row tiles
// and the output GEMM splits the hidden dimension kTwSplit ways, so that a
// few hundred rows still fill the GPU; tile rows are padded to whole groups
// of 8 row tiles (tw_tile_map).
constexpr int64_t kTwSmallRows = 16384;
constexpr int kTwSplit = 4;
bool transition_wide_small(int64_t rows) { return rows <= kTwSmallRows; }
int64_t transition_wide_rows(int64_t rows) {
  const int64_t q = transition_wide_small(rows) ? 8 * 128 : 8 * kTwTX;
  return (rows + q - 1) / q * q;
}
// fp32 arithmetic with few rows (fewer than 512 blocks of 16): the hidden
// chunks split over S workgroups per row block, S the largest divisor of
// the chunks per wave (4C / 32 / 4) that keeps the grid within 1024
// workgroups.  1: no split.  Not with the pair-bias epilogue.
int transition_f32_splits(const odde_transition_args* a) {
  if ((a->compute_dtype != ODDE_F32 && a->compute_dtype != ODDE_F32X3) || a->n_factor != 4 ||
      a->pb_heads)
    return 1;
  if (a->c != 64 && a->c != 128 && a->c != 256 && a->c != 384) return 1;
  const int64_t nblk = (a->rows + 15) / 16;
  if (nblk >= 512 || nblk == 0) return 1;
  const int per_wave = a->c / 32;  // 4C / 32 chunks over 4 waves
  int best = 1;
  for (int d = 1; d <= per_wave; ++d)
    if (per_wave % d == 0 && nblk * d <= 1024) best = d;
  return best;
}

// ODDE_F32X3: W_a, W_b and W_o split once per call into bf16 hi | lo rows
uint64_t transition_split_bytes(const odde_transition_args* a) {
  return a->compute_dtype == ODDE_F32X3 ? (uint64_t)3 * a->n_factor * a->c * a->c * 4 : 0;
}
// fp32 workspace: the split-hidden partial sums, then the split weights
uint64_t transition_part_bytes(const odde_transition_args* a) {
  const int splits = transition_f32_splits(a);
  if (splits <= 1) return 0;
  return ((uint64_t)splits * (uint64_t)a->rows * (uint64_t)a->c * 4 + 255) & ~uint64_t(255);
}
uint64_t transition_ws_bytes(const odde_transition_args* a) {
  const uint64_t f32 = transition_part_bytes(a) + transition_split_bytes(a);
  if (f32) return f32 + 256;
  if (!transition_wide(a->c, a->n_factor, a->compute_dtype)) return 0;
  // normalised rows [Mp][C] and hidden activations [Mp][4C], bf16; with the
  // split output GEMM its fp32 partial sums [kTwSplit][Mp][C]
  const uint64_t mp = (uint64_t)transition_wide_rows(a->rows);
  const uint64_t part = transition_wide_small(a->rows) ? (uint64_t)kTwSplit * mp * a->c * 4 : 0;
  return mp * 5 * a->c * 2 + part + 256;
}

template <typename ZT>
int run_transition_wide(const odde_transition_args* a, hipStream_t st) {
  const int C = a->c;
  const int64_t rows = a->rows, mp = transition_wide_rows(rows);
  bf16* yn = static_cast<bf16*>(a->workspace);
  bf16* h = yn + mp * C;
  LaunchScope ls(ODDE_K_TRANSITION, st);
  const int lg = (int)std::min<int64_t>((rows + 15) / 16, 4096);
  // rows as one view row of length `rows` (x = 0, y = row)
  hipLaunchKernelGGL((ln_view_bf16_kernel<ZT, 384>), dim3(lg), dim3(256), 0, st,
                     static_cast<const ZT*>(a->x), (int64_t)0, (int64_t)C, (int)rows, 1,
                     (int)rows, a->ln_w, a->ln_b, a->eps, yn);
  const int ncol1 = 8 * C / kTwTY, ncol2 = C / kTwTY;
  const bf16* wa = static_cast<const bf16*>(a->w_a);
  const bf16* wb = static_cast<const bf16*>(a->w_b);
  const bf16* wo = static_cast<const bf16*>(a->w_o);
  const ZT* x = static_cast<const ZT*>(a->x);
  ZT* out = static_cast<ZT*>(a->out);
  if (transition_wide_small(rows)) {
    const int row_tiles = (int)(mp / 128);
    float* part = reinterpret_cast<float*>(h + mp * 4 * C);
    hipLaunchKernelGGL(transition_wide_gate_kernel<128>, dim3(row_tiles * ncol1), dim3(512), 0, st,
                       yn, wa, wb, h, C, ncol1);
    hipLaunchKernelGGL((transition_wide_out_kernel<ZT, 128, kTwSplit>),
                       dim3(row_tiles * ncol2, kTwSplit), dim3(512), 0, st, h, wo, x, out, part,
                       rows, mp, C, a->add_residual, ncol2);
    const int rg = (int)std::min<int64_t>((rows * C / 4 + 255) / 256, 2048);
    hipLaunchKernelGGL((transition_wide_reduce_kernel<ZT, kTwSplit>), dim3(rg), dim3(256), 0, st,
                       part, x, out, rows, mp, C, a->add_residual);
  } else {
    // the gate GEMM (N = 8C): 256 x 256 tiles, 64-k pipelined stages (each
    // wave 64 x 128, fewer LDS bytes per MFMA than 256 x 128 tiles)
    const int row_tiles = (int)(mp / kTwTX), ncol1w = 8 * C / 256;
    hipLaunchKernelGGL((transition_wide_gate_kernel<kTwTX, 256, 64>), dim3(row_tiles * ncol1w),
                       dim3(512), 0, st, yn, wa, wb, h, C, ncol1w);
    hipLaunchKernelGGL((transition_wide_out_kernel<ZT, kTwTX, 1>), dim3(row_tiles * ncol2),
                       dim3(512), 0, st, h, wo, x, out, nullptr, rows, mp, C, a->add_residual,
                       ncol2);
  }
  if (a->pb_heads) {
    TransitionArgs<ZT, bf16> p;
    p.out = static_cast<ZT*>(a->out);
    p.rows = rows;
    p.pb_ln_w = a->pb_ln_w;
    p.pb_ln_b = a->pb_ln_b;
    p.pb_w = static_cast<const bf16*>(a->pb_w);
    p.pb_out = a->pb_out;
    p.pb_eps = a->pb_eps;
    // without an LN bias the kernel reads a row of zeros, written into the
    // hidden buffer (no longer needed once the output GEMM has run)
    float* zero = reinterpret_cast<float*>(h);
    if (!a->pb_ln_b) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(1), dim3(256), 0, st, zero, C);
      p.pb_zero = zero;
    } else {
      p.pb_zero = a->pb_ln_b;
    }
    const int grid = (int)std::min<int64_t>((rows + 63) / 64, 4096);
    hipLaunchKernelGGL((transition_pair_bias_kernel<ZT, 12>), dim3(grid), dim3(256), 0, st, p);
  }
  return check_launch("transition (wide)");
}

// kX3: the products in three bf16 parts (ODDE_F32X3)
template <bool kX3>
int run_transition_f32(const odde_transition_args* a, hipStream_t st) {
  TransitionArgs<float, float> p;
  p.x = static_cast<const float*>(a->x);
  p.out = static_cast<float*>(a->out);
  p.ln_w = a->ln_w; p.ln_b = a->ln_b;
  p.wa = static_cast<const float*>(a->w_a);
  p.wb = static_cast<const float*>(a->w_b);
  p.wo = static_cast<const float*>(a->w_o);
  p.rows = a->rows; p.add = a->add_residual; p.eps = a->eps;
  p.pb_ln_w = a->pb_ln_w; p.pb_ln_b = a->pb_ln_b;
  p.pb_w = static_cast<const float*>(a->pb_w);
  p.pb_out = a->pb_heads ? a->pb_out : nullptr;
  p.pb_eps = a->pb_eps;
  p.pb_zero = nullptr;
  const int64_t nblk = (p.rows + 15) / 16;
  const int grid = (int)std::min<int64_t>(nblk, 8 * 256);
  if constexpr (kX3) {
    // the weights as bf16 hi | lo rows (W_o's hidden units permuted within
    // blocks of 32), split once for this call
    const int C = a->c, HID = a->n_factor * a->c;
    char* d = static_cast<char*>(a->workspace) + transition_part_bytes(a);
    launch_split_x3(a->w_a, HID, C, d, false, st);
    p.wa = reinterpret_cast<const float*>(d);
    d += (size_t)HID * C * 4;
    launch_split_x3(a->w_b, HID, C, d, false, st);
    p.wb = reinterpret_cast<const float*>(d);
    d += (size_t)HID * C * 4;
    launch_split_x3(a->w_o, C, HID, d, true, st);
    p.wo = reinterpret_cast<const float*>(d);
  }
  LaunchScope ls(ODDE_K_TRANSITION, st);
  // the staged form when its tiles fill the GPU and the weights can be
  // staged by 16-byte direct loads
  const bool aligned16 = ((reinterpret_cast<uintptr_t>(p.wa) | reinterpret_cast<uintptr_t>(p.wb) |
                           reinterpret_cast<uintptr_t>(p.wo)) & 15) == 0;
  if (aligned16 && a->n_factor == 4 && (a->c == 64 || a->c == 128) && p.rows >= 256 * 64) {
    if (p.rows >= 256 * 128) {  // 8 waves (128 rows) per workgroup, 2 per SIMD
      const int64_t ntiles = (p.rows + 127) / 128;
      const int g2 = (int)std::min<int64_t>(ntiles, a->c == 64 ? 2 * 256 : 256);
      if (a->c == 64)
        hipLaunchKernelGGL((transition_f32_pipe_kernel<float, 2, 8, kX3>), dim3(g2), dim3(512), 0, st, p, ntiles);
      else
        hipLaunchKernelGGL((transition_f32_pipe_kernel<float, 4, 8, kX3>), dim3(g2), dim3(512), 0, st, p, ntiles);
    } else {  // 4 waves (64 rows) per workgroup: more workgroups for fewer rows
      const int64_t ntiles = (p.rows + 63) / 64;
      const int g2 = (int)std::min<int64_t>(ntiles, a->c == 64 ? 3 * 256 : 256);
      if (a->c == 64)
        hipLaunchKernelGGL((transition_f32_pipe_kernel<float, 2, 4, kX3>), dim3(g2), dim3(256), 0, st, p, ntiles);
      else
        hipLaunchKernelGGL((transition_f32_pipe_kernel<float, 4, 4, kX3>), dim3(g2), dim3(256), 0, st, p, ntiles);
    }
    return check_launch("transition (fp32)");
  }
  const int splits = transition_f32_splits(a);
  if (splits > 1) {
    const uint64_t need = (uint64_t)splits * (uint64_t)p.rows * (uint64_t)a->c * 4;
    if (!a->workspace || a->workspace_bytes < need || (reinterpret_cast<uintptr_t>(a->workspace) & 15))
      return set_error(ODDE_EINVAL, "transition (fp32, split hidden): workspace missing or too small");
    p.part = static_cast<float*>(a->workspace);
    const dim3 g3((unsigned)nblk, (unsigned)splits);
    switch (a->c) {
      case 64: hipLaunchKernelGGL((transition_f32_kernel<float, 2, kX3>), g3, dim3(256), 0, st, p, nblk); break;
      case 128: hipLaunchKernelGGL((transition_f32_kernel<float, 4, kX3>), g3, dim3(256), 0, st, p, nblk); break;
      case 256: hipLaunchKernelGGL((transition_f32_kernel<float, 8, kX3>), g3, dim3(256), 0, st, p, nblk); break;
      default: hipLaunchKernelGGL((transition_f32_kernel<float, 12, kX3>), g3, dim3(256), 0, st, p, nblk); break;
    }
    const int64_t n4 = p.rows * a->c / 4;
    const int rg = (int)std::min<int64_t>((n4 + 255) / 256, 1024);
    hipLaunchKernelGGL((transition_f32_reduce_kernel<float>), dim3(rg), dim3(256), 0, st, p, splits,
                       a->c);
    return check_launch("transition (fp32, split hidden)");
  }
  switch (a->c) {
    case 64: hipLaunchKernelGGL((transition_f32_kernel<float, 2, kX3>), dim3(grid), dim3(256), 0, st, p, nblk); break;
    case 128: hipLaunchKernelGGL((transition_f32_kernel<float, 4, kX3>), dim3(grid), dim3(256), 0, st, p, nblk); break;
    case 256: hipLaunchKernelGGL((transition_f32_kernel<float, 8, kX3>), dim3(grid), dim3(256), 0, st, p, nblk); break;
    case 384: hipLaunchKernelGGL((transition_f32_kernel<float, 12, kX3>), dim3(grid), dim3(256), 0, st, p, nblk); break;
    default: return set_error(ODDE_EUNSUPPORTED, "transition: c in {64, 128, 256, 384} with n = 4");
  }
  return check_launch("transition (fp32)");
}

template <typename ZT, typename CT>
int run_transition(const odde_transition_args* a, hipStream_t st) {
  if (transition_wide(a->c, a->n_factor, a->compute_dtype)) return run_transition_wide<ZT>(a, st);
  TransitionArgs<ZT, CT> p;
  p.x = static_cast<const ZT*>(a->x);
  p.out = static_cast<ZT*>(a->out);
  p.ln_w = a->ln_w; p.ln_b = a->ln_b;
  p.wa = static_cast<const CT*>(a->w_a);
  p.wb = static_cast<const CT*>(a->w_b);
  p.wo = static_cast<const CT*>(a->w_o);
  p.rows = a->rows; p.add = a->add_residual; p.eps = a->eps;
  p.pb_ln_w = a->pb_ln_w; p.pb_ln_b = a->pb_ln_b;
  p.pb_w = static_cast<const CT*>(a->pb_w);
  p.pb_out = a->pb_heads ? a->pb_out : nullptr;
  p.pb_eps = a->pb_eps;
  LaunchScope ls(ODDE_K_TRANSITION, st);
  if (a->c == 128 && a->n_factor == 4) {
    const int64_t ntiles = (p.rows + kTpRows - 1) / kTpRows;
    const int grid = (int)std::min<int64_t>(ntiles, 2 * 256);
    const bool pb = p.pb_out != nullptr;
    if (p.add && pb)
      hipLaunchKernelGGL((transition_pipe_kernel<ZT, true, true>), dim3(grid), dim3(256), 0, st, p,
                         ntiles);
    else if (p.add)
      hipLaunchKernelGGL((transition_pipe_kernel<ZT, true, false>), dim3(grid), dim3(256), 0, st,
                         p, ntiles);
    else if (pb)
      hipLaunchKernelGGL((transition_pipe_kernel<ZT, false, true>), dim3(grid), dim3(256), 0, st,
                         p, ntiles);
    else
      hipLaunchKernelGGL((transition_pipe_kernel<ZT, false, false>), dim3(grid), dim3(256), 0, st,
                         p, ntiles);
  }
  else if (a->c == 64 && a->n_factor == 4) launch_tr<ZT, CT, 2, 4>(p, st);
  else if (a->c == 256 && a->n_factor == 4) launch_tr<ZT, CT, 8, 4>(p, st);
  else return set_error(ODDE_EUNSUPPORTED, "transition: c in {64, 128, 256, 384} with n = 4");
  return check_launch("transition");
}

}  // namespace

extern "C" {

int odde_transition_workspace_bytes(const odde_transition_args* a, uint64_t* bytes) {
  if (!a || !bytes) return set_error(ODDE_EINVAL, "transition: null argument");
  if (a->struct_size != sizeof(odde_transition_args))
    return set_error(ODDE_EINVAL, "transition: struct_size mismatch (ABI version skew)");
  if (a->rows < 0 || a->c <= 0 || a->n_factor <= 0)
    return set_error(ODDE_EINVAL, "transition: bad sizes");
  *bytes = transition_ws_bytes(a);
  return ODDE_OK;
}

int odde_transition_fwd(const odde_transition_args* a, void* stream) {
  if (!a) return set_error(ODDE_EINVAL, "transition: null args");
  if (a->struct_size != sizeof(odde_transition_args))
    return set_error(ODDE_EINVAL, "transition: struct_size mismatch (ABI version skew)");
  if (a->rows < 0 || a->c <= 0 || a->n_factor <= 0)
    return set_error(ODDE_EINVAL, "transition: bad sizes");
  if (a->rows >= (int64_t(1) << 31))
    return set_error(ODDE_EUNSUPPORTED, "transition: at most 2^31 - 1 rows per call");
  if (!valid_dtype(a->x_dtype) ||
      !(valid_dtype(a->compute_dtype) || a->compute_dtype == ODDE_F32X3))
    return set_error(ODDE_EINVAL, "transition: bad dtype");
  if ((a->compute_dtype == ODDE_F32 || a->compute_dtype == ODDE_F32X3) && a->x_dtype != ODDE_F32)
    return set_error(ODDE_EUNSUPPORTED, "transition: fp32 arithmetic needs float32 rows");
  if (a->n_factor != 4 || (a->c != 64 && a->c != 128 && a->c != 256 && a->c != 384))
    return set_error(ODDE_EUNSUPPORTED, "transition: c in {64, 128, 256, 384} with n = 4");
  if (!a->x || !a->out || !a->ln_w || !a->ln_b || !a->w_a || !a->w_b || !a->w_o)
    return set_error(ODDE_EINVAL, "transition: null tensor pointer");
  if ((reinterpret_cast<uintptr_t>(a->x) | reinterpret_cast<uintptr_t>(a->out)) & 15)
    return set_error(ODDE_EINVAL, "transition: x/out must be 16-byte aligned");
  const uint64_t need = transition_ws_bytes(a);
  if (need && a->rows > 0 && (!a->workspace || a->workspace_bytes < need))
    return set_error(ODDE_EWORKSPACE, "transition: workspace too small");
  if (need && (reinterpret_cast<uintptr_t>(a->workspace) & 255))
    return set_error(ODDE_EWORKSPACE, "transition: workspace must be 256-byte aligned");
  if (a->pb_heads != 0) {
    if (a->pb_heads != 16)
      return set_error(ODDE_EUNSUPPORTED, "transition: pair-bias projection needs 16 heads");
    if (!a->pb_ln_w || !a->pb_w || !a->pb_out)
      return set_error(ODDE_EINVAL, "transition: null pair-bias pointer");
    if ((reinterpret_cast<uintptr_t>(a->pb_ln_w) | reinterpret_cast<uintptr_t>(a->pb_ln_b) |
         reinterpret_cast<uintptr_t>(a->pb_w)) & 15)
      return set_error(ODDE_EINVAL, "transition: pair-bias parameters must be 16-byte aligned");
  }
  if (a->rows == 0) return ODDE_OK;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->compute_dtype == ODDE_F32) return run_transition_f32<false>(a, st);
  if (a->compute_dtype == ODDE_F32X3) return run_transition_f32<true>(a, st);
  if (a->x_dtype == ODDE_F32) return run_transition<float, bf16>(a, st);
  return run_transition<bf16, bf16>(a, st);
}

}  // extern "C"
