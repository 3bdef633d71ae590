// Shared device helpers for the gfx950 (CDNA4) pair-stack kernels.
//
// Everything here is built around one MFMA tile: the 16x16 output block with
// a 32-deep contraction ("K32 fragment").  Lane l of a wave64 holds
//   * for an A operand: row (l % 16), eight contraction slots of group l / 16;
//   * for a B operand: column (l % 16), the same eight slots of group l / 16;
//   * for the f32x4 accumulator: column (l % 16), rows 4 * (l / 16) + r.
// Only the row/column ownership and the accumulator layout are relied upon:
// A and B always use the same slot -> contraction-index map, so the order in
// which the hardware walks the 32 slots does not matter.
//
// bf16 fragments feed v_mfma_f32_16x16x32_bf16 (one instruction); f32
// fragments feed eight v_mfma_f32_16x16x4_f32 (slot e of every group in
// instruction e), giving true fp32 products for the fp32 tier.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace odde {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// ----------------------------------------------------------------------------
// scalar conversions
// ----------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <> __device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
// x rounded to T's precision and widened back
template <typename T> __device__ __forceinline__ float round_to(float x) { return (float)from_f32<T>(x); }

// ----------------------------------------------------------------------------
// K32 fragments
// ----------------------------------------------------------------------------
template <typename CT> struct Frag;

template <> struct Frag<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void zero() {
    for (int e = 0; e < 8; ++e) v[e] = (bf16)0.0f;
  }
  __device__ __forceinline__ void load(const bf16* p) { v = *reinterpret_cast<const bf16x8*>(p); }
  __device__ __forceinline__ void set(int e, float x) { v[e] = (bf16)x; }
  __device__ __forceinline__ float get(int e) const { return (float)v[e]; }
};

template <> struct Frag<float> {
  f32x4 lo, hi;
  __device__ __forceinline__ void zero() {
    lo = f32x4{0.f, 0.f, 0.f, 0.f};
    hi = lo;
  }
  __device__ __forceinline__ void load(const float* p) {
    lo = *reinterpret_cast<const f32x4*>(p);
    hi = *reinterpret_cast<const f32x4*>(p + 4);
  }
  __device__ __forceinline__ void set(int e, float x) {
    if (e < 4) lo[e] = x; else hi[e - 4] = x;
  }
  __device__ __forceinline__ float get(int e) const { return e < 4 ? lo[e] : hi[e - 4]; }
};

template <> struct Frag<f16> {
  f16x8 v;
  __device__ __forceinline__ void zero() {
    for (int e = 0; e < 8; ++e) v[e] = (f16)0.0f;
  }
  __device__ __forceinline__ void load(const f16* p) { v = *reinterpret_cast<const f16x8*>(p); }
  __device__ __forceinline__ void set(int e, float x) { v[e] = (f16)x; }
  __device__ __forceinline__ float get(int e) const { return (float)v[e]; }
};

// acc += A * B over one 32-deep slot set.
__device__ __forceinline__ void mma(f32x4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const Frag<f16>& a, const Frag<f16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, b.v, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const Frag<float>& a, const Frag<float>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[0], b.lo[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[1], b.lo[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[2], b.lo[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[3], b.lo[3], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[0], b.hi[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[1], b.hi[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[2], b.hi[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[3], b.hi[3], acc, 0, 0, 0);
}

// An f32 fragment as a pair of bf16 fragments, x = hi + lo + O(2^-18 |x|):
// hi = bf16(x) to nearest, lo = bf16(x - hi).  Products of two such pairs as
// hi*hi + hi*lo + lo*hi on the bf16 MFMA (fp32 accumulation) carry ~2^-16 of
// relative error: the three-part fp32 form (ODDE_F32X3), for callers that
// allow reduced-precision fp32 products.  Same lane layout as Frag<float>
// (lane l: row l % 16, k = 8 (l / 16) + e), so the accumulators of the two
// forms match element for element.
__device__ __forceinline__ void split_x3(const Frag<float>& f, Frag<bf16>& hi, Frag<bf16>& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = f.get(e);
    const bf16 h = (bf16)x;
    hi.v[e] = h;
    lo.v[e] = (bf16)(x - (float)h);
  }
}
__device__ __forceinline__ void mma_x3(f32x4& acc, const Frag<bf16>& ah, const Frag<bf16>& al,
                                       const Frag<bf16>& bh, const Frag<bf16>& bl) {
  mma(acc, al, bh);
  mma(acc, ah, bl);
  mma(acc, ah, bh);
}
__device__ __forceinline__ bf16x8 as_bf16x8(const f32x4& v) {
  bf16x8 r;
  __builtin_memcpy(&r, &v, sizeof(r));
  return r;
}
struct FragX3 {
  Frag<bf16> hi, lo;
  __device__ __forceinline__ void zero() {
    hi.zero();
    lo.zero();
  }
  __device__ __forceinline__ void load(const float* p) {
    Frag<float> f;
    f.load(p);
    split_x3(f, hi, lo);
  }
  __device__ __forceinline__ void from(const Frag<float>& f) { split_x3(f, hi, lo); }
};
__device__ __forceinline__ void mma(f32x4& acc, const FragX3& a, const FragX3& b) {
  mma_x3(acc, a.hi, a.lo, b.hi, b.lo);
}
// The fragment type a kernel multiplies with: CT's own, or the three-part
// pair for f32 data (kX3).
template <typename CT, bool kX3>
using MulFrag = typename std::conditional<kX3, FragX3, Frag<CT>>::type;
// x as a multiplication fragment (a split for the three-part form)
__device__ __forceinline__ void to_mul(const Frag<float>& f, FragX3& m) { m.from(f); }
template <typename CT>
__device__ __forceinline__ void to_mul(const Frag<CT>& f, Frag<CT>& m) { m = f; }

// ----------------------------------------------------------------------------
// small vector stores of 4 consecutive elements
// ----------------------------------------------------------------------------
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16)a; v[1] = (bf16)b; v[2] = (bf16)c; v[3] = (bf16)d;
  *reinterpret_cast<bf16x4*>(p) = v;
}
__device__ __forceinline__ void store4(f16* p, float a, float b, float c, float d) {
  f16x4 v;
  v[0] = (f16)a; v[1] = (f16)b; v[2] = (f16)c; v[3] = (f16)d;
  *reinterpret_cast<f16x4*>(p) = v;
}
// Data a kernel touches exactly once (the pair tiles it streams, the planes
// it writes) is loaded and stored non-temporally: the nt cache policy, which
// on this GPU raises a streaming copy from about 5.7 to 6.2 TB/s and an
// in-place read-modify-write from 5.5 to 6.2 TB/s (the lines are not kept
// for reuse).  Operands that several workgroups re-read through L2 keep the
// default policy.
constexpr int kStream = 2;  // the nt bit of the cache-policy field
template <typename V>
__device__ __forceinline__ void store_stream(V* p, const V& v) {
  __builtin_nontemporal_store(v, p);
}
template <typename V>
__device__ __forceinline__ V load_stream(const V* p) {
  return __builtin_nontemporal_load(p);
}
__device__ __forceinline__ void store4_stream(float* p, float a, float b, float c, float d) {
  store_stream(reinterpret_cast<f32x4*>(p), f32x4{a, b, c, d});
}
__device__ __forceinline__ void store4_stream(bf16* p, float a, float b, float c, float d) {
  bf16x4 v;
  v[0] = (bf16)a; v[1] = (bf16)b; v[2] = (bf16)c; v[3] = (bf16)d;
  store_stream(reinterpret_cast<bf16x4*>(p), v);
}
// Exchange a 16-byte value between the two lanes of each pair (2k, 2k + 1)
// (DPP quad permutation [1, 0, 3, 2]).  Every lane of the wave must be active.
template <typename V>
__device__ __forceinline__ V swap_lane_pairs(const V& v) {
  static_assert(sizeof(V) == 16, "16-byte values");
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  i32x4_t x = __builtin_bit_cast(i32x4_t, v);
#pragma unroll
  for (int k = 0; k < 4; ++k) x[k] = __builtin_amdgcn_mov_dpp(x[k], 0xB1, 0xF, 0xF, true);
  return __builtin_bit_cast(V, x);
}

// Streaming stores of whole 128-byte lines.  Each lane of a pair (2k, 2k + 1)
// holds two 16-byte chunks of its own line: lo for slot slot_lo and hi for
// slot slot_hi (the four lanes l, l + 16, l + 32, l + 48 hold four disjoint
// slot pairs that together cover the line).  Storing lo, then hi, would leave
// each instruction with half lines, which the streaming policy writes back
// poorly; here the pair exchanges one chunk, so the first instruction writes
// the even lane's whole line and the second the odd lane's.  `partner` is the
// other lane's line; own_ok and partner_ok say whether the two lines are
// stored at all.  Every lane of the wave must be active.
template <typename V>
__device__ __forceinline__ void store_line_pair_at(V* own, V* partner, int slot_lo, int slot_hi,
                                                   const V& lo, const V& hi, bool own_ok = true,
                                                   bool partner_ok = true) {
  const bool odd = threadIdx.x & 1;
  // even lanes receive the odd lane's lo, odd lanes the even lane's hi
  const V got = swap_lane_pairs(odd ? lo : hi);
  const int slot = odd ? slot_hi : slot_lo;
  if (odd ? partner_ok : own_ok) store_stream((odd ? partner : own) + slot, odd ? got : lo);
  if (odd ? own_ok : partner_ok) store_stream((odd ? own : partner) + slot, odd ? hi : got);
}
// the slot pair (s, s + 4), s = 0..3
template <typename V>
__device__ __forceinline__ void store_line_pair(V* own, V* partner, int s, const V& lo, const V& hi,
                                                bool own_ok = true, bool partner_ok = true) {
  store_line_pair_at(own, partner, s, s + 4, lo, hi, own_ok, partner_ok);
}

__device__ __forceinline__ void load4(const float* p, float* o) {
  f32x4 v = *reinterpret_cast<const f32x4*>(p);
  o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
}
__device__ __forceinline__ void load4(const bf16* p, float* o) {
  bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  o[0] = (float)v[0]; o[1] = (float)v[1]; o[2] = (float)v[2]; o[3] = (float)v[3];
}

// 8 contiguous elements -> float
__device__ __forceinline__ void load8(const float* p, float* o) {
  f32x4 a = *reinterpret_cast<const f32x4*>(p);
  f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  for (int e = 0; e < 4; ++e) { o[e] = a[e]; o[e + 4] = b[e]; }
}
__device__ __forceinline__ void load8(const bf16* p, float* o) {
  bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
  for (int e = 0; e < 8; ++e) o[e] = (float)v[e];
}

// ----------------------------------------------------------------------------
// cross-lane reductions inside a wave64 over the four 16-lane groups
// (lanes l, l^16, l^32, l^48 hold the same row / column).
// ----------------------------------------------------------------------------
__device__ __forceinline__ float xor_shfl(float v, int mask) {
  return __shfl_xor(v, mask, 64);
}
__device__ __forceinline__ float group_sum(float v) {
  v += xor_shfl(v, 16);
  v += xor_shfl(v, 32);
  return v;
}
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, xor_shfl(v, 16));
  v = fmaxf(v, xor_shfl(v, 32));
  return v;
}

// Same reductions with the gfx950 lane-swap instructions (one v_permlane*_swap
// each instead of an LDS-crossbar permute): after swapping a register with a
// copy of itself, the two results hold the values of lanes l and l^32 (or
// l^16), so one max/add completes that butterfly step.
__device__ __forceinline__ float swap32_max(float v) {
  auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float swap16_max(float v) {
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float swap32_add(float v) {
  auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float swap16_add(float v) {
  auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float group_max_fast(float v) { return swap32_max(swap16_max(v)); }
__device__ __forceinline__ float group_sum_fast(float v) { return swap32_add(swap16_add(v)); }

// 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal (about 1 ulp
// each): an IEEE division here would cost a dozen instructions per element.
// Saturates correctly: exp2 -> inf gives 0, exp2 -> 0 gives 1.
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
// sigmoid(x) from xs = -x log2(e), for products whose weights carry the factor
constexpr float kNegLog2e = -1.4426950408889634f;
__device__ __forceinline__ float sigmoid_nl2e(float xs) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(xs));
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes
// land at lds + 16 l.  `base` / `bytes` describe a raw buffer (offsets at or
// past `bytes` read as zero); voff is the lane's byte offset, soff a uniform
// one.  Against global_load_lds this keeps one 32-bit offset per lane
// instead of a 64-bit address.
// kPolicy is the instruction's cache-policy field (0, or kStream).
template <int kPolicy = 0>
__device__ __forceinline__ void buffer_load_lds16(const void* base, uint32_t bytes, void* lds,
                                                  uint32_t voff, uint32_t soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16,
                                           voff, soff, 0, kPolicy);
#endif
}
__host__ __device__ __forceinline__ uint32_t clamp_bytes(uint64_t b) {
  return b > 0xffffffffull ? 0xffffffffu : (uint32_t)b;
}

// Workgroup barrier without the memory fence __syncthreads() carries (that
// fence waits for every outstanding global load, which would drain loads
// issued ahead of time).  Callers first wait for what they need themselves
// (s_waitcnt on their own loads and LDS traffic); the empty asm statements
// keep the compiler from moving memory operations across the barrier.
__device__ __forceinline__ void barrier_nofence() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Barrier for LDS hand-offs only: this wave's LDS reads and writes are done
// (lgkmcnt), its global loads and stores may still be in flight.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  barrier_nofence();
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// ----------------------------------------------------------------------------
// Row loader with fused LayerNorm: a wave owns 16 rows of C channels and ends
// with the normalised rows as K32 fragments (kC = C / 32 of them): lane l
// holds row (l % 16), channels 32 s + 8 (l / 16) + e.  Statistics are fp32,
// two-pass (mean, then centred second moment), eps as given.  Rows flagged
// invalid produce zero fragments.
// ----------------------------------------------------------------------------
template <typename ZT, typename CT, int C>
__device__ __forceinline__ void ln_rows_to_frags(const ZT* row_ptr, bool valid,
                                                 const float* __restrict__ ln_w,
                                                 const float* __restrict__ ln_b, float eps,
                                                 Frag<CT> (&frag)[C / 32]) {
  constexpr int kC = C / 32;
  const int g = lane_id() >> 4;
  float x[kC][8];
  float s = 0.f;
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    if (valid) {
      load8(row_ptr + 32 * t + 8 * g, x[t]);
    } else {
      for (int e = 0; e < 8; ++e) x[t][e] = 0.f;
    }
    for (int e = 0; e < 8; ++e) s += x[t][e];
  }
  const float mean = group_sum_fast(s) * (1.0f / C);
  float q = 0.f;
#pragma unroll
  for (int t = 0; t < kC; ++t)
    for (int e = 0; e < 8; ++e) {
      const float d = x[t][e] - mean;
      q += d * d;
    }
  const float rstd = rsqrtf(group_sum_fast(q) * (1.0f / C) + eps);
#pragma unroll
  for (int t = 0; t < kC; ++t) {
    float w[8], b[8];
    load8(ln_w + 32 * t + 8 * g, w);
    load8(ln_b + 32 * t + 8 * g, b);
    for (int e = 0; e < 8; ++e) {
      const float y = valid ? (x[t][e] - mean) * rstd * w[e] + b[e] : 0.f;
      frag[t].set(e, y);
    }
  }
}

// Load a K32 fragment of a weight matrix W[out][K] (row-major, K contiguous):
// lane l takes output row (o0 + l % 16) and contraction slots 32 t + 8 g.
// Rows at or beyond n_out read as zero.
template <typename CT>
__device__ __forceinline__ void load_w_frag(const CT* __restrict__ w, int ld, int o0, int n_out,
                                            int t, Frag<CT>& f) {
  const int o = o0 + (lane_id() & 15);
  const int g = lane_id() >> 4;
  if (o < n_out) f.load(w + (size_t)o * ld + 32 * t + 8 * g);
  else f.zero();
}
// Three-part weight fragments from weights split once per call
// (split_x3_rows_kernel): `w_split` holds the bytes of an [n_out][2 ld] bf16
// array whose row o is hi = bf16(W[o][:]) followed by lo = bf16(W[o][:] - hi)
// (the same 4 bytes per weight as the f32 array it replaces).
__device__ __forceinline__ void load_w_frag(const float* __restrict__ w_split, int ld, int o0,
                                            int n_out, int t, FragX3& f) {
  const int o = o0 + (lane_id() & 15);
  const int g = lane_id() >> 4;
  if (o < n_out) {
    const bf16* p = reinterpret_cast<const bf16*>(w_split) + (size_t)o * 2 * ld + 32 * t + 8 * g;
    f.hi.load(p);
    f.lo.load(p + ld);
  } else {
    f.zero();
  }
}

// A weight fragment from a weight row staged in LDS with the global row's
// bytes: fp32 (8 floats at k = 32 t + 8 g) or three-part (the row's 2 ld
// bf16, hi then lo, as load_w_frag reads them from the split weights).
__device__ __forceinline__ void staged_w_frag(const float* row, int ld, int t, Frag<float>& f) {
  (void)ld;
  f.load(row + 32 * t + 8 * (lane_id() >> 4));
}
__device__ __forceinline__ void staged_w_frag(const float* row, int ld, int t, FragX3& f) {
  const bf16* p = reinterpret_cast<const bf16*>(row) + 32 * t + 8 * (lane_id() >> 4);
  f.hi.load(p);
  f.lo.load(p + ld);
}
// W [rows][cols] f32 -> [rows][2 cols] bf16: row r = hi = bf16(W[r][:]) to
// nearest, then lo = bf16(W[r][:] - hi).  With kPerm32 the columns are
// permuted within each block of 32, column 16 s + 4 q + e to 8 q + 4 s + e,
// so that the 8 columns {4q .. 4q+3, 16+4q .. 16+4q+3} are contiguous (the
// transition's W_o, whose GEMM2 fragment slots of lane group q are those
// hidden units).
template <bool kPerm32>
__global__ __launch_bounds__(256) void split_x3_rows_kernel(const float* __restrict__ src,
                                                            bf16* __restrict__ dst, int rows,
                                                            int cols) {
  const int64_t total = (int64_t)rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * 256) {
    const int64_t r = i / cols;
    const int c = (int)(i - r * cols);
    int cc = c;
    if constexpr (kPerm32) {
      const int m = c & 31;
      cc = (c & ~31) + 8 * ((m >> 2) & 3) + 4 * (m >> 4) + (m & 3);
    }
    const float x = src[i];
    const bf16 h = (bf16)x;
    bf16* row = dst + r * 2 * cols;
    row[cc] = h;
    row[cols + cc] = (bf16)(x - (float)h);
  }
}
inline void launch_split_x3(const void* src, int rows, int cols, void* dst, bool perm32,
                            hipStream_t st) {
  const int64_t total = (int64_t)rows * cols;
  const int grid = (int)(total / 256 + 1 < 1024 ? total / 256 + 1 : 1024);
  if (perm32)
    hipLaunchKernelGGL((split_x3_rows_kernel<true>), dim3(grid), dim3(256), 0, st,
                       static_cast<const float*>(src), static_cast<bf16*>(dst), rows, cols);
  else
    hipLaunchKernelGGL((split_x3_rows_kernel<false>), dim3(grid), dim3(256), 0, st,
                       static_cast<const float*>(src), static_cast<bf16*>(dst), rows, cols);
}
// bf16 weights as fp16 fragments (exact: fp16 holds every bf16 value of the
// weights' range, |w| >= 2^-14, to more mantissa bits than bf16 has)
__device__ __forceinline__ void load_w_frag(const bf16* __restrict__ w, int ld, int o0, int n_out,
                                            int t, Frag<f16>& f) {
  Frag<bf16> b;
  load_w_frag(w, ld, o0, n_out, t, b);
#pragma unroll
  for (int e = 0; e < 8; ++e) f.v[e] = (f16)(float)b.v[e];
}
// ... scaled by `scale` on the way (one rounding of scale * w to fp16, 11
// significant bits): folds a constant factor of the product into the weights
__device__ __forceinline__ void load_w_frag_scaled(const bf16* __restrict__ w, int ld, int o0,
                                                   int n_out, int t, float scale, Frag<f16>& f) {
  Frag<bf16> b;
  load_w_frag(w, ld, o0, n_out, t, b);
#pragma unroll
  for (int e = 0; e < 8; ++e) f.v[e] = (f16)(scale * (float)b.v[e]);
}

}  // namespace odde
