// LayerNorm over the last n2 elements of n1 contiguous rows: forward
// (out, mean, invvar) and backward (grad_input, grad_gamma, grad_beta), the
// contract of the reference's fast LayerNorm extension
// (opendde/model/layer_norm/kernel/layer_norm_cuda.cpp:63-179).
//
// HBM-bound: the forward reads x once and writes out once (+8 bytes of
// statistics per row); the backward reads x and dout once and writes
// grad_input once.  Statistics and every sum are f32.
//
// Row kernels (n2 a multiple of the 16-byte vector, 16-byte aligned tensors,
// n2 <= 2048): a row is owned by a group of G lanes (G a power of two <= 64)
// holding NV 16-byte vectors each, so a whole row sits in registers and the
// two-pass statistics (mean, then sum of squared deviations) read HBM once.
// The group reduction is an xor butterfly, so every lane of a group ends with
// the same bits.  Each group keeps R rows in flight per iteration.  gamma and
// beta are converted to f32 once per lane and kept in registers.
//
// Backward column sums (grad_gamma, grad_beta) are fused into the row kernel:
// each lane accumulates dout*xhat and dout for its columns over the rows its
// group visits; the groups of a wave are summed by butterfly, the four waves
// of a workgroup in a fixed order through LDS, and each workgroup writes one
// partial row to the workspace.  A second kernel sums the partial rows in a
// fixed order, so results are deterministic for a given (n1, n2, dtype).
//
// Any other shape (odd n2, misaligned tensors, n2 > 2048) takes the generic
// kernels: a wave per row with strided scalar access, and a column-partial
// kernel for grad_gamma / grad_beta.
#include <algorithm>
#include <mutex>
#include <string>

#include "common.hpp"
#include "runtime.hpp"

namespace odde {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kLnThreads = 256;      // 4 waves per workgroup
constexpr int kLnMaxVecFloats = 32;  // NV * VEC bound of the row kernels
constexpr int kLnMaxRowN2 = 64 * kLnMaxVecFloats;
constexpr int kLnFwdMaxBlocks = 2048;
constexpr int kLnBwdMaxBlocks = 1024;
constexpr int64_t kLnGenericMaxParts = 4096;

template <typename T> struct VecOf { static constexpr int N = 16 / sizeof(T); };

// 16 bytes of T -> f32
__device__ __forceinline__ void unpack(const u32x4& u, float* f, float*) {
  f[0] = __uint_as_float(u[0]);
  f[1] = __uint_as_float(u[1]);
  f[2] = __uint_as_float(u[2]);
  f[3] = __uint_as_float(u[3]);
}
__device__ __forceinline__ void unpack(const u32x4& u, float* f, bf16*) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(u[i] << 16);
    f[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
  }
}
__device__ __forceinline__ void unpack(const u32x4& u, float* f, f16*) {
  f16x8 h = __builtin_bit_cast(f16x8, u);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = (float)h[i];
}

// f32 -> 16 bytes of T (round to nearest even)
__device__ __forceinline__ u32x4 pack(const float* f, float*) {
  return u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]),
               __float_as_uint(f[3])};
}
__device__ __forceinline__ u32x4 pack(const float* f, bf16*) {
  bf16x8 b;
#pragma unroll
  for (int i = 0; i < 8; ++i) b[i] = (bf16)f[i];
  return __builtin_bit_cast(u32x4, b);
}
__device__ __forceinline__ u32x4 pack(const float* f, f16*) {
  f16x8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (f16)f[i];
  return __builtin_bit_cast(u32x4, h);
}

template <typename T> __device__ __forceinline__ void load_vec(const T* p, float* f) {
  unpack(*reinterpret_cast<const u32x4*>(p), f, (T*)nullptr);
}
template <typename T> __device__ __forceinline__ void store_vec(T* p, const float* f) {
  *reinterpret_cast<u32x4*>(p) = pack(f, (T*)nullptr);
}

// Sum over the G = 1 << lg lanes of an aligned lane group (xor butterfly:
// every lane of the group ends with the same value).
__device__ __forceinline__ float group_sum(float s, int lg) {
  for (int o = 1; o < (1 << lg); o <<= 1) s += __shfl_xor(s, o);
  return s;
}

// ---------------------------------------------------------------------------
// row kernels
// ---------------------------------------------------------------------------

// Per-lane f32 copy of this lane's columns of a [n2] parameter (identity
// value `dflt` when the pointer is null or the slot is past the row end).
template <typename T, int NV>
__device__ __forceinline__ void load_param(const T* p, int j, int lg, int V, float dflt,
                                           float (&f)[NV][VecOf<T>::N]) {
  constexpr int VEC = VecOf<T>::N;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int v = j + (k << lg);
    if (p && v < V) {
      load_vec(p + v * VEC, f[k]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) f[k][e] = dflt;
    }
  }
}

template <typename T, int NV, int R>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_rows_kernel(
    const T* __restrict__ x, const T* __restrict__ gamma, const T* __restrict__ beta,
    T* __restrict__ out, float* __restrict__ mean, float* __restrict__ invvar, int64_t n1, int n2,
    int lg, float eps) {
  constexpr int VEC = VecOf<T>::N;
  const int V = n2 / VEC;
  const int j = threadIdx.x & ((1 << lg) - 1);
  const int64_t group = (int64_t(blockIdx.x) * kLnThreads + threadIdx.x) >> lg;
  const int64_t ngroups = (int64_t(gridDim.x) * kLnThreads) >> lg;
  const float inv_n2 = 1.0f / float(n2);

  float g[NV][VEC], b[NV][VEC];
  load_param<T, NV>(gamma, j, lg, V, 1.0f, g);
  load_param<T, NV>(beta, j, lg, V, 0.0f, b);

  for (int64_t base = 0; base < n1; base += R * ngroups) {
    float f[R][NV][VEC];
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const int64_t r = base + t * ngroups + group;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int v = j + (k << lg);
        if (r < n1 && v < V) {
          load_vec(x + r * n2 + v * VEC, f[t][k]);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) f[t][k][e] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const int64_t r = base + t * ngroups + group;
      if (r >= n1) break;  // uniform over the group
      float s = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < VEC; ++e) s += f[t][k][e];
      const float mu = group_sum(s, lg) * inv_n2;
      float q = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        if (j + (k << lg) < V) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const float d = f[t][k][e] - mu;
            q += d * d;
          }
        }
      }
      const float var = group_sum(q, lg) * inv_n2;
      const float iv = 1.0f / sqrtf(var + eps);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int v = j + (k << lg);
        if (v < V) {
          float o[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e) o[e] = (f[t][k][e] - mu) * iv * g[k][e] + b[k][e];
          store_vec(out + r * n2 + v * VEC, o);
        }
      }
      if (j == 0) {
        mean[r] = mu;
        invvar[r] = iv;
      }
    }
  }
}

// grad_input for the rows of each group; optional per-workgroup partial sums
// part[blockIdx.x][0][c] = sum dout*xhat, part[blockIdx.x][1][c] = sum dout.
template <typename T, int NV, int R>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_rows_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ invvar, const T* __restrict__ gamma, T* __restrict__ dx,
    float* __restrict__ part, int64_t n1, int n2, int lg) {
  constexpr int VEC = VecOf<T>::N;
  __shared__ float red[2 * kLnMaxRowN2];
  const int V = n2 / VEC;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = threadIdx.x & ((1 << lg) - 1);
  const int64_t group = (int64_t(blockIdx.x) * kLnThreads + threadIdx.x) >> lg;
  const int64_t ngroups = (int64_t(gridDim.x) * kLnThreads) >> lg;
  const float inv_n2 = 1.0f / float(n2);

  float g[NV][VEC];
  load_param<T, NV>(gamma, j, lg, V, 1.0f, g);
  float ag[NV][VEC], ab[NV][VEC];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < VEC; ++e) ag[k][e] = ab[k][e] = 0.0f;

  for (int64_t base = 0; base < n1; base += R * ngroups) {
    float xf[R][NV][VEC], df[R][NV][VEC];
    float mu[R], iv[R];
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const int64_t r = base + t * ngroups + group;
      mu[t] = r < n1 ? mean[r] : 0.0f;
      iv[t] = r < n1 ? invvar[r] : 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int v = j + (k << lg);
        if (r < n1 && v < V) {
          load_vec(x + r * n2 + v * VEC, xf[t][k]);
          load_vec(dout + r * n2 + v * VEC, df[t][k]);
        } else {
#pragma unroll
          for (int e = 0; e < VEC; ++e) xf[t][k][e] = df[t][k][e] = 0.0f;
        }
      }
    }
#pragma unroll
    for (int t = 0; t < R; ++t) {
      const int64_t r = base + t * ngroups + group;
      if (r >= n1) break;  // uniform over the group
      float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float xh = (xf[t][k][e] - mu[t]) * iv[t];
          const float gg = df[t][k][e] * g[k][e];
          xf[t][k][e] = xh;
          s1 += gg;
          s2 += gg * xh;
          ag[k][e] += df[t][k][e] * xh;
          ab[k][e] += df[t][k][e];
        }
      s1 = group_sum(s1, lg) * inv_n2;
      s2 = group_sum(s2, lg) * inv_n2;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int v = j + (k << lg);
        if (v < V) {
          float o[VEC];
#pragma unroll
          for (int e = 0; e < VEC; ++e)
            o[e] = iv[t] * (df[t][k][e] * g[k][e] - s1 - xf[t][k][e] * s2);
          store_vec(dx + r * n2 + v * VEC, o);
        }
      }
    }
  }
  if (!part) return;  // uniform: no parameter gradients requested

  // groups of the wave -> lanes 0..G-1
  for (int o = 1 << lg; o < 64; o <<= 1) {
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        ag[k][e] += __shfl_xor(ag[k][e], o);
        ab[k][e] += __shfl_xor(ab[k][e], o);
      }
  }
  // waves -> LDS, in wave order
  for (int w = 0; w < kLnThreads / 64; ++w) {
    if (wave == w && lane < (1 << lg)) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        const int v = j + (k << lg);
        if (v < V) {
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            const int c = v * VEC + e;
            red[c] = (w == 0 ? 0.0f : red[c]) + ag[k][e];
            red[n2 + c] = (w == 0 ? 0.0f : red[n2 + c]) + ab[k][e];
          }
        }
      }
    }
    __syncthreads();
  }
  float* dst = part + int64_t(blockIdx.x) * 2 * n2;
  for (int i = threadIdx.x; i < 2 * n2; i += kLnThreads) dst[i] = red[i];
}

// ---------------------------------------------------------------------------
// generic kernels (any n2, any alignment): one wave per row
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float s) {
  for (int o = 1; o < 64; o <<= 1) s += __shfl_xor(s, o);
  return s;
}

template <typename T>
__global__ __launch_bounds__(kLnThreads) void ln_fwd_generic_kernel(
    const T* __restrict__ x, const T* __restrict__ gamma, const T* __restrict__ beta,
    T* __restrict__ out, float* __restrict__ mean, float* __restrict__ invvar, int64_t n1, int n2,
    float eps) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = int64_t(gridDim.x) * (kLnThreads / 64);
  const float inv_n2 = 1.0f / float(n2);
  for (int64_t r = int64_t(blockIdx.x) * (kLnThreads / 64) + (threadIdx.x >> 6); r < n1; r += nw) {
    const T* xr = x + r * n2;
    float s = 0.0f;
    for (int c = lane; c < n2; c += 64) s += to_f32(xr[c]);
    const float mu = wave_sum(s) * inv_n2;
    float q = 0.0f;
    for (int c = lane; c < n2; c += 64) {
      const float d = to_f32(xr[c]) - mu;
      q += d * d;
    }
    const float iv = 1.0f / sqrtf(wave_sum(q) * inv_n2 + eps);
    T* orow = out + r * n2;
    for (int c = lane; c < n2; c += 64) {
      float o = (to_f32(xr[c]) - mu) * iv;
      if (gamma) o *= to_f32(gamma[c]);
      if (beta) o += to_f32(beta[c]);
      orow[c] = from_f32<T>(o);
    }
    if (lane == 0) {
      mean[r] = mu;
      invvar[r] = iv;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_generic_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ invvar, const T* __restrict__ gamma, T* __restrict__ dx, int64_t n1,
    int n2) {
  const int lane = threadIdx.x & 63;
  const int64_t nw = int64_t(gridDim.x) * (kLnThreads / 64);
  const float inv_n2 = 1.0f / float(n2);
  for (int64_t r = int64_t(blockIdx.x) * (kLnThreads / 64) + (threadIdx.x >> 6); r < n1; r += nw) {
    const T* xr = x + r * n2;
    const T* dr = dout + r * n2;
    const float mu = mean[r], iv = invvar[r];
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = lane; c < n2; c += 64) {
      const float gg = to_f32(dr[c]) * (gamma ? to_f32(gamma[c]) : 1.0f);
      s1 += gg;
      s2 += gg * (to_f32(xr[c]) - mu) * iv;
    }
    s1 = wave_sum(s1) * inv_n2;
    s2 = wave_sum(s2) * inv_n2;
    T* orow = dx + r * n2;
    for (int c = lane; c < n2; c += 64) {
      const float gg = to_f32(dr[c]) * (gamma ? to_f32(gamma[c]) : 1.0f);
      const float xh = (to_f32(xr[c]) - mu) * iv;
      orow[c] = from_f32<T>(iv * (gg - s1 - xh * s2));
    }
  }
}

// part[p][0][c] = sum over rows [p*rows_per_part, ...) of dout*xhat,
// part[p][1][c] = the same of dout.  Block (64, 4): x = column, y = row lane.
template <typename T>
__global__ __launch_bounds__(kLnThreads) void ln_bwd_cols_generic_kernel(
    const T* __restrict__ dout, const T* __restrict__ x, const float* __restrict__ mean,
    const float* __restrict__ invvar, float* __restrict__ part, int64_t n1, int n2,
    int rows_per_part) {
  __shared__ float sg[4][64], sb[4][64];
  const int c = blockIdx.x * 64 + threadIdx.x;
  const int64_t r0 = int64_t(blockIdx.y) * rows_per_part;
  const int64_t r1 = r0 + rows_per_part < n1 ? r0 + rows_per_part : n1;
  float ag = 0.0f, ab = 0.0f;
  if (c < n2) {
    for (int64_t r = r0 + threadIdx.y; r < r1; r += 4) {
      const float d = to_f32(dout[r * n2 + c]);
      ag += d * (to_f32(x[r * n2 + c]) - mean[r]) * invvar[r];
      ab += d;
    }
  }
  sg[threadIdx.y][threadIdx.x] = ag;
  sb[threadIdx.y][threadIdx.x] = ab;
  __syncthreads();
  if (threadIdx.y == 0 && c < n2) {
    float* dst = part + int64_t(blockIdx.y) * 2 * n2;
    dst[c] = (sg[0][threadIdx.x] + sg[1][threadIdx.x]) + (sg[2][threadIdx.x] + sg[3][threadIdx.x]);
    dst[n2 + c] =
        (sb[0][threadIdx.x] + sb[1][threadIdx.x]) + (sb[2][threadIdx.x] + sb[3][threadIdx.x]);
  }
}

// grad_gamma[c] = sum_p part[p][0][c]; grad_beta[c] = sum_p part[p][1][c].
// Block (64, 16), grid (ceil(n2 / 64), 2): blockIdx.y selects the output.
template <typename T>
__global__ __launch_bounds__(1024) void ln_param_grad_reduce_kernel(
    const float* __restrict__ part, int nparts, int n2, T* __restrict__ grad_gamma,
    T* __restrict__ grad_beta) {
  __shared__ float acc[16][65];
  T* dst = blockIdx.y == 0 ? grad_gamma : grad_beta;
  if (!dst) return;  // uniform over the workgroup
  const int c = blockIdx.x * 64 + threadIdx.x;
  float s = 0.0f;
  if (c < n2)
    for (int p = threadIdx.y; p < nparts; p += 16) s += part[(int64_t(p) * 2 + blockIdx.y) * n2 + c];
  acc[threadIdx.y][threadIdx.x] = s;
  __syncthreads();
  for (int h = 8; h > 0; h >>= 1) {
    if (threadIdx.y < h) acc[threadIdx.y][threadIdx.x] += acc[threadIdx.y + h][threadIdx.x];
    __syncthreads();
  }
  if (threadIdx.y == 0 && c < n2) dst[c] = from_f32<T>(acc[0][threadIdx.x]);
}

// ---------------------------------------------------------------------------
// host planning
// ---------------------------------------------------------------------------

struct LnPlan {
  bool rows = false;  // row kernels (else generic)
  int lg = 0, nv = 0, r = 1;
  int64_t blocks = 0;  // grid of the chosen kernel
  int64_t nparts = 0;  // partial rows of the backward column sums
};

inline int elem_size(int dt) { return dt == ODDE_F32 ? 4 : 2; }

// Row split of the generic column-sum kernel: at least 256 rows per part, at
// most kLnGenericMaxParts parts.
inline int64_t generic_rows_per_part(int64_t n1) {
  return std::max<int64_t>(256, (n1 + kLnGenericMaxParts - 1) / kLnGenericMaxParts);
}
inline int64_t generic_parts(int64_t n1) {
  const int64_t rpp = generic_rows_per_part(n1);
  return (n1 + rpp - 1) / rpp;
}

// Shape part of the plan: row kernels need n2 to be a whole number of 16-byte
// vectors and at most 32 f32 values per lane.  Among lane-group sizes
// G = 64, 32, ..., 1 the one leaving the fewest idle vector slots wins (ties:
// the larger G).
LnPlan plan_shape(int64_t n1, int n2, int dt, bool backward) {
  LnPlan p;
  const int vec = 16 / elem_size(dt);
  if (n2 % vec == 0 && n2 <= kLnMaxRowN2) {
    const int V = n2 / vec, max_nv = kLnMaxVecFloats / vec;
    int best_waste = 1 << 30;
    for (int lg = 6; lg >= 0; --lg) {
      const int G = 1 << lg, nv = (V + G - 1) / G;
      if (nv > max_nv) continue;
      if (G * nv - V < best_waste) {
        best_waste = G * nv - V;
        p.lg = lg;
        p.nv = nv;
      }
    }
    p.rows = p.nv > 0;
  }
  if (p.rows) {
    p.r = p.nv == 1 ? 4 : p.nv == 2 ? 2 : 1;
    const int64_t rows_per_block = int64_t(kLnThreads >> p.lg) * p.r;
    const int64_t cap = backward ? kLnBwdMaxBlocks : kLnFwdMaxBlocks;
    p.blocks = std::min<int64_t>((n1 + rows_per_block - 1) / rows_per_block, cap);
    p.nparts = p.blocks;
  } else {
    p.blocks = std::min<int64_t>((n1 + 3) / 4, kLnFwdMaxBlocks);
    p.nparts = generic_parts(n1);
  }
  return p;
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <typename T, int NV>
void launch_fwd_rows(const LnPlan& p, const odde_layer_norm_args* a, hipStream_t st) {
  constexpr int R = NV == 1 ? 4 : NV == 2 ? 2 : 1;
  hipLaunchKernelGGL((ln_fwd_rows_kernel<T, NV, R>), dim3(p.blocks), dim3(kLnThreads), 0, st,
                     (const T*)a->x, (const T*)a->gamma, (const T*)a->beta, (T*)a->out, a->mean,
                     a->invvar, a->n1, a->n2, p.lg, a->eps);
}

template <typename T, int NV>
void launch_bwd_rows(const LnPlan& p, const odde_layer_norm_bwd_args* a, float* part,
                     hipStream_t st) {
  constexpr int R = NV == 1 ? 4 : NV == 2 ? 2 : 1;
  hipLaunchKernelGGL((ln_bwd_rows_kernel<T, NV, R>), dim3(p.blocks), dim3(kLnThreads), 0, st,
                     (const T*)a->dout, (const T*)a->x, a->mean, a->invvar, (const T*)a->gamma,
                     (T*)a->grad_input, part, a->n1, a->n2, p.lg);
}

template <typename T>
int run_fwd(const odde_layer_norm_args* a, hipStream_t st) {
  const LnPlan p = plan_shape(a->n1, a->n2, a->dtype, false);
  const bool use_rows = p.rows && aligned16(a->x) && aligned16(a->out) && aligned16(a->gamma) &&
                        aligned16(a->beta);
  LaunchScope ls(ODDE_K_LAYER_NORM, st);
  if (use_rows) {
    switch (p.nv) {
      case 1: launch_fwd_rows<T, 1>(p, a, st); break;
      case 2: launch_fwd_rows<T, 2>(p, a, st); break;
      case 3: launch_fwd_rows<T, 3>(p, a, st); break;
      case 4: launch_fwd_rows<T, 4>(p, a, st); break;
      case 5: if constexpr (sizeof(T) == 4) { launch_fwd_rows<T, 5>(p, a, st); break; } [[fallthrough]];
      case 6: if constexpr (sizeof(T) == 4) { launch_fwd_rows<T, 6>(p, a, st); break; } [[fallthrough]];
      case 7: if constexpr (sizeof(T) == 4) { launch_fwd_rows<T, 7>(p, a, st); break; } [[fallthrough]];
      case 8: if constexpr (sizeof(T) == 4) { launch_fwd_rows<T, 8>(p, a, st); break; } [[fallthrough]];
      default: return set_error(ODDE_EINVAL, "layer_norm: internal plan error");
    }
  } else {
    const int64_t blocks = std::min<int64_t>((a->n1 + 3) / 4, kLnFwdMaxBlocks);
    hipLaunchKernelGGL((ln_fwd_generic_kernel<T>), dim3(blocks), dim3(kLnThreads), 0, st,
                       (const T*)a->x, (const T*)a->gamma, (const T*)a->beta, (T*)a->out, a->mean,
                       a->invvar, a->n1, a->n2, a->eps);
  }
  return check_launch("layer_norm forward");
}

template <typename T>
int run_bwd(const odde_layer_norm_bwd_args* a, uint64_t need_ws, hipStream_t st,
            bool events = true) {
  const LnPlan p = plan_shape(a->n1, a->n2, a->dtype, true);
  const bool use_rows = p.rows && aligned16(a->x) && aligned16(a->dout) &&
                        aligned16(a->grad_input) && aligned16(a->gamma);
  const bool want_params = a->grad_gamma || a->grad_beta;
  float* part = want_params ? static_cast<float*>(a->workspace) : nullptr;
  const int64_t nparts = a->n1 == 0 ? 0 : use_rows ? p.blocks : generic_parts(a->n1);
  if (want_params && uint64_t(nparts) * 2 * uint64_t(a->n2) * sizeof(float) > need_ws)
    return set_error(ODDE_EINVAL, "layer_norm backward: internal workspace plan error");
  LaunchScope ls(ODDE_K_LAYER_NORM_BWD, st, events);
  if (a->n1 > 0 && use_rows) {
    switch (p.nv) {
      case 1: launch_bwd_rows<T, 1>(p, a, part, st); break;
      case 2: launch_bwd_rows<T, 2>(p, a, part, st); break;
      case 3: launch_bwd_rows<T, 3>(p, a, part, st); break;
      case 4: launch_bwd_rows<T, 4>(p, a, part, st); break;
      case 5: if constexpr (sizeof(T) == 4) { launch_bwd_rows<T, 5>(p, a, part, st); break; } [[fallthrough]];
      case 6: if constexpr (sizeof(T) == 4) { launch_bwd_rows<T, 6>(p, a, part, st); break; } [[fallthrough]];
      case 7: if constexpr (sizeof(T) == 4) { launch_bwd_rows<T, 7>(p, a, part, st); break; } [[fallthrough]];
      case 8: if constexpr (sizeof(T) == 4) { launch_bwd_rows<T, 8>(p, a, part, st); break; } [[fallthrough]];
      default: return set_error(ODDE_EINVAL, "layer_norm: internal plan error");
    }
  } else if (a->n1 > 0) {
    const int64_t blocks = std::min<int64_t>((a->n1 + 3) / 4, kLnFwdMaxBlocks);
    hipLaunchKernelGGL((ln_bwd_generic_kernel<T>), dim3(blocks), dim3(kLnThreads), 0, st,
                       (const T*)a->dout, (const T*)a->x, a->mean, a->invvar, (const T*)a->gamma,
                       (T*)a->grad_input, a->n1, a->n2);
    if (want_params)
      hipLaunchKernelGGL((ln_bwd_cols_generic_kernel<T>), dim3((a->n2 + 63) / 64, nparts),
                         dim3(64, 4), 0, st, (const T*)a->dout, (const T*)a->x, a->mean,
                         a->invvar, part, a->n1, a->n2, int(generic_rows_per_part(a->n1)));
  }
  if (want_params)
    hipLaunchKernelGGL((ln_param_grad_reduce_kernel<T>), dim3((a->n2 + 63) / 64, 2),
                       dim3(64, 16), 0, st, part, int(nparts), a->n2, (T*)a->grad_gamma,
                       (T*)a->grad_beta);
  return check_launch("layer_norm backward");
}

bool valid_ln_dtype(int dt) { return dt == ODDE_F32 || dt == ODDE_BF16 || dt == ODDE_F16; }

// Partial column sums of the allocation-free backward: a fixed device array
// (each GPU holds its own copy at its own address for the life of the
// process).  Host code never passes `scratch` itself to a kernel: its name on
// the host is a stand-in, not a device address.  The device address is
// looked up once per device with hipGetSymbolAddress and cached.
constexpr uint64_t kLnScratchBytes = uint64_t(16) << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kLnScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_address(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return set_error(ODDE_EHIP, "layer_norm backward (no-alloc): no current HIP device");
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      return set_error(ODDE_EHIP, std::string("layer_norm backward (no-alloc): "
                                              "hipGetSymbolAddress(scratch) failed: ") +
                                      hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return ODDE_OK;
}

int check_bwd_args(const odde_layer_norm_bwd_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "layer_norm backward: null args");
  if (a->struct_size != sizeof(odde_layer_norm_bwd_args))
    return set_error(ODDE_EINVAL, "layer_norm backward: struct_size mismatch (ABI version skew)");
  if (a->n1 < 0 || a->n2 <= 0) return set_error(ODDE_EINVAL, "layer_norm backward: bad sizes");
  if (!valid_ln_dtype(a->dtype)) return set_error(ODDE_EINVAL, "layer_norm backward: bad dtype");
  if (a->n1 > 0 && (!a->dout || !a->x || !a->mean || !a->invvar || !a->grad_input))
    return set_error(ODDE_EINVAL, "layer_norm backward: null tensor pointer");
  return ODDE_OK;
}

uint64_t bwd_workspace(int64_t n1, int n2, int dt) {
  LnPlan rows = plan_shape(n1, n2, dt, true);
  const int64_t parts = std::max<int64_t>(rows.rows ? rows.nparts : 0, generic_parts(n1));
  return uint64_t(parts) * 2 * uint64_t(n2) * sizeof(float);
}

}  // namespace
}  // namespace odde

using namespace odde;

extern "C" {

int odde_layer_norm_fwd(const odde_layer_norm_args* a, void* stream) {
  if (!a) return set_error(ODDE_EINVAL, "layer_norm: null args");
  if (a->struct_size != sizeof(odde_layer_norm_args))
    return set_error(ODDE_EINVAL, "layer_norm: struct_size mismatch (ABI version skew)");
  if (a->n1 < 0 || a->n2 <= 0) return set_error(ODDE_EINVAL, "layer_norm: bad sizes");
  if (!valid_ln_dtype(a->dtype)) return set_error(ODDE_EINVAL, "layer_norm: bad dtype");
  if (!(a->eps >= 0.0f)) return set_error(ODDE_EINVAL, "layer_norm: eps must be >= 0");
  if (a->n1 == 0) return ODDE_OK;
  if (!a->x || !a->out || !a->mean || !a->invvar)
    return set_error(ODDE_EINVAL, "layer_norm: null tensor pointer");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == ODDE_F32) return run_fwd<float>(a, st);
  if (a->dtype == ODDE_BF16) return run_fwd<bf16>(a, st);
  return run_fwd<f16>(a, st);
}

int odde_layer_norm_bwd_workspace_bytes(const odde_layer_norm_bwd_args* a, uint64_t* bytes) {
  if (!a || !bytes) return set_error(ODDE_EINVAL, "layer_norm backward: null argument");
  if (a->struct_size != sizeof(odde_layer_norm_bwd_args))
    return set_error(ODDE_EINVAL, "layer_norm backward: struct_size mismatch (ABI version skew)");
  if (a->n1 < 0 || a->n2 <= 0) return set_error(ODDE_EINVAL, "layer_norm backward: bad sizes");
  if (!valid_ln_dtype(a->dtype)) return set_error(ODDE_EINVAL, "layer_norm backward: bad dtype");
  *bytes = bwd_workspace(a->n1, a->n2, a->dtype);
  return ODDE_OK;
}

int odde_layer_norm_bwd(const odde_layer_norm_bwd_args* a, void* stream) {
  if (const int rc = check_bwd_args(a)) return rc;
  const bool want_params = a->grad_gamma || a->grad_beta;
  const uint64_t need = bwd_workspace(a->n1, a->n2, a->dtype);
  if (want_params && need > 0) {
    if (!a->workspace || a->workspace_bytes < need)
      return set_error(ODDE_EWORKSPACE, "layer_norm backward: workspace too small");
    if (reinterpret_cast<uintptr_t>(a->workspace) & 15)
      return set_error(ODDE_EWORKSPACE, "layer_norm backward: workspace must be 16-byte aligned");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == ODDE_F32) return run_bwd<float>(a, need, st);
  if (a->dtype == ODDE_BF16) return run_bwd<bf16>(a, need, st);
  return run_bwd<f16>(a, need, st);
}

int odde_layer_norm_bwd_noalloc(const odde_layer_norm_bwd_args* a, void* stream) {
  if (const int rc = check_bwd_args(a)) return rc;
  const bool want_params = a->grad_gamma || a->grad_beta;
  const uint64_t need = bwd_workspace(a->n1, a->n2, a->dtype);
  odde_layer_norm_bwd_args b = *a;
  b.workspace = nullptr;
  b.workspace_bytes = 0;
  if (want_params && need > 0) {
    if (need > kLnScratchBytes)
      return set_error(ODDE_EUNSUPPORTED,
                       "layer_norm backward (no-alloc): the partial column sums need " +
                           std::to_string(need) + " bytes, more than the " +
                           std::to_string(kLnScratchBytes) +
                           "-byte scratch array; use odde_layer_norm_bwd with a workspace");
    void* p = nullptr;
    if (const int rc = scratch_address(&p)) return rc;
    b.workspace = p;
    b.workspace_bytes = kLnScratchBytes;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->dtype == ODDE_F32) return run_bwd<float>(&b, need, st, false);
  if (a->dtype == ODDE_BF16) return run_bwd<bf16>(&b, need, st, false);
  return run_bwd<f16>(&b, need, st, false);
}

}  // extern "C"
