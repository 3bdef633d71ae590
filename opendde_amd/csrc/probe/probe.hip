// Machine-rate probes, built into their own measurement library
// (libopendde_amd_probe.so, declared in include/opendde_amd_probe.h), apart
// from the product library: the MFMA throughput this GPU actually sustains,
// the triangle-attention core's instruction mix with no memory traffic, and
// the streaming HBM rate, so that kernel figures can be quoted against
// measured peaks as well as the data sheet's.  The caller times a probe with
// events on the stream it passes.
#include <string>

#include "../../../include/opendde_amd_probe.h"
#include "../common.hpp"

namespace odde {

namespace {
thread_local std::string g_probe_error;

int probe_error(const char* msg) {
  g_probe_error = msg;
  return -1;
}

int probe_launched(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e == hipSuccess) return 0;
  g_probe_error = std::string(what) + ": " + hipGetErrorString(e);
  return -2;
}
}  // namespace

// MFMA rate: every wave runs 8 independent accumulator chains of one MFMA
// shape for `iters` rounds; nothing is loaded, one conditional store per lane
// keeps the results live.

template <bool kBf16>
__global__ __launch_bounds__(256) void mfma_probe_kernel(float* __restrict__ sink, int64_t iters) {
  constexpr int NACC = 8;
  f32x4 acc[NACC];
#pragma unroll
  for (int k = 0; k < NACC; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float seed = 1e-3f * (float)(threadIdx.x & 63);
  if constexpr (kBf16) {
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (bf16)(seed + e);
      b[e] = (bf16)(seed - e);
    }
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int k = 0; k < NACC; ++k)
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[k], 0, 0, 0);
  } else {
    const float a = seed + 1.f, b = seed - 1.f;
    for (int64_t i = 0; i < iters; ++i)
#pragma unroll
      for (int k = 0; k < NACC; ++k)
        acc[k] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[k], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < NACC; ++k) s += acc[k][0] + acc[k][1] + acc[k][2] + acc[k][3];
  if (s == 1234.5f) sink[threadIdx.x] = s;  // practically never; keeps the chains live
}

// The attention core's per-key-block instruction mix at its tile (two rows x
// 64 queries per wave, 32 keys per block, head dim 32): 40 MFMA 16x16x32
// bf16 (QK^T 16, PV 16, row sums 8), 64 v_exp_f32 (2 x 64 x 32 scores / 64
// lanes) and 32 v_cvt_pk_bf16_f32 (the bf16 P operand), with no memory
// traffic.  kParts: 1 = the MFMAs alone, 2 = the exponentials alone (the
// packs have no consumer there and are dropped), 3 = the whole mix.  The exponentials are 64
// independent chains x <- exp2(-x) (bounded, fixed point ~0.64); the packed
// results feed the next iteration's MFMA A operands, as P feeds PV.
template <int kParts>
__global__ __launch_bounds__(256) void mix_probe_kernel(float* __restrict__ sink, int64_t iters) {
  constexpr bool kM = kParts & 1, kV = kParts & 2;
  f32x4 acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float seed = 1e-3f * (float)(threadIdx.x & 63);
  float e[64];
#pragma unroll
  for (int k = 0; k < 64; ++k) e[k] = seed + 0.01f * k;
  bf16x8 p[8], b;
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int t = 0; t < 8; ++t) p[k][t] = (bf16)(seed + t);
#pragma unroll
  for (int t = 0; t < 8; ++t) b[t] = (bf16)(seed - t);
  for (int64_t it = 0; it < iters; ++it) {
    if constexpr (kM) {
#pragma unroll
      for (int k = 0; k < 40; ++k)
        acc[k & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p[k & 7], b, acc[k & 7], 0, 0, 0);
    }
    if constexpr (kV) {
#pragma unroll
      for (int k = 0; k < 64; ++k) e[k] = __builtin_amdgcn_exp2f(-e[k]);
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int t = 0; t < 8; ++t) p[k][t] = (bf16)e[8 * k + t];  // v_cvt_pk_bf16_f32 pairs
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += acc[k][0] + (float)p[k][0];
#pragma unroll
  for (int k = 0; k < 64; ++k) s += e[k];
  if (s == 1234.5f) sink[threadIdx.x] = s;  // practically never; keeps the work live
}

// Streaming bandwidth: each thread moves 4 x 16 bytes per trip of a grid-
// stride loop with the non-temporal policy (kStream), as the row-tile kernels
// stream pair data.  kMode 0: read only (a practically-never-taken store keeps
// the loads live); 1: copy; 2: rewrite dst in place with its own bits.
template <int kMode>
__global__ __launch_bounds__(256) void stream_probe_kernel(const f32x4* __restrict__ src,
                                                           f32x4* __restrict__ dst, uint64_t n16) {
  constexpr int U = 4;
  const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  i32x4_t acc = {0, 0, 0, 0};
  for (uint64_t i = (uint64_t)blockIdx.x * 256 * U + threadIdx.x; i < n16; i += stride) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (i + u * 256 < n16) v[u] = load_stream((kMode == 2 ? dst : src) + i + u * 256);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (i + u * 256 >= n16) continue;
      if constexpr (kMode == 0) {
        acc ^= __builtin_bit_cast(i32x4_t, v[u]);
      } else {
        asm volatile("" : "+v"(v[u]));  // the in-place rewrite is not elided
        store_stream(dst + i + u * 256, v[u]);
      }
    }
  }
  if constexpr (kMode == 0)
    if ((acc[0] & acc[1] & acc[2] & acc[3]) == 0x7f7f7f7f)
      reinterpret_cast<float*>(dst)[threadIdx.x] = 1.f;  // practically never
}

}  // namespace odde

using namespace odde;

extern "C" {

const char* odde_probe_last_error(void) { return g_probe_error.c_str(); }

int odde_probe_mfma(int dtype, int64_t iters, int grid, float* sink, double* flops,
                    void* stream) {
  if (!sink || !flops || iters <= 0 || grid <= 0)
    return probe_error("probe_mfma: bad argument");
  if (dtype != ODDE_PROBE_BF16 && dtype != ODDE_PROBE_F32)
    return probe_error("probe_mfma: dtype must be ODDE_PROBE_BF16 or ODDE_PROBE_F32");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // flops per instruction: 2 * 16 * 16 * K (K = 32 bf16, 4 f32)
  const double per = 2.0 * 16 * 16 * (dtype == ODDE_PROBE_BF16 ? 32 : 4);
  *flops = per * 8.0 * (double)iters * 4.0 * (double)grid;  // 8 chains, 4 waves per workgroup
  if (dtype == ODDE_PROBE_BF16)
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(grid), dim3(256), 0, st, sink, iters);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(grid), dim3(256), 0, st, sink, iters);
  return probe_launched("probe_mfma");
}

int odde_probe_stream(int mode, const void* src, void* dst, uint64_t bytes, void* stream) {
  if (mode < 0 || mode > 2) return probe_error("probe_stream: mode must be 0, 1 or 2");
  if (!dst || (mode != 2 && !src) || bytes == 0 || bytes % 16 != 0)
    return probe_error("probe_stream: bad argument (bytes: a positive multiple of 16)");
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0)
    return probe_error("probe_stream: buffers must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  const uint64_t n16 = bytes / 16;
  const uint64_t want = (n16 + 1023) / 1024;  // 4 chunks per thread per trip
  const int grid = (int)(want < 8192 ? want : 8192);
  const f32x4* s4 = static_cast<const f32x4*>(src);
  f32x4* d4 = static_cast<f32x4*>(dst);
  switch (mode) {
    case 0: hipLaunchKernelGGL(stream_probe_kernel<0>, dim3(grid), dim3(256), 0, st, s4, d4, n16); break;
    case 1: hipLaunchKernelGGL(stream_probe_kernel<1>, dim3(grid), dim3(256), 0, st, s4, d4, n16); break;
    default: hipLaunchKernelGGL(stream_probe_kernel<2>, dim3(grid), dim3(256), 0, st, s4, d4, n16);
  }
  return probe_launched("probe_stream");
}

int odde_probe_mix(int parts, int64_t iters, int grid, float* sink, double* flops,
                   void* stream) {
  if (!sink || !flops || iters <= 0 || grid <= 0)
    return probe_error("probe_mix: bad argument");
  if (parts < 1 || parts > 3) return probe_error("probe_mix: parts must be 1, 2 or 3");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the attention flops one iteration stands for: QK^T and PV of 2 rows x 64
  // queries x 32 keys x head dim 32 (2 * 2 * 2 * 64 * 32 * 32), per wave
  *flops = 524288.0 * (double)iters * 4.0 * (double)grid;
  switch (parts) {
    case 1: hipLaunchKernelGGL(mix_probe_kernel<1>, dim3(grid), dim3(256), 0, st, sink, iters); break;
    case 2: hipLaunchKernelGGL(mix_probe_kernel<2>, dim3(grid), dim3(256), 0, st, sink, iters); break;
    default: hipLaunchKernelGGL(mix_probe_kernel<3>, dim3(grid), dim3(256), 0, st, sink, iters);
  }
  return probe_launched("probe_mix");
}

}  // extern "C"
