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
// keeps the results live.  kMode 0: bf16 with one fixed operand pair;
// 1: f32; 2: bf16 with four operand pairs of pseudo-random values in
// [-0.5, 0.5) per lane, taken in turn (the operands change from one
// instruction to the next, as in a GEMM; the matrix pipe's switching power,
// and with it the clock this GPU sustains under its power limit, depends on
// the data).

template <int kMode>
__global__ __launch_bounds__(256) void mfma_probe_kernel(float* __restrict__ sink, int64_t iters) {
  constexpr int NACC = 8;
  f32x4 acc[NACC];
#pragma unroll
  for (int k = 0; k < NACC; ++k) acc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  const float seed = 1e-3f * (float)(threadIdx.x & 63);
  if constexpr (kMode == 0) {
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
  } else if constexpr (kMode == 2) {
    bf16x8 a[4], b[4];
    uint32_t h = (uint32_t)threadIdx.x * 2654435761u + (uint32_t)blockIdx.x * 40503u + 12345u;
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h = h * 1664525u + 1013904223u;
        a[t][e] = (bf16)((float)(h >> 8) * (1.0f / 16777216.0f) - 0.5f);
        h = h * 1664525u + 1013904223u;
        b[t][e] = (bf16)((float)(h >> 8) * (1.0f / 16777216.0f) - 0.5f);
      }
    // two rounds per trip, so that every operand index is a constant
    for (int64_t i = 0; i < iters; i += 2)
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int k = 0; k < NACC; ++k)
          acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[k & 3], b[(k >> 2) + 2 * r], acc[k],
                                                           0, 0, 0);
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

// The same mix split between the two waves that share a SIMD: in a
// workgroup of 8 waves (waves w and w + 4 on one SIMD), waves 0-3 issue only
// the 40 MFMAs of an iteration and waves 4-7 only its 64 exponentials and 32
// packs, so that every cycle one wave of each SIMD has MFMA work and the
// other VALU work: the most co-issue the two kinds can get on this GPU.
// Per iteration a wave pair performs the mix of one wave of mix_probe_kernel.
__global__ __launch_bounds__(512) void mix_split_probe_kernel(float* __restrict__ sink,
                                                              int64_t iters) {
  const bool mfma_wave = (threadIdx.x >> 6) < 4;
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
  if (mfma_wave) {
    for (int64_t it = 0; it < iters; ++it)
#pragma unroll
      for (int k = 0; k < 40; ++k)
        acc[k & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p[k & 7], b, acc[k & 7], 0, 0, 0);
  } else {
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
      for (int k = 0; k < 64; ++k) e[k] = __builtin_amdgcn_exp2f(-e[k]);
#pragma unroll
      for (int k = 0; k < 8; ++k)
#pragma unroll
        for (int t = 0; t < 8; ++t) p[k][t] = (bf16)e[8 * k + t];  // v_cvt_pk_bf16_f32 pairs
      if (e[0] == 12345.f) {  // practically never; keeps every pack live
#pragma unroll
        for (int k = 0; k < 8; ++k)
          *reinterpret_cast<bf16x8*>(sink + 4 * k) = p[k];
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k) s += acc[k][0] + (float)p[k][0];
#pragma unroll
  for (int k = 0; k < 64; ++k) s += e[k];
  if (s == 1234.5f) sink[threadIdx.x & 255] = s;  // practically never
}

// Streaming bandwidth: each thread moves 4 x 16 bytes per trip of a grid-
// stride loop with the non-temporal policy (kStream), as the row-tile kernels
// stream pair data; whole trips run without bounds checks, the ragged end
// (fewer than grid x 1024 chunks) with them.  kMode 0: read only (a
// practically-never-taken store keeps the loads live); 1: copy; 2: rewrite
// dst in place with its own bits.
template <int kMode>
__global__ __launch_bounds__(256) void stream_probe_kernel(const f32x4* __restrict__ src,
                                                           f32x4* __restrict__ dst, uint64_t n16) {
  constexpr int U = 4;
  const uint64_t stride = (uint64_t)gridDim.x * 256 * U;
  const uint64_t whole = n16 / stride * stride;
  typedef int i32x4_t __attribute__((ext_vector_type(4)));
  i32x4_t acc = {0, 0, 0, 0};
  const f32x4* in = kMode == 2 ? dst : src;
  uint64_t i = (uint64_t)blockIdx.x * 256 * U + threadIdx.x;
  for (; i < whole; i += stride) {
    f32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = load_stream(in + i + u * 256);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if constexpr (kMode == 0) {
        acc ^= __builtin_bit_cast(i32x4_t, v[u]);
      } else {
        asm volatile("" : "+v"(v[u]));  // the in-place rewrite is not elided
        store_stream(dst + i + u * 256, v[u]);
      }
    }
  }
  // the ragged end: this thread's chunks of the last, partial trip
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint64_t j = i + u * 256;
    if (j >= n16) continue;
    f32x4 v = load_stream(in + j);
    if constexpr (kMode == 0) {
      acc ^= __builtin_bit_cast(i32x4_t, v);
    } else {
      asm volatile("" : "+v"(v));
      store_stream(dst + j, v);
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
  if (dtype != ODDE_PROBE_BF16 && dtype != ODDE_PROBE_F32 && dtype != ODDE_PROBE_BF16_RANDOM)
    return probe_error(
        "probe_mfma: dtype must be ODDE_PROBE_BF16, ODDE_PROBE_F32 or ODDE_PROBE_BF16_RANDOM");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // flops per instruction: 2 * 16 * 16 * K (K = 32 bf16, 4 f32)
  const double per = 2.0 * 16 * 16 * (dtype == ODDE_PROBE_F32 ? 4 : 32);
  if (dtype == ODDE_PROBE_BF16_RANDOM) iters += iters & 1;  // whole trips of two rounds
  *flops = per * 8.0 * (double)iters * 4.0 * (double)grid;  // 8 chains, 4 waves per workgroup
  if (dtype == ODDE_PROBE_BF16)
    hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3(grid), dim3(256), 0, st, sink, iters);
  else if (dtype == ODDE_PROBE_BF16_RANDOM)
    hipLaunchKernelGGL(mfma_probe_kernel<2>, dim3(grid), dim3(256), 0, st, sink, iters);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3(grid), dim3(256), 0, st, sink, iters);
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
  const int grid = (int)(want < 16384 ? want : 16384);
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
  if (parts < 1 || parts > 4) return probe_error("probe_mix: parts must be 1, 2, 3 or 4");
  hipStream_t st = static_cast<hipStream_t>(stream);
  // the attention flops one iteration stands for: QK^T and PV of 2 rows x 64
  // queries x 32 keys x head dim 32 (2 * 2 * 2 * 64 * 32 * 32), per wave
  *flops = 524288.0 * (double)iters * 4.0 * (double)grid;
  if (parts == 4) {  // workgroups of 8 waves: 4 wave pairs, one mix per pair and iteration
    hipLaunchKernelGGL(mix_split_probe_kernel, dim3(grid), dim3(512), 0, st, sink, iters);
    return probe_launched("probe_mix");
  }
  switch (parts) {
    case 1: hipLaunchKernelGGL(mix_probe_kernel<1>, dim3(grid), dim3(256), 0, st, sink, iters); break;
    case 2: hipLaunchKernelGGL(mix_probe_kernel<2>, dim3(grid), dim3(256), 0, st, sink, iters); break;
    default: hipLaunchKernelGGL(mix_probe_kernel<3>, dim3(grid), dim3(256), 0, st, sink, iters);
  }
  return probe_launched("probe_mix");
}

}  // extern "C"
