// Machine-rate probe: the MFMA throughput this GPU actually sustains, so that
// kernel figures can be quoted against a measured peak as well as the data
// sheet's.  Every wave runs 8 independent accumulator chains of one MFMA
// shape for `iters` rounds; nothing is loaded, one conditional store per lane
// keeps the results live.
#include "common.hpp"
#include "runtime.hpp"

namespace odde {

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

}  // namespace odde

using namespace odde;

extern "C" {

int odde_probe_mfma(int dtype, int64_t iters, int grid, float* sink, double* flops,
                    void* stream) {
  if (!sink || !flops || iters <= 0 || grid <= 0)
    return set_error(ODDE_EINVAL, "probe_mfma: bad argument");
  if (dtype != ODDE_BF16 && dtype != ODDE_F32)
    return set_error(ODDE_EINVAL, "probe_mfma: dtype must be ODDE_BF16 or ODDE_F32");
  hipStream_t st = static_cast<hipStream_t>(stream);
  LaunchScope ls(ODDE_K_PROBE, st);
  // flops per instruction: 2 * 16 * 16 * K (K = 32 bf16, 4 f32)
  const double per = 2.0 * 16 * 16 * (dtype == ODDE_BF16 ? 32 : 4);
  *flops = per * 8.0 * (double)iters * 4.0 * (double)grid;  // 8 chains, 4 waves per workgroup
  if (dtype == ODDE_BF16)
    hipLaunchKernelGGL(mfma_probe_kernel<true>, dim3(grid), dim3(256), 0, st, sink, iters);
  else
    hipLaunchKernelGGL(mfma_probe_kernel<false>, dim3(grid), dim3(256), 0, st, sink, iters);
  return check_launch("probe_mfma");
}

}  // extern "C"
