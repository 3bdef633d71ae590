// Single-track attention with an additive pair bias, in fp32 (the
// AttentionPairBias core: primitives._attention, opendde/model/modules/
// primitives.py:220-258, which upcasts q, k, v and the bias to fp32 and runs
// SDPA with scale 1):
//   out[h][i][:] = sum_j softmax_j(q[h][i] . k[h][j] + bias[h][i][j]) v[h][j][:]
//
// One workgroup of 256 threads per (head, 16 queries), so that a head of
// 1024 queries fills 64 workgroups and the pair stack's 16 heads give four
// workgroups per CU.  Key blocks of 128 are staged in LDS as f32 (K and V,
// head dim D; the next block and this thread's bias values are loaded into
// registers while a block is computed); the 16 threads of a query take keys
// part, part + 16, ... of each block, keep their own running max, sum and output (the online
// softmax), and merge the 16 partial results (max-rescaled) by lane shuffles
// at the end.  All arithmetic is f32; the exponentials are exp2 of
// log2e-scaled logits.
#include "common.hpp"
#include "runtime.hpp"

namespace odde {

constexpr int kBaTPQ = 16;             // threads per query
constexpr int kBaQ = 256 / kBaTPQ;     // queries per workgroup
constexpr int kBaK = 128;              // keys per staged block
constexpr int kBaKPT = kBaK / kBaTPQ;  // keys per thread per block
constexpr int kBaMaxD = 64;

struct BiasAttnArgs {
  const void* q; const void* k; const void* v;
  int64_t q_sh, q_sn, k_sh, k_sn, v_sh, v_sn;  // head and row strides (elements)
  const float* bias;                          // [H][Nq][Nk] or null
  void* out;
  int64_t o_sh, o_sn;
  int nq, nk;
};

// The next key block's K and V values (kBaK * D of each, spread over the 256
// threads) and this thread's bias values, loaded into registers while the
// current block is computed.
template <typename T, int D>
struct BaPrefetch {
  static constexpr int PER = (kBaK * D + 255) / 256;
  T kv[2][PER];
  float b[kBaKPT];
};

template <typename T, int D>
__global__ __launch_bounds__(256) void bias_attn_kernel(BiasAttnArgs a) {
  constexpr int LDK = D + 4;  // LDS row pitch (floats): the parts' rows land on distinct banks
  using PF = BaPrefetch<T, D>;
  __shared__ __attribute__((aligned(16))) float ks[kBaK * LDK];
  __shared__ __attribute__((aligned(16))) float vs[kBaK * LDK];
  const int h = blockIdx.y, i0 = blockIdx.x * kBaQ;
  const int t = threadIdx.x, qi = t / kBaTPQ, part = t % kBaTPQ;
  const int i = i0 + qi;
  const bool valid = i < a.nq;
  const T* qp = static_cast<const T*>(a.q) + h * a.q_sh + (int64_t)(valid ? i : 0) * a.q_sn;
  float q[D];
#pragma unroll
  for (int d = 0; d < D; ++d) q[d] = to_f32(qp[d]) * kLog2e;
  const float* brow = a.bias ? a.bias + ((int64_t)h * a.nq + (valid ? i : 0)) * a.nk : nullptr;
  float m = -INFINITY, lsum = 0.f, o[D];
#pragma unroll
  for (int d = 0; d < D; ++d) o[d] = 0.f;
  const T* kb = static_cast<const T*>(a.k) + h * a.k_sh;
  const T* vb = static_cast<const T*>(a.v) + h * a.v_sh;
  PF pf;
  auto fetch = [&](int j0) {
    const int nj = min(kBaK, a.nk - j0);
#pragma unroll
    for (int u = 0; u < PF::PER; ++u) {
      const int e = t + 256 * u, r = e / D, d = e % D;
      const bool in = e < kBaK * D && r < nj;
      pf.kv[0][u] = in ? kb[(int64_t)(j0 + r) * a.k_sn + d] : T(0.f);
      pf.kv[1][u] = in ? vb[(int64_t)(j0 + r) * a.v_sn + d] : T(0.f);
    }
#pragma unroll
    for (int u = 0; u < kBaKPT; ++u) {
      const int r = kBaTPQ * u + part;
      pf.b[u] = (brow && r < nj) ? brow[j0 + r] : 0.f;
    }
  };
  fetch(0);
  for (int j0 = 0; j0 < a.nk; j0 += kBaK) {
    const int nj = min(kBaK, a.nk - j0);
    __syncthreads();  // the previous block's K, V are no longer read
#pragma unroll
    for (int u = 0; u < PF::PER; ++u) {
      const int e = t + 256 * u;
      if (e < kBaK * D) {
        const int r = e / D, d = e % D;
        ks[r * LDK + d] = to_f32(pf.kv[0][u]);
        vs[r * LDK + d] = to_f32(pf.kv[1][u]);
      }
    }
    float bcur[kBaKPT];
#pragma unroll
    for (int u = 0; u < kBaKPT; ++u) bcur[u] = pf.b[u];
    __syncthreads();
    if (j0 + kBaK < a.nk) fetch(j0 + kBaK);  // in flight during this block
    // this thread's keys of the block: logits (log2 units), block max
    float s[kBaKPT];
    float bm = -INFINITY;
#pragma unroll
    for (int u = 0; u < kBaKPT; ++u) {
      const int r = kBaTPQ * u + part;
      const float* kr = ks + r * LDK;
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; ++d) acc = fmaf(q[d], kr[d], acc);
      acc = fmaf(bcur[u], kLog2e, acc);
      s[u] = r < nj ? acc : -INFINITY;
      bm = fmaxf(bm, s[u]);
    }
    const float mn = fmaxf(m, bm);
    if (mn > -INFINITY) {
      const float scale = __builtin_amdgcn_exp2f(m - mn);  // 0 on the first block
      lsum *= scale;
#pragma unroll
      for (int d = 0; d < D; ++d) o[d] *= scale;
#pragma unroll
      for (int u = 0; u < kBaKPT; ++u) {
        const float p = __builtin_amdgcn_exp2f(s[u] - mn);  // 0 for keys past the end
        lsum += p;
        const float* vr = vs + (kBaTPQ * u + part) * LDK;
#pragma unroll
        for (int d = 0; d < D; ++d) o[d] = fmaf(p, vr[d], o[d]);
      }
      m = mn;
    }
  }
  // merge the parts of the query (consecutive lanes of one wave)
#pragma unroll
  for (int x = 1; x < kBaTPQ; x <<= 1) {
    const float m2 = __shfl_xor(m, x, 64);
    const float l2 = __shfl_xor(lsum, x, 64);
    const float mn = fmaxf(m, m2);
    const float s1 = mn > -INFINITY ? __builtin_amdgcn_exp2f(m - mn) : 0.f;
    const float s2 = mn > -INFINITY ? __builtin_amdgcn_exp2f(m2 - mn) : 0.f;
    lsum = lsum * s1 + l2 * s2;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const float o2 = __shfl_xor(o[d], x, 64);
      o[d] = o[d] * s1 + o2 * s2;
    }
    m = mn;
  }
  if (!valid) return;
  const float inv = 1.0f / lsum;
  T* op = static_cast<T*>(a.out) + h * a.o_sh + (int64_t)i * a.o_sn;
  // part p writes dims p, p + 16, ...
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (d % kBaTPQ == part) op[d] = from_f32<T>(o[d] * inv);
}

namespace {

template <typename T>
int launch_bias_attn(const odde_bias_attn_args* x, hipStream_t st) {
  BiasAttnArgs a;
  a.q = x->q; a.k = x->k; a.v = x->v;
  a.q_sh = x->q_sh; a.q_sn = x->q_sn; a.k_sh = x->k_sh; a.k_sn = x->k_sn;
  a.v_sh = x->v_sh; a.v_sn = x->v_sn;
  a.bias = x->bias; a.out = x->out; a.o_sh = x->o_sh; a.o_sn = x->o_sn;
  a.nq = x->n_q; a.nk = x->n_k;
  LaunchScope ls(ODDE_K_BIAS_ATTN, st);
  dim3 grid((x->n_q + kBaQ - 1) / kBaQ, x->heads);
  switch (x->head_dim) {
#define ODDE_BA(D) \
    case D: hipLaunchKernelGGL((bias_attn_kernel<T, D>), grid, dim3(256), 0, st, a); break;
    ODDE_BA(8) ODDE_BA(16) ODDE_BA(24) ODDE_BA(32) ODDE_BA(48) ODDE_BA(64)
#undef ODDE_BA
    default: return set_error(ODDE_EUNSUPPORTED, "bias_attn: head_dim in {8, 16, 24, 32, 48, 64}");
  }
  return check_launch("bias_attn");
}

}  // namespace
}  // namespace odde

using namespace odde;

extern "C" int odde_bias_attn_fwd(const odde_bias_attn_args* x, void* stream) {
  if (!x) return set_error(ODDE_EINVAL, "bias_attn: null args");
  if (x->struct_size != sizeof(odde_bias_attn_args))
    return set_error(ODDE_EINVAL, "bias_attn: struct_size mismatch (ABI version skew)");
  if (x->n_q < 0 || x->n_k < 0 || x->heads < 0 || x->head_dim <= 0)
    return set_error(ODDE_EINVAL, "bias_attn: bad sizes");
  if (x->head_dim > kBaMaxD)
    return set_error(ODDE_EUNSUPPORTED, "bias_attn: head_dim in {8, 16, 24, 32, 48, 64}");
  if (!valid_dtype(x->dtype)) return set_error(ODDE_EINVAL, "bias_attn: bad dtype");
  if (x->n_q == 0 || x->heads == 0) return ODDE_OK;
  if (x->n_k == 0) return set_error(ODDE_EINVAL, "bias_attn: no keys");
  if (!x->q || !x->k || !x->v || !x->out) return set_error(ODDE_EINVAL, "bias_attn: null tensor pointer");
  if (x->heads > 65535) return set_error(ODDE_EUNSUPPORTED, "bias_attn: at most 65535 heads");
  hipStream_t st = static_cast<hipStream_t>(stream);
  return x->dtype == ODDE_F32 ? launch_bias_attn<float>(x, st) : launch_bias_attn<bf16>(x, st);
}
