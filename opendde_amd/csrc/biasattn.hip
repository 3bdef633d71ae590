// Single-track attention with an additive pair bias, in fp32 (the
// AttentionPairBias core: primitives._attention, opendde/model/modules/
// primitives.py:220-258, which upcasts q, k, v and the bias to fp32 and runs
// SDPA with scale 1):
//   out[h][i][:] = sum_j softmax_j(s q[h][i] . k[h][j] + bias[h][i][j]) v[h][j][:]
// with the query scale s (Attention._prep_qkv's 1 / sqrt(c_hidden),
// primitives.py:755-756) and, optionally, the output gate of
// Attention._wrap_up (primitives.py:772-776), out *= sigmoid(gate), applied
// at the store.
//
// One workgroup per (head, 64 queries); within it, KS groups of 4 waves
// (KS = 4 for head dims up to 32, else 1) take disjoint ranges of key blocks
// and merge their partial softmaxes at the end; wave w of a group takes
// queries 16 w .. 16 w + 15.  Key blocks of 64 are staged in LDS as f32 by
// 16-byte loads (the next block's are loaded into registers while a block is
// computed).  Per 16 keys of a block, on the fp32 MFMA
// (v_mfma_f32_16x16x4_f32, true fp32 products):
//   S^T[key][query] = K Q^T over head-dim steps of 4 (lane: key l % 16 of the
//   A operand, query l % 16 of B, dims 4 s + l / 16),
//   plus the bias, online softmax per query (running max across the four
//   16-lane groups, exp2 of log2e-scaled logits),
//   O^T[dim][query] += V^T P^T in four key steps: step kk takes the
//   accumulator's register kk of every lane (key 4 (l / 16) + kk) as the B
//   operand and V[key 4 (l / 16) + kk][dim l % 16] as the A operand, so P
//   needs no shuffle.
#include "common.hpp"
#include "runtime.hpp"

namespace odde {

constexpr int kBaMaxD = 64;
constexpr int kBaK = 64;  // keys per staged block

struct BiasAttnArgs {
  const void* q; const void* k; const void* v;
  int64_t q_sh, q_sn, k_sh, k_sn, v_sh, v_sn;  // head and row strides (elements)
  const float* bias;                          // [H][Nq][Nk] or null
  void* out;
  int64_t o_sh, o_sn;
  const void* gate;  // [H][Nq][D] strides g_sh, g_sn, or null: out *= sigmoid(gate)
  int64_t g_sh, g_sn;
  float q_scale;     // multiplies q . k
  int nq, nk;
};

__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Keys are split over KS groups of four waves (KS = 4 for head dims up to 32,
// whose K/V blocks are small): group s runs the online softmax over its own
// range of key blocks with its own LDS staging, and the groups' partial
// (max, sum, output) are merged in LDS at the end.  With one workgroup per
// (head, 64 queries) a single group would leave one wave per SIMD.
template <int D> struct BaSplit { static constexpr int KS = D <= 32 ? 4 : 1; };

template <typename T, int D>
__global__ __launch_bounds__(256 * BaSplit<D>::KS) void bias_attn_kernel(BiasAttnArgs a) {
  constexpr int KS = BaSplit<D>::KS;
  constexpr int NS = D / 4;          // head-dim steps of the QK^T product
  constexpr int NT = (D + 15) / 16;  // 16-dim tiles of the output
  constexpr int LD = D + 1;          // LDS row pitch (floats)
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int CPR = D / VEC;       // 16-byte chunks per key row
  constexpr int CHUNKS = kBaK * CPR; // per operand and block
  constexpr int PER = (CHUNKS + 255) / 256;
  static_assert(D % VEC == 0, "rows of whole 16-byte chunks");
  typedef T tvec __attribute__((ext_vector_type(VEC)));
  // group s stages its K block at kv + 2 s kBaK LD and its V block right after
  __shared__ float kv[KS * 2 * kBaK * LD];
  const int sp = wave_id() / 4, w = wave_id() % 4, tid = threadIdx.x % 256;
  const int l = lane_id(), g = l >> 4, r16 = l & 15;
  const int h = blockIdx.y, qi = blockIdx.x * 64 + 16 * w + r16;
  const bool qvalid = qi < a.nq;
  const T* qp = static_cast<const T*>(a.q) + h * a.q_sh + (int64_t)(qvalid ? qi : 0) * a.q_sn;
  float qf[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) qf[s] = qvalid ? to_f32(qp[4 * s + g]) * (a.q_scale * kLog2e) : 0.f;
  const T* kb = static_cast<const T*>(a.k) + h * a.k_sh;
  const T* vb = static_cast<const T*>(a.v) + h * a.v_sh;
  const float* brow = a.bias ? a.bias + ((int64_t)h * a.nq + (qvalid ? qi : 0)) * a.nk : nullptr;
  const bool bvec = (a.nk & 3) == 0;
  // this group's key blocks [blk0, blk1); every group runs nbs steps so that
  // the workgroup's barriers match
  const int nblk = (a.nk + kBaK - 1) / kBaK, nbs = (nblk + KS - 1) / KS;
  const int blk0 = sp * nbs, blk1 = min(nblk, blk0 + nbs);

  tvec kr[PER], vr[PER];  // the next block's chunks
  auto fetch = [&](int j0) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int c = tid + 256 * u, key = j0 + c / CPR, d0 = (c % CPR) * VEC;
      const bool in = c < CHUNKS && key < a.nk;
      tvec zk, zv;
      for (int e = 0; e < VEC; ++e) zk[e] = zv[e] = (T)0.f;
      kr[u] = in ? *reinterpret_cast<const tvec*>(kb + (int64_t)key * a.k_sn + d0) : zk;
      vr[u] = in ? *reinterpret_cast<const tvec*>(vb + (int64_t)key * a.v_sn + d0) : zv;
    }
  };
  float m = -INFINITY, lsum = 0.f;
  f32x4 o[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (blk0 < blk1) fetch(blk0 * kBaK);
  float* kss = kv + 2 * sp * kBaK * LD;
  float* vss = kss + kBaK * LD;
  for (int b = 0; b < nbs; ++b) {
    const int blk = blk0 + b, j0 = blk * kBaK;
    const bool live = blk < blk1;
    __syncthreads();  // the previous block is no longer read
    if (live) {
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int c = tid + 256 * u;
        if (c < CHUNKS) {
          const int key = c / CPR, d0 = (c % CPR) * VEC;
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            kss[key * LD + d0 + e] = to_f32(kr[u][e]);
            vss[key * LD + d0 + e] = to_f32(vr[u][e]);
          }
        }
      }
    }
    __syncthreads();
    if (!live) continue;
    if (blk + 1 < blk1) fetch(j0 + kBaK);  // in flight during this block
    const int nsub = min(kBaK, a.nk - j0);
    for (int sb = 0; sb < nsub; sb += 16) {
      const int k0 = j0 + sb;
      // bias[qi][k0 + 4 g + r]
      float bc[4] = {0.f, 0.f, 0.f, 0.f};
      if (brow) {
        if (bvec && k0 + 4 * g + 3 < a.nk) {
          const f32x4 b4 = *reinterpret_cast<const f32x4*>(brow + k0 + 4 * g);
#pragma unroll
          for (int r = 0; r < 4; ++r) bc[r] = b4[r];
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (k0 + 4 * g + r < a.nk) bc[r] = brow[k0 + 4 * g + r];
        }
      }
      f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NS; ++s)  // [key 4g + r][query r16]
        sacc = mfma4(kss[(sb + r16) * LD + 4 * s + g], qf[s], sacc);
      float sv[4], bm = -INFINITY;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int key = k0 + 4 * g + r;
        sv[r] = key < a.nk ? fmaf(bc[r], kLog2e, sacc[r]) : -INFINITY;
        bm = fmaxf(bm, sv[r]);
      }
      bm = group_max_fast(bm);
      const float mn = fmaxf(m, bm);  // finite: every 16-key step has a key
      const float scale = __builtin_amdgcn_exp2f(m - mn);  // 0 at the first step
      lsum *= scale;
#pragma unroll
      for (int t = 0; t < NT; ++t) o[t] *= scale;
      m = mn;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[r] = __builtin_amdgcn_exp2f(sv[r] - mn);
        lsum += p[r];
      }
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const int d = 16 * t + r16;
          const float vv = d < D ? vss[(sb + 4 * g + kk) * LD + d] : 0.f;
          o[t] = mfma4(vv, p[kk], o[t]);  // [dim][query r16]
        }
    }
  }
  lsum = group_sum_fast(lsum);
  if constexpr (KS > 1) {
    // merge the groups' partial softmaxes: groups 1.. leave (m, lsum, o) per
    // lane in LDS (the staging area, free once every group left its loop) and
    // group 0 merges them into its own
    constexpr int W = 2 + 4 * NT;  // floats per lane
    static_assert((KS - 1) * 256 * W <= KS * 2 * kBaK * LD, "merge area fits the staging area");
    __syncthreads();
    if (sp > 0) {
      float* dst = kv + ((sp - 1) * 256 + w * 64 + l) * W;
      dst[0] = m;
      dst[1] = lsum;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[2 + 4 * t + r] = o[t][r];
    }
    __syncthreads();
    if (sp > 0) return;
#pragma unroll
    for (int s = 1; s < KS; ++s) {
      const float* src = kv + ((s - 1) * 256 + w * 64 + l) * W;
      const float ms = src[0];
      const float mn = fmaxf(m, ms);  // finite: group 0 always holds key 0
      const float fa = __builtin_amdgcn_exp2f(m - mn), fb = __builtin_amdgcn_exp2f(ms - mn);
      lsum = lsum * fa + src[1] * fb;
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) o[t][r] = o[t][r] * fa + src[2 + 4 * t + r] * fb;
      m = mn;
    }
  }
  if (!qvalid) return;
  const float inv = 1.0f / lsum;
  T* op = static_cast<T*>(a.out) + h * a.o_sh + (int64_t)qi * a.o_sn;
  const T* gp = a.gate ? static_cast<const T*>(a.gate) + h * a.g_sh + (int64_t)qi * a.g_sn : nullptr;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int d = 16 * t + 4 * g + r;
      if (d >= D) continue;
      float y = o[t][r] * inv;
      if (gp) y *= sigmoidf_(to_f32(gp[d]));
      op[d] = from_f32<T>(y);
    }
}

namespace {

template <typename T>
int launch_bias_attn(const odde_bias_attn_args* x, hipStream_t st) {
  BiasAttnArgs a;
  a.q = x->q; a.k = x->k; a.v = x->v;
  a.q_sh = x->q_sh; a.q_sn = x->q_sn; a.k_sh = x->k_sh; a.k_sn = x->k_sn;
  a.v_sh = x->v_sh; a.v_sn = x->v_sn;
  a.bias = x->bias; a.out = x->out; a.o_sh = x->o_sh; a.o_sn = x->o_sn;
  a.gate = x->gate; a.g_sh = x->g_sh; a.g_sn = x->g_sn;
  a.q_scale = x->q_scale == 0.f ? 1.f : x->q_scale;
  a.nq = x->n_q; a.nk = x->n_k;
  LaunchScope ls(ODDE_K_BIAS_ATTN, st);
  dim3 grid((x->n_q + 63) / 64, x->heads);
  switch (x->head_dim) {
#define ODDE_BA(D) \
    case D:                                                                            \
      hipLaunchKernelGGL((bias_attn_kernel<T, D>), grid, dim3(256 * BaSplit<D>::KS), 0, st, a); \
      break;
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
  {
    const int64_t es = x->dtype == ODDE_F32 ? 4 : 2;
    if (((reinterpret_cast<uintptr_t>(x->k) | reinterpret_cast<uintptr_t>(x->v)) & 15) ||
        ((x->k_sh * es) | (x->k_sn * es) | (x->v_sh * es) | (x->v_sn * es)) & 15)
      return set_error(ODDE_EINVAL, "bias_attn: k and v rows must be 16-byte aligned");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  return x->dtype == ODDE_F32 ? launch_bias_attn<float>(x, st) : launch_bias_attn<bf16>(x, st);
}
