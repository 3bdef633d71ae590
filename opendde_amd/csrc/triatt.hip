// Triangle attention (starting node over a strided pair view) for gfx950.
//
// Three kernels, stream ordered:
//   1. triatt_proj  — LayerNorm + one pass of bias-free projections per pair
//                     row: q (pre-scaled by log2(e)/sqrt(D)), k, v, sigmoid(g),
//                     the triangle bias (pre-scaled by log2(e)) and the
//                     additive mask row, written in the layouts the core
//                     reads with whole-fragment 16-byte loads.
//   2. triatt_core  — flash-style attention: per (row i, head h, 32-query
//                     tile) stream 32-key blocks, S^T = bias + mask + K Q^T
//                     on MFMA (bias folded into the accumulator init), online
//                     softmax in fp32 with exp2, O^T += V^T P^T on MFMA with
//                     P kept in registers; epilogue 1/l and the sigmoid gate.
//                     The N x N x N logits never touch memory.
//   3. triatt_out   — o W_o^T on MFMA plus the residual add, written through
//                     the (possibly transposed) output strides.
//
// Workspace layouts (CT = compute type, Jp = N rounded up to 64):
//   q, k, gate : [I][H][Jp][32]
//   v          : [I][H][Jp/32][2][64][8]   MFMA-ready V^T fragments: block of
//                32 keys x 32 channels; channel half db, lane (d%16 + 16*g),
//                slot e holds key 4g+e (e<4) or 16+4g+(e-4) (e>=4)
//   bias       : [Bb][H][Jp][Jp]   (log2e-scaled tri bias; Bb bias batches)
//   mb         : [I][Jp] f32       (log2e-scaled additive mask; -inf on pads)
//   o          : [I][Jp][H*32]     (gated attention output, module path)
#include "common.hpp"
#include "runtime.hpp"

namespace odde {

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
  CT* bias;
  float* mb;
  int n, jp, heads;
  float q_scale;   // log2(e) / sqrt(D)
  float mask_inf;  // inf * log2(e)
  float eps;
};

__device__ __forceinline__ size_t vperm_offset(int row, int h, int heads, int jp, int j, int d) {
  const int kb = j >> 5, jj = j & 31;
  const int half = jj >> 4, gp = (jj & 15) >> 2, e = 4 * half + (jj & 3);
  const int db = d >> 4, dl = d & 15;
  return (((((size_t)row * heads + h) * (jp >> 5) + kb) * 2 + db) * 64 + dl + 16 * gp) * 8 + e;
}

template <typename ZT, typename CT, int kC>
__global__ __launch_bounds__(256) void triatt_proj_kernel(TriattProjArgs<ZT, CT> a) {
  constexpr int C = kC * 32;
  const int i = blockIdx.y;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int j0 = blockIdx.x * 64 + w * 16;
  const int jl = j0 + r16;
  const bool valid = jl < a.n;
  const ZT* rowp = a.z + (int64_t)i * a.z_s0 + (int64_t)(valid ? jl : 0) * a.z_s1;
  Frag<CT> x[kC];
  ln_rows_to_frags<ZT, CT, C>(rowp, valid, a.ln_w, a.ln_b, a.eps, x);

  const int H = a.heads, HD = H * 32, jp = a.jp;

  // q, k, gate: product W x^T -> lane holds pair row jl, channels o..o+3.
  for (int ob = 0; ob < HD / 16; ++ob) {
    f32x4 aq = {0.f, 0.f, 0.f, 0.f}, ak = aq, ag = aq;
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      Frag<CT> f;
      load_w_frag(a.wq, C, ob * 16, HD, t, f);
      mma(aq, f, x[t]);
      load_w_frag(a.wk, C, ob * 16, HD, t, f);
      mma(ak, f, x[t]);
      load_w_frag(a.wg, C, ob * 16, HD, t, f);
      mma(ag, f, x[t]);
    }
    const int o = ob * 16 + 4 * g;
    const int h = o >> 5, d = o & 31;
    const size_t off = (((size_t)i * H + h) * jp + jl) * 32 + d;
    const float s = a.q_scale;
    store4(a.q + off, aq[0] * s, aq[1] * s, aq[2] * s, aq[3] * s);
    store4(a.k + off, ak[0], ak[1], ak[2], ak[3]);
    store4(a.gate + off, sigmoidf_(ag[0]), sigmoidf_(ag[1]), sigmoidf_(ag[2]), sigmoidf_(ag[3]));
  }

  // v: product x W^T -> lane holds channel o, pair rows j0+4g .. +3.
  const int jb = j0 + 4 * g;
  for (int ob = 0; ob < HD / 16; ++ob) {
    f32x4 av = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      Frag<CT> f;
      load_w_frag(a.wv, C, ob * 16, HD, t, f);
      mma(av, x[t], f);
    }
    const int o = ob * 16 + r16;
    store4(a.v + vperm_offset(i, o >> 5, H, jp, jb, o & 31), av[0], av[1], av[2], av[3]);
  }

  // triangle bias: channel h = r16 (< H), rows jb..jb+3 -> bias[h][i][jb..]
  {
    f32x4 ab = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kC; ++t) {
      Frag<CT> f;
      load_w_frag(a.wb, C, 0, H, t, f);
      mma(ab, x[t], f);
    }
    if (r16 < H) {
      const float s = kLog2e;
      store4(a.bias + ((size_t)r16 * jp + i) * jp + jb, ab[0] * s, ab[1] * s, ab[2] * s,
             ab[3] * s);
    }
  }

  // additive mask row: mb[i][j] = inf*(mask-1)*log2e, -inf past the last token
  if (g == 0) {
    float v = -INFINITY;
    if (valid) {
      const float m = a.mask ? a.mask[(int64_t)i * a.m_s0 + (int64_t)jl * a.m_s1] : 1.0f;
      v = (m - 1.0f) * a.mask_inf;
    }
    a.mb[(size_t)i * jp + jl] = v;
  }
}

// ---------------------------------------------------------------------------
// 2. flash core
// ---------------------------------------------------------------------------
template <typename CT>
struct TriattCoreArgs {
  const CT* q;
  const CT* k;
  const CT* v;
  const CT* bias;
  const float* mb;
  const CT* gate;  // may be null
  CT* out;
  int64_t o_row, o_h, o_j;  // element strides of out[row][h][q][d]
  int rows, heads, n, jp, rows_per_bias;
};

template <typename CT>
__global__ __launch_bounds__(256) void triatt_core_kernel(TriattCoreArgs<CT> a) {
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int row = blockIdx.y * 4 + w;
  if (row >= a.rows) return;  // no barriers in this kernel: an early exit is safe
  const int h = blockIdx.z;
  const int q0 = blockIdx.x * 32;
  const int jp = a.jp, n = a.n;
  const size_t rh = (size_t)row * a.heads + h;
  const CT* Q = a.q + rh * jp * 32;
  const CT* K = a.k + rh * jp * 32;
  const CT* V = a.v + rh * jp * 32;
  const CT* B = a.bias + ((size_t)(row / a.rows_per_bias) * a.heads + h) * jp * jp;
  const float* MB = a.mb + (size_t)row * jp;

  Frag<CT> qf[2];
  const CT* brow[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qq = q0 + 16 * qb + r16;
    qf[qb].load(Q + (size_t)qq * 32 + 8 * g);
    brow[qb] = B + (size_t)min(qq, n - 1) * jp;
  }

  f32x4 o[2][2];
#pragma unroll
  for (int db = 0; db < 2; ++db)
    for (int qb = 0; qb < 2; ++qb) o[db][qb] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m[2] = {-1e30f, -1e30f};
  float lsum[2] = {0.f, 0.f};

  for (int k0 = 0; k0 < jp; k0 += 32) {
    Frag<CT> kf[2];
    float mbv[2][4];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      kf[kb].load(K + (size_t)(k0 + 16 * kb + r16) * 32 + 8 * g);
      load4(MB + k0 + 16 * kb + 4 * g, mbv[kb]);
    }
    f32x4 s[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        float bv[4];
        load4(brow[qb] + k0 + 16 * kb + 4 * g, bv);
        s[kb][qb] = f32x4{bv[0] + mbv[kb][0], bv[1] + mbv[kb][1], bv[2] + mbv[kb][2],
                          bv[3] + mbv[kb][3]};
        mma(s[kb][qb], kf[kb], qf[qb]);
      }
    Frag<CT> pf[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float mx = s[0][qb][0];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        for (int r = 0; r < 4; ++r) mx = fmaxf(mx, s[kb][qb][r]);
      mx = group_max(mx);
      const float mnew = fmaxf(m[qb], mx);
      const float sc = __builtin_amdgcn_exp2f(m[qb] - mnew);
      m[qb] = mnew;
      float ps = 0.f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        for (int r = 0; r < 4; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[kb][qb][r] - mnew);
          ps += p;
          pf[qb].set(4 * kb + r, p);
        }
      lsum[qb] = lsum[qb] * sc + ps;
#pragma unroll
      for (int db = 0; db < 2; ++db) o[db][qb] *= sc;
    }
    const CT* vb = V + (size_t)(k0 >> 5) * 1024;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      Frag<CT> vf;
      vf.load(vb + (db * 64 + l) * 8);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) mma(o[db][qb], vf, pf[qb]);
    }
  }

#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const float inv = 1.0f / group_sum(lsum[qb]);
    const int qq = q0 + 16 * qb + r16;
    if (qq >= n) continue;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
      const int d0 = 16 * db + 4 * g;
      float ov[4];
      for (int r = 0; r < 4; ++r) ov[r] = o[db][qb][r] * inv;
      if (a.gate) {
        float gv[4];
        load4(a.gate + (rh * jp + qq) * 32 + d0, gv);
        for (int r = 0; r < 4; ++r) ov[r] *= gv[r];
      }
      store4(a.out + (int64_t)row * a.o_row + (int64_t)h * a.o_h + (int64_t)qq * a.o_j + d0,
             ov[0], ov[1], ov[2], ov[3]);
    }
  }
}

// ---------------------------------------------------------------------------
// 3. output projection + residual
// ---------------------------------------------------------------------------
template <typename ZT, typename CT>
struct TriattOutArgs {
  const CT* o;  // [I][Jp][HD]
  const CT* wo; // [C][HD]
  const ZT* res;
  int64_t r_s0, r_s1;
  ZT* out;
  int64_t o_s0, o_s1;
  int n, jp, c;
  int add;
};

template <typename ZT, typename CT, int kHD>
__global__ __launch_bounds__(256) void triatt_out_kernel(TriattOutArgs<ZT, CT> a) {
  constexpr int HD = kHD * 32;
  const int i = blockIdx.y;
  const int w = wave_id(), l = lane_id(), g = l >> 4, r16 = l & 15;
  const int jl = blockIdx.x * 64 + w * 16 + r16;
  const bool valid = jl < a.n;
  Frag<CT> x[kHD];
  const CT* orow = a.o + ((size_t)i * a.jp + jl) * HD;
#pragma unroll
  for (int t = 0; t < kHD; ++t) {
    if (valid) x[t].load(orow + 32 * t + 8 * g);
    else x[t].zero();
  }
  for (int cb = 0; cb < a.c / 16; ++cb) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < kHD; ++t) {
      Frag<CT> f;
      load_w_frag(a.wo, HD, cb * 16, a.c, t, f);
      mma(acc, f, x[t]);
    }
    if (!valid) continue;
    const int c0 = cb * 16 + 4 * g;
    float base[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.add) load4(a.res + (int64_t)i * a.r_s0 + (int64_t)jl * a.r_s1 + c0, base);
    store4(a.out + (int64_t)i * a.o_s0 + (int64_t)jl * a.o_s1 + c0, base[0] + acc[0],
           base[1] + acc[1], base[2] + acc[2], base[3] + acc[3]);
  }
}

// ---------------------------------------------------------------------------
// 4. relayout for the core-only slot: strided q/k/v/bias/mask -> core layouts
// ---------------------------------------------------------------------------
template <typename CT>
struct RelayoutArgs {
  const CT* q; int64_t q_sb, q_si, q_sh, q_sj;
  const CT* k; int64_t k_sb, k_si, k_sh, k_sj;
  const CT* v; int64_t v_sb, v_si, v_sh, v_sj;
  const float* bias; int64_t b_sb, b_sh, b_sq, b_sk;
  const uint8_t* mask; int64_t m_sb, m_si, m_sk;
  CT* wq; CT* wk; CT* wv; CT* wbias; float* wmb;
  int batch, rows, heads, n, jp;
  float q_scale, mask_inf;
};

// One thread per (row r = b*I+i, head h, key j) moves 32 channels of q, k, v;
// threads with h == 0 also write the additive mask row.
template <typename CT>
__global__ __launch_bounds__(256) void triatt_relayout_kernel(RelayoutArgs<CT> a) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)a.batch * a.rows * a.heads * a.jp;
  if (tid >= total) return;
  const int j = (int)(tid % a.jp);
  const int h = (int)((tid / a.jp) % a.heads);
  const int64_t r = tid / ((int64_t)a.jp * a.heads);
  const int b = (int)(r / a.rows), i = (int)(r % a.rows);
  const bool valid = j < a.n;
  const size_t off = (((size_t)r * a.heads + h) * a.jp + j) * 32;
  const CT* qs = a.q + b * a.q_sb + i * a.q_si + h * a.q_sh + (int64_t)(valid ? j : 0) * a.q_sj;
  const CT* ks = a.k + b * a.k_sb + i * a.k_si + h * a.k_sh + (int64_t)(valid ? j : 0) * a.k_sj;
  const CT* vs = a.v + b * a.v_sb + i * a.v_si + h * a.v_sh + (int64_t)(valid ? j : 0) * a.v_sj;
  for (int d = 0; d < 32; ++d) {
    const float qv = valid ? to_f32(qs[d]) * a.q_scale : 0.f;
    const float kv = valid ? to_f32(ks[d]) : 0.f;
    const float vv = valid ? to_f32(vs[d]) : 0.f;
    a.wq[off + d] = from_f32<CT>(qv);
    a.wk[off + d] = from_f32<CT>(kv);
    a.wv[vperm_offset((int)r, h, a.heads, a.jp, j, d)] = from_f32<CT>(vv);
  }
  if (h == 0) {
    float mv = -INFINITY;
    if (valid) {
      const bool keep = a.mask ? a.mask[b * a.m_sb + i * a.m_si + (int64_t)j * a.m_sk] != 0 : true;
      mv = keep ? 0.f : -a.mask_inf;
    }
    a.wmb[(size_t)r * a.jp + j] = mv;
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
  a.wbias[tid] = from_f32<CT>(bv);
}

}  // namespace odde

// ===========================================================================
// host side
// ===========================================================================
using namespace odde;

namespace {

struct TriattWs {
  void* q; void* k; void* v; void* gate; void* o; void* bias; float* mb;
  uint64_t bytes;
};

TriattWs carve_triatt(void* base, uint64_t size, int n, int heads, int dt) {
  const int jp = round_up(n, 64);
  const uint64_t es = dtype_size(dt);
  const uint64_t per = (uint64_t)n * heads * jp * 32;
  Carver c(base, size);
  TriattWs w;
  w.q = c.take<char>(per * es);
  w.k = c.take<char>(per * es);
  w.v = c.take<char>(per * es);
  w.gate = c.take<char>(per * es);
  w.o = c.take<char>(per * es);
  w.bias = c.take<char>((uint64_t)heads * jp * jp * es);
  w.mb = c.take<float>((uint64_t)n * jp);
  w.bytes = (c.used + 255) & ~uint64_t(255);
  return w;
}

int check_triatt(const odde_triatt_args* a) {
  if (!a) return set_error(ODDE_EINVAL, "triatt: null args");
  if (a->struct_size != sizeof(odde_triatt_args))
    return set_error(ODDE_EINVAL, "triatt: struct_size mismatch (ABI version skew)");
  if (a->n <= 0 || a->c <= 0 || a->heads <= 0)
    return set_error(ODDE_EINVAL, "triatt: n, c and heads must be positive");
  if (a->head_dim != 32) return set_error(ODDE_EUNSUPPORTED, "triatt: head_dim must be 32");
  if (a->heads > 16) return set_error(ODDE_EUNSUPPORTED, "triatt: at most 16 heads");
  if (!valid_dtype(a->z_dtype) || !valid_dtype(a->compute_dtype))
    return set_error(ODDE_EINVAL, "triatt: bad dtype");
  if (a->z_dtype == ODDE_BF16 && a->compute_dtype == ODDE_F32)
    return set_error(ODDE_EUNSUPPORTED, "triatt: bf16 storage with f32 compute");
  return ODDE_OK;
}

template <typename ZT, typename CT, int kC>
void launch_proj(const TriattProjArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  dim3 grid(jp / 64, n);
  hipLaunchKernelGGL((triatt_proj_kernel<ZT, CT, kC>), grid, dim3(256), 0, st, p);
}

template <typename ZT, typename CT, int kHD>
void launch_out(const TriattOutArgs<ZT, CT>& p, int n, int jp, hipStream_t st) {
  dim3 grid(jp / 64, n);
  hipLaunchKernelGGL((triatt_out_kernel<ZT, CT, kHD>), grid, dim3(256), 0, st, p);
}

template <typename CT>
int launch_core(const TriattCoreArgs<CT>& p, hipStream_t st) {
  dim3 grid(p.jp / 32, (p.rows + 3) / 4, p.heads);
  LaunchScope ls(ODDE_K_TRIATT_CORE, st);
  hipLaunchKernelGGL((triatt_core_kernel<CT>), grid, dim3(256), 0, st, p);
  return check_launch("triatt_core");
}

template <typename ZT, typename CT>
int run_triatt(const odde_triatt_args* a, hipStream_t st) {
  const int n = a->n, H = a->heads, C = a->c, HD = H * 32;
  const int jp = round_up(n, 64);
  TriattWs ws = carve_triatt(a->workspace, a->workspace_bytes, n, H, a->compute_dtype);

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
  p.q = static_cast<CT*>(ws.q); p.k = static_cast<CT*>(ws.k); p.v = static_cast<CT*>(ws.v);
  p.gate = static_cast<CT*>(ws.gate); p.bias = static_cast<CT*>(ws.bias); p.mb = ws.mb;
  p.n = n; p.jp = jp; p.heads = H;
  p.q_scale = kLog2e / sqrtf((float)a->head_dim);
  p.mask_inf = a->inf * kLog2e;
  p.eps = a->eps;
  {
    LaunchScope ls(ODDE_K_TRIATT_PROJ, st);
    switch (C) {
      case 64: launch_proj<ZT, CT, 2>(p, n, jp, st); break;
      case 128: launch_proj<ZT, CT, 4>(p, n, jp, st); break;
      case 256: launch_proj<ZT, CT, 8>(p, n, jp, st); break;
      case 384: launch_proj<ZT, CT, 12>(p, n, jp, st); break;
      default: return set_error(ODDE_EUNSUPPORTED, "triatt: c must be 64, 128, 256 or 384");
    }
    int rc = check_launch("triatt_proj");
    if (rc) return rc;
  }

  TriattCoreArgs<CT> c;
  c.q = p.q; c.k = p.k; c.v = p.v; c.bias = p.bias; c.mb = p.mb; c.gate = p.gate;
  c.out = static_cast<CT*>(ws.o);
  c.o_row = (int64_t)jp * HD; c.o_h = 32; c.o_j = HD;
  c.rows = n; c.heads = H; c.n = n; c.jp = jp; c.rows_per_bias = n;
  int rc = launch_core<CT>(c, st);
  if (rc) return rc;

  TriattOutArgs<ZT, CT> o;
  o.o = static_cast<const CT*>(ws.o);
  o.wo = static_cast<const CT*>(a->w_o);
  o.res = static_cast<const ZT*>(a->z); o.r_s0 = a->z_s0; o.r_s1 = a->z_s1;
  o.out = static_cast<ZT*>(a->out); o.o_s0 = a->out_s0; o.o_s1 = a->out_s1;
  o.n = n; o.jp = jp; o.c = C; o.add = a->add_residual;
  {
    LaunchScope ls(ODDE_K_TRIATT_OUT, st);
    switch (HD) {
      case 64: launch_out<ZT, CT, 2>(o, n, jp, st); break;
      case 128: launch_out<ZT, CT, 4>(o, n, jp, st); break;
      case 256: launch_out<ZT, CT, 8>(o, n, jp, st); break;
      case 384: launch_out<ZT, CT, 12>(o, n, jp, st); break;
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
  *bytes = carve_triatt(nullptr, 0, a->n, a->heads, a->compute_dtype).bytes;
  return ODDE_OK;
}

int odde_triatt_fwd(const odde_triatt_args* a, void* stream) {
  int rc = check_triatt(a);
  if (rc) return rc;
  if (!a->z || !a->out || !a->ln_w || !a->ln_b || !a->w_bias || !a->w_q || !a->w_k ||
      !a->w_v || !a->w_g || !a->w_o)
    return set_error(ODDE_EINVAL, "triatt: null tensor pointer");
  const uint64_t need = carve_triatt(nullptr, 0, a->n, a->heads, a->compute_dtype).bytes;
  if (!a->workspace || a->workspace_bytes < need ||
      (reinterpret_cast<uintptr_t>(a->workspace) & 255))
    return set_error(ODDE_EWORKSPACE, "triatt: workspace missing, too small or not 256-byte aligned");
  const int zes = dtype_size(a->z_dtype);
  if ((reinterpret_cast<uintptr_t>(a->z) | reinterpret_cast<uintptr_t>(a->out)) & 15 ||
      ((a->z_s0 | a->z_s1 | a->out_s0 | a->out_s1) * zes) & 15)
    return set_error(ODDE_EINVAL, "triatt: z/out rows must be 16-byte aligned");
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (a->z_dtype == ODDE_F32 && a->compute_dtype == ODDE_F32) return run_triatt<float, float>(a, st);
  if (a->z_dtype == ODDE_F32 && a->compute_dtype == ODDE_BF16) return run_triatt<float, bf16>(a, st);
  return run_triatt<bf16, bf16>(a, st);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// core-only slot
// ---------------------------------------------------------------------------
namespace {

struct CoreWs { void* q; void* k; void* v; void* bias; float* mb; uint64_t bytes; };

CoreWs carve_core(void* base, uint64_t size, const odde_triatt_core_args* a) {
  const int jp = round_up(a->n, 64);
  const uint64_t es = dtype_size(a->dtype);
  const uint64_t rows = (uint64_t)a->batch * a->rows;
  const uint64_t per = rows * a->heads * jp * 32;
  Carver c(base, size);
  CoreWs w;
  w.q = c.take<char>(per * es);
  w.k = c.take<char>(per * es);
  w.v = c.take<char>(per * es);
  w.bias = c.take<char>((uint64_t)a->batch * a->heads * jp * jp * es);
  w.mb = c.take<float>(rows * jp);
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
  if (!valid_dtype(a->dtype)) return set_error(ODDE_EINVAL, "triatt_core: bad dtype");
  return ODDE_OK;
}

template <typename CT>
int run_core(const odde_triatt_core_args* a, hipStream_t st) {
  const int jp = round_up(a->n, 64);
  CoreWs ws = carve_core(a->workspace, a->workspace_bytes, a);
  RelayoutArgs<CT> r;
  r.q = static_cast<const CT*>(a->q); r.q_sb = a->q_sb; r.q_si = a->q_si; r.q_sh = a->q_sh; r.q_sj = a->q_sj;
  r.k = static_cast<const CT*>(a->k); r.k_sb = a->k_sb; r.k_si = a->k_si; r.k_sh = a->k_sh; r.k_sj = a->k_sj;
  r.v = static_cast<const CT*>(a->v); r.v_sb = a->v_sb; r.v_si = a->v_si; r.v_sh = a->v_sh; r.v_sj = a->v_sj;
  r.bias = a->bias; r.b_sb = a->b_sb; r.b_sh = a->b_sh; r.b_sq = a->b_sq; r.b_sk = a->b_sk;
  r.mask = a->mask; r.m_sb = a->m_sb; r.m_si = a->m_si; r.m_sk = a->m_sk;
  r.wq = static_cast<CT*>(ws.q); r.wk = static_cast<CT*>(ws.k); r.wv = static_cast<CT*>(ws.v);
  r.wbias = static_cast<CT*>(ws.bias); r.wmb = ws.mb;
  r.batch = a->batch; r.rows = a->rows; r.heads = a->heads; r.n = a->n; r.jp = jp;
  r.q_scale = a->scale * kLog2e;
  r.mask_inf = a->inf_value * kLog2e;
  {
    const int64_t total = (int64_t)a->batch * a->rows * a->heads * jp;
    const int64_t total_b = (int64_t)a->batch * a->heads * jp * jp;
    LaunchScope ls(ODDE_K_TRIATT_RELAYOUT, st);
    hipLaunchKernelGGL((triatt_relayout_kernel<CT>), dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, st, r);
    hipLaunchKernelGGL((triatt_bias_relayout_kernel<CT>),
                       dim3((unsigned)((total_b + 255) / 256)), dim3(256), 0, st, r);
    int rc = check_launch("triatt_relayout");
    if (rc) return rc;
  }
  TriattCoreArgs<CT> c;
  c.q = r.wq; c.k = r.wk; c.v = r.wv; c.bias = r.wbias; c.mb = r.wmb; c.gate = nullptr;
  c.out = static_cast<CT*>(a->out);
  c.o_row = a->o_si;  // rows are (b, i) with o_sb == rows * o_si checked by the caller
  c.o_h = a->o_sh; c.o_j = a->o_sj;
  c.rows = a->batch * a->rows; c.heads = a->heads; c.n = a->n; c.jp = jp;
  c.rows_per_bias = a->rows;
  return launch_core<CT>(c, st);
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
