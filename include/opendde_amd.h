/*
 * opendde_amd — C ABI of the MI355X (gfx950) Pairformer pair-stack kernels.
 *
 * Plain C: fixed-width integers, raw device pointers, element strides, a HIP
 * stream handle passed as void*.  No torch types.  The library never
 * allocates device memory: callers pass a workspace sized by the matching
 * *_workspace_bytes query.  Every entry point returns 0 on success or a
 * negative ODDE_E* status, with a message in odde_last_error() (thread
 * local).  All work is enqueued on the given stream; nothing synchronises.
 *
 * Pair tensors are addressed as  p[x][y][c] = base + x*s0 + y*s1 + c
 * (element strides; the channel stride must be 1).  Every kernel treats its
 * view as the *starting-node / natural* orientation; the ending-node
 * (transposed) form is the same call with s0 and s1 swapped for z, the mask
 * and the output, so no transposed copy of z is ever made.
 */
#ifndef OPENDDE_AMD_H
#define OPENDDE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ODDE_ABI_VERSION 1

/* element types */
#define ODDE_F32 0
#define ODDE_BF16 1
#define ODDE_F16 2 /* LayerNorm entry points only */
/* compute_dtype of odde_triatt_fwd, odde_trimul_fwd and odde_transition_fwd
 * (their workspaces then also hold the weights split into bf16 hi | lo rows,
 * written once per call):
 * f32 data and weights, the products on the bf16 MFMA in three parts (each
 * operand as a bf16 pair hi + lo; hi*hi + hi*lo + lo*hi, f32 accumulation;
 * about 2^-16 of relative error per product): every projection, the
 * attention core, the outputs and the transition's GEMMs, and the triangle
 * contraction where Np is a multiple of 256 (true fp32 products otherwise;
 * the transition's pair-bias projection stays true fp32).  The f32 mode for
 * callers that allow reduced-precision products: the reference's kernel
 * slot and its linear layers take TF32 (2^-11) from
 * torch.backends.cuda.matmul.allow_tf32 (opendde/model/triangular/
 * triangular.py:55-56), which its inference default enables
 * (opendde/config/model_base.py:35, opendde/model/opendde.py:106). */
#define ODDE_F32X3 3

/* status codes */
#define ODDE_OK 0
#define ODDE_EINVAL -1       /* bad argument (shape, stride, dtype, null) */
#define ODDE_EUNSUPPORTED -2 /* valid but not implemented (e.g. head_dim != 32) */
#define ODDE_EWORKSPACE -3   /* workspace too small or misaligned */
#define ODDE_EHIP -4         /* HIP runtime / launch error */

/* Kernel ids for odde_launch_count / odde_timing_query. */
#define ODDE_K_TRIATT_PROJ 0
#define ODDE_K_TRIATT_CORE 1
#define ODDE_K_TRIATT_OUT 2
#define ODDE_K_TRIMUL_PROJ 3
#define ODDE_K_TRIMUL_CONTRACT 4
#define ODDE_K_TRIMUL_OUT 5
#define ODDE_K_TRIATT_RELAYOUT 6
#define ODDE_K_TRANSITION 7
#define ODDE_K_LAYER_NORM 8
#define ODDE_K_LAYER_NORM_BWD 9
#define ODDE_K_OPM 10
#define ODDE_K_BIAS_ATTN 11
#define ODDE_K_COUNT 12

int odde_abi_version(void);
const char* odde_last_error(void);

/*
 * Triangle attention, whole module (starting node over the given view):
 *   x = LN(z);  tri_bias[h,q,k] = x[q,k] . w_bias[h];  q,k,v,g = x W^T per head
 *   o[i,q] = softmax_k( q[i,q].k[i,k]/sqrt(D) + inf*(mask[i,k]-1) + tri_bias[q,k] ) v[i,k]
 *   update[i,q] = W_o( sigmoid(g[i,q]) * o[i,q] )
 *   out = (add_residual ? z : 0) + update          (out may alias z)
 * Replaces the reference's TriangleAttention.forward + Attention.forward
 * (opendde/model/triangular/triangular.py:648-706,
 *  opendde/model/triangular/layers.py:426-481) on a GPU tensor.
 * Weights are in compute_dtype, row-major [out][in]; LN params are f32.
 */
typedef struct odde_triatt_args {
  uint32_t struct_size; /* sizeof(odde_triatt_args) */
  int32_t n;            /* tokens: the view is n x n */
  int32_t c;            /* channels of z */
  int32_t heads;        /* H */
  int32_t head_dim;     /* D (32) */
  int32_t z_dtype;      /* ODDE_F32 / ODDE_BF16: z, out */
  int32_t compute_dtype;/* ODDE_F32 / ODDE_BF16: weights, intermediates, MFMA */
  int32_t add_residual;
  const void* z;
  int64_t z_s0, z_s1;
  const float* mask; /* may be NULL (all ones) */
  int64_t mask_s0, mask_s1;
  void* out;
  int64_t out_s0, out_s1;
  const float* ln_w;
  const float* ln_b;
  const void* w_bias; /* [H][C]  (TriangleAttention.linear)   */
  const void* w_q;    /* [H*D][C] mha.linear_q                */
  const void* w_k;
  const void* w_v;
  const void* w_g;    /* [H*D][C] mha.linear_g                */
  const void* w_o;    /* [C][H*D] mha.linear_o                */
  float inf;          /* 1e9 */
  float eps;          /* 1e-5 */
  void* workspace;
  uint64_t workspace_bytes;
  /* Leading batch dims flattened to one count (the reference's modules take
   * z [*, N, N, C], triangular.py:648-706).  batch = 0 or 1: one view.  With
   * batch = B > 1, view b reads z + b*z_sb and mask + b*mask_sb and writes
   * out + b*out_sb (strides in elements; mask_sb may be 0 for a broadcast
   * mask).  One call runs the B views in order on the stream, sharing one
   * workspace of the size odde_triatt_workspace_bytes reports. */
  int32_t batch;
  int64_t z_sb, mask_sb, out_sb;
} odde_triatt_args;

int odde_triatt_workspace_bytes(const odde_triatt_args* args, uint64_t* bytes);
int odde_triatt_fwd(const odde_triatt_args* args, void* hip_stream);

/*
 * Triangle attention core only — the slot the reference fills with
 * cuequivariance_triangular_attn(q, k, v, bias, mask, scale)
 * (opendde/model/triangular/layers.py:484-494, called at :462-472):
 *   out[b,i,h,q,:] = softmax_k( scale*q.k + bias[b,h,q,k] + mask_term ) v[b,i,h,k,:]
 * q, k, v, out: [B][I][H][J][D] with arbitrary element strides (D contiguous);
 * bias: [B][H][J][J] f32 (the reference passes [B,1,H,J,J]);
 * mask: [B][I][J] uint8, nonzero = keep; dropped keys get -inf_value
 * (the reference's torch path uses -1e9, layers.py:472 / triangular.py:677);
 * mask may be NULL.  dtype is that of q, k, v and out.
 */
typedef struct odde_triatt_core_args {
  uint32_t struct_size;
  int32_t batch, rows, heads, n, head_dim; /* B, I, H, J, D */
  int32_t dtype;
  const void* q; int64_t q_sb, q_si, q_sh, q_sj;
  const void* k; int64_t k_sb, k_si, k_sh, k_sj;
  const void* v; int64_t v_sb, v_si, v_sh, v_sj;
  const float* bias; int64_t b_sb, b_sh, b_sq, b_sk;
  const uint8_t* mask; int64_t m_sb, m_si, m_sk;
  void* out; int64_t o_sb, o_si, o_sh, o_sj;
  float scale;
  float inf_value; /* 1e9 */
  void* workspace;
  uint64_t workspace_bytes;
} odde_triatt_core_args;

int odde_triatt_core_workspace_bytes(const odde_triatt_core_args* args, uint64_t* bytes);
int odde_triatt_core_fwd(const odde_triatt_core_args* args, void* hip_stream);

/*
 * Triangle multiplicative update, whole module:
 *   x = LN_in(z); a = mask*sigmoid(x Wag^T)*(x Wap^T); b likewise
 *   outgoing: p[i,j] = sum_k a[i,k]*b[j,k];  incoming: p[i,j] = sum_k a[k,i]*b[k,j]
 *   update = (LN_out(p) W_z^T) * sigmoid(x W_g^T)
 *   out = (add_residual ? z : 0) + update          (out may alias z)
 * Argument list of kernel_triangular_mult
 * (opendde/model/triangular/triangular.py:17-30, called at :498-515):
 * p_in_weight = cat(linear_a_p, linear_b_p), g_in_weight = cat(linear_a_g,
 * linear_b_g), p_out_weight = linear_z, g_out_weight = linear_g.
 */
typedef struct odde_trimul_args {
  uint32_t struct_size;
  int32_t n;
  int32_t c;        /* c_z */
  int32_t c_hidden; /* Ch */
  int32_t z_dtype;
  int32_t compute_dtype;
  int32_t outgoing; /* 1 = outgoing (Alg. 11), 0 = incoming (Alg. 12) */
  int32_t add_residual;
  const void* z;
  int64_t z_s0, z_s1;
  const float* mask; /* may be NULL */
  int64_t mask_s0, mask_s1;
  void* out;
  int64_t out_s0, out_s1;
  const float* norm_in_weight;
  const float* norm_in_bias;
  const float* norm_out_weight;
  const float* norm_out_bias;
  const void* p_in_weight;  /* [2*Ch][C] */
  const void* g_in_weight;  /* [2*Ch][C] */
  const void* p_out_weight; /* [C][Ch]   */
  const void* g_out_weight; /* [C][C]    */
  float eps;
  void* workspace;
  uint64_t workspace_bytes;
  /* Optional (may be NULL): p_out_weight in f32.  With bf16 compute the
   * output projection takes LN_out(p) W_z^T as rstd (p W'^T - mean s) + c,
   * W' = W_z diag(norm_out_weight) rounded to bf16 once, s = row sums of W',
   * c = W_z norm_out_bias: p enters the MFMA as stored, with no second
   * rounding after the LayerNorm.  W' is formed from this f32 copy when it
   * is given (one rounding), else from the bf16 p_out_weight. */
  const float* p_out_weight_f32;
  /* Leading batch dims, with the meaning they have in odde_triatt_args; the
   * reference's module takes z [*, N, N, C] (triangular.py:459-567). */
  int32_t batch;
  int64_t z_sb, mask_sb, out_sb;
} odde_trimul_args;

int odde_trimul_workspace_bytes(const odde_trimul_args* args, uint64_t* bytes);
int odde_trimul_fwd(const odde_trimul_args* args, void* hip_stream);

/*
 * Fused SwiGLU transition on rows of c channels (block member of the pair
 * stack; replaces Transition.forward, opendde/model/modules/primitives.py:
 * 182-217, whose flat row chunking is numerically neutral):
 *   y = LN(x); out = (add_residual ? x : 0) + (silu(y W_a^T) * (y W_b^T)) W_o^T
 * x, out: [rows][c] contiguous (out may alias x); W_a, W_b: [n*c][c],
 * W_o: [c][n*c] in compute_dtype; LN params f32.  c in {64, 128, 256, 384},
 * n = 4.  compute_dtype ODDE_BF16 takes f32 or bf16 rows; ODDE_F32 (true
 * fp32 products) and ODDE_F32X3 (three-part products) take f32 rows.
 * Optional (pb_heads = 16; 0 = off): the pair-bias projection that the single
 * track's AttentionPairBias takes from the updated pair tensor
 * (linear_nobias_z(layernorm_z(z)), opendde/model/modules/transformer.py:
 * 599-602), computed from the rows as written:
 *   pb_out[h][r] = sum_c LN'(out[r])[c] * pb_w[h][c]     (f32, [16][rows])
 * with LN' = LayerNorm(pb_ln_w, pb_ln_b (may be NULL), pb_eps); pb_w is
 * [16][c] in compute_dtype.  This saves the separate pass over all of z.
 * Wide rows (c = 384) in bf16 arithmetic run as a LayerNorm pass and two
 * GEMMs whose hidden activations live in the workspace
 * (odde_transition_workspace_bytes; 0 for the fused kernels, which need
 * none), and the pair-bias projection as a pass over the rows written.
 * fp32 arithmetic with few rows keeps split-hidden partial sums there, and
 * ODDE_F32X3 the weights split into bf16 hi | lo rows (3 n c^2 floats).
 */
typedef struct odde_transition_args {
  uint32_t struct_size;
  int32_t c;
  int32_t n_factor;
  int32_t x_dtype;
  int32_t compute_dtype;
  int32_t add_residual;
  int64_t rows;
  const void* x;
  void* out;
  const float* ln_w;
  const float* ln_b;
  const void* w_a;
  const void* w_b;
  const void* w_o;
  float eps;
  int32_t pb_heads;
  const float* pb_ln_w;
  const float* pb_ln_b;
  const void* pb_w;
  float* pb_out;
  float pb_eps;
  void* workspace;
  uint64_t workspace_bytes;
} odde_transition_args;

int odde_transition_workspace_bytes(const odde_transition_args* args, uint64_t* bytes);
int odde_transition_fwd(const odde_transition_args* args, void* hip_stream);

/*
 * LayerNorm over the last n2 elements of n1 contiguous rows, forward and
 * backward: the contract of the reference's optional fast LayerNorm
 * extension (its 8 entry points forward_{none,with_bias,with_weight,
 * with_both}_affine / backward_*, opendde/model/layer_norm/layer_norm.py:
 * 31-40, bound in kernel/layer_norm_cuda.cpp:143-180), selected there by
 * LAYERNORM_TYPE=fast_layernorm (opendde/model/triangular/layers.py:24-29).
 *   forward:  mean[r], invvar[r] = 1/sqrt(var[r] + eps) (f32, biased var);
 *             out = (x - mean) * invvar * gamma + beta
 *   backward: xhat = (x - mean) * invvar, g = dout * gamma,
 *             grad_input = invvar * (g - (sum g + xhat * sum g*xhat) / n2)
 *             grad_gamma = sum_rows dout * xhat, grad_beta = sum_rows dout
 * x, out, dout, grad_input, gamma, beta, grad_gamma, grad_beta share dtype
 * (ODDE_F32, ODDE_BF16 or ODDE_F16; statistics and sums are f32), all
 * contiguous [n1][n2] / [n2].  gamma / beta (and their gradients) may be
 * NULL; a NULL grad_gamma / grad_beta skips that sum.  When either is
 * requested the backward needs a workspace (16-byte aligned) for partial
 * column sums, of the size odde_layer_norm_bwd_workspace_bytes returns (a
 * function of n1, n2 and dtype only).  Results are deterministic.  n1 == 0
 * writes zero parameter gradients.
 */
typedef struct odde_layer_norm_args {
  uint32_t struct_size;
  int32_t dtype;
  int64_t n1;
  int32_t n2;
  float eps;
  const void* x;
  const void* gamma; /* may be NULL */
  const void* beta;  /* may be NULL */
  void* out;
  float* mean;
  float* invvar;
} odde_layer_norm_args;

typedef struct odde_layer_norm_bwd_args {
  uint32_t struct_size;
  int32_t dtype;
  int64_t n1;
  int32_t n2;
  const void* dout;
  const float* mean;
  const float* invvar;
  const void* x;
  const void* gamma;   /* may be NULL (then g = dout) */
  void* grad_input;
  void* grad_gamma;    /* may be NULL */
  void* grad_beta;     /* may be NULL */
  void* workspace;
  uint64_t workspace_bytes;
} odde_layer_norm_bwd_args;

int odde_layer_norm_fwd(const odde_layer_norm_args* args, void* hip_stream);
int odde_layer_norm_bwd_workspace_bytes(const odde_layer_norm_bwd_args* args, uint64_t* bytes);
int odde_layer_norm_bwd(const odde_layer_norm_bwd_args* args, void* hip_stream);

/*
 * odde_layer_norm_bwd without a workspace and without any allocation.  No
 * counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments and results as odde_layer_norm_bwd; the
 * workspace fields are ignored.  The partial column sums go to a fixed
 * 16 MiB device array inside the library (one per GPU, held until the
 * process ends): a call whose partial sums need more
 * (odde_layer_norm_bwd_workspace_bytes > 16 MiB, i.e. a large n2) returns
 * ODDE_EUNSUPPORTED.  Every call on one GPU shares that array, so calls that
 * overlap on one GPU (concurrent streams, or host threads) race; serialise
 * them.  Nothing in the array needs clearing between calls (every partial
 * row a call reads, it writes first).  Instrumentation events are not
 * recorded for it (odde_timing_*); the launch counter still counts it.
 */
int odde_layer_norm_bwd_noalloc(const odde_layer_norm_bwd_args* args, void* hip_stream);

/*
 * Attention with an additive bias in fp32: the core of the single track's
 * AttentionPairBias (replaces primitives._attention, opendde/model/modules/
 * primitives.py:220-258, which upcasts q, k, v and the bias to fp32 and runs
 * SDPA with scale 1; called from Attention.forward, :800-857):
 *   out[h][i][:] = sum_j softmax_j(s q[h][i] . k[h][j] + bias[h][i][j]) v[h][j][:]
 *                  (* sigmoid(gate[h][i][:]) when gate is given)
 * q, k, v, out: element (h, i, d) at base + h*s_h + i*s_n + d (head_dim
 * contiguous), dtype f32 or bf16 (out in the same dtype); k and v rows
 * 16-byte aligned; bias: f32 [heads][n_q][n_k] contiguous, or NULL.
 * head_dim in {8, 16, 24, 32, 48, 64}.  No workspace.
 * Optional: q_scale s (0 is read as 1; Attention._prep_qkv's q / sqrt(c_hidden),
 * primitives.py:755-756, applied in fp32), and gate (NULL = none; same dtype
 * and layout rules as q, strides g_sh, g_sn): the output gating
 * o * sigmoid(linear_g(q_x)) of Attention._wrap_up (primitives.py:772-776)
 * fused into the store.
 */
typedef struct odde_bias_attn_args {
  uint32_t struct_size;
  int32_t n_q;
  int32_t n_k;
  int32_t heads;
  int32_t head_dim;
  int32_t dtype;
  const void* q;
  int64_t q_sh, q_sn;
  const void* k;
  int64_t k_sh, k_sn;
  const void* v;
  int64_t v_sh, v_sn;
  const float* bias;
  void* out;
  int64_t o_sh, o_sn;
  const void* gate;
  int64_t g_sh, g_sn;
  float q_scale;
} odde_bias_attn_args;

int odde_bias_attn_fwd(const odde_bias_attn_args* args, void* hip_stream);

/*
 * OuterProductMean, the MSA -> pair update of the MSA module (replaces
 * OuterProductMean._forward / _opm, opendde/model/triangular/layers.py:
 * 525-616, called by MSABlock.forward, opendde/model/modules/pairformer.py:
 * 1289-1292; its row chunking is numerically neutral):
 *   y = LN(m[s][i]); a = mask[s][i] * (y W_1^T); b = mask[s][i] * (y W_2^T)
 *   upd[i][j][z] = (sum_{c1,c2} W_out[z][c1*32 + c2] sum_s a[s][i][c1] b[s][j][c2]
 *                   + b_out[z]) / (sum_s mask[s][i] mask[s][j] + eps)
 *   out = (add_residual ? out : 0) + upd    (upd rounded to bf16 first)
 * m: [n_seq][n_res][c_m] contiguous (f32 or bf16); mask: f32 [n_seq][n_res]
 * or NULL (all ones); out: [n_res][n_res][c_z] contiguous (f32 or bf16).
 * W_12 = [W_1; W_2]: [2*c_hidden][c_m], W_out: [c_z][c_hidden^2] in
 * compute_dtype (bf16 only); LN params, b_out (may be NULL) f32.  c_hidden =
 * 32; c_m in {32, 64, 128}; c_z in {64, 128, 256, 384}.  The workspace
 * (odde_opm_workspace_bytes, 256-byte aligned) holds a and b transposed, MSA
 * rows innermost.
 */
typedef struct odde_opm_args {
  uint32_t struct_size;
  int32_t n_seq;
  int32_t n_res;
  int32_t c_m;
  int32_t c_hidden;
  int32_t c_z;
  int32_t m_dtype;
  int32_t out_dtype;
  int32_t compute_dtype;
  int32_t add_residual;
  const void* m;
  const float* mask;
  const float* ln_w;
  const float* ln_b;
  const void* w_12;
  const void* w_out;
  const float* b_out;
  float ln_eps;
  float eps;
  void* out;
  void* workspace;
  uint64_t workspace_bytes;
} odde_opm_args;

int odde_opm_workspace_bytes(const odde_opm_args* args, uint64_t* bytes);
int odde_opm_fwd(const odde_opm_args* args, void* hip_stream);

/* Instrumentation (no counterpart in the reference): per-kernel launch
 * counters (always on), and optional HIP-event timing of every launch on the
 * stream it runs on.  odde_timing_query synchronises on the recorded events. */
int64_t odde_launch_count(int kernel_id);
int odde_timing_enable(int on);
int odde_timing_reset(void);
int odde_timing_query(int kernel_id, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* OPENDDE_AMD_H */
