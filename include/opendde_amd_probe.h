/* Measurement library of opendde_amd: machine-rate probes for benchmarks.
 *
 * Built apart from the product library, as libopendde_amd_probe.so; it has no
 * counterpart in the reference and nothing in the Pairformer path uses it.
 * Each probe launches on `hip_stream` and returns at once (0, or a negative
 * status with a message in odde_probe_last_error()); time it with events on
 * that stream. */
#ifndef OPENDDE_AMD_PROBE_H
#define OPENDDE_AMD_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ODDE_PROBE_F32 0
#define ODDE_PROBE_BF16 1
#define ODDE_PROBE_BF16_RANDOM 2

/* Message of the last failed probe call on this thread ("" if none). */
const char* odde_probe_last_error(void);

/* MFMA rate: launches `grid` workgroups of 4 waves that each run 8
 * independent MFMA accumulator chains of `iters` instructions (dtype
 * ODDE_PROBE_BF16: v_mfma_f32_16x16x32_bf16 on one fixed operand pair;
 * ODDE_PROBE_BF16_RANDOM: the same instruction on pseudo-random operands that
 * change from one instruction to the next, as a GEMM's do -- the rate this
 * GPU sustains under its power limit on real data; ODDE_PROBE_F32:
 * v_mfma_f32_16x16x4_f32) and returns the flops it performs in *flops.
 * `sink`: 256 floats of device memory (practically never written). */
int odde_probe_mfma(int dtype, int64_t iters, int grid, float* sink, double* flops,
                    void* hip_stream);

/* Co-issue: the triangle-attention core's per-key-block instruction mix at
 * its tile -- 40 MFMA 16x16x32 bf16, 64 v_exp_f32, 32 v_cvt_pk_bf16_f32 per
 * iteration, no memory traffic -- on `grid` workgroups of 4 waves.  parts:
 * 1 = the MFMAs alone, 2 = the exponentials alone, 3 = the whole mix,
 * 4 = the mix split between the two waves that share a SIMD (one issues the
 * MFMAs, the other the exponentials and packs; `grid` workgroups of 8 waves,
 * one mix per wave pair and iteration): the most co-issue of the two kinds.
 * *flops: the attention flops the iterations stand for (QK^T and PV of 2 rows
 * x 64 queries x 32 keys x head dim 32 per wave and iteration), so flops /
 * time is the core's ceiling on this GPU. */
int odde_probe_mix(int parts, int64_t iters, int grid, float* sink, double* flops,
                   void* hip_stream);

/* Streaming bandwidth: the HBM rate a kernel that touches its data once can
 * reach with the non-temporal cache policy the row-tile kernels use.  mode 0
 * reads `bytes` of src (dst: at least 256 floats, practically never
 * written); mode 1 copies src to dst; mode 2 rewrites dst in place with its
 * own contents (src unused).  bytes: a positive multiple of 16; 16-byte
 * aligned buffers.  The traffic is `bytes` for mode 0 and 2 * bytes
 * otherwise. */
int odde_probe_stream(int mode, const void* src, void* dst, uint64_t bytes, void* hip_stream);

#ifdef __cplusplus
}
#endif
#endif /* OPENDDE_AMD_PROBE_H */
