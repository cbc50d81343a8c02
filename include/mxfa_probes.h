/*
 * mxfa_probes.h - measurement probes of libmxfa (gfx950): the ceilings the
 * flash-attention kernels of mxfa.h are measured against, and a replay of the
 * alternative to the separate dQ pass. Not part of the attention interface;
 * same conventions and status codes as mxfa.h.
 */
#ifndef MXFA_PROBES_H
#define MXFA_PROBES_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Roofline probes: measured ceilings next to the published peaks.
 * Replace the reference's throughput audit, common/kernels/isa.cu:11-63
 * (fma_f32 / dp4a_s32 / fma_h2 chains and the stream_f4 read) driven by
 * common/examples/isa.rs:17-88, with the pipes this path runs on. The caller
 * times the launches (e.g. with events on `stream`). */

/* Floats in the probes' device sink (one per probe thread). */
int mxfa_probe_sink_len(void);
/* Launches `iters` x 8 independent MFMAs per wave over 2048 x 256 threads:
 * v_mfma_f32_16x16x32_bf16 for MXFA_BF16, v_mfma_f32_16x16x4_f32 for
 * MXFA_F32. Writes the flops the launch performs to *flops. `sink` is a device
 * float[mxfa_probe_sink_len()] (written; the values are meaningless). */
int mxfa_probe_mfma(int dtype, int iters, float *sink, double *flops, void *stream);
/* The same with v_mfma_f32_32x32x16_bf16 (4 independent accumulators per
 * wave, iters x 4 MFMAs per wave), the other bf16 MFMA shape: its rate is the
 * 16x16x32 one's (the kernels use 16x16x32). */
int mxfa_probe_mfma32(int iters, float *sink, double *flops, void *stream);

/* Instruction-mix ceilings. Each wave runs `iters` rounds of 32
 * v_mfma_f32_16x16x32_bf16 (8 independent accumulators) with the mix's other
 * instructions spread evenly over them, none waiting on another: the rate at
 * which a SIMD issues that mix, with `waves_per_simd` waves per SIMD (1-8;
 * 256 x waves_per_simd work-groups of 4 waves). The mixes replay, per 32
 * MFMAs, the instruction counts rocprofv3 measures for the bf16 d = 64 causal
 * kernels (SQ_INSTS_VALU less SQ_INSTS_MFMA, SQ_INSTS_VALU_TRANS_F32,
 * SQ_INSTS_LDS, per SQ_INSTS_MFMA), as v_exp_f32 / v_mul_f32 /
 * v_cvt_pk_bf16_f32 / ds_read_b128 / ds_read_b64_tr_b16:
 *   MXFA_PROBE_MIX_MFMA      the MFMAs alone
 *   MXFA_PROBE_MIX_DKV       dK/dV pass: 16 exp, 48 mul, 16 cvt, 12 b128, 16 tr
 *   MXFA_PROBE_MIX_DKV_VALU  its VALU part alone
 *   MXFA_PROBE_MIX_DKV_LDS   its LDS part alone
 *   MXFA_PROBE_MIX_DQ        dQ pass: 21 exp, 60 mul, 11 cvt, 10 b128, 11 tr
 *   MXFA_PROBE_MIX_FWD       forward: 32 exp, 106 mul, 16 cvt, 8 b128, 16 tr
 *   MXFA_PROBE_MIX32_*       the MFMA-only, dK/dV, dQ and forward mixes with
 *                            the same work issued as 16 v_mfma_f32_32x32x16_bf16
 *                            per round (4 independent accumulators), the other
 *                            instructions unchanged
 * Writes the launch's MFMA flops to *flops. Not the reference's: its audit
 * (isa.cu:11-63) times one instruction kind at a time. */
enum {
    MXFA_PROBE_MIX_MFMA = 0,
    MXFA_PROBE_MIX_DKV = 1,
    MXFA_PROBE_MIX_DKV_VALU = 2,
    MXFA_PROBE_MIX_DKV_LDS = 3,
    MXFA_PROBE_MIX_DQ = 4,
    MXFA_PROBE_MIX_FWD = 5,
    MXFA_PROBE_MIX32_MFMA = 6,
    MXFA_PROBE_MIX32_DKV = 7,
    MXFA_PROBE_MIX32_DQ = 8,
    MXFA_PROBE_MIX32_FWD = 9
};
int mxfa_probe_mix(int mix, int waves_per_simd, int iters, float *sink, double *flops, void *stream);
/* Work-group timeline of the forward and the backward. With the timeline
 * build of the code object loaded (mxfa_gfx950_timeline.hsaco beside
 * libmxfa.so, selected with mxfa_set_code_object before the device loads it),
 * thread 0 of every forward, dQ and dK/dV work-group stamps the 100 MHz
 * real-time counter at its start, once its first stage is staged, at the end
 * of its loop and once its stores are acknowledged, and records its kind and
 * block ((kind << 32) | block; kind 0 = dQ, query block; 1 = dK/dV, key block;
 * 2 = forward, query block), its stages and where it ran ((XCC_ID << 32) |
 * HW_ID): eight uint64 per linear work-group index ((blockIdx.z * gridDim.y +
 * blockIdx.y) * gridDim.x + blockIdx.x; the last one zero), for the first 65536 work-groups of each
 * launch, each launch
 * overwriting the last one's. Copies up to `bytes` of them to host `dst` (a
 * synchronous device-to-host copy; dst may be NULL) and writes their size to
 * *avail. MXFA_ERR_UNSUPPORTED with the normal code object. */
int mxfa_probe_wg_times(void *dst, size_t bytes, size_t *avail);
/* Launches a grid-stride streaming read of `bytes` (a multiple of 16) at `x`,
 * the stream_f4 shape (isa.cu:55-63). */
int mxfa_probe_read(const void *x, size_t bytes, float *sink, void *stream);
/* Launches a grid-stride copy of `bytes` (a multiple of 16) from x to y. */
int mxfa_probe_copy(const void *x, void *y, size_t bytes, void *stream);
/* Replays the global writes a dQ pass fused into the dK/dV pass would make at a
 * causal shape with `bh` (batch, head) pairs, N = n (a multiple of 128) and
 * d = 64: the work-group of each 128-key block adds one 64 x 64 fp32 partial
 * tile per 64-query stage from its diagonal stage on. atomic = 1: fp32 atomic
 * adds of 1.0 (on a zeroed `acc`, element (h, row, x) ends at row / 128 + 1);
 * atomic = 0: plain stores of the same bytes. `acc` is a device
 * float[bh * n * 64]; the payload bytes are written to *bytes. No counterpart
 * in the reference: it measures the alternative that the reference's separate
 * dQ pass (attention_bwd.cu:96-158) avoids. */
int mxfa_probe_dq_atomic(float *acc, int bh, int n, int atomic, double *bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFA_PROBES_H */
