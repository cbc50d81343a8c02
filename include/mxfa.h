/*
 * mxfa.h - C ABI of the MI355X (gfx950) flash-attention training path.
 *
 * Drop-in for the host wrappers and kernels of the 02-flash-attention crate of
 * glaucomaa/mx230. Every entry point below names the reference interface it
 * replaces (paths relative to the reference repository).
 *
 * Conventions
 *   - Plain C types only: device pointers are `void*` / `float*` obtained from
 *     hipMalloc (or any allocator of device memory); `stream` is a
 *     hipStream_t passed as `void*` (NULL = the null stream).
 *   - Layouts (row-major, contiguous):
 *       Q, O, dO, dQ : [B][Hq][N][d]
 *       K, V, dK, dV : [B][Hkv][N][d]
 *       LSE, Delta   : [B][Hq][N]  (always fp32; LSE in natural-log units)
 *     With B = Hq = Hkv = 1 and d = 64 this is exactly the reference's
 *     [N][64] layout (attention_flash.cu:17-89).
 *     Query head h reads KV head h / (Hq / Hkv) (grouped-query attention,
 *     03-llm-engine/src/cpu.rs:194,224); dK / dV of a KV head are the sum
 *     over the query heads that share it.
 *   - dtype MXFA_F32: every tensor above is fp32. dtype MXFA_BF16: Q, K, V,
 *     O, dO, dQ, dK, dV are bf16 (raw uint16 storage), LSE and Delta fp32,
 *     and all accumulation is fp32.
 *   - All launches are asynchronous on `stream`. The run_* entry points never
 *     synchronise and never allocate device memory. The library's own state
 *     is the one-launch backward's: a static 4 MB array of Delta flags per
 *     device, a launch counter (epoch), the counter of mxfa_bwd_delta_fallbacks
 *     and the settings of mxfa_set_bwd_options. Launches in flight together
 *     on one device are safe (see mxfa_bwd_one_launch); ordering is the
 *     caller's stream order.
 *   - The roofline and measurement probes are declared in mxfa_probes.h.
 *   - Errors are returned as negative codes (see mxfa_status); nothing aborts
 *     and no C++ exception crosses this boundary. The reference panics on a
 *     launch failure (02-flash-attention/src/main.rs:87,122,142,172,204,209).
 *   - Device pointers must be 16-byte aligned.
 */
#ifndef MXFA_H
#define MXFA_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MXFA_OK = 0,
    MXFA_ERR_NULL = -1,        /* a required pointer is NULL */
    MXFA_ERR_SHAPE = -2,       /* B, Hq, Hkv, N, d or Hq % Hkv invalid */
    MXFA_ERR_DTYPE = -3,       /* unknown dtype */
    MXFA_ERR_UNSUPPORTED = -4, /* valid shape, but no kernel (e.g. d not in {64, 128}) */
    MXFA_ERR_ALIGN = -5,       /* a device pointer is not 16-byte aligned */
    MXFA_ERR_LAUNCH = -6,      /* the HIP runtime rejected a launch */
    MXFA_ERR_DEVICE = -7,      /* no usable gfx950 device */
    MXFA_ERR_WORKSPACE = -8,   /* a workspace smaller than mxfa_{bwd,prefill}_workspace_bytes(shape) */
    MXFA_ERR_CODE_OBJECT = -9, /* the gfx950 code object is missing, malformed, for another
                                  processor, or lacks a kernel */
    MXFA_ERR_SCRATCH = -10     /* mxfa_run_bwd_noalloc: the shape needs more than
                                  mxfa_bwd_noalloc_scratch_bytes() */
} mxfa_status;

typedef enum { MXFA_F32 = 0, MXFA_BF16 = 1 } mxfa_dtype;

typedef struct {
    int B;        /* batch */
    int Hq;       /* query heads */
    int Hkv;      /* key/value heads; Hq % Hkv == 0 */
    int N;        /* sequence length (queries = keys) */
    int d;        /* head dim: 64 or 128 */
    int causal;   /* 0 or 1: key j visible to query i iff j <= i (main.rs:218) */
    int dtype;    /* mxfa_dtype */
    float scale;  /* softmax scale; 0 selects 1/sqrt(d) (main.rs:214) */
} mxfa_shape;

/* Library version as MAJOR*10000 + MINOR*100 + PATCH. */
int mxfa_version(void);

/* Human-readable text of a status code (static storage). */
const char *mxfa_strerror(int status);

/* The kernels are not part of libmxfa.so: they are one gfx950 code object,
 * mxfa_gfx950.hsaco (built by hipcc beside the library), loaded per device with
 * hipModuleLoadData and launched by name. */

/* Checks that `device` exists and is a gfx950 (MI355X), makes it current and
 * loads the code object on it (MXFA_ERR_CODE_OBJECT if that fails).
 * Optional: the run_* entry points load it on the current device at their
 * first launch there, and return MXFA_ERR_CODE_OBJECT if they cannot.
 * Replaces CudaContext::new(0) + load_kernels / load_bwd, which load the PTX
 * modules and look the kernels up by name
 * (02-flash-attention/src/main.rs:392-415, 514). */
int mxfa_init(int device);

/* Unloads the code object from every device it was loaded on (each device's
 * work must have completed); a later launch loads it again. */
int mxfa_shutdown(void);

/* Sets the code object file later loads read (NULL: mxfa_gfx950.hsaco in the
 * directory of libmxfa.so). Devices that already loaded one keep it until
 * mxfa_shutdown. Returns MXFA_OK; the file is checked when loaded.
 * Replaces the PTX paths the reference's build.rs exports to the crate
 * (kernel-build/src/lib.rs:37-55, :89-115). */
int mxfa_set_code_object(const char *path);

/* Checks a code object file on the host, with no device access (NULL: the
 * file later loads read): present and readable, a 64-bit little-endian ELF for
 * EM_AMDGPU with the AMDGPU HSA OS/ABI, built for gfx950. MXFA_OK or
 * MXFA_ERR_CODE_OBJECT. The counterpart of load_ptx's guard against an empty
 * stub module (common/src/lib.rs:11-18). */
int mxfa_check_code_object(const char *path);

/* Validates a shape exactly as every run_* entry point does; no GPU access. */
int mxfa_check_shape(const mxfa_shape *shape);

/* Forward, O only.
 * Replaces run_flash (02-flash-attention/src/main.rs:68-88) and kernel
 * attn_flash (02-flash-attention/kernels/attention_flash.cu:91-94). */
int mxfa_run_flash(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                   void *o, void *stream);

/* Forward, O and the per-row log-sum-exp L_i = m_i + ln(l_i).
 * Replaces run_flash_lse (main.rs:102-123) and attn_flash_lse
 * (attention_flash.cu:97-100, LSE at :85-87). */
int mxfa_run_flash_lse(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       void *o, float *lse, void *stream);

/* Delta_i = sum_x dO[i][x] * O[i][x] (fp32 accumulation).
 * Replaces run_preprocess (main.rs:126-143) and attn_bwd_preprocess
 * (attention_bwd.cu:32-44). */
int mxfa_run_preprocess(const mxfa_shape *shape, const void *dout, const void *o, float *delta,
                        void *stream);

/* dQ pass only (overwrites dQ; atomic-free).
 * Replaces the attn_bwd_dq launch of run_bwd_flash (main.rs:202-204,
 * attention_bwd.cu:96-158). */
int mxfa_run_bwd_dq(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                    const void *dout, const float *lse, const float *delta, void *dq,
                    void *stream);

/* dK/dV pass only (overwrites dK, dV; atomic-free; with Hq > Hkv the sum over
 * the query heads of a group is done inside the kernel).
 * Replaces the attn_bwd_dkv launch of run_bwd_flash (main.rs:206-209,
 * attention_bwd.cu:165-243). */
int mxfa_run_bwd_dkv(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                     const void *dout, const float *lse, const float *delta, void *dk,
                     void *dv, void *stream);

/* The tiled backward: dK/dV pass then dQ pass, same stream, outputs
 * overwritten (no zeroing needed).
 * Replaces run_bwd_flash (02-flash-attention/src/main.rs:179-210). */
int mxfa_run_bwd_flash(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       const void *dout, const float *lse, const float *delta, void *dq,
                       void *dk, void *dv, void *stream);

/* dQ pass that also computes Delta = rowsum(dO * O) for its query rows and
 * writes it to `delta` (the preprocess launch, attention_bwd.cu:32-44,
 * folded into the attn_bwd_dq launch, :96-158). */
int mxfa_run_bwd_dq_delta(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                          const void *dout, const float *lse, float *delta, void *dq, void *stream);

/* The whole backward from O in two launches: the dQ pass computes
 * Delta = rowsum(dO * O) itself (writing it to `delta`, B*Hq*N fp32, which the
 * caller owns as for mxfa_run_preprocess) and the dK/dV pass reads it.
 * Replaces the sequence run_preprocess + run_bwd_flash (main.rs:126-143,
 * :179-210; attention_bwd.cu:32-44, :96-243) with the preprocess launch folded
 * into the dQ pass; results equal that sequence's up to the summation order of
 * Delta. */
int mxfa_run_bwd(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                 const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv,
                 void *stream);

/* 1 if mxfa_run_bwd and mxfa_run_bwd_ws run the dQ and dK/dV work of this
 * shape in one launch (for a GQA split through a workspace, the adding of the
 * split's partial sums included), else 0 (a dQ launch and a dK/dV launch, or
 * an invalid shape).
 * The one-launch form (bf16, d = 64 or 128) runs the dQ work-groups first;
 * they publish Delta per 128-row query block, and the dK/dV work-groups of the
 * same launch wait for the blocks they need. Each wait is bounded in time
 * (mxfa_bwd_options.delta_wait_us): after it the work-group computes those
 * Delta rows from O and dO itself, with the same arithmetic as the dQ
 * work-groups, so the results equal the two-launch form's bitwise either way.
 * mxfa_bwd_options.one_launch = 0 selects two launches, and so does a stream
 * under graph capture (a replayed launch would reuse the capture's flag
 * epoch); this query answers for an ordinary stream.
 * No counterpart in the reference: it tells callers (and benchmarks) which
 * kernels the backward from O (main.rs:126-143, :179-210) becomes. */
int mxfa_bwd_one_launch(const mxfa_shape *shape);

/* Process-wide settings of the one-launch backward, read at every launch
 * (default {1, 200, 2000000}). Meant for tests and measurement; settings changed while
 * other threads launch take effect at their next launch.
 * No counterpart in the reference (its backward is always two launches,
 * main.rs:179-210). */
typedef struct {
    int one_launch;    /* 1: one launch where available (bf16); 0: always two */
    int delta_wait_us; /* bound of each Delta wait in microseconds; < 0: never
                          wait, always compute Delta in the dK/dV work-group */
    int reduce_wait_us; /* bound of each wait of a GQA split's reduce work-
                           group for its shares, microseconds, >= 0 (see
                           mxfa_bwd_reduce_timeouts) */
} mxfa_bwd_options;
int mxfa_set_bwd_options(const mxfa_bwd_options *options);
int mxfa_get_bwd_options(mxfa_bwd_options *options);

/* Delta blocks (64 query rows of one head) that the one-launch backward's
 * dK/dV work-groups computed themselves on the current device, because their
 * wait ran out, since the library was loaded. A synchronous device-to-host
 * copy: call it after the launches of interest have completed. 0 in normal
 * operation; a count does not change results (see mxfa_bwd_one_launch). */
int mxfa_bwd_delta_fallbacks(unsigned long long *count);

/* Work-groups of the one-launch backward that add a GQA split's partial sums
 * and whose wait for them ran out, on the current device since the library
 * was loaded (a synchronous device-to-host copy, as above). Those work-groups
 * run after all of the split's work-groups have been dispatched, so the wait
 * ends in normal operation and the count stays 0; a count means the dK and dV
 * rows of those work-groups were written as NaN. The wait is bounded
 * (mxfa_bwd_options.reduce_wait_us, default 2 s) so that a launch always
 * ends.
 * No counterpart in the reference (no GQA, and its backward is two launches,
 * main.rs:179-210). */
int mxfa_bwd_reduce_timeouts(unsigned long long *count);

/* Bytes of device workspace the _ws entry points below can use (0 for an
 * invalid shape). dQ is a separate atomic-free pass and needs none. With GQA
 * (Hq > Hkv), when the key blocks alone would leave the GPU underfilled, the
 * dK/dV pass splits the work of each key block (its group's query heads, each
 * from the diagonal) over several work-groups, a causal block with more
 * queries over more of them: each writes fp32 partial dK/dV sums to the
 * workspace, and they are added in a fixed order (deterministic, atomic-free)
 * by the last work-groups of the one-launch backward, else by a second
 * launch. The size is 2 * planes * B * Hkv * N * d * 4 bytes, planes being
 * the most work-groups any key block takes, then 8 bytes per work-group of
 * the split (the flags by which the one-launch backward's adding work-groups
 * learn that a share's sums are written: each launch writes its own value,
 * so the workspace needs no clearing); 0 when no split helps (always without
 * GQA). A call uses its workspace until it completes: calls in flight at the
 * same time need their own.
 * The reference has no GQA (d = 64, one head, attention_bwd.cu:165-243); this
 * sizes the scratch of its dK/dV pass generalised to GQA groups. */
size_t mxfa_bwd_workspace_bytes(const mxfa_shape *shape);

/* mxfa_run_bwd_dkv with a caller-owned workspace (16-byte aligned, at least
 * mxfa_bwd_workspace_bytes(shape) bytes, else MXFA_ERR_ALIGN or
 * MXFA_ERR_WORKSPACE). workspace == NULL is allowed and runs the unsplit pass
 * (= mxfa_run_bwd_dkv). Results equal the unsplit pass's up to the summation
 * order over the query heads of a group; the workspace holds nothing the
 * caller needs afterwards.
 * Replaces the attn_bwd_dkv launch (attention_bwd.cu:165-243, main.rs:206-209)
 * for GQA shapes. */
int mxfa_run_bwd_dkv_ws(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                        const void *dout, const float *lse, const float *delta, void *dk,
                        void *dv, void *workspace, size_t workspace_bytes, void *stream);

/* mxfa_run_bwd with a caller-owned workspace for its dK/dV pass (as
 * mxfa_run_bwd_dkv_ws; NULL = mxfa_run_bwd).
 * Replaces run_preprocess + run_bwd_flash (main.rs:126-143, :179-210) as
 * mxfa_run_bwd does. */
int mxfa_run_bwd_ws(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                    const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv,
                    void *workspace, size_t workspace_bytes, void *stream);

/* mxfa_run_bwd_ws without a workspace argument and without allocating: the
 * split dK/dV pass keeps its fp32 partial sums and share flags in a static
 * device array of the library, mxfa_bwd_noalloc_scratch_bytes() (65 MiB) per
 * device, held from the
 * library's set-up on the device (mxfa_init, else this entry point's first
 * call there) until the process ends. Shapes whose mxfa_bwd_workspace_bytes
 * exceed it return MXFA_ERR_SCRATCH before any device work. No hipMalloc,
 * hipFree or other allocating call; the array needs no clearing (every call
 * overwrites what it reads). All calls on one device share the array and
 * keep the last call's contents, so calls that overlap on one device race
 * (serialise them, e.g. on one stream); results equal mxfa_run_bwd_ws's.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation). */
int mxfa_run_bwd_noalloc(const mxfa_shape *shape, const void *q, const void *k, const void *v, const void *o,
                         const void *dout, const float *lse, float *delta, void *dq, void *dk, void *dv,
                         void *stream);
size_t mxfa_bwd_noalloc_scratch_bytes(void);

/* Naive backward baseline: one thread per query row, dK/dV scattered with
 * atomic adds. fp32 only. dQ, dK, dV MUST be zeroed by the caller.
 * Replaces run_bwd_naive (main.rs:147-173) and attn_bwd_naive
 * (attention_bwd.cu:48-90). */
int mxfa_run_bwd_naive(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       const void *dout, const float *lse, const float *delta, void *dq,
                       void *dk, void *dv, void *stream);

/* Bytes of the N x N fp32 score scratch mxfa_run_naive_fwd needs
 * (B * Hq * N * N * 4). */
size_t mxfa_naive_scratch_bytes(const mxfa_shape *shape);

/* Naive forward baseline that materialises the scores: S = QK^T * scale
 * (masked to -inf above the diagonal when causal), row softmax in place,
 * O = S V. fp32 only; `s` holds mxfa_naive_scratch_bytes bytes.
 * Replaces Naive::run (main.rs:32-66) and attn_scores / attn_softmax /
 * attn_av (attention_naive.cu:8-70). */
int mxfa_run_naive_fwd(const mxfa_shape *shape, const void *q, const void *k, const void *v,
                       float *s, void *o, void *stream);

/* ---- Inference-side forward (prefill): token-major rows over a KV cache.
 * Replaces `attn_prefill` (03-llm-engine/kernels/llm.cu:3806-3815, body
 * :3674-3804; launched by gpu.rs:3235-3289): query row i of this chunk sits at
 * absolute position pos0 + i and attends to cache rows 0 .. pos0 + i (causal
 * with a diagonal offset). Q row i holds head h at elements
 * [h * head_dim, (h + 1) * head_dim) of a row q_stride elements long (the
 * fused QKV row in the reference); the K and V caches hold position j in rows
 * kv_stride elements long, KV head h / (n_head / n_kv_head) at
 * [kvh * head_dim, ...); the output row i likewise with out_stride. Rows
 * 0 .. pos0 + n_tok - 1 of both caches must be filled (the reference copies
 * the chunk's own K/V in first, copy_kv_batch at llm.cu:3635). Generalisations: bf16 as well
 * as fp32, head_dim 128 (bf16), any scale; the reference is fp32, head_dim 64,
 * scale 1/8. No LSE is written. */
typedef struct {
    int n_tok;      /* query rows of this chunk */
    int n_head;     /* query heads */
    int n_kv_head;  /* KV heads; n_head % n_kv_head == 0 */
    int head_dim;   /* 64 (fp32, bf16) or 128 (bf16) */
    int pos0;       /* absolute position of query row 0 */
    int q_stride;   /* elements between query rows (>= n_head * head_dim) */
    int kv_stride;  /* elements between cache rows (>= n_kv_head * head_dim) */
    int out_stride; /* elements between output rows (>= n_head * head_dim) */
    int dtype;      /* mxfa_dtype */
    float scale;    /* 0 -> 1/sqrt(head_dim) */
} mxfa_prefill_shape;

/* MXFA_OK if the prefill shape is supported; strides whose rows would not start
 * on 16-byte boundaries give MXFA_ERR_ALIGN, and pos0 + max(n_tok, n_head)
 * above 2^31 - 129 gives MXFA_ERR_SHAPE (a single row runs its GQA group's
 * heads as rows at positions pos0, pos0 + 1, ...). */
int mxfa_check_prefill(const mxfa_prefill_shape *shape);
int mxfa_run_prefill(const mxfa_prefill_shape *shape, const void *q, const void *kcache, const void *vcache,
                     void *out, void *stream);

/* The prefill over a paged KV cache. Replaces `attn_prefill_paged`
 * (03-llm-engine/kernels/llm.cu:3827-3836, body :3674-3804 with
 * PAGED = true; launched by gpu.rs:3270-3289): the same as mxfa_run_prefill,
 * except that logical cache position t sits in cache row
 * block_table[t / block_size] * block_size + t % block_size (kv_row<true>,
 * llm.cu:959-963), rows kv_stride elements apart from kcache / vcache.
 * block_table: int32 on the device, entries for positions 0 .. pos0 + n_tok - 1,
 * each a physical block inside the caches (not checked: a bad entry reads
 * outside them, as in the reference). block_size: a power of two (the
 * reference engine's KV_BLOCK is 16, gpu.rs:209); others give
 * MXFA_ERR_UNSUPPORTED. Outputs are bitwise those of mxfa_run_prefill over the
 * gathered, contiguous cache. */
int mxfa_run_prefill_paged(const mxfa_prefill_shape *shape, const void *q, const void *kcache, const void *vcache,
                           void *out, const int *block_table, int block_size, void *stream);

/* The prefill with its keys split over work-groups, for chunks whose query
 * blocks alone would leave most of the GPU idle (a few hundred tokens after a
 * long history, or a single decode-like row). Replaces the same
 * `attn_prefill` launch as mxfa_run_prefill (llm.cu:3806-3815, gpu.rs:3235-3289),
 * which has no counterpart of the split: each work-group takes a range of the
 * cache's 64-key stages of one 64-query block and writes its unnormalised
 * output and its rows' running max and sum to `workspace` (fp32); a second
 * launch adds the ranges (out = sum_s w_s O_s / sum_s w_s l_s with
 * w_s = 2^(m_s - max m)). Same arguments as mxfa_run_prefill, plus the
 * workspace: mxfa_prefill_workspace_bytes(shape) bytes, 16-byte aligned,
 * device memory (no contents needed; calls that share one race). When that
 * size is 0 the shape needs no split and this is mxfa_run_prefill (workspace
 * may be NULL). A smaller workspace gives MXFA_ERR_WORKSPACE. Results equal
 * mxfa_run_prefill's to fp32 rounding of the merge, not bitwise. */
size_t mxfa_prefill_workspace_bytes(const mxfa_prefill_shape *shape);
int mxfa_run_prefill_ws(const mxfa_prefill_shape *shape, const void *q, const void *kcache, const void *vcache,
                        void *out, void *workspace, size_t workspace_bytes, void *stream);
/* mxfa_run_prefill_paged with the same key split (replaces the
 * `attn_prefill_paged` launch, llm.cu:3827-3836, gpu.rs:3270-3289): the
 * paged cache arguments of mxfa_run_prefill_paged and the workspace of
 * mxfa_run_prefill_ws, sized by mxfa_prefill_workspace_bytes(shape) (the
 * same for both caches). Outputs are bitwise those of mxfa_run_prefill_ws over
 * the gathered, contiguous cache. */
int mxfa_run_prefill_paged_ws(const mxfa_prefill_shape *shape, const void *q, const void *kcache,
                              const void *vcache, void *out, const int *block_table, int block_size,
                              void *workspace, size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFA_H */
