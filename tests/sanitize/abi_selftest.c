/*
 * Host-side checks of libmxfa's C ABI under AddressSanitizer and
 * UndefinedBehaviorSanitizer (tests/sanitize/Makefile builds the library's
 * host code with them). Only argument validation, size queries and settings
 * run: every run_* call here is rejected before any launch, so nothing
 * touches a device (this is safe with or without a GPU). Exit status 0 = all
 * checks passed.
 */
#include <float.h>
#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "../../include/mxfa.h"
#include "../../include/mxfa_probes.h"

static int g_fail = 0;
#define EXPECT(expr, want)                                                                  \
    do {                                                                                    \
        long long got_ = (long long)(expr);                                                 \
        if (got_ != (long long)(want)) {                                                    \
            fprintf(stderr, "FAIL %s:%d: %s = %lld, want %lld\n", __FILE__, __LINE__, #expr, \
                    got_, (long long)(want));                                               \
            ++g_fail;                                                                       \
        }                                                                                   \
    } while (0)

static mxfa_shape shape(int B, int Hq, int Hkv, int N, int d, int causal, int dtype, float scale) {
    mxfa_shape s = {B, Hq, Hkv, N, d, causal, dtype, scale};
    return s;
}

int main(void) {
    /* fake device addresses: aligned, misaligned; never dereferenced */
    void *p = (void *)(uintptr_t)4096, *mis = (void *)(uintptr_t)4100;
    float *fp = (float *)p;

    EXPECT(mxfa_version() > 0, 1);
    for (int st = -9; st <= 1; ++st) EXPECT(strlen(mxfa_strerror(st)) > 0, 1);

    /* shapes */
    mxfa_shape ok = shape(4, 12, 12, 4096, 64, 1, MXFA_BF16, 0.0f);
    EXPECT(mxfa_check_shape(&ok), MXFA_OK);
    EXPECT(mxfa_check_shape(NULL), MXFA_ERR_NULL);
    mxfa_shape s = ok;
    s.dtype = 7;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_DTYPE);
    s = ok; s.B = 0;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.N = -5;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.Hq = 3; s.Hkv = 2;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.causal = 2;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.scale = -1.0f;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.scale = INFINITY;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.scale = NAN;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = ok; s.d = 96;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_UNSUPPORTED);
    s = ok; s.d = 128; s.dtype = MXFA_F32;
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_UNSUPPORTED);
    /* products past every index type the kernels use */
    s = shape(INT_MAX, INT_MAX, 1, 1, 64, 0, MXFA_BF16, 0.0f);
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = shape(1, 1, 1, INT_MAX, 64, 0, MXFA_BF16, 0.0f);
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    s = shape(65535, 32768, 32768, 4194240, 128, 0, MXFA_BF16, 0.0f);
    EXPECT(mxfa_check_shape(&s), MXFA_ERR_SHAPE);
    EXPECT(mxfa_bwd_workspace_bytes(&s), 0);

    /* size queries */
    EXPECT(mxfa_bwd_workspace_bytes(NULL), 0);
    EXPECT(mxfa_bwd_workspace_bytes(&ok), 0);
    s = shape(2, 14, 2, 4096, 64, 1, MXFA_BF16, 0.0f);
    EXPECT(mxfa_bwd_workspace_bytes(&s), 2LL * 8 * 2 * 2 * 4096 * 64 * 4 + 8 * 908); /* cfg4: 8 planes, 908 shares */
    EXPECT(mxfa_naive_scratch_bytes(&ok), 4LL * 12 * 4096 * 4096 * 4);
    EXPECT(mxfa_naive_scratch_bytes(NULL), 0);
    EXPECT(mxfa_bwd_one_launch(&ok), 1);
    EXPECT(mxfa_bwd_one_launch(NULL), 0);

    /* settings */
    mxfa_bwd_options o, o0;
    EXPECT(mxfa_get_bwd_options(&o0), MXFA_OK);
    EXPECT(mxfa_get_bwd_options(NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_set_bwd_options(NULL), MXFA_ERR_NULL);
    o.one_launch = 0;
    o.delta_wait_us = INT_MAX;
    EXPECT(mxfa_set_bwd_options(&o), MXFA_OK);
    EXPECT(mxfa_bwd_one_launch(&ok), 0);
    o.one_launch = 5;
    EXPECT(mxfa_set_bwd_options(&o), MXFA_ERR_SHAPE);
    EXPECT(mxfa_set_bwd_options(&o0), MXFA_OK);
    EXPECT(mxfa_bwd_delta_fallbacks(NULL), MXFA_ERR_NULL);

    /* entry points reject bad arguments before launching */
    EXPECT(mxfa_run_flash(&ok, p, p, p, NULL, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_flash(&ok, p, mis, p, p, NULL), MXFA_ERR_ALIGN);
    EXPECT(mxfa_run_flash_lse(&ok, p, p, p, p, NULL, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_flash_lse(NULL, p, p, p, p, fp, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_preprocess(&ok, p, p, NULL, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_bwd_dq(&ok, p, p, p, p, fp, fp, mis, NULL), MXFA_ERR_ALIGN);
    EXPECT(mxfa_run_bwd_dkv(&ok, p, p, p, p, fp, NULL, p, p, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_bwd_flash(&ok, p, p, p, p, fp, fp, p, p, NULL, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_bwd_dq_delta(&ok, p, p, p, p, p, fp, fp, NULL, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_bwd(&ok, p, p, p, p, p, fp, fp, p, p, mis, NULL), MXFA_ERR_ALIGN);
    s = shape(2, 14, 2, 4096, 64, 1, MXFA_BF16, 0.0f);
    const size_t need = mxfa_bwd_workspace_bytes(&s);
    EXPECT(mxfa_run_bwd_ws(&s, p, p, p, p, p, fp, fp, p, p, p, p, need - 1, NULL), MXFA_ERR_WORKSPACE);
    EXPECT(mxfa_run_bwd_ws(&s, p, p, p, p, p, fp, fp, p, p, p, mis, need, NULL), MXFA_ERR_ALIGN);
    EXPECT(mxfa_run_bwd_dkv_ws(&s, p, p, p, p, fp, fp, p, p, p, 0, NULL), MXFA_ERR_WORKSPACE);
    EXPECT(mxfa_run_bwd_naive(&ok, p, p, p, p, fp, fp, p, p, p, NULL), MXFA_ERR_UNSUPPORTED);
    s = ok; s.dtype = MXFA_F32;
    EXPECT(mxfa_run_bwd_naive(&s, p, p, p, p, fp, fp, p, NULL, p, NULL), MXFA_ERR_NULL);
    EXPECT(mxfa_run_naive_fwd(&ok, p, p, p, fp, p, NULL), MXFA_ERR_UNSUPPORTED);
    EXPECT(mxfa_run_naive_fwd(&s, p, p, p, NULL, p, NULL), MXFA_ERR_NULL);

    /* the no-alloc backward: over its scratch, or missing pointers */
    EXPECT(mxfa_bwd_noalloc_scratch_bytes(), 65LL << 20);
    s = shape(1, 64, 4, 8192, 64, 1, MXFA_BF16, 0.0f);
    EXPECT(mxfa_run_bwd_noalloc(&s, p, p, p, p, p, fp, fp, p, p, p, NULL), MXFA_ERR_SCRATCH);
    EXPECT(mxfa_run_bwd_noalloc(&ok, p, p, p, p, p, fp, fp, p, NULL, p, NULL), MXFA_ERR_NULL);

    /* prefill */
    mxfa_prefill_shape pf = {16, 12, 4, 64, 100, 12 * 64 + 2 * 4 * 64, 4 * 64, 12 * 64, MXFA_BF16, 0.0f};
    EXPECT(mxfa_check_prefill(&pf), MXFA_OK);
    EXPECT(mxfa_check_prefill(NULL), MXFA_ERR_NULL);
    mxfa_prefill_shape pb = pf;
    pb.q_stride = 12 * 64 - 1;
    EXPECT(mxfa_check_prefill(&pb), MXFA_ERR_SHAPE);
    pb = pf; pb.kv_stride = 4 * 64 + 1;
    EXPECT(mxfa_check_prefill(&pb), MXFA_ERR_ALIGN);
    pb = pf; pb.pos0 = INT_MAX - 10;
    EXPECT(mxfa_check_prefill(&pb), MXFA_ERR_SHAPE);
    pb = pf; pb.n_head = 5;
    EXPECT(mxfa_check_prefill(&pb), MXFA_ERR_SHAPE);
    pb = pf; pb.head_dim = 128; pb.dtype = MXFA_F32;
    EXPECT(mxfa_check_prefill(&pb), MXFA_ERR_UNSUPPORTED);
    EXPECT(mxfa_run_prefill(&pf, p, p, NULL, p, NULL), MXFA_ERR_NULL);

    /* probes */
    double d = 0.0;
    EXPECT(mxfa_probe_mfma(7, 16, fp, &d, NULL), MXFA_ERR_DTYPE);
    EXPECT(mxfa_probe_mfma32(0, fp, &d, NULL), MXFA_ERR_SHAPE);
    EXPECT(mxfa_probe_mfma32(4, (float *)mis, &d, NULL), MXFA_ERR_ALIGN);
    EXPECT(mxfa_probe_read(p, 24, fp, NULL), MXFA_ERR_SHAPE);
    EXPECT(mxfa_probe_copy(p, mis, 32, NULL), MXFA_ERR_ALIGN);
    EXPECT(mxfa_probe_dq_atomic(fp, 1, 192, 1, &d, NULL), MXFA_ERR_SHAPE);

    /* code object checks (host only) */
    EXPECT(mxfa_check_code_object("/nonexistent/mxfa_gfx950.hsaco"), MXFA_ERR_CODE_OBJECT);
    EXPECT(mxfa_check_code_object("/proc/self/exe"), MXFA_ERR_CODE_OBJECT);
    EXPECT(mxfa_set_code_object("/nonexistent/mxfa_gfx950.hsaco"), MXFA_OK);
    EXPECT(mxfa_check_code_object(NULL), MXFA_ERR_CODE_OBJECT);
    EXPECT(mxfa_set_code_object(NULL), MXFA_OK);

    /* device selection: an index that no machine has */
    EXPECT(mxfa_init(-1), MXFA_ERR_DEVICE);
    EXPECT(mxfa_shutdown(), MXFA_OK);

    if (g_fail) {
        fprintf(stderr, "%d check(s) failed\n", g_fail);
        return 1;
    }
    printf("abi selftest: all checks passed\n");
    return 0;
}
