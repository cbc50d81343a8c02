/*
 * Self-test of the CPU oracle (oracle.c) for the host sanitizer builds
 * (`make -f oracle/Makefile sanitize` / `tsan`): runs every exported function
 * on small inputs, including the edge sizes (N = 1, ragged N, d = 128, GQA,
 * more threads than slices), so AddressSanitizer, UndefinedBehaviorSanitizer
 * and ThreadSanitizer see every code path, and checks what the mathematics
 * fixes, so a run that only avoids crashing does not pass:
 *   - pseudo_rand: deterministic, in [-1, 1) (common/src/lib.rs:104-113);
 *   - max_rel_err / allclose_err: the known answers of common/src/lib.rs:84-102;
 *   - forward: rows of O are convex combinations of V rows (each O element
 *     lies within the column's range over the visible V rows), causal row 0 is
 *     V row 0 and its LSE is scale q0.k0;
 *   - backward: sum_j dV_j = sum_i dO_i and sum_j dK_j = 0 (per head);
 *   - the reference's finite-difference gate fd_check < 5e-2 (main.rs:504-508);
 *   - the multi-head paths are independent of the thread count, bit for bit.
 * Test infrastructure, like oracle.c. Exit status 0 = all checks passed.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

void orc_pseudo_rand(float *out, size_t n, uint64_t seed);
void orc_normal(float *out, size_t n, uint64_t seed, float mult);
void orc_bf16_round(float *x, size_t n);
float orc_max_rel_err(const float *got, const float *want, size_t n);
float orc_allclose_err(const float *got, const float *want, size_t n, float rtol, float atol);
void orc_cpu_attention(const float *q, const float *k, const float *v, float *o, float *lse, int n, int d,
                       int causal, float scale);
void orc_cpu_attention_bwd(const float *q, const float *k, const float *v, const float *dout, float *dq,
                           float *dk, float *dv, int n, int d, int causal, float scale);
float orc_fd_check(int n, int d, int causal);
void orc_delta(const float *dout, const float *o, float *delta, size_t rows, int d);
int orc_mha_fwd(int B, int Hq, int Hkv, int N, int d, int causal, float scale, const float *q, const float *k,
                const float *v, float *o, float *lse, int nthreads);
int orc_mha_bwd(int B, int Hq, int Hkv, int N, int d, int causal, float scale, const float *q, const float *k,
                const float *v, const float *dout, float *dq, float *dk, float *dv, int nthreads);

static int g_fail = 0;
#define CHECK(cond, ...)                        \
    do {                                        \
        if (!(cond)) {                          \
            fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);       \
            fprintf(stderr, "\n");              \
            ++g_fail;                           \
        }                                       \
    } while (0)

static float *fbuf(size_t n) {
    /* exact sizes: an access one past the end is an ASan report */
    float *p = (float *)malloc((n ? n : 1) * sizeof(float));
    if (!p) abort();
    return p;
}

static void utilities(void) {
    float a[1000], b[1000];
    orc_pseudo_rand(a, 1000, 42);
    orc_pseudo_rand(b, 1000, 42);
    CHECK(memcmp(a, b, sizeof a) == 0, "pseudo_rand not deterministic");
    for (int i = 0; i < 1000; ++i) CHECK(a[i] >= -1.0f && a[i] < 1.0f, "pseudo_rand out of range at %d", i);
    orc_pseudo_rand(b, 1000, 43);
    CHECK(memcmp(a, b, sizeof a) != 0, "seeds 42 and 43 agree");

    const float w[3] = {1.0f, 2.0f, 3.0f}, g[3] = {1.0f, 2.2f, 3.0f};
    CHECK(orc_max_rel_err(w, w, 3) == 0.0f, "max_rel_err(a, a)");
    CHECK(fabsf(orc_max_rel_err(g, w, 3) - 0.1f) < 1e-6f, "max_rel_err known answer");
    const float want[2] = {0.0f, 100.0f}, ok[2] = {0.05f, 101.0f}, bad[2] = {0.10f, 102.0f};
    CHECK(orc_allclose_err(ok, want, 2, 1e-2f, 5e-2f) <= 1.0f + 1e-6f, "allclose_err within");
    CHECK(orc_allclose_err(bad, want, 2, 1e-2f, 5e-2f) > 1.0f, "allclose_err beyond");

    float z[7];
    orc_normal(z, 7, 9, 1.0f); /* odd length: the last Box-Muller pair is cut */
    for (int i = 0; i < 7; ++i) CHECK(isfinite(z[i]), "normal not finite");
    orc_bf16_round(z, 7);
    for (int i = 0; i < 7; ++i) {
        uint32_t u;
        memcpy(&u, &z[i], 4);
        CHECK((u & 0xffffu) == 0, "bf16_round left low bits");
    }
}

/* One head at (n, d, causal): forward invariants, backward closed forms, and
 * orc_delta against the sum of p dP it must equal. */
static void one_head(int n, int d, int causal) {
    const size_t nd = (size_t)n * d;
    const float scale = 1.0f / sqrtf((float)d);
    float *q = fbuf(nd), *k = fbuf(nd), *v = fbuf(nd), *dout = fbuf(nd), *o = fbuf(nd), *lse = fbuf(n);
    float *dq = fbuf(nd), *dk = fbuf(nd), *dv = fbuf(nd), *delta = fbuf(n);
    orc_normal(q, nd, 1, 1.0f);
    orc_normal(k, nd, 2, 1.0f);
    orc_normal(v, nd, 3, 1.0f);
    orc_normal(dout, nd, 4, 1.0f);
    orc_cpu_attention(q, k, v, o, lse, n, d, causal, scale);
    for (int i = 0; i < n; ++i) {
        const int cols = causal ? i + 1 : n;
        CHECK(isfinite(lse[i]), "lse not finite (n=%d row %d)", n, i);
        for (int x = 0; x < d; ++x) {
            float lo = INFINITY, hi = -INFINITY;
            for (int j = 0; j < cols; ++j) {
                lo = fminf(lo, v[(size_t)j * d + x]);
                hi = fmaxf(hi, v[(size_t)j * d + x]);
            }
            const float ox = o[(size_t)i * d + x];
            CHECK(ox >= lo - 1e-5f && ox <= hi + 1e-5f, "O outside the hull (n=%d row %d col %d)", n, i, x);
        }
    }
    if (causal) {
        float s0 = 0.0f;
        for (int x = 0; x < d; ++x) s0 += q[x] * k[x];
        CHECK(fabsf(lse[0] - s0 * scale) <= 1e-5f * (1.0f + fabsf(s0 * scale)), "causal LSE_0");
        for (int x = 0; x < d; ++x) CHECK(fabsf(o[x] - v[x]) <= 1e-6f, "causal O_0 != V_0");
    }
    orc_cpu_attention_bwd(q, k, v, dout, dq, dk, dv, n, d, causal, scale);
    orc_delta(dout, o, delta, (size_t)n, d);
    for (int x = 0; x < d; ++x) {
        double sdv = 0.0, sdo = 0.0, sdk = 0.0, adk = 0.0;
        for (int j = 0; j < n; ++j) {
            sdv += dv[(size_t)j * d + x];
            sdo += dout[(size_t)j * d + x];
            sdk += dk[(size_t)j * d + x];
            adk += fabs(dk[(size_t)j * d + x]);
        }
        CHECK(fabs(sdv - sdo) <= 1e-4 * (1.0 + fabs(sdo)), "sum dV != sum dO (n=%d col %d)", n, x);
        CHECK(fabs(sdk) <= 1e-4 * (1.0 + adk), "sum dK != 0 (n=%d col %d)", n, x);
    }
    for (int i = 0; i < n; ++i) CHECK(isfinite(delta[i]), "delta not finite");
    free(q); free(k); free(v); free(dout); free(o); free(lse);
    free(dq); free(dk); free(dv); free(delta);
}

/* GQA batch through the threaded paths: thread counts 1, 3 and more threads
 * than slices give the same bits. */
static void multi_head(int B, int Hq, int Hkv, int N, int d, int causal) {
    const size_t qn = (size_t)B * Hq * N * d, kn = (size_t)B * Hkv * N * d, ln = (size_t)B * Hq * N;
    float *q = fbuf(qn), *k = fbuf(kn), *v = fbuf(kn), *dout = fbuf(qn);
    float *o[3], *lse[3], *dq[3], *dk[3], *dv[3];
    orc_normal(q, qn, 11, 0.5f);
    orc_normal(k, kn, 12, 0.5f);
    orc_normal(v, kn, 13, 0.5f);
    orc_normal(dout, qn, 14, 1.0f);
    const int threads[3] = {1, 3, 2 * B * Hq + 1};
    for (int t = 0; t < 3; ++t) {
        o[t] = fbuf(qn); lse[t] = fbuf(ln); dq[t] = fbuf(qn); dk[t] = fbuf(kn); dv[t] = fbuf(kn);
        CHECK(orc_mha_fwd(B, Hq, Hkv, N, d, causal, 0.125f, q, k, v, o[t], lse[t], threads[t]) == 0, "mha_fwd");
        CHECK(orc_mha_bwd(B, Hq, Hkv, N, d, causal, 0.125f, q, k, v, dout, dq[t], dk[t], dv[t], threads[t]) == 0,
              "mha_bwd");
        if (t > 0) {
            CHECK(memcmp(o[t], o[0], qn * 4) == 0 && memcmp(lse[t], lse[0], ln * 4) == 0, "fwd depends on threads");
            CHECK(memcmp(dq[t], dq[0], qn * 4) == 0 && memcmp(dk[t], dk[0], kn * 4) == 0 &&
                      memcmp(dv[t], dv[0], kn * 4) == 0,
                  "bwd depends on threads");
        }
    }
    CHECK(orc_mha_fwd(B, 3, 2, N, d, causal, 0.125f, q, k, v, o[0], NULL, 1) == -1, "Hq %% Hkv accepted");
    for (int t = 0; t < 3; ++t) {
        free(o[t]); free(lse[t]); free(dq[t]); free(dk[t]); free(dv[t]);
    }
    free(q); free(k); free(v); free(dout);
}

int main(int argc, char **argv) {
    /* "threads": only the threaded paths (the ThreadSanitizer build) */
    const int threads_only = argc > 1 && strcmp(argv[1], "threads") == 0;
    if (!threads_only) {
        utilities();
        const int ns[5] = {1, 2, 33, 64, 97};
        for (int i = 0; i < 5; ++i) {
            one_head(ns[i], 64, 0);
            one_head(ns[i], 64, 1);
        }
        one_head(40, 128, 1);
        for (int causal = 0; causal < 2; ++causal) {
            const float e = orc_fd_check(32, 64, causal);
            CHECK(e < 5e-2f, "fd_check(32, causal=%d) = %g", causal, e);
        }
    }
    multi_head(2, 4, 2, 24, 64, 1);
    multi_head(1, 3, 1, 17, 64, 0);
    if (g_fail) {
        fprintf(stderr, "%d check(s) failed\n", g_fail);
        return 1;
    }
    printf("oracle selftest: all checks passed%s\n", threads_only ? " (threads)" : "");
    return 0;
}
