/*
 * CPU restatement of the reference's flash-attention CPU path (glaucomaa/mx230,
 * crate 02-flash-attention, plus the utilities of crate `common`).
 *
 * THIS FILE IS TEST INFRASTRUCTURE. It is the checker: only tests/, the
 * smoke() entry point and bench.py's cpu_baseline leg may load it. The product
 * library (libmxfa.so) neither links nor calls anything here.
 *
 * The reference oracle is Rust (02-flash-attention/src/main.rs:213-390,
 * common/src/lib.rs:46-78). Rust is not available in this image, so the
 * functions below restate it loop for loop, in the same accumulation order, in
 * fp32 with no contraction (build with -ffp-contract=off, no fast-math): Rust
 * neither fuses a*b+c nor reorders sums, and its f32::exp / f32::ln call libm
 * expf / logf, which is what this file calls.
 *
 * Extensions required by the measured configurations (not in the reference,
 * which is single-head, d = 64, fp32):
 *   - a [B][H][N][d] batch/head loop with grouped-query attention, using the
 *     reference engine's head mapping kvh = h / (Hq / Hkv)
 *     (03-llm-engine/src/cpu.rs:194,224);
 *   - head dim d as a parameter (64 or 128);
 *   - the log-sum-exp L = m + ln(l) (the value attention_flash.cu:85-87 emits);
 *   - a seeded N(0,1) generator (Box-Muller over the reference's xorshift64*);
 *   - bf16 round-to-nearest-even, so the bf16 configurations can be checked on
 *     the bf16-rounded inputs.
 *
 * Mutation hooks: building with -DORC_MUTANT=<k> plants one deliberate
 * mistake (see ORC_MUTANT below). The oracle's own tests build those variants
 * to prove each pin catches a plausible error. Normal builds define none.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifndef ORC_MUTANT
#define ORC_MUTANT 0
#endif

/* ---------------------------------------------------------------- PRNG -- */

/* common/src/lib.rs:67-78 `pseudo_rand`: xorshift64* mapped to [-1, 1).
 * (r >> 40) < 2^24 is exact in f32, so the result is bit-identical. */
void orc_pseudo_rand(float *out, size_t n, uint64_t seed) {
    for (size_t i = 0; i < n; ++i) {
        seed ^= seed >> 12;
        seed ^= seed << 25;
        seed ^= seed >> 27;
        uint64_t r = seed * 0x2545F4914F6CDD1DULL;
        out[i] = (float)(r >> 40) / (float)(1ULL << 23) - 1.0f;
    }
}

/* Seeded N(0,1) samples, multiplied by `mult`: the same xorshift64* stream,
 * 53-bit uniforms in (0,1), Box-Muller in double, rounded once to f32.
 * Extension (the reference only has uniform inputs). */
void orc_normal(float *out, size_t n, uint64_t seed, float mult) {
    uint64_t s = seed ? seed : 0x9E3779B97F4A7C15ULL;
    const double two_pi = 6.283185307179586476925286766559;
    size_t i = 0;
    while (i < n) {
        double u[2];
        for (int t = 0; t < 2; ++t) {
            s ^= s >> 12;
            s ^= s << 25;
            s ^= s >> 27;
            uint64_t r = s * 0x2545F4914F6CDD1DULL;
            u[t] = ((double)(r >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        }
        double rad = sqrt(-2.0 * log(u[0]));
        double z0 = rad * cos(two_pi * u[1]);
        double z1 = rad * sin(two_pi * u[1]);
        out[i++] = (float)(z0 * (double)mult);
        if (i < n) out[i++] = (float)(z1 * (double)mult);
    }
}

/* fp32 -> bf16 (round to nearest, ties to even) -> fp32, in place. */
static inline float bf16_round1(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7f800000u) == 0x7f800000u) {
        if (u & 0x007fffffu) u |= 0x00400000u; /* keep NaN quiet */
        u &= 0xffff0000u;
    } else {
        u += 0x7fffu + ((u >> 16) & 1u);
        u &= 0xffff0000u;
    }
    memcpy(&x, &u, 4);
    return x;
}

void orc_bf16_round(float *x, size_t n) {
    for (size_t i = 0; i < n; ++i) x[i] = bf16_round1(x[i]);
}

/* ------------------------------------------------------------- metrics -- */

/* common/src/lib.rs:46-52 `max_rel_err`. */
float orc_max_rel_err(const float *got, const float *want, size_t n) {
    float worst = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float w = fabsf(want[i]);
        float e = fabsf(got[i] - want[i]) / (w > 1e-6f ? w : 1e-6f);
        worst = fmaxf(worst, e);
    }
    return worst;
}

/* common/src/lib.rs:58-64 `allclose_err`: max |g-w| / (atol + rtol |w|). */
float orc_allclose_err(const float *got, const float *want, size_t n, float rtol, float atol) {
    float worst = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        float e = fabsf(got[i] - want[i]) / (atol + rtol * fabsf(want[i]));
        worst = fmaxf(worst, e);
    }
    return worst;
}

/* ------------------------------------------------------ single head -- */

/* 02-flash-attention/src/main.rs:213-241 `cpu_attention`, with the head dim
 * as a parameter and the per-row log-sum-exp L_i = m_i + ln(l_i) added
 * (the quantity attention_flash.cu:85-87 writes). `lse` may be NULL. */
void orc_cpu_attention(const float *q, const float *k, const float *v, float *o, float *lse,
                       int n, int d, int causal, float scale) {
    float *s = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    memset(o, 0, (size_t)n * d * sizeof(float));
    for (int i = 0; i < n; ++i) {
        int cols = causal ? i + 1 : n;
        float m = -INFINITY;
        for (int j = 0; j < cols; ++j) {
            float dot = 0.0f;
            for (int x = 0; x < d; ++x) dot += q[(size_t)i * d + x] * k[(size_t)j * d + x];
            s[j] = dot * scale;
            m = fmaxf(m, s[j]);
        }
        float l = 0.0f;
        for (int j = 0; j < cols; ++j) {
            s[j] = expf(s[j] - m);
            l += s[j];
        }
        for (int j = 0; j < cols; ++j) {
            float p = s[j] / l;
            for (int x = 0; x < d; ++x) o[(size_t)i * d + x] += p * v[(size_t)j * d + x];
        }
        if (lse) {
#if ORC_MUTANT == 1 /* planted: drop the running max from the log-sum-exp */
            lse[i] = logf(l);
#else
            lse[i] = m + logf(l);
#endif
        }
    }
    free(s);
}

/* 02-flash-attention/src/main.rs:246-300 `cpu_attention_bwd`: gradients of
 * the scalar loss <O, dO> w.r.t. Q, K, V (outputs are zeroed first, as the
 * reference allocates them with vec![0.0; ..]). */
void orc_cpu_attention_bwd(const float *q, const float *k, const float *v, const float *dout,
                           float *dq, float *dk, float *dv, int n, int d, int causal,
                           float scale) {
    size_t nd = (size_t)n * d;
    memset(dq, 0, nd * sizeof(float));
    memset(dk, 0, nd * sizeof(float));
    memset(dv, 0, nd * sizeof(float));
    float *p = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    float *dp = (float *)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    for (int i = 0; i < n; ++i) {
        int cols = causal ? i + 1 : n;
        float m = -INFINITY;
        for (int j = 0; j < cols; ++j) {
            float dot = 0.0f;
            for (int x = 0; x < d; ++x) dot += q[(size_t)i * d + x] * k[(size_t)j * d + x];
            p[j] = dot * scale;
            m = fmaxf(m, p[j]);
        }
        float l = 0.0f;
        for (int j = 0; j < cols; ++j) {
            p[j] = expf(p[j] - m);
            l += p[j];
        }
        for (int j = 0; j < cols; ++j) p[j] /= l;
        /* dP_ij = dO_i . v_j ; Delta_i = sum_j p_ij dP_ij  (main.rs:280-289) */
        float delta = 0.0f;
        for (int j = 0; j < cols; ++j) {
            float acc = 0.0f;
            for (int x = 0; x < d; ++x) acc += dout[(size_t)i * d + x] * v[(size_t)j * d + x];
            dp[j] = acc;
            delta += p[j] * acc;
        }
        for (int j = 0; j < cols; ++j) {
#if ORC_MUTANT == 2 /* planted: drop the Delta term of the softmax VJP */
            float ds = p[j] * dp[j] * scale;
#elif ORC_MUTANT == 3 /* planted: wrong sign of the Delta term */
            float ds = p[j] * (dp[j] + delta) * scale;
#else
            float ds = p[j] * (dp[j] - delta) * scale;
#endif
            for (int x = 0; x < d; ++x) {
#if ORC_MUTANT == 4 /* planted: dV uses dO of the key row (transposed index) */
                dv[(size_t)j * d + x] += p[j] * dout[(size_t)j * d + x];
#else
                dv[(size_t)j * d + x] += p[j] * dout[(size_t)i * d + x];
#endif
#if ORC_MUTANT == 5 /* planted: dK accumulates k instead of q (swapped operand) */
                dk[(size_t)j * d + x] += ds * k[(size_t)j * d + x];
#else
                dk[(size_t)j * d + x] += ds * q[(size_t)i * d + x];
#endif
#if ORC_MUTANT == 6 /* planted: dQ missing the softmax scale */
                dq[(size_t)i * d + x] += (ds / scale) * k[(size_t)j * d + x];
#else
                dq[(size_t)i * d + x] += ds * k[(size_t)j * d + x];
#endif
            }
        }
    }
    free(p);
    free(dp);
}

/* 02-flash-attention/src/main.rs:304-333 `attn_loss`: <O, dO> with the
 * forward in f64. */
double orc_attn_loss(const float *q, const float *k, const float *v, const float *dout, int n,
                     int d, int causal) {
    double scale = 1.0 / sqrt((double)d);
    double loss = 0.0;
    double *s = (double *)malloc((size_t)(n > 0 ? n : 1) * sizeof(double));
    for (int i = 0; i < n; ++i) {
        int cols = causal ? i + 1 : n;
        double m = -INFINITY;
        for (int j = 0; j < cols; ++j) {
            double dot = 0.0;
            for (int x = 0; x < d; ++x)
                dot += (double)q[(size_t)i * d + x] * (double)k[(size_t)j * d + x];
            s[j] = dot * scale;
            m = fmax(m, s[j]);
        }
        double l = 0.0;
        for (int j = 0; j < cols; ++j) {
            s[j] = exp(s[j] - m);
            l += s[j];
        }
        for (int x = 0; x < d; ++x) {
            double o = 0.0;
            for (int j = 0; j < cols; ++j) o += s[j] / l * (double)v[(size_t)j * d + x];
            loss += o * (double)dout[(size_t)i * d + x];
        }
    }
    free(s);
    return loss;
}

/* 02-flash-attention/src/main.rs:339-390 `fd_check`: central differences of
 * attn_loss at six spread indices of each of Q, K, V against the analytic
 * gradient; returns the worst |fd - g| / (1e-3 + |g|). Inputs are
 * pseudo_rand seeds 21..24 (main.rs:340-343). Requires n >= 4. */
float orc_fd_check(int n, int d, int causal) {
    size_t nd = (size_t)n * d;
    float *q = malloc(nd * 4), *k = malloc(nd * 4), *v = malloc(nd * 4), *g = malloc(nd * 4);
    float *dq = malloc(nd * 4), *dk = malloc(nd * 4), *dv = malloc(nd * 4);
    orc_pseudo_rand(q, nd, 21);
    orc_pseudo_rand(k, nd, 22);
    orc_pseudo_rand(v, nd, 23);
    orc_pseudo_rand(g, nd, 24);
    float scale = 1.0f / sqrtf((float)d);
    orc_cpu_attention_bwd(q, k, v, g, dq, dk, dv, n, d, causal, scale);

    const float eps = 1e-3f;
    /* main.rs:348 with D -> d (needs d >= 64 and n >= 4) */
    size_t idxs[6] = {0, 1, (size_t)d + 7, 3 * (size_t)d + 31, (size_t)(n / 2) * d + 17,
                      (size_t)(n - 1) * d + 63};
    float worst = 0.0f;
    for (int t = 0; t < 6; ++t) {
        size_t idx = idxs[t];
        float *ins[3] = {q, k, v};
        float grads[3] = {dq[idx], dk[idx], dv[idx]};
        for (int which = 0; which < 3; ++which) {
            float *a = ins[which];
            float orig = a[idx];
            a[idx] = orig + eps;
            double lp = orc_attn_loss(q, k, v, g, n, d, causal);
            a[idx] = orig - eps;
            double lm = orc_attn_loss(q, k, v, g, n, d, causal);
            a[idx] = orig;
            float fd = (float)((lp - lm) / (2.0 * (double)eps));
            float err = fabsf(fd - grads[which]) / (1e-3f + fabsf(grads[which]));
            worst = fmaxf(worst, err);
        }
    }
    free(q); free(k); free(v); free(g); free(dq); free(dk); free(dv);
    return worst;
}

/* attention_bwd.cu:32-44 `attn_bwd_preprocess`: Delta_i = sum_x dO[i,x] O[i,x],
 * over `rows` rows of width d, summed in x order. */
void orc_delta(const float *dout, const float *o, float *delta, size_t rows, int d) {
    for (size_t i = 0; i < rows; ++i) {
        float acc = 0.0f;
        for (int x = 0; x < d; ++x) acc += dout[i * d + x] * o[i * d + x];
        delta[i] = acc;
    }
}

/* ----------------------------------------------- batched / grouped -- */

/* Q, O, dQ: [B][Hq][N][d]; K, V, dK, dV: [B][Hkv][N][d]; LSE: [B][Hq][N].
 * Query head h reads KV head h / (Hq / Hkv) (03-llm-engine/src/cpu.rs:194,224). */
typedef struct {
    const float *q, *k, *v, *dout;
    float *o, *lse, *dq, *dk_h, *dv_h; /* dk_h / dv_h: per query head, [B][Hq][N][d] */
    int B, Hq, Hkv, N, d, causal;
    float scale;
    int next, total, bwd;
    pthread_mutex_t mu;
} orc_job;

static void run_slice(orc_job *jb, int t) {
    int b = t / jb->Hq, h = t % jb->Hq;
    int kvh = h / (jb->Hq / jb->Hkv);
    size_t nd = (size_t)jb->N * jb->d;
    size_t qo = ((size_t)b * jb->Hq + h) * nd;
    size_t ko = ((size_t)b * jb->Hkv + kvh) * nd;
    if (!jb->bwd) {
        orc_cpu_attention(jb->q + qo, jb->k + ko, jb->v + ko, jb->o + qo,
                          jb->lse ? jb->lse + ((size_t)b * jb->Hq + h) * jb->N : NULL, jb->N,
                          jb->d, jb->causal, jb->scale);
    } else {
        orc_cpu_attention_bwd(jb->q + qo, jb->k + ko, jb->v + ko, jb->dout + qo, jb->dq + qo,
                              jb->dk_h + qo, jb->dv_h + qo, jb->N, jb->d, jb->causal, jb->scale);
    }
}

static void *worker(void *arg) {
    orc_job *jb = (orc_job *)arg;
    for (;;) {
        pthread_mutex_lock(&jb->mu);
        int t = jb->next++;
        pthread_mutex_unlock(&jb->mu);
        if (t >= jb->total) break;
        run_slice(jb, t);
    }
    return NULL;
}

static void run_job(orc_job *jb, int nthreads) {
    jb->next = 0;
    jb->total = jb->B * jb->Hq;
    pthread_mutex_init(&jb->mu, NULL);
    if (nthreads <= 1) {
        worker(jb);
    } else {
        pthread_t *th = malloc(sizeof(pthread_t) * (size_t)nthreads);
        for (int i = 0; i < nthreads; ++i) pthread_create(&th[i], NULL, worker, jb);
        for (int i = 0; i < nthreads; ++i) pthread_join(th[i], NULL);
        free(th);
    }
    pthread_mutex_destroy(&jb->mu);
}

/* Forward over all (b, h) slices; `lse` may be NULL. Returns 0, or -1 on a
 * shape that the head mapping cannot serve. */
int orc_mha_fwd(int B, int Hq, int Hkv, int N, int d, int causal, float scale, const float *q,
                const float *k, const float *v, float *o, float *lse, int nthreads) {
    if (B < 0 || N < 0 || d <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv) return -1;
    orc_job jb;
    memset(&jb, 0, sizeof jb);
    jb.q = q; jb.k = k; jb.v = v; jb.o = o; jb.lse = lse;
    jb.B = B; jb.Hq = Hq; jb.Hkv = Hkv; jb.N = N; jb.d = d; jb.causal = causal; jb.scale = scale;
    run_job(&jb, nthreads);
    return 0;
}

/* Backward over all (b, h) slices. dK / dV of a KV head are the sum, in
 * increasing query-head order, of the per-query-head gradients of the heads
 * that share it, so the result does not depend on `nthreads`. */
int orc_mha_bwd(int B, int Hq, int Hkv, int N, int d, int causal, float scale, const float *q,
                const float *k, const float *v, const float *dout, float *dq, float *dk,
                float *dv, int nthreads) {
    if (B < 0 || N < 0 || d <= 0 || Hq <= 0 || Hkv <= 0 || Hq % Hkv) return -1;
    size_t nd = (size_t)N * d;
    size_t qsz = (size_t)B * Hq * nd;
    float *dk_h = malloc((qsz ? qsz : 1) * sizeof(float));
    float *dv_h = malloc((qsz ? qsz : 1) * sizeof(float));
    orc_job jb;
    memset(&jb, 0, sizeof jb);
    jb.q = q; jb.k = k; jb.v = v; jb.dout = dout; jb.dq = dq; jb.dk_h = dk_h; jb.dv_h = dv_h;
    jb.B = B; jb.Hq = Hq; jb.Hkv = Hkv; jb.N = N; jb.d = d; jb.causal = causal; jb.scale = scale;
    jb.bwd = 1;
    run_job(&jb, nthreads);
    int group = Hq / Hkv;
    for (int b = 0; b < B; ++b) {
        for (int kvh = 0; kvh < Hkv; ++kvh) {
            float *dko = dk + ((size_t)b * Hkv + kvh) * nd;
            float *dvo = dv + ((size_t)b * Hkv + kvh) * nd;
            memset(dko, 0, nd * sizeof(float));
            memset(dvo, 0, nd * sizeof(float));
            for (int g = 0; g < group; ++g) {
                size_t qo = ((size_t)b * Hq + (size_t)kvh * group + g) * nd;
                for (size_t e = 0; e < nd; ++e) {
                    dko[e] += dk_h[qo + e];
                    dvo[e] += dv_h[qo + e];
                }
            }
        }
    }
    free(dk_h);
    free(dv_h);
    return 0;
}

int orc_mutant(void) { return ORC_MUTANT; }
