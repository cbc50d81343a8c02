// Flash-attention forward for gfx950: O = softmax(Q K^T * scale) V and the
// per-row log-sum-exp, one pass over K/V with an online softmax.
//
// Follows the algorithm of attention_flash.cu:17-89 (online softmax, causal
// tile break, LSE = m + ln l at :85-87), re-tiled for CDNA4:
//   * workgroup = 4 waves = 128 queries of one (batch, head); each wave owns
//     32 queries, whose Q rows sit in registers as MFMA B operands (64 and
//     16 on grids too small to fill the GPU otherwise);
//   * K/V advance 64 keys per stage through double-buffered LDS, filled by
//     direct global->LDS loads issued one stage ahead;
//   * scores are computed transposed, S^T = K Q^T, so each lane owns one query
//     column: the running max / sum stay per lane and only the max needs a
//     cross-lane reduction (two permlane swaps);
//   * the output is accumulated transposed, O^T = V^T P^T, so the per-query
//     rescale factor is a per-lane scalar as well;
//   * exponentials are base 2: the fp32 scores are multiplied by
//     scale log2(e) (bf16, which keeps Q exact) or Q is (fp32);
//   * after the first stage the running max is only raised (and O and the sum
//     rescaled) when some p of a row exceeds 2^16 (fwd_stage_lazy), detected
//     from the per-lane row sums without computing a row maximum;
//   * only stages that straddle the causal diagonal or the end of the sequence
//     run the masking code (a separate instantiation of the stage body).
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

// Masking of a stage's scores, one compare per score: key k0 + 32 blk +
// bidx(t, g, r) is masked when it is past the lane's query position (causal)
// or past the last key, i.e. when its offset from the lane's first key of the
// stage, 32 blk + bidx(t, g, r) - bidx(0, g, 0) (a compile-time constant), is
// above the lane's limit below.
template <class Pol, bool CAUSAL>
__device__ __forceinline__ int fwd_mask_limit(int qpos, int k0, int Nk, int g) {
    return (CAUSAL ? min(qpos, Nk - 1) : Nk - 1) - k0 - Pol::bidx(0, g, 0);
}
template <class Pol>
__device__ __forceinline__ constexpr int fwd_mask_offset(int blk, int t, int g, int r) {
    return 32 * blk + Pol::bidx(t, g, r) - Pol::bidx(0, g, 0);
}

// One 64-key stage for one wave: scores in log2 units (x xmul when Q is kept
// exact, else qf holds Q scale log2(e)), online-softmax update,
// O^T += V^T P^T. PRIO: the matrix products run at raised wave priority.
// qpos0: position of the wave's first query row; Nk: key rows. EMPTY_ROWS:
// rows may have every key of the stage masked (a key split's first stage).
template <class Pol, int QT, bool CAUSAL, bool MASK, bool PRIO = false, bool EMPTY_ROWS = false>
__device__ __forceinline__ void fwd_stage(f32x4 (&acc)[Pol::D / 16][QT], float (&m)[QT], float (&lsum)[QT],
                                          const typename Pol::Frag (&qf)[QT][Pol::NC],
                                          const typename Pol::T *sk, const typename Pol::T *sv, int k0, int qpos0,
                                          int Nk, int g, int l16, float xmul) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
    f32x4 s[2][2][QT];  // [block][t][qt]
    wave_priority<PRIO>(1);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            Frag a[NC];
            Pol::lds_row_frags(a, sk, 32 * blk + Pol::arow(t, l16), g);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                f32x4 c = zero4();
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                s[blk][t][qt] = c;
            }
        }
    }
    wave_priority<PRIO>(0);
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int lim = fwd_mask_limit<Pol, CAUSAL>(qpos0 + 16 * qt + l16, k0, Nk, g);
        float mx = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = Pol::kExactScale ? s[blk][t][qt][r] * xmul : s[blk][t][qt][r];
                    if constexpr (MASK) v = fwd_mask_offset<Pol>(blk, t, g, r) > lim ? -INFINITY : v;
                    s[blk][t][qt][r] = v;
                    mx = fmaxf(mx, v);
                }
            }
        }
        mx = xg_max(mx);
        const float mnew = fmaxf(m[qt], mx);
        // a row with every key of the stage masked keeps m = -inf and gets
        // p = 0 (2^(-inf - 0)), not 2^(-inf - -inf) = NaN
        const float mref = EMPTY_ROWS && mnew == -INFINITY ? 0.f : mnew;
        const float corr = fast_exp2(m[qt] - mref);
        m[qt] = mnew;
        float ls = lsum[qt] * corr;
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) acc[xt][qt] *= corr;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = fast_exp2(s[blk][t][qt][r] - mref);
                    s[blk][t][qt][r] = pv;
                    ls += pv;
                }
            }
        }
        lsum[qt] = ls;
    }
    wave_priority<PRIO>(1);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        typename Pol::ChainB cb[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) cb[qt] = Pol::pack(s[blk][0][qt], s[blk][1][qt]);
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sv, 16 * xt, 32 * blk, g, l16);
            }
        }
    }
    wave_priority<PRIO>(0);
}

// fwd_stage for every stage after the first, with lazy rescaling. Key 0 is
// visible to every query (pos0 >= 0), so after the first stage m is finite for
// every row; a key split's work-group may leave a row at m = -inf after its
// first stage only when the row precedes every key of the split (causal), so
// every later stage masks the whole row (p = 0, nothing to rescale). The scores come out of the MFMAs relative to the running max m
// (the accumulators start at -m), and p = 2^(s - m) is taken optimistically
// with the old m. A lane's per-row sum of its p over the stage (16 keys)
// bounds each of them, so when no such sum exceeds kLazySum no p does either:
// O and the row sums then simply accumulate (m stays within log2(kLazySum) of
// the row's true running max, so nothing overflows or underflows in fp32 and
// the largest p of a row stays in [1, kLazySum]). Otherwise (an overflow shows
// as an infinite sum) the stage is redone exactly: the scores are recomputed
// from LDS, m rises to the row's max, O and the sum are rescaled, and the
// exponentials are taken again. LSE = m + log2(l) holds for any m used
// consistently, so the result is the online softmax's up to rounding. No row
// maximum is computed on the common path.
constexpr float kLazySum = 65536.0f;

// Scores of one 64-key stage relative to m: s = K Q^T scale log2(e) - m, with
// masked keys (MASK) at -inf. With Pol::kExactScale the accumulators start at
// -m / xmul and the fp32 result is multiplied by xmul = scale log2(e).
template <class Pol, int QT, bool CAUSAL, bool MASK, bool PRIO = false>
__device__ __forceinline__ void fwd_scores(f32x4 (&s)[2][2][QT], const float (&m)[QT],
                                           const typename Pol::Frag (&qf)[QT][Pol::NC], const typename Pol::T *sk,
                                           int k0, int qpos0, int Nk, int g, int l16, float xmul) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC;
    const float im = Pol::kExactScale ? 1.0f / xmul : 1.0f;
    f32x4 nm[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const float n = -m[qt] * im;
        nm[qt] = f32x4{n, n, n, n};
    }
    wave_priority<PRIO>(1);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            Frag a[NC];
            Pol::lds_row_frags(a, sk, 32 * blk + Pol::arow(t, l16), g);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                f32x4 c = nm[qt];
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                s[blk][t][qt] = Pol::kExactScale ? c * xmul : c;
            }
        }
    }
    wave_priority<PRIO>(0);
    if constexpr (MASK) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int lim = fwd_mask_limit<Pol, CAUSAL>(qpos0 + 16 * qt + l16, k0, Nk, g);
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        if (fwd_mask_offset<Pol>(blk, t, g, r) > lim) s[blk][t][qt][r] = -INFINITY;
                    }
                }
            }
        }
    }
}

// p = 2^s in place, added to l (row qt of this lane).
template <int QT>
__device__ __forceinline__ void fwd_exp_sum(f32x4 (&s)[2][2][QT], float (&l)[QT]) {
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        float ls = l[qt];
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float pv = fast_exp2(s[blk][t][qt][r]);
                    s[blk][t][qt][r] = pv;
                    ls += pv;
                }
            }
        }
        l[qt] = ls;
    }
}

template <class Pol, int QT, bool CAUSAL, bool MASK, bool PRIO = false>
__device__ __forceinline__ void fwd_stage_lazy(f32x4 (&acc)[Pol::D / 16][QT], float (&m)[QT], float (&lsum)[QT],
                                               const typename Pol::Frag (&qf)[QT][Pol::NC],
                                               const typename Pol::T *sk, const typename Pol::T *sv, int k0,
                                               int qpos0, int Nk, int g, int l16, float xmul) {
    constexpr int XT = Pol::D / 16;
    f32x4 s[2][2][QT];  // [block][t][qt]
    fwd_scores<Pol, QT, CAUSAL, MASK, PRIO>(s, m, qf, sk, k0, qpos0, Nk, g, l16, xmul);
    float l0[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) l0[qt] = lsum[qt];
    fwd_exp_sum(s, lsum);
    bool over = false;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) over = over || lsum[qt] > l0[qt] + kLazySum;
    if (__builtin_amdgcn_ballot_w64(over) != 0) {
        // some p of the wave exceeded kLazySum: redo the stage with m raised to
        // each row's max (rows whose max did not rise keep shift 0)
        fwd_scores<Pol, QT, CAUSAL, MASK, PRIO>(s, m, qf, sk, k0, qpos0, Nk, g, l16, xmul);
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            float v = -INFINITY;
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) v = fmaxf(v, s[blk][t][qt][r]);
                }
            }
            const float shift = fmaxf(xg_max(v), 0.f);
            const float corr = fast_exp2(-shift);
            m[qt] += shift;
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) acc[xt][qt] *= corr;
            lsum[qt] = l0[qt] * corr;
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[blk][t][qt][r] -= shift;
                }
            }
        }
        fwd_exp_sum(s, lsum);
    }
    wave_priority<PRIO>(1);
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        typename Pol::ChainB cb[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) cb[qt] = Pol::pack(s[blk][0][qt], s[blk][1][qt]);
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sv, 16 * xt, 32 * blk, g, l16);
            }
        }
    }
    wave_priority<PRIO>(0);
}

// One work-group of the forward, grid (B Hq, query blocks). QT: 16-query
// tiles per wave (the work-group takes 64 QT queries); the kernels are
// compiled for a number of waves per SIMD (the names' w*). PAGED: K/V rows
// through Params::block_table (the kernels named *_pg). SPLIT (kernels *_sp,
// grid.z = the splits): work-group z takes stages [z nsteps / S, (z + 1)
// nsteps / S) of its query block's keys and writes its unnormalised O and
// its rows' running max and sum to Params::fwd_part; fwd_merge adds the
// splits.
template <class Pol, bool CAUSAL, int QT, bool PAGED = false, bool SPLIT = false>
__device__ __forceinline__ void fwd_entry(const Params &p) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int BQ = 64 * QT, BK = Pol::ROWS;
    // bf16: the matrix products at raised wave priority, the softmax at normal
    // (A/B on one box: cfg4 78.1 -> 74.3 us, cfg5 d = 128 51.0 -> 47.2,
    // non-causal B2 H12 N4096 112.2 -> 109.7; the 64-query d = 64 launches
    // lost 1-3% with it)
    constexpr bool kPrio = Pol::kExactScale && (QT == 2 || D == 128);

    __shared__ __attribute__((aligned(16))) T sK[2][BK * D];
    __shared__ __attribute__((aligned(16))) T sV[2][BK * D];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N, Nk = p.Nk, pos0 = p.pos0;
    const int nqb = (N + BQ - 1) / BQ;
    // causal: heaviest first, in the order balanced per CU over the work-groups
    // resident at once (cu_order_wg; ranks are heads fastest)
    const int rank = CAUSAL ? cu_order_wg((int)(blockIdx.y * gridDim.x + blockIdx.x), p.cu_run, p.cu_runs)
                            : (int)(blockIdx.y * gridDim.x + blockIdx.x);
    const int bh = rank % (int)gridDim.x;
    const int qb = CAUSAL ? nqb - 1 - rank / (int)gridDim.x : rank / (int)gridDim.x;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const T *Q = static_cast<const T *>(p.q) + b * p.q_bs + h * p.q_hs;
    const size_t kvoff = b * p.kv_bs + kvh * p.kv_hs;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int q0 = qb * BQ + wave * 16 * QT;
    const int qpos0 = pos0 + q0;  // position of the wave's first query row
    wg_time(0);

    Frag qf[QT][NC];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) Pol::gmem_row_frags(qf[qt], Q, q0 + 16 * qt + l16, N, p.q_rs, g);
    // fp32: Q scale log2(e), so the scores come out of the MFMAs in log2
    // units; bf16 keeps Q exact and scales the fp32 scores instead
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) {
            if (!Pol::kExactScale) qf[qt][kc] = Pol::scaled(qf[qt][kc], p.scale_log2);
        }
    }
    f32x4 acc[XT][QT];
    float m[QT], lsum[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) acc[xt][qt] = zero4();
        m[qt] = -INFINITY;
        lsum[qt] = 0.f;
    }

    const int kend = CAUSAL ? min(Nk, pos0 + qb * BQ + BQ) : Nk;
    const int nsteps = (kend + BK - 1) / BK;
    // this work-group's stages [s_lo, s_hi) (SPLIT: its share; the first one
    // it runs takes the plain softmax body, the running max starting at -inf)
    const int s_lo = SPLIT ? (int)((long long)blockIdx.z * nsteps / gridDim.z) : 0;
    const int s_hi = SPLIT ? (int)((long long)(blockIdx.z + 1) * nsteps / gridDim.z) : nsteps;
    wg_info(2, qb, s_hi - s_lo);

    const RowPlan<Pol> plan(tid);
    // PAGED: the table entries of stage 0 now, then each stage fetches those
    // of the stage after the one it stages
    PagedRows<Pol> paged;
    auto stage_next = [&](T *sk, T *sv, int k0) __attribute__((always_inline)) {
        if constexpr (PAGED) {
            paged.stage(sk, sv, K, V, k0, Nk, p.bs_shift, plan, wave, p.kv_rs);
            if (k0 + BK < Nk) paged.fetch(p.block_table, p.bs_shift, k0 + BK, Nk, plan);
        } else {
            stage_kv<Pol>(sk, sv, K, V, k0, Nk, plan, wave, p.kv_rs);
        }
    };
    if (!SPLIT || s_lo < s_hi) {
        if constexpr (PAGED) paged.fetch(p.block_table, p.bs_shift, s_lo * BK, Nk, plan);
        stage_next(sK[0], sV[0], s_lo * BK);
    }
    wait_stage();
    __syncthreads();
    wg_time(1);

    // Leading stages that no wave masks (all their keys exist and precede the
    // workgroup's first query position) run in pairs with the LDS buffer a
    // compile-time constant, so the tile addresses fold into the instructions'
    // immediate offsets; the rest choose buffer and masking at run time.
    // The first stage runs the plain online-softmax body (the running max
    // starts at -inf); later ones the lazy-rescaling body.
    auto main_stage = [&](auto buf, auto first, int st) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < s_hi) stage_next(sK[B ^ 1], sV[B ^ 1], (st + 1) * BK);
        if constexpr (decltype(first)::value) {
            fwd_stage<Pol, QT, CAUSAL, false, kPrio>(acc, m, lsum, qf, sK[B], sV[B], st * BK, qpos0, Nk, g, l16,
                                                     p.scale_log2);
        } else {
            fwd_stage_lazy<Pol, QT, CAUSAL, false, kPrio>(acc, m, lsum, qf, sK[B], sV[B], st * BK, qpos0, Nk, g, l16,
                                                          p.scale_log2);
        }
        wait_stage();
        __syncthreads();
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    const int nmain = min(min(s_hi, Nk / BK), CAUSAL ? (pos0 + qb * BQ + 1) / BK : s_hi);
    int st = s_lo;
    if (nmain > st) main_stage(B0{}, std::true_type{}, st++);
    for (; st + 1 < nmain; st += 2) {
        main_stage(B1{}, std::false_type{}, st);
        main_stage(B0{}, std::false_type{}, st + 1);
    }
    if (st < nmain) main_stage(B1{}, std::false_type{}, st++);
    // the remaining stages may straddle the diagonal or the end of the keys:
    // one masked body each for the first stage and the later ones (a wave
    // that skips a stage skips every later one, so its first run stage is
    // the work-group's first)
    for (; st < s_hi; ++st) {
        const int cur = (st - s_lo) & 1;
        if (st + 1 < s_hi) stage_next(sK[cur ^ 1], sV[cur ^ 1], (st + 1) * BK);
        const int k0 = st * BK;
        // a wave whose queries all precede the stage's keys has nothing to do
        if (!CAUSAL || k0 <= qpos0 + 16 * QT - 1) {
            if (st == s_lo) {
                fwd_stage<Pol, QT, CAUSAL, true, kPrio, SPLIT>(acc, m, lsum, qf, sK[cur], sV[cur], k0, qpos0, Nk, g,
                                                               l16, p.scale_log2);
            } else {
                fwd_stage_lazy<Pol, QT, CAUSAL, true, kPrio>(acc, m, lsum, qf, sK[cur], sV[cur], k0, qpos0, Nk, g, l16,
                                                             p.scale_log2);
            }
        }
        wait_stage();
        __syncthreads();
    }

    wg_time(2);
    if constexpr (SPLIT) {
        // the split's partial: O unnormalised, then (running max, sum) per row
        const size_t rows = (size_t)gridDim.z * p.B * p.Hq * N;
        const size_t r0 = ((size_t)blockIdx.z * p.B * p.Hq + bh) * N;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qi = q0 + 16 * qt + l16;
            const float ltot = xg_sum(lsum[qt]);
            if (qi < N) {
                float *po = p.fwd_part + (r0 + qi) * D;
#pragma unroll
                for (int xt = 0; xt < XT; ++xt) store4<float>(po + 16 * xt + 4 * g, acc[xt][qt], 1.0f);
                if (g == 0) {
                    float *pml = p.fwd_part + rows * D + 2 * (r0 + qi);
                    *reinterpret_cast<float2 *>(pml) = make_float2(m[qt], ltot);
                }
            }
        }
        wg_time_after_stores();
        return;
    }
    T *O = static_cast<T *>(p.o) + b * p.o_bs + h * p.o_hs;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        const float ltot = xg_sum(lsum[qt]);
        const float inv = 1.0f / ltot;
        if constexpr (std::is_same<T, u16>::value) {
            // bf16 rows, 16 bytes per lane (rows start on 16-byte boundaries)
            T *row = O + (size_t)min(qi, N - 1) * p.o_rs;
#pragma unroll
            for (int xt = 0; xt < XT; xt += 2)
                store8_pair_bf16(row, 16 * xt, g, acc[xt][qt], acc[xt + 1][qt], inv, qi < N);
        } else if (qi < N) {
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) store4<T>(O + (size_t)qi * p.o_rs + 16 * xt + 4 * g, acc[xt][qt], inv);
        }
        if (qi < N && p.lse != nullptr && g == 0) p.lse[(size_t)bh * N + qi] = (m[qt] + fast_log2(ltot)) * kLn2;
    }
    wg_time_after_stores();
}

// Adds the S key splits of a split forward (fwd_entry<..., SPLIT>), one
// thread per four elements of a query row: with M the largest of the splits'
// running maxima (log2 units), O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M)
// l_s, in split order, written as the forward writes O. A split that holds
// no key of the row has m = -inf and weight 0. Every load is issued before
// the first is used (the loops unrolled to MAXS >= S), so a call costs one
// memory latency rather than one per split; MAXS = 8 keeps the registers of
// the common case low (the 32-split form takes 205 VGPRs).
constexpr int kFwdMaxSplits = 32;

template <class T, int D, int MAXS>
__device__ __forceinline__ void fwd_merge_body(const Params &p, int S) {
    constexpr int C = D / 4;
    const size_t rows = (size_t)p.B * p.Hq * p.N;
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * C) return;
    const size_t r = t / C;
    const int c = (int)(t % C);
    const float2 *ml = reinterpret_cast<const float2 *>(p.fwd_part + (size_t)S * rows * D);
    float2 v[MAXS];
    float4 a[MAXS];
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < S) {
            v[sp] = ml[sp * rows + r];
            a[sp] = *reinterpret_cast<const float4 *>(p.fwd_part + (sp * rows + r) * D + 4 * c);
        }
    }
    // the split holding key 0 (visible to every row) makes M finite
    float M = -INFINITY;
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) M = sp < S ? fmaxf(M, v[sp].x) : M;
    float L = 0.f;
    f32x4 o = zero4();
#pragma unroll
    for (int sp = 0; sp < MAXS; ++sp) {
        if (sp < S) {
            const float w = fast_exp2(v[sp].x - M);
            L += w * v[sp].y;
            o[0] += w * a[sp].x;
            o[1] += w * a[sp].y;
            o[2] += w * a[sp].z;
            o[3] += w * a[sp].w;
        }
    }
    const int bh = (int)(r / p.N), qi = (int)(r % p.N);
    const int b = bh / p.Hq, h = bh % p.Hq;
    T *O = static_cast<T *>(p.o) + b * p.o_bs + h * p.o_hs + (size_t)qi * p.o_rs + 4 * c;
    store4<T>(O, o, 1.0f / L);
    if (p.lse != nullptr && c == 0) p.lse[r] = (M + fast_log2(L)) * kLn2;
}

// The code object's forward kernels (fa_kernels.h): policy, causal, waves
// per SIMD, query tiles per wave.
#if defined(__HIP_DEVICE_COMPILE__)
#define MXFA_FWD(NAME, POL, CAUSAL, WPS, QT)                                                            \
    extern "C" __global__ __launch_bounds__(256, WPS) void NAME(Params p) { fwd_entry<POL, CAUSAL, QT>(p); }
#define MXFA_FWD_PG(NAME, POL, WPS, QT)                                                                 \
    extern "C" __global__ __launch_bounds__(256, WPS) void NAME(Params p) { fwd_entry<POL, true, QT, true>(p); }
MXFA_FWD(mxfa_fwd_b64_c_w3_q2, PolBF16<64>, true, 3, 2)
MXFA_FWD(mxfa_fwd_b64_c_w2_q2, PolBF16<64>, true, 2, 2)
MXFA_FWD(mxfa_fwd_b64_c_w3_q1, PolBF16<64>, true, 3, 1)
MXFA_FWD(mxfa_fwd_b64_n_w2_q2, PolBF16<64>, false, 2, 2)
MXFA_FWD(mxfa_fwd_b64_n_w3_q1, PolBF16<64>, false, 3, 1)
MXFA_FWD(mxfa_fwd_b128_c_w2_q2, PolBF16<128>, true, 2, 2)
MXFA_FWD(mxfa_fwd_b128_c_w2_q1, PolBF16<128>, true, 2, 1)
MXFA_FWD(mxfa_fwd_b128_n_w2_q2, PolBF16<128>, false, 2, 2)
// fp32: 64-query work-groups at two waves per SIMD (218 VGPRs). The 128-query
// form ran at one wave (331 registers) and was slower at every shape measured
// (causal B4 H12 N1024 75.6 -> 69.6 us, B1 H12 N4096 275 -> 232, B4 H12 N4096
// 886 -> 803; non-causal B1 H1 N256 22.5 -> 13.9, B4 H12 N1024 145 -> 108,
// B1 H12 N32768 25.5 -> 23.9 ms; the prefill of 512 tokens after 3584 at 14
// query heads 274 -> 151 us)
MXFA_FWD(mxfa_fwd_f64_c_w2_q1, PolF32<64>, true, 2, 1)
MXFA_FWD(mxfa_fwd_f64_n_w2_q1, PolF32<64>, false, 2, 1)
// the prefill over a paged cache (causal, as the prefill always is)
// (the table entries take registers: the three-wave 128-query d = 64 and the
// 128-query d = 128 forms would spill in their loops, so paged launches use
// two waves at d = 64 and 64-query work-groups at d = 128)
MXFA_FWD_PG(mxfa_fwd_b64_c_w2_q2_pg, PolBF16<64>, 2, 2)
MXFA_FWD_PG(mxfa_fwd_b64_c_w3_q1_pg, PolBF16<64>, 3, 1)
MXFA_FWD_PG(mxfa_fwd_b128_c_w2_q1_pg, PolBF16<128>, 2, 1)
MXFA_FWD_PG(mxfa_fwd_f64_c_w2_q1_pg, PolF32<64>, 2, 1)
// the prefill split over its keys (causal, 64-query work-groups) and the
// merge of the splits
#define MXFA_FWD_SP(NAME, POL, WPS, PG)                                                                \
    extern "C" __global__ __launch_bounds__(256, WPS) void NAME(Params p) { fwd_entry<POL, true, 1, PG, true>(p); }
MXFA_FWD_SP(mxfa_fwd_b64_c_w3_q1_sp, PolBF16<64>, 3, false)
MXFA_FWD_SP(mxfa_fwd_b128_c_w2_q1_sp, PolBF16<128>, 2, false)
MXFA_FWD_SP(mxfa_fwd_f64_c_w2_q1_sp, PolF32<64>, 2, false)
MXFA_FWD_SP(mxfa_fwd_b64_c_w3_q1_pg_sp, PolBF16<64>, 3, true)
MXFA_FWD_SP(mxfa_fwd_b128_c_w2_q1_pg_sp, PolBF16<128>, 2, true)
MXFA_FWD_SP(mxfa_fwd_f64_c_w2_q1_pg_sp, PolF32<64>, 2, true)
#define MXFA_FWD_MERGE(NAME, T, D, MAXS)                                                               \
    extern "C" __global__ __launch_bounds__(256) void NAME(Params p, int splits) {                     \
        fwd_merge_body<T, D, MAXS>(p, splits);                                                         \
    }
MXFA_FWD_MERGE(mxfa_fwd_merge8_b64, u16, 64, 8)
MXFA_FWD_MERGE(mxfa_fwd_merge8_b128, u16, 128, 8)
MXFA_FWD_MERGE(mxfa_fwd_merge8_f64, float, 64, 8)
MXFA_FWD_MERGE(mxfa_fwd_merge32_b64, u16, 64, kFwdMaxSplits)
MXFA_FWD_MERGE(mxfa_fwd_merge32_b128, u16, 128, kFwdMaxSplits)
MXFA_FWD_MERGE(mxfa_fwd_merge32_f64, float, 64, kFwdMaxSplits)
#undef MXFA_FWD
#undef MXFA_FWD_PG
#undef MXFA_FWD_SP
#undef MXFA_FWD_MERGE
#endif

// The kernel of (policy, causal) compiled for `wps` waves per SIMD with `qt`
// query tiles per wave (one of the list above); paged: its *_pg form (causal
// kernels only).
template <class Pol, bool CAUSAL>
static KernelId fwd_kernel_id(int wps, int qt, bool paged) {
    if constexpr (Pol::kExactScale && Pol::D == 64) {
        if (CAUSAL && paged) return qt == 1 ? k_mxfa_fwd_b64_c_w3_q1_pg : k_mxfa_fwd_b64_c_w2_q2_pg;
        if (CAUSAL) return qt == 1 ? k_mxfa_fwd_b64_c_w3_q1 : wps == 3 ? k_mxfa_fwd_b64_c_w3_q2 : k_mxfa_fwd_b64_c_w2_q2;
        return qt == 1 ? k_mxfa_fwd_b64_n_w3_q1 : k_mxfa_fwd_b64_n_w2_q2;
    } else if constexpr (Pol::kExactScale) {
        if (CAUSAL && paged) return k_mxfa_fwd_b128_c_w2_q1_pg;
        if (CAUSAL) return qt == 1 ? k_mxfa_fwd_b128_c_w2_q1 : k_mxfa_fwd_b128_c_w2_q2;
        return k_mxfa_fwd_b128_n_w2_q2;
    } else {
        if (CAUSAL && paged) return k_mxfa_fwd_f64_c_w2_q1_pg;
        return CAUSAL ? k_mxfa_fwd_f64_c_w2_q1 : k_mxfa_fwd_f64_n_w2_q1;
    }
}

template <class Pol, bool CAUSAL, int QT>
static hipError_t launch_fwd_qt(Params p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hq, (p.N + 64 * QT - 1) / (64 * QT));
    constexpr int kHi = Pol::kWavesFwdCausal;
    int wps = QT == 1 ? kHi : Pol::kWaves;
    if constexpr (CAUSAL && kHi > Pol::kWaves && QT > 1) {
        // enough causal work-groups to fill kHi per CU (256 CUs); not paged
        if ((long long)grid.x * grid.y >= 256LL * kHi && p.block_table == nullptr) wps = kHi;
    }
    const KernelId id = fwd_kernel_id<Pol, CAUSAL>(wps, QT, p.block_table != nullptr);
    if (CAUSAL) cu_balance(&p, id, (long long)grid.x * grid.y);
    void *args[] = {&p};
    return launch_kernel(id, grid, dim3(256), args, stream);
}

// bf16 launches whose 128-query work-groups would not fill every resident
// slot (256 CUs x the 128-query kernel's waves per SIMD: 3 at d = 64, 2 at
// d = 128) take 64-query work-groups (one 16-query tile per wave): twice the
// work-groups and half the critical path (the heaviest block's keys times its
// queries), for twice the LDS reads per MFMA. Measured on the MI355X: causal
// B1 H12 N4096 d64 54.3 -> 40.3 us, B1 H8 N2048 d128 43.4 -> 28.8 us,
// non-causal B1 H12 N4096 d64 74.6 -> 65.5 us; at 768 work-groups (causal B1
// H12 N8192 d64) 125 against 135 us keeps 128 queries, and so does d = 128 at
// 512 (causal B1 H32 Hkv4 N2048: 44.6 against 45.5 us). Non-causal d = 128
// keeps them (B1 H8 N4096: 77.2 against 80.2 us). A d = 128 prefill takes
// 64-query work-groups at any grid, as its paged form must (the 128-query
// d = 128 kernel would spill with the block-table registers): the wave's
// rows decide when the lazy rescale redoes a stage, so both tilings must match
// for the paged prefill to give the contiguous one's bits.
template <class Pol, bool CAUSAL>
static hipError_t launch_fwd_t(const Params &p, hipStream_t stream) {
    if constexpr (Pol::kExactScale && (CAUSAL || Pol::D == 64)) {
        constexpr long long kSlots = 256LL * Pol::kWavesFwdCausal;
        const long long wg = (long long)p.B * p.Hq * ((p.N + 127) / 128);
        if (wg < kSlots || (Pol::D == 128 && p.prefill != 0))
            return launch_fwd_qt<Pol, CAUSAL, 1>(p, stream);
    }
    if constexpr (!Pol::kExactScale) return launch_fwd_qt<Pol, CAUSAL, 1>(p, stream);  // fp32: see the kernels
    return launch_fwd_qt<Pol, CAUSAL, 2>(p, stream);
}

// Splits of the prefill's keys: none (1) when the 64-query work-groups
// already fill the resident slots (256 CUs x waves per SIMD) halfway, or when
// the heaviest query block has under 16 key stages (bf16; 8 for fp32), where
// the merging launch costs more than the split saves (measured on the MI355X,
// Qwen2.5 heads, 512 tokens at position 0, 8 stages: bf16 19.7 -> 24.6 us
// with 2 splits, fp32 36.5 -> 32.6 us); else enough to fill them, with at
// least 2 key stages per split and at most kFwdMaxSplits splits.
int fwd_splits(const Params &p, int dtype_bf16, int d) {
    const long long wgs = (long long)p.B * p.Hq * ((p.N + 63) / 64);
    const long long slots = 256LL * (dtype_bf16 && d == 64 ? 3 : 2);
    if (2 * wgs >= slots) return 1;
    const long long stages = (std::min(p.Nk, p.pos0 + p.N) + 63) / 64;  // the heaviest block's
    if (stages < (dtype_bf16 ? 16 : 8)) return 1;
    long long s = (slots + wgs - 1) / wgs;
    s = std::min(s, std::max(1LL, stages / 2));
    return (int)std::min(s, (long long)kFwdMaxSplits);
}

size_t fwd_split_workspace_bytes(const Params &p, int d, int splits) {
    if (splits <= 1) return 0;
    return (size_t)splits * p.B * p.Hq * p.N * (size_t)(d + 2) * sizeof(float);
}

hipError_t launch_fwd_split(const Params &p, int dtype_bf16, int d, int splits, hipStream_t stream) {
    if (p.fwd_part == nullptr || splits < 2 || splits > kFwdMaxSplits) return hipErrorInvalidValue;
    const bool pg = p.block_table != nullptr;
    const KernelId kf =
        dtype_bf16 ? (d == 64 ? (pg ? k_mxfa_fwd_b64_c_w3_q1_pg_sp : k_mxfa_fwd_b64_c_w3_q1_sp)
                              : (pg ? k_mxfa_fwd_b128_c_w2_q1_pg_sp : k_mxfa_fwd_b128_c_w2_q1_sp))
                   : (pg ? k_mxfa_fwd_f64_c_w2_q1_pg_sp : k_mxfa_fwd_f64_c_w2_q1_sp);
    const bool m8 = splits <= 8;
    const KernelId km = dtype_bf16 ? (d == 64 ? (m8 ? k_mxfa_fwd_merge8_b64 : k_mxfa_fwd_merge32_b64)
                                              : (m8 ? k_mxfa_fwd_merge8_b128 : k_mxfa_fwd_merge32_b128))
                                   : (m8 ? k_mxfa_fwd_merge8_f64 : k_mxfa_fwd_merge32_f64);
    Params q = p;
    void *args[] = {&q};
    hipError_t e = launch_kernel(kf, dim3(p.B * p.Hq, (p.N + 63) / 64, splits), dim3(256), args, stream);
    if (e != hipSuccess) return e;
    const size_t n = (size_t)p.B * p.Hq * p.N * (d / 4);
    int s = splits;
    void *margs[] = {&q, &s};
    return launch_kernel(km, dim3((unsigned)((n + 255) / 256)), dim3(256), margs, stream);
}

hipError_t launch_fwd(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream) {
    if (p.block_table != nullptr && !causal) return hipErrorInvalidValue;  // paged kernels are causal
#define MXFA_FWD(POL, DD)                                                            \
    if (d == DD) return causal ? launch_fwd_t<POL<DD>, true>(p, stream)            \
                               : launch_fwd_t<POL<DD>, false>(p, stream);
    if (dtype_bf16) {
        MXFA_FWD(PolBF16, 64)
        MXFA_FWD(PolBF16, 128)
    } else {
        MXFA_FWD(PolF32, 64)
    }
#undef MXFA_FWD
    return hipErrorInvalidValue;
}

}  // namespace mxfa
