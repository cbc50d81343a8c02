// Flash-attention forward for gfx950: O = softmax(Q K^T * scale) V and the
// per-row log-sum-exp, one pass over K/V with an online softmax.
//
// Follows the algorithm of attention_flash.cu:17-89 (online softmax, causal
// tile break, LSE = m + ln l at :85-87), re-tiled for CDNA4:
//   * workgroup = 4 waves = 128 queries of one (batch, head); each wave owns
//     32 queries, whose Q rows sit in registers as MFMA B operands;
//   * K/V advance 64 keys per stage through double-buffered LDS, filled by
//     direct global->LDS loads issued one stage ahead;
//   * scores are computed transposed, S^T = K Q^T, so each lane owns one query
//     column: the running max / sum stay per lane and only the max needs a
//     cross-lane reduction (two permlane swaps);
//   * the output is accumulated transposed, O^T = V^T P^T, so the per-query
//     rescale factor is a per-lane scalar as well;
//   * exponentials are base 2 with log2(e) folded into the scale;
//   * after the first stage the running max is only raised (and O and the sum
//     rescaled) when a score exceeds it by a factor above 2^8 (fwd_stage_lazy);
//   * only stages that straddle the causal diagonal or the end of the sequence
//     run the masking code (a separate instantiation of the stage body).
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

// One 64-key stage for one wave: scores (in log2 units: qf holds Q scale
// log2(e)), online-softmax update, O^T += V^T P^T.
// qpos0: position of the wave's first query row; Nk: key rows.
template <class Pol, bool CAUSAL, bool MASK>
__device__ __forceinline__ void fwd_stage(f32x4 (&acc)[Pol::D / 16][2], float (&m)[2], float (&lsum)[2],
                                          const typename Pol::Frag (&qf)[2][Pol::NC],
                                          const typename Pol::T *sk, const typename Pol::T *sv, int k0, int qpos0,
                                          int Nk, int g, int l16) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
    f32x4 s[2][2][2];  // [block][t][qt]
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            Frag a[NC];
            Pol::lds_row_frags(a, sk, 32 * blk + Pol::arow(t, l16), g);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f32x4 c = zero4();
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                s[blk][t][qt] = c;
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qpos = qpos0 + 16 * qt + l16;
        float mx = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float v = s[blk][t][qt][r];
                    if constexpr (MASK) {
                        const int key = k0 + 32 * blk + Pol::bidx(t, g, r);
                        v = (key >= Nk || (CAUSAL && key > qpos)) ? -INFINITY : v;
                    }
                    s[blk][t][qt][r] = v;
                    mx = fmaxf(mx, v);
                }
            }
        }
        mx = xg_max(mx);
        const float mnew = fmaxf(m[qt], mx);
        const float corr = fast_exp2(m[qt] - mnew);
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
                    const float pv = fast_exp2(s[blk][t][qt][r] - mnew);
                    s[blk][t][qt][r] = pv;
                    ls += pv;
                }
            }
        }
        lsum[qt] = ls;
    }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        typename Pol::ChainB cb[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) cb[qt] = Pol::pack(s[blk][0][qt], s[blk][1][qt]);
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sv, 16 * xt, 32 * blk, g, l16);
        }
    }
}

// fwd_stage for every stage after the first, with lazy rescaling. Key 0 is
// visible to every query (pos0 >= 0), so after the first stage m is finite for
// every row. The scores come out of the MFMAs relative to the running max (the
// accumulators start at -m), and m, O and the sum are only rescaled when some
// score of the wave exceeds its row's m by more than kLazy (log2 units).
// Otherwise p = 2^(s - m) with the old m, so p <= 2^kLazy: m never exceeds the
// row's true running max and never falls more than kLazy below it, so the
// largest p of each row lies in [1, 2^kLazy] and neither it nor the fp32 sum
// can overflow or underflow. The result is the online softmax's up to
// rounding, since LSE = m + log2(l) holds for any m used consistently.
constexpr float kLazy = 8.0f;

template <class Pol, bool CAUSAL, bool MASK>
__device__ __forceinline__ void fwd_stage_lazy(f32x4 (&acc)[Pol::D / 16][2], float (&m)[2], float (&lsum)[2],
                                               const typename Pol::Frag (&qf)[2][Pol::NC],
                                               const typename Pol::T *sk, const typename Pol::T *sv, int k0,
                                               int qpos0, int Nk, int g, int l16) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
    f32x4 s[2][2][2];  // [block][t][qt]
    const f32x4 nm[2] = {f32x4{-m[0], -m[0], -m[0], -m[0]}, f32x4{-m[1], -m[1], -m[1], -m[1]}};
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            Frag a[NC];
            Pol::lds_row_frags(a, sk, 32 * blk + Pol::arow(t, l16), g);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f32x4 c = nm[qt];
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                s[blk][t][qt] = c;
            }
        }
    }
    float mx[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qpos = qpos0 + 16 * qt + l16;
        float v = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = s[blk][t][qt][r];
                    if constexpr (MASK) {
                        const int key = k0 + 32 * blk + Pol::bidx(t, g, r);
                        x = (key >= Nk || (CAUSAL && key > qpos)) ? -INFINITY : x;
                        s[blk][t][qt][r] = x;
                    }
                    v = fmaxf(v, x);
                }
            }
        }
        mx[qt] = xg_max(v);
    }
    if (__builtin_amdgcn_ballot_w64(mx[0] > kLazy || mx[1] > kLazy) != 0) {
        // some row of the wave moved up by more than kLazy: rescale (rows whose
        // max did not rise keep shift 0) and shift its scores in place, so the
        // exponentials below serve both cases from the same registers
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const float shift = fmaxf(mx[qt], 0.f);
            const float corr = fast_exp2(-shift);
            m[qt] += shift;
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) acc[xt][qt] *= corr;
            lsum[qt] *= corr;
#pragma unroll
            for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[blk][t][qt][r] -= shift;
                }
            }
        }
    }
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        float ls = lsum[qt];
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
        lsum[qt] = ls;
    }
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        typename Pol::ChainB cb[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) cb[qt] = Pol::pack(s[blk][0][qt], s[blk][1][qt]);
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sv, 16 * xt, 32 * blk, g, l16);
        }
    }
}

// WPS: waves per SIMD the kernel is compiled for.
template <class Pol, bool CAUSAL, int WPS>
__global__ __launch_bounds__(256, WPS) void fwd_kernel(Params p) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int BQ = 128, BK = Pol::ROWS;

    __shared__ __attribute__((aligned(16))) T sK[2][BK * D];
    __shared__ __attribute__((aligned(16))) T sV[2][BK * D];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N, Nk = p.Nk, pos0 = p.pos0;
    const int bh = blockIdx.x;
    const int nqb = (N + BQ - 1) / BQ;
    const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;  // heaviest first
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const T *Q = static_cast<const T *>(p.q) + b * p.q_bs + h * p.q_hs;
    const size_t kvoff = b * p.kv_bs + kvh * p.kv_hs;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int q0 = qb * BQ + wave * 32;
    const int qpos0 = pos0 + q0;  // position of the wave's first query row

    Frag qf[2][NC];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        Pol::gmem_row_frags(qf[qt], Q + (size_t)qi * p.q_rs, g, qi < N);
        // Q scale log2(e): the scores come out of the MFMAs in log2 units
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) qf[qt][kc] = Pol::scaled(qf[qt][kc], p.scale_log2);
    }
    f32x4 acc[XT][2];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) acc[xt][0] = acc[xt][1] = zero4();
    float m[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.f, 0.f};

    const int kend = CAUSAL ? min(Nk, pos0 + qb * BQ + BQ) : Nk;
    const int nsteps = (kend + BK - 1) / BK;

    const RowPlan<Pol> plan(tid);
    stage_kv<Pol>(sK[0], sV[0], K, V, 0, Nk, plan, wave, p.kv_rs);
    wait_stage();
    __syncthreads();

    // Leading stages that no wave masks (all their keys exist and precede the
    // workgroup's first query position) run in pairs with the LDS buffer a
    // compile-time constant, so the tile addresses fold into the instructions'
    // immediate offsets; the rest choose buffer and masking at run time.
    // The first stage runs the plain online-softmax body (the running max
    // starts at -inf); later ones the lazy-rescaling body.
    auto main_stage = [&](auto buf, auto first, int st) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < nsteps) stage_kv<Pol>(sK[B ^ 1], sV[B ^ 1], K, V, (st + 1) * BK, Nk, plan, wave, p.kv_rs);
        if constexpr (decltype(first)::value) {
            fwd_stage<Pol, CAUSAL, false>(acc, m, lsum, qf, sK[B], sV[B], st * BK, qpos0, Nk, g, l16);
        } else {
            fwd_stage_lazy<Pol, CAUSAL, false>(acc, m, lsum, qf, sK[B], sV[B], st * BK, qpos0, Nk, g, l16);
        }
        wait_stage();
        __syncthreads();
    };
    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    const int nmain = min(min(nsteps, Nk / BK), CAUSAL ? (pos0 + qb * BQ + 1) / BK : nsteps);
    int st = 0;
    if (nmain > 0) main_stage(B0{}, std::true_type{}, st++);
    for (; st + 1 < nmain; st += 2) {
        main_stage(B1{}, std::false_type{}, st);
        main_stage(B0{}, std::false_type{}, st + 1);
    }
    if (st < nmain) main_stage(B1{}, std::false_type{}, st++);
    // the remaining stages may straddle the diagonal or the end of the keys:
    // one masked body each for the first stage and the later ones
    for (; st < nsteps; ++st) {
        const int cur = st & 1;
        if (st + 1 < nsteps) stage_kv<Pol>(sK[cur ^ 1], sV[cur ^ 1], K, V, (st + 1) * BK, Nk, plan, wave, p.kv_rs);
        const int k0 = st * BK;
        // a wave whose queries all precede the stage's keys has nothing to do
        if (!CAUSAL || k0 <= qpos0 + 31) {
            if (st == 0) {
                fwd_stage<Pol, CAUSAL, true>(acc, m, lsum, qf, sK[cur], sV[cur], k0, qpos0, Nk, g, l16);
            } else {
                fwd_stage_lazy<Pol, CAUSAL, true>(acc, m, lsum, qf, sK[cur], sV[cur], k0, qpos0, Nk, g, l16);
            }
        }
        wait_stage();
        __syncthreads();
    }

    T *O = static_cast<T *>(p.o) + b * p.o_bs + h * p.o_hs;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        const float ltot = xg_sum(lsum[qt]);
        const float inv = 1.0f / ltot;
        if (qi < N) {
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) store4<T>(O + (size_t)qi * p.o_rs + 16 * xt + 4 * g, acc[xt][qt], inv);
            if (p.lse != nullptr && g == 0) p.lse[(size_t)bh * N + qi] = (m[qt] + fast_log2(ltot)) * kLn2;
        }
    }
}

template <class Pol, bool CAUSAL>
static hipError_t launch_fwd_t(const Params &p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hq, (p.N + 127) / 128);
    constexpr int kHi = Pol::kWavesFwdCausal;
    if constexpr (CAUSAL && kHi > Pol::kWaves) {
        // enough causal work-groups to fill kHi per CU (256 CUs)
        if ((long long)grid.x * grid.y >= 256LL * kHi) {
            hipLaunchKernelGGL((fwd_kernel<Pol, CAUSAL, kHi>), grid, dim3(256), 0, stream, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((fwd_kernel<Pol, CAUSAL, Pol::kWaves>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_fwd(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream) {
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
