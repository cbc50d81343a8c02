// Flash-attention backward for gfx950 (FA-2 structure, recompute from LSE).
//
// Math (attention_bwd.cu:8-14): with p_ij = exp(s_ij * scale - L_i),
//   Delta_i = sum_x dO[i,x] O[i,x]
//   dP_ij   = dO_i . v_j
//   dS_ij   = p_ij (dP_ij - Delta_i)          (the softmax scale is applied once,
//   dV_j    = sum_i p_ij dO_i                  to dK and dQ, at the end)
//   dK_j    = scale * sum_i dS_ij q_i
//   dQ_i    = scale * sum_j dS_ij k_j
//
// Two atomic-free passes, as in attention_bwd.cu:96-243, re-tiled for CDNA4:
//   * dK/dV pass: a work-group owns 4 Tile::ROWS keys of one (batch, KV head);
//     each of its 4 waves owns Tile::ROWS keys whose K/V rows sit in registers
//     and whose dK/dV accumulate in registers. Q/dO/LSE/Delta stream through
//     double-buffered LDS (direct global->LDS loads issued one stage ahead),
//     64 queries per stage, for every query head of the KV head's group in
//     turn, so the grouped-query reduction of dK/dV happens inside the kernel
//     with no atomics and no extra memory.
//   * dQ pass: a work-group owns 4 Tile::ROWS queries of one (batch, query
//     head), Q/dO rows in registers; K/V stream through LDS 64 keys per stage.
//     It recomputes S and dP (the price of staying atomic-free and O(N) in
//     memory).
// The per-wave register state and arithmetic of each pass is a tile class
// (DqTile16, DkvTile16: 16x16 MFMA tiles, 32 rows per wave at d = 64).
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <chrono>
#include <cstring>
#include <random>
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

// ------------------------------------------------------------ preprocess

// Delta_i = sum_x dO[i][x] * O[i][x], 8 lanes per row (attention_bwd.cu:32-44).
template <class T, int D>
__device__ __forceinline__ void preprocess_body(const T *dout, const T *o, float *delta, long rows) {
    const long t = (long)blockIdx.x * 256 + threadIdx.x;
    const long row = t >> 3;
    const int part = (int)(t & 7);
    constexpr int PER = D / 8;  // elements per lane
    float acc = 0.f;
    if (row < rows) {
        const T *a = dout + row * D + part * PER;
        const T *b = o + row * D + part * PER;
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int i = 0; i < PER; i += 4) {
                const float4 x = *reinterpret_cast<const float4 *>(a + i);
                const float4 y = *reinterpret_cast<const float4 *>(b + i);
                acc += x.x * y.x;
                acc += x.y * y.y;
                acc += x.z * y.z;
                acc += x.w * y.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < PER; i += 8) {
                const uint4 x = *reinterpret_cast<const uint4 *>(a + i);
                const uint4 y = *reinterpret_cast<const uint4 *>(b + i);
                const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ys[4] = {y.x, y.y, y.z, y.w};
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    acc += __uint_as_float(xs[w] << 16) * __uint_as_float(ys[w] << 16);
                    acc += __uint_as_float(xs[w] & 0xffff0000u) * __uint_as_float(ys[w] & 0xffff0000u);
                }
            }
        }
    }
    acc += __shfl_xor(acc, 4, 8);
    acc += __shfl_xor(acc, 2, 8);
    acc += __shfl_xor(acc, 1, 8);
    if (row < rows && part == 0) delta[row] = acc;
}

// One dK/dV stage: the Pol::ROWS query rows from row `row` of Q and dO (row =
// bh N + qs: query qs of head bh; nvalid = N - qs of them exist), and their
// LSE and Delta, into LDS buffers.
// The buffers are given as LDS addresses.
template <class Pol, int NT = 256, bool STAGE_DELTA = true>
__device__ __forceinline__ void stage_qdo(uint32_t sq, uint32_t sdo, uint32_t sl, uint32_t sd, const Params &p,
                                          size_t row, int nvalid, const RowPlan<Pol, NT> &pl, int wave, int lane) {
    using T = typename Pol::T;
    const size_t off = row * Pol::D;
    stage_rows<Pol, NT>(sq, static_cast<const T *>(p.q) + off, nvalid, pl, wave);
    stage_rows<Pol, NT>(sdo, static_cast<const T *>(p.dout) + off, nvalid, pl, wave);
    // rows past N: LSE = +inf makes their p (and so dS) exactly 0
    if (wave == 0) stage_vec64(sl, p.lse + row, nvalid, lane, &kPosInf);
    if (STAGE_DELTA && wave == 1) stage_vec64(sd, p.delta + row, nvalid, lane, p.delta + row);
}

// Delta flags of the one-launch backward (see Params::epoch). Zero at load;
// launch epochs start at 1, so no flag matches before it is published. And,
// counted since the code object was loaded (read by name, see module.cpp):
// the stages whose Delta a dK/dV work-group of the one-launch backward
// computed itself (its wait ran out), and the reduce work-groups whose wait
// for their shares ran out (outputs NaN).
#if defined(__HIP_DEVICE_COMPILE__)
__device__ uint32_t g_delta_flags[kFlagSlots * kMaxFlagBlocks];
extern "C" __device__ unsigned long long mxfa_delta_fallbacks;
__device__ unsigned long long mxfa_delta_fallbacks;
extern "C" __device__ unsigned long long mxfa_reduce_timeouts;
__device__ unsigned long long mxfa_reduce_timeouts;
#else
extern __device__ uint32_t g_delta_flags[kFlagSlots * kMaxFlagBlocks];
extern "C" __device__ unsigned long long mxfa_delta_fallbacks;
extern "C" __device__ unsigned long long mxfa_reduce_timeouts;
#endif
constexpr int kFlagRows = 128;  // query rows per flag: one dQ work-group's block

// ---------------------------------------------------------------- wave tiles
//
// dQ tiles hold ROWS queries of one wave: Q and -dO (registers), the LSE
// offset and Delta of each query, and the dQ accumulators. load() fills them
// (DELTA: computing Delta = rowsum(dO * O) from O, which store_delta() writes
// to p.delta, write-through when PUBLISH), stage() runs one 64-key stage of K
// and V from LDS, store() writes dQ. delta_fallback() computes Delta of 64 rows on one
// wave with exactly the arithmetic of load(), so both give the same bits.
//
// dK/dV tiles hold ROWS keys of one wave: K and -V (registers) and the dK/dV
// accumulators; stage() runs one 64-query stage of Q, dO, LSE and Delta from
// LDS. Both accumulate dS / scale with the sign flipped (the dP accumulators
// start at Delta with the -V or -dO operand, so they come out as Delta - dP);
// store() multiplies by -scale. PRIO: the matrix products run at raised wave
// priority and the softmax part at normal priority (the one-launch backward,
// where dQ and dK/dV waves share each SIMD).

// 16x16 MFMA tiles (Pol = PolF32<64> or PolBF16<128>): lane l holds column
// l%16 and rows 4(l/16) + r of each 16x16 C tile. W2 (bf16 d = 64, the
// one-launch backward of small grids): compiled for two waves per SIMD, with
// the stages' LDS operands read ahead of their products (stage_batched).
template <class Pol_, int QT, bool W2 = false>
struct DqTile16 {
    using Pol = Pol_;
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    static constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    static constexpr int ROWS = 16 * QT;
    static constexpr int kWaves = W2 ? 2 : Pol::kWavesDq;
    static constexpr bool kPrioFused = D == 64;

    Frag qf[QT][NC], dof[QT][NC];
    float nL2[QT], Dl[QT];
    f32x4 acc[XT][QT];

    // Delta of the 16 d-element chunks the lane group g holds, (t0 + t2) +
    // (t1 + t3) over the groups (xg_sum)
    __device__ static __forceinline__ float group_part(const Frag (&a)[NC], const Frag (&b)[NC]) {
        float t = 0.f;
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) t += Pol::dot(a[kc], b[kc]);
        return t;
    }

    // The wave's rows: every load is issued first (branch-free), so they are
    // in flight together. DELTA: Delta = rowsum(dO * O) from O, which
    // store_delta() writes; otherwise Delta is read from p.delta.
    template <bool DELTA>
    __device__ __forceinline__ void load(const Params &p, int bh, int q0, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        const int N = p.N;
        const size_t hrow = (size_t)bh * N;
        const T *Q = static_cast<const T *>(p.q) + hrow * D;
        const T *dO = static_cast<const T *>(p.dout) + hrow * D;
        Frag of[DELTA ? QT : 1][NC];
        float lse[QT];
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qi = q0 + 16 * qt + l16, qc = min(qi, N - 1);
            Pol::gmem_row_frags(qf[qt], Q, qi, N, D, g);
            Pol::gmem_row_frags(dof[qt], dO, qi, N, D, g);
            if constexpr (DELTA) {
                Pol::gmem_row_frags(of[qt], static_cast<const T *>(p.o_in) + hrow * D, qi, N, D, g);
            } else {
                Dl[qt] = p.delta[hrow + qc];
            }
            lse[qt] = p.lse[hrow + qc];
        }
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const bool ok = q0 + 16 * qt + l16 < N;
            if constexpr (DELTA) {
                // the lane holds 16 of the row's d elements; the 4 lane groups
                // g = 0..3 together hold the row (rows past N: zeros, Delta 0)
                Dl[qt] = xg_sum(group_part(dof[qt], of[qt]));
            } else {
                Dl[qt] = ok ? Dl[qt] : 0.f;
            }
#pragma unroll
            for (int kc = 0; kc < NC; ++kc) {
                if (!Pol::kExactScale) qf[qt][kc] = Pol::scaled(qf[qt][kc], p.scale_log2);
                dof[qt][kc] = Pol::neg(dof[qt][kc]);
            }
            nL2[qt] = ok ? lse[qt] * (Pol::kExactScale ? -1.0f / p.scale : -kLog2e) : 0.f;
        }
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) acc[xt][qt] = zero4();
        }
    }

    // Writes the Delta rows load<true>() computed to p.delta; PUBLISH: written
    // through to memory.
    template <bool PUBLISH>
    __device__ __forceinline__ void store_delta(const Params &p, int bh, int q0, int lane) const {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qi = q0 + 16 * qt + l16;
            if (qi < p.N && g == 0) {
                float *dst = p.delta + (size_t)bh * p.N + qi;
                if constexpr (PUBLISH) {
                    store_wt(dst, __float_as_uint(Dl[qt]));
                } else {
                    *dst = Dl[qt];
                }
            }
        }
    }

    // Rows qs .. qs + 63 of head bh, lane r: row qs + r (0 past N).
    __device__ static __forceinline__ void delta_fallback(float *sd, const Params &p, size_t bh, int qs, int N,
                                                          int lane) {
        const int row = qs + lane;
        float acc = 0.f;
        if (row < N) {
            const size_t off = (bh * N + row) * D;
            const Frag *o = reinterpret_cast<const Frag *>(static_cast<const T *>(p.o_in) + off);
            const Frag *d = reinterpret_cast<const Frag *>(static_cast<const T *>(p.dout) + off);
            // group_part of each lane group g (t = 0, then t += dot in kc
            // order), one chunk pair at a time: this runs inside the dK/dV
            // loop, where the accumulators leave no room for the whole row
            float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < NC; ++kc) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    t[g] += Pol::dot(d[4 * kc + g], o[4 * kc + g]);
                    __builtin_amdgcn_sched_barrier(0);
                    asm volatile("" ::: "memory");
                }
            }
            acc = (t[0] + t[2]) + (t[1] + t[3]);
        }
        sd[lane] = acc;
    }

    // The score accumulators start at nL2, so they come out as the exponents
    // of P, times xmul where the policy keeps Q exact (Pol::kExactScale: qf
    // holds Q, nL2 is -L / scale, xmul = scale log2(e)); otherwise qf holds
    // Q scale log2(e) and nL2 is -L log2(e).
    template <bool CAUSAL, bool MASK, bool PRIO>
    __device__ __forceinline__ void stage(const T *sk, const T *sv, int k0, int q0, int N, int lane, float xmul) {
        if constexpr (kBatchedReads) {
            stage_batched<CAUSAL, MASK>(sk, sv, k0, q0, N, lane, xmul);
            return;
        }
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            f32x4 s[2][QT], dp[2][QT];  // [t][qt]
            wave_priority<PRIO>(1);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                Frag a[NC];
                const int n = 32 * blk + Pol::arow(t, l16);
                Pol::lds_row_frags(a, sk, n, g);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    f32x4 c = f32x4{nL2[qt], nL2[qt], nL2[qt], nL2[qt]};
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                    s[t][qt] = c;
                }
                Pol::lds_row_frags(a, sv, n, g);
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    f32x4 c = f32x4{Dl[qt], Dl[qt], Dl[qt], Dl[qt]};
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], dof[qt][kc], c);
                    dp[t][qt] = c;
                }
            }
            wave_priority<PRIO>(0);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int qi = q0 + 16 * qt + l16;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = s[t][qt][r];
                        if constexpr (MASK) {
                            const int key = k0 + 32 * blk + Pol::bidx(t, g, r);
                            x = (key >= N || (CAUSAL && key > qi)) ? -INFINITY : x;
                        }
                        const float pv = fast_exp2(Pol::kExactScale ? x * xmul : x);
                        s[t][qt][r] = pv * dp[t][qt][r];  // -dS / scale
                    }
                }
            }
            typename Pol::ChainB cb[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) cb[qt] = Pol::pack(s[0][qt], s[1][qt]);
            wave_priority<PRIO>(1);
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sk, 16 * xt, 32 * blk, g, l16);
                }
            }
            wave_priority<PRIO>(0);
        }
    }

    // The same stage with every LDS operand of a 32-key block read ahead of the
    // products that take it (W2: two waves per SIMD leave the registers for it;
    // as DkvTile16's stage_batched, the same arithmetic in the same order as
    // stage()).
    static constexpr bool kBatchedReads = W2;
    template <bool CAUSAL, bool MASK>
    __device__ __forceinline__ void stage_batched(const T *sk, const T *sv, int k0, int q0, int N, int lane,
                                                  float xmul) {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            Frag ak[2][NC], av[2][NC];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int n = 32 * blk + Pol::arow(t, l16);
                Pol::lds_row_frags(ak[t], sk, n, g);
                Pol::lds_row_frags(av[t], sv, n, g);
            }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 s[2][QT], dp[2][QT];  // [t][qt]
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    f32x4 c = f32x4{nL2[qt], nL2[qt], nL2[qt], nL2[qt]};
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(ak[t][kc], qf[qt][kc], c);
                    s[t][qt] = c;
                }
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) {
                    f32x4 c = f32x4{Dl[qt], Dl[qt], Dl[qt], Dl[qt]};
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(av[t][kc], dof[qt][kc], c);
                    dp[t][qt] = c;
                }
            }
            Frag ok[XT];
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) ok[xt] = Pol::chain_a(sk, 16 * xt, 32 * blk, g, l16);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) {
                const int qi = q0 + 16 * qt + l16;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float x = s[t][qt][r];
                        if constexpr (MASK) {
                            const int key = k0 + 32 * blk + Pol::bidx(t, g, r);
                            x = (key >= N || (CAUSAL && key > qi)) ? -INFINITY : x;
                        }
                        const float pv = fast_exp2(Pol::kExactScale ? x * xmul : x);
                        s[t][qt][r] = pv * dp[t][qt][r];  // -dS / scale
                    }
                }
            }
            typename Pol::ChainB cb[QT];
#pragma unroll
            for (int qt = 0; qt < QT; ++qt) cb[qt] = Pol::pack(s[0][qt], s[1][qt]);
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
                for (int qt = 0; qt < QT; ++qt) acc[xt][qt] = Pol::mma(ok[xt], cb[qt], acc[xt][qt]);
            }
        }
    }

    __device__ __forceinline__ void store(const Params &p, int bh, int q0, int lane) const {
        const int g = lane >> 4, l16 = lane & 15;
        const int N = p.N;
        T *dQ = static_cast<T *>(p.dq) + (size_t)bh * N * D;
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) {
            const int qi = q0 + 16 * qt + l16;
            if constexpr (std::is_same<T, u16>::value) {
                // bf16 rows, 16 bytes per lane
                const size_t row = (size_t)min(qi, N - 1) * D;
#pragma unroll
                for (int xt = 0; xt < XT; xt += 2)
                    store8_pair_bf16(dQ + row, 16 * xt, g, acc[xt][qt], acc[xt + 1][qt], -p.scale, qi < N);
            } else if (qi < N) {
#pragma unroll
                for (int xt = 0; xt < XT; ++xt)
                    store4<T>(dQ + (size_t)qi * D + 16 * xt + 4 * g, acc[xt][qt], -p.scale);
            }
        }
    }
};

// P2 (bf16, a softmax scale that is a power of two, as 1/sqrt(64) is): K is
// held as -K scale, which is exact, so the score accumulators start at L
// itself and come out as L - s scale; the exponent is that times -log2(e). This
// saves the per-block multiply of the staged LSE rows (16 VALU per stage at
// d = 64) and its wait before the first score MFMA.
template <class Pol_, int KT, bool P2 = false, bool W2 = false>
struct DkvTile16 {
    using Pol = Pol_;
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    static constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    static constexpr int ROWS = 16 * KT;
    static constexpr int kWaves = W2 ? 2 : Pol::kWavesDkv;
    static constexpr bool kPrioFused = D == 64;

    Frag kf[KT][NC], vf[KT][NC];
    f32x4 accK[XT][KT], accV[XT][KT];
    float lmul, xmul;

    // The score accumulators' start for 4 query rows from their staged LSE.
    __device__ __forceinline__ f32x4 nl_of(const float *l) const {
        if constexpr (P2) return *reinterpret_cast<const f32x4 *>(l);
        return *reinterpret_cast<const f32x4 *>(l) * lmul;
    }

    // K and V rows under a branch per row (gmem_row_frags_if): the branch-free
    // form issues the loads together, but measured no faster here (they
    // overlap the first stage's loads either way) and made the register
    // allocator spill inside the two-launch dK/dV kernel's stage loops
    __device__ __forceinline__ void load(const Params &p, const T *K, const T *V, int kw0, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
        const int N = p.N;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const int key = kw0 + 16 * kt + l16;
            Pol::gmem_row_frags_if(kf[kt], K + (size_t)key * D, g, key < N);
            Pol::gmem_row_frags_if(vf[kt], V + (size_t)key * D, g, key < N);
#pragma unroll
            for (int kc = 0; kc < NC; ++kc) {
                if constexpr (P2) {
                    kf[kt][kc] = Pol::scaled(kf[kt][kc], -p.scale);
                } else if constexpr (!Pol::kExactScale) {
                    kf[kt][kc] = Pol::scaled(kf[kt][kc], p.scale_log2);
                }
                vf[kt][kc] = Pol::neg(vf[kt][kc]);
            }
        }
        lmul = Pol::kExactScale ? -1.0f / p.scale : -kLog2e;
        xmul = P2 ? -kLog2e : p.scale_log2;
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) accK[xt][kt] = accV[xt][kt] = zero4();
        }
    }

    // The score accumulators start at L lmul, so they come out as the
    // exponents of P, times xmul where the policy keeps K exact
    // (Pol::kExactScale: kf holds K, lmul = -1 / scale, xmul = scale
    // log2(e)); otherwise kf holds K scale log2(e) and lmul = -log2(e). With
    // P2 they start at L and kf holds -K scale, xmul = -log2(e).
    template <bool CAUSAL, bool MASK, bool PRIO>
    __device__ __forceinline__ void stage(const T *sq, const T *sdo, const float *sl, const float *sd, int qs, int kw0,
                                          int lane) {
        if constexpr (kBatchedReads) {
            stage_batched<CAUSAL, MASK>(sq, sdo, sl, sd, qs, kw0, lane);
            return;
        }
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            f32x4 s[2][KT], dp[2][KT];  // [t][kt]
            wave_priority<PRIO>(1);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                // block rows bidx(t, g, 0..3) are consecutive: one 16-byte LDS read
                const int q4 = 32 * blk + Pol::bidx(t, g, 0);
                const f32x4 nl = nl_of(sl + q4);
                const f32x4 dl = *reinterpret_cast<const f32x4 *>(sd + q4);
                Frag a[NC];
                const int n = 32 * blk + Pol::arow(t, l16);
                Pol::lds_row_frags(a, sq, n, g);
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    f32x4 c = nl;
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], kf[kt][kc], c);
                    s[t][kt] = c;
                }
                Pol::lds_row_frags(a, sdo, n, g);
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    f32x4 c = dl;
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], vf[kt][kc], c);
                    dp[t][kt] = c;
                }
            }
            wave_priority<PRIO>(0);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int kt = 0; kt < KT; ++kt) {
                        float x = Pol::kExactScale || P2 ? s[t][kt][r] * xmul : s[t][kt][r];
                        if constexpr (MASK) {
                            // causal: query qs + 32 blk + bidx(t, g, r) before key kw0 + 16 kt + l16
                            const bool before = Pol::bidx(t, g, r) - l16 < kw0 - qs + 16 * kt - 32 * blk;
                            x = before ? -INFINITY : x;
                        }
                        const float pv = fast_exp2(x);
                        s[t][kt][r] = pv;
                        dp[t][kt][r] = pv * dp[t][kt][r];  // -dS / scale
                    }
                }
            }
            typename Pol::ChainB cp[KT], cds[KT];
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                cp[kt] = Pol::pack(s[0][kt], s[1][kt]);
                cds[kt] = Pol::pack(dp[0][kt], dp[1][kt]);
            }
            wave_priority<PRIO>(1);
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    accV[xt][kt] = Pol::chain(accV[xt][kt], cp[kt], sdo, 16 * xt, 32 * blk, g, l16);
                    accK[xt][kt] = Pol::chain(accK[xt][kt], cds[kt], sq, 16 * xt, 32 * blk, g, l16);
                }
            }
            wave_priority<PRIO>(0);
        }
    }

    // The same stage with every LDS operand of a 32-query block read ahead of the
    // products that take it (kBatchedReads: d = 128, one key tile per wave at
    // two waves per SIMD, where the default order reads each operand one or two
    // MFMAs before its use and the wave then waits out the LDS latency; and the
    // two-wave W2 tiles at d = 64, which have the registers for it): all the
    // score and dP operands first, then the products; the chained products'
    // operands right after those, so they arrive while the softmax runs. The
    // scheduling barriers keep the compiler from sinking the reads back to
    // their uses. The arithmetic and its order are those of stage().
    static constexpr bool kBatchedReads = (D == 128 && KT == 1) || W2;
    template <bool CAUSAL, bool MASK>
    __device__ __forceinline__ void stage_batched(const T *sq, const T *sdo, const float *sl, const float *sd, int qs,
                                                  int kw0, int lane) {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int blk = 0; blk < 2; ++blk) {
            Frag aq[2][NC], ad[2][NC];
            f32x4 nl[2], dl[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int q4 = 32 * blk + Pol::bidx(t, g, 0);
                nl[t] = nl_of(sl + q4);
                dl[t] = *reinterpret_cast<const f32x4 *>(sd + q4);
                const int n = 32 * blk + Pol::arow(t, l16);
                Pol::lds_row_frags(aq[t], sq, n, g);
                Pol::lds_row_frags(ad[t], sdo, n, g);
            }
            __builtin_amdgcn_sched_barrier(0);
            f32x4 s[2][KT], dp[2][KT];  // [t][kt]
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    f32x4 c = nl[t];
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(aq[t][kc], kf[kt][kc], c);
                    s[t][kt] = c;
                }
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    f32x4 c = dl[t];
#pragma unroll
                    for (int kc = 0; kc < NC; ++kc) c = Pol::mma(ad[t][kc], vf[kt][kc], c);
                    dp[t][kt] = c;
                }
            }
            Frag ov[XT], ok[XT];
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
                ov[xt] = Pol::chain_a(sdo, 16 * xt, 32 * blk, g, l16);
                ok[xt] = Pol::chain_a(sq, 16 * xt, 32 * blk, g, l16);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
#pragma unroll
                    for (int kt = 0; kt < KT; ++kt) {
                        float x = Pol::kExactScale || P2 ? s[t][kt][r] * xmul : s[t][kt][r];
                        if constexpr (MASK) {
                            const bool before = Pol::bidx(t, g, r) - l16 < kw0 - qs + 16 * kt - 32 * blk;
                            x = before ? -INFINITY : x;
                        }
                        const float pv = fast_exp2(x);
                        s[t][kt][r] = pv;
                        dp[t][kt][r] = pv * dp[t][kt][r];  // -dS / scale
                    }
                }
            }
            typename Pol::ChainB cp[KT], cds[KT];
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                cp[kt] = Pol::pack(s[0][kt], s[1][kt]);
                cds[kt] = Pol::pack(dp[0][kt], dp[1][kt]);
            }
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    accV[xt][kt] = Pol::mma(ov[xt], cp[kt], accV[xt][kt]);
                    accK[xt][kt] = Pol::mma(ok[xt], cds[kt], accK[xt][kt]);
                }
            }
        }
    }

    // Scaled dK and dV (dst = K-shaped outputs of type T), or with SPLIT the
    // unscaled fp32 partial sums (dst = the share's workspace planes).
    template <class U, bool WT = false>
    __device__ __forceinline__ void store(U *dK, U *dV, int kw0, int N, float kmul, int lane) const {
        const int g = lane >> 4, l16 = lane & 15;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const int key = kw0 + 16 * kt + l16;
            if constexpr (std::is_same<U, u16>::value) {
                // bf16 rows, 16 bytes per lane
                const size_t row = (size_t)min(key, N - 1) * D;
#pragma unroll
                for (int xt = 0; xt < XT; xt += 2) {
                    store8_pair_bf16(dK + row, 16 * xt, g, accK[xt][kt], accK[xt + 1][kt], kmul, key < N);
                    store8_pair_bf16(dV + row, 16 * xt, g, accV[xt][kt], accV[xt + 1][kt], 1.0f, key < N);
                }
            } else if (key < N) {
#pragma unroll
                for (int xt = 0; xt < XT; ++xt) {
                    if constexpr (WT) {  // partial sums (kmul = 1) for a reduce in the same launch
                        // from the wave's first key row (a wave-uniform base), within its rows
                        const uint32_t bytes = (uint32_t)(min(ROWS, N - kw0) * D * 4);
                        const uint32_t off = (uint32_t)(((key - kw0) * D + 16 * xt + 4 * g) * 4);
                        store4_wt(reinterpret_cast<float *>(dK + (size_t)kw0 * D), bytes, off, accK[xt][kt]);
                        store4_wt(reinterpret_cast<float *>(dV + (size_t)kw0 * D), bytes, off, accV[xt][kt]);
                    } else {
                        store4<U>(dK + (size_t)key * D + 16 * xt + 4 * g, accK[xt][kt], kmul);
                        store4<U>(dV + (size_t)key * D + 16 * xt + 4 * g, accV[xt][kt], 1.0f);
                    }
                }
            }
        }
    }
};

// ------------------------------------------------------------------ dQ pass

// LDS of a dQ work-group: double-buffered K and V tiles.
template <class Pol>
struct DqSmem {
    __attribute__((aligned(16))) typename Pol::T sK[2][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) typename Pol::T sV[2][Pol::ROWS * Pol::D];
};

// The dQ work of query block qb (4 Tile::ROWS rows) of (batch, query head) bh.
// DELTA: compute Delta_i = sum_x dO[i,x] O[i,x] here (O from p.o_in) and write
// it to p.delta for the dK/dV pass, instead of reading it from there.
// PUBLISH (with DELTA, in the one-launch backward): Delta is written through
// to memory once the first stage is staged, and the block's flag set to
// p.epoch after the first stage, whose wait sees those stores acknowledged.
template <class Tile, bool CAUSAL, bool DELTA, bool PUBLISH = false>
__device__ __forceinline__ void dq_body(const Params &p, int bh, int qb, DqSmem<typename Tile::Pol> &sm) {
    using Pol = typename Tile::Pol;
    constexpr int NW = 4;
    constexpr int BQ = Tile::ROWS * NW, BK = Pol::ROWS, NT = 64 * NW;
    static_assert(BQ % BK == 0, "causal: the masked tail is the work-group's BQ / BK diagonal stages");
    constexpr bool kPrio = PUBLISH && Tile::kPrioFused;
    using T = typename Pol::T;
    auto &sK = sm.sK;
    auto &sV = sm.sV;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int N = p.N;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const size_t kvoff = ((size_t)b * p.Hkv + kvh) * N * Pol::D;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int q0 = qb * BQ + wave * Tile::ROWS;
    wg_time(0);

    // the first stage's K/V loads and the tile's loads are in flight together
    const RowPlan<Pol, NT> plan(tid);
    stage_kv<Pol, NT>(sK[0], sV[0], K, V, 0, N, plan, wave);
    Tile t;
    t.template load<DELTA>(p, bh, q0, lane);
    if constexpr (DELTA && !PUBLISH) t.template store_delta<false>(p, bh, q0, lane);

    const int kend = CAUSAL ? min(N, qb * BQ + BQ) : N;
    const int nsteps = (kend + BK - 1) / BK;
    wg_info(0, qb, nsteps);

    wait_stage();
    __syncthreads();
    wg_time(1);
    // PUBLISH: the Delta stores go out now, and stage 0's wait (every wave's
    // s_waitcnt, then the barrier) sees them acknowledged before thread 0 sets
    // the flag; so no wave waits for a write-through on its own
    static_assert(!PUBLISH || (DELTA && BQ == kFlagRows), "a published block is one work-group's Delta rows");
    if constexpr (PUBLISH) t.template store_delta<true>(p, bh, q0, lane);
    auto publish = [&](int st) __attribute__((always_inline)) {
        if constexpr (PUBLISH) {
            if (st == 0 && tid == 0) {
                const int nfb = (N + kFlagRows - 1) / kFlagRows;
                store_wt(g_delta_flags + (size_t)p.flag_slot * kMaxFlagBlocks + (size_t)bh * nfb + qb, p.epoch);
            }
        }
    };

    // Every stage but the last kTail is unmasked for every wave (causal: its
    // keys all precede the workgroup's first query; otherwise: only the last
    // stage can be ragged). Those run in pairs with the LDS buffer a
    // compile-time constant, so the tile addresses fold into the instructions'
    // immediate offsets; the last kTail stages choose their buffer and masking
    // at run time.
    auto main_stage = [&](auto buf, int st) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < nsteps) stage_kv<Pol, NT>(sK[B ^ 1], sV[B ^ 1], K, V, (st + 1) * BK, N, plan, wave);
        t.template stage<CAUSAL, false, kPrio>(sK[B], sV[B], st * BK, q0, N, lane, p.scale_log2);
        wait_stage();
        __syncthreads();
        publish(st);
    };
    constexpr int kTail = BQ / BK > 2 ? BQ / BK : 2;
    const int nmain = nsteps - min(nsteps, kTail);
    int st = 0;
    for (; st + 1 < nmain; st += 2) {
        main_stage(std::integral_constant<int, 0>{}, st);
        main_stage(std::integral_constant<int, 1>{}, st + 1);
    }
    if (st < nmain) main_stage(std::integral_constant<int, 0>{}, st++);
    for (; st < nsteps; ++st) {
        const int cur = st & 1;
        if (st + 1 < nsteps) stage_kv<Pol, NT>(sK[cur ^ 1], sV[cur ^ 1], K, V, (st + 1) * BK, N, plan, wave);
        const int k0 = st * BK;
        // one (masked) body for these stages: a second, unmasked body behind a
        // branch makes the register allocator spill at three waves per SIMD
        if (!CAUSAL || k0 <= q0 + Tile::ROWS - 1) {
            t.template stage<CAUSAL, true, kPrio>(sK[cur], sV[cur], k0, q0, N, lane, p.scale_log2);
        }
        wait_stage();
        __syncthreads();
        publish(st);
    }
    wg_time(2);
    t.store(p, bh, q0, lane);
    wg_time_after_stores();
}

// The dQ pass as its own launch, grid (B Hq, query blocks). Causal: query
// blocks from the last (the most keys) to the first.
template <class Tile, bool CAUSAL, bool DELTA>
__device__ __forceinline__ void dq_entry(const Params &p) {
    __shared__ DqSmem<typename Tile::Pol> sm;
    const int nqb = (p.N + 4 * Tile::ROWS - 1) / (4 * Tile::ROWS);
    const int i = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    const int rank = CAUSAL ? cu_order_wg(i, p.cu_run, p.cu_runs) : i;  // heaviest first, balanced per CU
    const int qb = CAUSAL ? nqb - 1 - rank / (int)gridDim.x : rank / (int)gridDim.x;
    dq_body<Tile, CAUSAL, DELTA>(p, rank % (int)gridDim.x, qb, sm);
}

// ---------------------------------------------------------------- dK/dV pass

// LDS of a dK/dV work-group: double-buffered Q / dO tiles and their LSE /
// Delta rows (loads are issued one stage ahead).
template <class Pol>
struct DkvSmem {
    static constexpr int NBUF = 2;
    __attribute__((aligned(16))) typename Pol::T sQ[NBUF][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) typename Pol::T sdO[NBUF][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) float sL[NBUF][Pol::ROWS];
    __attribute__((aligned(16))) float sD[NBUF][Pol::ROWS];
    uint32_t sF[2];  // one-launch backward: the flags of the next stages' Delta blocks
};

// The dK/dV work wk (dkv_work): key block wk.kb (4 Tile::ROWS keys) of
// (batch, KV head) wk.bkv, share wk.sp of wk.ns, i.e. the share's run of the
// group's query heads' stages (head-major, each head's from the diagonal).
// WAIT (one-launch backward): Delta comes from the dQ work-groups of the same
// launch; wave 1 stages a stage's Delta rows only once their block's flag
// reads p.epoch (see issue below), else computes them as DqTile does.
template <class Tile, bool CAUSAL, bool WAIT = false, class DqTile = void>
__device__ __forceinline__ void dkv_body(const Params &p, const DkvWork wk, DkvSmem<typename Tile::Pol> &sm) {
    using Pol = typename Tile::Pol;
    using T = typename Pol::T;
    constexpr int D = Pol::D;
    constexpr int NW = 4, NT = 64 * NW;  // threads per workgroup
    constexpr int BKV = Tile::ROWS * NW;  // keys per workgroup
    constexpr int BQ = Pol::ROWS;          // queries per stage
    static_assert(BKV % BQ == 0, "causal start must align to a stage");
    constexpr bool kPrio = WAIT && Tile::kPrioFused;
    constexpr int NBUF = DkvSmem<Pol>::NBUF;
    auto &sQ = sm.sQ;
    auto &sdO = sm.sdO;
    auto &sL = sm.sL;
    auto &sD = sm.sD;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int N = p.N;
    const int kb = wk.kb, bkv = wk.bkv;  // bkv = b * Hkv + kvh
    const int b = bkv / p.Hkv, kvh = bkv % p.Hkv;
    const size_t kvoff = (size_t)bkv * N * D;
    const int kw0 = kb * BKV + wave * Tile::ROWS;  // first key of this wave
    wg_time(0);

    const int qstart = CAUSAL ? kb * BKV : 0;
    const int nqs = (N - qstart + BQ - 1) / BQ;  // stages per query head
    // the share's stages [g0, g0 + nsteps) of the group's p.group * nqs
    int g0 = 0, nsteps = p.group * nqs;
    if (wk.ns > 1) {
        g0 = (int)((long long)wk.sp * nsteps / wk.ns);
        nsteps = (int)((long long)(wk.sp + 1) * nsteps / wk.ns) - g0;
    }
    const size_t bh0 = (size_t)b * p.Hq + (size_t)kvh * p.group;  // the group's first query head
    wg_info(1, kb, nsteps);

    // Stages are loaded strictly in order. The next one's query head ld_bh,
    // its place ld_i in that head, its first query ld_qs and row ld_row =
    // ld_bh N + ld_qs, and the head's first Delta flag ld_fb = ld_bh nfb are
    // kept incrementally (wave-uniform, so in scalar registers): a stage then
    // costs a few scalar adds, not the products of the full index.
    const RowPlan<Pol, NT> plan(tid);
    int ld_i = 0;
    if (g0 > 0) ld_i = g0 - (g0 / nqs) * nqs;
    const int i_first = ld_i;  // the first stage's place in its query head
    // WAIT: the flag of each stage's Delta block is fetched into sm.sF one
    // issue ahead, with a load that misses the caches (as are the Delta rows
    // themselves: the dQ work-group that wrote them may sit on another XCD).
    // It is checked before the Delta rows are staged; a flag not yet set is
    // polled for at most p.delta_wait ticks of the real-time counter, and then
    // the wave computes the rows itself, in the dQ tile's order (the same
    // bits), and counts the event in mxfa_delta_fallbacks. The first stage,
    // with nothing fetched ahead, is polled directly.
    const int nfb = (N + kFlagRows - 1) / kFlagRows;
    const uint32_t *flags = g_delta_flags + (size_t)p.flag_slot * kMaxFlagBlocks;
    size_t ld_bh = bh0 + (size_t)(g0 / nqs);
    int ld_qs = qstart + ld_i * BQ;
    size_t ld_row = ld_bh * N + ld_qs;
    size_t ld_fb = ld_bh * nfb;
    // the buffers' LDS addresses (buffer bf: the first's plus bf times a buffer)
    const uint32_t lds_q = lds_addr(&sQ[0][0]), lds_do = lds_addr(&sdO[0][0]);
    const uint32_t lds_l = lds_addr(&sL[0][0]), lds_d = lds_addr(&sD[0][0]), lds_f = lds_addr(&sm.sF[0]);
    auto issue = [&](int st) __attribute__((always_inline)) {
        const int bf = (int)((unsigned)st % NBUF);
        const size_t bh = ld_bh, row = ld_row, fb = ld_fb;
        const int qs = ld_qs;
        const uint32_t ld_sd = lds_d + bf * (uint32_t)sizeof(sD[0]);
        stage_qdo<Pol, NT, !WAIT>(lds_q + bf * (uint32_t)sizeof(sQ[0]), lds_do + bf * (uint32_t)sizeof(sdO[0]),
                                  lds_l + bf * (uint32_t)sizeof(sL[0]), ld_sd, p, row, N - qs, plan, wave, lane);
        ld_qs += BQ;
        ld_row += BQ;
        if (++ld_i == nqs) {  // the next query head's first stage
            ld_i = 0;
            ld_qs = qstart;
            ld_row = row + (size_t)(N - qs) + (size_t)qstart;
            ++ld_bh;
            ld_fb += nfb;
        }
        if constexpr (WAIT) {
            if (wave == 1) {
                const uint32_t *f = flags + fb + (uint32_t)qs / kFlagRows;
                // delta_wait < 0 trusts no flag (every stage takes the fallback)
                bool ready = p.delta_wait >= 0 && st > 0 && sm.sF[st & 1] == p.epoch;
                if (!ready && p.delta_wait >= 0) {
                    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                    for (;;) {
                        ready = __builtin_amdgcn_readfirstlane(load_uc_sync(f)) == p.epoch;
                        if (ready || __builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)p.delta_wait) break;
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                if (ready) {
                    lds_dma4_uc(ld_sd, p.delta + row + min(lane, N - 1 - qs));
                } else {
                    DqTile::delta_fallback(sD[bf], p, bh, qs, N, lane);
                    if (lane == 0) atomicAdd(&mxfa_delta_fallbacks, 1ull);
                }
            }
            // the next stage's flag; one lane: the DMA writes each active
            // lane's dword at base + 4 lane
            if (wave == 1 && st + 1 < nsteps && lane == 0) {
                lds_dma4_uc(lds_f + ((st + 1) & 1) * 4u, flags + ld_fb + (uint32_t)ld_qs / kFlagRows);
            }
        }
    };
    // the first stage's loads (and its flag poll) go out before the tile's
    // own, so both are in flight together
    if (nsteps > 0) issue(0);
    Tile t;
    t.load(p, static_cast<const T *>(p.k) + kvoff, static_cast<const T *>(p.v) + kvoff, kw0, lane);
    wait_stage();
    __syncthreads();
    wg_time(1);

    // One stage: prefetch stage st + 1, compute stage st, then wait for stage
    // st + 1 and barrier. Causal: the stages that straddle the diagonal are
    // the first BKV / BQ of each query head (queries from kb * BKV); they run
    // in a loop of their own with the masked body, so neither loop carries the
    // other's code (two bodies behind one branch make the register allocator
    // spill).
    auto run = [&](int st, int i) __attribute__((always_inline)) {
        const int cur = (int)((unsigned)st % NBUF);
        if (st + 1 < nsteps) issue(st + 1);
        const int qs = qstart + i * BQ;
        // a wave whose keys all follow the stage's queries has nothing to do
        if (qs + BQ - 1 >= kw0) {
            t.template stage<CAUSAL, true, kPrio>(sQ[cur], sdO[cur], sL[cur], sD[cur], qs, kw0, lane);
        }
        wait_stage();
        barrier_lds();
    };
    // The unmasked stages with the LDS buffer a compile-time constant, so the
    // tile addresses fold into the instructions' immediate offsets. No wave
    // skips them: their queries follow all the workgroup's keys.
    auto run_fixed = [&](auto buf, int st, int i) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < nsteps) issue(st + 1);
        const int qs = qstart + i * BQ;
        t.template stage<CAUSAL, false, kPrio>(sQ[B], sdO[B], sL[B], sD[B], qs, kw0, lane);
        wait_stage();
        barrier_lds();
    };
    using Buf0 = std::integral_constant<int, 0>;
    using Buf1 = std::integral_constant<int, 1>;
    // rows past N get p = 0 from LSE = +inf, so only the causal diagonal masks
    // each query head of the share's run: stages [i, iend) of its nqs
    const int ndiag = CAUSAL ? min(nqs, BKV / BQ) : 0;
    for (int st = 0, i = i_first; st < nsteps; i = 0) {
        const int iend = min(nqs, i + (nsteps - st));
        // the diagonal stages (at most BKV / BQ: a loop of known length)
        const int dend = min(ndiag, iend);
#pragma unroll
        for (int j = 0; j < BKV / BQ; ++j) {
            if (i < dend) run(st++, i++);
        }
        if (i < iend && (st & 1)) run_fixed(Buf1{}, st++, i++);
        for (; i + 1 < iend; i += 2, st += 2) {
            run_fixed(Buf0{}, st, i);
            run_fixed(Buf1{}, st + 1, i + 1);
        }
        if (i < iend) run_fixed(Buf0{}, st++, i);
    }

    wg_time(2);
    if (p.dkv_split > 1) {
        // this share's fp32 partial sums (unscaled); dkv_reduce_body adds the
        // block's shares and applies the scale
        const size_t plane = (size_t)p.B * p.Hkv * N * D;
        float *wK = p.dkv_ws + (size_t)wk.sp * plane + kvoff;
        if (WAIT && p.red_rows > 0) {
            t.template store<float, true>(wK, wK + (size_t)p.dkv_split * plane, kw0, N, 1.0f, lane);
        } else {
            t.store(wK, wK + (size_t)p.dkv_split * plane, kw0, N, 1.0f, lane);
        }
    } else {
        t.store(static_cast<T *>(p.dk) + kvoff, static_cast<T *>(p.dv) + kvoff, kw0, N, -p.scale, lane);
    }
    wg_time_after_stores();
}

// The dK/dV pass as its own launch, a 1-D grid of dkv_work's work-groups.
// Causal: key block 0 (the most queries) is dispatched first.
template <class Tile, bool CAUSAL>
__device__ __forceinline__ void dkv_entry(const Params &p) {
    __shared__ DkvSmem<typename Tile::Pol> sm;
    const DkvWork wk = dkv_work(p, blockIdx.x, 4 * Tile::ROWS, Tile::Pol::ROWS, CAUSAL);
    if (wk.kb * 4 * Tile::ROWS >= p.N) return;
    dkv_body<Tile, CAUSAL>(p, wk, sm);
}

// The whole backward from O in one launch (bf16): work-groups [0, fused_ndq)
// run the dQ pass with Delta, query blocks in increasing order (so Delta
// appears in the order the dK/dV work-groups consume it: each walks its query
// rows upward from its diagonal), and publish Delta per block; the rest run
// the dK/dV pass, key block 0 first, and wait for the blocks they stage. The
// dQ work-groups have lower indices, so they are dispatched first and never
// wait; every wait of a dK/dV work-group is bounded in time
// (Params::delta_wait). This removes one kernel boundary per backward.
template <class Pol>
union FusedSmem {
    DqSmem<Pol> dq;
    DkvSmem<Pol> dkv;
};

// The reduce of a GQA split inside the one-launch backward: work-group r adds
// the shares' planes for red_rows = 16 keys of one key block (d / 64 float4s
// of each plane per thread), in share order, as dkv_reduce_body does. Work-
// groups go key block 0 first (the shares' order), then (batch, KV head),
// then the block's chunk of rows. The shares have lower indices, so each is
// dispatched before any reduce work-group and waits for nothing it runs; the
// wait is bounded all the same (Params::red_wait), after which the outputs
// are NaN and mxfa_reduce_timeouts counts the work-group.
template <class Tile, bool CAUSAL>
__device__ __forceinline__ void dkv_reduce_rows(const Params &p, int r, uint32_t *s_ok) {
    using T = typename Tile::Pol::T;
    constexpr int D = Tile::D, BKV = 4 * Tile::ROWS, BQ = Tile::Pol::ROWS;
    constexpr int RR = 16, NCH = BKV / RR, V = RR * D / 1024;  // V: float4s per thread per plane
    static_assert(BKV % RR == 0 && V * 1024 == RR * D, "a key block is whole chunks of whole float4 rows");
    const int N = p.N, nbkv = p.B * p.Hkv;
    const int c = r % NCH, bkv = (r / NCH) % nbkv, kb = r / (NCH * nbkv);
    const int key0 = kb * BKV + c * RR;
    if (key0 >= N) return;
    wg_time(0);
    // the block's shares are dkv_work indices [w0, w0 + ns)
    const int w0 = dkv_first_work(p, bkv, kb, BKV, BQ, CAUSAL);
    const int ns = dkv_block_shares(p, (N - (CAUSAL ? kb * BKV : 0) + BQ - 1) / BQ);
    wg_info(3, kb, ns);
    const int tid = threadIdx.x;
    if (tid < 64) {
        const unsigned long long *flags = p.share_flags + w0;
        bool ok = true;
        for (int s0 = 0; s0 < ns && ok; s0 += 64) {
            const int s = s0 + tid;
            const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (;;) {
                const bool ready = s >= ns || load2_uc_sync(flags + s) == p.share_nonce;
                if (__builtin_amdgcn_ballot_w64(!ready) == 0) break;
                if (__builtin_amdgcn_s_memrealtime() - t0 > (uint64_t)p.red_wait) {
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(2);
            }
        }
        if (tid == 0) {
            *s_ok = ok ? 1u : 0u;
            if (!ok) atomicAdd(&mxfa_reduce_timeouts, 1ull);
        }
    }
    __syncthreads();
    wg_time(1);
    const bool ok = *s_ok != 0;
    const size_t plane = (size_t)p.B * p.Hkv * N * D;
    const size_t off = ((size_t)bkv * N + key0) * D;  // the chunk's first element
    const uint32_t bytes = (uint32_t)(min(RR, N - key0) * D * 4);
    const float *wk = p.dkv_ws + off, *wv = p.dkv_ws + (size_t)p.dkv_split * plane + off;
    f32x4 ak[V], av[V];
#pragma unroll
    for (int v = 0; v < V; ++v) {
        ak[v] = load4_uc(wk, bytes, 16u * (tid + 256 * v));
        av[v] = load4_uc(wv, bytes, 16u * (tid + 256 * v));
    }
    for (int s0 = 1; s0 < ns; s0 += 8) {
        f32x4 xk[8][V], xv[8][V];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < ns) {
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    xk[j][v] = load4_uc(wk + (size_t)(s0 + j) * plane, bytes, 16u * (tid + 256 * v));
                    xv[j][v] = load4_uc(wv + (size_t)(s0 + j) * plane, bytes, 16u * (tid + 256 * v));
                }
            }
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < ns) {
#pragma unroll
                for (int v = 0; v < V; ++v) {
                    ak[v] += xk[j][v];
                    av[v] += xv[j][v];
                }
            }
        }
    }
    wg_time(2);
#pragma unroll
    for (int v = 0; v < V; ++v) {
        if (!ok) ak[v] = av[v] = f32x4{NAN, NAN, NAN, NAN};
        const uint32_t i4 = tid + 256 * v;  // the chunk's float4 index
        if (16u * i4 < bytes) {
            store4<T>(static_cast<T *>(p.dk) + off + 4 * i4, ak[v], -p.scale);
            store4<T>(static_cast<T *>(p.dv) + off + 4 * i4, av[v], 1.0f);
        }
    }
    wg_time_after_stores();
}

template <class DqT, class DkvT, bool CAUSAL>
__device__ __forceinline__ void bwd_fused_entry(const Params &p) {
    static_assert(std::is_same<typename DqT::Pol, typename DkvT::Pol>::value, "one LDS layout");
    __shared__ FusedSmem<typename DqT::Pol> sm;
    const int bid = blockIdx.x;
    if (bid < p.fused_ndq) {
        const int nbh = p.B * p.Hq;
        dq_body<DqT, CAUSAL, true, true>(p, bid % nbh, bid / nbh, sm.dq);
    } else if (bid < p.fused_ndq + p.fused_ndkv) {
        const int w = bid - p.fused_ndq;
        const DkvWork wk = dkv_work(p, w, 4 * DkvT::ROWS, DkvT::Pol::ROWS, CAUSAL);
        if (wk.kb * 4 * DkvT::ROWS >= p.N) return;
        dkv_body<DkvT, CAUSAL, true, DqT>(p, wk, sm.dkv);
        if (p.red_rows > 0) {
            // the share's planes are in memory once every wave's stores are
            // acknowledged: then its flag
            wait_stores();
            __syncthreads();
            if (threadIdx.x == 0) store2_wt(p.share_flags + w, p.share_nonce);
        }
    } else {
        dkv_reduce_rows<DkvT, CAUSAL>(p, bid - p.fused_ndq - p.fused_ndkv, &sm.dkv.sF[0]);
    }
}

// dK / dV of a split dK/dV pass: for each key row, the sum of its key block's
// shares' fp32 partial planes in share order (so the result is
// deterministic), times -scale for dK. n4 = float4 groups per plane
// ([B Hkv][N][d]), d4 = d / 4; keys in blocks of bkv_rows, queries in stages
// of bq; the dV planes follow the dK planes.
template <class T>
__device__ __forceinline__ void dkv_reduce_body(const Params &p, unsigned n4, int d4, int bkv_rows, int bq,
                                                int causal) {
    const f32x4 *w = reinterpret_cast<const f32x4 *>(p.dkv_ws);
    T *dk = static_cast<T *>(p.dk), *dv = static_cast<T *>(p.dv);
    const unsigned stride = gridDim.x * 256u;
    for (unsigned i = blockIdx.x * 256u + threadIdx.x; i < 2 * n4; i += stride) {
        const bool isv = i >= n4;
        const unsigned j = isv ? i - n4 : i;
        const int kb = (int)((j / (unsigned)d4) % (unsigned)p.N) / bkv_rows;
        const int ns = dkv_block_shares(p, (p.N - (causal ? kb * bkv_rows : 0) + bq - 1) / bq);
        const f32x4 *src = w + (isv ? (size_t)p.dkv_split * n4 : 0) + j;
        f32x4 a = src[0];
        for (int s = 1; s < ns; ++s) a += src[(size_t)s * n4];
        if (isv) {
            store4<T>(dv + 4 * (size_t)j, a, 1.0f);
        } else {
            store4<T>(dk + 4 * (size_t)j, a, -p.scale);
        }
    }
}

// ------------------------------------------------------------------ kernels

// The tiles of each dtype / head dim.
using DqB64 = DqTile16<PolBF16<64>, PolBF16<64>::kDqTiles>;
using DkvB64 = DkvTile16<PolBF16<64>, 2>;
using DkvB64P2 = DkvTile16<PolBF16<64>, 2, true>;
// the one launch of small grids (launch_fused_k): two waves per SIMD, LDS reads batched
using DqB64W2 = DqTile16<PolBF16<64>, PolBF16<64>::kDqTiles, true>;
using DkvB64W2 = DkvTile16<PolBF16<64>, 2, false, true>;
using DkvB64P2W2 = DkvTile16<PolBF16<64>, 2, true, true>;
using DqF32 = DqTile16<PolF32<64>, PolF32<64>::kDqTiles>;
using DkvF32 = DkvTile16<PolF32<64>, 2>;
using DqB128 = DqTile16<PolBF16<128>, PolBF16<128>::kDqTiles>;
using DkvB128 = DkvTile16<PolBF16<128>, 1>;

// The code object's kernels (names: fa_kernels.h), one per instantiation.
#if defined(__HIP_DEVICE_COMPILE__)
#define MXFA_PREPROCESS(NAME, T, D)                                                                      \
    extern "C" __global__ __launch_bounds__(256) void NAME(const T *dout, const T *o, float *delta, long rows) { \
        preprocess_body<T, D>(dout, o, delta, rows);                                                     \
    }
#define MXFA_DQ(NAME, TILE, CAUSAL, DELTA)                                                               \
    extern "C" __global__ __launch_bounds__(256, TILE::kWaves) void NAME(Params p) {                    \
        dq_entry<TILE, CAUSAL, DELTA>(p);                                                                \
    }
#define MXFA_DKV(NAME, TILE, CAUSAL)                                                                     \
    extern "C" __global__ __launch_bounds__(256, TILE::kWaves) void NAME(Params p) { dkv_entry<TILE, CAUSAL>(p); }
#define MXFA_FUSED(NAME, DQT, DKVT, CAUSAL)                                                              \
    extern "C" __global__ __launch_bounds__(256, DKVT::kWaves < DQT::kWaves ? DKVT::kWaves : DQT::kWaves) void \
    NAME(Params p) {                                                                                     \
        bwd_fused_entry<DQT, DKVT, CAUSAL>(p);                                                           \
    }
#define MXFA_REDUCE(NAME, T)                                                                             \
    extern "C" __global__ __launch_bounds__(256) void NAME(Params p, unsigned n4, int d4, int bkv_rows, int bq, \
                                                           int causal) {                                 \
        dkv_reduce_body<T>(p, n4, d4, bkv_rows, bq, causal);                                             \
    }
MXFA_PREPROCESS(mxfa_preprocess_b64, u16, 64)
MXFA_PREPROCESS(mxfa_preprocess_b128, u16, 128)
MXFA_PREPROCESS(mxfa_preprocess_f64, float, 64)
MXFA_DQ(mxfa_dq_b64_c, DqB64, true, false)
MXFA_DQ(mxfa_dq_b64_c_d, DqB64, true, true)
MXFA_DQ(mxfa_dq_b64_n, DqB64, false, false)
MXFA_DQ(mxfa_dq_b64_n_d, DqB64, false, true)
MXFA_DQ(mxfa_dq_b128_c, DqB128, true, false)
MXFA_DQ(mxfa_dq_b128_c_d, DqB128, true, true)
MXFA_DQ(mxfa_dq_b128_n, DqB128, false, false)
MXFA_DQ(mxfa_dq_b128_n_d, DqB128, false, true)
MXFA_DQ(mxfa_dq_f64_c, DqF32, true, false)
MXFA_DQ(mxfa_dq_f64_c_d, DqF32, true, true)
MXFA_DQ(mxfa_dq_f64_n, DqF32, false, false)
MXFA_DQ(mxfa_dq_f64_n_d, DqF32, false, true)
MXFA_DKV(mxfa_dkv_b64_c, DkvB64, true)
MXFA_DKV(mxfa_dkv_b64_n, DkvB64, false)
MXFA_DKV(mxfa_dkv_b64_c_p2, DkvB64P2, true)
MXFA_DKV(mxfa_dkv_b64_n_p2, DkvB64P2, false)
MXFA_DKV(mxfa_dkv_b128_c, DkvB128, true)
MXFA_DKV(mxfa_dkv_b128_n, DkvB128, false)
MXFA_DKV(mxfa_dkv_f64_c, DkvF32, true)
MXFA_DKV(mxfa_dkv_f64_n, DkvF32, false)
MXFA_FUSED(mxfa_bwd_b64_c, DqB64, DkvB64, true)
MXFA_FUSED(mxfa_bwd_b64_n, DqB64, DkvB64, false)
MXFA_FUSED(mxfa_bwd_b64_c_p2, DqB64, DkvB64P2, true)
MXFA_FUSED(mxfa_bwd_b64_n_p2, DqB64, DkvB64P2, false)
MXFA_FUSED(mxfa_bwd_b64_c_w2, DqB64W2, DkvB64W2, true)
MXFA_FUSED(mxfa_bwd_b64_n_w2, DqB64W2, DkvB64W2, false)
MXFA_FUSED(mxfa_bwd_b64_c_p2_w2, DqB64W2, DkvB64P2W2, true)
MXFA_FUSED(mxfa_bwd_b64_n_p2_w2, DqB64W2, DkvB64P2W2, false)
MXFA_FUSED(mxfa_bwd_b128_c, DqB128, DkvB128, true)
MXFA_FUSED(mxfa_bwd_b128_n, DqB128, DkvB128, false)
MXFA_REDUCE(mxfa_dkv_reduce_bf16, u16)
MXFA_REDUCE(mxfa_dkv_reduce_f32, float)
#undef MXFA_PREPROCESS
#undef MXFA_DQ
#undef MXFA_DKV
#undef MXFA_FUSED
#undef MXFA_REDUCE
#endif

// ----------------------------------------------------------------- launchers

// The kernels of each (dtype, head dim): the tiles and their code-object
// names, [causal] and [causal][computes Delta].
struct KernelsB64 {
    using Dq = DqB64;
    using Dkv = DkvB64;
    static constexpr KernelId dq[2][2] = {{k_mxfa_dq_b64_n, k_mxfa_dq_b64_n_d}, {k_mxfa_dq_b64_c, k_mxfa_dq_b64_c_d}};
    static constexpr KernelId dkv[2] = {k_mxfa_dkv_b64_n, k_mxfa_dkv_b64_c};
    static constexpr KernelId fused[2] = {k_mxfa_bwd_b64_n, k_mxfa_bwd_b64_c};
    // the same with DkvB64P2, for a softmax scale that is a power of two
    static constexpr bool kHasP2 = true;
    static constexpr KernelId dkv_p2[2] = {k_mxfa_dkv_b64_n_p2, k_mxfa_dkv_b64_c_p2};
    static constexpr KernelId fused_p2[2] = {k_mxfa_bwd_b64_n_p2, k_mxfa_bwd_b64_c_p2};
    // the one launch at two waves per SIMD with batched LDS reads (DqB64W2,
    // DkvB64W2 / DkvB64P2W2), for launches whose dQ and dK/dV work-groups
    // the three-wave kernel would hold all at once: each work-group then runs
    // faster, and the heaviest ones set the launch's time (A/B, µs: causal
    // B4 H12 N1024 41.6 -> 34.5, B2 H12 N2048 65.4 -> 56.5, B1 H16 N2048
    // 58.0 -> 50.2; grids of two rounds and more ran 3-8% slower with it)
    static constexpr bool kHasW2 = true;
    static constexpr KernelId fused_w2[2] = {k_mxfa_bwd_b64_n_w2, k_mxfa_bwd_b64_c_w2};
    static constexpr KernelId fused_p2_w2[2] = {k_mxfa_bwd_b64_n_p2_w2, k_mxfa_bwd_b64_c_p2_w2};
    static constexpr KernelId reduce = k_mxfa_dkv_reduce_bf16;
};
struct KernelsB128 {
    using Dq = DqB128;
    using Dkv = DkvB128;
    static constexpr KernelId dq[2][2] = {{k_mxfa_dq_b128_n, k_mxfa_dq_b128_n_d},
                                          {k_mxfa_dq_b128_c, k_mxfa_dq_b128_c_d}};
    static constexpr KernelId dkv[2] = {k_mxfa_dkv_b128_n, k_mxfa_dkv_b128_c};
    static constexpr KernelId fused[2] = {k_mxfa_bwd_b128_n, k_mxfa_bwd_b128_c};
    static constexpr bool kHasP2 = false;
    static constexpr KernelId dkv_p2[2] = {k_mxfa_dkv_b128_n, k_mxfa_dkv_b128_c};
    static constexpr KernelId fused_p2[2] = {k_mxfa_bwd_b128_n, k_mxfa_bwd_b128_c};
    static constexpr bool kHasW2 = false;
    static constexpr KernelId fused_w2[2] = {k_mxfa_bwd_b128_n, k_mxfa_bwd_b128_c};
    static constexpr KernelId fused_p2_w2[2] = {k_mxfa_bwd_b128_n, k_mxfa_bwd_b128_c};
    static constexpr KernelId reduce = k_mxfa_dkv_reduce_bf16;
};
struct KernelsF64 {
    using Dq = DqF32;
    using Dkv = DkvF32;
    static constexpr KernelId dq[2][2] = {{k_mxfa_dq_f64_n, k_mxfa_dq_f64_n_d}, {k_mxfa_dq_f64_c, k_mxfa_dq_f64_c_d}};
    static constexpr KernelId dkv[2] = {k_mxfa_dkv_f64_n, k_mxfa_dkv_f64_c};
    static constexpr bool kHasP2 = false;
    static constexpr KernelId dkv_p2[2] = {k_mxfa_dkv_f64_n, k_mxfa_dkv_f64_c};
    static constexpr KernelId reduce = k_mxfa_dkv_reduce_f32;
};

// A softmax scale that is a power of two (the default 1/sqrt(64) = 1/8 is):
// the kernels with the P2 dK/dV tile hold K scale exactly in bf16.
static bool scale_is_pow2(float scale) {
    int e = 0;
    return scale > 0.0f && std::frexp(scale, &e) == 0.5f;
}

hipError_t launch_preprocess(const Params &p, int dtype_bf16, int d, hipStream_t stream) {
    long rows = (long)p.B * p.Hq * p.N;
    const dim3 grid((unsigned)((rows * 8 + 255) / 256));
    KernelId id;
    if (dtype_bf16 && d == 64) {
        id = k_mxfa_preprocess_b64;
    } else if (dtype_bf16 && d == 128) {
        id = k_mxfa_preprocess_b128;
    } else if (!dtype_bf16 && d == 64) {
        id = k_mxfa_preprocess_f64;
    } else {
        return hipErrorInvalidValue;
    }
    const void *dout = p.dout, *o = p.o_in;
    float *delta = p.delta;
    void *args[] = {&dout, &o, &delta, &rows};
    return launch_kernel(id, grid, dim3(256), args, stream);
}

template <class K>
static hipError_t launch_dq_k(Params p, int causal, int delta, hipStream_t stream) {
    constexpr int BQ = 4 * K::Dq::ROWS;
    const dim3 grid(p.B * p.Hq, (p.N + BQ - 1) / BQ);
    const KernelId id = K::dq[causal ? 1 : 0][delta ? 1 : 0];
    if (causal) cu_balance(&p, id, (long long)grid.x * grid.y);
    void *args[] = {&p};
    return launch_kernel(id, grid, dim3(256), args, stream);
}

hipError_t launch_bwd_dq(const Params &p, int dtype_bf16, int d, int causal, int delta, hipStream_t stream) {
    if (dtype_bf16 && d == 64) return launch_dq_k<KernelsB64>(p, causal, delta, stream);
    if (dtype_bf16 && d == 128) return launch_dq_k<KernelsB128>(p, causal, delta, stream);
    if (!dtype_bf16 && d == 64) return launch_dq_k<KernelsF64>(p, causal, delta, stream);
    return hipErrorInvalidValue;
}

// Launch-wide settings of the one-launch backward (mxfa_set_bwd_options).
static std::atomic<unsigned> g_epoch{0};
static std::atomic<int> g_one_launch{1};
static std::atomic<int> g_delta_wait_us{200};
static std::atomic<int> g_reduce_wait_us{2000000};

void set_bwd_options(int one_launch, int delta_wait_us, int reduce_wait_us) {
    g_one_launch.store(one_launch);
    g_delta_wait_us.store(delta_wait_us);
    g_reduce_wait_us.store(reduce_wait_us);
}
void get_bwd_options(int *one_launch, int *delta_wait_us, int *reduce_wait_us) {
    *one_launch = g_one_launch.load();
    *delta_wait_us = g_delta_wait_us.load();
    *reduce_wait_us = g_reduce_wait_us.load();
}

bool bwd_fused_available(const Params &p, int dtype_bf16, int d, hipStream_t stream) {
    if (!dtype_bf16 || (d != 64 && d != 128)) return false;
    // a launch captured into a graph would replay with the epoch of its
    // capture, so a replay could take the previous replay's flags for its own
    // Delta: graphs get the two-launch form
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (stream != nullptr && hipStreamIsCapturing(stream, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone) {
        return false;
    }
    const long long nfb = (p.N + kFlagRows - 1) / kFlagRows;
    if ((long long)p.B * p.Hq * nfb > kMaxFlagBlocks) return false;
    return g_one_launch.load() != 0;
}

template <class K>
static hipError_t launch_dkv_reduce(const Params &p, int causal, hipStream_t stream) {
    using Tile = typename K::Dkv;
    const size_t n4 = (size_t)p.B * p.Hkv * p.N * (Tile::D / 4);
    if (2 * n4 >= 0xffffffffULL) return hipErrorInvalidValue;
    const size_t blocks = std::min<size_t>((2 * n4 + 255) / 256, 4096);
    unsigned n4u = (unsigned)n4;
    int d4 = Tile::D / 4, bkv_rows = 4 * Tile::ROWS, bq = Tile::Pol::ROWS;
    void *args[] = {const_cast<Params *>(&p), &n4u, &d4, &bkv_rows, &bq, &causal};
    return launch_kernel(K::reduce, dim3((unsigned)blocks), dim3(256), args, stream);
}

// The split of a dK/dV pass over its GQA group's query heads (Params::
// dkv_split and the two fields after it), for the pass's tile:
//  * none (dkv_split = 1) without GQA or when the key blocks alone give the
//    launch at least two work-groups per resident slot (256 CUs x the kernel's
//    work-groups per CU);
//  * else every key block gets at least dkv_min_shares shares: the smallest
//    divisor of the group that gives two work-groups per slot, else the whole
//    group (one query head per share);
//  * and a causal block with more stages gets more shares, about
//    dkv_share_stages stages each: the stages one slot runs on average over a
//    one-launch backward (dK/dV stages plus half the dQ stages, which cost
//    about half as much, over the slots), but at least 8 (a work-group's
//    prologue and epilogue take about as long as 3-4 stages) and no more than
//    twice the minimum shares per block. A share's stages run one after
//    another, so the heaviest share is the launch's critical path: at cfg5
//    d = 64 (B1 Hq32 Hkv4 N2048), one query head per share left key block 0's
//    32 stages per share as the last work-groups to end, with most slots idle.
template <class Tile>
static void dkv_plan_t(Params &p, bool causal) {
    p.dkv_split = p.dkv_min_shares = 1;
    p.dkv_share_stages = 1 << 30;
    if (p.group <= 1) return;
    constexpr int BKV = 4 * Tile::ROWS, BQ = Tile::Pol::ROWS;
    constexpr long long kSlots = 256LL * Tile::kWaves;
    const long long nbkv = (long long)p.B * p.Hkv, nkb = (p.N + BKV - 1) / BKV;
    int s = p.group;
    for (int c = 1; c < p.group; ++c) {
        if (p.group % c == 0 && nbkv * nkb * c >= 2 * kSlots) {
            s = c;
            break;
        }
    }
    if (s == 1) return;
    // stages of the dK/dV work (every query head of every key block) and of
    // the dQ work (128-query blocks over 64-key stages)
    long long dkv_stages = 0, dq_stages = 0;
    for (long long kb = 0; kb < nkb; ++kb) dkv_stages += (p.N - (causal ? kb * BKV : 0) + BQ - 1) / BQ;
    for (long long qb = 0; qb < (p.N + 127) / 128; ++qb) {
        dq_stages += ((causal ? std::min<long long>(p.N, 128 * (qb + 1)) : p.N) + 63) / 64;
    }
    const long long per_slot = (dkv_stages * p.group * nbkv + dq_stages * p.B * p.Hq / 2 + kSlots - 1) / kSlots;
    const long long most_stages = (long long)p.group * ((p.N + BQ - 1) / BQ);  // key block 0's
    const long long w = std::max({per_slot, 8LL, (most_stages + 2 * s - 1) / (2 * s)});
    p.dkv_split = 2;  // marks the split for dkv_block_shares
    p.dkv_min_shares = s;
    p.dkv_share_stages = (int)std::min<long long>(w, 1 << 30);
    int most = 1;
    for (long long kb = 0; kb < nkb; ++kb) {
        most = std::max(most, dkv_block_shares(p, (int)((p.N - (causal ? kb * BKV : 0) + BQ - 1) / BQ)));
    }
    p.dkv_split = most;
}

// The work-groups of a dK/dV pass (dkv_work's order) with p's split.
template <class Tile>
static long long dkv_work_groups(const Params &p, bool causal) {
    constexpr int BKV = 4 * Tile::ROWS, BQ = Tile::Pol::ROWS;
    const long long nbkv = (long long)p.B * p.Hkv, nkb = (p.N + BKV - 1) / BKV;
    if (p.dkv_split <= 1) return nbkv * nkb;
    long long n = 0;
    for (long long kb = 0; kb < nkb; ++kb) {
        n += nbkv * dkv_block_shares(p, (int)((p.N - (causal ? kb * BKV : 0) + BQ - 1) / BQ));
    }
    return n;
}

int dkv_split(const Params &p, int dtype_bf16, int d, int causal) {
    Params q = p;
    if (dtype_bf16) {
        if (d == 64) dkv_plan_t<DkvB64>(q, causal != 0);
        if (d == 128) dkv_plan_t<DkvB128>(q, causal != 0);
    } else if (d == 64) {
        dkv_plan_t<DkvF32>(q, causal != 0);
    }
    return q.dkv_split;
}

// Bytes of the fp32 partial planes of a split (p.dkv_split set): dK's planes,
// then dV's.
static size_t dkv_planes_bytes(const Params &p, int d) {
    return 2 * (size_t)p.dkv_split * p.B * p.Hkv * p.N * d * sizeof(float);
}

// The workspace of a split dK/dV pass: its planes, then the one-launch
// backward's share flags (8 bytes per share, dkv_work's order); 0 without a
// split.
template <class Tile>
static size_t dkv_workspace_bytes_t(Params p, bool causal) {
    dkv_plan_t<Tile>(p, causal);
    if (p.dkv_split <= 1) return 0;
    return dkv_planes_bytes(p, Tile::D) + 8 * (size_t)dkv_work_groups<Tile>(p, causal);
}

size_t dkv_workspace_bytes(const Params &p, int dtype_bf16, int d, int causal) {
    if (dtype_bf16 && d == 64) return dkv_workspace_bytes_t<DkvB64>(p, causal != 0);
    if (dtype_bf16 && d == 128) return dkv_workspace_bytes_t<DkvB128>(p, causal != 0);
    if (!dtype_bf16 && d == 64) return dkv_workspace_bytes_t<DkvF32>(p, causal != 0);
    return 0;
}

// A share-flag value for the next launch with an in-launch reduce: distinct for
// every launch of the process (a counter through a bijective 64-bit mix) and,
// through a random start, unrelated to any earlier process's values, so a
// flag left in the workspace by an earlier launch, or whatever the workspace
// memory held before, equals it only with probability 2^-64.
static unsigned long long next_share_nonce() {
    static const unsigned long long base = [] {
        unsigned long long r = 0;
        try {  // no exception may leave the C ABI: without an entropy source, the clocks alone
            std::random_device rd;
            r = ((unsigned long long)rd() << 32) ^ (unsigned long long)rd();
        } catch (...) {
        }
        const unsigned long long t = (unsigned long long)std::chrono::steady_clock::now().time_since_epoch().count();
        const unsigned long long w =
            (unsigned long long)std::chrono::system_clock::now().time_since_epoch().count();
        return r ^ (t * 0x9E3779B97F4A7C15ull) ^ (w * 0xC2B2AE3D27D4EB4Full);
    }();
    static std::atomic<unsigned long long> count{0};
    unsigned long long x = base + 0x9E3779B97F4A7C15ull * (count.fetch_add(1) + 1);
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;  // splitmix64's finaliser
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

template <class K>
static hipError_t launch_fused_k(Params p, int causal, hipStream_t stream) {
    // with a workspace, GQA shapes split each group's query heads as in the
    // dK/dV pass; the shares' partial sums are added by the launch's last
    // work-groups (dkv_reduce_rows), else by a second launch
    dkv_plan_t<typename K::Dkv>(p, causal != 0);
    if (p.dkv_ws == nullptr) p.dkv_split = 1;
    if (p.dkv_split == 1) p.dkv_ws = nullptr;
    const long long nfb = (p.N + kFlagRows - 1) / kFlagRows;
    const long long ndq = (long long)p.B * p.Hq * nfb;
    const long long ndkv = dkv_work_groups<typename K::Dkv>(p, causal != 0);
    if (ndq + ndkv > 0x7fffffffLL) return hipErrorInvalidValue;
    unsigned e = ++g_epoch;
    if (e == 0) e = ++g_epoch;  // 0 is the flags' initial value
    p.epoch = e;
    p.flag_slot = (int)(e % kFlagSlots);
    // microseconds -> ticks of the 100 MHz real-time counter
    const int wait_us = g_delta_wait_us.load();
    p.delta_wait = wait_us < 0 ? -1 : (int)std::min(100LL * wait_us, 0x7fffffffLL);
    p.fused_ndq = (int)ndq;
    p.fused_ndkv = (int)ndkv;
    // a split's reduce runs in the same launch, after the shares, whose flags
    // follow the planes in the workspace (dkv_workspace_bytes)
    long long nred = 0;
    p.red_rows = 0;
    if (p.dkv_split > 1) {
        constexpr int BKV = 4 * K::Dkv::ROWS, RR = 16;  // dkv_reduce_rows' keys per work-group
        nred = (long long)p.B * p.Hkv * ((p.N + BKV - 1) / BKV) * (BKV / RR);
        p.red_rows = RR;
        p.red_wait = (int)std::min(100LL * g_reduce_wait_us.load(), 0x7fffffffLL);  // 100 MHz ticks
        p.share_flags = reinterpret_cast<unsigned long long *>(reinterpret_cast<char *>(p.dkv_ws) +
                                                               dkv_planes_bytes(p, K::Dkv::D));
        p.share_nonce = next_share_nonce();
    }
    if (ndq + ndkv + nred > 0x7fffffffLL) return hipErrorInvalidValue;
    // the two-wave form where the three-wave kernel would hold every dQ and
    // dK/dV work-group at once (256 CUs x its work-groups per CU); the split
    // plan above is the three-wave tile's either way, so both give the same bits
    const bool w2 = K::kHasW2 && ndq + ndkv <= 256LL * K::Dkv::kWaves;
    const bool p2 = K::kHasP2 && scale_is_pow2(p.scale);
    const int c = causal ? 1 : 0;
    const KernelId id = w2 ? (p2 ? K::fused_p2_w2[c] : K::fused_w2[c]) : (p2 ? K::fused_p2[c] : K::fused[c]);
    void *args[] = {&p};
    const hipError_t err = launch_kernel(id, dim3((unsigned)(ndq + ndkv + nred)), dim3(256), args, stream);
    if (err != hipSuccess || p.dkv_split == 1 || p.red_rows > 0) return err;
    return launch_dkv_reduce<K>(p, causal, stream);
}

hipError_t launch_bwd_fused(const Params &p, int d, int causal, hipStream_t stream) {
    if (d == 64) return launch_fused_k<KernelsB64>(p, causal, stream);
    if (d == 128) return launch_fused_k<KernelsB128>(p, causal, stream);
    return hipErrorInvalidValue;
}

template <class K>
static hipError_t launch_dkv_k(Params p, int causal, hipStream_t stream) {
    using Tile = typename K::Dkv;
    // with a workspace, GQA shapes whose key blocks alone underfill the GPU
    // split each group's query heads over several work-groups
    dkv_plan_t<Tile>(p, causal != 0);
    if (p.dkv_ws == nullptr) p.dkv_split = 1;
    if (p.dkv_split == 1) p.dkv_ws = nullptr;
    const long long n = dkv_work_groups<Tile>(p, causal != 0);
    if (n > 0x7fffffffLL) return hipErrorInvalidValue;
    void *args[] = {&p};
    const KernelId id = K::kHasP2 && scale_is_pow2(p.scale) ? K::dkv_p2[causal ? 1 : 0] : K::dkv[causal ? 1 : 0];
    const hipError_t e = launch_kernel(id, dim3((unsigned)n), dim3(256), args, stream);
    if (e != hipSuccess || p.dkv_split == 1) return e;
    return launch_dkv_reduce<K>(p, causal, stream);
}

hipError_t launch_bwd_dkv(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream) {
    if (dtype_bf16 && d == 64) return launch_dkv_k<KernelsB64>(p, causal, stream);
    if (dtype_bf16 && d == 128) return launch_dkv_k<KernelsB128>(p, causal, stream);
    if (!dtype_bf16 && d == 64) return launch_dkv_k<KernelsF64>(p, causal, stream);
    return hipErrorInvalidValue;
}

}  // namespace mxfa
