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
//   * dkv_kernel: a workgroup owns 64*KT keys of one (batch, KV head); each of
//     its 4 waves owns 16*KT keys whose K/V rows sit in registers and whose
//     dK/dV accumulate in registers (bf16, d = 64: three work-groups per CU).
//     Q/dO/LSE/Delta stream through double-buffered LDS (direct global->LDS
//     loads issued one stage ahead), 64 queries per stage, for every query head of the
//     KV head's group in turn, so the grouped-query reduction of dK/dV happens
//     inside the kernel with no atomics and no extra memory.
//   * dq_kernel: a workgroup owns 128 queries of one (batch, query head) (32
//     per wave, Q/dO rows in registers); K/V stream through LDS 64 keys per
//     stage. It recomputes S and dP (the price of staying atomic-free and O(N)
//     in memory).
#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

// ------------------------------------------------------------ preprocess

// Delta_i = sum_x dO[i][x] * O[i][x], 8 lanes per row (attention_bwd.cu:32-44).
template <class T, int D>
__global__ __launch_bounds__(256) void preprocess_kernel(const T *dout, const T *o, float *delta,
                                                         long rows) {
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

// One dK/dV stage: the Pol::ROWS query rows from qs of Q and dO of head bh,
// and their LSE and Delta, into LDS buffers.
template <class Pol, int NT = 256, bool STAGE_DELTA = true>
__device__ __forceinline__ void stage_qdo(typename Pol::T *sq, typename Pol::T *sdo, float *sl, float *sd,
                                          const Params &p, size_t bh, int qs, int N, const RowPlan<Pol, NT> &pl,
                                          int wave, int lane) {
    using T = typename Pol::T;
    const size_t off = (bh * N + qs) * Pol::D;
    stage_rows<Pol, NT>(sq, static_cast<const T *>(p.q) + off, N - qs, pl, wave);
    stage_rows<Pol, NT>(sdo, static_cast<const T *>(p.dout) + off, N - qs, pl, wave);
    // rows past N: LSE = +inf makes their p (and so dS) exactly 0
    if (wave == 0) stage_vec64(sl, p.lse + bh * N + qs, N - qs, lane, &kPosInf);
    if (STAGE_DELTA && wave == 1) stage_vec64(sd, p.delta + bh * N + qs, N - qs, lane, p.delta + bh * N + qs);
}

// Delta of the Pol::ROWS rows from qs of head bh, computed by one wave from O
// and dO (lane r: row qs + r) into LDS: the one-launch backward's fallback
// when a block's flag has not appeared.
template <class Pol>
__device__ __forceinline__ void delta_rows_direct(float *sd, const Params &p, size_t bh, int qs, int N, int lane) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    const int row = qs + lane;
    float acc = 0.f;
    if (row < N) {
        const size_t off = (bh * N + row) * Pol::D;
        const Frag *o = reinterpret_cast<const Frag *>(static_cast<const T *>(p.o_in) + off);
        const Frag *d = reinterpret_cast<const Frag *>(static_cast<const T *>(p.dout) + off);
#pragma unroll
        for (int c = 0; c < Pol::D / Pol::EPC; ++c) acc += Pol::dot(d[c], o[c]);
    }
    sd[lane] = acc;
}

// Delta flags of the one-launch backward (see Params::epoch). Zero at load;
// launch epochs start at 1, so no flag matches before it is published.
__device__ uint32_t g_delta_flags[kFlagSlots * kMaxFlagBlocks];
constexpr int kFlagRows = 128;  // query rows per flag: one dQ work-group's block

// ------------------------------------------------------------------ dQ pass

// One 64-key stage of the dQ pass for one wave (16 QT queries). The score
// accumulators start at nL2, so they come out as the exponents of P, times
// xmul where the policy keeps Q exact (Pol::kExactScale: qf holds Q, nL2 is
// -L / scale, xmul = scale log2(e)); otherwise qf holds Q scale log2(e) and
// nL2 is -L log2(e). dof holds -dO and the dP accumulators start at Delta, so
// they come out as Delta - dP and the MFMAs accumulate -dQ / scale (the
// epilogue multiplies by -scale). PRIO: the matrix products run at raised
// wave priority, the softmax part at normal priority (the one-launch backward,
// where dQ and dK/dV work-groups share each SIMD).
template <class Pol, int QT, bool CAUSAL, bool MASK, bool PRIO = false>
__device__ __forceinline__ void dq_stage(f32x4 (&acc)[Pol::D / 16][QT], const typename Pol::Frag (&qf)[QT][Pol::NC],
                                         const typename Pol::Frag (&dof)[QT][Pol::NC], const float (&nL2)[QT],
                                         const float (&Dl)[QT], const typename Pol::T *sk,
                                         const typename Pol::T *sv, int k0, int q0, int N, int g, int l16,
                                         float xmul) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
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

// DELTA: compute Delta_i = sum_x dO[i,x] O[i,x] here (O from p.o_in, the
// same fp32 products as preprocess_kernel, summed in another order) and write
// it to p.delta for the dK/dV pass, instead of reading it from there.
// LDS of a dQ work-group: double-buffered K and V tiles.
template <class Pol>
struct DqSmem {
    __attribute__((aligned(16))) typename Pol::T sK[2][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) typename Pol::T sV[2][Pol::ROWS * Pol::D];
};

// The dQ work of query block qb (16 QT NW rows) of (batch, query head) bh.
// QT: 16-query tiles per wave; NW: waves per work-group. PUBLISH (with
// DELTA, in the one-launch backward): Delta is written through to memory and
// then the block's flag set to p.epoch, before the main loop.
template <class Pol, bool CAUSAL, int NW, bool DELTA, int QT, bool PUBLISH = false>
__device__ __forceinline__ void dq_body(const Params &p, int bh, int qb, DqSmem<Pol> &sm) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int BQ = 16 * QT * NW, BK = Pol::ROWS, NT = 64 * NW;
    static_assert(BQ % BK == 0, "causal: the masked tail is the work-group's BQ / BK diagonal stages");
    // raised priority for the matrix products in the one launch at d = 64
    // (at d = 128 it measured 7-13% slower)
    constexpr bool kPrio = PUBLISH && D == 64;
    auto &sK = sm.sK;
    auto &sV = sm.sV;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const T *Q = static_cast<const T *>(p.q) + (size_t)bh * N * D;
    const T *dO = static_cast<const T *>(p.dout) + (size_t)bh * N * D;
    const size_t kvoff = ((size_t)b * p.Hkv + kvh) * N * D;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int q0 = qb * BQ + wave * 16 * QT;

    Frag qf[QT][NC], dof[QT][NC];
    float nL2[QT], Dl[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        const bool ok = qi < N;
        Pol::gmem_row_frags(qf[qt], Q + (size_t)qi * D, g, ok);
        Pol::gmem_row_frags(dof[qt], dO + (size_t)qi * D, g, ok);
        if constexpr (DELTA) {
            // the lane holds 16 of the row's d elements; the 4 lane groups
            // g = 0..3 together hold the row
            Frag of[NC];
            Pol::gmem_row_frags(of, static_cast<const T *>(p.o_in) + (size_t)bh * N * D + (size_t)qi * D, g, ok);
            float dsum = 0.f;
#pragma unroll
            for (int kc = 0; kc < NC; ++kc) dsum += Pol::dot(dof[qt][kc], of[kc]);
            Dl[qt] = xg_sum(dsum);
            if (ok && g == 0) {
                if constexpr (PUBLISH) {
                    store_wt(p.delta + (size_t)bh * N + qi, __float_as_uint(Dl[qt]));
                } else {
                    p.delta[(size_t)bh * N + qi] = Dl[qt];
                }
            }
        } else {
            Dl[qt] = ok ? p.delta[(size_t)bh * N + qi] : 0.f;
        }
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) {
            if (!Pol::kExactScale) qf[qt][kc] = Pol::scaled(qf[qt][kc], p.scale_log2);
            dof[qt][kc] = Pol::neg(dof[qt][kc]);
        }
        nL2[qt] = ok ? p.lse[(size_t)bh * N + qi] * (Pol::kExactScale ? -1.0f / p.scale : -kLog2e) : 0.f;
    }
    f32x4 acc[XT][QT];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
        for (int qt = 0; qt < QT; ++qt) acc[xt][qt] = zero4();
    }

    if constexpr (PUBLISH) {
        static_assert(DELTA && BQ == kFlagRows, "a published block is one work-group's Delta rows");
        // every wave's Delta stores acknowledged (written through), then the flag
        wait_stores();
        __syncthreads();
        if (tid == 0) {
            const int nfb = (N + kFlagRows - 1) / kFlagRows;
            store_wt(g_delta_flags + (size_t)p.flag_slot * kMaxFlagBlocks + (size_t)bh * nfb + qb, p.epoch);
        }
    }

    const int kend = CAUSAL ? min(N, qb * BQ + BQ) : N;
    const int nsteps = (kend + BK - 1) / BK;

    const RowPlan<Pol, NT> plan(tid);
    stage_kv<Pol, NT>(sK[0], sV[0], K, V, 0, N, plan, wave);
    wait_stage();
    __syncthreads();

    // Every stage but the last kTail is unmasked for every wave (causal: its
    // keys all precede the workgroup's first query; otherwise: only the last
    // stage can be ragged). Those run in pairs with the LDS buffer a
    // compile-time constant, so the tile addresses fold into the instructions'
    // immediate offsets; the last kTail stages choose their buffer and masking
    // at run time.
    auto main_stage = [&](auto buf, int st) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < nsteps) stage_kv<Pol, NT>(sK[B ^ 1], sV[B ^ 1], K, V, (st + 1) * BK, N, plan, wave);
        dq_stage<Pol, QT, CAUSAL, false, kPrio>(acc, qf, dof, nL2, Dl, sK[B], sV[B], st * BK, q0, N, g, l16,
                                                  p.scale_log2);
        wait_stage();
        __syncthreads();
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
        if (!CAUSAL || k0 <= q0 + 16 * QT - 1) {
            dq_stage<Pol, QT, CAUSAL, true, kPrio>(acc, qf, dof, nL2, Dl, sK[cur], sV[cur], k0, q0, N, g, l16,
                                                     p.scale_log2);
        }
        wait_stage();
        __syncthreads();
    }

    T *dQ = static_cast<T *>(p.dq) + (size_t)bh * N * D;
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        if (qi < N) {
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) store4<T>(dQ + (size_t)qi * D + 16 * xt + 4 * g, acc[xt][qt], -p.scale);
        }
    }
}

// Causal: query blocks from the last (the most keys) to the first.
template <class Pol, bool CAUSAL, int NW, bool DELTA, int QT>
__global__ __launch_bounds__(64 * NW, Pol::kWavesDq) void dq_kernel(Params p) {
    __shared__ DqSmem<Pol> sm;
    const int nqb = (p.N + 16 * QT * NW - 1) / (16 * QT * NW);
    const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;
    dq_body<Pol, CAUSAL, NW, DELTA, QT>(p, blockIdx.x, qb, sm);
}

// ---------------------------------------------------------------- dK/dV pass

// Building blocks of the ping-pong dK/dV kernel (bf16, d = 64, 32 keys per
// wave), split so the LDS reads of a block's operands can be issued a phase
// before the MFMAs that use them.
namespace pp {

constexpr int kNbuf = 4;
constexpr int kTileBytes = 64 * 64 * 2;                    // one 64 x 64 bf16 tile
constexpr int kVecOff = kNbuf * 2 * kTileBytes;            // LSE / Delta vectors
constexpr int kSmemBytes = kVecOff + kNbuf * 2 * 64 * 4;   // 66 KB
static_assert(kVecOff >= 8 * 8 * 64 * 16, "the exchange of partial sums fits the tile area");

// The LDS operands of one block's chained GEMMs: dO^T and Q^T, 16 columns of
// d (xt) by the block's 32 query rows, read transposed.
template <class Pol>
__device__ __forceinline__ void chain_operands(bf16x8 (&cdo)[4], bf16x8 (&cq)[4], const u16 *sq, const u16 *sdo,
                                               int blk, int g, int l16) {
#pragma unroll
    for (int xt = 0; xt < 4; ++xt) {
        cdo[xt] = Pol::chain_a(sdo, 16 * xt, blk, g, l16);
        cq[xt] = Pol::chain_a(sq, 16 * xt, blk, g, l16);
    }
}

// Chained GEMMs of one block: dV^T += dO^T P^T and (-dK / scale)^T += Q^T dS^T.
template <class Pol>
__device__ __forceinline__ void chain_block(f32x4 (&accK)[4][2], f32x4 (&accV)[4][2], const bf16x8 (&cp)[2],
                                            const bf16x8 (&cds)[2], const bf16x8 (&cdo)[4], const bf16x8 (&cq)[4]) {
#pragma unroll
    for (int xt = 0; xt < 4; ++xt) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            accV[xt][kt] = Pol::mma(cdo[xt], cp[kt], accV[xt][kt]);
            accK[xt][kt] = Pol::mma(cq[xt], cds[kt], accK[xt][kt]);
        }
    }
}

// The row-form LDS operands of one block's scores: Q and dO rows arow(t, .)
// and Delta of rows bidx(t, g, 0..3).
struct ScoreOps {
    bf16x8 q[2][2], d[2][2];  // [t][kc]
    f32x4 dl[2], nl[2];       // Delta and LSE x lmul of the rows
};
template <class Pol>
__device__ __forceinline__ void score_operands(ScoreOps &o, const u16 *sq, const u16 *sdo, const float *sl,
                                               const float *sd, int blk, int g, int l16, float lmul) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int n = blk + Pol::arow(t, l16);
        Pol::lds_row_frags(o.q[t], sq, n, g);
        Pol::lds_row_frags(o.d[t], sdo, n, g);
        o.dl[t] = *reinterpret_cast<const f32x4 *>(sd + blk + Pol::bidx(t, g, 0));
        o.nl[t] = *reinterpret_cast<const f32x4 *>(sl + blk + Pol::bidx(t, g, 0)) * lmul;
    }
}

// Scores K Q^T + C with C = L lmul (the exponents of P up to the factor
// softmax_block applies: kf holds K and lmul = -1 / scale with exact scaling,
// else kf holds K scale log2(e) and lmul = -log2(e)), and Delta - dP =
// Delta + (-V) dO^T of one block.
template <class Pol>
__device__ __forceinline__ void score_block(f32x4 (&s)[2][2], f32x4 (&dp)[2][2], const bf16x8 (&kf)[2][2],
                                            const bf16x8 (&vf)[2][2], const ScoreOps &o) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            f32x4 c = o.nl[t];
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) c = Pol::mma(o.q[t][kc], kf[kt][kc], c);
            s[t][kt] = c;
            c = o.dl[t];
#pragma unroll
            for (int kc = 0; kc < 2; ++kc) c = Pol::mma(o.d[t][kc], vf[kt][kc], c);
            dp[t][kt] = c;
        }
    }
}

// P = exp2(S scale log2(e) - L log2(e)) (s holds the exponents, or with
// exact scaling the exponents / (scale log2(e)), multiplied back here) and
// -dS / scale = P (Delta - dP), packed as the chain operands. MASK (causal):
// query row bidx of the block precedes key 16 kt + l16 of the wave iff
// bidx - l16 < moff + 16 kt, where moff = first key of the wave - first query
// of the block (0 on the diagonal, >= 32 for a block wholly before the keys,
// whose P is then all zero).
template <class Pol, bool MASK>
__device__ __forceinline__ void softmax_block(f32x4 (&s)[2][2], f32x4 (&dp)[2][2], bf16x8 (&cp)[2],
                                              bf16x8 (&cds)[2], int moff, int g, int l16, float xmul) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
#pragma unroll
            for (int kt = 0; kt < 2; ++kt) {
                float x = s[t][kt][r];
                if constexpr (MASK) x = Pol::bidx(t, g, r) - l16 < moff + 16 * kt ? -INFINITY : x;
                const float pv = fast_exp2(Pol::kExactScale ? x * xmul : x);
                s[t][kt][r] = pv;
                dp[t][kt][r] = pv * dp[t][kt][r];
            }
        }
    }
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        cp[kt] = Pol::pack(s[0][kt], s[1][kt]);
        cds[kt] = Pol::pack(dp[0][kt], dp[1][kt]);
    }
}

}  // namespace pp

// One 64-query stage of the dK/dV pass for one wave (16*KT keys). The score
// accumulators start at L lmul, so they come out as the exponents of P, times
// xmul where the policy keeps K exact (Pol::kExactScale: kf holds K, lmul =
// -1 / scale, xmul = scale log2(e)); otherwise kf holds K scale log2(e) and
// lmul = -log2(e). vf holds -V and the dP accumulators start at Delta, so
// they come out as Delta - dP and accK accumulates -dK / scale (the epilogue
// multiplies by -scale). PRIO: the matrix products run at raised wave
// priority, the softmax part at normal priority (the one-launch backward).
template <class Pol, int KT, bool CAUSAL, bool MASK, bool PRIO = false>
__device__ __forceinline__ void dkv_stage(f32x4 (&accK)[Pol::D / 16][KT], f32x4 (&accV)[Pol::D / 16][KT],
                                          const typename Pol::Frag (&kf)[KT][Pol::NC],
                                          const typename Pol::Frag (&vf)[KT][Pol::NC], const typename Pol::T *sq,
                                          const typename Pol::T *sdo, const float *sl, const float *sd, int qs,
                                          int kw0, int N, int g, int l16, float lmul, float xmul) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        f32x4 s[2][KT], dp[2][KT];  // [t][kt]
        wave_priority<PRIO>(1);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            // block rows bidx(t, g, 0..3) are consecutive: one 16-byte LDS read
            const int q4 = 32 * blk + Pol::bidx(t, g, 0);
            const f32x4 nl = *reinterpret_cast<const f32x4 *>(sl + q4) * lmul;
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
                    float x = s[t][kt][r];
                    if constexpr (MASK) {
                        // causal: query qs + 32 blk + bidx(t, g, r) before key kw0 + 16 kt + l16
                        const bool before = Pol::bidx(t, g, r) - l16 < kw0 - qs + 16 * kt - 32 * blk;
                        x = before ? -INFINITY : x;
                    }
                    const float pv = fast_exp2(Pol::kExactScale ? x * xmul : x);
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

// LDS of a dK/dV work-group: an NBUF-deep ring of Q / dO tiles and their
// LSE / Delta rows (loads are issued NBUF - 1 stages ahead).
template <class Pol>
struct DkvSmem {
    static constexpr int NBUF = Pol::kDkvBuffers;
    __attribute__((aligned(16))) typename Pol::T sQ[NBUF][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) typename Pol::T sdO[NBUF][Pol::ROWS * Pol::D];
    __attribute__((aligned(16))) float sL[NBUF][Pol::ROWS];
    __attribute__((aligned(16))) float sD[NBUF][Pol::ROWS];
    uint32_t sF[2];  // one-launch backward: the flags of the next stages' Delta blocks
};

// The dK/dV work of key block kb (16 KT NW keys) of grid column bx =
// (batch, KV head) * dkv_split + share. WAIT (one-launch backward): Delta
// comes from the dQ work-groups of the same launch; wave 1 stages a stage's
// Delta rows only once their block's flag reads p.epoch (see issue below).
template <class Pol, int KT, bool CAUSAL, int NW, bool WAIT = false>
__device__ __forceinline__ void dkv_body(const Params &p, int bx, int kb, DkvSmem<Pol> &sm) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int NT = 64 * NW;       // threads per workgroup
    constexpr int BKV = 16 * KT * NW; // keys per workgroup
    constexpr int BQ = Pol::ROWS;     // queries per stage
    static_assert(BKV % BQ == 0, "causal start must align to a stage");
    // raised priority for the matrix products in the one launch at d = 64
    // (at d = 128 it measured 7-13% slower)
    constexpr bool kPrio = WAIT && D == 64;
    constexpr int NBUF = DkvSmem<Pol>::NBUF;
    auto &sQ = sm.sQ;
    auto &sdO = sm.sdO;
    auto &sL = sm.sL;
    auto &sD = sm.sD;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N;
    const int nsplit = p.dkv_split;
    const int bkv = bx / nsplit;       // b * Hkv + kvh
    const int sp = bx - bkv * nsplit;  // which share of the group's query heads
    const int b = bkv / p.Hkv, kvh = bkv % p.Hkv;
    const int h0 = sp * p.group / nsplit, nh = (sp + 1) * p.group / nsplit - h0;
    const size_t kvoff = (size_t)bkv * N * D;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int kw0 = kb * BKV + wave * 16 * KT;  // first key of this wave

    Frag kf[KT][NC], vf[KT][NC];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int key = kw0 + 16 * kt + l16;
        Pol::gmem_row_frags(kf[kt], K + (size_t)key * D, g, key < N);
        Pol::gmem_row_frags(vf[kt], V + (size_t)key * D, g, key < N);
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) {
            if (!Pol::kExactScale) kf[kt][kc] = Pol::scaled(kf[kt][kc], p.scale_log2);
            vf[kt][kc] = Pol::neg(vf[kt][kc]);
        }
    }
    const float lmul = Pol::kExactScale ? -1.0f / p.scale : -kLog2e;
    const float xmul = p.scale_log2;
    f32x4 accK[XT][KT], accV[XT][KT];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) accK[xt][kt] = accV[xt][kt] = zero4();
    }

    const int qstart = CAUSAL ? kb * BKV : 0;
    const int nqs = (N - qstart + BQ - 1) / BQ;  // stages per query head
    const int nsteps = nqs * nh;
    const size_t bh0 = (size_t)b * p.Hq + (size_t)kvh * p.group + h0;

    // Stages are loaded strictly in order; (ld_h, ld_i) = query head and stage
    // within it of the next one (kept incrementally: no division per stage).
    const RowPlan<Pol, NT> plan(tid);
    int ld_h = 0, ld_i = 0;
    // WAIT: the flag of each stage's Delta block is fetched into sm.sF one
    // issue ahead, with a load that misses the caches (as are the Delta rows
    // themselves: the dQ work-group that wrote them may sit on another XCD).
    // It is checked before the Delta rows are staged; a flag not yet set is
    // polled (up to p.delta_spin times), and then the wave computes the rows
    // itself. The first stage, with nothing fetched ahead, is polled directly.
    // Either way the rows hold Delta of the launch's own O and dO.
    const int nfb = (N + kFlagRows - 1) / kFlagRows;
    const uint32_t *flags = g_delta_flags + (size_t)p.flag_slot * kMaxFlagBlocks;
    auto issue = [&](int st) __attribute__((always_inline)) {
        const int bf = st % NBUF;
        const size_t bh = bh0 + ld_h;
        const int qs = qstart + ld_i * BQ;
        stage_qdo<Pol, NT, !WAIT>(sQ[bf], sdO[bf], sL[bf], sD[bf], p, bh, qs, N, plan, wave, lane);
        if (++ld_i == nqs) {
            ld_i = 0;
            ++ld_h;
        }
        if constexpr (WAIT) {
            static_assert(NBUF == 2, "flags are fetched one issue ahead");
            if (wave == 1) {
                const uint32_t *f = flags + bh * nfb + qs / kFlagRows;
                // delta_spin < 0 trusts no flag (every stage takes the fallback)
                bool ready = p.delta_spin >= 0 && st > 0 && sm.sF[st & 1] == p.epoch;
                for (int i = 0; !ready && i < p.delta_spin; ++i) {
                    ready = __builtin_amdgcn_readfirstlane(load_uc_sync(f)) == p.epoch;
                    if (!ready) __builtin_amdgcn_s_sleep(2);
                }
                if (ready) {
                    lds_dma4_uc(lds_addr(sD[bf]), p.delta + bh * N + min(qs + lane, N - 1));
                } else {
                    delta_rows_direct<Pol>(sD[bf], p, bh, qs, N, lane);
                }
                // one lane: the DMA writes each active lane's dword at base + 4 lane
                if (ld_h < nh && lane == 0) {
                    const int qs_next = qstart + ld_i * BQ;
                    lds_dma4_uc(lds_addr(&sm.sF[(st + 1) & 1]), flags + (bh0 + ld_h) * nfb + qs_next / kFlagRows);
                }
            }
        }
    };
    // loads of one stage per thread: the Q and dO tiles (+1 vector on waves
    // 0-1, which the waits below may over-wait by one load)
    constexpr int kLoads = 2 * tile_loads<Pol, NT>();
#pragma unroll
    for (int i = 0; i < NBUF - 1; ++i) {
        if (i < nsteps) issue(i);
    }
    if (NBUF > 2 && nsteps > 1) {
        wait_vmcnt<kLoads>();
    } else {
        wait_stage();
    }
    __syncthreads();

    // One stage: prefetch stage st + NBUF - 1, compute stage st, then wait for
    // stage st + 1 and barrier. Causal: the stages that straddle the diagonal
    // are the first ceil(BKV / BQ) of each query head (queries from kb * BKV);
    // they run in a loop of their own with the masked body, so neither loop
    // carries the other's code (two bodies behind one branch make the register
    // allocator spill).
    auto run = [&](auto mask_tag, int st, int i) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int cur = st % NBUF;
        const bool ahead = st + NBUF - 1 < nsteps;
        if (ahead) issue(st + NBUF - 1);
        const int qs = qstart + i * BQ;
        // a wave whose keys all follow the stage's queries has nothing to do
        if (!CAUSAL || qs + BQ - 1 >= kw0) {
            dkv_stage<Pol, KT, CAUSAL, MASK, kPrio>(accK, accV, kf, vf, sQ[cur], sdO[cur], sL[cur], sD[cur], qs, kw0,
                                                   N, g, l16, lmul, xmul);
        }
        if (NBUF > 2 && ahead) {
            wait_vmcnt<kLoads>();
        } else {
            wait_stage();
        }
        barrier_lds();
    };
    // The unmasked stages with the LDS buffer a compile-time constant (two
    // buffers), so the tile addresses fold into the instructions' immediate
    // offsets. No wave skips them: their queries follow all the workgroup's keys.
    auto run_fixed = [&](auto buf, int st, int i) __attribute__((always_inline)) {
        constexpr int B = decltype(buf)::value;
        if (st + 1 < nsteps) issue(st + 1);
        const int qs = qstart + i * BQ;
        dkv_stage<Pol, KT, CAUSAL, false, kPrio>(accK, accV, kf, vf, sQ[B], sdO[B], sL[B], sD[B], qs, kw0, N, g, l16,
                                                lmul, xmul);
        wait_stage();
        barrier_lds();
    };
    using Buf0 = std::integral_constant<int, 0>;
    using Buf1 = std::integral_constant<int, 1>;
    // rows past N get p = 0 from LSE = +inf, so only the causal diagonal masks
    const int ndiag = CAUSAL ? min(nqs, BKV / BQ) : 0;
    for (int hh = 0, st = 0; hh < nh; ++hh) {
        for (int i = 0; i < ndiag; ++i, ++st) run(std::true_type{}, st, i);
        if constexpr (NBUF == 2) {
            int i = ndiag;
            if (i < nqs && (st & 1)) run_fixed(Buf1{}, st++, i++);
            for (; i + 1 < nqs; i += 2, st += 2) {
                run_fixed(Buf0{}, st, i);
                run_fixed(Buf1{}, st + 1, i + 1);
            }
            if (i < nqs) run_fixed(Buf0{}, st++, i);
        } else {
            for (int i = ndiag; i < nqs; ++i, ++st) run(std::false_type{}, st, i);
        }
    }

    if (nsplit > 1) {
        // this share's fp32 partial sums (unscaled); dkv_reduce_kernel adds
        // the shares and applies the scale
        const size_t plane = (size_t)p.B * p.Hkv * N * D;
        float *wK = p.dkv_ws + (size_t)sp * plane + kvoff;
        float *wV = wK + (size_t)nsplit * plane;
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const int key = kw0 + 16 * kt + l16;
            if (key < N) {
#pragma unroll
                for (int xt = 0; xt < XT; ++xt) {
                    store4<float>(wK + (size_t)key * D + 16 * xt + 4 * g, accK[xt][kt], 1.0f);
                    store4<float>(wV + (size_t)key * D + 16 * xt + 4 * g, accV[xt][kt], 1.0f);
                }
            }
        }
        return;
    }
    T *dK = static_cast<T *>(p.dk) + kvoff;
    T *dV = static_cast<T *>(p.dv) + kvoff;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int key = kw0 + 16 * kt + l16;
        if (key < N) {
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) {
                store4<T>(dK + (size_t)key * D + 16 * xt + 4 * g, accK[xt][kt], -p.scale);
                store4<T>(dV + (size_t)key * D + 16 * xt + 4 * g, accV[xt][kt], 1.0f);
            }
        }
    }
}

// Causal: key block 0 (the most queries) is dispatched first.
template <class Pol, int KT, bool CAUSAL, int NW>
__global__ __launch_bounds__(64 * NW, Pol::kWavesDkv) void dkv_kernel(Params p) {
    __shared__ DkvSmem<Pol> sm;
    dkv_body<Pol, KT, CAUSAL, NW>(p, blockIdx.x, blockIdx.y, sm);
}

// The whole backward from O in one launch (bf16): work-groups [0, fused_ndq)
// run the dQ pass with Delta, query blocks in increasing order (so Delta
// appears in the order the dK/dV work-groups consume it: each walks its query
// rows upward from its diagonal), and publish Delta per block; the rest run
// the dK/dV pass, key block 0 first, and wait for the blocks they stage. The
// dQ work-groups have lower indices, so they are dispatched first and never
// wait; every wait of a dK/dV work-group is bounded (Params::delta_spin).
// This removes one kernel boundary per backward.
template <class Pol>
union FusedSmem {
    DqSmem<Pol> dq;
    DkvSmem<Pol> dkv;
};

template <class Pol, int KT, bool CAUSAL>
__global__ __launch_bounds__(256, Pol::kWavesDkv < Pol::kWavesDq ? Pol::kWavesDkv : Pol::kWavesDq) void
bwd_fused_kernel(Params p) {
    __shared__ FusedSmem<Pol> sm;
    const int bid = blockIdx.x;
    if (bid < p.fused_ndq) {
        const int nbh = p.B * p.Hq;
        dq_body<Pol, CAUSAL, Pol::kDqWavesPerGroup, true, Pol::kDqTiles, true>(p, bid % nbh, bid / nbh, sm.dq);
    } else {
        const int w = bid - p.fused_ndq, nbk = p.B * p.Hkv * p.dkv_split;
        dkv_body<Pol, KT, CAUSAL, 4, true>(p, w % nbk, w / nbk, sm.dkv);
    }
}

// dK / dV of a split dK/dV pass: the sum of the nsplit fp32 partial planes in
// split order (so the result is deterministic), times -scale for dK. n4 =
// float4 groups per plane; the dV planes follow the dK planes.
template <class T>
__global__ __launch_bounds__(256) void dkv_reduce_kernel(const float *ws, T *dk, T *dv, size_t n4, int nsplit,
                                                         float kscale) {
    const f32x4 *w = reinterpret_cast<const f32x4 *>(ws);
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < 2 * n4; i += stride) {
        const bool isv = i >= n4;
        const size_t j = isv ? i - n4 : i;
        const f32x4 *src = w + (isv ? (size_t)nsplit * n4 : 0) + j;
        f32x4 a = src[0];
        for (int s = 1; s < nsplit; ++s) a += src[(size_t)s * n4];
        if (isv) {
            store4<T>(dv + 4 * j, a, 1.0f);
        } else {
            store4<T>(dk + 4 * j, a, kscale);
        }
    }
}

// ------------------------------------------------- dK/dV pass, ping-pong form

// The dK/dV pass for bf16, d = 64, with two wave groups per workgroup that
// take turns on the matrix cores. A workgroup owns 128 keys; waves w and w + 4
// (which the hardware places on the same SIMD) both own keys 32w..32w+31.
// Group A (waves 0-3) takes query block 0 (rows 0-31) of every 64-query stage
// and group B (waves 4-7) block 1, so each wave handles one block per stage in
// two phases:
//   M: the chained GEMMs of its previous block (dV += P^T dO, dK += dS^T Q,
//      16 MFMAs, their LDS operands already in registers) and the scores and
//      dP of the current block (16 MFMAs);
//   V: the softmax recompute and dS of the current block (VALU and exp), the
//      transposed LDS reads of that block's chain operands for the next M, and
//      the group's share of the global->LDS loads of stage + 2.
// Group B runs one phase behind group A and a barrier separates the phases,
// so while one wave of a SIMD issues MFMAs the other issues VALU, LDS and
// global-load work. The loads are split between the groups (B: Q tiles,
// A: dO tiles and the LSE / Delta vectors) because a wave stalls on issuing
// more than a couple of wide loads at once. Stages rotate through a 4-deep LDS
// ring (a stage's buffer is last read by group B's V one stage later). At the
// end the two groups exchange partial sums through LDS: A stores dK, B dV.

template <bool CAUSAL>
__global__ __launch_bounds__(512) void dkv_pp_kernel(Params p) {
    using Pol = PolBF16<64>;
    using T = u16;
    constexpr int D = 64, XT = 4, KT = 2, BKV = 128, BQ = 64, NBUF = pp::kNbuf;

    __shared__ __attribute__((aligned(16))) char smem[pp::kSmemBytes];
    auto tq = [&](int b) { return reinterpret_cast<T *>(smem + b * 2 * pp::kTileBytes); };
    auto tdo = [&](int b) { return reinterpret_cast<T *>(smem + b * 2 * pp::kTileBytes + pp::kTileBytes); };
    auto vl = [&](int b) { return reinterpret_cast<float *>(smem + pp::kVecOff + b * 512); };
    auto vd = [&](int b) { return reinterpret_cast<float *>(smem + pp::kVecOff + b * 512 + 256); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pair = wave & 3, grp = wave >> 2;
    const int gtid = tid & 255;  // thread index within the group
    const int g = lane >> 4, l16 = lane & 15;
    const int blk = 32 * grp;  // this wave's query block within a stage
    const int N = p.N;
    const int bkv = blockIdx.x;
    const int kb = blockIdx.y;
    const int b = bkv / p.Hkv, kvh = bkv % p.Hkv;
    const size_t kvoff = (size_t)bkv * N * D;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int kw0 = kb * BKV + 32 * pair;

    bf16x8 kf[KT][2], vf[KT][2];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int key = kw0 + 16 * kt + l16;
        Pol::gmem_row_frags(kf[kt], K + (size_t)key * D, g, key < N);
        Pol::gmem_row_frags(vf[kt], V + (size_t)key * D, g, key < N);
#pragma unroll
        for (int kc = 0; kc < 2; ++kc) {
            if (!Pol::kExactScale) kf[kt][kc] = Pol::scaled(kf[kt][kc], p.scale_log2);
            vf[kt][kc] = Pol::neg(vf[kt][kc]);
        }
    }
    const float lmul = Pol::kExactScale ? -1.0f / p.scale : -kLog2e;
    const float xmul = p.scale_log2;
    f32x4 accK[XT][KT], accV[XT][KT];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) accK[xt][kt] = accV[xt][kt] = zero4();
    }

    const int qstart = CAUSAL ? kb * BKV : 0;
    const int nqs = (N - qstart + BQ - 1) / BQ;  // stages per query head
    const int nsteps = nqs * p.group;
    const size_t bh0 = (size_t)b * p.Hq + (size_t)kvh * p.group;

    // Loads of stage st: group B stages the Q tile (2 loads per thread),
    // group A the dO tile and, on its waves 0 and 1, the LSE / Delta vectors.
    // Every wave issues the stages in order; (ld_h, ld_i) = query head and
    // stage within it of the next one (kept incrementally: no division).
    int ld_h = 0, ld_i = 0;
    auto issue = [&](int st) __attribute__((always_inline)) {
        const int bf = st % NBUF;
        const size_t bh = bh0 + ld_h;
        const int qs = qstart + ld_i * BQ;
        if (++ld_i == nqs) {
            ld_i = 0;
            ++ld_h;
        }
        const size_t off = (bh * N + qs) * D;
        if (grp == 1) {
            stage_rows<Pol>(tq(bf), static_cast<const T *>(p.q) + off, N - qs, gtid, pair);
        } else {
            stage_rows<Pol>(tdo(bf), static_cast<const T *>(p.dout) + off, N - qs, gtid, pair);
            if (pair == 0) stage_vec64(vl(bf), p.lse + bh * N + qs, N - qs, lane, &kPosInf);
            if (pair == 1) stage_vec64(vd(bf), p.delta + bh * N + qs, N - qs, lane, p.delta + bh * N + qs);
        }
    };
    // waits until this wave's loads of all but its most recent issue() landed
    auto wait_older = [&]() __attribute__((always_inline)) {
        if (grp == 0 && pair < 2) {
            wait_vmcnt<3>();
        } else {
            wait_vmcnt<2>();
        }
    };
    // end of segment 2 st + 1: stage st + 1 must have landed; this wave's loads
    // of stage st + 2 (issued this or the previous segment) may stay in flight
    auto wait_next = [&](int st) __attribute__((always_inline)) {
        if (st + 1 < nsteps) {
            if (st + 2 < nsteps) {
                wait_older();
            } else {
                wait_stage();
            }
        }
    };

    issue(0);
    if (nsteps > 1) issue(1);
    wait_stage();
    barrier_phase();

    // Per-wave pipeline state: scores awaiting their softmax (M -> V), chain
    // operands awaiting their GEMMs (V -> next M). Every block is computed:
    // causal blocks wholly before the wave's keys are masked to P = 0 rather
    // than skipped (a skipped phase would only wait longer at the barrier).
    f32x4 s[2][KT], dp[2][KT];
    bf16x8 cp[KT], cds[KT], cdo[XT], cq[XT];
    pp::ScoreOps so;
    auto v_phase = [&](int st, int i) __attribute__((always_inline)) {
        const int bf = st % NBUF;
        const int moff = kw0 - (qstart + i * BQ + blk);
        pp::chain_operands<Pol>(cdo, cq, tq(bf), tdo(bf), blk, g, l16);
        if (CAUSAL && moff >= 0) {
            pp::softmax_block<Pol, true>(s, dp, cp, cds, moff, g, l16, xmul);
        } else {
            pp::softmax_block<Pol, false>(s, dp, cp, cds, 0, g, l16, xmul);
        }
    };
    auto m_phase = [&](int st) __attribute__((always_inline)) {
        const int cb = st % NBUF;
        pp::score_operands<Pol>(so, tq(cb), tdo(cb), vl(cb), vd(cb), blk, g, l16, lmul);
        pp::chain_block<Pol>(accK, accV, cp, cds, cdo, cq);
        pp::score_block<Pol>(s, dp, kf, vf, so);
    };
    auto first_scores = [&]() __attribute__((always_inline)) {
        pp::score_operands<Pol>(so, tq(0), tdo(0), vl(0), vd(0), blk, g, l16, lmul);
        pp::score_block<Pol>(s, dp, kf, vf, so);
    };

    // Segment 2 st: A runs M(st), B V(st - 1); segment 2 st + 1: A V(st),
    // B M(st). Each group runs a loop of its own (one branch around a whole
    // loop, not one per phase, so each loop keeps only its own pipeline state
    // live); both execute the same sequence of 2 nsteps + 1 barriers, which is
    // what keeps them in step (s_barrier counts waves, not call sites). Each
    // group issues its share of stage st + 2 at the start of its V phase (B in
    // segment 2 st, A in 2 st + 1), once stage st - 2's buffer is free.
    if (grp == 0) {
        first_scores();
        barrier_phase();
        if (nsteps > 2) issue(2);
        v_phase(0, 0);
        wait_next(0);
        barrier_phase();
        for (int st = 1, i = 0; st < nsteps; ++st) {
            if (++i == nqs) i = 0;
            m_phase(st);
            barrier_phase();
            if (st + 2 < nsteps) issue(st + 2);
            v_phase(st, i);
            wait_next(st);
            barrier_phase();
        }
        pp::chain_block<Pol>(accK, accV, cp, cds, cdo, cq);
    } else {
        if (nsteps > 2) issue(2);
        barrier_phase();
        first_scores();
        wait_next(0);
        barrier_phase();
        int ip = 0;  // stage index within its query head, of stage st - 1
        for (int st = 1; st < nsteps; ++st) {
            if (st + 2 < nsteps) issue(st + 2);
            v_phase(st - 1, ip);
            barrier_phase();
            m_phase(st);
            wait_next(st);
            barrier_phase();
            if (++ip == nqs) ip = 0;
        }
        v_phase(nsteps - 1, ip);
        pp::chain_block<Pol>(accK, accV, cp, cds, cdo, cq);
    }
    barrier_phase();

    // exchange: group A publishes its dV partials, group B its dK partials.
    // (Selected by value: a conditional between two array elements would take
    // their addresses and move the accumulators out of registers.)
    f32x4 give[XT][KT], keep[XT][KT];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) {
            const f32x4 k4 = accK[xt][kt], v4 = accV[xt][kt];
            give[xt][kt] = grp == 0 ? v4 : k4;
            keep[xt][kt] = grp == 0 ? k4 : v4;
        }
    }
    f32x4 *xch = reinterpret_cast<f32x4 *>(smem);
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
        for (int kt = 0; kt < KT; ++kt) xch[(wave * 8 + xt * KT + kt) * 64 + lane] = give[xt][kt];
    }
    barrier_phase();
    const int other = wave ^ 4;
    T *out = static_cast<T *>(grp == 0 ? p.dk : p.dv) + kvoff;
    const float mul = grp == 0 ? -p.scale : 1.0f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
        const int key = kw0 + 16 * kt + l16;
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
            const f32x4 sum = keep[xt][kt] + xch[(other * 8 + xt * KT + kt) * 64 + lane];
            if (key < N) store4<T>(out + (size_t)key * D + 16 * xt + 4 * g, sum, mul);
        }
    }
}

// ----------------------------------------------------------------- launchers

hipError_t launch_preprocess(const Params &p, int dtype_bf16, int d, hipStream_t stream) {
    const long rows = (long)p.B * p.Hq * p.N;
    const dim3 grid((unsigned)((rows * 8 + 255) / 256));
    if (dtype_bf16) {
        if (d == 64) hipLaunchKernelGGL((preprocess_kernel<u16, 64>), grid, dim3(256), 0, stream,
                                        static_cast<const u16 *>(p.dout), static_cast<const u16 *>(p.o_in), p.delta, rows);
        else if (d == 128) hipLaunchKernelGGL((preprocess_kernel<u16, 128>), grid, dim3(256), 0, stream,
                                              static_cast<const u16 *>(p.dout), static_cast<const u16 *>(p.o_in), p.delta, rows);
        else return hipErrorInvalidValue;
    } else {
        if (d == 64) hipLaunchKernelGGL((preprocess_kernel<float, 64>), grid, dim3(256), 0, stream,
                                        static_cast<const float *>(p.dout), static_cast<const float *>(p.o_in), p.delta, rows);
        else return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <class Pol, bool CAUSAL>
static hipError_t launch_dq_t(const Params &p, int delta, hipStream_t stream) {
    constexpr int QT = Pol::kDqTiles, NW = Pol::kDqWavesPerGroup, BQ = 16 * QT * NW;
    const dim3 grid(p.B * p.Hq, (p.N + BQ - 1) / BQ);
    if (delta) {
        hipLaunchKernelGGL((dq_kernel<Pol, CAUSAL, NW, true, QT>), grid, dim3(64 * NW), 0, stream, p);
    } else {
        hipLaunchKernelGGL((dq_kernel<Pol, CAUSAL, NW, false, QT>), grid, dim3(64 * NW), 0, stream, p);
    }
    return hipGetLastError();
}

hipError_t launch_bwd_dq(const Params &p, int dtype_bf16, int d, int causal, int delta, hipStream_t stream) {
#define MXFA_DQ(POL, DD)                                                        \
    if (d == DD) return causal ? launch_dq_t<POL<DD>, true>(p, delta, stream)  \
                               : launch_dq_t<POL<DD>, false>(p, delta, stream);
    if (dtype_bf16) {
        MXFA_DQ(PolBF16, 64)
        MXFA_DQ(PolBF16, 128)
    } else {
        MXFA_DQ(PolF32, 64)
    }
#undef MXFA_DQ
    return hipErrorInvalidValue;
}

static std::atomic<unsigned> g_epoch{0};

static int env_int(const char *name, int dflt) {
    const char *e = std::getenv(name);
    return e != nullptr && *e != '\0' ? std::atoi(e) : dflt;
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
    return env_int("MXFA_BWD_FUSED", 1) != 0;
}

template <class T>
static hipError_t launch_dkv_reduce(const Params &p, int d, hipStream_t stream);

template <class Pol, int KT, bool CAUSAL>
static hipError_t launch_fused_t(Params p, hipStream_t stream) {
    constexpr int BKV = 16 * KT * 4;
    // with a workspace, GQA shapes split each group's query heads as in the
    // dK/dV pass; the shares' partial sums are added by a second launch
    p.dkv_split = p.dkv_ws != nullptr ? dkv_split(p, 1, Pol::D) : 1;
    if (p.dkv_split == 1) p.dkv_ws = nullptr;
    const long long nfb = (p.N + kFlagRows - 1) / kFlagRows;
    const long long ndq = (long long)p.B * p.Hq * nfb;
    const long long ndkv = (long long)p.B * p.Hkv * p.dkv_split * ((p.N + BKV - 1) / BKV);
    if (ndq + ndkv > 0x7fffffffLL) return hipErrorInvalidValue;
    unsigned e = ++g_epoch;
    if (e == 0) e = ++g_epoch;  // 0 is the flags' initial value
    p.epoch = e;
    p.flag_slot = (int)(e % kFlagSlots);
    p.delta_spin = env_int("MXFA_DELTA_SPIN", 4096);
    p.fused_ndq = (int)ndq;
    hipLaunchKernelGGL((bwd_fused_kernel<Pol, KT, CAUSAL>), dim3((unsigned)(ndq + ndkv)), dim3(256), 0, stream, p);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess || p.dkv_split == 1) return err;
    return launch_dkv_reduce<u16>(p, Pol::D, stream);
}

hipError_t launch_bwd_fused(const Params &p, int d, int causal, hipStream_t stream) {
    if (d == 64) return causal ? launch_fused_t<PolBF16<64>, 2, true>(p, stream)
                               : launch_fused_t<PolBF16<64>, 2, false>(p, stream);
    if (d == 128) return causal ? launch_fused_t<PolBF16<128>, 1, true>(p, stream)
                                : launch_fused_t<PolBF16<128>, 1, false>(p, stream);
    return hipErrorInvalidValue;
}

// The ping-pong dK/dV kernel is opt-in (MXFA_DKV_KERNEL=pingpong, read on
// every call): at B=4, H=12, N=4096, d=64 causal it ran 0.29-0.30 ms against
// 0.24 ms for the 4-wave kernel of the time (now ~0.19 ms at three waves per
// SIMD), because its softmax-phase waves stall on issuing the global->LDS
// loads (which the 4-wave kernel hides behind the other work-groups on each
// SIMD); its MFMA phase alone runs near the matrix-core rate.
static bool dkv_pingpong_selected() {
    const char *e = std::getenv("MXFA_DKV_KERNEL");
    return e != nullptr && std::strcmp(e, "pingpong") == 0;
}

template <bool CAUSAL>
static hipError_t launch_dkv_pp(const Params &p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hkv, (p.N + 127) / 128);
    hipLaunchKernelGGL((dkv_pp_kernel<CAUSAL>), grid, dim3(512), 0, stream, p);
    return hipGetLastError();
}

template <class Pol, int KT, bool CAUSAL, int NW = 4>
static hipError_t launch_dkv_t(const Params &p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hkv * p.dkv_split, (p.N + 16 * KT * NW - 1) / (16 * KT * NW));
    hipLaunchKernelGGL((dkv_kernel<Pol, KT, CAUSAL, NW>), grid, dim3(64 * NW), 0, stream, p);
    return hipGetLastError();
}

// How many work-groups share the query heads of a key block's GQA group: the
// smallest divisor of the group that gives the launch at least two
// work-groups per resident slot (256 CUs x the kernel's work-groups per CU),
// else the whole group (one query head per work-group). 1 without GQA or when
// the key blocks alone fill the GPU twice over. A share's heads run one after
// another, so its causal key block 0 is the launch's critical path: at cfg5
// d = 128 (128 key blocks, 512 slots) 8 shares ran 144 us against 157 us for
// the 4 that one slot each would give.
template <class Pol, int KT, int NW = 4>
static int dkv_split_t(const Params &p) {
    if (p.group <= 1) return 1;
    constexpr int BKV = 16 * KT * NW;
    constexpr long long kSlots = 256LL * Pol::kWavesDkv;
    const long long base = (long long)p.B * p.Hkv * ((p.N + BKV - 1) / BKV);
    for (int s = 1; s < p.group; ++s) {
        if (p.group % s == 0 && base * s >= 2 * kSlots) return s;
    }
    return p.group;
}

int dkv_split(const Params &p, int dtype_bf16, int d) {
    if (dtype_bf16) {
        if (d == 64) return dkv_split_t<PolBF16<64>, 2>(p);
        if (d == 128) return dkv_split_t<PolBF16<128>, 1>(p);
    } else if (d == 64) {
        return dkv_split_t<PolF32<64>, 2>(p);
    }
    return 1;
}

template <class T>
static hipError_t launch_dkv_reduce(const Params &p, int d, hipStream_t stream) {
    const size_t n4 = (size_t)p.B * p.Hkv * p.N * (d / 4);
    const size_t blocks = std::min<size_t>((2 * n4 + 255) / 256, 4096);
    hipLaunchKernelGGL((dkv_reduce_kernel<T>), dim3((unsigned)blocks), dim3(256), 0, stream, p.dkv_ws,
                       static_cast<T *>(p.dk), static_cast<T *>(p.dv), n4, p.dkv_split, -p.scale);
    return hipGetLastError();
}

hipError_t launch_bwd_dkv(const Params &pin, int dtype_bf16, int d, int causal, hipStream_t stream) {
    // with a workspace, GQA shapes whose key blocks alone underfill the GPU
    // split each group's query heads over several work-groups
    Params p = pin;
    p.dkv_split = p.dkv_ws != nullptr ? dkv_split(p, dtype_bf16, d) : 1;
    if (p.dkv_split == 1) p.dkv_ws = nullptr;
    hipError_t e = hipErrorInvalidValue;
#define MXFA_DKV(POL, DD, KT)                                                                    \
    if (d == DD) e = causal ? launch_dkv_t<POL<DD>, KT, true>(p, stream)                         \
                            : launch_dkv_t<POL<DD>, KT, false>(p, stream);
    if (dtype_bf16) {
        if (d == 64 && p.dkv_split == 1 && dkv_pingpong_selected()) {
            return causal ? launch_dkv_pp<true>(p, stream) : launch_dkv_pp<false>(p, stream);
        }
        MXFA_DKV(PolBF16, 64, 2)
        else MXFA_DKV(PolBF16, 128, 1)
    } else {
        MXFA_DKV(PolF32, 64, 2)
    }
#undef MXFA_DKV
    if (e != hipSuccess || p.dkv_split == 1) return e;
    return dtype_bf16 ? launch_dkv_reduce<u16>(p, d, stream) : launch_dkv_reduce<float>(p, d, stream);
}

}  // namespace mxfa
