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
//     dK/dV accumulate in registers. Q/dO/LSE/Delta stream through
//     double-buffered LDS (direct global->LDS loads issued one stage ahead),
//     64 queries per stage, for every query head of the
//     KV head's group in turn, so the grouped-query reduction of dK/dV happens
//     inside the kernel with no atomics and no extra memory.
//   * dq_kernel: a workgroup owns 128 queries of one (batch, query head) (32
//     per wave, Q/dO rows in registers); K/V stream through LDS 64 keys per
//     stage. It recomputes S and dP (the price of staying atomic-free and O(N)
//     in memory).
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
template <class Pol>
__device__ __forceinline__ void stage_qdo(typename Pol::T *sq, typename Pol::T *sdo, float *sl, float *sd,
                                          const Params &p, size_t bh, int qs, int N, int tid, int wave,
                                          int lane) {
    using T = typename Pol::T;
    const size_t off = (bh * N + qs) * Pol::D;
    stage_rows<Pol>(sq, static_cast<const T *>(p.q) + off, N - qs, tid, wave);
    stage_rows<Pol>(sdo, static_cast<const T *>(p.dout) + off, N - qs, tid, wave);
    // rows past N: LSE = +inf makes their p (and so dS) exactly 0
    if (wave == 0) stage_vec64(sl, p.lse + bh * N + qs, N - qs, lane, &kPosInf);
    if (wave == 1) stage_vec64(sd, p.delta + bh * N + qs, N - qs, lane, p.delta + bh * N + qs);
}

// ------------------------------------------------------------------ dQ pass

// One 64-key stage of the dQ pass for one wave (32 queries). dof holds -dO and
// the dP accumulators start at Delta, so they come out as Delta - dP and the
// MFMAs accumulate -dQ / scale (the epilogue multiplies by -scale).
template <class Pol, bool CAUSAL, bool MASK>
__device__ __forceinline__ void dq_stage(f32x4 (&acc)[Pol::D / 16][2], const typename Pol::Frag (&qf)[2][Pol::NC],
                                         const typename Pol::Frag (&dof)[2][Pol::NC], const float (&L2)[2],
                                         const float (&Dl)[2], const typename Pol::T *sk,
                                         const typename Pol::T *sv, int k0, int q0, int N, float scale_log2,
                                         int g, int l16) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        f32x4 s[2][2], dp[2][2];  // [t][qt]
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            Frag a[NC];
            const int n = 32 * blk + Pol::arow(t, l16);
            Pol::lds_row_frags(a, sk, n, g);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f32x4 c = zero4();
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], qf[qt][kc], c);
                s[t][qt] = c;
            }
            Pol::lds_row_frags(a, sv, n, g);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                f32x4 c = f32x4{Dl[qt], Dl[qt], Dl[qt], Dl[qt]};
#pragma unroll
                for (int kc = 0; kc < NC; ++kc) c = Pol::mma(a[kc], dof[qt][kc], c);
                dp[t][qt] = c;
            }
        }
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) {
            const int qi = q0 + 16 * qt + l16;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float x = s[t][qt][r] * scale_log2 - L2[qt];
                    if constexpr (MASK) {
                        const int key = k0 + 32 * blk + Pol::bidx(t, g, r);
                        x = (key >= N || (CAUSAL && key > qi)) ? -INFINITY : x;
                    }
                    const float pv = fast_exp2(x);
                    s[t][qt][r] = pv * dp[t][qt][r];  // -dS / scale
                }
            }
        }
        typename Pol::ChainB cb[2];
#pragma unroll
        for (int qt = 0; qt < 2; ++qt) cb[qt] = Pol::pack(s[0][qt], s[1][qt]);
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) acc[xt][qt] = Pol::chain(acc[xt][qt], cb[qt], sk, 16 * xt, 32 * blk, g, l16);
        }
    }
}

template <class Pol, bool CAUSAL>
__global__ __launch_bounds__(256, Pol::kWaves) void dq_kernel(Params p) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int BQ = 128, BK = Pol::ROWS;

    __shared__ __attribute__((aligned(16))) T sK[2][BK * D];
    __shared__ __attribute__((aligned(16))) T sV[2][BK * D];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N;
    const int bh = blockIdx.x;
    const int nqb = (N + BQ - 1) / BQ;
    const int qb = CAUSAL ? (nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const T *Q = static_cast<const T *>(p.q) + (size_t)bh * N * D;
    const T *dO = static_cast<const T *>(p.dout) + (size_t)bh * N * D;
    const size_t kvoff = ((size_t)b * p.Hkv + kvh) * N * D;
    const T *K = static_cast<const T *>(p.k) + kvoff;
    const T *V = static_cast<const T *>(p.v) + kvoff;
    const int q0 = qb * BQ + wave * 32;

    Frag qf[2][NC], dof[2][NC];
    float L2[2], Dl[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        const bool ok = qi < N;
        Pol::gmem_row_frags(qf[qt], Q + (size_t)qi * D, g, ok);
        Pol::gmem_row_frags(dof[qt], dO + (size_t)qi * D, g, ok);
#pragma unroll
        for (int kc = 0; kc < NC; ++kc) dof[qt][kc] = Pol::neg(dof[qt][kc]);
        L2[qt] = ok ? p.lse[(size_t)bh * N + qi] * kLog2e : 0.f;
        Dl[qt] = ok ? p.delta[(size_t)bh * N + qi] : 0.f;
    }
    f32x4 acc[XT][2];
#pragma unroll
    for (int xt = 0; xt < XT; ++xt) acc[xt][0] = acc[xt][1] = zero4();

    const int kend = CAUSAL ? min(N, qb * BQ + BQ) : N;
    const int nsteps = (kend + BK - 1) / BK;

    stage_kv<Pol>(sK[0], sV[0], K, V, 0, N, tid, wave);
    wait_stage();
    __syncthreads();

    for (int st = 0; st < nsteps; ++st) {
        const int cur = st & 1;
        if (st + 1 < nsteps) stage_kv<Pol>(sK[cur ^ 1], sV[cur ^ 1], K, V, (st + 1) * BK, N, tid, wave);
        const int k0 = st * BK;
        if (!CAUSAL || k0 <= q0 + 31) {
            const bool need_mask = (k0 + BK > N) || (CAUSAL && k0 + BK - 1 > q0);
            if (need_mask) {
                dq_stage<Pol, CAUSAL, true>(acc, qf, dof, L2, Dl, sK[cur], sV[cur], k0, q0, N, p.scale_log2, g, l16);
            } else {
                dq_stage<Pol, CAUSAL, false>(acc, qf, dof, L2, Dl, sK[cur], sV[cur], k0, q0, N, p.scale_log2, g, l16);
            }
        }
        wait_stage();
        __syncthreads();
    }

    T *dQ = static_cast<T *>(p.dq) + (size_t)bh * N * D;
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int qi = q0 + 16 * qt + l16;
        if (qi < N) {
#pragma unroll
            for (int xt = 0; xt < XT; ++xt) store4<T>(dQ + (size_t)qi * D + 16 * xt + 4 * g, acc[xt][qt], -p.scale);
        }
    }
}

// ---------------------------------------------------------------- dK/dV pass

// One 64-query stage of the dK/dV pass for one wave (16*KT keys). vf holds -V
// and the dP accumulators start at Delta, so they come out as Delta - dP and
// accK accumulates -dK / scale (the epilogue multiplies by -scale).
template <class Pol, int KT, bool CAUSAL, bool MASK>
__device__ __forceinline__ void dkv_stage(f32x4 (&accK)[Pol::D / 16][KT], f32x4 (&accV)[Pol::D / 16][KT],
                                          const typename Pol::Frag (&kf)[KT][Pol::NC],
                                          const typename Pol::Frag (&vf)[KT][Pol::NC], const typename Pol::T *sq,
                                          const typename Pol::T *sdo, const float *sl, const float *sd, int qs,
                                          int kw0, int N, float scale_log2, int g, int l16) {
    using Frag = typename Pol::Frag;
    constexpr int NC = Pol::NC, XT = Pol::D / 16;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
        f32x4 s[2][KT], dp[2][KT];  // [t][kt]
        f32x4 L2[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            // block rows bidx(t, g, 0..3) are consecutive: one 16-byte LDS read
            const int q4 = 32 * blk + Pol::bidx(t, g, 0);
            L2[t] = *reinterpret_cast<const f32x4 *>(sl + q4) * kLog2e;
            const f32x4 dl = *reinterpret_cast<const f32x4 *>(sd + q4);
            Frag a[NC];
            const int n = 32 * blk + Pol::arow(t, l16);
            Pol::lds_row_frags(a, sq, n, g);
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                f32x4 c = zero4();
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
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
#pragma unroll
                for (int kt = 0; kt < KT; ++kt) {
                    float x = s[t][kt][r] * scale_log2 - L2[t][r];
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
#pragma unroll
        for (int xt = 0; xt < XT; ++xt) {
#pragma unroll
            for (int kt = 0; kt < KT; ++kt) {
                accV[xt][kt] = Pol::chain(accV[xt][kt], cp[kt], sdo, 16 * xt, 32 * blk, g, l16);
                accK[xt][kt] = Pol::chain(accK[xt][kt], cds[kt], sq, 16 * xt, 32 * blk, g, l16);
            }
        }
    }
}

template <class Pol, int KT, bool CAUSAL>
__global__ __launch_bounds__(256, Pol::kWavesDkv) void dkv_kernel(Params p) {
    using T = typename Pol::T;
    using Frag = typename Pol::Frag;
    constexpr int D = Pol::D, NC = Pol::NC, XT = D / 16;
    constexpr int BKV = 64 * KT;      // keys per workgroup
    constexpr int BQ = Pol::ROWS;     // queries per stage
    static_assert(BKV % BQ == 0, "causal start must align to a stage");

    // NBUF-deep ring of stages: loads are issued NBUF-1 stages ahead
    constexpr int NBUF = Pol::kDkvBuffers;
    __shared__ __attribute__((aligned(16))) T sQ[NBUF][BQ * D];
    __shared__ __attribute__((aligned(16))) T sdO[NBUF][BQ * D];
    __shared__ __attribute__((aligned(16))) float sL[NBUF][BQ];
    __shared__ __attribute__((aligned(16))) float sD[NBUF][BQ];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, l16 = lane & 15;
    const int N = p.N;
    const int bkv = blockIdx.x;  // b * Hkv + kvh
    const int kb = blockIdx.y;   // causal: block 0 (most queries) is dispatched first
    const int b = bkv / p.Hkv, kvh = bkv % p.Hkv;
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
        for (int kc = 0; kc < NC; ++kc) vf[kt][kc] = Pol::neg(vf[kt][kc]);
    }
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

    auto issue = [&](int st) __attribute__((always_inline)) {
        const int bf = st % NBUF;
        stage_qdo<Pol>(sQ[bf], sdO[bf], sL[bf], sD[bf], p, bh0 + st / nqs, qstart + (st % nqs) * BQ, N, tid,
                       wave, lane);
    };
    // loads of one stage per thread: the Q and dO tiles (+1 vector on waves
    // 0-1, which the waits below may over-wait by one load)
    constexpr int kLoads = 2 * tile_loads<Pol>();
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
    auto run = [&](auto mask_tag, int st) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int cur = st % NBUF;
        const bool ahead = st + NBUF - 1 < nsteps;
        if (ahead) issue(st + NBUF - 1);
        const int qs = qstart + (st % nqs) * BQ;
        // a wave whose keys all follow the stage's queries has nothing to do
        if (!CAUSAL || qs + BQ - 1 >= kw0) {
            dkv_stage<Pol, KT, CAUSAL, MASK>(accK, accV, kf, vf, sQ[cur], sdO[cur], sL[cur], sD[cur], qs, kw0, N,
                                             p.scale_log2, g, l16);
        }
        if (NBUF > 2 && ahead) {
            wait_vmcnt<kLoads>();
        } else {
            wait_stage();
        }
        barrier_lds();
    };
    // rows past N get p = 0 from LSE = +inf, so only the causal diagonal masks
    const int ndiag = CAUSAL ? min(nqs, BKV / BQ) : 0;
    for (int hh = 0, st = 0; hh < p.group; ++hh) {
        for (int i = 0; i < ndiag; ++i, ++st) run(std::true_type{}, st);
        for (int i = ndiag; i < nqs; ++i, ++st) run(std::false_type{}, st);
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
static hipError_t launch_dq_t(const Params &p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hq, (p.N + 127) / 128);
    hipLaunchKernelGGL((dq_kernel<Pol, CAUSAL>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd_dq(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream) {
#define MXFA_DQ(POL, DD)                                                        \
    if (d == DD) return causal ? launch_dq_t<POL<DD>, true>(p, stream)         \
                               : launch_dq_t<POL<DD>, false>(p, stream);
    if (dtype_bf16) {
        MXFA_DQ(PolBF16, 64)
        MXFA_DQ(PolBF16, 128)
    } else {
        MXFA_DQ(PolF32, 64)
    }
#undef MXFA_DQ
    return hipErrorInvalidValue;
}

template <class Pol, int KT, bool CAUSAL>
static hipError_t launch_dkv_t(const Params &p, hipStream_t stream) {
    const dim3 grid(p.B * p.Hkv, (p.N + 64 * KT - 1) / (64 * KT));
    hipLaunchKernelGGL((dkv_kernel<Pol, KT, CAUSAL>), grid, dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_bwd_dkv(const Params &p, int dtype_bf16, int d, int causal, hipStream_t stream) {
#define MXFA_DKV(POL, DD, KT)                                                          \
    if (d == DD) return causal ? launch_dkv_t<POL<DD>, KT, true>(p, stream)           \
                               : launch_dkv_t<POL<DD>, KT, false>(p, stream);
    if (dtype_bf16) {
        MXFA_DKV(PolBF16, 64, 2)
        MXFA_DKV(PolBF16, 128, 1)
    } else {
        MXFA_DKV(PolF32, 64, 2)
    }
#undef MXFA_DKV
    return hipErrorInvalidValue;
}

}  // namespace mxfa
