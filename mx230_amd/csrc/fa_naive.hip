// Naive fp32 baselines, kept for the naive-vs-flash comparison the reference
// reports (02-flash-attention/README.md:12-21, 81-87). Deliberately simple:
//   * forward materialises the B*Hq x N x N score matrix
//     (attention_naive.cu:8-70: scores, in-place row softmax, S*V);
//   * backward is one thread per query row with dK/dV scattered by atomic adds
//     (attention_bwd.cu:48-90); with GQA the atomics also sum over the query
//     heads of a group. Outputs must be zeroed by the caller.
#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

// S[bh][i][j] = scale * q_i . k_j, -inf above the diagonal when causal.
template <int D>
__device__ __forceinline__ void naive_scores_body(const Params &p, float *S, int causal) {
    const int j = blockIdx.x * 16 + threadIdx.x;
    const int i = blockIdx.y * 16 + threadIdx.y;
    const int bh = blockIdx.z;
    const int N = p.N;
    if (i >= N || j >= N) return;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const float *q = static_cast<const float *>(p.q) + ((size_t)bh * N + i) * D;
    const float *k = static_cast<const float *>(p.k) + (((size_t)b * p.Hkv + kvh) * N + j) * D;
    float acc = 0.f;
#pragma unroll 8
    for (int x = 0; x < D; ++x) acc += q[x] * k[x];
    S[((size_t)bh * N + i) * N + j] = (causal && j > i) ? -INFINITY : acc * p.scale;
}

// In-place softmax of one row per workgroup (256 threads).
__device__ __forceinline__ void naive_softmax_body(float *S, int N) {
    __shared__ float red[256];
    float *row = S + ((size_t)blockIdx.y * N + blockIdx.x) * N;
    const int t = threadIdx.x;
    float m = -INFINITY;
    for (int j = t; j < N; j += 256) m = fmaxf(m, row[j]);
    red[t] = m;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] = fmaxf(red[t], red[t + w]);
        __syncthreads();
    }
    m = red[0];
    __syncthreads();
    float l = 0.f;
    for (int j = t; j < N; j += 256) {
        const float e = fast_exp2((row[j] - m) * kLog2e);
        row[j] = e;
        l += e;
    }
    red[t] = l;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] += red[t + w];
        __syncthreads();
    }
    const float inv = 1.0f / red[0];
    for (int j = t; j < N; j += 256) row[j] *= inv;
}

// O[bh][i][x] = sum_j S[bh][i][j] V[j][x]; block (D, 4) covers 4 rows.
template <int D>
__device__ __forceinline__ void naive_av_body(const Params &p, const float *S) {
    const int x = threadIdx.x;
    const int i = blockIdx.x * 4 + threadIdx.y;
    const int bh = blockIdx.y;
    const int N = p.N;
    if (i >= N) return;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const float *v = static_cast<const float *>(p.v) + ((size_t)b * p.Hkv + kvh) * N * D;
    const float *s = S + ((size_t)bh * N + i) * N;
    float acc = 0.f;
    for (int j = 0; j < N; ++j) acc += s[j] * v[(size_t)j * D + x];
    static_cast<float *>(p.o)[((size_t)bh * N + i) * D + x] = acc;
}

template <int D>
__device__ __forceinline__ void naive_bwd_body(const Params &p, int causal) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const int bh = blockIdx.y;
    const int N = p.N;
    if (i >= N) return;
    const int b = bh / p.Hq, h = bh % p.Hq, kvh = h / p.group;
    const size_t qoff = ((size_t)bh * N + i) * D;
    const size_t kvoff = ((size_t)b * p.Hkv + kvh) * N * D;
    const float *Q = static_cast<const float *>(p.q), *dO = static_cast<const float *>(p.dout);
    const float *K = static_cast<const float *>(p.k) + kvoff, *V = static_cast<const float *>(p.v) + kvoff;
    float *dK = static_cast<float *>(p.dk) + kvoff, *dV = static_cast<float *>(p.dv) + kvoff;
    float q[D], doi[D], dq[D];
#pragma unroll
    for (int x = 0; x < D; ++x) {
        q[x] = Q[qoff + x];
        doi[x] = dO[qoff + x];
        dq[x] = 0.f;
    }
    const float L2 = p.lse[(size_t)bh * N + i] * kLog2e;
    const float Di = p.delta[(size_t)bh * N + i];
    const int jmax = causal ? i : N - 1;
    for (int j = 0; j <= jmax; ++j) {
        const float *kj = K + (size_t)j * D, *vj = V + (size_t)j * D;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int x = 0; x < D; ++x) {
            s += q[x] * kj[x];
            dp += doi[x] * vj[x];
        }
        const float pv = fast_exp2(s * p.scale_log2 - L2);
        const float ds = pv * (dp - Di) * p.scale;
#pragma unroll
        for (int x = 0; x < D; ++x) {
            atomicAdd(&dV[(size_t)j * D + x], pv * doi[x]);
            atomicAdd(&dK[(size_t)j * D + x], ds * q[x]);
            dq[x] += ds * kj[x];
        }
    }
    float *dQ = static_cast<float *>(p.dq) + qoff;
#pragma unroll
    for (int x = 0; x < D; ++x) dQ[x] = dq[x];
}

// The code object's naive kernels (fa_kernels.h), d = 64.
#if defined(__HIP_DEVICE_COMPILE__)
extern "C" __global__ __launch_bounds__(256) void mxfa_naive_scores(Params p, float *S, int causal) {
    naive_scores_body<64>(p, S, causal);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_naive_softmax(float *S, int N) { naive_softmax_body(S, N); }
extern "C" __global__ __launch_bounds__(256) void mxfa_naive_av(Params p, const float *S) { naive_av_body<64>(p, S); }
extern "C" __global__ __launch_bounds__(256) void mxfa_naive_bwd(Params p, int causal) {
    naive_bwd_body<64>(p, causal);
}
#endif

hipError_t launch_naive_fwd(const Params &pin, float *S, int d, int causal, hipStream_t stream) {
    if (d != 64) return hipErrorInvalidValue;
    Params p = pin;
    int N = p.N;
    const unsigned BH = (unsigned)(p.B * p.Hq);
    const unsigned t16 = (unsigned)((p.N + 15) / 16);
    void *sargs[] = {&p, &S, &causal};
    hipError_t e = launch_kernel(k_mxfa_naive_scores, dim3(t16, t16, BH), dim3(16, 16), sargs, stream);
    if (e != hipSuccess) return e;
    void *margs[] = {&S, &N};
    e = launch_kernel(k_mxfa_naive_softmax, dim3((unsigned)p.N, BH), dim3(256), margs, stream);
    if (e != hipSuccess) return e;
    const float *Sc = S;
    void *aargs[] = {&p, &Sc};
    return launch_kernel(k_mxfa_naive_av, dim3((unsigned)((p.N + 3) / 4), BH), dim3(64, 4), aargs, stream);
}

hipError_t launch_bwd_naive(const Params &pin, int d, int causal, hipStream_t stream) {
    if (d != 64) return hipErrorInvalidValue;
    Params p = pin;
    const dim3 grid((unsigned)((p.N + 255) / 256), (unsigned)(p.B * p.Hq));
    void *args[] = {&p, &causal};
    return launch_kernel(k_mxfa_naive_bwd, grid, dim3(256), args, stream);
}

}  // namespace mxfa
