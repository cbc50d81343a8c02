// Roofline probes: the measured ceilings of the MI355X pipes the flash-attention
// kernels run on, reported next to AMD's published peaks.
//
// They follow the idea of the reference's instruction-throughput audit
// (common/kernels/isa.cu:11-63 and common/examples/isa.rs:17-88: every thread
// runs several independent chains of the instruction under test, and the
// accumulators are written out so nothing is eliminated), re-targeted at what
// bounds this path on CDNA4: the bf16 and fp32 MFMA pipes and HBM streaming.
#include "fa_device.h"
#include "fa_launch.h"

namespace mxfa {

namespace {

constexpr int kProbeBlocks = 2048;  // 8 per CU: up to 8 waves per SIMD
constexpr int kProbeThreads = 256;
constexpr int kChains = 8;          // independent accumulators per wave

// Each wave issues iters x kChains MFMAs whose accumulators do not depend on
// each other, so the matrix pipe, not the dependent-issue latency, is the limit.
template <bool BF16>
__device__ __forceinline__ void probe_mfma_body(float *sink, int iters) {
    const int tid = threadIdx.x;
    f32x4 acc[kChains];
#pragma unroll
    for (int j = 0; j < kChains; ++j) acc[j] = zero4();
    // the loop body is kUnroll x kChains MFMAs and nothing else (checked in the
    // ISA): the accumulators stay in place across iterations
    constexpr int kUnroll = 4;
    const int outer = (iters + kUnroll - 1) / kUnroll;
    if constexpr (BF16) {
        bf16x8 a, b;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            a[e] = (__bf16)(0.001f * (float)((tid + e) & 7));
            b[e] = (__bf16)(0.002f * (float)((tid ^ e) & 7));
        }
        // (asm: with the builtin the compiler rotates the accumulators through
        // AGPRs, 56 moves per 32 MFMAs; here they stay in their VGPRs. A and B
        // are loop-invariant and each accumulator recurs every kChains MFMAs.)
        for (int i = 0; i < outer; ++i) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
                for (int j = 0; j < kChains; ++j)
                    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc[j]) : "v"(a), "v"(b));
            }
        }
        asm volatile("s_nop 7\n\ts_nop 7" ::: "memory");  // results settle before the VALU reads them
    } else {
        const float a = 0.001f * (float)(tid & 7), b = 0.002f * (float)((tid >> 3) & 7);
        for (int i = 0; i < outer; ++i) {
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
                for (int j = 0; j < kChains; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[j], 0, 0, 0);
            }
        }
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kChains; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    sink[blockIdx.x * kProbeThreads + tid] = s;
}

// The same for v_mfma_f32_32x32x16_bf16 (the other bf16 MFMA shape):
// 4 independent 16-register accumulators per wave.
constexpr int kChains32 = 4;
[[maybe_unused]] __device__ __forceinline__ void probe_mfma32_body(float *sink, int iters) {
    const int tid = threadIdx.x;
    f32x16 acc[kChains32];
#pragma unroll
    for (int j = 0; j < kChains32; ++j) acc[j] = f32x16{};
    constexpr int kUnroll = 4;
    const int outer = (iters + kUnroll - 1) / kUnroll;
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(0.001f * (float)((tid + e) & 7));
        b[e] = (__bf16)(0.002f * (float)((tid ^ e) & 7));
    }
    for (int i = 0; i < outer; ++i) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
#pragma unroll
            for (int j = 0; j < kChains32; ++j)
                asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc[j]) : "v"(a), "v"(b));
        }
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");  // results settle before the VALU reads them
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kChains32; ++j) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[j][r];
    }
    sink[blockIdx.x * kProbeThreads + tid] = s;
}

// Streaming read of n16 16-byte vectors, grid-stride (the stream_f4 shape).
[[maybe_unused]] __device__ __forceinline__ void probe_read_body(const float4 *x, size_t n16, float *sink) {
    float s = 0.f;
    for (size_t i = (size_t)blockIdx.x * kProbeThreads + threadIdx.x; i < n16; i += (size_t)gridDim.x * kProbeThreads) {
        const float4 v = x[i];
        s += v.x + v.y + v.z + v.w;
    }
    sink[blockIdx.x * kProbeThreads + threadIdx.x] = s;
}

// Streaming copy of n16 16-byte vectors, grid-stride.
[[maybe_unused]] __device__ __forceinline__ void probe_copy_body(const float4 *x, float4 *y, size_t n16) {
    for (size_t i = (size_t)blockIdx.x * kProbeThreads + threadIdx.x; i < n16; i += (size_t)gridDim.x * kProbeThreads)
        y[i] = x[i];
}

// The global writes of a dQ pass fused into the dK/dV pass, causal, d = 64:
// work-group (head, key block kb of 128 keys) adds one 64 x 64 fp32 partial
// tile per 64-query stage from its diagonal stage 2 kb to the last, each wave
// a quarter of the tile (16 lane-contiguous rows of 64 floats). ATOMIC: fp32
// atomic adds of 1 (no return); else plain stores of the same bytes.
// Key block 0 (the most stages) is dispatched first, as in the dK/dV pass.
template <bool ATOMIC>
__device__ __forceinline__ void probe_dq_atomic_body(float *acc, int n) {
    const int h = blockIdx.x, kb = blockIdx.y;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int nqs = n / 64;
    float *base = acc + (size_t)h * n * 64 + wave * 1024 + lane;
    for (int i = 2 * kb; i < nqs; ++i) {
        float *tile = base + (size_t)i * 64 * 64;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            if constexpr (ATOMIC) {
                atomicAdd(tile + j * 64, 1.0f);
            } else {
                tile[j * 64] = (float)i;
            }
        }
    }
}

}  // namespace

// The code object's probe kernels (fa_kernels.h).
#if defined(__HIP_DEVICE_COMPILE__)
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_mfma_bf16(float *sink, int iters) {
    probe_mfma_body<true>(sink, iters);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_mfma_f32(float *sink, int iters) {
    probe_mfma_body<false>(sink, iters);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_mfma32_bf16(float *sink, int iters) {
    probe_mfma32_body(sink, iters);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_read_f4(const float4 *x, size_t n16, float *sink) {
    probe_read_body(x, n16, sink);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_copy_f4(const float4 *x, float4 *y, size_t n16) {
    probe_copy_body(x, y, n16);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_dq_atomic_add(float *acc, int n) {
    probe_dq_atomic_body<true>(acc, n);
}
extern "C" __global__ __launch_bounds__(256) void mxfa_probe_dq_atomic_store(float *acc, int n) {
    probe_dq_atomic_body<false>(acc, n);
}
#endif

int probe_sink_len() { return kProbeBlocks * kProbeThreads; }

double probe_dq_atomic_bytes(int bh, int n) {
    const long long nqs = n / 64, nkb = n / 128;
    long long tiles = 0;
    for (long long kb = 0; kb < nkb; ++kb) tiles += nqs - 2 * kb;
    return (double)bh * (double)tiles * 64.0 * 64.0 * 4.0;
}

hipError_t launch_probe_dq_atomic(float *acc, int bh, int n, int atomic, hipStream_t stream) {
    const dim3 grid(bh, n / 128);
    void *args[] = {&acc, &n};
    return launch_kernel(atomic ? k_mxfa_probe_dq_atomic_add : k_mxfa_probe_dq_atomic_store, grid,
                         dim3(kProbeThreads), args, stream);
}

double probe_mfma_flops(int bf16, int iters) {
    const double per_mfma = bf16 ? 2.0 * 16 * 16 * 32 : 2.0 * 16 * 16 * 4;
    const double waves = (double)kProbeBlocks * (kProbeThreads / 64);
    const int rounded = (iters + 3) / 4 * 4;  // the kernel runs whole unrolled rounds of 4
    return waves * (double)rounded * kChains * per_mfma;
}

hipError_t launch_probe_mfma(int bf16, int iters, float *sink, hipStream_t stream) {
    void *args[] = {&sink, &iters};
    return launch_kernel(bf16 ? k_mxfa_probe_mfma_bf16 : k_mxfa_probe_mfma_f32, dim3(kProbeBlocks),
                         dim3(kProbeThreads), args, stream);
}

double probe_mfma32_flops(int iters) {
    const double waves = (double)kProbeBlocks * (kProbeThreads / 64);
    const int rounded = (iters + 3) / 4 * 4;
    return waves * (double)rounded * kChains32 * (2.0 * 32 * 32 * 16);
}

hipError_t launch_probe_mfma32(int iters, float *sink, hipStream_t stream) {
    void *args[] = {&sink, &iters};
    return launch_kernel(k_mxfa_probe_mfma32_bf16, dim3(kProbeBlocks), dim3(kProbeThreads), args, stream);
}

hipError_t launch_probe_read(const void *x, size_t bytes, float *sink, hipStream_t stream) {
    size_t n16 = bytes / 16;
    void *args[] = {&x, &n16, &sink};
    return launch_kernel(k_mxfa_probe_read_f4, dim3(kProbeBlocks), dim3(kProbeThreads), args, stream);
}

hipError_t launch_probe_copy(const void *x, void *y, size_t bytes, hipStream_t stream) {
    size_t n16 = bytes / 16;
    void *args[] = {&x, &y, &n16};
    return launch_kernel(k_mxfa_probe_copy_f4, dim3(kProbeBlocks), dim3(kProbeThreads), args, stream);
}

}  // namespace mxfa
