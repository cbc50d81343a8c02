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

// Instruction-mix ceilings: how fast a SIMD issues the instruction mix of a
// flash-attention kernel when nothing in it waits on anything else. Each
// iteration is 32 v_mfma_f32_16x16x32_bf16 on 8 independent accumulators,
// with E v_exp_f32, M v_mul_f32, C v_cvt_pk_bf16_f32, B ds_read_b128 and
// R ds_read_b64_tr_b16 spread evenly over them (instruction j of a kind with
// count K after MFMA floor(32 j / K)); every 4 MFMAs the wave waits for the
// LDS reads issued 4 MFMAs earlier, so at most one group's reads are in
// flight. The counts replay the per-MFMA counts rocprofv3 measures for the
// kernels (SQ_INSTS_VALU, SQ_INSTS_VALU_TRANS_F32, SQ_INSTS_LDS,
// SQ_INSTS_MFMA), so a kernel's MFMA rate over its mix's rate is the share
// of its instruction-issue ceiling that it reaches. The destinations are
// read-write operands (each its own registers, kept live across the loop), so
// the compiler does not fold the results of one kind into shared registers.
constexpr int kMixSlots = 32;

__device__ __forceinline__ constexpr int mix_first(int count, int slot) {
    return (slot * count + kMixSlots - 1) / kMixSlots;  // first j with 32 j / count >= slot
}
[[maybe_unused]] __device__ __forceinline__ constexpr int mix_reads(int b, int r, int s0, int s1) {
    return mix_first(b, s1) - mix_first(b, s0) + mix_first(r, s1) - mix_first(r, s0);
}

// BIG: the same flops as 16 v_mfma_f32_32x32x16_bf16 per round (one on
// every other slot, 4 independent accumulators), with the same other
// instructions: whether the larger MFMA shape, which issues half as many MFMA
// instructions for the work, raises a mix's ceiling.
template <int E, int M, int C, int B, int R, bool BIG = false>
__device__ __forceinline__ void probe_mix_body(float *sink, int iters) {
    __shared__ __attribute__((aligned(16))) float lds[4096];  // 16 KB
    const int tid = threadIdx.x, lane = tid & 63;
    for (int i = tid; i < 4096; i += kProbeThreads) lds[i] = 0.001f * (float)(i & 255);
    __syncthreads();
    f32x4 acc[8];
    f32x16 acc32[4];
    float xe[8], xm[8];
    uint32_t u[4];
    f32x4 rb[4];
    double rt[4];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        acc[j] = zero4();
        xe[j] = 0.001f * (float)(tid + j);
        xm[j] = 1.0f + 0.001f * (float)(tid ^ j);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        u[j] = 0;
        rb[j] = zero4();
        rt[j] = 0.0;
#pragma unroll
        for (int e = 0; e < 16; ++e) acc32[j][e] = 0.f;
    }
    bf16x8 a, b;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        a[e] = (__bf16)(0.001f * (float)((tid + e) & 7));
        b[e] = (__bf16)(0.002f * (float)((tid ^ e) & 7));
    }
    // byte address of this lane's 16 bytes in the first 1 KB (in bounds: the
    // largest read ends at 8 KB)
    const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)lds + 16u * lane;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int s = 0; s < kMixSlots; ++s) {
            if constexpr (BIG) {
                if (s % 2 == 0)
                    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc32[(s / 2) & 3]) : "v"(a), "v"(b));
            } else {
                asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc[s & 7]) : "v"(a), "v"(b));
            }
#pragma unroll
            for (int j = mix_first(E, s); j < mix_first(E, s + 1); ++j) asm volatile("v_exp_f32 %0, %0" : "+v"(xe[j & 7]));
#pragma unroll
            for (int j = mix_first(M, s); j < mix_first(M, s + 1); ++j)
                asm volatile("v_mul_f32 %0, %0, %1" : "+v"(xm[j & 7]) : "v"(xm[(j + 4) & 7]));
#pragma unroll
            for (int j = mix_first(C, s); j < mix_first(C, s + 1); ++j)
                asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "+v"(u[j & 3]) : "v"(xe[(j + 1) & 7]), "v"(xm[(j + 2) & 7]));
#pragma unroll
            for (int j = mix_first(B, s); j < mix_first(B, s + 1); ++j)
                asm volatile("ds_read_b128 %0, %1 offset:%2" : "+v"(rb[j & 3]) : "v"(la), "i"((j & 3) * 1024));
#pragma unroll
            for (int j = mix_first(R, s); j < mix_first(R, s + 1); ++j)
                asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "+v"(rt[j & 3]) : "v"(la), "i"(4096 + (j & 3) * 1024));
            if (s % 4 == 3) {
                // the reads of this group of 4 MFMAs may stay in flight
                const int n = mix_reads(B, R, s - 3, s + 1);
                asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(n < 15 ? n : 15) : "memory");
            }
        }
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_waitcnt lgkmcnt(0)" ::: "memory");
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) sum += acc[j][0] + xe[j] + xm[j];
#pragma unroll
    for (int j = 0; j < 4; ++j) sum += (float)u[j] + rb[j][0] + (float)rt[j] + acc32[j][0];
    sink[blockIdx.x * kProbeThreads + tid] = sum;
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
// instruction mixes (counts per 32 MFMAs; the rows of MXFA_PROBE_MIX_* in
// mxfa_probes.h)
#define MXFA_MIX(NAME, E, M, C, B, R, BIG)                                                                  \
    extern "C" __global__ __launch_bounds__(256) void NAME(float *sink, int iters) {                        \
        probe_mix_body<E, M, C, B, R, BIG>(sink, iters);                                                    \
    }
MXFA_MIX(mxfa_probe_mix_mfma, 0, 0, 0, 0, 0, false)
MXFA_MIX(mxfa_probe_mix_dkv, 16, 48, 16, 12, 16, false)
MXFA_MIX(mxfa_probe_mix_dkv_valu, 16, 48, 16, 0, 0, false)
MXFA_MIX(mxfa_probe_mix_dkv_lds, 0, 0, 0, 12, 16, false)
MXFA_MIX(mxfa_probe_mix_dq, 21, 60, 11, 10, 11, false)
MXFA_MIX(mxfa_probe_mix_fwd, 32, 106, 16, 8, 16, false)
MXFA_MIX(mxfa_probe_mix32_mfma, 0, 0, 0, 0, 0, true)
MXFA_MIX(mxfa_probe_mix32_dkv, 16, 48, 16, 12, 16, true)
MXFA_MIX(mxfa_probe_mix32_dq, 21, 60, 11, 10, 11, true)
MXFA_MIX(mxfa_probe_mix32_fwd, 32, 106, 16, 8, 16, true)
#undef MXFA_MIX
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

static const KernelId kMixKernels[] = {k_mxfa_probe_mix_mfma,    k_mxfa_probe_mix_dkv,     k_mxfa_probe_mix_dkv_valu,
                                       k_mxfa_probe_mix_dkv_lds, k_mxfa_probe_mix_dq,      k_mxfa_probe_mix_fwd,
                                       k_mxfa_probe_mix32_mfma,  k_mxfa_probe_mix32_dkv,   k_mxfa_probe_mix32_dq,
                                       k_mxfa_probe_mix32_fwd};

int probe_mix_count() { return (int)(sizeof(kMixKernels) / sizeof(kMixKernels[0])); }

// One work-group (4 waves, one per SIMD) per CU per wave of occupancy.
double probe_mix_flops(int waves_per_simd, int iters) {
    return 256.0 * waves_per_simd * 4.0 * (double)iters * kMixSlots * (2.0 * 16 * 16 * 32);
}

hipError_t launch_probe_mix(int mix, int waves_per_simd, int iters, float *sink, hipStream_t stream) {
    if (mix < 0 || mix >= probe_mix_count() || waves_per_simd < 1 || waves_per_simd > kProbeBlocks / 256)
        return hipErrorInvalidValue;
    void *args[] = {&sink, &iters};
    return launch_kernel(kMixKernels[mix], dim3(256 * waves_per_simd), dim3(kProbeThreads), args, stream);
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
