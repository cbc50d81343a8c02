// Device-side building blocks shared by the flash-attention kernels (gfx950).
//
// Tiling vocabulary used throughout:
//   * A "tile" is a 16x16 MFMA output. Lane l of a wave holds column l%16 and
//     rows 4*(l/16) + r, r = 0..3 (the C layout of every 16x16 MFMA).
//   * A "block" is 32 consecutive keys (or queries): the reduction depth of one
//     chained bf16 MFMA (16x16x32) or of eight fp32 MFMAs (16x16x4).
//   * The first GEMM of a chain (scores, dP) produces two 16-row tiles t = 0,1
//     per block. Its A-operand rows are permuted (Pol::arow) so that the lane
//     holding C element (t, r) of column c holds block row Pol::bidx(t, g, r),
//     g = l/16. For bf16 that puts rows 8g..8g+7 in one lane, which is exactly
//     one k-slice of the next MFMA: the scores feed the next GEMM (P*V, dS*K,
//     P^T*dO, dS^T*Q) straight from registers, no shuffle.
//   * "Row form" LDS tiles are [n][D] (rows = keys or queries), 16-byte chunks
//     XOR-swizzled per row. The bf16 chained GEMMs contract over n, so they also
//     stage a transposed "col form" tile [D][64] (chunks swizzled per row);
//     the fp32 chained GEMMs read the row form one element at a time.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxfa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16;

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct Params {
    const void *q, *k, *v, *dout, *o_in;
    void *o;
    float *lse, *delta;
    void *dq, *dk, *dv;
    int B, Hq, Hkv, N, group;
    float scale, scale_log2;
};

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Reductions across the four lane groups g = l/16 that share a column l%16
// (lanes l, l^16, l^32, l^48), with the gfx950 permlane swaps. Both results of
// a swap are combined, so every lane ends with the same value.
__device__ __forceinline__ float xg_max(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
__device__ __forceinline__ float xg_sum(float x) {
    auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ u16 to_bf16_bits(float x) {
    __bf16 h = (__bf16)x;
    return __builtin_bit_cast(u16, h);
}

// ------------------------------------------------------------------ policies

// bf16 inputs, fp32 accumulation: v_mfma_f32_16x16x32_bf16.
template <int D_>
struct PolBF16 {
    static constexpr int D = D_;
    using T = u16;
    using Frag = bf16x8;
    static constexpr int EPC = 8;      // elements per 16-byte chunk
    static constexpr int NC = D / 32;  // MFMAs over D per first-GEMM tile
    static constexpr bool kColForm = true;

    __device__ static __forceinline__ int arow(int t, int m) {
        return ((m >> 2) << 3) + (t << 2) + (m & 3);
    }
    __device__ static __forceinline__ int bidx(int t, int g, int r) { return (g << 3) + (t << 2) + r; }
    // row-form swizzle: the 8 rows one ds_read_b128 phase touches (arow of
    // m = 0..7 or 8..15) land in 8 distinct 16-byte bank groups
    __device__ static __forceinline__ int rswz(int n) { return (n & 3) | ((n >> 1) & 4); }
    __device__ static __forceinline__ int cswz(int y) { return (y ^ (y >> 3)) & 7; }

    __device__ static __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // k-slot (g, e) of MFMA c <-> element 32c + 8g + e of the row
    __device__ static __forceinline__ void lds_row_frags(Frag (&f)[NC], const T *tile, int n, int g) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const int chunk = 4 * c + g;
            f[c] = *reinterpret_cast<const Frag *>(tile + n * D + ((chunk ^ rswz(n)) * EPC));
        }
    }
    __device__ static __forceinline__ void gmem_row_frags(Frag (&f)[NC], const T *row, int g, bool valid) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (valid) {
                f[c] = *reinterpret_cast<const Frag *>(row + 32 * c + 8 * g);
            } else {
                f[c] = Frag{};
            }
        }
    }
    // acc += Other[y][blk .. blk+31] * chain, where chain element (t, r) of this
    // lane is block row bidx(t, g, r) and Other comes from the col-form tile.
    __device__ static __forceinline__ f32x4 chain(f32x4 acc, const f32x4 &c0, const f32x4 &c1,
                                                  const T *col_tile, int y, int blk, int g) {
        Frag b;
        b[0] = (__bf16)c0[0];
        b[1] = (__bf16)c0[1];
        b[2] = (__bf16)c0[2];
        b[3] = (__bf16)c0[3];
        b[4] = (__bf16)c1[0];
        b[5] = (__bf16)c1[1];
        b[6] = (__bf16)c1[2];
        b[7] = (__bf16)c1[3];
        const int chunk = (blk >> 3) + g;
        const Frag a = *reinterpret_cast<const Frag *>(col_tile + y * 64 + ((chunk ^ cswz(y)) * EPC));
        return mma(a, b, acc);
    }
};

// fp32 parity path: v_mfma_f32_16x16x4_f32.
template <int D_>
struct PolF32 {
    static constexpr int D = D_;
    using T = float;
    using Frag = float;
    static constexpr int EPC = 4;
    static constexpr int NC = D / 4;
    static constexpr bool kColForm = false;

    __device__ static __forceinline__ int arow(int t, int m) { return (t << 4) + m; }
    __device__ static __forceinline__ int bidx(int t, int g, int r) { return (t << 4) + (g << 2) + r; }
    __device__ static __forceinline__ int rswz(int n) { return n & 7; }
    __device__ static __forceinline__ int cswz(int) { return 0; }

    __device__ static __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
    }
    // k-slot g of MFMA s <-> element (D/4)*g + s of the row
    __device__ static __forceinline__ void lds_row_frags(Frag (&f)[NC], const T *tile, int n, int g) {
#pragma unroll
        for (int i = 0; i < NC / 4; ++i) {
            const int chunk = (NC / 4) * g + i;
            const float4 v = *reinterpret_cast<const float4 *>(tile + n * D + ((chunk ^ rswz(n)) * EPC));
            f[4 * i + 0] = v.x;
            f[4 * i + 1] = v.y;
            f[4 * i + 2] = v.z;
            f[4 * i + 3] = v.w;
        }
    }
    __device__ static __forceinline__ void gmem_row_frags(Frag (&f)[NC], const T *row, int g, bool valid) {
#pragma unroll
        for (int i = 0; i < NC / 4; ++i) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (valid) v = *reinterpret_cast<const float4 *>(row + NC * g + 4 * i);
            f[4 * i + 0] = v.x;
            f[4 * i + 1] = v.y;
            f[4 * i + 2] = v.z;
            f[4 * i + 3] = v.w;
        }
    }
    // Other comes from the row-form tile [n][D]: the k-slot g of MFMA (t, r) is
    // block row 16t + 4g + r, matching the C layout of the chain tiles.
    __device__ static __forceinline__ f32x4 chain(f32x4 acc, const f32x4 &c0, const f32x4 &c1,
                                                  const T *row_tile, int y, int blk, int g) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = blk + (t << 4) + (g << 2) + r;
                const float a = row_tile[n * D + (((y >> 2) ^ rswz(n)) << 2) + (y & 3)];
                acc = mma(a, t ? c1[r] : c0[r], acc);
            }
        }
        return acc;
    }
};

// --------------------------------------------------------------- LDS staging

// One "stage block": 8 consecutive rows x one 16-byte chunk of a 64 x D tile.
// Block b of a tile covers rows 8*(b / CPR) .. +7 and chunk b % CPR, CPR = D /
// EPC chunks per row, so 8 (bf16) or 16 (fp32) consecutive threads read whole
// rows (coalesced).
template <class Pol>
struct StageBlock {
    static constexpr int CPR = Pol::D / Pol::EPC;
    static constexpr int PER_TILE = 8 * CPR;
    uint4 r[8];

    __device__ __forceinline__ void load(const typename Pol::T *src, int nvalid, int b) {
        const int cb = b % CPR, rb = b / CPR;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int row = 8 * rb + e;
            if (row < nvalid) {
                r[e] = *reinterpret_cast<const uint4 *>(src + (size_t)row * Pol::D + cb * Pol::EPC);
            } else {
                r[e] = make_uint4(0u, 0u, 0u, 0u);
            }
        }
    }
    __device__ __forceinline__ void store_row(typename Pol::T *tile, int b) const {
        const int cb = b % CPR, rb = b / CPR;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int n = 8 * rb + e;
            *reinterpret_cast<uint4 *>(tile + n * Pol::D + ((cb ^ Pol::rswz(n)) * Pol::EPC)) = r[e];
        }
    }
    // bf16 only: transpose the 8x8 block in registers and write it to the
    // col-form tile [D][64]: row y = 8*cb + c holds column c of the block at
    // chunk rb.
    __device__ __forceinline__ void store_col(typename Pol::T *ctile, int b) const {
        const int cb = b % CPR, rb = b / CPR;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int word = c >> 1;
            uint32_t out[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = reinterpret_cast<const uint32_t *>(&r[2 * k])[word];
                const uint32_t hi = reinterpret_cast<const uint32_t *>(&r[2 * k + 1])[word];
                out[k] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
            }
            const int y = 8 * cb + c;
            *reinterpret_cast<uint4 *>(ctile + y * 64 + ((rb ^ Pol::cswz(y)) * 8)) =
                make_uint4(out[0], out[1], out[2], out[3]);
        }
    }
};

// Store four consecutive elements x0..x0+3 of one output row.
template <class T>
__device__ __forceinline__ void store4(T *dst, f32x4 v, float mul);

template <>
__device__ __forceinline__ void store4<float>(float *dst, f32x4 v, float mul) {
    *reinterpret_cast<float4 *>(dst) = make_float4(v[0] * mul, v[1] * mul, v[2] * mul, v[3] * mul);
}
template <>
__device__ __forceinline__ void store4<u16>(u16 *dst, f32x4 v, float mul) {
    const uint32_t a = (uint32_t)to_bf16_bits(v[0] * mul) | ((uint32_t)to_bf16_bits(v[1] * mul) << 16);
    const uint32_t b = (uint32_t)to_bf16_bits(v[2] * mul) | ((uint32_t)to_bf16_bits(v[3] * mul) << 16);
    *reinterpret_cast<uint2 *>(dst) = make_uint2(a, b);
}

}  // namespace mxfa
