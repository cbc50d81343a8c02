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
//   * LDS tiles are row form, [n][D] (rows = keys or queries), with 16-byte
//     chunks XOR-swizzled per row. The chained GEMMs contract over n: bf16 reads
//     their operand transposed with ds_read_b64_tr_b16, fp32 reads it one
//     element at a time.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxfa {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
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
    // Forward layout, in elements: batch, head and row strides of Q and O and
    // of K/V, the number of key rows, and the causal offset (query row i sits
    // at position pos0 + i and sees keys 0..pos0 + i). The packed training
    // layout [B][H][N][d] has Nk = N and pos0 = 0; the backward and naive
    // kernels assume it.
    long long q_bs, q_hs, kv_bs, kv_hs, o_bs, o_hs;
    int q_rs, kv_rs, o_rs, Nk, pos0;
    // Paged K/V (the prefill over a block-table cache): with block_table set,
    // key row t of K and V is cache row (block_table[t >> bs_shift] <<
    // bs_shift) + (t & (2^bs_shift - 1)), counted in rows of kv_rs elements
    // from the K/V base of the head; null: cache row t.
    const int *block_table;
    int bs_shift;
    // Split forward (fwd_entry<..., SPLIT>, the prefill with a workspace):
    // per split s and row r of the B*Hq*N query rows, the unnormalised O at
    // fwd_part[(s rows + r) D], then (running max in log2 units, sum) at
    // fwd_part[S rows D + 2 (s rows + r)].
    float *fwd_part;
    // dK/dV pass with dkv_split > 1: the group's query heads' stages of a
    // key block (group x its stages per head, in head order) are split into
    // dkv_block_shares(...) contiguous runs, one work-group each; share s
    // writes fp32 partial sums to plane s of dkv_ws ([dkv_split][B*Hkv][N][d]
    // for dK, then the same for dV; dkv_split = the most shares of any block)
    // and each block's planes are added in share order, by a reduce launch
    // or by the one-launch backward's last work-groups (red_rows below).
    float *dkv_ws;
    int dkv_split, dkv_min_shares, dkv_share_stages;
    // One-launch backward (bwd_fused_entry, kernels mxfa_bwd_*): work-groups [0, fused_ndq) run
    // the dQ pass and publish Delta per 128-row query block with flag value
    // epoch in slot flag_slot of g_delta_flags; the rest run the dK/dV pass
    // and wait for those flags, at most delta_wait ticks of the 100 MHz
    // real-time counter per block, then compute Delta themselves
    // (delta_wait < 0: always compute it).
    unsigned epoch;
    int flag_slot, delta_wait, fused_ndq;
    // Causal work order of a launch whose first work-groups are resident at
    // once (cu_order_wg): runs of cu_run linear work-group indices, every
    // other one of the first cu_runs reversed; cu_runs < 2: the kernel's own.
    int cu_run, cu_runs;
    // One-launch backward: work-groups [fused_ndq, fused_ndq + fused_ndkv)
    // run the dK/dV pass. With a GQA split and red_rows > 0 the shares write
    // their planes through to memory and then set their flag, share_flags[w]
    // (dkv_work's index w; in the launch's workspace, after the planes), to
    // share_nonce, a 64-bit value no other launch of the process uses; the
    // work-groups after them each add the planes of red_rows keys of one key
    // block (dkv_reduce_rows) once its shares' flags hold the nonce, polling
    // at most red_wait ticks; red_rows = 0: a reduce launch follows instead.
    int fused_ndkv, red_rows, red_wait;
    unsigned long long *share_flags;
    unsigned long long share_nonce;
    // A prefill launch (contiguous or paged cache): the tiles are chosen as
    // the paged cache's kernels allow, so both give the same bits.
    int prefill;
};

// Where a launch's first work-groups are resident at once, the dispatcher
// gives work-group i (linear index, x fastest) to XCD i mod 8, and each XCD
// deals its work-groups round robin over its CUs, so with C CUs i and i + C
// land on the same CU (seen in the timeline build's HW_ID and XCC_ID fields:
// for 1024 forward work-groups of a causal B1 H32 N2048, per-CU stage counts
// 52-80 against a mean of 66, and CU end times following them). A causal
// launch runs its work heaviest first, so CU c's first work-groups take ranks
// c, c + C, c + 2C, ..., whose stages all fall with c. Reversing every other
// run of C ranks among the resident ones gives each CU one heavy and one light
// rank per pair of runs; with an odd count of runs (C even) the last three go
// as a triple, position c of them taking c, C - 1 - 2c (c < C/2) or
// 2C - 2 - 2c, and (c + C/2) mod C, which sum to 3(C - 1)/2 rounded. So every
// CU gets the same stages up to rounding (the work falling steadily with the
// rank). Work-groups past `runs` runs (dispatched as slots free up) keep
// their order. run <= 1 or runs < 2: i itself.
__host__ __device__ inline int cu_order_wg(int i, int run, int runs) {
    if (run <= 1 || runs < 2) return i;
    const int k = i / run, c = i - k * run;
    if (k >= runs) return i;
    const int t = (runs & 1) && (run & 1) == 0 ? runs - 3 : runs;  // runs [t, runs): the triple
    if (k < t) return (k & 1) ? k * run + run - 1 - c : i;
    const int half = run / 2;
    if (k == t) return i;
    if (k == t + 1) return k * run + (c < half ? run - 1 - 2 * c : 2 * run - 2 - 2 * c);
    return k * run + (c + half) % run;
}

// Delta flags of the one-launch backward: kFlagSlots slots (one per launch,
// round robin, so launches in flight at once on one device do not share
// flags) of kMaxFlagBlocks flags, one per (batch, query head, 128-row block).
constexpr int kFlagSlots = 4;
constexpr int kMaxFlagBlocks = 1 << 18;

// Shares of a dK/dV key block whose queries take nqs stages per query head:
// its group x nqs stages in runs of about dkv_share_stages, never fewer than
// dkv_min_shares runs nor more runs than stages (1 without a split).
__host__ __device__ inline int dkv_block_shares(const Params &p, int nqs) {
    if (p.dkv_split <= 1) return 1;
    const int t = p.group * nqs;
    const int n = t / p.dkv_share_stages + (t % p.dkv_share_stages != 0 ? 1 : 0);
    const int s = n > p.dkv_min_shares ? n : p.dkv_min_shares;
    return s < t ? s : t;
}

// The work of work-group w of a dK/dV pass (keys in blocks of bkv_rows,
// queries in stages of bq): key block kb, causal key block 0 (the most
// queries) first, then (batch, KV head) bkv, then share sp of the block's ns.
// kb is the number of key blocks when w is past the pass's last work-group.
struct DkvWork {
    int bkv, kb, sp, ns;
};
__host__ __device__ inline DkvWork dkv_work(const Params &p, int w, int bkv_rows, int bq, bool causal) {
    const int nbkv = p.B * p.Hkv, nkb = (p.N + bkv_rows - 1) / bkv_rows;
    if (p.dkv_split <= 1) return {w % nbkv, w / nbkv, 0, 1};
    if (!causal) {
        const int ns = dkv_block_shares(p, (p.N + bq - 1) / bq), per = nbkv * ns, r = w % per;
        return {r / ns, w / per, r % ns, ns};
    }
    for (int kb = 0; kb < nkb; ++kb) {
        const int ns = dkv_block_shares(p, (p.N - kb * bkv_rows + bq - 1) / bq);
        if (w < nbkv * ns) return {w / ns, kb, w % ns, ns};
        w -= nbkv * ns;
    }
    return {0, nkb, 0, 1};
}

// The dkv_work index of share 0 of key block kb of (batch, KV head) bkv; the
// block's other shares follow it.
__host__ __device__ inline int dkv_first_work(const Params &p, int bkv, int kb, int bkv_rows, int bq, bool causal) {
    const int nbkv = p.B * p.Hkv;
    if (p.dkv_split <= 1) return kb * nbkv + bkv;
    if (!causal) return (kb * nbkv + bkv) * dkv_block_shares(p, (p.N + bq - 1) / bq);
    int w = 0;
    for (int k = 0; k < kb; ++k) w += nbkv * dkv_block_shares(p, (p.N - k * bkv_rows + bq - 1) / bq);
    return w + bkv * dkv_block_shares(p, (p.N - kb * bkv_rows + bq - 1) / bq);
}

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

// Makes x opaque to the optimiser (an empty asm that "modifies" it), so a value
// computed once before a loop is not recomputed inside it.
template <class X>
__device__ __forceinline__ void pin_regs(X &x) {
    asm volatile("" : "+v"(x));
}

// sum_e a[e] b[e] over 8 bf16 pairs in fp32, in a fixed order with explicit
// fused multiply-adds (each bf16 product is exact in fp32). Every computation
// of Delta = rowsum(dO * O) that must agree bit for bit with another goes
// through this.
__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b) {
    float d = (float)a[0] * (float)b[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) d = __builtin_fmaf((float)a[e], (float)b[e], d);
    return d;
}

// fp32 -> bf16 bits, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ u16 to_bf16_bits(float x) {
    __bf16 h = (__bf16)x;
    return __builtin_bit_cast(u16, h);
}

// ------------------------------------------------------------------ policies

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// bf16 inputs, fp32 accumulation: v_mfma_f32_16x16x32_bf16.
//
// LDS tiles (64 rows x D) are stored column-group major: the 32 bytes of
// columns 16x..16x+15 of all 64 rows are contiguous (2 KB per group). Within a
// group, row r (bits r0..r5) sits at slot prow(r), whose bits are
// (r0, r1, r3^r4, r2, r4, r5), and its two 16-byte halves swap when r3 is set.
// Then, with either 128 or 256 bytes of banks per cycle,
//   * the 16-byte A-operand reads of rows arow(t, 0..15) hit 16 distinct
//     16-byte slots of a 256-byte window (8 distinct in every 128 bytes), and
//   * the transposing reads (ds_read_b64_tr_b16) of 4 consecutive rows of a
//     group touch 128 contiguous bytes, and the two 16-lane groups g, g+1 (rows
//     r, r+8) land in different 128-byte halves of a 256-byte window;
// and the row bits that depend on the loop position (r2: tile t or half h,
// r5: block) and the group map to fixed slot bits, so those offsets are plain
// additions that fold into the instructions' immediate offsets.
template <int D_>
struct PolBF16 {
    static constexpr int D = D_;
    using T = u16;
    using Frag = bf16x8;
    static constexpr int EPC = 8;      // elements per 16-byte chunk
    static constexpr int NC = D / 32;  // MFMAs over D per first-GEMM tile
    static constexpr int ROWS = 64;    // rows of every LDS tile
    // waves per SIMD the forward (kWaves), dQ (kWavesDq) and dK/dV (kWavesDkv)
    // kernels are compiled for: the largest count that fits without spills in
    // their loops. Three work-groups per CU also balance the causal passes:
    // their 128-row work-groups (64 - 2i stages of 64 for i = 0..31 at
    // N = 4096) pair up into equal loads over 768 slots. The forward also has
    // a three-wave form (kWavesFwdCausal) for causal launches of at least 768
    // work-groups; on smaller causal grids and non-causal launches it is no
    // faster than two. At d = 128 all three kernels run two waves per SIMD
    // (dK/dV is held there by its 66 KB of LDS; the non-causal forward spills
    // 64 bytes per lane at two and still ran 22% faster than at one).
    // The register-resident operand of each score GEMM (Q in the forward and
    // the dQ pass, K in the dK/dV pass) stays as given and the fp32 scores are
    // multiplied by scale log2(e) (one v_mul per score): rounding the scaled
    // operand to bf16 instead puts an error of about |S log2(e)| 2^-9 into
    // every exponent, correlated along a row or a key, which grows with the
    // logits and reaches the outputs through LSE.
    static constexpr bool kExactScale = true;
    static constexpr int kWaves = 2;
    static constexpr int kWavesFwdCausal = D == 64 ? 3 : 2;
    static constexpr int kWavesDq = D == 64 ? 3 : 2;
    // dQ pass: 16-query tiles per wave and waves per work-group. 64 queries
    // per wave halve the LDS reads per MFMA but need two waves per SIMD, and
    // ran 9-10% slower (48 queries: 8%); 16 queries at five waves per SIMD
    // double them and ran 13% slower
    static constexpr int kDqTiles = 2;
    static constexpr int kDqWavesPerGroup = 4;
    static constexpr int kWavesDkv = D == 64 ? 3 : 2;
    // dK/dV stage ring depth (loads issued kDkvBuffers - 1 stages ahead); a
    // third buffer measured no faster at d = 64
    static constexpr int kDkvBuffers = 2;

    __device__ static __forceinline__ int arow(int t, int m) {
        return ((m >> 2) << 3) + (t << 2) + (m & 3);
    }
    __device__ static __forceinline__ int bidx(int t, int g, int r) { return (g << 3) + (t << 2) + r; }

    // slot of row r within a column group, and its inverse
    __device__ static __forceinline__ int prow(int r) {
        return (r & 3) | ((((r >> 3) ^ (r >> 4)) & 1) << 2) | (((r >> 2) & 1) << 3) | (r & 48);
    }
    __device__ static __forceinline__ int prow_inv(int s) {
        const int b4 = (s >> 4) & 1, b3 = ((s >> 2) & 1) ^ b4;
        return (s & 3) | (((s >> 3) & 1) << 2) | (b3 << 3) | (s & 48);
    }
    // byte offset of 16-byte chunk `chunk` (columns 8 chunk..+7) of row `row`
    __device__ static __forceinline__ int chunk_off(int row, int chunk) {
        return (chunk >> 1) * (ROWS * 32) + prow(row) * 32 + (((chunk & 1) ^ ((row >> 3) & 1)) << 4);
    }
    // inverse map for the stager: the chunk stored at 16-byte position P
    __device__ static __forceinline__ void chunk_at(int P, int &row, int &chunk) {
        const int grp = P / (ROWS * 2), rem = P % (ROWS * 2);
        row = prow_inv(rem >> 1);
        chunk = 2 * grp + ((rem & 1) ^ ((row >> 3) & 1));
    }

    __device__ static __forceinline__ f32x4 mma(Frag a, Frag b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // k-slot (g, e) of MFMA c <-> element 32c + 8g + e of the row
    __device__ static __forceinline__ void lds_row_frags(Frag (&f)[NC], const T *tile, int n, int g) {
        const char *base = reinterpret_cast<const char *>(tile);
#pragma unroll
        for (int c = 0; c < NC; ++c) f[c] = *reinterpret_cast<const Frag *>(base + chunk_off(n, 4 * c + g));
    }
    // the row's fragments if valid, else zeros (the loads under a branch)
    __device__ static __forceinline__ void gmem_row_frags_if(Frag (&f)[NC], const T *row, int g, bool valid) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (valid) {
                f[c] = *reinterpret_cast<const Frag *>(row + 32 * c + 8 * g);
            } else {
                f[c] = Frag{};
            }
        }
    }
    // row i of n rows (row stride rs elements), zeros for i >= n (n >= 1): the
    // loads read row min(i, n - 1), so they take no branch and a tile's loads
    // issue together
    __device__ static __forceinline__ void gmem_row_frags(Frag (&f)[NC], const T *rows, int i, int n, size_t rs,
                                                          int g) {
        const bool valid = i < n;
        const T *row = rows + (size_t)(valid ? i : n - 1) * rs;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const Frag v = *reinterpret_cast<const Frag *>(row + 32 * c + 8 * g);
            f[c] = valid ? v : Frag{};
        }
    }
    // sum of the element products, in fp32
    __device__ static __forceinline__ float dot(Frag a, Frag b) { return dot8(a, b); }
    // every element times s, rounded to bf16 (nearest even), pinned in
    // registers like neg()
    __device__ static __forceinline__ Frag scaled(Frag f, float s) {
        Frag r;
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (__bf16)((float)f[e] * s);
        pin_regs(r);
        return r;
    }
    // flips the sign of every element (bf16 sign bits, two per dword). The
    // result is pinned (pin_regs) so the compiler keeps the negated fragment
    // live instead of recomputing it from the original inside the stage loop.
    __device__ static __forceinline__ Frag neg(Frag f) {
        typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
        Frag r = __builtin_bit_cast(Frag, __builtin_bit_cast(u32x4, f) ^ 0x80008000u);
        pin_regs(r);
        return r;
    }
    // The chain operand of one 32-row block: this lane's elements (t, r) of the
    // two C tiles, as bf16, k-slot e = 4t + r <-> block row bidx(t, g, r) = 8g + e.
    using ChainB = Frag;
    __device__ static __forceinline__ ChainB pack(const f32x4 &c0, const f32x4 &c1) {
        Frag b;
        b[0] = (__bf16)c0[0];
        b[1] = (__bf16)c0[1];
        b[2] = (__bf16)c0[2];
        b[3] = (__bf16)c0[3];
        b[4] = (__bf16)c1[0];
        b[5] = (__bf16)c1[1];
        b[6] = (__bf16)c1[2];
        b[7] = (__bf16)c1[3];
        return b;
    }
    // acc += Other * chain over the 32-row block starting at blk, where Other[y][n]
    // = tile[n][y0 + y] is read transposed from the tile with ds_read_b64_tr_b16
    // (lane (g, j) of a 16-lane group addresses row blk + 8g + 4h + j/4,
    // columns y0 + 4(j%4)..+3, and receives column y0 + j of those 4 rows):
    // k-slot e of both operands <-> row blk + 8g + e.
    __device__ static __forceinline__ Frag chain_a(const T *tile, int y0, int blk, int g, int l16) {
        const char *base = reinterpret_cast<const char *>(tile);
        const int r0 = blk + 8 * g + (l16 >> 2);
        const int col = y0 + 4 * (l16 & 3);
        const int off_lo = chunk_off(r0, col >> 3) + ((col & 7) << 1);
        const int off_hi = chunk_off(r0 + 4, col >> 3) + ((col & 7) << 1);
        const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(base + off_lo));
        const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4 *)(base + off_hi));
        return __builtin_bit_cast(Frag, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
    __device__ static __forceinline__ f32x4 chain(f32x4 acc, const ChainB &b, const T *tile, int y0, int blk,
                                                  int g, int l16) {
        return mma(chain_a(tile, y0, blk, g, l16), b, acc);
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
    static constexpr int ROWS = 64;
    // fp32 operands: the scale folds into the operand with a 2^-24 rounding
    static constexpr bool kExactScale = false;
    // the forward runs 64-query work-groups at two waves per SIMD (fa_fwd.hip)
    static constexpr int kWaves = 2;
    static constexpr int kWavesFwdCausal = 2;
    // dQ pass: one 16-query tile per wave at two waves per SIMD (202 VGPRs);
    // two tiles at one wave ran slower (B1 H1 N256 backward 70.8 -> 57.5 us,
    // B4 H12 N1024 causal 244 -> 235, B1 H12 N4096 non-causal 1812 -> 1604).
    // dK/dV keeps 32 keys per wave at one wave: 16 keys spill at two
    static constexpr int kWavesDq = 2;
    static constexpr int kDqTiles = 1;
    static constexpr int kDqWavesPerGroup = 4;
    static constexpr int kWavesDkv = 1;
    static constexpr int kDkvBuffers = 2;

    __device__ static __forceinline__ int arow(int t, int m) { return (t << 4) + m; }
    __device__ static __forceinline__ int bidx(int t, int g, int r) { return (t << 4) + (g << 2) + r; }
    // Row-major tiles, 16-byte chunks XOR-swizzled by the low row bits.
    __device__ static __forceinline__ int rswz(int n) { return n & 7; }
    __device__ static __forceinline__ int chunk_off(int row, int chunk) {
        return row * (D * 4) + ((chunk ^ rswz(row)) << 4);
    }
    __device__ static __forceinline__ void chunk_at(int P, int &row, int &chunk) {
        row = P / (D / 4);
        chunk = (P % (D / 4)) ^ rswz(row);
    }

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
    __device__ static __forceinline__ void gmem_row_frags_if(Frag (&f)[NC], const T *row, int g, bool valid) {
#pragma unroll
        for (int j = 0; j < NC / 4; ++j) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (valid) v = *reinterpret_cast<const float4 *>(row + NC * g + 4 * j);
            f[4 * j + 0] = v.x;
            f[4 * j + 1] = v.y;
            f[4 * j + 2] = v.z;
            f[4 * j + 3] = v.w;
        }
    }
    // row i of n rows (row stride rs elements), zeros for i >= n (n >= 1),
    // branch-free as in PolBF16
    __device__ static __forceinline__ void gmem_row_frags(Frag (&f)[NC], const T *rows, int i, int n, size_t rs,
                                                          int g) {
        const bool valid = i < n;
        const T *row = rows + (size_t)(valid ? i : n - 1) * rs;
#pragma unroll
        for (int j = 0; j < NC / 4; ++j) {
            const float4 v = *reinterpret_cast<const float4 *>(row + NC * g + 4 * j);
            f[4 * j + 0] = valid ? v.x : 0.f;
            f[4 * j + 1] = valid ? v.y : 0.f;
            f[4 * j + 2] = valid ? v.z : 0.f;
            f[4 * j + 3] = valid ? v.w : 0.f;
        }
    }
    __device__ static __forceinline__ Frag neg(Frag f) { return -f; }
    __device__ static __forceinline__ Frag scaled(Frag f, float s) { return f * s; }
    __device__ static __forceinline__ float dot(Frag a, Frag b) { return a * b; }
    // The chain operand of one 32-row block: the two C tiles themselves.
    struct ChainB {
        f32x4 c0, c1;
    };
    __device__ static __forceinline__ ChainB pack(const f32x4 &c0, const f32x4 &c1) { return ChainB{c0, c1}; }
    // Other[y][n] = tile[n][y0 + y] read element-wise: the k-slot g of MFMA
    // (t, r) is block row 16t + 4g + r, matching the C layout of the chain tiles.
    __device__ static __forceinline__ f32x4 chain(f32x4 acc, const ChainB &b, const T *tile, int y0, int blk,
                                                  int g, int l16) {
        const int y = y0 + l16;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int n = blk + (t << 4) + (g << 2) + r;
                const float a = tile[n * D + (((y >> 2) ^ rswz(n)) << 2) + (y & 3)];
                acc = mma(a, t ? b.c1[r] : b.c0[r], acc);
            }
        }
        return acc;
    }
};

// --------------------------------------------------------------- LDS staging

// Wave-wide direct global->LDS loads (global_load_lds_dwordx4 / _dword: no
// VGPRs, no VALU). Lane i's bytes from src land at LDS address base + 16 i
// (+ 4 i for the dword form); base is wave-uniform and goes through M0.
//
// They are issued from asm on purpose. The compiler's wait-count pass cannot
// tell which LDS buffer an in-flight global->LDS load writes, so after a
// builtin load it makes the next LDS read of ANY buffer wait for it
// (s_waitcnt vmcnt(0)): a prefetch of the next stage would then complete
// before the current stage computes. Loads it does not see leave the waits
// to the kernels: wait_stage() / wait_vmcnt<>() and a barrier before a stage
// is read, and a barrier after a buffer's last read before it is refilled.
// M0 is saved and restored around each load, so the compiler's own uses of
// M0 are unaffected; the s_nop covers the M0-write -> LDS-DMA hazard.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
#if defined(__HIP_DEVICE_COMPILE__)  // the host pass rejects the address-space cast
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
#else
    return 0;
#endif
}
__device__ __forceinline__ void lds_dma16(uint32_t base, const void *src) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(src), "s"(__builtin_amdgcn_readfirstlane(base)));
#endif
}
__device__ __forceinline__ void lds_dma4(uint32_t base, const void *src) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
        "global_load_lds_dword %1, off\n\ts_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(src), "s"(__builtin_amdgcn_readfirstlane(base)));
#endif
}

// Accesses for data that work-groups on different XCDs exchange within one
// launch (each XCD has its own L2, which the hardware does not keep coherent
// with the others): system-coherent (sc0 sc1) stores write through every
// cache level, and loads of that kind miss them, so both meet in memory.
// lds_dma4_uc: lds_dma4 with such a load.
__device__ __forceinline__ void lds_dma4_uc(uint32_t base, const void *src) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t"
        "global_load_lds_dword %1, off sc0 sc1\n\ts_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(src), "s"(__builtin_amdgcn_readfirstlane(base)));
#endif
}
// A write-through store of one dword.
__device__ __forceinline__ void store_wt(void *dst, uint32_t v) {
    asm volatile("global_store_dword %0, %1, off sc0 sc1" ::"v"(dst), "v"(v) : "memory");
}
// A write-through store of four floats at byte offset off of base (wave-
// uniform); offsets at or past `bytes` are dropped. A builtin, not inline asm:
// a store of more than 64 bits whose data registers a VALU instruction
// overwrites within two wait states needs the compiler's hazard padding, and
// the compiler cannot see inside an asm statement (a build that kept the dK/dV
// accumulators in AGPRs moved the next one into the data registers right after
// such an asm store, and the stored partial sums were wrong).
__device__ __forceinline__ void store4_wt(float *base, uint32_t bytes, uint32_t off, f32x4 v) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 17);  // cache policy sc0 | sc1
}
// Four floats at byte offset off of base (wave-uniform) past the caches;
// offsets at or past `bytes` read as 0.
__device__ __forceinline__ f32x4 load4_uc(const float *base, uint32_t bytes, uint32_t off) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), 0, bytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 17);  // cache policy sc0 | sc1
}
// A load past the caches, complete on return (it waits for every outstanding
// vector-memory operation of the wave).
__device__ __forceinline__ uint32_t load_uc_sync(const void *src) {
    uint32_t v;
    asm volatile("global_load_dword %0, %1, off sc0 sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(src) : "memory");
    return v;
}
// The same for 8 bytes (naturally aligned: one access, never half old and
// half new), and a write-through store of 8 bytes.
__device__ __forceinline__ unsigned long long load2_uc_sync(const unsigned long long *src) {
    unsigned long long v;
    asm volatile("global_load_dwordx2 %0, %1, off sc0 sc1\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(src) : "memory");
    return v;
}
__device__ __forceinline__ void store2_wt(unsigned long long *dst, unsigned long long v) {
    asm volatile("global_store_dwordx2 %0, %1, off sc0 sc1" ::"v"(dst), "v"(v) : "memory");
}
// Waits until this wave's stores have been acknowledged.
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Timeline build (-DMXFA_WG_TIMELINE: `make timeline`, mxfa_gfx950_timeline.hsaco):
// thread 0 of every work-group of the forward, of the dQ and dK/dV bodies and
// of the one-launch backward's reduce stamps the 100 MHz real-time counter at
// its start (0), once its first stage is staged (1; the reduce: once its
// shares are done), at the end of its loop (2) and once its stores are
// acknowledged (3), into mxfa_wg_times[8 g + i] for its linear work-group
// index g ((z Y + y) X + x over the grid, so each split of a split forward has
// its own slot), and records what it ran: (kind << 32) | block at 8 g + 4
// (kind 0 = dQ, block = query block; 1 = dK/dV, block = key block; 2 =
// forward, block = query block; 3 = reduce, block = key block), its stages
// (the reduce: its shares) at 8 g + 5 and where it ran at 8 g + 6 ((XCC_ID
// << 32) | HW_ID; read by mxfa_probe_wg_times). In every other build these
// compile to nothing.
#if defined(__HIP_DEVICE_COMPILE__) && defined(MXFA_WG_TIMELINE)
constexpr unsigned kTimelineGroups = 1u << 16;
extern "C" __device__ unsigned long long mxfa_wg_times[kTimelineGroups * 8];
__device__ unsigned long long mxfa_wg_times[kTimelineGroups * 8];
__device__ __forceinline__ void wg_put(int i, unsigned long long v) {
    const unsigned g = (blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x;
    if (threadIdx.x == 0 && g < kTimelineGroups) {
        *reinterpret_cast<volatile unsigned long long *>(mxfa_wg_times + 8 * (size_t)g + i) = v;
    }
}
__device__ __forceinline__ void wg_time(int i) { wg_put(i, __builtin_amdgcn_s_memrealtime()); }
__device__ __forceinline__ void wg_info(unsigned kind, int block, int stages) {
    wg_put(4, ((unsigned long long)kind << 32) | (unsigned)block);
    wg_put(5, (unsigned)stages);
    // where it runs: the HW_ID register (CU, shader array and engine fields)
    // and the XCC_ID register (the XCD)
    wg_put(6, ((unsigned long long)__builtin_amdgcn_s_getreg(20 | (15 << 11)) << 32) |
                  (unsigned)__builtin_amdgcn_s_getreg(4 | (31 << 11)));
}
__device__ __forceinline__ void wg_time_after_stores() {
    wait_stores();
    wg_time(3);
}
#else
__device__ __forceinline__ void wg_time(int) {}
__device__ __forceinline__ void wg_info(unsigned, int, int) {}
__device__ __forceinline__ void wg_time_after_stores() {}
#endif

// Issue priority of the calling wave (0 or 1; the scheduling barriers keep the
// compiler from moving instructions across the change). ON = false compiles
// to nothing.
template <bool ON>
__device__ __forceinline__ void wave_priority(int hi) {
    if constexpr (ON) {
        __builtin_amdgcn_sched_barrier(0);
        if (hi) {
            __builtin_amdgcn_s_setprio(1);
        } else {
            __builtin_amdgcn_s_setprio(0);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Copies rows [0, Pol::ROWS) of a row-major [*, D] matrix into an LDS tile in
// the policy's layout: load k of the wave fills 16-byte positions
// P = k NT + 64 wave + lane, and each lane fetches the global chunk that
// belongs at its position. Rows >= nvalid re-read row nvalid-1 (in bounds; the
// kernels mask or zero their scores). Called by all NT threads of the
// workgroup.
template <class Pol, int NT = 256>
__device__ __forceinline__ void stage_rows(typename Pol::T *tile, const typename Pol::T *src, int nvalid,
                                           int tid, int wave, int row_stride = Pol::D) {
    constexpr int CPR = Pol::D / Pol::EPC;
    constexpr int NCH = Pol::ROWS * CPR;
    static_assert(NCH % NT == 0, "whole wave-wide loads");
    const uint32_t base = lds_addr(tile) + wave * 64 * 16;
#pragma unroll
    for (int k = 0; k < NCH / NT; ++k) {
        const int P = k * NT + tid;
        int row, c;
        Pol::chunk_at(P, row, c);
        const int grow = min(row, nvalid - 1);
        lds_dma16(base + k * NT * 16, src + (size_t)grow * row_stride + c * Pol::EPC);
    }
}

// The same load with the global address split into a wave-uniform base (an
// SGPR pair) and a 32-bit per-lane byte offset: the instruction's saddr form.
__device__ __forceinline__ void lds_dma16_s(uint32_t base, const void *sbase, uint32_t voff) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t save;
    asm volatile(
        "s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
        : "=&s"(save)
        : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(base)));
#endif
}

// Where each of a thread's staging loads of a tile reads from: load k fills
// 16-byte position P = k NT + tid of the tile, which holds chunk c of row r
// (Pol::chunk_at). Computed once per kernel and kept packed in one register
// per load (r in bits 0-7, the chunk's byte offset within the row above), so
// a stage's loads cost a few VALU operations each instead of the layout
// arithmetic.
template <class Pol, int NT = 256>
struct RowPlan {
    static constexpr int NK = Pol::ROWS * (Pol::D / Pol::EPC) / NT;
    static_assert(NK * NT == Pol::ROWS * (Pol::D / Pol::EPC), "whole wave-wide loads");
    uint32_t rc[NK];
    __device__ explicit RowPlan(int tid) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            int row, c;
            Pol::chunk_at(k * NT + tid, row, c);
            rc[k] = (uint32_t)row | ((uint32_t)(c * 16) << 8);
        }
    }
};

// stage_rows with a RowPlan: rows >= nvalid re-read row nvalid - 1, as there.
// The tile as an LDS address (tile_lds), or as a pointer below.
template <class Pol, int NT = 256>
__device__ __forceinline__ void stage_rows(uint32_t tile_lds, const typename Pol::T *src, int nvalid,
                                           const RowPlan<Pol, NT> &pl, int wave, int row_stride = Pol::D) {
    const uint32_t base = tile_lds + wave * 64 * 16;
    const uint32_t rs_bytes = (uint32_t)row_stride * sizeof(typename Pol::T);
#pragma unroll
    for (int k = 0; k < RowPlan<Pol, NT>::NK; ++k) {
        const uint32_t grow = (uint32_t)min((int)(pl.rc[k] & 255u), nvalid - 1);
        lds_dma16_s(base + k * NT * 16, src, grow * rs_bytes + (pl.rc[k] >> 8));
    }
}
template <class Pol, int NT = 256>
__device__ __forceinline__ void stage_rows(typename Pol::T *tile, const typename Pol::T *src, int nvalid,
                                           const RowPlan<Pol, NT> &pl, int wave, int row_stride = Pol::D) {
    stage_rows<Pol, NT>(lds_addr(tile), src, nvalid, pl, wave, row_stride);
}

// One K/V stage: Pol::ROWS key rows from k0 of K and V (rows row_stride
// elements apart) into LDS buffers.
template <class Pol, int NT = 256>
__device__ __forceinline__ void stage_kv(typename Pol::T *sk, typename Pol::T *sv, const typename Pol::T *K,
                                         const typename Pol::T *V, int k0, int N, int tid, int wave,
                                         int row_stride = Pol::D) {
    stage_rows<Pol, NT>(sk, K + (size_t)k0 * row_stride, N - k0, tid, wave, row_stride);
    stage_rows<Pol, NT>(sv, V + (size_t)k0 * row_stride, N - k0, tid, wave, row_stride);
}
template <class Pol, int NT = 256>
__device__ __forceinline__ void stage_kv(typename Pol::T *sk, typename Pol::T *sv, const typename Pol::T *K,
                                         const typename Pol::T *V, int k0, int N, const RowPlan<Pol, NT> &pl,
                                         int wave, int row_stride = Pol::D) {
    stage_rows<Pol, NT>(sk, K + (size_t)k0 * row_stride, N - k0, pl, wave, row_stride);
    stage_rows<Pol, NT>(sv, V + (size_t)k0 * row_stride, N - k0, pl, wave, row_stride);
}

// A paged K/V stage (Params::block_table): per staging load of the thread,
// the block-table entry of its row in the next stage to be staged. fetch()
// loads them for the stage at k0 (rows past N take row N - 1, as stage_rows
// does); stage() issues that stage's loads from them. A caller fetches one
// stage ahead of the loads, so the table loads complete within the stage
// before and the staging loads never wait for them.
template <class Pol, int NT = 256>
struct PagedRows {
    static constexpr int NK = RowPlan<Pol, NT>::NK;
    int blk[NK];

    __device__ __forceinline__ void fetch(const int *bt, int shift, int k0, int N, const RowPlan<Pol, NT> &pl) {
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int t = min(k0 + (int)(pl.rc[k] & 255u), N - 1);
            blk[k] = bt[t >> shift];
        }
    }
    // rows k0 .. k0 + Pol::ROWS - 1 of K and V (cache rows row_stride
    // elements apart) into the LDS tiles, as stage_kv does for a contiguous cache
    __device__ __forceinline__ void stage(typename Pol::T *sk, typename Pol::T *sv, const typename Pol::T *K,
                                          const typename Pol::T *V, int k0, int N, int shift,
                                          const RowPlan<Pol, NT> &pl, int wave, int row_stride) const {
        const uint32_t bk = lds_addr(sk) + wave * 64 * 16, bv = lds_addr(sv) + wave * 64 * 16;
        const int mask = (1 << shift) - 1;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
            const int t = min(k0 + (int)(pl.rc[k] & 255u), N - 1);
            const size_t off = (((size_t)blk[k] << shift) + (size_t)(t & mask)) * (size_t)row_stride +
                               (pl.rc[k] >> 8) / sizeof(typename Pol::T);
            lds_dma16(bk + k * NT * 16, K + off);
            lds_dma16(bv + k * NT * 16, V + off);
        }
    }
};

// Read by lanes past the end of a staged vector (see stage_vec64). Device
// variables and kernels are defined in the code object only (the device
// pass); the host library, compiled for the host alone, sees declarations.
#if defined(__HIP_DEVICE_COMPILE__)
__device__ const float kPosInf = __builtin_inff();
#else
extern __device__ const float kPosInf;
#endif

// 64 fp32 values src[l] (l < nvalid, else *pad) -> dst[l], by one wave (dst
// as an LDS address, or as a pointer).
__device__ __forceinline__ void stage_vec64(uint32_t dst_lds, const float *src, int nvalid, int lane,
                                            const float *pad) {
    lds_dma4(dst_lds, lane < nvalid ? src + lane : pad);
}
__device__ __forceinline__ void stage_vec64(float *dst, const float *src, int nvalid, int lane, const float *pad) {
    stage_vec64(lds_addr(dst), src, nvalid, lane, pad);
}

// Waits for this wave's outstanding global->LDS loads (the caller then
// barriers so every wave's loads are visible).
__device__ __forceinline__ void wait_stage() { __builtin_amdgcn_s_waitcnt(0); }

// Workgroup barrier that waits only for this wave's LDS operations.
// __syncthreads() also waits for every outstanding vector-memory operation
// (s_waitcnt vmcnt(0) before s_barrier), which would drain global->LDS loads
// issued for later stages; this one leaves them in flight. The asm is a
// compiler memory barrier, so no LDS access moves across it.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// barrier_lds() that also fences the instruction scheduler: register-only
// instructions (MFMAs above all) are not moved across it either. The asm alone
// orders memory accesses only, and the scheduler otherwise sinks MFMAs past
// the barrier into the next phase.
__device__ __forceinline__ void barrier_phase() {
    __builtin_amdgcn_sched_barrier(0);
    barrier_lds();
    __builtin_amdgcn_sched_barrier(0);
}

// Waits until at most VM of this wave's vector-memory loads are outstanding
// (s_waitcnt vmcnt(VM); expcnt and lgkmcnt left unconstrained): with loads
// issued for two stages ahead, the older stage is complete while the newer
// one stays in flight.
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(VM >= 0 && VM < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Global->LDS loads one thread of an NT-thread workgroup issues for one
// Pol::ROWS x D tile.
template <class Pol, int NT = 256>
constexpr int tile_loads() {
    return Pol::ROWS * (Pol::D / Pol::EPC) / NT;
}

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

// Two C tiles of one output row in bf16, 16 bytes per lane: in the 16x16 C
// layout a holds elements x0 + 4g .. +3 of the lane's row and b elements
// x0 + 16 + 4g .. +3 (g = lane / 16). Lanes of lane groups g and g + 1 (g
// even; the same row) swap halves with v_permlane16_swap, so a lane of an even
// group writes elements x0 + 4g .. +7 and one of an odd group x0 + 12 + 4g ..
// +7: a store instruction covers 64 bytes of each of its 16 rows instead of
// 32. Every lane takes part in the swap; only the store is predicated (both
// lanes of a pair have the same row, so the same `valid`).
__device__ __forceinline__ void store8_pair_bf16(u16 *row, int x0, int g, f32x4 a, f32x4 b, float mul,
                                                 bool valid) {
    const uint32_t a0 = (uint32_t)to_bf16_bits(a[0] * mul) | ((uint32_t)to_bf16_bits(a[1] * mul) << 16);
    const uint32_t a1 = (uint32_t)to_bf16_bits(a[2] * mul) | ((uint32_t)to_bf16_bits(a[3] * mul) << 16);
    const uint32_t b0 = (uint32_t)to_bf16_bits(b[0] * mul) | ((uint32_t)to_bf16_bits(b[1] * mul) << 16);
    const uint32_t b1 = (uint32_t)to_bf16_bits(b[2] * mul) | ((uint32_t)to_bf16_bits(b[3] * mul) << 16);
    // even groups keep their own a and take the odd partner's; odd groups
    // take the even partner's b and keep their own
    const auto s0 = __builtin_amdgcn_permlane16_swap(a0, b0, false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(a1, b1, false, false);
    if (valid) {
        const int off = x0 + ((g & 1) ? 12 + 4 * g : 4 * g);
        *reinterpret_cast<uint4 *>(row + off) = make_uint4(s0[0], s1[0], s0[1], s1[1]);
    }
}

}  // namespace mxfa
