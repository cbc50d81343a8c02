// The kernels of the gfx950 code object (mxfa_gfx950.hsaco), by name.
//
// This list is the one source of the names: the device sources define one
// `extern "C" __global__` kernel per entry (each an instantiation of a
// templated body), and the host library looks every entry up with
// hipModuleGetFunction when it loads the code object; a name missing from
// the code object fails that load. Naming: pass, dtype and head dim (b64 =
// bf16 d = 64, b128, f64 = fp32 d = 64), c / n = causal / not, then the
// variant (waves per SIMD w*, query tiles per wave q*, d = computes Delta,
// pg = K/V through a block table, sp = one split of the keys, p2 = a softmax
// scale that is a power of two).
#pragma once

#define MXFA_KERNEL_LIST(X)                                                                   \
    /* forward (fa_fwd.hip): waves per SIMD, 16-query tiles per wave */                      \
    X(mxfa_fwd_b64_c_w3_q2) X(mxfa_fwd_b64_c_w2_q2) X(mxfa_fwd_b64_c_w3_q1)                   \
    X(mxfa_fwd_b64_n_w2_q2) X(mxfa_fwd_b64_n_w3_q1)                                           \
    X(mxfa_fwd_b128_c_w2_q2) X(mxfa_fwd_b128_c_w2_q1) X(mxfa_fwd_b128_n_w2_q2)                \
    X(mxfa_fwd_f64_c_w2_q1) X(mxfa_fwd_f64_n_w2_q1)                                           \
    X(mxfa_fwd_b64_c_w2_q2_pg) X(mxfa_fwd_b64_c_w3_q1_pg) X(mxfa_fwd_b128_c_w2_q1_pg)          \
    X(mxfa_fwd_f64_c_w2_q1_pg)                                                                \
    X(mxfa_fwd_b64_c_w3_q1_sp) X(mxfa_fwd_b128_c_w2_q1_sp) X(mxfa_fwd_f64_c_w2_q1_sp)          \
    X(mxfa_fwd_b64_c_w3_q1_pg_sp) X(mxfa_fwd_b128_c_w2_q1_pg_sp) X(mxfa_fwd_f64_c_w2_q1_pg_sp) \
    X(mxfa_fwd_merge8_b64) X(mxfa_fwd_merge8_b128) X(mxfa_fwd_merge8_f64)                     \
    X(mxfa_fwd_merge32_b64) X(mxfa_fwd_merge32_b128) X(mxfa_fwd_merge32_f64)                  \
    /* backward (fa_bwd.hip) */                                                               \
    X(mxfa_preprocess_b64) X(mxfa_preprocess_b128) X(mxfa_preprocess_f64)                     \
    X(mxfa_dq_b64_c) X(mxfa_dq_b64_c_d) X(mxfa_dq_b64_n) X(mxfa_dq_b64_n_d)                   \
    X(mxfa_dq_b128_c) X(mxfa_dq_b128_c_d) X(mxfa_dq_b128_n) X(mxfa_dq_b128_n_d)               \
    X(mxfa_dq_f64_c) X(mxfa_dq_f64_c_d) X(mxfa_dq_f64_n) X(mxfa_dq_f64_n_d)                   \
    X(mxfa_dkv_b64_c) X(mxfa_dkv_b64_n) X(mxfa_dkv_b128_c) X(mxfa_dkv_b128_n)                 \
    X(mxfa_dkv_f64_c) X(mxfa_dkv_f64_n) X(mxfa_dkv_b64_c_p2) X(mxfa_dkv_b64_n_p2)             \
    X(mxfa_bwd_b64_c) X(mxfa_bwd_b64_n) X(mxfa_bwd_b128_c) X(mxfa_bwd_b128_n)                 \
    X(mxfa_bwd_b64_c_p2) X(mxfa_bwd_b64_n_p2)                                                 \
    X(mxfa_bwd_b64_c_w2) X(mxfa_bwd_b64_n_w2) X(mxfa_bwd_b64_c_p2_w2) X(mxfa_bwd_b64_n_p2_w2)  \
    X(mxfa_dkv_reduce_bf16) X(mxfa_dkv_reduce_f32)                                            \
    /* naive baselines (fa_naive.hip) */                                                      \
    X(mxfa_naive_scores) X(mxfa_naive_softmax) X(mxfa_naive_av) X(mxfa_naive_bwd)            \
    /* probes (probe.hip) */                                                                  \
    X(mxfa_probe_mfma_bf16) X(mxfa_probe_mfma_f32) X(mxfa_probe_mfma32_bf16)                  \
    X(mxfa_probe_read_f4) X(mxfa_probe_copy_f4) X(mxfa_probe_dq_atomic_add)                   \
    X(mxfa_probe_dq_atomic_store) X(mxfa_probe_mix_mfma) X(mxfa_probe_mix_dkv)                  \
    X(mxfa_probe_mix_dkv_valu) X(mxfa_probe_mix_dkv_lds) X(mxfa_probe_mix_dq) X(mxfa_probe_mix_fwd)         \
    X(mxfa_probe_mix32_mfma) X(mxfa_probe_mix32_dkv) X(mxfa_probe_mix32_dq) X(mxfa_probe_mix32_fwd)

namespace mxfa {

enum KernelId {
#define MXFA_KID(n) k_##n,
    MXFA_KERNEL_LIST(MXFA_KID)
#undef MXFA_KID
    kNumKernels
};

}  // namespace mxfa
