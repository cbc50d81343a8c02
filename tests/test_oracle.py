"""Pins the CPU oracle (oracle/oracle.c) before anything is checked against it.

Known-answer tests mirror the reference's own unit tests
(common/src/lib.rs:84-113); golden vectors come from float64 torch SDPA
(tests/golden/make_golden.py); the finite-difference gate is the reference's
(02-flash-attention/src/main.rs:339-390, 504-508); the rest are closed forms,
special cases and brute force. No GPU needed.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
from oracle_pins import (_rand_case, golden_cases, pin_fd, pin_golden, pin_invariants,
                         rel_max_err)


@pytest.fixture(scope="module")
def lib():
    return oracle.load()


# ------------------------------------------------ common/src/lib.rs tests --

def test_pseudo_rand_is_deterministic_and_bounded(lib):
    # common/src/lib.rs:104-113
    a = oracle.pseudo_rand(1000, 42)
    b = oracle.pseudo_rand(1000, 42)
    assert np.array_equal(a, b)
    assert a.size == 1000
    assert np.all((a >= -1.0) & (a < 1.0))
    assert not np.array_equal(oracle.pseudo_rand(1000, 43), a)


def test_pseudo_rand_matches_numpy_restatement(lib):
    """An independent uint64 restatement of xorshift64* (common/src/lib.rs:67-78)."""
    def ref(n, seed):
        s = np.uint64(seed)
        out = np.empty(n, np.float32)
        with np.errstate(over="ignore"):
            for i in range(n):
                s ^= s >> np.uint64(12)
                s ^= s << np.uint64(25)
                s ^= s >> np.uint64(27)
                r = s * np.uint64(0x2545F4914F6CDD1D)
                out[i] = np.float32(int(r >> np.uint64(40))) / np.float32(1 << 23) - np.float32(1.0)
        return out
    for seed in (1, 2, 3, 4, 11, 21, 12345678901234):
        assert np.array_equal(oracle.pseudo_rand(257, seed), ref(257, seed))
    # the values are multiples of 2^-23 in [-1, 1): exactly representable
    x = oracle.pseudo_rand(4096, 5).astype(np.float64)
    assert np.all(np.round(x * 2 ** 23) == x * 2 ** 23)


def test_max_rel_err_basics(lib):
    # common/src/lib.rs:84-91
    a = np.array([1.0, 2.0, 3.0], np.float32)
    assert oracle.max_rel_err(a, a) == 0.0
    got = np.array([1.0, 2.2, 3.0], np.float32)
    assert abs(oracle.max_rel_err(got, a) - 0.1) < 1e-6


def test_allclose_err_threshold(lib):
    # common/src/lib.rs:93-102
    want = np.array([0.0, 100.0], np.float32)
    got = np.array([0.05, 101.0], np.float32)
    assert oracle.allclose_err(got, want, 1e-2, 5e-2) <= 1.0 + 1e-6
    bad = np.array([0.10, 102.0], np.float32)
    assert oracle.allclose_err(bad, want, 1e-2, 5e-2) > 1.0


# ---------------------------------------------------------------- goldens --

@pytest.mark.parametrize("path", golden_cases(), ids=lambda p: os.path.basename(p)[:-4])
def test_oracle_matches_golden(lib, path):
    assert pin_golden(lib, path) == {}


def test_golden_set_is_complete():
    names = {os.path.basename(p) for p in golden_cases()}
    assert len(names) >= 8
    assert any("gqa" in n for n in names) and any("d128" in n for n in names)
    assert any("n1_" in n for n in names) and any("ragged" in n for n in names)


# ------------------------------------------------ reference's FD gate -----

@pytest.mark.parametrize("causal", [False, True])
def test_fd_check(lib, causal):
    assert pin_fd(lib, causal) == {}
    # the reference README reports ~1e-5 for this check
    assert oracle.fd_check(128, causal) < 1e-3


# ------------------------------------------------------------- invariants --

@pytest.mark.parametrize("causal", [False, True])
def test_vjp_invariants(lib, causal):
    assert pin_invariants(lib, causal) == {}


def test_delta_is_rowsum_of_p_dp(lib):
    """Delta_i = rowsum(dO * O) (attention_bwd.cu:32-44) equals sum_j p_ij dP_ij,
    which is what makes sum_j dS_ij vanish; checked against float64 numpy."""
    N, d = 33, 64
    q, k, v, do = (x[0, 0] for x in _rand_case(N, d, 1, 1, 1))
    o, _ = oracle.cpu_attention(q, k, v, N, d, True)
    dl = oracle.delta(do, o, d)
    s = q.astype(np.float64) @ k.astype(np.float64).T * oracle.default_scale(d)
    s[np.triu_indices(N, 1)] = -np.inf
    p = np.exp(s - s.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    want = (p * (do.astype(np.float64) @ v.astype(np.float64).T)).sum(1)
    assert rel_max_err(dl, want) < 1e-5


@pytest.mark.parametrize("causal", [False, True])
def test_v_scaling_is_exact(lib, causal):
    """Scaling V by 2 scales O, dQ, dK by exactly 2 and leaves dV, LSE unchanged."""
    B, Hq, Hkv, N, d = 1, 2, 2, 24, 64
    q, k, v, do = _rand_case(N, d, B, Hq, Hkv)
    o1, l1 = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, causal)
    o2, l2 = oracle.mha_fwd(q, k, 2 * v, B, Hq, Hkv, N, d, causal)
    g1 = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, causal)
    g2 = oracle.mha_bwd(q, k, 2 * v, do, B, Hq, Hkv, N, d, causal)
    assert np.array_equal(o2, 2 * o1) and np.array_equal(l1, l2)
    assert np.array_equal(g2[0], 2 * g1[0]) and np.array_equal(g2[1], 2 * g1[1])
    assert np.array_equal(g2[2], g1[2])


@pytest.mark.parametrize("causal", [False, True])
def test_key_shift_invariance(lib, causal):
    """K_j -> K_j + c for all j leaves O, dQ, dV unchanged, shifts LSE_i by
    scale * q_i . c, and leaves dK unchanged (dK does not depend on K's offset)."""
    N, d = 28, 64
    q, k, v, do = (x[0, 0] for x in _rand_case(N, d, 1, 1, 1, mult=0.5))
    c = oracle.normal(d, 99, 0.25)
    o1, l1 = oracle.cpu_attention(q, k, v, N, d, causal)
    o2, l2 = oracle.cpu_attention(q, k + c, v, N, d, causal)
    assert rel_max_err(o2, o1) < 2e-5
    shift = q.astype(np.float64) @ c.astype(np.float64) * oracle.default_scale(d)
    assert np.abs(l2 - l1 - shift).max() < 2e-5 * np.abs(l1).max()
    g1 = oracle.cpu_attention_bwd(q, k, v, do, N, d, causal)
    g2 = oracle.cpu_attention_bwd(q, k + c, v, do, N, d, causal)
    for a, b in zip(g1, g2):
        assert rel_max_err(b, a) < 5e-5


def test_permutation_equivariance(lib):
    """Non-causal: permuting key/value rows permutes dK/dV and leaves O, LSE, dQ."""
    N, d = 30, 64
    q, k, v, do = (x[0, 0] for x in _rand_case(N, d, 1, 1, 1))
    perm = np.random.default_rng(3).permutation(N)
    o1, l1 = oracle.cpu_attention(q, k, v, N, d, False)
    o2, l2 = oracle.cpu_attention(q, k[perm], v[perm], N, d, False)
    assert rel_max_err(o2, o1) < 2e-5 and rel_max_err(l2, l1) < 2e-6
    dq1, dk1, dv1 = oracle.cpu_attention_bwd(q, k, v, do, N, d, False)
    dq2, dk2, dv2 = oracle.cpu_attention_bwd(q, k[perm], v[perm], do, N, d, False)
    assert rel_max_err(dq2, dq1) < 5e-5
    assert rel_max_err(dk2, dk1[perm]) < 5e-5 and rel_max_err(dv2, dv1[perm]) < 5e-5


@pytest.mark.parametrize("causal", [False, True])
def test_gqa_equals_repeated_mha(lib, causal):
    """GQA (Hq = 3 Hkv) equals MHA on K/V repeated per group, with dK/dV summed
    over each group's query heads."""
    B, Hq, Hkv, N, d = 2, 6, 2, 20, 64
    q, k, v, do = _rand_case(N, d, B, Hq, Hkv)
    g = Hq // Hkv
    kr, vr = np.repeat(k, g, axis=1), np.repeat(v, g, axis=1)
    o1, l1 = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, causal)
    o2, l2 = oracle.mha_fwd(q, kr, vr, B, Hq, Hq, N, d, causal)
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2)
    dq1, dk1, dv1 = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, causal)
    dq2, dk2, dv2 = oracle.mha_bwd(q, kr, vr, do, B, Hq, Hq, N, d, causal)
    assert np.array_equal(dq1, dq2)
    sk = dk2.reshape(B, Hkv, g, N, d).sum(axis=2, dtype=np.float64)
    sv = dv2.reshape(B, Hkv, g, N, d).sum(axis=2, dtype=np.float64)
    assert rel_max_err(dk1, sk) < 1e-6 and rel_max_err(dv1, sv) < 1e-6


def test_thread_count_does_not_change_results(lib):
    B, Hq, Hkv, N, d = 2, 4, 2, 32, 64
    q, k, v, do = _rand_case(N, d, B, Hq, Hkv)
    a = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, True, nthreads=1)
    b = oracle.mha_bwd(q, k, v, do, B, Hq, Hkv, N, d, True, nthreads=4)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)
    fa = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, True, nthreads=1)
    fb = oracle.mha_fwd(q, k, v, B, Hq, Hkv, N, d, True, nthreads=3)
    assert np.array_equal(fa[0], fb[0]) and np.array_equal(fa[1], fb[1])


# ----------------------------------------------------------- special cases --

@pytest.mark.parametrize("d", [64, 128])
def test_causal_row_zero(lib, d):
    """Causal row 0 sees only key 0: O_0 = V_0, LSE_0 = scale q_0.k_0, dQ_0 = 0."""
    N = 16
    q, k, v, do = (x[0, 0] for x in _rand_case(N, d, 1, 1, 1))
    o, lse = oracle.cpu_attention(q, k, v, N, d, True)
    assert np.array_equal(o[0], v[0])
    want = float(np.dot(q[0].astype(np.float64), k[0].astype(np.float64))) * oracle.default_scale(d)
    assert abs(lse[0] - want) < 1e-5 * max(1.0, abs(want))
    dq, _, _ = oracle.cpu_attention_bwd(q, k, v, do, N, d, True)
    assert np.abs(dq[0]).max() < 1e-6


@pytest.mark.parametrize("causal", [False, True])
def test_zero_keys_give_uniform_attention(lib, causal):
    """K = 0: P is uniform over the visible keys, so O_i is the mean of the
    visible V rows, LSE_i = ln(#visible) and dQ = 0."""
    N, d = 21, 64
    q, _, v, do = (x[0, 0] for x in _rand_case(N, d, 1, 1, 1))
    k = np.zeros_like(q)
    o, lse = oracle.cpu_attention(q, k, v, N, d, causal)
    cnt = np.arange(1, N + 1) if causal else np.full(N, N)
    vm = np.cumsum(v.astype(np.float64), 0) / cnt[:, None] if causal else \
        np.broadcast_to(v.astype(np.float64).mean(0), (N, d))
    assert rel_max_err(o, vm) < 2e-6
    assert np.abs(lse - np.log(cnt)).max() < 2e-6
    dq, _, _ = oracle.cpu_attention_bwd(q, k, v, do, N, d, causal)
    assert np.abs(dq).max() == 0.0


def test_single_token(lib):
    """N = 1: O = V, LSE = s, dQ = dK = 0, dV = dO."""
    d = 64
    q, k, v, do = (x[0, 0] for x in _rand_case(1, d, 1, 1, 1))
    for causal in (False, True):
        o, lse = oracle.cpu_attention(q, k, v, 1, d, causal)
        assert np.array_equal(o, v)
        dq, dk, dv = oracle.cpu_attention_bwd(q, k, v, do, 1, d, causal)
        assert np.abs(dq).max() == 0 and np.abs(dk).max() == 0
        assert np.array_equal(dv, do)


def test_brute_force_tiny(lib):
    """Tiny shapes: float64 direct softmax (numpy) for O/LSE, and float64
    central differences of <O, dO> over EVERY input entry for the gradients."""
    rng = np.random.default_rng(11)
    for n, d, causal in [(3, 4, False), (4, 8, True), (5, 2, True)]:
        q, k, v, do = (rng.standard_normal((n, d)).astype(np.float32) for _ in range(4))
        scale = oracle.default_scale(d)

        def fwd(q, k, v):
            s = q @ k.T * scale
            if causal:
                s = np.where(np.tril(np.ones((n, n), bool)), s, -np.inf)
            m = s.max(1, keepdims=True)
            p = np.exp(s - m)
            lsum = p.sum(1, keepdims=True)
            return (p / lsum) @ v, (m + np.log(lsum))[:, 0]

        q64, k64, v64, do64 = (x.astype(np.float64) for x in (q, k, v, do))
        o_ref, lse_ref = fwd(q64, k64, v64)
        o, lse = oracle.cpu_attention(q, k, v, n, d, causal)
        assert rel_max_err(o, o_ref) < 1e-6 and rel_max_err(lse, lse_ref) < 1e-6

        grads = oracle.cpu_attention_bwd(q, k, v, do, n, d, causal)
        eps = 1e-6
        for which, g in enumerate(grads):
            fd = np.zeros((n, d))
            for idx in np.ndindex(n, d):
                xs = [q64.copy(), k64.copy(), v64.copy()]
                xs[which][idx] += eps
                lp = (fwd(*xs)[0] * do64).sum()
                xs[which][idx] -= 2 * eps
                lm = (fwd(*xs)[0] * do64).sum()
                fd[idx] = (lp - lm) / (2 * eps)
            assert rel_max_err(g, fd) < 1e-5, (n, d, causal, which)


# ------------------------------------------------------------- generators --

def test_bf16_round_known_values_and_torch(lib):
    one = 1.0
    vals = np.array([one, one + 2 ** -8, one + 3 * 2 ** -8, -one - 2 ** -8, 0.0, -0.0,
                     3.0e38, np.inf, -np.inf], np.float32)
    want = np.array([one, one, one + 2 ** -6, -one, 0.0, -0.0, 2.9981e38, np.inf, -np.inf],
                    np.float32)
    got = oracle.bf16_round(vals)
    assert np.array_equal(got[:6], want[:6])
    assert np.isinf(got[-2]) and np.isinf(got[-1]) and got[-2] > 0 > got[-1]
    import torch
    x = oracle.normal(100000, 5, 3.0)
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(oracle.bf16_round(x), ref)


def test_normal_generator(lib):
    x = oracle.normal(1 << 20, 1).astype(np.float64)
    assert abs(x.mean()) < 5e-3 and abs(x.std() - 1.0) < 5e-3
    assert np.array_equal(oracle.normal(1001, 9, 0.5), oracle.normal(1001, 9, 0.5))
    assert np.array_equal(oracle.normal(1000, 9, 0.5), 0.5 * oracle.normal(1000, 9, 1.0))
