"""Pins the CPU oracle to the reference's own known answers.

Every unit test of the reference crate for the hot path is restated here
(resolver.rs:133-189, config.rs:131-153, mat.rs:152-176,
cross_entropy.rs:92-148, kl.rs:160-223, quant.rs:209-275), plus checks
that the mathematics fixes independently of the oracle's formulas
(textbook cross-entropy against a smoothed target distribution, brute-force
f64 GEMMs, finite-difference KL gradients, published SplitMix64 outputs).
"""
import math

import numpy as np
import pytest

import oracle as O
from orda_hip.types import ChunkSize, KernelConfig, Profile


# --------------------------------------------------------------- resolver.rs
def test_fixed_chunking():
    # resolver.rs:137-150
    p = O.resolve_chunk_size(1000, ChunkSize.Fixed(256), None, None)
    assert (p.chunk_size, p.num_chunks) == (256, 4)
    p = O.resolve_chunk_size(100, ChunkSize.Fixed(4096), None, None)
    assert (p.chunk_size, p.num_chunks) == (100, 1)


def test_auto_without_vocab_is_single_chunk():
    # resolver.rs:152-162
    p = O.resolve_chunk_size(8192, ChunkSize.Auto, None, None)
    assert (p.chunk_size, p.num_chunks) == (8192, 1)


def test_chunks_from_raw_matches_python_rule():
    # resolver.rs:164-174
    assert O.chunks_from_raw(0.0) == 1
    assert O.chunks_from_raw(1.49) == 1
    assert O.chunks_from_raw(1.5) == 2
    assert O.chunks_from_raw(3.0) == 4
    assert O.chunks_from_raw(6.0) == 8


def test_auto_large_vocab_example():
    # resolver.rs:176-185: README case BT=8192, V=131072 -> 16 x 512
    p = O.resolve_chunk_size(8192, ChunkSize.Auto, 131072, None)
    assert (p.num_chunks, p.chunk_size) == (16, 512)


def test_doubling_schedule_escalates_to_limit():
    # resolver.rs:187-193
    assert O.chunk_doubling_schedule(10_000, 4, 32) == [4, 8, 16, 32]
    assert O.chunk_doubling_schedule(20, 4, 1000) == [4, 8, 16, 20]


@pytest.mark.parametrize("bt,v,plan", [
    (256, 8192, (256, 1)),        # Tied 256/512/8192
    (2048, 32000, (1024, 2)),     # Tied 2048/4096/32000
    (4096, 32000, (1024, 4)),     # Separate 4096/32000
    (4096, 65536, (512, 8)),      # Precomputed 4096/65536
    (8192, 131072, (512, 16)),    # Tied 8192/4096/131072
])
def test_benchmark_shape_plans(bt, v, plan):
    """The closed form of resolver.rs:69-97 worked by hand for each shape."""
    max_useful = max(bt // 512, 1)
    raw = max((bt / 1024) * (v / 32768) ** 2, bt / 4096)
    n = 1 if raw < 1.5 else 2 ** (math.floor(math.log2(raw / 1.5)) + 1)
    n = max(min(n, 2 * max_useful, max_useful, bt), 1)
    assert (-(-bt // n), n) == plan
    p = O.resolve_chunk_size(bt, ChunkSize.Auto, v, None)
    assert (p.chunk_size, p.num_chunks) == plan


def test_auto_respects_max_chunks_and_bt():
    p = O.resolve_chunk_size(8192, ChunkSize.Auto, 131072, 4)
    assert (p.chunk_size, p.num_chunks) == (2048, 4)
    # tiny BT: max_useful = 1
    p = O.resolve_chunk_size(7, ChunkSize.Auto, 10**6, None)
    assert (p.chunk_size, p.num_chunks) == (7, 1)
    assert O.default_max_chunks_limit(8192) == 32
    assert O.default_max_chunks_limit(100) == 2


# --------------------------------------------------------------- config.rs
def test_config_profiles_and_pow2():
    # config.rs:131-153
    assert not KernelConfig.from_profile(Profile.Balanced).fast_math
    assert KernelConfig.from_profile(Profile.Fast).fast_math
    assert not KernelConfig.from_profile(Profile.Debug).fast_math
    for p in [1, 2, 4, 8, 1024, 32768]:
        assert O.is_power_of_two(p)
    for n in [0, 3, 6, 100, 65535]:
        assert not O.is_power_of_two(n)


# --------------------------------------------------------------- mat.rs
def test_matmul_known_answers():
    # mat.rs:152-176
    c = O.matmul_nt(np.array([[1, 2, 3]], np.float32),
                    np.array([[1, 0, 0], [0, 1, 1]], np.float32))
    assert c.tolist() == [[1.0, 5.0]]
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[1, 0, 1], [0, 1, 0]], np.float32)
    assert O.matmul_tn(a, b).tolist() == [[1, 3, 1], [2, 4, 2]]
    assert O.matmul_nn(a, b).tolist() == [[1, 2, 1], [3, 4, 3]]


def test_matmul_brute_force_f64():
    rng = np.random.default_rng(0)
    a = rng.standard_normal((13, 37)).astype(np.float32)
    b = rng.standard_normal((29, 37)).astype(np.float32)
    d = rng.standard_normal((37, 11)).astype(np.float32)
    e = rng.standard_normal((13, 11)).astype(np.float32)
    ref_nt = a.astype(np.float64) @ b.astype(np.float64).T
    ref_nn = a.astype(np.float64) @ d.astype(np.float64)
    ref_tn = a.astype(np.float64).T @ e.astype(np.float64)
    np.testing.assert_allclose(O.matmul_nt(a, b), ref_nt, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.matmul_nn(a, d), ref_nn, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(O.matmul_tn(a, e), ref_tn, rtol=1e-5, atol=1e-5)
    # matmul_nt's dot is sequential f32 from 0 (mat.rs:72-75)
    acc = np.float32(0.0)
    for p in range(37):
        acc = np.float32(acc + np.float32(a[3, p] * b[5, p]))
    assert O.matmul_nt(a, b)[3, 5] == acc


# --------------------------------------------------------------- cross_entropy.rs
def _softmax64(x):
    x = np.asarray(x, np.float64)
    e = np.exp(x - x.max())
    return e / e.sum()


def test_nll_equals_negative_log_softmax_of_target():
    # cross_entropy.rs:92-100
    x = [1.0, 2.0, 0.5, -1.0]
    nll = O.ce_loss_row(x, 1, -100, 0.0)
    assert abs(nll - (-math.log(_softmax64(x)[1]))) < 1e-6


def test_grad_is_softmax_minus_onehot():
    # cross_entropy.rs:102-121
    x = [0.3, -0.7, 1.1, 0.0]
    _, g = O.ce_fwdbwd_row(x, 2, -100, 0.0, 1.0)
    p = _softmax64(x)
    p[2] -= 1.0
    np.testing.assert_allclose(g, p, atol=1e-6)
    assert abs(float(np.sum(g, dtype=np.float64))) < 1e-5


def test_ignored_row_is_zero():
    # cross_entropy.rs:123-129
    nll, g = O.ce_fwdbwd_row([3.0, 1.0, -2.0], -100, -100, 0.0, 1.0)
    assert nll == 0.0 and np.all(g == 0.0)


def test_scale_scales_gradient():
    # cross_entropy.rs:131-139
    x = [0.5, -0.5, 1.0]
    _, g1 = O.ce_fwdbwd_row(x, 0, -100, 0.0, 1.0)
    _, g2 = O.ce_fwdbwd_row(x, 0, -100, 0.0, 2.5)
    np.testing.assert_allclose(g2, 2.5 * g1, atol=1e-6)


def test_label_smoothing_grad_sums_to_zero():
    # cross_entropy.rs:141-148
    _, g = O.ce_fwdbwd_row([0.2, 1.3, -0.4, 0.9, 0.0], 3, -100, 0.1, 1.0)
    assert abs(float(np.sum(g, dtype=np.float64))) < 1e-5


@pytest.mark.parametrize("alpha", [0.0, 0.1, 0.37, 1.0])
def test_label_smoothing_is_textbook_cross_entropy(alpha):
    """nll = -Σ q_j log p_j with q = (1-α)·onehot + α/V, and
    grad = scale·(p − q): derived from the definition, not the oracle's
    rearranged lse form."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal(23).astype(np.float32) * 3
    y, scale = 5, 0.75
    p = _softmax64(x)
    q = np.full(23, alpha / 23)
    q[y] += 1 - alpha
    nll, g = O.ce_fwdbwd_row(x, y, -100, alpha, scale)
    assert abs(nll - float(-(q * np.log(p)).sum())) < 2e-6 * max(1.0, abs(nll))
    np.testing.assert_allclose(g, scale * (p - q), atol=1e-7, rtol=1e-6)


# --------------------------------------------------------------- kl.rs
def test_identical_distributions_have_zero_kl():
    # kl.rs:160-165
    row = [0.3, 1.2, -0.7, 2.1, 0.0]
    assert abs(O.forward_kl_row(row, row, 1.5)) < 1e-12


def test_kl_is_nonnegative():
    # kl.rs:167-175
    s = [0.1, 0.2, 0.3, -1.0, 2.0]
    t = [1.0, -0.5, 0.0, 0.7, 0.2]
    for temp in [0.5, 1.0, 1.5, 4.0]:
        assert O.forward_kl_row(s, t, temp) >= -1e-12


def test_kl_matches_closed_form_two_class():
    # kl.rs:177-197
    T = 2.0
    s, t = [0.7, -0.4], [-0.2, 1.1]

    def sig(a, b):
        za, zb = float(np.float32(a)) * (1 / T), float(np.float32(b)) * (1 / T)
        m = max(za, zb)
        d = math.exp(za - m) + math.exp(zb - m)
        return math.exp(za - m) / d, math.exp(zb - m) / d
    ps0, ps1 = sig(*s)
    pt0, pt1 = sig(*t)
    expected = pt0 * (math.log(pt0) - math.log(ps0)) + pt1 * (math.log(pt1) - math.log(ps1))
    assert abs(O.forward_kl_row(s, t, T) - expected) < 1e-12


def test_kl_ignored_rows_contribute_zero():
    # kl.rs:199-207
    lc = np.array([[1, 2, 3], [0.5, -0.5, 0]], np.float32)
    kl, g = O.kl_reference_chunk(lc, [-100], 1, 0.4, 1.5, 1, -100, True)
    assert kl == 0.0 and np.all(g == 0.0)


def test_kl_grad_matches_temperature_scaling():
    # kl.rs:209-222
    lc = np.array([[0.2, 0.5, -0.1], [1.0, -1.0, 0.3]], np.float32)
    kw, temp = 0.4, 1.5
    _, g = O.kl_reference_chunk(lc, [1], 1, kw, temp, 1, -100, True)
    ps, _ = O.softmax_logsoftmax(lc[0], 1 / temp)
    pt, _ = O.softmax_logsoftmax(lc[1], 1 / temp)
    gs = np.float32(kw) * np.float32(temp)
    np.testing.assert_allclose(g[0], (gs * (ps - pt)).astype(np.float32), atol=1e-6)


def test_kl_gradient_is_derivative_of_scaled_kl():
    """d/ds [kd·T²·KL(p_t || p_s)] = kd·T·(p_s − p_t), checked by central
    differences of the f64 row KL (independent of kl_chunk's grad formula)."""
    rng = np.random.default_rng(3)
    v, kd, T = 9, 0.6, 1.7
    lc = rng.standard_normal((2, v)).astype(np.float32)
    kl, g = O.kl_chunk(lc, [2], 1, kd, T, -100, 1.0, True)
    # kl_chunk reports Σ KL_row·T² (T² computed in f32)
    t_sq = float(np.float32(T) * np.float32(T))
    assert abs(kl - O.forward_kl_row(lc[0], lc[1], T) * t_sq) < 1e-6
    eps = 1e-3
    for j in range(v):
        sp, sm = lc[0].astype(np.float64), lc[0].astype(np.float64)
        sp = sp.copy(); sp[j] += eps
        sm = sm.copy(); sm[j] -= eps
        f = lambda s: kd * T * T * _kl64(s, lc[1].astype(np.float64), T)  # noqa: E731
        num = (f(sp) - f(sm)) / (2 * eps)
        assert abs(num - g[0, j]) < 1e-5, (j, num, g[0, j])


def _kl64(s, t, T):
    ps, pt = _softmax64(s / T), _softmax64(t / T)
    return float((pt * (np.log(pt) - np.log(ps))).sum())


# --------------------------------------------------------------- quant.rs
def test_round_half_even_cases():
    # quant.rs:209-217
    for x, r in [(0.5, 0.0), (1.5, 2.0), (2.5, 2.0), (-1.5, -2.0), (2.4, 2.0), (2.6, 3.0),
                 (-2.5, -2.0), (-0.5, -0.0), (3.5, 4.0)]:
        assert O.round_half_even(x) == r
    # agrees with IEEE round-to-nearest-even (numpy.rint) on many f32 values
    xs = np.concatenate([np.arange(-300, 300) / 2, np.random.default_rng(0).normal(0, 60, 2000)])
    xs = xs.astype(np.float32)
    assert all(O.round_half_even(float(x)) == float(np.rint(x)) for x in xs)


def test_deterministic_roundtrip_bounded_error():
    # quant.rs:219-232
    m = np.array([[1.0, -2.0, 0.5, 3.0], [-0.1, 0.2, -0.3, 0.05]], np.float32)
    q, s = O.quantize_rowwise_int8(m)
    deq = O.dequantize(q, s)
    for r in range(2):
        assert np.all(np.abs(m[r] - deq[r]) <= 0.5 * s[r] + 1e-6)
    # scale = max(amax, 1e-12)/127 in f32; amax row maps to ±127
    assert s[0] == np.float32(3.0) / np.float32(127.0)
    assert q[0, 3] == 127 and q[1, 2] == -127


def test_stochastic_is_unbiased():
    # quant.rs:234-251
    m = np.array([[0.37, -1.23, 2.71]], np.float32)
    rng = O.Rng(12345)
    acc = np.zeros(3)
    n = 20_000
    for _ in range(n):
        q, s = O.quantize_rowwise_int8_stochastic(m, rng)
        acc += O.dequantize(q, s)[0]
    assert np.all(np.abs(acc / n - m[0]) < 1e-2)


def test_grad_w_target_rows_are_exact():
    # quant.rs:253-269
    g = np.array([[10, -10], [0.123, 0.456], [-7, 7], [0.01, -0.02]], np.float32)
    assert O.unique_targets([0, 2, -100], -100, 4) == [0, 2]
    deq, _, _ = O.quant_dequant_grad_w(g, [0, 2, -100], -100)
    assert np.array_equal(deq[0], g[0]) and np.array_equal(deq[2], g[2])
    assert np.all(np.abs(deq[1] - g[1]) < 0.02)


def test_splitmix64_published_outputs():
    """Vigna's splitmix64.c reference sequence: state 0 gives
    0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
    0xF88BB8A8724C81EC; state 1234567 starts 6457827717110365317,
    3203168211198807973. Rng::new(seed) pre-adds the gamma (quant.rs:24-26),
    so Rng(0)'s first draw is the second output of state 0."""
    import ctypes
    st = ctypes.c_uint64(0)
    outs = [O.lib().ora_rng_next_u64(ctypes.byref(st)) for _ in range(4)]
    assert outs == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                    0xF88BB8A8724C81EC]
    st = ctypes.c_uint64(1234567)
    assert [O.lib().ora_rng_next_u64(ctypes.byref(st)) for _ in range(2)] == \
        [6457827717110365317, 3203168211198807973]
    r = O.Rng(0)
    assert r.next_u64() == 0x6E789E6AA1B965F4
    # next_f32 = (u64 >> 40) * 2^-24 (quant.rs:39-43)
    assert O.Rng(0).next_f32() == np.float32((0x6E789E6AA1B965F4 >> 40) * 2.0 ** -24)


def test_stochastic_codes_follow_rng_stream_row_major():
    """The code at flat index e uses the e-th draw of Rng(seed), including
    target rows (quant.rs:129-136, 163-187)."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal((5, 7)).astype(np.float32)
    _, q, s = O.quant_dequant_grad_w(g, [1, 3], -100, stochastic=True, seed=99)
    r = O.Rng(99)
    for i in range(5):
        for j in range(7):
            scaled = np.float32(g[i, j] / s[i])
            fl = np.floor(scaled)
            u = r.next_f32()
            exp = np.clip(fl + (1.0 if (scaled - fl) > np.float32(u) else 0.0), -127, 127)
            assert q[i, j] == int(exp)
