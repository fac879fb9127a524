"""Decode attention of the oracle, pinned bit-for-bit to the reference's own CPU mirror
(runtime_vk/attn_vk.h compiled into oracle/_ref) and by closed forms."""
import ctypes

from fractions import Fraction

import numpy as np
import pytest

import oracle
from oracle import F16, Q8_0


def make_cache(nfill, k_fmt, v_fmt, seed=0, cap=None, outliers=0, **kw):
    c = oracle.HostCache(n_layers=1, cap=cap or nfill, k_fmt=k_fmt, v_fmt=v_fmt, **kw)
    k, v = oracle.synth_kv(nfill, 4, 256, seed, 0, outliers=outliers)
    c.append(0, 0, k, v)
    return c, k, v


def q_gate(seed, n=1):
    q = oracle.normal(n * 16 * 256, seed, 77).reshape(n, 16, 256)
    g = oracle.normal(n * 16 * 256, seed, 78).reshape(n, 16, 256)
    return (q[0], g[0]) if n == 1 else (q, g)


def test_config1_matches_reference_mirror_bitwise():
    """BASELINE config 1 (1 layer, 256 tokens, f16 K/V, seed 0) through the reference's
    attn_score_row / attn_softmax_row / P16 / attn_pv_row / attn_gate_row."""
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    nfill = 256
    c, _, _ = make_cache(nfill, F16, F16, seed=0)
    q, g = q_gate(0)
    with oracle.exp_mode(1):                      # the mirror calls std::exp(float)
        out, og, sc, pr, p16 = c.decode(0, nfill, q, g, debug=True)
    q16 = oracle.f32_to_f16(q).view(np.uint32).reshape(16, 128)
    kc = np.ascontiguousarray(c.k_data[0]).view(np.uint32)
    vc = np.ascontiguousarray(c.v_data[0]).view(np.uint32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    for h in range(16):
        rs, rp = np.empty(nfill, np.float32), np.empty(nfill, np.float32)
        r16 = np.empty(nfill, np.uint16)
        ro, rg = np.empty(256, np.float32), np.empty(256, np.float32)
        qh = np.ascontiguousarray(q16[h])
        gh = np.ascontiguousarray(g[h])
        R.ref_decode_row(256, 16, 4, ctypes.c_float(0.0625), P(qh), P(kc), P(vc), h // 4, nfill,
                         P(gh), P(rs), P(rp), P(r16), P(ro), P(rg))
        assert oracle.bit_diff(sc[h], rs) == 0
        assert oracle.bit_diff(pr[h], rp) == 0
        assert np.array_equal(p16[h], r16)
        assert oracle.bit_diff(out[h], ro) == 0
        assert oracle.bit_diff(og[h], rg) == 0


def test_reference_rows_driver_matches_rows():
    """ref_decode_rows (the reference's rows under OpenMP, timed as the CPU baseline) gives, for 2
    layers x 16 heads, the oracle's pre-gate output of each layer's rows, bit for bit."""
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref not built (reference checkout absent)")
    nfill = 300
    c, _, _ = make_cache(nfill, F16, F16, seed=3)
    c2, _, _ = make_cache(nfill, F16, F16, seed=4)
    q = np.stack([q_gate(3)[0], q_gate(4)[0]])
    g = np.zeros_like(q)
    kc = np.ascontiguousarray(np.stack([c.k_data[0], c2.k_data[0]])).view(np.uint32)
    vc = np.ascontiguousarray(np.stack([c.v_data[0], c2.v_data[0]])).view(np.uint32)
    q16 = np.ascontiguousarray(oracle.f32_to_f16(q).view(np.uint32))
    out = np.empty((2, 16, 256), np.float32)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    R.ref_decode_rows(256, 16, 4, ctypes.c_float(0.0625), 2, P(q16), P(kc), P(vc), kc[0].size, nfill,
                      P(g), P(out), 4)
    with oracle.exp_mode(1):
        for i, cc in enumerate((c, c2)):
            want, _ = cc.decode(0, nfill, q[i])
            assert oracle.bit_diff(out[i], want) == 0


def test_single_key_probability_is_one():
    c, _, v = make_cache(1, Q8_0, Q8_0, seed=5)
    q, _ = q_gate(5)
    out, _, _, pr, p16 = c.decode(0, 1, q, debug=True)
    assert np.all(pr == 1.0) and np.all(p16 == 0x3C00)
    for h in range(16):
        assert np.array_equal(out[h], c.row(1, 0, 0, h // 4))


def test_identical_keys_uniform_and_mean():
    n = 64
    c = oracle.HostCache(n_layers=1, cap=n, k_fmt=F16, v_fmt=F16)
    k1, _ = oracle.synth_kv(1, 4, 256, 9, 0)
    _, v = oracle.synth_kv(n, 4, 256, 9, 1)
    c.append(0, 0, np.repeat(k1, n, axis=0), v)
    q, _ = q_gate(9)
    out, _, _, pr, p16 = c.decode(0, n, q, debug=True)
    assert np.all(pr == np.float32(1.0 / n)) and np.all(p16 == oracle.f32_to_f16(np.float32(1 / n)))
    vc = np.stack([[c.row(1, 0, j, g) for g in range(4)] for j in range(n)])   # [n][4][256]
    # PV with p = 1/64 exact: the sum is 1/64 * serial sum of V, computed in fp32 ascending
    for h in range(16):
        acc = np.zeros(256, np.float32)
        for j in range(n):
            acc = acc + np.float32(1 / n) * vc[j, h // 4]
        assert np.array_equal(acc, out[h])


def test_gqa_identical_queries_identical_rows():
    c, _, _ = make_cache(300, Q8_0, Q8_0, seed=4, outliers=3)
    q, _ = q_gate(4)
    q[4:8] = q[4]
    out, _, sc, _, _ = c.decode(0, 300, q, debug=True)
    for h in range(5, 8):
        assert np.array_equal(sc[h], sc[4]) and np.array_equal(out[h], out[4])


def test_sum_of_probabilities_and_dead_order():
    c, _, _ = make_cache(1000, Q8_0, Q8_0, seed=2, outliers=3)
    q, _ = q_gate(2)
    _, _, _, pr, _ = c.decode(0, 1000, q, debug=True)
    assert np.all(np.abs(pr.astype(np.float64).sum(axis=1) - 1) < 1e-4)


def test_ideal_leg_against_numpy_float64():
    n = 200
    c, _, _ = make_cache(n, Q8_0, F16, seed=3, outliers=3)
    q, _ = q_gate(3)
    K = np.stack([[c.row(0, 0, j, g) for g in range(4)] for j in range(n)]).astype(np.float64)
    V = np.stack([[c.row(1, 0, j, g) for g in range(4)] for j in range(n)]).astype(np.float64)
    for rb in (0, 1, 3):
        got = c.ideal(0, n, q, round_bits=rb)
        qq = oracle.f16_to_f32(oracle.f32_to_f16(q)).astype(np.float64) if rb & 1 else q.astype(np.float64)
        for h in range(16):
            s = K[:, h // 4] @ qq[h] * 0.0625
            p = np.exp(s - s.max())
            p /= p.sum()
            if rb & 2:
                p = oracle.f16_to_f32(oracle.f32_to_f16(p.astype(np.float32))).astype(np.float64)
            np.testing.assert_allclose(got[h], p @ V[:, h // 4], rtol=1e-10, atol=1e-12)
    # the fp32 mirror against its fp64 twin (same fp16 roundings): the gap is dominated by fp16
    # probabilities that land on the other side of a rounding boundary (~1 fp16 ulp each)
    out, _ = c.decode(0, n, q)
    assert oracle.rel_err(out, c.ideal(0, n, q, round_bits=3)) < 1e-3


def test_paged_equals_contiguous():
    n, page = 700, 64
    rng = np.random.default_rng(1)
    pool = 16
    bt = rng.permutation(pool)[None, :].astype(np.int32)
    cp = oracle.HostCache(n_layers=1, cap=pool * page, page_tokens=page, max_pages=pool,
                          block_table=bt)
    cc = oracle.HostCache(n_layers=1, cap=n)
    k, v = oracle.synth_kv(n, 4, 256, 6, 0, outliers=3)
    cp.append(0, 0, k, v)
    cc.append(0, 0, k, v)
    # gather indices: slot = bt[pos // page] * page + pos % page
    for pos in (0, 63, 64, 65, 699):
        assert cp.slot(0, pos) == bt[0, pos // page] * page + pos % page
    for pos in range(n):
        assert np.array_equal(cp.k_data[0, cp.slot(0, pos)], cc.k_data[0, pos])
    q, g = q_gate(6)
    a, ag = cp.decode(0, n, q, g)
    b, bg = cc.decode(0, n, q, g)
    assert oracle.bit_diff(a, b) == 0 and oracle.bit_diff(ag, bg) == 0


def test_prefill_rows_equal_decode():
    pos0, nq = 50, 5
    c, _, _ = make_cache(pos0 + nq, Q8_0, Q8_0, seed=8)
    q, g = q_gate(8, nq)
    out, og = c.prefill(0, pos0, q, g)
    for i in range(nq):
        o, gg = c.decode(0, pos0 + i + 1, q[i], g[i])
        assert oracle.bit_diff(out[i], o) == 0 and oracle.bit_diff(og[i], gg) == 0


def test_threads_do_not_change_numbers():
    c, _, _ = make_cache(500, Q8_0, Q8_0, seed=12)
    q, g = q_gate(12)
    a, ag = c.decode(0, 500, q, g, nthreads=1)
    b, bg = c.decode(0, 500, q, g, nthreads=4)
    assert oracle.bit_diff(a, b) == 0 and oracle.bit_diff(ag, bg) == 0


def test_exp_modes_differ_only_where_libm_is_not_correctly_rounded():
    c, _, _ = make_cache(2048, Q8_0, Q8_0, seed=13, outliers=3)
    q, g = q_gate(13)
    a, ag, _, pa, _ = c.decode(0, 2048, q, g, debug=True)
    with oracle.exp_mode(1):
        b, bg, _, pb, _ = c.decode(0, 2048, q, g, debug=True)
    # almost every probability is bit-identical, and the outputs agree far inside the tolerance
    assert (pa != pb).mean() < 0.01
    assert oracle.rel_err(a, b) < 1e-4 and oracle.rel_err(ag, bg) < 1e-4


def _exact_q8_inner(q16_row, i8_block):
    """The exact rational sum of q16 * int8 over one block, rounded once to fp32. The sum is a
    multiple of 2^-24 below 2^28, so float() of the Fraction is exact and only np.float32 rounds."""
    s = sum((Fraction(float(a)) * int(b) for a, b in zip(q16_row, i8_block)), Fraction(0))
    return np.float32(float(s))


def test_q8_k_dot_is_block_factored():
    """q8_0 K: score = sum in block order of f16(scale) * inner_b, inner_b = the exact sum of
    q16 * int8 over the block rounded once to fp32 (checked here with exact rational arithmetic)."""
    n = 8
    c, _, _ = make_cache(n, Q8_0, F16, seed=14, outliers=3)
    q, _ = q_gate(14)
    # edge operands: fp16 subnormal q, a max-magnitude q and a q that rounds to zero
    q[0, 3] = 3e-7
    q[1, 40] = 60000.0
    q[2, 7] = 1e-9
    _, _, sc, _, _ = c.decode(0, n, q, debug=True)
    q16 = oracle.f16_to_f32(oracle.f32_to_f16(q))
    i8 = c.k_data[0].view(np.int8).reshape(n, 4, 8, 32)
    s = c.k_scales[0].view(np.float16).reshape(n, 4, 8).astype(np.float32)
    for h in range(16):
        for j in range(n):
            acc = np.float32(0)
            for b in range(8):
                inner = _exact_q8_inner(q16[h, 32 * b:32 * b + 32], i8[j, h // 4, b])
                acc = np.float32(acc + np.float32(s[j, h // 4, b] * inner))
            assert acc == sc[h, j]


def test_q8_k_inner_is_correctly_rounded_not_serial():
    """A block whose serial fp32 chain rounds differently from the exact sum: the oracle's score
    follows the exact sum (the property that makes the inner sum order-free)."""
    n = 1
    c, _, _ = make_cache(n, Q8_0, F16, seed=3, outliers=0)
    i8 = c.k_data[0].view(np.int8).reshape(n, 4, 8, 32).copy()
    i8[0, 0, 0, :] = 0
    i8[0, 0, 0, 0], i8[0, 0, 0, 1], i8[0, 0, 0, 2] = 127, 1, -127
    c.k_data[0][:] = i8.view(np.uint8).reshape(c.k_data[0].shape)
    q = np.zeros((16, 256), np.float32)
    q[0, 0], q[0, 1], q[0, 2] = 2048.0, 2.0 ** -14, 2048.0   # serial: (2048*127 + tiny) - 2048*127 = 0
    _, _, sc, _, _ = c.decode(0, n, q, debug=True)
    sc0 = np.float32(c.k_scales[0].view(np.float16).reshape(n, 4, 8)[0, 0, 0])
    assert sc[0, 0] == np.float32(sc0 * np.float32(2.0 ** -14))
    serial = np.float32(np.float32(2048.0 * 127) + np.float32(2.0 ** -14)) - np.float32(2048.0 * 127)
    assert serial == 0.0 and sc[0, 0] != 0.0
