"""The oracle's QK RMS norm + rope (bko_norm_rope_row) against the reference's own attn_rms_norm /
attn_rope compiled from runtime_vk/attn_vk.h (oracle/_ref), and against what the mathematics fixes:
position 0 is the weighted norm alone, dims past n_rot pass through, the rotation keeps each pair's
length, a float64 recomputation agrees to ~1e-6, and the correctly rounded transcendentals (the
kernel contract) differ from the C library's float ones in only a few rows' last bits."""
import numpy as np
import pytest

import oracle

HD = 256


def rows(n, seed):
    x = oracle.normal(n * HD, seed, 900).reshape(n, HD)
    x[3] *= 40.0                                  # a large row
    x[5] *= 1e-3                                  # a small one
    w = 1.0 + 0.1 * oracle.normal(HD, seed, 901)
    return x.astype(np.float32), w.astype(np.float32)


def ideal(x, w, pos, nrot=oracle.NROT, eps=oracle.EPS, base=oracle.FREQ_BASE):
    x = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.sum(x * x) / HD + eps)
    n = x * inv * w.astype(np.float64)
    y = n.copy()
    half = nrot // 2
    p = np.arange(half)
    # the angle as the reference forms it in fp32 (theta, then pos * theta rounded): a large
    # position moves it by up to half an fp32 ulp of pos*theta, which no later step recovers
    ex = (np.float32(-2.0) * p.astype(np.float32)) / np.float32(nrot)
    th = (np.float64(base) ** ex.astype(np.float64)).astype(np.float32)
    a = (np.float32(pos) * th).astype(np.float64)
    y[:half] = n[:half] * np.cos(a) - n[half:nrot] * np.sin(a)
    y[half:nrot] = n[half:nrot] * np.cos(a) + n[:half] * np.sin(a)
    return y


@pytest.mark.skipif(oracle.ref() is None, reason="reference mirror not built (oracle/_ref)")
def test_libm_mode_is_the_reference_mirror_bit_for_bit():
    x, w = rows(40, 1)
    for i, pos in enumerate([0, 1, 7, 100, 4095, 32768, 65535, 123457] * 5):
        got = oracle.norm_rope_row(x[i], w, pos, libm_float=True)
        want = oracle.ref_norm_rope_row(x[i], w, pos)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (i, pos)


@pytest.mark.skipif(oracle.ref() is None, reason="reference mirror not built (oracle/_ref)")
def test_correctly_rounded_mode_against_the_mirror():
    """The kernel contract (correctly rounded pow/cos/sin) against the mirror's powf/cosf/sinf: the
    rows agree bit for bit except where a C-library float function is not correctly rounded (about a
    third of the rows have one such element), and there by about one fp32 ulp of the row's scale."""
    x, w = rows(64, 2)
    diff_rows = 0
    for i in range(64):
        pos = 37 * i * i + 5
        a = oracle.norm_rope_row(x[i], w, pos)
        b = oracle.ref_norm_rope_row(x[i], w, pos)
        if not np.array_equal(a, b):
            diff_rows += 1
            assert np.max(np.abs(a - b)) <= 4e-7 * np.max(np.abs(b))
    print(f"rows differing from the C library's float transcendentals: {diff_rows}/64")


def test_closed_forms():
    x, w = rows(8, 3)
    for i in range(8):
        y0 = oracle.norm_rope_row(x[i], w, 0)
        ss = np.float32(0)
        for v in x[i]:
            ss = np.float32(ss + np.float32(v * v))
        inv = np.float32(1) / np.sqrt(np.float32(ss / np.float32(HD) + np.float32(oracle.EPS)))
        n = (x[i] * inv) * w
        assert np.array_equal(y0, n)                       # cos 0 = 1, sin 0 = 0
        y = oracle.norm_rope_row(x[i], w, 12345)
        assert np.array_equal(y[oracle.NROT:], n[oracle.NROT:])
        h = oracle.NROT // 2
        l0 = np.hypot(n[:h].astype(np.float64), n[h:oracle.NROT])
        l1 = np.hypot(y[:h].astype(np.float64), y[h:oracle.NROT])
        assert np.allclose(l0, l1, rtol=1e-6, atol=1e-9)
        assert np.allclose(y, ideal(x[i], w, 12345), rtol=2e-5, atol=2e-6 * np.abs(n).max())


def test_norm_rope_append_host():
    """The fused append: Q rows come back normed + roped, K rows land in the cache normed + roped
    (fp16 here, so the cache holds f16(y)), V rows land raw."""
    c = oracle.HostCache(n_layers=1, cap=16, k_fmt=oracle.F16, v_fmt=oracle.F16)
    q = oracle.normal(2 * 16 * HD, 4, 1).reshape(2, 16, HD)
    k = oracle.normal(2 * 4 * HD, 4, 2).reshape(2, 4, HD)
    v = oracle.normal(2 * 4 * HD, 4, 3).reshape(2, 4, HD)
    qw = (1 + 0.1 * oracle.normal(HD, 4, 4)).astype(np.float32)
    kw = (1 + 0.1 * oracle.normal(HD, 4, 5)).astype(np.float32)
    qo = c.norm_rope_append(0, 6, q, k, v, qw, kw)
    for t in range(2):
        assert np.array_equal(qo[t, 3], oracle.norm_rope_row(q[t, 3], qw, 6 + t))
        kr = oracle.norm_rope_row(k[t, 2], kw, 6 + t)
        assert np.array_equal(c.row(0, 0, 6 + t, 2), kr.astype(np.float16).astype(np.float32))
        assert np.array_equal(c.row(1, 0, 6 + t, 1), v[t, 1].astype(np.float16).astype(np.float32))
