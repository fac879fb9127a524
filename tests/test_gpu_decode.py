"""GPU parity of the decode path (libbkv.so through the C ABI) against the CPU oracle.
Bar: q8_0/fp16 cache bytes and scales bit-exact; attention outputs within max relative error
1e-4 (max |gpu - oracle| / max |oracle| per head row), bit-diff counts printed."""
import numpy as np
import pytest
import torch

import oracle
from bonsai_vk_amd import BKV_F16, BKV_Q8_0
from tests.gpu_util import fill, pair, qg, report, same_bytes, say

TOL = 1e-4
pytestmark = pytest.mark.gpu


@pytest.fixture(params=["fused", "split"])
def path(request, monkeypatch):
    """Run a test through both decode implementations (the library reads BKV_DECODE per call)."""
    if request.param == "split":
        monkeypatch.setenv("BKV_DECODE", "split")
    else:
        monkeypatch.delenv("BKV_DECODE", raising=False)
    return request.param
FMTS = [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16), (BKV_F16, BKV_Q8_0), (BKV_Q8_0, BKV_F16)]


@pytest.mark.parametrize("kf,vf", FMTS)
def test_append_bit_exact(kf, vf):
    say(f"append kf={kf} vf={vf}")
    dev, host = pair(2, 300, kf, vf)
    k, v = oracle.synth_kv(300, 4, 256, 21, 1, outliers=3)
    # special values: zeros, a dead block, exact ties at d = 1, huge, tiny, NaN, inf
    k[0, 0, :32] = 0
    v[1, 2, 32:64] = 1e-37
    k[2, 1, 0:8] = [127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 126.5, -126.5]
    k[2, 1, 8:32] = 0
    v[3, 0, 5] = np.nan
    v[3, 3, 100] = np.inf
    k[4, 2, 200] = 7e4
    host.append(1, 0, k, v)
    dev.append(1, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    torch.cuda.synchronize()
    assert same_bytes(dev, host) == [0] * len(same_bytes(dev, host))


@pytest.mark.parametrize("kf,vf", FMTS)
@pytest.mark.parametrize("nfill", [1, 17, 256, 1000, 4097])
def test_decode_matches_oracle(kf, vf, nfill, path):
    say(f"decode kf={kf} vf={vf} nfill={nfill} path={path}")
    dev, host = pair(1, nfill, kf, vf)
    fill(dev, host, 0, nfill, seed=nfill)
    q, g = qg(nfill, 0)
    want, wg = host.decode(0, nfill, q, g, nthreads=8)
    out, og = dev.decode(0, nfill, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert report("out", out.cpu().numpy(), want) <= TOL
    assert report("gated", og.cpu().numpy(), wg) <= TOL


def test_config1_f16_256():
    """1 layer, 256 cached f16 tokens, 16Q/4KV, seed 0."""
    dev, host = pair(1, 256, BKV_F16, BKV_F16)
    fill(dev, host, 0, 256, seed=0, outliers=0)
    q, g = qg(0, 0)
    want, _ = host.decode(0, 256, q)
    out, _ = dev.decode(0, 256, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    assert report("config1", out.cpu().numpy(), want) <= TOL


def test_config2_decode_step_8_layers(path):
    """8 layers at 4096 context, q8_0 K+V, one token appended per layer with the
    fused decode_step, then GQA attention; cache bytes bit-exact afterwards."""
    n = 4096
    dev, host = pair(8, n + 1, BKV_Q8_0, BKV_Q8_0)
    worst = 0.0
    for layer in range(8):
        fill(dev, host, layer, n, seed=1)
        kn, vn = oracle.synth_kv(1, 4, 256, 101, layer, outliers=3)
        host.append(layer, n, kn, vn)
        q, g = qg(1, layer)
        want, wg = host.decode(layer, n + 1, q, g, nthreads=8)
        out, og = dev.decode_step(layer, n, torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda(),
                                  torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
        torch.cuda.synchronize()
        worst = max(worst, report(f"layer {layer}", out.cpu().numpy(), want),
                    oracle.rel_err(og.cpu().numpy(), wg))
    assert same_bytes(dev, host) == [0, 0, 0, 0]
    assert worst <= TOL


def test_decode_step_equals_append_then_decode(path):
    n = 2000
    a, _ = pair(1, n + 1, BKV_Q8_0, BKV_Q8_0)
    b, host = pair(1, n + 1, BKV_Q8_0, BKV_Q8_0)
    fill(a, host, 0, n, seed=3)
    fill(b, host, 0, n, seed=3)
    kn, vn = oracle.synth_kv(1, 4, 256, 33, 0)
    q, _ = qg(3, 0)
    kt, vt, qt = (torch.from_numpy(x).cuda() for x in (kn, vn, q))
    o1, _ = a.decode_step(0, n, kt, vt, qt)
    b.append(0, n, kt, vt)
    o2, _ = b.decode(0, n + 1, qt)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)
    assert all(torch.equal(x, y) for x, y in zip(a.host_arrays(), b.host_arrays()) if x is not None)


def test_deterministic_repeat(path):
    n = 20000
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n, seed=5)
    q, _ = qg(5, 0)
    qt = torch.from_numpy(q).cuda()
    o1, _ = dev.decode(0, n, qt)
    o1 = o1.clone()
    o2, _ = dev.decode(0, n, qt)
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


@pytest.mark.parametrize("kf,vf,n,seed", [(BKV_Q8_0, BKV_Q8_0, 4097, 1), (BKV_F16, BKV_F16, 3000, 7),
                                          (BKV_Q8_0, BKV_Q8_0, 40000, 2)])
def test_scores_probabilities_and_sum_bit_exact(kf, vf, n, seed, path):
    """The intermediates the reference's bitwise gate (BONSAI_QCHECK stages A/B) compares: every score,
    every e_j = exp(s_j*scale - max) and the serial fp32 softmax sum match the oracle bit for bit, and
    so do the fp16 probabilities formed from them."""
    say(f"bit-exact intermediates kf={kf} n={n}")
    dev, host = pair(1, n, kf, vf)
    fill(dev, host, 0, n, seed=seed)
    q, _ = qg(seed, 0)
    want, _, sc, pr, p16 = host.decode(0, n, q, debug=True, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    score, e, ssum, status = dev.debug_intermediates(n)
    say(f"decode path {dev.decode_path(n)}")
    if score is not None:                     # the fused path keeps scores in registers
        assert oracle.bit_diff(score.numpy(), sc) == 0
    e_want = np.exp((sc * np.float32(0.0625) - (sc * np.float32(0.0625)).max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float32)
    assert oracle.bit_diff(e.numpy(), e_want) == 0
    assert int(status.sum()) == 0, "the exact walk fell back to the serial loop"
    p_gpu = (e.numpy() / ssum.numpy()[:, None]).astype(np.float32)
    assert oracle.bit_diff(p_gpu, pr) == 0
    assert np.array_equal(oracle.f32_to_f16(p_gpu), p16)
    assert report("out", out.cpu().numpy(), want) <= TOL


def test_identical_keys_uniform_attention(path):
    """All scores equal: every e_j = 1 and the serial sum is exactly n; p = 1/n in fp16."""
    n = 5000
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    k1, _ = oracle.synth_kv(1, 4, 256, 9, 0)
    _, v = oracle.synth_kv(n, 4, 256, 9, 1)
    k = np.repeat(k1, n, axis=0)
    host.append(0, 0, k, v)
    dev.append(0, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    q, _ = qg(9, 0)
    want, _ = host.decode(0, n, q)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    _, e, ssum, status = dev.debug_intermediates(n)
    assert torch.all(e == 1.0) and torch.all(ssum == float(n)) and int(status.sum()) == 0
    assert report("uniform", out.cpu().numpy(), want) <= TOL
