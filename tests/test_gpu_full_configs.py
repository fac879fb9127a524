"""BASELINE configs 3 and 4 at their true shapes, against the CPU oracle.

Config 3: 8 layers, q8_0 K+V, 32768 cached tokens, then 48 consecutive decode steps (keys 32769 ..
32816), each appending one token per layer; seed 2. Every step of every layer runs on the device;
the oracle checks all 8 layers at steps 0, 1 and 47 (the steps between only move the context on),
and the whole cache is compared byte for byte at the end.

Config 4: 65536 cached tokens in 256-token pages from a pool of 320, a seeded random permutation of
the pool as each layer's block table, one decode step (key 65537) on each of the 8 layers, f16 and
q8_0 caches; seed 3. Every layer has its own block table and its own appended token and query; the
65536 cached tokens are one seeded draw shared by the layers (what changes between layers is where
the table puts them). The f16-vs-q8_0 difference of the outputs is printed (the reference's own
comparison of the two variants) next to each variant's parity.

Bar: cache bytes bit-exact; outputs within max relative error 1e-4 per head row."""
import numpy as np
import pytest
import torch

import oracle
from bonsai_vk_amd import BKV_F16, BKV_Q8_0
from tests.gpu_util import fill, pair, qg, report, same_bytes, say

TOL = 1e-4
pytestmark = pytest.mark.gpu


def test_config3_32k_48_steps():
    n0, steps, layers = 32768, 48, 8
    check = {0, 1, steps - 1}
    say(f"config3: {layers} layers, q8_0, {n0} cached tokens, {steps} steps")
    dev, host = pair(layers, n0 + steps, BKV_Q8_0, BKV_Q8_0)
    for layer in range(layers):
        fill(dev, host, layer, n0, seed=2)
    kn, vn = oracle.synth_kv(steps * layers, 4, 256, 2, 0, outliers=3, stream_base=50000)
    worst = 0.0
    for i in range(steps):
        for layer in range(layers):
            t = i * layers + layer
            q, g = qg(200 + i, layer)
            host.append(layer, n0 + i, kn[t:t + 1], vn[t:t + 1])
            out, og = dev.decode_step(layer, n0 + i, torch.from_numpy(kn[t:t + 1]).cuda(),
                                      torch.from_numpy(vn[t:t + 1]).cuda(), torch.from_numpy(q).cuda(),
                                      torch.from_numpy(g).cuda())
            if i in check:
                want, wg = host.decode(layer, n0 + i + 1, q, g, nthreads=16)
                torch.cuda.synchronize()
                worst = max(worst, report(f"config3 step {i} layer {layer}", out.cpu().numpy(), want),
                            oracle.rel_err(og.cpu().numpy(), wg))
    torch.cuda.synchronize()
    diffs = same_bytes(dev, host)
    say(f"config3: cache byte diffs {diffs}, worst rel err {worst:.3e}")
    assert diffs == [0] * len(diffs)
    assert worst <= TOL


_config4_outs = {}


@pytest.mark.parametrize("fmt", [BKV_F16, BKV_Q8_0])
def test_config4_paged_65k_8_layers(fmt):
    n, page, pool, layers = 65536, 256, 320, 8
    rng = np.random.default_rng(3)
    bt = np.stack([rng.permutation(pool) for _ in range(layers)]).astype(np.int32)
    assert len({tuple(r) for r in bt}) == layers            # distinct tables
    kn, vn = oracle.synth_kv(layers, 4, 256, 3, 0, outliers=3, stream_base=60000)
    k, v = oracle.synth_kv(n, 4, 256, 3, 0, outliers=3)
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    say(f"config4: fmt {fmt}, {n} tokens, page {page}, pool {pool}, {layers} layers")
    dev, host = pair(layers, pool * page, fmt, fmt, page_tokens=page, max_pages=pool, block_table=bt)
    worst = 0.0
    for layer in range(layers):
        host.append(layer, 0, k, v)
        for s0 in range(0, n, 16384):
            dev.append(layer, s0, kd[s0:s0 + 16384], vd[s0:s0 + 16384])
        q, g = qg(3, layer)
        host.append(layer, n, kn[layer:layer + 1], vn[layer:layer + 1])
        want, wg = host.decode(layer, n + 1, q, g, nthreads=16)
        out, og = dev.decode_step(layer, n, torch.from_numpy(kn[layer:layer + 1]).cuda(),
                                  torch.from_numpy(vn[layer:layer + 1]).cuda(),
                                  torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
        torch.cuda.synchronize()
        _config4_outs[(fmt, layer)] = out.cpu().numpy()
        worst = max(worst, report(f"config4 fmt {fmt} layer {layer}", _config4_outs[(fmt, layer)], want),
                    oracle.rel_err(og.cpu().numpy(), wg))
    diffs = same_bytes(dev, host)
    say(f"config4 fmt {fmt}: cache byte diffs {diffs}")
    assert diffs == [0] * len(diffs)
    assert worst <= TOL
    for layer in range(layers):
        if (BKV_F16, layer) in _config4_outs and (BKV_Q8_0, layer) in _config4_outs:
            say(f"config4 layer {layer}: q8_0 vs f16 output, max rel diff "
                f"{oracle.rel_err(_config4_outs[(BKV_Q8_0, layer)], _config4_outs[(BKV_F16, layer)]):.3e}")
