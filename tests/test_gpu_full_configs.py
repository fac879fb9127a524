"""BASELINE configs 3 and 4 at their true shapes, against the CPU oracle.

Config 3: 8 layers, q8_0 K+V, 32768 cached tokens, then 48 consecutive decode steps (keys 32769 ..
32816), each appending one token per layer; seed 2. Every step of every layer runs on the device;
the oracle checks all 8 layers at steps 0, 1 and 47 (the steps between only move the context on),
and the whole cache is compared byte for byte at the end.

Config 4: 65536 cached tokens in 256-token pages from a pool of 320, a seeded random permutation of
the pool as each layer's block table, one decode step (key 65537), f16 and q8_0 caches; seed 3. Two
layers with distinct block tables stand for the 8 (the layers share no state; what changes between
them is the table). The f16-vs-q8_0 difference of the outputs is printed (the reference's own
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


def test_config4_paged_65k_f16_and_q8():
    n, page, pool, layers = 65536, 256, 320, 2
    rng = np.random.default_rng(3)
    bt = np.stack([rng.permutation(pool) for _ in range(layers)]).astype(np.int32)
    kn, vn = oracle.synth_kv(layers, 4, 256, 3, 0, outliers=3, stream_base=60000)
    outs = {}
    for fmt in (BKV_F16, BKV_Q8_0):
        say(f"config4: fmt {fmt}, {n} tokens, page {page}, pool {pool}")
        dev, host = pair(layers, pool * page, fmt, fmt, page_tokens=page, max_pages=pool, block_table=bt)
        worst = 0.0
        for layer in range(layers):
            fill(dev, host, layer, n, seed=3)
            q, g = qg(3, layer)
            host.append(layer, n, kn[layer:layer + 1], vn[layer:layer + 1])
            want, wg = host.decode(layer, n + 1, q, g, nthreads=16)
            out, og = dev.decode_step(layer, n, torch.from_numpy(kn[layer:layer + 1]).cuda(),
                                      torch.from_numpy(vn[layer:layer + 1]).cuda(),
                                      torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
            torch.cuda.synchronize()
            outs[(fmt, layer)] = out.cpu().numpy()
            worst = max(worst, report(f"config4 fmt {fmt} layer {layer}", outs[(fmt, layer)], want),
                        oracle.rel_err(og.cpu().numpy(), wg))
        diffs = same_bytes(dev, host)
        say(f"config4 fmt {fmt}: cache byte diffs {diffs}")
        assert diffs == [0] * len(diffs)
        assert worst <= TOL
        del dev, host
    for layer in range(layers):
        say(f"config4 layer {layer}: q8_0 vs f16 output, max rel diff "
            f"{oracle.rel_err(outs[(BKV_Q8_0, layer)], outs[(BKV_F16, layer)]):.3e}")
