"""GPU parity of the fused append front end (bkv_qk_norm_rope_append through the C ABI) against the
oracle's restatement of the reference's attn_rms_norm / attn_rope (runtime_vk/attn_vk.h:102-122,
pinned against the reference's compiled mirror in tests/test_oracle_norm_rope.py). Bar: the roped Q
rows and every cache byte bit-exact (integer / byte work plus correctly rounded fp32 arithmetic),
then attention over the result within 1e-4 of the oracle."""
import numpy as np
import pytest
import torch

import oracle
from bonsai_vk_amd import BKV_F16, BKV_Q8_0
from tests.gpu_util import pair, report, same_bytes, say

pytestmark = pytest.mark.gpu


def inputs(n, seed):
    q = oracle.normal(n * 16 * 256, seed, 700).reshape(n, 16, 256) * 3.0
    k = oracle.normal(n * 4 * 256, seed, 701).reshape(n, 4, 256) * 3.0
    v = oracle.normal(n * 4 * 256, seed, 702).reshape(n, 4, 256) * 0.5
    qw = (1.0 + 0.2 * oracle.normal(256, seed, 703)).astype(np.float32)
    kw = (1.0 + 0.2 * oracle.normal(256, seed, 704)).astype(np.float32)
    k[1, 2] *= 1e-3
    return [np.ascontiguousarray(a, np.float32) for a in (q, k, v)] + [qw, kw]


@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16), (BKV_F16, BKV_Q8_0)])
@pytest.mark.parametrize("pos0", [0, 1000, 65000])
def test_norm_rope_append_bit_exact(kf, vf, pos0):
    say(f"norm_rope kf={kf} vf={vf} pos0={pos0}")
    n = 24
    dev, host = pair(1, pos0 + n, kf, vf)
    q, k, v, qw, kw = inputs(n, pos0 + 1)
    want = host.norm_rope_append(0, pos0, q, k, v, qw, kw)
    got = dev.norm_rope_append(0, pos0, *(torch.from_numpy(a).cuda() for a in (q, k, v, qw, kw)))
    torch.cuda.synchronize()
    got = got.cpu().numpy()
    bad = int((got.view(np.uint32) != want.view(np.uint32)).sum())
    say(f"  q_out bit-diff {bad}/{want.size}")
    assert bad == 0
    assert not any(same_bytes(dev, host))


def test_norm_rope_then_decode_and_rope_geometry():
    """Append 300 tokens through the front end, then decode the last token's roped Q: matches the
    oracle; other rope geometries (nrot 0, nrot 256, another base) stay bit-exact."""
    n = 300
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    q, k, v, qw, kw = inputs(n, 9)
    want_q = host.norm_rope_append(0, 0, q, k, v, qw, kw)
    got_q = dev.norm_rope_append(0, 0, *(torch.from_numpy(a).cuda() for a in (q, k, v, qw, kw)))
    want, _ = host.decode(0, n, want_q[-1], nthreads=8)
    out, _ = dev.decode(0, n, got_q[-1].contiguous())
    torch.cuda.synchronize()
    assert report("roped decode", out.cpu().numpy(), want) <= 1e-4
    for nrot, base in [(0, 1e7), (256, 1e4), (32, 5e5)]:
        d2, h2 = pair(1, 40, BKV_F16, BKV_Q8_0)
        qq, kk, vv, a1, a2 = inputs(8, nrot + 3)
        wq = h2.norm_rope_append(0, 30, qq, kk, vv, a1, a2, nrot=nrot, base=base)
        gq = d2.norm_rope_append(0, 30, *(torch.from_numpy(a).cuda() for a in (qq, kk, vv, a1, a2)),
                                 nrot=nrot, freq_base=base)
        torch.cuda.synchronize()
        assert np.array_equal(gq.cpu().numpy().view(np.uint32), wq.view(np.uint32)), nrot
        assert not any(same_bytes(d2, h2))
