"""GPU parity of the chunked prefill (bkv_attn_prefill_chunk through the C ABI) against the CPU
oracle, whose prefill is the decode row repeated per query (the reference's own prefill,
runtime_vk/attn_vk.h:261-311 once per token). The default path reproduces the serial scores, row
max, softmax sum and fp16 probabilities bit for bit and sums PV on the matrix cores. Bar: max
relative error 1e-4 per head row (max |gpu - oracle| / max |oracle|), bit-diff counts printed."""
import numpy as np
import pytest
import torch

import oracle
from bonsai_vk_amd import BKV_F16, BKV_Q8_0
from tests.gpu_util import fill, pair, qg, report, same_bytes, say

TOL = 1e-4
pytestmark = pytest.mark.gpu
FMTS = [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16), (BKV_F16, BKV_Q8_0), (BKV_Q8_0, BKV_F16)]


def run_pair(dev, host, layer, pos0, n_q, seed, gate=True):
    q, g = qg(seed, layer, n=n_q)
    if not gate:
        g = None
    want, wg = host.prefill(layer, pos0, q, g, nthreads=8)
    out, og = dev.prefill_chunk(layer, pos0, torch.from_numpy(q).cuda(),
                                None if g is None else torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    r = report(f"prefill pos0={pos0} n_q={n_q}", out.cpu().numpy(), want)
    if gate:
        r = max(r, report("gated", og.cpu().numpy(), wg))
    return r


@pytest.mark.parametrize("kf,vf", FMTS)
@pytest.mark.parametrize("pos0,n_q", [(0, 1), (0, 37), (5, 16), (200, 70), (1000, 130), (3000, 300)])
def test_prefill_matches_oracle(kf, vf, pos0, n_q):
    say(f"prefill kf={kf} vf={vf} pos0={pos0} n_q={n_q}")
    n = pos0 + n_q
    dev, host = pair(1, n, kf, vf)
    fill(dev, host, 0, n, seed=n_q)
    assert run_pair(dev, host, 0, pos0, n_q, seed=pos0 + 1) <= TOL


@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_Q8_0, BKV_F16), (BKV_F16, BKV_Q8_0)])
@pytest.mark.parametrize("pos0,n_q", [(240, 16), (496, 16), (752, 16), (1008, 16), (1520, 16), (0, 600)])
def test_prefill_tile_edges(kf, vf, pos0, n_q):
    """Chunks whose workgroups end exactly on the exact kernel's tile edges (256-key score tiles,
    512-key fp16-K super tiles, 192-key exp steps, 64-key PV tiles: 256, 512, 768, 1024 and 1536
    keys), and a chunk of two 512-query slices."""
    say(f"prefill tile edges kf={kf} vf={vf} pos0={pos0} n_q={n_q}")
    n = pos0 + n_q
    dev, host = pair(1, n, kf, vf)
    fill(dev, host, 0, n, seed=n + 3)
    assert run_pair(dev, host, 0, pos0, n_q, seed=pos0 + 7) <= TOL


def test_prefill_without_gate_and_layer_offset():
    dev, host = pair(3, 700, BKV_Q8_0, BKV_Q8_0)
    for layer in range(3):
        fill(dev, host, layer, 700, seed=9)
    assert run_pair(dev, host, 2, 600, 100, seed=4, gate=False) <= TOL


@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16)])
def test_prefill_paged(kf, vf):
    """64-token pages, a seeded permutation of a 48-page pool as the block table: matches the oracle,
    and equals the contiguous cache's result bit for bit."""
    page, pool, pos0, n_q = 64, 48, 2500, 170
    rng = np.random.default_rng(5)
    bt = np.stack([rng.permutation(pool) for _ in range(2)]).astype(np.int32)
    say(f"prefill paged kf={kf} vf={vf}")
    dev, host = pair(2, pool * page, kf, vf, page_tokens=page, max_pages=pool, block_table=bt)
    flat, _ = pair(2, pool * page, kf, vf)
    k, v = fill(dev, host, 1, pos0 + n_q, seed=6)
    flat.append(1, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    q, g = qg(6, 1, n=n_q)
    want, _ = host.prefill(1, pos0, q, g, nthreads=8)
    out, _ = dev.prefill_chunk(1, pos0, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    o2, _ = flat.prefill_chunk(1, pos0, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert report("paged prefill", out.cpu().numpy(), want) <= TOL
    assert torch.equal(out, o2)


def test_prefill_equals_decode_rows():
    """Each prefill row against the device decode of the same query at nfill = pos0 + i + 1 (the
    reference's prefill-vs-decode equality leg, align_attn.cpp:1330-1385), to the tolerance."""
    pos0, n_q = 1500, 40
    dev, host = pair(1, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, pos0 + n_q, seed=12)
    q, _ = qg(12, 0, n=n_q)
    qd = torch.from_numpy(q).cuda()
    out, _ = dev.prefill_chunk(0, pos0, qd)
    worst = 0.0
    for i in range(0, n_q, 7):
        o, _ = dev.decode(0, pos0 + i + 1, qd[i].contiguous())
        torch.cuda.synchronize()
        worst = max(worst, oracle.rel_err(out[i].cpu().numpy(), o.cpu().numpy()))
    say(f"prefill vs decode rows: max rel err {worst:.3e}")
    assert worst <= TOL


def test_prefill_deterministic():
    pos0, n_q = 900, 50
    dev, host = pair(1, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, pos0 + n_q, seed=13)
    q, g = qg(13, 0, n=n_q)
    qd, gd = torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda()
    a, ag = dev.prefill_chunk(0, pos0, qd, gd)
    b, bg = dev.prefill_chunk(0, pos0, qd, gd)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ag, bg)


def test_config5_sampled_rows():
    """BASELINE config 5 at its true shape for one layer: 512 queries appended onto 8192 cached
    tokens, q8_0 K+V, seed 4; sampled query rows checked against the oracle's decode row."""
    pos0, n_q = 8192, 512
    dev, host = pair(1, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, pos0 + n_q, seed=4, outliers=0)
    q, g = qg(4, 0, n=n_q)
    out, og = dev.prefill_chunk(0, pos0, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    out, og = out.cpu().numpy(), og.cpu().numpy()
    worst = 0.0
    for i in [0, 1, 15, 16, 17, 100, 255, 256, 400, 510, 511]:
        want, wg = host.decode(0, pos0 + i + 1, q[i], g[i], nthreads=8)
        worst = max(worst, oracle.rel_err(out[i], want), oracle.rel_err(og[i], wg))
    say(f"config5 sampled rows: max rel err {worst:.3e}")
    assert worst <= TOL


def test_config5_full_layer():
    """BASELINE config 5 at its true shape for one layer, every row: 512 queries appended onto 8192
    cached tokens (q8_0 K+V, seed 4, prefill_step: the chunk's K/V appended, then its attention),
    all 512 x 16 output rows and the gated rows against the oracle's prefill."""
    pos0, n_q = 8192, 512
    dev, host = pair(1, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, pos0, seed=4, outliers=0)
    k, v = oracle.synth_kv(n_q, 4, 256, 4, 0, outliers=0, stream_base=70000)
    q, g = qg(4, 0, n=n_q)
    host.append(0, pos0, k, v)
    want, wg = host.prefill(0, pos0, q, g, nthreads=16)
    out, og = dev.prefill_step(0, pos0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                               torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert not any(same_bytes(dev, host))
    assert report("config5 all rows", out.cpu().numpy(), want) <= TOL
    assert report("config5 all rows, gated", og.cpu().numpy(), wg) <= TOL


def test_config5_8_layers():
    """BASELINE config 5 on all 8 layers: per layer its own 8192 cached tokens and 512-token chunk
    (q8_0 K+V, seed 4, layer-dependent draws), prefill_step on each layer into one 8-layer cache.
    Every cache byte of every layer, and every one of the 512 x 16 output rows (and gated rows) of
    every layer, against the oracle."""
    pos0, n_q, layers = 8192, 512, 8
    dev, host = pair(layers, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    worst = 0.0
    for layer in range(layers):
        say(f"config5 layer {layer}")
        fill(dev, host, layer, pos0, seed=4 + layer, outliers=0)
        k, v = oracle.synth_kv(n_q, 4, 256, 4, layer, outliers=0, stream_base=70000)
        q, g = qg(4, layer, n=n_q)
        host.append(layer, pos0, k, v)
        want, wg = host.prefill(layer, pos0, q, g, nthreads=16)
        out, og = dev.prefill_step(layer, pos0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                                   torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
        torch.cuda.synchronize()
        worst = max(worst, report(f"config5 layer {layer}", out.cpu().numpy(), want),
                    report(f"config5 layer {layer}, gated", og.cpu().numpy(), wg))
    diffs = same_bytes(dev, host)
    say(f"config5 8 layers: cache byte diffs {diffs}")
    assert diffs == [0] * len(diffs)
    assert worst <= TOL


def test_prefill_errors():
    from bonsai_vk_amd import BkvError
    dev, _ = pair(1, 100, BKV_Q8_0, BKV_Q8_0)
    q = torch.zeros((10, 16, 256), device="cuda")
    with pytest.raises(BkvError):
        dev.prefill_chunk(0, 95, q)          # pos0 + n_q beyond the cache
    with pytest.raises(BkvError):
        dev.prefill_chunk(1, 0, q)           # no such layer


def test_prefill_and_decode_share_a_workspace():
    """The exact prefill's scratch lies past every array a decode can use, so decode calls (the
    resident kernel polls its partials for generation tags) and short prefill chunks (decode rows)
    on the same workspace stay correct after a prefill has filled its scratch."""
    import ctypes
    from bonsai_vk_amd import lib
    from bonsai_vk_amd._lib import check
    pos0, n_q = 700, 40
    n = pos0 + n_q
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n, seed=21)
    q, _ = qg(21, 0, n=n_q)
    qd = torch.from_numpy(q).cuda()
    ws = dev.prefill_workspace(n)
    want, _ = host.prefill(0, pos0, q, None, nthreads=8)
    for rep in range(3):
        out, _ = dev.prefill_chunk(0, pos0, qd)
        o = torch.empty((16, 256), device="cuda")
        check(lib().bkv_attn_decode(ctypes.byref(dev.desc), 0, n, qd[-1].data_ptr(), None,
                                    o.data_ptr(), None, ws.data_ptr(), ws.numel(), dev._stream()),
              "bkv_attn_decode")
        short, _ = dev.prefill_chunk(0, pos0 + 30, qd[30:35].contiguous())
        torch.cuda.synchronize()
        assert report(f"shared ws prefill rep {rep}", out.cpu().numpy(), want) <= TOL
        assert report(f"shared ws decode rep {rep}", o.cpu().numpy(), want[-1]) <= TOL
        assert report(f"shared ws short chunk rep {rep}", short.cpu().numpy(), want[30:35]) <= TOL


@pytest.mark.parametrize("mode", ["exact", "mfma"])
@pytest.mark.parametrize("n_q", [5, 40])
def test_prefill_interleaved_qg(mode, n_q, monkeypatch):
    """bkv_attn_prefill_chunk_qg reads q and the gate from [n][nh][2*hd] rows (q then gate per head)
    and equals the de-interleaved call bit for bit, on the exact path (and its decode-row path for
    short chunks) and on the MFMA-order variant."""
    if mode == "mfma":
        monkeypatch.setenv("BKV_PREFILL", "mfma")
    pos0 = 300
    dev, host = pair(1, pos0 + n_q, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, pos0 + n_q, seed=43)
    q, g = qg(43, 0, n=n_q)
    qd, gd = torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda()
    inter = torch.cat([qd, gd], dim=2).contiguous()
    a, ag = dev.prefill_chunk(0, pos0, qd, gd)
    b, bg = dev.prefill_chunk_qg(0, pos0, inter)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ag, bg)


def test_prefill_step_is_append_then_chunk():
    """bkv_prefill_step (append the chunk, then its attention) leaves the oracle's cache bytes and
    gives the oracle's prefill rows; a prompt fed as three chunks equals one decode step per token
    (the engine's prompt loop, runtime_vk/bonsai_forward.h:2752-2759) to the tolerance."""
    from tests.gpu_util import same_bytes
    n0, chunks = 500, [40, 17, 90]
    n = n0 + sum(chunks)
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n0, seed=51)
    k, v = oracle.synth_kv(n - n0, 4, 256, 52, 0, outliers=3)
    q, g = qg(52, 0, n=n - n0)
    pos = n0
    for c in chunks:
        i = pos - n0
        host.append(0, pos, k[i:i + c], v[i:i + c])
        want, wg = host.prefill(0, pos, q[i:i + c], g[i:i + c], nthreads=8)
        out, og = dev.prefill_step(0, pos, torch.from_numpy(k[i:i + c]).cuda(),
                                   torch.from_numpy(v[i:i + c]).cuda(), torch.from_numpy(q[i:i + c]).cuda(),
                                   torch.from_numpy(g[i:i + c]).cuda())
        torch.cuda.synchronize()
        assert report(f"prefill_step pos={pos} n={c}", out.cpu().numpy(), want) <= TOL
        assert oracle.rel_err(og.cpu().numpy(), wg) <= TOL
        pos += c
    assert not any(same_bytes(dev, host))


@pytest.mark.parametrize("pos0,n_q", [(1000, 40), (3000, 300)])
def test_prefill_q8k_query_exponent_spread(pos0, n_q):
    """q8_0 K prefill of queries whose q rows spread over many binades (every 7th query as
    test_gpu_decode.spread_q builds it: one workgroup's group past the int8 digits' range takes the
    fp64 path), against the oracle."""
    from tests.test_gpu_decode import spread_q
    say(f"prefill q exponent spread pos0={pos0} n_q={n_q}")
    n = pos0 + n_q
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n, seed=n_q + 5)
    q, g = qg(pos0 + 11, 0, n=n_q)
    for i in range(0, n_q, 7):
        q[i] = spread_q(q[i])
    want, wg = host.prefill(0, pos0, q, g, nthreads=8)
    out, og = dev.prefill_chunk(0, pos0, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    r = max(report("prefill", out.cpu().numpy(), want), report("gated", og.cpu().numpy(), wg))
    assert r <= TOL
