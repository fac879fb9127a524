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


PATHS = {"stream": 3, "resident": 2, "split": 0}


@pytest.fixture(params=list(PATHS))
def path(request, monkeypatch):
    """Run a test through every decode implementation (the library reads BKV_DECODE per call)."""
    monkeypatch.setenv("BKV_DECODE", request.param)
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
                                          (BKV_Q8_0, BKV_Q8_0, 40000, 2), (BKV_Q8_0, BKV_Q8_0, 65537, 3),
                                          (BKV_F16, BKV_F16, 65537, 5), (BKV_F16, BKV_Q8_0, 4097, 11),
                                          (BKV_F16, BKV_Q8_0, 32769, 12), (BKV_F16, BKV_Q8_0, 90, 13)])
def test_scores_probabilities_and_sum_bit_exact(kf, vf, n, seed, path, monkeypatch):
    """The intermediates the reference's bitwise gate (BONSAI_QCHECK stages A/B) compares: every score,
    every e_j = exp(s_j*scale - max) and the serial fp32 softmax sum match the oracle bit for bit, and
    so do the fp16 probabilities formed from them."""
    monkeypatch.setenv("BKV_KEEP_INTERMEDIATES", "1")
    say(f"bit-exact intermediates kf={kf} n={n}")
    dev, host = pair(1, n, kf, vf)
    fill(dev, host, 0, n, seed=seed)
    q, _ = qg(seed, 0)
    want, _, sc, pr, p16 = host.decode(0, n, q, debug=True, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    score, e, ssum, status = dev.debug_intermediates(n)
    say(f"decode path {dev.decode_path(n)}")
    if score is not None:                     # the single-launch paths keep scores in registers
        assert oracle.bit_diff(score.numpy(), sc) == 0
    e_want = np.exp((sc * np.float32(0.0625) - (sc * np.float32(0.0625)).max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float32)
    assert oracle.bit_diff(e.numpy(), e_want) == 0
    assert int(status.sum()) == 0, "the exact walk fell back to the serial loop"
    p_gpu = (e.numpy() / ssum.numpy()[:, None]).astype(np.float32)
    assert oracle.bit_diff(p_gpu, pr) == 0
    assert np.array_equal(oracle.f32_to_f16(p_gpu), p16)
    assert report("out", out.cpu().numpy(), want) <= TOL


def test_identical_keys_uniform_attention(path, monkeypatch):
    """All scores equal: every e_j = 1 and the serial sum is exactly n; p = 1/n in fp16."""
    monkeypatch.setenv("BKV_KEEP_INTERMEDIATES", "1")
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


@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16)])
def test_paged_matches_oracle_and_contiguous(kf, vf, path):
    """Paged cache (64-token pages, a seeded random permutation of a 48-page pool as each layer's block
    table): the oracle's paged decode matches, and the result equals the contiguous cache's bit for bit
    (same keys in the same order, only their slots differ)."""
    n, page, pool = 2900, 64, 48
    rng = np.random.default_rng(3)
    bt = np.stack([rng.permutation(pool)[:pool] for _ in range(2)]).astype(np.int32)
    say(f"paged kf={kf} vf={vf} n={n} path={path}")
    dev, host = pair(2, pool * page, kf, vf, page_tokens=page, max_pages=pool, block_table=bt)
    flat, _ = pair(2, pool * page, kf, vf)
    k, v = fill(dev, host, 1, n, seed=3)
    flat.append(1, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    q, g = qg(3, 1)
    want, wg = host.decode(1, n, q, g, nthreads=8)
    out, og = dev.decode(1, n, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    o2, _ = flat.decode(1, n, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert same_bytes(dev, host) == [0] * len(same_bytes(dev, host))
    assert report("paged", out.cpu().numpy(), want) <= TOL
    assert oracle.rel_err(og.cpu().numpy(), wg) <= TOL
    assert torch.equal(out, o2)


@pytest.mark.parametrize("page", [1, 3])
@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_F16)])
def test_small_pages(kf, vf, page, path):
    """Pages of 1 and 3 tokens at 8200 keys: a workgroup's 129 keys span 129 pages, more than the
    resident kernel's LDS page table holds, so the call takes the split path; or 44 pages, the
    resident kernel with a page size that is no power of two. Matches the oracle and equals the
    contiguous cache."""
    n = 8200
    pool = -(-n // page) + 5
    bt = np.random.default_rng(11).permutation(pool)[None].astype(np.int32)
    say(f"small pages kf={kf} vf={vf} page={page} path={path}")
    dev, host = pair(1, pool * page, kf, vf, page_tokens=page, max_pages=pool, block_table=bt)
    flat, _ = pair(1, pool * page, kf, vf)
    if path in ("resident", "stream"):
        assert dev.decode_path(n) == (0 if page == 1 else PATHS[path] if kf == BKV_Q8_0 else 2)
    k, v = fill(dev, host, 0, n, seed=11)
    flat.append(0, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    q, g = qg(11, 0)
    want, _ = host.decode(0, n, q, g, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    o2, _ = flat.decode(0, n, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert report(f"pages of {page}", out.cpu().numpy(), want) <= TOL
    if dev.decode_path(n) == flat.decode_path(n):
        assert torch.equal(out, o2)
    else:                                  # other kernels, other PV summation order
        assert oracle.rel_err(out.cpu().numpy(), o2.cpu().numpy()) <= TOL


@pytest.mark.parametrize("n", [32768, 33792, 33793])
def test_register_v_boundary(n):
    """The stream kernel keeps a workgroup's q8_0 V rows in registers up to 512 + 16 keys: 32768
    keys (no tail) and 33792 (the longest tail) take it, 33793 the resident kernel's two-pass form;
    all match the oracle, through decode_step (the appended token lands in the last workgroup's
    range)."""
    say(f"register-V boundary n={n}")
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n - 1, seed=31)
    k, v = oracle.synth_kv(1, 4, 256, 32, 0, outliers=3)
    q, g = qg(31, 0)
    host.append(0, n - 1, k, v)
    want, wg = host.decode(0, n, q, g, nthreads=8)
    out, og = dev.decode_step(0, n - 1, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda(),
                              torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert dev.decode_path(n) == (3 if n <= 33792 else 2)
    assert report(f"n={n}", out.cpu().numpy(), want) <= TOL
    assert oracle.rel_err(og.cpu().numpy(), wg) <= TOL
    assert same_bytes(dev, host) == [0, 0, 0, 0]


@pytest.mark.parametrize("kf,vf", [(BKV_F16, BKV_Q8_0), (BKV_Q8_0, BKV_F16)])
def test_mixed_formats_multipass(kf, vf):
    """Mixed K/V formats beyond the register-V range: 40000 keys (the resident kernel's two-pass
    form), against the oracle."""
    n = 40000
    dev, host = pair(1, n, kf, vf)
    fill(dev, host, 0, n, seed=44)
    q, g = qg(44, 0)
    want, wg = host.decode(0, n, q, g, nthreads=8)
    out, og = dev.decode(0, n, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert dev.decode_path(n) == 2
    assert report(f"mixed kf={kf} vf={vf} n={n}", out.cpu().numpy(), want) <= TOL
    assert oracle.rel_err(og.cpu().numpy(), wg) <= TOL


@pytest.mark.parametrize("n,path_want", [(131072, 2), (131073, 0)])
def test_longest_resident_context(n, path_want):
    """64 x 4 x 512 = 131072 keys is the longest context the resident kernel holds (four passes per
    workgroup); one more key takes the split path. Both match the oracle."""
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n, seed=45, chunk=16384)
    q, _ = qg(45, 0)
    want, _ = host.decode(0, n, q, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    assert dev.decode_path(n) == path_want
    assert report(f"n={n} path={path_want}", out.cpu().numpy(), want) <= TOL


def test_workspace_error_flag(path):
    """bkv_workspace_error: clean after ordinary decodes. A timed-out call is imitated from the
    host: the error word set and the sync area and tagged partials poisoned with junk (counters
    mid-protocol, a generation far ahead, tags of the next generations). The check reports
    BKV_ETIMEOUT, leaves the whole workspace zeroed, and the decodes after it match the oracle."""
    from bonsai_vk_amd import BkvError
    dev, host = pair(1, 600, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, 600, seed=41)
    q, _ = qg(41, 0)
    want, _ = host.decode(0, 600, q, nthreads=8)
    dev.decode(0, 600, torch.from_numpy(q).cuda())
    dev.check_workspace()
    off = dev.error_word_offset()
    ws = dev.workspace
    g = torch.Generator(device="cuda").manual_seed(5)
    junk = torch.randint(0, 256, (ws.numel(),), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    ws.copy_(junk)                            # every byte, sync lines and tagged partials included
    words = ws[:256 * 1024].view(torch.int32)
    words[::16] = 3                           # small counters and generations: a protocol mid-call
    ws[off:off + 4].view(torch.int32).fill_(1)
    with pytest.raises(BkvError) as e:
        dev.check_workspace()
    assert e.value.code == -8
    assert int(ws.count_nonzero()) == 0       # re-initialised
    dev.check_workspace()                     # clean now
    for i in range(3):
        out, _ = dev.decode(0, 600, torch.from_numpy(q).cuda())
        torch.cuda.synchronize()
        assert report(f"after the error check, call {i}", out.cpu().numpy(), want) <= TOL
    dev.check_workspace()


def test_paths_switch_on_one_workspace(monkeypatch):
    """The path a call takes follows its context on one workspace: split past 131,072 keys, the
    stream kernel for a window of 3,000 of them, the resident kernel for 40,000, and back. Every
    call matches the oracle: no path reads what another left in the workspace."""
    monkeypatch.delenv("BKV_DECODE", raising=False)
    n = 140000
    dev, _ = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    k, v = oracle.synth_kv(n, 4, 256, 61, 0, outliers=3)
    for s0 in range(0, n, 16384):
        dev.append(0, s0, torch.from_numpy(k[s0:s0 + 16384]).cuda(), torch.from_numpy(v[s0:s0 + 16384]).cuda())
    q, _ = qg(61, 0)
    qd = torch.from_numpy(q).cuda()
    wants = {}
    for kstart in (0, n - 3000, n - 40000):                 # the oracle of each window: its keys alone
        _, host = pair(1, n - kstart, BKV_Q8_0, BKV_Q8_0)
        host.append(0, 0, k[kstart:], v[kstart:])
        wants[kstart] = host.decode(0, n - kstart, q, nthreads=16)[0]
        del host
    for kstart, want_path in [(0, 0), (n - 3000, 3), (n - 40000, 2), (0, 0), (n - 3000, 3), (n - 40000, 2),
                              (n - 3000, 3)]:
        say(f"window [{kstart}, {n}) path {want_path}")
        assert dev.decode_path(n - kstart) == want_path
        out, _ = dev.decode_window(0, kstart, n, qd)
        torch.cuda.synchronize()
        assert report(f"window [{kstart}, {n})", out.cpu().numpy(), wants[kstart]) <= TOL
    dev.check_workspace()


def test_consecutive_decode_steps(path):
    """BASELINE config 3's pattern at a smaller context: consecutive decode_steps on one workspace
    (each call appends one token and attends over all of them), every step checked against the
    oracle, across layers that share the workspace."""
    n0, steps = 3000, 6
    dev, host = pair(2, n0 + steps, BKV_Q8_0, BKV_Q8_0)
    for layer in range(2):
        fill(dev, host, layer, n0, seed=2)
    kn, vn = oracle.synth_kv(steps * 2, 4, 256, 77, 0, outliers=3)
    worst = 0.0
    for i in range(steps):
        for layer in range(2):
            t = 2 * i + layer
            host.append(layer, n0 + i, kn[t:t + 1], vn[t:t + 1])
            q, _ = qg(20 + i, layer)
            want, _ = host.decode(layer, n0 + i + 1, q, nthreads=8)
            out, _ = dev.decode_step(layer, n0 + i, torch.from_numpy(kn[t:t + 1]).cuda(),
                                     torch.from_numpy(vn[t:t + 1]).cuda(), torch.from_numpy(q).cuda())
            torch.cuda.synchronize()
            worst = max(worst, report(f"step {i} layer {layer}", out.cpu().numpy(), want))
    assert same_bytes(dev, host) == [0, 0, 0, 0]
    assert worst <= TOL


def test_decode_path_selection(monkeypatch):
    """The stream kernel is the default for q8_0 K and V up to 64 x 528 keys, the resident kernel
    beyond (and for the other formats); BKV_DECODE forces the others."""
    dev, _ = pair(1, 70000, BKV_Q8_0, BKV_Q8_0)
    monkeypatch.delenv("BKV_DECODE", raising=False)
    assert dev.decode_path(1) == 3 and dev.decode_path(32769) == 3 and dev.decode_path(65537) == 2
    for name, code in PATHS.items():
        monkeypatch.setenv("BKV_DECODE", name)
        assert dev.decode_path(32769) == code


def test_fill_synthetic_and_dump(path):
    """bkv_kv_fill_synthetic leaves the reference's fixture bytes (0x3C003C00 everywhere) in every
    layer, decode over them matches the oracle's decode of the same fixture, and the TSV dump of the
    device cache equals the host cache's dump (kv_dump format) after real appends on top."""
    from bonsai_vk_amd import kvdump
    n = 600
    dev, host = pair(2, n, BKV_Q8_0, BKV_Q8_0)
    dev.fill_synthetic()
    host.fill_synthetic()
    torch.cuda.synchronize()
    assert same_bytes(dev, host) == [0] * len(same_bytes(dev, host))
    q, g = qg(31, 1)
    want, _ = host.decode(1, n, q, nthreads=8)
    out, _ = dev.decode(1, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    assert report("synthetic fill", out.cpu().numpy(), want) <= TOL
    k, v = oracle.synth_kv(40, 4, 256, 32, 0, outliers=3)
    host.append(0, 5, k, v)
    dev.append(0, 5, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    torch.cuda.synchronize()
    assert kvdump.dump_cache(dev, 0, 60) == kvdump.dump_cache(host, 0, 60)


def test_interleaved_qg_entry_points(path, monkeypatch):
    """bkv_attn_decode_qg / bkv_decode_step_qg read q and the gate from the engine's interleaved
    attn_q output (per head: 256 q then 256 gate, the layout deint_qg splits); results equal the
    de-interleaved calls bit for bit, gated output included."""
    monkeypatch.setenv("BKV_KEEP_INTERMEDIATES", "0")
    n = 2000
    dev, host = pair(1, n + 2, BKV_Q8_0, BKV_Q8_0)
    twin, _ = pair(1, n + 2, BKV_Q8_0, BKV_Q8_0)
    k, v = fill(dev, host, 0, n, seed=41)
    twin.append(0, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    q, g = qg(41, 0)
    qd, gd = torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda()
    inter = torch.cat([qd, gd], dim=1).contiguous()          # [16][512]: q then gate per head
    a, ag = dev.decode(0, n, qd, gd)
    b, bg = dev.decode_qg(0, n, inter)
    c, cg = dev.decode_qg(0, n, inter, gated=False)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ag, bg) and torch.equal(a, c) and cg is None
    kn, vn = oracle.synth_kv(1, 4, 256, 42, 0, outliers=3)
    kd, vd = torch.from_numpy(kn).cuda(), torch.from_numpy(vn).cuda()
    s1, s1g = dev.decode_step(0, n, kd, vd, qd, gd)
    s2, s2g = twin.decode_step_qg(0, n, kd, vd, inter)
    torch.cuda.synchronize()
    assert torch.equal(s1, s2) and torch.equal(s1g, s2g)
    assert not any(same_bytes(dev, oracle_like(twin)))
    want, wg = host.decode(0, n, q, g, nthreads=8)
    assert report("qg", b.cpu().numpy(), want) <= TOL


def oracle_like(cache):
    """the device arrays of another device cache, shaped like an oracle HostCache for same_bytes"""
    class _H:
        def arrays(self):
            return [None if a is None else a.numpy() for a in cache.host_arrays()]
    return _H()


@pytest.mark.parametrize("page", [0, 64])
def test_decode_window_equals_evicted_prefix(path, page):
    """bkv_attn_decode_window over keys [kstart, nfill) equals, bit for bit, the decode of a cache
    holding only those keys (the reference's eviction masks the farthest blocks out of the softmax
    with -INF, which adds exactly nothing), and matches the oracle."""
    n, kstart = 2600, 640
    pool = 48
    bt = np.stack([np.random.default_rng(7).permutation(pool)]).astype(np.int32) if page else None
    kw = dict(page_tokens=page, max_pages=pool, block_table=bt) if page else {}
    dev, _ = pair(1, pool * 64 if page else n, BKV_Q8_0, BKV_Q8_0, **kw)
    win, host = pair(1, n - kstart, BKV_Q8_0, BKV_Q8_0)
    k, v = oracle.synth_kv(n, 4, 256, 61, 0, outliers=3)
    dev.append(0, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    win.append(0, 0, torch.from_numpy(k[kstart:]).cuda(), torch.from_numpy(v[kstart:]).cuda())
    host.append(0, 0, k[kstart:], v[kstart:])
    q, g = qg(61, 0)
    qd, gd = torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda()
    a, ag = dev.decode_window(0, kstart, n, qd, gd)
    b, bg = win.decode(0, n - kstart, qd, gd)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and torch.equal(ag, bg)
    want, _ = host.decode(0, n - kstart, q, nthreads=8)
    assert report("window", a.cpu().numpy(), want) <= TOL


@pytest.mark.parametrize("nfill", [600, 4097, 20000, 40000])
def test_q8v_scale_spread_and_peaked_scores(nfill, path):
    """The matrix-core PV rounds each p16 * scale to a fixed-point grid set by the largest one: V
    blocks whose scales span 2^-12 .. 2^12 and a few dominant keys (p near 1 beside p near 0) keep
    the output within the bar on every path (contiguous q8_0 K and V; 40000 keys take the
    resident kernel's two-pass form, 600 a stream plan with a tail)."""
    say(f"scale spread nfill={nfill} path={path}")
    dev, host = pair(1, nfill, BKV_Q8_0, BKV_Q8_0)
    k, v = oracle.synth_kv(nfill, 4, 256, 77, 0, outliers=3)
    rng = np.random.default_rng(nfill)
    e = rng.integers(-12, 13, size=(nfill, 4, 8)).astype(np.float32)
    v = (v.reshape(nfill, 4, 8, 32) * np.exp2(e)[..., None]).reshape(nfill, 4, 256).astype(np.float32)
    for j in rng.integers(0, nfill, size=3):   # a few keys aligned with every query: peaked rows
        k[j] = 6.0 * np.sign(k[j]) * np.abs(k[j]).mean()
    host.append(0, 0, k, v)
    for s0 in range(0, nfill, 8192):
        s1 = min(nfill, s0 + 8192)
        dev.append(0, s0, torch.from_numpy(k[s0:s1]).cuda(), torch.from_numpy(v[s0:s1]).cuda())
    q, g = qg(nfill, 0)
    want, wg = host.decode(0, nfill, q, g, nthreads=8)
    out, og = dev.decode(0, nfill, torch.from_numpy(q).cuda(), torch.from_numpy(g).cuda())
    torch.cuda.synchronize()
    assert report("out", out.cpu().numpy(), want) <= TOL
    assert report("gated", og.cpu().numpy(), wg) <= TOL


def spread_q(q, lead=()):
    """q rows (heads on the second-to-last axis) whose fp16 values span many binades: head 1 holds
    300 beside 1e-6 (digits past 31 bits: the fp64 path), head 4 a block of values near 1e-4 beside
    a block near 40 (a wide spread that still fits), head 9 fp16 subnormals."""
    q = q.copy()
    q[lead + (1, 0)] = 300.0
    q[lead + (1, 37)] = 1e-6
    q[lead + (4, slice(0, 32))] *= 1e-4
    q[lead + (4, slice(224, 256))] *= 40.0
    q[lead + (9, slice(100, 110))] = 3e-7 * np.arange(1, 11, dtype=np.float32)
    return q


@pytest.mark.parametrize("n", [4097, 40000])
def test_q8k_query_exponent_spread(n, path, monkeypatch):
    """q8_0 K scores of q rows whose exponents spread over many binades (spread_q): the group past
    the int8 digits' range takes the fp64 path, the others the matrix cores; every e, the sum and
    the fp16 probabilities bit-exact, the output within the bar."""
    monkeypatch.setenv("BKV_KEEP_INTERMEDIATES", "1")
    say(f"q exponent spread n={n} path={path}")
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    fill(dev, host, 0, n, seed=21)
    q = spread_q(qg(21, 0)[0])
    want, _, sc, pr, p16 = host.decode(0, n, q, debug=True, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    score, e, ssum, status = dev.debug_intermediates(n)
    if score is not None:
        assert oracle.bit_diff(score.numpy(), sc) == 0
    e_want = np.exp((sc * np.float32(0.0625) - (sc * np.float32(0.0625)).max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float32)
    assert oracle.bit_diff(e.numpy(), e_want) == 0
    p_gpu = (e.numpy() / ssum.numpy()[:, None]).astype(np.float32)
    assert oracle.bit_diff(p_gpu, pr) == 0
    assert np.array_equal(oracle.f32_to_f16(p_gpu), p16)
    assert report("out", out.cpu().numpy(), want) <= TOL


def test_many_specials_first_and_second_workgroup(path, monkeypatch):
    """Keys shaped so that the exact-sum walk has more specials than the copies handed over with the
    records cover: the first 40 keys point away from their group's queries (e ~ 1e-15: every step of
    the running sum below 2^-17 is a special), the rest of the first workgroup's keys hold e ~ 2^-12,
    and the second workgroup's normal keys carry the sum across several binades (one special per
    crossing). e, the serial sum and p16 stay bit-exact, with no fallback to the serial loop on the
    single-launch paths."""
    monkeypatch.setenv("BKV_KEEP_INTERMEDIATES", "1")
    n, kpw = 4097, 125                         # 33 workgroups of 125 keys per group at this context
    dev, host = pair(1, n, BKV_Q8_0, BKV_Q8_0)
    k, v = oracle.synth_kv(n, 4, 256, 23, 0, outliers=3)
    q, _ = qg(23, 0)
    qsum = q.reshape(4, 4, 256).sum(axis=1)    # [kv group][dim]: the group's four query rows
    k[:40] = -2.0 * qsum[None]
    k[40:kpw] = -0.3 * qsum[None] + 0.1 * k[40:kpw]
    host.append(0, 0, k, v)
    dev.append(0, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    want, _, sc, pr, p16 = host.decode(0, n, q, debug=True, nthreads=8)
    out, _ = dev.decode(0, n, torch.from_numpy(q).cuda())
    torch.cuda.synchronize()
    _, e, ssum, status = dev.debug_intermediates(n)
    x = sc * np.float32(0.0625)
    e_want = np.exp((x - x.max(axis=1, keepdims=True)).astype(np.float64)).astype(np.float32)
    run = np.cumsum(e_want.astype(np.float64), axis=1)
    # what the shape promises: > 32 tiny-sum specials in workgroup 0, >= 2 binade crossings in workgroup 1
    assert np.all(run[:, 33] < 2.0 ** -17)
    assert np.all(np.floor(np.log2(run[:, 2 * kpw - 1])) - np.floor(np.log2(run[:, kpw - 1])) >= 2)
    assert oracle.bit_diff(e.numpy(), e_want) == 0
    if path != "split":                       # (the split path's larger chunks overflow their record
        assert int(status.sum()) == 0, "the exact walk fell back to the serial loop"   # and take it)
    p_gpu = (e.numpy() / ssum.numpy()[:, None]).astype(np.float32)
    assert oracle.bit_diff(p_gpu, pr) == 0
    assert np.array_equal(oracle.f32_to_f16(p_gpu), p16)
    assert report("out", out.cpu().numpy(), want) <= TOL
