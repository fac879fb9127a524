"""q8_0 quantise-on-write of the oracle (attn_norm_rope2.comp:102-115, :184-217), pinned by the
format's invariants, special cases, brute force over tiny blocks and the reference's own dumps."""
import os

import numpy as np

import oracle

GOLD = os.path.join(os.path.dirname(__file__), "golden", "kv_dump_v4.npz")


def f16(x):
    return np.float32(x).astype(np.float16).astype(np.float32)


def test_invariants_random_blocks():
    rng = np.random.default_rng(3)
    for t in range(3000):
        x = rng.standard_normal(32).astype(np.float32) * np.float32(10.0 ** rng.uniform(-6, 3))
        if t % 3 == 0:
            x[rng.integers(0, 32, 2)] *= 8
        q, s = oracle.q8_block(x)
        amax = np.abs(x).max()
        d = np.float32(amax) / np.float32(127)
        assert s == np.float32(d).astype(np.float16).view(np.uint16)
        assert np.abs(q.astype(int)).max() == 127          # the absmax element lands on +-127
        assert np.all(np.abs(q.astype(int)) <= 127)
        # each byte is within half a step of x/d (the unrounded fp32 id = 1/d)
        idv = np.float32(1) / d
        assert np.all(np.abs(x * idv - q) <= 0.5 + 1e-6)
        # the absmax element's sign survives
        i = np.argmax(np.abs(x))
        assert np.sign(q[i]) == np.sign(x[i])


def test_dead_and_tiny_blocks():
    q, s = oracle.q8_block(np.zeros(32, np.float32))
    assert not q.any() and s == 0
    x = np.full(32, 1e-36, np.float32)              # amax <= 1e-35: d = 0, id = 0
    q, s = oracle.q8_block(x)
    assert not q.any() and s == 0
    x = np.zeros(32, np.float32)
    x[5] = -2e-35                                    # live, but d underflows fp16 -> stored 0
    q, s = oracle.q8_block(x)
    assert q[5] == -127 and s == 0 and np.count_nonzero(q) == 1


def test_tie_rule_switch():
    # amax = 127 gives d = 1, id = 1 exactly, so x = k + 0.5 are exact ties
    x = np.array([127.0, 2.5, -2.5, 3.5, 0.5, -0.5, 126.5, -126.5] + [0.0] * 24, np.float32)
    q_rne, _ = oracle.q8_block(x, rhaz=0)
    q_haz, _ = oracle.q8_block(x, rhaz=1)
    assert list(q_rne[:8]) == [127, 2, -2, 4, 0, 0, 126, -126]
    assert list(q_haz[:8]) == [127, 3, -3, 4, 1, -1, 127, -127]
    assert oracle.q8_ties(x) == 7


def test_nonfinite_policy():
    x = np.ones(32, np.float32)
    x[3] = np.nan
    q, s = oracle.q8_block(x)                      # NaN does not raise amax; its byte is 0
    assert q[3] == 0 and q[0] == 127
    assert s == 0x2008 == int(np.float16(np.float32(1.0) / np.float32(127.0)).view(np.uint16))   # RNE fp16 of d = 1/127
    x = np.ones(32, np.float32)
    x[7] = np.inf                                  # amax = inf: d = inf, id = 0 -> all bytes 0
    q, s = oracle.q8_block(x)
    assert not q.any() and s == 0x7C00


def test_brute_force_tiny_blocks():
    """Every block over a small alphabet: the bytes are the nearest integers to x*id, ties even."""
    vals = np.array([0.0, 0.25, -0.5, 1.0, -1.75, 3.0, 127.0, -63.5], np.float32)
    rng = np.random.default_rng(11)
    for _ in range(2000):
        x = vals[rng.integers(0, len(vals), 32)]
        q, s = oracle.q8_block(x)
        amax = np.abs(x).max()
        if amax == 0:
            assert not q.any() and s == 0
            continue
        d = np.float32(amax) / np.float32(127)
        idv = np.float32(1) / d
        t = (x * idv).astype(np.float64)
        # brute force over the 255 candidate bytes: nearest, ties to even
        cand = np.arange(-127, 128)
        dist = np.abs(t[:, None] - cand[None, :])
        best = dist.min(axis=1, keepdims=True)
        ok = dist == best
        choice = np.array([c[o][np.argmin(np.abs(c[o]) % 2 != 0)] if o.sum() > 1 else c[o][0]
                           for c, o in zip(np.broadcast_to(cand, dist.shape), ok)])
        assert np.array_equal(q.astype(int), choice)


def test_reference_dump_requantised():
    """The reference's q8_0 V dump (runs/kv_q8_0_v4.tsv) against the oracle re-quantising the fp16 V
    of the same prompt (runs/kv_none_v4.tsv). The q8 run quantised fp32 V, the none run stored it
    rounded to fp16, so a byte may move where fp16 rounding crosses a rounding boundary - counted.
    Position 0 is layer 0's first write, identical input in both runs."""
    z = np.load(GOLD)
    # both runs store the same fp16 K (the in-run proof that the dumps are comparable)
    assert np.array_equal(z["k_none"][0], z["k_q8run"][0])
    v = z["v_none"][0].astype(np.float32)                # [4][256]
    qi, sc = z["v_q8_int"][0], z["v_q8_scale"][0]
    byte_diff = scale_diff = 0
    for h in range(4):
        for b in range(8):
            blk = v[h, 32 * b:32 * b + 32]
            q, s = oracle.q8_block(blk)
            ref_s = int(sc[h, b].view(np.uint16))
            if s != ref_s:
                scale_diff += 1
                # the fp32 amax the reference saw lies within half an fp16 ulp of the fp16 amax;
                # its scale must be what the same recipe gives at one end of that interval
                a16 = np.float16(np.abs(blk).max())
                ulp = np.float32(np.spacing(a16))
                ends = [np.float32(a16) - ulp / 2, np.float32(a16) + ulp / 2]
                cands = {int(np.float16(np.float32(e) / np.float32(127)).view(np.uint16)) for e in ends}
                assert ref_s in cands, (h, b, hex(s), hex(ref_s), cands)
            dq = np.abs(q.astype(int) - qi[h, 32 * b:32 * b + 32].astype(int))
            assert dq.max() <= 1
            byte_diff += int(dq.sum())
    assert scale_diff <= 12, scale_diff     # of 32 blocks
    assert byte_diff <= 16, byte_diff       # of 1024 bytes
    # invariants on every dumped block of the q8_0 run: |q| <= 127 and a live block reaches 127
    qa = np.abs(z["v_q8_int"].astype(int)).reshape(37, 4, 8, 32)
    live = z["v_q8_scale"].astype(np.float32) != 0
    assert np.all(qa.max(axis=3)[live] == 127)
    assert np.all(qa <= 127)
