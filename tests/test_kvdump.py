"""The TSV dump (bonsai_vk_amd.kvdump) prints a cache exactly as the reference's kv_dump does
(runtime_vk/bonsai_forward.h:1404-1488): the arena bytes of the reference's two layer-0 runs are
rebuilt from kv_dump_v4.npz, and the dump of them must reproduce the reference's own lines
(tests/golden/kv_*_v4_excerpt.tsv, excerpts of runs/kv_q8_0_v4.tsv and runs/kv_none_v4.tsv)
character for character. Also: the synthetic fill fixture of the host cache."""
import os

import numpy as np

import oracle
from bonsai_vk_amd import kvdump

HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = os.path.join(HERE, "golden")


def excerpt(name):
    with open(os.path.join(GOLD, name)) as f:
        return [l.rstrip("\n") for l in f]


def rebuilt(v_q8):
    """A host cache of 256 slots holding the 37 positions of the reference run."""
    z = np.load(os.path.join(GOLD, "kv_dump_v4.npz"))
    c = oracle.HostCache(n_layers=1, cap=256, k_fmt=oracle.F16, v_fmt=oracle.Q8_0 if v_q8 else oracle.F16)
    n = z["k_none"].shape[0]
    if v_q8:
        c.k_data[0, :n] = z["k_q8run"].reshape(n, -1).view(np.uint8)
        c.v_data[0, :n] = z["v_q8_int"].reshape(n, -1).view(np.uint8)
        c.v_scales[0, :n] = z["v_q8_scale"].reshape(n, -1).view(np.uint8)
    else:
        c.k_data[0, :n] = z["k_none"].reshape(n, -1).view(np.uint8)
        c.v_data[0, :n] = z["v_none"].reshape(n, -1).view(np.uint8)
    return c, n


def check_against(lines, want):
    by_pos = {}
    for l in lines[1:]:
        by_pos.setdefault(int(l.split()[1]), []).append(l)
    assert lines[0] == want[0]
    got = []
    for p in sorted({int(l.split()[1]) for l in want[1:]}):
        got += by_pos[p]
    assert got == want[1:]


def test_q8_v_dump_matches_reference_lines():
    c, n = rebuilt(True)
    lines = kvdump.dump_cache(c, 0, n)
    assert len(lines) == 1 + n * (4 * 256 + 4 * (8 + 256))
    check_against(lines, excerpt("kv_q8_0_v4_excerpt.tsv"))


def test_f16_v_dump_matches_reference_lines():
    c, n = rebuilt(False)
    lines = kvdump.dump_cache(c, 0, n)
    check_against(lines, excerpt("kv_none_v4_excerpt.tsv"))


def test_max_pos_and_q8_k_header():
    c = oracle.HostCache(n_layers=2, cap=64, k_fmt=oracle.Q8_0, v_fmt=oracle.Q8_0)
    k, v = oracle.synth_kv(10, 4, 256, 3, 1, outliers=3)
    c.append(1, 0, k, v)
    lines = kvdump.dump_cache(c, 1, 10, max_pos=4)
    assert lines[0].startswith("# layer 1  positions 4  nkv 4  hd 256  v_q8 1  kk 256 kvd 256 kvs 16  kks 16")
    assert len(lines) == 1 + 4 * (4 * 256 + 4 * (8 + 256))
    # K lines are the q8_0 reconstruction: f16(scale) * int8, the same rows the oracle decodes with
    kq = np.array([float(l.split()[4]) for l in lines[1:] if l.startswith("K 2 3 ")], np.float32)
    assert np.array_equal(kq, c.row(0, 1, 2, 3))


def test_fill_synthetic_host():
    c = oracle.HostCache(n_layers=2, cap=8, k_fmt=oracle.F16, v_fmt=oracle.Q8_0)
    c.fill_synthetic()
    lines = kvdump.dump_cache(c, 1, 1)
    vals = {l.split()[0]: set() for l in lines[1:]}
    for l in lines[1:]:
        vals[l.split()[0]].add(float(l.split()[4]))
    assert vals == {"K": {1.0}, "S": {1.0}, "V": {0.0, 60.0}}
