"""Writes tests/golden/kv_dump_v4.npz from the reference's committed KV dumps (data, not code):
  runs/kv_none_v4.tsv  - layer-0 arena of a run with fp16 V (BONSAI_KV_V_QUANT=none), 37 positions
  runs/kv_q8_0_v4.tsv  - the same prompt and binary with q8_0 V: reconstructed V and fp16 scales S
Both were written by kv_dump (runtime_vk/bonsai_forward.h:1404-1488). Run in the build container
only (the reference checkout is absent on the GPU box):  python tests/golden/make_kv_fixtures.py
"""
import os
import sys

import numpy as np

REF = os.environ.get("BONSAI_REF", "/root/reference")
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kv_dump_v4.npz")


def read(path):
    K, V, S = {}, {}, {}
    with open(path) as f:
        for line in f:
            if line.startswith("#"):
                continue
            t, p, h, i, val = line.split()
            key = (int(p), int(h), int(i))
            {"K": K, "V": V, "S": S}[t][key] = np.float32(float(val))
    return K, V, S


def dense(dct, npos, nkv, n):
    a = np.zeros((npos, nkv, n), np.float32)
    for (p, h, i), v in dct.items():
        a[p, h, i] = v
    return a


def main():
    kn, vn, _ = read(os.path.join(REF, "runs", "kv_none_v4.tsv"))
    kq, vq, sq = read(os.path.join(REF, "runs", "kv_q8_0_v4.tsv"))
    npos, nkv, hd = 37, 4, 256
    k_none, v_none = dense(kn, npos, nkv, hd), dense(vn, npos, nkv, hd)
    k_q8, v_q8, s_q8 = dense(kq, npos, nkv, hd), dense(vq, npos, nkv, hd), dense(sq, npos, nkv, hd // 32)
    # q8_0 V as (int8, fp16 scale): V = S * int exactly (kv_dump prints float(scale) * float(byte))
    s_rep = np.repeat(s_q8, 32, axis=2)
    qint = np.where(s_rep != 0, v_q8 / np.where(s_rep != 0, s_rep, 1), 0)
    assert np.all(qint == np.round(qint)), "V is not an integer multiple of its block scale"
    assert np.all(np.abs(qint) <= 127)
    assert np.all(s_rep * qint.astype(np.float32) == v_q8)
    np.savez_compressed(
        OUT,
        k_none=k_none.astype(np.float16), v_none=v_none.astype(np.float16),
        k_q8run=k_q8.astype(np.float16), v_q8_int=qint.astype(np.int8),
        v_q8_scale=s_q8.astype(np.float16))
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    sys.exit(main())
