"""Helpers for the GPU parity tests: build matching device (libbkv) and host (oracle) caches."""
import numpy as np
import torch

import oracle
from bonsai_vk_amd import KvCache


def say(*a):
    print(*a, flush=True)


def pair(n_layers, cap, k_fmt, v_fmt, page_tokens=0, max_pages=0, block_table=None, max_ctx=None):
    dev = KvCache(n_layers=n_layers, cap=cap, k_fmt=k_fmt, v_fmt=v_fmt, page_tokens=page_tokens,
                  max_pages=max_pages, block_table=block_table, max_ctx=max_ctx)
    host = oracle.HostCache(n_layers=n_layers, cap=cap, k_fmt=k_fmt, v_fmt=v_fmt,
                            page_tokens=page_tokens, max_pages=max_pages, block_table=block_table)
    return dev, host


def fill(dev, host, layer, n, seed, outliers=3, chunk=8192):
    """append n synthetic tokens to both caches (device through bkv_kv_append)"""
    k, v = oracle.synth_kv(n, dev.nkv, dev.hd, seed, layer, outliers=outliers)
    host.append(layer, 0, k, v)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        dev.append(layer, s, torch.from_numpy(k[s:e]).cuda(), torch.from_numpy(v[s:e]).cuda())
    return k, v


def qg(seed, layer, nh=16, hd=256, n=None):
    shape = (nh, hd) if n is None else (n, nh, hd)
    m = int(np.prod(shape))
    q = oracle.normal(m, seed, 500 + 7 * layer).reshape(shape)
    g = oracle.normal(m, seed, 501 + 7 * layer).reshape(shape)
    return q, g


def same_bytes(dev, host):
    d = dev.host_arrays()
    out = []
    for a, b in zip(d, host.arrays()):
        if b is None:
            continue
        out.append(int((a.numpy() != b).sum()))
    return out


def report(tag, got, want):
    r = oracle.rel_err(got, want)
    bd = oracle.bit_diff(got, want)
    say(f"{tag}: max rel err {r:.3e}, bit-diff {bd}/{np.asarray(want).size}")
    return r
