"""KV-cache dump in the reference's TSV format (kv_dump, runtime_vk/bonsai_forward.h:1404-1488), so a
cache held by libbkv can be diffed line for line against the reference's runs/kv_*.tsv with the
reference's own tools/kv_compare.py.

One file covers one layer's first min(nfill, max_pos) positions:
    # layer L  positions N  nkv H  hd D  v_q8 Q  kk A kvd B kvs C  per-layer W words
    K p h d value          fp16 K, every element (d ascending, heads ascending)
    S p h b value          q8_0 V: the fp16 scale of block b (8 lines per head, before its V lines)
    V p h d value          V, fp16 or the q8_0 reconstruction float(fp16 scale) * int8
values printed as %.9g of the fp32 value. kk / kvd / kvs are u32 words per slot of K, V data and V
scales (KvGeom, runtime_vk/kv_guard.h:118-130); per-layer = cap * (kk + kvd + kvs).
A q8_0 K (which the reference never stores) prints its reconstructed values on the K lines, and the
header then carries an extra "kks" field (K scale words per slot) before "per-layer".
"""
import numpy as np

F16, Q8_0 = 0, 1


def _fmt(x):
    return "%.9g" % float(x)


def dump_lines(arrays, layer, nfill, cap, nkv=4, hd=256, k_fmt=F16, v_fmt=Q8_0, max_pos=None,
               block_table=None, page_tokens=0):
    """Lines (without newlines) of the dump of one layer. arrays: (k_data, k_scales, v_data,
    v_scales) as uint8 arrays [n_layers][cap][row bytes] (None where absent)."""
    kd, ks, vd, vs = [None if a is None else np.asarray(a) for a in arrays]
    npos = nfill if max_pos is None else min(nfill, max_pos)
    kk = nkv * hd // (4 if k_fmt == Q8_0 else 2)
    kvd = nkv * hd // (4 if v_fmt == Q8_0 else 2)
    kvs = nkv * hd // 64 if v_fmt == Q8_0 else 0
    kks = nkv * hd // 64 if k_fmt == Q8_0 else 0
    extra = f"  kks {kks}" if k_fmt == Q8_0 else ""
    yield (f"# layer {layer}  positions {npos}  nkv {nkv}  hd {hd}  v_q8 {int(v_fmt == Q8_0)}  "
           f"kk {kk} kvd {kvd} kvs {kvs}{extra}  per-layer {cap * (kk + kvd + kvs + kks)} words")

    def slot(p):
        if not page_tokens:
            return p
        return int(block_table[layer][p // page_tokens]) * page_tokens + p % page_tokens

    def q8_values(data, scales, sl):
        b = data[layer, sl].view(np.int8).reshape(nkv, hd).astype(np.float32)
        sc = scales[layer, sl].view(np.float16).reshape(nkv, hd // 32).astype(np.float32)
        return sc, b * np.repeat(sc, 32, axis=1)       # fp32 products, as the reference prints them

    for p in range(npos):
        sl = slot(p)
        if k_fmt == Q8_0:
            kv = q8_values(kd, ks, sl)[1]
        else:
            kv = kd[layer, sl].view(np.float16).reshape(nkv, hd).astype(np.float32)
        for h in range(nkv):
            for d in range(hd):
                yield f"K {p} {h} {d} {_fmt(kv[h, d])}"
        if v_fmt == Q8_0:
            sc, vv = q8_values(vd, vs, sl)
            for h in range(nkv):
                for b in range(hd // 32):
                    yield f"S {p} {h} {b} {_fmt(sc[h, b])}"
                for d in range(hd):
                    yield f"V {p} {h} {d} {_fmt(vv[h, d])}"
        else:
            vv = vd[layer, sl].view(np.float16).reshape(nkv, hd).astype(np.float32)
            for h in range(nkv):
                for d in range(hd):
                    yield f"V {p} {h} {d} {_fmt(vv[h, d])}"


def dump_cache(cache, layer, nfill, path=None, max_pos=None):
    """Dump a bonsai_vk_amd.KvCache (device arrays are copied to the host) or an oracle.HostCache.
    Returns the lines; writes them to `path` when given."""
    arrs = cache.host_arrays() if hasattr(cache, "host_arrays") else cache.arrays()
    arrs = [None if a is None else (a.numpy() if hasattr(a, "numpy") else a) for a in arrs]
    bt = getattr(cache, "block_table_host", None)
    if bt is None:
        bt = getattr(cache, "block_table", None)
        if bt is not None and hasattr(bt, "cpu"):
            bt = bt.cpu().numpy()
    lines = list(dump_lines(arrs, layer, nfill, cache.cap, cache.nkv, cache.hd, cache.k_fmt,
                            cache.v_fmt, max_pos, bt, getattr(cache, "page_tokens", 0) or 0))
    if path is not None:
        with open(path, "w") as f:
            f.write("\n".join(lines) + "\n")
    return lines
