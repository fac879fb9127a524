"""CPU oracle of the KV-cache path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker; the product library never calls it. It wraps oracle/libbko.so (bkv_oracle.c, a
plain-C restatement of hiyoing/bonsai-vk's KV path, each function citing the reference file:line it
follows) and, when built, oracle/_ref/libattnref.so (the reference's own CPU mirror compiled from its
sources by oracle/Makefile).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libbko.so")
REF_LIB = os.path.join(HERE, "_ref", "libattnref.so")
F16, Q8_0 = 0, 1


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class Desc(ctypes.Structure):
    """struct bkv_cache_desc with HOST pointers."""
    _fields_ = [
        ("n_layers", ctypes.c_int32), ("nh", ctypes.c_int32), ("nkv", ctypes.c_int32),
        ("hd", ctypes.c_int32), ("cap", ctypes.c_int32), ("k_fmt", ctypes.c_int32),
        ("v_fmt", ctypes.c_int32), ("page_tokens", ctypes.c_int32), ("max_pages", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("k_data", ctypes.c_void_p), ("k_scales", ctypes.c_void_p),
        ("v_data", ctypes.c_void_p), ("v_scales", ctypes.c_void_p),
        ("layer_stride_bytes", ctypes.c_uint64 * 4),
        ("block_table", ctypes.c_void_p),
    ]


_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        P, D, u32, i32, sz = ctypes.c_void_p, ctypes.POINTER(Desc), ctypes.c_uint32, ctypes.c_int, ctypes.c_size_t
        sig = {
            "bko_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "bko_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "bko_f32_to_f16_array": (None, [P, P, sz]),
            "bko_f16_to_f32_array": (None, [P, P, sz]),
            "bko_q8_block": (None, [P, i32, P, P]),
            "bko_q8_block_ties": (i32, [P]),
            "bko_slot": (ctypes.c_int64, [D, i32, ctypes.c_int64]),
            "bko_kv_append": (None, [D, i32, u32, i32, P, P, i32]),
            "bko_load_row": (None, [D, i32, i32, ctypes.c_int64, i32, P]),
            "bko_attn_decode": (None, [D, i32, u32, P, P, P, P, P, P, P, i32]),
            "bko_attn_decode_heads": (None, [D, i32, u32, P, P, P, P, i32, i32]),
            "bko_attn_decode_ideal": (None, [D, i32, u32, P, i32, P]),
            "bko_attn_prefill": (None, [D, i32, u32, i32, P, P, P, P, i32]),
            "bko_splitmix64": (ctypes.c_uint64, [ctypes.c_uint64]),
            "bko_fill_normal": (None, [P, sz, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]),
            "bko_outlier_channels": (None, [ctypes.c_uint64, i32, i32, i32, i32, P]),
            "bko_apply_outliers": (None, [P, i32, i32, i32, ctypes.c_uint64, i32, i32, ctypes.c_float]),
            "bko_now": (ctypes.c_double, []),
            "bko_set_exp_mode": (None, [i32]),
            "bko_max_threads": (i32, []),
            "bko_norm_rope_row": (None, [i32, i32, ctypes.c_float, ctypes.c_float, P, P, u32, i32, P]),
            "bko_norm_rope_append": (None, [D, i32, u32, i32, P, P, P, P, P, i32, ctypes.c_float,
                                            ctypes.c_float, i32, P]),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def ref():
    """The reference's own mirror (oracle/_ref), or None when it was not built here."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB):
        L = ctypes.CDLL(REF_LIB)
        L.ref_f32_to_f16_bits.restype, L.ref_f32_to_f16_bits.argtypes = ctypes.c_uint16, [ctypes.c_float]
        L.ref_f16_to_f32.restype, L.ref_f16_to_f32.argtypes = ctypes.c_float, [ctypes.c_uint16]
        P = ctypes.c_void_p
        L.ref_decode_row.restype = None
        L.ref_decode_row.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, P, P, P,
                                     ctypes.c_int, ctypes.c_int, P, P, P, P, P, P]
        L.ref_decode_rows.restype = None
        L.ref_decode_rows.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, P,
                                      P, P, ctypes.c_size_t, ctypes.c_int, P, P, ctypes.c_int]
        L.ref_norm_rope_row.restype = None
        L.ref_norm_rope_row.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float, P, P,
                                        ctypes.c_int, P]
        _ref = L
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# the reference model's rope geometry (attn_vk.h:65-77: n_rot 64, eps 1e-6, freq_base 1e7)
NROT, EPS, FREQ_BASE = 64, 1.0e-6, 10000000.0


def norm_rope_row(x, w, pos, nrot=NROT, eps=EPS, base=FREQ_BASE, libm_float=False):
    """bko_norm_rope_row: one row's RMS norm, weight and rope (fp32)."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    lib().bko_norm_rope_row(x.size, nrot, eps, base, _p(x), _p(w), pos, int(libm_float), _p(y))
    return y


def ref_norm_rope_row(x, w, pos, nrot=NROT, eps=EPS, base=FREQ_BASE):
    """The reference's attn_rms_norm + attn_rope compiled from attn_vk.h, or None when not built."""
    R = ref()
    if R is None:
        return None
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    y = np.empty_like(x)
    R.ref_norm_rope_row(x.size, nrot, eps, base, _p(x), _p(w), pos, _p(y))
    return y


class exp_mode:
    """context manager: 0 = correctly rounded exp (default), 1 = libm expf (the reference mirror's)"""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        lib().bko_set_exp_mode(self.mode)

    def __exit__(self, *a):
        lib().bko_set_exp_mode(0)


# ------------------------------------------------------------------ fp16 / q8_0
def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty(x.shape, dtype=np.uint16)
    lib().bko_f32_to_f16_array(_p(x), _p(h), x.size)
    return h


def f16_to_f32(h):
    h = np.ascontiguousarray(h, dtype=np.uint16)
    x = np.empty(h.shape, dtype=np.float32)
    lib().bko_f16_to_f32_array(_p(h), _p(x), h.size)
    return x


def q8_block(x, rhaz=0):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == 32
    q = np.empty(32, dtype=np.uint8)
    s = np.zeros(1, dtype=np.uint16)
    lib().bko_q8_block(_p(x), rhaz, _p(q), _p(s))
    return q.view(np.int8), int(s[0])


def q8_ties(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    return lib().bko_q8_block_ties(_p(x))


# ------------------------------------------------------------------ synthetic data
def normal(n, seed, stream, sigma=1.0):
    x = np.empty(int(n), dtype=np.float32)
    lib().bko_fill_normal(_p(x), x.size, seed, stream, sigma)
    return x


def outlier_channels(seed, layer, head, hd=256, n_out=3):
    ch = np.empty(n_out, dtype=np.int32)
    lib().bko_outlier_channels(seed, layer, head, hd, n_out, _p(ch))
    return ch


def synth_kv(n_tok, nkv, hd, seed, layer, outliers=3, k_sigma=1.0, v_sigma=0.5, stream_base=0):
    """K ~ N(0,1) with `outliers` seeded channels per (layer, kv head) scaled x8, V ~ N(0, v_sigma)."""
    k = normal(n_tok * nkv * hd, seed, stream_base + 1000 * layer + 1, k_sigma).reshape(n_tok, nkv, hd)
    v = normal(n_tok * nkv * hd, seed, stream_base + 1000 * layer + 2, v_sigma).reshape(n_tok, nkv, hd)
    if outliers:
        lib().bko_apply_outliers(_p(k), n_tok, nkv, hd, seed, layer, outliers, 8.0)
    return k, v


# ------------------------------------------------------------------ host cache
class HostCache:
    """The cache layout of include/bkv.h in host memory, driven by the oracle."""

    def __init__(self, n_layers=1, nh=16, nkv=4, hd=256, cap=256, k_fmt=Q8_0, v_fmt=Q8_0,
                 page_tokens=0, max_pages=0, block_table=None, scale=None, rhaz=0):
        self.n_layers, self.nh, self.nkv, self.hd, self.cap = n_layers, nh, nkv, hd, cap
        self.k_fmt, self.v_fmt, self.rhaz = k_fmt, v_fmt, rhaz
        self.page_tokens, self.max_pages = page_tokens, max_pages
        rowb = lambda f: nkv * hd * (2 if f == F16 else 1)
        srow = nkv * (hd // 32) * 2
        self.k_data = np.zeros((n_layers, cap, rowb(k_fmt)), np.uint8)
        self.v_data = np.zeros((n_layers, cap, rowb(v_fmt)), np.uint8)
        self.k_scales = np.zeros((n_layers, cap, srow), np.uint8) if k_fmt == Q8_0 else None
        self.v_scales = np.zeros((n_layers, cap, srow), np.uint8) if v_fmt == Q8_0 else None
        self.block_table = None if block_table is None else np.ascontiguousarray(block_table, np.int32)
        d = Desc()
        d.n_layers, d.nh, d.nkv, d.hd, d.cap = n_layers, nh, nkv, hd, cap
        d.k_fmt, d.v_fmt, d.page_tokens, d.max_pages = k_fmt, v_fmt, page_tokens, max_pages
        d.scale = float(scale if scale is not None else 1.0 / hd ** 0.5)
        for i, a in enumerate((self.k_data, self.k_scales, self.v_data, self.v_scales)):
            if a is not None:
                setattr(d, ("k_data", "k_scales", "v_data", "v_scales")[i], a.ctypes.data)
                d.layer_stride_bytes[i] = a.strides[0]
        d.block_table = None if self.block_table is None else self.block_table.ctypes.data
        self.desc = d

    def arrays(self):
        return [self.k_data, self.k_scales, self.v_data, self.v_scales]

    def load_arrays(self, arrs):
        """Copy device-cache contents (KvCache.host_arrays()) into this cache."""
        for mine, theirs in zip(self.arrays(), arrs):
            if mine is not None:
                mine[...] = np.asarray(theirs)

    def norm_rope_append(self, layer, pos0, q_in, k_in, v_in, qn_w, kn_w, nrot=NROT, eps=EPS,
                         base=FREQ_BASE):
        """bko_norm_rope_append: returns the normed + roped Q [n][nh][hd]; K (normed + roped) and V go
        into the cache at pos0.."""
        q_in, k_in, v_in, qn_w, kn_w = (np.ascontiguousarray(a, np.float32) for a in (q_in, k_in, v_in, qn_w, kn_w))
        n = q_in.shape[0]
        q_out = np.empty_like(q_in)
        lib().bko_norm_rope_append(ctypes.byref(self.desc), layer, pos0, n, _p(q_in), _p(k_in), _p(v_in),
                                   _p(qn_w), _p(kn_w), nrot, eps, base, self.rhaz, _p(q_out))
        return q_out

    def fill_synthetic(self):
        """The reference's timing fixture (runtime_vk/bonsai_forward.h:1355-1370): the whole KV arena
        filled with the word 0x3C003C00 (fp16 1.0 pairs; q8_0 bytes 0/60 with fp16 scale 1.0)."""
        for a in self.arrays():
            if a is not None:
                a.view(np.uint32)[...] = 0x3C003C00

    def slot(self, layer, pos):
        return lib().bko_slot(ctypes.byref(self.desc), layer, pos)

    def append(self, layer, pos, k, v):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        lib().bko_kv_append(ctypes.byref(self.desc), layer, pos, k.shape[0], _p(k), _p(v), self.rhaz)

    def row(self, which, layer, pos, head):
        out = np.empty(self.hd, np.float32)
        lib().bko_load_row(ctypes.byref(self.desc), which, layer, pos, head, _p(out))
        return out

    def decode(self, layer, nfill, q, gate=None, nthreads=1, debug=False):
        q = np.ascontiguousarray(q, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        out = np.empty((self.nh, self.hd), np.float32)
        og = None if g is None else np.empty_like(out)
        sc = pr = p16 = None
        if debug:
            sc = np.empty((self.nh, nfill), np.float32)
            pr = np.empty((self.nh, nfill), np.float32)
            p16 = np.empty((self.nh, nfill), np.uint16)
        lib().bko_attn_decode(ctypes.byref(self.desc), layer, nfill, _p(q), _p(g), _p(out), _p(og),
                              _p(sc), _p(pr), _p(p16), nthreads)
        if debug:
            return out, og, sc, pr, p16
        return out, og

    def decode_heads(self, layer, nfill, q, h0, h1, gate=None):
        q = np.ascontiguousarray(q, np.float32)
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        out = np.zeros((self.nh, self.hd), np.float32)
        og = None if g is None else np.zeros_like(out)
        lib().bko_attn_decode_heads(ctypes.byref(self.desc), layer, nfill, _p(q), _p(g), _p(out),
                                    _p(og), h0, h1)
        return out, og

    def ideal(self, layer, nfill, q, round_bits=3):
        q = np.ascontiguousarray(q, np.float32)
        out = np.empty((self.nh, self.hd), np.float64)
        lib().bko_attn_decode_ideal(ctypes.byref(self.desc), layer, nfill, _p(q), round_bits, _p(out))
        return out

    def prefill(self, layer, pos0, q, gate=None, nthreads=1):
        q = np.ascontiguousarray(q, np.float32)
        n = q.shape[0]
        g = None if gate is None else np.ascontiguousarray(gate, np.float32)
        out = np.empty((n, self.nh, self.hd), np.float32)
        og = None if g is None else np.empty_like(out)
        lib().bko_attn_prefill(ctypes.byref(self.desc), layer, pos0, n, _p(q), _p(g), _p(out), _p(og),
                               nthreads)
        return out, og


def rel_err(got, want):
    """max |got - want| / max |want| per head row, maximised over rows (the tolerance measure)."""
    got = np.asarray(got, np.float64).reshape(-1, np.asarray(want).shape[-1])
    want = np.asarray(want, np.float64).reshape(got.shape)
    den = np.maximum(np.abs(want).max(axis=1), 1e-30)
    return float((np.abs(got - want).max(axis=1) / den).max())


def bit_diff(got, want):
    """number of fp32 elements whose bit patterns differ"""
    return int((np.asarray(got, np.float32).view(np.uint32) != np.asarray(want, np.float32).view(np.uint32)).sum())
