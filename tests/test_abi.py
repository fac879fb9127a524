"""The C-ABI library loads, exports every symbol include/bkv.h declares, and its host-side
validation follows KvGeom (runtime_vk/kv_guard.h:94-150). No compute call is made here."""
import ctypes
import os
import re

import pytest

from bonsai_vk_amd import _lib
from bonsai_vk_amd._lib import BKV_F16, BKV_Q8_0, BkvCacheDesc
from bonsai_vk_amd.cache import KvGeom

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared():
    txt = open(os.path.join(ROOT, "include", "bkv.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(bkv_[a-z_0-9]+)\s*\(", txt)))


def test_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared()
    assert names, "no declarations parsed"
    for n in names:
        assert hasattr(L, n), n
    assert sorted(_lib.EXPORTS) == names


def desc(**kw):
    d = BkvCacheDesc()
    d.n_layers, d.nh, d.nkv, d.hd, d.cap = 8, 16, 4, 256, 4096
    d.k_fmt = d.v_fmt = BKV_Q8_0
    d.scale = 0.0625
    d.k_data, d.k_scales, d.v_data, d.v_scales = 0x100000, 0x200000, 0x300000, 0x400000
    for i, sb in enumerate((1024, 64, 1024, 64)):
        d.layer_stride_bytes[i] = sb * 4096
    for k, v in kw.items():
        setattr(d, k, v)
    return d


def call(name, *a):
    return getattr(_lib.lib(), name)(*a)


def test_geometry_rules_and_errors():
    ok = desc()
    assert call("bkv_geom_check", ctypes.byref(ok)) == 0
    assert call("bkv_geom_check", ctypes.byref(desc(hd=250))) == -2          # hd % 4 / % 32
    assert call("bkv_geom_check", ctypes.byref(desc(hd=96))) == -2           # hd/32 odd
    assert call("bkv_geom_check", ctypes.byref(desc(nh=15))) == -2           # nh % nkv
    assert call("bkv_geom_check", ctypes.byref(desc(k_scales=None))) == -1
    assert call("bkv_geom_check", ctypes.byref(desc(v_data=0x300008))) == -4
    assert call("bkv_geom_check", ctypes.byref(desc(k_fmt=7))) == -1
    assert call("bkv_geom_check", ctypes.byref(desc(page_tokens=256, max_pages=4))) == -1  # no table
    paged = desc(page_tokens=256, max_pages=256, block_table=0x500000)
    assert call("bkv_geom_check", ctypes.byref(paged)) == 0
    assert call("bkv_max_positions", ctypes.byref(paged)) == 65536
    assert call("bkv_max_positions", ctypes.byref(ok)) == 4096
    # the reference's per-slot bytes: K fp16 2048, V q8_0 data 1024 + scales 64 (3136 B/slot/layer)
    ref = desc(k_fmt=BKV_F16, k_scales=None)
    assert [call("bkv_slot_bytes", ctypes.byref(ref), i) for i in range(4)] == [2048, 0, 1024, 64]
    for e in range(-7, 1):
        assert call("bkv_strerror", e)


def test_cap_and_workspace_checks_before_any_launch():
    d = desc()
    z = ctypes.c_void_p(0x600000)
    # pos + n_tok > cap -> ECAP (the KvGuard REFUSE case), checked on the host
    assert call("bkv_kv_append", ctypes.byref(d), 0, 4096, 1, z, z, None) == -3
    assert call("bkv_kv_append", ctypes.byref(d), 8, 0, 1, z, z, None) == -1       # bad layer
    assert call("bkv_attn_decode", ctypes.byref(d), 0, 0, z, None, z, None, z, 1 << 30, None) == -3
    ws = call("bkv_workspace_bytes", ctypes.byref(d), 0, 4096)
    assert ws > 0
    assert call("bkv_attn_decode", ctypes.byref(d), 0, 4096, z, None, z, None, z, ws - 1, None) == -5
    assert call("bkv_attn_decode", ctypes.byref(d), 0, 16, z, z, z, None, z, ws, None) == -1   # gate w/o out
    # workspace bounds grow with the context
    sizes = [call("bkv_workspace_bytes", ctypes.byref(desc(cap=70000)), 0, n)
             for n in (1, 100, 4096, 5000, 32768, 65536, 70000)]
    assert sizes == sorted(sizes)


def test_unsupported_shapes_are_refused():
    d = desc(hd=128)
    z = ctypes.c_void_p(0x600000)
    assert call("bkv_geom_check", ctypes.byref(d)) == 0
    assert call("bkv_kv_append", ctypes.byref(d), 0, 0, 1, z, z, None) == -7


def test_kvgeom_mirror():
    g = KvGeom(nkv=4, hd=256, n_attn=8, v_q8=1, k_q8=0)
    assert g.check() == ""
    assert (g.w_k, g.w_vd, g.w_vs) == (512, 256, 16)
    assert g.w_layer * 4 == 3136
    assert g.bytes_slot == 25088                      # 24.50 KiB/token over 8 layers
    assert KvGeom(hd=96).check() and KvGeom(hd=250).check()
    g2 = KvGeom(v_q8=1, k_q8=1)
    assert g2.w_layer * 4 == 2176                     # both q8_0: 2176 B/slot/layer


def test_library_missing_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "nope.so"))
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError):
        _lib.lib()
