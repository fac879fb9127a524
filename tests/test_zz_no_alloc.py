"""bkv_decode_step_static (the workspace in a static device array, no allocation) against
bkv_decode_step on the same inputs, through the C ABI: two calls in a row, the second over a
smaller context, each bit-identical to the workspace entry point (same kernels, same cache bytes,
same outputs), and the size limit rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from bonsai_vk_amd import BKV_F16, BKV_Q8_0, KvCache
from bonsai_vk_amd._lib import check, lib
from tests.gpu_util import say

pytestmark = pytest.mark.gpu


def _filled(n, kf, vf, seed):
    c = KvCache(n_layers=2, cap=n + 8, k_fmt=kf, v_fmt=vf)
    k, v = oracle.synth_kv(n, 4, 256, seed, 1, outliers=3)
    c.append(1, 0, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    return c


def _step(c, pos, k, v, q, g, static):
    out = torch.full((16, 256), np.nan, device="cuda")
    og = torch.full((16, 256), np.nan, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    d = ctypes.byref(c.desc)
    if static:
        rc = lib().bkv_decode_step_static(d, 1, pos, k.data_ptr(), v.data_ptr(), q.data_ptr(), g.data_ptr(),
                                          out.data_ptr(), og.data_ptr(), st)
    else:
        rc = lib().bkv_decode_step(d, 1, pos, k.data_ptr(), v.data_ptr(), q.data_ptr(), g.data_ptr(),
                                   out.data_ptr(), og.data_ptr(), c.workspace.data_ptr(), c.workspace.numel(), st)
    check(rc, "static" if static else "workspace")
    torch.cuda.synchronize()
    return out.cpu(), og.cpu()


@pytest.mark.parametrize("kf,vf", [(BKV_Q8_0, BKV_Q8_0), (BKV_F16, BKV_Q8_0)])
def test_static_matches_workspace(kf, vf):
    assert lib().bkv_static_scratch_bytes() == 16 << 20
    for call, n in enumerate([20000, 3000]):          # the second call: a smaller context
        say(f"no-alloc decode_step kf={kf} vf={vf} call={call} pos={n}")
        a, b = _filled(n, kf, vf, 40 + call), _filled(n, kf, vf, 40 + call)
        gen = torch.Generator(device="cuda").manual_seed(7 + call)
        k, v, q, g = (torch.randn(s, generator=gen, device="cuda") for s in [(4, 256), (4, 256), (16, 256), (16, 256)])
        want = _step(a, n, k, v, q, g, static=False)
        got = _step(b, n, k, v, q, g, static=True)
        for w, x in zip(want, got):
            assert torch.isfinite(w).all()
            assert torch.equal(w.view(torch.int32), x.view(torch.int32))
        for x, y in zip(a.host_arrays(), b.host_arrays()):
            if x is not None:
                assert torch.equal(x, y)


def test_static_rejects_oversize():
    n = 100000                                         # its decode plan exceeds the 16 MiB array
    c = KvCache(n_layers=1, cap=n + 8, max_ctx=1)
    lay = (ctypes.c_uint64 * 6)()
    check(lib().bkv_debug_layout(ctypes.byref(c.desc), n + 1, lay), "layout")
    assert lay[5] > lib().bkv_static_scratch_bytes()
    z = torch.zeros(16, 256, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib().bkv_decode_step_static(ctypes.byref(c.desc), 0, n, z.data_ptr(), z.data_ptr(), z.data_ptr(),
                                      None, z.data_ptr(), None, st)
    assert rc == -9                                    # BKV_ESCRATCH, nothing launched
    torch.cuda.synchronize()
    assert int(c.k_data.count_nonzero()) == 0          # the cache was not written


def _hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return h


def test_static_error_word_and_reset():
    """bkv_static_error: clean after ordinary static calls. A timed-out static call is imitated from
    the host (the array's error word set): the check reports BKV_ETIMEOUT and zeroes the array, the
    next check is clean, and static calls after it (and after bkv_static_reset) equal the workspace
    entry point bit for bit."""
    n = 3000
    a, b = _filled(n, BKV_Q8_0, BKV_Q8_0, 60), _filled(n, BKV_Q8_0, BKV_Q8_0, 60)
    gen = torch.Generator(device="cuda").manual_seed(61)
    k, v, q, g = (torch.randn(s, generator=gen, device="cuda") for s in [(4, 256), (4, 256), (16, 256), (16, 256)])
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    d = ctypes.byref(b.desc)
    _step(a, n, k, v, q, g, static=False)
    _step(b, n, k, v, q, g, static=True)
    assert lib().bkv_static_error(d, st) == 0
    addr = ctypes.c_void_p()
    check(lib().bkv_static_debug_address(ctypes.byref(addr)), "address")
    assert addr.value
    off = (ctypes.c_uint64 * 1)()
    check(lib().bkv_error_words(d, off), "error word")
    hip = _hip()
    one = ctypes.c_uint32(1)
    torch.cuda.synchronize()
    assert hip.hipMemcpy(addr.value + off[0], ctypes.byref(one), 4, 1) == 0      # host to device
    assert lib().bkv_static_error(d, st) == -8                                   # BKV_ETIMEOUT
    head = np.zeros(1 << 16, np.uint32)
    assert hip.hipMemcpy(head.ctypes.data, addr.value, head.nbytes, 2) == 0      # device to host
    assert int(np.count_nonzero(head)) == 0                                      # zeroed
    assert lib().bkv_static_error(d, st) == 0
    for reset in (False, True):
        if reset:
            check(lib().bkv_static_reset(st), "reset")
        pos = n + 1 + int(reset)
        want = _step(a, pos, k, v, q, g, static=False)
        got = _step(b, pos, k, v, q, g, static=True)
        for w, x in zip(want, got):
            assert torch.equal(w.view(torch.int32), x.view(torch.int32))
