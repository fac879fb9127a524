"""The arena planner and the block-level policy (bonsai_vk_amd.guard) against the reference's rules
(runtime_vk/kv_guard.h:579-648, runtime_vk/bonsai_forward.h:1717-1834), case by case."""
from bonsai_vk_amd.cache import KvGeom
from bonsai_vk_amd.guard import KV_EVICT, KV_OK, KV_REFUSE, KV_WARN, KvGuard, autofit_cap


def test_geometry_bytes_match_the_reference_arena():
    g = KvGeom()                                   # fp16 K, q8_0 V: the reference's default
    assert (g.w_k, g.w_vd, g.w_vs, g.w_layer) == (512, 256, 16, 784)
    assert g.bytes_slot == 784 * 4 * 8 == 25088    # 24.50 KiB/token (runs/kvfx_c32768_q2048_v1.log:44)
    assert KvGeom(v_q8=0).w_layer == 1024


def test_autofit():
    per = 25088
    assert autofit_cap(1 << 30, 400 << 20, 100 << 20, per, 1 << 20) == 21900   # (2^30 - 500 MiB) // 25088 = 21901, made even
    assert autofit_cap(1 << 30, 400 << 20, 100 << 20, per, 2048) == 2048      # the kernel row limit
    assert autofit_cap(1000 + 3 * per, 500, 500, per, 99) == 2               # 3 slots fit -> even 2
    assert autofit_cap(1000, 600, 400, per, 99) is None                      # nothing fits


def test_decisions():
    g = KvGeom()
    kg = KvGuard(blk_slots=64).init(g, 1024, 1 << 30, evict=False)
    assert (kg.n_blk, kg.bytes_per_blk) == (16, 64 * g.bytes_slot)
    assert kg.decide(1024)[0] == KV_REFUSE                                   # geometry ceiling
    assert kg.decide(1023, value=1e9, have_counter=False)[0] == KV_OK        # no counter: no judgement
    assert kg.decide(640, value=100.0, have_counter=True, growing=False)[0] == KV_WARN   # a spike
    assert kg.decide(640, value=100.0, have_counter=True, growing=True)[0] == KV_REFUSE
    assert kg.decide(640, value=40.0, have_counter=True, growing=True)[0] == KV_WARN
    assert kg.decide(640, value=10.0, have_counter=True, growing=True)[0] == KV_OK
    ev = KvGuard(blk_slots=64).init(g, 1024, 1 << 30, evict=True)
    assert ev.decide(640, value=100.0, have_counter=True, growing=True)[0] == KV_EVICT
    assert ev.live_low == 64                                  # the window now starts one block later
    assert ev.decide(63, value=100.0, have_counter=True, growing=True)[0] == KV_REFUSE   # block 0
    small = KvGuard(blk_slots=64).init(g, 100, 1 << 30, evict=True)          # one whole block only
    assert small.decide(70, value=100.0, have_counter=True, growing=True)[0] == KV_REFUSE
    assert (kg.n_refuse, kg.n_warn, ev.n_evict) == (2, 2, 1)
    assert "16 blocks of 64 positions" in kg.report() and "evict off" in kg.report()
