"""KV arena planning and the block-level refuse / evict policy, restated from the reference's host
side so an engine that moves onto libbkv keeps the same decisions:

  autofit_cap ... the OOM fallback of fwd_init (runtime_vk/bonsai_forward.h:1717-1834): with the
                  device budget, the resident weights and the cap-independent bytes known, the
                  largest EVEN cap whose cap-proportional bytes still fit, clamped to the widest row
                  the attention kernel takes; None when no cap fits at all.
  KvGuard ....... KvGuard (runtime_vk/kv_guard.h:579-648): blocks of blk_slots positions, and one
                  decision per block boundary from the next position and the spill metric.

KV_EVICT is returned as the reference returns it (evict the farthest block). Acting on it means
excluding that block's keys from the softmax, which the reference does with -INF in its additive
score mask; with libbkv the engine advances live_low by one block and attends with
bkv_attn_decode_window(kstart = live_low), the same computation (a -INF key adds exactly +0).
"""
from dataclasses import dataclass, field

from .cache import KvGeom

KV_OK, KV_WARN, KV_REFUSE, KV_EVICT = 0, 1, 2, 3


def autofit_cap(heap_bytes, weights_bytes, fixed_bytes, per_slot_bytes, row_limit):
    """The usable cap of the reference's OOM fallback (bonsai_forward.h:1760-1790): avail = heap -
    weights - cap-independent bytes; fit = avail // per_slot, made even (P16 packs key pairs), then
    clamped to row_limit. None when avail <= 0 (no cap fits; nothing may be dispatched)."""
    avail = int(heap_bytes) - int(weights_bytes) - int(fixed_bytes)
    if avail <= 0:
        return None
    fit = avail // int(per_slot_bytes)
    if fit & 1:
        fit -= 1
    return min(fit, int(row_limit))


@dataclass
class KvGuard:
    """kv_guard.h:579-648. init() sizes the blocks; decide() is the one decision point."""
    g: KvGeom = field(default_factory=KvGeom)
    cap: int = 0
    blk_slots: int = 64
    n_blk: int = 0
    bytes_per_blk: int = 0
    ceiling_bytes: int = 0
    allow_evict: bool = False
    g_spill_soft: float = 32.0
    g_spill_hard: float = 64.0
    live_low: int = 0
    n_refuse: int = 0
    n_evict: int = 0
    n_warn: int = 0

    def init(self, geom, cap, kv_ceiling_bytes, evict):
        self.g, self.cap, self.allow_evict = geom, int(cap), bool(evict)
        self.blk_slots = max(1, int(self.blk_slots))
        self.n_blk = self.cap // self.blk_slots
        self.bytes_per_blk = self.blk_slots * geom.bytes_slot
        self.ceiling_bytes = int(kv_ceiling_bytes)
        return self

    def decide(self, next_pos, value=0.0, have_counter=False, growing=False):
        """(action, why) at a block boundary (kv_guard.h:620-637): the geometry ceiling first; no
        counter -> OK; past the hard threshold AND growing -> evict the farthest block when allowed
        and there is one to spare (block index >= 1, at least 2 blocks), else refuse; past the soft
        threshold -> warn. The action counters advance as the reference's do."""
        b = int(next_pos) // self.blk_slots
        if next_pos >= self.cap:
            self.n_refuse += 1
            return KV_REFUSE, "KV arena full: the position reaches cap"
        if not have_counter:
            return KV_OK, ""
        if value > self.g_spill_hard and growing:
            if self.allow_evict and b >= 1 and self.n_blk >= 2:
                self.n_evict += 1
                self.live_low += self.blk_slots
                return KV_EVICT, "spill: evict the farthest KV block"
            self.n_refuse += 1
            return KV_REFUSE, "spill: refuse new KV blocks"
        if value > self.g_spill_soft:
            self.n_warn += 1
            return KV_WARN, "spill: past the soft threshold, watching"
        return KV_OK, ""

    def report(self):
        """the reference's one-line summary (kv_guard.h:639-645)"""
        M = 1048576.0
        return (f"  KV block hook: {self.cap} slots = {self.n_blk} blocks of {self.blk_slots} positions, "
                f"{self.bytes_per_blk / M:.2f} MiB per block ({self.g.bytes_slot / 1024.0:.2f} KiB/slot x "
                f"{self.g.n_attn} layers x {self.blk_slots}), ceiling {self.ceiling_bytes / M:.2f} MiB, "
                f"evict {'ENABLED (BONSAI_KV_EVICT=1)' if self.allow_evict else 'off'}")
