"""Host mirror of the reference's KV arena geometry and attention call sites, over the C ABI.

KvGeom restates KvGeom (hiyoing/bonsai-vk runtime_vk/kv_guard.h:94-150): the per-slot word counts of
the K, V-data and V-scale sub-arenas and the three divisibility rules. KvCache owns device memory
(torch tensors, one allocation per sub-arena for all layers) and issues bkv_kv_append /
bkv_attn_decode / bkv_decode_step / bkv_attn_prefill_chunk on the current torch stream, the way the
engine's attn_block (runtime_vk/bonsai_forward.h:581-645) records its three attention dispatches.
"""
import ctypes
from dataclasses import dataclass

import torch

from ._lib import (BKV_F16, BKV_OP_DECODE, BKV_OP_PREFILL, BKV_Q8_0, BkvCacheDesc, check, lib)


@dataclass
class KvGeom:
    """Per-slot geometry in u32 words (kv_guard.h:118-130). k_q8 extends the reference (which never
    compresses K) with the same q8_0 layout V uses."""
    nkv: int = 4
    hd: int = 256
    n_attn: int = 8
    blk: int = 32
    v_q8: int = 1
    k_q8: int = 0

    def check(self):
        """KvGeom::check (kv_guard.h:103-113): returns '' or the reason the geometry is refused."""
        if self.hd % 4:
            return f"hd % 4 == {self.hd % 4}: a q8_0 data word would straddle elements"
        if self.hd % self.blk:
            return f"hd % blk == {self.hd % self.blk}: a block would straddle head rows"
        if (self.hd // self.blk) % 2:
            return f"hd/blk == {self.hd // self.blk} is odd: two-per-word scale packing would straddle a head"
        if self.blk != 32:
            return f"block size {self.blk} is not ggml's QK8_0 = 32"
        return ""

    @property
    def nblk_head(self):
        return self.hd // self.blk

    def words(self, q8):
        """(data words, scale words) per slot per layer of one tensor."""
        if q8:
            return self.nkv * self.hd // 4, self.nkv * self.nblk_head // 2
        return self.nkv * self.hd // 2, 0

    @property
    def w_k(self):
        return sum(self.words(self.k_q8))

    @property
    def w_vd(self):
        return self.words(self.v_q8)[0]

    @property
    def w_vs(self):
        return self.words(self.v_q8)[1]

    @property
    def w_layer(self):
        return self.w_k + self.w_vd + self.w_vs

    @property
    def bytes_slot(self):
        return self.w_layer * 4 * self.n_attn


class KvCache:
    """Device KV cache of n_layers attention layers (contiguous or paged) plus a decode workspace."""

    def __init__(self, n_layers=8, nh=16, nkv=4, hd=256, cap=4096, k_fmt=BKV_Q8_0, v_fmt=BKV_Q8_0,
                 page_tokens=0, max_pages=0, block_table=None, scale=None, device="cuda",
                 max_ctx=None):
        self.n_layers, self.nh, self.nkv, self.hd, self.cap = n_layers, nh, nkv, hd, cap
        self.k_fmt, self.v_fmt = k_fmt, v_fmt
        self.page_tokens, self.max_pages = page_tokens, max_pages
        self.device = torch.device(device)
        self.scale = float(scale if scale is not None else 1.0 / (hd ** 0.5))
        geom = KvGeom(nkv=nkv, hd=hd, n_attn=n_layers, v_q8=int(v_fmt == BKV_Q8_0),
                      k_q8=int(k_fmt == BKV_Q8_0))
        why = geom.check()
        if why:
            raise ValueError(why)
        self.geom = geom

        def alloc(fmt, scales):
            if scales and fmt != BKV_Q8_0:
                return None
            if scales:
                row = nkv * (hd // 32) * 2
            else:
                row = nkv * hd * (2 if fmt == BKV_F16 else 1)
            return torch.zeros((n_layers, cap, row), dtype=torch.uint8, device=self.device)

        self.k_data = alloc(k_fmt, False)
        self.k_scales = alloc(k_fmt, True)
        self.v_data = alloc(v_fmt, False)
        self.v_scales = alloc(v_fmt, True)
        if page_tokens:
            if block_table is None:
                raise ValueError("paged cache needs a block table [n_layers][max_pages]")
            self.block_table = torch.as_tensor(block_table, dtype=torch.int32).to(self.device).contiguous()
            assert tuple(self.block_table.shape) == (n_layers, max_pages)
        else:
            self.block_table = None

        d = BkvCacheDesc()
        d.n_layers, d.nh, d.nkv, d.hd, d.cap = n_layers, nh, nkv, hd, cap
        d.k_fmt, d.v_fmt, d.page_tokens, d.max_pages = k_fmt, v_fmt, page_tokens, max_pages
        d.scale = self.scale
        arrs = [self.k_data, self.k_scales, self.v_data, self.v_scales]
        for i, a in enumerate(arrs):
            if a is not None:
                setattr(d, ("k_data", "k_scales", "v_data", "v_scales")[i], a.data_ptr())
                d.layer_stride_bytes[i] = a.stride(0)
        d.block_table = self.block_table.data_ptr() if self.block_table is not None else None
        self.desc = d
        check(lib().bkv_geom_check(ctypes.byref(d)), "bkv_geom_check")
        self.max_positions = lib().bkv_max_positions(ctypes.byref(d))
        self.max_ctx = max_ctx or self.max_positions
        ws = lib().bkv_workspace_bytes(ctypes.byref(d), BKV_OP_DECODE, self.max_ctx)
        self.workspace = torch.empty(ws, dtype=torch.uint8, device=self.device)
        check(lib().bkv_workspace_init(ctypes.byref(d), self.workspace.data_ptr(), ws, self._stream()),
              "bkv_workspace_init")

    # ---------------------------------------------------------------- helpers
    @staticmethod
    def _ptr(t):
        return None if t is None else t.data_ptr()

    def _f32(self, t, shape):
        t = torch.as_tensor(t, dtype=torch.float32, device=self.device).contiguous()
        assert tuple(t.shape) == tuple(shape), (tuple(t.shape), shape)
        return t

    @staticmethod
    def _stream():
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    # ---------------------------------------------------------------- the path
    def append(self, layer, pos, k, v):
        """kv_append: k, v [n_tok][nkv][hd] fp32 (post-RoPE K, raw V) at positions pos.."""
        n = k.shape[0]
        k = self._f32(k, (n, self.nkv, self.hd))
        v = self._f32(v, (n, self.nkv, self.hd))
        check(lib().bkv_kv_append(ctypes.byref(self.desc), layer, pos, n, k.data_ptr(),
                                  v.data_ptr(), self._stream()), "bkv_kv_append")

    def decode(self, layer, nfill, q, gate=None, out=None, out_gated=None):
        q = self._f32(q, (self.nh, self.hd))
        out = torch.empty((self.nh, self.hd), dtype=torch.float32, device=self.device) if out is None else out
        if gate is not None:
            gate = self._f32(gate, (self.nh, self.hd))
            if out_gated is None:
                out_gated = torch.empty_like(out)
        check(lib().bkv_attn_decode(ctypes.byref(self.desc), layer, nfill, q.data_ptr(),
                                    self._ptr(gate), out.data_ptr(), self._ptr(out_gated),
                                    self.workspace.data_ptr(), self.workspace.numel(),
                                    self._stream()), "bkv_attn_decode")
        return out, out_gated

    def decode_step(self, layer, pos, k, v, q, gate=None, out=None, out_gated=None):
        k = self._f32(k, (1, self.nkv, self.hd))
        v = self._f32(v, (1, self.nkv, self.hd))
        q = self._f32(q, (self.nh, self.hd))
        out = torch.empty((self.nh, self.hd), dtype=torch.float32, device=self.device) if out is None else out
        if gate is not None:
            gate = self._f32(gate, (self.nh, self.hd))
            if out_gated is None:
                out_gated = torch.empty_like(out)
        check(lib().bkv_decode_step(ctypes.byref(self.desc), layer, pos, k.data_ptr(), v.data_ptr(),
                                    q.data_ptr(), self._ptr(gate), out.data_ptr(),
                                    self._ptr(out_gated), self.workspace.data_ptr(),
                                    self.workspace.numel(), self._stream()), "bkv_decode_step")
        return out, out_gated

    def prefill_chunk(self, layer, pos0, q, gate=None):
        n = q.shape[0]
        q = self._f32(q, (n, self.nh, self.hd))
        out = torch.empty((n, self.nh, self.hd), dtype=torch.float32, device=self.device)
        out_gated = None
        if gate is not None:
            gate = self._f32(gate, (n, self.nh, self.hd))
            out_gated = torch.empty_like(out)
        ws = self.prefill_workspace(pos0 + n)
        check(lib().bkv_attn_prefill_chunk(ctypes.byref(self.desc), layer, pos0, n, q.data_ptr(),
                                           self._ptr(gate), out.data_ptr(), self._ptr(out_gated),
                                           ws.data_ptr(), ws.numel(), self._stream()),
              "bkv_attn_prefill_chunk")
        return out, out_gated

    def norm_rope_append(self, layer, pos0, q_in, k_in, v_in, qn_w, kn_w, nrot=64, eps=1e-6,
                         freq_base=1e7):
        """bkv_qk_norm_rope_append: K normed + roped and V appended at pos0..; returns the roped Q."""
        n = q_in.shape[0]
        q_in = self._f32(q_in, (n, self.nh, self.hd))
        k_in = self._f32(k_in, (n, self.nkv, self.hd))
        v_in = self._f32(v_in, (n, self.nkv, self.hd))
        qn_w = self._f32(qn_w, (self.hd,))
        kn_w = self._f32(kn_w, (self.hd,))
        q_out = torch.empty_like(q_in)
        check(lib().bkv_qk_norm_rope_append(ctypes.byref(self.desc), layer, pos0, n, q_in.data_ptr(),
                                            k_in.data_ptr(), v_in.data_ptr(), qn_w.data_ptr(),
                                            kn_w.data_ptr(), nrot, eps, freq_base, q_out.data_ptr(),
                                            self._stream()), "bkv_qk_norm_rope_append")
        return q_out

    def prefill_step(self, layer, pos0, k, v, q, gate=None):
        """bkv_prefill_step: append the chunk's K/V (q8_0 / fp16 on write), then its causal attention."""
        n = q.shape[0]
        k = self._f32(k, (n, self.nkv, self.hd))
        v = self._f32(v, (n, self.nkv, self.hd))
        q = self._f32(q, (n, self.nh, self.hd))
        out = torch.empty((n, self.nh, self.hd), dtype=torch.float32, device=self.device)
        out_gated = None
        if gate is not None:
            gate = self._f32(gate, (n, self.nh, self.hd))
            out_gated = torch.empty_like(out)
        ws = self.prefill_workspace(pos0 + n)
        check(lib().bkv_prefill_step(ctypes.byref(self.desc), layer, pos0, n, k.data_ptr(), v.data_ptr(),
                                     q.data_ptr(), self._ptr(gate), out.data_ptr(), self._ptr(out_gated),
                                     ws.data_ptr(), ws.numel(), self._stream()), "bkv_prefill_step")
        return out, out_gated

    def prefill_workspace(self, max_ctx):
        need = lib().bkv_workspace_bytes(ctypes.byref(self.desc), BKV_OP_PREFILL, max_ctx)
        if getattr(self, "_pws", None) is None or self._pws.numel() < need:
            self._pws = torch.empty(need, dtype=torch.uint8, device=self.device)
            check(lib().bkv_workspace_init(ctypes.byref(self.desc), self._pws.data_ptr(), need,
                                           self._stream()), "bkv_workspace_init")
        return self._pws

    def decode_window(self, layer, kstart, nfill, q, gate=None):
        """bkv_attn_decode_window: attention over keys [kstart, nfill) (an evicted prefix)."""
        q = self._f32(q, (self.nh, self.hd))
        out = torch.empty((self.nh, self.hd), dtype=torch.float32, device=self.device)
        og = None
        if gate is not None:
            gate = self._f32(gate, (self.nh, self.hd))
            og = torch.empty_like(out)
        check(lib().bkv_attn_decode_window(ctypes.byref(self.desc), layer, kstart, nfill, q.data_ptr(),
                                           self._ptr(gate), out.data_ptr(), self._ptr(og),
                                           self.workspace.data_ptr(), self.workspace.numel(),
                                           self._stream()), "bkv_attn_decode_window")
        return out, og

    def decode_qg(self, layer, nfill, qg, gated=True):
        """bkv_attn_decode_qg: q and gate from the interleaved attn_q output [nh][2*hd]."""
        qg = self._f32(qg, (self.nh, 2 * self.hd))
        out = torch.empty((self.nh, self.hd), dtype=torch.float32, device=self.device)
        og = torch.empty_like(out) if gated else None
        check(lib().bkv_attn_decode_qg(ctypes.byref(self.desc), layer, nfill, qg.data_ptr(), out.data_ptr(),
                                       self._ptr(og), self.workspace.data_ptr(), self.workspace.numel(),
                                       self._stream()), "bkv_attn_decode_qg")
        return out, og

    def decode_step_qg(self, layer, pos, k, v, qg, gated=True):
        """bkv_decode_step_qg: append the token, then attention with the interleaved q/gate rows."""
        k = self._f32(k, (1, self.nkv, self.hd))
        v = self._f32(v, (1, self.nkv, self.hd))
        qg = self._f32(qg, (self.nh, 2 * self.hd))
        out = torch.empty((self.nh, self.hd), dtype=torch.float32, device=self.device)
        og = torch.empty_like(out) if gated else None
        check(lib().bkv_decode_step_qg(ctypes.byref(self.desc), layer, pos, k.data_ptr(), v.data_ptr(),
                                       qg.data_ptr(), out.data_ptr(), self._ptr(og),
                                       self.workspace.data_ptr(), self.workspace.numel(), self._stream()),
              "bkv_decode_step_qg")
        return out, og

    def prefill_chunk_qg(self, layer, pos0, qg, gated=True):
        """bkv_attn_prefill_chunk_qg: qg [n][nh][2*hd]."""
        n = qg.shape[0]
        qg = self._f32(qg, (n, self.nh, 2 * self.hd))
        out = torch.empty((n, self.nh, self.hd), dtype=torch.float32, device=self.device)
        og = torch.empty_like(out) if gated else None
        ws = self.prefill_workspace(pos0 + n)
        check(lib().bkv_attn_prefill_chunk_qg(ctypes.byref(self.desc), layer, pos0, n, qg.data_ptr(),
                                              out.data_ptr(), self._ptr(og), ws.data_ptr(), ws.numel(),
                                              self._stream()), "bkv_attn_prefill_chunk_qg")
        return out, og

    def fill_synthetic(self):
        """bkv_kv_fill_synthetic: every slot of every layer holds the word 0x3C003C00 (the reference's
        kv_fill_synthetic timing fixture, runtime_vk/bonsai_forward.h:1355-1370)."""
        check(lib().bkv_kv_fill_synthetic(ctypes.byref(self.desc), self._stream()), "bkv_kv_fill_synthetic")

    def decode_path(self, nfill):
        """3: stream single launch (the default for q8_0 K and V), 2: resident single launch, 0: split path"""
        return lib().bkv_decode_path(ctypes.byref(self.desc), nfill)

    def check_workspace(self):
        """bkv_workspace_error on the decode workspace (synchronises the stream): raises BkvError
        (BKV_ETIMEOUT) if a decode since the last check gave up waiting, and clears the flag."""
        check(lib().bkv_workspace_error(ctypes.byref(self.desc), self.workspace.data_ptr(),
                                        self.workspace.numel(), self._stream()), "bkv_workspace_error")

    def error_word_offset(self):
        """Byte offset of the single-launch kernels' error word in the workspace."""
        out = (ctypes.c_uint64 * 1)()
        check(lib().bkv_error_words(ctypes.byref(self.desc), out), "bkv_error_words")
        return int(out[0])

    # ---------------------------------------------------------------- inspection
    def debug_intermediates(self, nfill):
        """After a decode over nfill keys (stream-synchronised): scores [nh][nfill], e [nh][nfill],
        exact softmax sums [nh] and walker status [nh], read from the workspace."""
        out = (ctypes.c_uint64 * 6)()
        check(lib().bkv_debug_layout(ctypes.byref(self.desc), nfill, out), "bkv_debug_layout")
        ld, o_s, o_e, o_sum, o_st = (int(x) for x in out[:5])
        ws = self.workspace
        f = lambda off, n: ws[off:off + 4 * n].view(torch.float32)
        nh = self.nh
        score = f(o_s, nh * ld).view(nh, ld)[:, :nfill].cpu() if o_s else None
        e = f(o_e, nh * ld).view(nh, ld)[:, :nfill].cpu()
        ssum = f(o_sum, nh).cpu()
        status = ws[o_st:o_st + 4 * nh].view(torch.int32).cpu()
        return score, e, ssum, status

    
    def host_arrays(self):
        """The four sub-arenas as CPU uint8 tensors [n_layers][cap][row bytes] (None if absent)."""
        return [None if a is None else a.cpu() for a in
                (self.k_data, self.k_scales, self.v_data, self.v_scales)]
