"""Per-phase clocks of the resident decode kernel (one launch per layer), for finding where a
layer's time goes. Needs the instrumented build:

    python -m bonsai_vk_amd.build --timestamps
    BKV_LIBRARY=bonsai_vk_amd/libbkv_ts.so python -m bonsai_vk_amd.phase_times [ctx] [--paged] [--b2b] [--f16k]

With BKV_EXPERIMENT_TS every workgroup's thread 0 writes the GPU wall clock (100 MHz) at each phase
boundary into the workspace at byte 131072 ([workgroup][16] u32). The probe runs six decode_steps
of one q8_0 layer at ctx keys (256-token pages with --paged; fp16 K with --f16k), and prints min / median / max over
the workgroups of the last call, in microseconds from the first workgroup's start.
"""
import os
import sys

import numpy as np
import torch

from bonsai_vk_amd import BKV_Q8_0, KvCache

# slot -> phase, in launch order, of the default kernel (stream_kernel; thread 0's clocks)
PHASES_STREAM = [(0, "start"), (14, "K tile landed (wave 0)"), (1, "scores done (wave 0)"),
                 (9, "stats stored"), (2, "barrier A passed"), (3, "e pass done"),
                 (13, "spec PV done (wave 0)"), (4, "barrier B passed"), (5, "walk done"),
                 (12, "p16 done"), (15, "corrections done"), (10, "PV rows reduced"),
                 (6, "partials stored"), (7, "merge polled"), (8, "end")]
# the same for resident_kernel (BKV_DECODE=resident; slot 15 is wave 7's end of PV)
PHASES = [(0, "start"), (1, "scores done (wave 0)"), (2, "barrier A passed"), (10, "e main pass"),
          (11, "e tail + p16'"), (3, "records stored"), (4, "barrier B passed"), (5, "walk done"),
          (12, "p16 done"), (13, "PV done (wave 0)"), (15, "PV done (wave 7)"), (14, "PV rows reduced"),
          (6, "partials stored"), (7, "merge polled"), (8, "end")]
TS_WORD = 131072 // 4


def probe(ctx=32768, paged=False, calls=6, b2b=False, k_fmt=BKV_Q8_0):
    """Timestamps [workgroups][16] (raw 100 MHz clocks) of the last of `calls` decode_steps; b2b:
    the calls run back to back as in the bench (one synchronisation at the end), otherwise each
    call starts on an idle GPU."""
    if paged:
        npg = (ctx + calls + 255) // 256
        bt = np.random.default_rng(3).permutation(npg).astype(np.int32)[None]
        cache = KvCache(n_layers=1, cap=npg * 256, k_fmt=k_fmt, v_fmt=BKV_Q8_0, max_ctx=ctx + calls,
                        page_tokens=256, max_pages=npg, block_table=bt)
    else:
        cache = KvCache(n_layers=1, cap=ctx + calls, k_fmt=k_fmt, v_fmt=BKV_Q8_0, max_ctx=ctx + calls)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    for s in range(0, ctx, 8192):
        e = min(ctx, s + 8192)
        cache.append(0, s, torch.randn(e - s, 4, 256, generator=g, device="cuda"),
                     torch.randn(e - s, 4, 256, generator=g, device="cuda") * 0.5)
    k = torch.randn(1, 4, 256, device="cuda")
    v = torch.randn(1, 4, 256, device="cuda")
    q = torch.randn(16, 256, device="cuda")
    nwg = torch.cuda.get_device_properties(0).multi_processor_count
    ts = tw = None
    import ctypes
    from bonsai_vk_amd._lib import lib
    for i in range(calls):
        cache.decode_step(0, ctx + i, k, v, q)
        if b2b and i < calls - 1:
            continue
        torch.cuda.synchronize()
        ts = cache.workspace.view(torch.int32)[TS_WORD:TS_WORD + nwg * 16].cpu().numpy()
        out = (ctypes.c_uint64 * 6)()
        lib().bkv_debug_layout(ctypes.byref(cache.desc), ctx + i + 1, out)
        o = (int(out[5]) - 262144) // 4
        tw = cache.workspace.view(torch.int32)[o:o + nwg * 128].cpu().numpy()
    ts = ts.astype(np.int64).reshape(nwg, 16)
    probe.per_wave = tw.astype(np.int64).reshape(nwg, 8, 16)[ts[:, 0] != 0]
    if not ts[:, 8].any():
        raise RuntimeError("no timestamps written: load the instrumented build "
                           "(BKV_LIBRARY=bonsai_vk_amd/libbkv_ts.so after build --timestamps)")
    return ts[ts[:, 0] != 0]


def main(argv):
    ctx = int(next((a for a in argv if not a.startswith("-")), 32768))
    from bonsai_vk_amd import BKV_F16
    ts = probe(ctx, "--paged" in argv, b2b="--b2b" in argv, k_fmt=BKV_F16 if "--f16k" in argv else BKV_Q8_0)
    phases = PHASES if os.environ.get("BKV_DECODE") == "resident" else PHASES_STREAM
    t0 = ts[:, 0].min()
    print(f"ctx {ctx}{' paged' if '--paged' in argv else ''}{' back to back' if '--b2b' in argv else ''}: phase clocks in us from the first "
          f"workgroup's start, min / median / max over {len(ts)} workgroups")
    for slot, name in phases:
        col = (ts[:, slot] - t0) / 100.0
        print(f"  {name:22s} {col.min():8.2f} {np.median(col):8.2f} {col.max():8.2f}")
    pw = getattr(probe, "per_wave", None)
    if phases is PHASES_STREAM and pw is not None and pw.any():
        names = ["K tile landed", "tile scored", "tail scored", "max barrier passed", "spec PV done"]
        print("  per wave (median over workgroups): " + ", ".join(names))
        for wv in range(8):
            cells = []
            for j in range(len(names)):
                col = pw[:, wv, j]
                cells.append(f"{(np.median(col) - t0) / 100.0:7.2f}" if col.any() else "      -")
            # slots 5 (wall) and 6 / 7 (shader cycles): the clock rate over the scoring phase
            dw = (pw[:, wv, 2] - pw[:, wv, 5]).astype(np.float64)
            dc = ((pw[:, wv, 7] - pw[:, wv, 6]) & 0xFFFFFFFF).astype(np.float64)
            ok = dw > 0
            ghz = f"   score clock {np.median(dc[ok] / dw[ok]) / 10.0:5.2f} GHz over {np.median(dw[ok]) / 100.0:5.2f} us" if ok.any() else ""
            print(f"    wave {wv}: " + " ".join(cells) + ghz)
        print("  the PV (median): start, first round of 32 keys done, partial formed")
        for wv in range(8):
            cells = [f"{(np.median(pw[:, wv, j]) - t0) / 100.0:7.2f}" if pw[:, wv, j].any() else "      -" for j in (13, 14, 15)]
            print(f"    wave {wv}: " + " ".join(cells))
        print("  the walk (waves 0-3, median): records scanned, specials loaded, segments checked, "
              "chain done; specials walked")
        for wv in range(4):
            cells = [f"{(np.median(pw[:, wv, 8 + j]) - t0) / 100.0:7.2f}" for j in range(4)]
            print(f"    wave {wv}: " + " ".join(cells) + f"   {int(np.median(pw[:, wv, 12]))}")


if __name__ == "__main__":
    main(sys.argv[1:])
