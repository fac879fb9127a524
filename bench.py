"""bench.py - decode attention + KV append over a 32K q8_0 cache, 8 layers, on one MI355X.

One step = one decode token: for each of the 8 attention layers, bkv_decode_step appends the token's
K/V (q8_0 quantise-on-write) and runs GQA attention (16 Q / 4 KV heads, d 256) over the whole cache.
The cache is prefilled with seeded synthetic K/V (K ~ N(0,1) with 3 channels per (layer, kv head)
scaled x8, V ~ N(0, 0.5) std, Q ~ N(0,1)) so that the timed steps attend over 32769..32768+K keys
Inputs are resident in HBM before the timed region.

A second object on the same line, "prefill", times BASELINE config 5: 512 new q8_0 tokens appended
onto an 8192-token cache, then causal GQA attention for the 512 queries over 8 layers
(bkv_attn_prefill_chunk), on the exact path (the default) and on the MFMA-order variant.
A third, "other_configs", gives us/token and roofline fractions of BASELINE configs 2 (8 layers at
4096 keys) and 4 (65536 keys, 256-token pages of a 320-page pool, f16 and q8_0), and of config 3's
shape with fp16 K + q8_0 V and with the gate read and the gated output written.

    python bench.py [--steps 48] [--warmup 4] [--ctx 32768] [--no-cpu] [--no-prefill] [--no-configs]
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def algorithmic_bytes(n, gated=False):
    """Compulsory HBM bytes of one layer's decode step over n keys (q8_0 K+V, d 256, 4 KV heads):
    K/V read 2176 B/key, append write 2176 B, K/V fp32 input 8192 B, Q 16384 B, out 16384 B
    (+ gate read and gated write 32768 B)."""
    return 2176 * n + 43136 + (32768 if gated else 0)


def algorithmic_bytes_f16(n):
    """As algorithmic_bytes for an f16 K+V cache: read 4096 B/key, append write 4096 B, K/V input
    8192 B, Q 16384 B, out 16384 B."""
    return 4096 * n + 45056


def algorithmic_bytes_f16k_q8v(n, gated=False):
    """As algorithmic_bytes for f16 K (2048 B/key) and q8_0 V (1088 B/key): read 3136 B/key, append
    write 3136 B, K/V input 8192 B, Q 16384 B, out 16384 B (+ gate 32768 B)."""
    return 3136 * n + 44096 + (32768 if gated else 0)


def time_decode(cache, layers, n0, steps, warmup, seed, gated=False):
    """Mean us/token of `steps` decode_steps x `layers` layers over keys n0 + 1 .. (after `warmup`
    untimed ones, which the caller counts into n0), with HIP events around the timed region.
    gated: each call also reads a gate and writes the gated output."""
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    tot = warmup + steps
    knew = torch.randn(tot, layers, 1, 4, 256, generator=g, device="cuda")
    vnew = torch.randn(tot, layers, 1, 4, 256, generator=g, device="cuda") * 0.5
    q = torch.randn(tot, layers, 16, 256, generator=g, device="cuda")
    gate = torch.randn(tot, layers, 16, 256, generator=g, device="cuda") if gated else None
    out = torch.empty(layers, 16, 256, device="cuda")
    og = torch.empty(layers, 16, 256, device="cuda") if gated else None
    base = n0 - warmup

    def step(i):
        for layer in range(layers):
            cache.decode_step(layer, base + i, knew[i, layer], vnew[i, layer], q[i, layer],
                              None if gate is None else gate[i, layer], out[layer],
                              None if og is None else og[layer])

    for i in range(warmup):
        step(i)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record()
    for i in range(steps):
        step(warmup + i)
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) * 1e3 / steps


def other_configs(steps=16, warmup=2):
    """BASELINE configs 2 (8 layers, 4096 keys, q8_0) and 4 (65536 keys in 256-token pages of a
    320-page pool, seeded permuted block tables, f16 and q8_0), us/token over `steps` decode steps
    (each appending one token per layer) and the fraction of the HBM roofline."""
    import numpy as np
    import torch
    from bonsai_vk_amd import BKV_F16, BKV_Q8_0, KvCache
    res = {}
    L = 8
    cache = KvCache(n_layers=L, cap=4096 + steps + warmup + 1, k_fmt=BKV_Q8_0, v_fmt=BKV_Q8_0)
    gen_cache(cache, 4096 - warmup, seed=1, layers=L)
    us = time_decode(cache, L, 4096, steps, warmup, seed=11)
    b = sum(L * algorithmic_bytes(4097 + i) for i in range(steps)) / steps
    res["config2_q8_4k"] = {"us_per_token": round(us, 2), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    del cache
    bt = np.stack([np.random.default_rng(3).permutation(320) for _ in range(L)]).astype(np.int32)
    for name, fmt, fb in (("config4_paged_f16_64k", BKV_F16, algorithmic_bytes_f16),
                          ("config4_paged_q8_64k", BKV_Q8_0, algorithmic_bytes)):
        torch.cuda.empty_cache()
        cache = KvCache(n_layers=L, cap=320 * 256, k_fmt=fmt, v_fmt=fmt, page_tokens=256,
                        max_pages=320, block_table=bt)
        gen_cache(cache, 65536 - warmup, seed=3, layers=L)
        us = time_decode(cache, L, 65536, steps, warmup, seed=13)
        b = sum(L * fb(65537 + i) for i in range(steps)) / steps
        res[name] = {"us_per_token": round(us, 2), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        del cache
    # config 3's shape with fp16 K and q8_0 V, and with the gate (q8_0 K+V)
    for name, kf, fb, gated in (("config3_f16k_q8v_32k", BKV_F16, algorithmic_bytes_f16k_q8v, False),
                                ("config3_q8_32k_gated", BKV_Q8_0, algorithmic_bytes, True)):
        torch.cuda.empty_cache()
        cache = KvCache(n_layers=L, cap=32768 + steps + 1, k_fmt=kf, v_fmt=BKV_Q8_0)
        gen_cache(cache, 32768 - warmup, seed=2, layers=L)
        us = time_decode(cache, L, 32768, steps, warmup, seed=17, gated=gated)
        b = sum(L * fb(32769 + i, gated) for i in range(steps)) / steps
        res[name] = {"us_per_token": round(us, 2), "frac": round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                     "path": {3: "stream", 2: "resident", 0: "split"}[cache.decode_path(32769)]}
        del cache
    torch.cuda.empty_cache()
    return res


def gen_cache(cache, n, seed, layers):
    import torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    chunk = 8192
    for layer in range(layers):
        ch = torch.stack([torch.randperm(256, generator=g, device="cuda")[:3] for _ in range(4)])
        scale = torch.ones(4, 256, device="cuda")
        scale.scatter_(1, ch, 8.0)
        for s in range(0, n, chunk):
            e = min(n, s + chunk)
            k = torch.randn(e - s, 4, 256, generator=g, device="cuda") * scale
            v = torch.randn(e - s, 4, 256, generator=g, device="cuda") * 0.5
            cache.append(layer, s, k, v)
    torch.cuda.synchronize()


def kernel_name(cache, n):
    """The launch(es) one decode_step call makes at n keys."""
    return {3: "stream_kernel (one launch per layer, one workgroup per CU: append, QK, exact sum, PV, "
               "merge)",
            2: "resident_kernel (one launch per layer, one workgroup per CU: append, QK, exact sum, "
               "PV, merge)",
            0: "qk_kernel + e_kernel + pv_kernel + merge_kernel (four launches per layer)"}[cache.decode_path(n)]


# the sources whose code a decode launch runs: a traffic summary measured on other code is stale
TRAFFIC_SOURCES = ["bkv_stream.hip", "bkv_resident.hip", "bkv_res_shared.h", "bkv_device.h", "bkv_common.h",
                   "bkv_exp.h", "bkv_q8dot.h", "bkv_pv8.h", "bkv_internal.h"]


def kernel_sources_sha():
    """sha256 (first 16 hex digits) of the decode kernels' sources, as the traffic summaries
    record it"""
    import hashlib
    h = hashlib.sha256()
    for f in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, "bonsai_vk_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def launched_kernel(cache, n):
    """rocprof's name of the single-launch kernel a contiguous q8_0 K+V decode_step at n keys runs
    (None for the split path)"""
    path = cache.decode_path(n)
    if path == 3:
        # the library's plan: 64 workgroups per KV group (256 CUs, nkv 4), at least 128 keys each;
        # workgroups of at most 128 keys run the short instantiation
        wgs = min(64, -(-n // 128))
        short = -(-n // wgs) <= 128
        return f"void bkv::stream_kernel<1, false, {'true' if short else 'false'}>(bkv::ResArgs)"
    if path == 2:
        return "void bkv::resident_kernel<1, 1, true, false>(bkv::ResArgs)"
    return None


def measured_traffic(cache, n):
    """HBM bytes per launch of the single-launch kernel this workload takes, from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary (profiles/<kernel>_q8_32k_traffic.json); None when
    that summary is absent, names another kernel than the one this run launches, or was measured on
    other kernel sources (its source_sha differs from the tree's)."""
    name = {3: "stream_kernel", 2: "resident_kernel"}.get(cache.decode_path(n))
    if name is None:
        return None
    path = os.path.join(ROOT, "profiles", f"{name}_q8_32k_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        summary = json.load(f)
    if summary.get("kernel") != launched_kernel(cache, n) or summary.get("source_sha") != kernel_sources_sha():
        return None
    return summary.get("hbm_bytes_per_launch")


def check_no_timeout(cache, where):
    """A decode whose bounded wait gave up produced no valid output: stop with an error instead of
    reporting its time."""
    from bonsai_vk_amd import BkvError
    try:
        cache.check_workspace()
    except BkvError as e:
        print(f"bench.py: a decode call timed out ({where}): {e}", file=sys.stderr, flush=True)
        sys.exit(3)


def host_threads():
    """(threads this process may run on, the machine's logical CPU count)"""
    n = os.cpu_count() or 1
    aff = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else n
    return max(1, aff), n


def cpu_baseline(ctx, seed=2, budget_s=12.0):
    """The reference's own CPU path on the host cores: its compiled mirror (oracle/_ref
    ref_decode_rows: attn_vk.h:156-212 score / softmax / P16 / PV / gate per head row) over the 128
    (layer, head) rows of one decode token at ctx+1 keys, OpenMP over every core this process may
    use. The mirror's arenas are fp16 (the reference's CPU twin has no q8_0 path), one distinct arena
    per layer. Beside it: the same rows single-threaded (one row x 128) and this build's CPU oracle
    on the q8_0 cache (one layer x 8). Returns the baseline object."""
    import ctypes
    import numpy as np
    import oracle
    cores, nproc = host_threads()
    n = ctx + 1
    res = {"unit": "us/token", "cores": cores, "nproc": nproc}
    R = oracle.ref()
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    if R is not None:
        rng = np.random.default_rng(seed)
        L, words = 8, n * 4 * 128
        kc = np.empty((L, words), np.uint32)
        vc = np.empty((L, words), np.uint32)
        for l in range(L):
            kc[l] = rng.standard_normal(2 * words, np.float32).astype(np.float16).view(np.uint32)
            vc[l] = (rng.standard_normal(2 * words, np.float32) * 0.5).astype(np.float16).view(np.uint32)
        q16 = rng.standard_normal((L * 16, 256), np.float32).astype(np.float16).view(np.uint32).copy()
        gate = rng.standard_normal((L * 16, 256), np.float32)
        out = np.empty((L * 16, 256), np.float32)
        args = lambda layers, thr: (256, 16, 4, ctypes.c_float(0.0625), layers, P(q16), P(kc), P(vc), words, n,
                                    P(gate), P(out), thr)
        reps, t0 = 0, time.perf_counter()
        while reps < 1 or (time.perf_counter() - t0 < budget_s and reps < 100):
            R.ref_decode_rows(*args(L, cores))
            reps += 1
        per_token = (time.perf_counter() - t0) / reps
        t1 = time.perf_counter()
        R.ref_decode_rows(*args(1, 1))             # one layer's 16 rows on one thread
        single = (time.perf_counter() - t1) * 8
        res.update({"value": per_token * 1e6, "kind": "reference",
                    "sample": f"reference mirror (oracle/_ref ref_decode_rows) over 8 layers x 16 heads "
                              f"at {n} fp16 keys, {reps} tokens on {cores} threads",
                    "single_thread_us_per_token": single * 1e6})
        del kc, vc
    # this build's oracle on the q8_0 workload itself
    host = oracle.HostCache(n_layers=1, cap=n, k_fmt=oracle.Q8_0, v_fmt=oracle.Q8_0)
    k, v = oracle.synth_kv(n, 4, 256, seed, 0, outliers=3)
    host.append(0, 0, k, v)
    q = oracle.normal(16 * 256, seed, 5).reshape(16, 256)
    reps, t0 = 0, time.perf_counter()
    while reps < 1 or (time.perf_counter() - t0 < budget_s / 2 and reps < 100):
        host.decode(0, n, q, nthreads=cores)
        reps += 1
    per_layer = (time.perf_counter() - t0) / reps
    res["port_q8_us_per_token"] = per_layer * 8 * 1e6
    res["port_sample"] = f"CPU oracle decode of 1 layer (16 heads) at {n} q8_0 keys, {reps} reps, x8 layers"
    if "value" not in res:                     # the reference checkout was absent where oracle/_ref was built
        res.update({"value": res["port_q8_us_per_token"], "kind": "port", "sample": res["port_sample"]})
    return res




def prefill_flops(pos0, n_q, nh=16, hd=256):
    """QK^T + PV flops of one layer's causal chunk: 2*2*hd per (row, visible key)."""
    return 4 * hd * nh * sum(pos0 + i + 1 for i in range(n_q))


def prefill_leg(cpu=True, reps=5):
    """BASELINE config 5 on the GPU (exact path and the MFMA-order variant) and the CPU oracle on
    a bounded sample (a few query rows, scaled to the chunk)."""
    import torch
    from bonsai_vk_amd import BKV_Q8_0, KvCache
    pos0, n_q, L = 8192, 512, 8
    n = pos0 + n_q
    cache = KvCache(n_layers=L, cap=n, k_fmt=BKV_Q8_0, v_fmt=BKV_Q8_0)
    g = torch.Generator(device="cuda")
    g.manual_seed(4)
    for layer in range(L):
        k = torch.randn(n, 4, 256, generator=g, device="cuda")
        v = torch.randn(n, 4, 256, generator=g, device="cuda") * 0.5
        cache.append(layer, 0, k, v)
    q = torch.randn(L, n_q, 16, 256, generator=g, device="cuda")

    def run():
        for layer in range(L):
            cache.prefill_chunk(layer, pos0, q[layer])

    res = {}
    for mode in ("exact", "mfma"):
        if mode == "mfma":
            os.environ["BKV_PREFILL"] = "mfma"
        run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            run()
        e1.record()
        torch.cuda.synchronize()
        res[mode] = e0.elapsed_time(e1) / reps * 1e3   # us per 8-layer chunk
        os.environ.pop("BKV_PREFILL", None)
    fl = L * prefill_flops(pos0, n_q)
    # the exact path's score sweep on the int8 matrix cores: each (query, head) row is 4 base-256
    # digit rows of its fp16 value, so 4 x 2 x 256 int8 ops per (row, key), over the causal key range
    # pos0 + i + 1 of query i, 16 heads per query
    score_ops = L * 16 * sum(pos0 + i + 1 for i in range(n_q)) * 4 * 2 * 256
    out = {"workload": "bkv_attn_prefill_chunk x 8 layers: 512 q8_0 queries onto 8192 cached keys "
                       "(BASELINE config 5)",
           "unit": "us/chunk", "value": round(res["exact"], 1),
           "us_per_layer": round(res["exact"] / L, 1),
           "algorithmic_tflops": round(fl / (res["exact"] * 1e-6) / 1e12, 2),
           "bound": "vector ALUs (correctly rounded exp in fp64, serial sums, the p16 quotients, the "
                    "serial outer chain of each q8_0 score), with the scores' inner sums on the int8 "
                    "matrix cores",
           "score_int8_mfma_tops_over_chunk": round(score_ops / (res["exact"] * 1e-6) / 1e12, 1),
           "int8_mfma_peak_tops": 5000.0,
           "mfma_variant": {"value": round(res["mfma"], 1), "unit": "us/chunk",
                            "algorithmic_tflops": round(fl / (res["mfma"] * 1e-6) / 1e12, 1),
                            "peak_tflops": 2500.0,
                            "note": "scores and sums in MFMA order: not bit-identical probabilities"}}
    if cpu:
        import numpy as np
        import oracle
        cores = host_threads()[0]
        host = oracle.HostCache(n_layers=1, cap=n, k_fmt=oracle.Q8_0, v_fmt=oracle.Q8_0)
        kk, vv = oracle.synth_kv(n, 4, 256, 4, 0, outliers=0)
        host.append(0, 0, kk, vv)
        qh = oracle.normal(16 * 256, 4, 5).reshape(16, 256)
        rows = [0, 255, 511]
        t0 = time.perf_counter()
        for i in rows:
            host.decode(0, pos0 + i + 1, qh, nthreads=cores)
        per_row = (time.perf_counter() - t0) / len(rows)
        out["cpu_baseline"] = {"value": round(per_row * n_q * L * 1e6, 1), "unit": "us/chunk",
                               "cores": cores, "kind": "port",
                               "sample": f"oracle rows {rows} of one layer (16 heads each), x512 rows x8 layers"}
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=48)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the config-5 prefill leg")
    ap.add_argument("--no-configs", action="store_true", help="skip the config-2 and config-4 timings")
    ap.add_argument("--gate", action="store_true", help="also read the gate and write GOUT")
    ap.add_argument("--copy-calib", type=int, default=0, metavar="MIB",
                    help="after the timed region, copy a MIB MiB buffer once (a reference kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the KV path is sharded across GPUs by "
              "KV head or sequence in design only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from bonsai_vk_amd import BKV_Q8_0, KvCache

    L, K, W, ctx = args.layers, args.steps, args.warmup, args.ctx
    RP = 16                                 # roofline pass: steps after the timed region
    cap = ctx + K + RP + 1
    cache = KvCache(n_layers=L, cap=cap, k_fmt=BKV_Q8_0, v_fmt=BKV_Q8_0, max_ctx=cap)
    prefill = ctx - W                       # warmup appends positions ctx-W .. ctx-1
    gen_cache(cache, prefill, seed=2, layers=L)
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    nstep = W + K + RP
    knew = torch.randn(nstep, L, 1, 4, 256, generator=g, device="cuda")
    vnew = torch.randn(nstep, L, 1, 4, 256, generator=g, device="cuda") * 0.5
    q = torch.randn(nstep, L, 16, 256, generator=g, device="cuda")
    gate = torch.randn(nstep, L, 16, 256, generator=g, device="cuda") if args.gate else None
    out = torch.empty(L, 16, 256, device="cuda")
    og = torch.empty(L, 16, 256, device="cuda") if args.gate else None

    def step(i):
        pos = prefill + i
        for layer in range(L):
            cache.decode_step(layer, pos, knew[i, layer], vnew[i, layer], q[i, layer],
                              None if gate is None else gate[i, layer], out[layer],
                              None if og is None else og[layer])

    for i in range(W):
        step(i)
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for i in range(K):
        step(W + i)
    t_end.record()
    torch.cuda.synchronize()
    check_no_timeout(cache, "timed region")
    ms_total = t_start.elapsed_time(t_end)
    ms_step = ms_total / K
    ns = [ctx + 1 + i for i in range(K)]
    bytes_step = sum(L * algorithmic_bytes(n, args.gate) for n in ns) / K

    # roofline pass (not part of the timed region): HIP events on the launch stream at step
    # boundaries only, so the per-launch average carries no per-call event overhead
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(RP + 1)]
    evs[0].record()
    for i in range(RP):
        step(W + K + i)
        evs[i + 1].record()
    torch.cuda.synchronize()
    check_no_timeout(cache, "roofline pass")
    avg_call_s = sum(evs[i].elapsed_time(evs[i + 1]) for i in range(RP)) / RP / L / 1e3
    rp_bytes = sum(algorithmic_bytes(ctx + 1 + K + i, args.gate) for i in range(RP)) / RP
    achieved = rp_bytes / avg_call_s / 1e9

    if args.copy_calib:
        src = torch.empty(args.copy_calib << 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()

    line = {
        "metric": "us/token decode attn+KV append at 32K ctx (8 layers); achieved HBM GB/s % peak",
        "value": round(ms_step * 1e3, 3), "unit": "us/token", "n_gpus": 1, "steps": K,
        "warmup": W, "ms_per_step": round(ms_step, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded torch.randn K/V/Q, 3 outlier K channels x8 per layer/head)",
        "config": {"workload": "bkv_decode_step x 8 layers, q8_0 K+V, keys 32769..32768+steps "
                               "(BASELINE config 3)", "ctx": ctx, "layers": L, "nh": 16, "nkv": 4,
                   "kv_format": "q8_0 K+V (fp32 scores and accumulation, fp64 exact-sum bookkeeping)",
                   "hd": 256, "gate": bool(args.gate)},
        "achieved_gbs_step": round(bytes_step / (ms_step / 1e3) / 1e9, 1),
        "roofline": {"bound": "hbm", "kernel": kernel_name(cache, ns[0]),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(cache, ns[0]),
                     "algorithmic_bytes": round(rp_bytes),
                     "avg_call_us": round(avg_call_s * 1e6, 3)},
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(ctx)
    if not args.no_configs:
        del cache
        torch.cuda.empty_cache()
        cache = None
        line["other_configs"] = other_configs()
    if not args.no_prefill:
        del cache
        torch.cuda.empty_cache()
        line["prefill"] = prefill_leg(cpu=not args.no_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
