"""Build libbkv.so (the gfx950 KV-cache path) in-tree with hipcc.

    python -m bonsai_vk_amd.build               # or bonsai_vk_amd.build.build()
    python -m bonsai_vk_amd.build --timestamps  # libbkv_ts.so: the decode kernel records per-phase
                                                # clocks (read by bonsai_vk_amd.phase_times)
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libbkv.so")
LIB_TS = os.path.join(HERE, "libbkv_ts.so")
SOURCES = ["bkv_api.cpp", "bkv_decode.hip", "bkv_resident.hip", "bkv_stream.hip", "bkv_prefill.hip", "bkv_norm_rope.hip", "bkv_static.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
    # packed fp32 ops stay off: the gfx950 pool has shown silent wrong results from some v_pk_*_f32 forms
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # correctly rounded fp32 divide/sqrt: the q8_0 scale d = amax/127 and id = 1/d must round exactly
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math", "-ffp-contract=off",
    "-Wall", "-Wno-unused-function",
]


def build(verbose=False, jobs=None, timestamps=False):
    """Compile every source to an object in parallel (under bonsai_vk_amd/_build), then link.
    timestamps: the instrumented library libbkv_ts.so instead (objects under _build_ts)."""
    from concurrent.futures import ThreadPoolExecutor
    obj_dir = os.path.join(HERE, "_build_ts" if timestamps else "_build")
    out = LIB_TS if timestamps else LIB
    os.makedirs(obj_dir, exist_ok=True)
    cflags = [f for f in FLAGS if f != "-shared"] + (["-DBKV_EXPERIMENT_TS"] if timestamps else [])

    def compile_one(src):
        obj = os.path.join(obj_dir, src + ".o")
        cmd = [HIPCC] + cflags + ["-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        return obj, r

    n = jobs or min(len(SOURCES), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(n) as ex:
        results = list(ex.map(compile_one, SOURCES))
    for obj, r in results:
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed compiling {os.path.basename(obj)}")
    cmd = [HIPCC, "--offload-arch=gfx950", "-fPIC", "-shared", "-o", out + ".tmp"] + [o for o, _ in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"hipcc failed linking {os.path.basename(out)}")
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, timestamps="--timestamps" in sys.argv[1:]))
