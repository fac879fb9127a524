"""ctypes binding of libbkv.so (include/bkv.h). Loading fails loudly when the library is missing:
there is no CPU fallback behind this package."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# BKV_LIBRARY points the binding at another build of the same sources (e.g. one compiled with
# per-phase timestamps for profiling); the default is the in-tree libbkv.so
LIB_PATH = os.environ.get("BKV_LIBRARY") or os.path.join(HERE, "libbkv.so")

BKV_F16, BKV_Q8_0 = 0, 1
BKV_OP_DECODE, BKV_OP_PREFILL = 0, 1
BKV_PREFILL_MAX_Q = 4096

ERRORS = {
    0: "BKV_OK", -1: "BKV_EINVAL", -2: "BKV_ESHAPE", -3: "BKV_ECAP", -4: "BKV_EALIGN",
    -5: "BKV_EWORKSPACE", -6: "BKV_EHIP", -7: "BKV_EUNSUPPORTED", -8: "BKV_ETIMEOUT", -9: "BKV_ESCRATCH",
}

# every symbol include/bkv.h declares
EXPORTS = [
    "bkv_geom_check", "bkv_slot_bytes", "bkv_max_positions", "bkv_kv_append", "bkv_attn_decode",
    "bkv_decode_step", "bkv_attn_prefill_chunk", "bkv_workspace_bytes", "bkv_strerror",
    "bkv_last_hip_error", "bkv_version", "bkv_debug_layout", "bkv_workspace_init", "bkv_decode_path",
    "bkv_kv_fill_synthetic", "bkv_attn_decode_qg", "bkv_decode_step_qg", "bkv_attn_prefill_chunk_qg", "bkv_prefill_step", "bkv_qk_norm_rope_append", "bkv_attn_decode_window",
    "bkv_workspace_error", "bkv_error_words", "bkv_decode_step_static", "bkv_static_scratch_bytes",
    "bkv_static_error", "bkv_static_reset", "bkv_static_debug_address",
]


class BkvCacheDesc(ctypes.Structure):
    """Mirror of struct bkv_cache_desc."""
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


class BkvError(RuntimeError):
    def __init__(self, code, where=""):
        self.code = code
        name = ERRORS.get(code, str(code))
        msg = f"{where}: {name} ({lib().bkv_strerror(code).decode()})"
        if code == -6:
            msg += " " + lib().bkv_last_hip_error().decode()
        super().__init__(msg)


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built: run bonsai_vk_amd.build.build() "
                          "(there is no CPU fallback for the KV-cache path)")
    L = ctypes.CDLL(LIB_PATH)
    P, D, i32, u32, sz = ctypes.c_void_p, ctypes.POINTER(BkvCacheDesc), ctypes.c_int, ctypes.c_uint32, ctypes.c_size_t
    sig = {
        "bkv_geom_check": (i32, [D]),
        "bkv_slot_bytes": (ctypes.c_uint64, [D, i32]),
        "bkv_max_positions": (ctypes.c_int64, [D]),
        "bkv_kv_append": (i32, [D, i32, u32, i32, P, P, P]),
        "bkv_attn_decode": (i32, [D, i32, u32, P, P, P, P, P, sz, P]),
        "bkv_decode_step": (i32, [D, i32, u32, P, P, P, P, P, P, P, sz, P]),
        "bkv_attn_prefill_chunk": (i32, [D, i32, u32, i32, P, P, P, P, P, sz, P]),
        "bkv_workspace_bytes": (sz, [D, i32, u32]),
        "bkv_strerror": (ctypes.c_char_p, [i32]),
        "bkv_last_hip_error": (ctypes.c_char_p, []),
        "bkv_version": (ctypes.c_char_p, []),
        "bkv_debug_layout": (i32, [D, u32, ctypes.POINTER(ctypes.c_uint64)]),
        "bkv_workspace_init": (i32, [D, P, sz, P]),
        "bkv_decode_path": (i32, [D, u32]),
        "bkv_kv_fill_synthetic": (i32, [D, P]),
        "bkv_attn_decode_qg": (i32, [D, i32, u32, P, P, P, P, sz, P]),
        "bkv_decode_step_qg": (i32, [D, i32, u32, P, P, P, P, P, P, sz, P]),
        "bkv_attn_prefill_chunk_qg": (i32, [D, i32, u32, i32, P, P, P, P, sz, P]),
        "bkv_prefill_step": (i32, [D, i32, u32, i32, P, P, P, P, P, P, P, sz, P]),
        "bkv_attn_decode_window": (i32, [D, i32, u32, u32, P, P, P, P, P, sz, P]),
        "bkv_workspace_error": (i32, [D, P, sz, P]),
        "bkv_error_words": (i32, [D, ctypes.POINTER(ctypes.c_uint64)]),
        "bkv_decode_step_static": (i32, [D, i32, u32, P, P, P, P, P, P, P]),
        "bkv_static_scratch_bytes": (sz, []),
        "bkv_static_error": (i32, [D, P]),
        "bkv_static_reset": (i32, [P]),
        "bkv_static_debug_address": (i32, [ctypes.POINTER(ctypes.c_void_p)]),
        "bkv_qk_norm_rope_append": (i32, [D, i32, u32, i32, P, P, P, P, P, i32, ctypes.c_float,
                                          ctypes.c_float, P, P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype, f.argtypes = res, args
    _lib = L
    return L


def check(rc, where):
    if rc != 0:
        raise BkvError(rc, where)
