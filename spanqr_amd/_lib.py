"""ctypes binding of libspanqr.so, the MI355X C ABI declared in include/spanqr.h, and its in-tree build.

The library is built ahead of time with hipcc for gfx950 (no runtime compilation). If it is missing, every entry
point raises: there is no CPU or PyTorch fallback for the hot path.
"""
import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libspanqr.so")
SRC = os.path.join(_HERE, "csrc", "spanqr.hip")
INCLUDE = os.path.join(os.path.dirname(_HERE), "include", "spanqr.h")

# hipcc flags: gfx950 only; packed fp32 VALU ops disabled (the kernels never rely on them); no fast-math so every
# fp32 operation keeps IEEE rounding and subnormals.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

# plan queries (include/spanqr.h)
(Q_K, Q_R, Q_SPLITS, Q_SPLIT_ROWS, Q_CHOL_GRID, Q_WORKSPACE_MB, Q_DEVICE, Q_BATCH, Q_CHOL_BATCH, Q_BLOCKS,
 Q_SOLVE_ROWS, Q_BLOCK_WIDTH, Q_NORM_PARTIALS) = range(13)
MAX_BATCH = 32   # SPANQR_MAX_BATCH
MAX_R = 4096     # SPANQR_MAX_R
# kernels for spanqr_profile_kernel
(K_AMAX, K_GRAM_PASS1, K_GRAM, K_REDUCE, K_CHOL, K_TRSM_PASS1, K_TRSM, K_NS_APPLY, K_CHOL_SOLVE_PASS1,
 K_CHOL_SOLVE) = range(10)

# every exported symbol of include/spanqr.h: (restype, argtypes)
_P, _I, _L, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float
SIGNATURES = {
    "spanqr_plan_create": (_I, [_I, _I, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "spanqr_plan_create_batched": (_I, [_I, _I, _I, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "spanqr_plan_create_borth": (_I, [_I, _I, _I, _I, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "spanqr_plan_destroy": (None, [_P]),
    "spanqr_plan_query": (_L, [_P, _I]),
    "spanqr_orth_f32": (_I, [_P, _P, _L, _P, _L, _F, _F, _F, _I, _P]),
    "spanqr_orth_batched_f32": (_I, [_P, _I, _P, _L, _P, _L, _F, _F, _F, _I, _P]),
    "spanqr_orth_f32_noalloc": (_I, [_I, _I, _P, _L, _P, _L, _F, _F, _F, _I, _P]),
    "spanqr_profile_orth": (_I, [_P, _P, _L, _P, _L, _F, _F, _F, _I, _P, _P, _I, ctypes.POINTER(ctypes.c_int)]),
    "spanqr_profile_chol": (_I, [_P, _P, _P, _F, _F, _P, ctypes.POINTER(ctypes.c_double), _P]),
    "spanqr_profile_kernel": (_I, [_P, _I, _I, ctypes.POINTER(ctypes.c_float), _P]),
    "spanqr_last_error": (ctypes.c_char_p, []),
    "spanqr_dust_host": (_I, [_I, _I, _P]),
    "spanqr_split_rows": (_I, [_I, _I]),
    "spanqr_norm_partials": (_I, [_I, _I]),
    "spanqr_stage_amax": (_I, [_P, _P, _L, _P]),
    "spanqr_stage_gram": (_I, [_P, _P, _L, _I, _I, _P, _P, _P]),
    "spanqr_stage_chol": (_I, [_P, _P, _P, _F, _F, _P, _P, _P, _P]),
    "spanqr_stage_trsm": (_I, [_P, _P, _L, _I, _F, _P, _P, _P, _L, _P]),
    "spanqr_stage_ns": (_I, [_P, _P, _L, _I, _P, _L, _P]),
    "spanqr_plan_copy_dust": (_I, [_P, _P, _P]),
    "spanqr_plan_copy_scalars": (_I, [_P, _P, _P]),
    "spanqr_plan_status": (_I, [_P, _P]),
    "spanqr_chol32": (_I, [_P, _P, _L, _P, _P, _L, _P, _P]),
    "spanqr_debug_spin_limit": (_I, [ctypes.c_uint]),
    "spanqr_chol64_plan_create": (_I, [_I, _I, ctypes.POINTER(ctypes.c_void_p)]),
    "spanqr_chol64_plan_destroy": (None, [_P]),
    "spanqr_chol64": (_I, [_P, _P, _L, _P, _P, _P, _P, _P, _P]),
    "spanqr_chol64_status": (_I, [_P, _P]),
}

_lib = None


class SpanqrError(RuntimeError):
    """a C ABI call returned an error (message from spanqr_last_error)"""


def build(verbose=False):
    """compile libspanqr.so in place (hipcc cross-compiles gfx950 without a GPU)"""
    cmd = ["hipcc", *HIPCC_FLAGS, "-o", LIB_PATH, SRC]
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    return LIB_PATH


def lib():
    """the loaded library (raises if it has not been built)"""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing; build it with spanqr_amd._lib.build() "
                              "(or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc):
    if rc != 0:
        raise SpanqrError(lib().spanqr_last_error().decode(errors="replace") or f"spanqr error {rc}")


def exported_symbols_in_header():
    """names of the functions declared in include/spanqr.h"""
    import re
    with open(INCLUDE) as f:
        text = f.read()
    return sorted(set(re.findall(r"\b(spanqr_[a-z0-9_]+)\s*\(", text)))
