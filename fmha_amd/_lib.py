"""ctypes binding of libfmha_decode.so (declarations in include/fmha_decode.h).

The library must have been built (fmha_amd/_build.py); there is no fallback
implementation: a missing library is an error.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# FMHA_DECODE_LIB selects another build of the same sources (the
# host-sanitizer build of tests/test_sanitizers.py); by default the in-tree
# library that fmha_amd/_build.py writes.
LIB_PATH = os.environ.get("FMHA_DECODE_LIB") or os.path.join(_HERE, "libfmha_decode.so")

# Every symbol include/fmha_decode.h declares.
EXPORTED = (
    "fmha_decode_fwd",
    "fmha_decode_fwd_fast",
    "fmha_decode_fwd_fp32_weights",
    "fmha_decode_fwd_exact",
    "fmha_decode_fwd_uniform",
    "fmha_decode_fwd_uniform_fast",
    "fmha_decode_fwd_strided",
    "fmha_decode_fwd_paged",
    "fmha_decode_splitkv_workspace_size",
    "fmha_decode_fwd_splitkv",
    "fmha_decode_fwd_splitkv_noalloc",
    "fmha_decode_fwd_splitkv_strided",
    "fmha_decode_fwd_splitkv_paged",
    "fmha_decode_error_string",
    "fmha_decode_last_error_detail",
    "fmha_decode_last_plan",
    "fmha_decode_version",
)

_lib = None


def load():
    """Load the library once and declare its signatures."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = ctypes.CDLL(LIB_PATH)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
    lib.fmha_decode_fwd.restype = ctypes.c_int
    lib.fmha_decode_fwd.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_fast.restype = ctypes.c_int
    lib.fmha_decode_fwd_fast.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_fp32_weights.restype = ctypes.c_int
    lib.fmha_decode_fwd_fp32_weights.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_exact.restype = ctypes.c_int
    lib.fmha_decode_fwd_exact.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_uniform.restype = ctypes.c_int
    lib.fmha_decode_fwd_uniform.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_uniform_fast.restype = ctypes.c_int
    lib.fmha_decode_fwd_uniform_fast.argtypes = [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32]
    i64 = ctypes.c_int64
    lib.fmha_decode_fwd_strided.restype = ctypes.c_int
    lib.fmha_decode_fwd_strided.argtypes = [vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i32, i32, i32, i32, i32,
                                            i32, f32]
    lib.fmha_decode_fwd_paged.restype = ctypes.c_int
    lib.fmha_decode_fwd_paged.argtypes = [vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, i32, i32, f32]
    sz = ctypes.c_size_t
    lib.fmha_decode_splitkv_workspace_size.restype = sz
    lib.fmha_decode_splitkv_workspace_size.argtypes = [i32, i32, i32, i32, i32]
    lib.fmha_decode_fwd_splitkv.restype = ctypes.c_int
    lib.fmha_decode_fwd_splitkv.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32, vp, sz]
    lib.fmha_decode_fwd_splitkv_noalloc.restype = ctypes.c_int
    lib.fmha_decode_fwd_splitkv_noalloc.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, f32]
    lib.fmha_decode_fwd_splitkv_strided.restype = ctypes.c_int
    lib.fmha_decode_fwd_splitkv_strided.argtypes = [vp, vp, vp, vp, vp, vp, i32, i64, i64, i64, i32, i32, i32, i32,
                                                    i32, i32, f32, vp, sz]
    lib.fmha_decode_fwd_splitkv_paged.restype = ctypes.c_int
    lib.fmha_decode_fwd_splitkv_paged.argtypes = [vp, vp, vp, vp, vp, vp, i32, vp, i32, i32, i32, i32, i32, i32, i32,
                                                  i32, f32, vp, sz]
    lib.fmha_decode_error_string.restype = ctypes.c_char_p
    lib.fmha_decode_error_string.argtypes = [ctypes.c_int]
    lib.fmha_decode_last_error_detail.restype = ctypes.c_char_p
    lib.fmha_decode_last_error_detail.argtypes = []
    lib.fmha_decode_last_plan.restype = ctypes.c_char_p
    lib.fmha_decode_last_plan.argtypes = []
    lib.fmha_decode_version.restype = ctypes.c_int
    lib.fmha_decode_version.argtypes = []
    _lib = lib
    return lib
