"""CPU oracle for the decode-attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker or as the timed CPU baseline; the product
(fmha_amd/) never does.

* liboracle.so (fmha_oracle.cpp): the restated reference CPU loop
  (fmha_host.cpp:169-245, with the grouped-query KV-head mapping), a float64
  variant, the comparison gate, the reference's length generator
  (fmha_host.cpp:58-72) and the rounding helpers.
* _ref/libfmha_ref.so (ref_shim.cpp, built only where /root/reference is
  mounted): the reference's own fmha_host.cpp and kernel headers compiled in
  place, used to pin the restatement and to run the reference GPU kernels.

Arrays are numpy: bf16 and fp16 tensors travel as uint16 bit patterns.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# FMHA_ORACLE_LIB selects another build of the same source (the sanitizer
# build of tests/test_sanitizers.py).
LIB_PATH = os.environ.get("FMHA_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libfmha_ref.so")

# Floor of the half-width of the relative perturbation of a softmax weight
# that the gate tolerates at a bf16 rounding midpoint; per head the oracle
# widens it to 4x its own float32 error (see head_f32 in fmha_oracle.cpp).
SLACK_EPS = 2.0 ** -19

_lib = None
_ref = None


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        vp, i64, i32, f32, f64 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float,
                                  ctypes.c_double)
        L.oracle_decode.restype = ctypes.c_int
        L.oracle_decode.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32, f32, i32, vp, vp, f64, i32, i32]
        L.oracle_decode_f64.restype = ctypes.c_int
        L.oracle_decode_f64.argtypes = [vp, vp, vp, vp, i64, i32, i32, i32, f64, vp, i32, i32, vp]
        L.oracle_compare.restype = None
        L.oracle_compare.argtypes = [vp, vp, vp, i64, f64, f64, vp]
        L.oracle_generate_seqlens.restype = None
        L.oracle_generate_seqlens.argtypes = [i64, i32, f64, ctypes.c_uint32, vp]
        L.oracle_f32_to_bf16.restype = None
        L.oracle_f32_to_bf16.argtypes = [vp, i64, vp]
        L.oracle_f32_to_f16.restype = None
        L.oracle_f32_to_f16.argtypes = [vp, i64, vp]
        L.oracle_exp_nearest.restype = None
        L.oracle_exp_nearest.argtypes = [vp, i64, vp]
        _lib = L
    return _lib


def _u16(a):
    a = np.ascontiguousarray(a)
    if a.dtype != np.uint16:
        raise TypeError("expected uint16 bit patterns")
    return a


def decode(q, k, v, cu, hq, hkv, d, scale, p_mode=0, with_slack=False, slack_eps=SLACK_EPS,
           nthreads=0, max_seqlen=16, slack_fixed=False):
    """Restated reference loop.  q [B,Hq,D], k/v [rows,Hkv,D] as uint16 bf16
    bits; cu int32 [B+1]; lengths up to max_seqlen (the reference's 16 by
    default).  p_mode 0: bf16 weights (the reference loop), 1: fp32
    weights, 2: bf16 weights from exp_nearest in place of the C library's
    expf.  Returns (o fp16 bits [B,Hq,D], slack or None).  The slack's
    half-width is max(slack_eps, 4x the oracle's own float32 error) per head,
    or exactly slack_eps with slack_fixed."""
    if slack_fixed:
        slack_eps = -abs(slack_eps)
    q, k, v = _u16(q), _u16(k), _u16(v)
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    B = cu.shape[0] - 1
    o = np.empty((B, hq, d), dtype=np.uint16)
    slack = np.empty((B, hq, d), dtype=np.float32) if with_slack else None
    nt = nthreads if nthreads > 0 else (os.cpu_count() or 1)
    rc = lib().oracle_decode(_p(q), _p(k), _p(v), _p(cu), B, hq, hkv, d, float(scale), p_mode,
                             _p(o), _p(slack), float(slack_eps), nt, max_seqlen)
    if rc != 0:
        raise ValueError("oracle_decode rejected its arguments")
    return o, slack


def exp_nearest(x):
    """The exponential of decode(p_mode=2): float32 x -> the float nearest
    exp(x), evaluated in double and rounded once."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().oracle_exp_nearest(_p(x), x.size, _p(out))
    return out


def decode_f64(q, k, v, cu, hq, hkv, d, scale, nthreads=0, max_seqlen=16, with_bound=False):
    """Float64 decode attention; returns float64 [B,Hq,D], or (that, bound)
    with with_bound: the per-element bound on |o - t| that a bf16-weight
    float32 implementation meets without tie slack (head_f64 in
    fmha_oracle.cpp)."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    B = cu.shape[0] - 1
    o = np.empty((B, hq, d), dtype=np.float64)
    bound = np.empty((B, hq, d), dtype=np.float64) if with_bound else None
    nt = nthreads if nthreads > 0 else (os.cpu_count() or 1)
    rc = lib().oracle_decode_f64(_p(q), _p(k), _p(v), _p(cu), B, hq, hkv, d, float(scale), _p(o), nt,
                                 max_seqlen, _p(bound))
    if rc != 0:
        raise ValueError("oracle_decode_f64 rejected its arguments")
    return (o, bound) if with_bound else o


def compare(o, r, slack=None, atol=2e-3, rtol=1e-2):
    """Gate |o-r| <= atol + rtol*|r| + slack per element (o, r fp16 bits)."""
    o, r = _u16(o).ravel(), _u16(r).ravel()
    if o.shape != r.shape:
        raise ValueError("shape mismatch")
    s = None if slack is None else np.ascontiguousarray(slack, dtype=np.float32).ravel()
    stats = np.zeros(9, dtype=np.float64)
    lib().oracle_compare(_p(o), _p(r), _p(s), o.size, atol, rtol, _p(stats))
    return {
        "fails": int(stats[0]), "slack_elems": int(stats[1]), "max_abs": float(stats[2]),
        "max_rel": float(stats[3]), "ref_rule_fails": int(stats[4]), "nonfinite": int(stats[5]),
        "first_fail": int(stats[6]), "n": int(stats[7]), "ref_rule_fails_raw": int(stats[8]),
        "atol": atol, "rtol": rtol,
    }


def generate_seqlens(batch, max_seqlen=16, lam=4.0, seed=42):
    out = np.empty(batch, dtype=np.int32)
    lib().oracle_generate_seqlens(batch, max_seqlen, lam, seed, _p(out))
    return out


def f32_to_bf16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(_p(x), x.size, _p(out))
    return out


def f32_to_f16(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16(_p(x), x.size, _p(out))
    return out


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_to_f32(bits):
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------
# The reference compiled in place (oracle/_ref), when it was built.
# ---------------------------------------------------------------------------
def ref_available():
    return os.path.exists(REF_LIB_PATH)


def ref_lib():
    global _ref
    if _ref is None:
        if not ref_available():
            raise RuntimeError(f"{REF_LIB_PATH} not built (needs /root/reference)")
        R = ctypes.CDLL(REF_LIB_PATH)
        vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        R.ref_generate_seqlens.restype = None
        R.ref_generate_seqlens.argtypes = [i32, i32, vp]
        R.ref_do_validation.restype = ctypes.c_int
        R.ref_do_validation.argtypes = [i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]
        for name in ("ref_launch_mfma_4x4x4", "ref_launch_vectorized_fma", "ref_launch_mfma",
                     "ref_launch_mfma_v3"):
            fn = getattr(R, name)
            fn.restype = ctypes.c_int
            fn.argtypes = [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, f32]
        _ref = R
    return _ref


def ref_do_validation(q, k, v, cu, hq, hkv, d, gpu_o=None):
    """Run the reference's do_validation (fmha_host.cpp:158-284).  Returns
    (ref_o fp16 bits [B,Hq,D], passed).  The reference prints to stdout."""
    q, k, v = _u16(q), _u16(k), _u16(v)
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    B = cu.shape[0] - 1
    ref_o = np.empty((B, hq, d), dtype=np.uint16)
    g = np.zeros((B, hq, d), dtype=np.uint16) if gpu_o is None else _u16(gpu_o)
    ok = ref_lib().ref_do_validation(B, hq, hkv, d, _p(cu), _p(q), _p(k), _p(v), _p(ref_o), _p(g))
    return ref_o, bool(ok)


def ref_generate_seqlens(batch, max_seqlen=16):
    out = np.empty(batch, dtype=np.int32)
    ref_lib().ref_generate_seqlens(batch, max_seqlen, _p(out))
    return out
