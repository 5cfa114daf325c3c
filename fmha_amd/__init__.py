"""fmha_amd -- MI355X (gfx950) decode attention: seqlen_q = 1, KV length
0..16 per sequence, bf16 Q/K/V, fp32 accumulation, fp16 output, with
grouped-query attention.  The kernels are hand-written HIP in fmha_amd/csrc;
the C ABI is include/fmha_decode.h; this package is its host-side interface.
"""
from .decode import (MAX_SEQLEN_KV, NOALLOC_SCRATCH_BYTES, FmhaDecodeError, fmha_decode, fmha_decode_paged,
                     fmha_decode_splitkv, fmha_decode_strided, launch_fmha_decode, launch_fmha_decode_exact,
                     launch_fmha_decode_fast, launch_fmha_decode_uniform_fast,
                     launch_fmha_decode_fp32_weights, launch_fmha_decode_paged,
                     launch_fmha_decode_splitkv, launch_fmha_decode_splitkv_paged, launch_fmha_decode_splitkv_strided,
                     launch_fmha_decode_strided, launch_fmha_decode_uniform, last_plan, splitkv_workspace_size)
from ._lib import LIB_PATH, EXPORTED

__all__ = [
    "MAX_SEQLEN_KV",
    "NOALLOC_SCRATCH_BYTES",
    "FmhaDecodeError",
    "fmha_decode",
    "fmha_decode_strided",
    "fmha_decode_paged",
    "launch_fmha_decode_strided",
    "launch_fmha_decode_paged",
    "fmha_decode_splitkv",
    "launch_fmha_decode_splitkv",
    "launch_fmha_decode_splitkv_strided",
    "launch_fmha_decode_splitkv_paged",
    "splitkv_workspace_size",
    "launch_fmha_decode",
    "launch_fmha_decode_fp32_weights",
    "launch_fmha_decode_exact",
    "launch_fmha_decode_fast",
    "launch_fmha_decode_uniform_fast",
    "launch_fmha_decode_uniform",
    "last_plan",
    "LIB_PATH",
    "EXPORTED",
]
