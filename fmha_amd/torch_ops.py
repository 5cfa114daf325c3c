"""PyTorch custom-op registration of the decode-attention kernel.

Importing this module registers
  torch.ops.fmha_amd.decode(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, fp32_weights=False) -> O
  torch.ops.fmha_amd.decode_out(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, out, fp32_weights=False) -> ()
with fake (meta) implementations, so the kernel can sit inside torch.compile
graphs.  Both call the C ABI through fmha_amd.decode.fmha_decode; there is no
other implementation behind them.

Arguments are those of fmha_decode: cu_seqlens_kv may be None (uniform
lengths), seqlen_kv < 0 means "infer from k's shape", softmax_scale <= 0
means 1/sqrt(head_dim), fp32_weights keeps the softmax weights in fp32 (the
numerics of the reference's fmha_vectorized_fma; needs cu_seqlens_kv).
"""
from typing import Optional

import torch

from .decode import fmha_decode


def _args(cu_seqlens_kv, seqlen_kv, softmax_scale):
    seq = None if (cu_seqlens_kv is not None or seqlen_kv < 0) else int(seqlen_kv)
    scale = None if softmax_scale <= 0 else float(softmax_scale)
    return seq, scale


@torch.library.custom_op("fmha_amd::decode", mutates_args=(), device_types="cuda")
def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_kv: Optional[torch.Tensor],
           seqlen_kv: int, softmax_scale: float, fp32_weights: bool = False) -> torch.Tensor:
    seq, scale = _args(cu_seqlens_kv, seqlen_kv, softmax_scale)
    return fmha_decode(q, k, v, cu_seqlens_kv=cu_seqlens_kv, seqlen_kv=seq, softmax_scale=scale,
                       fp32_weights=fp32_weights)


@decode.register_fake
def _decode_fake(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, fp32_weights=False):
    return torch.empty(q.shape, dtype=torch.float16, device=q.device)


@torch.library.custom_op("fmha_amd::decode_out", mutates_args=("out",), device_types="cuda")
def decode_out(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_kv: Optional[torch.Tensor],
               seqlen_kv: int, softmax_scale: float, out: torch.Tensor, fp32_weights: bool = False) -> None:
    seq, scale = _args(cu_seqlens_kv, seqlen_kv, softmax_scale)
    fmha_decode(q, k, v, cu_seqlens_kv=cu_seqlens_kv, seqlen_kv=seq, softmax_scale=scale, out=out,
                fp32_weights=fp32_weights)


@decode_out.register_fake
def _decode_out_fake(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, out, fp32_weights=False):
    return None
