"""PyTorch custom-op registration of the decode-attention kernel.

Importing this module registers
  torch.ops.fmha_amd.decode(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, fp32_weights=False,
                            exact=False) -> O
  torch.ops.fmha_amd.decode_out(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, out, fp32_weights=False,
                                exact=False) -> ()
  torch.ops.fmha_amd.decode_splitkv(q, k, v, cu_seqlens_kv, max_seqlen_kv, softmax_scale) -> O
  torch.ops.fmha_amd.decode_strided(q, k, v, seqlens_kv, softmax_scale) -> O
  torch.ops.fmha_amd.decode_paged(q, k_cache, v_cache, block_table, seqlens_kv, softmax_scale,
                                  max_seqlen_kv=-1) -> O
with fake (meta) implementations, so the kernels can sit inside torch.compile
graphs.  Each calls the C ABI through the matching fmha_amd.decode function
(fmha_decode, fmha_decode_splitkv, fmha_decode_strided, fmha_decode_paged);
there is no other implementation behind them.  The split-KV, strided and
paged ops allocate their workspace through torch's caching allocator.

Arguments are those of fmha_decode: cu_seqlens_kv may be None (uniform
lengths), seqlen_kv < 0 means "infer from k's shape", softmax_scale <= 0
means 1/sqrt(head_dim), fp32_weights keeps the softmax weights in fp32 (the
numerics of the reference's fmha_vectorized_fma; needs cu_seqlens_kv),
exact computes the reference CPU loop's arithmetic step for step (its
outputs bit for bit; needs cu_seqlens_kv and Hq == Hkv).
decode_strided takes k/v as [B, S, Hkv, D] views (any strides with a unit
innermost one: BHSD caches as k.transpose(1, 2)); decode_paged's
max_seqlen_kv < 0 keeps the bound of 16.
"""
from typing import Optional

import torch

from .decode import fmha_decode, fmha_decode_paged, fmha_decode_splitkv, fmha_decode_strided


def _args(cu_seqlens_kv, seqlen_kv, softmax_scale):
    seq = None if (cu_seqlens_kv is not None or seqlen_kv < 0) else int(seqlen_kv)
    scale = None if softmax_scale <= 0 else float(softmax_scale)
    return seq, scale


@torch.library.custom_op("fmha_amd::decode", mutates_args=(), device_types="cuda")
def decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_kv: Optional[torch.Tensor],
           seqlen_kv: int, softmax_scale: float, fp32_weights: bool = False, exact: bool = False) -> torch.Tensor:
    seq, scale = _args(cu_seqlens_kv, seqlen_kv, softmax_scale)
    return fmha_decode(q, k, v, cu_seqlens_kv=cu_seqlens_kv, seqlen_kv=seq, softmax_scale=scale,
                       fp32_weights=fp32_weights, exact=exact)


@decode.register_fake
def _decode_fake(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, fp32_weights=False, exact=False):
    return torch.empty(q.shape, dtype=torch.float16, device=q.device)


@torch.library.custom_op("fmha_amd::decode_out", mutates_args=("out",), device_types="cuda")
def decode_out(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_kv: Optional[torch.Tensor],
               seqlen_kv: int, softmax_scale: float, out: torch.Tensor, fp32_weights: bool = False,
               exact: bool = False) -> None:
    seq, scale = _args(cu_seqlens_kv, seqlen_kv, softmax_scale)
    fmha_decode(q, k, v, cu_seqlens_kv=cu_seqlens_kv, seqlen_kv=seq, softmax_scale=scale, out=out,
                fp32_weights=fp32_weights, exact=exact)


@decode_out.register_fake
def _decode_out_fake(q, k, v, cu_seqlens_kv, seqlen_kv, softmax_scale, out, fp32_weights=False, exact=False):
    return None


def _scale(softmax_scale):
    return None if softmax_scale <= 0 else float(softmax_scale)


def _like_q(q):
    return torch.empty(q.shape, dtype=torch.float16, device=q.device)


@torch.library.custom_op("fmha_amd::decode_splitkv", mutates_args=(), device_types="cuda")
def decode_splitkv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_kv: torch.Tensor,
                   max_seqlen_kv: int, softmax_scale: float) -> torch.Tensor:
    return fmha_decode_splitkv(q, k, v, cu_seqlens_kv, max_seqlen_kv, softmax_scale=_scale(softmax_scale))


@decode_splitkv.register_fake
def _decode_splitkv_fake(q, k, v, cu_seqlens_kv, max_seqlen_kv, softmax_scale):
    return _like_q(q)


@torch.library.custom_op("fmha_amd::decode_strided", mutates_args=(), device_types="cuda")
def decode_strided(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seqlens_kv: Optional[torch.Tensor],
                   softmax_scale: float) -> torch.Tensor:
    return fmha_decode_strided(q, k, v, seqlens_kv=seqlens_kv, softmax_scale=_scale(softmax_scale))


@decode_strided.register_fake
def _decode_strided_fake(q, k, v, seqlens_kv, softmax_scale):
    return _like_q(q)


@torch.library.custom_op("fmha_amd::decode_paged", mutates_args=(), device_types="cuda")
def decode_paged(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, block_table: torch.Tensor,
                 seqlens_kv: torch.Tensor, softmax_scale: float, max_seqlen_kv: int = -1) -> torch.Tensor:
    return fmha_decode_paged(q, k_cache, v_cache, block_table, seqlens_kv, softmax_scale=_scale(softmax_scale),
                             max_seqlen_kv=None if max_seqlen_kv < 0 else int(max_seqlen_kv))


@decode_paged.register_fake
def _decode_paged_fake(q, k_cache, v_cache, block_table, seqlens_kv, softmax_scale, max_seqlen_kv=-1):
    return _like_q(q)
