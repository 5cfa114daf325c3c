"""Host-side interface of the decode-attention path.

Two levels, both thin wrappers over the C ABI in include/fmha_decode.h:

* launch_fmha_decode / launch_fmha_decode_uniform -- pointer level, the same
  parameters, order and meaning as the reference's launch helper
  launch_fmha_mfma_4x4x4 (fmha_mfma_4x4x4_kernel.hpp:370-376) without the
  caller-chosen grid/block; a rejected call raises FmhaDecodeError instead of
  failing silently.
* fmha_decode -- tensor level, for torch device tensors: checks shapes,
  dtypes and devices, allocates O if not given, launches on torch's current
  stream.  fmha_decode_strided and fmha_decode_paged do the same for strided
  (BSHD / BHSD / padded) and paged KV caches.
"""
import math

from . import _lib

MAX_SEQLEN_KV = 16
# Bytes of the device array fmha_decode_fwd_splitkv_noalloc uses as its
# workspace (FMHA_DECODE_NOALLOC_SCRATCH_BYTES in include/fmha_decode.h).
NOALLOC_SCRATCH_BYTES = 64 << 20


class FmhaDecodeError(RuntimeError):
    """A call the library rejected (code is the hipError_t value returned)."""

    def __init__(self, code, message, detail):
        super().__init__(f"fmha_decode error {code} ({message}): {detail}")
        self.code = code
        self.detail = detail


def last_plan():
    """The kernels the most recent call on this thread launched, as the
    library describes them (fmha_decode_last_plan): a list of strings such
    as "split(D=128 G=4 layout=packed sub_units=1 blocks=64 ...)"."""
    text = _lib.load().fmha_decode_last_plan().decode()
    return [p for p in text.split("; ") if p]


def _raise_if(rc):
    if rc != 0:
        lib = _lib.load()
        raise FmhaDecodeError(rc, lib.fmha_decode_error_string(rc).decode(),
                              lib.fmha_decode_last_error_detail().decode())


def launch_fmha_decode(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv,
                       seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """Variable-length decode attention on raw device pointers (ints).

    stream is a hipStream_t as an int (0 = null stream).  Mirrors
    launch_fmha_mfma_4x4x4 (fmha_mfma_4x4x4_kernel.hpp:370-376).  Up to 2
    query heads per KV head the outputs are the reference CPU loop's
    (fmha_host.cpp:179-244) bit for bit; above, tree-order sums (within the
    comparison gate).
    """
    rc = _lib.load().fmha_decode_fwd(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q,
                                     num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                     float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_fast(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv,
                            seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """launch_fmha_decode with tree-order sums and the device expf: the same
    semantics within the comparison gate, not the CPU loop's bits."""
    rc = _lib.load().fmha_decode_fwd_fast(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q,
                                          num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                          float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_fp32_weights(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv,
                                    seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """launch_fmha_decode with fp32 softmax weights: the semantics of the
    reference's fmha_vectorized_fma (fmha_vectorized_fma_kernel.hpp:243-296)."""
    rc = _lib.load().fmha_decode_fwd_fp32_weights(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q,
                                                  num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                                  float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_exact(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q, num_heads_kv,
                             seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """launch_fmha_decode with the reference CPU loop's arithmetic step for
    step (fmha_host.cpp:179-244) for every call: its outputs bit for bit
    wherever that loop's expf returns the nearest float; more than 8 query
    heads per KV head are rejected."""
    rc = _lib.load().fmha_decode_fwd_exact(stream, Q, K, V, O, cu_seqlens_kv, batch, num_heads_q,
                                           num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                           float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_uniform(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q, num_heads_kv,
                               seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """Uniform-length decode attention (K/V as [batch, seqlen_kv, Hkv, D]);
    numerics as launch_fmha_decode."""
    rc = _lib.load().fmha_decode_fwd_uniform(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q,
                                             num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                             float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_uniform_fast(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q, num_heads_kv,
                                    seqlen_q, head_dim_q, head_dim_kv, softmax_scale):
    """launch_fmha_decode_uniform with the numerics of launch_fmha_decode_fast."""
    rc = _lib.load().fmha_decode_fwd_uniform_fast(stream, Q, K, V, O, seqlen_kv, batch, num_heads_q,
                                                  num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                                  float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_strided(stream, Q, K, V, O, seqlens_kv, seqlen_kv, kv_batch_stride, kv_row_stride,
                               kv_head_stride, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q,
                               head_dim_kv, softmax_scale):
    """Decode attention over strided K/V (strides in elements); seqlens_kv is
    a device pointer to int32 lengths or 0 for a uniform length."""
    rc = _lib.load().fmha_decode_fwd_strided(stream, Q, K, V, O, seqlens_kv, seqlen_kv, kv_batch_stride,
                                             kv_row_stride, kv_head_stride, batch, num_heads_q, num_heads_kv,
                                             seqlen_q, head_dim_q, head_dim_kv, float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_paged(stream, Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv,
                             page_size, batch, num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                             softmax_scale):
    """Decode attention over a paged [pages, page_size, Hkv, D] cache."""
    rc = _lib.load().fmha_decode_fwd_paged(stream, Q, K_cache, V_cache, O, block_table, block_table_stride,
                                           seqlens_kv, page_size, batch, num_heads_q, num_heads_kv, seqlen_q,
                                           head_dim_q, head_dim_kv, float(softmax_scale))
    _raise_if(rc)


def launch_fmha_decode_splitkv_strided(stream, Q, K, V, O, seqlens_kv, max_seqlen_kv, kv_batch_stride,
                                       kv_row_stride, kv_head_stride, batch, num_heads_q, num_heads_kv, seqlen_q,
                                       head_dim_q, head_dim_kv, softmax_scale, workspace, workspace_bytes):
    """Strided K/V with lengths up to max_seqlen_kv (any size), using a
    caller-provided device workspace; seqlens_kv is a device pointer or 0."""
    rc = _lib.load().fmha_decode_fwd_splitkv_strided(stream, Q, K, V, O, seqlens_kv, max_seqlen_kv, kv_batch_stride,
                                                     kv_row_stride, kv_head_stride, batch, num_heads_q, num_heads_kv,
                                                     seqlen_q, head_dim_q, head_dim_kv, float(softmax_scale),
                                                     workspace, workspace_bytes)
    _raise_if(rc)


def launch_fmha_decode_splitkv_paged(stream, Q, K_cache, V_cache, O, block_table, block_table_stride, seqlens_kv,
                                     page_size, max_seqlen_kv, batch, num_heads_q, num_heads_kv, seqlen_q,
                                     head_dim_q, head_dim_kv, softmax_scale, workspace, workspace_bytes):
    """Paged [pages, page_size, Hkv, D] cache with lengths up to
    max_seqlen_kv (any size), using a caller-provided device workspace."""
    rc = _lib.load().fmha_decode_fwd_splitkv_paged(stream, Q, K_cache, V_cache, O, block_table, block_table_stride,
                                                   seqlens_kv, page_size, max_seqlen_kv, batch, num_heads_q,
                                                   num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                                   float(softmax_scale), workspace, workspace_bytes)
    _raise_if(rc)


def splitkv_workspace_size(batch, num_heads_q, num_heads_kv, max_seqlen_kv, head_dim):
    """Bytes of device workspace fmha_decode_fwd_splitkv needs (0 if the
    arguments are invalid)."""
    return int(_lib.load().fmha_decode_splitkv_workspace_size(batch, num_heads_q, num_heads_kv, max_seqlen_kv,
                                                              head_dim))


def launch_fmha_decode_splitkv(stream, Q, K, V, O, cu_seqlens_kv, max_seqlen_kv, batch, num_heads_q,
                               num_heads_kv, seqlen_q, head_dim_q, head_dim_kv, softmax_scale, workspace,
                               workspace_bytes):
    """Decode attention for lengths up to max_seqlen_kv (any size) over the
    packed layout, using a caller-provided device workspace."""
    rc = _lib.load().fmha_decode_fwd_splitkv(stream, Q, K, V, O, cu_seqlens_kv, max_seqlen_kv, batch,
                                             num_heads_q, num_heads_kv, seqlen_q, head_dim_q, head_dim_kv,
                                             float(softmax_scale), workspace, workspace_bytes)
    _raise_if(rc)


def fmha_decode_splitkv(q, k, v, cu_seqlens_kv, max_seqlen_kv, softmax_scale=None, out=None, workspace=None):
    """Decode attention with lengths beyond 16: q [B, Hq, 1, D] or [B, Hq, D],
    k/v packed [rows, Hkv, D] bfloat16, cu_seqlens_kv int32 [B+1], every
    length <= max_seqlen_kv.  workspace: a uint8 device tensor of at least
    splitkv_workspace_size(...) bytes (allocated here when None)."""
    import torch
    B, Hq, D = _q_shape(q)
    out = _check_q_out(q, out)
    for name, t in (("k", k), ("v", v)):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 3 or not t.is_contiguous() or t.shape[2] != D:
            raise ValueError(f"{name} must be a contiguous bfloat16 GPU tensor [rows, Hkv, D]")
    _check_device(q, k=k, v=v)
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    if (cu_seqlens_kv.dtype != torch.int32 or cu_seqlens_kv.numel() != B + 1
            or cu_seqlens_kv.device != q.device or not cu_seqlens_kv.is_contiguous()):
        raise ValueError("cu_seqlens_kv must be a contiguous int32 tensor [batch+1] on q's device")
    Hkv = k.shape[1]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    need = splitkv_workspace_size(B, Hq, Hkv, int(max_seqlen_kv), D)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    if workspace.dtype != torch.uint8 or workspace.device != q.device or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor on q's device")
    stream = torch.cuda.current_stream(q.device).cuda_stream
    launch_fmha_decode_splitkv(stream, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                               cu_seqlens_kv.data_ptr(), int(max_seqlen_kv), B, Hq, Hkv, 1, D, D, softmax_scale,
                               workspace.data_ptr(), workspace.numel())
    return out


def _q_shape(q):
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("q must have seqlen_q == 1")
        return q.shape[0], q.shape[1], q.shape[3]
    if q.dim() == 3:
        return tuple(q.shape)
    raise ValueError("q must be [B, Hq, 1, D] or [B, Hq, D]")


def _check_q_out(q, out):
    import torch
    if q.dtype != torch.bfloat16 or not q.is_cuda or not q.is_contiguous():
        raise ValueError("q must be a contiguous bfloat16 GPU tensor")
    if out is None:
        return torch.empty(q.shape, dtype=torch.float16, device=q.device)
    if out.dtype != torch.float16 or out.shape != q.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous float16 tensor shaped like q")
    _check_device(q, out=out)
    return out


def _check_device(q, **tensors):
    """Every tensor must live on q's device: the kernels dereference their
    pointers there, and a host or other-device pointer would fault."""
    for name, t in tensors.items():
        if t is not None and t.device != q.device:
            raise ValueError(f"{name} must be on q's device ({q.device}), not {t.device}")


def _check_lengths(t, B, device):
    import torch
    if t is None:
        return 0
    if t.dtype != torch.int32 or t.numel() != B or t.device != device or not t.is_contiguous():
        raise ValueError("seqlens_kv must be a contiguous int32 tensor [batch] on q's device")
    return t.data_ptr()


def _workspace(workspace, need, device):
    import torch
    if workspace is None:
        return torch.empty(max(need, 1), dtype=torch.uint8, device=device)
    if workspace.dtype != torch.uint8 or workspace.device != device or not workspace.is_contiguous():
        raise ValueError("workspace must be a contiguous uint8 tensor on q's device")
    return workspace


def fmha_decode_strided(q, k, v, seqlens_kv=None, softmax_scale=None, out=None, workspace=None):
    """Decode attention for K/V given as any [B, S, Hkv, D] view with unit
    innermost stride: a contiguous padded BSHD cache, or a BHSD cache passed
    as k.transpose(1, 2).  seqlens_kv (int32 [B]) gives each batch's length
    (rows past it are never read; a length above S gives NaN); without it
    every batch uses all S rows.  S may exceed 16: the call then goes through
    fmha_decode_fwd_splitkv_strided with workspace (a uint8 device tensor of
    splitkv_workspace_size(B, Hq, Hkv, S, D) bytes, allocated here when
    None)."""
    import torch
    B, Hq, D = _q_shape(q)
    out = _check_q_out(q, out)
    for name, t in (("k", k), ("v", v)):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 4 or t.shape[0] != B or t.shape[3] != D:
            raise ValueError(f"{name} must be a bfloat16 GPU tensor [B, S, Hkv, D]")
        if t.stride(3) != 1:
            raise ValueError(f"{name} must have unit stride in the head dimension")
    _check_device(q, k=k, v=v)
    if k.shape != v.shape or k.stride() != v.stride():
        raise ValueError("k and v must have the same shape and strides")
    S, Hkv = k.shape[1], k.shape[2]
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    lens = _check_lengths(seqlens_kv, B, q.device)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if S > MAX_SEQLEN_KV:
        ws = _workspace(workspace, splitkv_workspace_size(B, Hq, Hkv, S, D), q.device)
        launch_fmha_decode_splitkv_strided(stream, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lens, S,
                                           k.stride(0), k.stride(1), k.stride(2), B, Hq, Hkv, 1, D, D, softmax_scale,
                                           ws.data_ptr(), ws.numel())
        return out
    launch_fmha_decode_strided(stream, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), lens, S,
                               k.stride(0), k.stride(1), k.stride(2), B, Hq, Hkv, 1, D, D, softmax_scale)
    return out


def fmha_decode_paged(q, k_cache, v_cache, block_table, seqlens_kv, softmax_scale=None, out=None,
                      max_seqlen_kv=None, workspace=None):
    """Decode attention over a paged cache: k_cache/v_cache [pages, page_size,
    Hkv, D] bfloat16, block_table int32 [B, max_pages], seqlens_kv int32 [B].
    Lengths above max_seqlen_kv (default 16, the reference's bound) or above
    max_pages * page_size give NaN.  With max_seqlen_kv given the call goes
    through fmha_decode_fwd_splitkv_paged with workspace (a uint8 device
    tensor of splitkv_workspace_size(B, Hq, Hkv, max_seqlen_kv, D) bytes,
    allocated here when None; for max_seqlen_kv <= 16 it is used only by a
    group size above 8 whose rows may reach past a batch's first page).
    Without max_seqlen_kv, a group size above 8 needs pages of at least
    min(16, max_pages * page_size) rows (FmhaDecodeError otherwise)."""
    import torch
    B, Hq, D = _q_shape(q)
    out = _check_q_out(q, out)
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if t.dtype != torch.bfloat16 or not t.is_cuda or t.dim() != 4 or not t.is_contiguous() or t.shape[3] != D:
            raise ValueError(f"{name} must be a contiguous bfloat16 GPU tensor [pages, page_size, Hkv, D]")
    _check_device(q, k_cache=k_cache, v_cache=v_cache)
    if k_cache.shape != v_cache.shape:
        raise ValueError("k_cache and v_cache must have the same shape")
    if (block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B
            or block_table.stride(1) != 1 or block_table.device != q.device):
        raise ValueError("block_table must be int32 [B, max_pages] with unit column stride on q's device")
    lens = _check_lengths(seqlens_kv, B, q.device)
    if lens == 0:
        raise ValueError("seqlens_kv is required for a paged cache")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if max_seqlen_kv is not None:
        Hkv = k_cache.shape[2]
        ws = _workspace(workspace, splitkv_workspace_size(B, Hq, Hkv, int(max_seqlen_kv), D), q.device)
        launch_fmha_decode_splitkv_paged(stream, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                                         block_table.data_ptr(), block_table.stride(0), lens, k_cache.shape[1],
                                         int(max_seqlen_kv), B, Hq, Hkv, 1, D, D, softmax_scale, ws.data_ptr(),
                                         ws.numel())
        return out
    launch_fmha_decode_paged(stream, q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
                             block_table.data_ptr(), block_table.stride(0), lens, k_cache.shape[1], B, Hq,
                             k_cache.shape[2], 1, D, D, softmax_scale)
    return out


def fmha_decode(q, k, v, cu_seqlens_kv=None, seqlen_kv=None, softmax_scale=None, out=None, fp32_weights=False,
                exact=False, fast=False):
    """Decode attention on torch tensors; returns O (fp16, shaped like q).

    q: [B, Hq, 1, D] or [B, Hq, D], bfloat16, contiguous, on a GPU.
    k, v: [rows, Hkv, D] packed (with cu_seqlens_kv) or [B, S, Hkv, D]
      (uniform, with seqlen_kv or inferred from the shape); bfloat16.
    cu_seqlens_kv: int32 [B+1] on the same device, or None.
    softmax_scale: defaults to 1/sqrt(D), as the reference passes
      (fmha_host.cpp:371).
    Numerics (at most one flag): by default the reference CPU loop's
      arithmetic step for step up to 2 query heads per KV head (its outputs
      bit for bit wherever its expf returns the nearest float) and tree-order
      sums above;
    exact: the loop's arithmetic for every call (with cu_seqlens_kv up to 8
      query heads per KV head, with uniform lengths up to 2; others are
      rejected);
    fast: tree-order sums and the device expf (fmha_decode_fwd_fast,
      fmha_decode_fwd_uniform_fast);
    fp32_weights: keep the softmax weights in fp32 (fmha_vectorized_fma's
      semantics) instead of rounding them to bf16; needs cu_seqlens_kv.
    """
    import torch

    if q.dim() == 4:
        if q.shape[2] != 1:
            raise ValueError("q must have seqlen_q == 1")
        B, Hq, _, D = q.shape
    elif q.dim() == 3:
        B, Hq, D = q.shape
    else:
        raise ValueError("q must be [B, Hq, 1, D] or [B, Hq, D]")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16 (got {t.dtype})")
        if not t.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    Hkv = k.shape[-2]
    if k.shape[-1] != D:
        raise ValueError("k/v head_dim must equal q head_dim")
    if int(bool(fp32_weights)) + int(bool(exact)) + int(bool(fast)) > 1:
        raise ValueError("fp32_weights, exact and fast are different numerics; pick one")
    _check_device(q, k=k, v=v)
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    if out is None:
        out = torch.empty(q.shape, dtype=torch.float16, device=q.device)
    elif out.dtype != torch.float16 or out.shape != q.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous float16 tensor shaped like q")
    else:
        _check_device(q, out=out)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    if cu_seqlens_kv is not None:
        if cu_seqlens_kv.dtype != torch.int32 or cu_seqlens_kv.numel() != B + 1:
            raise ValueError("cu_seqlens_kv must be int32 with batch+1 entries")
        if cu_seqlens_kv.device != q.device or not cu_seqlens_kv.is_contiguous():
            raise ValueError("cu_seqlens_kv must be a contiguous tensor on q's device")
        if k.dim() != 3:
            raise ValueError("packed k/v must be [rows, Hkv, D]")
        launch = (launch_fmha_decode_fp32_weights if fp32_weights else
                  launch_fmha_decode_exact if exact else
                  launch_fmha_decode_fast if fast else launch_fmha_decode)
        launch(stream, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
               cu_seqlens_kv.data_ptr(), B, Hq, Hkv, 1, D, D, softmax_scale)
    else:
        if fp32_weights:
            raise ValueError("fp32_weights needs the packed layout with cu_seqlens_kv")
        if exact and Hq // Hkv > 2:
            # fmha_decode_fwd_uniform takes the exact numerics up to 2 query
            # heads per KV head; fmha_decode_fwd_exact (cu_seqlens_kv) up to 8
            raise ValueError("exact with uniform lengths takes at most 2 query heads per KV head (got %d); "
                             "pass cu_seqlens_kv for up to 8" % (Hq // Hkv))
        if seqlen_kv is None:
            if k.dim() != 4 or k.shape[0] != B:
                raise ValueError("uniform k/v must be [B, S, Hkv, D] when seqlen_kv is not given")
            seqlen_kv = k.shape[1]
        if k.numel() != B * seqlen_kv * Hkv * D:
            raise ValueError("k/v size does not match batch * seqlen_kv * Hkv * D")
        launch = launch_fmha_decode_uniform_fast if fast else launch_fmha_decode_uniform
        launch(stream, q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
               seqlen_kv, B, Hq, Hkv, 1, D, D, softmax_scale)
    return out
