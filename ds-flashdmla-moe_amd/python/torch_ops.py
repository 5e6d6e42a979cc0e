"""The ops registered with PyTorch's dispatcher: ``torch.ops.flashdmla.*``.

The reference's layout names ``csrc/torch_bindings.cpp`` ("pybind11/ATen entry points",
README.md:35) under its autograd wrappers; neither file exists.  This module is that layer for
this backend: each op is a ``torch.library`` custom op whose CUDA (HIP) kernel is the matching
C-ABI call of ``libflashdmla.so`` (through python/ops.py), with a fake implementation for shape
inference (meta tensors, tracing) and, for the two forwards, an autograd formula that runs the
matching backward op.  Only GPU tensors have a kernel: CPU tensors raise, as everywhere else.

    torch.ops.flashdmla.fwd_cache_latent(q, k_lat, d_v, softmax_scale, causal) -> (o, m, l)
    torch.ops.flashdmla.bwd_cache_latent(q, k_lat, o, do, m, l, d_v, softmax_scale, causal) -> (dq, dk_lat)
    torch.ops.flashdmla.fwd_onthefly(q, k, v, wk, wv, softmax_scale, causal) -> (o, m, l)
    torch.ops.flashdmla.bwd_onthefly(q, k, v, wk, wv, o, do, m, l, softmax_scale, causal)
        -> (dq, dk, dv, dwk, dwv)
    torch.ops.flashdmla.decode_plan(cache_seqlens, num_heads, max_pages) -> plan
    torch.ops.flashdmla.decode_paged(q, kv_pool, block_table, cache_seqlens, d_v, softmax_scale, plan)
        -> (o, lse)
    torch.ops.flashdmla.kv_append(kv_pool, block_table, cache_seqlens, new_kv, new_lens) -> ()   (kv_pool in place)
    torch.ops.flashdmla.lse_combine(part_o, part_lse, num_splits) -> (o, lse)

Shapes and conventions are those of python/ops.py.  m and l are outputs without a gradient;
the backwards return dk_lat and dwk / dwv in float32 (the autograd formulas cast them to the
input dtypes).  The host-side checks of python/ops.py that synchronize (check_range,
check_indices) are not part of these signatures.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor
from torch.library import custom_op

from . import _lib, ops

_F32 = torch.float32
_BF16 = torch.bfloat16


# ---- cache-latent forward / backward ---------------------------------------------------------
@custom_op("flashdmla::fwd_cache_latent", mutates_args=(), device_types="cuda")
def fwd_cache_latent(q: Tensor, k_lat: Tensor, d_v: int, softmax_scale: Optional[float],
                     causal: bool) -> Tuple[Tensor, Tensor, Tensor]:
    o, m, l = ops.flash_dmla_fwd(q, k_lat, d_v, softmax_scale, causal, return_stats=True)
    return o, m, l


@fwd_cache_latent.register_fake
def _(q, k_lat, d_v, softmax_scale, causal):
    B, H, Sq, _ = q.shape
    return (q.new_empty((B, H, Sq, d_v), dtype=_BF16), q.new_empty((B, H, Sq), dtype=_F32),
            q.new_empty((B, H, Sq), dtype=_F32))


@custom_op("flashdmla::bwd_cache_latent", mutates_args=(), device_types="cuda")
def bwd_cache_latent(q: Tensor, k_lat: Tensor, o: Tensor, do: Tensor, m: Tensor, l: Tensor, d_v: int,
                     softmax_scale: Optional[float], causal: bool) -> Tuple[Tensor, Tensor]:
    return ops.flash_dmla_bwd(q, k_lat, o, do, m, l, d_v, softmax_scale, causal)


@bwd_cache_latent.register_fake
def _(q, k_lat, o, do, m, l, d_v, softmax_scale, causal):
    return q.new_empty(q.shape, dtype=q.dtype), k_lat.new_empty(k_lat.shape, dtype=_F32)


def _fwd_cl_setup(ctx, inputs, output):
    q, k_lat, d_v, softmax_scale, causal = inputs
    o, m, l = output
    ctx.mark_non_differentiable(m, l)
    ctx.save_for_backward(q, k_lat, o, m, l)
    ctx.args = (d_v, softmax_scale, causal)


def _fwd_cl_backward(ctx, do, _dm, _dl):
    q, k_lat, o, m, l = ctx.saved_tensors
    d_v, softmax_scale, causal = ctx.args
    dq, dk = torch.ops.flashdmla.bwd_cache_latent(q, k_lat, o, do.contiguous(), m, l, d_v, softmax_scale, causal)
    return dq, dk.to(k_lat.dtype), None, None, None


fwd_cache_latent.register_autograd(_fwd_cl_backward, setup_context=_fwd_cl_setup)


# ---- on-the-fly forward / backward -----------------------------------------------------------
@custom_op("flashdmla::fwd_onthefly", mutates_args=(), device_types="cuda")
def fwd_onthefly(q: Tensor, k: Tensor, v: Tensor, wk: Tensor, wv: Tensor, softmax_scale: Optional[float],
                 causal: bool) -> Tuple[Tensor, Tensor, Tensor]:
    o, m, l = ops.flash_dmla_fwd_onthefly(q, k, v, wk, wv, softmax_scale, causal, return_stats=True)
    return o, m, l


@fwd_onthefly.register_fake
def _(q, k, v, wk, wv, softmax_scale, causal):
    B, H, Sq, _ = q.shape
    return (q.new_empty((B, H, Sq, wk.shape[2]), dtype=_BF16), q.new_empty((B, H, Sq), dtype=_F32),
            q.new_empty((B, H, Sq), dtype=_F32))


@custom_op("flashdmla::bwd_onthefly", mutates_args=(), device_types="cuda")
def bwd_onthefly(q: Tensor, k: Tensor, v: Tensor, wk: Tensor, wv: Tensor, o: Tensor, do: Tensor, m: Tensor,
                 l: Tensor, softmax_scale: Optional[float],
                 causal: bool) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    return ops.flash_dmla_bwd_onthefly(q, k, v, wk, wv, o, do, m, l, softmax_scale, causal)


@bwd_onthefly.register_fake
def _(q, k, v, wk, wv, o, do, m, l, softmax_scale, causal):
    return (q.new_empty(q.shape, dtype=_BF16), k.new_empty(k.shape, dtype=_BF16), v.new_empty(v.shape, dtype=_BF16),
            wk.new_empty(wk.shape, dtype=_F32), wv.new_empty(wv.shape, dtype=_F32))


def _fwd_otf_setup(ctx, inputs, output):
    q, k, v, wk, wv, softmax_scale, causal = inputs
    o, m, l = output
    ctx.mark_non_differentiable(m, l)
    ctx.save_for_backward(q, k, v, wk, wv, o, m, l)
    ctx.args = (softmax_scale, causal)


def _fwd_otf_backward(ctx, do, _dm, _dl):
    q, k, v, wk, wv, o, m, l = ctx.saved_tensors
    softmax_scale, causal = ctx.args
    dq, dk, dv, dwk, dwv = torch.ops.flashdmla.bwd_onthefly(q, k, v, wk, wv, o, do.contiguous(), m, l,
                                                            softmax_scale, causal)
    return dq, dk, dv, dwk.to(wk.dtype), dwv.to(wv.dtype), None, None


fwd_onthefly.register_autograd(_fwd_otf_backward, setup_context=_fwd_otf_setup)


# ---- paged decode, its plan, the append and the split-KV combine ------------------------------
@custom_op("flashdmla::decode_plan", mutates_args=(), device_types="cuda")
def decode_plan(cache_seqlens: Tensor, num_heads: int, max_pages: int) -> Tensor:
    return ops.flash_dmla_decode_plan(cache_seqlens, num_heads, max_pages)


@decode_plan.register_fake
def _(cache_seqlens, num_heads, max_pages):
    nbytes = int(_lib.lib().dmla_decode_plan_bytes(cache_seqlens.shape[0], num_heads, max_pages))
    return cache_seqlens.new_empty((nbytes // 4,), dtype=torch.int32)


@custom_op("flashdmla::decode_paged", mutates_args=(), device_types="cuda")
def decode_paged(q: Tensor, kv_pool: Tensor, block_table: Tensor, cache_seqlens: Tensor, d_v: int,
                 softmax_scale: Optional[float], plan: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
    o, lse = ops.flash_dmla_decode_paged(q, kv_pool, block_table, cache_seqlens, d_v, softmax_scale,
                                         return_lse=True, plan=plan)
    return o, lse


@decode_paged.register_fake
def _(q, kv_pool, block_table, cache_seqlens, d_v, softmax_scale, plan):
    B, H, _ = q.shape
    return q.new_empty((B, H, d_v), dtype=_BF16), q.new_empty((B, H), dtype=_F32)


@custom_op("flashdmla::kv_append", mutates_args=("kv_pool",), device_types="cuda")
def kv_append(kv_pool: Tensor, block_table: Tensor, cache_seqlens: Tensor, new_kv: Tensor,
              new_lens: Optional[Tensor]) -> None:
    ops.flash_dmla_kv_append(kv_pool, block_table, cache_seqlens, new_kv, new_lens)


@kv_append.register_fake
def _(kv_pool, block_table, cache_seqlens, new_kv, new_lens):
    return None


@custom_op("flashdmla::lse_combine", mutates_args=(), device_types="cuda")
def lse_combine(part_o: Tensor, part_lse: Tensor, num_splits: Optional[Tensor]) -> Tuple[Tensor, Tensor]:
    o, lse = ops.flash_dmla_lse_combine(part_o, part_lse, num_splits, return_lse=True)
    return o, lse


@lse_combine.register_fake
def _(part_o, part_lse, num_splits):
    B, _, H, d = part_o.shape
    return part_o.new_empty((B, H, d), dtype=_BF16), part_o.new_empty((B, H), dtype=_F32)
