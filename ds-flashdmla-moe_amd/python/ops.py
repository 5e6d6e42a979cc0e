"""Flash-DMLA operators: ``torch.autograd.Function`` wrappers over the gfx950 HIP kernels.

This is the Python API the reference's README promises ("minimal autograd.Function wrappers",
README.md:25 and the absent python/ops.py of README.md:54-56).  Every op calls
``libflashdmla.so`` through its C ABI on the current HIP stream; there is no CPU or PyTorch
fallback -- a missing library or a non-GPU tensor raises.

Conventions (the reference fixes none of them; see the oracle for the restated math):
  * q [B, H, S, 576] bf16 and a head-shared latent cache k_lat [B, S_k, 576] bf16; V_lat is
    k_lat[..., :d_v] with d_v = 512.
  * softmax_scale defaults to 1/sqrt(d_qk).
  * causal masks key j > i + (S_k - S_q) (bottom-right aligned; j > i when S_q == S_k).
  * m, l are the row max and row sum in natural-log units of the scaled scores
    (m = max_j scale*q.k_j, l = sum_j exp(scale*q.k_j - m)), as in fa_fwd.cu:81-123.
"""
from __future__ import annotations

import ctypes
import functools
import math
from typing import Optional, Tuple

import torch

from . import _lib

D_QK = 576
D_V = 512
PAGE_SIZE = 64


def _stream(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _check_bf16(name: str, t: torch.Tensor, ndim: int) -> None:
    _require(isinstance(t, torch.Tensor), f"{name} must be a tensor")
    _require(t.is_cuda, f"{name} must be a GPU tensor (the HIP kernels have no CPU path)")
    _require(t.dtype == torch.bfloat16, f"{name} must be bfloat16, got {t.dtype}")
    _require(t.dim() == ndim, f"{name} must have {ndim} dims, got shape {tuple(t.shape)}")
    _require(t.stride(-1) == 1, f"{name} must be contiguous in its last dim")


def _same_device(**tensors: Optional[torch.Tensor]) -> None:
    """Raises unless every given tensor lives on one device (the kernels read them all there)."""
    devs = {name: t.device for name, t in tensors.items() if t is not None}
    _require(len(set(devs.values())) <= 1, "tensors must be on one device, got " +
             ", ".join(f"{n} on {d}" for n, d in devs.items()))


def _check_fp16_range(name: str, t: torch.Tensor) -> None:
    """Raises unless every entry of t is finite and inside fp16's range (|x| <= 65504): the
    kernels convert these operands to fp16, which saturates beyond it.  One device sync."""
    if t.numel() == 0:
        return
    _require(bool(torch.isfinite(t).all()) and float(t.abs().max()) <= 65504.0,
             f"{name} has entries outside fp16's finite range (|x| <= 65504)")


def _check_latent_range(name: str, x: torch.Tensor, w: torch.Tensor, mul: float) -> None:
    """Raises unless the on-the-fly projection x[b, s, h, :] @ w[h] * mul stays inside fp16's
    range for every row, by the bound max_s sum_i |x[.., s, h, i]| * max |w[h]| * mul: the dQ
    kernel of the on-the-fly backward stores K_lat * scale * log2(e) and V_lat in fp16.  One
    device sync."""
    if x.numel() == 0:
        return
    row_l1 = x.float().abs().sum(dim=-1).amax(dim=(0, 1))          # [H]
    w_max = w.float().abs().amax(dim=(1, 2))                        # [H]
    bound = float((row_l1 * w_max).max()) * mul
    _require(math.isfinite(bound) and bound <= 65504.0,
             f"{name}'s projection may leave fp16's finite range (bound {bound:.4g} > 65504)")


def _on_tensor_device(fn):
    """Runs an op with the device of its first GPU tensor argument current.  The library sizes
    its work and workspace, finds its static scratch and launches on the current device, so
    that must be the device the tensors live on (what a device guard does in a PyTorch
    extension); with one GPU this changes nothing."""
    @functools.wraps(fn)
    def wrapped(*args, **kwargs):
        for a in (*args, *kwargs.values()):
            if isinstance(a, torch.Tensor) and a.is_cuda:
                with torch.cuda.device(a.device):
                    return fn(*args, **kwargs)
        return fn(*args, **kwargs)
    return wrapped


def _scale(softmax_scale: Optional[float], d_qk: int) -> float:
    return float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(d_qk)


@_on_tensor_device
def flash_dmla_fwd(
    q: torch.Tensor,
    k_lat: torch.Tensor,
    d_v: int = D_V,
    softmax_scale: Optional[float] = None,
    causal: bool = True,
    return_stats: bool = True,
) -> Tuple[torch.Tensor, Optional[torch.Tensor], Optional[torch.Tensor]]:
    """Cache-latent DMLA forward: returns (o [B,H,Sq,d_v] bf16, m, l [B,H,Sq] fp32).

    o[b,h,i] = softmax(scale * q[b,h,i] . k_lat[b]^T (+ causal mask)) . k_lat[b][:, :d_v].
    """
    _check_bf16("q", q, 4)
    _check_bf16("k_lat", k_lat, 3)
    B, H, Sq, Dqk = q.shape
    _require(k_lat.shape[0] == B and k_lat.shape[2] == Dqk,
             f"k_lat shape {tuple(k_lat.shape)} does not match q {tuple(q.shape)}")
    _same_device(q=q, k_lat=k_lat)
    Sk = k_lat.shape[1]
    o = torch.empty((B, H, Sq, d_v), dtype=torch.bfloat16, device=q.device)
    m = l = None
    if return_stats:
        m = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
        l = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
    _lib.call(
        "dmla_fwd_cache_latent",
        _ptr(q), _ptr(k_lat), _ptr(o), _ptr(m), _ptr(l),
        B, H, Sq, Sk, Dqk, d_v,
        q.stride(0), q.stride(1), q.stride(2),
        k_lat.stride(0), k_lat.stride(1),
        o.stride(0), o.stride(1), o.stride(2),
        _scale(softmax_scale, Dqk), 1 if causal else 0, _stream(q),
    )
    return o, m, l


@_on_tensor_device
def flash_dmla_fwd_onthefly(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    wk: torch.Tensor,
    wv: torch.Tensor,
    softmax_scale: Optional[float] = None,
    causal: bool = True,
    return_stats: bool = False,
    check_range: bool = False,
):
    """On-the-fly DMLA forward: K_lat = K WK and V_lat = V WV per head inside the kernel.

    q [B, H, Sq, 64]; k, v [B, Sk, H, 128]; wk, wv [H, 128, 64] (all bf16).  Returns o
    [B, H, Sq, 64] bf16, or (o, m, l) with return_stats.  softmax_scale defaults to 1/sqrt(64).
    The scores take q as given (bf16) against K_lat * scale * log2(e) kept as a bf16 hi + lo
    pair; V_lat and P enter the PV product as fp16 (V_lat saturates beyond 65504).  Inputs must
    be finite.  check_range=True verifies on the host (one device sync) that q, k, v, wk, wv
    are finite and within fp16's range (the backward converts all of them to fp16).
    """
    _check_bf16("q", q, 4)
    for name, t in (("k", k), ("v", v)):
        _check_bf16(name, t, 4)
    for name, t in (("wk", wk), ("wv", wv)):
        _check_bf16(name, t, 3)
    B, H, Sq, Dl = q.shape
    Sk, Din = k.shape[1], k.shape[3]
    _require(tuple(k.shape) == (B, Sk, H, Din) and tuple(v.shape) == (B, Sk, H, Din),
             "k and v must both be [B, Sk, H, d_in] with q's B and H")
    _require(tuple(wk.shape) == (H, Din, Dl) and tuple(wv.shape) == (H, Din, Dl),
             "wk and wv must be [H, d_in, d_lat]")
    _require(wk.stride() == wv.stride(), "wk and wv must share strides")
    _same_device(q=q, k=k, v=v, wk=wk, wv=wv)
    if check_range:
        for name, t in (("q", q), ("k", k), ("v", v), ("wk", wk), ("wv", wv)):
            _check_fp16_range(name, t)
    o = torch.empty((B, H, Sq, Dl), dtype=torch.bfloat16, device=q.device)
    m = l = None
    if return_stats:
        m = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
        l = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device)
    _lib.call(
        "dmla_fwd_onthefly",
        _ptr(q), _ptr(k), _ptr(v), _ptr(wk), _ptr(wv), _ptr(o), _ptr(m), _ptr(l),
        B, H, Sq, Sk, Din, Dl,
        q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2), wk.stride(0), wk.stride(1),
        o.stride(0), o.stride(1), o.stride(2),
        _scale(softmax_scale, Dl), 1 if causal else 0, _stream(q),
    )
    return (o, m, l) if return_stats else o


@_on_tensor_device
def flash_dmla_decode_plan(cache_seqlens: torch.Tensor, num_heads: int, max_pages: int) -> torch.Tensor:
    """Decode tile-scheduler plan (int32 tensor) for this batch on the current device.

    It depends on cache_seqlens only, so one plan serves every layer of a decode step: pass it
    to flash_dmla_decode_paged(..., plan=plan).  Layout in include/flashdmla.h.
    """
    _require(cache_seqlens.dtype == torch.int32 and cache_seqlens.dim() == 1 and cache_seqlens.is_cuda
             and cache_seqlens.is_contiguous(), "cache_seqlens must be a contiguous 1-D int32 GPU tensor")
    B = cache_seqlens.shape[0]
    nbytes = int(_lib.lib().dmla_decode_plan_bytes(B, num_heads, max_pages))
    _require(nbytes > 0, "decode plan: B, num_heads and max_pages must be positive")
    plan = torch.empty((nbytes // 4,), dtype=torch.int32, device=cache_seqlens.device)
    _lib.call("dmla_decode_plan", _ptr(cache_seqlens), B, num_heads, max_pages, _ptr(plan), nbytes,
              _stream(cache_seqlens))
    return plan


@_on_tensor_device
def flash_dmla_decode_paged(
    q: torch.Tensor,
    kv_pool: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    d_v: int = D_V,
    softmax_scale: Optional[float] = None,
    return_lse: bool = False,
    check_indices: bool = False,
    plan: Optional[torch.Tensor] = None,
):
    """Paged-KV DMLA decode for one query token per sequence.

    q [B, H, 576] bf16; kv_pool [num_pages, 64, 576] bf16; block_table [B, max_pages] int32;
    cache_seqlens [B] int32.  Returns o [B, H, d_v] bf16 (and lse [B, H] fp32 natural log when
    return_lse).  Token t of sequence b is kv_pool[block_table[b, t // 64], t % 64].
    check_indices=True validates the table and lengths on the host (one device sync) and raises
    instead of producing NaN rows for out-of-range pages.  plan: a flash_dmla_decode_plan of
    the same cache_seqlens, H and max_pages (computed here when None).
    """
    _check_bf16("q", q, 3)
    _check_bf16("kv_pool", kv_pool, 3)
    _require(block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.is_cuda,
             "block_table must be a 2-D int32 GPU tensor")
    _require(block_table.stride(1) == 1, "block_table must be contiguous in its last dim")
    _require(cache_seqlens.dtype == torch.int32 and cache_seqlens.dim() == 1 and cache_seqlens.is_cuda,
             "cache_seqlens must be a 1-D int32 GPU tensor")
    _require(cache_seqlens.is_contiguous(), "cache_seqlens must be contiguous")
    B, H, Dqk = q.shape
    num_pages, page, Dk = kv_pool.shape
    _require(Dk == Dqk, f"kv_pool last dim {Dk} != q last dim {Dqk}")
    _require(page == PAGE_SIZE, f"page size must be {PAGE_SIZE}, got {page}")
    _require(block_table.shape[0] == B and cache_seqlens.shape[0] == B, "batch size mismatch")
    _same_device(q=q, kv_pool=kv_pool, block_table=block_table, cache_seqlens=cache_seqlens, plan=plan)
    max_pages = block_table.shape[1]
    if check_indices:
        bt = block_table.cpu()
        sl = cache_seqlens.cpu()
        _require(bool((sl >= 0).all()), "cache_seqlens must be >= 0")
        _require(int(sl.max()) <= max_pages * PAGE_SIZE if B else True,
                 "a cache_seqlens entry exceeds the block table capacity")
        for b in range(B):
            n = (int(sl[b]) + PAGE_SIZE - 1) // PAGE_SIZE
            used = bt[b, :n]
            _require(bool(((used >= 0) & (used < num_pages)).all()),
                     f"block_table row {b} holds a page index outside [0, {num_pages})")
    o = torch.empty((B, H, d_v), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, H), dtype=torch.float32, device=q.device) if return_lse else None
    ws_bytes = int(_lib.lib().dmla_decode_workspace_bytes(B, H, d_v, max_pages))
    if plan is None:
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
        _lib.call(
            "dmla_decode_paged",
            _ptr(q), _ptr(kv_pool), _ptr(block_table), _ptr(cache_seqlens), _ptr(o), _ptr(lse),
            B, H, Dqk, d_v, page, num_pages, max_pages,
            q.stride(0), q.stride(1), kv_pool.stride(0), kv_pool.stride(1), block_table.stride(0),
            o.stride(0), o.stride(1),
            _scale(softmax_scale, Dqk), _ptr(ws), ws_bytes, _stream(q),
        )
    else:
        plan_bytes = int(_lib.lib().dmla_decode_plan_bytes(B, H, max_pages))
        _require(plan.dtype == torch.int32 and plan.is_cuda and plan.is_contiguous()
                 and plan.numel() * 4 >= plan_bytes, "plan must come from flash_dmla_decode_plan for this batch")
        ws_bytes -= plan_bytes
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
        _lib.call(
            "dmla_decode_paged_planned",
            _ptr(q), _ptr(kv_pool), _ptr(block_table), _ptr(cache_seqlens), _ptr(o), _ptr(lse),
            B, H, Dqk, d_v, page, num_pages, max_pages,
            q.stride(0), q.stride(1), kv_pool.stride(0), kv_pool.stride(1), block_table.stride(0),
            o.stride(0), o.stride(1),
            _scale(softmax_scale, Dqk), _ptr(plan), _ptr(ws), ws_bytes, _stream(q),
        )
    return (o, lse) if return_lse else o


@_on_tensor_device
def flash_dmla_kv_append(
    kv_pool: torch.Tensor,
    block_table: torch.Tensor,
    cache_seqlens: torch.Tensor,
    new_kv: torch.Tensor,
    new_lens: Optional[torch.Tensor] = None,
    check_indices: bool = False,
) -> None:
    """Writes new latent rows into the paged cache in place (the producer of decode's pages).

    kv_pool [num_pages, P, d] bf16; block_table [B, max_pages] int32; cache_seqlens [B] int32
    (rows already cached; not updated); new_kv [B, n_new, d] bf16; new_lens [B] int32 or None.
    Row t of sequence b lands at position cache_seqlens[b] + t.  Rows whose page slot or page
    index is out of range are skipped; check_indices=True raises afterwards (one device sync).
    """
    _check_bf16("kv_pool", kv_pool, 3)
    _check_bf16("new_kv", new_kv, 3)
    for name, t, nd in (("block_table", block_table, 2), ("cache_seqlens", cache_seqlens, 1)):
        _require(t.dtype == torch.int32 and t.dim() == nd and t.is_cuda, f"{name} must be a {nd}-D int32 GPU tensor")
    _require(block_table.stride(-1) == 1 and cache_seqlens.is_contiguous(), "index tensors must be contiguous")
    B, n_new, d = new_kv.shape
    num_pages, P, dk = kv_pool.shape
    _require(dk == d, "kv_pool and new_kv row widths differ")
    _require(block_table.shape[0] == B and cache_seqlens.shape[0] == B, "batch size mismatch")
    _same_device(kv_pool=kv_pool, block_table=block_table, cache_seqlens=cache_seqlens, new_kv=new_kv,
                 new_lens=new_lens)
    if new_lens is not None:
        _require(new_lens.dtype == torch.int32 and new_lens.dim() == 1 and new_lens.is_cuda and new_lens.is_contiguous()
                 and new_lens.shape[0] == B, "new_lens must be a contiguous [B] int32 GPU tensor")
    flag = torch.zeros(1, dtype=torch.int32, device=kv_pool.device) if check_indices else None
    _lib.call(
        "dmla_kv_append",
        _ptr(kv_pool), _ptr(block_table), _ptr(cache_seqlens), _ptr(new_lens), _ptr(new_kv), _ptr(flag),
        B, n_new, d, P, num_pages, block_table.shape[1],
        kv_pool.stride(0), kv_pool.stride(1), block_table.stride(0), new_kv.stride(0), new_kv.stride(1),
        _stream(kv_pool),
    )
    if check_indices:
        _require(int(flag.item()) == 0, "kv append: a row's page slot or page index was out of range (row skipped)")


@_on_tensor_device
def flash_dmla_lse_combine(
    part_o: torch.Tensor,
    part_lse: torch.Tensor,
    num_splits: Optional[torch.Tensor] = None,
    return_lse: bool = False,
):
    """Merges split-KV partials: part_o [B, S, H, d] fp32 (each normalised over its split),
    part_lse [B, S, H] fp32 natural log, num_splits [B] int32 or None (all S).  Returns
    o [B, H, d] bf16 (and lse [B, H] fp32 with return_lse)."""
    _require(part_o.dtype == torch.float32 and part_o.is_cuda and part_o.dim() == 4 and part_o.stride(-1) == 1,
             "part_o must be a [B, S, H, d] float32 GPU tensor, contiguous in d")
    B, S, H, d = part_o.shape
    _require(part_lse.dtype == torch.float32 and part_lse.is_cuda and tuple(part_lse.shape) == (B, S, H),
             "part_lse must be a [B, S, H] float32 GPU tensor")
    if num_splits is not None:
        _require(num_splits.dtype == torch.int32 and num_splits.is_cuda and num_splits.is_contiguous()
                 and tuple(num_splits.shape) == (B,), "num_splits must be a contiguous [B] int32 GPU tensor")
    _same_device(part_o=part_o, part_lse=part_lse, num_splits=num_splits)
    o = torch.empty((B, H, d), dtype=torch.bfloat16, device=part_o.device)
    lse = torch.empty((B, H), dtype=torch.float32, device=part_o.device) if return_lse else None
    _lib.call(
        "dmla_lse_combine",
        _ptr(part_o), _ptr(part_lse), _ptr(num_splits), _ptr(o), _ptr(lse), B, H, S, d,
        part_o.stride(0), part_o.stride(1), part_o.stride(2), part_lse.stride(0), part_lse.stride(1),
        part_lse.stride(2), o.stride(0), o.stride(1), _stream(part_o),
    )
    return (o, lse) if return_lse else o


class FlashDMLACacheLatent(torch.autograd.Function):
    """o = FlashDMLACacheLatent.apply(q, k_lat, d_v, softmax_scale, causal).

    Saves (q, k_lat, o, m, l) for the backward, which reuses the row statistics instead of
    recomputing them (README.md:12).
    """

    @staticmethod
    def forward(ctx, q, k_lat, d_v=D_V, softmax_scale=None, causal=True):
        o, m, l = flash_dmla_fwd(q, k_lat, d_v, softmax_scale, causal, return_stats=True)
        ctx.save_for_backward(q, k_lat, o, m, l)
        ctx.d_v = d_v
        ctx.softmax_scale = softmax_scale
        ctx.causal = causal
        return o

    @staticmethod
    def backward(ctx, do):
        q, k_lat, o, m, l = ctx.saved_tensors
        dq, dk_lat = flash_dmla_bwd(q, k_lat, o, do.to(torch.bfloat16).contiguous(), m, l, ctx.d_v,
                                    ctx.softmax_scale, ctx.causal)
        return dq, dk_lat.to(k_lat.dtype), None, None, None


@_on_tensor_device
def flash_dmla_bwd(
    q: torch.Tensor,
    k_lat: torch.Tensor,
    o: torch.Tensor,
    do: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    d_v: int = D_V,
    softmax_scale: Optional[float] = None,
    causal: bool = True,
    dq_dtype: Optional[torch.dtype] = None,
    dk_dtype: torch.dtype = torch.float32,
    check_range: bool = False,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Cache-latent DMLA backward from the saved statistics: returns (dq, dk_lat).

    dq [B, H, Sq, 576] (dq_dtype, default q.dtype) and dk_lat [B, Sk, 576] (dk_dtype, default
    float32: dk_lat sums P^T dO and dS^T q over every head and position, so its large entries
    would lose more to a bf16 rounding than the accumulation itself does).  dk_lat already holds
    the V_lat gradient in its first d_v columns.  m, l must be the forward's statistics.
    The second-stage products (dS^T q, P^T dO, dS K) run on fp16 operands, with q, dO and
    k_lat converted exactly; check_range=True verifies on the host (one device sync) that they
    stay inside fp16's range instead of saturating.
    """
    _check_bf16("q", q, 4)
    _check_bf16("k_lat", k_lat, 3)
    _check_bf16("o", o, 4)
    _check_bf16("do", do, 4)
    B, H, Sq, Dqk = q.shape
    Sk = k_lat.shape[1]
    _require(k_lat.shape[0] == B and k_lat.shape[2] == Dqk, "k_lat shape does not match q")
    _require(tuple(o.shape) == (B, H, Sq, d_v), f"o must be [B, H, Sq, {d_v}]")
    _require(tuple(do.shape) == (B, H, Sq, d_v), f"do must be [B, H, Sq, {d_v}]")
    for name, t in (("m", m), ("l", l)):
        _require(t.dtype == torch.float32 and t.is_cuda and t.is_contiguous() and tuple(t.shape) == (B, H, Sq),
                 f"{name} must be a contiguous float32 GPU tensor [B, H, Sq]")
    _same_device(q=q, k_lat=k_lat, o=o, do=do, m=m, l=l)
    if check_range:
        for name, t in (("q", q), ("k_lat", k_lat), ("do", do)):
            _check_fp16_range(name, t)
    dq_dtype = q.dtype if dq_dtype is None else dq_dtype
    _require(dq_dtype in (torch.bfloat16, torch.float32) and dk_dtype in (torch.bfloat16, torch.float32),
             "gradient dtypes must be bfloat16 or float32")
    dq = torch.empty((B, H, Sq, Dqk), dtype=dq_dtype, device=q.device)
    dk = torch.empty((B, Sk, Dqk), dtype=dk_dtype, device=q.device)
    ws_bytes = int(_lib.lib().dmla_bwd_workspace_bytes(B, H, Sq, Sk, Dqk, d_v, 1 if causal else 0))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    _lib.call(
        "dmla_bwd_cache_latent",
        _ptr(q), _ptr(k_lat), _ptr(o), _ptr(do), _ptr(m), _ptr(l), _ptr(dq), _ptr(dk),
        B, H, Sq, Sk, Dqk, d_v,
        q.stride(0), q.stride(1), q.stride(2), k_lat.stride(0), k_lat.stride(1),
        o.stride(0), o.stride(1), o.stride(2), do.stride(0), do.stride(1), do.stride(2),
        dq.stride(0), dq.stride(1), dq.stride(2), dk.stride(0), dk.stride(1),
        1 if dq_dtype == torch.float32 else 0, 1 if dk_dtype == torch.float32 else 0,
        _scale(softmax_scale, Dqk), 1 if causal else 0, _ptr(ws), ws_bytes, _stream(q),
    )
    return dq, dk


@_on_tensor_device
def flash_dmla_bwd_onthefly(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    wk: torch.Tensor,
    wv: torch.Tensor,
    o: torch.Tensor,
    do: torch.Tensor,
    m: torch.Tensor,
    l: torch.Tensor,
    softmax_scale: Optional[float] = None,
    causal: bool = True,
    dw_dtype: torch.dtype = torch.float32,
    check_range: bool = False,
    dq_dtype: Optional[torch.dtype] = None,
    dkv_dtype: Optional[torch.dtype] = None,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """On-the-fly DMLA backward from the saved statistics: returns (dq, dk, dv, dwk, dwv).

    Shapes as for flash_dmla_fwd_onthefly; dq [B, H, Sq, 64] in dq_dtype (default q.dtype),
    dk and dv [B, Sk, H, 128] in dkv_dtype (default k.dtype); dwk and dwv [H, 128, 64] in
    dw_dtype (default float32: they sum over every batch element and position, and at config-4
    sizes reach ~30, where a bf16 rounding alone is 0.06).  Each may be bfloat16 or float32.
    m, l must be the forward's statistics (return_stats=True).
    The dk / dv / weight side runs on bf16 operands, every rounded intermediate carried as a
    bf16 pair hi + lo; dq runs on fp16 operands (q, do converted exactly, K_lat * scale *
    log2(e) and V_lat rounded to fp16).  check_range=True verifies on the host (one device sync)
    that q and do, and a bound of those projections, stay inside fp16's range.
    """
    _check_bf16("q", q, 4)
    _check_bf16("o", o, 4)
    _check_bf16("do", do, 4)
    for name, t in (("k", k), ("v", v)):
        _check_bf16(name, t, 4)
    for name, t in (("wk", wk), ("wv", wv)):
        _check_bf16(name, t, 3)
    B, H, Sq, Dl = q.shape
    Sk, Din = k.shape[1], k.shape[3]
    _require(tuple(k.shape) == (B, Sk, H, Din) and tuple(v.shape) == (B, Sk, H, Din),
             "k and v must both be [B, Sk, H, d_in] with q's B and H")
    _require(tuple(wk.shape) == (H, Din, Dl) and tuple(wv.shape) == (H, Din, Dl),
             "wk and wv must be [H, d_in, d_lat]")
    _require(wk.stride() == wv.stride(), "wk and wv must share strides")
    _require(tuple(o.shape) == (B, H, Sq, Dl) and tuple(do.shape) == (B, H, Sq, Dl), "o and do must be [B, H, Sq, d_lat]")
    for name, t in (("m", m), ("l", l)):
        _require(t.dtype == torch.float32 and t.is_cuda and t.is_contiguous() and tuple(t.shape) == (B, H, Sq),
                 f"{name} must be a contiguous float32 GPU tensor [B, H, Sq]")
    _same_device(q=q, k=k, v=v, wk=wk, wv=wv, o=o, do=do, m=m, l=l)
    scale = _scale(softmax_scale, Dl)
    if check_range:
        for name, t in (("q", q), ("do", do)):
            _check_fp16_range(name, t)
        _check_latent_range("k", k, wk, scale / math.log(2.0))
        _check_latent_range("v", v, wv, 1.0)
    dq_dtype = q.dtype if dq_dtype is None else dq_dtype
    dkv_dtype = k.dtype if dkv_dtype is None else dkv_dtype
    _require(all(t in (torch.bfloat16, torch.float32) for t in (dq_dtype, dkv_dtype, dw_dtype)),
             "gradient dtypes must be bfloat16 or float32")
    dq = torch.empty((B, H, Sq, Dl), dtype=dq_dtype, device=q.device)
    dk = torch.empty((B, Sk, H, Din), dtype=dkv_dtype, device=q.device)
    dv = torch.empty_like(dk)
    dwk = torch.empty((H, Din, Dl), dtype=dw_dtype, device=q.device)
    dwv = torch.empty_like(dwk)
    if B * H == 0:
        return dq, dk, dv, dwk, dwv
    if Sq == 0 or Sk == 0:   # nothing attends: every gradient is zero
        return dq.zero_(), dk.zero_(), dv.zero_(), dwk.zero_(), dwv.zero_()
    ws_bytes = int(_lib.lib().dmla_bwd_onthefly_workspace_bytes(B, H, Sq, Sk, Din, Dl))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=q.device)
    _lib.call(
        "dmla_bwd_onthefly",
        _ptr(q), _ptr(k), _ptr(v), _ptr(wk), _ptr(wv), _ptr(o), _ptr(do), _ptr(m), _ptr(l),
        _ptr(dq), _ptr(dk), _ptr(dv), _ptr(dwk), _ptr(dwv),
        B, H, Sq, Sk, Din, Dl,
        q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2), wk.stride(0), wk.stride(1),
        o.stride(0), o.stride(1), o.stride(2), do.stride(0), do.stride(1), do.stride(2),
        dq.stride(0), dq.stride(1), dq.stride(2), dk.stride(0), dk.stride(1), dk.stride(2),
        dwk.stride(0), dwk.stride(1), 1 if dq_dtype == torch.float32 else 0,
        1 if dkv_dtype == torch.float32 else 0, 1 if dw_dtype == torch.float32 else 0,
        scale, 1 if causal else 0, _ptr(ws), ws_bytes, _stream(q),
    )
    return dq, dk, dv, dwk, dwv


class FlashDMLAOnTheFly(torch.autograd.Function):
    """o = FlashDMLAOnTheFly.apply(q, k, v, wk, wv, softmax_scale, causal).

    Saves q, k, v, wk, wv, o and the row statistics m, l; backward(do) returns the gradients
    of q, k, v, wk and wv (flash_dmla_bwd_onthefly; the weight gradients are summed in fp32 and
    cast to the weights' dtype by autograd).
    """

    @staticmethod
    def forward(ctx, q, k, v, wk, wv, softmax_scale=None, causal=True):
        o, m, l = flash_dmla_fwd_onthefly(q, k, v, wk, wv, softmax_scale, causal, return_stats=True)
        ctx.save_for_backward(q, k, v, wk, wv, o, m, l)
        ctx.softmax_scale = softmax_scale
        ctx.causal = causal
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, wk, wv, o, m, l = ctx.saved_tensors
        dq, dk, dv, dwk, dwv = flash_dmla_bwd_onthefly(q, k, v, wk, wv, o, do.contiguous(), m, l,
                                                       ctx.softmax_scale, ctx.causal)
        return dq, dk, dv, dwk, dwv, None, None


def flash_dmla(q, k_lat, d_v=D_V, softmax_scale=None, causal=True):
    """Differentiable cache-latent DMLA attention (functional form of FlashDMLACacheLatent)."""
    return FlashDMLACacheLatent.apply(q, k_lat, d_v, softmax_scale, causal)


def flash_dmla_onthefly(q, k, v, wk, wv, softmax_scale=None, causal=True):
    """Differentiable on-the-fly DMLA attention (functional form of FlashDMLAOnTheFly)."""
    return FlashDMLAOnTheFly.apply(q, k, v, wk, wv, softmax_scale, causal)
