"""CPU restatement of the reference's (Flash-)DMLA attention math.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (ds-flashdmla-moe_amd/) imports this
module; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only
as the checker or as the timed CPU baseline.

The reference (yfeng445/ds-flashdmla-moe) ships no DMLA kernel and no Python: its DMLA
semantics exist as README prose (README.md:12-15) plus generic single-head attention kernels
whose math this module restates in PyTorch eager (fp32 by default, fp64 for pinning):

  * exact three-pass softmax of csrc/attention/vanallia_attn.cu:31-82 (row max :33-50,
    row sum :52-69, weighted V :71-82)                                -> attention_exact
  * the online m / l / alpha recurrence and the 1/l guard of csrc/attention/fa_fwd.cu:81-123
    (identical tile update in csrc/attention/fa2_fwd.cu:88-129)        -> attention_online
  * the cache-latent mode (README.md:15): all heads share K_lat and V_lat = K_lat[..., :d_v]
                                                                        -> dmla_fwd_cache_latent
  * the on-the-fly mode (README.md:14): K_lat, V_lat = K WK, V WV per head
                                                                        -> dmla_fwd_onthefly
  * the backward skeleton of csrc/attention/fa2_bwd.cu:198-310 (D = rowsum(dO*O),
    dS = P*(dP - D), dV = P^T dO, dK = dS^T Q, dQ = dS K), with the softmax scale applied to
    dQ/dK (missing at fa2_bwd.cu:251-254, :306-309) and the statistics taken from the forward
    (README.md:12) instead of recomputed                               -> dmla_bwd_cache_latent
  * the same backward in the on-the-fly mode, through the projections K WK, V WV to the
    gradients of K, V, WK and WV (README.md:14 makes WK / WV learnable)
                                                                        -> dmla_bwd_onthefly
  * paged decode (no reference counterpart; benchmark config 3): contiguous attention over the
    tokens gathered through the block table                           -> dmla_decode_paged
  * the paged-cache append that produces those pages and the split-KV LSE combine (no
    reference counterparts)                                           -> kv_append, lse_combine

Conventions the reference leaves open, fixed here and in the kernels alike:
  * causal: key j is masked when j > i + (Sk - Sq) (j > i for Sq == Sk);
  * m = max_j scale*q_i.k_j and l = sum_j exp(scale*q_i.k_j - m) in natural-log units;
    a row with no unmasked key has o = 0, m = -inf, l = 0 (fa_fwd.cu:117-118);
  * WK, WV are [H, d_in, d_lat] and project K[b, s, h, :] @ WK[h].

Every function here is pinned by tests/test_oracle.py against brute-force fp64 loops, a
library routine (torch scaled_dot_product_attention / autograd / gradcheck), closed-form
invariants and the committed golden fixture of config 1.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

Tensor = torch.Tensor


def default_scale(d_qk: int) -> float:
    return 1.0 / math.sqrt(d_qk)


def causal_mask(sq: int, sk: int, device=None) -> Tensor:
    """Boolean [sq, sk] mask, True where key j is masked for query i (j > i + sk - sq)."""
    i = torch.arange(sq, device=device).unsqueeze(1)
    j = torch.arange(sk, device=device).unsqueeze(0)
    return j > i + (sk - sq)


def masked_scores(q: Tensor, k: Tensor, scale: float, causal: bool) -> Tensor:
    """scale * q . k^T with -inf at masked positions; q [..., Sq, D], k [..., Sk, D]."""
    s = scale * torch.matmul(q, k.transpose(-1, -2).contiguous())
    if causal:
        s = s.masked_fill(causal_mask(q.shape[-2], k.shape[-2], q.device), float("-inf"))
    return s


def attention_exact(q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool
                    ) -> Tuple[Tensor, Tensor, Tensor]:
    """Three-pass softmax attention (vanallia_attn.cu:31-82) returning (o, m, l).

    m = row max of the masked scaled scores, l = sum exp(s - m), o = sum exp(s - m) v / l with
    the l > 0 guard of fa_fwd.cu:117-118 (fully masked rows give o = 0, m = -inf, l = 0).
    """
    s = masked_scores(q, k, scale, causal)
    if s.shape[-1] == 0:   # no keys at all: every row is fully masked
        m = torch.full(s.shape[:-1], float("-inf"), dtype=s.dtype, device=s.device)
        return (torch.zeros(s.shape[:-1] + (v.shape[-1],), dtype=s.dtype, device=s.device), m,
                torch.zeros_like(m))
    m = s.amax(dim=-1)
    m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    e = torch.exp(s - m_safe.unsqueeze(-1))
    l = e.sum(dim=-1)
    inv = torch.where(l > 0, 1.0 / l, torch.zeros_like(l))
    o = torch.matmul(e, v) * inv.unsqueeze(-1)
    return o, m, l


def attention_online(q: Tensor, k: Tensor, v: Tensor, scale: float, causal: bool, block: int = 16
                     ) -> Tuple[Tensor, Tensor, Tensor]:
    """Tile-by-tile online softmax with the recurrence of fa_fwd.cu:81-123.

    Per key tile: m_new = max(m_prev, m_tile) (:83); alpha = 0 if m_prev = -inf else
    exp(m_prev - m_new) (:84); l_new = l_prev*alpha + sum exp(s - m_new) (:116);
    O_new = O_prev * (l_prev*alpha/l_new) + (1/l_new) * sum exp(s - m_new) v (:117-136), with
    1/l_new guarded to 0.  O is kept normalised between tiles as in the reference.
    """
    sq, sk = q.shape[-2], k.shape[-2]
    batch = q.shape[:-2]
    m = torch.full(batch + (sq,), float("-inf"), dtype=q.dtype, device=q.device)
    l = torch.zeros(batch + (sq,), dtype=q.dtype, device=q.device)
    o = torch.zeros(batch + (sq, v.shape[-1]), dtype=q.dtype, device=q.device)
    mask = causal_mask(sq, sk, q.device) if causal else None
    for j0 in range(0, sk, block):
        kt, vt = k[..., j0:j0 + block, :], v[..., j0:j0 + block, :]
        s = scale * torch.matmul(q, kt.transpose(-1, -2).contiguous())
        if mask is not None:
            s = s.masked_fill(mask[:, j0:j0 + block], float("-inf"))
        m_tile = s.amax(dim=-1)
        m_new = torch.maximum(m, m_tile)
        alpha = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(m), torch.exp(m - m_new))
        m_new_safe = torch.where(torch.isfinite(m_new), m_new, torch.zeros_like(m_new))
        e = torch.exp(s - m_new_safe.unsqueeze(-1))
        l_new = l * alpha + e.sum(dim=-1)
        inv = torch.where(l_new > 0, 1.0 / l_new, torch.zeros_like(l_new))
        prev = torch.where(l_new > 0, l * alpha * inv, torch.zeros_like(l_new))
        o = o * prev.unsqueeze(-1) + inv.unsqueeze(-1) * torch.matmul(e, vt)
        m, l = m_new, l_new
    return o, m, l


def dmla_fwd_cache_latent(q: Tensor, k_lat: Tensor, d_v: int, scale: Optional[float] = None,
                          causal: bool = True, dtype: torch.dtype = torch.float32
                          ) -> Tuple[Tensor, Tensor, Tensor]:
    """Cache-latent DMLA forward (README.md:15).

    q [B, H, Sq, D], k_lat [B, Sk, D] shared by the H heads, V_lat = k_lat[..., :d_v].
    Returns o [B, H, Sq, d_v], m and l [B, H, Sq] in `dtype`.  Loops over the batch to bound
    the [H, Sq, Sk] score matrix.
    """
    scale = default_scale(q.shape[-1]) if scale is None else scale
    outs, ms, ls = [], [], []
    for b in range(q.shape[0]):
        qb = q[b].to(dtype)
        kb = k_lat[b].to(dtype)
        o, m, l = attention_exact(qb, kb.unsqueeze(0), kb[:, :d_v].unsqueeze(0), scale, causal)
        outs.append(o)
        ms.append(m)
        ls.append(l)
    return torch.stack(outs), torch.stack(ms), torch.stack(ls)


def project_latent(x: Tensor, w: Tensor) -> Tensor:
    """x [B, S, H, d_in] @ w [H, d_in, d_lat] per head -> [B, H, S, d_lat] (README.md:14)."""
    return torch.einsum("bshd,hdl->bhsl", x, w)


def dmla_fwd_onthefly(q: Tensor, k: Tensor, v: Tensor, wk: Tensor, wv: Tensor,
                      scale: Optional[float] = None, causal: bool = True,
                      dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor, Tensor]:
    """On-the-fly DMLA forward: K_lat = K WK, V_lat = V WV per head, then attention.

    q [B, H, Sq, d_lat]; k, v [B, Sk, H, d_in]; wk, wv [H, d_in, d_lat].
    """
    scale = default_scale(q.shape[-1]) if scale is None else scale
    k_lat = project_latent(k.to(dtype), wk.to(dtype))
    v_lat = project_latent(v.to(dtype), wv.to(dtype))
    return attention_exact(q.to(dtype), k_lat, v_lat, scale, causal)


def gather_pages(kv_pool: Tensor, block_table: Tensor, seqlen: int, page_size: int) -> Tensor:
    """The first `seqlen` tokens of one sequence: token t is kv_pool[block_table[t // P], t % P]."""
    n_pages = (seqlen + page_size - 1) // page_size
    pages = block_table[:n_pages].long()
    return kv_pool[pages].reshape(-1, kv_pool.shape[-1])[:seqlen]


def dmla_decode_paged(q: Tensor, kv_pool: Tensor, block_table: Tensor, cache_seqlens: Tensor,
                      d_v: int, scale: Optional[float] = None, dtype: torch.dtype = torch.float32
                      ) -> Tuple[Tensor, Tensor]:
    """Paged decode: q [B, H, D] attends the gathered latent tokens of its sequence (no mask).

    Returns o [B, H, d_v] and lse [B, H] = m + ln(l) (natural log; -inf for empty contexts).
    """
    scale = default_scale(q.shape[-1]) if scale is None else scale
    page_size = kv_pool.shape[1]
    outs, lses = [], []
    for b in range(q.shape[0]):
        kv = gather_pages(kv_pool, block_table[b], int(cache_seqlens[b]), page_size).to(dtype)
        o, m, l = attention_exact(q[b].to(dtype).unsqueeze(1), kv.unsqueeze(0), kv[:, :d_v].unsqueeze(0),
                                  scale, False)
        outs.append(o.squeeze(1))
        lses.append((m + torch.log(l)).squeeze(1))
    return torch.stack(outs), torch.stack(lses)


def decode_plan(cache_seqlens, n_ranges: int, max_pages: int, page_size: int = 64, tile: int = 32,
                seg_cost: int = 10):
    """The decode tile-scheduler plan for R = n_ranges (no reference counterpart).

    The 32-token tiles of all sequences, in order, are cut into R ranges that are equal in a
    weighted space where every nonempty sequence is preceded by seg_cost virtual tiles (the
    fixed cost of a segment): range r starts at weighted position r*W, W = ceil(weighted/R),
    which maps to the tile at that position, or to the sequence's first tile when the position
    is among its virtual tiles.  Returns the int32 list header[8] + tile_prefix[B+1] +
    split_base[B+1] + num_splits[B] + first_range[B] + range_start[R+1] + range_first_b[R]
    with the layout of include/flashdmla.h."""
    B, R = len(cache_seqlens), n_ranges
    tiles = [(min(max(int(x), 0), max_pages * page_size) + tile - 1) // tile for x in cache_seqlens]
    tp = [0]
    for n in tiles:
        tp.append(tp[-1] + n)
    total = tp[-1]
    wstart, ne = [], 0          # weighted start of each sequence
    for b in range(B):
        wstart.append(tp[b] + seg_cost * ne)
        ne += tiles[b] > 0
    weighted = total + seg_cost * ne
    W = max(1, -(-weighted // R))
    rs = []
    for r in range(R):
        pos = r * W
        if pos >= weighted:
            rs.append(total)
            continue
        b = max(i for i in range(B) if wstart[i] <= pos)
        rs.append(min(tp[b] + max(0, pos - wstart[b] - seg_cost), tp[b + 1]))
    rs.append(total)

    def range_of(t):
        return max(r for r in range(R) if rs[r] <= t)

    ns, fr = [], []
    for b in range(B):
        if tiles[b]:
            fr.append(range_of(tp[b]))
            ns.append(range_of(tp[b + 1] - 1) - fr[-1] + 1)
        else:
            fr.append(0)
            ns.append(0)
    sb = [0]
    for n in ns:
        sb.append(sb[-1] + n)
    rfb = [max(b for b in range(B) if tp[b] <= rs[r]) for r in range(R)]
    return [B, R, W, total, sb[-1], seg_cost, 0, 0] + tp + sb + ns + fr + rs + rfb


def decode_ranges(B: int, H: int, max_pages: int, cu_count: int, page_size: int = 64, tile: int = 32,
                  seg_cost: int = 10, max_seg_pages: int = 128) -> int:
    """Range count R of a decode plan (no reference counterpart): one range per CU and group of
    64 heads (a multiple of 8 from 8 on), raised so that a range spans at most
    2*max_seg_pages - 2 tiles when every sequence is full."""
    hg = -(-H // 64)
    r = cu_count // hg
    if r >= 8:
        r -= r % 8
    max_seg_tiles = 2 * max_seg_pages - 2
    weighted_max = B * max_pages * (page_size // tile) + seg_cost * B
    return max(r, -(-weighted_max // max_seg_tiles), 1)


def plan_segment_pages(plan, cache_seqlens, page_size: int = 64, tile: int = 32):
    """Pages spanned by each (range, sequence) segment of a decode plan, as the decode kernel
    walks them: the segment's tiles [s0, s1) of sequence b cover pages s0//2 .. ceil(s1/2)-1."""
    B = len(cache_seqlens)
    R = plan[1]
    tp = plan[8:8 + B + 1]
    rs = plan[8 + 4 * B + 2:8 + 4 * B + 2 + R + 1]
    per = page_size // tile
    out = []
    for r in range(R):
        t0, t1 = rs[r], rs[r + 1]
        for b in range(B):
            s0, s1 = max(t0, tp[b]) - tp[b], min(t1, tp[b + 1]) - tp[b]
            if s0 < s1:
                out.append(-(-s1 // per) - s0 // per)
    return out


def kv_append(kv_pool: Tensor, block_table: Tensor, cache_seqlens: Tensor, new_kv: Tensor,
              new_lens: Optional[Tensor] = None) -> Tensor:
    """Paged KV-cache append (no reference counterpart; the producer side of gather_pages).

    Token t of sequence b's new rows (t < new_lens[b], default all) lands at position
    cache_seqlens[b] + t: page block_table[b, pos // P], row pos % P.  Returns the new pool.
    """
    out = kv_pool.clone()
    page_size = kv_pool.shape[1]
    for b in range(new_kv.shape[0]):
        n = new_kv.shape[1] if new_lens is None else int(new_lens[b])
        for t in range(n):
            pos = int(cache_seqlens[b]) + t
            out[int(block_table[b, pos // page_size]), pos % page_size] = new_kv[b, t]
    return out


def lse_combine(part_o: Tensor, part_lse: Tensor, num_splits: Optional[Tensor] = None,
                dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """Merges split-KV partials: part_o [B, S, H, D] (each normalised over its split's keys),
    part_lse [B, S, H] natural log.  o = sum_s w_s o_s / sum_s w_s with w_s = exp(lse_s - max),
    lse = max + log(sum_s w_s); splits >= num_splits[b] are ignored; no finite lse -> o = 0,
    lse = -inf; a NaN lse -> o and lse NaN.  The combine of split-KV decoding (no reference
    counterpart)."""
    B, S = part_o.shape[0], part_o.shape[1]
    po, pl = part_o.to(dtype), part_lse.to(dtype)
    if num_splits is not None:
        valid = torch.arange(S).view(1, S, 1) < num_splits.view(B, 1, 1).to(torch.long)
        pl = torch.where(valid, pl, torch.full_like(pl, float("-inf")))
    mx = pl.amax(dim=1)
    ref = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
    w = torch.exp(pl - ref.unsqueeze(1))
    wsum = w.sum(dim=1)
    # an empty split (lse -inf) contributes nothing whatever its o holds; NaN propagates
    contrib = torch.where(torch.isneginf(pl).unsqueeze(-1), torch.zeros_like(po), w.unsqueeze(-1) * po)
    den = torch.where(wsum > 0, wsum, torch.ones_like(wsum))
    o = contrib.sum(dim=1) / den.unsqueeze(-1)
    lse = torch.where(wsum > 0, ref + torch.log(den), mx)
    bad = torch.isnan(pl).any(dim=1)
    o = torch.where(bad.unsqueeze(-1), torch.full_like(o, float("nan")), o)
    lse = torch.where(bad, torch.full_like(lse, float("nan")), lse)
    return o, lse


def dmla_bwd_cache_latent(q: Tensor, k_lat: Tensor, o: Tensor, do: Tensor, m: Tensor, l: Tensor,
                          d_v: int, scale: Optional[float] = None, causal: bool = True,
                          dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor]:
    """Cache-latent DMLA backward from the saved statistics (fa2_bwd.cu:198-310, corrected).

    P = exp(scale*q.k - m) / l, D = rowsum(dO * O), dP = dO V^T, dS = P * (dP - D),
    dQ = scale dS K, dK = scale sum_h dS^T Q, dV = sum_h P^T dO, dK_lat = dK + [dV, 0].
    Returns (dq [B, H, Sq, D], dk_lat [B, Sk, D]) in `dtype`.
    """
    scale = default_scale(q.shape[-1]) if scale is None else scale
    dqs, dks = [], []
    for b in range(q.shape[0]):
        qb, kb = q[b].to(dtype), k_lat[b].to(dtype)
        ob, dob = o[b].to(dtype), do[b].to(dtype)
        mb, lb = m[b].to(dtype), l[b].to(dtype)
        s = masked_scores(qb, kb.unsqueeze(0), scale, causal)
        m_safe = torch.where(torch.isfinite(mb), mb, torch.zeros_like(mb))
        inv_l = torch.where(lb > 0, 1.0 / lb, torch.zeros_like(lb))
        p = torch.exp(s - m_safe.unsqueeze(-1)) * inv_l.unsqueeze(-1)
        v = kb[:, :d_v]
        delta = (dob * ob).sum(dim=-1)
        dp = torch.matmul(dob, v.t().contiguous())
        ds = p * (dp - delta.unsqueeze(-1))
        dq = scale * torch.matmul(ds, kb)
        dk = scale * torch.matmul(ds.transpose(-1, -2).contiguous(), qb).sum(dim=0)
        dv = torch.matmul(p.transpose(-1, -2).contiguous(), dob).sum(dim=0)
        dk[:, :d_v] += dv
        dqs.append(dq)
        dks.append(dk)
    return torch.stack(dqs), torch.stack(dks)


def dmla_bwd_onthefly(q: Tensor, k: Tensor, v: Tensor, wk: Tensor, wv: Tensor, o: Tensor, do: Tensor,
                      m: Tensor, l: Tensor, scale: Optional[float] = None, causal: bool = True,
                      dtype: torch.dtype = torch.float32) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """On-the-fly DMLA backward from the saved statistics (fa2_bwd.cu:198-310 corrected, plus
    the projection gradients that README.md:14's learnable WK / WV imply).

    K_lat = K WK, V_lat = V WV per head; P = exp(scale*q.K_lat - m) / l, D = rowsum(dO * O),
    dS = P * (dP - D) with dP = dO V_lat^T; dQ = scale dS K_lat, dK_lat = scale dS^T Q,
    dV_lat = P^T dO; dK[b,s,h] = dK_lat[b,h,s] WK[h]^T, dWK[h] = sum_{b,s} K[b,s,h]^T dK_lat[b,h,s]
    (same for V / WV).  Returns (dq, dk, dv, dwk, dwv) in `dtype`.
    """
    scale = default_scale(q.shape[-1]) if scale is None else scale
    q, k, v, wk, wv = (t.to(dtype) for t in (q, k, v, wk, wv))
    o, do, m, l = o.to(dtype), do.to(dtype), m.to(dtype), l.to(dtype)
    k_lat, v_lat = project_latent(k, wk), project_latent(v, wv)            # [B, H, Sk, d_lat]
    s = masked_scores(q, k_lat, scale, causal)
    m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    inv_l = torch.where(l > 0, 1.0 / l, torch.zeros_like(l))
    p = torch.exp(s - m_safe.unsqueeze(-1)) * inv_l.unsqueeze(-1)
    delta = (do * o).sum(dim=-1)
    dp = torch.matmul(do, v_lat.transpose(-1, -2).contiguous())
    ds = p * (dp - delta.unsqueeze(-1))
    dq = scale * torch.matmul(ds, k_lat)
    dk_lat = scale * torch.matmul(ds.transpose(-1, -2).contiguous(), q)
    dv_lat = torch.matmul(p.transpose(-1, -2).contiguous(), do)
    dk = torch.einsum("bhsl,hdl->bshd", dk_lat, wk)
    dv = torch.einsum("bhsl,hdl->bshd", dv_lat, wv)
    dwk = torch.einsum("bshd,bhsl->hdl", k, dk_lat)
    dwv = torch.einsum("bshd,bhsl->hdl", v, dv_lat)
    return dq, dk, dv, dwk, dwv


def dmla_grads_onthefly_autograd(q: Tensor, k: Tensor, v: Tensor, wk: Tensor, wv: Tensor, do: Tensor,
                                 scale: Optional[float] = None, causal: bool = True,
                                 dtype: torch.dtype = torch.float64) -> Tuple[Tensor, ...]:
    """(dq, dk, dv, dwk, dwv) of sum(o * do) by torch.autograd through the exact on-the-fly forward."""
    xs = [t.detach().to(dtype).requires_grad_(True) for t in (q, k, v, wk, wv)]
    o, _, _ = dmla_fwd_onthefly(*xs, scale, causal, dtype)
    (o * do.to(dtype)).sum().backward()
    return tuple(t.grad for t in xs)


def dmla_grads_autograd(q: Tensor, k_lat: Tensor, do: Tensor, d_v: int, scale: Optional[float] = None,
                        causal: bool = True, dtype: torch.dtype = torch.float64) -> Tuple[Tensor, Tensor]:
    """(dq, dk_lat) of sum(o * do) by torch.autograd through the exact forward (library check)."""
    qx = q.detach().to(dtype).requires_grad_(True)
    kx = k_lat.detach().to(dtype).requires_grad_(True)
    o, _, _ = dmla_fwd_cache_latent(qx, kx, d_v, scale, causal, dtype)
    (o * do.to(dtype)).sum().backward()
    return qx.grad, kx.grad
