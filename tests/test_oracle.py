"""Pins the CPU oracle (oracle/dmla_ref.py) before any kernel is compared against it.

Each oracle function is checked against something that does not restate its own formula:
the golden fixture of config 1 (brute-force fp64 row loops + torch.autograd), a library
routine (scaled_dot_product_attention, torch.autograd, gradcheck), closed forms and
invariants.  The planted-mistake tests at the end show that these checks reject plausible
errors (a dropped scale, a wrong V slice, a transposed operand, a missing V-fold).
"""
import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import seeded
from oracle import dmla_ref as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "cfg1_tiny.npz")


def _golden():
    return np.load(GOLDEN, allow_pickle=False)


# ---------------------------------------------------------------- golden fixture (config 1)
def test_golden_forward_cfg1():
    g = _golden()
    q, k = torch.from_numpy(g["q"]), torch.from_numpy(g["k_lat"])
    o, m, l = R.dmla_fwd_cache_latent(q, k, int(g["d_v"]), float(g["scale"]), True, torch.float32)
    np.testing.assert_allclose(o.numpy(), g["o"], atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(m.numpy(), g["m"], atol=2e-6, rtol=1e-6)
    np.testing.assert_allclose(l.numpy(), g["l"], atol=0, rtol=2e-6)


def test_golden_forward_cfg1_fp64_tight():
    g = _golden()
    q, k = torch.from_numpy(g["q"]).double(), torch.from_numpy(g["k_lat"]).double()
    o, m, l = R.dmla_fwd_cache_latent(q, k, 32, 1 / 8, True, torch.float64)
    np.testing.assert_allclose(o.numpy(), g["o"], atol=1e-6, rtol=1e-6)
    np.testing.assert_allclose((m + torch.log(l)).numpy(), g["lse"], atol=1e-6, rtol=0)


def test_golden_backward_cfg1():
    g = _golden()
    q, k, do = (torch.from_numpy(g[n]).double() for n in ("q", "k_lat", "do"))
    o, m, l = R.dmla_fwd_cache_latent(q, k, 32, 1 / 8, True, torch.float64)
    dq, dk = R.dmla_bwd_cache_latent(q, k, o, do, m, l, 32, 1 / 8, True, torch.float64)
    np.testing.assert_allclose(dq.numpy(), g["dq"], atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(dk.numpy(), g["dk_lat"], atol=1e-5, rtol=1e-5)


# ---------------------------------------------------------------- library cross-checks
@pytest.mark.parametrize("sq,sk,causal", [(37, 37, True), (16, 53, True), (29, 41, False)])
def test_forward_matches_sdpa(sq, sk, causal):
    B, H, D, DV = 2, 3, 40, 24
    q = seeded((B, H, sq, D), 1, dtype=torch.float64)
    k = seeded((B, sk, D), 2, dtype=torch.float64)
    scale = 0.3
    o, m, l = R.dmla_fwd_cache_latent(q, k, DV, scale, causal, torch.float64)
    mask = None
    if causal:
        mask = ~R.causal_mask(sq, sk)  # True = attend (bottom-right aligned)
    ref = F.scaled_dot_product_attention(
        q, k.unsqueeze(1).expand(B, H, sk, D), k[..., :DV].unsqueeze(1).expand(B, H, sk, DV),
        attn_mask=mask, scale=scale)
    torch.testing.assert_close(o, ref, atol=1e-12, rtol=1e-12)
    s = scale * torch.einsum("bhid,bjd->bhij", q, k)
    if causal:
        s = s.masked_fill(R.causal_mask(sq, sk), float("-inf"))
    torch.testing.assert_close(m + torch.log(l), torch.logsumexp(s, -1), atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(m, s.amax(-1), atol=0, rtol=0)


def test_backward_matches_autograd_and_gradcheck():
    B, H, S, D, DV = 2, 2, 11, 12, 8
    q = seeded((B, H, S, D), 3, dtype=torch.float64)
    k = seeded((B, S, D), 4, dtype=torch.float64)
    do = seeded((B, H, S, DV), 5, dtype=torch.float64)
    o, m, l = R.dmla_fwd_cache_latent(q, k, DV, 0.4, True, torch.float64)
    dq, dk = R.dmla_bwd_cache_latent(q, k, o, do, m, l, DV, 0.4, True, torch.float64)
    dq2, dk2 = R.dmla_grads_autograd(q, k, do, DV, 0.4, True)
    torch.testing.assert_close(dq, dq2, atol=1e-12, rtol=1e-10)
    torch.testing.assert_close(dk, dk2, atol=1e-12, rtol=1e-10)

    def f(qq, kk):
        return R.dmla_fwd_cache_latent(qq, kk, DV, 0.4, True, torch.float64)[0]

    assert torch.autograd.gradcheck(f, (q[:1, :1, :5].clone().requires_grad_(True),
                                        k[:1, :5].clone().requires_grad_(True)))


def _otf_inputs(B, H, sq, sk, din, dl, seed):
    q = seeded((B, H, sq, dl), seed, dtype=torch.float64)
    k = seeded((B, sk, H, din), seed + 1, dtype=torch.float64)
    v = seeded((B, sk, H, din), seed + 2, dtype=torch.float64)
    wk = seeded((H, din, dl), seed + 3, 0.4, dtype=torch.float64)
    wv = seeded((H, din, dl), seed + 4, 0.4, dtype=torch.float64)
    do = seeded((B, H, sq, dl), seed + 5, dtype=torch.float64)
    return q, k, v, wk, wv, do


@pytest.mark.parametrize("sq,sk,causal", [(9, 13, True), (13, 9, True), (11, 11, False), (7, 16, False)])
def test_onthefly_backward_matches_autograd(sq, sk, causal):
    q, k, v, wk, wv, do = _otf_inputs(2, 3, sq, sk, 10, 6, 40 + sq)
    o, m, l = R.dmla_fwd_onthefly(q, k, v, wk, wv, 0.4, causal, torch.float64)
    got = R.dmla_bwd_onthefly(q, k, v, wk, wv, o, do, m, l, 0.4, causal, torch.float64)
    ref = R.dmla_grads_onthefly_autograd(q, k, v, wk, wv, do, 0.4, causal)
    for name, a, b in zip(("dq", "dk", "dv", "dwk", "dwv"), got, ref):
        assert a.shape == b.shape, name
        torch.testing.assert_close(a, b, atol=1e-12, rtol=1e-10, msg=name)
    if causal and sq > sk:   # rows before the first key see nothing and get no gradient
        assert torch.equal(got[0][:, :, :sq - sk], torch.zeros_like(got[0][:, :, :sq - sk]))


def test_onthefly_backward_gradcheck():
    q, k, v, wk, wv, _ = _otf_inputs(1, 2, 5, 6, 3, 4, 60)

    def f(*xs):
        return R.dmla_fwd_onthefly(*xs, 0.5, True, torch.float64)[0]

    assert torch.autograd.gradcheck(f, tuple(t.clone().requires_grad_(True) for t in (q, k, v, wk, wv)))


# ---------------------------------------------------------------- closed forms / invariants
def test_causal_first_row_is_first_value():
    q = seeded((1, 2, 9, 16), 6, dtype=torch.float64)
    k = seeded((1, 9, 16), 7, dtype=torch.float64)
    o, m, l = R.dmla_fwd_cache_latent(q, k, 8, 0.5, True, torch.float64)
    torch.testing.assert_close(o[0, :, 0], k[0, 0, :8].expand(2, 8), atol=0, rtol=0)
    torch.testing.assert_close(l[0, :, 0], torch.ones(2, dtype=torch.float64))


def test_zero_query_gives_prefix_mean():
    k = seeded((1, 10, 16), 8, dtype=torch.float64)
    q = torch.zeros(1, 3, 10, 16, dtype=torch.float64)
    o, _, l = R.dmla_fwd_cache_latent(q, k, 8, 0.5, True, torch.float64)
    prefix_mean = torch.cumsum(k[0, :, :8], 0) / torch.arange(1, 11, dtype=torch.float64).unsqueeze(1)
    torch.testing.assert_close(o[0, 1], prefix_mean, atol=1e-14, rtol=1e-14)
    torch.testing.assert_close(l[0, 0], torch.arange(1, 11, dtype=torch.float64))


def test_head_permutation_equivariance():
    q = seeded((2, 5, 7, 16), 9, dtype=torch.float64)
    k = seeded((2, 7, 16), 10, dtype=torch.float64)
    perm = torch.tensor([3, 0, 4, 1, 2])
    o, m, l = R.dmla_fwd_cache_latent(q, k, 8, 0.5, True, torch.float64)
    o2, m2, l2 = R.dmla_fwd_cache_latent(q[:, perm], k, 8, 0.5, True, torch.float64)
    torch.testing.assert_close(o2, o[:, perm], atol=0, rtol=0)
    torch.testing.assert_close(l2, l[:, perm], atol=0, rtol=0)


def test_fully_masked_rows_follow_the_guard():
    # Sq > Sk with bottom-right alignment leaves the first Sq - Sk rows without keys.
    q = seeded((1, 1, 6, 8), 11, dtype=torch.float64)
    k = seeded((1, 4, 8), 12, dtype=torch.float64)
    o, m, l = R.dmla_fwd_cache_latent(q, k, 4, 0.5, True, torch.float64)
    assert torch.all(o[0, 0, :2] == 0) and torch.all(l[0, 0, :2] == 0)
    assert torch.all(torch.isinf(m[0, 0, :2])) and torch.all(m[0, 0, :2] < 0)
    assert torch.all(l[0, 0, 2:] > 0)


@pytest.mark.parametrize("block", [1, 5, 16, 64])
def test_online_recurrence_equals_exact(block):
    q = seeded((2, 3, 33, 16), 13, dtype=torch.float64)
    k = seeded((2, 1, 33, 16), 14, dtype=torch.float64)
    v = k[..., :8]
    o, m, l = R.attention_exact(q, k, v, 0.7, True)
    o2, m2, l2 = R.attention_online(q, k, v, 0.7, True, block)
    torch.testing.assert_close(o2, o, atol=1e-13, rtol=1e-12)
    torch.testing.assert_close(m2, m, atol=0, rtol=0)
    torch.testing.assert_close(l2, l, atol=1e-12, rtol=1e-12)


def test_onthefly_is_cache_latent_per_head():
    B, H, S, DIN, DL = 2, 3, 13, 10, 6
    q = seeded((B, H, S, DL), 15, dtype=torch.float64)
    k = seeded((B, S, H, DIN), 16, dtype=torch.float64)
    v = seeded((B, S, H, DIN), 17, dtype=torch.float64)
    wk = seeded((H, DIN, DL), 18, dtype=torch.float64)
    wv = seeded((H, DIN, DL), 19, dtype=torch.float64)
    o, m, l = R.dmla_fwd_onthefly(q, k, v, wk, wv, 0.4, True, torch.float64)
    for h in range(H):
        kl = k[:, :, h] @ wk[h]
        vl = v[:, :, h] @ wv[h]
        ref = F.scaled_dot_product_attention(q[:, h], kl, vl, is_causal=True, scale=0.4)
        torch.testing.assert_close(o[:, h], ref, atol=1e-12, rtol=1e-12)


def test_decode_paged_equals_contiguous_and_ignores_page_order():
    B, H, D, DV, P = 3, 4, 16, 8, 4
    lens = torch.tensor([1, 9, 14], dtype=torch.int32)
    n_pages = [(int(n) + P - 1) // P for n in lens]
    total = sum(n_pages)
    seqs = [seeded((int(n), D), 20 + i, dtype=torch.float64) for i, n in enumerate(lens)]
    q = seeded((B, H, D), 30, dtype=torch.float64)
    for perm_seed in (0, 1):
        perm = torch.randperm(total, generator=torch.Generator().manual_seed(perm_seed))
        pool = torch.full((total, P, D), float("nan"), dtype=torch.float64)  # unused rows are NaN
        table = torch.zeros(B, 4, dtype=torch.int32)
        c = 0
        for b in range(B):
            for j in range(n_pages[b]):
                page = int(perm[c]); c += 1
                table[b, j] = page
                rows = seqs[b][j * P:(j + 1) * P]
                pool[page, :rows.shape[0]] = rows
        o, lse = R.dmla_decode_paged(q, pool, table, lens, DV, 0.5, torch.float64)
        for b in range(B):
            ref, m, l = R.attention_exact(q[b].unsqueeze(1), seqs[b].unsqueeze(0), seqs[b][:, :DV].unsqueeze(0), 0.5, False)
            torch.testing.assert_close(o[b], ref.squeeze(1), atol=1e-14, rtol=1e-13)
            torch.testing.assert_close(lse[b], (m + torch.log(l)).squeeze(1), atol=1e-13, rtol=1e-13)


# ---------------------------------------------------------------- planted mistakes
def _mutant_bwd(q, k, o, do, m, l, d_v, scale, mistake):
    s = R.masked_scores(q[0], k[0].unsqueeze(0), scale, True)
    p = torch.exp(s - m[0].unsqueeze(-1)) / l[0].unsqueeze(-1)
    v = k[0, :, :d_v]
    delta = (do[0] * o[0]).sum(-1)
    dp = do[0] @ v.t()
    ds = p * dp if mistake == "no_delta" else p * (dp - delta.unsqueeze(-1))
    dq_scale = 1.0 if mistake == "dq_no_scale" else scale
    dq = dq_scale * ds @ k[0]
    dk = scale * (ds.transpose(-1, -2) @ q[0]).sum(0)
    if mistake != "no_v_fold":
        dk[:, :d_v] += (p.transpose(-1, -2) @ do[0]).sum(0)
    return dq.unsqueeze(0), dk.unsqueeze(0)


@pytest.mark.parametrize("mistake", ["dq_no_scale", "no_v_fold", "no_delta"])
def test_planted_backward_mistakes_are_caught(mistake):
    g = _golden()
    q, k, do = (torch.from_numpy(g[n]).double() for n in ("q", "k_lat", "do"))
    o, m, l = R.dmla_fwd_cache_latent(q, k, 32, 1 / 8, True, torch.float64)
    dq, dk = _mutant_bwd(q, k, o, do, m, l, 32, 1 / 8, mistake)
    bad = not (np.allclose(dq.numpy(), g["dq"], atol=1e-5) and np.allclose(dk.numpy(), g["dk_lat"], atol=1e-5))
    assert bad, f"golden gradients failed to catch the planted mistake {mistake}"


def _mutant_otf_bwd(q, k, v, wk, wv, o, do, m, l, scale, mistake):
    kl, vl = R.project_latent(k, wk), R.project_latent(v, wv)
    s = R.masked_scores(q, kl, scale, True)
    p = torch.exp(s - m.unsqueeze(-1)) / l.unsqueeze(-1)
    ds = p * (do @ vl.transpose(-1, -2) - (do * o).sum(-1, keepdim=True))
    dkl = (1.0 if mistake == "dk_lat_no_scale" else scale) * ds.transpose(-1, -2) @ q
    dvl = p.transpose(-1, -2) @ do
    dk = torch.einsum("bhsl,hdl->bshd", dkl, wv if mistake == "dk_through_wv" else wk)
    dwk = torch.einsum("bshd,bhsl->hdl", k, dvl if mistake == "dwk_from_dv_lat" else dkl)
    dwv = torch.einsum("bshd,bhsl->hdl", k if mistake == "dwv_from_k" else v, dvl)
    return scale * ds @ kl, dk, torch.einsum("bhsl,hdl->bshd", dvl, wv), dwk, dwv


@pytest.mark.parametrize("mistake", ["dk_lat_no_scale", "dk_through_wv", "dwk_from_dv_lat", "dwv_from_k"])
def test_planted_onthefly_backward_mistakes_are_caught(mistake):
    q, k, v, wk, wv, do = _otf_inputs(2, 2, 8, 8, 6, 6, 70)
    o, m, l = R.dmla_fwd_onthefly(q, k, v, wk, wv, 0.4, True, torch.float64)
    ref = R.dmla_grads_onthefly_autograd(q, k, v, wk, wv, do, 0.4, True)
    got = _mutant_otf_bwd(q, k, v, wk, wv, o, do, m, l, 0.4, mistake)
    same = all(torch.allclose(a, b, atol=1e-6) for a, b in zip(got, ref))
    assert not same, f"autograd failed to catch the planted mistake {mistake}"
    assert all(torch.allclose(a, b, atol=1e-10) for a, b in zip(_mutant_otf_bwd(q, k, v, wk, wv, o, do, m, l, 0.4, "none"), ref))


@pytest.mark.parametrize("mistake", ["v_wrong_slice", "k_transposed_dims", "unscaled_m", "mask_off_by_one"])
def test_planted_forward_mistakes_are_caught(mistake):
    g = _golden()
    q, k = torch.from_numpy(g["q"]).double(), torch.from_numpy(g["k_lat"]).double()
    if mistake == "v_wrong_slice":
        o, m, l = R.attention_exact(q[0], k, k[..., -32:], 1 / 8, True)
    elif mistake == "k_transposed_dims":
        o, m, l = R.attention_exact(q[0], k.flip(-1), k[..., :32], 1 / 8, True)
    elif mistake == "mask_off_by_one":   # each row also sees the next key
        s = (q[0] @ k.transpose(-1, -2)) / 8
        n = s.shape[-1]
        mask = torch.arange(n).view(1, n) > torch.arange(n).view(n, 1) + 1
        s = s.masked_fill(mask, float("-inf"))
        m = s.amax(-1)
        p = torch.exp(s - m.unsqueeze(-1))
        o = (p / p.sum(-1, keepdim=True)) @ k[0, :, :32]
    else:
        o, m, l = R.attention_exact(q[0], k, k[..., :32], 1 / 8, True)
        m = m * 8.0
    same = (np.allclose(o.numpy(), g["o"][0], atol=1e-5) and np.allclose(m.numpy(), g["m"][0], atol=1e-5))
    assert not same, f"golden forward failed to catch the planted mistake {mistake}"


# ---------------------------------------------------------------- paged append and combine
def test_kv_append_round_trips_through_gather():
    g = torch.Generator().manual_seed(41)
    P, D, n_pages = 8, 16, 12
    pool = torch.randn(n_pages, P, D, generator=g)
    table = torch.randperm(n_pages, generator=g)[:12].view(2, 6)   # disjoint pages per sequence
    lens = torch.tensor([5, 13])
    new = torch.randn(2, 11, D, generator=g)
    new_lens = torch.tensor([11, 3])
    out = R.kv_append(pool, table, lens, new, new_lens)
    for b in range(2):
        before = R.gather_pages(pool, table[b], int(lens[b]), P)
        after = R.gather_pages(out, table[b], int(lens[b] + new_lens[b]), P)
        assert torch.equal(after, torch.cat([before, new[b, : int(new_lens[b])]]))
    # rows outside the appended positions are untouched
    touched = torch.zeros(n_pages, P, dtype=torch.bool)
    for b in range(2):
        for t in range(int(new_lens[b])):
            pos = int(lens[b]) + t
            touched[int(table[b, pos // P]), pos % P] = True
    assert torch.equal(out[~touched], pool[~touched])


def test_lse_combine_of_key_splits_is_full_attention():
    g = torch.Generator().manual_seed(43)
    H, N, D, DV = 3, 50, 16, 8
    q = torch.randn(1, H, 1, D, generator=g, dtype=torch.float64)
    k = torch.randn(1, N, D, generator=g, dtype=torch.float64)
    cuts = [0, 7, 7, 30, N]   # includes an empty split
    parts_o, parts_l = [], []
    for a, b in zip(cuts[:-1], cuts[1:]):
        if b > a:
            o, m, l = R.attention_exact(q[0], k[:, a:b], k[:, a:b, :DV], 0.3, False)
            parts_o.append(o[:, 0])
            parts_l.append((m + torch.log(l))[:, 0])
        else:
            parts_o.append(torch.full((H, DV), float("nan"), dtype=torch.float64))
            parts_l.append(torch.full((H,), float("-inf"), dtype=torch.float64))
    po = torch.stack(parts_o).unsqueeze(0)
    pl = torch.stack(parts_l).unsqueeze(0)
    o, lse = R.lse_combine(po, pl, dtype=torch.float64)
    o_ref, m_ref, l_ref = R.attention_exact(q[0], k, k[..., :DV], 0.3, False)
    torch.testing.assert_close(o[0], o_ref[:, 0], atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(lse[0], (m_ref + torch.log(l_ref))[:, 0], atol=1e-12, rtol=1e-12)
    # num_splits drops the trailing splits: the combine of the first two equals attention over keys 0..6
    o2, _ = R.lse_combine(po, pl, torch.tensor([2]), dtype=torch.float64)
    o_pre, _, _ = R.attention_exact(q[0], k[:, :7], k[:, :7, :DV], 0.3, False)
    torch.testing.assert_close(o2[0], o_pre[:, 0], atol=1e-12, rtol=1e-12)
    # no finite lse -> o = 0, lse = -inf
    o3, l3 = R.lse_combine(po[:, 1:2], pl[:, 1:2], dtype=torch.float64)
    assert torch.all(o3 == 0) and torch.all(torch.isneginf(l3))


# ---------------------------------------------------------------- decode plan
def _walk_plan(plan, lens):
    """Walks the ranges like the decode kernel; returns {(b, tile): range} and splits per b."""
    B = len(lens)
    hdr = plan[:8]
    tp = plan[8:8 + B + 1]
    sb = plan[8 + B + 1:8 + 2 * (B + 1)]
    o = 8 + 2 * (B + 1)
    ns, fr = plan[o:o + B], plan[o + B:o + 2 * B]
    nr = hdr[1]
    rs = plan[o + 2 * B:o + 2 * B + nr + 1]
    rfb = plan[o + 2 * B + nr + 1:o + 2 * B + 2 * nr + 1]
    seen, splits, segs = {}, [0] * B, [0] * nr
    for r in range(nr):
        t0, t1 = rs[r], rs[r + 1]
        if t0 >= t1:
            continue
        b = rfb[r]
        assert tp[b] <= t0 < tp[b + 1]
        while b < B and tp[b] < t1:
            s0, s1 = max(t0, tp[b]), min(t1, tp[b + 1])
            if s0 < s1:
                assert r - fr[b] == splits[b]          # split index = order of the pieces
                splits[b] += 1
                segs[r] += 1
                for t in range(s0, s1):
                    assert (b, t - tp[b]) not in seen
                    seen[(b, t - tp[b])] = r
            b += 1
    return hdr, tp, sb, ns, rs, seen, splits, segs


@pytest.mark.parametrize("lens,nr", [([5, 0, 70, 1, 64, 0], 4), ([1000, 3000, 10, 8192], 16), ([0, 0], 3),
                                     ([33], 8), ([7] * 50, 8), ([3000] + [1] * 30, 5)])
def test_decode_plan_covers_every_tile_once(lens, nr):
    plan = R.decode_plan(lens, nr, 128)
    hdr, tp, sb, ns, rs, seen, splits, segs = _walk_plan(plan, lens)
    B = len(lens)
    assert hdr[0] == B and hdr[1] == nr and hdr[5] == 10
    total = sum((x + 31) // 32 for x in lens)
    assert hdr[3] == total and len(seen) == total and rs[0] == 0 and rs[-1] == total
    assert all(rs[i] <= rs[i + 1] for i in range(nr))
    assert splits == ns and sb == [sum(ns[:i]) for i in range(B + 1)] and hdr[4] == sum(ns)


def test_decode_plan_balances_tiles_plus_segment_costs():
    # benchmark config 3 shape: 64 contexts in [1024, 8192], 128 ranges
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 8193, (64,), generator=g).tolist()
    plan = R.decode_plan(lens, 128, 128)
    hdr, tp, sb, ns, rs, seen, splits, segs = _walk_plan(plan, lens)
    W, c = hdr[2], hdr[5]
    assert c == 10
    cost = [(rs[r + 1] - rs[r]) + c * segs[r] for r in range(128)]
    # every range's weighted cost is within one segment cost of W (the first segment included)
    assert max(cost) <= W + c and min(x for x in cost if x) >= W - 2 * c


@pytest.mark.parametrize("cus", [256, 304, 80])
@pytest.mark.parametrize("H", [128, 16, 200])
def test_decode_segments_fit_the_page_registers(cus, H):
    """The decode kernel holds a segment's page indices in two VGPRs (128 pages): with the range
    count of decode_ranges no segment of any plan spans more, over full and ragged batches."""
    g = torch.Generator().manual_seed(cus + H)
    for B in (1, 7, 64, 128, 300):
        for max_pages in (1, 2, 127, 128, 129, 256, 1000):
            R_ = R.decode_ranges(B, H, max_pages, cus)
            full = [max_pages * 64] * B
            ragged = torch.randint(0, max_pages * 64 + 1, (B,), generator=g).tolist()
            for lens in (full, ragged):
                plan = R.decode_plan(lens, R_, max_pages)
                pages = R.plan_segment_pages(plan, lens)
                assert max(pages, default=0) <= 128, (B, H, max_pages, R_, max(pages))


def test_decode_range_bound_without_segment_costs_overflows():
    # Planted mistake: sizing R from the tiles alone (no per-segment weight) lets the ranges of
    # 64 full 16K-token sequences on 256 CUs span 130 pages, which the check above rejects.
    B, H, max_pages, cus = 64, 128, 256, 256
    r = (cus // 2) - (cus // 2) % 8
    bad_R = max(r, -(-(B * max_pages * 2) // 254))
    plan = R.decode_plan([max_pages * 64] * B, bad_R, max_pages)
    assert max(R.plan_segment_pages(plan, [max_pages * 64] * B)) > 128
    assert R.decode_ranges(B, H, max_pages, cus) > bad_R


def test_attention_with_no_keys_is_the_fully_masked_case():
    q = torch.randn(2, 3, 8, dtype=torch.float64)
    k = torch.zeros(2, 0, 8, dtype=torch.float64)
    o, m, l = R.attention_exact(q, k, k[..., :4], 0.5, False)
    assert o.shape == (2, 3, 4) and torch.all(o == 0) and torch.all(torch.isneginf(m)) and torch.all(l == 0)
    o2, lse = R.dmla_decode_paged(torch.randn(2, 4, 16), torch.randn(3, 64, 16), torch.zeros(2, 1, dtype=torch.int32),
                                  torch.tensor([0, 5]), 8, 0.3)
    assert torch.all(o2[0] == 0) and torch.all(torch.isneginf(lse[0])) and torch.isfinite(lse[1]).all()
