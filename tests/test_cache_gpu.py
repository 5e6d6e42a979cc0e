"""The paged-cache append (dmla_kv_append) and the standalone split-KV combine
(dmla_lse_combine) on the GPU.

The append is a pure copy, so it must match the oracle bit for bit; appended pages must then
decode like the oracle's attention over the gathered context.  The combine is checked against
the oracle combine and against full attention over the union of the splits' keys.
"""
import math

import pytest
import torch

from conftest import assert_out_close, seeded
from oracle import dmla_ref as R
from python import ops

SCALE = 1.0 / math.sqrt(192.0)


def _paged(B, lens, extra, seed, n_spare=3):
    g = torch.Generator().manual_seed(seed)
    need = [(int(l) + e + 63) // 64 for l, e in zip(lens, extra)]
    n_pages = sum(need) + n_spare
    pool = (torch.randn(n_pages, 64, 576, generator=g) * 0.5).to(torch.bfloat16)
    perm = torch.randperm(n_pages, generator=g)
    table = torch.full((B, max(need)), -1, dtype=torch.int32)
    c = 0
    for b in range(B):
        table[b, : need[b]] = perm[c: c + need[b]].to(torch.int32)
        c += need[b]
    return pool, table


@pytest.mark.gpu
def test_kv_append_is_bit_exact(gpu):
    B = 4
    lens = torch.tensor([0, 63, 64, 200], dtype=torch.int32)
    new_lens = torch.tensor([70, 1, 130, 0], dtype=torch.int32)
    pool, table = _paged(B, lens, new_lens.tolist(), seed=5)
    new = seeded((B, 130, 576), 6, 0.5, torch.bfloat16)
    ref = R.kv_append(pool, table, lens, new, new_lens)
    pg = pool.to(gpu)
    ops.flash_dmla_kv_append(pg, table.to(gpu), lens.to(gpu), new.to(gpu), new_lens.to(gpu), check_indices=True)
    assert torch.equal(pg.cpu(), ref)


@pytest.mark.gpu
def test_kv_append_then_decode(gpu):
    B, H = 3, 128
    lens = torch.tensor([100, 1, 700], dtype=torch.int32)
    n_new = 40
    pool, table = _paged(B, lens, [n_new] * B, seed=8)
    new = seeded((B, n_new, 576), 9, 0.5, torch.bfloat16)
    q = seeded((B, H, 576), 10, 0.5, torch.bfloat16)
    pg, tg = pool.to(gpu), table.to(gpu)
    ops.flash_dmla_kv_append(pg, tg, lens.to(gpu), new.to(gpu))
    total = lens + n_new
    o = ops.flash_dmla_decode_paged(q.to(gpu), pg, tg, total.to(gpu), 512, SCALE)
    o_ref, _ = R.dmla_decode_paged(q.float(), R.kv_append(pool, table, lens, new).float(), table, total, 512, SCALE)
    assert_out_close(o, o_ref)


@pytest.mark.gpu
def test_kv_append_skips_and_flags_bad_pages(gpu):
    B = 2
    lens = torch.tensor([10, 10], dtype=torch.int32)
    pool, table = _paged(B, lens, [80, 5], seed=12)
    table[0, 1] = pool.shape[0] + 7          # second page of sequence 0: out of range
    new = seeded((B, 80, 576), 13, 0.5, torch.bfloat16)
    new_lens = torch.tensor([80, 5], dtype=torch.int32)
    pg = pool.to(gpu)
    with pytest.raises(ValueError, match="out of range"):
        ops.flash_dmla_kv_append(pg, table.to(gpu), lens.to(gpu), new.to(gpu), new_lens.to(gpu), check_indices=True)
    # the rows on valid pages were written exactly as the oracle writes them
    good = table.clone()
    good[0, 1] = -1
    expect = pool.clone()
    for b in range(B):
        for t in range(int(new_lens[b])):
            pos = int(lens[b]) + t
            page = int(good[b, pos // 64])
            if page >= 0:
                expect[page, pos % 64] = new[b, t]
    assert torch.equal(pg.cpu(), expect)


@pytest.mark.gpu
def test_lse_combine_matches_oracle_and_full_attention(gpu):
    B, S, H, d = 3, 5, 8, 512
    g = torch.Generator().manual_seed(21)
    q = (torch.randn(B, H, 576, generator=g) * 0.5).to(torch.bfloat16).float()
    keys = (torch.randn(B, 300, 576, generator=g) * 0.5).to(torch.bfloat16).float()
    cuts = [0, 40, 40, 170, 260, 300]      # one empty split
    po = torch.full((B, S, H, d), float("nan"))
    pl = torch.full((B, S, H), float("-inf"))
    for b in range(B):
        for s, (a, e) in enumerate(zip(cuts[:-1], cuts[1:])):
            if e > a:
                o, m, l = R.attention_exact(q[b].unsqueeze(1), keys[b:b + 1, a:e], keys[b:b + 1, a:e, :d], SCALE, False)
                po[b, s] = o[:, 0]
                pl[b, s] = (m + torch.log(l))[:, 0]
    num = torch.tensor([5, 3, 1], dtype=torch.int32)
    o, lse = ops.flash_dmla_lse_combine(po.to(gpu), pl.to(gpu), num.to(gpu), return_lse=True)
    o_ref, lse_ref = R.lse_combine(po, pl, num)
    assert_out_close(o, o_ref)
    assert (lse.cpu() - lse_ref).abs().max().item() <= 1e-5
    # sequence 0 used every split: full attention over all 300 keys
    of, mf, lf = R.attention_exact(q[0].unsqueeze(1), keys[0:1], keys[0:1, :, :d], SCALE, False)
    assert_out_close(o[0], of[:, 0])
    assert (lse[0].cpu() - (mf + torch.log(lf))[:, 0]).abs().max().item() <= 1e-4
