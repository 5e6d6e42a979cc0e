"""Parity of the paged decode kernel (dmla_decode_paged) with the fp32 oracle."""
import math

import pytest
import torch

from conftest import assert_out_close, seeded
from oracle import dmla_ref as R
from python import ops

SCALE = 1.0 / math.sqrt(192.0)


def _paged(lens, H, seed, page=64, extra_pages=0, poison_tail=True):
    """Seeded q, a randomly permuted page pool and its block table for the given lengths."""
    B = len(lens)
    n_pages = [(n + page - 1) // page for n in lens]
    total = sum(n_pages) + extra_pages
    max_pages = max(max(n_pages), 1)
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(total, generator=g)
    pool = (torch.randn(total, page, 576, generator=g) * 0.5).to(torch.bfloat16)
    if poison_tail:
        # Rows past each sequence's end hold NaN: the kernel must never let them reach o.
        pool_tail = torch.full((page, 576), float("nan")).to(torch.bfloat16)
    table = torch.zeros(B, max_pages, dtype=torch.int32)
    c = 0
    for b in range(B):
        for j in range(n_pages[b]):
            table[b, j] = int(perm[c])
            c += 1
        if poison_tail and lens[b] % page:
            last = int(table[b, n_pages[b] - 1])
            pool[last, lens[b] % page:] = pool_tail[lens[b] % page:]
    q = (torch.randn(B, H, 576, generator=g) * 0.5).to(torch.bfloat16)
    return q, pool, table, torch.tensor(lens, dtype=torch.int32)


def _check(gpu, q, pool, table, lens, oracle_device="cpu"):
    o, lse = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), lens.to(gpu),
                                         512, SCALE, return_lse=True)
    torch.cuda.synchronize()
    dev = gpu if oracle_device == "gpu" else "cpu"
    o_ref, lse_ref = R.dmla_decode_paged(q.to(dev).float(), pool.to(dev).float(), table.to(dev),
                                         lens.to(dev), 512, SCALE)
    assert_out_close(o, o_ref)
    d = (lse - lse_ref.to(lse.device)).abs().max().item()
    assert d <= 1e-3, f"lse max-abs {d:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize(
    "lens,H",
    [
        ([1, 63, 64, 65, 130], 128),   # 1-token context, partial and exact pages
        ([700, 5, 2048], 128),         # long enough to split across workgroups
        ([100, 33], 16),               # fewer heads than a workgroup
        ([256, 257, 300], 96),         # two head groups, the second partial
    ],
)
def test_decode_small(gpu, lens, H):
    q, pool, table, sl = _paged(lens, H, seed=sum(lens) + H)
    _check(gpu, q, pool, table, sl)


@pytest.mark.gpu
def test_decode_score_growth_takes_the_exact_max_pass(gpu):
    # Each sequence's scores grow along its context by ~86 (log2 units) -- far past the 2^32
    # headroom over a segment's first-tile max -- so every segment restarts on the exact-max
    # path; the long contexts also split across workgroups, whose partials the combine merges.
    lens = [700, 2100, 37, 64]
    H, page = 128, 64
    q, pool, table, sl = _paged(lens, H, seed=17)
    pool = pool.float()
    q = q.float()
    for b, n in enumerate(lens):
        for t in range(n):
            pool[int(table[b, t // page]), t % page, 512] = 30.0 * t / max(n - 1, 1)
    q[..., 512] = 4.0
    q, pool = q.to(torch.bfloat16), pool.to(torch.bfloat16)
    o, lse = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, 0.5,
                                         return_lse=True)
    torch.cuda.synchronize()
    o_ref, lse_ref = R.dmla_decode_paged(q.float(), pool.float(), table, sl, 512, 0.5)
    assert_out_close(o, o_ref)
    d = (lse.cpu() - lse_ref).abs().max().item()
    assert d <= 1e-3, f"lse max-abs {d:.3e}"


@pytest.mark.gpu
def test_decode_page_order_does_not_matter(gpu):
    q, pool, table, sl = _paged([500, 333], 128, seed=11)
    o1 = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE)
    # Move every page to a new physical slot and rewrite the table accordingly.
    perm = torch.randperm(pool.shape[0], generator=torch.Generator().manual_seed(3))
    pool2 = torch.empty_like(pool)
    pool2[perm] = pool
    table2 = perm[table.long()].to(torch.int32)
    o2 = ops.flash_dmla_decode_paged(q.to(gpu), pool2.to(gpu), table2.to(gpu), sl.to(gpu), 512, SCALE)
    assert torch.equal(o1, o2)


@pytest.mark.gpu
def test_decode_bad_page_index_gives_nan_not_a_fault(gpu):
    q, pool, table, sl = _paged([128, 128], 128, seed=12)
    table[1, 1] = pool.shape[0] + 5  # out of range: must not be dereferenced
    o = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE)
    torch.cuda.synchronize()
    assert torch.isnan(o[1].float()).all()
    assert torch.isfinite(o[0].float()).all()
    with pytest.raises(ValueError, match="page index"):
        ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE,
                                    check_indices=True)


@pytest.mark.gpu
def test_decode_config3_full_shape(gpu):
    # benchmark config 3: B=64, H=128, contexts uniform in [1024, 8192], 64-token pages in a
    # seeded random permutation.
    g = torch.Generator().manual_seed(3)
    lens = torch.randint(1024, 8193, (64,), generator=g).tolist()
    q, pool, table, sl = _paged(lens, 128, seed=3, poison_tail=False)
    _check(gpu, q, pool, table, sl, oracle_device="gpu")


@pytest.mark.gpu
def test_decode_long_contexts_stay_within_segment_pages(gpu):
    # 64 full 16K-token sequences: the plan's ranges must keep each segment within the 128 page
    # indices a workgroup holds (a range count sized from the tiles alone made 130-page segments
    # that read wrapped page indices).  The plan stored by the kernel is checked page by page.
    lens = [16384] * 64
    q, pool, table, sl = _paged(lens, 128, seed=21, poison_tail=False)
    _check(gpu, q, pool, table, sl, oracle_device="gpu")
    plan = ops.flash_dmla_decode_plan(sl.to(gpu), 128, table.shape[1]).cpu().tolist()
    assert max(R.plan_segment_pages(plan, lens)) <= 128


def _lse_close(lse, lse_ref, tol=1e-3):
    lse, lse_ref = lse.cpu(), lse_ref.cpu()
    inf = torch.isinf(lse_ref)
    assert torch.equal(torch.isinf(lse), inf) and bool((lse[inf] == lse_ref[inf]).all())
    if (~inf).any():
        d = (lse[~inf] - lse_ref[~inf]).abs().max().item()
        assert d <= tol, f"lse max-abs {d:.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("lens,max_pages", [
    ([5, 0, 70, 1, 64, 0, 4000, 31], 64),
    ([8192] * 3 + [1] * 40, 128),
    ([0, 0, 0], 4),
    (list(range(1, 3000, 37)), 48),
])
def test_decode_plan_matches_oracle(gpu, lens, max_pages):
    sl = torch.tensor(lens, dtype=torch.int32)
    plan = ops.flash_dmla_decode_plan(sl.to(gpu), 128, max_pages).cpu().tolist()
    nr = plan[1]
    ref = R.decode_plan(lens, nr, max_pages)
    assert plan[:len(ref)] == ref


@pytest.mark.gpu
def test_decode_ranges_spanning_many_sequences_and_empty_ones(gpu):
    # 300 short sequences (some empty): each range covers many of them, most sequences are split
    g = torch.Generator().manual_seed(77)
    lens = torch.randint(0, 160, (300,), generator=g).tolist()
    lens[:5] = [0, 0, 1, 0, 159]
    q, pool, table, sl = _paged(lens, 128, seed=78)
    o, lse = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE,
                                         return_lse=True)
    o_ref, lse_ref = R.dmla_decode_paged(q.float(), pool.float(), table, sl, 512, SCALE)
    assert_out_close(o, o_ref)
    _lse_close(lse, lse_ref)
    empty = sl == 0
    assert bool((o.cpu()[empty] == 0).all())


@pytest.mark.gpu
def test_decode_with_a_shared_plan_is_bit_identical(gpu):
    lens = [3000, 17, 0, 8000, 640]
    q, pool, table, sl = _paged(lens, 128, seed=91)
    q2 = seeded(tuple(q.shape), 92, 0.5, torch.bfloat16)
    args = (pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE)
    plan = ops.flash_dmla_decode_plan(sl.to(gpu), 128, table.shape[1])
    for qq in (q, q2):   # one plan, two "layers"
        a, la = ops.flash_dmla_decode_paged(qq.to(gpu), *args, return_lse=True)
        b, lb = ops.flash_dmla_decode_paged(qq.to(gpu), *args, return_lse=True, plan=plan)
        assert torch.equal(a, b) and torch.equal(la, lb)


@pytest.mark.gpu
def test_decode_inline_plan_stores_the_plan_kernels_plan(gpu):
    """For batches up to 512 sequences dmla_decode_paged builds the plan inside the decode kernel
    and stores it at the start of the workspace (where the combine reads it): that stored plan
    must equal the standalone plan kernel's, entry for entry."""
    from python import _lib
    lens = [3000, 17, 0, 8000, 640, 1, 64, 4097]
    q, pool, table, sl = _paged(lens, 128, seed=95)
    qg, pg, tg, sg = q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu)
    B, H, max_pages = len(lens), 128, table.shape[1]
    ws_bytes = int(_lib.lib().dmla_decode_workspace_bytes(B, H, 512, max_pages))
    plan_bytes = int(_lib.lib().dmla_decode_plan_bytes(B, H, max_pages))
    ws = torch.full((ws_bytes,), 0x5A, dtype=torch.uint8, device=gpu)
    o = torch.empty((B, H, 512), dtype=torch.bfloat16, device=gpu)
    _lib.call("dmla_decode_paged", qg.data_ptr(), pg.data_ptr(), tg.data_ptr(), sg.data_ptr(), o.data_ptr(), None,
              B, H, 576, 512, 64, pool.shape[0], max_pages, qg.stride(0), qg.stride(1), pg.stride(0), pg.stride(1),
              tg.stride(0), o.stride(0), o.stride(1), SCALE, ws.data_ptr(), ws_bytes,
              torch.cuda.current_stream().cuda_stream)
    plan = ops.flash_dmla_decode_plan(sg, H, max_pages)
    torch.cuda.synchronize()
    ref = plan.cpu()
    n = 8 + 4 * B + 2 + 2 * int(ref[1]) + 1   # header, per-sequence arrays, range arrays
    stored = ws[:plan_bytes].view(torch.int32).cpu()[:n]
    bad = (stored != ref[:n]).nonzero().flatten().tolist()
    assert not bad, f"plan entries differ at {bad[:8]}: stored {stored[bad[:8]].tolist()} vs {ref[bad[:8]].tolist()}"


@pytest.mark.gpu
def test_decode_inline_plan_at_its_batch_limit(gpu):
    """512 sequences, the largest batch whose plan the decode kernel builds itself (one sequence
    per thread of the workgroup, the last one included)."""
    g = torch.Generator().manual_seed(99)
    lens = torch.randint(0, 80, (512,), generator=g).tolist()
    lens[-1] = 200   # the last thread's sequence spans several tiles
    q, pool, table, sl = _paged(lens, 16, seed=100)
    o, lse = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE,
                                         return_lse=True)
    o_ref, lse_ref = R.dmla_decode_paged(q.float(), pool.float(), table, sl, 512, SCALE)
    assert_out_close(o, o_ref)
    _lse_close(lse, lse_ref)


@pytest.mark.gpu
def test_decode_large_batch_uses_the_plan_kernel(gpu):
    """600 short sequences: past the inline-plan limit, the plan kernel runs first."""
    g = torch.Generator().manual_seed(97)
    lens = torch.randint(0, 96, (600,), generator=g).tolist()
    q, pool, table, sl = _paged(lens, 16, seed=98)
    o, lse = ops.flash_dmla_decode_paged(q.to(gpu), pool.to(gpu), table.to(gpu), sl.to(gpu), 512, SCALE,
                                         return_lse=True)
    o_ref, lse_ref = R.dmla_decode_paged(q.float(), pool.float(), table, sl, 512, SCALE)
    assert_out_close(o, o_ref)
    _lse_close(lse, lse_ref)   # empty sequences: lse -inf on both sides


@pytest.mark.gpu
@pytest.mark.parametrize("lens", [[131072], [1, 98304, 3]])
def test_decode_one_very_long_context(gpu, lens):
    """One sequence of 128K (or 96K beside two tiny ones) tokens: the plan splits it over every
    workgroup, so a single sequence is merged from the most partials the combine ever sees."""
    q, pool, table, sl = _paged(lens, 128, seed=len(lens) + 31, poison_tail=False)
    plan = ops.flash_dmla_decode_plan(sl.to(gpu), 128, table.shape[1]).cpu().tolist()
    assert max(R.plan_segment_pages(plan, lens)) <= 128
    _check(gpu, q, pool, table, sl, oracle_device="gpu")
