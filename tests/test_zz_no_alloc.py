"""dmla_decode_paged_noalloc (the decode entry point that allocates nothing) against
dmla_decode_paged with a caller workspace, both called through the C ABI.

The two run the same kernels on the same plan, so outputs and log-sum-exps must be bit-identical.
Two calls in a row, the second with a smaller batch, show that whatever the first call left in
the shared static scratch does not leak into the second; an oversized batch is rejected with
DMLA_ERR_WORKSPACE before anything is launched.
"""
import ctypes
import math

import pytest
import torch

from python import _lib

SCALE = 1.0 / math.sqrt(192.0)


def _batch(lens, H, seed):
    g = torch.Generator().manual_seed(seed)
    n_pages = [(n + 63) // 64 for n in lens]
    total = sum(n_pages)
    perm = torch.randperm(total, generator=g)
    pool = (torch.randn(total, 64, 576, generator=g) * 0.5).to(torch.bfloat16)
    table = torch.zeros(len(lens), max(n_pages), dtype=torch.int32)
    c = 0
    for b, n in enumerate(n_pages):
        table[b, :n] = perm[c:c + n].to(torch.int32)
        c += n
    q = (torch.randn(len(lens), H, 576, generator=g) * 0.5).to(torch.bfloat16)
    return q, pool, table, torch.tensor(lens, dtype=torch.int32)


def _args(q, pool, table, sl, o, lse):
    P = ctypes.c_void_p
    B, H = q.shape[0], q.shape[1]
    return ([P(q.data_ptr()), P(pool.data_ptr()), P(table.data_ptr()), P(sl.data_ptr()), P(o.data_ptr()),
             P(lse.data_ptr()), B, H, 576, 512, 64, pool.shape[0], table.shape[1],
             q.stride(0), q.stride(1), pool.stride(0), pool.stride(1), table.stride(0), o.stride(0), o.stride(1)],
            ctypes.c_float(SCALE))


def _both(gpu, lens, H, seed):
    lib = _lib.lib()
    q, pool, table, sl = (t.to(gpu) for t in _batch(lens, H, seed))
    B = len(lens)
    stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
    o1 = torch.empty(B, H, 512, dtype=torch.bfloat16, device=gpu)
    l1 = torch.empty(B, H, dtype=torch.float32, device=gpu)
    o2, l2 = torch.empty_like(o1), torch.empty_like(l1)
    ws_bytes = int(lib.dmla_decode_workspace_bytes(B, H, 512, table.shape[1]))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    head, scale = _args(q, pool, table, sl, o1, l1)
    rc = lib.dmla_decode_paged(*head, scale, ctypes.c_void_p(ws.data_ptr()), ws_bytes, stream)
    assert rc == 0, lib.dmla_last_error()
    head, scale = _args(q, pool, table, sl, o2, l2)
    rc = lib.dmla_decode_paged_noalloc(*head, scale, stream)
    assert rc == 0, lib.dmla_last_error()
    torch.cuda.synchronize()
    assert torch.isfinite(o2.float()).all()
    assert torch.equal(o1, o2), "outputs differ"
    assert torch.equal(l1, l2), "log-sum-exps differ"


@pytest.mark.gpu
def test_noalloc_decode_matches_the_workspace_entry_point(gpu):
    g = torch.Generator().manual_seed(3)
    big = torch.randint(1024, 8193, (64,), generator=g).tolist()    # benchmark config 3
    print("no-alloc decode: call 1, B=64 H=128 (config 3 lengths)", flush=True)
    _both(gpu, big, 128, seed=31)
    print("no-alloc decode: call 2, B=5 H=128 (smaller batch after a larger one)", flush=True)
    _both(gpu, [1, 64, 700, 33, 2000], 128, seed=32)


@pytest.mark.gpu
def test_noalloc_decode_rejects_a_batch_beyond_its_scratch(gpu):
    lib = _lib.lib()
    B, H, max_pages = 1024, 128, 256
    assert lib.dmla_decode_workspace_bytes(B, H, 512, max_pages) > (64 << 20)
    q = torch.zeros(1, dtype=torch.bfloat16, device=gpu)
    P = ctypes.c_void_p
    rc = lib.dmla_decode_paged_noalloc(P(q.data_ptr()), P(q.data_ptr()), P(q.data_ptr()), P(q.data_ptr()),
                                       P(q.data_ptr()), P(None), B, H, 576, 512, 64, 1 << 20, max_pages,
                                       H * 576, 576, 64 * 576, 576, max_pages, H * 512, 512, ctypes.c_float(SCALE),
                                       P(None))
    assert rc == _lib.DMLA_ERR_WORKSPACE
    assert b"static scratch" in lib.dmla_last_error()
