"""The ops inside HIP graphs (torch.cuda.CUDAGraph): capture once, replay many times.

A serving loop replays one captured decode step per token, and a training step can be captured
whole.  The library allocates nothing, records no memset and never synchronizes, so its
kernels capture as plain kernel nodes; torch provides the outputs and workspaces from the
graph's pool.  Each test replays its graph several times with new inputs copied in eagerly
between the replays (and a synchronization after each) and checks every replay bit for bit
against an eager call on the same inputs.
"""
import math

import pytest
import torch

from conftest import seeded
from python import ops
from test_decode_gpu import _paged

SCALE = 1.0 / math.sqrt(192.0)


def _capture(fn):
    # torch's recipe: warm up on a side stream, then capture on the graph's own stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


@pytest.mark.gpu
def test_decode_step_replays_in_a_graph(gpu):
    q0, pool, table, lens = _paged([700, 5, 2048, 64, 1300], 128, seed=61)
    q = q0.to(gpu)
    pool, table, lens = pool.to(gpu), table.to(gpu), lens.to(gpu)

    def step():
        return ops.flash_dmla_decode_paged(q, pool, table, lens, 512, SCALE, return_lse=True)

    graph, (o_g, lse_g) = _capture(step)
    for r in range(4):
        q.copy_(seeded(tuple(q.shape), 200 + r, 0.5, torch.bfloat16).to(gpu))   # eager work
        graph.replay()
        torch.cuda.synchronize()
        o_e, lse_e = step()
        torch.cuda.synchronize()
        assert torch.equal(o_g, o_e), f"replay {r}: o differs from the eager call"
        assert torch.equal(lse_g, lse_e), f"replay {r}: lse differs from the eager call"


@pytest.mark.gpu
def test_prefill_forward_and_backward_replay_in_a_graph(gpu):
    B, H, S = 1, 16, 300
    q = seeded((B, H, S, 576), 71, 0.5, torch.bfloat16).to(gpu)
    k = seeded((B, S, 576), 72, 0.5, torch.bfloat16).to(gpu)
    do = seeded((B, H, S, 512), 73, 1.0, torch.bfloat16).to(gpu)

    def step():
        o, m, l = ops.flash_dmla_fwd(q, k, 512, SCALE, True)
        dq, dk = ops.flash_dmla_bwd(q, k, o, do, m, l, 512, SCALE, True)
        return o, dq, dk

    graph, outs_g = _capture(step)
    for r in range(3):
        q.copy_(seeded(tuple(q.shape), 300 + r, 0.5, torch.bfloat16).to(gpu))
        do.copy_(seeded(tuple(do.shape), 400 + r, 1.0, torch.bfloat16).to(gpu))
        graph.replay()
        torch.cuda.synchronize()
        outs_e = step()
        torch.cuda.synchronize()
        for name, g, e in zip(("o", "dq", "dk_lat"), outs_g, outs_e):
            assert torch.equal(g, e), f"replay {r}: {name} differs from the eager call"


@pytest.mark.gpu
def test_ops_launch_on_the_current_stream(gpu):
    # Ops take the caller's current stream: an append and the decode that reads its rows,
    # issued back to back on a side stream with no host synchronization in between, are
    # ordered by that stream; results equal the same calls on the default stream.  The rows
    # appended (inside each sequence's last page) held NaN before, so a decode that ran ahead
    # of the append would not be finite.
    q0, pool0, table0, lens0 = _paged([300, 60, 1000], 32, seed=92)
    q, table, lens = q0.to(gpu), table0.to(gpu), lens0.to(gpu)
    new = seeded((3, 4, 576), 93, 0.5, torch.bfloat16).to(gpu)
    grown = lens + 4

    def run():
        pool = pool0.to(gpu)
        ops.flash_dmla_kv_append(pool, table, lens, new)
        return ops.flash_dmla_decode_paged(q, pool, table, grown, 512, SCALE, return_lse=True)

    o_ref, lse_ref = run()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        o_s, lse_s = run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(o_s).all()) and bool(torch.isfinite(lse_s).all())
    assert torch.equal(o_s, o_ref) and torch.equal(lse_s, lse_ref)
