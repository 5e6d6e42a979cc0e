"""torch.ops.flashdmla.* on the GPU: each registered op returns exactly what the python/ops.py
call it wraps returns (same kernels, bit for bit), autograd through the two registered forwards
gives the gradients of the autograd.Function wrappers, and torch.library.opcheck accepts the
schemas, fake implementations and autograd registrations.  Parity of the kernels themselves
with the fp32 oracle is tested per op in the other test modules.
"""
import math

import pytest
import torch

from python import ops
import python  # noqa: F401  (registers torch.ops.flashdmla.*)
from conftest import seeded
from test_bwd_gpu import _inputs as cl_inputs
from test_decode_gpu import _paged
from test_otf_bwd_gpu import _inputs as otf_inputs

SCALE = 1.0 / math.sqrt(192.0)
F = torch.ops.flashdmla


def _same(a, b, what):
    # bit for bit: the paged pools carry NaN rows past each sequence (decode must never read
    # them), and NaN compares unequal to itself
    assert a.dtype == b.dtype and a.shape == b.shape, what
    bits = {2: torch.int16, 4: torch.int32, 8: torch.int64}
    if a.is_floating_point():
        a, b = a.view(bits[a.element_size()]), b.view(bits[b.element_size()])
    assert torch.equal(a, b), f"{what} differs"


@pytest.mark.gpu
def test_cache_latent_ops_match_the_python_api(gpu):
    q, k, do = (t.to(gpu) for t in cl_inputs(1, 5, 70, 90, seed=81))
    o, m, l = F.fwd_cache_latent(q, k, 512, SCALE, True)
    o2, m2, l2 = ops.flash_dmla_fwd(q, k, 512, SCALE, True)
    for a, b, n in ((o, o2, "o"), (m, m2, "m"), (l, l2, "l")):
        _same(a, b, n)
    dq, dk = F.bwd_cache_latent(q, k, o, do, m, l, 512, SCALE, True)
    dq2, dk2 = ops.flash_dmla_bwd(q, k, o, do, m, l, 512, SCALE, True)
    _same(dq, dq2, "dq")
    _same(dk, dk2, "dk_lat")


@pytest.mark.gpu
def test_onthefly_ops_match_the_python_api(gpu):
    q, k, v, wk, wv, do = (t.to(gpu) for t in otf_inputs(1, 2, 100, 130, seed=82))
    o, m, l = F.fwd_onthefly(q, k, v, wk, wv, 0.125, True)
    o2, m2, l2 = ops.flash_dmla_fwd_onthefly(q, k, v, wk, wv, 0.125, True, return_stats=True)
    for a, b, n in ((o, o2, "o"), (m, m2, "m"), (l, l2, "l")):
        _same(a, b, n)
    g = F.bwd_onthefly(q, k, v, wk, wv, o, do, m, l, 0.125, True)
    g2 = ops.flash_dmla_bwd_onthefly(q, k, v, wk, wv, o, do, m, l, 0.125, True)
    for a, b, n in zip(g, g2, ("dq", "dk", "dv", "dwk", "dwv")):
        _same(a, b, n)


@pytest.mark.gpu
def test_decode_ops_match_the_python_api(gpu):
    q, pool, table, lens = (t.to(gpu) for t in _paged([300, 64, 1000], 16, seed=83))
    plan = F.decode_plan(lens, 16, table.shape[1])
    plan2 = ops.flash_dmla_decode_plan(lens, 16, table.shape[1])
    # the entries the plan defines: header, 4 per-sequence arrays (two of B + 1), two per-range
    # arrays (R + 1, R); the rest of the buffer is padding nobody writes
    B, R = lens.shape[0], int(plan2[1])
    used = 8 + 2 * (B + 1) + 2 * B + (R + 1) + R
    _same(plan[:used], plan2[:used], "plan")
    o, lse = F.decode_paged(q, pool, table, lens, 512, SCALE, None)
    o2, lse2 = ops.flash_dmla_decode_paged(q, pool, table, lens, 512, SCALE, return_lse=True)
    _same(o, o2, "o")
    _same(lse, lse2, "lse")
    o3, lse3 = F.decode_paged(q, pool, table, lens, 512, SCALE, plan)
    _same(o3, o2, "o with a plan")
    _same(lse3, lse2, "lse with a plan")

    # the append writes the pool in place, as the Python call does on a copy
    new = seeded((3, 5, 576), 84, 0.5, torch.bfloat16).to(gpu)
    short = torch.tensor([10, 20, 30], dtype=torch.int32, device=gpu)
    pa, pb = pool.clone(), pool.clone()
    assert F.kv_append(pa, table, short, new, None) is None
    ops.flash_dmla_kv_append(pb, table, short, new)
    _same(pa, pb, "pool after the append")

    part_o = seeded((2, 3, 4, 512), 85, 1.0, torch.float32).to(gpu)
    part_lse = seeded((2, 3, 4), 86, 1.0, torch.float32).to(gpu)
    ns = torch.tensor([3, 2], dtype=torch.int32, device=gpu)
    o, lse = F.lse_combine(part_o, part_lse, ns)
    o2, lse2 = ops.flash_dmla_lse_combine(part_o, part_lse, ns, return_lse=True)
    _same(o, o2, "combined o")
    _same(lse, lse2, "combined lse")


@pytest.mark.gpu
def test_autograd_through_the_registered_forwards(gpu):
    q, k, do = (t.to(gpu) for t in cl_inputs(1, 4, 66, 66, seed=87))
    qa, ka = q.clone().requires_grad_(), k.clone().requires_grad_()
    (F.fwd_cache_latent(qa, ka, 512, SCALE, True)[0].float() * do.float()).sum().backward()
    qb, kb = q.clone().requires_grad_(), k.clone().requires_grad_()
    (ops.FlashDMLACacheLatent.apply(qb, kb, 512, SCALE, True).float() * do.float()).sum().backward()
    _same(qa.grad, qb.grad, "dq through the registered op")
    _same(ka.grad, kb.grad, "dk_lat through the registered op")

    xs = [t.to(gpu) for t in otf_inputs(1, 2, 80, 80, seed=88)]
    do = xs.pop()
    xa = [t.clone().requires_grad_() for t in xs]
    (F.fwd_onthefly(*xa, 0.125, True)[0].float() * do.float()).sum().backward()
    xb = [t.clone().requires_grad_() for t in xs]
    (ops.FlashDMLAOnTheFly.apply(*xb, 0.125, True).float() * do.float()).sum().backward()
    for a, b, n in zip(xa, xb, ("dq", "dk", "dv", "dwk", "dwv")):
        _same(a.grad, b.grad, f"{n} through the registered op")


@pytest.mark.gpu
def test_opcheck_accepts_the_registrations(gpu):
    checks = ("test_schema", "test_autograd_registration", "test_faketensor")
    q, k, _ = (t.to(gpu) for t in cl_inputs(1, 2, 40, 40, seed=89))
    torch.library.opcheck(F.fwd_cache_latent.default, (q.requires_grad_(), k, 512, SCALE, True), test_utils=checks)
    qp, pool, table, lens = (t.to(gpu) for t in _paged([200, 70], 8, seed=90))
    torch.library.opcheck(F.decode_paged.default, (qp, pool, table, lens, 512, SCALE, None), test_utils=checks)
    new = seeded((2, 3, 576), 91, 0.5, torch.bfloat16).to(gpu)
    torch.library.opcheck(F.kv_append.default, (pool.clone(), table, lens, new, None), test_utils=checks)


@pytest.mark.gpu
def test_torch_compile_traces_the_ops(gpu):
    # Dynamo + AOTAutograd over the registered ops (fake implementations for tracing, the
    # autograd formula for the backward graph, auto-functionalization of the in-place append),
    # run eagerly from the traced graphs: results equal the uncompiled calls bit for bit.
    torch._dynamo.reset()
    q, k, do = (t.to(gpu) for t in cl_inputs(1, 3, 70, 90, seed=92))

    def train_step(q, k, do):
        o = F.fwd_cache_latent(q, k, 512, SCALE, True)[0]
        (o.float() * do.float()).sum().backward()
        return o

    compiled = torch.compile(train_step, backend="aot_eager", fullgraph=False)
    qa, ka = q.clone().requires_grad_(), k.clone().requires_grad_()
    oa = compiled(qa, ka, do)
    qb, kb = q.clone().requires_grad_(), k.clone().requires_grad_()
    ob = train_step(qb, kb, do)
    _same(oa.detach(), ob.detach(), "o under torch.compile")
    _same(qa.grad, qb.grad, "dq under torch.compile")
    _same(ka.grad, kb.grad, "dk_lat under torch.compile")

    qp, pool, table, lens = (t.to(gpu) for t in _paged([300, 60, 1000], 16, seed=93))
    new = seeded((3, 1, 576), 94, 0.5, torch.bfloat16).to(gpu)

    def decode_step(qp, pool, table, lens, new):
        F.kv_append(pool, table, lens, new, None)
        grown = lens + 1
        plan = F.decode_plan(grown, 16, table.shape[1])
        return F.decode_paged(qp, pool, table, grown, 512, SCALE, plan)

    step = torch.compile(decode_step, backend="aot_eager", fullgraph=True)
    pa, pb = pool.clone(), pool.clone()
    oa, lsea = step(qp, pa, table, lens, new)
    ob, lseb = decode_step(qp, pb, table, lens, new)
    _same(pa, pb, "pool after the traced append")
    _same(oa, ob, "decode o under torch.compile")
    _same(lsea, lseb, "decode lse under torch.compile")
