"""Parity of the on-the-fly forward (dmla_fwd_onthefly) with the fp32 oracle.

The oracle projects K_lat = K WK and V_lat = V WV in fp32 and runs exact attention; the kernel
projects on MFMA, rounds V_lat and P to fp16 before the PV product and keeps K_lat as an fp16
hi + lo pair for the scores.  Outputs are held to the north-star tolerance (max-abs 2e-2,
mean-rel 1e-2) and the statistics to 1e-3 (m max-abs, l max-rel), as in every other mode.
Inputs follow benchmark config 4: q, k, v ~ N(0, 1), wk and wv Xavier-uniform (bound
sqrt(6 / (128 + 64))), scale 1/8.
"""
import math

import pytest
import torch

from conftest import assert_out_close, assert_stats_close, seeded
from oracle import dmla_ref as R
from python import ops


def _inputs(B, H, Sq, Sk, seed):
    q = seeded((B, H, Sq, 64), seed, 1.0, torch.bfloat16)
    k = seeded((B, Sk, H, 128), seed + 1, 1.0, torch.bfloat16)
    v = seeded((B, Sk, H, 128), seed + 2, 1.0, torch.bfloat16)
    bound = math.sqrt(6.0 / (128 + 64))
    g = torch.Generator().manual_seed(seed + 3)
    wk = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16)
    wv = ((torch.rand(H, 128, 64, generator=g) * 2 - 1) * bound).to(torch.bfloat16)
    return q, k, v, wk, wv


def _check(gpu, B, H, Sq, Sk, causal, seed, ref_device="cpu", scale=0.125):
    q, k, v, wk, wv = _inputs(B, H, Sq, Sk, seed)
    o, m, l = ops.flash_dmla_fwd_onthefly(q.to(gpu), k.to(gpu), v.to(gpu), wk.to(gpu), wv.to(gpu), scale, causal,
                                          return_stats=True)
    torch.cuda.synchronize()
    dev = gpu if ref_device == "gpu" else torch.device("cpu")
    o_ref, m_ref, l_ref = R.dmla_fwd_onthefly(q.to(dev), k.to(dev), v.to(dev), wk.to(dev), wv.to(dev), scale, causal)
    assert_out_close(o, o_ref)
    dm, dl = assert_stats_close(m, l, m_ref, l_ref)
    print(f"on-the-fly B={B} H={H} Sq={Sq} Sk={Sk}: m max-abs {dm:.2e}, l max-rel {dl:.2e}")
    return o


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B,H,Sq,Sk,causal",
    [
        (1, 2, 64, 64, True),       # one key tile
        (2, 4, 600, 600, True),     # two 512-row query tiles, ragged keys
        (1, 3, 100, 300, False),    # non-causal, Sq < Sk
        (1, 2, 130, 500, True),     # bottom-right aligned causal
        (1, 2, 150, 40, True),      # Sq > Sk: leading rows see no key
        (1, 1, 1, 1, True),         # single token
    ],
)
def test_otf_small_shapes(gpu, B, H, Sq, Sk, causal):
    _check(gpu, B, H, Sq, Sk, causal, seed=B * 100 + H * 10 + Sq)


@pytest.mark.gpu
def test_otf_score_growth_moves_the_reference(gpu):
    # Scores grow along the keys, so the running reference max moves many times.
    B, H, S = 1, 2, 700
    q, k, v, wk, wv = _inputs(B, H, S, S, seed=9)
    ramp = torch.linspace(0.0, 6.0, S).view(1, S, 1, 1)
    k = (k.float() * 0.2 + ramp).to(torch.bfloat16)
    q = (q.float().abs()).to(torch.bfloat16)
    o = ops.flash_dmla_fwd_onthefly(q.to(gpu), k.to(gpu), v.to(gpu), wk.to(gpu), wv.to(gpu), 0.125, True)
    o_ref, _, _ = R.dmla_fwd_onthefly(q, k, v, wk, wv, 0.125, True)
    assert_out_close(o, o_ref)


@pytest.mark.gpu
def test_otf_config4_full_shape(gpu):
    # benchmark config 4: B=2, H=32, S=4096, causal; the oracle runs in fp32 on the GPU.
    _check(gpu, 2, 32, 4096, 4096, True, seed=0, ref_device="gpu")


@pytest.mark.gpu
def test_otf_strided_views(gpu):
    q, k, v, wk, wv = _inputs(1, 4, 200, 200, seed=13)
    kb = torch.cat([k, k], dim=-1)[..., :128]   # non-contiguous head / row strides
    qb = torch.cat([q, q], dim=-1)[..., 64:]
    o = ops.flash_dmla_fwd_onthefly(qb.to(gpu), kb.to(gpu), v.to(gpu), wk.to(gpu), wv.to(gpu), 0.125, True)
    o_ref, _, _ = R.dmla_fwd_onthefly(q, k, v, wk, wv, 0.125, True)
    assert_out_close(o, o_ref)
