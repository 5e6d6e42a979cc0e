"""Parity of the cache-latent prefill kernel (dmla_fwd_cache_latent) with the fp32 oracle.

Inputs are generated on the CPU from seeded generators and cast to bf16; the oracle consumes
the bf16->fp32 upcasts, so both sides see bit-identical data.  Small cases run the oracle on
the CPU; the full benchmark config 2 shape runs the same oracle code on the GPU in fp32.
"""
import math

import pytest
import torch

from conftest import assert_out_close, assert_stats_close, seeded
from oracle import dmla_ref as R
from python import ops

SCALE = 1.0 / math.sqrt(192.0)


def _inputs(B, H, Sq, Sk, seed, scale=0.5):
    q = seeded((B, H, Sq, 576), seed, scale, torch.bfloat16)
    k = seeded((B, Sk, 576), seed + 1, scale, torch.bfloat16)
    return q, k


def _check(gpu, q, k, causal, scale=SCALE, oracle_device="cpu"):
    o, m, l = ops.flash_dmla_fwd(q.to(gpu), k.to(gpu), 512, scale, causal)
    torch.cuda.synchronize()
    dev = gpu if oracle_device == "gpu" else "cpu"
    o_ref, m_ref, l_ref = R.dmla_fwd_cache_latent(q.to(dev).float(), k.to(dev).float(), 512, scale, causal)
    assert_out_close(o, o_ref)
    assert_stats_close(m, l, m_ref, l_ref)


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B,H,Sq,Sk,causal",
    [
        (1, 16, 64, 64, True),     # exactly one 64-row tile, two key tiles
        (2, 16, 200, 200, True),   # ragged: S not a multiple of the tile
        (1, 3, 77, 77, True),      # heads not dividing the 64-row workgroup
        (1, 1, 130, 130, True),    # one head: the workgroup spans 64 positions
        (2, 16, 96, 96, False),    # non-causal
        (1, 8, 40, 100, True),     # Sq < Sk: bottom-right aligned causal
        (1, 4, 50, 30, True),      # Sq > Sk: first rows have no key (o = 0, m = -inf, l = 0)
        (1, 128, 1, 1, True),      # single token
    ],
)
def test_fwd_small_shapes(gpu, B, H, Sq, Sk, causal):
    q, k = _inputs(B, H, Sq, Sk, seed=B * 1000 + H * 10 + Sq)
    _check(gpu, q, k, causal)


@pytest.mark.gpu
def test_fwd_strided_views(gpu):
    # q and k_lat as views into wider buffers (row strides > 576).
    qb = seeded((2, 16, 70, 640), 7, 0.5, torch.bfloat16)
    kb = seeded((2, 70, 704), 8, 0.5, torch.bfloat16)
    q, k = qb[..., :576], kb[..., 64:640]
    o, m, l = ops.flash_dmla_fwd(q.to(gpu), k.to(gpu), 512, SCALE, True)
    o_ref, m_ref, l_ref = R.dmla_fwd_cache_latent(q.float(), k.float(), 512, SCALE, True)
    assert_out_close(o, o_ref)
    assert_stats_close(m, l, m_ref, l_ref)


@pytest.mark.gpu
def test_fwd_score_growth_takes_the_exact_max_pass(gpu):
    # Scores grow along the keys by far more than the 2^32 headroom over the first tile's max,
    # forcing the recompute-with-exact-max path of the kernel.
    B, H, S = 1, 16, 256
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, H, S, 576, generator=g) * 0.1
    k = torch.randn(B, S, 576, generator=g) * 0.1
    q[..., 512] = 4.0
    k[..., 512] = torch.linspace(0.0, 30.0, S)
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    _check(gpu, q, k, True, scale=0.5)


@pytest.mark.gpu
def test_fwd_score_jump_in_the_last_tile(gpu):
    # Keys of the last 32-key tile score ~86 (log2 units) above all earlier keys: only rows
    # that reach that tile overflow, and only there -- the restart must still be taken.
    B, H, S = 1, 16, 256
    g = torch.Generator().manual_seed(6)
    q = torch.randn(B, H, S, 576, generator=g) * 0.1
    k = torch.randn(B, S, 576, generator=g) * 0.1
    q[..., 512] = 4.0
    k[..., 512] = 0.0
    k[:, S - 32:, 512] = 30.0
    q, k = q.to(torch.bfloat16), k.to(torch.bfloat16)
    _check(gpu, q, k, True, scale=0.5)


@pytest.mark.gpu
def test_fwd_config2_full_shape(gpu):
    # benchmark config 2: B=4, H=16, S=2048, 576/512, N(0,1)*0.5, scale 1/sqrt(192), causal.
    q, k = _inputs(4, 16, 2048, 2048, seed=2)
    _check(gpu, q, k, True, oracle_device="gpu")


@pytest.mark.gpu
def test_fwd_is_deterministic(gpu):
    q, k = _inputs(1, 16, 300, 300, seed=3)
    a = ops.flash_dmla_fwd(q.to(gpu), k.to(gpu), 512, SCALE, True)
    b = ops.flash_dmla_fwd(q.to(gpu), k.to(gpu), 512, SCALE, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
