"""Seeded random shapes through every op, against the same fp32 references as the per-op tests.

The per-op tests pick their shapes by hand (tile edges, ragged rows, head counts that do not
divide a tile, Sq != Sk).  These cases draw batch, heads, lengths, causality and, for decode,
per-sequence context lengths from a fixed seed, so each round runs the same shapes, which
cover combinations the hand-picked lists do not.  Each op is checked by its own test module's
helper, at the north-star tolerance (2e-2 max-abs / 1e-2 mean-rel, statistics 1e-3).
"""
import random

import pytest

import test_bwd_gpu as BW
import test_decode_gpu as D
import test_fwd_gpu as F
import test_otf_bwd_gpu as OB
import test_otf_gpu as OF


def _length(rng, hi):
    # half of the draws short (one or two tiles), half anywhere up to hi
    return rng.randint(1, min(hi, 70)) if rng.random() < 0.5 else rng.randint(1, hi)


def _cases(kind, n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        causal = rng.random() < 0.6
        if kind == "fwd":
            B, H = rng.randint(1, 3), rng.choice([1, 3, 7, 16, 17, 33, 100, 128])
            Sq, Sk = _length(rng, 400), _length(rng, 400)
            Sq = max(1, min(Sq, 60000 // (B * H)))
            out.append((B, H, Sq, Sk, causal))
        elif kind == "bwd":
            B, H = rng.randint(1, 2), rng.choice([1, 3, 5, 16, 17, 33, 64])
            Sq, Sk = _length(rng, 300), _length(rng, 300)
            Sq = max(1, min(Sq, 20000 // (B * H)))
            out.append((B, H, Sq, Sk, causal))
        elif kind == "decode":
            lens = [rng.choice([rng.randint(1, 200), rng.randint(1, 3000), 64 * rng.randint(1, 20)])
                    for _ in range(rng.randint(1, 12))]
            out.append((tuple(lens), rng.choice([1, 8, 48, 65, 96, 127, 128]), rng.randint(0, 3)))
        else:   # on-the-fly forward / backward
            hi = 600 if kind == "otf" else 300
            out.append((rng.randint(1, 2), rng.randint(1, 3), _length(rng, hi), _length(rng, hi), causal))
    return out


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,Sq,Sk,causal", _cases("fwd", 12, 101))
def test_random_fwd(gpu, B, H, Sq, Sk, causal):
    q, k = F._inputs(B, H, Sq, Sk, seed=B * 7919 + H * 31 + Sq)
    F._check(gpu, q, k, causal)


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,Sq,Sk,causal", _cases("bwd", 12, 102))
def test_random_bwd(gpu, B, H, Sq, Sk, causal):
    q, k, do = BW._inputs(B, H, Sq, Sk, seed=B * 7919 + H * 31 + Sq)
    BW._check(gpu, q, k, do, causal, autograd=False)


@pytest.mark.gpu
@pytest.mark.parametrize("lens,H,extra_pages", _cases("decode", 12, 103))
def test_random_decode(gpu, lens, H, extra_pages):
    q, pool, table, lt = D._paged(list(lens), H, seed=len(lens) * 131 + H, extra_pages=extra_pages)
    D._check(gpu, q, pool, table, lt)


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,Sq,Sk,causal", _cases("otf", 10, 104))
def test_random_onthefly_fwd(gpu, B, H, Sq, Sk, causal):
    OF._check(gpu, B, H, Sq, Sk, causal, seed=B * 7919 + H * 31 + Sq)


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,Sq,Sk,causal", _cases("otf_bwd", 10, 105))
def test_random_onthefly_bwd(gpu, B, H, Sq, Sk, causal):
    OB._check(gpu, B, H, Sq, Sk, causal, seed=B * 7919 + H * 31 + Sq, autograd=False)
