"""Parity of the cache-latent backward (dmla_bwd_cache_latent) with fp32 references.

Each case runs this library's forward, then its backward from the saved (o, m, l), and checks
dq and dk_lat twice:
  * against the closed-form oracle backward fed with the same o, m, l -- isolates the
    backward kernels;
  * against fp32 torch.autograd through the exact forward -- the end-to-end gradient the
    baseline config 5 names.
Both at the north-star tolerance (max-abs 2e-2, mean-rel 1e-2).  dk_lat is compared in fp32,
the op's default output type: its largest entries (a key seen by every later row of all heads
collects sum_i P_ij dO_i over thousands of rows) reach ~20 at config 5, where a bf16 rounding
alone is 0.06.  dO ~ N(0, 1) as in config 5.
"""
import math

import pytest
import torch

from conftest import OUT_MAX_ABS, assert_out_close, seeded
from oracle import dmla_ref as R
from python import ops

SCALE = 1.0 / math.sqrt(192.0)


def _inputs(B, H, Sq, Sk, seed, scale=0.5):
    q = seeded((B, H, Sq, 576), seed, scale, torch.bfloat16)
    k = seeded((B, Sk, 576), seed + 1, scale, torch.bfloat16)
    do = seeded((B, H, Sq, 512), seed + 2, 1.0, torch.bfloat16)
    return q, k, do


def _run(gpu, q, k, do, causal, scale=SCALE, **kw):
    qg, kg, dog = q.to(gpu), k.to(gpu), do.to(gpu)
    o, m, l = ops.flash_dmla_fwd(qg, kg, 512, scale, causal)
    dq, dk = ops.flash_dmla_bwd(qg, kg, o, dog, m, l, 512, scale, causal, **kw)
    torch.cuda.synchronize()
    return o, m, l, dq, dk


def _check(gpu, q, k, do, causal, scale=SCALE, ref_device="cpu", autograd=True):
    o, m, l, dq, dk = _run(gpu, q, k, do, causal, scale)
    assert dq.dtype == torch.bfloat16 and dk.dtype == torch.float32
    dev = gpu if ref_device == "gpu" else torch.device("cpu")
    qf, kf, dof = q.to(dev).float(), k.to(dev).float(), do.to(dev).float()
    dq_ref, dk_ref = R.dmla_bwd_cache_latent(qf, kf, o.to(dev).float(), dof, m.to(dev), l.to(dev), 512, scale,
                                             causal)
    # One key: every row that sees it has softmax 1 and the exact dS = dP - D is 0, so the exact
    # dq is 0.  What remains is rounding: D comes from the saved bf16 O, dP from V itself, in the
    # oracle as in the kernel.  Only the absolute bar applies to dq then (mean-rel against a
    # reference that is itself rounding noise means nothing), against fp32 autograd (exactly 0)
    # with the bf16 O's share (oracle - autograd) allowed, as test_bwd_single_key states.
    single_key = k.shape[1] == 1
    if single_key:
        err = (dq.float() - dq_ref.to(dq.device)).abs().max().item()
        assert err <= OUT_MAX_ABS, f"dq of a single key vs oracle backward: max-abs {err:.3e}"
    else:
        assert_out_close(dq, dq_ref, "dq vs oracle backward")
    assert_out_close(dk, dk_ref, "dk_lat vs oracle backward")
    if autograd:
        dq_ag, dk_ag = R.dmla_grads_autograd(qf, kf, dof, 512, scale, causal, torch.float32)
        if single_key:
            same_o = (dq_ref - dq_ag).abs().max().item()
            err = (dq.float() - dq_ag.to(dq.device)).abs().max().item()
            assert err <= same_o + OUT_MAX_ABS, f"dq of a single key vs fp32 autograd: max-abs {err:.3e}"
        else:
            assert_out_close(dq, dq_ag, "dq vs fp32 autograd")
        assert_out_close(dk, dk_ag, "dk_lat vs fp32 autograd")
    return dq, dk


@pytest.mark.gpu
@pytest.mark.parametrize("B,H,Sq", [(2, 33, 117), (1, 64, 1)])
def test_bwd_single_key(gpu, B, H, Sq):
    """One key seen by every row: softmax is exactly 1, so the exact dq and the rope dims of
    dk_lat are 0 (fp32 autograd gives 0 exactly), while dk_lat[:, :, :512] is the folded dV =
    sum of dO over rows and heads.  The kernel's dS = dP - D is pure rounding (the bf16 O against
    V itself), so its dq must stay within the absolute bar; a relative measure of it against the
    oracle's own rounding noise is meaningless, and the closed-form comparison is skipped."""
    q, k, do = _inputs(B, H, Sq, 1, seed=B * 1000 + H + Sq)
    _, _, _, dq, dk = _run(gpu, q, k, do, False)
    dq_ag, dk_ag = R.dmla_grads_autograd(q.float(), k.float(), do.float(), 512, SCALE, False, torch.float32)
    assert dq_ag.abs().max().item() == 0.0 and dk_ag[..., 512:].abs().max().item() == 0.0
    assert dq.float().abs().max().item() <= 2e-2, "dq of a single key"
    assert dk[..., 512:].abs().max().item() <= 2e-2, "rope dims of dk_lat of a single key"
    assert_out_close(dk[..., :512], dk_ag[..., :512], "folded dV of a single key")


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B,H,Sq,Sk,causal",
    [
        (1, 16, 64, 64, True),      # one key block (a pair with itself), two row tiles
        (1, 16, 128, 128, True),    # one key-block pair
        (2, 16, 200, 200, True),    # ragged rows and keys, several pairs
        (1, 3, 77, 77, True),       # heads not dividing the 32-row tile
        (1, 1, 130, 130, True),     # one head
        (2, 16, 96, 96, False),     # non-causal
        (1, 8, 100, 300, False),    # non-causal, Sq < Sk
        (1, 8, 40, 100, True),      # Sq < Sk: bottom-right aligned causal
        (1, 4, 150, 70, True),      # Sq > Sk: the first rows see no key and get no gradient
        (1, 128, 8, 8, True),       # many heads, few positions
    ],
)
def test_bwd_small_shapes(gpu, B, H, Sq, Sk, causal):
    q, k, do = _inputs(B, H, Sq, Sk, seed=B * 1000 + H * 10 + Sq)
    _check(gpu, q, k, do, causal)


@pytest.mark.gpu
def test_bwd_many_segments(gpu):
    # 16 key blocks, 8 pairs, up to 32 row segments per pair: work items that switch key block
    # mid-item and dK partials summed across segments.
    q, k, do = _inputs(1, 16, 1024, 1024, seed=11)
    _check(gpu, q, k, do, True, ref_device="gpu")


@pytest.mark.gpu
def test_bwd_strided_views_and_fp32_outputs(gpu):
    qb = seeded((2, 16, 70, 640), 7, 0.5, torch.bfloat16)
    kb = seeded((2, 70, 704), 8, 0.5, torch.bfloat16)
    dob = seeded((2, 16, 70, 576), 9, 1.0, torch.bfloat16)
    q, k, do = qb[..., :576], kb[..., 64:640], dob[..., 32:544]
    o, m, l, dq, dk = _run(gpu, q, k, do, True, dq_dtype=torch.float32, dk_dtype=torch.bfloat16)
    assert dq.dtype == torch.float32 and dk.dtype == torch.bfloat16
    dq_ref, dk_ref = R.dmla_bwd_cache_latent(q.float(), k.float(), o.cpu().float(), do.float(), m.cpu(), l.cpu(),
                                             512, SCALE, True)
    assert_out_close(dq, dq_ref, "dq fp32")
    # bf16 dk_lat: the tolerance plus 2^-9 relative, half of bf16's own rounding bound (2^-8).
    diff = (dk.float().cpu() - dk_ref).abs()
    assert (diff <= 2e-2 + dk_ref.abs() * 2.0 ** -9).all(), f"dk bf16 max diff {diff.max().item():.3e}"


@pytest.mark.gpu
def test_bwd_dq_row_stride_not_a_multiple_of_8(gpu):
    # A bf16 dq whose strides are multiples of 8 elements leaves as whole 16-byte pieces staged
    # through LDS; any other stride takes the per-element stores.  Both store the same rounded
    # accumulators, so a dq written into a [.., 577]-wide buffer equals the contiguous one bit
    # for bit (and the 577th column stays untouched).
    from python import _lib
    B, H, Sq, Sk = 1, 16, 200, 200
    q, k, do = (t.to(gpu) for t in _inputs(B, H, Sq, Sk, seed=77))
    o, m, l = ops.flash_dmla_fwd(q, k, 512, SCALE, True)
    dq_ref, dk_ref = ops.flash_dmla_bwd(q, k, o, do, m, l, 512, SCALE, True)
    wide = torch.full((B, H, Sq, 577), 7.0, dtype=torch.bfloat16, device=gpu)
    dq = wide[..., :576]
    dk = torch.empty_like(dk_ref)
    ws_bytes = int(_lib.lib().dmla_bwd_workspace_bytes(B, H, Sq, Sk, 576, 512, 1))
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=gpu)
    _lib.call(
        "dmla_bwd_cache_latent",
        ops._ptr(q), ops._ptr(k), ops._ptr(o), ops._ptr(do), ops._ptr(m), ops._ptr(l), ops._ptr(dq), ops._ptr(dk),
        B, H, Sq, Sk, 576, 512,
        q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1),
        o.stride(0), o.stride(1), o.stride(2), do.stride(0), do.stride(1), do.stride(2),
        dq.stride(0), dq.stride(1), dq.stride(2), dk.stride(0), dk.stride(1),
        0, 1, SCALE, 1, ops._ptr(ws), ws_bytes, ops._stream(q),
    )
    torch.cuda.synchronize()
    assert torch.equal(dq, dq_ref), "strided bf16 dq differs from the contiguous one"
    assert torch.equal(dk, dk_ref)
    assert (wide[..., 576] == 7.0).all(), "the column past dq was written"


@pytest.mark.gpu
def test_bwd_config5_full_shape(gpu):
    # benchmark config 5: B=4, H=16, S=2048, causal, dO ~ N(0, 1); references in fp32 on the GPU.
    q, k, do = _inputs(4, 16, 2048, 2048, seed=0)
    _check(gpu, q, k, do, True, ref_device="gpu")


@pytest.mark.gpu
def test_bwd_is_deterministic(gpu):
    q, k, do = _inputs(2, 16, 300, 300, seed=21)
    _, _, _, dq1, dk1 = _run(gpu, q, k, do, True)
    _, _, _, dq2, dk2 = _run(gpu, q, k, do, True)
    assert torch.equal(dq1, dq2) and torch.equal(dk1, dk2)


@pytest.mark.gpu
@pytest.mark.parametrize("shift", [20, 40])
def test_bwd_small_gradients_scale_exactly(gpu, shift):
    """Gradients as small as training produces (|dO| ~ 1e-6 and far below).  The fp16 operands of
    the second-stage products would turn such values into subnormals; the backward instead scales
    dO and dS' by a power of two chosen on the device from max |dO| and the results back, so
    dO 2^-shift yields exactly 2^-shift times the gradients of dO, bit for bit, and the parity of
    the unscaled case carries over at every scale."""
    q, k, do = _inputs(1, 16, 256, 256, seed=41)
    small = (do.float() * 2.0 ** -shift).to(torch.bfloat16)   # exact: a power of two
    _, _, _, dq, dk = _run(gpu, q, k, do, True)
    _, _, _, dqs, dks = _run(gpu, q, k, small, True)
    assert dk.abs().max().item() > 0.1
    assert torch.equal(dqs.float() * 2.0 ** shift, dq.float()), "dq of a scaled dO"
    assert torch.equal(dks * 2.0 ** shift, dk), "dk_lat of a scaled dO"


@pytest.mark.gpu
def test_bwd_zero_output_gradient_gives_zero(gpu):
    """dO = 0: the largest |dO| is 0, the gradient exponent stays 0, and every gradient is 0."""
    q, k, do = _inputs(1, 16, 200, 200, seed=43)
    _, _, _, dq, dk = _run(gpu, q, k, torch.zeros_like(do), True)
    assert int(torch.count_nonzero(dq)) == 0 and int(torch.count_nonzero(dk)) == 0


@pytest.mark.gpu
def test_autograd_function_matches_fp32_autograd(gpu):
    q, k, do = _inputs(1, 4, 96, 96, seed=31)
    qg = q.to(gpu).requires_grad_(True)
    kg = k.to(gpu).requires_grad_(True)
    out = ops.flash_dmla(qg, kg, 512, SCALE, True)
    out.backward(do.to(gpu))
    assert qg.grad.dtype == torch.bfloat16 and kg.grad.dtype == torch.bfloat16
    dq_ag, dk_ag = R.dmla_grads_autograd(q.float(), k.float(), do.float(), 512, SCALE, True, torch.float32)
    assert_out_close(qg.grad, dq_ag, "dq through autograd.Function")
    diff = (kg.grad.float().cpu() - dk_ag).abs()
    assert (diff <= 2e-2 + dk_ag.abs() * 2.0 ** -9).all(), f"dk bf16 max diff {diff.max().item():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize(
    "B,H,Sq,Sk,causal,dk_dtype",
    [
        (2, 4, 600, 600, True, torch.float32),    # many chunks, dk accumulated in the fp32 output
        (2, 4, 600, 600, True, torch.bfloat16),   # the same through the workspace accumulator
        (1, 3, 300, 500, True, torch.float32),    # bottom-right causal, heads not dividing a tile
        (1, 4, 200, 350, False, torch.float32),   # non-causal: every group holds every key block
    ],
)
def test_bwd_row_chunks(gpu, monkeypatch, B, H, Sq, Sk, causal, dk_dtype):
    # A 96 KB cap on dS' storage (the default is 2 GiB) cuts these rows into several chunks of
    # 128-row groups; each chunk's dq rows are final and dk_lat sums over the chunks.
    monkeypatch.setenv("DMLA_BWD_DS_CAP_BYTES", str(96 * 1024))
    from python import _lib
    small = _lib.lib().dmla_bwd_workspace_bytes(B, H, Sq, Sk, 576, 512, 1 if causal else 0)
    q, k, do = _inputs(B, H, Sq, Sk, seed=B * 7 + H * 3 + Sq)
    o, m, l, dq, dk = _run(gpu, q, k, do, causal, dk_dtype=dk_dtype)
    dq_ref, dk_ref = R.dmla_bwd_cache_latent(q.float(), k.float(), o.cpu().float(), do.float(), m.cpu(), l.cpu(),
                                             512, SCALE, causal)
    assert_out_close(dq, dq_ref, "dq (row chunks)")
    if dk_dtype == torch.float32:
        assert_out_close(dk, dk_ref, "dk_lat (row chunks)")
    else:
        diff = (dk.float().cpu() - dk_ref).abs()
        assert (diff <= 2e-2 + dk_ref.abs() * 2.0 ** -9).all(), f"dk bf16 max diff {diff.max().item():.3e}"
    # the same call without the cap (one chunk) agrees to fp32 summation-order differences
    monkeypatch.delenv("DMLA_BWD_DS_CAP_BYTES")
    assert _lib.lib().dmla_bwd_workspace_bytes(B, H, Sq, Sk, 576, 512, 1 if causal else 0) != small
    _, _, _, dq1, dk1 = _run(gpu, q, k, do, causal, dk_dtype=dk_dtype)
    assert torch.equal(dq, dq1), "dq rows do not depend on the chunking"
    # fp32 sums in another order: ~1e-6 in fp32, up to one bf16 step (2^-7 relative) in bf16
    tol = 1e-3 + dk1.float().abs() * (2.0 ** -7 if dk_dtype == torch.bfloat16 else 0.0)
    assert ((dk.float() - dk1.float()).abs() <= tol).all()


@pytest.mark.gpu
def test_bwd_long_sequence_is_chunked(gpu, monkeypatch):
    # S = 8192 (B = 1, H = 16): the causal dS' blocks alone are ~1.1 GB; under a 512 MiB cap
    # (the default 2 GiB holds them in one chunk) the rows run in three chunks; references in
    # fp32 on the GPU.
    from python import _lib
    monkeypatch.setenv("DMLA_BWD_DS_CAP_BYTES", str(512 << 20))
    ws = _lib.lib().dmla_bwd_workspace_bytes(1, 16, 8192, 8192, 576, 512, 1)
    assert ws < (512 << 20) + (200 << 20), ws
    q, k, do = _inputs(1, 16, 8192, 8192, seed=5)
    _check(gpu, q, k, do, True, ref_device="gpu", autograd=False)
