"""torch.ops.flashdmla.*: the dispatcher-level entry points (CPU checks; the GPU parity of the
same ops is in test_torch_ops_gpu.py).

Every op is registered with its schema, infers output shapes and dtypes on meta tensors
(fake implementations, what tracing uses), and has no CPU kernel: a CPU tensor raises.
"""
import pytest
import torch

import python  # noqa: F401  (registers torch.ops.flashdmla.*)

OPS = ("fwd_cache_latent", "bwd_cache_latent", "fwd_onthefly", "bwd_onthefly", "decode_plan",
       "decode_paged", "kv_append", "lse_combine")
META = dict(device="meta")


def _t(shape, dtype=torch.bfloat16):
    return torch.empty(shape, dtype=dtype, **META)


def test_every_op_is_registered_with_its_schema():
    for name in OPS:
        assert hasattr(torch.ops.flashdmla, name), name
    s = str(torch.ops.flashdmla.kv_append.default._schema)
    assert "Tensor(a0!) kv_pool" in s, s   # the append writes the pool in place
    s = str(torch.ops.flashdmla.decode_paged.default._schema)
    assert "Tensor? plan" in s and "float? softmax_scale" in s, s


def test_fake_shapes_of_the_attention_ops():
    B, H, Sq, Sk = 2, 3, 5, 7
    q, k = _t((B, H, Sq, 576)), _t((B, Sk, 576))
    o, m, l = torch.ops.flashdmla.fwd_cache_latent(q, k, 512, None, True)
    assert (o.shape, o.dtype, m.shape, m.dtype, l.shape) == ((B, H, Sq, 512), torch.bfloat16, (B, H, Sq),
                                                             torch.float32, (B, H, Sq))
    dq, dk = torch.ops.flashdmla.bwd_cache_latent(q, k, o, o, m, l, 512, 0.1, True)
    assert (dq.shape, dq.dtype, dk.shape, dk.dtype) == (q.shape, torch.bfloat16, k.shape, torch.float32)

    qo, kk, vv, w = _t((B, H, Sq, 64)), _t((B, Sk, H, 128)), _t((B, Sk, H, 128)), _t((H, 128, 64))
    o, m, l = torch.ops.flashdmla.fwd_onthefly(qo, kk, vv, w, w, None, False)
    assert (o.shape, m.shape) == ((B, H, Sq, 64), (B, H, Sq))
    grads = torch.ops.flashdmla.bwd_onthefly(qo, kk, vv, w, w, o, o, m, l, 0.125, True)
    assert [tuple(g.shape) for g in grads] == [qo.shape, kk.shape, vv.shape, w.shape, w.shape]
    assert [g.dtype for g in grads] == [torch.bfloat16] * 3 + [torch.float32] * 2


def test_fake_shapes_of_the_decode_ops():
    B, H, P = 4, 128, 9
    sl = _t((B,), torch.int32)
    plan = torch.ops.flashdmla.decode_plan(sl, H, 16)
    assert plan.dtype == torch.int32 and plan.dim() == 1 and plan.numel() > 0
    o, lse = torch.ops.flashdmla.decode_paged(_t((B, H, 576)), _t((P, 64, 576)), _t((B, 16), torch.int32), sl,
                                              512, None, plan)
    assert (o.shape, o.dtype, lse.shape, lse.dtype) == ((B, H, 512), torch.bfloat16, (B, H), torch.float32)
    assert torch.ops.flashdmla.kv_append(_t((P, 64, 576)), _t((B, 16), torch.int32), sl, _t((B, 3, 576)), None) is None
    o, lse = torch.ops.flashdmla.lse_combine(_t((B, 5, H, 512), torch.float32), _t((B, 5, H), torch.float32), None)
    assert (o.shape, lse.shape) == ((B, H, 512), (B, H))


def test_cpu_tensors_have_no_kernel():
    q, k = torch.zeros(1, 1, 4, 576, dtype=torch.bfloat16), torch.zeros(1, 4, 576, dtype=torch.bfloat16)
    with pytest.raises(NotImplementedError):
        torch.ops.flashdmla.fwd_cache_latent(q, k, 512, None, True)
