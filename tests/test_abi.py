"""The C ABI (include/flashdmla.h): the library loads, exports every declared entry point and
rejects bad arguments with a status and message -- all without touching a GPU.

Every call below returns before any kernel launch (argument errors, missing workspace or an
empty problem), so the fake device pointers are never dereferenced."""
import ctypes
import os
import re

import pytest
import torch

from conftest import ROOT

from python import _lib, ops

HEADER = os.path.join(ROOT, "include", "flashdmla.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dmla_[a-z0-9_]+)\s*\(", text)))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = declared_functions()
    assert "dmla_fwd_cache_latent" in names and "dmla_decode_paged" in names
    for n in names:
        assert hasattr(lib, n), f"{n} declared in flashdmla.h but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature in python/_lib.py"
    assert lib.dmla_version() >= 100


def _fwd(**kw):
    args = dict(q=1 << 20, k=1 << 20, o=1 << 20, m=None, l=None, B=1, H=16, Sq=8, Sk=8, dqk=576, dv=512,
                scale=0.07, causal=1)
    args.update(kw)
    P = ctypes.c_void_p
    return _lib.lib().dmla_fwd_cache_latent(
        P(args["q"]), P(args["k"]), P(args["o"]), P(args["m"]), P(args["l"]),
        args["B"], args["H"], args["Sq"], args["Sk"], args["dqk"], args["dv"],
        16 * 8 * 576, 8 * 576, 576, 8 * 576, 576, 16 * 8 * 512, 8 * 512, 512,
        args["scale"], args["causal"], None)


def test_fwd_argument_errors():
    assert _fwd(q=None) == _lib.DMLA_ERR_INVALID_ARG
    assert b"null" in _lib.lib().dmla_last_error()
    assert _fwd(dqk=64, dv=32) == _lib.DMLA_ERR_UNSUPPORTED
    assert _fwd(scale=-1.0) == _lib.DMLA_ERR_INVALID_ARG
    assert _fwd(scale=float("inf")) == _lib.DMLA_ERR_INVALID_ARG
    assert _fwd(q=(1 << 20) + 2) == _lib.DMLA_ERR_INVALID_ARG  # misaligned
    assert _fwd(m=1 << 20) == _lib.DMLA_ERR_INVALID_ARG        # m without l
    assert _fwd(B=-1) == _lib.DMLA_ERR_INVALID_ARG
    # Empty problems succeed without launching anything.
    assert _fwd(B=0) == _lib.DMLA_OK
    assert _fwd(Sq=0) == _lib.DMLA_OK
    assert _lib.lib().dmla_last_error() == b""


def test_decode_argument_errors():
    P = ctypes.c_void_p
    lib = _lib.lib()

    def call(**kw):
        a = dict(q=1 << 20, kv=1 << 20, bt=1 << 20, sl=1 << 20, o=1 << 20, B=2, H=128, dqk=576, dv=512,
                 page=64, num_pages=10, max_pages=4, bt_sb=4, ws=None, ws_bytes=0)
        a.update(kw)
        return lib.dmla_decode_paged(P(a["q"]), P(a["kv"]), P(a["bt"]), P(a["sl"]), P(a["o"]), None,
                                     a["B"], a["H"], a["dqk"], a["dv"], a["page"], a["num_pages"], a["max_pages"],
                                     128 * 576, 576, 64 * 576, 576, a["bt_sb"], 128 * 512, 512, 0.07,
                                     P(a["ws"]), a["ws_bytes"], None)

    assert call(bt=None) == _lib.DMLA_ERR_INVALID_ARG
    assert call(page=32) == _lib.DMLA_ERR_UNSUPPORTED
    assert call(bt_sb=2) == _lib.DMLA_ERR_INVALID_ARG
    assert call(num_pages=0) == _lib.DMLA_ERR_INVALID_ARG
    assert call(B=0) == _lib.DMLA_OK
    need = lib.dmla_decode_workspace_bytes(64, 128, 512, 128)
    assert need > 0
    assert call(B=64, max_pages=128, bt_sb=128) == _lib.DMLA_ERR_WORKSPACE


def test_python_wrappers_reject_cpu_tensors_and_bad_shapes():
    q = torch.zeros(1, 16, 8, 576, dtype=torch.bfloat16)
    k = torch.zeros(1, 8, 576, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        ops.flash_dmla_fwd(q, k)
    with pytest.raises(ValueError):
        ops.flash_dmla_fwd(q.float(), k)
    with pytest.raises(ValueError):
        ops.flash_dmla_decode_paged(q[:, :, 0], k, torch.zeros(1, 1, dtype=torch.int32),
                                    torch.ones(1, dtype=torch.int32))


def test_error_message_is_raised_as_exception():
    with pytest.raises(_lib.DmlaUnsupported, match="576"):
        _lib.check("dmla_fwd_cache_latent", _fwd(dqk=64, dv=32))


def _bwd(ws_bytes=None, **kw):
    args = dict(q=1 << 20, k=1 << 20, o=1 << 20, do=1 << 20, m=1 << 20, l=1 << 20, dq=1 << 20, dk=1 << 20,
                B=1, H=16, Sq=64, Sk=64, dqk=576, dv=512, scale=0.07, causal=1, ws=1 << 20)
    args.update(kw)
    P = ctypes.c_void_p
    lib = _lib.lib()
    need = lib.dmla_bwd_workspace_bytes(args["B"], args["H"], args["Sq"], args["Sk"], args["dqk"], args["dv"],
                                        args["causal"])
    return lib.dmla_bwd_cache_latent(
        P(args["q"]), P(args["k"]), P(args["o"]), P(args["do"]), P(args["m"]), P(args["l"]), P(args["dq"]),
        P(args["dk"]), args["B"], args["H"], args["Sq"], args["Sk"], args["dqk"], args["dv"],
        16 * 64 * 576, 64 * 576, 576, 64 * 576, 576, 16 * 64 * 512, 64 * 512, 512, 16 * 64 * 512, 64 * 512, 512,
        16 * 64 * 576, 64 * 576, 576, 64 * 576, 576, 0, 1, args["scale"], args["causal"], P(args["ws"]),
        need - 256 if ws_bytes is None else ws_bytes, None)


def test_bwd_workspace_query_and_argument_errors():
    lib = _lib.lib()
    need = lib.dmla_bwd_workspace_bytes(1, 16, 64, 64, 576, 512, 1)
    assert need > 0 and need % 256 == 0
    assert lib.dmla_bwd_workspace_bytes(1, 16, 64, 64, 64, 32, 1) == 0       # unsupported dims
    assert lib.dmla_bwd_workspace_bytes(0, 16, 64, 64, 576, 512, 1) == 0     # empty problem
    # The workspace holds the dS' blocks of every (16-row, 16-key) pair: at least 2 bytes per
    # (row, key) of the problem.
    assert lib.dmla_bwd_workspace_bytes(1, 16, 512, 512, 576, 512, 1) >= 2 * 16 * 512 * 512
    assert _bwd() == _lib.DMLA_ERR_WORKSPACE                                 # 256 bytes short
    assert b"workspace" in lib.dmla_last_error()
    assert _bwd(q=None) == _lib.DMLA_ERR_INVALID_ARG
    assert _bwd(m=(1 << 20) + 4) == _lib.DMLA_ERR_INVALID_ARG                # misaligned m
    assert _bwd(dqk=64, dv=32) == _lib.DMLA_ERR_UNSUPPORTED
    assert _bwd(scale=0.0) == _lib.DMLA_ERR_INVALID_ARG
    assert _bwd(Sk=0, ws_bytes=0) == _lib.DMLA_ERR_INVALID_ARG
    assert _bwd(B=0, ws_bytes=0) == _lib.DMLA_OK                             # empty: nothing launched
    assert lib.dmla_last_error() == b""


def test_bwd_python_wrapper_rejects_cpu_tensors():
    q = torch.zeros(1, 2, 4, 576, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 576, dtype=torch.bfloat16)
    o = torch.zeros(1, 2, 4, 512, dtype=torch.bfloat16)
    m = torch.zeros(1, 2, 4)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.flash_dmla_bwd(q, k, o, o, m, m)


def test_kv_append_and_combine_argument_errors():
    lib = _lib.lib()
    P = ctypes.c_void_p

    def append(**kw):
        a = dict(pool=1 << 20, bt=1 << 20, sl=1 << 20, new=1 << 20, B=2, n=3, d=576, ps=64, npg=10, mp=4,
                 kv_sp=64 * 576, kv_ss=576, bt_sb=4)
        a.update(kw)
        return lib.dmla_kv_append(P(a["pool"]), P(a["bt"]), P(a["sl"]), None, P(a["new"]), None, a["B"], a["n"],
                                  a["d"], a["ps"], a["npg"], a["mp"], a["kv_sp"], a["kv_ss"], a["bt_sb"],
                                  3 * 576, 576, None)
    assert append(pool=None) == _lib.DMLA_ERR_INVALID_ARG
    assert append(d=12) == _lib.DMLA_ERR_UNSUPPORTED
    assert append(kv_ss=8) == _lib.DMLA_ERR_INVALID_ARG           # row stride below d
    assert append(bt_sb=2) == _lib.DMLA_ERR_INVALID_ARG           # table stride below max pages
    assert append(new=(1 << 20) + 8) == _lib.DMLA_ERR_INVALID_ARG  # misaligned
    assert append(n=0) == _lib.DMLA_OK and append(B=0) == _lib.DMLA_OK

    def combine(**kw):
        a = dict(po=1 << 20, pl=1 << 20, o=1 << 20, B=2, H=4, S=3, d=512)
        a.update(kw)
        return lib.dmla_lse_combine(P(a["po"]), P(a["pl"]), None, P(a["o"]), None, a["B"], a["H"], a["S"], a["d"],
                                    3 * 4 * 512, 4 * 512, 512, 12, 4, 1, 4 * 512, 512, None)
    assert combine(po=None) == _lib.DMLA_ERR_INVALID_ARG
    assert combine(S=0) == _lib.DMLA_ERR_INVALID_ARG
    assert combine(d=6) == _lib.DMLA_ERR_UNSUPPORTED
    assert combine(B=1 << 16, H=1 << 15) == _lib.DMLA_ERR_UNSUPPORTED   # B * H = 2^31, before any launch
    assert combine(B=0) == _lib.DMLA_OK


def test_onthefly_bwd_workspace_query_and_argument_errors():
    lib = _lib.lib()
    P = ctypes.c_void_p
    need = lib.dmla_bwd_onthefly_workspace_bytes(2, 4, 100, 300, 128, 64)
    assert need > 0 and need % 256 == 0
    # per padded key: fp16 K_lat and V_lat, dK_lat and dV_lat as bf16 hi and lo planes; lse2
    # and -D per padded row
    assert need >= 6 * 2 * 4 * 384 * 64 * 2 + 2 * 2 * 4 * 128 * 4
    assert lib.dmla_bwd_onthefly_workspace_bytes(2, 4, 100, 300, 64, 64) == 0      # unsupported d_in
    assert lib.dmla_bwd_onthefly_workspace_bytes(0, 4, 100, 300, 128, 64) == 0     # empty problem
    assert lib.dmla_bwd_onthefly_workspace_bytes(1, 1, 1 << 25, 8, 128, 64) == 0   # above 2^24

    def call(ws_short=256, **kw):
        a = dict(q=1 << 20, dq=1 << 20, m=1 << 20, B=1, H=2, Sq=64, Sk=64, din=128, dlat=64, scale=0.125, ks=2 * 128,
                 ws=1 << 20)
        a.update(kw)
        ok = lib.dmla_bwd_onthefly_workspace_bytes(a["B"], a["H"], a["Sq"], a["Sk"], 128, 64)
        ptrs = [P(a["q"])] + [P(1 << 20)] * 6 + [P(a["m"]), P(1 << 20), P(a["dq"])] + [P(1 << 20)] * 4
        return lib.dmla_bwd_onthefly(
            *ptrs, a["B"], a["H"], a["Sq"], a["Sk"], a["din"], a["dlat"],
            2 * 64 * 64, 64 * 64, 64, 64 * a["ks"], a["ks"], 128, 64 * a["ks"], a["ks"], 128, 128 * 64, 64,
            2 * 64 * 64, 64 * 64, 64, 2 * 64 * 64, 64 * 64, 64, 2 * 64 * 64, 64 * 64, 64,
            64 * 256, 256, 128, 128 * 64, 64, 0, 0, 1, a["scale"], 1, P(a["ws"]), max(ok - ws_short, 0), None)

    assert call() == _lib.DMLA_ERR_WORKSPACE                         # 256 bytes short
    assert b"workspace" in lib.dmla_last_error()
    assert call(q=None) == _lib.DMLA_ERR_INVALID_ARG
    assert call(dq=(1 << 20) + 2) == _lib.DMLA_ERR_INVALID_ARG       # misaligned
    assert call(ks=2 * 128 + 4) == _lib.DMLA_ERR_INVALID_ARG         # k row stride not a multiple of 8
    assert call(din=64) == _lib.DMLA_ERR_UNSUPPORTED
    assert call(scale=0.0) == _lib.DMLA_ERR_INVALID_ARG
    assert call(Sk=0) == _lib.DMLA_ERR_INVALID_ARG
    assert call(Sq=1 << 25) == _lib.DMLA_ERR_UNSUPPORTED
    assert call(ks=1 << 24) == _lib.DMLA_ERR_UNSUPPORTED               # row stride past the copy offsets
    assert call(B=0, ws_short=0) == _lib.DMLA_OK                     # empty: nothing launched
    assert lib.dmla_last_error() == b""


def test_onthefly_bwd_python_wrapper_rejects_cpu_tensors():
    q = torch.zeros(1, 2, 4, 64, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 2, 128, dtype=torch.bfloat16)
    w = torch.zeros(2, 128, 64, dtype=torch.bfloat16)
    m = torch.zeros(1, 2, 4)
    with pytest.raises(ValueError, match="GPU tensor"):
        ops.flash_dmla_bwd_onthefly(q, k, k, w, w, q, q, m, m)


def test_latent_range_check_bounds_the_projection():
    # The on-the-fly backward's dQ kernel stores K_lat * scale * log2(e) and V_lat in fp16;
    # check_range bounds them by max_s sum_i |x_i| * max |w| before any launch.
    x = torch.ones(1, 3, 2, 128)
    w = torch.full((2, 128, 64), 0.5)
    ops._check_latent_range("k", x, w, 1.0)              # 128 * 0.5 = 64
    w[1, 5, 7] = 600.0
    with pytest.raises(ValueError, match="k's projection"):
        ops._check_latent_range("k", x, w, 1.0)          # head 1: 128 * 600 > 65504
    ops._check_latent_range("k", x, w, 0.5)              # scaled below the bound


def test_fp16_range_check_rejects_values_the_kernels_would_saturate():
    # The on-the-fly forward and both backwards convert their operands to fp16; with
    # check_range=True the wrappers refuse inputs beyond fp16's range or non-finite ones.
    ok = torch.tensor([0.5, -65280.0, 3.0])  # the largest bf16 below 65504.to(torch.bfloat16)
    ops._check_fp16_range("q", ok)
    ops._check_fp16_range("q", ok[:0])
    for bad in ([1.0, 70000.0], [float("nan"), 1.0], [-float("inf")]):
        with pytest.raises(ValueError, match="fp16's finite range"):
            ops._check_fp16_range("q", torch.tensor(bad).to(torch.bfloat16))


def test_same_device_check_names_the_tensors_on_other_devices():
    # Every op checks that its tensors share one device before any launch (absent optional
    # tensors are skipped).
    a, b = torch.zeros(2), torch.zeros(2, device="meta")
    ops._same_device(q=a, k=torch.ones(3), plan=None)
    with pytest.raises(ValueError, match="k on meta"):
        ops._same_device(q=a, k=b)


def test_onthefly_forward_argument_errors():
    lib = _lib.lib()
    P = ctypes.c_void_p

    def call(ks=128 * 2, vs=128 * 2, din=128, B=1):
        ptrs = [P(1 << 20)] * 6 + [P(1 << 20), P(1 << 20)]
        return lib.dmla_fwd_onthefly(*ptrs, B, 2, 64, 64, din, 64, 2 * 64 * 64, 64 * 64, 64,
                                     64 * ks, ks, 128, 64 * vs, vs, 128, 128 * 64, 64,
                                     2 * 64 * 64, 64 * 64, 64, 0.125, 1, None)

    assert call(din=64) == _lib.DMLA_ERR_UNSUPPORTED
    assert call(ks=1 << 24) == _lib.DMLA_ERR_UNSUPPORTED   # the copies' 32-bit lane offsets
    assert call(vs=1 << 24) == _lib.DMLA_ERR_UNSUPPORTED
    assert call(ks=2 * 128 + 4) == _lib.DMLA_ERR_INVALID_ARG
    assert call(B=0) == _lib.DMLA_OK                        # empty: nothing launched


def test_onthefly_forward_wrapper_takes_check_range():
    import inspect
    assert "check_range" in inspect.signature(ops.flash_dmla_fwd_onthefly).parameters


def test_bwd_workspace_grows_linearly_with_the_sequence():
    # dS' storage covers only the causal blocks and is capped (row chunks past the cap), so the
    # workspace no longer grows as S^2: ~linear terms (K^T, statistics, partials) plus the cap.
    lib = _lib.lib()
    ws = {S: lib.dmla_bwd_workspace_bytes(4, 16, S, S, 576, 512, 1) for S in (2048, 8192, 16384, 65536)}
    full_square = lambda S: 4 * 16 * S * S * 2        # the former layout's dS' alone
    assert ws[2048] < 0.75 * full_square(2048) + (200 << 20)
    assert ws[65536] < 5 * ws[16384]                  # S^2 growth would be 16x
    assert ws[65536] < (5 << 30) and full_square(65536) > (500 << 30)
    non_causal = lib.dmla_bwd_workspace_bytes(4, 16, 2048, 2048, 576, 512, 0)
    assert non_causal > ws[2048]
