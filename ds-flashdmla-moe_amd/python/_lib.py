"""ctypes binding of ``libflashdmla.so``, the C ABI declared in ``include/flashdmla.h``.

The shared library is built in-tree (``ds-flashdmla-moe_amd/libflashdmla.so``) by
``make -C ds-flashdmla-moe_amd/csrc`` or ``__graft_entry__.build()``.  There is no fallback:
every op fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
PKG_ROOT = os.path.dirname(_HERE)
# DMLA_LIBRARY names another build of the same ABI (the sanitizer build of csrc/Makefile).
LIB_PATH = os.environ.get("DMLA_LIBRARY") or os.path.join(PKG_ROOT, "libflashdmla.so")

DMLA_OK = 0
DMLA_ERR_INVALID_ARG = -1
DMLA_ERR_UNSUPPORTED = -2
DMLA_ERR_WORKSPACE = -3
DMLA_ERR_HIP = -4


class DmlaError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, name: str, code: int, message: str):
        super().__init__(f"{name} failed with status {code}: {message}")
        self.code = code


class DmlaInvalidArgument(DmlaError, ValueError):
    pass


class DmlaUnsupported(DmlaError, NotImplementedError):
    pass


_i64 = ctypes.c_int64
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float
_int = ctypes.c_int

# name -> (restype, argtypes); mirrors include/flashdmla.h exactly.
SIGNATURES = {
    "dmla_version": (_int, []),
    "dmla_last_error": (ctypes.c_char_p, []),
    "dmla_fwd_cache_latent": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr]  # q, k_lat, o, m, l
        + [_i64] * 6  # B, H, Sq, Sk, d_qk, d_v
        + [_i64] * 8  # q_sb q_sh q_ss k_sb k_ss o_sb o_sh o_ss
        + [_f32, _int, _ptr],  # scale, causal, stream
    ),
    "dmla_fwd_onthefly": (
        _int,
        [_ptr] * 8  # q, k, v, wk, wv, o, m, l
        + [_i64] * 6  # B, H, Sq, Sk, d_in, d_lat
        + [_i64] * 14  # q(3) k(3) v(3) w(2) o(3) strides
        + [_f32, _int, _ptr],  # scale, causal, stream
    ),
    "dmla_decode_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "dmla_decode_paged": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr]  # q, kv_pool, block_table, seqlens, o, lse
        + [_i64] * 7  # B, H, d_qk, d_v, page_size, num_pages, max_pages_per_seq
        + [_i64] * 7  # q_sb q_sh kv_sp kv_ss bt_sb o_sb o_sh
        + [_f32, _ptr, _i64, _ptr],  # scale, workspace, workspace_bytes, stream
    ),
    "dmla_decode_paged_noalloc": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr]  # q, kv_pool, block_table, seqlens, o, lse
        + [_i64] * 7  # B, H, d_qk, d_v, page_size, num_pages, max_pages_per_seq
        + [_i64] * 7  # q_sb q_sh kv_sp kv_ss bt_sb o_sb o_sh
        + [_f32, _ptr],  # scale, stream
    ),
    "dmla_decode_plan_bytes": (_i64, [_i64, _i64, _i64]),
    "dmla_decode_plan": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr]),
    "dmla_decode_paged_planned": (
        _int,
        [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr]  # q, kv_pool, block_table, seqlens, o, lse
        + [_i64] * 7  # B, H, d_qk, d_v, page_size, num_pages, max_pages_per_seq
        + [_i64] * 7  # q_sb q_sh kv_sp kv_ss bt_sb o_sb o_sh
        + [_f32, _ptr, _ptr, _i64, _ptr],  # scale, plan, workspace, workspace_bytes, stream
    ),
    "dmla_kv_append": (
        _int,
        [_ptr] * 6  # kv_pool, block_table, cache_seqlens, new_lens, new_kv, bad_index_flag
        + [_i64] * 6  # B, n_new, d, page_size, num_pages, max_pages_per_seq
        + [_i64] * 5  # kv_sp kv_ss bt_sb nk_sb nk_ss
        + [_ptr],  # stream
    ),
    "dmla_lse_combine": (
        _int,
        [_ptr] * 5  # part_o, part_lse, num_splits, o, lse
        + [_i64] * 4  # B, H, max_splits, d
        + [_i64] * 8  # po_sb po_ss po_sh lse_sb lse_ss lse_sh o_sb o_sh
        + [_ptr],  # stream
    ),
    "dmla_bwd_workspace_bytes": (_i64, [_i64] * 6 + [_int]),  # B H Sq Sk d_qk d_v causal
    "dmla_bwd_cache_latent": (
        _int,
        [_ptr] * 8  # q, k_lat, o, dout, m, l, dq, dk_lat
        + [_i64] * 6  # B, H, Sq, Sk, d_qk, d_v
        + [_i64] * 16  # q(3) k(2) o(3) dout(3) dq(3) dk(2) strides
        + [_int, _int, _f32, _int, _ptr, _i64, _ptr],  # dq_fp32 dk_fp32 scale causal ws ws_bytes stream
    ),
    "dmla_bwd_onthefly_workspace_bytes": (_i64, [_i64] * 6),  # B H Sq Sk d_in d_lat
    "dmla_bwd_onthefly": (
        _int,
        [_ptr] * 14  # q, k, v, wk, wv, o, dout, m, l, dq, dk, dv, dwk, dwv
        + [_i64] * 6  # B, H, Sq, Sk, d_in, d_lat
        + [_i64] * 25  # q(3) k(3) v(3) w(2) o(3) dout(3) dq(3) dk(3) dw(2) strides
        + [_int] * 3  # dq_fp32 dkv_fp32 dw_fp32
        + [_f32, _int, _ptr, _i64, _ptr],  # scale causal ws ws_bytes stream
    ),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads the shared library once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `make -C {os.path.join(PKG_ROOT, 'csrc')}` "
                "or __graft_entry__.build()"
            )
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def check(name: str, rc: int) -> None:
    """Turns a C-ABI status into an exception carrying dmla_last_error()."""
    if rc == DMLA_OK:
        return
    msg = (lib().dmla_last_error() or b"").decode(errors="replace")
    if rc == DMLA_ERR_INVALID_ARG:
        raise DmlaInvalidArgument(name, rc, msg)
    if rc == DMLA_ERR_UNSUPPORTED:
        raise DmlaUnsupported(name, rc, msg)
    raise DmlaError(name, rc, msg)


def call(name: str, *args) -> None:
    check(name, getattr(lib(), name)(*args))
