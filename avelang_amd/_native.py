"""ctypes binding of ``libgdn.so`` (the gfx950 C ABI declared in include/gdn.h).

The library is built in-tree by ``avelang_amd.build``.  There is no
fallback: if the library is missing or fails to load, every operator
raises.  ``torch`` is imported first so that the library binds to the HIP
runtime torch already loaded (one runtime, one device context per process).
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (load torch's HIP runtime before libgdn.so)

LIB_PATH = Path(__file__).resolve().parent / "libgdn.so"

# Entry points declared in include/gdn.h; tests check every one is exported.
EXPORTS = (
    "gdn_chunk_fwd",
    "gdn_chunk_workspace_bytes",
    "gdn_chunk_fwd_save",
    "gdn_chunk_bwd",
    "gdn_chunk_bwd_workspace_bytes",
    "gdn_recurrent_fwd",
    "gdn_last_error",
    "gdn_abi_version",
    "gdn_cu_seqlens_check",
    "gdn_chunk_fwd_noalloc",
    "gdn_chunk_fwd_gating",
    "gdn_recurrent_fwd_gating",
    # include/gdn_layer.h
    "gdn_gating_fwd",
    "gdn_gating_bwd",
    "gdn_gating_bwd_workspace_bytes",
    "gdn_l2norm_fwd",
    "gdn_causal_conv1d_fwd",
    "gdn_causal_conv1d_update",
    "gdn_rmsnorm_gated_fwd",
    "gdn_recurrent_fwd_indexed",
    "gdn_recurrent_fwd_spec",
)

GDN_DTYPE_F32 = 0
GDN_DTYPE_BF16 = 1
GDN_DTYPE_F16 = 2

GDN_OK = 0
GDN_ERR_NULL = -1
GDN_ERR_SHAPE = -2
GDN_ERR_SEQLENS = -3
GDN_ERR_WORKSPACE = -4
GDN_ERR_ALIAS = -5

_lock = threading.Lock()
_lib = None

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t
_ll = ctypes.c_longlong


class NativeLibraryError(RuntimeError):
    """libgdn.so is missing or cannot be loaded."""


def lib():
    """Load (once) and return the ctypes handle of libgdn.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryError(
                f"{LIB_PATH} is not built; run `python -m avelang_amd.build` "
                "(there is no CPU fallback for the GDN operators)")
        try:
            h = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - environment specific
            raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        h.gdn_chunk_fwd.restype = _i
        h.gdn_chunk_fwd.argtypes = [
            _vp, _vp, _vp, _vp, _vp,          # q k v g beta
            _vp, _vp, _vp, _vp,               # h0 ht o cu_seqlens
            _i, _i, _i, _i, _i, _i, _i,       # B T Hqk Hv K V N
            _f, _i, _vp, _sz, _vp,            # scale l2norm ws ws_bytes stream
        ]
        h.gdn_chunk_workspace_bytes.restype = _sz
        h.gdn_chunk_workspace_bytes.argtypes = [_i] * 9
        h.gdn_chunk_fwd_save.restype = _i
        h.gdn_chunk_fwd_save.argtypes = h.gdn_chunk_fwd.argtypes
        h.gdn_chunk_bwd.restype = _i
        h.gdn_chunk_bwd.argtypes = [
            _vp, _vp, _vp, _vp, _vp, _vp,     # q k v g beta h0
            _vp, _vp,                         # dO dht
            _vp, _vp, _vp, _vp, _vp, _vp,     # dq dk dv dg dbeta dh0
            _vp,                              # cu_seqlens
            _i, _i, _i, _i, _i, _i, _i,       # B T Hqk Hv K V N
            _f, _i, _i, _vp, _sz, _vp,        # scale l2norm saved ws ws_bytes stream
        ]
        h.gdn_chunk_bwd_workspace_bytes.restype = _sz
        h.gdn_chunk_bwd_workspace_bytes.argtypes = [_i] * 9
        h.gdn_recurrent_fwd.restype = _i
        h.gdn_recurrent_fwd.argtypes = [
            _vp, _vp, _vp, _vp, _vp,
            _vp, _vp, _vp, _vp,
            _i, _i, _i, _i, _i, _i, _i,
            _f, _i, _vp,
        ]
        h.gdn_last_error.restype = ctypes.c_char_p
        h.gdn_last_error.argtypes = []
        h.gdn_abi_version.restype = _i
        h.gdn_abi_version.argtypes = []
        h.gdn_chunk_fwd_noalloc.restype = _i
        h.gdn_chunk_fwd_noalloc.argtypes = h.gdn_recurrent_fwd.argtypes
        _gate = [_vp, _vp, _vp, _vp, _i, _i, _i, _f, _f]   # A_log, a, b, dt_bias, dtypes, softplus
        h.gdn_chunk_fwd_gating.restype = _i
        h.gdn_chunk_fwd_gating.argtypes = ([_vp] * 3 + _gate + [_vp] * 4 + [_i] * 7
                                           + [_f, _i, _vp, _sz, _vp])
        h.gdn_recurrent_fwd_gating.restype = _i
        h.gdn_recurrent_fwd_gating.argtypes = ([_vp] * 3 + _gate + [_vp] * 5 + [_i] * 8
                                               + [_f, _i, _vp])
        h.gdn_cu_seqlens_check.restype = _i
        h.gdn_cu_seqlens_check.argtypes = [_vp, _i, _i]
        h.gdn_gating_fwd.restype = _i
        h.gdn_gating_fwd.argtypes = [
            _vp, _vp, _vp, _vp, _vp, _vp,     # A_log a b dt_bias g beta
            _ll, _i, _i, _i, _i,              # rows H a_dtype b_dtype p_dtype
            _f, _f, _vp,                      # softplus beta, threshold, stream
        ]
        h.gdn_gating_bwd_workspace_bytes.restype = _sz
        h.gdn_gating_bwd_workspace_bytes.argtypes = [_ll, _i]
        h.gdn_gating_bwd.restype = _i
        h.gdn_gating_bwd.argtypes = [
            _vp, _vp, _vp, _vp, _vp, _vp,     # A_log a b dt_bias dg dbeta
            _vp, _vp, _vp, _vp,               # dA_log da db ddt_bias
            _ll, _i, _i, _i, _i,              # rows H a_dtype b_dtype p_dtype
            _f, _f, _vp, _sz, _vp,            # softplus beta, threshold, ws, ws bytes, stream
        ]
        h.gdn_l2norm_fwd.restype = _i
        h.gdn_l2norm_fwd.argtypes = [_vp, _vp, _ll, _i, _f, _i, _vp]
        h.gdn_causal_conv1d_fwd.restype = _i
        h.gdn_causal_conv1d_fwd.argtypes = (
            [_vp] * 7                         # x weight bias seq_idx init final out
            + [_i] * 4                        # B D T W
            + [_ll] * 6                       # x strides, out strides
            + [_i, _i, _i, _vp])              # silu dtype w_dtype stream
        h.gdn_causal_conv1d_update.restype = _i
        h.gdn_causal_conv1d_update.argtypes = (
            [_vp] * 6                         # x conv_state weight bias indices out
            + [_i] * 6                        # B D L W S num_slots
            + [_ll] * 6
            + [_i, _i, _i, _vp])
        h.gdn_rmsnorm_gated_fwd.restype = _i
        h.gdn_rmsnorm_gated_fwd.argtypes = [_vp, _vp, _vp, _vp, _ll, _i, _f, _i, _i, _vp]
        h.gdn_recurrent_fwd_indexed.restype = _i
        h.gdn_recurrent_fwd_indexed.argtypes = (
            [_vp] * 10                        # q k v g beta h0 ht o cu_seqlens state_indices
            + [_i] * 8                        # B T Hqk Hv K V N num_slots
            + [_f, _i, _vp])
        h.gdn_recurrent_fwd_spec.restype = _i
        h.gdn_recurrent_fwd_spec.argtypes = (
            [_vp] * 9                         # q k v g beta pool o cu_seqlens state_indices
            + [_i, _vp]                       # index_stride num_accepted_tokens
            + [_i] * 8                        # B T Hqk Hv K V N num_slots
            + [_f, _i, _vp])
        _lib = h
        return _lib


def last_error() -> str:
    return lib().gdn_last_error().decode(errors="replace")


def check(rc: int, what: str) -> None:
    """Raise for a non-zero ABI return code (ValueError for argument errors)."""
    if rc == GDN_OK:
        return
    msg = last_error()
    if rc < 0:
        raise ValueError(f"{what}: {msg} (code {rc})")
    raise RuntimeError(f"{what}: {msg} (hipError {rc})")
