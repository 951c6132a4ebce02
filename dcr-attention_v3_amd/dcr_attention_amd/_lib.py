"""ctypes binding of ``libdcr_sparse_decode.so`` (the C ABI in
``include/dcr_sparse_decode.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already loaded (both carry the soname ``libamdhip64.so.7``); kernels are
enqueued on torch's current stream.  There is no fallback: if the library is
missing every entry point raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_native", "libdcr_sparse_decode.so")
ABI_VERSION = 6

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

STATUS = {0: "ok", -1: "invalid argument", -2: "unsupported shape", -3: "workspace too small",
          -4: "HIP error"}

# name -> (restype, argtypes); mirrors include/dcr_sparse_decode.h
_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
SIGNATURES = {
    "dcr_abi_version": (_i, []),
    "dcr_status_string": (ctypes.c_char_p, [_i]),
    "dcr_last_error": (ctypes.c_char_p, []),
    "dcr_compute_uq": (_i, [_vp, _i, _vp, _i, _i, _f, _vp]),
    "dcr_score_pass": (_i, [_vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "dcr_topk_select_workspace_bytes": (_sz, [_i, _i]),
    "dcr_topk_select": (_i, [_vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "dcr_gather_attn_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "dcr_gather_attn": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _sz,
                             _vp]),
    "dcr_qaxis_select_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "dcr_qaxis_select": (_i, [_vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _vp, _sz, _vp]),
    "dcr_sparse_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "dcr_sparse_decode": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _vp,
                              _sz, _vp]),
    "dcr_sparse_decode_static": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f,
                                     _vp]),
    "dcr_set_sparse_path": (_i, [_i]),
    "dcr_set_score_form": (_i, [_i]),
    "dcr_sparse_decode_launches": (_i, [_i] * 7),
    "dcr_fused_errors": (_i, [_i, ctypes.POINTER(ctypes.c_uint)]),
    "dcr_dense_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "dcr_dense_decode": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "dcr_rank_local_fwd": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _vp]),
    "dcr_rank_local_fwd_gather": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp] + [_i] * 8 + [_f, _vp]),
    "dcr_profile_begin": (_i, []),
    "dcr_profile_end": (_i, [ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_double),
                             ctypes.POINTER(ctypes.c_int), _i]),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise RuntimeError if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"HIP library not built: {LIB_PATH} is missing "
                    "(run `make -C dcr-attention_v3_amd` or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.dcr_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH}: ABI {lib.dcr_abi_version()} != {ABI_VERSION}")
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    """Map a dcr_status to a Python exception (RuntimeError, like a failed launch)."""
    if rc != 0:
        msg = load().dcr_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {STATUS.get(rc, rc)}: {msg}")


class KernelTimer:
    """Per-kernel HIP-event timing of every launch the library makes while
    active (dcr_profile_begin / dcr_profile_end).  ``result`` maps kernel
    name -> (total_us, launches) after the block exits."""

    def __init__(self):
        self.result = {}

    def __enter__(self):
        check(load().dcr_profile_begin(), "dcr_profile_begin")
        return self

    def __exit__(self, *exc):
        n_max = 32
        names = (ctypes.c_char_p * n_max)()
        tot = (ctypes.c_double * n_max)()
        cnt = (ctypes.c_int * n_max)()
        n = load().dcr_profile_end(names, tot, cnt, n_max)
        if n < 0:
            check(n, "dcr_profile_end")
        self.result = {names[i].decode(): (tot[i], cnt[i]) for i in range(n)}
        return False


PATH_AUTO, PATH_CLASSIC, PATH_FUSED, PATH_UNION = 0, 1, 2, 3


def set_sparse_path(path: int) -> int:
    """Select the sparse decode launch sequence (PATH_AUTO: the library's
    choice, currently PATH_CLASSIC; PATH_CLASSIC: score, select, index-list
    attention; PATH_FUSED: one launch where the shape allows it; PATH_UNION:
    union-gather attention for fp16/bf16); returns the previous setting."""
    rc = load().dcr_set_sparse_path(int(path))
    if rc < 0:
        check(rc, "dcr_set_sparse_path")
    return rc


SCORE_AUTO, SCORE_VALU = 0, 1


def set_score_form(form: int) -> int:
    """Select the score pass's form (SCORE_AUTO: MFMA where it fits;
    SCORE_VALU: always VALU); returns the previous setting."""
    rc = load().dcr_set_score_form(int(form))
    if rc < 0:
        check(rc, "dcr_set_score_form")
    return rc


def fused_errors(clear: bool = False) -> int:
    """The one-launch path's sticky error word on the current device (0 = no
    barrier ever gave up)."""
    v = ctypes.c_uint(0)
    check(load().dcr_fused_errors(1 if clear else 0, ctypes.byref(v)), "dcr_fused_errors")
    return v.value


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    """Scratch from torch's caching allocator (512-byte aligned)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def require_device(*tensors: torch.Tensor, what: str) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(f"{what} requires HIP device tensors (got device {t.device}).")


def kv_head_stride(K: torch.Tensor, V: torch.Tensor = None, name: str = "K_cache") -> int:
    """Rows between consecutive KV heads (``ldn``) of a [B, H_kv, N, D] cache view.

    Accepted layouts: contiguous (ldn = N); the first N rows of a preallocated
    [B, H_kv, N_max, D] cache (ldn = N_max); every n_rep-th head of a
    GQA-repeated [B, H, N, D] tensor, ``K[:, ::n_rep]`` (ldn = n_rep * N).
    Rows must be contiguous and the batch stride H_kv * ldn rows.  V, when
    given, must have the same strides.  Raises AssertionError otherwise (the
    reference asserts contiguity, topk_axis_pass1.py:125-126)."""
    B, H_kv, N, D = K.shape
    st = K.stride()
    assert st[3] == 1 and (N == 1 or st[2] == D), f"{name} rows must be contiguous"
    assert st[1] % D == 0 and st[1] // D >= N, f"{name} head stride {st[1]} is not a row multiple >= N*D"
    ldn = st[1] // D
    assert B == 1 or st[0] == H_kv * st[1], f"{name} batch stride {st[0]} != H_kv * head stride"
    if V is not None:
        assert V.shape == K.shape, "V_cache shape must equal K_cache shape"
        assert V.stride() == K.stride() or (B == 1 and V.stride()[1:] == K.stride()[1:]), \
            "V_cache must have the same layout as K_cache"
    assert ldn < 2 ** 31, f"{name} head stride too large"
    return ldn
