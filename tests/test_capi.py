"""The C-ABI library loads and exports every symbol include/*.h declares.

CPU only: no compute calls (there is no HIP device here); only entry points
that do not touch the device (version, status strings, workspace sizing and
argument validation) are called.
"""
from __future__ import annotations

import ctypes
import glob
import os
import re

import pytest
import torch

from dcr_attention_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(dcr_\w+)\s*\(", text, flags=re.M):
            names.add(m.group(1))
    return names


def test_library_built_and_loads():
    assert os.path.exists(_lib.LIB_PATH), "run __graft_entry__.build() first"
    lib = _lib.load()
    assert lib.dcr_abi_version() == _lib.ABI_VERSION


def test_every_declared_symbol_is_exported_and_bound():
    declared = _declared_functions()
    assert len(declared) >= 15, declared
    lib = _lib.load()
    for name in sorted(declared):
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert declared == set(_lib.SIGNATURES), "ctypes signature table out of sync with header"


def test_status_strings():
    lib = _lib.load()
    assert lib.dcr_status_string(0) == b"ok"
    assert lib.dcr_status_string(-3) == b"workspace too small"


def test_workspace_sizes():
    lib = _lib.load()
    # C2: u 32 KiB + scores 8 MiB + 16 histogram slabs per row (1 MiB of 16-bit counts) + idx 2.5 MB + partials
    ws = lib.dcr_sparse_decode_workspace_bytes(4, 32, 8, 32768, 64, 4916, 1)
    assert 4 * 32 * 32768 * 2 + 128 * 16 * 256 * 2 + 128 * 4916 * 4 < ws < 64 << 20
    assert ws % 256 == 0
    sel = lib.dcr_qaxis_select_workspace_bytes(4, 32, 8, 32768, 64, 1)
    assert sel < ws and sel % 256 == 0
    assert lib.dcr_topk_select_workspace_bytes(128, 32768) == 128 * 8 * 256 * 2
    assert lib.dcr_sparse_decode_workspace_bytes(0, 32, 8, 32768, 64, 4916, 1) == 0
    assert lib.dcr_sparse_decode_workspace_bytes(4, 32, 8, 32768, 64, 4916, 9) == 0


def test_argument_validation_without_device():
    """Invalid arguments are rejected before any launch (safe with no GPU)."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x1000)
    buf = ctypes.create_string_buffer(1 << 16)
    ws = ctypes.c_void_p((ctypes.addressof(buf) + 255) & ~255)
    # k >= N
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 32, 8, 100, 100, 64, 100, 1e-12,
                               ws, 1 << 15, None)
    assert rc == -1 and b"k=100" in lib.dcr_last_error()
    # H not divisible by Hkv
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 30, 8, 100, 100, 64, 10, 1e-12,
                               ws, 1 << 15, None)
    assert rc == -1
    # unsupported head dim / group size
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 32, 8, 100, 100, 96, 10, 1e-12,
                               ws, 1 << 15, None)
    assert rc == -2
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 24, 8, 100, 100, 64, 10, 1e-12,
                               ws, 1 << 15, None)
    assert rc == -2
    # N beyond the top-k limit (2^24; rows over 131072 positions are supported)
    rc = lib.dcr_topk_select(fake, fake, 1, (1 << 24) + 1, 10, ws, 1 << 15, None)
    assert rc == -2
    # workspace too small / misaligned
    need = lib.dcr_sparse_decode_workspace_bytes(1, 32, 8, 4096, 64, 615, 1)
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 32, 8, 4096, 4096, 64, 615, 1e-12,
                               ws, need - 1, None)
    assert rc == -3
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 32, 8, 4096, 4096, 64, 615, 1e-12,
                               ctypes.c_void_p(ws.value + 4), need, None)
    assert rc == -3
    # null pointers and bad dtype
    rc = lib.dcr_gather_attn(None, fake, fake, 1, fake, fake, 1, 32, 8, 100, 100, 64, 10, ws, 1 << 15,
                             None)
    assert rc == -1 and b"null pointer" in lib.dcr_last_error()
    rc = lib.dcr_compute_uq(fake, 7, fake, 4, 64, 1e-12, None)
    assert rc == -1
    # KV head stride smaller than N
    rc = lib.dcr_sparse_decode(fake, fake, fake, 1, fake, None, 1, 32, 8, 4096, 4095, 64, 615,
                               1e-12, ws, need, None)
    assert rc == -1 and b"ldn=4095" in lib.dcr_last_error()
    # rank-local: window, head dim and grid limits; the gather form's head
    # mapping and cache row stride
    rc = lib.dcr_rank_local_fwd(fake, fake, fake, 1, fake, fake, fake, 4, 8, 100, 64, -1, 0.125, None)
    assert rc == -1 and b"k_window" in lib.dcr_last_error()
    rc = lib.dcr_rank_local_fwd(fake, fake, fake, 1, fake, fake, fake, 4, 8, 100, 96, 8, 0.125, None)
    assert rc == -2
    rc = lib.dcr_rank_local_fwd(fake, fake, fake, 1, fake, fake, fake, 70000, 8, 100, 64, 8, 0.125, None)
    assert rc == -2
    rc = lib.dcr_rank_local_fwd_gather(fake, fake, fake, 1, fake, fake, fake, fake, 1, 6, 4, 1, 100, 100,
                                       64, 8, 0.125, None)
    assert rc == -1 and b"multiple" in lib.dcr_last_error()
    rc = lib.dcr_rank_local_fwd_gather(fake, fake, fake, 1, fake, fake, fake, fake, 1, 8, 2, 1, 100, 99,
                                       64, 8, 0.125, None)
    assert rc == -1 and b"ldn=99" in lib.dcr_last_error()
    rc = lib.dcr_rank_local_fwd_gather(fake, fake, fake, 1, None, fake, fake, fake, 1, 8, 2, 1, 100, 100,
                                       64, 8, 0.125, None)
    assert rc == -1 and b"null pointer" in lib.dcr_last_error()


def test_kv_head_stride_layouts():
    """Accepted cache views: contiguous, a prefix of a preallocated cache, the
    un-repeat view K[:, ::n_rep] of a GQA-repeated tensor."""
    K = torch.zeros(2, 8, 100, 64)
    assert _lib.kv_head_stride(K) == 100
    big = torch.zeros(2, 8, 256, 64)
    assert _lib.kv_head_stride(big[:, :, :100]) == 256
    rep = torch.zeros(2, 32, 100, 64)
    assert _lib.kv_head_stride(rep[:, ::4]) == 400
    with pytest.raises(AssertionError):
        _lib.kv_head_stride(K.transpose(2, 3).contiguous().transpose(2, 3))
    with pytest.raises(AssertionError):
        _lib.kv_head_stride(big[:, :4, :100])   # batch stride != H_kv * head stride
    with pytest.raises(AssertionError):
        _lib.kv_head_stride(K, torch.zeros(2, 8, 100, 64)[:, :, :99])


def test_python_api_rejects_host_tensors():
    from dcr_attention_amd.kernel.hip import topk_qaxis_attention, topk_pass2_select
    Q = torch.zeros(1, 32, 64, dtype=torch.float16)
    K = torch.zeros(1, 8, 128, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="HIP device"):
        topk_qaxis_attention(Q, K, K, 10)
    with pytest.raises(RuntimeError, match="HIP device"):
        topk_pass2_select(torch.zeros(1, 4, 100, dtype=torch.bfloat16), 10)


def test_missing_library_raises(monkeypatch, tmp_path):
    """No CPU fallback: without the built library every entry point raises."""
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", str(tmp_path / "libdcr_sparse_decode.so"))
    with pytest.raises(RuntimeError, match="not built"):
        _lib.load()


def test_static_entry_point_rejects_oversize_before_any_device_call():
    """dcr_sparse_decode_static checks the shape against its static scratch
    (DCR_STATIC_SCRATCH_BYTES) before it touches a device."""
    lib = _lib.load()
    fake = ctypes.c_void_p(0x10000)
    rc = lib.dcr_sparse_decode_static(fake, fake, fake, 2, fake, None, 16, 32, 8, 65536, 65536, 128,
                                      6554, 1e-12, None)
    assert rc == -3 and b"static scratch" in lib.dcr_last_error()
    rc = lib.dcr_sparse_decode_static(fake, fake, fake, 1, fake, None, 1, 32, 8, 100, 100, 64, 100,
                                      1e-12, None)
    assert rc == -1 and b"k=100" in lib.dcr_last_error()


def test_sparse_path_switch_and_launch_count_without_device():
    """dcr_set_sparse_path returns the previous setting and rejects unknown
    values; dcr_sparse_decode_launches rejects what dcr_sparse_decode would and
    reports 3 launches under DCR_PATH_CLASSIC (no device needed for either)."""
    lib = _lib.load()
    prev = _lib.set_sparse_path(_lib.PATH_CLASSIC)
    try:
        assert _lib.set_sparse_path(_lib.PATH_CLASSIC) == _lib.PATH_CLASSIC
        assert lib.dcr_set_sparse_path(7) == -1 and b"unknown sparse path" in lib.dcr_last_error()
        assert lib.dcr_sparse_decode_launches(4, 32, 8, 32768, 64, 4916, 1) == 3
        assert lib.dcr_sparse_decode_launches(4, 30, 8, 32768, 64, 4916, 1) < 0     # H % Hkv
        assert lib.dcr_sparse_decode_launches(4, 32, 8, 100, 64, 100, 1) < 0        # k >= N
        assert lib.dcr_sparse_decode_launches(4, 32, 8, 100, 64, 10, 9) < 0         # dtype
    finally:
        _lib.set_sparse_path(prev)
