"""dcr_sparse_decode_static (the entry point that allocates nothing) against
dcr_sparse_decode on the same inputs, through the C ABI.

The two entry points run the same kernels in the same order on different
scratch memory (the library's static device array vs a caller workspace), so
indices and outputs must be bit-identical; the indices are also checked
against the CPU oracle.  Two calls in a row, the second on a smaller input
(the static array keeps the first call's contents), with free device memory
unchanged across them, then a third at the first shape; a shape that needs
more than the static maximum is rejected with DCR_ERR_WORKSPACE.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import cpu
from dcr_attention_amd import _lib
from dcr_attention_amd.synthetic import make_qkv

pytestmark = pytest.mark.gpu
DEV = "cuda"
DCR_ERR_WORKSPACE = -3
STATIC_MAX = 32 * 1024 * 1024  # DCR_STATIC_SCRATCH_BYTES


class _Case:
    """Device inputs and preallocated outputs of one shape."""

    def __init__(self, B, H, Hkv, N, D, k, dtype, seed):
        self.shape = (B, H, Hkv, N, D, k)
        self.dtype = dtype
        self.Q, self.K, self.V = make_qkv(B, H, Hkv, N, D, dtype, seed=seed, n_sinks=4, n_outlier=2)
        self.Qd, self.Kd, self.Vd = (t.to(DEV) for t in (self.Q, self.K, self.V))
        self.out_ws = torch.empty(B, H, D, dtype=dtype, device=DEV)
        self.out_st = torch.empty(B, H, D, dtype=dtype, device=DEV)
        self.idx_ws = torch.empty(B, H, k, dtype=torch.int32, device=DEV)
        self.idx_st = torch.empty(B, H, k, dtype=torch.int32, device=DEV)
        lib = _lib.load()
        self.ws_bytes = lib.dcr_sparse_decode_workspace_bytes(B, H, Hkv, N, D, k, _lib.DTYPE_CODE[dtype])
        assert 0 < self.ws_bytes <= STATIC_MAX
        self.ws = _lib.workspace(self.ws_bytes, torch.device(DEV))

    def run_workspace(self):
        B, H, Hkv, N, D, k = self.shape
        lib = _lib.load()
        rc = lib.dcr_sparse_decode(self.Qd.data_ptr(), self.Kd.data_ptr(), self.Vd.data_ptr(),
                                   _lib.DTYPE_CODE[self.dtype], self.out_ws.data_ptr(),
                                   self.idx_ws.data_ptr(), B, H, Hkv, N, N, D, k, 1e-12,
                                   self.ws.data_ptr(), self.ws_bytes, _lib.stream_of(self.Qd))
        _lib.check(rc, "dcr_sparse_decode")

    def run_static(self):
        B, H, Hkv, N, D, k = self.shape
        lib = _lib.load()
        rc = lib.dcr_sparse_decode_static(self.Qd.data_ptr(), self.Kd.data_ptr(), self.Vd.data_ptr(),
                                          _lib.DTYPE_CODE[self.dtype], self.out_st.data_ptr(),
                                          self.idx_st.data_ptr(), B, H, Hkv, N, N, D, k, 1e-12,
                                          _lib.stream_of(self.Qd))
        _lib.check(rc, "dcr_sparse_decode_static")

    def check(self):
        torch.cuda.synchronize()
        assert torch.equal(self.idx_st, self.idx_ws)
        assert torch.equal(self.out_st, self.out_ws)
        k = self.shape[-1]
        ref_idx = cpu.topk(cpu.scores(self.K, cpu.compute_uq(self.Q)), k)
        assert torch.equal(self.idx_st.cpu(), ref_idx)
        ref = cpu.attention_f64(self.Q, self.K, self.V, ref_idx)
        tol = torch.full_like(ref, 2e-3 if self.dtype == torch.float16 else 5e-3)
        if self.dtype == torch.bfloat16:  # the suite's bf16 bar: max(5e-3, one bf16 ulp)
            tol = torch.maximum(tol, torch.ldexp(torch.ones_like(ref), torch.frexp(ref)[1] - 8))
        assert ((self.out_st.double().cpu() - ref).abs() <= tol).all()


def test_static_matches_workspace_entry_point_twice_then_smaller():
    big = _Case(4, 32, 8, 32768, 64, 4916, torch.float16, seed=21)      # C2 (17 MB of scratch)
    small = _Case(1, 32, 8, 4096, 64, 615, torch.bfloat16, seed=22)     # C1 heads, bf16
    print(f"static scratch: C2 needs {big.ws_bytes} B, small case {small.ws_bytes} B", flush=True)

    big.run_workspace()
    small.run_workspace()
    big.run_static()            # first call on this device: looks up the array's address
    small.run_static()
    torch.cuda.synchronize()
    for c in (big, small):      # poison the outputs the measured calls write
        c.out_st.fill_(float("nan"))
        c.idx_st.fill_(-1)
    torch.cuda.synchronize()
    free0, _ = torch.cuda.mem_get_info()
    big.run_static()            # two calls in a row, nothing else between them
    small.run_static()          # the smaller input over the first call's leftovers
    torch.cuda.synchronize()
    free1, _ = torch.cuda.mem_get_info()
    assert free1 == free0, f"device memory changed across static calls: {free0} -> {free1}"
    big.check()
    small.check()
    big.out_st.fill_(float("nan"))
    big.run_static()            # back to the larger shape after the smaller one
    big.check()


def test_static_rejects_shapes_beyond_the_maximum():
    lib = _lib.load()
    B, H, Hkv, N, D, k = 16, 32, 8, 65536, 128, 6554                    # C5: ~126 MiB of scratch
    need = lib.dcr_sparse_decode_workspace_bytes(B, H, Hkv, N, D, k, 2)
    assert need > STATIC_MAX
    fake = ctypes.c_void_p(0x10000)
    rc = lib.dcr_sparse_decode_static(fake, fake, fake, 2, fake, None, B, H, Hkv, N, N, D, k, 1e-12,
                                      None)
    assert rc == DCR_ERR_WORKSPACE
    assert b"static" in lib.dcr_last_error()
