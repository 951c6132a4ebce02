"""The fused merge of attn_kernel, union_attn_kernel and dense_kernel (the last workgroup of
a GQA group merges the group's split-k partials) is ordered by the instructions the compiler emits,
not by C++ release/acquire fences, so this test pins that instruction order in
the gfx950 assembly of every fused instance built from csrc/attn.hip:

  1. every global store before the ticket is an agent-coherent store (sc1:
     the lowering of the agent-scope atomic partial stores);
  2. after the last of them, `s_waitcnt vmcnt(0)` (the wave's stores are
     complete), then `s_barrier` (every wave of the workgroup has passed its
     wait), then the ticket's `global_atomic_add`;
  3. every global load after the ticket is agent-coherent (sc1), so the merging
     workgroup reads the partials past its own L2.

A compiler change that reorders these fails here, on the host (hipcc emits the
device assembly without a GPU).
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "dcr-attention_v3_amd")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# The library's own flags (dcr-attention_v3_amd/Makefile), device code only.
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(PKG, "csrc"),
         "--cuda-device-only", "-S"]
KERNEL = re.compile(r"^(_Z\S*attn_kernelILi(\d)ELi(\d+)ELi(\d)ELb(\d)ELb(\d)ELi(\d)E\S*):")


@pytest.fixture(scope="module")
def attn_asm(tmp_path_factory):
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("isa") / "attn.s"
    subprocess.run([HIPCC, *FLAGS, os.path.join(PKG, "csrc", "attn.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    return out.read_text().splitlines()


def _fused_bodies(lines):
    """{mangled name: body lines} of the attn_kernel instances with FUSE = true."""
    bodies, cur, name = {}, None, None
    for ln in lines:
        m = KERNEL.match(ln)
        if m:
            name = m.group(1)
            cur = [] if m.group(5) == "1" else None
            continue
        if cur is not None:
            if ln.startswith(".Lfunc_end"):
                bodies[name] = cur
                cur = None
            else:
                cur.append(ln.strip())
    return bodies


UNION = re.compile(r"^(_Z\S*union_attn_kernelILi(\d)ELi(\d+)ELi(\d)ELi(\d)E\S*):")


def _union_bodies(lines):
    """{mangled name: body lines} of the union_attn_kernel instances (all merge)."""
    bodies, cur, name = {}, None, None
    for ln in lines:
        m = UNION.match(ln)
        if m:
            name, cur = m.group(1), []
            continue
        if cur is not None:
            if ln.startswith(".Lfunc_end"):
                bodies[name] = cur
                cur = None
            else:
                cur.append(ln.strip())
    return bodies


def _check_order(name, body):
    atomics = [i for i, s in enumerate(body) if s.startswith("global_atomic_add")]
    assert len(atomics) == 1, f"{name}: {len(atomics)} ticket atomics"
    a = atomics[0]
    stores = [i for i, s in enumerate(body[:a]) if s.startswith("global_store")]
    assert stores, f"{name}: no partial stores before the ticket"
    for i in stores:
        assert re.search(r"\bsc1\b", body[i]), f"{name}: non-coherent store before the ticket: {body[i]}"
    last = stores[-1]
    waits = [i for i in range(last + 1, a) if re.match(r"s_waitcnt\b.*\bvmcnt\(0\)", body[i])]
    assert waits, f"{name}: no s_waitcnt vmcnt(0) between the partial stores and the ticket"
    bars = [i for i in range(waits[0] + 1, a) if body[i] == "s_barrier"]
    assert bars, f"{name}: no s_barrier between the wait and the ticket"
    loads_after = [s for s in body[a + 1:] if s.startswith("global_load")]
    assert loads_after, f"{name}: the merge loads no partials"
    for s in loads_after:
        assert re.search(r"\bsc1\b", s), f"{name}: non-coherent load after the ticket: {s}"


def test_fused_merge_instruction_order(attn_asm):
    bodies = _fused_bodies(attn_asm)
    # fp32/fp16/bf16 x D 64/128 x n_rep 1/2/4/8, scored (fp16/bf16) and K-gathering forms
    assert len(bodies) >= 40, len(bodies)
    for name, body in bodies.items():
        _check_order(name, body)


def test_union_merge_instruction_order(attn_asm):
    """union_attn_kernel merges the same way (its partial stores, the wait,
    the barrier, the ticket, the coherent loads of combine_head)."""
    bodies = _union_bodies(attn_asm)
    # fp16/bf16 x D 64/128 x n_rep 1/2/4/8 x 4 or 8 positions per thread
    assert len(bodies) == 32, len(bodies)
    for name, body in bodies.items():
        _check_order(name, body)


DENSE = re.compile(r"^(_Z\S*dense_kernelILi(\d)ELi(\d+)ELi(\d)E\S*):")


def _dense_bodies(lines):
    """{mangled name: body lines} of the dense_kernel instances (all merge)."""
    bodies, cur, name = {}, None, None
    for ln in lines:
        m = DENSE.match(ln)
        if m:
            name, cur = m.group(1), []
            continue
        if cur is not None:
            if ln.startswith(".Lfunc_end"):
                bodies[name] = cur
                cur = None
            else:
                cur.append(ln.strip())
    return bodies


def test_dense_merge_instruction_order(attn_asm):
    """dense_kernel merges in the same order through its 64-bit self-resetting
    ticket: the first `global_atomic_add_x2` is the ticket (the others re-take
    it after a stale word); coherent partial stores, the wait and the barrier
    precede it, and the merge's loads after it are coherent."""
    bodies = _dense_bodies(attn_asm)
    # fp32/fp16/bf16 x D 64/128 x n_rep 1/2/4/8
    assert len(bodies) == 24, len(bodies)
    for name, body in bodies.items():
        first = next(i for i, ln in enumerate(body) if ln.startswith("global_atomic_add_x2"))
        # _check_order's view: the first add is the ticket; the re-takes after it are dropped
        view = [ln for i, ln in enumerate(body) if i <= first or not ln.startswith("global_atomic_add")]
        _check_order(name, view)


_GOOD = ["global_store_dword v[6:7], v3, off sc1", "global_store_dword v[6:7], v4, off offset:4 sc1",
         "s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier", "global_atomic_add v6, v6, v7, s[10:11] sc0",
         "s_waitcnt vmcnt(0)", "global_load_dword v22, v[8:9], off sc1", "s_endpgm"]


@pytest.mark.parametrize("mutate", [
    lambda b: [s for s in b if s != "s_barrier"],                                  # no barrier
    lambda b: [s for s in b if not s.startswith("s_waitcnt vmcnt(0) lgkmcnt")],    # no wait
    lambda b: [b[0], b[2], b[3], b[1], *b[4:]],                                    # store after the wait
    lambda b: [s.replace(" sc1", "") if s.startswith("global_store") else s for s in b],
    lambda b: [s.replace(" sc1", "") if s.startswith("global_load") else s for s in b],
    lambda b: [*b[:3], b[4], b[3], *b[5:]],                                        # ticket before the barrier
])
def test_checker_rejects_a_misordered_sequence(mutate):
    _check_order("good", _GOOD)
    with pytest.raises(AssertionError):
        _check_order("planted", mutate(list(_GOOD)))
