"""The built gfx950 code objects: kernels whose waits are hand-counted use no
scratch and spill nothing.

The forward chain (chunk_chain_sw_kernel) and the reverse chain
(chunk_rev_sw_kernel) wait for their own loads with exact vector-memory
counts (s_waitcnt vmcnt(n), avelang_amd/csrc/gdn_chunk_chain.hip and
gdn_chunk_rev.hip): a scratch spill or reload is one more vector-memory
operation in that in-order counter, which would let a wait pass before the
operand it guards has landed (a stale LDS read, not a fault).  The gradient
kernel (chunk_grad_kernel) reloads spilled values behind every outstanding
store, the cost its design avoids.  This test reads the AMDGPU metadata of
every kernel in avelang_amd/libgdn.so (the clang offload bundles of the
.hip_fatbin section, split here; the notes read with llvm-readelf) and
fails if any of these kernels has a private (scratch) segment or spills
VGPRs.  SGPR spills are allowed: with no private segment they go to VGPR
lanes (v_writelane / v_readlane), which are not memory operations.  Runs on
the CPU (no GPU needed).
"""
import os
import re
import struct
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "avelang_amd", "libgdn.so")
READELF = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "llvm-readelf")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
GUARDED = ("chunk_chain_sw_kernel", "chunk_rev_sw_kernel", "chunk_grad_kernel")


def _code_objects(blob):
    """gfx950 code objects of every offload bundle in a binary (clang offload
    bundle layout: magic, entry count, then per entry offset, size, triple
    length and triple; offsets relative to the bundle start)."""
    out = []
    at = blob.find(MAGIC)
    while at >= 0:
        p = at + len(MAGIC)
        (n,) = struct.unpack_from("<Q", blob, p)
        p += 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", blob, p)
            p += 24
            triple = blob[p:p + tlen].decode()
            p += tlen
            if "gfx950" in triple and size:
                out.append(blob[at + off:at + off + size])
        at = blob.find(MAGIC, at + 1)
    return out


def _kernel_metadata(co):
    with tempfile.NamedTemporaryFile(suffix=".co") as f:
        f.write(co)
        f.flush()
        notes = subprocess.run([READELF, "--notes", f.name], capture_output=True, text=True,
                               check=True).stdout
    kernels, cur = {}, None
    for line in notes.splitlines():
        m = re.match(r"\s+\.(name|private_segment_fixed_size|vgpr_spill_count|sgpr_spill_count):"
                     r"\s+(\S+)", line)
        if not m:
            continue
        key, val = m.groups()
        if key == "name":
            cur = kernels.setdefault(val, {})
        elif cur is not None:
            cur[key] = int(val)
    return kernels


@pytest.fixture(scope="module")
def kernels():
    if not os.path.exists(LIB):
        pytest.fail("avelang_amd/libgdn.so is not built (run __graft_entry__.build())")
    if not os.path.exists(READELF):
        pytest.skip("llvm-readelf not found")
    blob = open(LIB, "rb").read()
    cos = _code_objects(blob)
    assert cos, "no gfx950 code object found in libgdn.so"
    out = {}
    for co in cos:
        out.update(_kernel_metadata(co))
    return out


def test_guarded_kernels_are_present(kernels):
    for g in GUARDED:
        assert any(g in name for name in kernels), g


def _violations(kernels):
    bad = []
    for name, md in kernels.items():
        if any(g in name for g in GUARDED):
            for key in ("private_segment_fixed_size", "vgpr_spill_count"):
                if md.get(key, 0) != 0:
                    bad.append(f"{name}: {key} = {md[key]}")
    return bad


def test_guarded_kernels_use_no_scratch_and_spill_nothing(kernels):
    bad = _violations(kernels)
    assert not bad, "\n".join(bad)


def test_the_check_catches_scratch_and_spills():
    """Planted metadata: a guarded kernel with scratch or VGPR spills is flagged, an
    unguarded one or SGPR-only spills are not."""
    ok = {"private_segment_fixed_size": 0, "vgpr_spill_count": 0, "sgpr_spill_count": 9}
    assert _violations({"_ZN3gdn21chunk_chain_sw_kernelI": ok}) == []
    assert _violations({"_ZN3gdn16recurrent_kernelI": dict(ok, vgpr_spill_count=4)}) == []
    assert len(_violations({"_ZN3gdn19chunk_rev_sw_kernelI": dict(ok, private_segment_fixed_size=16)})) == 1
    assert len(_violations({"_ZN3gdn17chunk_grad_kernelI": dict(ok, vgpr_spill_count=2)})) == 1
