"""The built library's gfx950 code objects, read without a GPU: scratch use and register budgets of the bf16 kernels.

A kernel whose registers spill, or whose by-value argument block the compiler copies to per-lane scratch, still
rounds the same sums, so no parity test sees it; its launches then run several times slower. These checks read the
AMDGPU metadata note (a msgpack map) of every code object the host library carries in its .hip_fatbin section
(clang offload bundles, one per HIP source file).

Occupancy arithmetic on gfx950: a SIMD holds 512 VGPRs (architectural and accumulation registers together) per lane,
allocated in granules of 8, and a CU has 4 SIMDs. The bf16 engine's configurations (option 1 of psgdk_set_option)
map to template arguments <BM, BN, WGM, WGN, epilogue, load-only waves> as in _CFG below.
"""
import os
import re
import struct

import msgpack
import pytest

from psgd_pro_amd import _lib as L

_BUNDLE_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"
_TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
_NT_AMDGPU_METADATA = 32
_SHT_NOTE = 7

# (BM, BN, WGM, WGN, load-only waves) -> option 1 configuration
_CFG = {(256, 256, 2, 4, 0): 0, (128, 128, 2, 2, 0): 1, (256, 256, 2, 2, 0): 2, (256, 256, 2, 4, 4): 3,
        (128, 128, 2, 2, 4): 4}
# epilogues the size rule keeps off configurations 3 and 4 (factor update, Procrustes, r2 trace SYRK, Procrustes
# with bf16 (R Q)^T)
_HEAVY_EPI = {1, 2, 6, 7}


def _sections(b):
    """ELF64 section table: name -> (type, offset, size)."""
    shoff, = struct.unpack_from("<Q", b, 0x28)
    shentsize, shnum, shstrndx = struct.unpack_from("<HHH", b, 0x3A)
    hdr = [struct.unpack_from("<IIQQQQIIQQ", b, shoff + i * shentsize) for i in range(shnum)]
    stro = hdr[shstrndx][4]

    def name(o):
        return b[stro + o:b.index(b"\0", stro + o)].decode()

    return {name(h[0]): (h[1], h[4], h[5]) for h in hdr}


def _bundled_code_objects(fat):
    """The gfx950 entries of the concatenated offload bundles (magic, entry count, then offset, size, triple length
    and triple per entry; offsets from the bundle's start)."""
    out, p = [], fat.find(_BUNDLE_MAGIC)
    while p >= 0:
        n, = struct.unpack_from("<Q", fat, p + len(_BUNDLE_MAGIC))
        q, end = p + len(_BUNDLE_MAGIC) + 8, p
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", fat, q)
            triple = fat[q + 24:q + 24 + tlen].decode()
            q += 24 + tlen
            end = max(end, p + off + size)
            if triple == _TARGET:
                out.append(fat[p + off:p + off + size])
        p = fat.find(_BUNDLE_MAGIC, end)
    return out


def _metadata(co):
    for typ, off, size in _sections(co).values():
        if typ != _SHT_NOTE:
            continue
        q = off
        while q < off + size:
            namesz, descsz, ntype = struct.unpack_from("<III", co, q)
            name = co[q + 12:q + 12 + namesz].rstrip(b"\0")
            d0 = q + 12 + (namesz + 3) // 4 * 4
            if name == b"AMDGPU" and ntype == _NT_AMDGPU_METADATA:
                return msgpack.unpackb(co[d0:d0 + descsz], raw=False)
            q = d0 + (descsz + 3) // 4 * 4
    raise AssertionError("code object without an AMDGPU metadata note")


@pytest.fixture(scope="module")
def code_objects():
    if not os.path.exists(L.LIB_PATH):
        pytest.fail(f"{L.LIB_PATH} not built (python -m psgd_pro_amd.build)")
    so = open(L.LIB_PATH, "rb").read()
    secs = _sections(so)
    assert ".hip_fatbin" in secs, "the library carries no HIP fat binary"
    _, off, size = secs[".hip_fatbin"]
    fat = so[off:off + size]
    if not fat.startswith(_BUNDLE_MAGIC):
        pytest.skip("compressed offload bundle: the metadata checks read uncompressed bundles only")
    return [_metadata(co) for co in _bundled_code_objects(fat)]


@pytest.fixture(scope="module")
def kernels(code_objects):
    return {k[".name"]: k for md in code_objects for k in md["amdhsa.kernels"]}


def _bf16(kernels):
    """(cfg, epilogue) -> metadata of each gemm_bf16_kernel instantiation."""
    out = {}
    for name, k in kernels.items():
        m = re.search(r"16gemm_bf16_kernelI((?:Li\d+E)+)E", name)
        if m:
            bm, bn, wgm, wgn, epi, pw = map(int, re.findall(r"Li(\d+)E", m.group(1)))
            out[(_CFG[(bm, bn, wgm, wgn, pw)], epi)] = k
    return out


def test_every_code_object_is_gfx950(code_objects):
    assert code_objects
    for md in code_objects:
        assert md["amdhsa.target"] == "amdgcn-amd-amdhsa--gfx950"


def test_every_bf16_configuration_and_epilogue_is_built(kernels):
    got = _bf16(kernels)
    assert set(got) == {(c, e) for c in range(5) for e in range(8)}
    for (c, e), k in got.items():
        ws = 4 if c in (3, 4) else 0
        assert L.kernel_name(5000 + 10 * c + e).endswith(f", {e}{', 4' if ws else ''}>")
        waves = {0: 8, 1: 4, 2: 4, 3: 12, 4: 8}[c]
        assert k[".max_flat_workgroup_size"] == 64 * waves, (c, e)


def test_kernels_the_size_rule_launches_use_no_scratch(kernels):
    """Every kernel of the library runs without scratch memory, except bf16 instantiations that only a forced
    configuration reaches (configuration 2, and the heavy epilogues on configurations 3 and 4), whose spills stay a
    few hundred bytes: far below a copy of the by-value argument block (5 to 8 KB)."""
    forced_only = {id(k) for (c, e), k in _bf16(kernels).items() if c == 2 or (c in (3, 4) and e in _HEAVY_EPI)}
    for name, k in kernels.items():
        scratch, spills = k[".private_segment_fixed_size"], k[".vgpr_spill_count"]
        if id(k) in forced_only:
            assert scratch <= 512, (name, scratch)
        else:
            assert scratch == 0 and spills == 0, (name, scratch, spills)


def test_register_budgets_of_the_bf16_configurations(kernels):
    """Configuration 3 (12 waves per workgroup: 3 per SIMD) fits 168 registers; configuration 4 (8 waves per workgroup,
    two workgroups per CU: 4 per SIMD) fits 128; configuration 0 (8 waves: 2 per SIMD) fits 256. Checked for the
    epilogues the size rule gives each configuration."""
    budget = {0: 256, 3: 168, 4: 128}
    for (c, e), k in _bf16(kernels).items():
        if c in budget and not (c in (3, 4) and e in _HEAVY_EPI):
            assert k[".vgpr_count"] <= budget[c], (c, e, k[".vgpr_count"])
