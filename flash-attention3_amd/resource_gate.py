"""gfx950 resource gate for the built library (replaces the reference's
scripts/check_fused_bwd_kernel_gate.py:61-212, which checks its own custom-ISA
kernel for scratch use and spills).

Reads the AMDGPU code-object metadata of every gfx950 kernel in
lib/libshaobo_fa3_bwd.so -- the clang offload bundles in its .hip_fatbin
section, each holding one ELF code object, whose NT_AMDGPU_METADATA note
`llvm-readelf --notes` prints as YAML -- and checks, per kernel:

  * no private segment (scratch), no dynamic stack, no VGPR / SGPR spills;
  * LDS (group segment) within the 160 KiB of a gfx950 CU;
  * VGPRs (architectural + accumulation) within the budget that lets every
    wave of one full-size workgroup be resident: 512 registers per SIMD lane
    shared by ceil(workgroup waves / 4) waves.

Usage: python resource_gate.py [path/to/lib.so]   (exit status 1 on a violation)
"""
import math
import os
import struct
import subprocess
import sys
import tempfile

import yaml

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libshaobo_fa3_bwd.so")
READELF = "/opt/rocm/llvm/bin/llvm-readelf"
ARCH = "gfx950"
LDS_BYTES = 160 * 1024
VGPRS_PER_LANE = 512   # unified VGPR + AGPR file of one SIMD lane
SIMDS_PER_CU = 4
WAVE = 64
_MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(data, arch=ARCH):
    """The code objects for `arch` in every offload bundle inside `data`.

    Bundle layout: the magic, a little-endian uint64 entry count, then per
    entry uint64 offset (from the bundle start), uint64 size, uint64 triple
    length and the triple."""
    out = []
    i = data.find(_MAGIC)
    while i >= 0:
        (count,) = struct.unpack_from("<Q", data, i + len(_MAGIC))
        p = i + len(_MAGIC) + 8
        for _ in range(count):
            off, size, tlen = struct.unpack_from("<QQQ", data, p)
            p += 24
            triple = data[p:p + tlen].decode()
            p += tlen
            if triple.endswith("--" + arch) and size > 0:
                out.append(data[i + off:i + off + size])
        i = data.find(_MAGIC, i + 1)
    return out


def kernel_metadata(code_object, readelf=READELF):
    """amdhsa.kernels of one ELF code object, as a list of dicts."""
    with tempfile.NamedTemporaryFile(suffix=".elf") as f:
        f.write(code_object)
        f.flush()
        text = subprocess.run([readelf, "--notes", f.name], check=True, capture_output=True,
                              text=True).stdout
    start = text.index("---", text.index("AMDGPU Metadata:"))
    end = text.index("\n...", start)
    return yaml.safe_load(text[start:end])["amdhsa.kernels"]


def violations(kernel):
    """Gate failures of one kernel's metadata dict (empty list: it passes)."""
    name = kernel.get(".name", "?")
    bad = []
    if kernel.get(".private_segment_fixed_size", 0) != 0:
        bad.append(f"{name}: scratch {kernel['.private_segment_fixed_size']} B per lane")
    if kernel.get(".uses_dynamic_stack", False):
        bad.append(f"{name}: dynamic stack")
    for key in (".vgpr_spill_count", ".sgpr_spill_count"):
        if kernel.get(key, 0) != 0:
            bad.append(f"{name}: {key[1:]} = {kernel[key]}")
    lds = kernel.get(".group_segment_fixed_size", 0)
    if lds > LDS_BYTES:
        bad.append(f"{name}: LDS {lds} B > {LDS_BYTES} B")
    waves = math.ceil(kernel.get(".max_flat_workgroup_size", 256) / WAVE)
    per_simd = math.ceil(waves / SIMDS_PER_CU)
    budget = VGPRS_PER_LANE // per_simd
    # the accumulation registers start at a 4-register boundary after the
    # architectural ones
    regs = 4 * math.ceil(kernel.get(".vgpr_count", 0) / 4) + kernel.get(".agpr_count", 0)
    if regs > budget:
        bad.append(f"{name}: {regs} VGPRs > {budget} ({per_simd} waves per SIMD)")
    return bad


def check(path=LIB_PATH):
    """(kernels, violations) of the library at `path`."""
    with open(path, "rb") as f:
        data = f.read()
    kernels = [k for co in code_objects(data) for k in kernel_metadata(co)]
    return kernels, [v for k in kernels for v in violations(k)]


if __name__ == "__main__":
    kernels, bad = check(sys.argv[1] if len(sys.argv) > 1 else LIB_PATH)
    for k in kernels:
        print(f"{k['.name'][:90]:90s} vgpr {k.get('.vgpr_count')} agpr {k.get('.agpr_count')} "
              f"lds {k.get('.group_segment_fixed_size')} scratch "
              f"{k.get('.private_segment_fixed_size')}")
    for v in bad:
        print("VIOLATION", v)
    sys.exit(1 if bad or not kernels else 0)
