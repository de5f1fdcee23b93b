"""Instruction-level check of the built gfx950 code (CPU only).

A 128-bit buffer store reads its data VGPRs after it issues; a
v_accvgpr_read (emitted by inline asm, which the compiler's hazard check
does not pad) that overwrites one of them in the next cycle was measured to
replace that dword of the store in some lanes (the 8-wave epilogue wrote raw
fp32 accumulators into bf16 outputs).  Every such store is followed by an
s_nop 1 (store_b128 in include/hipgemm/detail/arch.hpp); this test
disassembles the built library and checks that no v_accvgpr_read writes a
data VGPR of a preceding >64-bit store with fewer than two wait states in
between, whatever the register allocation of the day.
"""
import os
import re
import shutil
import struct
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "hipgemm_amd", "libhipgemm.so")
OBJDUMP = "/opt/rocm/llvm/bin/llvm-objdump"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

STORE = re.compile(
    r"^\s*(buffer|global|flat)_store_(dwordx[34]|b96|b128)\s+v\[(\d+):(\d+)\]")
NEED = 2  # wait states required between the store and the writer


def code_objects(path):
    """The gfx950 code objects of every offload bundle in .hip_fatbin.

    Bundle layout (clang offload bundler, uncompressed): the magic string,
    u64 entry count, then per entry u64 offset, u64 size, u64 triple length
    and the triple; offsets are from the bundle's start.
    """
    tmp = path + ".fatbin.tmp"
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin",
                    path, tmp], check=True)
    try:
        data = open(tmp, "rb").read()
    finally:
        os.remove(tmp)
    out = []
    pos = data.find(MAGIC)
    while pos >= 0:
        n, = struct.unpack_from("<Q", data, pos + len(MAGIC))
        q = pos + len(MAGIC) + 8
        for _ in range(n):
            off, size, tlen = struct.unpack_from("<QQQ", data, q)
            triple = data[q + 24:q + 24 + tlen].decode()
            q += 24 + tlen
            if "gfx950" in triple and size:
                out.append(data[pos + off:pos + off + size])
        pos = data.find(MAGIC, pos + 1)
    return out


def hazards(asm_lines):
    hits = []
    for i, line in enumerate(asm_lines):
        m = STORE.match(line)
        if not m:
            continue
        data = set(range(int(m[3]), int(m[4]) + 1))
        ws = 0
        for nxt in asm_lines[i + 1:]:
            s = nxt.strip()
            if not s or s.startswith((";", "/", ".")) or s.endswith(">:"):
                continue
            op = s.split()[0]
            if op == "s_nop":
                ws += int(s.split()[1].split("/")[0], 0) + 1
            elif op.startswith("v_accvgpr_read"):
                dst = s.split()[1].rstrip(",")
                r = re.match(r"v(\d+)$", dst)
                if r and int(r[1]) in data:
                    hits.append(f"{line.strip()}  ->  {s}")
                    break
                ws += 1
            else:
                ws += 1
            if ws >= NEED:
                break
    return hits


@pytest.mark.skipif(not os.path.exists(LIB), reason="library not built")
@pytest.mark.skipif(not os.path.exists(OBJDUMP) or not shutil.which("objcopy"),
                    reason="llvm-objdump / objcopy not available")
def test_no_accvgpr_read_over_store_data(tmp_path):
    objs = code_objects(LIB)
    assert objs, "no gfx950 code objects found in the library"
    found, stores = [], 0
    for k, co in enumerate(objs):
        f = tmp_path / f"co{k}.o"
        f.write_bytes(co)
        asm = subprocess.run([OBJDUMP, "-d", "--no-show-raw-insn", str(f)],
                             check=True, capture_output=True, text=True).stdout
        lines = asm.splitlines()
        stores += sum(1 for l in lines if STORE.match(l))
        found += hazards(lines)
    assert stores > 0, "disassembly shows no 128-bit stores: scan is broken"
    assert not found, f"{len(found)} hazards, e.g.:\n" + "\n".join(found[:5])


def test_scanner_flags_the_measured_case():
    """The scanner itself, on the sequence that failed on the GPU."""
    bad = ["\tbuffer_store_dwordx4 v[18:21], v22, s[24:27], s28 offen nt",
           "\tv_accvgpr_read_b32 v18, a92"]
    ok1 = [bad[0], "\ts_nop 1", bad[1]]
    ok2 = [bad[0], "\ts_add_i32 s5, s5, 1", "\tv_add_u32_e32 v9, 1, v9", bad[1]]
    other = [bad[0], "\tv_accvgpr_read_b32 v22, a92"]
    assert len(hazards(bad)) == 1
    assert len(hazards([bad[0], "\ts_nop 0", bad[1]])) == 1
    assert hazards(ok1) == [] and hazards(ok2) == [] and hazards(other) == []
