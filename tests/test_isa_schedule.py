"""Instruction-order checks of the built gfx950 code (CPU only).

1. No buffer instruction sits in a readfirstlane loop.  A buffer resource
   the compiler takes for divergent (for instance one built from a quotient
   that integer division left in a VGPR) gets every instruction that uses it
   wrapped in a loop over the distinct values in the wave: four
   v_readfirstlane, two compares, an exec save and a branch per store.  The
   resources here are wave-uniform by construction (make_rsrc in
   include/hipgemm/detail/arch.hpp reads them from lane 0).
2. The K loops of every 16x16x128 4-wave kernel issue their LDS reads
   and DMAs one per MFMA block: never two DMAs or two reads back to back;
   and the steady loop (whole steps of the tile) has no VALU besides the
   MFMA (a per-lane K-tail select on each DMA there cost 2-4 %).  Given only a sched_group_barrier pattern, the scheduler clustered
   them in some quarters, and an unrelated change elsewhere in the kernel
   moved the clustering into the default instantiation (3-7 % slower); the
   order is now written out (`quarter` in gemm_4wave.hpp), and this checks
   the result.
"""
import os
import re
import shutil
import subprocess

import pytest

from test_isa_hazards import LIB, OBJDUMP, code_objects

LINE = re.compile(r"^\s+([a-z_0-9]+)\b(.*?)\s*//\s*([0-9A-Fa-f]+):(.*)$")
FUNC = re.compile(r"^([0-9a-f]+) <(\S+)>:$")
TARGET = re.compile(r"<(\S+)\+0x([0-9a-f]+)>")


def functions(asm):
    """{name: [(addr, mnemonic, "operands // comment")]} of one
    disassembly (the comment holds a branch's target as <function+offset>)."""
    out, cur, base = {}, None, 0
    for line in asm.splitlines():
        m = FUNC.match(line)
        if m:
            base, cur = int(m[1], 16), m[2]
            out[cur] = []
            continue
        m = LINE.match(line)
        if m and cur is not None:
            out[cur].append((int(m[3], 16), m[1], m[2] + " //" + m[4]))
    return out


def loops(insns, func_addr_of):
    """(start, end) index ranges of backward branches' loops."""
    idx = {a: i for i, (a, _, _) in enumerate(insns)}
    res = []
    for i, (a, op, rest) in enumerate(insns):
        if not op.startswith("s_cbranch") and op != "s_branch":
            continue
        t = TARGET.search(rest)
        if not t:
            continue
        dest = func_addr_of(t[1]) + int(t[2], 16)
        if dest <= a and dest in idx:
            res.append((idx[dest], i))
    return res


def readfirstlane_loops(insns, func_addr_of):
    hits = []
    for s, e in loops(insns, func_addr_of):
        body = [op for _, op, _ in insns[s:e + 1]]
        if (insns[e][1] == "s_cbranch_execnz" and "v_readfirstlane_b32" in body
                and any(op.startswith("s_and_saveexec") for op in body)
                and any(op.startswith("buffer_") for op in body)):
            hits.append((insns[s][0], insns[e][0]))
    return hits


def k_loops(insns, func_addr_of):
    """The K loops: loops of one step pair, 64-256 MFMA (the tile loop that
    holds them has more).  Each as (M / R / D pattern, non-MFMA VALU count)."""
    out = []
    for s, e in loops(insns, func_addr_of):
        body = insns[s:e + 1]
        n = sum(op.startswith("v_mfma") for _, op, _ in body)
        if not 64 <= n <= 256:
            continue
        pat, valu = "", 0
        for _, op, rest in body:
            if op.startswith("v_mfma"):
                pat += "M"
            elif op.startswith("ds_read"):
                pat += "R"
            elif op.startswith("buffer_load") and rest.split("//")[0].rstrip().endswith("lds"):
                pat += "D"
            elif op.startswith("v_"):
                valu += 1
        out.append((pat, valu))
    return out


def disassemble(tmp_path):
    out = []
    for k, co in enumerate(code_objects(LIB)):
        f = tmp_path / f"co{k}.o"
        f.write_bytes(co)
        asm = subprocess.run([OBJDUMP, "-d", "--no-show-raw-insn", str(f)],
                             check=True, capture_output=True, text=True).stdout
        out.append(asm)
    return out


def addr_map(asm):
    addrs = {}
    for line in asm.splitlines():
        m = FUNC.match(line)
        if m:
            addrs[m[2]] = int(m[1], 16)
    return addrs.__getitem__


needs_lib = [
    pytest.mark.skipif(not os.path.exists(LIB), reason="library not built"),
    pytest.mark.skipif(not os.path.exists(OBJDUMP) or not shutil.which("objcopy"),
                       reason="llvm-objdump / objcopy not available"),
]


@needs_lib[0]
@needs_lib[1]
def test_no_readfirstlane_loops(tmp_path):
    found, nfunc, nloop = [], 0, 0
    for asm in disassemble(tmp_path):
        fa = addr_map(asm)
        for name, insns in functions(asm).items():
            nfunc += 1
            nloop += len(loops(insns, fa))
            for a, b in readfirstlane_loops(insns, fa):
                found.append(f"{name} {a:#x}..{b:#x}")
    assert nfunc > 50 and nloop > 100, "few functions or loops: the scan is broken"
    assert not found, f"{len(found)} readfirstlane loops, e.g.:\n" + "\n".join(found[:5])


@needs_lib[0]
@needs_lib[1]
def test_4wave_16x16x128_loops_interleave(tmp_path):
    """Every K loop interleaves; each kernel without MX scales has a steady
    loop (the pairs that fetch whole steps of the tile) with no VALU besides
    the MFMA."""
    checked, bad, valu = 0, [], []
    for asm in disassemble(tmp_path):
        fa = addr_map(asm)
        for name, insns in functions(asm).items():
            if "4wave" not in name or not any(
                    "16x16x128" in op for _, op, _ in insns):
                continue
            ks = k_loops(insns, fa)
            if not ks:
                continue
            checked += 1
            # steady and edge (an edge loop may show two back edges)
            assert len(ks) >= 2, (name, len(ks))
            for pat, _ in ks:
                assert pat.count("D") >= 16 and pat.count("R") >= 32, (name, pat)
                if "DD" in pat or "RR" in pat:
                    bad.append(f"{name}: {pat}")
            # MX kernels load their block scales with VALU address work
            if "_mx" not in name and min(v for _, v in ks) != 0:
                valu.append(f"{name}: {[v for _, v in ks]}")
    # plain, MX and extended-epilogue units, every format
    assert checked >= 100, f"only {checked} 16x16x128 4-wave kernels found"
    assert not bad, f"{len(bad)} clustered loops, e.g.:\n" + "\n".join(bad[:3])
    assert not valu, f"{len(valu)} kernels with VALU in the steady loop:\n" + "\n".join(valu[:3])


def test_pattern_scanner():
    """The scanners themselves on hand-made sequences."""
    f = "<k+0x%x>"
    ins = [(0x0, "s_mov_b32", " s0, 0"),
           (0x4, "v_readfirstlane_b32", " s20, v2"),
           (0x8, "s_and_saveexec_b64", " s[0:1], s[0:1]"),
           (0xc, "buffer_store_dwordx4", " v[0:3], v4, s[20:23], s2 offen"),
           (0x10, "s_xor_b64", " exec, exec, s[0:1]"),
           (0x14, "s_cbranch_execnz", " 65530 " + f % 0x4)]
    assert len(readfirstlane_loops(ins, lambda n: 0)) == 1
    assert readfirstlane_loops(ins[:5], lambda n: 0) == []
    body = [(4 * i, op, r) for i, (op, r) in enumerate(
        [("s_nop", " 0")] + [("v_mfma_f32_16x16x128_f8f6f4", ""),
                             ("ds_read_b128", " v[0:3], v1")] * 64 +
        [("v_mfma_f32_16x16x128_f8f6f4", ""),
         ("buffer_load_dwordx4", " v1, s[4:7], s8 offen lds")] * 32)]
    body.append((4 * len(body), "v_cndmask_b32_e32", " v1, v2, v3, vcc"))
    body.append((4 * len(body), "s_cbranch_scc0", " 1 " + f % 0))
    (pat, valu), = k_loops(body, lambda n: 0)
    assert pat == "MR" * 64 + "MD" * 32 and valu == 1
    assert "DD" not in pat and "RR" not in pat
