"""The DPP source hazard of the indexer score's inline asm, checked on the
gfx950 code object this tree builds (CPU only; no GPU call).

k_iscore (deepseek-v4-in-c_amd/csrc/dsv4_mla.hip) fuses the q broadcast into
its fma as inline `v_fmac_f64_dpp ... row_newbcast`. The compiler does not
look inside inline asm for hazards, and the ISA requires two wait states
between a VALU write of a VGPR and a DPP read of it; chain_16 places an
`s_nop 1` for that. This test disassembles the built dsv4_mla.o and checks
every DPP instruction of the file (the compiler's own ones too): along every
path into it -- the fall-through and every branch that targets an
instruction in between -- no VALU instruction writes the DPP source within
the two wait states before it (an s_nop N counts N + 1).
"""
import os
import re
import shutil
import subprocess

import pytest

import common

LLVM = "/opt/rocm/llvm/bin"
OBJ = os.path.join(common.ROOT, "deepseek-v4-in-c_amd", "lib", "obj", "dsv4_mla.o")


def _disassemble(tmp):
    for tool in ("objcopy",):
        if not shutil.which(tool):
            pytest.skip("%s not available" % tool)
    for tool in ("clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, tool)):
            pytest.skip("%s not available" % tool)
    if not os.path.exists(OBJ):
        pytest.skip("the backend is not built (no %s)" % OBJ)
    fat, co = os.path.join(tmp, "mla.fat"), os.path.join(tmp, "mla.co")
    # objcopy rewrites its input when given no output file: it works on a
    # copy, so the build product keeps its bytes and its timestamp
    obj = os.path.join(tmp, "mla.o")
    shutil.copyfile(OBJ, obj)
    subprocess.run(["objcopy", "--dump-section", ".hip_fatbin=" + fat, obj, os.devnull],
                   check=True)
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                    "--input=" + fat, "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    "--output=" + co], check=True)
    out = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", co],
                         check=True, capture_output=True, text=True).stdout
    return out


_INS = re.compile(r"^\s+(\S+)\s*(.*?)\s*//\s*([0-9A-Fa-f]+):")


def _parse(listing):
    """[(addr, opcode, operand text)] in address order."""
    ins = []
    for line in listing.splitlines():
        m = _INS.match(line)
        if m:
            ins.append((int(m.group(3), 16), m.group(1), m.group(2)))
    return ins


def _vregs(op):
    op = op.strip()
    m = re.match(r"v\[(\d+):(\d+)\]", op)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)\b", op)
    return {int(m.group(1))} if m else set()


def _operands(text):
    return [o.strip() for o in text.split(",")] if text else []


def _branch_target(addr, opc, text):
    if not (opc.startswith("s_cbranch") or opc == "s_branch"):
        return None
    imm = int(text.split()[0])
    if imm >= 1 << 15:
        imm -= 1 << 16
    return addr + 4 + 4 * imm


def dpp_hazards(listing):
    """(DPP instructions checked, v_fmac_f64_dpp count, hazard descriptions)
    for an llvm-objdump listing."""
    ins = _parse(listing)
    at = {a: i for i, (a, _, _) in enumerate(ins)}
    preds = {i: [] for i in range(len(ins))}
    for i, (a, opc, text) in enumerate(ins):
        t = _branch_target(a, opc, text)
        if t is not None and t in at:
            preds[at[t]].append(i)
        if i + 1 < len(ins) and opc not in ("s_branch", "s_endpgm", "s_setpc_b64"):
            preds[i + 1].append(i)

    def waits(opc, text):
        return int(text.split()[0]) + 1 if opc == "s_nop" else 1

    def hazard(i, src, budget, seen):
        """A VALU write of src within `budget` wait states before i, along
        any path into i."""
        for p in preds[i]:
            if (p, budget) in seen:
                continue
            seen.add((p, budget))
            _, opc, text = ins[p]
            if opc.startswith("v_") and _vregs((_operands(text) or [""])[0]) & src:
                return ins[p]
            rest = budget - waits(opc, text)
            if rest > 0:
                r = hazard(p, src, rest, seen)
                if r:
                    return r
        return None

    checked, bad = 0, []
    for i, (a, opc, text) in enumerate(ins):
        if "_dpp" not in opc:
            continue
        ops = _operands(text)
        src = _vregs(ops[1].split()[0]) if len(ops) > 1 else set()
        if not src:
            continue
        checked += 1
        r = hazard(i, src, 2, set())
        if r:
            bad.append("%x %s %s <- %x %s %s" % (a, opc, text[:40], r[0], r[1], r[2][:40]))
    fused = sum(1 for _, opc, _ in ins if opc == "v_fmac_f64_dpp")
    return checked, fused, bad


def _listing(lines):
    """A synthetic objdump listing: (opcode operands) at 4-byte steps."""
    out = []
    for k, l in enumerate(lines):
        out.append("\t%s // %012X: 00000000" % (l, 0x1000 + 4 * k))
    return "\n".join(out)


DPP = "v_fmac_f64_dpp v[4:5], v[2:3], v[6:7] row_newbcast:0 row_mask:0xf bank_mask:0xf"


def test_checker_finds_planted_hazards():
    """The checker itself: a write of the DPP source right before it, or one
    wait state before it, or on a branch path into it, is a hazard; two wait
    states (s_nop 1, or two other instructions) are not."""
    cvt = "v_cvt_f64_f32 v[2:3], v1"
    assert len(dpp_hazards(_listing([cvt, DPP]))[2]) == 1
    assert len(dpp_hazards(_listing([cvt, "s_nop 0", DPP]))[2]) == 1
    assert len(dpp_hazards(_listing([cvt, "v_mov_b32 v9, v8", DPP]))[2]) == 1
    assert dpp_hazards(_listing([cvt, "s_nop 1", DPP]))[2] == []
    assert dpp_hazards(_listing([cvt, "v_mov_b32 v9, v8", "v_mov_b32 v10, v8", DPP]))[2] == []
    assert dpp_hazards(_listing(["v_cvt_f64_f32 v[8:9], v1", DPP]))[2] == []
    # a conditional branch from right after the write onto the DPP itself:
    # the fall-through path has its wait states, the taken path only the
    # branch's one (s_cbranch_scc1 2 at 0x1004 targets 0x1004 + 4 + 8)
    br = [cvt, "s_cbranch_scc1 2", "s_nop 1", "s_nop 1", DPP]
    assert len(dpp_hazards(_listing(br))[2]) == 1
    ok = [cvt, "s_nop 1", "s_cbranch_scc1 2", "s_nop 1", "s_nop 1", DPP]
    assert dpp_hazards(_listing(ok))[2] == []


def test_dpp_source_hazards_have_two_wait_states(tmp_path):
    checked, fused, bad = dpp_hazards(_disassemble(str(tmp_path)))
    print("dpp instructions checked: %d (v_fmac_f64_dpp: %d); hazards: %d"
          % (checked, fused, len(bad)))
    assert checked > 1000
    assert fused > 0                    # the score kernel's asm is in the object
    assert not bad, "\n".join(bad[:20])
