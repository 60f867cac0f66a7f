"""Instruction-order checks on this repository's own gfx950 build (CPU only).

The device code of libndattn.so is unbundled from its .hip_fatbin section and
disassembled with the ROCm llvm-objdump. Two rules the kernels' results depend
on are then checked over every kernel, one basic block at a time:

1. A VGPR written by a VALU instruction is not read by an MFMA (any operand)
   or by v_permlane*_swap fewer than two wait states later. The compiler
   inserts these waits for code it can see, never across an inline-asm
   instruction: an asm v_fma_mixhi_f16 one wait state ahead of the MFMA that
   read its result let the MFMA read the register's previous contents (a
   stale lo half of the softmax weights).
2. An MFMA accumulation chain keeps one opcode: no MFMA reads as its
   accumulator (srcC) the result of an earlier MFMA of another opcode. On
   gfx950 a 16x16x16 f16 MFMA issued straight after the 16x16x32 f16 MFMA
   whose result it accumulated onto gave wrong results (0.2-0.4 on unit-scale
   outputs), although the compiler's hazard model asks for no wait state
   there; the decode kernel now runs its 16-dim tail on the 16x16x32 opcode.

A planted mistake for each rule is checked first, on hand-written lines.
"""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "esp32-needle-3_amd", "libndattn.so")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"

INSN = re.compile(r"^\s+([a-z_0-9]+)\s*(.*?)\s*//\s*([0-9A-F]+):")
FUNC = re.compile(r"^([0-9a-f]+) <(\S+)>:")
TARGET_REF = re.compile(r"<(\S+)\+0x([0-9a-f]+)>")


def vregs(tok):
    tok = tok.strip()
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def operands(rest):
    return [o.strip() for o in rest.split(",")] if rest else []


def parse(lines):
    """Disassembly lines -> {kernel: [basic blocks of (opcode, operands)]}."""
    funcs, order = {}, []
    cur = None
    for ln in lines:
        m = FUNC.match(ln)
        if m:
            cur = m.group(2)
            funcs[cur] = (int(m.group(1), 16), [])
            order.append(cur)
            continue
        m = INSN.match(ln)
        if m and cur:
            funcs[cur][1].append((int(m.group(3), 16), m.group(1), m.group(2), ln))
    out = {}
    for name in order:
        base, insns = funcs[name]
        starts = set()
        for _, op, _, ln in insns:
            if op.startswith(("s_branch", "s_cbranch")):
                t = TARGET_REF.search(ln)
                if t and t.group(1) == name:
                    starts.add(base + int(t.group(2), 16))
        blocks, blk = [], []
        for addr, op, rest, _ in insns:
            if addr in starts and blk:
                blocks.append(blk)
                blk = []
            blk.append((op, operands(rest)))
            if op.startswith(("s_branch", "s_cbranch", "s_endpgm", "s_setpc")):
                blocks.append(blk)
                blk = []
        if blk:
            blocks.append(blk)
        out[name] = blocks
    return out


def is_valu(op):
    return op.startswith("v_") and not op.startswith(("v_mfma", "v_cmp", "v_readlane", "v_readfirstlane"))


def valu_to_mfma(blocks):
    """Rule 1 violations: (valu line, reader line, wait states)."""
    bad = []
    for blk in blocks:
        for i, (op, ops) in enumerate(blk):
            if not is_valu(op) or not ops:
                continue
            w = vregs(ops[0])
            if not w:
                continue
            ws = 0
            for op2, ops2 in blk[i + 1:]:
                if op2 == "s_nop":
                    ws += int(ops2[0], 0) + 1
                else:
                    if op2.startswith("v_mfma") or "permlane" in op2:
                        src = set()
                        for o in (ops2[1:] if op2.startswith("v_mfma") else ops2):
                            src |= vregs(o)
                        if w & src:
                            bad.append((op, op2, ws))
                    ws += 1
                if ws >= 2:
                    break
    return bad


def mixed_chains(blocks, window=64):
    """Rule 2 violations: MFMA pairs (writer, reader) of different opcodes
    where the reader's srcC overlaps the writer's result."""
    bad = []
    for blk in blocks:
        for i, (op, ops) in enumerate(blk):
            if not op.startswith("v_mfma"):
                continue
            dst = vregs(ops[0])
            for op2, ops2 in blk[i + 1:i + 1 + window]:
                if op2.startswith("v_mfma"):
                    if vregs(ops2[3]) & dst:
                        if op2 != op:
                            bad.append((op, op2))
                        break
                    if vregs(ops2[0]) & dst:
                        break
                elif ops2 and vregs(ops2[0]) & dst and not op2.startswith(("ds_write", "global_store", "buffer_store")):
                    break        # result overwritten before any MFMA reads it
    return bad


def test_planted_mistakes_are_caught():
    lines = [
        "0000000000000000 <k>:",
        "\tv_fma_mixhi_f16 v95, v87, -1.0, v97 op_sel:[1,0,0] op_sel_hi:[1,0,0] // 000000000000: 0",
        "\ts_nop 0                                                    // 000000000008: 0",
        "\tv_mfma_f32_16x16x32_f16 v[22:25], v[88:91], v[92:95], v[22:25] // 00000000000C: 0",
        "\tv_mfma_f32_16x16x16_f16 v[22:25], v[86:87], v[50:51], v[22:25] // 000000000014: 0",
        "\tv_max3_f32 v1, v2, v3, v4                                  // 00000000001C: 0",
        "\ts_nop 1                                                    // 000000000024: 0",
        "\tv_permlane32_swap_b32_e32 v1, v5                           // 000000000028: 0",
        "\ts_endpgm                                                   // 00000000002C: 0",
    ]
    blocks = parse(lines)["k"]
    assert valu_to_mfma(blocks) == [("v_fma_mixhi_f16", "v_mfma_f32_16x16x32_f16", 1)]
    assert mixed_chains(blocks) == [("v_mfma_f32_16x16x32_f16", "v_mfma_f32_16x16x16_f16")]


def _disassemble(tmp_path):
    if not os.path.exists(LIB):
        pytest.fail("libndattn.so is not built (run __graft_entry__.build())")
    for tool in ("llvm-objcopy", "clang-offload-bundler", "llvm-objdump"):
        if not os.path.exists(os.path.join(LLVM, tool)):
            pytest.skip("ROCm llvm tools absent")
    fat = tmp_path / "fat.bin"
    subprocess.run([os.path.join(LLVM, "llvm-objcopy"), "--dump-section", ".hip_fatbin=%s" % fat, LIB],
                   check=True)
    data = fat.read_bytes()
    offs = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert offs, "no offload bundle in libndattn.so"
    lines = []
    for n, (a, b) in enumerate(zip(offs, offs[1:] + [len(data)])):
        part = tmp_path / ("b%d.bin" % n)
        part.write_bytes(data[a:b])
        dev = tmp_path / ("b%d.o" % n)
        subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o",
                        "--input=%s" % part, "--targets=" + TARGET, "--output=%s" % dev], check=True)
        r = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", "--mcpu=gfx950", str(dev)],
                           check=True, capture_output=True, text=True)
        lines += r.stdout.splitlines()
    return parse(lines)


def test_built_kernels_keep_both_rules(tmp_path):
    kernels = _disassemble(tmp_path)
    names = list(kernels)
    assert any("decode_mfma_kernel" in k for k in names) and any("prefill_kernel" in k for k in names)
    n_mfma = sum(op.startswith("v_mfma") for blocks in kernels.values() for blk in blocks for op, _ in blk)
    assert n_mfma > 1000, n_mfma
    v1 = {k: valu_to_mfma(b) for k, b in kernels.items()}
    v2 = {k: mixed_chains(b) for k, b in kernels.items()}
    v1 = {k: v[:3] for k, v in v1.items() if v}
    v2 = {k: v[:3] for k, v in v2.items() if v}
    assert not v1, "VALU result read by an MFMA / permlane within 2 wait states: %s" % v1
    assert not v2, "MFMA chain mixes opcodes: %s" % v2
