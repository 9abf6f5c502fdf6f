"""Register budgets and hazards of the kernels, read from the compiler's resource remarks (hipcc -Rpass-analysis=
kernel-resource-usage on the library's own sources, gfx950; no GPU needed) and from the gfx950 assembly of the
same compile.

The streaming attention kernels wait for their HBM -> LDS copies with hand-counted `s_waitcnt vmcnt(N)`, so any
compiler-made vector memory access in them (a register spill to scratch) would make a wait return early and the
kernel read LDS before its data arrived: they must use no scratch, and between the 4/4 kernels' waits the
stream's own LDS DMAs must be the only vector memory instructions. The seal must not spill either (a spill there
once cost 30 MB of scratch traffic per commit). An MFMA must not read a register that an inline-asm VALU
instruction wrote less than two wait states before, nor an inline-asm VALU instruction read an MFMA result or
overwrite an MFMA accumulator too soon after the MFMA: the compiler inserts those wait states around its own
instructions but not around inline asm, and the 4/4 kernel feeds its asm-built fp16 operand pairs straight into
MFMAs. A compiler or source change that breaks this fails here, before anything runs on a GPU."""
import functools
import os
import re
import shutil
import subprocess
import tempfile

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "sj-kvarn-codec_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["-std=c++17", "-O3", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-x", "hip", "-S",
         "-Rpass-analysis=kernel-resource-usage", "--cuda-device-only"]


@functools.lru_cache(maxsize=None)
def compile_device(src):
    """(resource remarks, gfx950 assembly) of one source file"""
    with tempfile.TemporaryDirectory() as d:
        asm = os.path.join(d, "k.s")
        out = subprocess.run([HIPCC] + FLAGS + ["-o", asm, os.path.join(CSRC, src)], capture_output=True, text=True,
                             timeout=600)
        assert out.returncode == 0, out.stderr[-2000:]
        with open(asm) as f:
            return out.stderr, f.read()


def kernel_bodies(asm):
    """{symbol: lines} of the functions in an assembly listing"""
    bodies = {}
    for m in re.finditer(r"^(_Z\S+):\s*;", asm, re.M):
        bodies[m.group(1)] = asm[m.end():asm.find(".Lfunc_end", m.end())].split("\n")
    return bodies


def vgprs(text):
    """VGPR numbers named in an operand list (v7, v[4:7])"""
    regs = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]", text):
        regs.update(range(int(m.group(1)), int(m.group(2)) + 1))
    for m in re.finditer(r"\bv(\d+)\b", text):
        regs.add(int(m.group(1)))
    return regs


def parse_asm(lines):
    """(mnemonic, text, inside inline asm) per instruction; block labels as ("label", "", _)"""
    ins, in_asm = [], False
    for line in lines:
        t = line.strip()
        if "ASMSTART" in t or "ASMEND" in t:
            in_asm = "ASMSTART" in t
            continue
        if t.startswith(".LBB") or t.startswith("; %bb"):
            ins.append(("label", "", in_asm))
        elif t and not t.startswith(";") and not t.startswith("."):
            ins.append((t.split()[0], t, in_asm))
    return ins


def operands(text):
    parts = text.split(None, 1)
    return [p.strip() for p in parts[1].split(",")] if len(parts) > 1 else []


def written(op, text):
    """VGPRs an instruction writes (VALU and MFMA destinations, LDS and memory loads into registers)"""
    o = operands(text)
    if not o:
        return set()
    if op.startswith("v_") or (op.startswith("ds_") and not op.startswith("ds_write")) or \
            (op.startswith(("global_load", "buffer_load")) and "lds" not in op):
        return vgprs(o[0])
    return set()


TRANS = ("v_exp_", "v_log_", "v_rcp_", "v_rsq_", "v_sqrt_", "v_sin_", "v_cos_")


def asm_mfma_hazards(lines, valu_to_mfma=2, mfma_to_valu=11):
    """Inline-asm VALU instructions next to MFMAs without the wait states between them that the compiler inserts
    only around its own instructions (every instruction is one wait state, s_nop N is N + 1; the scan stops at a
    block label): an MFMA reading a VGPR whose last write was an asm VALU instruction fewer than valu_to_mfma wait
    states before; an asm VALU instruction reading an MFMA result, or writing a register an MFMA reads as its
    accumulator, fewer than mfma_to_valu wait states after the MFMA (the eight-pass MFMAs of these kernels); an asm
    VALU instruction reading a transcendental result with no wait state between."""
    ins = parse_asm(lines)
    bad = []
    for k, (op, text, asm) in enumerate(ins):
        if asm and op.startswith("v_") and k > 0:
            # a transcendental result needs one wait state before another VALU instruction reads it
            op2, text2, _ = ins[k - 1]
            if op2.startswith(TRANS) and written(op2, text2) & vgprs(",".join(operands(text)[1:])):
                bad.append(("transcendental write -> asm read", text2, text, 0))
        if op.startswith("v_mfma"):
            live, waits = vgprs(",".join(operands(text)[1:])), 0
            for j in range(k - 1, -1, -1):
                op2, text2, asm2 = ins[j]
                if op2 == "label" or waits >= valu_to_mfma or not live:
                    break
                w = written(op2, text2) & live
                if w and asm2 and op2.startswith("v_"):
                    bad.append(("asm write -> MFMA read", text2, text, waits))
                    break
                live -= w
                waits += int(text2.split()[1]) + 1 if op2 == "s_nop" else 1
        elif asm and op.startswith("v_"):
            o = operands(text)
            dst, live, waits = vgprs(o[0]) if o else set(), vgprs(",".join(o[1:])), 0
            for j in range(k - 1, -1, -1):
                op2, text2, _ = ins[j]
                if op2 == "label" or waits >= mfma_to_valu:
                    break
                w = written(op2, text2)
                if op2.startswith("v_mfma"):
                    o2 = operands(text2)
                    if w & live:
                        bad.append(("MFMA write -> asm read", text2, text, waits))
                    if len(o2) > 3 and vgprs(o2[3]) & dst:
                        bad.append(("MFMA accumulator read -> asm write", text2, text, waits))
                live -= w
                dst -= w
                waits += int(text2.split()[1]) + 1 if op2 == "s_nop" else 1
    return bad


def resources(src):
    stderr, _ = compile_device(src)
    res, name = {}, None
    for line in stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            res[name] = {}
            continue
        m = re.search(r"remark:\s+([A-Za-z /\[\]]+?):\s+(\d+)", line)
        if m and name:
            res[name][m.group(1).strip()] = int(m.group(2))
    return res


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_attention_kernels_use_no_scratch():
    res = resources("sjk_attend3.hip")
    kernels = [k for k in res if "attend4_kernel" in k or "attend3_kernel" in k or "attendsc_kernel" in k]
    assert len(kernels) >= 14, sorted(res)         # 4/4 and the other scalar bodies at D = 128 and 256, three
                                                   # trellis bodies, and their _dyn twins
    for k in kernels:
        assert res[k].get("ScratchSize [bytes/lane]", -1) == 0, (k, res[k])
        assert res[k].get("VGPRs Spill", -1) == 0, (k, res[k])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_inline_asm_keeps_its_wait_states():
    for src in ("sjk_attend3.hip", "sjk_seal.hip", "sjk_rows.hip"):
        _, asm = compile_device(src)
        bodies = kernel_bodies(asm)
        assert src != "sjk_attend3.hip" or sum("attend4_kernel" in k for k in bodies) == 4, sorted(bodies)
        for k, lines in bodies.items():
            bad = asm_mfma_hazards(lines)
            assert not bad, (src, k, bad[:3])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_4_4_stream_has_no_other_vector_memory_instructions():
    # between the first and the last hand-counted vmcnt wait of the 4/4 kernels the only vector memory instructions
    # are the stream's own LDS DMAs: any other (a flat or global access the compiler made, a spill) would be counted
    # by the waits and make one of them return early
    _, asm = compile_device("sjk_attend3.hip")
    bodies = {k: v for k, v in kernel_bodies(asm).items() if "attend4_kernel" in k}
    assert len(bodies) == 4, sorted(bodies)
    for k, lines in bodies.items():
        waits = [i for i in range(len(lines) - 1) if "ASMSTART" in lines[i] and "s_waitcnt vmcnt(" in lines[i + 1]]
        assert len(waits) >= 8, (k, len(waits))
        foreign = [t.strip() for t in lines[waits[0]:waits[-1]]
                   if t.strip().startswith(("flat_", "scratch_", "buffer_")) or
                   (t.strip().startswith("global_") and "_lds_" not in t.strip().split()[0])]
        assert not foreign, (k, foreign[:4])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
def test_seal_kernel_uses_no_scratch():
    res = resources("sjk_seal.hip")
    kernels = [k for k in res if "seal_kernel" in k]
    assert len(kernels) == 2, sorted(res)           # D = 128 and D = 256
    for k in kernels:
        assert res[k].get("ScratchSize [bytes/lane]", -1) == 0, (k, res[k])
