"""Register budgets of the kernels, read from the compiler's resource remarks (hipcc -Rpass-analysis=
kernel-resource-usage on the library's own sources, gfx950; no GPU needed).

The streaming attention kernels wait for their HBM -> LDS copies with hand-counted `s_waitcnt vmcnt(N)`, so any
compiler-made vector memory access in them (a register spill to scratch) would make a wait return early and the
kernel read LDS before its data arrived: they must use no scratch. The seal must not spill either (a spill there
once cost 30 MB of scratch traffic per commit). A compiler or source change that breaks this fails here, before
anything runs on a GPU."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "sj-kvarn-codec_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["-std=c++17", "-O3", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off",
         "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-gpu-flush-denormals-to-zero",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-x", "hip", "-c", "-o", os.devnull,
         "-Rpass-analysis=kernel-resource-usage", "--cuda-device-only"]


def resources(src):
    out = subprocess.run([HIPCC] + FLAGS + [os.path.join(CSRC, src)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stderr[-2000:]
    res, name = {}, None
    for line in out.stderr.splitlines():
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
def test_seal_kernel_uses_no_scratch():
    res = resources("sjk_seal.hip")
    kernels = [k for k in res if "seal_kernel" in k]
    assert len(kernels) == 2, sorted(res)           # D = 128 and D = 256
    for k in kernels:
        assert res[k].get("ScratchSize [bytes/lane]", -1) == 0, (k, res[k])
