"""Assembly checks of the hot kernels (CPU; needs hipcc, skipped without it).

The GEMM and the Q4_K GEMV load into LDS with inline-asm global_load_lds_dwordx4,
which writes M0 itself: it is correct only while the compiler keeps nothing of its own
in M0 across those statements, so the generated code must not touch M0 outside the
asm blocks.  The hot kernels must also stay free of register spills (scratch).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "mold_amd", "csrc")
HIPCC = shutil.which("hipcc") or ("/opt/rocm/bin/hipcc" if os.path.exists("/opt/rocm/bin/hipcc") else None)

pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")


def _asm(tmp_path, src, defines=()):
    out = tmp_path / (os.path.basename(src) + ".s")
    cmd = [HIPCC, "-O3", "-std=c++20", "-I" + os.path.join(ROOT, "include"), "--offload-arch=gfx950",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S",
           "-o", str(out), os.path.join(CSRC, src)] + ["-D" + d for d in defines]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    return out.read_text()


def _functions(text):
    """{mangled kernel name: (body lines, {metadata key: value})}"""
    out, cur = {}, None
    for line in text.splitlines():
        m = re.match(r"^(_Z\S+):", line)
        if m:
            cur = m.group(1)
            out[cur] = ([], {})
            continue
        if cur is None:
            continue
        meta = re.search(r"; (NumVgprs|ScratchSize): (\d+)", line)
        if meta:
            out[cur][1][meta.group(1)] = int(meta.group(2))
        else:
            out[cur][0].append(line)
    return out


def _m0_outside_asm(lines):
    bad, in_asm = [], False
    for line in lines:
        if "ASMSTART" in line:
            in_asm = True
        elif "ASMEND" in line:
            in_asm = False
        elif not in_asm and not line.lstrip().startswith(";") and re.search(r"\bm0\b", line):
            bad.append(line.strip())
    return bad


@pytest.mark.parametrize("src,defines,kernel", [
    ("mq_gemm.hip", ("MQ_GEMM_TYPE=Q4_K",), "gemm_fast_kernel"),
    ("mq_gemv.hip", (), "gemv_q4k_kernel"),
])
def test_lds_dma_kernels_leave_m0_alone_and_do_not_spill(tmp_path, src, defines, kernel):
    funcs = {k: v for k, v in _functions(_asm(tmp_path, src, defines)).items() if kernel in k}
    assert funcs, f"no {kernel} in the assembly of {src}"
    for name, (lines, meta) in funcs.items():
        assert not _m0_outside_asm(lines), (name, _m0_outside_asm(lines)[:3])
        assert meta.get("ScratchSize", 0) == 0, (name, meta)


VMEM_LOAD = re.compile(r"^\s*(global_|buffer_|flat_)load")


def test_gemv_pre_quantized_x_wait_covers_its_dma(tmp_path):
    """The Q4_K GEMV on pre-quantized x issues x's LDS DMA, then its first weight loads,
    then waits vmcnt(10) for x: every path from a DMA to that wait must issue at least
    10 vector loads after the DMA (the first pair's 10 or more), so the wait covers it."""
    funcs = {k: v for k, v in _functions(_asm(tmp_path, "mq_gemv.hip")).items()
             if "gemv_q4k_kernel" in k and "Q8kX" in k}
    assert funcs, "no gemv_q4k_kernel<.., Q8kX, ..> in the assembly"
    for name, (lines, _) in funcs.items():
        body = [ln.strip() for ln in lines if ln.strip() and not ln.strip().startswith(";")]
        waits = [i for i, ln in enumerate(body) if ln.startswith("s_waitcnt vmcnt(10)")]
        assert len(waits) == 1, (name, len(waits))
        w = waits[0]
        dmas = [i for i in range(w) if "global_load_lds_dwordx4" in body[i]]
        assert dmas, name
        loads = sum(1 for i in range(dmas[-1] + 1, w) if VMEM_LOAD.match(body[i]))
        assert loads >= 10, (name, loads)
        # no branch back into the DMA loop between the loads and the wait
        assert not any(re.match(r"s_cbranch|s_branch", body[i]) for i in range(dmas[-1] + 1 + loads, w)), name
