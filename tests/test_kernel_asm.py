"""Register discipline of the wide prefill GEMM's inline assembly (CPU only:
compiles k_prefill.hip for gfx950 and reads the assembly).

k_q4_gemm_wide issues its weight loads as inline assembly and waits for them
with hand-counted s_waitcnt vmcnt(N): the compiler treats an asm output as
ready at once, so nothing else may read, write or copy a destination register
of such a load until a wait has retired it. The check models the wave's
in-order vector-memory queue (the asm loads and the global->LDS DMA the
compiler emits) and fails on any other instruction that touches a register
of a load still in the queue. It also pins the waits the kernel's schedule
relies on."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "enginesmith-qwen35-08b-long-decode-m5max-round005_amd")
HIPCC = "/opt/rocm/bin/hipcc"


def _regs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def inflight_hazards(lines):
    """Instructions that touch a register of a vector load still in flight.
    Loads retire in issue order; s_waitcnt vmcnt(n) leaves the newest n."""
    queue, bad = [], []
    for i, line in enumerate(lines):
        t = line.strip()
        if t.startswith(("global_load_dwordx4", "global_load_ushort")):
            queue.append(_regs(t.split()[1].rstrip(",")))
            continue
        if t.startswith("global_load_lds"):
            queue.append(set())
            continue
        if t.startswith("s_waitcnt") and "vmcnt" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            queue = queue[len(queue) - n:] if 0 < n < len(queue) else ([] if n == 0 else queue)
            continue
        if t.startswith(("v_", "ds_", "global_store", "buffer_")):
            used = set()
            for tok in re.findall(r"v\[\d+:\d+\]|v\d+", t):
                used |= _regs(tok)
            if any(used & q for q in queue):
                bad.append((i, t))
    return bad


@pytest.fixture(scope="module")
def wide_asm(tmp_path_factory):
    if not os.path.exists(HIPCC) or shutil.which("ld.lld", path="/opt/rocm/llvm/bin") is None:
        pytest.skip("hipcc for gfx950 is not installed")
    out = tmp_path_factory.mktemp("asm") / "k_prefill.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fhip-fp32-correctly-rounded-divide-sqrt",
           "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), "-Xclang", "-target-feature", "-Xclang",
           "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(out),
           os.path.join(PKG, "csrc", "k_prefill.hip")]
    subprocess.run(cmd, check=True, capture_output=True, cwd=os.path.join(PKG, "csrc"))
    lines = out.read_text().splitlines()
    start = next(i for i, l in enumerate(lines) if re.match(r"^_ZN2es12_GLOBAL__N_114k_q4_gemm_wide\w*:", l))
    end = next(i for i in range(start, len(lines)) if "s_endpgm" in lines[i])
    return lines[start:end + 1]


def test_no_register_of_an_inflight_load_is_touched(wide_asm):
    bad = inflight_hazards(wide_asm)
    assert not bad, "touches an in-flight load register: " + "; ".join(f"{i}: {t}" for i, t in bad[:5])


def test_the_counted_waits_are_present(wide_asm):
    text = "\n".join(wide_asm)
    # the weight set of the next step (12 operations after it) and the X DMA (4 after it)
    assert text.count("s_waitcnt vmcnt(12)") >= 2
    assert text.count("s_waitcnt vmcnt(4)") >= 3
    assert len(re.findall(r"v_mfma_f32_32x32x16_bf16", text)) == 128  # two 64-column steps per loop pass


def test_the_checker_finds_a_planted_hazard():
    """A copy of a load's destination before its wait is flagged; after it, not."""
    planted = ["global_load_dwordx4 v[2:5], v[10:11], off",
               "global_load_lds_dwordx4 v[12:13], off",
               "v_mov_b32_e32 v20, v3",
               "s_waitcnt vmcnt(1)",
               "v_mov_b32_e32 v21, v4"]
    bad = inflight_hazards(planted)
    assert [i for i, _ in bad] == [2]
