"""Register and wait discipline of the prefill kernels' hand-counted memory
waits (CPU only: compiles k_prefill.hip for gfx950 and reads the assembly).

k_q4_gemm_wide issues its weight loads as inline assembly and waits for them
with hand-counted s_waitcnt vmcnt(N): the compiler treats an asm output as
ready at once, so nothing else may read, write or copy a destination register
of such a load until a wait has retired it. The check models the wave's
in-order vector-memory queue (every load, store and atomic, global or buffer,
and the DMA into LDS, which occupies a slot but writes no register), walks
each loop body twice so that a load issued late in an iteration meets the
instructions at the top of the next, and fails on any instruction that
touches a register of a load still in the queue.

k_attn_prefill stages each 32-key block of K and V with 8 DMA instructions
per wave and waits with vmcnt(16), vmcnt(8) or vmcnt(0) before the barrier
that publishes block kb (the two, one or no newer blocks still in flight):
that arithmetic holds only if the loop issues nothing else to the queue, which
is checked too."""
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


VMEM = re.compile(r"(global|buffer)_(load|store|atomic)")


def queue_entry(t):
    """Registers a vector-memory operation writes when it completes: the
    destination of a load, nothing for stores, atomics without return and
    loads into LDS (which still take a slot of the in-order queue)."""
    op = t.split()[0]
    if "_load" in op and not t.rstrip().endswith(" lds") and not op.startswith("global_load_lds"):
        return _regs(t.split()[1].rstrip(","))
    return set()


def walk(lines):
    """The lines in program order with every backward branch taken once more
    (each loop body walked a second time)."""
    labels = {l.strip().split(":")[0]: i for i, l in enumerate(lines) if re.match(r"^\.LBB\w*:", l.strip())}
    order, taken = [], set()
    for i, line in enumerate(lines):
        order.append(i)
        m = re.match(r"s_(cbranch_\w+|branch)\s+(\.LBB\w+)", line.strip())
        if m and m.group(2) in labels and labels[m.group(2)] < i and i not in taken:
            taken.add(i)
            order.extend(range(labels[m.group(2)], i + 1))
    return order


def inflight_hazards(lines):
    """Instructions that touch a register of a vector load still in flight.
    Operations retire in issue order; s_waitcnt vmcnt(n) leaves the newest n."""
    queue, bad = [], []
    for i in walk(lines):
        t = lines[i].strip()
        if VMEM.match(t):
            queue.append(queue_entry(t))
            continue
        if t.startswith("s_waitcnt") and "vmcnt" in t:
            n = int(re.search(r"vmcnt\((\d+)\)", t).group(1))
            queue = queue[len(queue) - n:] if n > 0 else []
            continue
        if t.startswith(("v_", "ds_")):
            used = set()
            for tok in re.findall(r"v\[\d+:\d+\]|v\d+", t):
                used |= _regs(tok)
            if any(used & q for q in queue):
                bad.append((i, t))
    return bad


def kernel_asm(tmp_path_factory, name):
    if not os.path.exists(HIPCC) or shutil.which("ld.lld", path="/opt/rocm/llvm/bin") is None:
        pytest.skip("hipcc for gfx950 is not installed")
    out = tmp_path_factory.getbasetemp() / "k_prefill.s"
    if not out.exists():
        cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fhip-fp32-correctly-rounded-divide-sqrt",
               "-ffp-contract=off", "-I" + os.path.join(ROOT, "include"), "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(out),
               os.path.join(PKG, "csrc", "k_prefill.hip")]
        subprocess.run(cmd, check=True, capture_output=True, cwd=os.path.join(PKG, "csrc"))
    lines = out.read_text().splitlines()
    start = next(i for i, l in enumerate(lines) if re.match(r"^_ZN2es12_GLOBAL__N_1\d+" + name + r"\w*:", l))
    end = next(i for i in range(start, len(lines)) if "s_endpgm" in lines[i])
    return lines[start:end + 1]


@pytest.fixture(scope="module")
def wide_asm(tmp_path_factory):
    return kernel_asm(tmp_path_factory, "k_q4_gemm_wide")


@pytest.fixture(scope="module")
def attn_asm(tmp_path_factory):
    return kernel_asm(tmp_path_factory, "k_attn_prefill")


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


def test_attention_prefill_registers(attn_asm):
    bad = inflight_hazards(attn_asm)
    assert not bad, "touches an in-flight load register: " + "; ".join(f"{i}: {t}" for i, t in bad[:5])


def test_attention_prefill_barrier_waits(attn_asm):
    """The key-block loop: from its head to the barrier that publishes block
    kb it issues no memory operation and waits with vmcnt(16), vmcnt(8) or
    vmcnt(0) only; from the barrier to the back edge it issues exactly the 8
    DMA instructions that stage block kb + 3 and nothing else, so the count
    of newer blocks in flight is what the waits assume."""
    lines = [l.strip() for l in attn_asm]
    barriers = [i for i, t in enumerate(lines) if t.startswith("s_barrier")]
    assert len(barriers) == 1, "one barrier per key block"
    bar = barriers[0]
    labels = {t.split(":")[0]: i for i, t in enumerate(lines) if re.match(r"^\.LBB\w*:", t)}
    back = next(i for i in range(bar, len(lines))
                if (m := re.match(r"s_(cbranch_\w+|branch)\s+(\.LBB\w+)", lines[i])) and labels[m.group(2)] < bar)
    head = labels[re.match(r"s_\w+\s+(\.LBB\w+)", lines[back]).group(1)]
    waits = [int(m.group(1)) for t in lines[head:bar] if (m := re.match(r"s_waitcnt vmcnt\((\d+)\)", t))]
    assert not any(VMEM.match(t) for t in lines[head:bar])
    assert waits and set(waits) == {0, 8, 16}, waits
    ops = [t for t in lines[bar:back] if VMEM.match(t)]
    assert len(ops) == 8 and all(t.startswith("buffer_load_dwordx4") and t.endswith(" lds") for t in ops), ops


def test_the_checker_follows_a_loop_back_edge():
    """A load issued at the end of a loop body and used at its top before a
    wait is flagged only when the back edge is walked."""
    planted = [".LBB0_1:",
               "v_mov_b32_e32 v20, v3",
               "s_waitcnt vmcnt(0)",
               "global_load_dwordx4 v[2:5], v[10:11], off",
               "buffer_store_dword v7, v8, s[0:3], 0 offen",
               "s_cbranch_scc1 .LBB0_1",
               "s_waitcnt vmcnt(0)"]
    bad = inflight_hazards(planted)
    assert [t for _, t in bad] == ["v_mov_b32_e32 v20, v3"]
