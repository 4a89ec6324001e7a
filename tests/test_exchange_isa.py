"""CPU: the split-K partial exchange of the decode kernels, checked in the gfx950 assembly hipcc emits.

Workgroups on different XCDs exchange partials through memory. Every access to a partial is an agent-scope
relaxed atomic, and the order between a workgroup's partial stores and the arrival that announces them is kept
by the instruction sequence itself (decode_common.h, ws_publish / ws_arrive / ws_acquire), not by the memory
model's fences (measured 4.3x slower). This test compiles the kernels to assembly on every run and checks that
sequence, so a change in how the compiler lowers these accesses fails here instead of silently on a GPU:

  * partial stores write through the L2 (`global_store* ... sc1`);
  * `s_waitcnt vmcnt(0)` and `s_barrier` come after the last of them and before the arrival's fetch-add
    (`global_atomic_add ... sc0`, which returns the count);
  * partial loads miss the L2 (`global_load* ... sc1`) and come only after the fetch-add.
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "bytes-per-token_amd" / "csrc"

# (source, mangled-name prefix of one instantiation that splits segments across workgroups)
KERNELS = [
    ("paged_decode_mfma.hip", "_ZN3bpt18decode_mfma_kernelILi1ELi1ELb1ELb0ELi4ELb0EEEvNS_12DecodeParamsE"),
    ("paged_decode_mfma.hip", "_ZN3bpt18decode_mfma_kernelILi1ELi1ELb1ELb0ELi2ELb0EEEvNS_12DecodeParamsE"),
    ("paged_decode.hip", "_ZN3bpt13decode_kernel"),
    ("kivi_decode.hip", "_ZN3bpt18kivi_decode_kernelILi0ELi2ELb0EE"),
]


def device_assembly(src: str, tmp: Path) -> str:
    from bpt_amd import _build

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc not available")
    out = tmp / (Path(src).stem + ".s")
    flags = [f for f in _build.HIPCC_FLAGS if f not in ("-fPIC",)]
    cmd = [hipcc, *flags, f"-I{ROOT / 'include'}", f"-I{CSRC}", "--cuda-device-only", "-S", str(CSRC / src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return out.read_text()


def kernel_body(asm: str, prefix: str) -> list[str]:
    m = re.search(r"^(" + re.escape(prefix) + r"\w*):", asm, flags=re.M)
    assert m, f"no kernel {prefix} in the assembly"
    end = asm.index(".Lfunc_end", m.end())
    lines = []
    for raw in asm[m.end():end].split("\n"):
        line = raw.split(";")[0].strip()
        if line and (not line.startswith(".") or re.match(r"^\.LBB\w+:", line)):
            lines.append(line)
    return lines


def basic_blocks(body: list[str]) -> tuple[list[list[str]], list[list[int]]]:
    """The kernel's basic blocks (instruction lists) and each block's successors (by index)."""
    blocks, names = [[]], ["entry"]
    for line in body:
        label = re.match(r"^(\.LBB\w+):", line)
        if label:
            blocks.append([])
            names.append(label.group(1))
            continue
        blocks[-1].append(line)
        if re.match(r"^s_(c?branch|setpc|endpgm)", line):
            blocks.append([])
            names.append(None)
    index = {n: i for i, n in enumerate(names) if n}
    succ = []
    for i, ins in enumerate(blocks):
        last = ins[-1] if ins else ""
        out = []
        target = re.match(r"^s_c?branch\w*\s+(\.LBB\w+)", last)
        if target:
            out.append(index[target.group(1)])
        if not re.match(r"^s_(branch|setpc|endpgm)\b", last) and i + 1 < len(blocks):
            out.append(i + 1)  # falls through
        succ.append(out)
    return blocks, succ


def is_partial_store(line: str) -> bool:
    return line.startswith("global_store") and re.search(r"\bsc1\b", line) is not None


def is_partial_load(line: str) -> bool:
    return line.startswith("global_load") and re.search(r"\bsc1\b", line) is not None


def check_exchange(body: list[str]) -> list[str]:
    """Dataflow over the kernel's control flow.

    Stores, per path: 0 clean, 1 partial stores waited for (s_waitcnt vmcnt(0)), 2 pending; a barrier turns
    1 into 0, and the fetch-add needs 0 on every path. Arrival, per path: 0 nothing, 1 past the fetch-add (its
    own wave ran it, or skipped it by an exec-mask branch while the workgroup's first thread ran it), 2 past a
    barrier after that; each partial load needs 2 on every path.
    """
    blocks, succ = basic_blocks(body)
    n = len(blocks)
    # Exec-mask branches that jump forward over a block holding the fetch-add (the waves with no lane that
    # runs it; the guarded region is laid out between the branch and its target).
    atomic_blocks = [b for b in range(n) if any(l.startswith("global_atomic_add") for l in blocks[b])]
    skips = {(b, t) for b in range(n) for t in succ[b]
             if blocks[b] and blocks[b][-1].startswith("s_cbranch_execz") and t > b + 1
             and any(b < a < t for a in atomic_blocks)}
    pend_in, arr_in = [None] * n, [None] * n
    pend_in[0], arr_in[0] = 0, 0
    problems, work = [], [0]
    while work:
        b = work.pop()
        pend, arr = pend_in[b], arr_in[b]
        for line in blocks[b]:
            if is_partial_store(line):
                pend = 2
            elif line.startswith("s_waitcnt") and "vmcnt(0)" in line and pend == 2:
                pend = 1
            elif line.startswith("s_barrier"):
                pend = 0 if pend == 1 else pend
                arr = 2 if arr == 1 else arr
            elif line.startswith("global_atomic_add"):
                if pend != 0:
                    problems.append(f"fetch-add reachable with partial stores not waited for and barriered: {line}")
                arr = 1
            elif is_partial_load(line) and arr != 2:
                problems.append(f"partial load reachable before the fetch-add and a barrier: {line}")
        for s2 in succ[b]:
            a2 = max(arr, 1) if (b, s2) in skips else arr
            new_p = pend if pend_in[s2] is None else max(pend_in[s2], pend)
            new_a = a2 if arr_in[s2] is None else min(arr_in[s2], a2)
            if new_p != pend_in[s2] or new_a != arr_in[s2]:
                pend_in[s2], arr_in[s2] = new_p, new_a
                work.append(s2)
    return sorted(set(problems))


@pytest.fixture(scope="module")
def assembly(tmp_path_factory):
    """The three sources' device assembly, compiled concurrently (each takes tens of seconds)."""
    from concurrent.futures import ThreadPoolExecutor

    tmp = tmp_path_factory.mktemp("isa")
    srcs = sorted({src for src, _ in KERNELS})
    with ThreadPoolExecutor(max_workers=len(srcs)) as pool:
        return dict(zip(srcs, pool.map(lambda s: device_assembly(s, tmp), srcs)))


@pytest.mark.parametrize("src,prefix", KERNELS)
def test_partial_exchange_sequence(src, prefix, assembly):
    body = kernel_body(assembly[src], prefix)
    assert any(l.startswith("global_atomic_add") and re.search(r"\bsc0\b", l) for l in body), "no returning fetch-add"
    assert any(is_partial_store(l) for l in body) and any(is_partial_load(l) for l in body)
    problems = check_exchange(body)
    assert not problems, problems[:5]


def test_checker_finds_a_missing_wait():
    """The checker itself: a path from a partial store to the fetch-add with no wait, or a load before it."""
    good = ["global_store_dwordx2 v[0:1], v[2:3], off sc1", "s_waitcnt vmcnt(0)", "s_barrier",
            "s_cbranch_execz .LBB0_1", "global_atomic_add v1, v2, v3, s[0:1] sc0", ".LBB0_1:", "s_waitcnt vmcnt(0)",
            "s_barrier", "global_load_dword v4, v[0:1], off sc1", "s_endpgm"]
    assert check_exchange(good) == []
    assert check_exchange([l for l in good if not l.startswith("s_waitcnt")])  # no wait
    assert check_exchange([l for l in good[:2] + good[3:]])  # no barrier before the fetch-add
    assert check_exchange(good[:7] + good[8:])  # no barrier between the fetch-add and the loads
    early = ["global_load_dword v4, v[0:1], off sc1"] + good
    assert check_exchange(early)
    # A branch around the wait leaves one path unwaited.
    branchy = ["global_store_dword v[0:1], v2, off sc1", "s_cbranch_scc1 .LBB0_2", "s_waitcnt vmcnt(0)", ".LBB0_2:",
               "s_barrier", "global_atomic_add v1, v2, v3, s[0:1] sc0", "s_endpgm"]
    assert check_exchange(branchy)
