"""Schedule invariants of the tiled MXFP4 GEMM (moe.hip::moe_mxfp4_gemm_kernel), checked on the
compiled gfx950 assembly (CPU only: hipcc cross-compiles).

The kernel waits for a pipeline stage with an explicit `s_waitcnt vmcnt(N)`: vector-memory
operations complete in issue order, so the wait is only right if exactly the expected loads were
issued after the stage's own, group by group.  The compiler is free to reorder independent loads
unless fenced, and spill code adds vector-memory operations, so both are pinned here:
  * inside every group loop, each group issues exactly LOADS operations (2 weight-tile register
    loads, 2 scale-row and ceil(MT/2) activation direct-to-LDS loads, MT = 2..6 row tiles: one loop
    per MT, two MTs per activation-load count 2 and 3) and the loop has no scratch access;
  * before every stage wait in a pass prologue, the operations since the last full drain end in
    whole groups of that composition (no later group's load moved ahead of an earlier group's);
    fewer than 3 groups after a drain are fine, the drain completed everything before it.
A reordering of this kind once let a wave read a stage whose activation block was still in flight.
"""
import os
import re
import shutil
import subprocess
from collections import Counter

import pytest

from flyai_amd import build as B

HIPCC = B.HIPCC if os.path.exists(B.HIPCC) else shutil.which("hipcc")
pytestmark = pytest.mark.skipif(HIPCC is None, reason="hipcc not available")

VMEM = re.compile(r"\s*(global_load\w*|global_store\w*|scratch_\w+|buffer_\w+)")


def _group(md):
    """One group's loads with md activation direct-to-LDS loads (md = ceil(MT / 2))."""
    return Counter({"global_load_dwordx4": 2, "global_load_lds_dword": 2, "global_load_lds_dwordx4": md})


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("asm") / "moe.s"
    flags = [f for f in B.FLAGS if f != "-fPIC"]
    r = subprocess.run([HIPCC, *flags, "-S", "--cuda-device-only", "-x", "hip",
                        os.path.join(B.CSRC, "moe.hip"), "-o", str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    text = out.read_text()
    bodies = {}
    for name in re.findall(r"\n(_ZN5flyai21moe_mxfp4_gemm_kernel\w+):", text):
        i = text.index("\n" + name + ":")
        bodies[name] = text[i:text.index(".Lfunc_end", i)].split("\n")
    assert len(bodies) == 2, "expected the gate_up and down instantiations"
    return bodies


def _ops(lines):
    return [m.group(1) for m in (VMEM.match(l) for l in lines) if m]


def test_group_loops_issue_exact_groups(gemm_asm):
    for name, body in gemm_asm.items():
        loops = [n for n, l in enumerate(body) if "Inner Loop Header" in l]
        assert len(loops) == 5, f"{name}: one group loop per row-tile count"
        seen = Counter()
        for lo in loops:
            hi = next(n for n in range(lo, len(body)) if re.search(r"s_cbranch\w* \.LBB", body[n]))
            waits = [n for n in range(lo, hi) if re.search(r"s_waitcnt vmcnt\(\d+\)", body[n])]
            assert waits, f"{name}: group loop without a stage wait"
            wait_n = {int(re.search(r"vmcnt\((\d+)\)", body[w]).group(1)) for w in waits}
            assert len(wait_n) == 1
            loads = wait_n.pop() // 2  # the stage wait leaves 2 younger groups in flight
            md = loads - 4
            assert md in (1, 2, 3)
            seen[md] += 1
            assert not any("scratch_" in body[n] for n in range(lo, hi)), f"{name}: spill code in a group loop"
            bounds = waits + [hi]
            for a, b in zip(bounds, bounds[1:]):
                assert Counter(_ops(body[a:b])) == _group(md), f"{name} MD={md}: group issue {_ops(body[a:b])}"
        assert seen == Counter({1: 1, 2: 2, 3: 2})


def test_prologue_issues_groups_in_order(gemm_asm):
    for name, body in gemm_asm.items():
        checked = 0
        for w, line in enumerate(body):
            m = re.search(r"s_waitcnt vmcnt\((15|18|21)\)", line)
            if not m:
                continue
            loads = int(m.group(1)) // 3
            md = loads - 4
            ops = []
            for n in range(w - 1, -1, -1):
                t = body[n].strip()
                if t.startswith("s_waitcnt vmcnt(0)") or t.startswith("s_barrier"):
                    break
                mm = VMEM.match(body[n])
                if mm:
                    ops.append(mm.group(1))
            ops.reverse()
            # the youngest 3 groups must be whole groups; if fewer loads follow the last drain, the
            # loads before it are complete and the rest must be the tail of one group
            whole = min(3, len(ops) // loads)
            for g in range(whole):
                chunk = ops[len(ops) - (g + 1) * loads:len(ops) - g * loads]
                assert Counter(chunk) == _group(md), f"{name} MD={md}: {ops}"
            if whole < 3:
                head = Counter(ops[:len(ops) - whole * loads])
                assert not head - _group(md), f"{name} MD={md}: {ops}"
            checked += 1
        assert checked == 5, f"{name}: expected one prologue wait per row-tile count"
