"""Static check of the generated gfx950 assembly for a fault class of inline-asm loads.

The kernels issue many of their vector loads through inline asm (explicit
`s_waitcnt vmcnt(n)` waits keep a fixed number of loads in flight). The
compiler treats an asm statement's output register as written when the
statement retires, but the load writes it only when its data returns. If the
compiler copies that register, or reuses it for another value, before a wait
covers the load, the returning data lands on whatever the register holds by
then. When that is an address, the next load faults.

This module compiles each HIP source to device assembly with the library's
own flags. For every inline-asm vector load (between `;;#ASMSTART` and
`;;#ASMEND`) it follows every control-flow path: both successors of a
conditional branch, backward branches included. The load counts as complete
at the first `s_waitcnt vmcnt(N)` with N <= the number of vector memory
operations issued after it, since they complete in order. Any other
instruction that reads or writes one of the load's destination registers
before that point is reported.

`main()` prints the findings for every source and returns 1 if there are any;
test_asm_hazards.py runs the check over all sources (CPU only; test tooling, not part of
the library).
"""
from __future__ import annotations

import concurrent.futures as cf
import importlib
import re
import subprocess
import sys
import tempfile
from pathlib import Path

_ROOT = Path(__file__).resolve().parents[1]
if str(_ROOT) not in sys.path:
    sys.path.insert(0, str(_ROOT))
import __graft_entry__  # noqa: E402  (loads the package directory as g4mi)

__graft_entry__.load_package()
_build = importlib.import_module("g4mi.build")
ARCH, CSRC, FILE_FLAGS, HIPCC_FLAGS, _hipcc = (_build.ARCH, _build.CSRC, _build.FILE_FLAGS, _build.HIPCC_FLAGS,
                                               _build._hipcc)

_VMEM = re.compile(r"^(global_|buffer_|flat_|scratch_)(load|store|atomic)")
_BRANCH = re.compile(r"^s_(c?branch)(\w*)\s+(\.LBB\w+)")
_LABEL = re.compile(r"^(\.LBB\w+):")
_WAIT = re.compile(r"vmcnt\((\d+)\)")


def _vregs(operands: str) -> set[int]:
    out: set[int] = set()
    for m in re.finditer(r"\bv\[(\d+):(\d+)\]|\bv(\d+)\b", operands):
        if m.group(3) is not None:
            out.add(int(m.group(3)))
        else:
            out.update(range(int(m.group(1)), int(m.group(2)) + 1))
    return out


def check_function(lines: list[str]) -> list[tuple[int, str, int, str]]:
    """(load line, load, offending line, offending instruction) for one function body."""
    labels = {}
    for i, line in enumerate(lines):
        m = _LABEL.match(line.strip())
        if m:
            labels[m.group(1)] = i
    findings = []
    for i, line in enumerate(lines):
        t = line.strip()
        if not (_VMEM.match(t) and "_load" in t and "lds" not in t):
            continue
        k = i - 1
        while k >= 0 and not lines[k].strip():
            k -= 1
        if k < 0 or not lines[k].strip().startswith(";;#ASMSTART"):
            continue  # a compiler-issued load: the compiler waits for it itself
        dst = _vregs(t.split(None, 1)[1].split(",")[0])
        stack = [(i + 1, 0)]
        seen: set[tuple[int, int]] = set()
        found = None
        while stack and found is None:
            j, after = stack.pop()
            while j < len(lines):
                state = (j, min(after, 64))
                if state in seen:
                    break
                seen.add(state)
                u = lines[j].strip()
                if u.startswith("s_waitcnt"):
                    m = _WAIT.search(u)
                    if m and int(m.group(1)) <= after:
                        break
                elif u.startswith("s_endpgm"):
                    break
                elif _VMEM.match(u):
                    if _vregs(u.split(None, 1)[1]) & dst:
                        found = (j, u)
                        break
                    after += 1
                elif u and not u.startswith((".", ";")) and not u.endswith(":"):
                    m = _BRANCH.match(u)
                    if m:
                        target = labels[m.group(3)]
                        if m.group(1) == "branch":
                            j = target
                            continue
                        stack.append((target, after))
                    elif _vregs(u.split(None, 1)[1] if " " in u else "") & dst:
                        found = (j, u)
                        break
                j += 1
        if found:
            findings.append((i, t) + found)
    return findings


def check_assembly(text: str) -> dict[str, list]:
    """Findings per kernel (mangled name) of one assembly file."""
    out = {}
    for m in re.finditer(r"^(_Z\w+):", text, flags=re.M):
        end = text.find(".Lfunc_end", m.end())
        f = check_function(text[m.end():end].splitlines())
        if f:
            out[m.group(1)] = f
    return out


def device_assembly(src: Path, out: Path) -> None:
    flags = [f for f in HIPCC_FLAGS if f != "-fPIC"]
    cmd = [_hipcc(), *flags, *FILE_FLAGS.get(src.name, []), "--offload-device-only", "-S", str(src), "-o", str(out)]
    p = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if p.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name} for {ARCH}:\n{p.stdout[-4000:]}")


def check_sources(srcs: list[Path] | None = None, jobs: int = 8) -> dict[str, dict[str, list]]:
    """Findings per source file (empty dicts when clean), and the number of kernels checked under key ''."""
    srcs = srcs or sorted(CSRC.glob("*.hip"))
    results: dict[str, dict[str, list]] = {}
    with tempfile.TemporaryDirectory() as td:
        outs = [Path(td) / (s.stem + ".s") for s in srcs]
        with cf.ThreadPoolExecutor(min(jobs, len(srcs))) as ex:
            list(ex.map(lambda p: device_assembly(*p), zip(srcs, outs)))
        kernels = 0
        for s, o in zip(srcs, outs):
            text = o.read_text()
            kernels += len(re.findall(r"^_Z\w+:", text, flags=re.M))
            results[s.name] = check_assembly(text)
    results[""] = {"kernels": kernels}  # type: ignore[dict-item]
    return results


def main() -> int:
    res = check_sources()
    bad = 0
    for name, per in res.items():
        if not name:
            continue
        for kern, f in per.items():
            bad += len(f)
            print(f"{name}: {kern}: {len(f)} finding(s)")
            for i, load, j, use in f[:3]:
                print(f"    load (line {i}): {load}\n    use  (line {j}): {use}")
    print(f"{res['']['kernels']} kernels checked, {bad} findings")
    return 1 if bad else 0
