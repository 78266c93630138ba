"""Kernel-instantiation coverage of the GPU test suite.

Every route of the dispatch trees ends in one instantiation of a kernel
template, so "every route is tested" is checked as "every kernel instantiation
in libnq_hip.so was launched by some -m gpu test".

    python tests/route_coverage.py <trace_dir> <times_file> > profiles/gpu_test_kernel_coverage.txt

builds the committed summary from a kernel trace of the GPU suite:

    cd /tmp && TMPDIR=/tmp NQ_TEST_TIMES=<times_file> rocprofv3 --kernel-trace --output-format csv \\
        -d <trace_dir> -o run -- python3 -m pytest <repo>/tests -m gpu -q -p no:cacheprovider

(NQ_TEST_TIMES makes tests/conftest.py log each test's start and end.) Each
line of the summary is `<kernel instantiation>\\t<dispatches>\\t<first test that
launched it>`. tests/test_route_coverage.py compares it with the
instantiations the library holds (host-side kernel handles, from nm).
"""
from __future__ import annotations

import bisect
import csv
import glob
import os
import re
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "nanoinfer_amd", "libnq_hip.so")
SUMMARY = os.path.join(ROOT, "profiles", "gpu_test_kernel_coverage.txt")


def demangle(names):
    """Itanium demangling with binutils' c++filt, which does not know the
    _Float16 code DF16_: it is rewritten to Dh (a builtin type as well, so the
    substitution numbering is unchanged) and shows as `half`."""
    names = [n.replace("DF16_", "Dh") if n.startswith("_Z") else n for n in names]
    if not names:
        return []
    r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True, check=True)
    return r.stdout.splitlines()


def key(demangled: str) -> str | None:
    """`void nq::(anonymous namespace)::gemv_q8_kernel<2, 4, float, ...>(args)` ->
    `gemv_q8_kernel<2, 4, float, ...>`; None for kernels outside namespace nq."""
    m = re.search(r"nq::\(anonymous namespace\)::(\w+(?:<.*>)?)\(", demangled)
    if not m:
        return None
    return m.group(1).replace("nq::(anonymous namespace)::", "").replace("_Float16", "half")


def library_kernels(lib: str = LIB) -> set[str]:
    """Kernel instantiations compiled into the library: the host-side kernel
    handles (data symbols named for each __global__ instantiation)."""
    out = subprocess.run(["nm", lib], capture_output=True, text=True, check=True).stdout
    mangled = [ln.split()[-1] for ln in out.splitlines()
               if len(ln.split()) == 3 and ln.split()[1] in "dD" and ln.split()[-1].startswith("_ZN2nq")]
    ks = {key(d) for d in demangle(mangled)}
    return {k for k in ks if k and "_kernel" in k}


def read_summary(path: str = SUMMARY) -> dict[str, tuple[int, str]]:
    got = {}
    with open(path) as f:
        for ln in f:
            if ln.startswith("#") or not ln.strip():
                continue
            name, count, test = ln.rstrip("\n").split("\t")
            got[name] = (int(count), test)
    return got


def summarize(trace_dir: str, times_file: str) -> str:
    f = glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True)
    if not f:
        raise SystemExit(f"no kernel_trace.csv under {trace_dir}")
    rows = list(csv.DictReader(open(f[0])))
    starts = [int(r["Start_Timestamp"]) for r in rows]
    spans = {"mono": [], "boot": []}
    for ln in open(times_file):
        clk, t0, t1, test = ln.rstrip("\n").split(" ", 3)
        spans[clk].append((int(t0), int(t1), test))
    # the clock whose test spans contain the kernel timestamps
    def hits(sp):
        b = sorted(sp)
        n = 0
        for t in starts[:: max(1, len(starts) // 200)]:
            i = bisect.bisect_right([s[0] for s in b], t) - 1
            n += i >= 0 and b[i][0] <= t <= b[i][1]
        return n
    clk = max(spans, key=lambda c: hits(spans[c]))
    sp = sorted(spans[clk])
    s0 = [s[0] for s in sp]
    names = demangle([r["Kernel_Name"] for r in rows])
    cov: dict[str, list] = {}
    for r, dn in zip(rows, names):
        k = key(dn)
        if not k:
            continue
        t = int(r["Start_Timestamp"])
        i = bisect.bisect_right(s0, t) - 1
        test = sp[i][2] if i >= 0 and sp[i][0] <= t <= sp[i][1] else "?"
        e = cov.setdefault(k, [0, test])
        e[0] += 1
        if e[1] == "?":
            e[1] = test
    lines = [f"# kernel instantiations launched by `pytest tests -m gpu` (clock: {clk}); "
             "see tests/route_coverage.py for the command",
             "# instantiation\tdispatches\tfirst test"]
    lines += [f"{k}\t{v[0]}\t{v[1]}" for k, v in sorted(cov.items())]
    return "\n".join(lines) + "\n"


if __name__ == "__main__":
    sys.stdout.write(summarize(sys.argv[1], sys.argv[2]))
