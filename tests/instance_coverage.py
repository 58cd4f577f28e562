"""Which kernel instances compiled into libdopt.so does a kernel trace never launch?

Run the GPU suite under a kernel trace on an MI355X, from /tmp with TMPDIR=/tmp (R = repository
root):

    rocprofv3 --kernel-trace --output-format csv -d /tmp/tt -o t -- python3 -m pytest -q $R/tests -m gpu

then, anywhere the library is built:

    python3 tests/instance_coverage.py /tmp/tt

It lists every `dopt::` kernel instance in the library's symbol table (`nm -C`) that no row of the
trace's *kernel_trace.csv files names, and exits 1 if there is one. Not a pytest module: it reads
the output of a profiled GPU run.
"""
import csv
import glob
import os
import re
import subprocess
import sys

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "deep_optimization_amd",
                   "libdopt.so")


def instance_name(name: str) -> str:
    """`dopt::kernel<args>` of a demangled symbol or trace name: no return type, no anonymous
    namespace, no parameter list."""
    name = name.replace("void ", "").replace("(anonymous namespace)::", "").strip()
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def built_instances(lib: str = LIB) -> set:
    out = subprocess.run(["nm", "-C", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    names = set()
    for line in out.splitlines():
        parts = line.split(" ", 2)
        if len(parts) == 3 and "dopt::" in parts[2] and "__device_stub__" not in parts[2] \
                and re.search(r"_kernel[<(]", parts[2]):
            names.add(instance_name(parts[2]))
    return names


def traced_instances(trace_dir: str) -> set:
    names = set()
    for path in glob.glob(os.path.join(trace_dir, "**", "*kernel_trace.csv"), recursive=True):
        with open(path) as f:
            for row in csv.DictReader(f):
                if "dopt::" in row["Kernel_Name"]:
                    names.add(instance_name(row["Kernel_Name"]))
    return names


def main(argv) -> int:
    if len(argv) != 2:
        print(__doc__)
        return 2
    built, traced = built_instances(), traced_instances(argv[1])
    missing = sorted(built - traced)
    print(f"{len(built)} kernel instances in {LIB}; {len(built) - len(missing)} launched in the trace")
    for name in missing:
        print("  not launched:", name)
    return 1 if missing else 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
