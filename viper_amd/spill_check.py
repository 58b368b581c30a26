#!/usr/bin/env python3
"""Scratch check of every kernel in the HIP library (maintainer tool, run by `make -C viper_amd spillcheck`).

Compiles each translation unit for gfx950 with the compiler's resource-usage remarks and reports every
kernel whose scratch size is not zero.  A kernel that spills its registers to scratch pays a memory
round trip per spilled value; the multi-row int8 GEMV once did so at every row load and ran 2.4x
slower.  Exits 1 if a kernel outside the known set below uses scratch:
  - qgemv_m1_kernel in its partials mode (MODE 1, the test entry viper_hip_qlinear_partials);
  - qgemv_m1_kernel for Q6 on 640 threads without an exact tiling (8-24 bytes: every LDS operand of a
    segment is read before the first dot, 2-6 registers past the 168-VGPR limit of 640 threads).
Usage: spill_check.py HIPCC FLAGS... -- SOURCES...
"""
import re
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor


def kernels_with_scratch(cmd, src):
    out = subprocess.run(cmd + ["--cuda-device-only", "-c", "-o", "/dev/null",
                                "-Rpass-analysis=kernel-resource-usage", src],
                         capture_output=True, text=True)
    if out.returncode != 0:
        sys.exit(f"{src}: compile failed\n{out.stderr[-2000:]}")
    found, name = [], None
    for line in out.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and name is not None and int(m.group(1)) > 0:
            found.append((name, int(m.group(1))))
    return found


def demangle(names):
    out = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True).stdout
    return out.splitlines()


def known(pretty):
    # qgemv_m1_kernel<F, TS, NTT, CPL, SENC, MODE, EXACT, PRO, MR, DELAY, KC>
    m = re.search(r"qgemv_m1_kernel<(\d+), (\d+), (\d+), (\d+), (\d+), (\d+), (true|false), (\d+), (\d+), (\d+), (\d+)>",
                  pretty)
    if not m:
        return False
    f, ntt, mode, exact = int(m.group(1)), int(m.group(3)), int(m.group(6)), m.group(7) == "true"
    return mode == 1 or (f == 6 and ntt == 640 and not exact)


def main():
    args = sys.argv[1:]
    cut = args.index("--")
    cmd, srcs = args[:cut], args[cut + 1:]
    with ThreadPoolExecutor(max_workers=8) as ex:
        results = list(ex.map(lambda s: (s, kernels_with_scratch(cmd, s)), srcs))
    bad = 0
    for src, found in results:
        if not found:
            continue
        pretty = demangle([n for n, _ in found])
        for (_, b), p in zip(found, pretty):
            tag = "known" if known(p) else "NEW"
            bad += tag == "NEW"
            print(f"{tag:5} {b:5} B/lane  {src}: {p[:200]}")
    total = sum(len(f) for _, f in results)
    print(f"spillcheck: {total} kernels use scratch, {bad} outside the known set")
    return 1 if bad else 0


if __name__ == "__main__":
    sys.exit(main())
