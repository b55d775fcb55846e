"""Per-kernel resource usage of the HIP library as the compiler reports it
(VGPRs, SGPRs, private scratch bytes per lane, occupancy in waves per SIMD),
one line per kernel instance: hipcc's kernel-resource-usage remarks for a
device-only compile of gaans_w64.hip with the build's flags.

Usage: python fast-compressai_amd/csrc/resource_report.py > report.txt
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import build  # noqa: E402


def main() -> None:
    flags = [f for f in build.FLAGS if f not in ("-shared", "-fPIC")]
    with tempfile.TemporaryDirectory() as tmp:
        cmd = [build.hipcc(), *flags, "--cuda-device-only", "-c", build.SOURCES[0], "-o",
               os.path.join(tmp, "dev.o"), "-Rpass-analysis=kernel-resource-usage"]
        res = subprocess.run(cmd, capture_output=True, text=True, check=True)
    shown = [os.path.relpath(c, build.REPO) if c.startswith(build.REPO) else c for c in cmd]
    shown[shown.index("-o") + 1] = "<tmp>/dev.o"
    print("command (python fast-compressai_amd/csrc/resource_report.py runs it): " + " ".join(shown))
    rows, cur = [], None
    for line in res.stderr.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = {"name": m.group(1)}
            rows.append(cur)
            continue
        for key in ("VGPRs", "SGPRs", "ScratchSize", "Occupancy"):
            m = re.search(key + r"[^:]*: (\d+)", line)
            if m and cur is not None and key not in cur:
                cur[key] = int(m.group(1))
    names = subprocess.run(["c++filt"], input="\n".join(r["name"] for r in rows),
                           capture_output=True, text=True).stdout.splitlines()
    print(f"{'kernel':58s} VGPRs SGPRs scratch(B/lane) occupancy(waves/SIMD)")
    for r, n in zip(rows, names):
        n = n.replace("(anonymous namespace)::", "").replace("void ", "")
        print(f"{n[:58]:58s} {r.get('VGPRs', 0):5d} {r.get('SGPRs', 0):5d} "
              f"{r.get('ScratchSize', 0):15d} {r.get('Occupancy', 0):9d}")


if __name__ == "__main__":
    main()
