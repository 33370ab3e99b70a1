"""Per-kernel register and scratch use of the gfx950 code, from the compiler's
own resource-usage remarks (hipcc -Rpass-analysis=kernel-resource-usage).

    python3 edgebert_amd/csrc/resource_report.py [--fail-on-scratch]

prints one line per kernel (VGPRs, AGPRs, scratch bytes per lane, SGPR / VGPR
spills, occupancy) for gemm.hip, attention.hip, rowops.hip and few.hip, and with
--fail-on-scratch exits 1 if any kernel spills or uses scratch."""
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-x", "hip", "-c", "-o", os.devnull, "-Rpass-analysis=kernel-resource-usage"]
KEYS = {"VGPRs": "vgpr", "AGPRs": "agpr", "ScratchSize [bytes/lane]": "scratch", "SGPRs Spill": "sgpr_spill",
        "VGPRs Spill": "vgpr_spill", "Occupancy [waves/SIMD]": "occupancy"}


def kernels(src):
    out = subprocess.run([HIPCC] + FLAGS + [os.path.join(HERE, src)], capture_output=True, text=True).stderr
    rows, cur = [], None
    for line in out.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = {"name": m.group(1)}
            rows.append(cur)
            continue
        for k, short in KEYS.items():
            m = re.search(r"remark:\s+" + re.escape(k) + r": (\d+)", line)
            if m and cur is not None:
                cur[short] = int(m.group(1))
    return rows


def demangle(names):
    r = subprocess.run(["c++filt"], input="\n".join(names), capture_output=True, text=True)
    return r.stdout.splitlines() if r.returncode == 0 else names


def main():
    bad = 0
    for src in ("gemm.hip", "attention.hip", "rowops.hip", "few.hip"):
        rows = kernels(src)
        names = demangle([r["name"] for r in rows])
        print(f"{src}: {len(rows)} kernels")
        for r, n in zip(rows, names):
            spill = r.get("scratch", 0) or r.get("sgpr_spill", 0) or r.get("vgpr_spill", 0)
            bad += bool(spill)
            print(f"  vgpr {r.get('vgpr', 0):3d} agpr {r.get('agpr', 0):3d} scratch {r.get('scratch', 0):3d} "
                  f"spill s/v {r.get('sgpr_spill', 0)}/{r.get('vgpr_spill', 0)} occ {r.get('occupancy', 0)}  "
                  f"{n.replace('ebh::', '')[:110]}")
    print(f"kernels with spills or scratch: {bad}")
    return 1 if bad and "--fail-on-scratch" in sys.argv else 0


if __name__ == "__main__":
    sys.exit(main())
