"""Build the gfx950 HIP library ``lib/librdna2_qgemm.so`` with an existing hipcc.

Mirrors the reference's build helper (rdna2-ops/rdna2_ops/build.py:14-36):
same flag discipline (``-O3 -ffp-contract=off -Rpass-analysis=kernel-resource-usage``),
a JSON build record next to the library, and no dependency beyond hipcc.
Each translation unit is compiled in parallel, then linked into one shared
library. Kernel register/LDS usage reported by the compiler is parsed into
``lib/kernel_resources.json`` (returned as kernel metadata by the operators).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import hashlib
import json
import os
from pathlib import Path
import re
import shutil
import subprocess
import time

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
INCLUDE = PACKAGE.parent.parent / "include"
LIB_DIR = PACKAGE / "lib"
LIB_NAME = "librdna2_qgemm.so"
ARCH = "gfx950"

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
    # Packed-fp32 VALU forms are kept out of the generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Rpass-analysis=kernel-resource-usage",
]


def _hipcc(explicit=None):
    path = explicit or os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; pass --hipcc or set HIPCC")
    return path


def sources():
    return sorted(CSRC.glob("*.hip"))


_RES = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|TotalSGPRs|ScratchSize \[bytes/lane\]|"
                  r"Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]|VGPRs Spill|SGPRs Spill): (.*)")


def _parse_resources(text):
    kernels, current = {}, None
    for line in text.splitlines():
        m = _RES.search(line)
        if not m:
            continue
        key, value = m.group(1), m.group(2).split(" [-Rpass")[0].strip()
        if key == "Function Name":
            current = kernels.setdefault(value, {})
            continue
        if current is not None:
            try:
                current[key] = int(value)
            except ValueError:
                current[key] = value
    return kernels


def build(hipcc=None, jobs=None, verbose=False):
    hipcc = _hipcc(hipcc)
    LIB_DIR.mkdir(exist_ok=True)
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(exist_ok=True)
    srcs = sources()
    t0 = time.perf_counter()

    def compile_one(src):
        obj = obj_dir / (src.stem + ".o")
        cmd = [hipcc, *COMMON_FLAGS, f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
        run = subprocess.run(cmd, capture_output=True, text=True, timeout=900)
        return src, obj, cmd, run

    results = []
    with cf.ThreadPoolExecutor(max_workers=jobs or min(8, len(srcs))) as pool:
        for src, obj, cmd, run in pool.map(compile_one, srcs):
            results.append((src, obj, cmd, run))
    log = []
    resources = {}
    failed = False
    for src, obj, cmd, run in results:
        log.append(" ".join(cmd) + "\n" + run.stdout + run.stderr)
        resources.update(_parse_resources(run.stderr))
        if run.returncode:
            failed = True
            print(run.stderr[-8000:], flush=True)
    out = LIB_DIR / LIB_NAME
    link = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *[str(o) for _, o, _, _ in results],
            "-o", str(out) + ".tmp"]
    if not failed:
        run = subprocess.run(link, capture_output=True, text=True, timeout=600)
        log.append(" ".join(link) + "\n" + run.stdout + run.stderr)
        if run.returncode:
            failed = True
            print(run.stderr[-8000:], flush=True)
        else:
            os.replace(str(out) + ".tmp", out)
    (LIB_DIR / "build.log").write_text("\n".join(log))
    version = subprocess.run([hipcc, "--version"], capture_output=True, text=True).stdout
    record = {
        "compile_flags": COMMON_FLAGS, "target": ARCH, "compiler_version": version,
        "sources": {s.name: hashlib.sha256(s.read_bytes()).hexdigest() for s in srcs},
        "internal_headers": {h.name: hashlib.sha256(h.read_bytes()).hexdigest() for h in sorted(CSRC.glob("*.h"))},
        "header_sha256": hashlib.sha256((INCLUDE / "qgemm.h").read_bytes()).hexdigest(),
        "seconds": time.perf_counter() - t0, "returncode": int(failed),
    }
    if not failed:
        record["library_sha256"] = hashlib.sha256(out.read_bytes()).hexdigest()
        (LIB_DIR / "kernel_resources.json").write_text(json.dumps(resources, indent=1, sort_keys=True) + "\n")
    (LIB_DIR / "build.json").write_text(json.dumps(record, indent=2) + "\n")
    if verbose:
        print(json.dumps({k: v for k, v in record.items() if k != "compiler_version"}), flush=True)
    if failed:
        raise RuntimeError("HIP build failed; see " + str(LIB_DIR / "build.log"))
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--hipcc", default=None)
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    build(args.hipcc, args.jobs, verbose=True)


if __name__ == "__main__":
    main()
