"""Build the gfx950 library libq4llm.so (and the native runner) in-tree with hipcc.

    python iree-adreno-genai-tuner_amd/build.py [--jobs N]

Every HIP/C++ source under csrc/ is compiled for gfx950 only, with packed-fp32 instructions
disabled (-packed-fp32-ops), into lib/. The output stays in the source tree so it ships with the
tree to the machine that runs it; nothing is installed.
"""

import argparse
import concurrent.futures as cf
import os
import pathlib
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas", "-Wno-unused-command-line-argument",
    f"-I{ROOT / 'include'}", f"-I{CSRC}",
]

LIB_SOURCES = [
    "q4_status.cpp", "q4_format.hip", "q4_gemv.hip", "q4_gemv_mx.hip", "gemm_f16.hip", "q4_linear.hip",
    "attn_bucket.hip", "llama_ops.hip", "q4llm_step.cpp", "roofline_probe.hip", "q4_t16.hip",
]


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    lang = [] if src.suffix == ".hip" else ["-x", "hip"]
    cmd = [HIPCC, *COMMON, *lang, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def build(jobs: int = 8, verbose: bool = True) -> pathlib.Path:
    """Compile every source and link lib/libq4llm.so; returns the library path."""
    LIB.mkdir(exist_ok=True)
    objdir = LIB / "obj"
    objdir.mkdir(exist_ok=True)
    srcs = [CSRC / s for s in LIB_SOURCES if (CSRC / s).exists()]
    objs = [objdir / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, srcs, objs))
    out = LIB / "libq4llm.so"
    tmp = LIB / "libq4llm.so.tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, out)
    runner_src = CSRC / "llm_runner.cpp"
    if runner_src.exists():
        exe = LIB / "llm-runner"
        cmd = [HIPCC, *COMMON, "-x", "hip", str(runner_src), "-o", str(exe), f"-L{LIB}", "-lq4llm",
               "-Wl,-rpath,$ORIGIN"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"runner build failed:\n{r.stderr}")
    if verbose:
        print(f"built {out} ({len(srcs)} sources)")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=min(8, os.cpu_count() or 1))
    a = ap.parse_args()
    build(a.jobs)
    return 0


if __name__ == "__main__":
    sys.exit(main())
