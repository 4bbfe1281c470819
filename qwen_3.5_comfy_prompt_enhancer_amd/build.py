"""Build libqlin.so (gfx950) in-tree with hipcc.

    python qwen_3.5_comfy_prompt_enhancer_amd/build.py [--jobs N]

Objects go to `_build/` at the repository root, the library to
`qwen_3.5_comfy_prompt_enhancer_amd/kernels/libqlin.so`, where the Python package
loads it.  Every HIP source is compiled with packed fp32 instructions disabled
(`-Xclang -target-feature -Xclang -packed-fp32-ops`).
"""
from __future__ import annotations

import argparse
import os
import pathlib
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = pathlib.Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "kernels" / "libqlin.so"
BUILD = ROOT / "_build"
ARCH = os.environ.get("QLIN_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


# Per-source flags.  The A16 prefill kernel (prefill_kernel.h, instantiated by
# prefill.hip and prefill_w4_*.hip) keeps its 128 fp32 accumulators per lane in
# architectural VGPRs (the VGPR form of MFMA): with accumulation registers the
# compiler rotates the loop-carried accumulators through copies every K tile.
_VGPR_FORM = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
EXTRA = {
    "prefill.hip": _VGPR_FORM,
    "prefill_w4_f16.hip": _VGPR_FORM,
    "prefill_w4_bf16.hip": _VGPR_FORM,
    "prefill_w4_f32.hip": _VGPR_FORM,
}


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def compile_one(src: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [HIPCC, *CFLAGS, *EXTRA.get(src.name, []), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(jobs: int | None = None) -> pathlib.Path:
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 1, 8)
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(compile_one, srcs))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    args = ap.parse_args()
    out = build(args.jobs)
    print(out)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
