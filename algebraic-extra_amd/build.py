"""Build libalgx.so (gfx950) in-tree with hipcc.

    python algebraic-extra_amd/build.py            # compile every csrc/*.hip, link
    python algebraic-extra_amd/build.py --asm      # also write gfx950 ISA to _build/

Each translation unit is compiled separately (in parallel) and linked into
``algebraic_amd/libalgx.so`` next to the Python package that loads it.
"""

import argparse
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "algebraic_amd", "libalgx.so")
ARCH = "gfx950"
# Extra flags per translation unit: the MFMA kernels keep their accumulators in
# architectural VGPRs so the VALU reads them without accvgpr copies.
EXTRA = {
    "attn_fwd_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "attn_bwd_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "head.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gemm_batched.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def flags():
    return [
        f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
        "-I", os.path.join(ROOT, "include"), "-I", CSRC,
        "-munsafe-fp-atomics",
        # Packed FP32 VALU forms stay disabled on this hardware pool.
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
    ]


def _compile(src, asm):
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    extra = EXTRA.get(os.path.basename(src), [])
    cmd = [hipcc()] + flags() + extra + ["-c", src, "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{res.stderr}")
    if asm:
        s = os.path.join(BUILD, os.path.basename(src) + ".s")
        subprocess.run([hipcc()] + flags() + extra + ["--cuda-device-only", "-S", src, "-o", s],
                       capture_output=True, text=True, check=True)
    return obj


def build(asm=False, jobs=None):
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    jobs = jobs or min(8, len(sources), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, asm), sources))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed\n{res.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--asm", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(asm=a.asm, jobs=a.j))
    sys.exit(0)
