"""Build libqim.so (the HIP kernels + C ABI) for gfx950 with hipcc.

Each csrc/*.hip file is compiled to an object under _build/ in parallel, then
linked into qwen_image_accel/libqim.so, where the package's ctypes loader looks
for it.  Usage:  python qwen-image-2.1-accel_amd/build_native.py
"""
import concurrent.futures
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "qwen_image_accel", "libqim.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -ffp-contract=off: no implicit a*b+c fusion, so every rounding point of the
#   reference's eager ops is kept (the reference launches its Triton kernels
#   with enable_fp_fusion=False); fmaf is used where the reference has an FMA.
# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 generated from float code.
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
    "-fno-gpu-rdc", "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
]


# Per-source additions.  qim_attention.hip: MFMA accumulators in architectural
#   VGPRs (the "VGPR form"), operands in AGPRs, so the softmax reads the score
#   tiles and the lazy O rescale multiplies O in place; the accumulation-
#   register form copies every tile through v_accvgpr_read/write instead.
EXTRA = {
    "qim_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _compile(src):
    obj = os.path.join(BUILD, os.path.basename(src).replace(".hip", ".o"))
    cmd = [HIPCC, *COMMON, *EXTRA.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    msgs = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                     if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msgs}")
    return obj, msgs


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        results = list(ex.map(_compile, sources))
    for obj, msgs in results:
        if verbose and msgs.strip():
            print(msgs)
    tmp = OUT + ".tmp"
    # -Bsymbolic: the library's own references (kernel stubs, helpers) bind
    # inside it, never to a same-named symbol of another loaded library.
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-Bsymbolic", "-o", tmp,
           *[o for o, _ in results]]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
