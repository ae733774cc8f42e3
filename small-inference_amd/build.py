"""Build recipe of libsmallinf_hip.so: hipcc for gfx950, in-tree, no torch extension machinery.

    python small-inference_amd/build.py        # or __graft_entry__.build()

The library is written next to the Python package (small-inference_amd/build/libsmallinf_hip.so) so that it
travels with the source tree to the GPU machine; engine/_hip.py loads it from there.
"""

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "build"
LIB = OUT_DIR / "libsmallinf_hip.so"
SOURCES = ["capi.hip", "decode.hip", "decode_int8.hip", "decode_valu_stream.hip", "metadata.hip", "prefill.hip",
           "quant_store.hip"]
PROBE_LIB = OUT_DIR / "libsmallinf_probe.so"  # measurement kernels for bench.py, outside the product ABI
PROBE_SOURCES = ["probe.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting packed fp32 VALU ops (v_pk_fma_f32 and kin); the kernels are written
# with scalar fp32 arithmetic only.
# Code object v5: loadable by torch's bundled HIP runtime (ROCm 7.0), which is the one in the process, since
# torch's libamdhip64 is loaded first and shares the SONAME libamdhip64.so.7 with ROCm's.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}", "-mcode-object-version=5",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         # MFMA accumulators in VGPRs: the default AGPR form makes the compiler copy every accumulator between
         # AGPRs and VGPRs around the softmax rescale of each key tile.
         "-mllvm", "-amdgpu-mfma-vgpr-form",
         # Leading scalar kernel arguments are preloaded into SGPRs at wave launch (the bf16 decode kernel passes
         # the fields of its first memory round trip that way); kernels whose leading argument is a struct are
         # unaffected.
         "-mllvm", "-amdgpu-kernarg-preload-count=16",
         "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas"]


def hipcc() -> str:
    """Path of hipcc (ROCm's, if not on PATH)."""
    return shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def _compile(sources: list[str], out: Path, verbose: bool) -> Path:
    tmp = out.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, "-I", str(ROOT / "include"), *[str(CSRC / s) for s in sources], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{proc.stdout}\n{proc.stderr}")
    # The host pass does not know the packed-fp32 feature flag and says so once per file; nothing else to show.
    notes = [ln for ln in proc.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if verbose and notes:
        print("\n".join(notes), file=sys.stderr)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile the decode-path library (and the bench's probe library); returns the main library's path.
    Always recompiles."""
    OUT_DIR.mkdir(exist_ok=True)
    _compile(PROBE_SOURCES, PROBE_LIB, verbose)
    return _compile(SOURCES, LIB, verbose)


if __name__ == "__main__":
    print(build(verbose=True))
