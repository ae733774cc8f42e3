"""Build recipe of the C oracle (TEST INFRASTRUCTURE ONLY): gcc, no fast-math, into oracle/_build/.

The reference (Shivram08/small-inference) is pure Python and torch; it has no C/C++ sources, so there is no
oracle/_ref build of it: its algorithm is restated in quant_ref.c and paged_ref.py instead.
"""

import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
OUT = HERE / "_build" / "liboracle_quant.so"


def build(verbose: bool = False) -> Path:
    """Compile quant_ref.c into liboracle_quant.so; always recompiles."""
    OUT.parent.mkdir(exist_ok=True)
    cc = shutil.which("gcc") or "cc"
    cmd = [cc, "-O2", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-std=c11", "-Wall",
           str(HERE / "quant_ref.c"), "-o", str(OUT), "-lm"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
