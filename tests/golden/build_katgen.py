"""Build tests/golden/libkatgen.so (test-only data replayer, see katgen.cpp)."""
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def build(verbose=False):
    src = HERE / "katgen.cpp"
    out = HERE / "libkatgen.so"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", str(src), "-o", str(out)]
    if verbose:
        print(" ".join(cmd))
    subprocess.run(cmd, check=True)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
