"""Build libmiracle_hip.so (gfx950) from ../csrc with its Makefile."""
import subprocess
from pathlib import Path

CSRC = Path(__file__).resolve().parent.parent / "csrc"


def build(jobs=8):
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", str(CSRC)], check=True)
    return CSRC.parent / "miracle_hip" / "_lib" / "libmiracle_hip.so"


if __name__ == "__main__":
    print(build())
