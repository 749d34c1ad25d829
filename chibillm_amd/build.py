"""Build recipe: every native artefact is compiled in-tree with make.

  chibillm_amd/libckv.so        HIP kernels + C ABI (hipcc --offload-arch=gfx950)
  chibillm_amd/libchibillm_host.so, host tests   C++ host layer over the ABI
  oracle/liboracle.so           CPU oracle (test infrastructure only)
  measure/libckv_probes.so      hardware-ceiling probes of bench.py (measurement only)
"""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TARGETS = [
    os.path.join(ROOT, "chibillm_amd", "csrc"),
    os.path.join(ROOT, "chibillm_amd", "host"),
    os.path.join(ROOT, "oracle"),
    os.path.join(ROOT, "measure"),
]


def build(jobs: int = 8) -> None:
    """Recompile everything (make -B), failing loudly on any error."""
    for directory in TARGETS:
        if not os.path.exists(os.path.join(directory, "Makefile")):
            continue
        subprocess.run(["make", "-B", f"-j{jobs}", "-C", directory], check=True)


if __name__ == "__main__":
    build()
