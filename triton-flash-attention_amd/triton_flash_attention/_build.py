"""Build recipe for libfa_gfx950.so (the HIP kernels and their C ABI).

The library is compiled in-tree with ``hipcc --offload-arch=gfx950`` so that
the shared object travels with the source tree. No JIT cache is involved.

    python -m triton_flash_attention._build        # (re)build the library
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
LIB_NAME = "libfa_gfx950.so"
LIB_PATH = PACKAGE_DIR / LIB_NAME

SOURCES = ("fa_fwd.hip", "fa_bwd.hip", "fa_capi.hip")
HEADERS = ("fa_common.hpp", "fa_kernels.hpp")

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in generated code.
# -amdgpu-mfma-vgpr-form: MFMA accumulators live in ordinary VGPRs, so the
#   per-row rescales of the accumulators need no AGPR<->VGPR copies.
HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
)


def hipcc() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    raise RuntimeError("hipcc not found: install ROCm or set ROCM_PATH")


def build_command(output: Path = LIB_PATH, extra: tuple[str, ...] = ()) -> list[str]:
    return [
        hipcc(),
        *HIPCC_FLAGS,
        *extra,
        f"-I{INCLUDE_DIR}",
        "-o",
        str(output),
        *(str(CSRC_DIR / s) for s in SOURCES),
    ]


def build(output: Path = LIB_PATH, verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 into ``output`` (always recompiles)."""
    tmp = output.with_name(output.name + ".tmp")
    cmd = build_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        # hipcc's host pass warns that it does not know the packed-fp32 feature;
        # only real diagnostics are worth showing.
        lines = [
            ln
            for ln in (proc.stderr or "").splitlines()
            if "packed-fp32-ops" not in ln
        ]
        raise RuntimeError("hipcc failed:\n" + "\n".join(lines[-60:]))
    os.replace(tmp, output)
    return output


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    path = build(verbose="-v" in argv)
    print(f"built {path}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
