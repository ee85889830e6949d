"""Build recipe for libfa_gfx950.so (the HIP kernels and their C ABI).

The library is compiled in-tree with ``hipcc --offload-arch=gfx950`` so that
the shared object travels with the source tree. No JIT cache is involved.

    python -m triton_flash_attention._build        # (re)build the library and the binding

The C++ autograd binding (csrc/fa_native.cpp, ``_fa_native.so``) is host code
only; it is compiled with g++ against PyTorch's headers (``build_native``).
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

SOURCES = ("fa_fwd.hip", "fa_bwd.hip", "fa_bwd_pair.hip", "fa_capi.hip")
HEADERS = ("fa_common.hpp", "fa_kernels.hpp", "fa_bwd_pipe.hpp")

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


def object_commands(obj_dir: Path, extra: tuple[str, ...] = ()) -> list[tuple[Path, list[str]]]:
    """One ``hipcc -c`` per source (each object carries its own gfx950 code
    object), so the translation units compile in parallel."""
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    out = []
    for s in SOURCES:
        obj = obj_dir / (Path(s).stem + ".o")
        out.append((obj, [hipcc(), *flags, *extra, f"-I{INCLUDE_DIR}", "-c", "-o", str(obj),
                          str(CSRC_DIR / s)]))
    return out


def _check(proc: subprocess.CompletedProcess) -> None:
    if proc.returncode != 0:
        # hipcc's host pass warns that it does not know the packed-fp32 feature;
        # only real diagnostics are worth showing.
        lines = [
            ln
            for ln in (proc.stderr or "").splitlines()
            if "packed-fp32-ops" not in ln
        ]
        raise RuntimeError("hipcc failed:\n" + "\n".join(lines[-60:]))


def build(output: Path = LIB_PATH, verbose: bool = False) -> Path:
    """Compile every HIP source for gfx950 into ``output`` (always recompiles).
    The sources compile as separate objects in parallel and are then linked."""
    import tempfile

    tmp = output.with_name(output.name + ".tmp")
    with tempfile.TemporaryDirectory(prefix="fa_build_") as d:
        jobs = object_commands(Path(d))
        procs = []
        for _, cmd in jobs:
            if verbose:
                print(" ".join(cmd), flush=True)
            procs.append(subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                          text=True))
        for (_, cmd), p in zip(jobs, procs):
            out, err = p.communicate()
            _check(subprocess.CompletedProcess(cmd, p.returncode, out, err))
        link = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
                *(str(o) for o, _ in jobs)]
        if verbose:
            print(" ".join(link), flush=True)
        _check(subprocess.run(link, capture_output=True, text=True))
    os.replace(tmp, output)
    return output


NATIVE_SOURCE = "fa_native.cpp"
NATIVE_PATH = PACKAGE_DIR / "_fa_native.so"


def native_command(output: Path = NATIVE_PATH) -> list[str]:
    """g++ line of the C++ autograd binding (host code only: PyTorch's headers
    and libraries, ROCm's HIP headers for torch's stream API)."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    libdirs = cpp_extension.library_paths()
    return [
        os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *(f"-I{p}" for p in cpp_extension.include_paths()),
        f"-I{sysconfig.get_paths()['include']}", f"-I{rocm}/include",
        str(CSRC_DIR / NATIVE_SOURCE), "-o", str(output),
        *(f"-L{p}" for p in libdirs), *(f"-Wl,-rpath,{p}" for p in libdirs),
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-ltorch_python",
    ]


def build_native(output: Path = NATIVE_PATH, verbose: bool = False) -> Path:
    """Compile the C++ autograd binding into ``output`` (always recompiles)."""
    tmp = output.with_name(output.name + ".tmp")
    cmd = native_command(tmp)
    if verbose:
        print(" ".join(cmd), flush=True)
    _check(subprocess.run(cmd, capture_output=True, text=True))
    os.replace(tmp, output)
    return output


def main(argv: list[str] | None = None) -> int:
    from concurrent.futures import ThreadPoolExecutor

    argv = sys.argv[1:] if argv is None else argv
    with ThreadPoolExecutor(max_workers=1) as pool:
        native = pool.submit(build_native, verbose="-v" in argv)
        print(f"built {build(verbose='-v' in argv)}")
        print(f"built {native.result()}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
