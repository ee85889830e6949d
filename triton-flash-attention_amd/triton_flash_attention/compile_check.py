"""Driver-free compile check of the gfx950 kernel library.

The MI355X counterpart of the reference's ``scripts/aot_compile_check.py``
(which AOT-compiles its forward, preprocess and backward kernels for an NVIDIA
target without a GPU, lines 81-156): this compiles every HIP source of the
library for ``--offload-arch=gfx950`` with the production flags into a
temporary file, no GPU or driver needed, and reads the compiler's per-kernel
resource report (VGPRs, AGPRs, scratch, occupancy, LDS). With ``--strict`` it
also fails when a kernel the default tiling table selects spills registers to
scratch memory: a spill reload inside a pipelined loop is a vector-memory load,
and waiting for it drains the kernel's DMA ring.

    python -m triton_flash_attention.compile_check [--arch gfx950] [--report] [--strict]
"""

from __future__ import annotations

import argparse
import re
import shutil
import subprocess
import sys
import tempfile
from dataclasses import dataclass
from pathlib import Path

from . import _build

SUPPORTED_ARCHS = ("gfx950",)

# Kernel instances the default tiling table (kDefault in csrc/fa_capi.hip) and
# its shape rules select, as demangled name prefixes, for D = 32, 64, 128, both
# mask modes and both element types (at D = 128 the forward takes the 8-wave
# pipelined kernel, and the 4-wave one for short queries; at D = 32 causal
# launches over few heads take the two-key-group forward, and the other causal
# launches from 512 queries its 16x16x32 form; small causal launches at D <= 64,
# and decoding at every head size, the 16x16x32 form with 64-query work-groups;
# at D <= 64 a backward
# whose dK/dV launch splits next to a short dQ launch runs the combined dK/dV + dQ
# kernel; dQ takes the pipelined kernel at D = 128 for short causal launches, and
# dQ and dK/dV their 16x16x32 forms at D = 64 and, without the mask, D = 32;
# short-query launches at D = 128 without the mask run the classic 4 x 32 dQ
# and dK/dV).
def _defaults() -> tuple[str, ...]:
    names = []
    for e in ("fa::F16", "fa::BF16"):
        for c in ("false", "true"):
            names += [f"fa::fwd_pipe_kernel<32, {c}, 4, 1, {e}, 1>",
                      f"fa::fwd_pipe_kernel<64, {c}, 4, 1, {e}, 1>",
                      f"fa::fwd_pipe_kernel<128, {c}, 8, 1, {e}, 1>", f"fa::fwd_kernel<128, {c}, 4, 32, {e}>",
                      f"fa::dkdv_pipe_kernel<32, {c}, 4, {e}>", f"fa::dkdv_pipe_kernel<64, {c}, 4, {e}>",
                      f"fa::dkdv_pipe_kernel<128, {c}, 4, {e}>", f"fa::dkdv_pipe16_kernel<64, {c}, 4, {e}>",
                      f"fa::dkdv_pipe16_kernel<32, false, 4, {e}>",
                      f"fa::dq_kernel<128, true, 4, 32, {e}>" if c == "true"
                      else f"fa::dq_pipe_kernel<128, false, 4, {e}, false>"]
            # dQ with and without the key-tail test (dq_tail_free)
            for t in ("false", "true"):
                names += [f"fa::dq_pipe_kernel<32, {c}, 4, {e}, {t}>",
                          f"fa::dq_pipe_kernel<64, {c}, 4, {e}, {t}>",
                          f"fa::bwd_pair_kernel<32, {c}, 4, {e}, {t}>",
                          f"fa::bwd_pair_kernel<64, {c}, 4, {e}, {t}>"]
            if c == "false":
                names.append(f"fa::dq_pipe_kernel<128, false, 4, {e}, true>")
                names += [f"fa::dq_pipe16_kernel<{d}, false, 4, {e}, {t}>"
                          for d in (32, 64) for t in ("false", "true")]
            else:
                names += [f"fa::dq_pipe_kernel<128, true, 4, {e}, {t}>" for t in ("false", "true")]
                names += [f"fa::dq_pipe16_kernel<64, true, 4, {e}, {t}>" for t in ("false", "true")]
        names.append(f"fa::fwd_pipe_kernel<32, true, 8, 1, {e}, 2>")
        names.append(f"fa::fwd_pipe16_kernel<32, true, {e}, 2>")
        names += [f"fa::fwd_pipe16_kernel<{d}, {c}, {e}, 1>"
                  for d in (32, 64, 128) for c in ("false", "true")]
        names += [f"fa::preprocess_kernel<{d}, {e}>" for d in (32, 64, 128)]
        names.append(f"fa::split_reduce_kernel<{e}>")
    names += [f"fa::{k}_kernel<128, false, 4, 32, {e}>" for k in ("dq", "dkdv")
              for e in ("fa::F16", "fa::BF16")]
    return tuple(names)


DEFAULT_KERNELS = _defaults()
# Default kernels allowed a measured spill (bytes per lane, at most): the
# short-query dK/dV at D = 128 asks for two waves per SIMD (256 registers) and
# reloads two 16-byte values per 32-query unit; with them it is 13-15 % faster
# than the pipelined kernel at one wave per SIMD for 4-64 queries (select_dkdv,
# csrc/fa_capi.hip). Any other spill, or a larger one, fails --strict.
ALLOWED_SPILLS = {f"fa::dkdv_kernel<128, false, 4, 32, {e}>": 52 for e in ("fa::F16", "fa::BF16")}
# The same table as (kernel kind, head_dim, causal) -> default variant index,
# for the test that keeps this list in step with kDefault (kinds: 0 fwd,
# 1 dK/dV, 2 dQ).
DEFAULT_VARIANTS = {
    (0, 32, False): 6, (0, 32, True): 6, (0, 64, False): 6, (0, 64, True): 6,
    (0, 128, False): 7, (0, 128, True): 7,
    (1, 32, False): 4, (1, 32, True): 4, (1, 64, False): 4, (1, 64, True): 4,
    (1, 128, False): 4, (1, 128, True): 4,
    (2, 32, False): 4, (2, 32, True): 4, (2, 64, False): 4, (2, 64, True): 4,
    (2, 128, False): 4, (2, 128, True): 1,
}


@dataclass
class KernelUsage:
    name: str
    vgprs: int = -1
    agprs: int = -1
    scratch: int = -1
    occupancy: int = -1
    lds: int = -1


_FIELDS = (
    ("vgprs", re.compile(r"remark:\s+VGPRs: (\d+)")),
    ("agprs", re.compile(r"remark:\s+AGPRs: (\d+)")),
    ("scratch", re.compile(r"remark:\s+ScratchSize \[bytes/lane\]: (\d+)")),
    ("occupancy", re.compile(r"remark:\s+Occupancy \[waves/SIMD\]: (\d+)")),
    ("lds", re.compile(r"remark:\s+LDS Size \[bytes/block\]: (\d+)")),
)
_NAME = re.compile(r"remark: Function Name: (\S+)")


_MANGLED = re.compile(r"^_ZN2fa(\d+)")
_TARG = re.compile(r"L([ib])(\d+)E|NS_\d+(F16|BF16)E")


def _short_name(mangled: str) -> str:
    """``fa::name<args>`` of this library's kernels (integer / bool template
    arguments only), for names a demangler leaves as they are."""
    m = _MANGLED.match(mangled)
    if m is None:
        return mangled
    n = int(m.group(1))
    start = m.end()
    name = mangled[start:start + n]
    rest = mangled[start + n:]
    args = []
    if rest.startswith("I"):
        body = rest[1:rest.index("EE") + 1] if "EE" in rest else ""
        for kind, val, elem in _TARG.findall(body):
            if elem:
                args.append("fa::" + elem)
            else:
                args.append(("true" if val == "1" else "false") if kind == "b" else val)
    return f"fa::{name}<{', '.join(args)}>(...)" if args else f"fa::{name}(...)"


def _demangle(names: list[str]) -> list[str]:
    tool = shutil.which("c++filt") or shutil.which("llvm-cxxfilt")
    out_names = names
    if tool is not None and names:
        out = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True)
        lines = out.stdout.splitlines()
        if out.returncode == 0 and len(lines) == len(names):
            out_names = lines
    return [_short_name(n) if n.startswith("_Z") else n for n in out_names]


def parse_resource_usage(text: str) -> list[KernelUsage]:
    """Kernel records from hipcc's ``-Rpass-analysis=kernel-resource-usage`` remarks."""
    kernels: list[KernelUsage] = []
    for line in text.splitlines():
        m = _NAME.search(line)
        if m:
            kernels.append(KernelUsage(m.group(1)))
            continue
        if not kernels:
            continue
        for field, pattern in _FIELDS:
            m = pattern.search(line)
            if m:
                setattr(kernels[-1], field, int(m.group(1)))
                break
    for k, name in zip(kernels, _demangle([k.name for k in kernels])):
        k.name = name.removeprefix("void ")
    return kernels


def compile_library(arch: str = "gfx950") -> tuple[list[KernelUsage], str]:
    """Compile the library into a temporary file; returns (kernels, diagnostics)."""
    if arch not in SUPPORTED_ARCHS:
        raise ValueError(f"unsupported arch {arch!r}: the kernels are written for {SUPPORTED_ARCHS}")
    with tempfile.TemporaryDirectory() as tmp:
        jobs = _build.object_commands(Path(tmp),
                                      extra=("-Rpass-analysis=kernel-resource-usage",))
        procs = [subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
                 for _, cmd in jobs]
        results = [(p.returncode, err) for p in procs for _, err in [p.communicate()]]
    stderr = "\n".join(err or "" for _, err in results)
    diag = "\n".join(ln for ln in stderr.splitlines()
                     if "packed-fp32-ops" not in ln and "remark:" not in ln)
    if any(rc != 0 for rc, _ in results):
        raise RuntimeError("hipcc failed:\n" + diag[-6000:])
    return parse_resource_usage(stderr), diag


def spilling_defaults(kernels: list[KernelUsage]) -> tuple[list[KernelUsage], list[str]]:
    """(default kernels that use scratch beyond ALLOWED_SPILLS, default kernels
    missing from the report)."""
    spills, missing = [], []
    for prefix in DEFAULT_KERNELS:
        found = [k for k in kernels if k.name.startswith(prefix + "(")]
        if not found:
            missing.append(prefix)
        spills += [k for k in found if k.scratch > ALLOWED_SPILLS.get(prefix, 0)]
    return spills, missing


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description="Driver-free gfx950 compile check")
    parser.add_argument("--arch", default="gfx950", help="offload target (only gfx950)")
    parser.add_argument("--report", action="store_true", help="print every kernel's resource usage")
    parser.add_argument("--strict", action="store_true",
                        help="fail if a default-tiling kernel spills to scratch")
    args = parser.parse_args(argv)
    try:
        kernels, _ = compile_library(args.arch)
    except (ValueError, RuntimeError) as e:
        print(f"compile check FAILED: {e}", file=sys.stderr)
        return 1
    if args.report:
        print(f"{'kernel':58s} {'VGPR':>5s} {'AGPR':>5s} {'scratch':>7s} {'waves/SIMD':>10s} {'LDS':>7s}")
        for k in kernels:
            print(f"{k.name[:58]:58s} {k.vgprs:5d} {k.agprs:5d} {k.scratch:7d} {k.occupancy:10d} {k.lds:7d}")
    spills, missing = spilling_defaults(kernels)
    if args.strict and (spills or missing):
        for k in spills:
            print(f"default kernel spills {k.scratch} bytes/lane to scratch: {k.name}", file=sys.stderr)
        for name in missing:
            print(f"default kernel not in the compiler report: {name}", file=sys.stderr)
        return 1
    print(f"compile check passed for {args.arch}: {len(kernels)} kernels (forward, preprocess, "
          f"dK/dV, dQ, split reduce; causal/bidirectional; D 32/64/128; MHA/GQA)"
          + ("; no scratch in the default tilings beyond the measured allowance"
             if args.strict else ""))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
