"""The driver-free gfx950 compile check (CPU only: hipcc cross-compiles).

Counterpart of the reference's AOT compile check (scripts/aot_compile_check.py:81-156).
"""

from __future__ import annotations

import pytest

from triton_flash_attention import _lib, compile_check

REMARKS = """\
fa_fwd.hip:61:1: remark: Function Name: _ZN2fa15fwd_pipe_kernelILi64ELb1ELi4ELi1ENS_3F16EEEvNS_7FwdArgsE [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     TotalSGPRs: 64 [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     VGPRs: 168 [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     Occupancy [waves/SIMD]: 3 [-Rpass-analysis=kernel-resource-usage]
fa_fwd.hip:61:1: remark:     LDS Size [bytes/block]: 49152 [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark: Function Name: _ZN2fa17preprocess_kernelILi32ENS_3F16EEEvPKDF16_S3_Pfl [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark:     VGPRs: 16 [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark:     AGPRs: 0 [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark:     Occupancy [waves/SIMD]: 8 [-Rpass-analysis=kernel-resource-usage]
fa_bwd.hip:37:1: remark:     LDS Size [bytes/block]: 0 [-Rpass-analysis=kernel-resource-usage]
"""


def test_resource_report_parsing():
    ks = compile_check.parse_resource_usage(REMARKS)
    # c++filt demangles the first; the second (fp16 pointer arguments) may stay
    # mangled there and is named by the fallback decoder instead.
    assert [k.name.split("(")[0] for k in ks] == ["fa::fwd_pipe_kernel<64, true, 4, 1, fa::F16>",
                                                  "fa::preprocess_kernel<32, fa::F16>"]
    fwd, pre = ks
    assert (fwd.vgprs, fwd.agprs, fwd.scratch, fwd.occupancy, fwd.lds) == (168, 0, 0, 3, 49152)
    assert (pre.vgprs, pre.scratch, pre.occupancy) == (16, 12, 8)
    spills, missing = compile_check.spilling_defaults(ks)
    assert [k.name.split("(")[0] for k in spills] == ["fa::preprocess_kernel<32, fa::F16>"]
    assert "fa::dkdv_pipe_kernel<64, true, 4, fa::BF16>" in missing


def test_spill_allowance_is_per_kernel_and_capped():
    """A default kernel listed in ALLOWED_SPILLS may spill up to its measured
    bytes per lane and no more; every other default kernel may not spill."""
    name, cap = next(iter(compile_check.ALLOWED_SPILLS.items()))
    assert name in compile_check.DEFAULT_KERNELS
    other = "fa::dq_kernel<128, false, 4, 32, fa::F16>"
    assert other in compile_check.DEFAULT_KERNELS and other not in compile_check.ALLOWED_SPILLS

    def spills(scratch_of):
        ks = [compile_check.KernelUsage(name=f"{n}(fa::BwdArgs)", scratch=scratch_of.get(n, 0))
              for n in compile_check.DEFAULT_KERNELS]
        return [k.name.split("(")[0] for k in compile_check.spilling_defaults(ks)[0]]

    assert spills({name: cap}) == []
    assert spills({name: cap + 4}) == [name]
    assert spills({other: 4}) == [other]


def test_fallback_names_for_undemangled_kernels():
    assert compile_check._short_name("_ZN2fa17preprocess_kernelILi128ENS_4BF16EEEvPKDF16_S3_Pfl") == \
        "fa::preprocess_kernel<128, fa::BF16>(...)"
    assert compile_check._short_name("_ZN2fa14dq_pipe_kernelILi32ELb0ELi4EEEvNS_7BwdArgsE") == \
        "fa::dq_pipe_kernel<32, false, 4>(...)"
    assert compile_check._short_name("_ZN2fa19split_reduce_kernelEPKfPDF16_S2_li") == \
        "fa::split_reduce_kernel(...)"


def test_default_kernel_list_follows_the_tiling_table():
    ok, why = _lib.available()
    assert ok, why
    for (kind, D, causal), variant in compile_check.DEFAULT_VARIANTS.items():
        assert _lib.get_tiling(kind, D, causal)["variant"] == variant, (kind, D, causal)
    assert len(compile_check.DEFAULT_VARIANTS) == 3 * 3 * 2


def test_unsupported_arch_is_rejected():
    with pytest.raises(ValueError, match="unsupported arch"):
        compile_check.compile_library("gfx942")


def test_library_compiles_for_gfx950_without_spills_in_the_defaults(capsys):
    assert compile_check.main(["--strict"]) == 0
    assert "compile check passed for gfx950" in capsys.readouterr().out
