"""Resource figures of the built library's gfx950 kernels, read from the
code objects' own AMDGPU metadata (no GPU needed): every kernel of the hot
path has zero scratch, zero VGPR/SGPR spills and fits the register and LDS
budgets of one CDNA4 CU."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "p40-kernel_amd"))

import kernel_resources as kr  # noqa: E402

pytestmark = pytest.mark.skipif(
    not (os.path.exists(kr.LIB) and os.path.exists(os.path.join(kr.LLVM, "llvm-objdump"))
         and os.path.exists(os.path.join(kr.LLVM, "llvm-readelf"))),
    reason="needs the built library and ROCm's llvm-objdump / llvm-readelf")


@pytest.fixture(scope="module")
def rows():
    r = kr.kernel_resources()
    assert r, "no gfx950 kernels found in the library"
    return r


def test_every_kernel_family_is_present(rows):
    fams = {kr.family(r) for r in rows}
    for f in ("gemv_nb_kernel", "gemv_stream_kernel", "gemm_wide_kernel", "gemm_f16_kernel", "gemm_bd_kernel",
              "gemm_small_kernel", "rot_quant_kernel", "rms_rot_quant_kernel", "swiglu_rot_quant_kernel",
              "quant_kernel", "repack_kernel", "chain_kernel"):
        assert f in fams, f


def _ffn_epilogue_instance(r):
    # gemv_nb_kernel<..., EPI = true>: the FFN gate/up launch with its glue
    return kr.family(r) == "gemv_nb_kernel" and r["name"].split(">(")[0].endswith("true")


def test_hot_path_kernels_use_no_scratch_and_do_not_spill(rows):
    hot = [r for r in rows if kr.is_hot_path(r)]
    assert len(hot) > 100
    bad = [(r["name"], r["scratch"], r["vgpr_spill"], r["dynamic_stack"]) for r in hot
           if r["scratch"] or r["vgpr_spill"] or r["dynamic_stack"]]
    assert not bad, bad
    # SGPR spills go to VGPR lanes (no memory); none on the hot path but the
    # FFN-epilogue instances, where at most a few are tolerated
    sgpr = [(r["name"], r["sgpr_spill"]) for r in hot
            if r["sgpr_spill"] and not (_ffn_epilogue_instance(r) and r["sgpr_spill"] <= 32)]
    assert not sgpr, sgpr


def test_no_kernel_uses_scratch_memory(rows):
    # the persistent chain kernel spills a few SGPRs into VGPR lanes, which is
    # not scratch memory; nothing in the library reads or writes scratch
    bad = [(r["name"], r["scratch"], r["vgpr_spill"]) for r in rows if r["scratch"] or r["vgpr_spill"]]
    assert not bad, bad


def test_kernels_fit_one_cu(rows):
    for r in rows:
        # 512 unified VGPR+AGPR per lane at one wave per SIMD, 160 KiB LDS per CU
        assert r["vgpr"] + r["agpr"] <= 512, r["name"]
        assert r["lds"] <= 160 * 1024, r["name"]
        assert r["max_wg"] <= 1024, r["name"]


def test_wide_prefill_kernel_keeps_two_waves_per_simd(rows):
    # 512 threads = 2 waves per SIMD; both tile shapes, with the activation
    # staged or DMA'd, must stay within 256 VGPRs so that the two waves fit,
    # and within the LDS budget of 1 block/CU
    wide = [r for r in rows if kr.family(r) == "gemm_wide_kernel"]
    assert len(wide) == 4
    for r in wide:
        assert r["max_wg"] == 512
        assert r["vgpr"] + r["agpr"] <= 256, (r["name"], r["vgpr"], r["agpr"])
