"""The checks triton-mla_amd/build.py runs on every build, on planted inputs:
the resource-report parser and its scratch/LDS gate, and the scan for reads
of an inline-asm MFMA result before the MFMA has finished. (The real build
runs them on the shipped code; here each must catch what it is for.)"""

import os
import sys

import pytest

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "triton-mla_amd"))
import build  # noqa: E402

REMARKS = """\
remark: /x/mla_decode.hip:717:0: Function Name: _ZN4tmla18mla_partial_kernelILi0ELi512ELi64ELi1ELb1ELb1ELb0EEEvNS_11PartialArgsE [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     VGPRs: 256 [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     AGPRs: 130 [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     ScratchSize [bytes/lane]: 0 [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     Dynamic Stack: False [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     LDS Size [bytes/block]: 148544 [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0: Function Name: _ZN4tmla18mla_partial_kernelILi0ELi512ELi64ELi4ELb1ELb1ELb1EEEvNS_11PartialArgsE [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     ScratchSize [bytes/lane]: 12 [-Rpass-analysis=kernel-resource-usage]
remark: /x/mla_decode.hip:717:0:     LDS Size [bytes/block]: 160832 [-Rpass-analysis=kernel-resource-usage]
"""


def test_resource_report_parsed():
    usage = build.parse_resource_usage(REMARKS)
    assert len(usage) == 2
    k1 = next(k for k in usage if "ELi1ELb1ELb1ELb0E" in k)
    assert usage[k1] == {"VGPRs": 256, "AGPRs": 130, "ScratchSize": 0, "LDS Size": 148544}
    build.check_resources(usage)  # the fp8 ring's 12 bytes are within its allowance


@pytest.mark.parametrize("edit, why", [
    (("ScratchSize [bytes/lane]: 0", "ScratchSize [bytes/lane]: 4"), "scratch"),
    (("ScratchSize [bytes/lane]: 12", "ScratchSize [bytes/lane]: 16"), "scratch"),
    (("148544", "163844"), "LDS"),
])
def test_resource_gate_fails(edit, why):
    usage = build.parse_resource_usage(REMARKS.replace(*edit))
    with pytest.raises(RuntimeError, match=why):
        build.check_resources(usage)


def _asm(tmp_path, body):
    p = tmp_path / "k.s"
    p.write_text("_Zkernel:\n" + body)
    return str(p)


def test_mfma_hazard_scan(tmp_path):
    mfma = "\tv_mfma_f32_32x32x16_bf16 v[0:15], v[32:35], v[36:39], v[0:15]\n"
    filler = "".join(f"\tv_add_u32_e32 v{100 + i}, v{101 + i}, v{102 + i}\n" for i in range(17))
    early = "\tv_max_f32_e32 v40, v3, v40\n"
    # read one instruction after the MFMA: flagged
    assert len(build.mfma_result_hazards(_asm(tmp_path, mfma + early))) == 1
    # 17 independent instructions are still too few; 18 (or s_nop wait states) suffice
    assert len(build.mfma_result_hazards(_asm(tmp_path, mfma + filler + early))) == 1
    assert build.mfma_result_hazards(_asm(tmp_path, mfma + filler + "\ts_nop 0\n" + early)) == []
    assert build.mfma_result_hazards(_asm(tmp_path, mfma + "\ts_nop 7\n\ts_nop 7\n\ts_nop 1\n" + early)) == []
    # a register-allocator copy of the accumulator in flight: flagged
    assert len(build.mfma_result_hazards(_asm(tmp_path, mfma + "\tv_mov_b32_e32 v60, v7\n"))) == 1
    # back-to-back accumulation into the same registers: the hardware's case
    assert build.mfma_result_hazards(_asm(tmp_path, mfma + mfma)) == []
    # an MFMA that reads the in-flight result as an A/B operand: flagged
    bad_ab = "\tv_mfma_f32_32x32x16_bf16 v[16:31], v[0:3], v[36:39], v[16:31]\n"
    assert len(build.mfma_result_hazards(_asm(tmp_path, mfma + bad_ab))) == 1
    # MFMAs into AGPRs are the compiler's own (it inserts their waits)
    agpr = "\tv_mfma_f32_32x32x16_bf16 a[0:15], v[32:35], v[36:39], a[0:15]\n"
    assert build.mfma_result_hazards(_asm(tmp_path, agpr + "\tv_mov_b32_e32 v60, v7\n")) == []
