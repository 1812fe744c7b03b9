"""The build's scratch guard: hipcc's kernel-resource remarks are parsed per
kernel, and the decode kernels' name patterns select what must not use
scratch memory (CPU)."""

from __future__ import annotations

import re

from breeze_amd import build as B

_TAG = " [-Rpass-analysis=kernel-resource-usage]"


def _remarks(name: str, vgpr: int, scratch: int) -> str:
    lines = [
        f"Function Name: {name}",
        "    TotalSGPRs: 64",
        f"    VGPRs: {vgpr}",
        "    AGPRs: 0",
        f"    ScratchSize [bytes/lane]: {scratch}",
        "    Occupancy [waves/SIMD]: 4",
    ]
    return "".join(f"csrc/x.hip:12:1: remark: {l}{_TAG}\n" for l in lines)


def test_parse_remarks():
    text = (
        "csrc/x.hip:3:5: warning: something unrelated\n"
        + _remarks("_ZN2bz9gemv_mfmaILi0ELi4ELi1ELi4ELb0EEEvNS_10GemvParamsE", 73, 32)
        + _remarks("_ZN2bz15head_f32_kernelILi1ELi8EEEvPKfS2_iiPfi", 40, 0)
    )
    got = B.kernel_resources(text)
    assert got == [
        ("_ZN2bz9gemv_mfmaILi0ELi4ELi1ELi4ELb0EEEvNS_10GemvParamsE", 73, 32),
        ("_ZN2bz15head_f32_kernelILi1ELi8EEEvPKfS2_iiPfi", 40, 0),
    ]


def _checked(name: str) -> bool:
    return any(re.search(t, name) for t in B.NO_SCRATCH)


def test_patterns_cover_the_decode_kernels():
    for name in (
        "_ZN2bz12gemv_persistILi0ELi1ELi2ELi2ELb1EEEvNS_10GemvParamsE",
        "_ZN2bz9gemv_mfmaILi2ELi2ELi1ELi4ELb0EEEvNS_10GemvParamsE",
        "_ZN2bz10gemv_i8mmaILi0ELi4ELi1ELi4ELb0EEEvNS_10GemvParamsEi",
        "_ZN2bz9gemv_tileILi0ELi2ELi1ELi4EEEvNS_10TileParamsE",
        "_ZN2bz11attn_kernelILi4ELi4ELb0ELb1EEEvNS_10AttnParamsE",
        "_ZN2bz11attn_kernelILi1ELi16ELb0ELb0EEEvNS_10AttnParamsE",
    ):
        assert _checked(name), name
    # fp32 caches and D = 512 are allowed scratch
    for name in (
        "_ZN2bz11attn_kernelILi4ELi16ELb1ELb0EEEvNS_10AttnParamsE",
        "_ZN2bz11attn_kernelILi8ELi4ELb0ELb1EEEvNS_10AttnParamsE",
    ):
        assert not _checked(name), name
