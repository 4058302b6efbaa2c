"""CPU check of the flash attention kernel's register budget (attention.hip,
attn_flash_kernel).

Four 32-query workgroups of four waves share a CU: 32 KB of LDS each and at
most 128 VGPRs per wave (four waves per SIMD out of 512 registers).  At 129
or more the hardware fits only three waves per SIMD, and the kernel loses
6-7% at 512 tokens.  This test compiles attention.hip to assembly and checks
every 4-wave instantiation's register count and that nothing spills.
"""
import pathlib
import re
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "longbow-fletcher_amd" / "csrc"


def test_flash_kernel_fits_four_waves_per_simd(tmp_path):
    import longbow_fletcher_amd.build as B
    if not shutil.which(B.HIPCC) and not pathlib.Path(B.HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path / "attention.s"
    cmd = [B.HIPCC, *B.COMMON, f"-I{CSRC}", *B.PER_FILE.get("attention.hip", []),
           "--cuda-device-only", "-S", "-o", str(out), str(CSRC / "attention.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    asm = out.read_text()
    found = 0
    for m in re.finditer(r"\.amdhsa_kernel (_ZN2fl17attn_flash_kernel\S*)(.*?)\.end_amdhsa_kernel",
                         asm, re.S):
        name, meta = m.group(1), m.group(2)
        assert re.search(r"\.amdhsa_private_segment_fixed_size 0\b", meta), f"{name} spills"
        if "ELi4ELb" not in name:  # the 2-wave variant serves sequences of <= 64 tokens
            continue
        found += 1
        vgprs = int(re.search(r"\.amdhsa_next_free_vgpr (\d+)", meta).group(1))
        assert vgprs <= 128, f"{name}: {vgprs} VGPRs, more than four waves per SIMD allow"
    assert found >= 6  # head size 64 (pre-scaled or not) and 32, fp16 and bf16
