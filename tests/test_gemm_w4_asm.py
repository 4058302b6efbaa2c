"""CPU checks of the four-wave GEMM's register discipline (gemm.hip,
gemm_w4_kernel).

Its K steps are asm blocks that keep fragments in v128-v255 and accumulators
in a0-a255 across statements; the compiler is only told that each block
clobbers them.  The kernel is correct only while the compiler's own code
between the blocks stays out of those registers and away from m0 (which the
blocks set for their DMA loads), and spills nothing.  These tests rebuild
the generated asm include and compile gemm.hip to assembly to check both.
"""
import pathlib
import re
import shutil
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "longbow-fletcher_amd" / "csrc"


def test_generated_include_is_current():
    sys.path.insert(0, str(CSRC))
    try:
        import gen_gemm_w4
    finally:
        sys.path.pop(0)
    assert (CSRC / "gemm_w4.inc").read_text() == gen_gemm_w4.generate()


def _kernels(asm: str, name: str = "gemm_w4_kernel"):
    pat = r"^(_ZN2fl%d%s\S*):.*?$(.*?)^\.Lfunc_end" % (len(name), name)
    for m in re.finditer(pat, asm, re.M | re.S):
        meta = re.search(r"\.amdhsa_kernel " + re.escape(m.group(1)) + r"(.*?)\.end_amdhsa_kernel",
                         asm, re.S).group(1)
        yield m.group(1), m.group(2), meta


def _compiler_lines(body: str):
    inside = False
    for ln in body.splitlines():
        if ";;#ASMSTART" in ln:
            inside = True
        elif ";;#ASMEND" in ln:
            inside = False
        elif not inside:
            code = ln.split(";")[0].strip()
            if code and not code.startswith(".") and not code.endswith(":"):
                yield code


@pytest.fixture(scope="module")
def gemm_asm(tmp_path_factory):
    import longbow_fletcher_amd.build as B
    if not shutil.which(B.HIPCC) and not pathlib.Path(B.HIPCC).exists():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm") / "gemm.s"
    cmd = [B.HIPCC, *B.COMMON, f"-I{CSRC}", *B.PER_FILE.get("gemm.hip", []), "--cuda-device-only",
           "-S", "-o", str(out), str(CSRC / "gemm.hip")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    return out.read_text()


def test_w4_kernel_register_discipline(gemm_asm):
    asm = gemm_asm
    found = 0
    for name, body, meta in _kernels(asm):
        found += 1
        assert re.search(r"\.amdhsa_private_segment_fixed_size 0\b", meta), f"{name} spills"
        assert re.search(r"\.amdhsa_accum_offset 256\b", meta), name
        mfmas = len(re.findall(r"v_mfma_f32_16x16x32_(?:f16|bf16)", body))
        assert mfmas >= 512, name
        if "_Li0ELi1E" in name:
            # STORE also has the half-tile steps (12 blocks of 32 MFMAs).
            assert mfmas >= 512 + 384, (name, mfmas)
        bad = []
        for code in _compiler_lines(body):
            if re.search(r"\bm0\b", code) or "scratch_" in code:
                bad.append(code)
                continue
            for kind, lo, hi in re.findall(r"\b([va])\[?(\d+)(?::(\d+))?\]?", code):
                if kind == "a" or int(hi or lo) >= 128:
                    bad.append(code)
                    break
        assert not bad, f"{name}: compiler code touches reserved registers: {bad[:5]}"
    assert found >= 6  # STORE, RoPE, SwiGLU x f16, bf16
