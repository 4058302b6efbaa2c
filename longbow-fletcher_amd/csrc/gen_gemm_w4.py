"""Writes gemm_w4.inc: the register-level K step of gemm_w4_kernel (gemm.hip).

The four-wave GEMM keeps its operands in fixed registers so that one K step
can be issued as a single asm block in a fixed order:

  a[4k .. 4k+3]            accumulator tile k = 8f + t (feature block f,
                           token block t) of the wave's 128x128 output block
  v[128 + 64P + 4t ..]     token fragment t of register set P (0 or 1)
  v[128 + 64P + 32 + 4f ..] feature fragment f of register set P

A step on set P starts with the DMA wait, the fragment wait and the
workgroup barrier, then issues its 64 MFMAs (token block major) and between
them the 16 LDS reads of the next step's fragments into set 1-P (one after
every third MFMA, from the first on) and the wave's 8 DMA loads of a later
step (one after MFMAs 4, 12, ..., 60).  The zero variants (a tile's first
step, accumulating into 0): 1 issues no DMA (the kernel loads that step's
slice before the previous tile's epilogue), 2 does.  FL_W4_FUSED_*: the
zero variant without DMA, cut into the halves of the previous tile's
epilogue row blocks (fused_half).

Asm operands of a step: %0 / %1 LDS byte address of this lane's token /
feature fragment 0 in the stage being read, %2..%9 the lanes' global byte
offsets of the 8 loads, %10 the LDS address of the wave's first load, %11 /
%12 the 64-bit token / weight base of the loaded K slice, %13 the vmcnt.

FL_W4_HSTEP_*: the step of a half-width tile (step_hf), with the same
operands and zero variants.

Run: python gen_gemm_w4.py  (rewrites gemm_w4.inc next to this file).
"""
import pathlib

HERE = pathlib.Path(__file__).resolve().parent
MNEMONIC = {"F16": "v_mfma_f32_16x16x32_f16", "BF16": "v_mfma_f32_16x16x32_bf16"}


def vreg(base, n=4):
    return f"v[{base}:{base + n - 1}]"


# MFMA index after which each of the 16 fragment reads / 8 DMA loads issues.
READ_AFTER = [3 * r for r in range(16)]
DMA_AFTER = [8 * j + 4 for j in range(8)]


def step(dtype, cur, zero, read_after=READ_AFTER, dma_after=DMA_AFTER):
    rc = 128 + 64 * cur
    rn = 128 + 64 * (1 - cur)
    out = ["s_waitcnt vmcnt(%13)", "s_waitcnt lgkmcnt(0)", "s_barrier"]
    for i in range(64):
        t, f = i >> 3, i & 7
        k = 8 * f + t
        acc = f"a[{4 * k}:{4 * k + 3}]"
        src_c = "0" if zero else acc
        out.append(f"{MNEMONIC[dtype]} {acc}, {vreg(rc + 32 + 4 * f)}, {vreg(rc + 4 * t)}, {src_c}")
        for r in (r for r in range(16) if read_after[r] == i):
            blk = r // 2
            if r % 2 == 0:
                out.append(f"ds_read_b128 {vreg(rn + 4 * blk)}, %0 offset:{blk * 1024}")
            else:
                out.append(f"ds_read_b128 {vreg(rn + 32 + 4 * blk)}, %1 offset:{blk * 1024}")
        for j in (j for j in range(8) if dma_after[j] == i and zero != 1):
            imm = j * 1024 if j < 4 else 16384 + (j - 4) * 1024
            out.append("s_mov_b32 m0, %10" if imm == 0 else f"s_add_u32 m0, %10, {imm}")
            out.append("s_nop 0")
            out.append(f"global_load_lds_dwordx4 %{2 + j}, {'%11' if j < 4 else '%12'}")
    return out


def fused_half(dtype, t, half):
    """Half h of row block t of a tile's epilogue fused with the next tile's
    first K step (set 0, accumulating into 0, no DMA): for each of the four
    feature blocks f, the four accumulator reads of tile k = 8f + t (outputs
    %0..%15) and then the MFMA that restarts tile k.  Each half also issues
    one of the 16 fragment reads of the step after (into set 1; %16 / %17 are
    this lane's token / feature fragment address in that stage).  The first
    half carries the step's fragment wait and barrier."""
    rc, rn = 128, 192
    out = ["s_waitcnt lgkmcnt(0)", "s_barrier"] if (t, half) == (0, 0) else []
    for j in range(4):
        f = 4 * half + j
        k = 8 * f + t
        out += [f"v_accvgpr_read_b32 %{4 * j + e}, a{4 * k + e}" for e in range(4)]
        out.append(f"{MNEMONIC[dtype]} a[{4 * k}:{4 * k + 3}], {vreg(rc + 32 + 4 * f)}, "
                   f"{vreg(rc + 4 * t)}, 0")
        if j == 1:
            r = 2 * t + half
            blk = r // 2
            if r % 2 == 0:
                out.append(f"ds_read_b128 {vreg(rn + 4 * blk)}, %16 offset:{blk * 1024}")
            else:
                out.append(f"ds_read_b128 {vreg(rn + 32 + 4 * blk)}, %17 offset:{blk * 1024}")
    return out


# Half-width step (a tile's last-round half, HALF_DMA_AFTER / step_hf): the
# full register map and the full step's DMA loads, operands and wait, but
# only feature blocks 0-3: 32 MFMAs (token block major) and 12 fragment reads
# of the next step (token blocks 0-7, feature blocks 0-3).
HALF_READ_AFTER = [(32 * r) // 12 for r in range(12)]
HALF_DMA_AFTER = [4 * j + 2 for j in range(8)]


def step_hf(dtype, cur, zero):
    rc = 128 + 64 * cur
    rn = 128 + 64 * (1 - cur)
    out = ["s_waitcnt vmcnt(%13)", "s_waitcnt lgkmcnt(0)", "s_barrier"]
    for i in range(32):
        t, f = i >> 2, i & 3
        k = 8 * f + t
        acc = f"a[{4 * k}:{4 * k + 3}]"
        src_c = "0" if zero else acc
        out.append(f"{MNEMONIC[dtype]} {acc}, {vreg(rc + 32 + 4 * f)}, {vreg(rc + 4 * t)}, {src_c}")
        for r in (r for r in range(12) if HALF_READ_AFTER[r] == i):
            if r < 8:
                out.append(f"ds_read_b128 {vreg(rn + 4 * r)}, %0 offset:{r * 1024}")
            else:
                out.append(f"ds_read_b128 {vreg(rn + 32 + 4 * (r - 8))}, %1 offset:{(r - 8) * 1024}")
        for j in (j for j in range(8) if HALF_DMA_AFTER[j] == i and zero != 1):
            imm = j * 1024 if j < 4 else 16384 + (j - 4) * 1024
            out.append("s_mov_b32 m0, %10" if imm == 0 else f"s_add_u32 m0, %10, {imm}")
            out.append("s_nop 0")
            out.append(f"global_load_lds_dwordx4 %{2 + j}, {'%11' if j < 4 else '%12'}")
    return out


def reads(cur):
    r0 = 128 + 64 * cur
    out = []
    for blk in range(8):
        out.append(f"ds_read_b128 {vreg(r0 + 4 * blk)}, %0 offset:{blk * 1024}")
        out.append(f"ds_read_b128 {vreg(r0 + 32 + 4 * blk)}, %1 offset:{blk * 1024}")
    out.append("s_waitcnt lgkmcnt(0)")
    return out


def as_c_string(lines):
    return " \\\n".join(f'  "{l}\\n\\t"' for l in lines)


def generate(**kw):
    parts = [
        "// Generated by gen_gemm_w4.py -- do not edit.  Register map and operand",
        "// numbering are described there.",
        "#pragma once",
        "",
        "#define FL_W4_CLOBBER_V " + ", ".join(f'"v{i}"' for i in range(128, 256)),
        "#define FL_W4_CLOBBER_A " + ", ".join(f'"a{i}"' for i in range(256)),
        "",
    ]
    for dtype in ("F16", "BF16"):
        for cur in (0, 1):
            for zero in (0, 1, 2):
                parts.append(f"#define FL_W4_STEP_{dtype}_{cur}_{zero} \\")
                parts.append(as_c_string(step(dtype, cur, zero, **kw)))
                parts.append("")
    for dtype in ("F16", "BF16"):
        for t in range(8):
            for half in (0, 1):
                parts.append(f"#define FL_W4_FUSED_{dtype}_{t}_{half} \\")
                parts.append(as_c_string(fused_half(dtype, t, half)))
                parts.append("")
    parts.append("#define FL_W4_READ_0 \\")
    parts.append(as_c_string(reads(0)))
    parts.append("")
    for dtype in ("F16", "BF16"):
        for cur in (0, 1):
            for zero in (0, 1, 2):
                parts.append(f"#define FL_W4_HSTEP_{dtype}_{cur}_{zero} \\")
                parts.append(as_c_string(step_hf(dtype, cur, zero)))
                parts.append("")
    # Accumulator tile k -> four floats, for the epilogue.
    parts.append("template <int K> struct W4Acc;")
    for k in range(64):
        regs = "\\n\\t".join(f"v_accvgpr_read_b32 %{e}, a{4 * k + e}" for e in range(4))
        parts.append(
            f"template <> struct W4Acc<{k}> {{ __device__ static inline float4_t read() {{ "
            f"float x, y, z, w; asm volatile(\"{regs}\" : \"=v\"(x), \"=v\"(y), \"=v\"(z), "
            f"\"=v\"(w)); return float4_t{{x, y, z, w}}; }} }};")
    parts.append("")
    return "\n".join(parts)


if __name__ == "__main__":
    (HERE / "gemm_w4.inc").write_text(generate())
