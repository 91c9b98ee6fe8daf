#!/usr/bin/env python3
"""Writes gemm_tune_list.h: the CDNA4 (gfx950) GEMM tune space of `kernelh tune`.

The reference's space is BM, BN in {64, 128, 256} x BK in {16, 32} x waves in
{4, 8} x unroll in {1, 2} x vec in {1, 2, 4}, pruned by LDS and VGPR estimates
(include/kernelh/compiler/autotuner.hpp:36-41, lib/compiler/autotuner.cpp:
754-799). Here the same axes are re-pruned for wave64, MFMA tiles and 160 KiB
of LDS per CU:

  MF      MFMA shape: 32 (v_mfma_f32_32x32x2f32) or 16 (v_mfma_f32_16x16x4f32);
          wave tiles are whole multiples of it.
  waves   4 (2 x 2 waves) or 8 (2 x 4 or 4 x 2) per workgroup.
  BM, BN  {64, 128, 256}, = MF x (accumulator blocks per wave) x (waves per side).
  BK      {16, 32} (an MF = 16 chunk is 16 deep, an MF = 32 chunk 8 deep).
  unroll  slabs in flight ahead of the MFMAs: 1 (register-staged, two LDS
          stages), 2 (direct-to-LDS into three stages, or register-staged two
          slabs ahead: "pf2").
  prio    MFMA-phase wave priority (s_setprio 1 while MFMAs issue): both
          values for the four-wave MF = 32 tiles, 1 elsewhere (measured +2% on
          the product tiles).
  vec     not a compile-time axis: every candidate loads float4s when k and n
          are multiples of 4 and aligned, and falls back to guarded scalar
          loads otherwise (the CSV reports which one the shape takes).

Prune rules (each drops configurations that cannot run two waves per SIMD,
which is what hides one wave's slab hand-over behind the other's MFMAs):
  1. accumulators <= 128 VGPRs per lane;
  2. accumulators + fragments (twice for the direct-to-LDS pipeline, which
     reads the next chunk while the current one computes) + register staging
     <= 200 VGPRs (the rest holds addresses);
  3. LDS <= 80 KiB for four-wave workgroups (two per CU), <= 160 KiB for
     eight-wave ones (one per CU);
  4. a slab splits into whole float4s over the workgroup's threads;
  5. pf2 only for 64 x 64 tiles (two register staging sets fit only there);
  6. MF = 16 direct-to-LDS only with BN >= 128 (with BN = 64 four B rows share
     one padded LDS group and the fragment reads of one half-wave collide on
     banks).
The product kernels (`gemm`, `gemm_mid`, `gemm_small`, `gemm_small_pf2`,
`gemm_ksplit`, `gemm_ksplit_deep`) are candidates too; the runtime lists them
beside these (khrt_gemm_candidate_get).

The entries are dealt round-robin into PARTS code objects so that they
compile in parallel. Run: python gemm_tune_space.py > gemm_tune_list.h
"""
import sys

PARTS = 4
PIPES = {"regs": 1, "dma": 2, "pf2": 3}  # gemm_tiles.h kPipeRegs / kPipeDma / kPipePrefetch2


def lds_bytes(mf, wgm, wgn, wtm, wtn, bk, pipe):
    """LdsNeed in gemm_tiles.h: the fast pipeline's stages or the generic
    path's single padded stage, whichever is larger, for A and for B."""
    bm, bn = mf * wtm * wgm, mf * wtn * wgn
    dma = pipe == "dma"
    brow = bn // 4
    rpi = (1 if brow >= 64 else 64 // brow) if dma else 1
    lda = bk if dma else bk + 4
    ldg = rpi * bn + 4
    a_stage, b_stage = bm * lda, (bk // rpi) * ldg
    ga, gb = bm * (bk + 4), bk * (bn + 4)
    stages = 3 if dma else 2
    return 4 * (max(stages * a_stage, ga) + max(stages * b_stage, gb))


def space():
    out = []
    for mf in (32, 16):
        for wgm, wgn in ((2, 2), (2, 4), (4, 2)):
            nt = 64 * wgm * wgn
            for bm in (64, 128, 256):
                for bn in (64, 128, 256):
                    if bm % (mf * wgm) or bn % (mf * wgn):
                        continue
                    wtm, wtn = bm // (mf * wgm), bn // (mf * wgn)
                    acc = wtm * wtn * (16 if mf == 32 else 4)
                    frag = 4 * wtm + 4 * wtn
                    for bk in (16, 32):
                        if (bm * bk // 4) % nt or (bk * bn // 4) % nt:
                            continue  # rule 4
                        for pipe in ("regs", "dma", "pf2"):
                            if pipe == "pf2" and (bm, bn) != (64, 64):
                                continue  # rule 5
                            if mf == 16 and pipe == "dma" and bn < 128:
                                continue  # rule 6
                            staging = 0 if pipe == "dma" else 4 * (bm * bk + bk * bn) // 4 // nt * (
                                2 if pipe == "pf2" else 1)
                            regs = acc + (2 * frag if pipe == "dma" else frag) + staging
                            budget = 160 * 1024 if nt == 512 else 80 * 1024
                            if acc > 128 or regs > 200:
                                continue  # rules 1, 2
                            if lds_bytes(mf, wgm, wgn, wtm, wtn, bk, pipe) > budget:
                                continue  # rule 3
                            prios = (0, 1) if (mf == 32 and nt == 256) else (1,)
                            for prio in prios:
                                out.append((mf, wgm, wgn, wtm, wtn, bk, prio, pipe))
    return out


def symbol(mf, wgm, wgn, wtm, wtn, bk, prio, pipe):
    return f"gemm_m{mf}_w{wgm}x{wgn}_t{wtm}x{wtn}_k{bk}_p{prio}_{pipe}"


def main() -> int:
    entries = space()
    parts = [[] for _ in range(PARTS)]
    for i, e in enumerate(entries):
        parts[i % PARTS].append(e)
    w = sys.stdout.write
    w("// Generated by gemm_tune_space.py, which states the space and its prune\n")
    w("// rules; regenerate with `python gemm_tune_space.py > gemm_tune_list.h`.\n")
    w(f"// {len(entries)} candidates in {PARTS} code objects (gemm_tune0 .. gemm_tune{PARTS - 1}).\n")
    w("// X(PART, MF, WGM, WGN, WTM, WTN, BK, PRIO, PIPE, SYMBOL): MFMA shape MF x MF,\n")
    w("// WGM x WGN waves, WTM x WTN accumulator blocks per wave, BK-deep slabs,\n")
    w("// MFMA-phase priority, pipeline (1 register-staged, 2 direct-to-LDS three\n")
    w("// stages, 3 register-staged two slabs ahead). Shared by gemm_tune.hip (one\n")
    w("// kernel per entry) and the runtime's candidate table, so they cannot drift.\n")
    w("#pragma once\n\n")
    w(f"#define KH_GEMM_TUNE_PARTS {PARTS}\n")
    w(f"#define KH_GEMM_TUNE_COUNT {len(entries)}\n\n")
    for p, es in enumerate(parts):
        w(f"#define KH_GEMM_TUNE_PART{p}(X) \\\n")
        for j, e in enumerate(es):
            mf, wgm, wgn, wtm, wtn, bk, prio, pipe = e
            tail = " \\\n" if j + 1 < len(es) else "\n\n"
            w(f"  X({p}, {mf}, {wgm}, {wgn}, {wtm}, {wtn}, {bk}, {prio}, {PIPES[pipe]}, {symbol(*e)}){tail}")
    w("#define KH_GEMM_TUNE_CONFIGS(X) " + " ".join(f"KH_GEMM_TUNE_PART{p}(X)" for p in range(PARTS)) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())
