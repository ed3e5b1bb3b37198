"""CPU model of the grouped GEMM's LDS layouts (parallel_amd/csrc/grouped_gemm.hip).

The kernel's DMA (buffer_load_dwordx4 ... lds) fills each 1 KiB block lane by
lane, so a lane fetches whichever global 16-byte chunk belongs at its slot;
fragment reads then locate each element with a per-lane offset.  This model
restates both sides' index formulas and checks (1) that the reader finds
every element where the writer put it and (2) that every read pass touches
distinct banks of the 64-bank (256 B/clk) gfx950 LDS: 16 lanes per
ds_read_b128 pass, 32 lanes per ds_read_b64_tr_b16 pass.  A swizzle designed
for 32 banks fails (2), which is what the SQ_LDS_BANK_CONFLICT counter showed
on the GPU before the change.
"""

import pytest


def kc_swizzle(r):  # K-contiguous: row bits 2-3
    return (r >> 2) & 3


def mc_swizzle(kk):  # M/N-contiguous: k-row & 3 selects the 64-byte bank quarter
    return 4 * (kk & 3)


def bank_conflicts(addrs, lanes_per_pass, width):
    n = 0
    for p in range(0, len(addrs), lanes_per_pass):
        banks = [((a // 4) + b) % 64 for a in addrs[p:p + lanes_per_pass] for b in range(width // 4)]
        n += len(banks) - len(set(banks))
    return n


def check_kc(R, swz):
    where = {}
    for li in range(R * 64 // 1024):  # 32-deep k-tile: 4 chunks of 16 B per row
        for lane in range(64):
            r = li * 16 + (lane >> 2)
            where[(r, (lane & 3) ^ swz(r))] = li * 1024 + lane * 16
    conflicts = 0
    for row0 in range(0, R, 32):
        for ks in range(2):
            addrs = []
            for lane in range(64):
                l32, kh = lane & 31, lane >> 5
                off = row0 * 64 + l32 * 64 + (((2 * ks + kh) ^ swz(l32)) << 4)
                assert where[(row0 + l32, 2 * ks + kh)] == off
                addrs.append(off)
            conflicts += bank_conflicts(addrs, 16, 16)
    return conflicts


def check_mc(R, WT, swz):
    cpk = R // 8
    where = {}
    for li in range(R * 64 // 1024):
        for lane in range(64):
            kk = li * (64 // cpk) + lane // cpk
            where[(kk, (lane % cpk) ^ swz(kk))] = li * 1024 + lane * 16
    conflicts = 0
    for wcb in range(0, R, WT):
        for t in range(WT // 32):
            for ks in range(2):
                for h in range(2):
                    addrs = []
                    for lane in range(64):
                        q, i = lane >> 4, lane & 15
                        krow = 8 * (q >> 1) + (i >> 2)
                        col = 16 * (q & 1) + 4 * (i & 3)
                        off = (krow * R * 2 + ((((wcb + 32 * t + col) >> 3) ^ swz(krow)) << 4)
                               + (((col >> 2) & 1) << 3) + 16 * ks * R * 2 + h * 4 * R * 2)
                        kr, gcol = 16 * ks + krow + 4 * h, wcb + 32 * t + col
                        assert where[(kr, gcol >> 3)] + (gcol & 7) * 2 == off
                        addrs.append(off)
                    conflicts += bank_conflicts(addrs, 32, 8)
    return conflicts


@pytest.mark.parametrize("R", [128, 256])
def test_k_contiguous_layout_is_consistent_and_conflict_free(R):
    assert check_kc(R, kc_swizzle) == 0


@pytest.mark.parametrize("R,WT", [(128, 64), (256, 64), (256, 128)])
def test_transpose_read_layout_is_consistent_and_conflict_free(R, WT):
    assert check_mc(R, WT, mc_swizzle) == 0


def test_model_flags_32_bank_swizzles():
    assert check_kc(256, lambda r: (r >> 1) & 3) > 0
    assert check_mc(256, 64, lambda kk: 2 * (kk & 3)) > 0
