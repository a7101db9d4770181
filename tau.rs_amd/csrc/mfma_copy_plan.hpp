// Per-lane addresses of the direct-to-LDS operand copies of mfma_gemm
// (grouped_gemm.hip), shared by the kernel and by the host checks that prove
// every copy of a stage lands in a distinct LDS chunk and reads inside its
// tensor (tests/mfma_copy_check.cpp).
//
// A stage holds BM rows of A and BN rows of B, BK elements deep, as 16-byte
// chunks (CPR = BK/8 per row).  Instruction i of wave w copies 1 KB: rows
// [q*RPI, (q+1)*RPI) with q = i*(NT/64) + w, lane l supplying row
// q*RPI + l/CPR into chunk slot l%CPR, which holds global chunk
// slot ^ swz(row).  FRAG16 weights are copied as whole 1 KB fragments:
// instruction q of a stage copies fragment (band q / (BK/32), K piece
// q % (BK/32)).
#pragma once
#include <stdint.h>

#include "host_device.hpp"

namespace tau_amd {

// XOR swizzle of the 16-byte chunk slot within a staged row.  LDS has 64
// banks of 4 bytes (256 bytes); a 16-lane phase of a fragment read touches 16
// consecutive rows at one chunk, so (row bank offset, swizzled slot) must be
// distinct over any 16 consecutive rows: 128-byte rows (BK=64) alternate two
// bank offsets, so the key is (row >> 1) & 7; 64-byte rows (BK=32) cycle four
// offsets, so the key is (row >> 2) & 3.
template <int CPR>
TAU_HOST_DEVICE inline int swz(int row) {
    if constexpr (CPR == 8) return (row >> 1) & 7;
    else return (row >> 2) & 3;
}

// Stage row and K offset (elements, within the BK-deep step) that lane `lane`
// of wave `wave` copies with its i-th row-major copy instruction.
template <int NT, int CPR>
TAU_HOST_DEVICE inline void row_copy_slot(int i, int wave, int lane, int& row, int& kchunk) {
    constexpr int RPI = 64 / CPR;
    row = (i * (NT / 64) + wave) * RPI + lane / CPR;
    kchunk = ((lane % CPR) ^ swz<CPR>(row)) * 8;
}

// Weight row (within one expert) of B-stage row r for output tile column c0:
// SiLU tiles take BN/2 gate rows then the matching BN/2 up rows (up row j =
// gate row j + w_up_offset).  Columns past n read row 0 (their outputs are
// never stored).
template <int BN, bool SILU>
TAU_HOST_DEVICE inline long weight_row(int r, int c0, int n, int w_up_offset) {
    if constexpr (SILU) {
        const int j = c0 + (r < BN / 2 ? r : r - BN / 2);
        return j < n ? (r < BN / 2 ? j : j + w_up_offset) : 0;
    } else {
        const int j = c0 + r;
        return j < n ? j : 0;
    }
}

// Element offset from the expert's weights of lane `lane`'s i-th B copy at K
// step 0 (step kb adds kb, or 16*kb for FRAG16).
template <int NT, int CPR, int BN, int BK, bool SILU, bool FRAG16>
TAU_HOST_DEVICE inline long b_copy_offset(int i, int wave, int lane, int c0, int n, int w_up_offset, int k) {
    const int q = i * (NT / 64) + wave;
    if constexpr (FRAG16) {
        const int band = q / (BK / 32), c = q % (BK / 32);
        return (weight_row<BN, SILU>(band * 16, c0, n, w_up_offset) >> 4) * 16L * k + c * 512 + lane * 8;
    } else {
        int r, kchunk;
        row_copy_slot<NT, CPR>(i, wave, lane, r, kchunk);
        return weight_row<BN, SILU>(r, c0, n, w_up_offset) * (long)k + kchunk;
    }
}

// A wave-uniform 64-bit address moved through two 32-bit scalar reads
// (readfirstlane works on 32-bit values) and joined again.  The words are
// unsigned: a low word with bit 31 set must not sign-extend into the high one.
TAU_HOST_DEVICE inline uint32_t address_hi(uint64_t a) { return (uint32_t)(a >> 32); }
TAU_HOST_DEVICE inline uint32_t address_lo(uint64_t a) { return (uint32_t)a; }
TAU_HOST_DEVICE inline uint64_t join_address(uint32_t hi, uint32_t lo) { return ((uint64_t)hi << 32) | (uint64_t)lo; }

}  // namespace tau_amd
