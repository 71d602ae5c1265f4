// nx_rows.hpp — row preconditions of the register-run kernels, in one place.
//
// k_block_prologue (RMSNorm + router logits, and the exact router logits
// alone) and k_rms_runs (exact RMSNorm) hold a whole row in registers, one run
// of float4s per lane.  Their loads clamp the float4 index into the row
// (min(i, H / 4 - 1)) and select zeros for indices past it afterwards, so that
// every load is issued before the first wait; a clamped index is in range only
// for a row of at least one whole float4 (with H = 0 it is -1: the float4
// before the row).  Every launcher of those kernels checks register_row_fits
// first.
//
// Plain C++ (no HIP): the CPU tests compile this header on its own.
#pragma once

namespace nx {

// widest rows of the register-run kernels, in floats: k_block_prologue's
// 64-lane chains of 112-column runs, k_rms_runs' 64 runs of 28 float4s
constexpr long kPrologueMaxH = 64 * 112;
constexpr long kRmsRunsMaxH = 64 * 28 * 4;

// a row of H floats suits a register-run kernel holding at most max_h: whole
// float4s, at least one, at most max_h
constexpr bool register_row_fits(long H, long max_h) {
  return H > 0 && H % 4 == 0 && H <= max_h;
}

}  // namespace nx
