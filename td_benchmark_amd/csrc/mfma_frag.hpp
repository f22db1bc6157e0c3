// The grouped GEMM's LDS row swizzle, FP8 fragment loader and MFMA call.
// Shared by csrc/gemm.hip and the test-only probe library (tests/csrc), which
// checks the operand layout and the matrix core's accumulation through this
// exact code.
#pragma once

#include "common.hpp"

namespace moe {

// LDS rows are 128 B (one 128-element K block of FP8).  The 16 B chunk index
// of a row is XORed with swz(row) = (row mod 8) ^ bit3(row), which depends
// only on the row's position inside its 16-row MFMA subtile.
MOE_HOST_DEVICE int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
// LDS slot of logical 16 B chunk c in row `row`, and its inverse (an involution).
MOE_HOST_DEVICE int slot_of(int c, int row) { return (c ^ swz(row)) & 7; }

// One v_mfma_scale_f32_16x16x128_f8f6f4 from a zero accumulator, OCP e4m3
// operands (format code 0) and unit block scales.
MOE_DEVICE v4f mfma_fp8(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// A 32-byte fragment (lane = row fr, K segment kseg: 32 contiguous K bytes)
// from two per-lane LDS bases plus a compile-time offset.
template <int OFF>
MOE_DEVICE v8i frag_at(const uint8_t* base0, const uint8_t* base1) {
  const v4i x = *reinterpret_cast<const v4i*>(base0 + OFF);
  const v4i y = *reinterpret_cast<const v4i*>(base1 + OFF);
  return (v8i){x[0], x[1], x[2], x[3], y[0], y[1], y[2], y[3]};
}

}  // namespace moe
