// Published-slot protocol of the decode kernels' split-K finish, as plain
// functions that compile for the host too (tests/native/slot_protocol_emu.cpp
// drives them from threads on the CPU).
//
// A slot is one 32-bit word of workspace per (split, row, column).  It reads 0
// while empty.  A publishing split stores the bitwise complement of its fp32
// partial, so every published value is non-zero; the one partial whose
// complement is 0, the NaN 0xFFFFFFFF, is published as the canonical quiet NaN
// 0x7FC00000 instead.  The finisher polls until every slot it needs is
// non-zero, sums the decoded values in split order, and stores 0 to every slot
// it read, so the slots are empty again when the call ends.
//
// The poll is bounded.  A finisher that exhausts its budget stores NaN outputs
// and sets kStatusSplitKTimeout in the workspace status word.  A publisher
// that arrives after such a give-up leaves its slot non-zero, so the status
// word also marks the workspace as poisoned: its slot half must be zeroed
// again before the next call uses it.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define W4A16_HD __host__ __device__ __forceinline__
#else
#define W4A16_HD inline
#endif

namespace w4a16 {

// Status word bits (the last aligned 32-bit word of a workspace).
constexpr uint32_t kStatusSplitKTimeout = 1u;

// Default poll budget of a finisher (rounds over its outstanding slots).
constexpr uint32_t kDefaultSpinLimit = 1u << 20;

W4A16_HD uint32_t f32_bits(float v) {
  uint32_t b;
  __builtin_memcpy(&b, &v, 4);
  return b;
}

W4A16_HD float bits_f32(uint32_t b) {
  float v;
  __builtin_memcpy(&v, &b, 4);
  return v;
}

// Slot word for a partial: never 0.
W4A16_HD uint32_t publish_bits(float v) {
  uint32_t b = f32_bits(v);
  if (b == 0xffffffffu) b = 0x7fc00000u;
  return ~b;
}

W4A16_HD bool slot_empty(uint32_t word) { return word == 0u; }

// The partial a non-empty slot holds.
W4A16_HD float slot_value(uint32_t word) { return bits_f32(~word); }

}  // namespace w4a16
