// Device-side building blocks shared by the W4A16 kernels (gfx950).
//
// Weight format (fixed by the reference, engine/kernels/quant.py:115-118,141-146):
//   packed[k/2, n] int8: bits 7..4 = q[2i, n] (even K row), bits 3..0 = q[2i+1, n]
//   (odd K row), both 4-bit two's complement in [-8, 7];
//   scale[k/128, n] fp32;  W[k, n] = q[k, n] * scale[k/128, n].
//
// Nibble -> bf16.  Flipping bit 3 of a two's complement nibble q gives
// u = q + 8 in [0, 15], and the bf16 bit pattern 0x4300 | u is exactly 128 + u.
// One byte permute plus an and/or therefore turns a packed byte into the bf16
// pair (128 + u_even, 128 + u_odd).  An MFMA over such operands yields
// sum_k x[k] * (q[k] + 136); the kernels remove 136 * sum_k x[k] per (row,
// group) before the scale is applied, which keeps every per-group partial
// exact up to fp32 accumulation rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace w4a16 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGroup = 128;                      // K rows per scale group
constexpr int kPackedRowsPerGroup = kGroup / 2;  // packed rows per group
constexpr uint32_t kBf16ExpBytes = 0x43434343u;  // high byte of bf16(128 + u) in every byte
constexpr uint32_t kBf16Base = 0x43004300u;      // bf16 128.0 in both halves
constexpr uint32_t kBf16Neg136 = 0xC308C308u;    // bf16 -136.0 in both halves
constexpr float kOffset = 136.0f;                // 128 (bf16 base) + 8 (nibble bias)

// Cache-policy bit of buffer instructions that makes an access coherent at
// agent scope across the XCD L2s (the bit agent-scope atomics use).
constexpr int kAgentCoherent = 16;
// Cache-policy bit for data read once (non-temporal).  Measured on MI355X over
// a 1.24 GB stream of 16-byte buffer loads: 6.98 TB/s with it, 6.41 without.
constexpr int kStream = 2;

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round-to-nearest-even fp32 -> bf16; NaN becomes the canonical quiet NaN
// 0x7FC0, the same rule torch uses for float -> bfloat16.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

// Two fp32 values -> a packed bf16 pair (a in the low half), round to nearest
// even, through gfx950's packed conversion (one VALU op).  Finite values and
// infinities round exactly as f32_to_bf16; a NaN stays a quiet NaN but keeps
// its sign and leading payload bits instead of becoming 0x7FC0.
typedef float f32x2v_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v_t{a, b}, bf16x2_t));
}

// 16x16x32 bf16 MFMA.  Operand layout (lane l): A[m = l%16][k = 8*(l/16) + j],
// B[k = 8*(l/16) + j][n = l%16] for j = 0..7; D[m = 4*(l/16) + r][n = l%16].
__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A 32-bit word of packed bytes (4 columns) spread to one nibble per byte:
// byte 2j of x01 / x23 is u = q + 8 of the even row of column j / j+2 (the high
// nibble), byte 2j+1 that of the odd row (the low nibble).  Every byte holds a
// clean value 0..15, so one byte permute against 0x43 bytes yields a bf16 pair.
struct Prep {
  uint32_t x01;  // columns 0 and 1
  uint32_t x23;  // columns 2 and 3
};

__device__ __forceinline__ Prep prep(uint32_t raw) {
  // q + 8 = q ^ 8 per nibble; xor-and with constants is one v_bitop3 each.
  const uint32_t lo = (raw ^ 0x08080808u) & 0x0F0F0F0Fu;         // odd rows
  const uint32_t hi = ((raw >> 4) ^ 0x08080808u) & 0x0F0F0F0Fu;  // even rows
  // v_perm_b32 byte pool: bytes 0-3 come from the second operand, 4-7 from the first.
  Prep w;
  w.x01 = __builtin_amdgcn_perm(hi, lo, 0x01050004u);
  w.x23 = __builtin_amdgcn_perm(hi, lo, 0x03070206u);
  return w;
}

// bf16 pair for byte c (0..3) of the raw word: low half 128 + u(even row),
// high half 128 + u(odd row); bytes 1 and 3 are the 0x43 exponent byte.
template <int C>
__device__ __forceinline__ uint32_t pair_of(Prep w) {
  return __builtin_amdgcn_perm(C < 2 ? w.x01 : w.x23, kBf16ExpBytes, (C & 1) ? 0x00070006u : 0x00050004u);
}

__device__ __forceinline__ uint32_t pair_dyn(Prep w, int c) {
  switch (c) {
    case 0: return pair_of<0>(w);
    case 1: return pair_of<1>(w);
    case 2: return pair_of<2>(w);
    default: return pair_of<3>(w);
  }
}

// Raw buffer resource over [base, base + bytes): untyped loads (DATA_FORMAT 32
// in the third descriptor word), no stride.  Offsets are 32-bit.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int BYTES, int AUX = 0>
__device__ __forceinline__ void buffer_load_bytes(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                  uint32_t (&out)[(BYTES + 3) / 4]) {
  if constexpr (BYTES == 16) {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
  } else if constexpr (BYTES == 8) {
    const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX));
    out[0] = v[0]; out[1] = v[1];
  } else if constexpr (BYTES == 4) {
    out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, AUX);
  } else {
    out[0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, AUX);
  }
}

// `BYTES` consecutive packed bytes from column `col` of one packed row, with
// generic loads.  FULL: the caller guarantees the span is in bounds and
// aligned, so the load is unconditional (no per-lane branch).  Otherwise
// columns at or beyond N read as 0 (q = 0).
template <int BYTES, bool FULL>
__device__ __forceinline__ void load_packed(const uint8_t* row, int col, int N, bool vec,
                                            uint32_t (&out)[(BYTES + 3) / 4]) {
  if (FULL || (vec && col + BYTES <= N)) {
    if constexpr (BYTES == 16) {
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(row + col);
      out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else if constexpr (BYTES == 8) {
      u32x2_t v = *reinterpret_cast<const u32x2_t*>(row + col);
      out[0] = v[0]; out[1] = v[1];
    } else if constexpr (BYTES == 4) {
      out[0] = *reinterpret_cast<const uint32_t*>(row + col);
    } else {
      out[0] = *reinterpret_cast<const uint16_t*>(row + col);
    }
  } else {
#pragma unroll
    for (int w = 0; w < (BYTES + 3) / 4; ++w) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < (BYTES < 4 ? BYTES : 4); ++b) {
        const int c = col + 4 * w + b;
        const uint32_t v = (c < N) ? (uint32_t)row[c] : 0u;
        acc |= v << (8 * b);
      }
      out[w] = acc;
    }
  }
}

// `CNT` consecutive fp32 scales from column `col`; columns >= N read 0.
template <int CNT, bool FULL>
__device__ __forceinline__ void load_scales(const float* row, int col, int N, bool vec, float (&s)[CNT]) {
  if (FULL || (vec && col + CNT <= N)) {
    if constexpr (CNT % 4 == 0) {
#pragma unroll
      for (int i = 0; i < CNT; i += 4) {
        f32x4_t v = *reinterpret_cast<const f32x4_t*>(row + col + i);
        s[i] = v[0]; s[i + 1] = v[1]; s[i + 2] = v[2]; s[i + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < CNT; ++i) s[i] = row[col + i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < CNT; ++i) s[i] = (col + i < N) ? row[col + i] : 0.0f;
  }
}

// 8 consecutive bf16 activations of one row (16 bytes).
__device__ __forceinline__ bf16x8_t load_x8(const uint16_t* p, bool vec) {
  if (vec) return *reinterpret_cast<const bf16x8_t*>(p);
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
  return as_bf16x8(v);
}

// Agent-coherent fp32 store / load used to publish split-K partials.
__device__ __forceinline__ void store_coherent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait until every vector memory operation this wave issued (loads, stores,
// direct-to-LDS copies) has completed.  gfx9 counts stores in vmcnt.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0f70); }

// Wait until at most N of this wave's vector memory operations are still
// outstanding (loads complete in issue order, so every older one has landed).
template <int N>
__device__ __forceinline__ void wait_vmem_n() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0f70 | (N & 15) | ((N >> 4) << 14));
}

}  // namespace w4a16
