// W4A16 fused linear for MI355X (gfx950): y[M,N] = x[M,K] (bf16) @ W[K,N],
// W stored as packed signed INT4 with one fp32 scale per 128-row K group.
//
// Weight format (fixed by the reference, engine/kernels/quant.py:115-118,141-146):
//   packed[k/2, n] int8: bits 7..4 = q[2i, n] (even K row), bits 3..0 = q[2i+1, n]
//   (odd K row), both 4-bit two's complement in [-8, 7];
//   scale[k/128, n] fp32;  W[k, n] = q[k, n] * scale[k/128, n].
// Contraction order (engine/kernels/quant.py:221-234): per 128-row group the dot
// product of bf16 activations with the integer weights is formed in fp32, then
// multiplied by the fp32 scale and added to an fp32 accumulator; the result is
// rounded once to bf16.
//
// Kernels in this file:
//   skinny_kernel   M <= 32 (decode, batched decode, speculative verify).  HBM bound.
//   rowsum_kernel   per-(group,row) activation sums used by gemm_kernel.
//   gemm_kernel     M > 32 (prefill).  MFMA bound.
//   dequant_kernel  packed -> dense weights (bit-exactness probe of the unpack).
//
// Nibble -> bf16 conversion used by both matrix kernels.  Flipping bit 3 of a
// two's complement nibble q gives u = q + 8 in [0, 15].  The bf16 bit pattern
// 0x4300 | u is exactly 128 + u, so one byte permute plus one and-or turns a
// packed byte into a pair of bf16 values (128 + u_even, 128 + u_odd).  The MFMA
// therefore produces sum_k x[k] * (q[k] + 136); the 136 * sum_k x[k] offset is
// removed per (row, group) before the scale is applied, which keeps the
// per-group partial exact up to fp32 accumulation rounding.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <type_traits>

#include "../../include/w4a16.h"

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kGroup = 128;                 // K rows per scale group
constexpr int kPackedRowsPerGroup = kGroup / 2;
constexpr uint32_t kBf16Base = 0x43004300u; // bf16 128.0 in both halves
constexpr uint32_t kBf16Neg136 = 0xC308C308u;
constexpr float kOffset = 136.0f;           // 128 (bf16 base) + 8 (nibble bias)
constexpr int kCounterBytes = 65536;        // split-K arrival counters at the head of the workspace
constexpr int kMaxStrips = kCounterBytes / 4;

struct LinearArgs {
  const uint16_t* x;   // bf16 activations [M, K], row stride ldx (elements)
  int64_t ldx;
  const uint8_t* packed;  // [K/2, N], row stride ldp (bytes)
  int64_t ldp;
  const float* scale;  // [K/128, N], row stride lds (elements)
  int64_t lds;
  uint16_t* y;         // bf16 output [M, N], row stride ldy (elements)
  int64_t ldy;
  int M, N, K;
  float* part;         // split-K partials [nsplit][M][N] (skinny) / row sums [K/128][M] (gemm)
  uint32_t* counters;  // one arrival counter per column strip, zero between calls
  int gps;             // groups per split (skinny)
  int nsplit;          // number of K splits (skinny)
  int vec;             // bit 0: packed/scale rows 16B aligned; bit 1: x rows 16B aligned;
                       // bit 2: y rows 8B aligned
  int mtiles, ntiles;  // gemm tile grid
#ifdef W4A16_EXP
  uint64_t* trace;     // per-wave phase timestamps (experiments only)
#endif
};

#ifdef W4A16_EXP
#define W4A16_MARK(i)                                                                                       \
  do {                                                                                                      \
    if (a.trace && (threadIdx.x & 63) == 0)                                                                 \
      a.trace[(((size_t)blockIdx.y * gridDim.x + blockIdx.x) * (blockDim.x / 64) + (threadIdx.x >> 6)) * 8 + \
              (i)] = __builtin_amdgcn_s_memrealtime();                                                      \
  } while (0)
#else
#define W4A16_MARK(i) \
  do {                \
  } while (0)
#endif

__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

// Round-to-nearest-even fp32 -> bf16; NaN becomes the canonical quiet NaN 0x7FC0,
// the same rule torch uses for float -> bfloat16.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4_t v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A 32-bit word of packed bytes (4 columns) prepared for pair extraction.
struct Prep {
  uint32_t p;  // nibble sign bits flipped: every nibble now holds u = q + 8
  uint32_t q;  // p >> 4: the high nibble of byte c sits in the low nibble of byte c
};

__device__ __forceinline__ Prep prep(uint32_t raw) {
  Prep w;
  w.p = raw ^ 0x88888888u;
  w.q = w.p >> 4;
  return w;
}

// bf16 pair for column c (0..3) of a prepared word: low half 128 + u(even row),
// high half 128 + u(odd row).
template <int C>
__device__ __forceinline__ uint32_t pair_of(Prep w) {
  // v_perm_b32 byte pool: bytes 0-3 come from the second operand, 4-7 from the first.
  const uint32_t y = __builtin_amdgcn_perm(w.p, w.q, (uint32_t)C | ((uint32_t)(4 + C) << 16));
  return (y & 0x000F000Fu) | kBf16Base;
}

__device__ __forceinline__ uint32_t pair_dyn(Prep w, int c) {
  switch (c) {
    case 0: return pair_of<0>(w);
    case 1: return pair_of<1>(w);
    case 2: return pair_of<2>(w);
    default: return pair_of<3>(w);
  }
}

// Raw buffer resource over [base, base + bytes): untyped dword loads
// (DATA_FORMAT 32 in the third descriptor word), no stride.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

template <int BYTES>
__device__ __forceinline__ void buffer_load_packed(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                   uint32_t (&out)[BYTES / 4]) {
  if constexpr (BYTES == 16) {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
    out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
  } else if constexpr (BYTES == 8) {
    const u32x2_t v = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
    out[0] = v[0]; out[1] = v[1];
  } else {
    out[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  }
}

// Load `bytes` (4, 8 or 16) consecutive packed bytes starting at column `col`
// of one packed row.  Columns at or beyond N read as 0 (q = 0).
// FULL: the caller guarantees the whole tile is in bounds and aligned, so the
// load is unconditional (no per-lane branch; all loads of a group can be in
// flight together).
template <int BYTES, bool FULL>
__device__ __forceinline__ void load_packed(const uint8_t* row, int col, int N, bool vec,
                                            uint32_t (&out)[BYTES / 4]) {
  if (FULL || (vec && col + BYTES <= N)) {
    if constexpr (BYTES == 16) {
      u32x4_t v = *reinterpret_cast<const u32x4_t*>(row + col);
      out[0] = v[0]; out[1] = v[1]; out[2] = v[2]; out[3] = v[3];
    } else if constexpr (BYTES == 8) {
      u32x2_t v = *reinterpret_cast<const u32x2_t*>(row + col);
      out[0] = v[0]; out[1] = v[1];
    } else {
      out[0] = *reinterpret_cast<const uint32_t*>(row + col);
    }
  } else {
#pragma unroll
    for (int w = 0; w < BYTES / 4; ++w) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int c = col + 4 * w + b;
        const uint32_t v = (c < N) ? (uint32_t)row[c] : 0u;
        acc |= v << (8 * b);
      }
      out[w] = acc;
    }
  }
}

// Load `CNT` consecutive fp32 scales from column `col`; columns >= N read 0.
template <int CNT, bool FULL>
__device__ __forceinline__ void load_scales(const float* row, int col, int N, bool vec, float (&s)[CNT]) {
  if (FULL || (vec && col + CNT <= N)) {
#pragma unroll
    for (int i = 0; i < CNT; i += 4) {
      f32x4_t v = *reinterpret_cast<const f32x4_t*>(row + col + i);
      s[i] = v[0]; s[i + 1] = v[1]; s[i + 2] = v[2]; s[i + 3] = v[3];
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

template <int CPL>
struct DecodeSlot {
  static constexpr int WPR = CPL / 4;
  uint32_t raw[4][4][WPR];
  float s[CPL];
};

// xs: LDS activations [M][kpitch] bf16; g_local = group index within the staged K range.
template <int CPL>
__device__ __forceinline__ void decode_compute(const DecodeSlot<CPL>& d, const uint16_t* xs, int kpitch, int g_local,
                                               int xrow_idx, int lk, uint32_t keep, f32x4_t (&total)[CPL]) {
  constexpr int WPR = CPL / 4;
  const bf16x8_t neg136 = as_bf16x8(u32x4_t{kBf16Neg136, kBf16Neg136, kBf16Neg136, kBf16Neg136});
  const uint16_t* xrow = xs + xrow_idx * kpitch + g_local * kGroup + lk * 8;
  bf16x8_t A[4];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xrow + st * 32);
    A[st] = as_bf16x8(v & keep);
  }
  f32x4_t cinit = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int st = 0; st < 4; ++st) cinit = mfma16(A[st], neg136, cinit);
  f32x4_t acc[CPL];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
#pragma unroll
    for (int wi = 0; wi < WPR; ++wi) {
      Prep pw[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) pw[r] = prep(d.raw[st][r][wi]);
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int t = wi * 4 + c4;
        const bf16x8_t B = as_bf16x8(u32x4_t{pair_dyn(pw[0], c4), pair_dyn(pw[1], c4),
                                             pair_dyn(pw[2], c4), pair_dyn(pw[3], c4)});
        acc[t] = mfma16(A[st], B, st == 0 ? cinit : acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < CPL; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) total[t][r] = __builtin_fmaf(acc[t][r], d.s[t], total[t][r]);
}

// ---------------------------------------------------------------------------
// Split-K finish shared by the M <= 32 kernels.  Each workgroup publishes its
// fp32 partial for (split, strip) with agent-scope relaxed atomic stores, which
// the hardware keeps coherent per access across the XCD L2s (no whole-L2
// writeback / invalidate as a release/acquire fence would need).  The
// workgroup barrier waits until those stores are acknowledged before thread 0
// bumps the strip's arrival counter; the last arrival, whose counter update
// has returned before it issues any load, sums all partials in split order
// (deterministic), writes bf16 and resets the counter to zero.  Partials are
// loaded 8 at a time so their latencies overlap.
// ---------------------------------------------------------------------------
template <int NT, class PartialFn>
__device__ __forceinline__ void splitk_finish(const LinearArgs& a, int strip, int n0, int wcols, int rows,
                                              PartialFn partial) {
  const int M = a.M, N = a.N;
  const int elems = rows * wcols;
  float* part = a.part + (size_t)blockIdx.y * M * N;
  for (int e = threadIdx.x; e < elems; e += NT) {
    const int m = e / wcols, c = e % wcols, n = n0 + c;
    if (n < N) __hip_atomic_store(part + (size_t)m * N + n, partial(e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  __shared__ int is_last;
  if (threadIdx.x == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(a.counters + strip, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == (uint32_t)(a.nsplit - 1));
  }
  __syncthreads();
  if (!is_last) return;
  for (int e = threadIdx.x; e < elems; e += NT) {
    const int m = e / wcols, c = e % wcols, n = n0 + c;
    if (n < N) {
      const float* src = a.part + (size_t)m * N + n;
      const size_t stride = (size_t)M * N;
      float v = 0.f;
      for (int sp0 = 0; sp0 < a.nsplit; sp0 += 8) {
        float t[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
          t[i] = sp0 + i < a.nsplit ? __hip_atomic_load(src + (size_t)(sp0 + i) * stride, __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT)
                                    : 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) v += t[i];
      }
      a.y[(int64_t)m * a.ldy + n] = f32_to_bf16(v);
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(a.counters + strip, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Skinny kernel (M <= 32).
//
// A wave owns 16*CPL output columns and a set of 128-row K groups.  Lane l
// covers columns col0 = n0 + CPL*(l%16) .. +CPL and, inside each 32-row K step,
// rows 8*(l/16) .. +8 (four packed rows).  Per group a lane issues 16 loads of
// CPL bytes (4 steps x 4 packed rows); 16 lanes read CPL*16 contiguous bytes of
// one packed row, so each wave load instruction covers four full row segments.
// Column t of the lane maps to MFMA instance t with virtual column l%16, so the
// lane's CPL output columns are contiguous.  MT M-subtiles of 16 rows reuse the
// same unpacked weights.
//
// Per group g and M-subtile:  acc = -136*sum_k x  (4 MFMAs against a -136 matrix),
// acc += x . (q + 136) over the 4 K steps, total += acc * scale[g, n].
// A wave keeps the next group's loads in flight while it computes the current
// one.
//
// The WAVES waves of a workgroup split the workgroup's groups round-robin and
// are summed through LDS.  Workgroups along gridDim.y split K further; each
// writes an fp32 partial and the last one to arrive for a column strip (arrival
// counter) adds the partials in split order and writes bf16.  The counter is
// reset to zero by that last workgroup, so the workspace needs zeroing once.
// ---------------------------------------------------------------------------
template <int MT, int CPL>
struct SkinnyGroup {
  static constexpr int WPR = CPL / 4;
  uint32_t raw[4][4][WPR];  // [K step][packed row][word]
  bf16x8_t A[MT][4];        // [M subtile][K step]
  float s[CPL];             // scales of the lane's columns
};

template <int MT, int CPL, bool FULL>
__device__ __forceinline__ void skinny_load(const LinearArgs& a, int g, int col0, int mrow0, int lk,
                                            uint32_t keep0, SkinnyGroup<MT, CPL>& d) {
  constexpr int WPR = CPL / 4;
  const bool vec_w = (a.vec & 1) != 0;
  const bool vec_x = (a.vec & 2) != 0;
#pragma unroll
  for (int st = 0; st < 4; ++st)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t pr = (int64_t)g * kPackedRowsPerGroup + st * 16 + lk * 4 + r;
#ifdef W4A16_EXP_NOLOAD
#pragma unroll
      for (int w = 0; w < WPR; ++w) d.raw[st][r][w] = (uint32_t)(col0 * 2654435761u + pr * 97u + w);
#else
      load_packed<CPL, FULL>(a.packed + pr * a.ldp, col0, a.N, vec_w, d.raw[st][r]);
#endif
    }
  // Activations: lane holds x[m][g*128 + 32*st + 8*lk .. +8] for m = 16*mt + l%16.
  // Rows past M load row M-1 (always valid) and are zeroed by a select, so the
  // loads carry no per-lane branch.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mrow0 + 16 * mt;
    const int mrow = m < a.M ? m : a.M - 1;
    const uint32_t keep = mt == 0 ? keep0 : (m < a.M ? 0xffffffffu : 0u);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      u32x4_t v = __builtin_bit_cast(
          u32x4_t, load_x8(a.x + (int64_t)mrow * a.ldx + (int64_t)g * kGroup + st * 32 + lk * 8, vec_x));
      d.A[mt][st] = as_bf16x8(v & keep);
    }
  }
  load_scales<CPL, FULL>(a.scale + (int64_t)g * a.lds, col0, a.N, vec_w, d.s);
  (void)WPR;
}

template <int MT, int CPL>
__device__ __forceinline__ void skinny_compute(const SkinnyGroup<MT, CPL>& d, f32x4_t (&total)[MT][CPL]) {
  constexpr int WPR = CPL / 4;
#ifdef W4A16_EXP_LOADONLY
  uint32_t h = 0;
  for (int st = 0; st < 4; ++st) for (int r = 0; r < 4; ++r) for (int w = 0; w < WPR; ++w) h ^= d.raw[st][r][w];
  total[0][0][0] += __uint_as_float(h & 0x3fffffu) + (float)d.A[0][0][0] + d.s[0];
  return;
#endif
  const bf16x8_t neg136 = as_bf16x8(u32x4_t{kBf16Neg136, kBf16Neg136, kBf16Neg136, kBf16Neg136});
  // Offset correction -136 * sum_{k in group} x[m, k], in MFMA output layout.
  f32x4_t cinit[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    f32x4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) c = mfma16(d.A[mt][st], neg136, c);
    cinit[mt] = c;
  }
  // Step-outer: the CPL column accumulators of a step are independent MFMAs.
  f32x4_t acc[MT][CPL];
#pragma unroll
  for (int st = 0; st < 4; ++st) {
#pragma unroll
    for (int wi = 0; wi < WPR; ++wi) {
      Prep pw[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) pw[r] = prep(d.raw[st][r][wi]);
#pragma unroll
      for (int c4 = 0; c4 < 4; ++c4) {
        const int t = wi * 4 + c4;
        const bf16x8_t B = as_bf16x8(u32x4_t{pair_dyn(pw[0], c4), pair_dyn(pw[1], c4),
                                             pair_dyn(pw[2], c4), pair_dyn(pw[3], c4)});
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][t] = mfma16(d.A[mt][st], B, st == 0 ? cinit[mt] : acc[mt][t]);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < CPL; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) total[mt][t][r] = __builtin_fmaf(acc[mt][t][r], d.s[t], total[mt][t][r]);
}

template <int MT, int CPL, int WAVES, bool FULL, bool PIPE>
__global__ __launch_bounds__(WAVES * 64) void skinny_kernel(LinearArgs a) {
  constexpr int WCOLS = 16 * CPL;    // columns per wave / workgroup
  constexpr int NT = WAVES * 64;
  extern __shared__ float red[];     // [WAVES][R rows][WCOLS]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int strip = blockIdx.x;
  const int n0 = strip * WCOLS;
  const int col0 = n0 + lc * CPL;
  const int G = a.K / kGroup;
  const int g_begin = blockIdx.y * a.gps;
  const int g_end = min(G, g_begin + a.gps);
  const int M = a.M;
  const int N = a.N;
  const uint32_t keep0 = lc < M ? 0xffffffffu : 0u;

  W4A16_MARK(0);
  f32x4_t total[MT][CPL];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < CPL; ++t) total[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // This wave's groups are g = g_begin + wave, + WAVES, ...  With PIPE the
  // next group's loads are issued before the current group is computed.
  int g = g_begin + wave;
  if (!PIPE) {
    for (; g < g_end; g += WAVES) {
      SkinnyGroup<MT, CPL> cur;
      skinny_load<MT, CPL, FULL>(a, g, col0, lc, lk, keep0, cur);
      W4A16_MARK(1);
      skinny_compute<MT, CPL>(cur, total);
    }
  } else if (g < g_end) {
    SkinnyGroup<MT, CPL> cur, nxt;
    skinny_load<MT, CPL, FULL>(a, g, col0, lc, lk, keep0, cur);
    while (true) {
      const int gn = g + WAVES;
      if (gn < g_end) skinny_load<MT, CPL, FULL>(a, gn, col0, lc, lk, keep0, nxt);
      skinny_compute<MT, CPL>(cur, total);
      if (gn >= g_end) break;
      const int gnn = gn + WAVES;
      if (gnn < g_end) skinny_load<MT, CPL, FULL>(a, gnn, col0, lc, lk, keep0, cur);
      skinny_compute<MT, CPL>(nxt, total);
      if (gnn >= g_end) break;
      g = gnn;
    }
  }

  W4A16_MARK(3);
  // ---- reduce the waves through LDS (rows < M only) ----
  const int R = min(M, 16 * MT);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + lk * 4 + r;
      if (m < R) {
        float* dst = red + ((size_t)wave * R + m) * WCOLS + lc * CPL;
#pragma unroll
        for (int t = 0; t < CPL; t += 4)
          *reinterpret_cast<f32x4_t*>(dst + t) =
              f32x4_t{total[mt][t][r], total[mt][t + 1][r], total[mt][t + 2][r], total[mt][t + 3][r]};
      }
    }
  __syncthreads();
  W4A16_MARK(4);

  const int elems = R * WCOLS;
  auto wave_sum = [&](int e) {
    float v = red[e];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[(size_t)w * elems + e];
    return v;
  };
  if (a.nsplit == 1) {
    for (int e = threadIdx.x; e < elems; e += NT) {
      const int m = e / WCOLS, c = e % WCOLS, n = n0 + c;
      if (n < N) a.y[(int64_t)m * a.ldy + n] = f32_to_bf16(wave_sum(e));
    }
    W4A16_MARK(5);
    return;
  }

  splitk_finish<NT>(a, strip, n0, WCOLS, R, wave_sum);
  W4A16_MARK(6);
}

// ---------------------------------------------------------------------------
// Decode GEMV kernel (M <= 16): the HBM-bound path of batch-1 decode.
//
// Workgroup = 4 waves on one strip of 16*CPL columns; blockIdx.y selects a
// range of gps groups (normally 4, one per wave).  Sized so that every
// workgroup of a launch is resident at once: the lean register budget
// (one group in flight per wave, 32-bit row offsets) allows 3+ workgroups per
// CU, and launches are planned as whole multiples of the CU count where the
// shape allows.  Order of work in a wave: issue the group's 16 weight loads
// and its scales, copy the workgroup's activations x[0:M, krange] into LDS,
// barrier, then unpack + MFMA with A fragments read from LDS.
// Lane mapping and arithmetic are those of skinny_kernel.
// ---------------------------------------------------------------------------
template <int CPL, bool FULL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 8))) void gemv_kernel(LinearArgs a) {
  constexpr int WPR = CPL / 4;
  constexpr int WCOLS = 16 * CPL;
  extern __shared__ __attribute__((aligned(16))) float smem[];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int strip = blockIdx.x;
  const int n0 = strip * WCOLS;
  const int col0 = n0 + lc * CPL;
  const int G = a.K / kGroup;
  const int g_begin = blockIdx.y * a.gps;
  const int g_end = min(G, g_begin + a.gps);
  const int M = a.M, N = a.N;
  const int kspan = (g_end - g_begin) * kGroup;
  const int kpitch = a.gps * kGroup + 8;   // +16 B per row against LDS bank conflicts
  const bool vec_w = (a.vec & 1) != 0;
  W4A16_MARK(0);

  // Weight loads for this wave's group.  FULL launches use buffer loads: the
  // per-lane offset (column, k-block row) is fixed and the row of each load
  // is a scalar offset, so no per-load address arithmetic is needed.
  int g = g_begin + wave;
  DecodeSlot<CPL> cur;
  const uint32_t ldp = (uint32_t)a.ldp;
  // (Only FULL launches use these; the resources are harmless otherwise.)
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.packed, (uint32_t)((size_t)(a.K / 2) * a.ldp));
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.scale, (uint32_t)((size_t)G * a.lds * 4));
  const uint32_t wvoff = (uint32_t)col0 + (uint32_t)(lk * 4) * ldp;
  const uint32_t svoff = (uint32_t)col0 * 4u;
  auto load_group = [&](int gg) {
    if constexpr (FULL) {
      const uint32_t gbase = (uint32_t)gg * kPackedRowsPerGroup * ldp;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          buffer_load_packed<CPL>(wrs, wvoff, gbase + (uint32_t)(st * 16 + r) * ldp, cur.raw[st][r]);
      const uint32_t soff = (uint32_t)gg * (uint32_t)a.lds * 4u;
#pragma unroll
      for (int t = 0; t < CPL; t += 4) {
        const f32x4_t v = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(srs, svoff + 4u * t, soff, 0));
        cur.s[t] = v[0]; cur.s[t + 1] = v[1]; cur.s[t + 2] = v[2]; cur.s[t + 3] = v[3];
      }
    } else {
      const uint8_t* base = a.packed + (int64_t)gg * kPackedRowsPerGroup * a.ldp;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const uint32_t off = (uint32_t)((st * 16 + lk * 4 + r) * ldp);
          load_packed<CPL, FULL>(base + off, col0, N, vec_w, cur.raw[st][r]);
        }
      load_scales<CPL, FULL>(a.scale + (int64_t)gg * a.lds, col0, N, vec_w, cur.s);
    }
  };
  if (g < g_end) load_group(g);
  W4A16_MARK(1);

  // Activations of the workgroup's K range -> LDS.
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  {
    const bool vec_x = (a.vec & 2) != 0;
    const int chunks = kspan / 8;
    for (int i = threadIdx.x; i < M * chunks; i += 256) {
      const int m = i / chunks, c = i % chunks;
      const uint16_t* src = a.x + (int64_t)m * a.ldx + (int64_t)g_begin * kGroup + c * 8;
      *reinterpret_cast<u32x4_t*>(xs + m * kpitch + c * 8) = __builtin_bit_cast(u32x4_t, load_x8(src, vec_x));
    }
  }
  __syncthreads();
  W4A16_MARK(2);

  const uint32_t keep = lc < M ? 0xffffffffu : 0u;
  const int xrow_idx = lc < M ? lc : M - 1;
  f32x4_t total[CPL];
#pragma unroll
  for (int t = 0; t < CPL; ++t) total[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  while (g < g_end) {
    decode_compute<CPL>(cur, xs, kpitch, g - g_begin, xrow_idx, lk, keep, total);
    g += 4;
    if (g < g_end) load_group(g);
  }
  W4A16_MARK(3);

  // Reduce the 4 waves through LDS (reusing the activation buffer).
  __syncthreads();
  float* red = smem;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = lk * 4 + r;
    if (m < M) {
      float* dst = red + ((size_t)wave * M + m) * WCOLS + lc * CPL;
#pragma unroll
      for (int t = 0; t < CPL; t += 4)
        *reinterpret_cast<f32x4_t*>(dst + t) = f32x4_t{total[t][r], total[t + 1][r], total[t + 2][r], total[t + 3][r]};
    }
  }
  __syncthreads();
  W4A16_MARK(4);
  const int elems = M * WCOLS;
  auto wave_sum = [&](int e) {
    return ((red[e] + red[(size_t)elems + e]) + red[(size_t)2 * elems + e]) + red[(size_t)3 * elems + e];
  };
  if (a.nsplit == 1) {
    for (int e = threadIdx.x; e < elems; e += 256) {
      const int m = e / WCOLS, c = e % WCOLS, n = n0 + c;
      if (n < N) a.y[(int64_t)m * a.ldy + n] = f32_to_bf16(wave_sum(e));
    }
    W4A16_MARK(5);
    return;
  }
  splitk_finish<256>(a, strip, n0, WCOLS, M, wave_sum);
  W4A16_MARK(6);
  (void)WPR;
}

// ---------------------------------------------------------------------------
// Row sums for the gemm offset correction: out[g*M + m] = 136 * sum_{k in g} x[m,k].
// 16 lanes per (row, group); each lane sums 8 values, then a butterfly over the
// 16 lanes (fixed order, deterministic).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rowsum_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                     int K, int vec_x, float* __restrict__ out) {
  const int G = K / kGroup;
  const int64_t item = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const bool valid = item < (int64_t)M * G;
  const int m = valid ? (int)(item / G) : 0;
  const int g = valid ? (int)(item % G) : 0;
  float s = 0.f;
  if (valid) {
    const bf16x8_t v = load_x8(x + (int64_t)m * ldx + (int64_t)g * kGroup + sub * 8, vec_x != 0);
    const u32x4_t w = __builtin_bit_cast(u32x4_t, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s += __uint_as_float(w[i] << 16);
      s += __uint_as_float(w[i] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) s += __shfl_xor(s, off, 16);
  if (valid && sub == 0) out[(int64_t)g * M + m] = kOffset * s;
}

// ---------------------------------------------------------------------------
// GEMM kernel (M > 32).
//
// Workgroup tile 128 rows x 256 columns, 4 waves side by side along N, each
// wave 128 x 64 (8 M-subtiles x 4 MFMA column blocks, 4 columns per lane).
// Per 128-row K group:
//  * the activation tile (128 x 128 bf16, 32 KB) is copied global -> LDS with
//    direct-to-LDS loads in MFMA fragment order (wave w copies K step w),
//    double buffered, together with the group's 128 row sums (rowsum_kernel);
//  * each wave loads its own packed weights (16 buffer loads of 4 bytes,
//    scalar row offsets) and scales one group ahead, in registers;
//  * running-ratio fold: the accumulator U is kept in units of the current
//    group's scale, U <- U * (s_prev / s) - 136 * rowsum, so one fp32
//    accumulator set suffices and the MFMAs accumulate straight into it;
//    the output is U * s_last (see clamp_scale for zero / tiny scales).
// Tiles are handed out XCD-major: workgroup b runs on XCD b % 8, and each XCD
// receives a contiguous range of tile ids, ordered in column bands of 4 row
// tiles, so the rows of x and the weight columns an XCD touches stay in its L2.
// ---------------------------------------------------------------------------
constexpr int kGemmRows = 128;
constexpr int kGemmCols = 256;
constexpr int kGemmMT = 8;      // 16-row subtiles per wave
constexpr int kGemmBand = 4;    // row tiles per column band

// Scale magnitudes below 1e-20 (zero, subnormal or tiny) are raised to 1e-20
// in the GEMM fold so that the running ratio stays finite; such a group then
// contributes at most 1e-20 * sum|x*q| instead of exactly 0.  Non-finite
// scales pass through and make the column non-finite, as in the reference.
__device__ __forceinline__ float clamp_scale(float s) {
  const float a = __builtin_fabsf(s);
  return a < 1e-20f ? __builtin_copysignf(1e-20f, s) : s;
}

template <bool FULL>
#ifndef W4A16_GEMM_WAVES
#define W4A16_GEMM_WAVES 2
#endif
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W4A16_GEMM_WAVES, 8))) void gemm_kernel(LinearArgs a) {
  __shared__ u32x4_t As[2][4 * kGemmMT * 64];  // [buf][step][subtile][lane] 16 B each
  __shared__ __attribute__((aligned(16))) float Cs[2][kGemmRows];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int M = a.M, N = a.N;
  const int G = a.K / kGroup;

  // ---- tile assignment ----
  const int tiles = a.mtiles * a.ntiles;
  int tid_lin = blockIdx.x;
  if ((gridDim.x & 7) == 0) {
    const int per_xcd = gridDim.x >> 3;
    tid_lin = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  }
  if (tid_lin >= tiles) return;
  const int band_size = kGemmBand * a.ntiles;
  const int band = tid_lin / band_size;
  const int first_m = band * kGemmBand;
  const int band_rows = min(kGemmBand, a.mtiles - first_m);
  const int in_band = tid_lin % band_size;
  const int m_tile = first_m + in_band % band_rows;
  const int n_tile = in_band / band_rows;
  const int m0 = m_tile * kGemmRows;
  const int col0 = n_tile * kGemmCols + wave * 64 + lc * 4;
  const bool vec_w = (a.vec & 1) != 0;

  // ---- operand sources ----
  const uint32_t ldp = (uint32_t)a.ldp;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(a.packed, (uint32_t)((size_t)(a.K / 2) * a.ldp));
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(a.scale, (uint32_t)((size_t)G * a.lds * 4));
  const uint32_t wvoff = (uint32_t)col0 + (uint32_t)(lk * 4) * ldp;
  // Activation rows this lane copies (clamped: rows past M compute values that are never stored).
  const uint16_t* xlane = a.x + (int64_t)(m0 + lc) * a.ldx + (wave * 4 + lk) * 8;
  const int64_t xstep = (int64_t)16 * a.ldx;     // 16 rows
  const int last_full = (M - 1 - m0 - lc) / 16;  // subtiles whose row m0 + 16i + lc < M
  int crow = m0 + (threadIdx.x & 127);
  crow = crow < M ? crow : M - 1;

  auto stage_a = [&](int g, int b) {
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i) {
      const int ii = i <= last_full ? i : last_full;
      const uint16_t* src = xlane + (int64_t)ii * xstep + (int64_t)g * kGroup;
      __builtin_amdgcn_global_load_lds((const void*)src,
                                       (void __attribute__((address_space(3)))*)&As[b][(wave * kGemmMT + i) * 64],
                                       16, 0, 0);
    }
    if (wave < 2)
      __builtin_amdgcn_global_load_lds((const void*)(a.part + (int64_t)g * M + crow),
                                       (void __attribute__((address_space(3)))*)&Cs[b][wave * 64], 4, 0, 0);
  };
  auto load_b = [&](int g, uint32_t (&raw)[4][4], float (&s)[4]) {
    if constexpr (FULL) {
      const uint32_t gbase = (uint32_t)g * kPackedRowsPerGroup * ldp;
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          raw[st][r] = __builtin_amdgcn_raw_buffer_load_b32(wrs, wvoff, gbase + (uint32_t)(st * 16 + r) * ldp, 0);
      const f32x4_t v = __builtin_bit_cast(
          f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(srs, (uint32_t)col0 * 4u, (uint32_t)g * (uint32_t)a.lds * 4u, 0));
      s[0] = v[0]; s[1] = v[1]; s[2] = v[2]; s[3] = v[3];
    } else {
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t pr = (int64_t)g * kPackedRowsPerGroup + st * 16 + lk * 4 + r;
          uint32_t w[1];
          load_packed<4, false>(a.packed + pr * a.ldp, col0, N, vec_w, w);
          raw[st][r] = w[0];
        }
      load_scales<4, false>(a.scale + (int64_t)g * a.lds, col0, N, vec_w, s);
    }
  };

  f32x4_t U[kGemmMT][4];
#pragma unroll
  for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) U[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint32_t raw[4][4];
  float s[4];
  float s_ref[4];      // scale U is currently expressed in (per column)
  load_b(0, raw, s);
  stage_a(0, 0);
#pragma unroll
  for (int t = 0; t < 4; ++t) s_ref[t] = clamp_scale(s[t]);

  for (int g = 0; g < G; ++g) {
    const int b = g & 1;
    // Direct-to-LDS copies of this group (issued one iteration earlier) must
    // have landed before the barrier publishes them.
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0)
    __syncthreads();

    const bool has_next = g + 1 < G;
    uint32_t raw_n[4][4];
    float s_n[4];
    if (has_next) {
      stage_a(g + 1, b ^ 1);
      load_b(g + 1, raw_n, s_n);
    }

    // Fold: U <- U * (s_ref / s) - 136 * rowsum.  (U is zero before the first
    // group, where the ratio is 1.)  s_ref / s uses the hardware reciprocal:
    // relative error ~1 ulp, the order of the fp32 rounding of the fold.
    float rho[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const float sc = clamp_scale(s[t]);
      rho[t] = s_ref[t] * __builtin_amdgcn_rcpf(sc);
      s_ref[t] = sc;
    }
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i) {
      const f32x4_t c4 = *reinterpret_cast<const f32x4_t*>(&Cs[b][16 * i + 4 * lk]);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) U[i][t][r] = __builtin_fmaf(U[i][t][r], rho[t], -c4[r]);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      Prep p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = prep(raw[st][r]);
      bf16x8_t B[4];
      B[0] = as_bf16x8(u32x4_t{pair_of<0>(p[0]), pair_of<0>(p[1]), pair_of<0>(p[2]), pair_of<0>(p[3])});
      B[1] = as_bf16x8(u32x4_t{pair_of<1>(p[0]), pair_of<1>(p[1]), pair_of<1>(p[2]), pair_of<1>(p[3])});
      B[2] = as_bf16x8(u32x4_t{pair_of<2>(p[0]), pair_of<2>(p[1]), pair_of<2>(p[2]), pair_of<2>(p[3])});
      B[3] = as_bf16x8(u32x4_t{pair_of<3>(p[0]), pair_of<3>(p[1]), pair_of<3>(p[2]), pair_of<3>(p[3])});
#pragma unroll
      for (int i = 0; i < kGemmMT; ++i) {
        const bf16x8_t A = __builtin_bit_cast(bf16x8_t, As[b][(st * kGemmMT + i) * 64 + lane]);
#pragma unroll
        for (int t = 0; t < 4; ++t) U[i][t] = mfma16(A, B[t], U[i][t]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }

    if (has_next) {
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int r = 0; r < 4; ++r) raw[st][r] = raw_n[st][r];
#pragma unroll
      for (int t = 0; t < 4; ++t) s[t] = s_n[t];
    }
  }

  // ---- store y = U * s_ref: lane holds rows m0 + 16i + 4lk + r, columns col0 .. col0+3 ----
  const float* outs = s_ref;
  const bool vec_y = FULL ? (a.vec & 4) != 0 : ((a.vec & 4) != 0 && col0 + 4 <= N);
#pragma unroll
  for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 16 * i + 4 * lk + r;
      if (m >= M) continue;
      uint16_t* dst = a.y + (int64_t)m * a.ldy + col0;
      const uint16_t h0 = f32_to_bf16(U[i][0][r] * outs[0]);
      const uint16_t h1 = f32_to_bf16(U[i][1][r] * outs[1]);
      const uint16_t h2 = f32_to_bf16(U[i][2][r] * outs[2]);
      const uint16_t h3 = f32_to_bf16(U[i][3][r] * outs[3]);
      if (vec_y) {
        *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{(uint32_t)h0 | ((uint32_t)h1 << 16),
                                                   (uint32_t)h2 | ((uint32_t)h3 << 16)};
      } else {
        if (col0 + 0 < N) dst[0] = h0;
        if (col0 + 1 < N) dst[1] = h1;
        if (col0 + 2 < N) dst[2] = h2;
        if (col0 + 3 < N) dst[3] = h3;
      }
    }
}

// ---------------------------------------------------------------------------
// Dequantize: out[k, n] = q[k, n] * s[k/128, n] (engine/kernels/quant.py:122-156).
// With a bf16 output the scale is first rounded to bf16, then the product is
// rounded to bf16, which is what `dequantize_weight_int4(packed, scale.to(bf16))`
// computes.  One thread per packed byte.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ packed, int64_t ldp,
                                                      const float* __restrict__ scale, int64_t lds,
                                                      void* __restrict__ out, int64_t ldo, int out_bf16,
                                                      int K, int N, int group_size) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)(K / 2) * N;
  if (idx >= total) return;
  const int i = (int)(idx / N);
  const int n = (int)(idx % N);
  const int8_t byte = (int8_t)packed[(int64_t)i * ldp + n];
  const int q_even = byte >> 4;                          // arithmetic shift: [-8, 7]
  const int q_odd = (int)(int8_t)(uint8_t)(byte << 4) >> 4;
  const int k = 2 * i;
  float s = scale[(int64_t)(k / group_size) * lds + n];
  if (out_bf16) {
    s = bf16_to_f32(f32_to_bf16(s));
    uint16_t* o = static_cast<uint16_t*>(out);
    o[(int64_t)k * ldo + n] = f32_to_bf16((float)q_even * s);
    o[(int64_t)(k + 1) * ldo + n] = f32_to_bf16((float)q_odd * s);
  } else {
    float* o = static_cast<float*>(out);
    o[(int64_t)k * ldo + n] = (float)q_even * s;
    o[(int64_t)(k + 1) * ldo + n] = (float)q_odd * s;
  }
}

// y = 0 for an empty contraction (K == 0), as the reference produces.
__global__ __launch_bounds__(256) void zero_kernel(uint16_t* __restrict__ y, int64_t ldy, int M, int N) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  y[(idx / N) * ldy + idx % N] = 0;
}

// ---------------------------------------------------------------------------
// Host-side planning.
// ---------------------------------------------------------------------------
struct Plan {
  int kind;    // 0 = skinny, 1 = gemm, 2 = gemv (M <= 16, activations in LDS)
  size_t lds_bytes;
  int mt, cpl, waves, pipe;  // skinny variant
  int strips, nsplit, gps;
  size_t ws_bytes;
};

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int env_int(const char* name, int dflt) {
#ifdef W4A16_EXP
  const char* v = getenv(name);
  if (v) return atoi(v);
#endif
  (void)name;
  return dflt;
}

Plan make_plan(int M, int N, int K) {
  Plan p{};
  const int G = K / kGroup;
  if (M > 32) {
    p.kind = 1;
    p.ws_bytes = (size_t)kCounterBytes + (size_t)G * M * sizeof(float);
    return p;
  }
  // GEMV kernel: 4 waves x one 128-row group each per workgroup; activations
  // of the workgroup's K range staged in LDS.
  if (M <= 16 && G > 0 && env_int("W4A16_GEMV", 1)) {
    p.kind = 2;
    p.cpl = env_int("W4A16_CPL", 8);
    p.strips = ceil_div(N, 16 * p.cpl);
    p.gps = env_int("W4A16_GPS", 4);
    p.nsplit = ceil_div(G, p.gps);
    p.lds_bytes = (size_t)M * (p.gps * kGroup + 8) * 2;
    const size_t rbytes = (size_t)4 * M * 16 * p.cpl * 4;
    if (rbytes > p.lds_bytes) p.lds_bytes = rbytes;
    p.ws_bytes = p.nsplit > 1 ? (size_t)kCounterBytes + (size_t)p.nsplit * M * N * sizeof(float) : 0;
    return p;
  }
  p.kind = 0;
  p.mt = M <= 16 ? 1 : 2;
  p.cpl = env_int("W4A16_CPL", 8);
  if (p.mt == 2 && p.cpl == 16) p.cpl = 8;
  const int R = M < 16 * p.mt ? M : 16 * p.mt;
  // Waves per workgroup: as many as the LDS reduction buffer allows (<= 64 KB).
  int waves = 16;
  while (waves > 4 && (size_t)waves * R * 16 * p.cpl * 4 > 65536) waves >>= 1;
  p.waves = env_int("W4A16_WAVES", waves);
  p.pipe = env_int("W4A16_PIPE", 0);
  p.strips = ceil_div(N, 16 * p.cpl);
  // Split K across workgroups until ~16 waves per CU are resident, keeping at
  // least one group per wave and the fp32 partial traffic (write + read) within
  // a quarter of the weight bytes.
  int nsplit = ceil_div(256 * 16, (int64_t)p.strips * p.waves);
  const int by_traffic = (int)((int64_t)K / (64 * (int64_t)M));
  if (nsplit > by_traffic) nsplit = by_traffic;
  const int max_split = ceil_div(G, p.waves);
  if (nsplit > max_split) nsplit = max_split;
  if (nsplit < 1) nsplit = 1;
  nsplit = env_int("W4A16_NSPLIT", nsplit);
  p.gps = G > 0 ? ceil_div(G, nsplit) : 0;
  p.nsplit = G > 0 ? ceil_div(G, p.gps) : 1;
  p.ws_bytes = p.nsplit > 1 ? (size_t)kCounterBytes + (size_t)p.nsplit * M * N * sizeof(float) : 0;
  return p;
}

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? W4A16_OK : W4A16_ERR_LAUNCH;
}

template <int CPL>
int launch_gemv_c(const LinearArgs& a, const Plan& p, hipStream_t stream) {
  // Buffer loads address at most 4 GiB per resource.
  const bool full = (a.vec & 1) && (a.N % (16 * CPL) == 0) && (size_t)(a.K / 2) * a.ldp < 0xffffffffull &&
                    (size_t)(a.K / kGroup) * a.lds * 4 < 0xffffffffull;
  if (full)
    hipLaunchKernelGGL((gemv_kernel<CPL, true>), dim3(p.strips, p.nsplit), dim3(256), p.lds_bytes, stream, a);
  else
    hipLaunchKernelGGL((gemv_kernel<CPL, false>), dim3(p.strips, p.nsplit), dim3(256), p.lds_bytes, stream, a);
  return launch_status();
}

int launch_gemv(const LinearArgs& a, const Plan& p, hipStream_t stream) {
  if (p.cpl == 4) return launch_gemv_c<4>(a, p, stream);
  if (p.cpl == 16) return launch_gemv_c<16>(a, p, stream);
  return launch_gemv_c<8>(a, p, stream);
}

template <int MT, int CPL, int WAVES, bool PIPE>
int launch_skinny_p(const LinearArgs& a, const Plan& p, hipStream_t stream) {
  const int R = a.M < 16 * MT ? a.M : 16 * MT;
  const size_t shmem = (size_t)WAVES * R * 16 * CPL * sizeof(float);
  const bool full = (a.vec & 1) && (a.N % (16 * CPL) == 0);
  if (full)
    hipLaunchKernelGGL((skinny_kernel<MT, CPL, WAVES, true, PIPE>), dim3(p.strips, p.nsplit), dim3(WAVES * 64),
                       shmem, stream, a);
  else
    hipLaunchKernelGGL((skinny_kernel<MT, CPL, WAVES, false, PIPE>), dim3(p.strips, p.nsplit), dim3(WAVES * 64),
                       shmem, stream, a);
  return launch_status();
}

template <int MT, int CPL, int WAVES>
int launch_skinny_w(const LinearArgs& a, const Plan& p, hipStream_t stream) {
  if (p.pipe) return launch_skinny_p<MT, CPL, WAVES, true>(a, p, stream);
  return launch_skinny_p<MT, CPL, WAVES, false>(a, p, stream);
}

template <int MT, int CPL>
int launch_skinny(const LinearArgs& a, const Plan& p, hipStream_t stream) {
  switch (p.waves) {
    case 16: return launch_skinny_w<MT, CPL, 16>(a, p, stream);
    case 8: return launch_skinny_w<MT, CPL, 8>(a, p, stream);
    default: return launch_skinny_w<MT, CPL, 4>(a, p, stream);
  }
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int w4a16_abi_version(void) { return W4A16_ABI_VERSION; }

const char* w4a16_error_string(int code) {
  switch (code) {
    case W4A16_OK: return "ok";
    case W4A16_ERR_NULL: return "null pointer argument";
    case W4A16_ERR_SHAPE: return "invalid shape (negative size or leading dimension smaller than the row)";
    case W4A16_ERR_K_GROUP: return "K must be a multiple of group_size (and even) for int4 packing";
    case W4A16_ERR_GROUP_SIZE: return "fused INT4 kernel requires group_size=128";
    case W4A16_ERR_WORKSPACE: return "workspace missing or smaller than w4a16_workspace_size()";
    case W4A16_ERR_LAUNCH: return "HIP kernel launch failed";
    case W4A16_ERR_DTYPE: return "unsupported dtype code";
    case W4A16_ERR_TOO_LARGE: return "problem exceeds the supported size";
    default: return "unknown w4a16 error";
  }
}

int w4a16_workspace_size(int M, int N, int K, int group_size, size_t* bytes) {
  if (!bytes) return W4A16_ERR_NULL;
  *bytes = 0;
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  if (group_size != kGroup) return W4A16_ERR_GROUP_SIZE;
  if (K % kGroup != 0) return W4A16_ERR_K_GROUP;
  if (M == 0 || N == 0) return W4A16_OK;
  const Plan p = make_plan(M, N, K);
  *bytes = p.ws_bytes;
  return W4A16_OK;
}

int w4a16_linear(const void* x, int64_t ldx, const int8_t* packed, int64_t ldp, const float* scale,
                 int64_t lds, void* y, int64_t ldy, int M, int N, int K, int group_size, void* workspace,
                 size_t workspace_bytes, void* stream) {
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  if (group_size != kGroup) return W4A16_ERR_GROUP_SIZE;
  if (K % kGroup != 0) return W4A16_ERR_K_GROUP;
  if (M == 0 || N == 0) return W4A16_OK;
  if (!y) return W4A16_ERR_NULL;
  if (K > 0 && (!x || !packed || !scale)) return W4A16_ERR_NULL;
  if (ldy < N || (K > 0 && (ldx < K || ldp < N || lds < N))) return W4A16_ERR_SHAPE;

  const Plan p = make_plan(M, N, K);
  if (p.ws_bytes > 0 && (!workspace || workspace_bytes < p.ws_bytes)) return W4A16_ERR_WORKSPACE;
  if (p.kind != 1 && p.nsplit > 1 && p.strips > kMaxStrips) return W4A16_ERR_TOO_LARGE;

  LinearArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.ldx = ldx;
  a.packed = reinterpret_cast<const uint8_t*>(packed);
  a.ldp = ldp;
  a.scale = scale;
  a.lds = lds;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = M;
  a.N = N;
  a.K = K;
  const bool vw = aligned16(packed) && (ldp % 16 == 0) && aligned16(scale) && (lds % 4 == 0);
  const bool vx = aligned16(x) && (ldx % 8 == 0);
  const bool vy = (((uintptr_t)y & 7u) == 0) && (ldy % 4 == 0);
  a.vec = (vw ? 1 : 0) | (vx ? 2 : 0) | (vy ? 4 : 0);
#ifdef W4A16_EXP
  a.trace = getenv("W4A16_TRACE") ? reinterpret_cast<uint64_t*>(strtoull(getenv("W4A16_TRACE"), nullptr, 0)) : nullptr;
#endif
  hipStream_t s = static_cast<hipStream_t>(stream);

  if (K == 0) {
    hipLaunchKernelGGL(zero_kernel, dim3(ceil_div((int64_t)M * N, 256)), dim3(256), 0, s, a.y, ldy, M, N);
    return launch_status();
  }

  if (p.kind == 1) {
    if (!vx) {
      // The gemm stages activations with 16-byte loads; unaligned activations
      // are processed 32 rows at a time by the skinny kernel instead.
      for (int m0 = 0; m0 < M; m0 += 32) {
        const int mc = M - m0 < 32 ? M - m0 : 32;
        int rc = w4a16_linear(static_cast<const uint16_t*>(x) + (int64_t)m0 * ldx, ldx, packed, ldp, scale, lds,
                              static_cast<uint16_t*>(y) + (int64_t)m0 * ldy, ldy, mc, N, K, group_size,
                              workspace, workspace_bytes, stream);
        if (rc != W4A16_OK) return rc;
      }
      return W4A16_OK;
    }
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    a.mtiles = ceil_div(M, kGemmRows);
    a.ntiles = ceil_div(N, kGemmCols);
    const int64_t items = (int64_t)M * (K / kGroup);
    hipLaunchKernelGGL(rowsum_kernel, dim3(ceil_div(items, 16)), dim3(256), 0, s, a.x, ldx, M, K, 1, a.part);
    int rc = launch_status();
    if (rc != W4A16_OK) return rc;
    int blocks = a.mtiles * a.ntiles;
    blocks = (blocks + 7) & ~7;
    if ((a.vec & 1) && N % kGemmCols == 0)
      hipLaunchKernelGGL(gemm_kernel<true>, dim3(blocks), dim3(256), 0, s, a);
    else
      hipLaunchKernelGGL(gemm_kernel<false>, dim3(blocks), dim3(256), 0, s, a);
    return launch_status();
  }

  a.gps = p.gps;
  a.nsplit = p.nsplit;
  if (p.nsplit > 1) {
    a.counters = static_cast<uint32_t*>(workspace);
    a.part = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  }
  if (p.kind == 2) return launch_gemv(a, p, s);
  if (p.mt == 1 && p.cpl == 16) return launch_skinny<1, 16>(a, p, s);
  if (p.mt == 1 && p.cpl == 4) return launch_skinny<1, 4>(a, p, s);
  if (p.mt == 1) return launch_skinny<1, 8>(a, p, s);
  if (p.cpl == 4) return launch_skinny<2, 4>(a, p, s);
  return launch_skinny<2, 8>(a, p, s);
}

int w4a16_dequant(const int8_t* packed, int64_t ldp, const float* scale, int64_t lds, void* out, int64_t ldo,
                  int out_dtype, int K, int N, int group_size, void* stream) {
  if (K < 0 || N < 0) return W4A16_ERR_SHAPE;
  if (group_size <= 0) return W4A16_ERR_GROUP_SIZE;
  if (K % group_size != 0 || K % 2 != 0) return W4A16_ERR_K_GROUP;
  if (out_dtype != W4A16_DTYPE_F32 && out_dtype != W4A16_DTYPE_BF16) return W4A16_ERR_DTYPE;
  if (K == 0 || N == 0) return W4A16_OK;
  if (!packed || !scale || !out) return W4A16_ERR_NULL;
  if (ldp < N || lds < N || ldo < N) return W4A16_ERR_SHAPE;
  const int64_t total = (int64_t)(K / 2) * N;
  hipLaunchKernelGGL(dequant_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     reinterpret_cast<const uint8_t*>(packed), ldp, scale, lds, out, ldo,
                     out_dtype == W4A16_DTYPE_BF16 ? 1 : 0, K, N, group_size);
  return launch_status();
}

}  // extern "C"
