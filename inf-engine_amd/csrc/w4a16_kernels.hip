// W4A16 fused linear for MI355X (gfx950): y[M,N] = x[M,K] (bf16) @ W[K,N],
// W stored as packed signed INT4 with one fp32 scale per 128-row K group
// (format and nibble arithmetic: w4a16_device.h).
//
// Contraction order (engine/kernels/quant.py:221-234): per 128-row group the
// dot product of bf16 activations with the integer weights is formed in fp32,
// then multiplied by the fp32 scale and added to an fp32 accumulator; the
// result is rounded once to bf16.
//
// A launch processes a table of up to kMaxProblems independent projections
// that share M (one problem for the drop-in int4_matmul; q/k/v or gate/up or
// a set of MoE experts for grouped calls).  Kernels:
//   gemv_kernel     M <= 32, or <= 64 on small shapes (decode, batched decode)  HBM bound
//   rowsum_kernel   per-(group,row) activation sums for gemm_kernel
//   gemm_kernel     larger M (prefill)                      MFMA bound
//   splitk_reduce_kernel  ordered sum of gemm_kernel's K-split partials
//   zero_kernel     y = 0 for K == 0
//   dequant_kernel  packed -> dense weights (bit-exactness probe of the unpack)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "../../include/w4a16.h"
#include "slot_protocol.h"
#include "w4a16_device.h"

using namespace w4a16;

namespace {

constexpr int kMaxProblems = W4A16_MAX_PROBLEMS;
static_assert(kStatusSplitKTimeout == W4A16_STATUS_SPLITK_TIMEOUT, "status bit of the C ABI");

// One projection of a launch, as the device sees it.
struct Problem {
  const uint16_t* x;   // bf16 [M, K], row stride ldx elements
  int64_t ldx;
  const uint8_t* packed;  // [K/2, N], row stride ldp bytes
  int64_t ldp;
  const float* scale;  // [K/128, N], row stride lds elements
  int64_t lds;
  uint16_t* y;         // bf16 [M, N], row stride ldy elements
  int64_t ldy;
  float* part;         // gemm: split-K partials [nsplit][M][N]; gemv: published
                       // partial slots [nsplit - 1][M][N] (workspace, zero between calls)
  float* rowsum;       // gemm: 136 * row sums [K/128][M] (workspace, maybe shared)
  int M, N, K;
  int wg_begin;        // first workgroup of this problem in the launch grid
  int rs_begin;        // rowsum_kernel: first workgroup (-1: row sums shared with another problem)
  int tiles_m, tiles_n;  // gemm tile grid; gemv: tiles_n = column strips
  int nsplit, gps;     // K split: nsplit ranges of gps groups
  int red_begin;       // splitk_reduce_kernel: first workgroup of this problem
  int vec;             // bit 0: packed and scale rows 16-byte aligned; bit 1: x rows 16-byte
                       // aligned; bit 2: y rows 8-byte aligned
};

struct Launch {
  Problem p[kMaxProblems];
  int count;
  int total_wgs;
  uint32_t* status;    // the workspace's status word (W4A16_STATUS_*), or null without a workspace
  uint32_t spin_limit; // polls before a split-K finisher gives up
};


// Problem owning workgroup `wg` (wave-uniform scan of <= 8 entries).
__device__ __forceinline__ int problem_of(const Launch& L, int wg) {
  int p = 0;
  for (int i = 1; i < L.count; ++i)
    if (wg >= L.p[i].wg_begin) p = i;
  return p;
}

// ---------------------------------------------------------------------------
// Split-K reduction of the decode kernel, without atomics.
//
// The workgroup of the last split (split == nsplit - 1) of a strip finishes
// it; the others publish their fp32 partial and exit.  Slot encoding, the
// empty test and the give-up rule are in slot_protocol.h: a slot reading 0 is
// still empty, published slots hold the complement of the partial.  The
// finisher polls the nsplit - 1 slots of each of its elements with
// agent-coherent loads, sums them in split order with its own partial last
// (deterministic), writes bf16 and zeroes the slots again, so the slots are
// empty at the start of every call.
//
// Why no workgroup can wait forever: the grid orders workgroups split-major
// ((strip, split) grids, or split-major ids within a problem), so a finisher
// is dispatched after every workgroup it waits for, and those never wait on
// anything.  The poll is still bounded (Launch::spin_limit); a finisher that
// gives up writes NaN and sets kStatusSplitKTimeout in the workspace status
// word, which the host reads after a synchronisation.
//
// An arrival counter instead (one agent-scope atomic per workgroup, the last
// arrival reduces) measures 1 us (8 splits) to 3.3 us (24 splits) slower per
// launch on MI355X: atomics on one address serialize.
// ---------------------------------------------------------------------------
// Poll-and-sum of nslots published slots (stride bytes apart) for a
// thread's EPT elements at byte offsets off[].  All of a thread's polls for a
// chunk of SCH slots are in flight at once, so a thread with several elements
// waits about one round trip per chunk rather than one per element.  Sums in
// slot order into v; zeroes what it read.
//
// The code is kept short and branch-free outside the spin loop: only the
// finishing workgroup runs it, so its instructions are not in the CU's
// instruction cache and every one of them is fetched on the critical path
// of the launch (MI355X: 512 added instructions there cost 0.25-0.8 us per
// launch).  Polls are unconditional buffer loads; slots past nslots lie
// beyond the resource's range and read 0 without touching memory, and are
// masked out.
template <int EPT>
__device__ __forceinline__ void sum_slots(__amdgpu_buffer_rsrc_t rs, int nslots, uint32_t stride,
                                          const uint32_t (&off)[EPT], const bool (&ok)[EPT], float (&v)[EPT],
                                          uint32_t limit, bool& timed_out) {
  constexpr int SCH = EPT >= 8 ? 2 : (EPT >= 4 ? 4 : 8);  // slots per chunk: EPT * SCH polls in flight
  for (int sp0 = 0; sp0 < nslots; sp0 += SCH) {
    uint32_t t[EPT][SCH];
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < SCH; ++i)
        t[j][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, off[j] + (uint32_t)(sp0 + i) * stride, 0, kAgentCoherent);
    // A slot is still empty when it reads 0, lies within nslots and belongs to one of our elements.
    auto empty = [&](int j, int i) { return slot_empty(t[j][i]) && sp0 + i < nslots && ok[j]; };
    // Wave-uniform loop: every round re-polls all SCH slots and keeps the
    // ones that had already arrived.
    for (uint32_t spins = 0;; ++spins) {
      bool missing = false;
#pragma unroll
      for (int j = 0; j < EPT; ++j)
#pragma unroll
        for (int i = 0; i < SCH; ++i) missing = missing | empty(j, i);  // bitwise: no short-circuit branches
      if (__builtin_amdgcn_ballot_w64(missing) == 0) break;
      // After a give-up the later chunks take what has arrived without
      // waiting, so a give-up costs one poll budget, not one per chunk.
      if (timed_out || spins >= limit) {
        timed_out = true;
        break;
      }
      asm volatile("" ::: "memory");  // every round reloads from memory
#pragma unroll
      for (int j = 0; j < EPT; ++j)
#pragma unroll
        for (int i = 0; i < SCH; ++i) {
          const uint32_t r =
              __builtin_amdgcn_raw_buffer_load_b32(rs, off[j] + (uint32_t)(sp0 + i) * stride, 0, kAgentCoherent);
          const uint32_t keep = t[j][i] != 0u ? ~0u : 0u;  // a mask, not a select, so the load stays unconditional
          t[j][i] = (t[j][i] & keep) | (r & ~keep);
        }
    }
#pragma unroll
    for (int j = 0; j < EPT; ++j)
#pragma unroll
      for (int i = 0; i < SCH; ++i) v[j] += sp0 + i < nslots ? slot_value(t[j][i]) : 0.f;
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j)
    for (int sp = 0; sp < nslots; ++sp)
      if (ok[j]) __builtin_amdgcn_raw_buffer_store_b32(0u, rs, off[j] + (uint32_t)sp * stride, 0, kAgentCoherent);
}

// x * sigmoid(x) in fp32 (engine/layers.py:28-30).
__device__ __forceinline__ float silu(float x) { return x / (1.f + __expf(-x)); }

// Split-K epilogue modes.
enum FinishMode {
  kFinishStore = 0,  // last split sums the partials and stores bf16 y
  kFinishGate = 1,   // gate of a SwiGLU pair: every split publishes (slots [nsplit][M][N])
  kFinishUp = 2,     // up of a SwiGLU pair: the last split also sums the gate's slots
                     // (problem `gate`) and stores bf16(silu(gate) * up)
};

// EPT: most elements (rows x columns of the strip) one thread handles.
template <int NT, int EPT, int MODE, class PartialFn>
__device__ __forceinline__ void splitk_finish(const Launch& L, const Problem& P, int M, int split, int n0, int wcols,
                                              int rows, PartialFn partial, const Problem* gate = nullptr) {
  const int N = P.N;
  const int elems = rows * wcols;
  // Slots are [nslots][M][N] fp32; byte offsets fit in 32 bits (make_plan).
  const uint32_t stride = (uint32_t)M * (uint32_t)N * 4u;
  const int last = P.nsplit - 1;
  const int nslots = MODE == kFinishGate ? P.nsplit : last;
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(P.part, stride * (uint32_t)nslots);
  if (MODE == kFinishGate || split != last) {
    const uint32_t dst = (uint32_t)split * stride;
    for (int e = threadIdx.x; e < elems; e += NT) {
      const int m = e / wcols, c = e % wcols, n = n0 + c;
      if (n < N)
        __builtin_amdgcn_raw_buffer_store_b32(publish_bits(partial(e)), rs, dst + ((uint32_t)m * N + n) * 4u, 0,
                                              kAgentCoherent);
    }
    return;
  }
  uint32_t off[EPT];
  bool ok[EPT];
  float own[EPT], v[EPT];
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    const int e = threadIdx.x + j * NT;
    const int m = e / wcols, c = e % wcols, n = n0 + c;
    ok[j] = e < elems && n < N;
    off[j] = ok[j] ? ((uint32_t)m * N + n) * 4u : 0u;
    own[j] = ok[j] ? partial(e) : 0.f;
    v[j] = 0.f;
  }
  bool timed_out = false;
  const uint32_t limit = L.spin_limit;
  sum_slots<EPT>(rs, last, stride, off, ok, v, limit, timed_out);
  if constexpr (MODE == kFinishUp) {
    float gv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) gv[j] = 0.f;
    const __amdgpu_buffer_rsrc_t grs = make_rsrc(gate->part, stride * (uint32_t)gate->nsplit);
    sum_slots<EPT>(grs, gate->nsplit, stride, off, ok, gv, limit, timed_out);
#pragma unroll
    for (int j = 0; j < EPT; ++j) v[j] = silu(gv[j]) * (v[j] + own[j]);
  } else {
#pragma unroll
    for (int j = 0; j < EPT; ++j) v[j] += own[j];
  }
#pragma unroll
  for (int j = 0; j < EPT; ++j) {
    if (!ok[j]) continue;
    const int e = threadIdx.x + j * NT;
    const int m = e / wcols, n = n0 + e % wcols;
    P.y[(int64_t)m * P.ldy + n] = timed_out ? (uint16_t)0x7fc0 : f32_to_bf16(v[j]);
  }
  // timed_out is wave-uniform (it follows a ballot); one lane per wave reports it.
  if (timed_out && (threadIdx.x & 63) == 0)
    __hip_atomic_fetch_or(L.status, kStatusSplitKTimeout, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------------------
// Decode GEMV kernel (M <= 64): the HBM-bound path of decode and of small
// batches (M > 16 runs two or four 16-row M subtiles that share every
// unpacked weight).
//
// Lane mapping: a wave owns 16*CPL output columns;
// lane l covers columns col0 = n0 + CPL*(l%16) .. +CPL and, inside each 32-row
// K step, rows 8*(l/16) .. +8, i.e. four packed rows.  Per 128-row group a
// lane issues 16 loads of CPL bytes (4 steps x 4 packed rows).  Column t of the
// lane is MFMA instance t with virtual column l%16, so a lane's CPL outputs
// are contiguous.  Per group:
//   acc = -136 * sum_k x   (4 MFMAs against a constant -136 operand),
//   acc += x . (q + 136)   (4 K steps x CPL MFMAs),   total += acc * scale.
//
// Workgroup = WAVES waves on one strip; blockIdx selects (problem, split,
// strip) and wave w takes group split*gps + w of the split's gps (= WAVES)
// groups.  Every wave issues all of its memory traffic before any arithmetic,
// in the order it is consumed: its activation fragments (lanes l%16 < M load
// row l%16 straight from global memory, the rest hold zeros), the group's
// scales, then the 16 weight loads.  A scheduling barrier keeps the compiler
// from sinking loads below the MFMAs, so a wave's loads are all in flight
// together and the waits that follow are partial (vmcnt counts down while the
// first K steps are already being multiplied).  Waves are then reduced
// through LDS; with K split across workgroups, splitk_finish sums the split
// partials in split order.
// ---------------------------------------------------------------------------
template <int CPL>
struct DecodeSlot {
  static constexpr int WPR = CPL / 4;
  uint32_t raw[4][4][WPR];  // [K step][packed row][word]
  float s[CPL];
};

// One group of one wave: A[st] are the activation fragments of the group's 4
// K steps (rows past M zero), d the group's packed weights and scales.
// MT 16-row M subtiles share every unpacked B fragment.
template <int CPL, int MT>
__device__ __forceinline__ void decode_group(const DecodeSlot<CPL>& d, const bf16x8_t (&A)[MT][4],
                                             f32x4_t (&total)[MT][CPL]) {
  constexpr int WPR = CPL / 4;
  const bf16x8_t neg136 = as_bf16x8(u32x4_t{kBf16Neg136, kBf16Neg136, kBf16Neg136, kBf16Neg136});
  f32x4_t cinit[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    cinit[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 4; ++st) cinit[mt] = mfma16(A[mt][st], neg136, cinit[mt]);
  }
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
        for (int mt = 0; mt < MT; ++mt) acc[mt][t] = mfma16(A[mt][st], B, st == 0 ? cinit[mt] : acc[mt][t]);
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

// One wave's share of a decode launch: the 128-row group g of problem P for
// the lane's CPL columns starting at col0, accumulated into total.  Activation
// fragments: lane (lc, lk) holds x[lc, g*128 + 32*st + 8*lk .. +8].  FULL
// launches load them unconditionally (lanes past M read zeros from outside the
// buffer's range), so no branch or wait sits before the weight loads.
template <int CPL, bool FULL, int MT>
__device__ __forceinline__ void decode_wave(const Problem& P, int g, int col0, int lc, int lk, int M,
                                            f32x4_t (&total)[MT][CPL]) {
  const int N = P.N;
  const int G = (uint32_t)P.K / kGroup;
  bf16x8_t A[MT][4];
  DecodeSlot<CPL> d;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int row = lc + 16 * mt;
    const uint32_t keep = row < M ? 0xffffffffu : 0u;
    if constexpr (FULL) {
      // Lanes of rows past M get an offset beyond the resource's range (x is
      // under 2 GB on this path, make_plan): their loads return zeros without
      // a memory access, so at M = 1 only 4 lanes of 64 fetch activations.
      const __amdgpu_buffer_rsrc_t xrs = make_rsrc(P.x, (uint32_t)((size_t)P.ldx * 2 * M));
      const uint32_t xoff =
          row < M ? ((uint32_t)row * (uint32_t)P.ldx + (uint32_t)(g * kGroup + lk * 8)) * 2u : 0x80000000u;
#pragma unroll
      for (int st = 0; st < 4; ++st)
        A[mt][st] = as_bf16x8(
            __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xrs, xoff + st * 64, 0, 0)));
    } else {
      const bool vec_x = (P.vec & 2) != 0;
      const uint16_t* xrow = P.x + (int64_t)(row < M ? row : 0) * P.ldx + (int64_t)g * kGroup + lk * 8;
#pragma unroll
      for (int st = 0; st < 4; ++st)
        A[mt][st] = as_bf16x8(__builtin_bit_cast(u32x4_t, load_x8(xrow + st * 32, vec_x)) & keep);
    }
  }
  if constexpr (FULL) {
    // Weights and scales are read once per call.  With 128-column strips a
    // row segment of a lane group is a whole 128-byte line, so the loads are
    // marked non-temporal (gate M=1 8.55 -> 8.33 us); with 64-column strips
    // two workgroups share each line and the hint costs a second fetch
    // (k_proj M=16 5.5 -> 6.5 us), so those keep the default policy.
    constexpr int kWeightPolicy = CPL == 8 ? kStream : 0;
    const uint32_t ldp = (uint32_t)P.ldp;
    const __amdgpu_buffer_rsrc_t wrs = make_rsrc(P.packed, (uint32_t)((size_t)(P.K / 2) * P.ldp));
    const __amdgpu_buffer_rsrc_t srs = make_rsrc(P.scale, (uint32_t)((size_t)G * P.lds * 4));
    const uint32_t soff = (uint32_t)g * (uint32_t)P.lds * 4u;
#pragma unroll
    for (int t = 0; t < CPL; t += 4) {
      const f32x4_t v = __builtin_bit_cast(
          f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(srs, (uint32_t)(col0 + t) * 4u, soff, kWeightPolicy));
      d.s[t] = v[0]; d.s[t + 1] = v[1]; d.s[t + 2] = v[2]; d.s[t + 3] = v[3];
    }
    const uint32_t wvoff = (uint32_t)col0 + (uint32_t)(lk * 4) * ldp;
    const uint32_t gbase = (uint32_t)g * kPackedRowsPerGroup * ldp;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        buffer_load_bytes<CPL, kWeightPolicy>(wrs, wvoff, gbase + (uint32_t)(st * 16 + r) * ldp, d.raw[st][r]);
  } else {
    const bool vw = (P.vec & 1) != 0;
    load_scales<CPL, false>(P.scale + (int64_t)g * P.lds, col0, N, vw, d.s);
    const uint8_t* base = P.packed + (int64_t)g * kPackedRowsPerGroup * P.ldp;
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        load_packed<CPL, false>(base + (int64_t)(st * 16 + lk * 4 + r) * P.ldp, col0, N, vw, d.raw[st][r]);
  }
  // Everything above is in flight before the first MFMA below.
  __builtin_amdgcn_sched_barrier(0);
  decode_group<CPL, MT>(d, A, total);
}

// MULTI: the launch holds several problems.  A single-problem launch reads its
// table entry at fixed kernel-argument offsets, so every field arrives with one
// round of scalar loads instead of two dependent ones.  MROWS (1, 4, 8 or 16)
// bounds M for every problem of the launch.  MROWS == 1 (batch-1 decode)
// compiles the row loops and reductions to their one-row form, which measures
// ~0.4 us faster per launch; the bound also sizes the split-K finisher's
// per-thread polls (splitk_finish).  PAIR: the launch is a SwiGLU pair, gate
// (problem 0) and up (problem 1) of the same shape and activations; gate's
// workgroups publish every split and up's finisher stores silu(gate) * up.
template <int CPL, int WAVES, bool FULL, bool MULTI, int MROWS, bool PAIR = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_kernel(Launch L) {
  constexpr int WCOLS = 16 * CPL;
  constexpr int NT = WAVES * 64;
  extern __shared__ __attribute__((aligned(16))) float smem[];  // [WAVES][M][WCOLS] wave totals

  const int pi = MULTI ? problem_of(L, blockIdx.x) : 0;
  // The empty asm makes the pointer fields live here, so they are fetched in
  // the same round of scalar loads as the tiling fields instead of after it.
  const Problem P = L.p[pi];
  asm volatile("" ::"s"(P.x), "s"(P.packed), "s"(P.scale), "s"(P.ldx), "s"(P.ldp), "s"(P.lds));
  // Single-problem launches use a (strip, split) grid: no division in the
  // prologue, which every wave of a CU runs on the shared scalar unit.
  int strip, split;
  if constexpr (MULTI) {
    const uint32_t local = blockIdx.x - (uint32_t)P.wg_begin;
    strip = (int)(local % (uint32_t)P.tiles_n);
    split = (int)(local / (uint32_t)P.tiles_n);
  } else {
    strip = blockIdx.x;
    split = blockIdx.y;
  }

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int n0 = strip * WCOLS;
  const int col0 = n0 + lc * CPL;
  const int M = MROWS == 1 ? 1 : P.M, N = P.N;
  const int G = (uint32_t)P.K / kGroup;
  const int g = split * P.gps + wave;
  const bool active = wave < P.gps && g < G;  // wave-uniform

  constexpr int MT = (MROWS + 15) / 16;
  f32x4_t total[MT][CPL];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < CPL; ++t) total[mt][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if (active) decode_wave<CPL, FULL, MT>(P, g, col0, lc, lk, M, total);

  // Reduce the waves through LDS.  Rows m = 16*mt + 4*lk + r of the MFMA output.
  float* red = smem;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + lk * 4 + r;
      if (m < M) {
        float* dst = red + ((size_t)wave * M + m) * WCOLS + lc * CPL;
#pragma unroll
        for (int t = 0; t < CPL; t += 4)
          *reinterpret_cast<f32x4_t*>(dst + t) =
              f32x4_t{total[mt][t][r], total[mt][t + 1][r], total[mt][t + 2][r], total[mt][t + 3][r]};
      }
    }
  __syncthreads();
  const int elems = M * WCOLS;
  auto wave_sum = [&](int e) {
    float v = red[e];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[(size_t)w * elems + e];
    return v;
  };
  constexpr int EPT = (MROWS * WCOLS + NT - 1) / NT;
  if constexpr (PAIR) {
    if (pi == 0)
      splitk_finish<NT, EPT, kFinishGate>(L, P, M, split, n0, WCOLS, M, wave_sum);
    else
      splitk_finish<NT, EPT, kFinishUp>(L, P, M, split, n0, WCOLS, M, wave_sum, &L.p[0]);
    return;
  }
  if (P.nsplit == 1) {
    for (int e = threadIdx.x; e < elems; e += NT) {
      const int m = e / WCOLS, c = e % WCOLS, n = n0 + c;
      if (n < N) P.y[(int64_t)m * P.ldy + n] = f32_to_bf16(wave_sum(e));
    }
    return;
  }
  splitk_finish<NT, EPT, kFinishStore>(L, P, M, split, n0, WCOLS, M, wave_sum);
}

// ---------------------------------------------------------------------------
// Row sums for the gemm offset correction: rowsum[g*M + m] = 136 * sum_{k in g} x[m,k].
// 16 lanes per (row, group); each lane sums 8 values, then a butterfly over the
// 16 lanes (fixed order, deterministic).  Problems that share x share the sums.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void rowsum_kernel(Launch L) {
  int pi = 0;
  for (int i = 0; i < L.count; ++i)
    if (L.p[i].rs_begin >= 0 && (int)blockIdx.x >= L.p[i].rs_begin) pi = i;
  const Problem& P = L.p[pi];
  const int M = P.M;
  const int G = P.K / kGroup;
  const int64_t item = (int64_t)(blockIdx.x - P.rs_begin) * 16 + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const bool valid = item < (int64_t)M * G;
  const int m = valid ? (int)(item / G) : 0;
  const int g = valid ? (int)(item % G) : 0;
  float s = 0.f;
  if (valid) {
    const bf16x8_t v = load_x8(P.x + (int64_t)m * P.ldx + (int64_t)g * kGroup + sub * 8, (P.vec & 2) != 0);
    const u32x4_t w = __builtin_bit_cast(u32x4_t, v);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s += __uint_as_float(w[i] << 16);
      s += __uint_as_float(w[i] & 0xffff0000u);
    }
  }
#pragma unroll
  for (int off = 8; off >= 1; off >>= 1) s += __shfl_xor(s, off, 16);
  if (valid && sub == 0) P.rowsum[(int64_t)g * M + m] = kOffset * s;
}

// ---------------------------------------------------------------------------
// GEMM kernel (prefill-sized M).
//
// Workgroup tile 128 rows x 64*CPL columns, 4 waves side by side along N, each
// wave 128 x 16*CPL (8 M-subtiles x CPL MFMA column blocks, CPL columns per
// lane: 4 for wide problems, 2 to double the tile count of narrow ones).
// Per 128-row K group:
//  * the activation tile (128 x 128 bf16, 32 KB) is copied global -> LDS with
//    direct-to-LDS loads in MFMA fragment order (wave w copies K step w),
//    double buffered, together with the group's 128 row sums (rowsum_kernel);
//  * each wave loads its own packed weights (16 buffer loads of CPL bytes,
//    scalar row offsets) and scales one group ahead, in registers;
//  * running-ratio fold: the accumulator U is kept in units of the current
//    group's scale, U <- U * (s_prev / s) - 136 * rowsum, so a single fp32
//    accumulator set suffices and the MFMAs accumulate straight into it; the
//    output is U * s_last (see clamp_scale for zero / tiny scales).
// blockIdx -> (problem, K split, tile).  Tiles are handed out XCD-major:
// workgroup b runs on XCD b % 8 and each XCD receives a contiguous range of
// work ids, ordered within a problem in column bands of 4 row tiles, so the
// rows of x and the weight columns an XCD touches stay in its L2.  With K
// split, each split stores its fp32 partial tile (already scaled) and
// splitk_reduce_kernel, launched next on the same stream, sums the splits in
// split order.
// ---------------------------------------------------------------------------
constexpr int kGemmRows = 128;
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

// B fragments of one K step: raw[r] holds packed row r's CPL bytes.  For CPL=2
// two rows share a word (row 2j in the low half, row 2j+1 in the high half).
template <int CPL>
__device__ __forceinline__ void gemm_unpack(const uint32_t (&raw)[4], bf16x8_t (&B)[CPL]) {
  if constexpr (CPL == 4) {
    Prep p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = prep(raw[r]);
    B[0] = as_bf16x8(u32x4_t{pair_of<0>(p[0]), pair_of<0>(p[1]), pair_of<0>(p[2]), pair_of<0>(p[3])});
    B[1] = as_bf16x8(u32x4_t{pair_of<1>(p[0]), pair_of<1>(p[1]), pair_of<1>(p[2]), pair_of<1>(p[3])});
    B[2] = as_bf16x8(u32x4_t{pair_of<2>(p[0]), pair_of<2>(p[1]), pair_of<2>(p[2]), pair_of<2>(p[3])});
    B[3] = as_bf16x8(u32x4_t{pair_of<3>(p[0]), pair_of<3>(p[1]), pair_of<3>(p[2]), pair_of<3>(p[3])});
  } else {
    const Prep p01 = prep(raw[0] | (raw[1] << 16));
    const Prep p23 = prep(raw[2] | (raw[3] << 16));
    B[0] = as_bf16x8(u32x4_t{pair_of<0>(p01), pair_of<2>(p01), pair_of<0>(p23), pair_of<2>(p23)});
    B[1] = as_bf16x8(u32x4_t{pair_of<1>(p01), pair_of<3>(p01), pair_of<1>(p23), pair_of<3>(p23)});
  }
}

// PAIR: a SwiGLU gate/up pair (problem 0 gate, problem 1 up, same shape and
// activations) in one launch.  Tiles are 128 rows x 128 output columns: waves
// 0-1 compute the gate's 128 columns and waves 2-3 the up projection's, each
// as an ordinary 64-column wave sharing the workgroup's activation tile.  The
// up waves then hand their scaled fp32 tile to the gate waves through the idle
// activation buffers, and those store bf16(silu(g) * u) from the fp32 sums
// (engine/llama_mlp.py:30-32).  (Gate and up columns side by side within a
// lane, with 2-byte weight loads, measured 2.3x slower.)
template <int CPL, bool FULL, int KW, bool PAIR = false>
__global__ __launch_bounds__(256 * KW) __attribute__((amdgpu_waves_per_eu(2, 8))) void gemm_kernel(Launch L) {
  static_assert(!PAIR || (CPL == 4 && FULL && KW == 1), "the SwiGLU pair GEMM is one shape");
  constexpr int WCOLS = 16 * CPL;       // columns per wave
  constexpr int kATile = 4 * kGemmMT * 64;  // 16-byte entries of one activation tile
  // Two activation buffers [step][subtile][lane] (16 B each) and two row-sum
  // buffers per K half, as separate objects so that alias analysis can tell a
  // copy into one from a read of the other.
  __shared__ u32x4_t As0[KW * kATile], As1[KW * kATile];
  __shared__ __attribute__((aligned(16))) float Cs0[KW * kGemmRows], Cs1[KW * kGemmRows];
  auto a_buf = [&](auto tag) -> u32x4_t* {
    if constexpr (decltype(tag)::value == 0) return As0; else return As1;
  };
  auto c_buf = [&](auto tag) -> float* {
    if constexpr (decltype(tag)::value == 0) return Cs0; else return Cs1;
  };

  // ---- work assignment ----
  int wid = blockIdx.x;
  if ((gridDim.x & 7) == 0) {
    const int per_xcd = gridDim.x >> 3;
    wid = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  }
  if (wid >= L.total_wgs) return;
  const int pi = PAIR ? 0 : problem_of(L, wid);
  const Problem& P = L.p[pi];
  const Problem& Pw = PAIR ? L.p[__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 7))] : P;  // this wave's weights
  const int tiles = P.tiles_m * P.tiles_n;
  const int local = wid - P.wg_begin;
  const int split = local / tiles;
  const int tile_lin = local % tiles;
  const int band_size = kGemmBand * P.tiles_n;
  const int band = tile_lin / band_size;
  const int first_m = band * kGemmBand;
  const int band_rows = min(kGemmBand, P.tiles_m - first_m);
  const int in_band = tile_lin % band_size;
  const int m_tile = first_m + in_band % band_rows;
  const int n_tile = in_band / band_rows;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x & 255) >> 6);  // column block
  const int kw = KW == 1 ? 0 : __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8);  // K half
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int M = P.M, N = P.N;
  const int G = P.K / kGroup;
  const int g_begin = split * P.gps;
  const int g_end = min(G, g_begin + P.gps);
  const int m0 = m_tile * kGemmRows;
  // Output column of the lane's first block (a pair: waves w and w + 2 share columns).
  const int col0 = PAIR ? n_tile * 128 + (wave & 1) * WCOLS + lc * CPL : n_tile * 4 * WCOLS + wave * WCOLS + lc * CPL;

  // ---- operand sources ----
  const uint32_t ldp = (uint32_t)Pw.ldp;
  const __amdgpu_buffer_rsrc_t wrs = make_rsrc(Pw.packed, (uint32_t)((size_t)(P.K / 2) * Pw.ldp));
  const __amdgpu_buffer_rsrc_t srs = make_rsrc(Pw.scale, (uint32_t)((size_t)G * Pw.lds * 4));
  const uint32_t wvoff = (uint32_t)col0 + (uint32_t)(lk * 4) * ldp;
  const bool w_small = (size_t)(P.K / 2) * Pw.ldp <= 0x80000000ull;
  // Activations come through a buffer resource based at this tile's first
  // row and ending after its last row inside M, so every copy is one 32-bit
  // per-lane offset (row lc of subtile 0 plus 16 rows per subtile) and a
  // scalar group offset.  Rows past M fall outside the resource and read as
  // zero: they compute values that are never stored.
  const int tile_rows = min(kGemmRows, M - m0);
  const __amdgpu_buffer_rsrc_t xrs =
      make_rsrc(P.x + (int64_t)m0 * P.ldx, (uint32_t)((size_t)tile_rows * P.ldx * 2));
  const uint32_t xv0 = ((uint32_t)lc * (uint32_t)P.ldx + (uint32_t)((wave * 4 + lk) * 8)) * 2u;
  const uint32_t xsub = (uint32_t)P.ldx * 32u;  // bytes per 16-row subtile
  const __amdgpu_buffer_rsrc_t crs = make_rsrc(P.rowsum, (uint32_t)((size_t)G * M * 4));
  const uint32_t cv = (uint32_t)min(m0 + (int)(threadIdx.x & 127), M - 1) * 4u;

  auto stage_a = [&](int g, auto buf_tag) {
    u32x4_t* as = a_buf(buf_tag) + kw * kATile;
    float* cs = c_buf(buf_tag) + kw * kGemmRows;
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xrs, (void __attribute__((address_space(3)))*)&as[(wave * kGemmMT + i) * 64],
                                               16, xv0 + (uint32_t)i * xsub, (uint32_t)g * (kGroup * 2), 0, 0);
    if (wave < 2)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(crs, (void __attribute__((address_space(3)))*)&cs[wave * 64], 4, cv,
                                               (uint32_t)g * (uint32_t)M * 4u, 0, 0);
  };
  // Packed weights of K step st of group g: 4 packed rows x CPL bytes per lane.
  auto load_b_step = [&](int g, int st, uint32_t (&raw)[4], uint32_t wv) {
    if constexpr (FULL) {
      const uint32_t gbase = (uint32_t)g * kPackedRowsPerGroup * ldp;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t w[1];
        buffer_load_bytes<CPL>(wrs, wv, gbase + (uint32_t)(st * 16 + r) * ldp, w);
        raw[r] = w[0];
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t pr = (int64_t)g * kPackedRowsPerGroup + st * 16 + lk * 4 + r;
        uint32_t w[1];
        load_packed<CPL, false>(Pw.packed + pr * Pw.ldp, col0, N, (P.vec & 1) != 0, w);
        raw[r] = w[0];
      }
    }
  };
  auto load_scales_b = [&](int g, float (&s)[CPL]) {
    if constexpr (FULL) {
      const uint32_t soff = (uint32_t)g * (uint32_t)Pw.lds * 4u;
      if constexpr (CPL == 4) {
        const f32x4_t v =
            __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(srs, (uint32_t)col0 * 4u, soff, 0));
        s[0] = v[0]; s[1] = v[1]; s[2] = v[2]; s[3] = v[3];
      } else {
        const f32x2_t v =
            __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(srs, (uint32_t)col0 * 4u, soff, 0));
        s[0] = v[0]; s[1] = v[1];
      }
    } else {
      load_scales<CPL, false>(Pw.scale + (int64_t)g * Pw.lds, col0, N, (P.vec & 1) != 0, s);
    }
  };
  auto load_b = [&](int g, uint32_t (&raw)[4][4], float (&s)[CPL]) {
#pragma unroll
    for (int st = 0; st < 4; ++st) load_b_step(g, st, raw[st], wvoff);
    load_scales_b(g, s);
  };

  f32x4_t U[kGemmMT][CPL];
#pragma unroll
  for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
    for (int t = 0; t < CPL; ++t) U[i][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Packed weights (4 K steps) and scales.  FULL tiles stream the weights
  // through one register set: right after step st of a group is unpacked, the
  // same registers receive step st of the next group, a whole group ahead of
  // its use.  That keeps 16 VGPRs free for deeper activation prefetch.  Other
  // tiles (whose loads are not one instruction per row) hold two sets: the
  // group computed from set BUF while the next one loads into set BUF ^ 1.
  // Scales always use two sets.  With KW == 2 the two K halves of the
  // workgroup (waves 0-3 and 4-7) take alternate groups of the range, each
  // with its own LDS buffers, and are summed through LDS at the end.
  constexpr bool kStreamB = FULL;
  // Vector memory operations issued after a group's activation copies: the
  // next group's scale load and 16 weight loads.
  constexpr int kLoadsAfterA = 1 + 16;
  uint32_t raw2[kStreamB ? 1 : 2][4][4];
  float s2[2][CPL];
  float s_ref[CPL];  // scale U is currently expressed in (per column)
  const int g_first = g_begin + kw;
  const int n_iter = (g_end - g_begin + KW - 1) / KW;  // iterations of every K half (barrier count)
#pragma unroll
  for (int t = 0; t < CPL; ++t) s_ref[t] = 1.f;
  if (g_first < g_end) {
    if constexpr (kStreamB) {
      stage_a(g_first, std::integral_constant<int, 0>{});
      __builtin_amdgcn_sched_barrier(0);
      load_scales_b(g_first, s2[0]);
#pragma unroll
      for (int st = 0; st < 4; ++st) load_b_step(g_first, st, raw2[0][st], wvoff);
    } else {
      load_b(g_first, raw2[0], s2[0]);
      stage_a(g_first, std::integral_constant<int, 0>{});
    }
  }
  if (g_first < g_end) {
#pragma unroll
    for (int t = 0; t < CPL; ++t) s_ref[t] = clamp_scale(s2[0][t]);
  }

  // One group.  BUF is the LDS buffer holding this group's activations; the
  // next group is staged into the other one.  BUF is a compile-time constant
  // (the loop below is unrolled by two) so that the compiler can tell the
  // direct-to-LDS copies into buffer BUF ^ 1 from the reads of buffer BUF:
  // with a run-time index it must assume they alias and waits for the copies
  // (vmcnt(0)) before the first LDS read, which serializes the prefetch.
  auto group = [&](auto buf_tag, int it) {
    constexpr int b = decltype(buf_tag)::value;
    const int g = g_first + it * KW;
    const u32x4_t* as = a_buf(buf_tag) + kw * kATile;
    const float* cs = c_buf(buf_tag) + kw * kGemmRows;
    uint32_t (&raw)[4][4] = raw2[kStreamB ? 0 : b];
    const float (&s)[CPL] = s2[b];
    // Direct-to-LDS copies of this group (issued one iteration earlier) must
    // have landed before the barrier publishes them.  When the weights stream,
    // only the loads issued after those copies may still be in flight.
    if constexpr (kStreamB)
      wait_vmem_n<kLoadsAfterA>();
    else
      wait_vmem();
    __syncthreads();
    if (g >= g_end) return;  // the K half with one group less: barriers only

    const bool has_next = g + KW < g_end;
    // After the last group the streamed loads have nothing to fetch: they go
    // to offset 2^31, past the weights' resource, and read zero without a
    // memory access (a resource over more than 2 GB re-reads this group).
    const int g_next = has_next ? g + KW : g;
    const uint32_t wv_next = (has_next || !w_small) ? wvoff : 0x80000000u;
    if (has_next) {
      stage_a(g + KW, std::integral_constant<int, b ^ 1>{});
      if constexpr (kStreamB) {
        __builtin_amdgcn_sched_barrier(0);  // the copies stay ahead of the loads counted above
        load_scales_b(g + KW, s2[b ^ 1]);
      } else {
        load_b(g + KW, raw2[b ^ 1], s2[b ^ 1]);
      }
    }

    // Fold: U <- U * (s_ref / s) - 136 * rowsum.  (U is zero before the first
    // group, so its ratio only has to be finite.)  s_ref / s uses the hardware
    // reciprocal: relative error ~1 ulp, the order of the fold's own rounding.
    // With 128-column tiles (CPL 2) the fold runs as one block before the
    // group's MFMAs; with 256-column tiles it is applied to each accumulator
    // right before its first MFMA of the group (each measured faster for its
    // tile width on MI355X).
    float rho[CPL];
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const float sc = clamp_scale(s[t]);
      rho[t] = s_ref[t] * __builtin_amdgcn_rcpf(sc);
      s_ref[t] = sc;
    }
    constexpr bool kFoldBlock = CPL == 2;
    if constexpr (kFoldBlock) {
#pragma unroll
      for (int i = 0; i < kGemmMT; ++i) {
        const f32x4_t c4 = *reinterpret_cast<const f32x4_t*>(&cs[16 * i + 4 * lk]);
#pragma unroll
        for (int t = 0; t < CPL; ++t)
#pragma unroll
          for (int r = 0; r < 4; ++r) U[i][t][r] = __builtin_fmaf(U[i][t][r], rho[t], -c4[r]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // With 128-column tiles each K step runs at raised wave priority, so the
    // two waves sharing a SIMD fall into alternating unpack / MFMA phases
    // (measured +10% at M = 2048 on q/o/down; no gain with 256-column tiles).
    constexpr bool kStepPrio = CPL == 2;
    // Activation fragments go through LDS reads one subtile pair ahead of
    // their MFMAs (pair q = subtiles 2(q%4), 2(q%4)+1 of step q/4), so four
    // fragments are in flight and each read has a pair's MFMAs to land.
    // The fences (an empty asm statement for the IR passes, a scheduling
    // barrier that only VALU and SALU work may cross) keep that order:
    // without them the compiler sinks every read next to its first use (two
    // fragments in flight, the wait on the LDS read exposed before every 8
    // MFMAs).
    constexpr int kPairs = 4 * kGemmMT / 2;
    constexpr int kAhead = 1;  // pairs read ahead (2 measured the same, 3 spills)
    bf16x8_t A[kAhead + 1][2];
    f32x4_t c4[kAhead + 1][2];
    auto read_pair = [&](int q, bf16x8_t (&a)[2], f32x4_t (&c)[2]) {
      const int st = q / (kGemmMT / 2);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int i = 2 * (q % (kGemmMT / 2)) + j;
        a[j] = __builtin_bit_cast(bf16x8_t, as[(st * kGemmMT + i) * 64 + lane]);
        if (!kFoldBlock && st == 0) c[j] = *reinterpret_cast<const f32x4_t*>(&cs[16 * i + 4 * lk]);
      }
    };
#pragma unroll
    for (int q = 0; q < kAhead; ++q) read_pair(q, A[q], c4[q]);
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      if constexpr (kStepPrio) __builtin_amdgcn_s_setprio(1);
      bf16x8_t B[CPL];
      gemm_unpack<CPL>(raw[st], B);
      // Unconditional (a branch here splits the step and stops the unpack from
      // interleaving with the MFMAs).
      // The scheduling barrier keeps the loads here (a group ahead of their
      // use) while every other kind of instruction may still move across it.
      if constexpr (kStreamB) {
        load_b_step(g_next, st, raw[st], wv_next);
        asm volatile("" ::: "memory");  // no IR pass sinks them either
        __builtin_amdgcn_sched_barrier(0x38F);
      }
#pragma unroll
      for (int pp = 0; pp < kGemmMT / 2; ++pp) {
        const int q = st * (kGemmMT / 2) + pp;
        if (q + kAhead < kPairs) read_pair(q + kAhead, A[(q + kAhead) % (kAhead + 1)], c4[(q + kAhead) % (kAhead + 1)]);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0x6);  // only VALU / SALU work (the unpack) may cross
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = 2 * pp + j;
#pragma unroll
          for (int t = 0; t < CPL; ++t) {
            if (!kFoldBlock && st == 0) {
#pragma unroll
              for (int r = 0; r < 4; ++r) U[i][t][r] = __builtin_fmaf(U[i][t][r], rho[t], -c4[q % (kAhead + 1)][j][r]);
            }
            U[i][t] = mfma16(A[q % (kAhead + 1)][j], B[t], U[i][t]);
          }
        }
      }
      if constexpr (kStepPrio) __builtin_amdgcn_s_setprio(0);
    }
  };
  for (int it = 0; it < n_iter; it += 2) {
    group(std::integral_constant<int, 0>{}, it);
    if (it + 1 < n_iter) group(std::integral_constant<int, 1>{}, it + 1);
  }

  if constexpr (KW == 2) {
    // K half 1 hands its scaled tile to half 0 through the (now idle)
    // activation buffers: subtiles 0-3 in As0, 4-7 in As1, fragment order.
    __syncthreads();
    if (kw == 1) {
#pragma unroll
      for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
          f32x4_t v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = U[i][t][r] * s_ref[t];
          u32x4_t* dst = i < kGemmMT / 2 ? As0 : As1;
          dst[((wave * (kGemmMT / 2) + (i % (kGemmMT / 2))) * CPL + t) * 64 + lane] = __builtin_bit_cast(u32x4_t, v);
        }
    }
    __syncthreads();
    if (kw == 1) return;
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
      for (int t = 0; t < CPL; ++t) {
        const u32x4_t* src = i < kGemmMT / 2 ? As0 : As1;
        const f32x4_t o = __builtin_bit_cast(
            f32x4_t, src[((wave * (kGemmMT / 2) + (i % (kGemmMT / 2))) * CPL + t) * 64 + lane]);
#pragma unroll
        for (int r = 0; r < 4; ++r) U[i][t][r] = __builtin_fmaf(U[i][t][r], s_ref[t], o[r]);
      }
#pragma unroll
    for (int t = 0; t < CPL; ++t) s_ref[t] = 1.f;
  }

  // ---- output: lane holds rows m0 + 16i + 4lk + r, columns col0 .. col0+CPL-1 ----
  if constexpr (PAIR) {
    // Up waves (2, 3) hand their scaled tile to the gate waves (0, 1) through
    // the activation buffers: subtiles 0-3 in As0, 4-7 in As1, fragment order.
    __syncthreads();  // every wave is past its last read of the activation tiles
    const int half = wave & 1;
    if (wave >= 2) {
#pragma unroll
      for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
        for (int t = 0; t < CPL; ++t) {
          f32x4_t v;
#pragma unroll
          for (int r = 0; r < 4; ++r) v[r] = U[i][t][r] * s_ref[t];
          u32x4_t* dst = i < kGemmMT / 2 ? As0 : As1;
          dst[((half * (kGemmMT / 2) + (i % (kGemmMT / 2))) * CPL + t) * 64 + lane] = __builtin_bit_cast(u32x4_t, v);
        }
    }
    __syncthreads();
    if (wave >= 2) return;
    // h[m, col0 .. col0 + 3] = bf16(silu(g) * u); y rows are 8-byte aligned (pair_gemm_ok).
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i) {
      f32x4_t u[CPL];
#pragma unroll
      for (int t = 0; t < CPL; ++t) {
        const u32x4_t* src = i < kGemmMT / 2 ? As0 : As1;
        u[t] = __builtin_bit_cast(f32x4_t, src[((half * (kGemmMT / 2) + (i % (kGemmMT / 2))) * CPL + t) * 64 + lane]);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * i + 4 * lk + r;
        if (m >= M) continue;
        float h[CPL];
#pragma unroll
        for (int t = 0; t < CPL; ++t) h[t] = silu(U[i][t][r] * s_ref[t]) * u[t][r];
        *reinterpret_cast<u32x2_t*>(P.y + (int64_t)m * P.ldy + col0) = u32x2_t{bf16x2_rne(h[0], h[1]), bf16x2_rne(h[2], h[3])};
      }
    }
    return;
  }
  if (P.nsplit == 1 && FULL && m0 + kGemmRows <= M && (P.vec & 4) != 0 &&
      (size_t)kGemmRows * P.ldy * 2 < 0xffffffffull) {
    // Whole tile in range: buffer stores off a resource at the tile's first
    // row, the lane's column offset in a VGPR and the row offset as a scalar,
    // so the stores need no per-row address arithmetic or bounds checks.
    const uint32_t ldy2 = (uint32_t)P.ldy * 2u;
    const __amdgpu_buffer_rsrc_t yrs = make_rsrc(P.y + (int64_t)m0 * P.ldy, kGemmRows * ldy2);
    const uint32_t yv = (uint32_t)(4 * lk) * ldy2 + (uint32_t)col0 * 2u;
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        uint32_t h2[CPL / 2];
#pragma unroll
        for (int t = 0; t < CPL; t += 2) h2[t / 2] = bf16x2_rne(U[i][t][r] * s_ref[t], U[i][t + 1][r] * s_ref[t + 1]);
        const uint32_t so = (uint32_t)(16 * i + r) * ldy2;
        if constexpr (CPL == 4)
          __builtin_amdgcn_raw_buffer_store_b64(u32x2_t{h2[0], h2[1]}, yrs, yv, so, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b32(h2[0], yrs, yv, so, 0);
      }
    return;
  }
  if (P.nsplit == 1) {
    const bool vec_y = FULL ? (P.vec & 4) != 0 : ((P.vec & 4) != 0 && col0 + CPL <= N);
#pragma unroll
    for (int i = 0; i < kGemmMT; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * i + 4 * lk + r;
        if (m >= M) continue;
        uint16_t* dst = P.y + (int64_t)m * P.ldy + col0;
        // Column pairs through the hardware packed conversion (one VALU op per two outputs).
        uint32_t h2[CPL / 2];
#pragma unroll
        for (int t = 0; t < CPL; t += 2) h2[t / 2] = bf16x2_rne(U[i][t][r] * s_ref[t], U[i][t + 1][r] * s_ref[t + 1]);
        if (vec_y) {
          if constexpr (CPL == 4)
            *reinterpret_cast<u32x2_t*>(dst) = u32x2_t{h2[0], h2[1]};
          else
            *reinterpret_cast<uint32_t*>(dst) = h2[0];
        } else {
#pragma unroll
          for (int t = 0; t < CPL; ++t)
            if (col0 + t < N) dst[t] = (uint16_t)(h2[t / 2] >> (16 * (t & 1)));
        }
      }
    return;
  }

  // ---- K split: store this split's fp32 tile (already scaled); splitk_reduce_kernel
  // sums the splits in order in the next launch ----
  float* part = P.part + (size_t)split * M * N;
#pragma unroll
  for (int i = 0; i < kGemmMT; ++i) {
    if (m0 + 16 * i >= M) break;  // wave-uniform: the rest of the tile is past M
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 16 * i + 4 * lk + r;
      if (m >= M) continue;
      float* dst = part + (size_t)m * N + col0;
      float v[CPL];
#pragma unroll
      for (int t = 0; t < CPL; ++t) v[t] = U[i][t][r] * s_ref[t];
      if (FULL) {
        if constexpr (CPL == 4)
          *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{v[0], v[1], v[2], v[3]};
        else
          *reinterpret_cast<f32x2_t*>(dst) = f32x2_t{v[0], v[1]};
      } else {
#pragma unroll
        for (int t = 0; t < CPL; ++t)
          if (col0 + t < N) dst[t] = v[t];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split-K reduction of the GEMM: y = bf16(sum over splits, in split order, of
// part[split]).  Four consecutive elements of the dense [M, N] partial per
// thread; grid = sum of red_wgs over the split problems of the launch.
// ---------------------------------------------------------------------------
constexpr int kReduceElems = 4 * 256;  // elements per workgroup

__global__ __launch_bounds__(256) void splitk_reduce_kernel(Launch L) {
  const int wg = blockIdx.x;
  int pi = 0;
  for (int i = 1; i < L.count; ++i)
    if (wg >= L.p[i].red_begin) pi = i;
  const Problem& P = L.p[pi];
  const int M = P.M, N = P.N;
  const int64_t total = (int64_t)M * N;
  const int64_t e0 = (int64_t)(wg - P.red_begin) * kReduceElems + 4 * threadIdx.x;
  if (e0 >= total) return;
  const size_t stride = (size_t)total;
  if ((N & 3) == 0 && (P.vec & 4)) {
    // Four elements in one row: 16-byte loads, one 8-byte store.
    const float* src = P.part + e0;
    f32x4_t acc = *reinterpret_cast<const f32x4_t*>(src);
    for (int sp = 1; sp < P.nsplit; ++sp) acc += *reinterpret_cast<const f32x4_t*>(src + sp * stride);
    const int64_t m = e0 / N, n = e0 % N;
    *reinterpret_cast<u32x2_t*>(P.y + m * P.ldy + n) =
        u32x2_t{(uint32_t)f32_to_bf16(acc[0]) | ((uint32_t)f32_to_bf16(acc[1]) << 16),
                (uint32_t)f32_to_bf16(acc[2]) | ((uint32_t)f32_to_bf16(acc[3]) << 16)};
  } else {
    for (int j = 0; j < 4; ++j) {
      const int64_t e = e0 + j;
      if (e >= total) break;
      float acc = P.part[e];
      for (int sp = 1; sp < P.nsplit; ++sp) acc += P.part[e + sp * stride];
      P.y[(e / N) * P.ldy + e % N] = f32_to_bf16(acc);
    }
  }
}

// ---------------------------------------------------------------------------
// Dense bf16 GEMV for the output projection (M <= 16):
// y[m, n] = sum_k x[m, k] * w[n, k], w in Linear layout [N, K] (row n is the
// weight vector of output n, contiguous along K), as
// `logits = x @ lm_head.T` (engine/llama_model.py:148).
//
// A wave owns 16 consecutive rows of w and streams them over the whole of K,
// so no partial leaves the wave.  Per 64-element K chunk a lane issues two
// 16-byte buffer loads of its row: lane l covers row n0 + l % 16 and bytes
// 16 * (l / 16) of each 64-byte half, so the 4 lanes of a row read 128
// contiguous bytes and each 16-byte load is one bf16 B fragment of
// v_mfma_f32_16x16x32_bf16 as loaded.  kDenseChunks chunks are in flight per
// lane, double buffered.  x[0:M, :] is staged in LDS with a zero row M for
// the MFMA rows past M.  Rows past N lie outside the wave's buffer resource
// and read as zero; they are never stored.
// ---------------------------------------------------------------------------
constexpr int kDenseChunks = 4;  // 64-element K chunks per pipeline stage

template <bool FULL>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8))) void bf16_gemv_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ w, int64_t ldw,
    uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xsd[];
  const int kpitch = K + 72;
  {
    const int chunks = K / 8;
    for (int i = threadIdx.x; i < M * chunks; i += 256) {
      const int m = i / chunks, c = i % chunks;
      *reinterpret_cast<u32x4_t*>(xsd + m * kpitch + c * 8) =
          __builtin_bit_cast(u32x4_t, load_x8(x + (int64_t)m * ldx + c * 8, true));
    }
    if (M < 16)
      for (int c = threadIdx.x; c < chunks; c += 256)
        *reinterpret_cast<u32x4_t*>(xsd + M * kpitch + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lc = lane & 15;
  const int lk = lane >> 4;
  const int n0 = (blockIdx.x * 4 + wave) * 16;
  if (n0 >= N) return;
  const int rows = min(16, N - n0);
  const uint32_t nrec = (uint32_t)((size_t)rows * ldw * 2);
  const __amdgpu_buffer_rsrc_t rs = make_rsrc(w + (int64_t)n0 * ldw, nrec);
  const uint32_t voff = (uint32_t)((size_t)lc * ldw * 2) + (uint32_t)lk * 16u;
  const uint16_t* xrow = xsd + (lc < M ? lc : M) * kpitch + lk * 8;

  u32x4_t buf[2][kDenseChunks][2];
  auto load_stage = [&](u32x4_t (&b)[kDenseChunks][2], int kc) {
#pragma unroll
    for (int c = 0; c < kDenseChunks; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kc + c * 64 + h * 32;  // first element of this lane group's 32-element block
        // Past K the lane's offset starts at the end of the resource, which reads as zero.
        const uint32_t v = (FULL || k + lk * 8 < K) ? voff : nrec;
        b[c][h] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, v, (uint32_t)(k * 2), 0));
      }
  };
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  auto compute_stage = [&](const u32x4_t (&b)[kDenseChunks][2], int kc) {
#pragma unroll
    for (int c = 0; c < kDenseChunks; ++c)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int k = kc + c * 64 + h * 32;
        // K is a multiple of 8, so each lane's 8-element block is wholly inside K
        // or past it; the LDS rows have 64 elements of slack for the read.
        u32x4_t a = *reinterpret_cast<const u32x4_t*>(xrow + k);
        if (!FULL) a = (k + lk * 8 < K) ? a : u32x4_t{0u, 0u, 0u, 0u};
        acc = mfma16(as_bf16x8(a), as_bf16x8(b[c][h]), acc);
      }
  };
  constexpr int kStage = 64 * kDenseChunks;
  int kc = 0;
  load_stage(buf[0], 0);
  if (kStage < K) load_stage(buf[1], kStage);
  for (;;) {
    compute_stage(buf[0], kc);
    kc += kStage;
    if (kc >= K) break;
    if (kc + kStage < K) load_stage(buf[0], kc + kStage);
    compute_stage(buf[1], kc);
    kc += kStage;
    if (kc >= K) break;
    if (kc + kStage < K) load_stage(buf[1], kc + kStage);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = lk * 4 + r;
    if (m < M && lc < rows) y[(int64_t)m * ldy + n0 + lc] = f32_to_bf16(acc[r]);
  }
}

// ---------------------------------------------------------------------------
// Dense bf16 GEMV for M <= 4 (the logits of decode steps), as bf16_gemv_kernel
// computes it but with the weight rows read as whole 1 KB pieces: a wave reads
// two rows of w at a time, each as 16-byte loads of 64 consecutive lanes (512
// elements per load), the pattern a flat streaming read uses, and multiplies
// with packed bf16 dot products (v_dot2c_f32_bf16, fp32 accumulation).  The
// 16-row MFMA layout reads 16 rows x 64 B per load instead, which measured
// ~5 TB/s against 1.24 GB of Qwen3-8B lm_head weights.  x[0:M, :] sits in LDS,
// zero-padded to whole 512-element segments; segments past K lie outside each
// row's buffer resource and read as zero.  Workgroups stride over row pairs,
// and each lane's partial dot products are reduced across the wave with a
// fixed butterfly, so results are deterministic.
// ---------------------------------------------------------------------------
constexpr int kRowSegs = 8;          // 512-element segments per row in flight per load round
constexpr int kRowsGrid = 1024;      // workgroups of the row kernel (4 per CU)

// The dot-product builtin takes bf16 pairs as 2 x 16-bit integer vectors (bit patterns).
typedef short bf16x2v_t __attribute__((ext_vector_type(2)));

template <int MR>
__global__ __launch_bounds__(256) void bf16_gemv_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const uint16_t* __restrict__ w, int64_t ldw,
                                                             uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                             int K) {
  extern __shared__ __attribute__((aligned(16))) uint16_t xsr[];  // [M][Kp] bf16
  const int nseg = (K + 511) / 512;
  const int kp = nseg * 512;
  for (int i = threadIdx.x; i < M * (kp / 8); i += 256) {
    const int m = i / (kp / 8), c = (i % (kp / 8)) * 8;
    *reinterpret_cast<u32x4_t*>(xsr + m * kp + c) =
        c < K ? __builtin_bit_cast(u32x4_t, load_x8(x + (int64_t)m * ldx + c, true)) : u32x4_t{0u, 0u, 0u, 0u};
  }
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int gw = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int nw = gridDim.x * 4;
  const uint32_t rowb = (uint32_t)K * 2u;
  for (int r0 = 2 * gw; r0 < N; r0 += 2 * nw) {
    const __amdgpu_buffer_rsrc_t rs0 = make_rsrc(w + (int64_t)r0 * ldw, rowb);
    const __amdgpu_buffer_rsrc_t rs1 = make_rsrc(w + (int64_t)(r0 + 1) * ldw, r0 + 1 < N ? rowb : 0u);
    float acc[MR][2];
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[m][0] = acc[m][1] = 0.f;
    for (int s0 = 0; s0 < nseg; s0 += kRowSegs) {
      u32x4_t wv[2][kRowSegs];
#pragma unroll
      for (int sg = 0; sg < kRowSegs; ++sg) {
        const uint32_t off = ((uint32_t)(s0 + sg) * 512u + (uint32_t)lane * 8u) * 2u;  // past K: zeros
        // Read-once weights: non-temporal (Qwen3-8B lm_head M=1 226 -> 199 us).
        wv[0][sg] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs0, off, 0, kStream));
        wv[1][sg] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs1, off, 0, kStream));
      }
      __builtin_amdgcn_sched_barrier(0);  // all 16 loads in flight before the first dot product
#pragma unroll
      for (int sg = 0; sg < kRowSegs; ++sg) {
        if (s0 + sg >= nseg) break;  // wave-uniform
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (m >= M) break;
          const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(xsr + m * kp + (s0 + sg) * 512 + lane * 8);
#pragma unroll
          for (int rr = 0; rr < 2; ++rr)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              // Copy the vector elements to scalars first: a bit cast of a
              // vector element (v[q]) compiles to element 0 for every q here.
              const uint32_t wq = wv[rr][sg][q], xq = xv[q];
              acc[m][rr] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v_t, wq),
                                                            __builtin_bit_cast(bf16x2v_t, xq), acc[m][rr], false);
            }
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) acc[m][rr] += __shfl_xor(acc[m][rr], o, 64);
    if (lane == 0)
      for (int m = 0; m < M && m < MR; ++m) {
        y[(int64_t)m * ldy + r0] = f32_to_bf16(acc[m][0]);
        if (r0 + 1 < N) y[(int64_t)m * ldy + r0 + 1] = f32_to_bf16(acc[m][1]);
      }
  }
}

// ---------------------------------------------------------------------------
// Dequantize: out[k, n] = q[k, n] * s[k/g, n] (engine/kernels/quant.py:122-156).
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
  const uint8_t byte = packed[(int64_t)i * ldp + n];
  const int q_even = (int8_t)byte >> 4;                  // arithmetic shift: [-8, 7]
  const int q_odd = (int8_t)(uint8_t)(byte << 4) >> 4;   // low nibble moved up, shifted back
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

// h = bf16(silu(h) * u) elementwise: the SwiGLU epilogue after separate gate
// (written to h) and up (u, contiguous [M, N]) projections.
__global__ __launch_bounds__(256) void silu_mul_kernel(uint16_t* __restrict__ h, int64_t ldh,
                                                       const uint16_t* __restrict__ u, int M, int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)M * N) return;
  const int64_t m = i / N, n = i % N;
  uint16_t* d = h + m * ldh + n;
  *d = f32_to_bf16(silu(bf16_to_f32(*d)) * bf16_to_f32(u[i]));
}

// ---------------------------------------------------------------------------
// Host-side planning.
// ---------------------------------------------------------------------------
enum Kind { kGemv = 0, kGemm = 1 };

inline int ceil_div(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }
inline size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
bool aligned(const void* p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

struct Plan {
  Kind kind;
  int cpl;
  int waves;           // gemv: waves per workgroup (4 or 8)
  int kw;              // gemm: K halves per workgroup (1, or 2 with 8 waves)
  bool full;           // every problem takes the unconditional (aligned, full tile) load path
  bool pair;           // SwiGLU pair (gemv only): problem 0 gate, problem 1 up
  size_t skip;         // bytes at the start of the upper workspace half reserved by the caller
  size_t lds_bytes;    // dynamic LDS (gemv)
  size_t ws_bytes;     // bytes of the plan's workspace half (see bind())
  bool too_large;      // gemv: a problem's split-K slots exceed the finish's 32-bit byte offsets
  int total_wgs;
  int rs_wgs;          // rowsum_kernel workgroups
  int red_wgs;         // splitk_reduce_kernel workgroups (gemm with split K)
  Launch L;            // device table (workspace pointers filled in by bind())
  size_t part_off[kMaxProblems], rowsum_off[kMaxProblems];
  int rowsum_src[kMaxProblems];  // problem whose row sums this one uses
};

// Validate one problem; returns a W4A16 status.
int check_problem(const w4a16_problem& q) {
  if (q.M < 0 || q.N < 0 || q.K < 0) return W4A16_ERR_SHAPE;
  if (q.K % kGroup != 0) return W4A16_ERR_K_GROUP;
  if (q.M == 0 || q.N == 0) return W4A16_OK;
  if (!q.y) return W4A16_ERR_NULL;
  if (q.K > 0 && (!q.x || !q.packed || !q.scale)) return W4A16_ERR_NULL;
  if (q.ldy < q.N || (q.K > 0 && (q.ldx < q.K || q.ldp < q.N || q.lds < q.N))) return W4A16_ERR_SHAPE;
  return W4A16_OK;
}

bool gemm_x_ok(const w4a16_problem& q) { return aligned(q.x, 16) && q.ldx % 8 == 0; }

// Kernel family of a problem.  M <= 32: decode kernel.  32 < M <= 64: the
// decode kernel as well (four M subtiles, one 8-wave workgroup per CU) when it
// launches at most 1024 workgroups, the GEMM otherwise (measured at M = 40
// and 64: Qwen3-8B q/k 1.6-1.8x faster than the GEMM, gate/down within 10%,
// Qwen3-32B gate/down 1.2-1.7x slower).
inline Kind kind_of(const w4a16_problem& q) {
  if (q.M <= 32) return kGemv;
  if (q.M > 64) return kGemm;
  const int64_t wgs = (int64_t)ceil_div(q.N, 64) * ceil_div(q.K / kGroup, 8);
  return wgs <= 1024 ? kGemv : kGemm;
}

// Plan one launch over problems that all have M > 0, N > 0, K > 0 and the
// same kind (kind_of).
Plan make_plan(const w4a16_problem* probs, int count, bool pair = false) {
  Plan pl{};
  pl.pair = pair;
  pl.L.count = count;
  int max_m = 0;
  for (int i = 0; i < count; ++i) max_m = std::max(max_m, probs[i].M);
  pl.kind = kind_of(probs[0]);
  bool full = true;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = probs[i];
    Problem& P = pl.L.p[i];
    P.x = static_cast<const uint16_t*>(q.x);
    P.ldx = q.ldx;
    P.packed = reinterpret_cast<const uint8_t*>(q.packed);
    P.ldp = q.ldp;
    P.scale = q.scale;
    P.lds = q.lds;
    P.y = static_cast<uint16_t*>(q.y);
    P.ldy = q.ldy;
    P.M = q.M;
    P.N = q.N;
    P.K = q.K;
    const bool vw = aligned(q.packed, 16) && q.ldp % 16 == 0 && aligned(q.scale, 16) && q.lds % 4 == 0;
    const bool vx = aligned(q.x, 16) && q.ldx % 8 == 0;
    const bool vy = aligned(q.y, 8) && q.ldy % 4 == 0;
    P.vec = (vw ? 1 : 0) | (vx ? 2 : 0) | (vy ? 4 : 0);
    P.rs_begin = -1;
    pl.rowsum_src[i] = i;
  }

  size_t ws = 0;
  if (pl.kind == kGemv) {
    // Decode shape choice (measured over the Qwen3-8B / 32B projections at
    // M = 1..32 on MI355X):
    //  * 128-column strips (CPL 8), or 64-column strips (CPL 4) when N is not
    //    a multiple of 128, when 128-column strips would give the launch fewer
    //    than 128 workgroups (k/v projections: more, smaller workgroups), or
    //    when M > 16 (two M subtiles: 103 instead of 140 VGPRs per lane);
    //  * 4 waves per workgroup (one 128-row group each), or 8 when M >= 8,
    //    when 4 would launch more than 1000 workgroups, or, with M >= 2, split
    //    K more than 20 ways: past that, reducing inside the workgroup beats
    //    more splits (Qwen3-8B down at M = 2 / 4: 10.2 / 10.6 -> 9.4 / 9.7 us;
    //    at M = 1 the 24 splits of 4 waves are faster, 9.07 -> 8.90 us);
    //    and 8 when K has 5..8 groups, so one workgroup covers K and there is
    //    no split-K finish (Qwen3-0.6B gate at M = 1: 3.9 -> 3.4 us).
    int max_m = 0, wg8 = 0, max_split4 = 0, n_odd = 0;
    for (int i = 0; i < count; ++i) {
      const int G = probs[i].K / kGroup;
      max_m = std::max(max_m, probs[i].M);
      wg8 += ceil_div(probs[i].N, 128) * ceil_div(G, 4);
      max_split4 = std::max(max_split4, ceil_div(G, 4));
      n_odd += probs[i].N % 128 != 0;
    }
    const int cpl = (n_odd > 0 || wg8 < 128 || max_m > 16) ? 4 : 8;
    pl.cpl = cpl;
    const int wcols = 16 * cpl;
    int wg4 = 0;
    for (int i = 0; i < count; ++i) wg4 += ceil_div(probs[i].N, wcols) * ceil_div(probs[i].K / kGroup, 4);
    pl.waves = (max_m >= 8 || wg4 > 1000 || (max_split4 > 20 && max_m >= 2) || max_split4 == 2) ? 8 : 4;
    int wg = 0;
    size_t lds = 0;
    for (int i = 0; i < count; ++i) {
      Problem& P = pl.L.p[i];
      const int G = P.K / kGroup;
      const int M = P.M;
      P.tiles_m = 1;
      P.tiles_n = ceil_div(P.N, wcols);
      P.gps = pl.waves;  // one 128-row group per wave
      P.nsplit = ceil_div(G, P.gps);
      lds = std::max(lds, (size_t)pl.waves * M * wcols * 4);
      P.wg_begin = wg;
      wg += P.tiles_n * P.nsplit;
      const size_t wbytes = (size_t)(P.K / 2) * P.ldp, sbytes = (size_t)G * P.lds * 4;
      const size_t xbytes = (size_t)P.ldx * 2 * M;
      full = full && (P.vec & 1) && (P.vec & 2) && P.N % wcols == 0 && wbytes < 0xffffffffull &&
             sbytes < 0xffffffffull && xbytes < 0x80000000ull;  // x: rows past M read at offset 2^31
      // Published slots: nsplit - 1 per strip (the last split finishes), all
      // nsplit for the gate of a pair (up's finisher reads them).
      const int nslots = pair && i == 0 ? P.nsplit : P.nsplit - 1;
      if (nslots > 0) {
        pl.part_off[i] = ws;
        ws = align256(ws + (size_t)nslots * M * P.N * 4);
        if ((size_t)P.nsplit * M * P.N * 4 >= 0xffffffffull) pl.too_large = true;
      }
    }
    pl.lds_bytes = lds;
    pl.total_wgs = wg;
  } else {
    // GEMM tile choice (measured on the Qwen3-8B / 32B shapes at M = 2048):
    //  * 128 x 256 tiles when there are at least 192 of them, else 128 x 128
    //    tiles with K split across workgroups;
    //  * with at most 256 such tiles (one per CU), 8-wave workgroups whose two
    //    K halves run side by side (KW 2): the CU still holds two waves per
    //    SIMD (q/o 92.7 -> 77 us, down 266 -> 208 us); above 256 tiles two
    //    4-wave workgroups per CU do better (32B down 674 vs 799 us).
    int t4 = 0;
    for (int i = 0; i < count; ++i) t4 += ceil_div(probs[i].M, kGemmRows) * ceil_div(probs[i].N, 256);
    pl.cpl = t4 < 192 ? 2 : 4;
    pl.kw = pl.cpl == 4 && t4 <= 256 ? 2 : 1;
    if (pl.cpl == 2) pl.kw = 1;
    const int tcols = 64 * pl.cpl;
    int tiles_total = 0;
    for (int i = 0; i < count; ++i) tiles_total += ceil_div(probs[i].M, kGemmRows) * ceil_div(probs[i].N, tcols);
    int wg = 0;
    for (int i = 0; i < count; ++i) {
      Problem& P = pl.L.p[i];
      const int G = P.K / kGroup;
      const int M = P.M;
      P.tiles_m = ceil_div(M, kGemmRows);
      P.tiles_n = ceil_div(P.N, tcols);
      const int tiles = P.tiles_m * P.tiles_n;
      // Split K when the launch has fewer than ~1.5 workgroups per CU slot,
      // keeping >= 4 groups per split.
      int nsplit = tiles_total >= 384 ? 1 : std::max(1, 512 / tiles_total);
      nsplit = std::min(nsplit, std::max(1, G / 4));
      if (pl.cpl == 4) nsplit = 1;  // 256-column tiles only when the chip is already full
      while (nsplit > 1 && (size_t)nsplit * M * P.N * 4 >= 0xffffffffull) --nsplit;  // 32-bit buffer offsets
      P.gps = ceil_div(G, nsplit);
      P.nsplit = ceil_div(G, P.gps);
      P.wg_begin = wg;
      wg += tiles * P.nsplit;
      const size_t wbytes = (size_t)(P.K / 2) * P.ldp, sbytes = (size_t)G * P.lds * 4;
      full = full && aligned(P.packed, pl.cpl) && P.ldp % pl.cpl == 0 && aligned(P.scale, 4 * pl.cpl) &&
             P.lds % pl.cpl == 0 && P.N % tcols == 0 && wbytes < 0xffffffffull && sbytes < 0xffffffffull;
      // Row sums, shared by problems with the same activations.
      for (int j = 0; j < i; ++j)
        if (probs[j].x == probs[i].x && probs[j].ldx == probs[i].ldx && probs[j].K == probs[i].K &&
            probs[j].M == probs[i].M && pl.rowsum_src[j] == j) {
          pl.rowsum_src[i] = j;
          break;
        }
      if (pl.rowsum_src[i] == i) {
        pl.rowsum_off[i] = ws;
        ws = align256(ws + (size_t)G * M * 4);
        P.rs_begin = pl.rs_wgs;
        pl.rs_wgs += ceil_div((int64_t)M * G, 16);
      }
      P.red_begin = pl.red_wgs;
      if (P.nsplit > 1) {
        pl.part_off[i] = ws;
        ws = align256(ws + (size_t)P.nsplit * M * P.N * 4);
        pl.red_wgs += ceil_div((int64_t)M * P.N, kReduceElems);
      }
    }
    pl.total_wgs = wg;
  }
  pl.full = full;
  pl.L.total_wgs = pl.total_wgs;
  pl.ws_bytes = ws;
  return pl;
}

// Point the device table at the workspace.  A workspace of W bytes is split
// in two halves: the decode kernels' published-partial slots live in the
// lower half, which is zero between calls (every finisher zeroes what it
// read), and the GEMM's row sums and split partials in the upper half, which
// holds garbage after a GEMM.  Keeping them apart is what lets the decode
// slots rely on "0 = empty" whatever ran before on the same workspace.
//
// The last aligned 32-bit word of the workspace is its status word
// (kStatusSplitKTimeout), zero as allocated; plan_bytes() leaves the last 128
// bytes outside both halves' scratch, so nothing else writes it.
std::atomic<uint32_t> g_spin_limit{kDefaultSpinLimit};

uint32_t* status_word(void* workspace, size_t workspace_bytes) {
  if (!workspace || workspace_bytes < 256) return nullptr;
  return reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + ((workspace_bytes - 4) & ~(size_t)3));
}

void bind(Plan& pl, void* workspace, size_t workspace_bytes) {
  char* ws = static_cast<char*>(workspace);
  char* upper = ws + ((workspace_bytes / 2) & ~(size_t)255) + pl.skip;
  pl.L.status = status_word(workspace, workspace_bytes);
  pl.L.spin_limit = g_spin_limit.load(std::memory_order_relaxed);
  for (int i = 0; i < pl.L.count; ++i) {
    Problem& P = pl.L.p[i];
    if (pl.kind == kGemm) {
      if (P.nsplit > 1) P.part = reinterpret_cast<float*>(upper + pl.part_off[i]);
      P.rowsum = reinterpret_cast<float*>(upper + pl.rowsum_off[pl.rowsum_src[i]]);
    } else if (P.nsplit > 1 || (pl.pair && i == 0)) {
      P.part = reinterpret_cast<float*>(ws + pl.part_off[i]);
    }
  }
}

// Workspace bytes a plan needs: twice its half, rounded.  The GEMM scratch
// sits after the caller's `skip` bytes in the upper half; decode slots use the
// lower half, which must then still be as large as `skip`.
size_t plan_bytes(const Plan& pl) {
  const size_t half = pl.kind == kGemm ? pl.skip + pl.ws_bytes : std::max(pl.skip, pl.ws_bytes);
  return half == 0 ? 0 : 2 * align256(half) + 256;
}

int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? W4A16_OK : W4A16_ERR_LAUNCH;
}

template <int CPL, int WAVES, bool MULTI, int MROWS, bool PAIR>
void launch_gemv_as(const Plan& pl, dim3 grid, hipStream_t s) {
  const dim3 block(WAVES * 64);
  if (pl.full)
    hipLaunchKernelGGL((gemv_kernel<CPL, WAVES, true, MULTI, MROWS, PAIR>), grid, block, pl.lds_bytes, s, pl.L);
  else
    hipLaunchKernelGGL((gemv_kernel<CPL, WAVES, false, MULTI, (MROWS > 32 ? 64 : (MROWS > 16 ? 32 : 16)), PAIR>), grid, block,
                       pl.lds_bytes, s, pl.L);
}

template <int CPL, int WAVES, bool MULTI, bool PAIR = false>
void launch_gemv_rows(const Plan& pl, dim3 grid, int max_m, hipStream_t s) {
  if (max_m == 1)
    launch_gemv_as<CPL, WAVES, MULTI, 1, PAIR>(pl, grid, s);
  else if (max_m <= 4)
    launch_gemv_as<CPL, WAVES, MULTI, 4, PAIR>(pl, grid, s);
  else if (max_m <= 8)
    launch_gemv_as<CPL, WAVES, MULTI, 8, PAIR>(pl, grid, s);
  else if (max_m <= 16)
    launch_gemv_as<CPL, WAVES, MULTI, 16, PAIR>(pl, grid, s);
  else if constexpr (CPL == 4 && WAVES == 8) {  // the only shape make_plan picks for M > 16
    if (max_m <= 32)
      launch_gemv_as<CPL, WAVES, MULTI, 32, PAIR>(pl, grid, s);
    else
      launch_gemv_as<CPL, WAVES, MULTI, 64, PAIR>(pl, grid, s);
  }
}

template <int CPL, int WAVES>
int launch_gemv(const Plan& pl, hipStream_t s) {
  int max_m = 0;
  for (int i = 0; i < pl.L.count; ++i) max_m = std::max(max_m, pl.L.p[i].M);
  if (pl.pair)
    launch_gemv_rows<CPL, WAVES, true, true>(pl, dim3(pl.total_wgs), max_m, s);
  else if (pl.L.count > 1)
    launch_gemv_rows<CPL, WAVES, true>(pl, dim3(pl.total_wgs), max_m, s);
  else
    launch_gemv_rows<CPL, WAVES, false>(pl, dim3(pl.L.p[0].tiles_n, pl.L.p[0].nsplit), max_m, s);
  return launch_status();
}

template <int CPL, int KW>
int launch_gemm(const Plan& pl, hipStream_t s) {
  const int grid = (pl.total_wgs + 7) & ~7;
  if (pl.full)
    hipLaunchKernelGGL((gemm_kernel<CPL, true, KW>), dim3(grid), dim3(256 * KW), 0, s, pl.L);
  else
    hipLaunchKernelGGL((gemm_kernel<CPL, false, KW>), dim3(grid), dim3(256 * KW), 0, s, pl.L);
  return launch_status();
}

// Problems that run() launches on their own: K == 0 (zero fill), or M > 32
// with activations the GEMM cannot stage with 16-byte copies.
bool separate(const w4a16_problem& q) { return q.K == 0 || (q.M > 32 && !gemm_x_ok(q)); }

// The launches of one call: problems with M > 0 and N > 0 grouped by kernel.
// The decode (M <= 32) and the GEMM group are one launch each.  Problems in
// `sep` are handled alone.
struct Batches {
  w4a16_problem gemv[kMaxProblems], gemm[kMaxProblems], sep[kMaxProblems];
  int n_gemv = 0, n_gemm = 0, n_sep = 0;
};

Batches split(const w4a16_problem* probs, int count) {
  Batches b;
  for (int i = 0; i < count; ++i) {
    const w4a16_problem& q = probs[i];
    if (q.M == 0 || q.N == 0) continue;
    if (separate(q)) {
      b.sep[b.n_sep++] = q;
      continue;
    }
    if (kind_of(q) == kGemv)
      b.gemv[b.n_gemv++] = q;
    else
      b.gemm[b.n_gemm++] = q;
  }
  return b;
}

// Unaligned activations with M > 32 go through the decode kernel 32 rows at a time.
template <class Fn>
int for_each_chunk(const w4a16_problem& q, Fn fn) {
  for (int m0 = 0; m0 < q.M; m0 += 32) {
    w4a16_problem c = q;
    c.x = static_cast<const uint16_t*>(q.x) + (int64_t)m0 * q.ldx;
    c.y = static_cast<uint16_t*>(q.y) + (int64_t)m0 * q.ldy;
    c.M = q.M - m0 < 32 ? q.M - m0 : 32;
    const int rc = fn(c);
    if (rc != W4A16_OK) return rc;
  }
  return W4A16_OK;
}

// Launch one planned batch (all problems of one kind).
int launch_plan(const w4a16_problem* probs, int count, void* workspace, size_t workspace_bytes, hipStream_t s,
                size_t skip = 0, bool pair = false) {
  Plan pl = make_plan(probs, count, pair);
  pl.skip = skip;
  const size_t need = plan_bytes(pl);
  if (need > 0 && (!workspace || workspace_bytes < need)) return W4A16_ERR_WORKSPACE;
  bind(pl, workspace, workspace_bytes);
  if (pl.too_large) return W4A16_ERR_TOO_LARGE;
  if (pl.kind == kGemv) {
    if (pl.waves == 8 && pl.cpl == 4) return launch_gemv<4, 8>(pl, s);
    int max_m = 0;
    for (int i = 0; i < count; ++i) max_m = std::max(max_m, probs[i].M);
    if (max_m > 16) return W4A16_ERR_LAUNCH;  // no kernel built for that shape
    if (pl.waves == 8) return launch_gemv<8, 8>(pl, s);
    return pl.cpl == 4 ? launch_gemv<4, 4>(pl, s) : launch_gemv<8, 4>(pl, s);
  }
  hipLaunchKernelGGL(rowsum_kernel, dim3(pl.rs_wgs), dim3(256), 0, s, pl.L);
  const int rc = launch_status();
  if (rc != W4A16_OK) return rc;
  const int rc2 = pl.cpl == 2 ? launch_gemm<2, 1>(pl, s) : (pl.kw == 2 ? launch_gemm<4, 2>(pl, s) : launch_gemm<4, 1>(pl, s));
  if (rc2 != W4A16_OK || pl.red_wgs == 0) return rc2;
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(pl.red_wgs), dim3(256), 0, s, pl.L);
  return launch_status();
}

// Workspace bytes launch_plan needs for one batch.
int plan_workspace(const w4a16_problem* probs, int count, size_t* bytes, size_t skip = 0, bool pair = false) {
  Plan pl = make_plan(probs, count, pair);
  pl.skip = skip;
  *bytes = std::max(*bytes, plan_bytes(pl));
  return W4A16_OK;
}

// The launches run in order on one stream, so they share the workspace.
int run(const w4a16_problem* probs, int count, void* workspace, size_t workspace_bytes, hipStream_t s,
        size_t skip = 0) {
  Batches b = split(probs, count);
  for (int i = 0; i < b.n_sep; ++i) {
    const w4a16_problem& q = b.sep[i];
    int rc;
    if (q.K == 0) {
      hipLaunchKernelGGL(zero_kernel, dim3(ceil_div((int64_t)q.M * q.N, 256)), dim3(256), 0, s,
                         static_cast<uint16_t*>(q.y), q.ldy, q.M, q.N);
      rc = launch_status();
    } else {
      rc = for_each_chunk(q, [&](const w4a16_problem& c) {
        return launch_plan(&c, 1, workspace, workspace_bytes, s, skip);
      });
    }
    if (rc != W4A16_OK) return rc;
  }
  if (b.n_gemv > 0) {
    const int rc = launch_plan(b.gemv, b.n_gemv, workspace, workspace_bytes, s, skip);
    if (rc != W4A16_OK) return rc;
  }
  if (b.n_gemm > 0) return launch_plan(b.gemm, b.n_gemm, workspace, workspace_bytes, s, skip);
  return W4A16_OK;
}

// Workspace run() needs for these problems (0 when none).
int workspace_for(const w4a16_problem* probs, int count, size_t* bytes, size_t skip = 0) {
  *bytes = 0;
  Batches b = split(probs, count);
  for (int i = 0; i < b.n_sep; ++i) {
    if (b.sep[i].K == 0) continue;
    const int rc =
        for_each_chunk(b.sep[i], [&](const w4a16_problem& c) { return plan_workspace(&c, 1, bytes, skip); });
    if (rc != W4A16_OK) return rc;
  }
  int rc = W4A16_OK;
  if (b.n_gemv > 0 && (rc = plan_workspace(b.gemv, b.n_gemv, bytes, skip)) != W4A16_OK) return rc;
  if (b.n_gemm > 0 && (rc = plan_workspace(b.gemm, b.n_gemm, bytes, skip)) != W4A16_OK) return rc;
  return W4A16_OK;
}

// SwiGLU h = silu(x @ Wg) * (x @ Wu) on the gate/up problem pair.  M <= 16:
// one decode launch whose finishers apply the epilogue to the fp32 sums.
// Larger M: gate into h and up into the first `ubytes` of the upper workspace
// half (one grouped launch), then silu_mul_kernel.
size_t swiglu_up_bytes(const w4a16_problem& q) { return kind_of(q) == kGemv ? 0 : align256((size_t)q.M * q.N * 2); }

// The SwiGLU pair at GEMM-sized M as one gemm_kernel<4, true, 1, true> launch
// (after the row sums): needs 128-column tiles in range and aligned operands
// (4-byte weight loads, 16-byte scale loads, 8-byte output stores), and at least
// one full round of tiles on the chip (there is no split-K in this shape).
// Otherwise swiglu() runs the grouped GEMM plus silu_mul_kernel.
bool pair_gemm_ok(const w4a16_problem pair[2]) {
  const w4a16_problem& g = pair[0];
  if (kind_of(g) != kGemm || g.N % 128 != 0 || !gemm_x_ok(g)) return false;
  if ((int64_t)ceil_div(g.M, kGemmRows) * (g.N / 128) < 256) return false;
  if (!aligned(g.y, 8) || g.ldy % 4 != 0) return false;
  for (int i = 0; i < 2; ++i) {
    const w4a16_problem& q = pair[i];
    if (!aligned(q.packed, 4) || q.ldp % 4 != 0 || !aligned(q.scale, 16) || q.lds % 4 != 0) return false;
    if ((size_t)(q.K / 2) * q.ldp >= 0xffffffffull || (size_t)(q.K / kGroup) * q.lds * 4 >= 0xffffffffull) return false;
  }
  return true;
}

Plan make_pair_plan(const w4a16_problem pair[2]) {
  Plan pl{};
  pl.kind = kGemm;
  pl.cpl = 4;
  pl.kw = 1;
  pl.full = true;
  pl.pair = true;
  pl.L.count = 2;
  for (int i = 0; i < 2; ++i) {
    const w4a16_problem& q = pair[i];
    Problem& P = pl.L.p[i];
    P.x = static_cast<const uint16_t*>(q.x);
    P.ldx = q.ldx;
    P.packed = reinterpret_cast<const uint8_t*>(q.packed);
    P.ldp = q.ldp;
    P.scale = q.scale;
    P.lds = q.lds;
    P.y = static_cast<uint16_t*>(q.y);
    P.ldy = q.ldy;
    P.M = q.M;
    P.N = q.N;
    P.K = q.K;
    P.rs_begin = -1;
    P.nsplit = 1;
    P.gps = q.K / kGroup;
    pl.rowsum_src[i] = 0;
  }
  Problem& P = pl.L.p[0];
  P.tiles_m = ceil_div(P.M, kGemmRows);
  P.tiles_n = P.N / 128;
  P.rs_begin = 0;
  pl.rowsum_off[0] = 0;
  pl.rs_wgs = ceil_div((int64_t)P.M * (P.K / kGroup), 16);
  pl.ws_bytes = align256((size_t)(P.K / kGroup) * P.M * 4);
  pl.total_wgs = P.tiles_m * P.tiles_n;
  pl.L.total_wgs = pl.total_wgs;
  return pl;
}

int swiglu(const w4a16_problem pair[2], void* workspace, size_t workspace_bytes, hipStream_t s) {
  const w4a16_problem& g = pair[0];
  if (g.M == 0 || g.N == 0) return W4A16_OK;
  if (g.K == 0) {
    hipLaunchKernelGGL(zero_kernel, dim3(ceil_div((int64_t)g.M * g.N, 256)), dim3(256), 0, s,
                       static_cast<uint16_t*>(g.y), g.ldy, g.M, g.N);
    return launch_status();
  }
  if (kind_of(g) == kGemv) return launch_plan(pair, 2, workspace, workspace_bytes, s, 0, true);
  if (pair_gemm_ok(pair)) {
    Plan pl = make_pair_plan(pair);
    if (!workspace || workspace_bytes < plan_bytes(pl)) return W4A16_ERR_WORKSPACE;
    bind(pl, workspace, workspace_bytes);
    hipLaunchKernelGGL(rowsum_kernel, dim3(pl.rs_wgs), dim3(256), 0, s, pl.L);
    const int rc = launch_status();
    if (rc != W4A16_OK) return rc;
    hipLaunchKernelGGL((gemm_kernel<4, true, 1, true>), dim3((pl.total_wgs + 7) & ~7), dim3(256), 0, s, pl.L);
    return launch_status();
  }
  const size_t ub = swiglu_up_bytes(g);
  if (!workspace || workspace_bytes < 2 * ub + 256) return W4A16_ERR_WORKSPACE;
  w4a16_problem q[2] = {pair[0], pair[1]};
  uint16_t* u = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + ((workspace_bytes / 2) & ~(size_t)255));
  q[1].y = u;
  q[1].ldy = g.N;
  const int rc = run(q, 2, workspace, workspace_bytes, s, ub);
  if (rc != W4A16_OK) return rc;
  hipLaunchKernelGGL(silu_mul_kernel, dim3(ceil_div((int64_t)g.M * g.N, 256)), dim3(256), 0, s,
                     static_cast<uint16_t*>(g.y), g.ldy, static_cast<const uint16_t*>(u), g.M, g.N);
  return launch_status();
}

int swiglu_workspace(const w4a16_problem pair[2], size_t* bytes) {
  *bytes = 0;
  const w4a16_problem& g = pair[0];
  if (g.M == 0 || g.N == 0 || g.K == 0) return W4A16_OK;
  if (kind_of(g) == kGemv) return plan_workspace(pair, 2, bytes, 0, true);
  // Enough for both GEMM-sized forms: the size query sees only shapes, and a
  // call whose operands are not aligned for the pair kernel takes the grouped
  // GEMM + silu_mul path.
  const size_t ub = swiglu_up_bytes(g);
  const int rc = workspace_for(pair, 2, bytes, ub);
  *bytes = std::max(*bytes, 2 * ub + 256);
  if (pair_gemm_ok(pair)) *bytes = std::max(*bytes, plan_bytes(make_pair_plan(pair)));
  return rc;
}

int check_all(const w4a16_problem* probs, int count, int group_size) {
  if (count < 0 || count > kMaxProblems) return W4A16_ERR_SHAPE;
  if (count > 0 && !probs) return W4A16_ERR_NULL;
  if (group_size != kGroup) return W4A16_ERR_GROUP_SIZE;
  for (int i = 0; i < count; ++i) {
    const int rc = check_problem(probs[i]);
    if (rc != W4A16_OK) return rc;
  }
  return W4A16_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (w4a16_linear_noalloc).
//
// One array per GPU in the library's own device memory, held until the
// process ends.  It stands in for the caller's workspace: the lower half holds
// the decode kernels' published-partial slots (zero between calls, like any
// workspace), the upper half the GEMM's row sums and split partials, and the
// last word the status word.  In host code `scratch` names a host-side shadow,
// not device memory: the device address comes from hipGetSymbolAddress, once
// per device with that device current, and only that pointer is ever passed
// to a kernel.  Every call on a GPU shares its array, so calls that overlap on
// one GPU (other streams, other threads) race.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = (size_t)96 << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

__global__ __launch_bounds__(256) void fill_zero_kernel(u32x4_t* __restrict__ p, size_t n16) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (size_t)gridDim.x * 256)
    p[i] = u32x4_t{0u, 0u, 0u, 0u};
}

bool capturing(hipStream_t s) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(s, &st) != hipSuccess || st != hipStreamCaptureStatusNone;
}

// Zero the whole scratch on `s` and wait for it.
int zero_scratch(void* p, hipStream_t s) {
  hipLaunchKernelGGL(fill_zero_kernel, dim3(1024), dim3(256), 0, s, static_cast<u32x4_t*>(p), kScratchBytes / 16);
  if (hipGetLastError() != hipSuccess) return W4A16_ERR_LAUNCH;
  return hipStreamSynchronize(s) == hipSuccess ? W4A16_OK : W4A16_ERR_LAUNCH;
}

// Device address of the current device's scratch, set up on the first call
// on that device.  Set-up is eager work: the address lookup and a zero fill on
// `s` that completes before the pointer is published, so a set-up scratch is
// zero for every stream.  Under graph capture that fill would become a node
// that re-zeroes 96 MiB on every replay, so a stream that is capturing is
// refused (W4A16_ERR_CAPTURING): one eager call (or w4a16_noalloc_status) on
// the device sets the scratch up.
int scratch_for_current_device(hipStream_t s, void** out) {
  *out = nullptr;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return W4A16_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (capturing(s)) return W4A16_ERR_CAPTURING;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return W4A16_ERR_LAUNCH;
    const int rc = zero_scratch(p, s);
    if (rc != W4A16_OK) return rc;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return W4A16_OK;
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
    case W4A16_ERR_SHAPE:
      return "invalid shape (negative size, leading dimension smaller than the row, or bad problem count)";
    case W4A16_ERR_K_GROUP: return "K must be a multiple of group_size (and even) for int4 packing";
    case W4A16_ERR_GROUP_SIZE: return "fused INT4 kernel requires group_size=128";
    case W4A16_ERR_WORKSPACE: return "workspace missing or smaller than w4a16_workspace_size()";
    case W4A16_ERR_LAUNCH: return "HIP kernel launch failed";
    case W4A16_ERR_DTYPE: return "unsupported dtype code";
    case W4A16_ERR_TOO_LARGE: return "problem exceeds the supported size";
    case W4A16_ERR_CAPTURING:
      return "the stream is capturing a graph and the call needs eager work first (set up the no-alloc scratch with "
             "one eager call or w4a16_noalloc_status)";
    default: return "unknown w4a16 error";
  }
}

int w4a16_workspace_size(int M, int N, int K, int group_size, size_t* bytes) {
  if (!bytes) return W4A16_ERR_NULL;
  *bytes = 0;
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  if (group_size != kGroup) return W4A16_ERR_GROUP_SIZE;
  if (K % kGroup != 0) return W4A16_ERR_K_GROUP;
  // The query sees shapes, not pointers.  Activations whose rows are not
  // 16-byte aligned send M > 32 through the decode kernel 32 rows at a time
  // (separate()), which can need more split-K slots than the GEMM plan of
  // aligned rows, so the size covers both.
  const uintptr_t a = 256;
  w4a16_problem q{reinterpret_cast<const void*>(a), K, reinterpret_cast<const int8_t*>(a), N,
                  reinterpret_cast<const float*>(a), N, reinterpret_cast<void*>(a), N, M, N, K};
  int rc = workspace_for(&q, 1, bytes);
  if (rc != W4A16_OK) return rc;
  q.x = reinterpret_cast<const void*>(a + 2);
  size_t unaligned = 0;
  rc = workspace_for(&q, 1, &unaligned);
  *bytes = std::max(*bytes, unaligned);
  return rc;
}

int w4a16_status_offset(size_t workspace_bytes, size_t* offset) {
  if (!offset) return W4A16_ERR_NULL;
  if (workspace_bytes < 256) return W4A16_ERR_WORKSPACE;
  *offset = (workspace_bytes - 4) & ~(size_t)3;
  return W4A16_OK;
}

uint32_t w4a16_debug_set_spin_limit(uint32_t polls) { return g_spin_limit.exchange(polls); }

int w4a16_workspace_size_grouped(const w4a16_problem* problems, int count, int group_size, size_t* bytes) {
  if (!bytes) return W4A16_ERR_NULL;
  *bytes = 0;
  const int rc = check_all(problems, count, group_size);
  if (rc != W4A16_OK) return rc;
  return workspace_for(problems, count, bytes);
}

int w4a16_linear_grouped(const w4a16_problem* problems, int count, int group_size, void* workspace,
                         size_t workspace_bytes, void* stream) {
  const int rc = check_all(problems, count, group_size);
  if (rc != W4A16_OK) return rc;
  return run(problems, count, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int w4a16_linear(const void* x, int64_t ldx, const int8_t* packed, int64_t ldp, const float* scale, int64_t lds,
                 void* y, int64_t ldy, int M, int N, int K, int group_size, void* workspace, size_t workspace_bytes,
                 void* stream) {
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  const w4a16_problem q{x, ldx, packed, ldp, scale, lds, y, ldy, M, N, K};
  return w4a16_linear_grouped(&q, 1, group_size, workspace, workspace_bytes, stream);
}

int w4a16_linear_noalloc(const void* x, int64_t ldx, const int8_t* packed, int64_t ldp, const float* scale,
                         int64_t lds, void* y, int64_t ldy, int M, int N, int K, int group_size, void* stream) {
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  const w4a16_problem q{x, ldx, packed, ldp, scale, lds, y, ldy, M, N, K};
  int rc = check_all(&q, 1, group_size);
  if (rc != W4A16_OK) return rc;
  size_t need = 0;
  rc = workspace_for(&q, 1, &need);
  if (rc != W4A16_OK) return rc;
  if (need > kScratchBytes) return W4A16_ERR_TOO_LARGE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (need == 0) return run(&q, 1, nullptr, 0, s);
  void* ws = nullptr;
  rc = scratch_for_current_device(s, &ws);
  if (rc != W4A16_OK) return rc;
  return run(&q, 1, ws, kScratchBytes, s);
}

int w4a16_capture_id(void* stream, unsigned long long* id) {
  if (!id) return W4A16_ERR_NULL;
  *id = 0;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  unsigned long long cid = 0;
  if (hipStreamGetCaptureInfo(static_cast<hipStream_t>(stream), &st, &cid) != hipSuccess) return W4A16_ERR_LAUNCH;
  if (st == hipStreamCaptureStatusActive) *id = cid;
  return W4A16_OK;
}

int w4a16_noalloc_status(void* stream, uint32_t* status) {
  if (!status) return W4A16_ERR_NULL;
  *status = 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (capturing(s)) return W4A16_ERR_CAPTURING;
  void* ws = nullptr;
  int rc = scratch_for_current_device(s, &ws);
  if (rc != W4A16_OK) return rc;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (hipStreamSynchronize(s) != hipSuccess) return W4A16_ERR_LAUNCH;
  size_t off = 0;
  w4a16_status_offset(kScratchBytes, &off);
  uint32_t word = 0;
  if (hipMemcpy(&word, static_cast<uint8_t*>(ws) + off, 4, hipMemcpyDeviceToHost) != hipSuccess) return W4A16_ERR_LAUNCH;
  // A give-up leaves late partials in the slot half: zero it all again.
  if (word) rc = zero_scratch(ws, s);
  *status = word;
  return rc;
}

int w4a16_workspace_size_swiglu(int M, int N, int K, int group_size, size_t* bytes) {
  if (!bytes) return W4A16_ERR_NULL;
  *bytes = 0;
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  if (group_size != kGroup) return W4A16_ERR_GROUP_SIZE;
  if (K % kGroup != 0) return W4A16_ERR_K_GROUP;
  // Aligned and unaligned activation rows, as in w4a16_workspace_size.
  const uintptr_t a = 256;
  w4a16_problem q{reinterpret_cast<const void*>(a), K, reinterpret_cast<const int8_t*>(a), N,
                  reinterpret_cast<const float*>(a), N, reinterpret_cast<void*>(a), N, M, N, K};
  w4a16_problem pair[2] = {q, q};
  int rc = swiglu_workspace(pair, bytes);
  if (rc != W4A16_OK) return rc;
  pair[0].x = pair[1].x = reinterpret_cast<const void*>(a + 2);
  size_t unaligned = 0;
  rc = swiglu_workspace(pair, &unaligned);
  *bytes = std::max(*bytes, unaligned);
  return rc;
}

int w4a16_swiglu(const void* x, int64_t ldx, const int8_t* gate_packed, int64_t gate_ldp, const float* gate_scale,
                 int64_t gate_lds, const int8_t* up_packed, int64_t up_ldp, const float* up_scale, int64_t up_lds,
                 void* h, int64_t ldh, int M, int N, int K, int group_size, void* workspace, size_t workspace_bytes,
                 void* stream) {
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  const w4a16_problem pair[2] = {{x, ldx, gate_packed, gate_ldp, gate_scale, gate_lds, h, ldh, M, N, K},
                                 {x, ldx, up_packed, up_ldp, up_scale, up_lds, h, ldh, M, N, K}};
  const int rc = check_all(pair, 2, group_size);
  if (rc != W4A16_OK) return rc;
  return swiglu(pair, workspace, workspace_bytes, static_cast<hipStream_t>(stream));
}

int w4a16_bf16_gemv(const void* x, int64_t ldx, const void* w, int64_t ldw, void* y, int64_t ldy, int M, int N,
                    int K, void* stream) {
  if (M < 0 || N < 0 || K < 0) return W4A16_ERR_SHAPE;
  if (M > 16) return W4A16_ERR_TOO_LARGE;
  if (M == 0 || N == 0) return W4A16_OK;
  if (!y) return W4A16_ERR_NULL;
  if (K == 0) {
    hipLaunchKernelGGL(zero_kernel, dim3(ceil_div((int64_t)M * N, 256)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<uint16_t*>(y), ldy, M, N);
    return launch_status();
  }
  if (!x || !w) return W4A16_ERR_NULL;
  if (ldx < K || ldw < K || ldy < N) return W4A16_ERR_SHAPE;
  // 16-byte loads: x and w rows 16-byte aligned, K a multiple of 8.
  if (K % 8 != 0 || ldx % 8 != 0 || ldw % 8 != 0 || !aligned(x, 16) || !aligned(w, 16)) return W4A16_ERR_SHAPE;
  if ((size_t)16 * ldw * 2 >= 0xffffffffull) return W4A16_ERR_TOO_LARGE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t lds_rows = (size_t)M * ((K + 511) / 512 * 512) * 2;
  if (M <= 4 && lds_rows <= 64 * 1024) {
    const int grid = (int)std::min<int64_t>(kRowsGrid, ceil_div(N, 8));
    const auto* xp = static_cast<const uint16_t*>(x);
    const auto* wp = static_cast<const uint16_t*>(w);
    auto* yp = static_cast<uint16_t*>(y);
    if (M == 1)
      hipLaunchKernelGGL(bf16_gemv_rows_kernel<1>, dim3(grid), dim3(256), lds_rows, s, xp, ldx, wp, ldw, yp, ldy, M, N, K);
    else if (M == 2)
      hipLaunchKernelGGL(bf16_gemv_rows_kernel<2>, dim3(grid), dim3(256), lds_rows, s, xp, ldx, wp, ldw, yp, ldy, M, N, K);
    else
      hipLaunchKernelGGL(bf16_gemv_rows_kernel<4>, dim3(grid), dim3(256), lds_rows, s, xp, ldx, wp, ldw, yp, ldy, M, N, K);
    return launch_status();
  }
  const size_t lds = (size_t)(M + 1) * (K + 72) * 2;
  if (lds > 160 * 1024) return W4A16_ERR_TOO_LARGE;
  const int grid = ceil_div(N, 64);
  const bool full = K % (64 * kDenseChunks) == 0;
  if (full)
    hipLaunchKernelGGL(bf16_gemv_kernel<true>, dim3(grid), dim3(256), lds, s, static_cast<const uint16_t*>(x), ldx,
                       static_cast<const uint16_t*>(w), ldw, static_cast<uint16_t*>(y), ldy, M, N, K);
  else
    hipLaunchKernelGGL(bf16_gemv_kernel<false>, dim3(grid), dim3(256), lds, s, static_cast<const uint16_t*>(x), ldx,
                       static_cast<const uint16_t*>(w), ldw, static_cast<uint16_t*>(y), ldy, M, N, K);
  return launch_status();
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
