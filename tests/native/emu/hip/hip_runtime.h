// Host stand-in for <hip/hip_runtime.h>: compiles the gfx950 kernel source
// (inf-engine_amd/csrc/w4a16_kernels.hip) as ordinary x86-64 C++ so that the
// kernels can run on the CPU under the wave emulator of emu_runtime.cpp.
//
// TEST INFRASTRUCTURE ONLY.  Each GPU thread is a fiber; the operations that
// exchange data between the lanes of a wave (MFMA, ballot, readfirstlane,
// shuffles) and __syncthreads are the points where fibers meet.  Buffer
// loads and stores apply the raw-buffer range rule of the hardware (an
// access past num_records reads zero / is dropped, per dword); every other
// memory access is an ordinary host access, so a kernel that leaves its
// buffers touches a guard page and is reported (emu_alloc in
// emu_runtime.cpp).  Direct-to-LDS copies land only when a wait
// (s_waitcnt vmcnt) covers them, as on the hardware.  Buffer accesses are
// also audited: their outcome must not depend on how the range check treats
// the scalar offset, and a load of data another workgroup stored in the same
// launch must be agent-coherent, as must that store.  Workgroups run one
// after another in dispatch order, or (decode kernels, emu_set_concurrency)
// several at once, interleaved at every meeting point.  What this does NOT
// model: timing, caches and the memory ordering they allow (every store is
// visible to every later load at once), and the exact rounding order of the
// matrix cores (the MFMA sums in fp32, k in order).
#pragma once

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include <functional>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline __attribute__((always_inline))
#define __launch_bounds__(...)
#define __shared__ static
#define __align__(n) __attribute__((aligned(n)))
// AMDGPU-only function attributes (occupancy hints) have no host meaning.
#define amdgpu_waves_per_eu(...) unused

typedef uint32_t emu_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t emu_u32x2 __attribute__((ext_vector_type(2)));
typedef float emu_f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 emu_bf16x8 __attribute__((ext_vector_type(8)));
typedef short emu_s16x2 __attribute__((ext_vector_type(2)));

struct dim3 {
  unsigned x, y, z;
  dim3(unsigned a = 1, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct emu_uint3 {
  unsigned x, y, z;
};

typedef int hipError_t;
enum { hipSuccess = 0, hipErrorInvalidValue = 1, hipErrorLaunchFailure = 719 };
typedef struct emu_stream_t* hipStream_t;

// A raw buffer resource: base address and size in bytes (stride 0).
struct emu_rsrc {
  const char* base;
  uint32_t num;
};
#define __amdgpu_buffer_rsrc_t emu_rsrc

// The integer min / max overloads HIP provides in device code.
inline int min(int a, int b) { return a < b ? a : b; }
inline int max(int a, int b) { return a > b ? a : b; }
inline unsigned min(unsigned a, unsigned b) { return a < b ? a : b; }
inline unsigned max(unsigned a, unsigned b) { return a > b ? a : b; }
inline long long min(long long a, long long b) { return a < b ? a : b; }
inline long long max(long long a, long long b) { return a > b ? a : b; }

namespace emu {

// Launch, lane and collective services (emu_runtime.cpp).
const emu_uint3* cur_tid();
const emu_uint3* cur_bid();
extern emu_uint3 g_grid_dim, g_block_dim;
void launch(const char* name, dim3 grid, dim3 block, size_t dyn_lds, const std::function<void()>& body);
void* dyn_lds();
void* static_lds(int id, size_t bytes);  // per-workgroup __shared__ array (prepare.py)
emu_f32x4 mfma_16x16x32_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x4 c);
uint64_t ballot(bool pred);
uint32_t readfirstlane(uint32_t v);
float shfl_xor(float v, int mask, int width);
void syncthreads();
int lane_id();
hipError_t last_error();
// Vector-memory bookkeeping of the calling lane: every buffer access counts
// as one operation in issue order; a direct-to-LDS copy reaches the LDS only
// when a wait (s_waitcnt vmcnt(n)) leaves at most n younger operations
// outstanding, as on the hardware, where such copies land asynchronously.
void vm_issue();
void count_load();  // buffer loads issued since emu_reset_load_count
// Cross-workgroup coherence audit (emu_runtime.cpp): within one launch, a
// buffer load of a dword that another workgroup stored must carry the
// agent-coherence bit, and so must that store; otherwise the run stops.
void note_store(const char* p, int bytes, int aux);
void check_load(const char* p, int bytes, int aux);
void vm_copy_to_lds(void* dst, const void* src, int bytes);
void waitcnt(int code);

inline emu_rsrc make_rsrc(const void* p, short, int num, int) { return emu_rsrc{static_cast<const char*>(p), (uint32_t)num}; }

// Stops the run: a buffer access whose outcome depends on a detail of the
// hardware's range check (emu_runtime.cpp).
[[noreturn]] void range_ambiguous();

// The kernels must not depend on two details of the raw-buffer range check
// that the emulated rule below fixes one way: whether the scalar offset
// (soffset) counts towards the check or only moves the address, and whether a
// multi-dword access that straddles num_records is checked per dword or as a
// whole.  Every access must therefore lie wholly in range or wholly out of
// range whichever way those are read, with no 32-bit wrap of the offset.
inline void range_rules_agree(emu_rsrc r, uint64_t vimm, uint32_t soff, int bytes) {
  const uint64_t full = vimm + soff;
  if (full >= (1ull << 32)) range_ambiguous();
  const bool in_v = vimm + bytes <= r.num, out_v = vimm >= r.num;
  const bool in_full = full + bytes <= r.num, out_full = full >= r.num;
  if (!((in_v && in_full) || (out_v && out_full))) range_ambiguous();
}

// Raw buffer rule: each dword (or the one 16-bit word) is in range when its
// last byte lies below num_records; out-of-range loads read zero and
// out-of-range stores are dropped.
template <int BYTES>
inline void buffer_load(emu_rsrc r, uint32_t voff, uint32_t soff, void* out, int aux) {
  vm_issue();
  count_load();
  range_rules_agree(r, voff, soff, BYTES);
  const uint64_t off = (uint64_t)voff + soff;
  const int unit = BYTES < 4 ? BYTES : 4;
  for (int i = 0; i < BYTES; i += unit) {
    if (off + i + unit <= r.num) {
      check_load(r.base + off + i, unit, aux);
      memcpy(static_cast<char*>(out) + i, r.base + off + i, unit);
    } else {
      memset(static_cast<char*>(out) + i, 0, unit);
    }
  }
}
template <int BYTES>
inline void buffer_store(emu_rsrc r, uint32_t voff, uint32_t soff, const void* in, int aux) {
  vm_issue();
  range_rules_agree(r, voff, soff, BYTES);
  const uint64_t off = (uint64_t)voff + soff;
  for (int i = 0; i < BYTES; i += 4)
    if (off + i + 4 <= r.num) {
      note_store(r.base + off + i, 4, aux);
      memcpy(const_cast<char*>(r.base) + off + i, static_cast<const char*>(in) + i, 4);
    }
}
inline emu_u32x4 load_b128(emu_rsrc r, uint32_t v, uint32_t s, int a) { emu_u32x4 o; buffer_load<16>(r, v, s, &o, a); return o; }
inline emu_u32x2 load_b64(emu_rsrc r, uint32_t v, uint32_t s, int a) { emu_u32x2 o; buffer_load<8>(r, v, s, &o, a); return o; }
inline uint32_t load_b32(emu_rsrc r, uint32_t v, uint32_t s, int a) { uint32_t o; buffer_load<4>(r, v, s, &o, a); return o; }
inline uint16_t load_b16(emu_rsrc r, uint32_t v, uint32_t s, int a) { uint16_t o; buffer_load<2>(r, v, s, &o, a); return o; }
inline void store_b32(uint32_t x, emu_rsrc r, uint32_t v, uint32_t s, int a) { buffer_store<4>(r, v, s, &x, a); }
inline void store_b64(emu_u32x2 x, emu_rsrc r, uint32_t v, uint32_t s, int a) { buffer_store<8>(r, v, s, &x, a); }
// Direct-to-LDS load: lane l's `size` bytes go to lds + offset + l * size once
// a later wait covers the copy (vm_copy_to_lds).
inline void load_lds(emu_rsrc r, void* lds, int size, uint32_t v, uint32_t s, int imm, int aux) {
  char* dst = static_cast<char*>(lds) + imm + lane_id() * size;
  char data[16];
  range_rules_agree(r, (uint64_t)v + imm, s, size);
  const uint64_t off = (uint64_t)v + imm + s;
  if (size != 16 && size != 4 && size != 2) __builtin_trap();
  const int unit = size < 4 ? size : 4;
  for (int i = 0; i < size; i += unit) {
    if (off + i + unit <= r.num) {
      check_load(r.base + off + i, unit, aux);
      memcpy(data + i, r.base + off + i, unit);
    } else {
      memset(data + i, 0, unit);
    }
  }
  vm_copy_to_lds(dst, data, size);
}

// v_perm_b32: bytes 0-3 of the pool are src1, 4-7 src0; selector bytes 8-11
// replicate a sign bit, 12 gives 0x00, 13 and above 0xff.
inline uint32_t perm(uint32_t s0, uint32_t s1, uint32_t sel) {
  const uint64_t pool = ((uint64_t)s0 << 32) | s1;
  uint32_t out = 0;
  for (int i = 0; i < 4; ++i) {
    const uint32_t b = (sel >> (8 * i)) & 0xff;
    uint32_t v;
    if (b < 8) v = (pool >> (8 * b)) & 0xff;
    else if (b < 12) v = ((pool >> (16 * (b - 8) + 15)) & 1) ? 0xff : 0x00;
    else if (b == 12) v = 0x00;
    else v = 0xff;
    out |= v << (8 * i);
  }
  return out;
}

inline float bf16_bits_to_f32(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}
inline float fdot2_bf16(emu_s16x2 a, emu_s16x2 b, float c, bool) {
  return bf16_bits_to_f32((uint16_t)a[0]) * bf16_bits_to_f32((uint16_t)b[0]) +
         bf16_bits_to_f32((uint16_t)a[1]) * bf16_bits_to_f32((uint16_t)b[1]) + c;
}
template <class T>
inline T atomic_or(T* p, T v) { const T old = *p; *p = old | v; return old; }
template <class T>
inline void atomic_store(T* p, T v) { *p = v; }
template <class T>
inline T atomic_load(const T* p) { return *p; }

}  // namespace emu

#define threadIdx (*emu::cur_tid())
#define blockIdx (*emu::cur_bid())
#define gridDim (emu::g_grid_dim)
#define blockDim (emu::g_block_dim)

#define __syncthreads() emu::syncthreads()
#define __shfl_xor(v, m, w) emu::shfl_xor((v), (m), (w))
#define __expf(x) expf(x)
#define __uint_as_float(u) __builtin_bit_cast(float, (uint32_t)(u))
#define __float_as_uint(f) __builtin_bit_cast(uint32_t, (float)(f))

#define __builtin_amdgcn_make_buffer_rsrc emu::make_rsrc
#define __builtin_amdgcn_raw_buffer_load_b128 emu::load_b128
#define __builtin_amdgcn_raw_buffer_load_b64 emu::load_b64
#define __builtin_amdgcn_raw_buffer_load_b32 emu::load_b32
#define __builtin_amdgcn_raw_buffer_load_b16 emu::load_b16
#define __builtin_amdgcn_raw_buffer_store_b32 emu::store_b32
#define __builtin_amdgcn_raw_buffer_store_b64 emu::store_b64
#define __builtin_amdgcn_raw_ptr_buffer_load_lds emu::load_lds
#define __builtin_amdgcn_perm emu::perm
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
#define __builtin_amdgcn_fdot2_f32_bf16 emu::fdot2_bf16
#define __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, cbsz, abid, blgp) emu::mfma_16x16x32_bf16((a), (b), (c))
#define __builtin_amdgcn_ballot_w64(p) emu::ballot(p)
#define __builtin_amdgcn_readfirstlane(v) ((int)emu::readfirstlane((uint32_t)(v)))
#define __builtin_amdgcn_sched_barrier(m) ((void)0)
#define __builtin_amdgcn_s_setprio(p) ((void)0)
#define __builtin_amdgcn_s_waitcnt(c) emu::waitcnt(c)

#define __HIP_MEMORY_SCOPE_AGENT 3
#define __hip_atomic_fetch_or(p, v, order, scope) emu::atomic_or((p), (v))
#define __hip_atomic_store(p, v, order, scope) emu::atomic_store((p), (v))
#define __hip_atomic_load(p, order, scope) emu::atomic_load((p))

#define hipLaunchKernelGGL(kernel, grid, block, lds, stream, ...) \
  emu::launch(#kernel, dim3(grid), dim3(block), (size_t)(lds), [=]() { kernel(__VA_ARGS__); })
#define HIP_SYMBOL(s) (&(s))
inline hipError_t hipGetLastError() { return emu::last_error(); }
inline hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
inline hipError_t hipGetSymbolAddress(void** p, const void* sym) { *p = const_cast<void*>(sym); return hipSuccess; }
// Stream capture, as the host sees it: emu_set_capturing (emu_runtime.cpp)
// makes every stream report that it is capturing a graph.
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
namespace emu { extern int g_capturing; }
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st) {
  *st = emu::g_capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}
inline hipError_t hipStreamGetCaptureInfo(hipStream_t, hipStreamCaptureStatus* st, unsigned long long* id) {
  *st = emu::g_capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  *id = emu::g_capturing ? (unsigned long long)emu::g_capturing : 0ull;
  return hipSuccess;
}
// Launches run to completion when they are made, so a stream is always idle.
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
enum hipMemcpyKind { hipMemcpyDeviceToHost = 2 };
inline hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind) { memcpy(dst, src, n); return hipSuccess; }
