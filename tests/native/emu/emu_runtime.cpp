// Wave emulator for running the gfx950 kernels on the CPU (tests only).
//
// A launch runs its workgroups one after another in dispatch order (x
// fastest, then y).  Inside a workgroup every thread is a fiber with its own
// stack; a fiber runs until it reaches a collective operation (MFMA, ballot,
// readfirstlane, shuffle: the 64 lanes of its wave meet) or __syncthreads
// (every live thread of the workgroup meets), then yields.  The last lane
// to arrive computes the operation for the whole wave.  Lanes that return
// leave the set a collective or barrier waits for, as exited waves do on the
// hardware.  Lanes of one wave that reach different collectives, a barrier
// that can never complete, or a kernel that touches memory outside its
// buffers (guard pages around every emu_alloc buffer and the dynamic LDS)
// stop the process with a message naming the kernel, workgroup and thread.
#include <hip/hip_runtime.h>

#include <signal.h>
#include <stdio.h>
#include <stdlib.h>
#include <sys/mman.h>
#include <unistd.h>

#include <vector>

namespace {

constexpr size_t kStackBytes = 256 * 1024;
constexpr int kMaxThreads = 1024;
constexpr size_t kMaxDynLds = 160 * 1024;

enum Coll { kNone = 0, kMfma, kBallot, kFirst, kShfl };

struct Payload {
  emu_bf16x8 a, b;
  emu_f32x4 c;
  uint64_t u;
  float f;
  int mask, width;
};

struct PendingCopy {
  uint64_t issue;
  char* dst;
  char data[16];
  int bytes;
};

struct Lane {
  uint64_t vm_issued = 0;
  std::vector<PendingCopy> pending;  // direct-to-LDS copies not yet landed
  void* sp = nullptr;
  char* stack = nullptr;
  emu_uint3 tid{0, 0, 0};
  bool done = false;
  int wait_kind = 0;  // 0 running, 1 collective, 2 barrier
  uint64_t coll_seq = 0, bar_seq = 0;
};

struct Wave {
  int alive = 0, arrived = 0;
  uint64_t seq = 0, completed = 0;
  int kind = kNone;
  Payload in[64];
  Payload out[64];
  bool present[64];
};

Lane g_lanes[kMaxThreads];
Wave g_waves[kMaxThreads / 64];
int g_nthreads = 0, g_alive = 0, g_bar_arrived = 0;
uint64_t g_bar_seq = 0, g_bar_done = 0;
Lane* g_cur = nullptr;
void* g_sched_sp = nullptr;
const std::function<void()>* g_body = nullptr;
char* g_lds = nullptr;
size_t g_lds_map = 0;
const char* g_kernel = "";
hipError_t g_error = hipSuccess;
// Order in which the scheduler visits a workgroup's threads each round:
// 0 ascending, 1 descending, 2 a fresh pseudo-random permutation per round.
// Results of a kernel without intra-workgroup races do not depend on it.
int g_schedule = 0;
uint64_t g_sched_state = 1;

extern "C" void emu_ctx_switch(void** save_sp, void* new_sp);
asm(R"(
  .text
  .globl emu_ctx_switch
  .type emu_ctx_switch,@function
emu_ctx_switch:
  pushq %rbp
  pushq %rbx
  pushq %r12
  pushq %r13
  pushq %r14
  pushq %r15
  movq %rsp, (%rdi)
  movq %rsi, %rsp
  popq %r15
  popq %r14
  popq %r13
  popq %r12
  popq %rbx
  popq %rbp
  ret
  .size emu_ctx_switch, .-emu_ctx_switch
)");

[[noreturn]] void fail(const char* what) {
  fprintf(stderr, "emu: %s in %s, workgroup (%u, %u), thread %u\n", what, g_kernel, emu::g_block_idx.x,
          emu::g_block_idx.y, g_cur ? g_cur->tid.x : 0u);
  fflush(stderr);
  _exit(97);
}

void yield() { emu_ctx_switch(&g_cur->sp, g_sched_sp); }

void compute(Wave& w) {
  switch (w.kind) {
    case kMfma: {
      // D[m][n] = sum_k A[m][k] B[k][n] + C[m][n]; lane l holds A[l%16][8(l/16)+j],
      // B[8(l/16)+j][l%16] and D[4(l/16)+r][l%16].
      float A[16][32], B[32][16], C[16][16];
      for (int l = 0; l < 64; ++l)
        for (int j = 0; j < 8; ++j) {
          A[l % 16][8 * (l / 16) + j] = (float)w.in[l].a[j];
          B[8 * (l / 16) + j][l % 16] = (float)w.in[l].b[j];
        }
      for (int l = 0; l < 64; ++l)
        for (int r = 0; r < 4; ++r) C[4 * (l / 16) + r][l % 16] = w.in[l].c[r];
      for (int m = 0; m < 16; ++m)
        for (int n = 0; n < 16; ++n) {
          float s = 0.f;
          for (int k = 0; k < 32; ++k) s += A[m][k] * B[k][n];
          C[m][n] += s;
        }
      for (int l = 0; l < 64; ++l)
        for (int r = 0; r < 4; ++r) w.out[l].c[r] = C[4 * (l / 16) + r][l % 16];
      break;
    }
    case kBallot: {
      uint64_t bits = 0;
      for (int l = 0; l < 64; ++l)
        if (w.present[l] && w.in[l].u) bits |= 1ull << l;
      for (int l = 0; l < 64; ++l) w.out[l].u = bits;
      break;
    }
    case kFirst: {
      int first = -1;
      for (int l = 0; l < 64 && first < 0; ++l)
        if (w.present[l]) first = l;
      for (int l = 0; l < 64; ++l) w.out[l].u = w.in[first].u;
      break;
    }
    case kShfl:
      for (int l = 0; l < 64; ++l) {
        const int src = (l ^ w.in[l].mask) & 63;
        w.out[l].f = (w.present[src] && (src / w.in[l].width) == (l / w.in[l].width)) ? w.in[src].f : w.in[l].f;
      }
      break;
  }
  for (int l = 0; l < 64; ++l) w.present[l] = false;
  w.arrived = 0;
  w.completed = w.seq;
  w.kind = kNone;
}

// The calling lane's part of a wave collective.
Payload& collective(int kind, const Payload& p) {
  Lane* me = g_cur;
  const int lane = me->tid.x & 63;
  Wave& w = g_waves[me->tid.x / 64];
  const uint64_t seq = ++me->coll_seq;
  if (w.arrived == 0) {
    w.seq = seq;
    w.kind = kind;
  } else if (w.seq != seq || w.kind != kind) {
    fail("lanes of one wave reached different collective operations");
  }
  w.in[lane] = p;
  w.present[lane] = true;
  if (++w.arrived == w.alive) {
    compute(w);
  } else {
    me->wait_kind = 1;
    yield();
  }
  return w.out[lane];
}

void land(Lane& L, uint64_t upto) {
  size_t keep = 0;
  for (size_t i = 0; i < L.pending.size(); ++i) {
    PendingCopy& c = L.pending[i];
    if (c.issue < upto)
      memcpy(c.dst, c.data, c.bytes);
    else
      L.pending[keep++] = c;
  }
  L.pending.resize(keep);
}

void trampoline() {
  (*g_body)();
  land(*g_cur, ~0ull);
  g_cur->done = true;
  --g_alive;
  Wave& w = g_waves[g_cur->tid.x / 64];
  --w.alive;
  if (w.arrived > 0 && w.arrived == w.alive) compute(w);
  if (g_bar_arrived > 0 && g_bar_arrived == g_alive) {
    g_bar_done = g_bar_seq;
    g_bar_arrived = 0;
  }
  emu_ctx_switch(&g_cur->sp, g_sched_sp);
  __builtin_trap();
}

// Fiber stack: return address of the first switch is the trampoline.
void init_lane(Lane& L) {
  if (!L.stack) {
    L.stack = static_cast<char*>(mmap(nullptr, kStackBytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
    if (L.stack == MAP_FAILED) fail("stack allocation failed");
  }
  uintptr_t top = (reinterpret_cast<uintptr_t>(L.stack) + kStackBytes) & ~(uintptr_t)15;
  void** sp = reinterpret_cast<void**>(top);
  *--sp = nullptr;                                  // alignment slot: trampoline entered with rsp % 16 == 8
  *--sp = reinterpret_cast<void*>(&trampoline);     // ret target
  for (int i = 0; i < 6; ++i) *--sp = nullptr;      // rbp rbx r12-r15
  L.sp = sp;
  L.done = false;
  L.wait_kind = 0;
  L.coll_seq = L.bar_seq = 0;
  L.vm_issued = 0;
  L.pending.clear();
}

bool ready(const Lane& L) {
  if (L.done) return false;
  if (L.wait_kind == 1) return g_waves[L.tid.x / 64].completed >= L.coll_seq;
  if (L.wait_kind == 2) return g_bar_done >= L.bar_seq;
  return true;
}

void segv_handler(int, siginfo_t* info, void*) {
  char buf[256];
  snprintf(buf, sizeof buf, "memory access outside every buffer at %p", info->si_addr);
  fail(buf);
}

struct InstallHandler {
  InstallHandler() {
    struct sigaction sa{};
    sa.sa_sigaction = segv_handler;
    sa.sa_flags = SA_SIGINFO | SA_ONSTACK;
    static char alt[64 * 1024];
    stack_t ss{};
    ss.ss_sp = alt;
    ss.ss_size = sizeof alt;
    sigaltstack(&ss, nullptr);
    sigaction(SIGSEGV, &sa, nullptr);
    sigaction(SIGBUS, &sa, nullptr);
  }
} g_install;

// `bytes` of memory between two inaccessible pages.  By default the buffer
// ends where the trailing guard page begins, so reads or writes past the end
// fault; with `front` it starts right after the leading guard page, so
// accesses before the start fault.
void* guarded(size_t bytes, size_t* mapped, bool front = false) {
  const size_t page = 4096;
  const size_t body = (bytes + page - 1) / page * page;
  const size_t total = body + 2 * page;
  char* m = static_cast<char*>(mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
  if (m == MAP_FAILED) return nullptr;
  mprotect(m, page, PROT_NONE);
  mprotect(m + page + body, page, PROT_NONE);
  *mapped = total;
  return front ? m + page : m + page + body - bytes;
}

}  // namespace

namespace emu {

emu_uint3 g_block_idx{0, 0, 0}, g_grid_dim{1, 1, 1}, g_block_dim{1, 1, 1};

const emu_uint3* cur_tid() { return &g_cur->tid; }
int lane_id() { return g_cur->tid.x & 63; }
void* dyn_lds() { return g_lds; }
hipError_t last_error() {
  const hipError_t e = g_error;
  g_error = hipSuccess;
  return e;
}

emu_f32x4 mfma_16x16x32_bf16(emu_bf16x8 a, emu_bf16x8 b, emu_f32x4 c) {
  Payload p{};
  p.a = a;
  p.b = b;
  p.c = c;
  return collective(kMfma, p).c;
}
uint64_t ballot(bool pred) {
  Payload p{};
  p.u = pred ? 1 : 0;
  return collective(kBallot, p).u;
}
uint32_t readfirstlane(uint32_t v) {
  Payload p{};
  p.u = v;
  return (uint32_t)collective(kFirst, p).u;
}
float shfl_xor(float v, int mask, int width) {
  Payload p{};
  p.f = v;
  p.mask = mask;
  p.width = width;
  return collective(kShfl, p).f;
}

void vm_issue() { ++g_cur->vm_issued; }

void vm_copy_to_lds(void* dst, const void* src, int bytes) {
  PendingCopy c;
  c.issue = g_cur->vm_issued++;
  c.dst = static_cast<char*>(dst);
  memcpy(c.data, src, bytes);
  c.bytes = bytes;
  g_cur->pending.push_back(c);
}

// s_waitcnt: the vmcnt field is bits 3:0 and 15:14 (6 bits); ops complete in
// issue order, so all but the `n` youngest have landed after the wait.
void waitcnt(int code) {
  const uint64_t n = (uint64_t)((code & 15) | (((code >> 14) & 3) << 4));
  Lane& L = *g_cur;
  if (L.vm_issued >= n) land(L, L.vm_issued - n);
}

void syncthreads() {
  Lane* me = g_cur;
  const uint64_t seq = ++me->bar_seq;
  if (g_bar_arrived == 0) g_bar_seq = seq;
  else if (g_bar_seq != seq) fail("threads reached different barriers");
  if (++g_bar_arrived == g_alive) {
    g_bar_done = seq;
    g_bar_arrived = 0;
  } else {
    me->wait_kind = 2;
    yield();
  }
}

void launch(const char* name, dim3 grid, dim3 block, size_t dyn, const std::function<void()>& body) {
  const int nt = (int)(block.x * block.y * block.z);
  g_kernel = name;
  if (nt <= 0 || nt > kMaxThreads || block.y != 1 || block.z != 1 || dyn > kMaxDynLds || grid.z != 1 ||
      grid.x == 0 || grid.y == 0) {
    fprintf(stderr, "emu: invalid launch of %s (grid %u x %u, block %u, lds %zu)\n", name, grid.x, grid.y, block.x, dyn);
    g_error = hipErrorInvalidValue;
    return;
  }
  size_t map = 0;
  char* lds_map_base = nullptr;
  if (dyn > 0) {
    g_lds = static_cast<char*>(guarded(dyn, &map));
    lds_map_base = g_lds + dyn - (map - 4096);  // start of the mapping
  } else {
    g_lds = nullptr;
  }
  g_grid_dim = emu_uint3{grid.x, grid.y, 1};
  g_block_dim = emu_uint3{block.x, 1, 1};
  g_body = &body;
  for (unsigned by = 0; by < grid.y; ++by)
    for (unsigned bx = 0; bx < grid.x; ++bx) {
      g_block_idx = emu_uint3{bx, by, 0};
      if (g_lds) memset(g_lds, 0xA5, dyn);  // LDS starts undefined: make stale reads visible
      g_nthreads = g_alive = nt;
      g_bar_arrived = 0;
      g_bar_seq = g_bar_done = 0;
      for (int w = 0; w < (nt + 63) / 64; ++w) {
        g_waves[w] = Wave{};
        g_waves[w].alive = std::min(64, nt - 64 * w);
      }
      for (int t = 0; t < nt; ++t) {
        init_lane(g_lanes[t]);
        g_lanes[t].tid = emu_uint3{(unsigned)t, 0, 0};
      }
      std::vector<int> order(nt);
      for (int t = 0; t < nt; ++t) order[t] = g_schedule == 1 ? nt - 1 - t : t;
      while (g_alive > 0) {
        bool progressed = false;
        if (g_schedule == 2)
          for (int t = nt - 1; t > 0; --t) {
            g_sched_state = g_sched_state * 6364136223846793005ull + 1442695040888963407ull;
            std::swap(order[t], order[(g_sched_state >> 33) % (uint64_t)(t + 1)]);
          }
        for (int oi = 0; oi < nt; ++oi) {
          Lane& L = g_lanes[order[oi]];
          if (!ready(L)) continue;
          L.wait_kind = 0;
          g_cur = &L;
          emu_ctx_switch(&g_sched_sp, L.sp);
          g_cur = nullptr;
          progressed = true;
        }
        if (!progressed) fail("deadlock: every live thread waits at a collective or barrier that cannot complete");
      }
    }
  if (lds_map_base) munmap(lds_map_base, map);
  g_lds = nullptr;
}

}  // namespace emu

// Scheduling order of the threads of a workgroup (see g_schedule).
extern "C" void emu_set_schedule(int mode, uint64_t seed) {
  g_schedule = mode;
  g_sched_state = seed * 2 + 1;
}

// Test-side allocation of "device" buffers with guard pages.
extern "C" void* emu_alloc(size_t bytes) {
  size_t mapped = 0;
  return guarded(bytes == 0 ? 1 : bytes, &mapped);
}

// As emu_alloc, but the guard page precedes the buffer (catches underflow).
extern "C" void* emu_alloc_front(size_t bytes) {
  size_t mapped = 0;
  return guarded(bytes == 0 ? 1 : bytes, &mapped, true);
}
