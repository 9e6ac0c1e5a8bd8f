// Wave emulator for running the gfx950 kernels on the CPU (tests only).
//
// Every GPU thread is a fiber with its own stack.  A fiber runs until it
// reaches a collective operation (MFMA, ballot, readfirstlane, shuffle: the
// 64 lanes of its wave meet) or __syncthreads (every live thread of the
// workgroup meets), then yields.  The last lane to arrive computes the
// operation for the whole wave.  Lanes that return leave the set a
// collective or barrier waits for, as exited waves do on the hardware.
//
// Workgroups are dispatched in order (x fastest, then y; or the reverse) into
// a number of resident slots (both set by emu_set_concurrency): one by
// default, so workgroups run one after another, or more, so that resident
// workgroups interleave at every meeting point -- a decode split-K finisher
// then polls while its publishers still run.  Every workgroup has its own
// LDS, static arrays included (static_lds).
//
// Lanes of one wave that reach different collectives, a state in which no
// live thread can move, or a kernel that touches memory outside its buffers
// (guard pages around every emu_alloc buffer and the dynamic LDS) stop the
// process with a message naming the kernel, workgroup and thread.
#include <hip/hip_runtime.h>

#include <signal.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <deque>
#include <unordered_map>
#include <vector>

namespace {

constexpr size_t kStackBytes = 128 * 1024;
constexpr int kMaxThreads = 1024;
constexpr size_t kMaxDynLds = 160 * 1024;
constexpr size_t kLdsBytes = 160 * 1024;  // LDS one gfx950 workgroup can hold

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

struct Block;

struct Lane {
  Block* blk = nullptr;
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

struct Block {
  emu_uint3 bid{0, 0, 0};
  int nt = 0, alive = 0, bar_arrived = 0;
  uint64_t bar_seq = 0, bar_done = 0;
  std::vector<Lane*> lanes;
  std::vector<int> order;
  Wave waves[kMaxThreads / 64];
  char* lds = nullptr;
  char* lds_map = nullptr;
  size_t lds_map_bytes = 0;
  size_t dyn_bytes = 0;
  // Static LDS objects of the kernel (__shared__ arrays), one guarded,
  // poisoned allocation each per workgroup.
  struct StaticLds {
    int id;
    char* p;
    char* map;
    size_t map_bytes, bytes;
  };
  std::vector<StaticLds> statics;
  size_t static_bytes = 0;
};

std::vector<Lane*> g_free_lanes;
Lane* g_cur = nullptr;
void* g_sched_sp = nullptr;
const std::function<void()>* g_body = nullptr;
const char* g_kernel = "";
hipError_t g_error = hipSuccess;
// Order in which the scheduler visits a workgroup's threads each round:
// 0 ascending, 1 descending, 2 a fresh pseudo-random permutation per round.
// Results of a kernel without intra-workgroup races do not depend on it.
int g_schedule = 0;
uint64_t g_sched_state = 1;
int g_concurrency = 1;     // resident workgroups of a decode-kernel launch
bool g_reverse = false;    // dispatch the last workgroup first

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
  const Block* b = g_cur ? g_cur->blk : nullptr;
  fprintf(stderr, "emu: %s in %s, workgroup (%u, %u), thread %u\n", what, g_kernel, b ? b->bid.x : 0u,
          b ? b->bid.y : 0u, g_cur ? g_cur->tid.x : 0u);
  fflush(stderr);
  _exit(97);
}

void yield() { emu_ctx_switch(&g_cur->sp, g_sched_sp); }

void compute(Wave& w) {
  switch (w.kind) {
    case kMfma: {
      // D[m][n] = sum_k A[m][k] B[k][n] + C[m][n]; lane l holds A[l%16][8(l/16)+j],
      // B[8(l/16)+j][l%16] and D[4(l/16)+r][l%16].  The matrix cores read every lane.
      for (int l = 0; l < 64; ++l)
        if (!w.present[l]) fail("MFMA issued by a wave with exited lanes");
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
      // The kernels use readfirstlane to move a wave-uniform value into a
      // scalar register; a value that differs between lanes is a bug there.
      int first = -1;
      for (int l = 0; l < 64 && first < 0; ++l)
        if (w.present[l]) first = l;
      for (int l = 0; l < 64; ++l)
        if (w.present[l] && w.in[l].u != w.in[first].u) fail("readfirstlane of a value that differs between lanes");
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
  Wave& w = me->blk->waves[me->tid.x / 64];
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
  Lane& me = *g_cur;
  Block& b = *me.blk;
  land(me, ~0ull);
  me.done = true;
  --b.alive;
  Wave& w = b.waves[me.tid.x / 64];
  --w.alive;
  if (w.arrived > 0 && w.arrived == w.alive) compute(w);
  if (b.bar_arrived > 0 && b.bar_arrived == b.alive) {
    b.bar_done = b.bar_seq;
    b.bar_arrived = 0;
  }
  emu_ctx_switch(&me.sp, g_sched_sp);
  __builtin_trap();
}

// Fiber stack: the return address of the first switch is the trampoline.
void init_lane(Lane& L) {
  if (!L.stack) {
    L.stack = static_cast<char*>(mmap(nullptr, kStackBytes, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
    if (L.stack == MAP_FAILED) fail("stack allocation failed");
  }
  uintptr_t top = (reinterpret_cast<uintptr_t>(L.stack) + kStackBytes) & ~(uintptr_t)15;
  void** sp = reinterpret_cast<void**>(top);
  *--sp = nullptr;                               // alignment slot: trampoline entered with rsp % 16 == 8
  *--sp = reinterpret_cast<void*>(&trampoline);  // ret target
  for (int i = 0; i < 6; ++i) *--sp = nullptr;   // rbp rbx r12-r15
  L.sp = sp;
  L.done = false;
  L.wait_kind = 0;
  L.coll_seq = L.bar_seq = 0;
  L.vm_issued = 0;
  L.pending.clear();
}

bool ready(const Lane& L) {
  if (L.done) return false;
  if (L.wait_kind == 1) return L.blk->waves[L.tid.x / 64].completed >= L.coll_seq;
  if (L.wait_kind == 2) return L.blk->bar_done >= L.bar_seq;
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
void* guarded(size_t bytes, size_t* mapped, char** base = nullptr, bool front = false) {
  const size_t page = 4096;
  const size_t body = (bytes + page - 1) / page * page;
  const size_t total = body + 2 * page;
  char* m = static_cast<char*>(mmap(nullptr, total, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0));
  if (m == MAP_FAILED) return nullptr;
  mprotect(m, page, PROT_NONE);
  mprotect(m + page + body, page, PROT_NONE);
  *mapped = total;
  if (base) *base = m;
  return front ? m + page : m + page + body - bytes;
}

Block* start_block(emu_uint3 bid, int nt, size_t dyn) {
  Block* b = new Block();
  b->bid = bid;
  b->nt = b->alive = nt;
  b->dyn_bytes = dyn;
  if (dyn > 0) {
    b->lds = static_cast<char*>(guarded(dyn, &b->lds_map_bytes, &b->lds_map));
    memset(b->lds, 0xA5, dyn);  // LDS starts undefined: make stale reads visible
  }
  for (int w = 0; w < (nt + 63) / 64; ++w) b->waves[w].alive = std::min(64, nt - 64 * w);
  for (int t = 0; t < nt; ++t) {
    Lane* L;
    if (!g_free_lanes.empty()) {
      L = g_free_lanes.back();
      g_free_lanes.pop_back();
    } else {
      L = new Lane();
    }
    init_lane(*L);
    L->tid = emu_uint3{(unsigned)t, 0, 0};
    L->blk = b;
    b->lanes.push_back(L);
    b->order.push_back(g_schedule == 1 ? nt - 1 - t : t);
  }
  return b;
}

void finish_block(Block* b) {
  for (Lane* L : b->lanes) g_free_lanes.push_back(L);
  if (b->lds_map) munmap(b->lds_map, b->lds_map_bytes);
  for (auto& st : b->statics) munmap(st.map, st.map_bytes);
  delete b;
}

// One round over a block's ready threads; returns whether any ran.
bool run_round(Block& b) {
  if (g_schedule == 2)
    for (int t = b.nt - 1; t > 0; --t) {
      g_sched_state = g_sched_state * 6364136223846793005ull + 1442695040888963407ull;
      std::swap(b.order[t], b.order[(g_sched_state >> 33) % (uint64_t)(t + 1)]);
    }
  bool progressed = false;
  for (int oi = 0; oi < b.nt; ++oi) {
    Lane& L = *b.lanes[b.order[oi]];
    if (!ready(L)) continue;
    L.wait_kind = 0;
    g_cur = &L;
    emu_ctx_switch(&g_sched_sp, L.sp);
    g_cur = nullptr;
    progressed = true;
  }
  return progressed;
}

}  // namespace

namespace emu {
extern std::unordered_map<uintptr_t, std::pair<uint64_t, bool>> g_written;  // coherence audit, below

emu_uint3 g_grid_dim{1, 1, 1}, g_block_dim{1, 1, 1};

const emu_uint3* cur_tid() { return &g_cur->tid; }
const emu_uint3* cur_bid() { return &g_cur->blk->bid; }
int lane_id() { return g_cur->tid.x & 63; }
void* dyn_lds() { return g_cur->blk->lds; }

// The workgroup's static LDS object `id` (one per __shared__ declarator of
// the source) of `bytes` bytes: allocated, guarded and poisoned on the first
// thread's call, shared by the workgroup's other threads.  Static plus
// dynamic LDS must fit the 160 KB a gfx950 workgroup can hold.
void* static_lds(int id, size_t bytes) {
  Block* b = g_cur->blk;
  for (auto& st : b->statics)
    if (st.id == id) {
      if (st.bytes != bytes) fail("static LDS object declared with two sizes");
      return st.p;
    }
  Block::StaticLds st{};
  st.id = id;
  st.bytes = bytes;
  st.p = static_cast<char*>(guarded(bytes, &st.map_bytes, &st.map));
  memset(st.p, 0xA5, bytes);
  b->statics.push_back(st);
  b->static_bytes += bytes;
  if (b->static_bytes + b->dyn_bytes > kLdsBytes) fail("static plus dynamic LDS exceeds 160 KB per workgroup");
  return st.p;
}
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

void range_ambiguous() {
  fail("buffer access in range by one reading of the range check and out of range by another (soffset counted or not, straddling num_records, or a 32-bit offset wrap)");
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
  Block& b = *me->blk;
  const uint64_t seq = ++me->bar_seq;
  if (b.bar_arrived == 0) b.bar_seq = seq;
  else if (b.bar_seq != seq) fail("threads reached different barriers");
  if (++b.bar_arrived == b.alive) {
    b.bar_done = seq;
    b.bar_arrived = 0;
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
  g_written.clear();
  g_grid_dim = emu_uint3{grid.x, grid.y, 1};
  g_block_dim = emu_uint3{block.x, 1, 1};
  g_body = &body;
  const int slots = std::max(1, g_concurrency);
  const uint64_t nblocks = (uint64_t)grid.x * grid.y;
  uint64_t next = 0;
  std::deque<Block*> resident;
  auto dispatch = [&]() {
    while ((int)resident.size() < slots && next < nblocks) {
      const uint64_t lin = g_reverse ? nblocks - 1 - next : next;
      ++next;
      resident.push_back(start_block(emu_uint3{(unsigned)(lin % grid.x), (unsigned)(lin / grid.x), 0}, nt, dyn));
    }
  };
  dispatch();
  while (!resident.empty()) {
    bool progressed = false;
    for (size_t i = 0; i < resident.size(); ++i) progressed |= run_round(*resident[i]);
    for (size_t i = 0; i < resident.size();) {
      if (resident[i]->alive == 0) {
        finish_block(resident[i]);
        resident.erase(resident.begin() + i);
      } else {
        ++i;
      }
    }
    dispatch();
    if (!progressed && !resident.empty()) {
      g_cur = resident.front()->lanes.front();
      fail("deadlock: every live thread waits at a collective or barrier that cannot complete");
    }
  }
}

}  // namespace emu

namespace emu {
int g_capturing = 0;
uint64_t g_loads = 0;  // fibers run one at a time: no atomics needed
void count_load() { ++g_loads; }

// Coherence audit: dword address -> (writing workgroup + 1, store was
// agent-coherent), for the current launch only (reset by launch()).
constexpr int kCoherentBit = 16;
std::unordered_map<uintptr_t, std::pair<uint64_t, bool>> g_written;
uint64_t cur_block_id() {
  const Block* b = g_cur ? g_cur->blk : nullptr;
  return b ? (uint64_t)b->bid.y * g_grid_dim.x + b->bid.x + 1 : 0;
}
void note_store(const char* p, int bytes, int aux) {
  for (int i = 0; i < bytes; i += 4)
    g_written[(uintptr_t)(p + i) & ~(uintptr_t)3] = {cur_block_id(), (aux & kCoherentBit) != 0};
}
void check_load(const char* p, int bytes, int aux) {
  if (g_written.empty()) return;
  for (int i = 0; i < bytes; i += 4) {
    const auto it = g_written.find((uintptr_t)(p + i) & ~(uintptr_t)3);
    if (it == g_written.end() || it->second.first == cur_block_id()) continue;
    if (!(aux & kCoherentBit) || !it->second.second)
      fail("a workgroup read data another workgroup stored in the same launch without agent-coherent accesses on "
           "both sides (on the chip the load can hit a stale line of its own cache)");
  }
}
}  // namespace emu

extern "C" void emu_set_capturing(int on) { emu::g_capturing = on; }
extern "C" uint64_t emu_load_count() { return emu::g_loads; }
extern "C" void emu_reset_load_count() { emu::g_loads = 0; }

// Scheduling order of the threads of a workgroup (see g_schedule).
extern "C" void emu_set_schedule(int mode, uint64_t seed) {
  g_schedule = mode;
  g_sched_state = seed * 2 + 1;
}

// Resident workgroups of decode-kernel launches (1: one after another), and
// whether workgroups are dispatched last-first.
extern "C" void emu_set_concurrency(int slots, int reverse) {
  g_concurrency = slots;
  g_reverse = reverse != 0;
}

// Test-side allocation of "device" buffers with guard pages; every mapping
// is recorded so that emu_free_all can release them between tests.
namespace {
std::vector<std::pair<char*, size_t>> g_buffers;

void* test_buffer(size_t bytes, bool front) {
  size_t mapped = 0;
  char* base = nullptr;
  void* p = guarded(bytes == 0 ? 1 : bytes, &mapped, &base, front);
  if (p) g_buffers.emplace_back(base, mapped);
  return p;
}
}  // namespace

extern "C" void* emu_alloc(size_t bytes) { return test_buffer(bytes, false); }

// As emu_alloc, but the guard page precedes the buffer (catches underflow).
extern "C" void* emu_alloc_front(size_t bytes) { return test_buffer(bytes, true); }

// Unmap every buffer emu_alloc / emu_alloc_front returned.
extern "C" void emu_free_all() {
  for (auto& b : g_buffers) munmap(b.first, b.second);
  g_buffers.clear();
}
