// Host-side invariants of the launch planner in inf-engine_amd/csrc/w4a16_kernels.hip,
// checked on the CPU over a sweep of shapes (single, grouped and SwiGLU-pair
// calls).  The planner decides grids, K splits, LDS and workspace layout; a
// mistake there turns into out-of-range device accesses or a split-K finisher
// waiting for a partial nobody publishes, so every property the kernels rely
// on is asserted here:
//   * the K split covers every group exactly (nsplit * gps >= G, no empty split);
//   * workgroup ranges of the problems are contiguous and split-major, so every
//     split-K finisher is dispatched after the workgroups it waits for;
//   * LDS fits the CU and holds the wave reduction;
//   * workspace regions are disjoint, the decode slots stay in the lower half,
//     the GEMM scratch in the upper half, and neither reaches the status word;
//   * w4a16_workspace_size() is enough for the plan an aligned call gets;
//   * FULL (unconditional-load) plans satisfy the alignment the kernels assume.
// Built by tests/test_plan_check.py with hipcc (the TU includes the kernel
// source, so it compiles the device code too); runs no HIP call.  Prints "ok".
#include "../../inf-engine_amd/csrc/w4a16_kernels.hip"

#include <cstdio>
#include <vector>

static int failures = 0;
static char ctx[256];
#define CHECK(c)                                                        \
  do {                                                                  \
    if (!(c)) {                                                         \
      if (failures < 40) std::printf("FAIL [%s] line %d: %s\n", ctx, __LINE__, #c); \
      ++failures;                                                       \
    }                                                                   \
  } while (0)

namespace {

uintptr_t g_next = (uintptr_t)1 << 32;
// A fake, 256-byte aligned device address (plans only look at alignment).
const void* fake(size_t bytes, uintptr_t misalign = 0) {
  const uintptr_t p = g_next + misalign;
  g_next += (bytes + 4096) & ~(uintptr_t)255;
  return reinterpret_cast<const void*>(p);
}

w4a16_problem make_problem(int M, int N, int K, uintptr_t mis_x = 0, int pad = 0) {
  w4a16_problem q{};
  q.ldx = K + pad;
  q.x = fake((size_t)M * q.ldx * 2, mis_x);
  q.ldp = N;
  q.packed = static_cast<const int8_t*>(fake((size_t)(K / 2) * N));
  q.lds = N;
  q.scale = static_cast<const float*>(fake((size_t)(K / kGroup) * N * 4));
  q.ldy = N;
  q.y = const_cast<void*>(fake((size_t)M * N * 2));
  q.M = M;
  q.N = N;
  q.K = K;
  return q;
}

struct Range {
  size_t lo, hi;
};

void check_disjoint(std::vector<Range> r) {
  for (size_t i = 0; i < r.size(); ++i)
    for (size_t j = i + 1; j < r.size(); ++j) CHECK(r[i].hi <= r[j].lo || r[j].hi <= r[i].lo);
}

void check_plan(const w4a16_problem* probs, int count, bool pair) {
  Plan pl = make_plan(probs, count, pair);
  const size_t need = plan_bytes(pl);
  // Bind to a workspace of exactly the planned size and inspect where things land.
  const size_t W = need;
  char* ws = reinterpret_cast<char*>((uintptr_t)1 << 44);
  if (need > 0) bind(pl, ws, W);
  const size_t half = (W / 2) & ~(size_t)255;
  const size_t status = W >= 256 ? ((W - 4) & ~(size_t)3) : W;
  std::vector<Range> regions;
  int wg = 0;
  for (int i = 0; i < count; ++i) {
    const Problem& P = pl.L.p[i];
    const int G = P.K / kGroup;
    CHECK(P.wg_begin == wg);
    CHECK(P.gps >= 1);
    CHECK((int64_t)P.nsplit * P.gps >= G);
    CHECK((int64_t)(P.nsplit - 1) * P.gps < G);
    if (pl.kind == kGemv) {
      CHECK(P.tiles_n == ceil_div(P.N, 16 * pl.cpl));
      CHECK(P.gps == pl.waves);
      wg += P.tiles_n * P.nsplit;
      CHECK(pl.lds_bytes >= (size_t)pl.waves * P.M * 16 * pl.cpl * 4);
      const int nslots = pair && i == 0 ? P.nsplit : P.nsplit - 1;
      if (nslots > 0 && !pl.too_large) {
        const char* base = reinterpret_cast<const char*>(P.part);
        CHECK(base >= ws);
        const size_t lo = (size_t)(base - ws), hi = lo + (size_t)nslots * P.M * P.N * 4;
        CHECK(hi <= half);  // decode slots: lower half only
        regions.push_back({lo, hi});
      }
      if (pl.full) {
        CHECK(P.N % (16 * pl.cpl) == 0);
        CHECK((P.vec & 3) == 3);
      }
    } else {
      CHECK(P.tiles_m == ceil_div(P.M, kGemmRows));
      CHECK(P.tiles_n == ceil_div(P.N, 64 * pl.cpl));
      wg += P.tiles_m * P.tiles_n * P.nsplit;
      if (P.nsplit > 1) {
        const size_t lo = (size_t)(reinterpret_cast<const char*>(P.part) - ws);
        const size_t hi = lo + (size_t)P.nsplit * P.M * P.N * 4;
        CHECK(lo >= half && hi + 128 <= W);
        regions.push_back({lo, hi});
      }
      if (pl.rowsum_src[i] == i) {
        const size_t lo = (size_t)(reinterpret_cast<const char*>(P.rowsum) - ws);
        const size_t hi = lo + (size_t)G * P.M * 4;
        CHECK(lo >= half && hi + 128 <= W);
        regions.push_back({lo, hi});
        CHECK(P.rs_begin >= 0);
      } else {
        const Problem& S = pl.L.p[pl.rowsum_src[i]];
        CHECK(S.x == P.x && S.M == P.M && S.K == P.K && S.ldx == P.ldx);
      }
    }
  }
  CHECK(wg == pl.total_wgs);
  CHECK(pl.lds_bytes <= 160 * 1024);
  for (const Range& r : regions) CHECK(r.hi <= status);
  check_disjoint(regions);
  if (pl.kind == kGemm) {
    // Row-sum and split-reduce workgroup ranges cover their elements.
    int rs = 0, red = 0;
    for (int i = 0; i < count; ++i) {
      const Problem& P = pl.L.p[i];
      if (pl.rowsum_src[i] == i) {
        CHECK(P.rs_begin == rs);
        rs += ceil_div((int64_t)P.M * (P.K / kGroup), 16);
      }
      CHECK(P.red_begin == red);
      if (P.nsplit > 1) red += ceil_div((int64_t)P.M * P.N, kReduceElems);
    }
    CHECK(rs == pl.rs_wgs);
    CHECK(red == pl.red_wgs);
  }
}

void check_call(const w4a16_problem* probs, int count) {
  Batches b = split(probs, count);
  if (b.n_gemv) check_plan(b.gemv, b.n_gemv, false);
  if (b.n_gemm) check_plan(b.gemm, b.n_gemm, false);
  for (int i = 0; i < b.n_sep; ++i)
    if (b.sep[i].K > 0)
      for_each_chunk(b.sep[i], [&](const w4a16_problem& c) {
        check_plan(&c, 1, false);
        return W4A16_OK;
      });
  // The size query covers every launch of the call.
  size_t bytes = 0;
  CHECK(workspace_for(probs, count, &bytes) == W4A16_OK);
  if (b.n_gemv) CHECK(bytes >= plan_bytes(make_plan(b.gemv, b.n_gemv)));
  if (b.n_gemm) CHECK(bytes >= plan_bytes(make_plan(b.gemm, b.n_gemm)));
}

}  // namespace

int main() {
  const int Ms[] = {1, 2, 3, 4, 7, 8, 15, 16, 17, 24, 31, 32, 33, 40, 64, 65, 100, 128, 300, 2048, 4096};
  const int Ks[] = {128, 256, 1024, 2048, 4096, 5120, 8192, 12288, 25600};
  const int Ns[] = {1, 17, 64, 100, 128, 640, 1024, 3072, 4096, 5120, 8192, 12288, 25600};
  int calls = 0;
  for (int M : Ms)
    for (int K : Ks)
      for (int N : Ns) {
        if ((double)M * K * N > 4.0e12) continue;
        std::snprintf(ctx, sizeof ctx, "single M=%d K=%d N=%d", M, K, N);
        const w4a16_problem q = make_problem(M, N, K);
        check_call(&q, 1);
        // The public size query (contiguous aligned operands) covers the plan.
        size_t bytes = 0;
        CHECK(w4a16_workspace_size(M, N, K, kGroup, &bytes) == W4A16_OK);
        Batches b = split(&q, 1);
        if (b.n_gemv) CHECK(bytes >= plan_bytes(make_plan(b.gemv, 1)));
        if (b.n_gemm) CHECK(bytes >= plan_bytes(make_plan(b.gemm, 1)));
        // Unaligned activations (row stride not a multiple of 8 elements).
        std::snprintf(ctx, sizeof ctx, "unaligned M=%d K=%d N=%d", M, K, N);
        const w4a16_problem u = make_problem(M, N, K, 2, 1);
        check_call(&u, 1);
        ++calls;
        // SwiGLU pair at decode-sized M.
        if (kind_of(q) == kGemv) {
          std::snprintf(ctx, sizeof ctx, "pair M=%d K=%d N=%d", M, K, N);
          const w4a16_problem pr[2] = {q, make_problem(M, N, K)};
          check_plan(pr, 2, true);
        }
      }
  // Grouped calls: q/k/v shapes sharing x, MoE-like experts with their own M.
  const int qkv[][3] = {{4096, 4096, 0}, {4096, 1024, 0}, {4096, 1024, 0}};
  for (int M : Ms) {
    std::snprintf(ctx, sizeof ctx, "qkv M=%d", M);
    w4a16_problem p[3];
    const w4a16_problem base = make_problem(M, qkv[0][1], qkv[0][0]);
    for (int i = 0; i < 3; ++i) {
      p[i] = make_problem(M, qkv[i][1], qkv[i][0]);
      p[i].x = base.x;
      p[i].ldx = base.ldx;
    }
    check_call(p, 3);
  }
  for (int e = 1; e <= kMaxProblems; ++e) {
    std::snprintf(ctx, sizeof ctx, "experts=%d", e);
    std::vector<w4a16_problem> p;
    for (int i = 0; i < e; ++i) p.push_back(make_problem(1 + (i * 7) % 40, 768, 2048));
    check_call(p.data(), e);
  }
  std::printf("%d shapes checked\n", calls);
  if (failures) {
    std::printf("%d failures\n", failures);
    return 1;
  }
  std::printf("ok\n");
  return 0;
}
