// Host emulation of the decode kernels' split-K slot protocol
// (inf-engine_amd/csrc/slot_protocol.h), driven from threads: publishers
// store encoded partials, a finisher polls with a bounded budget, sums in
// split order, re-zeroes the slots, and reports a give-up in a status word.
// Built and run by tests/test_slot_protocol.py; prints "ok" and exits 0 when
// every check passes.
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "slot_protocol.h"

using namespace w4a16;

static int failures = 0;
#define CHECK(c)                                                   \
  do {                                                             \
    if (!(c)) {                                                    \
      std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #c);     \
      ++failures;                                                  \
    }                                                              \
  } while (0)

struct Workspace {
  int nslots, elems;
  std::vector<std::atomic<uint32_t>> slots;  // [nslots][elems]
  std::atomic<uint32_t> status{0};
  Workspace(int ns, int e) : nslots(ns), elems(e), slots((size_t)ns * e) {
    for (auto& s : slots) s.store(0);
  }
  bool all_zero() const {
    for (auto& s : slots)
      if (s.load()) return false;
    return true;
  }
};

// A publishing split: slot word of every element of its partial.
static void publish(Workspace& ws, int split, const std::vector<float>& part) {
  for (int e = 0; e < ws.elems; ++e) ws.slots[(size_t)split * ws.elems + e].store(publish_bits(part[e]), std::memory_order_release);
}

// The finisher: wait for every slot (at most `limit` re-poll rounds), sum in
// split order with its own partial last, zero what it read, NaN + status bit
// on a give-up.  Returns the outputs.
static std::vector<float> finish(Workspace& ws, const std::vector<float>& own, uint32_t limit) {
  std::vector<float> out(ws.elems, 0.f);
  bool timed_out = false;
  std::vector<uint32_t> t((size_t)ws.nslots * ws.elems);
  for (size_t i = 0; i < t.size(); ++i) t[i] = ws.slots[i].load(std::memory_order_acquire);
  for (uint32_t spins = 0;; ++spins) {
    bool missing = false;
    for (uint32_t w : t) missing = missing || slot_empty(w);
    if (!missing) break;
    if (spins >= limit) {
      timed_out = true;
      break;
    }
    for (size_t i = 0; i < t.size(); ++i)
      if (slot_empty(t[i])) t[i] = ws.slots[i].load(std::memory_order_acquire);
  }
  for (int e = 0; e < ws.elems; ++e) {
    float v = 0.f;
    for (int sp = 0; sp < ws.nslots; ++sp) v += slot_value(t[(size_t)sp * ws.elems + e]);
    out[e] = timed_out ? NAN : v + own[e];
  }
  for (auto& s : ws.slots) s.store(0, std::memory_order_relaxed);
  if (timed_out) ws.status.fetch_or(kStatusSplitKTimeout);
  return out;
}

static uint32_t bits(float f) { uint32_t b; std::memcpy(&b, &f, 4); return b; }

int main() {
  // Encoding: never 0, decodes to the same bits, NaN 0xFFFFFFFF canonicalised.
  for (uint64_t b = 0; b <= 0xffffffffull; b += 0x10001ull) {
    const float v = bits_f32((uint32_t)b);
    const uint32_t w = publish_bits(v);
    CHECK(!slot_empty(w));
    if ((uint32_t)b != 0xffffffffu) CHECK(bits(slot_value(w)) == (uint32_t)b);
  }
  CHECK(publish_bits(bits_f32(0xffffffffu)) == ~0x7fc00000u);
  CHECK(bits(slot_value(publish_bits(bits_f32(0xffffffffu)))) == 0x7fc00000u);
  CHECK(!slot_empty(publish_bits(0.f)) && !slot_empty(publish_bits(-0.f)));
  CHECK(bits(slot_value(publish_bits(-0.f))) == 0x80000000u);

  // Normal calls: publishers race the finisher; the sum is in split order and
  // bit-identical on every repetition; the slots end empty.
  const int nsplit = 8, elems = 96;
  Workspace ws(nsplit - 1, elems);
  std::vector<std::vector<float>> parts(nsplit, std::vector<float>(elems));
  for (int sp = 0; sp < nsplit; ++sp)
    for (int e = 0; e < elems; ++e) parts[sp][e] = std::ldexp((float)((sp * 131 + e * 17) % 97) - 48.f, (sp * 7 + e) % 40 - 20);
  std::vector<float> expect(elems);
  for (int e = 0; e < elems; ++e) {
    float v = 0.f;
    for (int sp = 0; sp < nsplit - 1; ++sp) v += parts[sp][e];
    expect[e] = v + parts[nsplit - 1][e];
  }
  for (int rep = 0; rep < 50; ++rep) {
    std::vector<std::thread> pubs;
    for (int sp = 0; sp < nsplit - 1; ++sp) pubs.emplace_back(publish, std::ref(ws), sp, std::cref(parts[sp]));
    const std::vector<float> out = finish(ws, parts[nsplit - 1], kDefaultSpinLimit * 64);
    for (auto& t : pubs) t.join();
    for (int e = 0; e < elems; ++e) CHECK(bits(out[e]) == bits(expect[e]));
    CHECK(ws.all_zero());
    CHECK(ws.status.load() == 0);
  }

  // Give-up: one publisher arrives only after the finisher has given up.  The
  // outputs are NaN, the status bit is set, and the late slot is left
  // non-zero -- a poisoned workspace, which the host zeroes before reuse.
  {
    Workspace w2(3, 4);
    std::vector<float> p(4, 1.5f), own(4, 0.25f);
    publish(w2, 0, p);
    publish(w2, 1, p);
    const std::vector<float> out = finish(w2, own, 0);
    for (float v : out) CHECK(std::isnan(v));
    CHECK(w2.status.load() == kStatusSplitKTimeout);
    publish(w2, 2, p);  // the late publisher
    CHECK(!w2.all_zero());
    // Host recovery: zero the workspace (slots and status), then a full call.
    for (auto& s : w2.slots) s.store(0);
    w2.status.store(0);
    for (int sp = 0; sp < 3; ++sp) publish(w2, sp, p);
    const std::vector<float> ok = finish(w2, own, 0);
    for (float v : ok) CHECK(v == 1.5f * 3 + 0.25f);
    CHECK(w2.status.load() == 0 && w2.all_zero());
  }
  if (failures) return 1;
  std::printf("ok\n");
  return 0;
}
