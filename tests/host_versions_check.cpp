// Host-only checks of the state-version table and the copy-on-write page pool
// (csrc/state_table.h, csrc/page_pool.cpp), built with g++ by
// tests/test_host_versions.py.
//
// 1. VersionTable: the invariants of the reference's StateTable judge
//    (judges/state_table.cpp:7-20): constructor bounds, unpublished / foreign /
//    stale descriptors rejected field by field, double publish and double
//    release rejected, slot reuse with a new generation, byte budget, clear,
//    generation exhaustion.
// 2. PagePool: a random walk of branch / extend / release over a simulated KV
//    memory (page -> 16 token tags). After every operation each live version
//    must read back exactly its own lineage's tokens, and page references must
//    balance (all pages free once every version is released).
#include <cassert>
#include <cstdio>
#include <map>
#include <random>
#include <string>
#include <vector>

#include "page_pool.h"
#include "state_table.h"

using hb::PagePool;
using hb::VersionTable;

static size_t checks = 0;

template <class F>
static void rejects(F f) {
  bool thrown = false;
  try {
    f();
  } catch (const std::exception&) {
    thrown = true;
  }
  if (!thrown) {
    std::fprintf(stderr, "FAIL: expected a rejection (check %zu)\n", checks);
    std::exit(1);
  }
  ++checks;
}

#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond); \
      std::exit(1);                                                   \
    }                                                                 \
    ++checks;                                                         \
  } while (0)

static void table_checks() {
  rejects([] { VersionTable<int> t(0, 1, 4); });
  rejects([] { VersionTable<int> t(1, 0, 4); });
  rejects([] { VersionTable<int> t(1, 65, 4); });
  rejects([] { VersionTable<int> t(1, 1, 0); });
  rejects([] { VersionTable<int> t(1, 1, 4, 0); });
  VersionTable<std::string> t(7, 2, 8), other(9, 2, 8);
  StateId a = t.reserve(3, 4);
  CHECK(a.owner == 7 && a.position == 3 && a.bytes == 4 && a.generation == 1);
  rejects([&] { t.get(a); });  // reserved but unpublished
  t.publish(a, "root");
  rejects([&] { t.publish(a, "twice"); });
  StateId b = t.reserve(4, 4);
  t.publish(b, "child");
  rejects([&] { t.reserve(5, 1); });  // slots and bytes both exhausted
  rejects([&] { other.get(a); });
  for (int field = 0; field < 5; ++field) {
    StateId bad = a;
    if (field == 0) bad.owner += 1;
    if (field == 1) bad.slot = UINT64_MAX;
    if (field == 2) bad.generation += 1;
    if (field == 3) bad.position += 1;
    if (field == 4) bad.bytes += 1;
    rejects([&] { t.get(bad); });
    rejects([&] { t.release(bad); });
    rejects([&] { t.rollback(bad); });
  }
  t.release(a);
  rejects([&] { t.release(a); });
  StateId again = t.reserve(3, 4);
  CHECK(again.slot == a.slot && again.generation == a.generation + 1);
  rejects([&] { t.get(a); });  // the old id stays stale after slot reuse
  t.publish(again, "root2");
  CHECK(t.get(b) == "child" && t.get(again) == "root2");
  CHECK(t.residents() == 2 && t.bytes() == 8);
  t.release(b);
  t.release(again);
  CHECK(t.residents() == 0 && t.bytes() == 0);
  for (int n = 0; n < 20000; ++n) {
    StateId id = t.reserve(uint64_t(n) + 1, 8);
    rejects([&] { t.reserve(1, 1); });
    t.rollback(id);
    rejects([&] { t.get(id); });
    CHECK(t.bytes() == 0);
  }
  rejects([&] { t.reserve(0, 4); });
  rejects([&] { t.reserve(1, 0); });
  rejects([&] { t.reserve(1, UINT64_MAX); });
  StateId live = t.reserve(1, 8);
  t.publish(live, "live");
  t.clear();
  CHECK(t.residents() == 0 && t.bytes() == 0);
  rejects([&] { t.get(live); });
  VersionTable<int> short_lived(3, 1, 4, 2);
  for (int n = 0; n < 2; ++n) {
    StateId x = short_lived.reserve(1, 4);
    short_lived.publish(x, n);
    short_lived.release(x);
  }
  rejects([&] { short_lived.reserve(1, 4); });  // generation limit reached
}

struct SimVersion {
  std::vector<int32_t> pages;
  std::vector<uint32_t> tokens;  // expected content of positions 0..len-1
};

static void pool_walk(uint64_t seed, int pages, int page, int steps) {
  PagePool pool(pages, page);
  std::map<int32_t, std::vector<uint32_t>> memory;  // page -> token tags
  std::vector<SimVersion> live;
  std::mt19937_64 rng(seed);
  uint32_t next_tag = 1;
  auto read_back = [&](const SimVersion& v) {
    for (size_t pos = 0; pos < v.tokens.size(); ++pos) {
      const auto it = memory.find(v.pages[pos / page]);
      CHECK(it != memory.end() && it->second[pos % page] == v.tokens[pos]);
    }
  };
  for (int s = 0; s < steps; ++s) {
    const int op = int(rng() % 10);
    if (op < 2 && !live.empty()) {  // release
      const size_t i = rng() % live.size();
      pool.drop(live[i].pages);
      live.erase(live.begin() + long(i));
    } else {  // child of a random live version (or a fresh root)
      const bool root = live.empty() || rng() % 8 == 0;
      const SimVersion parent = root ? SimVersion{} : live[rng() % live.size()];
      const int p = int(parent.tokens.size()), n = 1 + int(rng() % 9);
      PagePool::Plan plan;
      try {
        plan = pool.extend(parent.pages, p, n);
      } catch (const std::runtime_error&) {  // pages exhausted: release something
        ++checks;
        continue;
      }
      if (rng() % 16 == 0) {  // a forward that failed: undo must restore everything
        pool.undo(plan);
        continue;
      }
      for (size_t i = 0; i + 1 < plan.pairs.size(); i += 2) memory[plan.pairs[i + 1]] = memory[plan.pairs[i]];
      SimVersion child{plan.pages, parent.tokens};
      for (int j = 0; j < n; ++j) {
        const int pos = p + j;
        auto& mem = memory[child.pages[pos / page]];
        mem.resize(page, 0);
        mem[pos % page] = next_tag;
        child.tokens.push_back(next_tag++);
      }
      CHECK(int(child.pages.size()) == (p + n + page - 1) / page);
      live.push_back(std::move(child));
    }
    for (const SimVersion& v : live) read_back(v);
  }
  for (const SimVersion& v : live) pool.drop(v.pages);
  CHECK(pool.free_pages() == size_t(pages));
}

int main() {
  table_checks();
  for (uint64_t seed = 1; seed <= 6; ++seed) pool_walk(seed, 96, 16, 3000);
  pool_walk(77, 24, 4, 4000);  // small pages, frequent exhaustion
  std::printf("PASS host version checks=%zu\n", checks);
  return 0;
}
