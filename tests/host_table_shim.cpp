// C entry points over the sessions' VersionTable (csrc/state_table.h) for the
// differential walk in tests/test_host_versions.py; built by that test with g++.
#include <cstdint>
#include <exception>

#include "state_table.h"

namespace {
template <class F>
int guarded(F f) {
  try {
    f();
    return 0;
  } catch (const std::exception&) {
    return -1;
  }
}
using Table = hb::VersionTable<int>;
}  // namespace

extern "C" {
void* hb_table_create(uint64_t owner, size_t slots, uint64_t bytes) {
  try {
    return new Table(owner, slots, bytes);
  } catch (const std::exception&) {
    return nullptr;
  }
}
void hb_table_destroy(void* t) { delete static_cast<Table*>(t); }
int hb_table_reserve(void* t, uint64_t position, uint64_t bytes, StateId* id) {
  return guarded([&] { *id = static_cast<Table*>(t)->reserve(position, bytes); });
}
int hb_table_publish(void* t, const StateId* id, int value) {
  return guarded([&] { static_cast<Table*>(t)->publish(*id, value); });
}
int hb_table_get(void* t, const StateId* id, int* value) {
  return guarded([&] { *value = static_cast<Table*>(t)->get(*id); });
}
int hb_table_rollback(void* t, const StateId* id) { return guarded([&] { static_cast<Table*>(t)->rollback(*id); }); }
int hb_table_release(void* t, const StateId* id) { return guarded([&] { static_cast<Table*>(t)->release(*id); }); }
uint64_t hb_table_bytes(void* t) { return static_cast<Table*>(t)->bytes(); }
size_t hb_table_residents(void* t) { return static_cast<Table*>(t)->residents(); }
void hb_table_clear(void* t) { static_cast<Table*>(t)->clear(); }
}
