// Generation-checked table of immutable state versions (StateTable / StateId,
// native/state_table.h:11-38). A version is reserved before the forward that
// produces it, then either published (value attached, id handed out) or
// rolled back. Every lookup checks the full descriptor: owner, slot,
// generation, position and charged bytes, so a stale or forged id fails
// instead of aliasing a newer version in the same slot. Single-threaded: the
// owning session is confined to its caller's worker thread.
#pragma once
#include <cstdint>
#include <limits>
#include <optional>
#include <stdexcept>
#include <vector>

#include "../../include/hip_bridge.h"

namespace hb {

template <class T, uint64_t kGenerationLimit = std::numeric_limits<uint64_t>::max()>
class VersionTable {
  static_assert(kGenerationLimit > 0, "generation limit");
  struct Slot {
    uint64_t generation = 0, position = 0, bytes = 0;
    bool held = false;
    std::optional<T> value;
  };

 public:
  VersionTable(uint64_t owner, size_t slots, uint64_t capacity) : owner_(owner), capacity_(capacity), slots_(slots) {
    if (owner == 0 || slots == 0 || slots > 64 || capacity == 0) throw std::invalid_argument("state table bounds");
  }

  // Takes the first free slot whose generation can still advance.
  StateId reserve(uint64_t position, uint64_t bytes) {
    if (position == 0 || bytes == 0 || bytes > capacity_ - used_)
      throw std::runtime_error("resident state byte budget exhausted");
    for (size_t i = 0; i < slots_.size(); ++i) {
      Slot& s = slots_[i];
      if (s.held || s.generation == kGenerationLimit) continue;
      s.generation += 1;
      s.position = position;
      s.bytes = bytes;
      s.held = true;
      used_ += bytes;
      return StateId{owner_, i, s.generation, position, bytes};
    }
    throw std::runtime_error("resident state slots exhausted");
  }

  void publish(const StateId& id, T value) {
    Slot& s = lookup(id);
    if (s.value) throw std::invalid_argument("state already published");
    s.value.emplace(std::move(value));
  }

  const T& get(const StateId& id) {
    Slot& s = lookup(id);
    if (!s.value) throw std::invalid_argument("unpublished state");
    return *s.value;
  }

  // Frees a reserved (published or not) version; its slot keeps the generation.
  void rollback(const StateId& id) {
    Slot& s = lookup(id);
    s.value.reset();
    s.held = false;
    used_ -= s.bytes;
  }

  // Releases a published version (an unpublished one is an error).
  void release(const StateId& id) {
    (void)get(id);
    rollback(id);
  }

  uint64_t bytes() const { return used_; }
  size_t residents() const {
    size_t n = 0;
    for (const Slot& s : slots_) n += s.held;
    return n;
  }
  // Invalidates every version (generations are kept, so old ids stay stale).
  void clear() {
    for (Slot& s : slots_) {
      s.value.reset();
      s.held = false;
    }
    used_ = 0;
  }
  // Visits every held, published value (for teardown of device resources).
  template <class F>
  void for_each(F&& f) {
    for (Slot& s : slots_)
      if (s.held && s.value) f(*s.value);
  }

 private:
  Slot& lookup(const StateId& id) {
    if (id.owner != owner_ || id.slot >= slots_.size()) throw std::invalid_argument("foreign state owner/slot");
    Slot& s = slots_[id.slot];
    if (!s.held || s.generation != id.generation || s.position != id.position || s.bytes != id.bytes)
      throw std::invalid_argument("stale state generation/geometry");
    return s;
  }

  uint64_t owner_, capacity_, used_ = 0;
  std::vector<Slot> slots_;
};

}  // namespace hb
