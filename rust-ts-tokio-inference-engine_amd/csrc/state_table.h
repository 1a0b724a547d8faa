// Version table of the device sessions: immutable state versions named by a
// StateId{owner, slot, generation, position, bytes} (40 B, the descriptor the
// reference hands to Rust, native/state_table.h:11).
//
// Design. A table has at most 64 slots, so slot occupancy is one 64-bit mask:
// a reservation takes the lowest clear bit of (held | retired) with a bit
// scan, and freeing a slot clears its bit. Each slot keeps the descriptor it
// last issued, whole; a lookup is "is the slot held, and is the caller's
// descriptor exactly the issued one". Generations count reservations per slot,
// so an id from before a slot's reuse never matches again; a slot whose
// generation reached the table's limit is retired for good.
//
// Observable contract (shared with the reference so callers see the same
// errors, in the same order):
//   constructor: owner != 0, 1 <= slots <= 64, budget > 0  ("state table bounds")
//   reserve: position > 0, bytes > 0, bytes within the remaining budget
//            ("resident state byte budget exhausted"); the lowest free slot
//            that is not retired ("resident state slots exhausted")
//   any lookup: owner or slot index wrong -> "foreign state owner/slot";
//            slot not held or any other field different ->
//            "stale state generation/geometry"
//   publish: once per reservation ("state already published")
//   get / release: published only ("unpublished state")
//   rollback frees a held slot, published or not; clear frees every slot and
//   keeps the generations, so every outstanding id turns stale.
// Single-threaded: a session is confined to its caller's worker thread.
#pragma once
#include <cstdint>
#include <limits>
#include <optional>
#include <stdexcept>
#include <vector>

#include "../../include/hip_bridge.h"

namespace hb {

template <class T>
class VersionTable {
 public:
  VersionTable(uint64_t owner, size_t slots, uint64_t budget,
               uint64_t generation_limit = std::numeric_limits<uint64_t>::max())
      : owner_(owner), budget_(budget), limit_(generation_limit) {
    if (owner == 0 || slots == 0 || slots > 64 || budget == 0 || generation_limit == 0)
      throw std::invalid_argument("state table bounds");
    n_ = slots;
    usable_ = slots == 64 ? ~uint64_t(0) : (uint64_t(1) << slots) - 1;
    issued_.resize(slots);
    values_.resize(slots);
  }

  StateId reserve(uint64_t position, uint64_t bytes) {
    if (position == 0 || bytes == 0 || bytes > budget_ - in_use_)
      throw std::runtime_error("resident state byte budget exhausted");
    const uint64_t open = usable_ & ~(held_ | retired_);
    if (!open) throw std::runtime_error("resident state slots exhausted");
    const unsigned slot = unsigned(__builtin_ctzll(open));
    const uint64_t generation = issued_[slot].generation + 1;
    issued_[slot] = StateId{owner_, slot, generation, position, bytes};
    held_ |= bit(slot);
    if (generation == limit_) retired_ |= bit(slot);
    in_use_ += bytes;
    return issued_[slot];
  }

  void publish(const StateId& id, T value) {
    std::optional<T>& v = values_[find(id)];
    if (v) throw std::invalid_argument("state already published");
    v.emplace(std::move(value));
  }

  const T& get(const StateId& id) {
    const std::optional<T>& v = values_[find(id)];
    if (!v) throw std::invalid_argument("unpublished state");
    return *v;
  }

  void rollback(const StateId& id) { free_slot(find(id)); }

  void release(const StateId& id) {
    const size_t slot = find(id);
    if (!values_[slot]) throw std::invalid_argument("unpublished state");
    free_slot(slot);
  }

  uint64_t bytes() const { return in_use_; }
  size_t residents() const { return size_t(__builtin_popcountll(held_)); }

  void clear() {
    for (uint64_t m = held_; m; m &= m - 1) values_[__builtin_ctzll(m)].reset();
    held_ = 0;
    in_use_ = 0;
  }

  // Every held, published value (teardown of the device resources they own).
  template <class F>
  void for_each(F&& f) {
    for (uint64_t m = held_; m; m &= m - 1)
      if (values_[__builtin_ctzll(m)]) f(*values_[__builtin_ctzll(m)]);
  }

 private:
  static uint64_t bit(size_t slot) { return uint64_t(1) << slot; }

  size_t find(const StateId& id) const {
    if (id.owner != owner_ || id.slot >= n_) throw std::invalid_argument("foreign state owner/slot");
    const StateId& mine = issued_[id.slot];
    if (!(held_ & bit(id.slot)) || mine.generation != id.generation || mine.position != id.position ||
        mine.bytes != id.bytes)
      throw std::invalid_argument("stale state generation/geometry");
    return size_t(id.slot);
  }

  void free_slot(size_t slot) {
    values_[slot].reset();
    held_ &= ~bit(slot);
    in_use_ -= issued_[slot].bytes;
  }

  uint64_t owner_, budget_, limit_;
  size_t n_ = 0;
  uint64_t usable_ = 0, held_ = 0, retired_ = 0, in_use_ = 0;
  std::vector<StateId> issued_;  // the descriptor each slot issued last
  std::vector<std::optional<T>> values_;
};

}  // namespace hb
