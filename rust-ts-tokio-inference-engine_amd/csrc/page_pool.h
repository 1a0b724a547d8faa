// Reference-counted page allocator for copy-on-write sharing of paged KV
// between immutable state versions. Host-only (no device code).
#pragma once
#include <algorithm>
#include <cstdint>
#include <stdexcept>
#include <vector>

namespace hb {

// Page allocator with reference counts and a per-page fill mark (the number of
// token positions any holder has written). A child starting at position p
// inherits its parent's full pages. It writes into the parent's last, partly
// filled page only when nobody has written past the parent's content there
// (fill == p mod page); otherwise it takes a fresh page and copies the parent's
// page into it first. Holders of a page never see positions at or above its
// fill mark, so shared pages are never changed under them.
class PagePool {
 public:
  PagePool(int pages, int page_tokens);
  struct Plan {
    std::vector<int32_t> pages;  // the child's page list
    std::vector<int32_t> pairs;  // (source, destination) page copies to run before the forward
    int claimed = -1, claimed_fill = 0;
  };
  // Pages for a child of `parent` (its page list) writing positions [p, p + n).
  Plan extend(const std::vector<int32_t>& parent, int p, int n);
  // Undoes extend() of a child whose forward did not happen or failed.
  void undo(Plan& plan);
  void drop(const std::vector<int32_t>& pages);
  size_t free_pages() const { return free_.size(); }

 private:
  int take();
  int page_ = 16;
  std::vector<int32_t> refs_, fill_, free_;
};

}  // namespace hb
