// Copy-on-write page allocator (see page_pool.h).
#include "page_pool.h"

namespace hb {

PagePool::PagePool(int pages, int page_tokens) : page_(page_tokens), refs_(pages, 0), fill_(pages, 0) {
  if (page_tokens <= 0 || pages < 0) throw std::invalid_argument("page pool geometry");
  for (int p = pages - 1; p >= 0; --p) free_.push_back(p);
}

int PagePool::take() {
  if (free_.empty()) throw std::runtime_error("KV pages exhausted");
  const int p = free_.back();
  free_.pop_back();
  refs_[p] = 1;
  fill_[p] = 0;
  return p;
}

PagePool::Plan PagePool::extend(const std::vector<int32_t>& parent, int p, int n) {
  Plan plan;
  try {
    const int full = p / page_, part = p % page_, end = p + n;
    if (p < 0 || n < 1 || int(parent.size()) < (p + page_ - 1) / page_)
      throw std::invalid_argument("parent page list shorter than its position");
    for (int j = 0; j < full; ++j) {
      ++refs_[parent[j]];
      plan.pages.push_back(parent[j]);
    }
    if (part) {
      const int q = parent[full];
      if (fill_[q] == part) {  // nobody wrote past the parent here: continue in place
        ++refs_[q];
        plan.pages.push_back(q);
        plan.claimed = q;
        plan.claimed_fill = part;
        fill_[q] = std::min(page_, end - full * page_);
      } else {  // a sibling line continued this page: copy it
        const int c = take();
        plan.pages.push_back(c);
        plan.pairs.push_back(q);
        plan.pairs.push_back(c);
        fill_[c] = std::min(page_, end - full * page_);
      }
    }
    while (int(plan.pages.size()) * page_ < end) {
      const int c = take();
      fill_[c] = std::min(page_, end - int(plan.pages.size()) * page_);
      plan.pages.push_back(c);
    }
  } catch (...) {
    undo(plan);
    throw;
  }
  return plan;
}

void PagePool::undo(Plan& plan) {
  if (plan.claimed >= 0) fill_[plan.claimed] = plan.claimed_fill;
  drop(plan.pages);
  plan = Plan{};
}

void PagePool::drop(const std::vector<int32_t>& pages) {
  for (int32_t p : pages)
    if (--refs_[p] == 0) free_.push_back(p);
}

}  // namespace hb
