// Host-side pieces of the dK/dV query-range split shared by the backward
// kernels for head dims up to 128 and for head dims 136..512: the makespan
// estimate the split count is chosen by, and a small cache of chosen counts.
#pragma once

#include <algorithm>
#include <cstdint>
#include <functional>
#include <mutex>
#include <vector>

namespace sa {

// Estimated makespan, in iterations, of one XCD's share of a dK/dV grid of
// nkb key blocks x units (batch, KV head) pairs, each block's iterations
// iters(kb) split n_split ways.  Blocks run in dispatch order (key block,
// unit, split) and are dealt to the 8 XCDs round-robin, so the XCD gets every
// 8th; it runs `slots` of them at once, each starting on the slot that frees
// first.  A block costs its share of the iterations plus `setup` (its loads
// of K and V and its stores); a fifth of the longest block is added for the
// ragged end.
template <typename Iters>
double dkdv_split_makespan(int nkb, int units, int n_split, int slots, double setup, Iters iters) {
    std::vector<double> heap(static_cast<size_t>(slots), 0.0);
    double longest = 0.0;
    int64_t id = 0;
    for (int kb = 0; kb < nkb; ++kb) {
        const int64_t it = iters(kb);
        for (int64_t j = 0; j < static_cast<int64_t>(units) * n_split; ++j, ++id) {
            if (id % 8) continue;
            const int64_t s = j % n_split;
            const double cost = static_cast<double>((s + 1) * it / n_split - s * it / n_split) + setup;
            longest = std::max(longest, cost);
            std::pop_heap(heap.begin(), heap.end(), std::greater<double>());
            heap.back() += cost;
            std::push_heap(heap.begin(), heap.end(), std::greater<double>());
        }
    }
    return *std::max_element(heap.begin(), heap.end()) + 0.2 * longest;
}

// The split counts of the last 16 shapes asked for (the estimate costs up to
// ~0.1 ms of host time, and a training step asks for the same shapes again).
class SplitCountCache {
  public:
    template <typename Compute>
    int get(const int (&key)[6], Compute compute) {
        {
            std::lock_guard<std::mutex> lock(mu_);
            for (int i = 0; i < n_cached_; ++i)
                if (std::equal(key, key + 6, cache_[i].key)) return cache_[i].n_split;
        }
        const int n = compute();
        std::lock_guard<std::mutex> lock(mu_);
        Entry& e = cache_[next_];
        std::copy(key, key + 6, e.key);
        e.n_split = n;
        next_ = (next_ + 1) % kEntries;
        n_cached_ = std::min(n_cached_ + 1, kEntries);
        return n;
    }

  private:
    static constexpr int kEntries = 16;
    struct Entry {
        int key[6];
        int n_split;
    };
    std::mutex mu_;
    Entry cache_[kEntries];
    int n_cached_ = 0, next_ = 0;
};

}  // namespace sa
