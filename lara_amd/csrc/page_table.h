// Host-side allocator of a paged K/V cache: a pool of fixed-size pages, one block table per
// sequence (page index of each page-sized run of token rows, -1 = unmapped) and
// least-recently-used eviction of whole sequences.
//
// The KV260 reloads its cache on every transaction (hw/rtl/mem/kv_cache_ram.sv:77-91,
// sw/attn_driver.py:418-422), so the reference has no cache manager; this is the serving-side
// counterpart that lets many sequences of different lengths share one HBM pool.  Plain C++
// (no HIP), so the logic is tested on the CPU.
#pragma once

#include <stdint.h>

#include <algorithm>
#include <vector>

namespace lara {

class PageTable {
  public:
    PageTable() = default;
    PageTable(int batch, int max_pages_per_seq, int n_pages)
        : batch_(batch), max_pages_(max_pages_per_seq), n_pages_(n_pages),
          table_((size_t)batch * max_pages_per_seq, -1), mapped_(batch, 0), last_use_(batch, 0) {
        free_.reserve(n_pages);
        for (int p = n_pages - 1; p >= 0; --p) free_.push_back(p);  // hands out 0, 1, 2, ... first
    }

    int batch() const { return batch_; }
    int max_pages() const { return max_pages_; }
    int n_pages() const { return n_pages_; }
    int free_pages() const { return (int)free_.size(); }
    int mapped(int b) const { return mapped_[b]; }
    const int32_t* row(int b) const { return table_.data() + (size_t)b * max_pages_; }
    const int32_t* data() const { return table_.data(); }
    uint64_t last_use(int b) const { return last_use_[b]; }

    // Marks sequence b as used now (the eviction order).
    void touch(int b) { last_use_[b] = ++clock_; }

    // Maps pages so that rows [0, n_rows) of sequence b are backed.  Returns false, changing
    // nothing, when the sequence would need more than max_pages or the pool has too few free
    // pages.
    bool reserve(int b, int n_rows, int page_size) {
        const int need = (n_rows + page_size - 1) / page_size;
        if (need > max_pages_) return false;
        const int extra = need - mapped_[b];
        if (extra <= 0) {
            touch(b);
            return true;
        }
        if (extra > (int)free_.size()) return false;
        int32_t* r = table_.data() + (size_t)b * max_pages_;
        for (int i = mapped_[b]; i < need; ++i) {
            r[i] = free_.back();
            free_.pop_back();
        }
        mapped_[b] = need;
        touch(b);
        return true;
    }

    // Returns every page of sequence b to the pool.
    void release(int b) {
        int32_t* r = table_.data() + (size_t)b * max_pages_;
        for (int i = mapped_[b] - 1; i >= 0; --i) {
            free_.push_back(r[i]);
            r[i] = -1;
        }
        mapped_[b] = 0;
    }

    // Releases whole sequences, least recently used first and skipping pinned ones, until at
    // least `need` pages are free.  Plans first: returns false and releases nothing when even
    // every unpinned sequence would not free enough.
    bool evict_lru(int need, const std::vector<char>& pinned, std::vector<int>* evicted) {
        evicted->clear();
        if ((int)free_.size() >= need) return true;
        std::vector<int> order;
        for (int b = 0; b < batch_; ++b)
            if (mapped_[b] > 0 && !(b < (int)pinned.size() && pinned[b])) order.push_back(b);
        std::stable_sort(order.begin(), order.end(),
                         [&](int x, int y) { return last_use_[x] < last_use_[y]; });
        int avail = (int)free_.size();
        size_t take = 0;
        while (take < order.size() && avail < need) avail += mapped_[order[take++]];
        if (avail < need) return false;
        for (size_t i = 0; i < take; ++i) {
            release(order[i]);
            evicted->push_back(order[i]);
        }
        return true;
    }

    // True when rows [row0, row0 + n) of sequence b are all backed.
    bool covers(int b, int64_t row0, int64_t n, int page_size) const {
        if (n <= 0) return true;
        return row0 >= 0 && (row0 + n + page_size - 1) / page_size <= mapped_[b];
    }

  private:
    int batch_ = 0, max_pages_ = 0, n_pages_ = 0;
    std::vector<int32_t> table_;
    std::vector<int> mapped_;
    std::vector<uint64_t> last_use_;
    std::vector<int32_t> free_;
    uint64_t clock_ = 0;
};

}  // namespace lara
