// Host-logic checks of the paged-cache allocator (lara_amd/csrc/page_table.h), built with g++
// and run by tests/test_page_table.py.  Prints "ok" and exits 0, or names the first failed
// check and exits 1.
#include "page_table.h"

#include <stdio.h>
#include <stdlib.h>

#include <random>
#include <set>
#include <vector>

using lara::PageTable;

static int failures = 0;
#define CHECK(cond)                                                       \
    do {                                                                  \
        if (!(cond)) {                                                    \
            printf("FAILED line %d: %s\n", __LINE__, #cond);              \
            ++failures;                                                   \
        }                                                                 \
    } while (0)

// Every page is either free or mapped exactly once; unmapped table slots hold -1.
static bool consistent(const PageTable& t) {
    std::set<int> seen;
    int mapped = 0;
    for (int b = 0; b < t.batch(); ++b) {
        for (int i = 0; i < t.max_pages(); ++i) {
            const int p = t.row(b)[i];
            if (i < t.mapped(b)) {
                if (p < 0 || p >= t.n_pages() || !seen.insert(p).second) return false;
            } else if (p != -1) {
                return false;
            }
        }
        mapped += t.mapped(b);
    }
    return mapped + t.free_pages() == t.n_pages();
}

int main() {
    const int P = 64;
    {
        PageTable t(3, 4, 6);  // 3 sequences, up to 4 pages (256 rows) each, 6 pages in the pool
        CHECK(t.free_pages() == 6);
        CHECK(t.reserve(0, 1, P));           // one row needs one page
        CHECK(t.mapped(0) == 1 && t.row(0)[0] == 0);
        CHECK(t.reserve(0, 64, P) && t.mapped(0) == 1);   // still one page
        CHECK(t.reserve(0, 65, P) && t.mapped(0) == 2 && t.row(0)[1] == 1);
        CHECK(!t.reserve(1, 5 * P, P));      // more than max_pages
        CHECK(t.mapped(1) == 0 && t.free_pages() == 4);
        CHECK(t.reserve(1, 3 * P, P) && t.free_pages() == 1);
        CHECK(!t.reserve(2, 2 * P, P));      // the pool is short: nothing changes
        CHECK(t.mapped(2) == 0 && t.free_pages() == 1);
        CHECK(t.covers(0, 0, 128, P) && !t.covers(0, 0, 129, P) && t.covers(0, 100, 28, P));
        CHECK(!t.covers(2, 0, 1, P) && t.covers(2, 0, 0, P));
        t.release(0);
        CHECK(t.mapped(0) == 0 && t.row(0)[0] == -1 && t.free_pages() == 3);
        CHECK(t.reserve(2, 3 * P, P));       // reuses the released pages
        CHECK(consistent(t));
    }
    {
        // LRU eviction: uses order the victims, pinned sequences are skipped, and an
        // impossible request releases nothing.
        PageTable t(4, 2, 8);
        for (int b = 0; b < 4; ++b) CHECK(t.reserve(b, 2 * P, P));
        CHECK(t.free_pages() == 0);
        t.touch(0);  // order of last use now: 1, 2, 3, 0
        std::vector<int> ev;
        std::vector<char> pin(4, 0);
        CHECK(t.evict_lru(2, pin, &ev) && ev.size() == 1 && ev[0] == 1 && t.free_pages() == 2);
        CHECK(t.evict_lru(2, pin, &ev) && ev.empty());  // already enough
        pin[2] = 1;
        CHECK(t.evict_lru(4, pin, &ev) && ev.size() == 1 && ev[0] == 3 && t.mapped(2) == 2);
        CHECK(!t.evict_lru(8, pin, &ev) && ev.empty() && t.mapped(0) == 2 && t.mapped(2) == 2);
        pin[2] = 0;
        CHECK(t.evict_lru(8, pin, &ev) && ev.size() == 2 && ev[0] == 2 && ev[1] == 0 && t.free_pages() == 8);
        CHECK(consistent(t));
    }
    {
        // Random operations keep the pool consistent.
        std::mt19937 rng(12345);
        PageTable t(16, 32, 200);
        for (int it = 0; it < 20000; ++it) {
            const int b = rng() % 16;
            const int op = rng() % 10;
            if (op < 6) {
                const int before_free = t.free_pages(), before = t.mapped(b);
                const int rows = rng() % (40 * P);
                const bool ok = t.reserve(b, rows, P);
                const int need = (rows + P - 1) / P;
                if (ok) {
                    CHECK(t.mapped(b) == (need > before ? need : before));
                } else {
                    CHECK(t.mapped(b) == before && t.free_pages() == before_free);
                    CHECK(need > 32 || need - before > before_free);
                }
            } else if (op < 8) {
                t.release(b);
            } else {
                std::vector<int> ev;
                std::vector<char> pin(16, 0);
                pin[rng() % 16] = 1;
                const int want = rng() % 201;
                const bool ok = t.evict_lru(want, pin, &ev);
                if (ok) CHECK(t.free_pages() >= want);
                else CHECK(ev.empty());
            }
            if (!consistent(t)) {
                printf("FAILED: inconsistent pool after %d operations\n", it);
                return 1;
            }
        }
    }
    if (failures) return 1;
    printf("ok\n");
    return 0;
}
