// The engine's host-side KV page bookkeeping (qraf_amd/csrc/kv_pages.cpp)
// built with AddressSanitizer and UndefinedBehaviorSanitizer and driven by
// seeded random operations: sequence create / release (valid and unknown
// ids), steps of random rows (decode rows, chunked prefill runs, repeated
// sequences, and invalid rows: unknown or released sequences, positions
// outside the cache, positions that skip past a sequence's length) and pools
// small enough to run out.  Each step's status is checked against the rules
// restated here (any invalid row: QRAF_HIP_ERR_INVALID; else more new pages
// than free: QRAF_HIP_ERR_NOMEM; else OK), a refused step must change
// nothing, an accepted one must extend every sequence's page list (earlier
// pages unchanged) with page-table rows matching it, and the whole state must
// stay consistent (every page free or held by one live sequence).
//
// usage: kv_pages_check [seed] [rounds]; prints one summary line, exit 0 on success.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <iterator>
#include <map>
#include <random>
#include <vector>

#include "../../qraf_amd/csrc/kv_pages.h"
#include "qraf_hip.h"

using qraf_hip::KvPages;

#define CHECK(cond, ...)                          \
    do {                                          \
        if (!(cond)) {                            \
            std::fprintf(stderr, "FAIL line %d: ", __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);    \
            std::fprintf(stderr, "\n");           \
            std::exit(1);                         \
        }                                         \
    } while (0)

struct Shadow {
    int len = 0;
    std::vector<int32_t> pages;  // as last seen in a page-table row
};

static int run(uint32_t seed, int rounds, long* n_ok, long* n_inval, long* n_nomem) {
    std::mt19937 rng(seed);
    auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
    const int page_size = 1 << uni(0, 5);           // 1 .. 32
    const int capacity = uni(1, 300);
    const int max_pages = (capacity + page_size - 1) / page_size;
    const int num_pages = uni(1, 3 * max_pages + 4);
    KvPages kv;
    CHECK(kv.init(num_pages, page_size, capacity) == QRAF_HIP_OK, "init");
    CHECK(kv.init(0, page_size, capacity) != QRAF_HIP_OK, "init with no pages accepted");
    CHECK(kv.init(num_pages, page_size, capacity) == QRAF_HIP_OK, "re-init");
    CHECK(kv.max_pages() == max_pages && kv.free_pages() == num_pages && kv.scratch_page() == num_pages, "sizes");
    std::map<int32_t, Shadow> live;
    std::vector<int32_t> released;
    for (int round = 0; round < rounds; round++) {
        const int op = uni(0, 9);
        if (op == 0 || live.empty()) {
            int32_t id = -1;
            CHECK(kv.seq_create(&id) == QRAF_HIP_OK, "create");
            CHECK(id >= 0 && !live.count(id), "create returned a live id %d", id);
            live[id] = Shadow{};
            int32_t len = -1;
            CHECK(kv.seq_length(id, &len) == QRAF_HIP_OK && len == 0, "new sequence length");
        } else if (op == 1) {
            // release: a live sequence, or an unknown / released id (refused)
            if (uni(0, 3) == 0) {
                const int32_t bad = uni(0, 2) ? -1 - uni(0, 5) : 1000 + uni(0, 5);
                CHECK(kv.seq_release(bad) == QRAF_HIP_ERR_INVALID, "release of unknown %d accepted", bad);
                for (int32_t r : released)
                    if (!live.count(r)) CHECK(kv.seq_release(r) == QRAF_HIP_ERR_INVALID, "double release of %d", r);
            } else {
                auto it = live.begin();
                std::advance(it, uni(0, (int)live.size() - 1));
                const int before = kv.free_pages();
                CHECK(kv.seq_release(it->first) == QRAF_HIP_OK, "release");
                CHECK(kv.free_pages() == before + (int)it->second.pages.size(), "pages not returned");
                released.push_back(it->first);
                live.erase(it);
            }
        } else {
            // a step: rows over some live sequences, each a run of consecutive
            // positions from its length (chunked prefill) or a repeated
            // position, plus sometimes an invalid row
            std::vector<int32_t> ids, pos;
            std::vector<int32_t> order;
            for (auto& kvp : live) order.push_back(kvp.first);
            std::shuffle(order.begin(), order.end(), rng);
            const int nseq = uni(1, (int)order.size());
            for (int k = 0; k < nseq; k++) {
                const int32_t id = order[k];
                const int len = live[id].len;
                const int run = uni(0, 3) == 0 ? uni(1, 2 * page_size + 3) : 1;
                const int start = uni(0, 4) == 0 && len > 0 ? uni(0, len - 1) : len;  // rewrite an earlier position
                for (int j = 0; j < run; j++) {
                    ids.push_back(id);
                    pos.push_back(start + j);
                }
            }
            const int bad = uni(0, 7);
            if (bad == 0 && !released.empty()) {
                ids.push_back(released[uni(0, (int)released.size() - 1)]);
                pos.push_back(0);
            } else if (bad == 1) {
                ids.push_back(order[0]);
                pos.push_back(capacity + uni(0, 3));
            } else if (bad == 2) {
                ids.push_back(order[0]);
                pos.push_back(-1 - uni(0, 3));
            } else if (bad == 3) {
                ids.push_back(order[0]);
                pos.push_back(live[order[0]].len + 2 + uni(0, 3) + (int)pos.size());  // skips past its length
            } else if (bad == 4) {
                ids.push_back(1 << 20);
                pos.push_back(0);
            }
            if (uni(0, 1)) {  // rows in a random order (a sequence's own rows keep theirs)
                std::vector<int> idx(ids.size());
                for (size_t i = 0; i < idx.size(); i++) idx[i] = (int)i;
                std::stable_sort(idx.begin(), idx.end(), [&](int a, int b) { return ids[a] < ids[b]; });
                std::vector<int32_t> i2, p2;
                for (int i : idx) {
                    i2.push_back(ids[i]);
                    p2.push_back(pos[i]);
                }
                ids.swap(i2);
                pos.swap(p2);
            }
            // the rules, restated: every row valid in order, then the pool
            const int n = (int)ids.size();
            bool valid = true;
            std::map<int32_t, int> step_len, step_pages;
            int need = 0;
            for (int i = 0; i < n && valid; i++) {
                const int32_t id = ids[i], p = pos[i];
                if (!live.count(id) || p < 0 || p >= capacity) {
                    valid = false;
                    break;
                }
                if (!step_len.count(id)) {
                    step_len[id] = live[id].len;
                    step_pages[id] = (int)live[id].pages.size();
                }
                if (p > step_len[id]) {
                    valid = false;
                    break;
                }
                step_len[id] = std::max(step_len[id], p + 1);
                const int pg = std::max(step_pages[id], p / page_size + 1);
                need += pg - step_pages[id];
                step_pages[id] = pg;
            }
            const int want = !valid ? QRAF_HIP_ERR_INVALID : need > kv.free_pages() ? QRAF_HIP_ERR_NOMEM : QRAF_HIP_OK;
            std::vector<int32_t> ptab((size_t)n * max_pages + 1, -7);
            const int free_before = kv.free_pages();
            int ctx = -1;
            const int rc = kv.plan_step(n, ids.data(), pos.data(), ptab.data(), &ctx);
            CHECK(rc == want, "step of %d rows: status %d, want %d", n, rc, want);
            if (rc != QRAF_HIP_OK) {
                CHECK(kv.free_pages() == free_before, "refused step changed the pool");
                for (auto& kvp : live) {
                    int32_t len = -1;
                    CHECK(kv.seq_length(kvp.first, &len) == QRAF_HIP_OK && len == kvp.second.len,
                          "refused step changed sequence %d", kvp.first);
                }
                (rc == QRAF_HIP_ERR_NOMEM ? *n_nomem : *n_inval) += 1;
            } else {
                *n_ok += 1;
                CHECK(kv.free_pages() == free_before - need, "pages taken %d, want %d", free_before - kv.free_pages(),
                      need);
                int want_ctx = 1;
                for (int i = 0; i < n; i++) {
                    Shadow& sh = live[ids[i]];
                    sh.len = std::max(sh.len, pos[i] + 1);
                    want_ctx = std::max(want_ctx, pos[i] + 1);
                    const int np = pos[i] / page_size + 1;
                    const int32_t* row = ptab.data() + (size_t)i * max_pages;
                    CHECK(np <= max_pages, "page index past max_pages");
                    // the sequence's earlier pages unchanged, its new ones valid, zeros past them
                    const int held = std::max(np, (int)sh.pages.size());
                    for (int j = 0; j < (int)sh.pages.size(); j++)
                        CHECK(row[j] == sh.pages[j], "sequence %d page %d moved", ids[i], j);
                    for (int j = 0; j < max_pages; j++) {
                        if (j < held) CHECK(row[j] >= 0 && row[j] < num_pages, "page id %d", row[j]);
                        else CHECK(row[j] == 0, "entry %d past the sequence's %d pages is %d", j, held, row[j]);
                    }
                    sh.pages.assign(row, row + held);
                }
                CHECK(ctx == want_ctx, "step_ctx %d, want %d", ctx, want_ctx);
                CHECK(ptab[(size_t)n * max_pages] == -7, "page table written past its rows");
                for (auto& kvp : live) {
                    int32_t len = -1;
                    CHECK(kv.seq_length(kvp.first, &len) == QRAF_HIP_OK && len == kvp.second.len,
                          "sequence %d length %d, want %d", kvp.first, len, kvp.second.len);
                }
            }
        }
        CHECK(kv.consistent(), "inconsistent state after round %d", round);
        int held = 0;
        for (auto& kvp : live) held += (kvp.second.len + page_size - 1) / page_size;
        CHECK(held + kv.free_pages() == num_pages, "pages held %d + free %d != %d", held, kv.free_pages(), num_pages);
    }
    // release everything: the whole pool comes back
    for (auto& kvp : live) CHECK(kv.seq_release(kvp.first) == QRAF_HIP_OK, "final release");
    CHECK(kv.free_pages() == num_pages && kv.consistent(), "pool not whole at the end");
    return 0;
}

int main(int argc, char** argv) {
    const uint32_t seed = argc > 1 ? (uint32_t)std::strtoul(argv[1], nullptr, 10) : 1;
    const int rounds = argc > 2 ? std::atoi(argv[2]) : 400;
    long ok = 0, inval = 0, nomem = 0;
    for (uint32_t s = seed; s < seed + 200; s++) run(s, rounds, &ok, &inval, &nomem);
    std::printf("kv_pages_check: 200 pools, %d rounds each: %ld steps accepted, %ld invalid refused, %ld refused "
                "for lack of pages\n",
                rounds, ok, inval, nomem);
    return 0;
}
