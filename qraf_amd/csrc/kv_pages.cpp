// kv_pages.cpp -- the engine's host-side KV page bookkeeping (see kv_pages.h).
#include "kv_pages.h"

#include <algorithm>

#include "qraf_hip.h"
#include "status.h"

namespace qraf_hip {

int KvPages::init(int num_pages, int page_size, int capacity) {
    QH_REQUIRE(num_pages > 0 && page_size > 0 && capacity > 0, QRAF_HIP_ERR_INVALID,
               "kv pages: %d pages of %d positions, capacity %d", num_pages, page_size, capacity);
    num_pages_ = num_pages;
    page_size_ = page_size;
    capacity_ = capacity;
    max_pages_ = (capacity + page_size - 1) / page_size;
    seqs_.clear();
    free_.resize((size_t)num_pages);
    for (int i = 0; i < num_pages; i++) free_[(size_t)i] = num_pages - 1 - i;  // page 0 is taken first
    step_stamp_ = 0;
    return QRAF_HIP_OK;
}

int KvPages::seq_create(int32_t* id) {
    QH_REQUIRE(id, QRAF_HIP_ERR_INVALID, "seq_create: null argument");
    for (size_t i = 0; i < seqs_.size(); i++)
        if (!seqs_[i].live) {
            seqs_[i].live = true;
            seqs_[i].len = 0;
            *id = (int32_t)i;
            return QRAF_HIP_OK;
        }
    seqs_.push_back({});
    seqs_.back().live = true;
    *id = (int32_t)seqs_.size() - 1;
    return QRAF_HIP_OK;
}

int KvPages::seq_release(int32_t id) {
    QH_REQUIRE(live(id), QRAF_HIP_ERR_INVALID, "seq_release: unknown sequence %d", id);
    Seq& sq = seqs_[(size_t)id];
    for (int32_t p : sq.pages) free_.push_back(p);
    sq.pages.clear();
    sq.len = 0;
    sq.live = false;
    return QRAF_HIP_OK;
}

int KvPages::seq_length(int32_t id, int32_t* len) const {
    QH_REQUIRE(len && live(id), QRAF_HIP_ERR_INVALID, "seq_length: unknown sequence %d", id);
    *len = seqs_[(size_t)id].len;
    return QRAF_HIP_OK;
}

int KvPages::plan_step(int n, const int32_t* seq_ids, const int32_t* positions, int32_t* ptab, int* step_ctx) {
    QH_REQUIRE(n > 0 && seq_ids && positions && ptab && step_ctx, QRAF_HIP_ERR_INVALID, "step: bad arguments");
    // validate, and count the pages each sequence needs (before allocating
    // any): per sequence, the length and page count so far in this step
    const uint64_t stamp = ++step_stamp_;
    int need = 0;
    for (int i = 0; i < n; i++) {
        const int32_t id = seq_ids[i], p = positions[i];
        QH_REQUIRE(live(id), QRAF_HIP_ERR_INVALID, "step: unknown sequence %d", id);
        QH_REQUIRE(p >= 0 && p < capacity_, QRAF_HIP_ERR_INVALID, "step: position %d outside the cache (%d)", p,
                   capacity_);
        Seq& sq = seqs_[(size_t)id];
        if (sq.stamp != stamp) {
            sq.stamp = stamp;
            sq.step_len = sq.len;
            sq.step_pages = (int)sq.pages.size();
        }
        // rows of one sequence add positions without gaps (earlier rows count)
        QH_REQUIRE(p <= sq.step_len, QRAF_HIP_ERR_INVALID, "step: sequence %d position %d skips past its length %d",
                   id, p, sq.step_len);
        sq.step_len = std::max(sq.step_len, p + 1);
        const int pages = std::max(sq.step_pages, p / page_size_ + 1);
        need += pages - sq.step_pages;
        sq.step_pages = pages;
    }
    QH_REQUIRE(need <= (int)free_.size(), QRAF_HIP_ERR_NOMEM, "step: KV page pool exhausted (%d pages needed, %zu free)",
               need, free_.size());
    int ctx = 1;
    for (int i = 0; i < n; i++) {
        Seq& sq = seqs_[(size_t)seq_ids[i]];
        while ((int)sq.pages.size() < positions[i] / page_size_ + 1) {
            sq.pages.push_back(free_.back());
            free_.pop_back();
        }
        sq.len = std::max(sq.len, positions[i] + 1);
        ctx = std::max(ctx, positions[i] + 1);
        int32_t* row = ptab + (size_t)i * max_pages_;
        for (int j = 0; j < max_pages_; j++) row[j] = j < (int)sq.pages.size() ? sq.pages[(size_t)j] : 0;
    }
    *step_ctx = ctx;
    return QRAF_HIP_OK;
}

bool KvPages::consistent() const {
    std::vector<int> owner((size_t)num_pages_, 0);
    for (int32_t p : free_) {
        if (p < 0 || p >= num_pages_ || owner[(size_t)p]++) return false;
    }
    for (const Seq& sq : seqs_) {
        if (!sq.live) {
            if (!sq.pages.empty() || sq.len) return false;
            continue;
        }
        if (sq.len < 0 || sq.len > capacity_) return false;
        if ((int)sq.pages.size() != (sq.len + page_size_ - 1) / page_size_) return false;
        for (int32_t p : sq.pages)
            if (p < 0 || p >= num_pages_ || owner[(size_t)p]++) return false;
    }
    for (int c : owner)
        if (c != 1) return false;
    return true;
}

}  // namespace qraf_hip
