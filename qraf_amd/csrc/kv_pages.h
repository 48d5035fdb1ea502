// kv_pages.h -- the engine's host-side KV page bookkeeping (plain C++, no GPU
// code; built into libqraf_hip.so and, with AddressSanitizer and
// UndefinedBehaviorSanitizer, into tests/cpp/kv_pages_check).
//
// The reference's KVCache (attention.cpp:14-52) holds one contiguous
// [max_seq_len] cache per layer for its single sequence; the engine instead
// gives every sequence pages of page_size positions from one pool of
// num_pages, so a continuous batch (batch_scheduler.h:54-283) admits a new
// request into the pages a finished one released.  This class owns that
// state: which sequences live, their lengths, the pages each holds (in
// position order) and the free list.  A step's rows are checked and their
// pages allocated in one call that changes nothing unless every row is valid
// and the pool holds every new page.
#pragma once

#include <cstdint>
#include <vector>

namespace qraf_hip {

class KvPages {
public:
    // num_pages pages of page_size positions; a sequence holds at most
    // capacity positions (max_pages() pages).  QRAF_HIP_ERR_INVALID for
    // non-positive sizes.
    int init(int num_pages, int page_size, int capacity);

    int seq_create(int32_t* id);   // a released id is reused first
    int seq_release(int32_t id);   // its pages return to the pool
    int seq_length(int32_t id, int32_t* len) const;
    bool live(int32_t id) const { return id >= 0 && id < (int32_t)seqs_.size() && seqs_[id].live; }

    int free_pages() const { return (int)free_.size(); }
    int max_pages() const { return max_pages_; }
    int num_pages() const { return num_pages_; }
    // one page past the pool: the page table's entry for the engine's pad rows
    int32_t scratch_page() const { return num_pages_; }

    // One step of n rows: row i adds position positions[i] of sequence
    // seq_ids[i].  Every sequence must live, every position lie in
    // [0, capacity) and not skip past the sequence's length (counting the
    // step's earlier rows: chunked prefill), and the pool must hold the pages
    // the new positions need; otherwise an error status (QRAF_HIP_ERR_INVALID,
    // QRAF_HIP_ERR_NOMEM) and no change.  On success the pages are taken from
    // the pool, the lengths updated, row i's page table (max_pages() entries,
    // 0 past the sequence's pages) written to ptab + i * max_pages(), and
    // *step_ctx set to the longest context (position + 1) of the step.
    int plan_step(int n, const int32_t* seq_ids, const int32_t* positions, int32_t* ptab, int* step_ctx);

    // Consistency of the whole state: every page either free or held by
    // exactly one live sequence, each sequence's page count that of its
    // length, released sequences holding none.  For the sanitized tests.
    bool consistent() const;

private:
    struct Seq {
        bool live = false;
        int len = 0;
        std::vector<int32_t> pages;
        uint64_t stamp = 0;  // the step that last validated this sequence
        int step_len = 0, step_pages = 0;
    };
    std::vector<Seq> seqs_;
    std::vector<int32_t> free_;
    int num_pages_ = 0, page_size_ = 0, capacity_ = 0, max_pages_ = 0;
    uint64_t step_stamp_ = 0;
};

}  // namespace qraf_hip
