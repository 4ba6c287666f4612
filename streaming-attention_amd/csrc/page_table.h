// Host-side bookkeeping of the paged KV cache: which pages each sequence
// owns, the committed lengths, the free list, and every check an append or a
// decode needs before a kernel is launched.  No HIP here: the device copy of
// the table and the lengths is written by the cache glue (kvcache.hip) from
// what this class decides, and the class is unit-tested on the CPU.
//
// The reference's dense cache has one length for the whole batch and throws
// on overflow (reference tensor_cpp/include/tensor_cpp/kv_cache.h:94-130); here
// each sequence has its own pages and length, and every overflow, bad index
// or page conflict is refused before any device work is enqueued.
#pragma once

#include <stdint.h>

#include <vector>

#include "sa_amd.h"

namespace sa {

struct Verdict {
    sa_status status;
    const char* msg;   // static text; "" when status == SA_OK
    bool ok() const { return status == SA_OK; }
};

class PageTable {
public:
    void init(int max_seqs, int max_pages_per_seq, int num_pages);
    // Every sequence back to length 0, every page back to the free list
    // (page 0 is handed out first).
    void reset();

    // Room for n_tokens tokens in total in seq, taking pages from the free list.
    Verdict reserve(int seq, int n_tokens);
    // Replace seq's pages with pages[0, n).  Every page must be in the pool,
    // listed once, and either free or already owned by seq.  A length beyond
    // the new capacity is cut to it (*len_cut tells the caller to publish it).
    Verdict set_pages(int seq, const int32_t* pages, int n, bool* len_cut);
    Verdict set_len(int seq, int len);
    // Rows ids[0, n) (NULL: 0 .. n-1) are cache rows; with unique, no row twice.
    Verdict check_rows(const int32_t* ids, int n, bool unique) const;
    // An append of S tokens to each row: every row has pages for len + S
    // tokens and, when rope_max_pos > 0, len + S <= rope_max_pos.
    Verdict check_append(const int32_t* ids, int n, int S, int rope_max_pos) const;
    // A decode over len + n_pending tokens of each row: every row has pages for
    // them.  Returns the longest such length and their sum.
    Verdict check_decode(const int32_t* ids, int n, int n_pending, int* max_len, long long* total) const;
    // len += n for each row, refused as a whole if any row would overflow.
    Verdict commit(const int32_t* ids, int n_rows, int n);

    int max_seqs() const { return max_seqs_; }
    int max_pages() const { return max_pages_; }
    int num_pages() const { return num_pages_; }
    int len(int seq) const { return lens_[seq]; }
    int capacity(int seq) const { return npages_[seq] * kPage; }
    int npages(int seq) const { return npages_[seq]; }
    int free_count() const { return (int)free_.size(); }
    int owner(int page) const { return owner_[page]; }
    const int32_t* row(int seq) const { return table_.data() + (size_t)seq * max_pages_; }
    bool valid_seq(int seq) const { return seq >= 0 && seq < max_seqs_; }

    static constexpr int kPage = SA_PAGE_TOKENS;

private:
    int max_seqs_ = 0, max_pages_ = 0, num_pages_ = 0;
    std::vector<int32_t> table_;   // [max_seqs][max_pages], -1 = no page
    std::vector<int> lens_;        // committed length per sequence
    std::vector<int> npages_;      // pages assigned per sequence
    std::vector<int32_t> free_;    // stack of free pages
    std::vector<int32_t> owner_;   // [num_pages]: owning sequence, -1 = free
};

}  // namespace sa
