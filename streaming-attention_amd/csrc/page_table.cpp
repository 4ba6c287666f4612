// Host bookkeeping of the paged KV cache (see page_table.h).
#include "page_table.h"

#include <algorithm>

namespace sa {

namespace {
constexpr Verdict kOk{SA_OK, ""};
Verdict refuse(sa_status st, const char* msg) { return Verdict{st, msg}; }
}  // namespace

void PageTable::init(int max_seqs, int max_pages_per_seq, int num_pages) {
    max_seqs_ = max_seqs;
    max_pages_ = max_pages_per_seq;
    num_pages_ = num_pages;
    reset();
}

void PageTable::reset() {
    table_.assign((size_t)max_seqs_ * max_pages_, -1);
    lens_.assign(max_seqs_, 0);
    npages_.assign(max_seqs_, 0);
    owner_.assign(num_pages_, -1);
    free_.resize(num_pages_);
    for (int i = 0; i < num_pages_; ++i) free_[i] = num_pages_ - 1 - i;
}

Verdict PageTable::reserve(int seq, int n_tokens) {
    if (!valid_seq(seq)) return refuse(SA_ERANGE, "sequence index out of range");
    if (n_tokens < 0) return refuse(SA_EINVAL, "n_tokens must be >= 0");
    const long long need = ((long long)n_tokens + kPage - 1) / kPage;
    if (need > max_pages_) return refuse(SA_EFULL, "KV cache full, cannot append more tokens");
    int have = npages_[seq];
    if (need <= have) return kOk;
    if ((long long)free_.size() < need - have) return refuse(SA_EFULL, "KV cache full, cannot append more tokens");
    int32_t* r = table_.data() + (size_t)seq * max_pages_;
    for (; have < need; ++have) {
        const int32_t p = free_.back();
        free_.pop_back();
        r[have] = p;
        owner_[p] = seq;
    }
    npages_[seq] = have;
    return kOk;
}

Verdict PageTable::set_pages(int seq, const int32_t* pages, int n, bool* len_cut) {
    if (len_cut) *len_cut = false;
    if (!valid_seq(seq)) return refuse(SA_ERANGE, "sequence index out of range");
    if (n < 0 || n > max_pages_ || (n > 0 && !pages)) return refuse(SA_EINVAL, "bad page list");
    std::vector<char> listed(num_pages_, 0);
    for (int j = 0; j < n; ++j) {
        const int32_t p = pages[j];
        if (p < 0 || p >= num_pages_) return refuse(SA_ERANGE, "page id out of range");
        if (listed[p]) return refuse(SA_EINVAL, "page listed twice");
        listed[p] = 1;
        if (owner_[p] != -1 && owner_[p] != seq) return refuse(SA_EINVAL, "page owned by another sequence");
    }
    int32_t* r = table_.data() + (size_t)seq * max_pages_;
    // The sequence's pages that are not kept go back to the free list.
    for (int j = 0; j < npages_[seq]; ++j) {
        const int32_t p = r[j];
        if (!listed[p]) {
            owner_[p] = -1;
            free_.push_back(p);
        }
    }
    // Listed pages that were free leave the free list.
    free_.erase(std::remove_if(free_.begin(), free_.end(), [&](int32_t p) { return listed[p] != 0; }),
                free_.end());
    for (int j = 0; j < max_pages_; ++j) r[j] = j < n ? pages[j] : -1;
    for (int j = 0; j < n; ++j) owner_[pages[j]] = seq;
    npages_[seq] = n;
    if (lens_[seq] > n * kPage) {
        lens_[seq] = n * kPage;
        if (len_cut) *len_cut = true;
    }
    return kOk;
}

Verdict PageTable::set_len(int seq, int len) {
    if (!valid_seq(seq)) return refuse(SA_ERANGE, "sequence index out of range");
    if (len < 0 || len > capacity(seq)) return refuse(SA_EFULL, "length exceeds reserved pages");
    lens_[seq] = len;
    return kOk;
}

Verdict PageTable::check_rows(const int32_t* ids, int n, bool unique) const {
    if (n < 0) return refuse(SA_EINVAL, "negative sequence count");
    if (!ids) {
        if (n > max_seqs_) return refuse(SA_ERANGE, "sequence index out of range");
        return kOk;
    }
    std::vector<char> seen(unique ? max_seqs_ : 0, 0);
    for (int i = 0; i < n; ++i) {
        if (!valid_seq(ids[i])) return refuse(SA_ERANGE, "sequence index out of range");
        if (unique) {
            if (seen[ids[i]]) return refuse(SA_EINVAL, "sequence listed twice");
            seen[ids[i]] = 1;
        }
    }
    return kOk;
}

Verdict PageTable::check_append(const int32_t* ids, int n, int S, int rope_max_pos) const {
    Verdict v = check_rows(ids, n, true);
    if (!v.ok()) return v;
    for (int i = 0; i < n; ++i) {
        const int s = ids ? ids[i] : i;
        const long long end = (long long)lens_[s] + S;
        if (end > capacity(s)) return refuse(SA_EFULL, "KV cache full, cannot append more tokens");
        if (rope_max_pos > 0 && end > rope_max_pos) return refuse(SA_ERANGE, "position beyond RoPE table");
    }
    return kOk;
}

Verdict PageTable::check_decode(const int32_t* ids, int n, int n_pending, int* max_len, long long* total) const {
    Verdict v = check_rows(ids, n, false);
    if (!v.ok()) return v;
    if (n_pending < 0) return refuse(SA_EINVAL, "n_pending must be >= 0");
    int mx = 0;
    long long sum = 0;
    for (int i = 0; i < n; ++i) {
        const int s = ids ? ids[i] : i;
        const long long L = (long long)lens_[s] + n_pending;
        if (L > capacity(s)) return refuse(SA_ERANGE, "Requested seq_len exceeds cached length");
        mx = std::max(mx, (int)L);
        sum += L;
    }
    if (max_len) *max_len = mx;
    if (total) *total = sum;
    return kOk;
}

Verdict PageTable::commit(const int32_t* ids, int n_rows, int n) {
    if (n < 0) return refuse(SA_EINVAL, "n must be >= 0");
    Verdict v = check_rows(ids, n_rows, true);
    if (!v.ok()) return v;
    for (int i = 0; i < n_rows; ++i) {
        const int s = ids ? ids[i] : i;
        if ((long long)lens_[s] + n > capacity(s)) return refuse(SA_EFULL, "KV cache full, cannot append more tokens");
    }
    for (int i = 0; i < n_rows; ++i) lens_[ids ? ids[i] : i] += n;
    return kOk;
}

}  // namespace sa
