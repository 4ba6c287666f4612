// CPU unit test of the paged cache's host bookkeeping (no GPU, no HIP):
// every refusal an append, decode, reserve, set_pages or commit can meet.
#include "page_table.h"

#include <cstdio>
#include <cstring>
#include <vector>

static int g_fail = 0;

#define EXPECT(cond)                                                       \
    do {                                                                   \
        if (!(cond)) {                                                     \
            std::printf("FAIL %s:%d: %s\n", __FILE__, __LINE__, #cond);    \
            ++g_fail;                                                      \
        }                                                                  \
    } while (0)

static bool is(const sa::Verdict& v, sa_status st, const char* needle = nullptr) {
    return v.status == st && (!needle || std::strstr(v.msg, needle));
}

int main() {
    sa::PageTable pt;
    pt.init(/*max_seqs*/ 4, /*max_pages*/ 4, /*num_pages*/ 6);
    EXPECT(pt.free_count() == 6);

    // reserve: pages in order 0, 1, ...; beyond the row or the pool is full
    EXPECT(is(pt.reserve(0, 4 * 64 + 1), SA_EFULL));
    EXPECT(pt.reserve(0, 130).ok());
    EXPECT(pt.npages(0) == 3 && pt.row(0)[0] == 0 && pt.row(0)[1] == 1 && pt.row(0)[2] == 2);
    EXPECT(pt.row(0)[3] == -1 && pt.capacity(0) == 192);
    EXPECT(is(pt.reserve(1, 4 * 64), SA_EFULL));          // 3 pages left
    EXPECT(pt.npages(1) == 0 && pt.free_count() == 3);     // refused as a whole
    EXPECT(is(pt.reserve(7, 1), SA_ERANGE));
    EXPECT(is(pt.reserve(1, -1), SA_EINVAL));
    EXPECT(pt.reserve(0, 100).ok() && pt.npages(0) == 3);  // already room

    // set_pages: ownership, duplicates, range
    EXPECT(is(pt.set_pages(1, std::vector<int32_t>{3, 1}.data(), 2, nullptr), SA_EINVAL, "another"));
    EXPECT(is(pt.set_pages(1, std::vector<int32_t>{3, 3}.data(), 2, nullptr), SA_EINVAL, "twice"));
    EXPECT(is(pt.set_pages(1, std::vector<int32_t>{6}.data(), 1, nullptr), SA_ERANGE));
    EXPECT(is(pt.set_pages(1, nullptr, 1, nullptr), SA_EINVAL));
    EXPECT(pt.free_count() == 3 && pt.npages(1) == 0);     // nothing changed
    EXPECT(pt.set_pages(1, std::vector<int32_t>{5, 3}.data(), 2, nullptr).ok());
    EXPECT(pt.owner(5) == 1 && pt.owner(3) == 1 && pt.owner(4) == -1 && pt.free_count() == 1);

    // shrinking a sequence cuts its length and frees the dropped pages
    EXPECT(pt.set_len(0, 150).ok());
    bool cut = false;
    EXPECT(pt.set_pages(0, std::vector<int32_t>{2, 0}.data(), 2, &cut).ok());
    EXPECT(cut && pt.len(0) == 128 && pt.capacity(0) == 128);
    EXPECT(pt.owner(1) == -1 && pt.free_count() == 2);
    EXPECT(pt.row(0)[0] == 2 && pt.row(0)[1] == 0 && pt.row(0)[2] == -1);
    EXPECT(pt.set_pages(0, std::vector<int32_t>{2, 0}.data(), 2, &cut).ok() && !cut);
    EXPECT(is(pt.set_len(0, 129), SA_EFULL) && pt.len(0) == 128);

    // append checks: capacity, RoPE table, bad and repeated rows
    const int32_t r01[] = {0, 1};
    const int32_t r00[] = {0, 0};
    const int32_t r09[] = {0, 9};
    EXPECT(is(pt.check_append(r01, 2, 1, 0), SA_EFULL));   // row 0 is full
    EXPECT(pt.check_append(r01 + 1, 1, 128, 0).ok());
    EXPECT(is(pt.check_append(r01 + 1, 1, 129, 0), SA_EFULL));
    EXPECT(is(pt.check_append(r01 + 1, 1, 10, 9), SA_ERANGE, "RoPE"));
    EXPECT(is(pt.check_append(r00, 2, 0, 0), SA_EINVAL, "twice"));
    EXPECT(is(pt.check_append(r09, 2, 0, 0), SA_ERANGE));
    EXPECT(is(pt.check_append(nullptr, 5, 1, 0), SA_ERANGE));
    EXPECT(is(pt.check_append(nullptr, 3, 1, 0), SA_EFULL));   // rows 0 (full) and 2 (no pages)

    // decode checks: pending tokens need pages; repeated rows are fine
    int mx = -1;
    long long tot = -1;
    EXPECT(pt.check_decode(r00, 2, 0, &mx, &tot).ok() && mx == 128 && tot == 256);
    EXPECT(is(pt.check_decode(r00, 2, 1, &mx, &tot), SA_ERANGE));
    EXPECT(pt.check_decode(r01 + 1, 1, 1, &mx, &tot).ok() && mx == 1 && tot == 1);
    EXPECT(is(pt.check_decode(r09, 2, 0, &mx, &tot), SA_ERANGE));
    EXPECT(is(pt.check_decode(r01, 2, -1, &mx, &tot), SA_EINVAL));

    // commit: all or nothing
    EXPECT(is(pt.commit(r01, 2, 1), SA_EFULL) && pt.len(1) == 0);
    EXPECT(pt.commit(r01 + 1, 1, 100).ok() && pt.len(1) == 100);
    EXPECT(is(pt.commit(r00, 2, 0), SA_EINVAL));

    // reset: everything back
    pt.reset();
    EXPECT(pt.free_count() == 6 && pt.len(1) == 0 && pt.npages(0) == 0 && pt.owner(3) == -1);
    EXPECT(pt.reserve(2, 64).ok() && pt.row(2)[0] == 0);

    if (g_fail) {
        std::printf("%d check(s) failed\n", g_fail);
        return 1;
    }
    std::printf("page table: all checks passed\n");
    return 0;
}
