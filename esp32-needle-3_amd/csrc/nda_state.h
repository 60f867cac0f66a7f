/* nda_state.h - host-side session bookkeeping of libndattn: per-sequence
 * state, the position -> slot arithmetic of the engine's KV ring, and the
 * page tables with their free list and journal. Plain C++ with no HIP
 * dependence: the library includes it, and so does a CPU check built with
 * address and undefined-behaviour sanitizers. */
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <algorithm>
#include <vector>

namespace nda_host {

constexpr uint32_t MIN_RECENT = 64;   // ND_MIN_RECENT, engine/src/nd_model.c:1311-1312

struct Prefix {
    bool used = false;
    uint32_t len = 0;       // positions stored: [0, len)
    uint32_t n_sink = 0;    // pinned count (clamped len)
    uint32_t refs = 0;      // sequences attached
};

// The engine's per-session position state (nd_model.h:132-148: pos, n_sink),
// plus the attached prefix segment and what a rewind restores.
struct SeqHost {
    uint32_t pos = 0, n_sink = 0;
    int32_t prefix = -1;
    bool has_snap = false;
    uint32_t snap_pos = 0;
    uint32_t stored_end = 0;   // one past the highest position stored
    uint32_t ring_lo = 0;      // ring positions in [n_sink, ring_lo) were overwritten before a rewind
};

// nd_model_set_sink's clamp: at least ND_MIN_RECENT ring slots stay
// (engine/src/nd_model.c:1314-1321).
inline uint32_t clamp_sink(uint32_t window, uint32_t n)
{
    uint32_t cap = window > MIN_RECENT ? window - MIN_RECENT : 0;
    return n < cap ? n : cap;
}

// Own slot of position p: kv_slot (engine/src/nd_model.c:1302-1309), with the
// sinks of an attached prefix living in the prefix's pages instead.
inline uint32_t own_slot(const SeqHost &s, uint32_t p, uint32_t window)
{
    if (s.prefix >= 0)
        return (p - s.n_sink) % (window - s.n_sink);
    if (p < s.n_sink)
        return p;
    return s.n_sink + (p - s.n_sink) % (window - s.n_sink);
}

// The positions a token at p attends (the dispatch of attention(),
// engine/src/nd_model.c:2451-2483), split into the shared-prefix run and the
// sequence's own slots [0, n_own).
struct Vis {
    uint32_t n_sh, n_own;
};

inline Vis visible(const SeqHost &s, uint32_t p, uint32_t window)
{
    uint32_t sinks = std::min(s.n_sink, p + 1);
    uint32_t rcap = window - s.n_sink;
    uint32_t rcount = (p + 1 <= s.n_sink) ? 0 : std::min(p + 1 - s.n_sink, rcap);
    Vis v;
    v.n_sh = s.prefix >= 0 ? sinks : 0;
    v.n_own = s.prefix >= 0 ? rcount : sinks + rcount;
    return v;
}

// Page tables of one context: per sequence and per prefix segment a row of
// page ids (-1: not backed), and the free list. Rows of sequences changed
// since the last upload are [dirty_lo, dirty_hi). While a transaction is
// open, every page a sequence row takes is journaled so it can be given back.
struct PageTables {
    uint32_t pages_per_seq = 0, log2_page = 0;
    std::vector<int32_t> pages, prefix_pages, free_pages;
    std::vector<size_t> journal;
    int txn_depth = 0;
    uint32_t dirty_lo = UINT32_MAX, dirty_hi = 0;
    bool prefix_dirty = true;

    // Low page ids are handed out first.
    void init(uint32_t max_seqs, uint32_t max_prefixes, uint32_t pps, uint32_t lg, uint64_t max_pages)
    {
        pages_per_seq = pps;
        log2_page = lg;
        pages.assign((size_t)max_seqs * pps, -1);
        prefix_pages.assign((size_t)max_prefixes * pps, -1);
        free_pages.resize(max_pages);
        for (uint64_t i = 0; i < max_pages; i++)
            free_pages[i] = (int32_t)(max_pages - 1 - i);
        dirty_lo = 0;
        dirty_hi = max_seqs;
    }

    int32_t *row(uint32_t seq) { return &pages[(size_t)seq * pages_per_seq]; }
    const int32_t *row(uint32_t seq) const { return &pages[(size_t)seq * pages_per_seq]; }
    int32_t *prefix_row(int32_t id) { return &prefix_pages[(size_t)id * pages_per_seq]; }

    void mark(uint32_t seq)
    {
        dirty_lo = std::min(dirty_lo, seq);
        dirty_hi = std::max(dirty_hi, seq + 1);
    }

    // Pages backing own slots [s0, s1) of a sequence would take.
    size_t need(uint32_t seq, uint32_t s0, uint32_t s1) const
    {
        if (s1 <= s0)
            return 0;
        const int32_t *r = row(seq);
        size_t n = 0;
        for (uint32_t i = s0 >> log2_page; i <= (s1 - 1) >> log2_page; i++)
            n += r[i] < 0;
        return n;
    }

    // Back own slots [s0, s1): all or nothing (false: too few free pages).
    bool back_slots(uint32_t seq, uint32_t s0, uint32_t s1)
    {
        if (s1 <= s0)
            return true;
        if (need(seq, s0, s1) > free_pages.size())
            return false;
        int32_t *r = row(seq);
        for (uint32_t i = s0 >> log2_page; i <= (s1 - 1) >> log2_page; i++) {
            if (r[i] < 0) {
                r[i] = free_pages.back();
                free_pages.pop_back();
                mark(seq);
                if (txn_depth)
                    journal.push_back((size_t)seq * pages_per_seq + i);
            }
        }
        return true;
    }

    // Back the own slots of positions [p0, p0 + n) (n >= 1, no wrap inside a
    // run): positions map to consecutive slots until the ring wraps, so the
    // walk goes run by run. False: the pool ran out, possibly after earlier
    // runs took pages (a transaction gives those back).
    bool back_positions(uint32_t seq, const SeqHost &s, uint32_t p0, uint32_t n, uint32_t window)
    {
        uint32_t p = p0, end = p0 + n;
        while (p < end) {
            uint32_t sl = own_slot(s, p, window);
            uint32_t run;
            if (s.prefix < 0 && p < s.n_sink)
                run = std::min(end, s.n_sink) - p;
            else {
                uint32_t ring_end = (s.prefix >= 0 ? 0u : s.n_sink) + (window - s.n_sink);
                run = std::min(end - p, ring_end - sl);
            }
            if (!back_slots(seq, sl, sl + run))
                return false;
            p += run;
        }
        return true;
    }

    size_t backed(uint32_t seq) const
    {
        const int32_t *r = row(seq);
        size_t n = 0;
        for (uint32_t i = 0; i < pages_per_seq; i++)
            n += r[i] >= 0;
        return n;
    }

    void release(uint32_t seq)
    {
        int32_t *r = row(seq);
        for (uint32_t i = 0; i < pages_per_seq; i++) {
            if (r[i] >= 0) {
                free_pages.push_back(r[i]);
                r[i] = -1;
            }
        }
        mark(seq);
    }

    // The first npages of a prefix segment's row: all or nothing.
    bool take_prefix(int32_t id, uint32_t npages)
    {
        if (npages > free_pages.size())
            return false;
        int32_t *r = prefix_row(id);
        for (uint32_t i = 0; i < npages; i++) {
            r[i] = free_pages.back();
            free_pages.pop_back();
        }
        prefix_dirty = true;
        return true;
    }

    void release_prefix(int32_t id)
    {
        int32_t *r = prefix_row(id);
        for (uint32_t i = 0; i < pages_per_seq; i++)
            if (r[i] >= 0) {
                free_pages.push_back(r[i]);
                r[i] = -1;
            }
        prefix_dirty = true;
    }
};

// The pages a call backs stay journaled until it commits; a call that fails
// part-way (the pool runs out for a later sequence, a buffer cannot grow)
// gives them back in reverse order, so the page tables and the free list are
// as before the call.
struct PageTxn {
    PageTables &t;
    size_t mark;
    bool open = true;
    explicit PageTxn(PageTables &t_) : t(t_), mark(t_.journal.size()) { t.txn_depth++; }
    PageTxn(const PageTxn &) = delete;
    PageTxn &operator=(const PageTxn &) = delete;
    void commit()
    {
        if (open) {
            open = false;
            t.txn_depth--;
            if (!t.txn_depth)
                t.journal.clear();
        }
    }
    ~PageTxn()
    {
        if (!open)
            return;
        while (t.journal.size() > mark) {
            const size_t idx = t.journal.back();
            t.journal.pop_back();
            t.free_pages.push_back(t.pages[idx]);
            t.pages[idx] = -1;
            t.mark((uint32_t)(idx / t.pages_per_seq));
        }
        t.txn_depth--;
    }
};

} // namespace nda_host
