// sanitize_check.cpp - host code of this repository run under the address
// and undefined-behaviour sanitizers (CPU only; built and run by
// tests/test_sanitizers.py):
//   1. the session bookkeeping of libndattn (esp32-needle-3_amd/csrc/
//      nda_state.h): slot arithmetic against the oracle's kv_slot, and
//      randomized page-table operations with their invariants checked after
//      every step;
//   2. the oracle (oracle/nd_oracle.c): sessions with snapshot / rewind /
//      prefix save-restore over several geometries, explicit runs, the front,
//      the threaded fp16 batch decode.
// Any sanitizer report aborts the run; a failed check exits non-zero.
#include "nd_oracle.h"
#include "nda_state.h"

#include <stdio.h>
#include <stdlib.h>

#include <random>
#include <set>
#include <vector>

using namespace nda_host;

static int failures = 0;
#define CHECK(cond)                                                              \
    do {                                                                         \
        if (!(cond)) {                                                           \
            fprintf(stderr, "check failed %s:%d: %s\n", __FILE__, __LINE__, #cond); \
            if (++failures > 20)                                                 \
                exit(1);                                                         \
        }                                                                        \
    } while (0)

// ---------------------------------------------------------------- slots

static void check_slots(std::mt19937 &rng)
{
    for (int trial = 0; trial < 2000; trial++) {
        const uint32_t W = 2 + rng() % 500;
        SeqHost s;
        const uint32_t req = rng() % (W + 10);
        s.n_sink = clamp_sink(W, req);
        CHECK(s.n_sink == ndo_clamp_sink(W, req));
        for (int k = 0; k < 20; k++) {
            const uint32_t p = rng() % (4 * W + 3);
            CHECK(own_slot(s, p, W) == ndo_kv_slot(W, s.n_sink, p));
            const Vis v = visible(s, p, W);
            // every visible position's slot lies in [0, n_own) and they are distinct
            const uint32_t sinks = std::min(s.n_sink, p + 1);
            CHECK(v.n_sh == 0 && v.n_own >= sinks && v.n_own <= W);
            std::set<uint32_t> seen;
            for (uint32_t q = 0; q < sinks; q++)
                seen.insert(own_slot(s, q, W));
            for (uint32_t q = p + 1 - (v.n_own - sinks); q <= p && v.n_own > sinks; q++)
                seen.insert(own_slot(s, q, W));
            CHECK(seen.size() == v.n_own);
            CHECK(seen.empty() || *seen.rbegin() < v.n_own);
        }
    }
    // attached: sinks come from the prefix, own slots are ring indices
    for (int trial = 0; trial < 500; trial++) {
        const uint32_t W = 70 + rng() % 400;
        SeqHost s;
        s.prefix = 0;
        s.n_sink = clamp_sink(W, 1 + rng() % W);
        const uint32_t p = s.n_sink + rng() % (3 * W);
        const Vis v = visible(s, p, W);
        CHECK(v.n_sh == s.n_sink && v.n_own == std::min(p + 1 - s.n_sink, W - s.n_sink));
        CHECK(own_slot(s, p, W) == (p - s.n_sink) % (W - s.n_sink));
    }
}

// ---------------------------------------------------------- page tables

struct Model {
    PageTables t;
    std::vector<SeqHost> seqs;
    uint32_t window, P;
    uint64_t max_pages;
};

static void invariants(const Model &m)
{
    std::vector<int> owner(m.max_pages, 0);
    for (int32_t x : m.t.pages)
        if (x >= 0) {
            CHECK(x < (int32_t)m.max_pages);
            owner[x]++;
        }
    for (int32_t x : m.t.prefix_pages)
        if (x >= 0)
            owner[x]++;
    for (int32_t x : m.t.free_pages) {
        CHECK(x >= 0 && x < (int32_t)m.max_pages);
        owner[x]++;
    }
    for (uint64_t i = 0; i < m.max_pages; i++)
        CHECK(owner[i] == 1);
    CHECK(m.t.txn_depth > 0 || m.t.journal.empty());
}

// Every own slot a sequence at m.seqs[q].pos has stored is backed.
static void covered(const Model &m, uint32_t q)
{
    const SeqHost &s = m.seqs[q];
    if (s.pos == 0)
        return;
    const Vis v = visible(s, s.pos - 1, m.window);
    for (uint32_t sl = 0; sl < v.n_own; sl++)
        CHECK(m.t.row(q)[sl / m.P] >= 0);
}

static void check_pages(std::mt19937 &rng)
{
    for (int round = 0; round < 40; round++) {
        Model m;
        const uint32_t lg = 4 + rng() % 3;
        m.P = 1u << lg;
        m.window = 32 + rng() % 300;
        const uint32_t pps = (m.window + m.P - 1) / m.P, nseq = 3 + rng() % 6, npre = 3;
        m.max_pages = 1 + rng() % (nseq * pps + 4);
        m.t.init(nseq, npre, pps, lg, m.max_pages);
        m.seqs.assign(nseq, SeqHost());
        for (auto &s : m.seqs)
            s.n_sink = rng() % 2 ? clamp_sink(m.window, rng() % m.window) : 0;
        invariants(m);
        for (int op = 0; op < 400; op++) {
            const uint32_t kind = rng() % 7;
            if (kind <= 2) {
                // a batch of appends / chunks: all or nothing
                const PageTables before = m.t;
                std::vector<uint32_t> ids, n;
                for (uint32_t q = 0; q < nseq; q++)
                    if (rng() % 2) {
                        ids.push_back(q);
                        const uint32_t room = m.window - (m.seqs[q].pos < m.window ? m.seqs[q].pos : 0);
                        n.push_back(kind == 0 ? 1 : 1 + rng() % std::max(1u, std::min(room, 40u)));
                    }
                bool ok = true;
                {
                    PageTxn txn(m.t);
                    for (size_t i = 0; i < ids.size() && ok; i++) {
                        SeqHost &s = m.seqs[ids[i]];
                        if (n[i] > 1 && s.pos + n[i] > m.window)
                            n[i] = 1;   // chunks do not wrap (the prefill refuses them)
                        ok = m.t.back_positions(ids[i], s, s.pos, n[i], m.window);
                    }
                    const bool forced = rng() % 8 == 0;   // a later step of the call fails
                    if (ok && !forced)
                        txn.commit();
                    else
                        ok = false;
                }
                invariants(m);
                if (ok) {
                    for (size_t i = 0; i < ids.size(); i++) {
                        m.seqs[ids[i]].pos += n[i];
                        covered(m, ids[i]);
                    }
                } else {
                    CHECK(m.t.pages == before.pages && m.t.free_pages == before.free_pages);
                }
            } else if (kind == 3) {
                const uint32_t q = rng() % nseq;
                m.t.release(q);
                m.seqs[q] = SeqHost();
                invariants(m);
            } else if (kind == 4) {
                const int32_t id = (int32_t)(rng() % npre);
                if (m.t.prefix_row(id)[0] < 0) {
                    const uint32_t np = 1 + rng() % pps;
                    const size_t free0 = m.t.free_pages.size();
                    const bool got = m.t.take_prefix(id, np);
                    CHECK(got == (np <= free0));
                } else {
                    m.t.release_prefix(id);
                }
                invariants(m);
            } else if (kind == 5) {
                // nested transactions: the inner one commits, the outer gives all back
                const PageTables before = m.t;
                const uint32_t q = rng() % nseq;
                {
                    PageTxn outer(m.t);
                    {
                        PageTxn inner(m.t);
                        (void)m.t.back_positions(q, m.seqs[q], m.seqs[q].pos, 1, m.window);
                        inner.commit();
                    }
                    CHECK(m.t.txn_depth == 1);
                }
                CHECK(m.t.pages == before.pages && m.t.free_pages == before.free_pages);
                invariants(m);
            } else {
                // backed and unbacked pages of a row add up to the row
                for (uint32_t q = 0; q < nseq; q++)
                    CHECK(m.t.backed(q) + m.t.need(q, 0, pps * m.P) == pps);
            }
        }
    }
}

// ------------------------------------------------------------- oracle

static std::vector<float> normal(std::mt19937 &rng, size_t n, float scale = 1.0f)
{
    std::normal_distribution<float> d(0.0f, scale);
    std::vector<float> x(n);
    for (auto &v : x)
        v = d(rng);
    return x;
}

static void check_oracle(std::mt19937 &rng)
{
    const uint32_t geoms[][6] = {{2, 8, 8, 64, 64, 96}, {1, 12, 2, 48, 64, 90}, {1, 14, 2, 36, 20, 70},
                                 {1, 5, 1, 64, 16, 40}, {1, 6, 3, 32, 32, 66}};
    for (const auto &g : geoms) {
        for (int dtype = 0; dtype < 2; dtype++) {
            ndo_session s;
            CHECK(ndo_session_init(&s, g[0], g[1], g[2], g[3], g[4], g[5], dtype) == 0);
            CHECK(ndo_session_front(&s, 3, 10000.0f) == 0);
            const uint32_t nh = g[1], nkv = g[2], qk = g[3], vd = g[4];
            std::vector<float> out(nh * vd);
            ndo_front_w fw;
            std::vector<float> tq = normal(rng, 3 * nh * qk, 0.3f), tk = normal(rng, 3 * nkv * qk, 0.3f),
                               tv = normal(rng, 3 * nkv * vd, 0.3f), nq = normal(rng, qk, 0.1f),
                               nk = normal(rng, qk, 0.1f);
            fw.tap_q = tq.data();
            fw.tap_k = tk.data();
            fw.tap_v = tv.data();
            fw.norm_q = nq.data();
            fw.norm_k = nk.data();
            ndo_prefix *saved = nullptr;
            for (int t = 0; t < 3 * (int)g[5]; t++) {
                if (t == 20) {
                    CHECK(ndo_snapshot(&s) == 0);
                    saved = ndo_prefix_save(&s);
                    CHECK(saved != nullptr);
                }
                if (t == 2 * (int)g[5])
                    CHECK(ndo_prefix_restore(&s, saved) == 0);
                if (t == 2 * (int)g[5] + 7)
                    ndo_rewind(&s);
                for (uint32_t li = 0; li < g[0]; li++) {
                    std::vector<float> q = normal(rng, nh * qk), k = normal(rng, nkv * qk),
                                       v = normal(rng, nkv * vd), gt = normal(rng, nh * vd);
                    ndo_front(&s, li, &fw, q.data(), k.data(), v.data());
                    ndo_attention(&s, li, q.data(), k.data(), v.data(), t % 3 ? gt.data() : nullptr, out.data());
                    for (float x : out)
                        CHECK(x == x);
                }
                ndo_step_end(&s);
            }
            ndo_prefix_free(saved);
            ndo_session_free(&s);
        }
    }
    // the threaded fp16 batch decode
    const uint32_t nseq = 37, nh = 8, d = 64;
    std::vector<uint32_t> len(nseq);
    std::vector<uint64_t> off(nseq);
    uint64_t tot = 0;
    for (uint32_t b = 0; b < nseq; b++) {
        len[b] = 1 + rng() % 300;
        off[b] = tot;
        tot += (uint64_t)len[b] * nh * d;
    }
    std::vector<uint16_t> kb(tot), vb(tot);
    for (uint64_t i = 0; i < tot; i++) {
        kb[i] = ndo_f32_to_f16(normal(rng, 1)[0]);
        vb[i] = ndo_f32_to_f16(normal(rng, 1)[0]);
    }
    std::vector<float> q = normal(rng, nseq * nh * d), kn = normal(rng, nseq * nh * d), vn = normal(rng, nseq * nh * d),
                       out1(nseq * nh * d), out8(nseq * nh * d);
    ndo_batch_f16 bt = {nseq, nh, nh, d, d, len.data(), off.data(), off.data(), kb.data(), vb.data(),
                        q.data(), kn.data(), vn.data(), nullptr, out1.data()};
    CHECK(ndo_decode_batch_f16(&bt, 1) == 0);
    bt.out = out8.data();
    CHECK(ndo_decode_batch_f16(&bt, 8) == 0);
    CHECK(out1 == out8);
}

int main()
{
    std::mt19937 rng(20261202);
    check_slots(rng);
    check_pages(rng);
    check_oracle(rng);
    if (failures) {
        fprintf(stderr, "%d checks failed\n", failures);
        return 1;
    }
    printf("sanitize_check: ok\n");
    return 0;
}
