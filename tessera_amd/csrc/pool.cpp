// The page pool for paged kept rows: tessera-kv's Pool (engine/ir/kv/src/
// pool.rs:71-450) as a C++ class behind a C ABI. The bookkeeping follows the
// reference call for call, since the page order it yields (and so every page
// table the attention kernels read) must be identical: lowest free page first,
// retained runs evicted by retirement number, a shared partial last page copied
// before a run writes into it, and every refusal checked before anything moves.
#include <algorithm>
#include <optional>
#include <set>
#include <vector>

#include "../../include/tessera_kv.h"

namespace {

struct Run {
    uint64_t tag;
    std::vector<uint32_t> pages;
    uint64_t rows, worst;
    std::optional<uint64_t> retired;  // retirement number; lowest is evicted first
};

struct Slot {
    uint32_t generation = 0;
    std::optional<Run> run;
};

}  // namespace

struct ts_kv_pool {
    uint64_t page;
    std::vector<uint32_t> live, kept;  // each page's live and retained holders
    std::set<uint32_t> free;
    std::vector<Slot> slots;
    uint64_t retirements = 0;
    uint64_t err_a = 0, err_b = 0;

    ts_kv_pool(uint32_t pages, uint32_t page_rows) : page(page_rows), live(pages, 0), kept(pages, 0) {
        for (uint32_t p = 0; p < pages; p++) free.insert(p);
    }

    uint64_t span(uint64_t rows) const { return (rows + page - 1) / page; }
    uint32_t holders(uint32_t p) const { return live[p] + kept[p]; }

    uint64_t spare() const {
        uint64_t reclaimable = 0;
        for (size_t i = 0; i < live.size(); i++) reclaimable += live[i] == 0 && kept[i] > 0;
        return free.size() + reclaimable;
    }

    // One if the next write lands in a shared page (pool.rs:402-407).
    uint64_t copies(uint64_t rows, const uint32_t *pages, size_t n) const {
        const bool partial = rows % page != 0;
        const bool shared = n > 0 && holders(pages[n - 1]) > 1;
        return partial && shared;
    }

    uint64_t need(const Run &r) const {
        return span(r.worst) - r.pages.size() + copies(r.rows, r.pages.data(), r.pages.size());
    }

    uint64_t promised() const {
        uint64_t s = 0;
        for (const Slot &sl : slots)
            if (sl.run && !sl.run->retired) s += need(*sl.run);
        return s;
    }

    int no_room(uint64_t n) {
        err_a = n;
        return TS_KV_NO_ROOM;
    }
    int past_worst(uint64_t rows, uint64_t worst) {
        err_a = rows;
        err_b = worst;
        return TS_KV_PAST_WORST;
    }
    int past_source(uint64_t rows) {
        err_a = rows;
        return TS_KV_PAST_SOURCE;
    }

    int fits(uint64_t n, uint64_t lost) {
        return promised() + n + lost <= spare() ? TS_KV_OK : no_room(n);
    }

    const Run *find(ts_kv_run id) const {
        if (id.at >= slots.size()) return nullptr;
        const Slot &s = slots[id.at];
        if (s.generation != id.generation || !s.run) return nullptr;
        return &*s.run;
    }
    Run &at(uint32_t i) { return *slots[i].run; }

    void unhold(uint32_t p, bool retained) {
        (retained ? kept : live)[p] -= 1;
        if (holders(p) == 0) free.insert(p);
    }

    void end(uint32_t i) {
        Slot &s = slots[i];
        s.generation += 1;
        Run r = std::move(*s.run);
        s.run.reset();
        for (uint32_t p : r.pages) unhold(p, r.retired.has_value());
    }

    // The lowest free page, after evicting retained runs if needed (pool.rs:359-372).
    uint32_t take() {
        while (free.empty()) {
            bool found = false;
            uint64_t best_ret = 0;
            uint32_t best_at = 0;
            for (uint32_t i = 0; i < slots.size(); i++) {
                const auto &r = slots[i].run;
                if (!r || !r->retired) continue;
                if (!found || *r->retired < best_ret || (*r->retired == best_ret && i < best_at)) {
                    found = true;
                    best_ret = *r->retired;
                    best_at = i;
                }
            }
            end(best_at);  // the room check promised a page
        }
        uint32_t p = *free.begin();
        free.erase(free.begin());
        live[p] = 1;
        return p;
    }

    ts_kv_run add(Run r) {
        uint32_t i = 0;
        while (i < slots.size() && slots[i].run) i++;
        if (i == slots.size()) slots.emplace_back();
        slots[i].run = std::move(r);
        return ts_kv_run{i, slots[i].generation};
    }

    bool consistent() const {
        std::vector<uint32_t> l(live.size(), 0), k(kept.size(), 0);
        for (const Slot &s : slots) {
            if (!s.run) continue;
            auto &c = s.run->retired ? k : l;
            for (uint32_t p : s.run->pages) c[p] += 1;
        }
        if (l != live || k != kept) return false;
        std::set<uint32_t> f;
        for (uint32_t p = 0; p < live.size(); p++)
            if (l[p] + k[p] == 0) f.insert(p);
        return f == free && promised() <= spare();
    }
};

extern "C" {

ts_kv_pool *tessera_kv_new(uint32_t pages, uint32_t page) {
    if (page == 0) return nullptr;
    return new ts_kv_pool(pages, page);
}

void tessera_kv_free(ts_kv_pool *p) { delete p; }

int tessera_kv_reserve(ts_kv_pool *p, uint64_t tag, uint64_t rows, uint64_t worst, ts_kv_run *out) {
    if (rows > worst) return p->past_worst(rows, worst);
    if (int e = p->fits(p->span(worst), 0)) return e;
    Run r{tag, {}, rows, worst, std::nullopt};
    for (uint64_t i = 0; i < p->span(rows); i++) r.pages.push_back(p->take());
    *out = p->add(std::move(r));
    return TS_KV_OK;
}

int tessera_kv_fork(ts_kv_pool *p, ts_kv_run source, uint64_t rows, uint64_t worst, ts_kv_run *out) {
    const Run *src = p->find(source);
    if (!src) return TS_KV_UNKNOWN;
    if (rows > src->rows) return p->past_source(src->rows);
    if (rows > worst) return p->past_worst(rows, worst);
    const size_t n = p->span(rows);
    uint64_t lost = 0;
    for (size_t i = 0; i < n; i++) lost += p->live[src->pages[i]] == 0;
    // A shared partial page costs each live holder one copy.
    const bool mine = rows % p->page != 0;
    const bool theirs = !src->retired && src->rows % p->page != 0 && n == src->pages.size() && n > 0 &&
                        p->holders(src->pages[n - 1]) == 1;
    const uint64_t need = p->span(worst) - n + mine + theirs;
    if (int e = p->fits(need, lost)) return e;
    Run r{src->tag, std::vector<uint32_t>(src->pages.begin(), src->pages.begin() + n), rows, worst, std::nullopt};
    for (uint32_t pg : r.pages) p->live[pg] += 1;
    *out = p->add(std::move(r));
    return TS_KV_OK;
}

static int live_at(const ts_kv_pool *p, ts_kv_run id) {
    const Run *r = p->find(id);
    if (!r) return TS_KV_UNKNOWN;
    if (r->retired) return TS_KV_RETAINED;
    return TS_KV_OK;
}

int tessera_kv_grow(ts_kv_pool *p, ts_kv_run run, uint64_t rows, ts_kv_copy *copy, uint32_t *n_copies) {
    if (n_copies) *n_copies = 0;
    if (int e = live_at(p, run)) return e;
    Run &r = p->at(run.at);
    if (rows > r.worst) return p->past_worst(rows, r.worst);
    if (rows <= r.rows) return TS_KV_OK;
    const uint64_t written = r.rows % p->page;
    if (!r.pages.empty() && written > 0 && p->holders(r.pages.back()) > 1) {
        const uint32_t from = r.pages.back();
        const uint32_t to = p->take();
        p->live[from] -= 1;
        p->at(run.at).pages.back() = to;
        if (copy) *copy = ts_kv_copy{from, to, written};
        if (n_copies) *n_copies = 1;
    }
    while (p->at(run.at).pages.size() < p->span(rows)) {
        const uint32_t pg = p->take();
        p->at(run.at).pages.push_back(pg);
    }
    p->at(run.at).rows = rows;
    return TS_KV_OK;
}

int tessera_kv_truncate(ts_kv_pool *p, ts_kv_run run, uint64_t rows) {
    if (int e = live_at(p, run)) return e;
    Run &r = p->at(run.at);
    if (rows >= r.rows) return TS_KV_OK;
    const size_t keep = p->span(rows);
    // The run may grow back. Shared pages stay held.
    const uint64_t regrow = r.pages.size() - keep + p->copies(rows, r.pages.data(), keep);
    uint64_t freed = 0;
    for (size_t i = keep; i < r.pages.size(); i++) freed += p->live[r.pages[i]] == 1;
    const uint64_t owed = freed + p->copies(r.rows, r.pages.data(), r.pages.size());
    if (int e = p->fits(regrow > owed ? regrow - owed : 0, 0)) return e;
    std::vector<uint32_t> dropped(r.pages.begin() + keep, r.pages.end());
    r.pages.resize(keep);
    r.rows = rows;
    for (uint32_t pg : dropped) p->unhold(pg, false);
    return TS_KV_OK;
}

int tessera_kv_retain(ts_kv_pool *p, ts_kv_run run) {
    if (int e = live_at(p, run)) return e;
    p->retirements += 1;
    Run &r = p->at(run.at);
    r.retired = p->retirements;
    for (uint32_t pg : r.pages) {
        p->live[pg] -= 1;
        p->kept[pg] += 1;
    }
    return TS_KV_OK;
}

int tessera_kv_adopt(ts_kv_pool *p, ts_kv_run run, uint64_t rows, uint64_t worst, ts_kv_run *out) {
    const Run *r = p->find(run);
    if (!r) return TS_KV_UNKNOWN;
    if (!r->retired) return TS_KV_LIVE;
    if (rows > r->rows) return p->past_source(r->rows);
    if (rows > worst) return p->past_worst(rows, worst);
    const size_t keep = p->span(rows);
    uint64_t lost = 0;
    for (size_t i = 0; i < keep; i++) lost += p->live[r->pages[i]] == 0;
    const uint64_t need = p->span(worst) - keep + p->copies(rows, r->pages.data(), keep);
    if (int e = p->fits(need, lost)) return e;
    Run &w = p->at(run.at);
    std::vector<uint32_t> dropped(w.pages.begin() + keep, w.pages.end());
    w.pages.resize(keep);
    for (uint32_t pg : dropped) p->unhold(pg, true);
    Run &x = p->at(run.at);
    x.rows = rows;
    x.worst = worst;
    x.retired.reset();
    for (uint32_t pg : x.pages) {
        p->kept[pg] -= 1;
        p->live[pg] += 1;
    }
    // The retained id is now stale.
    p->slots[run.at].generation += 1;
    *out = ts_kv_run{run.at, p->slots[run.at].generation};
    return TS_KV_OK;
}

int tessera_kv_release(ts_kv_pool *p, ts_kv_run run) {
    if (!p->find(run)) return TS_KV_UNKNOWN;
    p->end(run.at);
    return TS_KV_OK;
}

int tessera_kv_pages(const ts_kv_pool *p, ts_kv_run run, const uint32_t **pages, uint32_t *count) {
    const Run *r = p->find(run);
    if (!r) return TS_KV_UNKNOWN;
    *pages = r->pages.data();
    *count = (uint32_t)r->pages.size();
    return TS_KV_OK;
}

int tessera_kv_rows(const ts_kv_pool *p, ts_kv_run run, uint64_t *rows) {
    const Run *r = p->find(run);
    if (!r) return TS_KV_UNKNOWN;
    *rows = r->rows;
    return TS_KV_OK;
}

int tessera_kv_tag(const ts_kv_pool *p, ts_kv_run run, uint64_t *tag) {
    const Run *r = p->find(run);
    if (!r) return TS_KV_UNKNOWN;
    *tag = r->tag;
    return TS_KV_OK;
}

uint64_t tessera_kv_spare(const ts_kv_pool *p) { return p->spare(); }
uint64_t tessera_kv_promised(const ts_kv_pool *p) { return p->promised(); }

void tessera_kv_get_stats(const ts_kv_pool *p, ts_kv_stats *s) {
    uint64_t held = 0;
    for (uint32_t l : p->live) held += l > 0;
    *s = ts_kv_stats{p->live.size() * p->page, held * p->page, 0, 0, 0};
    for (const Slot &sl : p->slots) {
        if (!sl.run) continue;
        if (sl.run->retired) {
            s->kept_runs += 1;
            continue;
        }
        s->live_runs += 1;
        s->worst += p->span(sl.run->worst) * p->page;
    }
}

// FNV-1a over each page's holders, then each slot's generation and run (pool.rs:304-322).
uint64_t tessera_kv_digest(const ts_kv_pool *p) {
    uint64_t hash = 0xcbf29ce484222325ull;
    auto eat = [&](uint64_t x) {
        for (int b = 0; b < 8; b++) hash = (hash ^ ((x >> (8 * b)) & 0xff)) * 0x100000001b3ull;
    };
    for (size_t i = 0; i < p->live.size(); i++) eat(((uint64_t)p->live[i] << 32) | p->kept[i]);
    for (const Slot &s : p->slots) {
        eat(s.generation);
        if (!s.run) continue;
        eat(s.run->tag);
        eat(s.run->rows);
        eat(s.run->worst);
        eat(s.run->retired.value_or(0));
        for (uint32_t pg : s.run->pages) eat(pg);
    }
    return hash;
}

int tessera_kv_consistent(const ts_kv_pool *p) { return p->consistent() ? 1 : 0; }
uint64_t tessera_kv_error_value(const ts_kv_pool *p) { return p->err_a; }
uint64_t tessera_kv_error_value2(const ts_kv_pool *p) { return p->err_b; }

}  // extern "C"
