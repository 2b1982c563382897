// CPU oracle of the n-gram hint path: TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load this library, as the checker (or as the CPU baseline that is timed beside the GPU); nothing in
// the product calls it.
//
// A restatement, in plain C++ (std::thread, std::sort), of the reference's CPU algorithms for this path:
//   * oracle_query_counts: exact_match/src/kgram.rs count_with/scan/Contexts (:308-399, :406-489, :505-565), the
//     query-filtered counting: the distinct valid query k-contexts are indexed, the corpus is streamed, every hit is
//     verified token by token and (context id, next token) collected, then sorted per context; plus
//     old_records.val_count_features (src/retrieval_blog_post/old_records.py:236-294) for tot/dist/cnt with the
//     top-`cnt_top` rule, and the context's `ntop` most frequent next tokens (count descending, then token
//     ascending: kgram.rs:357-368).
//   * oracle_table_counts: exact_match/src/count_table.rs build_level/runs/query_counts (:491-631, :726-777,
//     :291-331), the corpus-wide table: every context of the corpus counted (here with exact 128-bit packed keys,
//     k <= 8), then queried.
//   * oracle_longest_match: the largest k <= cap whose query k-context is valid and occurred (kgram.rs kgram_stats'
//     "matched" at each k, :252-277, with the monotonicity of kgram.rs:12-15), and that context's most frequent next
//     token and its count.
//   * oracle_online: exact_match/src/online.rs's step rule (:1-17) and walks (Walker :574-672, Counter :674-705): per
//     level, occurrences (time alpha = 1 + max tau over their k + 1 tokens) and queries (time tau_in) sorted by
//     (context, time, occurrences first, position) and walked; hint rows (deepest level first) and count rows.
// Definitions (kgram.rs:7-9): a query position i's k-context is x[i-k+1..=i], valid iff avail[i] >= k; a corpus
// occurrence is any k tokens within one shard followed by a token of the same shard; tot = occurrences (u32; the
// caller checks >= 2^32), dist = distinct next tokens (saturated at 65535), cnt = the target's count if its rank
// (count descending, token ascending) is below cnt_top, else 0; all 0 where the context is invalid or never occurred.
#include <algorithm>
#include <parallel/algorithm>
#include <cstdio>
#include <cstdlib>
#include <chrono>
#include <cmath>
#include <functional>
#include <atomic>
#include <cstdint>
#include <cstring>
#include <thread>
#include <unordered_map>
#include <vector>

typedef uint64_t u64;
typedef uint32_t u32;
typedef uint16_t u16;
typedef int64_t i64;
typedef int32_t i32;
typedef unsigned __int128 u128;

static u64 mix(u64 h) {
    h ^= h >> 30;
    h *= 0xbf58476d1ce4e5b9ull;
    h ^= h >> 27;
    h *= 0x94d049bb133111ebull;
    return h ^ (h >> 31);
}

static u64 hash_tokens(const u16* t, int k) {
    u64 h = 0;
    for (int j = 0; j < k; ++j) h = h * 0x9e3779b185ebca87ull + (u64)t[j] + 1;
    return mix(h) | 1;
}

template <class F>
static void parallel_for(i64 n, int threads, F f) {
    if (threads <= 1 || n < 2) {
        f(0, n, 0);
        return;
    }
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t) {
        i64 a = n * t / threads, b = n * (t + 1) / threads;
        ts.emplace_back([=, &f] { f(a, b, t); });
    }
    for (auto& th : ts) th.join();
}

// The distinct valid query k-contexts (kgram.rs Contexts::new): an open-addressing table from a 64-bit hash to the
// ids of the contexts with that hash (a hash shared by different contexts keeps them apart: every lookup compares
// tokens, so the index is exact whatever the hash).
struct Contexts {
    int k;
    std::vector<u32> key_of;  // per position: id or UINT32_MAX
    std::vector<u32> reps;    // per id: a position
    std::vector<u64> slot_hash;
    std::vector<u32> slot_id;
    u64 mask;
    const u16* x;

    void build(const u16* x_, const i32* avail, i64 n, int k_) {
        x = x_;
        k = k_;
        key_of.assign(n, UINT32_MAX);
        reps.clear();
        u64 cap = 1024;
        while (cap < 2 * (u64)n + 2) cap <<= 1;
        slot_hash.assign(cap, 0);
        slot_id.assign(cap, 0);
        mask = cap - 1;
        for (i64 i = 0; i < n; ++i) {
            if (avail[i] < k) continue;
            const u16* c = x + i + 1 - k;
            u64 h = hash_tokens(c, k);
            u64 s = h & mask;
            while (true) {
                if (slot_hash[s] == 0) {
                    slot_hash[s] = h;
                    slot_id[s] = (u32)reps.size();
                    key_of[i] = (u32)reps.size();
                    reps.push_back((u32)i);
                    break;
                }
                if (slot_hash[s] == h) {
                    u32 id = slot_id[s];
                    const u16* r = x + reps[id] + 1 - k;
                    if (memcmp(r, c, 2 * (size_t)k) == 0) {
                        key_of[i] = id;
                        break;
                    }
                }
                s = (s + 1) & mask;
            }
        }
    }

    // The id of the context c (k tokens), or UINT32_MAX.
    u32 find(const u16* c) const {
        u64 h = hash_tokens(c, k);
        u64 s = h & mask;
        while (true) {
            if (slot_hash[s] == 0) return UINT32_MAX;
            if (slot_hash[s] == h) {
                u32 id = slot_id[s];
                if (memcmp(x + reps[id] + 1 - k, c, 2 * (size_t)k) == 0) return id;
            }
            s = (s + 1) & mask;
        }
    }
};

// One context's counted pairs: the next tokens and counts, ranked (count descending, token ascending).
struct Ranked {
    u64 total = 0;
    std::vector<std::pair<u32, u16>> ranked;  // (count, token)
};

static void rank_pairs(std::vector<std::pair<u32, u16>>& v) {
    std::sort(v.begin(), v.end(), [](const std::pair<u32, u16>& a, const std::pair<u32, u16>& b) {
        if (a.first != b.first) return a.first > b.first;
        return a.second < b.second;
    });
}

// Per-position outputs from per-context ranked lists.
static void position_outputs(const std::vector<u32>& ctx, const std::vector<Ranked>& per, const u16* tgt, i64 n,
                             int cnt_top, int ntop, u32* tot, u16* dist, u32* cnt, u16* top_tok, u32* top_cnt) {
    for (i64 i = 0; i < n; ++i) {
        if (tot) tot[i] = 0;
        if (dist) dist[i] = 0;
        if (cnt) cnt[i] = 0;
        for (int r = 0; r < ntop; ++r) {
            top_tok[i * ntop + r] = 0;
            top_cnt[i * ntop + r] = 0;
        }
        u32 id = ctx[i];
        if (id == UINT32_MAX) continue;
        const Ranked& c = per[id];
        if (c.total == 0) continue;
        if (tot) tot[i] = (u32)c.total;
        if (dist) dist[i] = (u16)std::min<size_t>(c.ranked.size(), 65535);
        if (cnt) {
            size_t lim = std::min<size_t>(c.ranked.size(), (size_t)cnt_top);
            for (size_t r = 0; r < lim; ++r)
                if (c.ranked[r].second == tgt[i]) {
                    cnt[i] = c.ranked[r].first;
                    break;
                }
        }
        for (int r = 0; r < ntop && r < (int)c.ranked.size(); ++r) {
            top_tok[i * ntop + r] = c.ranked[r].second;
            top_cnt[i * ntop + r] = c.ranked[r].first;
        }
    }
}

// Group (id << 16 | next) entries into per-context ranked lists. Each thread's entries are sorted and run-length
// encoded in parallel (Zipf-skewed pairs repeat a lot); then ranges of context ids are merged in parallel, each from
// its slice of every thread's runs.
static void group_entries(std::vector<std::vector<u64>>& acc, std::vector<Ranked>& per, int threads) {
    threads = std::max(1, threads);
    std::vector<std::vector<std::pair<u64, u64>>> runs(acc.size());
    parallel_for((i64)acc.size(), std::max(1, std::min<int>(threads, (int)acc.size())), [&](i64 a, i64 b, int) {
        for (i64 t = a; t < b; ++t) {
            std::vector<u64>& v = acc[t];
            std::sort(v.begin(), v.end());
            for (size_t i = 0; i < v.size();) {
                size_t j = i;
                while (j < v.size() && v[j] == v[i]) ++j;
                runs[t].push_back({v[i], (u64)(j - i)});
                i = j;
            }
            std::vector<u64>().swap(v);
        }
    });
    const i64 nids = (i64)per.size();
    const i64 R = std::min<i64>(std::max<i64>(nids, 1), 16 * (i64)threads);  // id ranges, taken dynamically
    std::atomic<i64> next_range(0);
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t)
        ts.emplace_back([&] {
            for (i64 r; (r = next_range++) < R;) {
                const u64 lo = (u64)(nids * r / R) << 16, hi = (u64)(nids * (r + 1) / R) << 16;
                std::vector<std::pair<u64, u64>> all;
                for (auto& rv : runs) {
                    auto a = std::lower_bound(rv.begin(), rv.end(), std::make_pair(lo, (u64)0));
                    auto b = std::lower_bound(rv.begin(), rv.end(), std::make_pair(hi, (u64)0));
                    all.insert(all.end(), a, b);
                }
                std::sort(all.begin(), all.end());
                for (size_t i = 0; i < all.size();) {
                    const u64 id = all[i].first >> 16;
                    Ranked& c = per[id];
                    size_t j = i;
                    while (j < all.size() && (all[j].first >> 16) == id) {
                        const u64 v = all[j].first;
                        u64 n = 0;
                        while (j < all.size() && all[j].first == v) n += all[j++].second;
                        c.ranked.push_back({(u32)n, (u16)(v & 0xFFFF)});
                        c.total += n;
                    }
                    rank_pairs(c.ranked);
                    i = j;
                }
            }
        });
    for (auto& th : ts) th.join();
}

extern "C" {

// Query-filtered counts of level k (see the file comment). `tok` holds the shards concatenated, shard s being
// [bounds[s], bounds[s + 1]); `x`, `tgt`, `avail` are the query positions' inputs, targets and segment lengths.
// Outputs per position (any may be null except top arrays when ntop > 0). `hits`, if not null, receives per corpus
// position whose k-context matched a query context (the next token's index, as kgram.rs's bitmap) a 1 byte.
// Returns the number of matched corpus occurrences, or -1 on bad arguments.
i64 oracle_query_counts(const u16* tok, const i64* bounds, int nshards, const u16* x, const u16* tgt,
                        const i32* avail, i64 n, int k, int cnt_top, int ntop, u32* tot, u16* dist, u32* cnt,
                        u16* top_tok, u32* top_cnt, uint8_t* hits, const uint8_t* gate, int threads) {
    if (k < 1 || n < 0 || nshards < 1 || ntop < 0) return -1;
    Contexts ctx;
    ctx.build(x, avail, n, k);
    std::vector<std::pair<i64, i64>> pieces;
    const i64 PIECE = 1 << 20;
    for (int s = 0; s < nshards; ++s)
        for (i64 p = bounds[s] + k; p < bounds[s + 1]; p += PIECE) pieces.push_back({p, std::min(bounds[s + 1], p + PIECE)});
    if (threads < 1) threads = 1;
    std::vector<std::vector<u64>> acc(threads);
    std::atomic<size_t> next_piece(0);
    std::vector<std::thread> ts;
    for (int t = 0; t < threads; ++t)
        ts.emplace_back([&, t] {
            while (true) {
                size_t q = next_piece++;
                if (q >= pieces.size()) break;
                for (i64 p = pieces[q].first; p < pieces[q].second; ++p) {
                    if (gate && !gate[p]) continue;  // its (k-1)-suffix never matched: neither can its k-context
                    u32 id = ctx.find(tok + p - k);
                    if (id == UINT32_MAX) continue;
                    if (hits) hits[p] = 1;
                    acc[t].push_back(((u64)id << 16) | tok[p]);
                }
            }
        });
    for (auto& th : ts) th.join();
    size_t total = 0;
    for (auto& a : acc) total += a.size();
    std::vector<Ranked> per(ctx.reps.size());
    group_entries(acc, per, threads);
    position_outputs(ctx.key_of, per, tgt, n, cnt_top, ntop, tot, dist, cnt, top_tok, top_cnt);
    if (getenv("ORACLE_TRACE")) fprintf(stderr, "oracle query_counts k=%d: %zu events\n", k, total);
    return (i64)total;
}

// Corpus-wide counts of level k <= 8 (count_table.rs): every context of every shard is counted, keyed by its tokens
// packed 16 bits each (exact), then each query position looks its context up. Same outputs as oracle_query_counts.
// Also returns (through the pointers, if not null) the level's distinct contexts and distinct (context, next) pairs.
i64 oracle_table_counts(const u16* tok, const i64* bounds, int nshards, const u16* x, const u16* tgt,
                        const i32* avail, i64 n, int k, int cnt_top, int ntop, u32* tot, u16* dist, u32* cnt,
                        u16* top_tok, u32* top_cnt, i64* n_contexts, i64* n_pairs, int threads) {
    if (k < 1 || k > 8 || n < 0 || nshards < 1) return -1;  // a context packs into 128 bits up to k = 8
    struct E {
        u128 ctx;
        u16 next;
        bool operator<(const E& o) const { return ctx != o.ctx ? ctx < o.ctx : next < o.next; }
    };
    auto pack = [k](const u16* c) {
        u128 v = 0;
        for (int j = 0; j < k; ++j) v = (v << 16) | c[j];
        return v;
    };
    std::vector<E> all;
    i64 events = 0;
    for (int s = 0; s < nshards; ++s) events += std::max<i64>(0, bounds[s + 1] - bounds[s] - k);
    all.resize(events);
    i64 at = 0;
    for (int s = 0; s < nshards; ++s)
        for (i64 p = bounds[s] + k; p < bounds[s + 1]; ++p) all[at++] = E{pack(tok + p - k), tok[p]};
    if (threads > 1) {
        // sort in parallel pieces, then merge
        std::vector<i64> cut;
        for (int t = 0; t <= threads; ++t) cut.push_back(events * t / threads);
        parallel_for(threads, threads, [&](i64 a, i64 b, int) {
            for (i64 t = a; t < b; ++t) std::sort(all.begin() + cut[t], all.begin() + cut[t + 1]);
        });
        for (int w = 1; w < threads; w *= 2)
            for (int t = 0; t + w < threads; t += 2 * w)
                std::inplace_merge(all.begin() + cut[t], all.begin() + cut[t + w],
                                   all.begin() + cut[std::min(threads, t + 2 * w)]);
    } else {
        std::sort(all.begin(), all.end());
    }
    // contexts: sorted packed keys with their ranked pairs
    std::vector<u128> keys;
    std::vector<Ranked> per;
    i64 pairs = 0;
    size_t i = 0;
    while (i < all.size()) {
        u128 c = all[i].ctx;
        Ranked r;
        size_t j = i;
        while (j < all.size() && all[j].ctx == c) {
            u16 t = all[j].next;
            size_t a = j;
            while (j < all.size() && all[j].ctx == c && all[j].next == t) ++j;
            r.ranked.push_back({(u32)(j - a), t});
        }
        r.total = j - i;
        pairs += r.ranked.size();
        rank_pairs(r.ranked);
        keys.push_back(c);
        per.push_back(std::move(r));
        i = j;
    }
    if (n_contexts) *n_contexts = (i64)keys.size();
    if (n_pairs) *n_pairs = pairs;
    std::vector<u32> ctx(n, UINT32_MAX);
    for (i64 q = 0; q < n; ++q) {
        if (avail[q] < k) continue;
        u128 c = pack(x + q + 1 - k);
        auto it = std::lower_bound(keys.begin(), keys.end(), c);
        if (it != keys.end() && *it == c) ctx[q] = (u32)(it - keys.begin());
    }
    position_outputs(ctx, per, tgt, n, cnt_top, ntop, tot, dist, cnt, top_tok, top_cnt);
    return events;
}

// Longest match: per query position, the largest k <= cap whose k-context is valid and occurred in the corpus (0 if
// none), that context's most frequent next token (count descending, token ascending) and its count. Two phases, both
// from the definitions: existence level by level (a corpus position can match at k only if it matched at k - 1,
// kgram.rs:12-15, so each level examines only the previous level's hit positions, kept as one bitmap per level), then,
// per level, the (context, next) pairs of only the contexts some position ends at, counted over that level's hits.
static inline bool bit_at(const std::vector<u64>& b, i64 p) { return (b[p >> 6] >> (p & 63)) & 1; }

int oracle_longest_match(const u16* tok, const i64* bounds, int nshards, const u16* x, const i32* avail, i64 n,
                         int cap, u32* length, u16* next, u32* count, int threads) {
    if (cap < 1 || n < 0 || nshards < 1) return -1;
    if (threads < 1) threads = 1;
    const i64 T = bounds[nshards];
    const i64 W = (T + 63) / 64;
    std::vector<i32> av(avail, avail + n);
    std::vector<u32> final_id(n, UINT32_MAX);
    std::vector<std::vector<u64>> hit(cap + 1);  // hit[k]: corpus positions whose k-context matched (bitmap)
    std::vector<Contexts> ctx(cap + 1);
    for (i64 i = 0; i < n; ++i) length[i] = 0, next[i] = 0, count[i] = 0;
    std::vector<std::pair<i64, i64>> pieces;
    for (int s = 0; s < nshards; ++s)
        for (i64 p = bounds[s]; p < bounds[s + 1]; p += 1 << 20) pieces.push_back({p, std::min(bounds[s + 1], p + (1 << 20))});
    const bool trace = getenv("ORACLE_TRACE") != nullptr;
    auto for_pieces = [&](auto body) {
        std::atomic<size_t> nxt(0);
        std::vector<std::thread> ts;
        auto last = std::chrono::steady_clock::now();
        for (int t = 0; t < threads; ++t)
            ts.emplace_back([&, t] {
                for (size_t q; (q = nxt++) < pieces.size();) {
                    body(pieces[q].first, pieces[q].second, t);
                    if (trace && t == 0 && std::chrono::steady_clock::now() - last > std::chrono::seconds(20)) {
                        fprintf(stderr, "  piece %zu of %zu\n", q, pieces.size());
                        last = std::chrono::steady_clock::now();
                    }
                }
            });
        for (auto& th : ts) th.join();
    };
    // shard of each corpus position, to keep a context inside its shard: position p's k-context is p-k..p-1
    auto shard_start = [&](i64 p) {
        return *(std::upper_bound(bounds, bounds + nshards + 1, p) - 1);
    };
    int top_level = 0;
    for (int k = 1; k <= cap; ++k) {
        bool any = false;
        for (i64 i = 0; i < n; ++i) any |= av[i] >= k;
        if (!any) break;
        ctx[k].build(x, av.data(), n, k);
        std::vector<uint8_t> found(ctx[k].reps.size(), 0);
        hit[k].assign(W, 0);
        for_pieces([&](i64 a, i64 b, int) {
            const i64 s0 = shard_start(a);
            for (i64 p = std::max(a, s0 + k); p < b; ++p) {
                if (k > 1 && !bit_at(hit[k - 1], p)) continue;
                const u32 id = ctx[k].find(tok + p - k);
                if (id == UINT32_MAX) continue;
                found[id] = 1;
                __atomic_fetch_or(&hit[k][p >> 6], 1ull << (p & 63), __ATOMIC_RELAXED);
            }
        });
        for (i64 i = 0; i < n; ++i) {
            if (av[i] < k) continue;
            const u32 id = ctx[k].key_of[i];
            if (id != UINT32_MAX && found[id]) {
                length[i] = (u32)k;
                final_id[i] = id;
            } else {
                av[i] = 0;  // no longer matching: out of the deeper levels
            }
        }
        top_level = k;
        if (getenv("ORACLE_TRACE")) fprintf(stderr, "exist k=%d %.3f\n", k, std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count());
    }
    // counting: per level, the contexts some position ends at, over that level's hit positions
    for (int k = 1; k <= top_level; ++k) {
        std::vector<uint8_t> wanted(ctx[k].reps.size(), 0);
        bool any = false;
        for (i64 i = 0; i < n; ++i)
            if (length[i] == (u32)k) wanted[final_id[i]] = 1, any = true;
        if (!any) continue;
        std::vector<std::vector<u64>> acc(threads);
        for_pieces([&](i64 a, i64 b, int t) {
            const i64 s0 = shard_start(a);
            for (i64 p = std::max(a, s0 + k); p < b; ++p) {
                if (!bit_at(hit[k], p)) continue;
                const u32 id = ctx[k].find(tok + p - k);
                if (id != UINT32_MAX && wanted[id]) acc[t].push_back(((u64)id << 16) | tok[p]);
            }
        });
        std::vector<Ranked> per(ctx[k].reps.size());
        group_entries(acc, per, threads);
        for (i64 i = 0; i < n; ++i)
            if (length[i] == (u32)k && !per[final_id[i]].ranked.empty()) {
                next[i] = per[final_id[i]].ranked[0].second;
                count[i] = per[final_id[i]].ranked[0].first;
            }
        if (getenv("ORACLE_TRACE")) fprintf(stderr, "count k=%d %.3f\n", k, std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count());
    }
    return 0;
}

// Online rows under the step rule (online.rs): tokens in parts [bounds[j], bounds[j + 1]); tau / tau_in per position
// (0xFFFFFFFF: never). Queries: positions with tau_in in [step_lo, step_hi) whose k-context lies in their segment
// (segments start at each part start and at every BOS). Hint rows for `levels` (deepest first; bucket = index in
// `buckets`; `entries` next tokens) into cell / next / weights; count rows for `count_levels` into tot / dist / cnt
// [n, nc] (cnt: the count of the query's own next token, if within its part). Outputs are written only where a row
// exists (callers zero them). Returns the queries hinted, or -1 on bad arguments.
i64 oracle_online(const u16* tok, i64 n, const i64* bounds, int nparts, const u32* tau, const u32* tau_in,
                  const int* levels, int nl, const int* buckets, int nb, int entries, const int* count_levels, int nc,
                  u32 step_lo, u32 step_hi, int16_t* cell, u16* next, u16* weights, u32* tot, u16* dist, u32* cnt,
                  int threads) {
    const u32 NONE = 0xFFFFFFFFu;
    if (entries < 1 || nparts < 1 || step_lo > step_hi) return -1;
    for (int i = 0; i < nl; ++i)
        if (levels[i] < 1 || levels[i] > 8) return -1;  // contexts pack into 128 bits up to 8 tokens
    for (int i = 0; i < nc; ++i)
        if (count_levels[i] < 1 || count_levels[i] > 8) return -1;
    std::vector<u32> seg(n), part_end(n), part_lo(n);
    for (int j = 0; j < nparts; ++j) {
        i64 s0 = bounds[j];
        for (i64 g = bounds[j]; g < bounds[j + 1]; ++g) {
            if (tok[g] == 50256) s0 = g;
            seg[g] = (u32)s0;
            part_end[g] = (u32)bounds[j + 1];
            part_lo[g] = (u32)bounds[j];
        }
    }
    if (n >= (i64)1 << 32) return -1;
    struct El {
        u128 key;  // the k tokens g-k+1..g packed 16 bits each, first token highest: exact, ordered like the tokens
        u32 tk;    // time << 1 | kind (0 occurrence, 1 query): ordered by time, then occurrences first
        u32 g;
    };
    auto pack = [&](i64 g, int k) {
        u128 v = 0;
        for (i64 q = g - k + 1; q <= g; ++q) v = (v << 16) | tok[q];
        return v;
    };
    std::vector<uint8_t> filled(n, 0);
    std::atomic<i64> hinted(0);
    const int T = std::max(1, threads);
    auto now = [] { return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count(); };
    // levels needed: hint levels (descending: a position's row comes from its deepest level) and count levels
    std::vector<int> all;
    for (int i = 0; i < nl; ++i) all.push_back(levels[i]);
    for (int i = 0; i < nc; ++i) all.push_back(count_levels[i]);
    std::sort(all.begin(), all.end(), std::greater<int>());
    all.erase(std::unique(all.begin(), all.end()), all.end());
    for (int k : all) {
        const double t0 = now();
        int li = -1, ci = -1;
        for (int i = 0; i < nl; ++i)
            if (levels[i] == k)
                for (int b = 0; b < nb; ++b)
                    if (buckets[b] == k) li = b;
        for (int i = 0; i < nc; ++i)
            if (count_levels[i] == k) ci = i;
        // the level's elements: occurrences (available at alpha = 1 + max tau over their k + 1 tokens) and queries,
        // built in parallel ranges of positions
        std::vector<std::vector<El>> part(T);
        parallel_for(n, T, [&](i64 lo, i64 hi, int t) {
            for (i64 g = lo; g < hi; ++g) {
                // occurrence ending at g: tokens g-k+1..g and next g+1 within g's part
                if (g - k + 1 >= (i64)part_lo[g] && g + 1 < (i64)part_end[g]) {
                    u32 a = 0;
                    bool ok = true;
                    for (i64 q = g - k + 1; q <= g + 1; ++q) {
                        if (tau[q] == NONE) ok = false;
                        else a = std::max(a, tau[q]);
                    }
                    if (ok && a + 1 < step_hi) part[t].push_back({pack(g, k), (a + 1) << 1, (u32)g});
                }
                if (tau_in[g] != NONE && tau_in[g] >= step_lo && tau_in[g] < step_hi && g - (i64)seg[g] + 1 >= k)
                    part[t].push_back({pack(g, k), (tau_in[g] << 1) | 1u, (u32)g});
            }
        });
        std::vector<El> els;
        for (auto& v : part) els.insert(els.end(), v.begin(), v.end()), std::vector<El>().swap(v);
        const double tb = now();
        __gnu_parallel::sort(els.begin(), els.end(), [](const El& x, const El& y) {
            if (x.key != y.key) return x.key < y.key;
            if (x.tk != y.tk) return x.tk < y.tk;
            return x.g < y.g;
        });
        const double t1 = now();
        // the walk: each context's elements in (time, occurrences first, position) order; chunks of whole contexts
        // walked in parallel (a query position is in one context per level)
        std::vector<size_t> cut(T + 1, els.size());
        cut[0] = 0;
        for (int t = 1; t < T; ++t) {
            size_t c = els.size() * t / T;
            while (c > 0 && c < els.size() && els[c].key == els[c - 1].key) ++c;
            cut[t] = std::max(c, cut[t - 1]);
        }
        parallel_for(T, T, [&](i64 t0c, i64 t1c, int) {
            std::vector<u32> counts(1 << 16, 0);
            for (i64 chunk = t0c; chunk < t1c; ++chunk) {
                size_t i = cut[chunk];
                const size_t end = cut[chunk + 1];
                while (i < end) {
                    size_t j = i;
                    while (j < els.size() && els[j].key == els[i].key) ++j;
                    std::vector<u16> touched;
                    std::vector<std::pair<u32, u16>> top;  // (count, token), best first
                    u32 total = 0;
                    auto better = [](std::pair<u32, u16> a, std::pair<u32, u16> b) {
                        return a.first > b.first || (a.first == b.first && a.second < b.second);
                    };
                    for (size_t e = i; e < j; ++e) {
                        const El& el = els[e];
                        if ((el.tk & 1) == 0) {
                            u16 t = tok[el.g + 1];
                            if (counts[t] == 0) touched.push_back(t);
                            u32 c = ++counts[t];
                            ++total;
                            int pos = -1;
                            for (size_t q = 0; q < top.size(); ++q)
                                if (top[q].second == t) pos = (int)q;
                            if (pos < 0) {
                                if ((int)top.size() < entries) {
                                    top.push_back({c, t});
                                    pos = (int)top.size() - 1;
                                } else if (better({c, t}, top[entries - 1])) {
                                    pos = entries - 1;
                                }
                            }
                            if (pos >= 0) {
                                top[pos] = {c, t};
                                while (pos > 0 && better(top[pos], top[pos - 1])) {
                                    std::swap(top[pos], top[pos - 1]);
                                    --pos;
                                }
                            }
                        } else if (total > 0) {
                            const i64 g = (i64)el.g;
                            if (ci >= 0) {
                                tot[g * nc + ci] = total;
                                dist[g * nc + ci] = (u16)std::min<size_t>(touched.size(), 65535);
                                cnt[g * nc + ci] = g + 1 < (i64)part_end[g] ? counts[tok[g + 1]] : 0;
                            }
                            if (li >= 0 && !filled[g]) {
                                static const u32 CE[6] = {2, 3, 5, 9, 17, 33};
                                static const double PE[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
                                int cb = 0, pb = 0;
                                for (u32 c : CE) cb += c <= total;
                                for (double p : PE) pb += p <= (double)top[0].first / (double)total;
                                cell[g] = (int16_t)(((1 + li) * 7 + cb) * 6 + pb);
                                double sum = 0;
                                for (auto& tc : top) sum += tc.first;
                                for (int r = 0; r < entries; ++r) {
                                    next[g * entries + r] = r < (int)top.size() ? top[r].second : 0;
                                    weights[g * entries + r] =
                                        r < (int)top.size() ? (u16)std::nearbyint((double)top[r].first / sum * 65535.0)
                                                            : 0;
                                }
                                filled[g] = 1;
                                ++hinted;
                            }
                        }
                    }
                    for (u16 t : touched) counts[t] = 0;
                    i = j;
                }
            }
        });
        if (getenv("ORACLE_TRACE"))
            fprintf(stderr, "online k=%d: %zu elements, built %.2f s, sorted %.2f s, walked %.2f s\n", k, els.size(),
                    tb - t0, t1 - tb, now() - t1);
    }
    return hinted;
}

}  // extern "C"
