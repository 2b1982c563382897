// Partitioned pair counting: the engine's count path without global atomics (no counterpart in the reference's
// libraries; it replaces, inside this build's hosts, the split-table counting of ng_scan_count and ng_table_compact).
//
//   1. ng_scan_emit (engine.hip) appends each hit's mix64(pair key) to its block's region;
//   2. ng_seg_offsets + ng_seg_gather pack the regions into one array of events;
//   3. the events are sorted by their top pbits (sort_pairs, keys only): partition p = events whose mixed key has top
//      bits p, i.e. a hash partition of the pairs; ng_part_bounds finds each partition's range;
//   4. ng_part_count: one block per group of partitions (about equal events each) counts each partition's events in
//      an LDS hash table (8192 slots in buckets of four; a partition reaching 7000 distinct pairs sets flags[0] bit 0
//      and the host repeats 3-4 with one more bit),
//      answers that partition's lookups (the query positions' (context, target) pairs, hashed and sorted the same way
//      by ng_part_lookups + sort_pairs), and appends the distinct pairs (unmixed) with their counts to the block's
//      segment, which ng_seg_gather packs again.
// Every event is read three times and written twice, in coalesced runs, and counted by LDS atomics; on MI355X global
// atomics run at about 27 G/s scattered and 80 M/s on one address, far below these streams.
#include "part.h"
#include "prim.h"
#include "scatter.h"

namespace {

// offsets[s] = cnt[0] + ... + cnt[s - 1], offsets[n] = the total: one block of 1024 threads, each a contiguous chunk.
__global__ void __launch_bounds__(1024) seg_offsets_k(const u32* __restrict__ cnt, i64 n, u64* __restrict__ off) {
    __shared__ u64 part[1024];
    const int t = threadIdx.x;
    const i64 per = (n + 1023) / 1024;
    const i64 a = t * per, b = a + per < n ? a + per : n;
    u64 sum = 0;
    for (i64 i = a; i < b; ++i) sum += cnt[i];
    part[t] = sum;
    __syncthreads();
    for (int d = 1; d < 1024; d <<= 1) {  // Hillis-Steele inclusive scan of the chunk sums
        const u64 v = t >= d ? part[t - d] : 0;
        __syncthreads();
        part[t] += v;
        __syncthreads();
    }
    u64 run = part[t] - sum;
    for (i64 i = a; i < b; ++i) {
        off[i] = run;
        run += cnt[i];
    }
    if (t == 1023) off[n] = part[1023];
}

// Segment s (src + base_s, cnt[s] items; base_s = bases[s], or s * region without bases) copied to dst + off[s].
__global__ void __launch_bounds__(256) seg_gather_k(const u64* __restrict__ src_k, const u32* __restrict__ src_v,
                                                    u64 region, const i64* __restrict__ bases, const u32* __restrict__ cnt,
                                                    i64 nseg, const u64* __restrict__ off, u64* __restrict__ dst_k,
                                                    u32* __restrict__ dst_v) {
    for (i64 s = blockIdx.x; s < nseg; s += gridDim.x) {
        const u64 base = bases ? (u64)bases[s] : (u64)s * region;
        const u32 c = !bases && (u64)cnt[s] > region ? (u32)region : cnt[s];  // a region holds at most `region`
        const u64 o = off[s];
        for (u32 i = threadIdx.x; i < c; i += 256) {
            dst_k[o + i] = src_k[base + i];
            if (src_v) dst_v[o + i] = src_v[base + i];
        }
    }
}

// An event's partition: its top pbits, numbered in the order the partition sort leaves them. msd 0: sorted by the
// top pbits (LSD). msd 1: first grouped by the top 8 bits, then stably sorted by the pbits - 8 bits below them, so
// partition (lo, hi) = (bits [64 - pbits, 56), bits [56, 64)) is numbered lo << 8 | hi.
__device__ __forceinline__ i64 part_id(u64 e, int pbits, int msd) {
    if (pbits <= 0) return 0;
    if (!msd || pbits <= 8) return (i64)(e >> (64 - pbits));
    const u64 lo = (e >> (64 - pbits)) & ((1ull << (pbits - 8)) - 1);
    return (i64)((lo << 8) | (e >> 56));
}

// start[p] = the first i with part_id(ev[i]) >= p, for p = 0..P (start[P] = n).
__global__ void part_bounds_k(const u64* __restrict__ ev, i64 n, int pbits, int msd, i64 P, i64* __restrict__ start) {
    const i64 p = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (p > P) return;
    i64 a = 0, b = n;
    if (p == P) a = n;
    else if (pbits > 0) {
        while (a < b) {
            const i64 m = (a + b) >> 1;
            if (part_id(ev[m], pbits, msd) < p) a = m + 1;
            else b = m;
        }
    }  // pbits 0: one partition starting at 0
    start[p] = a;
}

// Lookup j of query position i = pos[j] (pos NULL: i = j): the mixed pair key of its (context, target) if its
// context id is in [lo, hi) (else EMPTY, which no mixed pair key equals: mix64 is a bijection and its preimage of
// EMPTY is no pair key), value i.
__global__ void part_lookups_k(const int* __restrict__ ctx_of, const u16* __restrict__ tgt, const int* __restrict__ pos,
                               i64 n, i64 lo, i64 hi, u64* __restrict__ qk, u32* __restrict__ qv) {
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= n) return;
    const i64 i = pos ? pos[j] : j;
    const i64 c = ctx_of[i];
    qk[j] = (c >= lo && c < hi) ? mix64(((u64)c << 16) | tgt[i]) : EMPTY;
    qv[j] = (u32)i;
}

#define PT_SLOTS 8192    // 96 KB of LDS per block (keys and counts; measured faster than two blocks per CU of 6400)
#define PT_BUCKETS (PT_SLOTS / 4)
#define PT_BLOCK 1024
#define PT_ITEMS 4
#define PT_LIMIT 7000  // distinct pairs a partition may reach before it is declared overfull (with every thread's
                       // insert in flight the table stays below PT_SLOTS, so probes always meet their key or a free slot)

// The LDS table is bucketized: four keys per 32-byte bucket, filled from the front, buckets probed linearly from the
// key's home bucket. A key lies in the first bucket along its probe sequence that has a free slot, or before it, so
// one pair of 16-byte reads settles most probes: on MI355X the divergent one-slot probe loop cost about twice as
// much, in scalar exec-mask work per probe step.
__device__ __forceinline__ u32 pt_bucket(u64 key) { return (u32)(((u64)(u32)key * PT_BUCKETS) >> 32); }
__device__ __forceinline__ u32 pt_next(u32 b) { return b + 1 == PT_BUCKETS ? 0 : b + 1; }

__device__ __forceinline__ void pt_read4(const u64* tk, u32 b, u64& k0, u64& k1, u64& k2, u64& k3) {
    const ulonglong2 a = *(const ulonglong2*)(tk + 4 * b);
    const ulonglong2 c = *(const ulonglong2*)(tk + 4 * b + 2);
    k0 = a.x;
    k1 = a.y;
    k2 = c.x;
    k3 = c.y;
}

// Count `add` occurrences of `key`; returns whether it took a free slot. A lost race for a free slot re-reads the
// bucket. Unbounded: the occupancy limit keeps a free slot in the table.
__device__ __forceinline__ bool pt_add(u64* tk, u32* tc, u64 key, u32 add) {
    u32 b = pt_bucket(key);
    int slot = -1;
    bool fresh = false;
    while (slot < 0) {
        u64 k0, k1, k2, k3;
        pt_read4(tk, b, k0, k1, k2, k3);
        const int q = k0 == key ? 0 : k1 == key ? 1 : k2 == key ? 2 : k3 == key ? 3 : -1;
        const int e = k0 == EMPTY ? 0 : k1 == EMPTY ? 1 : k2 == EMPTY ? 2 : k3 == EMPTY ? 3 : -1;
        if (q >= 0) {
            slot = 4 * (int)b + q;
        } else if (e >= 0) {
            const u64 prev = atomicCAS((unsigned long long*)&tk[4 * b + e], EMPTY, key);
            if (prev == EMPTY || prev == key) {
                slot = 4 * (int)b + e;
                fresh = prev == EMPTY;
            }
        } else {
            b = pt_next(b);
        }
    }
    atomicAdd(&tc[slot], add);
    return fresh;
}

__device__ __forceinline__ u32 pt_find(const u64* tk, const u32* tc, u64 key) {
    u32 b = pt_bucket(key);
    while (true) {
        u64 k0, k1, k2, k3;
        pt_read4(tk, b, k0, k1, k2, k3);
        const int q = k0 == key ? 0 : k1 == key ? 1 : k2 == key ? 2 : k3 == key ? 3 : -1;
        if (q >= 0) return tc[4 * b + q];
        if (k3 == EMPTY) return 0;
        b = pt_next(b);
    }
}

// Block b counts the partitions it owns (part_owner) in turn. Its distinct pairs (at most its events) go to
// out[start[p0] ...]: segment b = (seg_base[b], seg_cnt[b]). qcnt[qv[j]] = the count of lookup j (0: absent).
// cb == 0: out_k = pair key, out_c = count. cb > 0 (context ids below 2^cb, cb <= 44): out_k = the packed word
// pair key << (48 - cb) | min(count, esc), esc = 2^(48 - cb) - 1, a count >= esc also put in the escape table.
__global__ void __launch_bounds__(PT_BLOCK) part_count_k(const u64* __restrict__ ev, const i64* __restrict__ start,
                                                        i64 P, const u64* __restrict__ qk,
                                                        const u32* __restrict__ qv, const i64* __restrict__ qstart,
                                                        u64* __restrict__ out_k, u32* __restrict__ out_c, int cb,
                                                        u64* esc_k, u32* esc_c, u64 esc_cap,
                                                        u32* __restrict__ seg_cnt, i64* __restrict__ seg_base,
                                                        u32* __restrict__ qcnt, u32* __restrict__ dhist, int dshift,
                                                        int dbits, u32* flags) {
    __shared__ __align__(16) u64 tk[PT_SLOTS];
    __shared__ u32 tc[PT_SLOTS];
    __shared__ u32 dh[SS_MAXB];  // with dhist: the block's packed words per dbits-bit digit at dshift
    __shared__ u32 cur;
    __shared__ u32 nocc;  // the partition's distinct pairs counted so far (updated once per wave and item)
    const int t = threadIdx.x, lane = lane_id();
    const i64 n_ev = start[P], G = gridDim.x;
    const i64 p0 = part_first(start, P, n_ev, G, blockIdx.x), p1 = part_first(start, P, n_ev, G, blockIdx.x + 1);
    if (p0 >= p1) {
        if (t == 0) {
            seg_cnt[blockIdx.x] = 0;
            seg_base[blockIdx.x] = 0;
        }
        if (dhist)
            for (int d = t; d < (1 << dbits); d += PT_BLOCK) dhist[(i64)d * G + blockIdx.x] = 0;
        return;
    }
    const i64 out_base = start[p0];
    if (t == 0) {
        cur = 0;
        nocc = 0;
    }
    if (dhist)
        for (int d = t; d < (1 << dbits); d += PT_BLOCK) dh[d] = 0;
    for (int j = t; j < PT_SLOTS; j += PT_BLOCK) {  // the output pass empties the slots for the next partition
        tk[j] = EMPTY;
        tc[j] = 0;
    }
    __syncthreads();
    // the events stream through in rounds of PT_ITEMS * PT_BLOCK; each round's loads are issued before the previous
    // round (or the previous partition's output) is worked through, so their latency is hidden
    constexpr i64 ROUND = (i64)PT_BLOCK * PT_ITEMS;
    auto load_round = [&](u64 (&dst)[PT_ITEMS], i64 i0, i64 end) {
#pragma unroll
        for (int r = 0; r < PT_ITEMS; ++r) {
            const i64 i = i0 + (i64)r * PT_BLOCK + t;
            dst[r] = i < end ? ev[i] : EMPTY;
        }
    };
    u64 ahead[PT_ITEMS];
    i64 ahead_of = -1;  // the partition whose first round `ahead` holds (block-uniform)
    for (i64 p = p0; p < p1; ++p) {
        const i64 a = start[p], b = start[p + 1], qa = qstart[p], qb = qstart[p + 1];
        // the partition's first lookups are loaded now, so that their latency overlaps the inserts
        const bool has_q = qa + t < qb;
        u64 lk = EMPTY;
        u32 lv = 0;
        if (has_q) {
            lk = qk[qa + t];
            lv = qv[qa + t];
        }
        if (ahead_of != p && a < b) load_round(ahead, a, b);
        for (i64 i0 = a; i0 < b; i0 += ROUND) {  // the same rounds for every wave
            u64 key[PT_ITEMS];
#pragma unroll
            for (int r = 0; r < PT_ITEMS; ++r) key[r] = ahead[r];
            if (i0 + ROUND < b) {
                load_round(ahead, i0 + ROUND, b);
                ahead_of = p;
            } else if (p + 1 < p1) {
                load_round(ahead, b, start[p + 2]);  // the next partition's first round
                ahead_of = p + 1;
            }
#pragma unroll
            for (int r = 0; r < PT_ITEMS; ++r) {
                const bool valid = key[r] != EMPTY;
                const u64 vb = __ballot(valid);
                if (!vb) continue;
                if (__builtin_amdgcn_readfirstlane(nocc) >= PT_LIMIT) {  // overfull: the host repartitions
                    if (lane == 0) atomicOr(&flags[0], 1u);
                    continue;
                }
                // the lanes holding the wave's first key add once (a hot pair would serialize the LDS atomics)
                const int ld = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)vb) - 1);
                const u64 k0 = readlane_u64(key[r], ld);
                const bool same = valid && key[r] == k0;
                const u64 m = __ballot(same);
                bool fresh = false;
                if (valid && (!same || lane == ld)) fresh = pt_add(tk, tc, key[r], same ? (u32)__popcll(m) : 1u);
                const u64 fb = __ballot(fresh);
                if (fb && lane == 0) atomicAdd(&nocc, (u32)__popcll(fb));
            }
        }
        lds_barrier();
        if (qb > qa) {  // block-uniform
            if (has_q) qcnt[lv] = lk == EMPTY ? 0u : pt_find(tk, tc, lk);
            for (i64 j = qa + PT_BLOCK + t; j < qb; j += PT_BLOCK) {
                const u64 key = qk[j];
                qcnt[qv[j]] = key == EMPTY ? 0u : pt_find(tk, tc, key);
            }
            lds_barrier();  // every lookup has probed before the output pass empties the slots
        }
        for (int j0 = 0; j0 < PT_SLOTS; j0 += PT_BLOCK) {
            const int j = j0 + t;
            const u64 key = j < PT_SLOTS ? tk[j] : EMPTY;
            const bool occ = key != EMPTY;
            const u64 bal = __ballot(occ);
            if (!bal) continue;
            u32 off = 0;
            if (lane == 0) off = atomicAdd(&cur, (u32)__popcll(bal));
            off = (u32)__shfl((int)off, 0, WAVE);
            if (occ) {
                const u64 at = (u64)out_base + off + (u64)__popcll(bal & lanemask_lt());
                const u64 pk = unmix64(key);
                const u32 n = tc[j];
                tk[j] = EMPTY;
                tc[j] = 0;
                if (cb == 0) {
                    out_k[at] = pk;
                    out_c[at] = n;
                } else {
                    const u64 esc = (1ull << (48 - cb)) - 1;
                    const u64 word = (pk << (48 - cb)) | ((u64)n < esc ? (u64)n : esc);
                    out_k[at] = word;
                    if ((u64)n >= esc) esc_put(esc_k, esc_c, esc_cap, pk, n, flags);
                    if (dhist) atomicAdd(&dh[(u32)(word >> dshift) & ((1u << dbits) - 1u)], 1u);
                }
            }
        }
        if (t == 0) nocc = 0;
        lds_barrier();  // the slots are empty again (the output stores need not have completed)
    }
    if (t == 0) {
        seg_cnt[blockIdx.x] = cur;
        seg_base[blockIdx.x] = out_base;
    }
    if (dhist)  // the last partition's barrier has ordered every count
        for (int d = t; d < (1 << dbits); d += PT_BLOCK) dhist[(i64)d * G + blockIdx.x] = dh[d];
}

// Per context from packed words sorted by context (word >> (64 - cb)): a wave per window of 64 words, staged in LDS.
// Each block is one wave, so that a wave held up by a long context holds up no other (with four waves a block, the
// barriers made every round wait for the block's slowest wave: 22-27% slower at c3's levels 2 and 3).
// A lane holding a context's first word whose context also ends in the window walks it in LDS alone (every such lane
// at once); the one context that runs past the window's end, if it starts there, is done by the whole wave over the
// following windows' leading words, counts summed and the top KT kept per lane, then reduced across the wave. No
// dependent global loads: every word is read by its own window and at most once more by the window of its context's
// first word. For present contexts only: dist[c] = its pairs, and its record rec[c] (CtxRecord<KT>::WORDS u32: total,
// pairs, the first KT tokens by (count desc, token asc) two per word, their counts; 0-padded; for KT 2 and 8 also the
// index of its first word), stored whole as 16-byte vectors; flags[0] bit 2 if a total reaches 2^32. dist may be
// NULL; with nstat: the contexts counted in nstat[1..256] (their sum) and, with deep, each context of more than
// deep_min pairs appended to deep (nstat[0] of them; callers size deep for U / (deep_min + 1) + 1).
#define SUMMARY_AHEAD 4  // windows of a long context loaded per step
#define SUMMARY_SHORT 12  // the longest context a lane walks alone within a window
#define SUMMARY_GRID 262144  // blocks (one wave each) at most (c3 level 2: 2^16 3% slower, 2^20 7% slower)

template <int KT>
__global__ void __launch_bounds__(WAVE) ctx_summary_k(const u64* __restrict__ w, i64 U, int cb,
                                                     const u64* __restrict__ esc_k, const u32* __restrict__ esc_c,
                                                     u64 esc_cap, u32* __restrict__ rec, u32* __restrict__ dist,
                                                     u32 deep_min, i64* __restrict__ deep, u32* __restrict__ nstat,
                                                     u32* flags) {
    u32 nctx = 0;  // contexts this lane summarized
    auto done = [&](u64 c, u32 pairs) {
        ++nctx;
        if (dist) dist[c] = pairs;
        if (deep && pairs > deep_min) deep[atomicAdd(&nstat[0], 1u)] = (i64)c;
    };
    __shared__ u64 sw[WAVE];
    using R = CtxRecord<KT>;
    __shared__ uint4 s_rec[WAVE * R::WORDS / 4];  // the short contexts' records of a window, stored together below
    __shared__ u64 s_ctx[WAVE];
    const int sh = 64 - cb, csh = 48 - cb;
    const u64 esc = (1ull << csh) - 1;
    const int lane = lane_id();
    auto count_of = [&](u64 word) -> u32 {
        const u64 n = word & esc;
        return n < esc ? (u32)n : esc_get(esc_k, esc_c, esc_cap, word >> csh);
    };
    const i64 nwin = (U + WAVE - 1) / WAVE;
    for (i64 wv = blockIdx.x; wv < nwin; wv += gridDim.x) {
        const i64 i = wv * WAVE + lane;
        const bool valid = i < U;
        const u64 word = valid ? w[i] : 0;
        const u64 ctx = word >> sh;
        sw[lane] = word;
        u64 prev = shfl_up_u64(word, 1);
        if (lane == 0) prev = (valid && i > 0) ? w[i - 1] : 0;
        u64 next = shfl_down_u64(word, 1);
        if (lane == WAVE - 1) next = i + 1 < U ? w[i + 1] : 0;
        const bool head = valid && (i == 0 || (prev >> sh) != ctx);
        const bool tail = valid && (i + 1 >= U || (next >> sh) != ctx);
        const u64 tails = __ballot(tail);
        // the context running past the window, when it starts in it: its next window is loaded now, so that the
        // load overlaps the lanes' walks below
        const bool open = head && !(tails >> lane);
        const u64 opens = __ballot(open);
        u64 ahead = 0;
        if (opens && wv * WAVE + WAVE + lane < U) ahead = w[wv * WAVE + WAVE + lane];
        __syncthreads();
        // a context that starts and ends in the window: walked by its first lane from LDS when short; a long one
        // (more than SUMMARY_SHORT words) by the whole wave below, one word per lane, so that one lane's long walk
        // does not hold up the wave
        int e = -1;  // this head's last word's lane
        if (head && (tails >> lane)) e = lane + __ffsll((unsigned long long)(tails >> lane)) - 1;
        const bool walk = e >= 0 && e - lane + 1 <= SUMMARY_SHORT;
        u64 longs = __ballot(e >= 0 && !walk);
        const u64 walks = __ballot(walk);
        if (walk) {
            u64 tl[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) tl[r] = 0;
            u64 s = 0;
            for (int j = lane; j <= e; ++j) {
                const u64 wj = sw[j];
                const u32 n = count_of(wj);
                s += n;
                topk_insert<KT>(tl, rank_score(wj >> csh, n));
            }
            done(ctx, (u32)(e - lane + 1));
            u32 v[R::WORDS];
            record_words<KT>(v, s, (u32)(e - lane + 1), tl, (u64)i);
            const int j = __popcll(walks & lanemask_lt());
#pragma unroll
            for (int q = 0; q < R::WORDS / 4; ++q)
                s_rec[j * (R::WORDS / 4) + q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
            s_ctx[j] = ctx;
            if (s >> 32) atomicOr(&flags[0], 4u);
        }
        if (walks) {  // wave-uniform: the records leave as 16-byte chunks of consecutive lanes, a record's chunks side
                      // by side (one request per record where a lane storing its own made one per chunk)
            __syncthreads();
            constexpr int CH = R::WORDS / 4;
            const int nrec = __popcll(walks);
            for (int q = lane; q < nrec * CH; q += WAVE)
                ((uint4*)(rec + s_ctx[q / CH] * R::WORDS))[q % CH] = s_rec[q];
        }
        while (longs) {  // wave-uniform
            const int h = __ffsll((unsigned long long)longs) - 1;
            longs &= longs - 1;
            const int eh = __shfl(e, h, WAVE);
            const bool in = lane >= h && lane <= eh;
            const u32 n = in ? count_of(word) : 0u;
            u64 part = n;
            u64 sc = in ? rank_score(word >> csh, n) : 0;
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) part += shfl_down_u64(part, d);
            part = bcast_u64(part, 0);
            u64 top[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) {  // KT rounds of a wave-wide maximum (scores are distinct within a context)
                u64 m = sc;
#pragma unroll
                for (int d = WAVE / 2; d > 0; d >>= 1) {
                    const u64 o = shfl_down_u64(m, d);
                    m = o > m ? o : m;
                }
                m = bcast_u64(m, 0);
                top[r] = m;
                if (m != 0 && sc == m) sc = 0;
            }
            if (lane == h) {
                done(ctx, (u32)(eh - h + 1));
                store_record<KT>(rec, ctx, part, (u32)(eh - h + 1), top, (u64)i);
                if (part >> 32) atomicOr(&flags[0], 4u);
            }
        }
        // the context running past the window: the whole wave, over the following windows
        if (opens) {
            const int h = __ffsll((unsigned long long)opens) - 1;
            const u64 hc = bcast_u64(ctx, h);
            const bool in = valid && lane >= h;
            u64 part = 0;
            u64 lt[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) lt[r] = 0;
            if (in) {
                part = count_of(word);
                lt[0] = rank_score(word >> csh, (u32)part);
            }
            u32 len = (u32)(WAVE - h);
            // the following windows: the next one already loaded (`ahead`), then SUMMARY_AHEAD windows per step, all
            // their loads issued before any is used (a long context costs one load latency per step, not per window)
            {
                const i64 j = wv * WAVE + WAVE + lane;
                const bool in2 = j < U && (ahead >> sh) == hc;
                const u64 m2 = __ballot(in2);
                if (in2) {
                    const u32 n = count_of(ahead);
                    part += n;
                    topk_insert<KT>(lt, rank_score(ahead >> csh, n));
                }
                len += (u32)__popcll(m2);
                bool cont = ((m2 >> (WAVE - 1)) & 1ull) && wv * WAVE + 2 * WAVE < U;
                for (i64 nx = wv * WAVE + 2 * WAVE; cont; nx += SUMMARY_AHEAD * WAVE) {
                    u64 w4[SUMMARY_AHEAD];
#pragma unroll
                    for (int q = 0; q < SUMMARY_AHEAD; ++q) {
                        const i64 jq = nx + q * WAVE + lane;
                        w4[q] = jq < U ? w[jq] : 0;
                    }
#pragma unroll
                    for (int q = 0; q < SUMMARY_AHEAD; ++q) {
                        if (!cont) break;  // wave-uniform
                        const i64 jq = nx + q * WAVE + lane;
                        const bool iq = jq < U && (w4[q] >> sh) == hc;
                        const u64 mq = __ballot(iq);
                        if (iq) {
                            const u32 n = count_of(w4[q]);
                            part += n;
                            topk_insert<KT>(lt, rank_score(w4[q] >> csh, n));
                        }
                        len += (u32)__popcll(mq);
                        cont = ((mq >> (WAVE - 1)) & 1ull) && nx + (q + 1) * WAVE < U;
                    }
                }
            }
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) part += shfl_down_u64(part, d);
            part = bcast_u64(part, 0);
            // merge the lanes' lists: KT rounds of a wave-wide maximum; the lane holding it moves to its next entry
            // (scores are distinct within a context, so exactly one lane holds a nonzero maximum)
            int headq = 0;
            u64 merged[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) {
                u64 mine = 0;
#pragma unroll
                for (int q = 0; q < KT; ++q)
                    if (q == headq) mine = lt[q];
                u64 m = mine;
#pragma unroll
                for (int d = WAVE / 2; d > 0; d >>= 1) {
                    const u64 o = shfl_down_u64(m, d);
                    m = o > m ? o : m;
                }
                m = bcast_u64(m, 0);
                merged[r] = m;
                if (m != 0 && mine == m) ++headq;
            }
            if (lane == h) {
                done(hc, len);
                store_record<KT>(rec, hc, part, len, merged, (u64)(wv * WAVE + h));
                if (part >> 32) atomicOr(&flags[0], 4u);
            }
        }
        __syncthreads();  // the window's staged words are read before the next round writes them
    }
    if (nstat) {  // one add per wave, spread over 256 counters
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) nctx += (u32)__shfl_down((int)nctx, d, WAVE);
        if (lane == 0 && nctx) atomicAdd(&nstat[1 + (blockIdx.x & 255)], nctx);
    }
}

// Per query position i whose context id c is in [lo, hi) and present (dist[c - lo] > 0): from its context's record
// (ctx_summary_k's) tot, dist (at most 65535), the first kout of ktop top entries; cnt = qcnt[i] (with thr: only if its
// score reaches thr[c]); mask bit li.
// A position's first kout (<= KT) entries, tokens tk and counts tc, into rows i of out_tok / out_tcnt ([., kout]): one
// store each where the row is a whole KT-entry vector (kout == KT, 4 or 8, rows aligned), else entry by entry.
template <int KT>
__device__ __forceinline__ void put_top(u16* __restrict__ out_tok, u32* __restrict__ out_tcnt, i64 i, int kout,
                                        const u16 (&tk)[KT], const u32 (&tc)[KT]) {
    if constexpr (KT == 4 || KT == 8) {
        if (kout == KT && !((uintptr_t)out_tok & 7) && !((uintptr_t)out_tcnt & 15)) {
#pragma unroll
            for (int h = 0; h < KT / 4; ++h) {
                *(ushort4*)(out_tok + i * KT + 4 * h) = make_ushort4(tk[4 * h], tk[4 * h + 1], tk[4 * h + 2], tk[4 * h + 3]);
                *(uint4*)(out_tcnt + i * KT + 4 * h) = make_uint4(tc[4 * h], tc[4 * h + 1], tc[4 * h + 2], tc[4 * h + 3]);
            }
            return;
        }
    }
#pragma unroll
    for (int r = 0; r < KT; ++r) {
        if (r < kout) {
            out_tok[i * kout + r] = tk[r];
            out_tcnt[i * kout + r] = tc[r];
        }
    }
}

template <int KT>
__global__ void __launch_bounds__(256) pos_summary_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi,
                                                     const u16* __restrict__ tgt, const u32* __restrict__ rec,
                                                     const u32* __restrict__ dist, const u64* __restrict__ thr,
                                                     const u32* __restrict__ qcnt, int kout, int li,
                                                     int* __restrict__ out_tot, int* __restrict__ out_dist,
                                                     int* __restrict__ out_cnt, u16* __restrict__ out_tok,
                                                     u32* __restrict__ out_tcnt, int* __restrict__ mask,
                                                     u32* __restrict__ hit_bits) {
    using R = CtxRecord<KT>;
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    i64 c = i < N ? ctx_of[i] : -1;
    const bool other = c >= 0 && (c < lo || c >= hi);  // a context of another id range: that range's call writes it
    const u32 d = c >= 0 && !other ? dist[c - lo] : 0u;
    if (hit_bits) {  // bit i: position i's context occurred (a wave's 64 positions are two words)
        const u64 m = __ballot(d != 0);
        if (lane_id() == 0 && i < N) {
            hit_bits[i >> 5] = (u32)m;
            hit_bits[(i >> 5) + 1] = (u32)(m >> 32);
        }
    }
    if (i >= N || other) return;
    if (d == 0) {  // no context, or one that never occurred: zeros (so the outputs need no fill before)
        out_tot[i] = 0;
        out_dist[i] = 0;
        out_cnt[i] = 0;
        const u16 zt[KT] = {};
        const u32 zc[KT] = {};
        put_top<KT>(out_tok, out_tcnt, i, kout, zt, zc);
        return;
    }
    c -= lo;
    u32 v[R::WORDS];
    const uint4* src = (const uint4*)(rec + c * R::WORDS);
#pragma unroll
    for (int q = 0; q < R::WORDS / 4; ++q) {
        const uint4 x = src[q];
        v[4 * q] = x.x;
        v[4 * q + 1] = x.y;
        v[4 * q + 2] = x.z;
        v[4 * q + 3] = x.w;
    }
    out_tot[i] = (int)v[0];
    out_dist[i] = (int)(d < 65535u ? d : 65535u);
    const u32 n = qcnt ? qcnt[i] : 0u;
    int cnt = 0;
    if (n) {
        const u64 th = thr ? thr[c] : 0;
        if (th == 0 || rank_score(((u64)c << 16) | tgt[i], n) >= th) cnt = (int)n;
    }
    out_cnt[i] = cnt;
    u16 tk[KT];
    u32 tc[KT];
#pragma unroll
    for (int r = 0; r < KT; ++r) {
        tk[r] = (u16)(v[2 + r / 2] >> (16 * (r & 1)));
        tc[r] = v[2 + R::TOKW + r];
    }
    put_top<KT>(out_tok, out_tcnt, i, kout, tk, tc);
    if (mask) mask[i] |= 1 << li;
}

}  // namespace

// offsets[s] = cnt[0] + ... + cnt[s - 1] for s = 0..nseg (u64[nseg + 1]; offsets[nseg] = the total).
extern "C" int ng_seg_offsets(const u32* cnt, i64 nseg, u64* offsets, void* stream) {
    if (nseg < 0) return -1;
    seg_offsets_k<<<1, 1024, 0, (hipStream_t)stream>>>(cnt, nseg, offsets);
    return (int)hipGetLastError();
}

// Segments packed: segment s = cnt[s] items at src + (bases ? bases[s] : s * region), copied to dst + offsets[s]
// (ng_seg_offsets'). src_v / dst_v (u32 values beside the u64 keys) may be NULL.
extern "C" int ng_seg_gather(const u64* src_k, const u32* src_v, u64 region, const i64* bases, const u32* cnt,
                             i64 nseg, const u64* offsets, u64* dst_k, u32* dst_v, void* stream) {
    if (nseg <= 0) return 0;
    if ((src_v == nullptr) != (dst_v == nullptr)) return -1;
    const i64 g = nseg < 16384 ? nseg : 16384;
    seg_gather_k<<<(unsigned)g, 256, 0, (hipStream_t)stream>>>(src_k, src_v, region, bases, cnt, nseg, offsets, dst_k,
                                                               dst_v);
    return (int)hipGetLastError();
}

// start[p] for p = 0..2^pbits (i64[2^pbits + 1]) of events sorted by their top pbits (0 <= pbits <= 24): msd 0 in
// key order; msd 1 grouped first by the top 8 bits (ng_seg_scatter), then stably by the pbits - 8 bits below them,
// partition (lo, hi) numbered lo << 8 | hi.
extern "C" int ng_part_bounds(const u64* ev, i64 n, int pbits, int msd, i64* start, void* stream) {
    if (pbits < 0 || pbits > 24 || n < 0 || (msd != 0 && msd != 1)) return -1;
    const i64 P = 1ll << pbits;
    part_bounds_k<<<grid_for(P + 1, 256), 256, 0, (hipStream_t)stream>>>(ev, n, pbits, msd, P, start);
    return (int)hipGetLastError();
}

// Buffer fills on the caller's stream (the hosts' zeroed and EMPTY-filled buffers, so that no framework kernel runs
// inside a build): n words of value v.
extern "C" int ng_fill_u32(u32* p, i64 n, u32 v, void* stream) {
    if (n < 0 || (n > 0 && p == nullptr)) return -1;
    return prim::fill_u32(p, v, n, (hipStream_t)stream);
}
extern "C" int ng_fill_u64(u64* p, i64 n, u64 v, void* stream) {
    if (n < 0 || (n > 0 && p == nullptr)) return -1;
    return prim::fill_u64(p, v, n, (hipStream_t)stream);
}

// Exclusive prefix sum of n u32 (out may alias in), *total (device, may be NULL) the sum as u64; CUB-style two-phase
// temp storage (temp NULL: *temp_bytes set).
extern "C" int ng_exclusive_scan_u32(void* temp, size_t* temp_bytes, const u32* in, u32* out, i64 n, u64* total,
                                     void* stream) {
    if (n < 0 || temp_bytes == nullptr) return -1;
    if (temp == nullptr) {
        *temp_bytes = prim::scan_u32_temp_bytes(n);
        return 0;
    }
    return prim::exclusive_scan_u32(in, out, n, total, temp, (hipStream_t)stream);
}

// A sort's first pass from segments (scatter.h's scatter_k): nseg segments of ev_count[s] keys at src + (bases ? bases[s] :
// s * R), scattered by the nbits-bit digit (key >> shift) & (2^nbits - 1) (nbits <= 11) to out at the offsets dpre
// (u32 [2^nbits * nseg], the exclusive scan of the producer's digit histograms, digit-major: ng_scan_emit's with
// shift 56 and 8 bits, ng_part_count's; fewer than 2^32 keys).
extern "C" int ng_seg_scatter(const u64* src, u64 R, const i64* bases, const u32* ev_count, const u32* dpre, i64 nseg,
                              int shift, int nbits, u64* out, u64 cap, void* stream) {
    if (nseg < 0 || nbits < 1 || nbits > 11 || shift < 0 || shift + nbits > 64 ||
        (bases == nullptr && (R == 0 || R > 0xFFFFFFFFull)))
        return -1;
    if (nseg == 0) return 0;
    const i64 g = nseg < 16384 ? nseg : 16384;
    const RegionSegs sg{R, bases, ev_count, dpre, nseg};
    if (nbits <= 8)
        scatter_k<256, u64, u64><<<(unsigned)g, SS_BLOCK, 0, (hipStream_t)stream>>>(src, sg, shift, nbits, out, cap);
    else
        scatter_k<SS_MAXB, u64, u64><<<(unsigned)g, SS_BLOCK, 0, (hipStream_t)stream>>>(src, sg, shift, nbits, out, cap);
    return (int)hipGetLastError();
}

// ng_seg_scatter with the keys narrowed to their low 32 bits on the way out (u32 out[cap]): for keys whose digit is
// their top nbits bits and whose bits below the digit fit 32 (shift <= 32), the first pass of the 32-bit count.
extern "C" int ng_seg_scatter_narrow(const u64* src, u64 R, const i64* bases, const u32* ev_count, const u32* dpre,
                                     i64 nseg, int shift, int nbits, u32* out, u64 cap, void* stream) {
    if (nseg < 0 || nbits < 1 || nbits > 11 || shift < 0 || shift > 32 ||
        (bases == nullptr && (R == 0 || R > 0xFFFFFFFFull)))
        return -1;
    if (nseg == 0) return 0;
    const i64 g = nseg < 16384 ? nseg : 16384;
    const RegionSegs sg{R, bases, ev_count, dpre, nseg};
    if (nbits <= 8)
        scatter_k<256, u64, u32><<<(unsigned)g, SS_BLOCK, 0, (hipStream_t)stream>>>(src, sg, shift, nbits, out, cap);
    else
        scatter_k<SS_MAXB, u64, u32><<<(unsigned)g, SS_BLOCK, 0, (hipStream_t)stream>>>(src, sg, shift, nbits, out, cap);
    return (int)hipGetLastError();
}

// The lookups of n query positions (pos[j], or j with pos NULL): qk[j] = mix64(ctx_of[i] << 16 | tgt[i]) for context
// ids in [lo, hi), else EMPTY; qv[j] = i.
extern "C" int ng_part_lookups(const int* ctx_of, const u16* tgt, const int* pos, i64 n, i64 lo, i64 hi, u64* qk,
                               u32* qv, void* stream) {
    if (n <= 0) return 0;
    part_lookups_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, tgt, pos, n, lo, hi, qk, qv);
    return (int)hipGetLastError();
}

// Count the sorted events partition by partition (start: ng_part_bounds' of 2^pbits partitions) with `grid` blocks
// (at most 65536) of consecutive partitions holding about n / grid events each: block b's distinct pairs (pair key, count) at out_k/out_c + seg_base[b], seg_cnt[b] of
// them (out_k/out_c hold as many items as ev). Lookups (qk sorted like ev, qv their query positions, qstart their
// bounds) get qcnt[qv[j]] = the pair's count or 0. dhist (may be NULL; packed words only): block b's words per
// dbits-bit digit (word >> dshift) & (2^dbits - 1) (dbits <= 11) at dhist[d * grid + b], for ng_seg_scatter. flags[0] bit 0: a partition reached 7000
// distinct pairs
// (its count is incomplete: repartition with one more bit).
extern "C" int ng_part_count(const u64* ev, const i64* start, int pbits, const u64* qk, const u32* qv,
                             const i64* qstart, u64* out_k, u32* out_c, int cb, u64* esc_k, u32* esc_c, u64 esc_cap,
                             u32* seg_cnt, i64* seg_base, u32* qcnt, u32* dhist, int dshift, int dbits, u32* flags,
                             int grid, void* stream) {
    if (pbits < 0 || pbits > 24 || grid <= 0 || grid > 65536 || cb < 0 || cb > 44) return -1;
    if (cb > 0 && (esc_k == nullptr || esc_c == nullptr || esc_cap == 0)) return -1;
    if (cb == 0 && out_c == nullptr) return -1;
    if (dhist && (cb == 0 || dbits < 1 || dbits > 11 || dshift < 0 || dshift + dbits > 64)) return -1;
    const i64 P = 1ll << pbits;
    part_count_k<<<grid, PT_BLOCK, 0, (hipStream_t)stream>>>(ev, start, P, qk, qv, qstart, out_k, out_c, cb, esc_k,
                                                             esc_c, esc_cap, seg_cnt, seg_base, qcnt, dhist, dshift,
                                                             dbits, flags);
    return (int)hipGetLastError();
}

// Per context from U packed words (ng_part_count's with cb > 0) sorted by context: dist[c] = its pairs and its record
// rec[c] (u32 words: total, pairs, the first topk (1, 2, 4, 8) tokens by (count desc, token asc) two per word, their
// counts; 4, 8, 8, 16 words for topk 1, 2, 4, 8; for topk 2 and 8 the index of the context's first word in the two
// words after the counts), written for contexts present only (callers zero dist; dist may be NULL). With nstat
// (u32[257], zeroed): the number of contexts is nstat[1] + ... + nstat[256], and with deep the contexts of more than
// deep_min pairs are appended to deep (nstat[0] of them; sized U / (deep_min + 1) + 1). flags[0] bit 2: a total
// reached 2^32.
extern "C" int ng_ctx_summary(const u64* w, i64 U, int cb, const u64* esc_k, const u32* esc_c, u64 esc_cap, int topk,
                              u32* rec, u32* dist, u32 deep_min, i64* deep, u32* nstat, u32* flags, void* stream) {
    if (cb <= 0 || cb > 44 || esc_cap == 0 || (deep && !nstat)) return -1;
    if (U <= 0) return 0;
    int g = grid_for((U + WAVE - 1) / WAVE, 1);  // a window per block and round
    g = g > SUMMARY_GRID ? SUMMARY_GRID : g;
    hipStream_t st = (hipStream_t)stream;
    switch (topk) {
        case 1: ctx_summary_k<1><<<g, WAVE, 0, st>>>(w, U, cb, esc_k, esc_c, esc_cap, rec, dist, deep_min, deep, nstat, flags); break;
        case 2: ctx_summary_k<2><<<g, WAVE, 0, st>>>(w, U, cb, esc_k, esc_c, esc_cap, rec, dist, deep_min, deep, nstat, flags); break;
        case 4: ctx_summary_k<4><<<g, WAVE, 0, st>>>(w, U, cb, esc_k, esc_c, esc_cap, rec, dist, deep_min, deep, nstat, flags); break;
        case 8: ctx_summary_k<8><<<g, WAVE, 0, st>>>(w, U, cb, esc_k, esc_c, esc_cap, rec, dist, deep_min, deep, nstat, flags); break;
        default: return -1;
    }
    return (int)hipGetLastError();
}

// Per query position from the per-context records and pair counts (ng_ctx_summary's) and the counted lookups qcnt: tot,
// dist, cnt (thr may be NULL: the CNT_TOP threshold scores), the first kout <= ktop top entries, mask bit li (mask may
// be NULL). Every position whose context is absent (ctx_of < 0) or did not occur (dist 0) gets zeros; those whose
// context id lies outside [lo, hi) are left as they are. hit_bits (may be NULL; lo 0, every id in range): bit i set
// where position i's context occurred (ceil(N / 64) * 2 u32 words, all written), for the next level's list.
extern "C" int ng_pos_summary(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u32* rec, const u32* dist,
                              const u64* thr, const u32* qcnt, int ktop, int kout, int li, int* out_tot, int* out_dist,
                              int* out_cnt, u16* out_tok, u32* out_tcnt, int* mask, u32* hit_bits, void* stream) {
    if (kout < 0 || kout > ktop || (mask && (li < 0 || li > 30)) || (hit_bits && lo != 0)) return -1;
    if (N <= 0) return 0;
    const int g = grid_for(N, 256);
    hipStream_t st = (hipStream_t)stream;
    switch (ktop) {
        case 1: pos_summary_k<1><<<g, 256, 0, st>>>(ctx_of, N, lo, hi, tgt, rec, dist, thr, qcnt, kout, li, out_tot, out_dist, out_cnt, out_tok, out_tcnt, mask, hit_bits); break;
        case 2: pos_summary_k<2><<<g, 256, 0, st>>>(ctx_of, N, lo, hi, tgt, rec, dist, thr, qcnt, kout, li, out_tot, out_dist, out_cnt, out_tok, out_tcnt, mask, hit_bits); break;
        case 4: pos_summary_k<4><<<g, 256, 0, st>>>(ctx_of, N, lo, hi, tgt, rec, dist, thr, qcnt, kout, li, out_tot, out_dist, out_cnt, out_tok, out_tcnt, mask, hit_bits); break;
        case 8: pos_summary_k<8><<<g, 256, 0, st>>>(ctx_of, N, lo, hi, tgt, rec, dist, thr, qcnt, kout, li, out_tot, out_dist, out_cnt, out_tok, out_tcnt, mask, hit_bits); break;
        default: return -1;
    }
    return (int)hipGetLastError();
}
