// Online rows under the step rule on the GPU: the incremental state behind ngram_amd/online.py's OnlineRows (the
// surface of exact_match/src/online.rs :102-1382; no counterpart in the reference's GPU libraries). Per level k the
// state persists between steps: a context table (u64 keys, slot = context id), a record per context (its total,
// distinct next tokens and top-E entries, count descending then token ascending: one 64-byte load), and a pair table
// of 16-byte slots ((slot << 16 | next) key beside its u32 count: one line per lookup). A step inserts the occurrences
// that become available in it, then answers its queries (online.rs:11-13: an occurrence counts for a step-s query
// iff all its tokens were trained before s). The top-E lists stay exact: a step's touched pairs are grouped by context
// (in LDS buckets, ng_online_merge, or by a sort, ng_online_top) and merged into their context's list with their new
// counts (counts only grow, so untouched tokens outside a list stay below its last entry).
#include "ngram_common.h"
#include "prim.h"

namespace {

__device__ __forceinline__ i64 octx_find_insert(u64* ck, u64 ccap, u64 key, u32* flags) {
    u64 s = __umul64hi(key, ccap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 cur = ck[s];
        if (cur == key) return (i64)s;
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&ck[s], EMPTY, key);
            if (prev == EMPTY || prev == key) return (i64)s;
        }
        s = s + 1 == ccap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 2u);
    return -1;
}

__device__ __forceinline__ i64 octx_find(const u64* __restrict__ ck, u64 ccap, u64 key) {
    u64 s = __umul64hi(key, ccap);
    for (u64 probe = 0; probe < ccap; ++probe) {
        const u64 cur = ck[s];
        if (cur == key) return (i64)s;
        if (cur == EMPTY) return -1;
        s = s + 1 == ccap ? 0 : s + 1;
    }
    return -1;
}

// The pair table: cap slots of 16 bytes, pt[2s] the key (EMPTY when free) and the low half of pt[2s + 1] its count.
__device__ __forceinline__ u32* opair_cnt(u64* pt, u64 s) { return (u32*)(pt + 2 * s + 1); }

// Count a pair; returns 1 if this call inserted it (its first occurrence), 0 if it was there, -1 if the table is full.
__device__ __forceinline__ int opair_add(u64* pt, u64 cap, u64 key, u32* flags) {
    u64 s = __umul64hi(mix64(key), cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 cur = pt[2 * s];
        if (cur == key) {
            atomicAdd(opair_cnt(pt, s), 1u);
            return 0;
        }
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&pt[2 * s], EMPTY, key);
            if (prev == EMPTY || prev == key) {
                atomicAdd(opair_cnt(pt, s), 1u);
                return prev == EMPTY ? 1 : 0;
            }
        }
        s = s + 1 == cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
    return -1;
}

__device__ __forceinline__ u32 opair_count(const u64* __restrict__ pt, u64 cap, u64 key) {
    u64 s = __umul64hi(mix64(key), cap);
    for (u64 probe = 0; probe < cap; ++probe) {
        const ulonglong2 v = *(const ulonglong2*)(pt + 2 * s);  // key and count in one load
        if (v.x == key) return (u32)v.y;
        if (v.x == EMPTY) return 0;
        s = s + 1 == cap ? 0 : s + 1;
    }
    return 0;
}

// A pair's slot, inserted if absent (-1 and flags[0] bit 0 if the table is full).
__device__ __forceinline__ i64 opair_slot(u64* pt, u64 cap, u64 key, u32* flags) {
    u64 s = __umul64hi(mix64(key), cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 cur = pt[2 * s];
        if (cur == key) return (i64)s;
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&pt[2 * s], EMPTY, key);
            if (prev == EMPTY || prev == key) return (i64)s;
        }
        s = s + 1 == cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
    return -1;
}

// A context's record, rw u32 words per context slot: [0] its total, [1] its distinct next tokens; where the level keeps
// top lists (rw = OREC_TOP: 64 bytes, four 16-byte loads) [2, 10) the counts and [10, 14) the tokens (two per word,
// the lower half first) of its top entries, count descending then token ascending (count 0: no entry). As a ranking
// score an entry is count << 16 | 65535 - token.
#define OREC_TOP 16
#define OREC_CNT 2

struct ORec {
    u32 tot, dist;
    u64 sc[8];
};

__device__ __forceinline__ void orec_load(const u32* __restrict__ r, ORec& o) {
    const uint4* q = (const uint4*)r;
    const uint4 a = q[0], b = q[1], c = q[2], d = q[3];
    o.tot = a.x;
    o.dist = a.y;
    const u32 cnt[8] = {a.z, a.w, b.x, b.y, b.z, b.w, c.x, c.y};
    const u32 tk[4] = {c.z, c.w, d.x, d.y};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const u32 t = (tk[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
        o.sc[j] = cnt[j] ? ((u64)cnt[j] << 16) | (0xFFFFu - t) : 0;
    }
}

// The record of total tot, distinct count dist and the entries sc[0, E) (scores, descending; later ones empty).
__device__ __forceinline__ void orec_store(u32* r, u32 tot, u32 dist, const u64 (&sc)[8], int E) {
    u32 cnt[8], tk[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const u64 v = j < E ? sc[j] : 0;
        cnt[j] = (u32)(v >> 16);
        tk[j >> 1] |= (v ? 0xFFFFu - (u32)(v & 0xFFFF) : 0u) << (16 * (j & 1));
    }
    uint4* q = (uint4*)r;
    q[0] = make_uint4(tot, dist, cnt[0], cnt[1]);
    q[1] = make_uint4(cnt[2], cnt[3], cnt[4], cnt[5]);
    q[2] = make_uint4(cnt[6], cnt[7], tk[0], tk[1]);
    q[3] = make_uint4(tk[2], tk[3], 0u, 0u);
}

// A context's total and distinct count grown by add and fresh (a record without top entries).
__device__ __forceinline__ void orec_add(u32* r, u32 add, u32 fresh) {
    uint2 v = *(uint2*)r;
    v.x += add;
    v.y += fresh;
    *(uint2*)r = v;
}

template <int K>
__device__ __forceinline__ u64 okey(const u16* e, int k) {
    if constexpr (K > 0) return ctx_key<K>(e);
    else return ctx_key_rt(e, k);
}

// Occurrence i ending at pos[i] (context tok[g-k+1..g], next tok[g+1]; the caller lists valid ones only); ev[i] = the
// pair key | tag (the level's tag, above every pair key's bits: several levels' events sort as one array).
template <int K>
__device__ __forceinline__ void insert_one(const u16* __restrict__ tok, const int* __restrict__ pos, i64 i, int k,
                                           u64* ck, u64 ccap, u64* pt, u64 pcap, u32* rec, int rw,
                                           u64* __restrict__ ev, u32* flags, u64 tag, bool count_pair = true) {
    const i64 g = pos[i];
    const u64 key = okey<K>(tok + g + 1, k);
    const i64 slot = octx_find_insert(ck, ccap, key, flags);
    if (slot < 0) {
        ev[i] = EMPTY;
        return;
    }
    const u64 pair = ((u64)slot << 16) | tok[g + 1];
    if (!count_pair) {  // the step's merge counts each distinct pair once (ng_online_top with add_counts)
        ev[i] = pair | tag;
        return;
    }
    const int added = opair_add(pt, pcap, pair, flags);
    if (added < 0) {
        ev[i] = EMPTY;
        return;
    }
    if (rec) {  // else the step's sorted pass (online_top_k) adds them, once per context
        atomicAdd(&rec[slot * rw], 1u);
        if (added) atomicAdd(&rec[slot * rw + 1], 1u);
    }
    ev[i] = pair | tag;
}

template <int K>
__global__ void online_insert_k(const u16* __restrict__ tok, const int* __restrict__ pos, i64 m, int k, u64* ck,
                                u64 ccap, u64* pt, u64 pcap, u32* rec, int rw, u64* __restrict__ ev, u32* flags,
                                u64 tag) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < m) insert_one<K>(tok, pos, i, k, ck, ccap, pt, pcap, rec, rw, ev, flags, tag);
}

// Every level's inserts of a step in one launch: each level's inserts are chains of dependent table round trips, and
// in one launch the levels' chains overlap (c4, inserts counting pairs: five launches 409 us per step, one 322 us;
// with the pairs counted in the step's merge instead, 110 us). Level t takes
// the blocks with blockIdx.y == t; its fields (ONLINE_INS_FIELDS i64 each, as ng_online_insert_levels documents) are
// picked by unrolled compares on that block-uniform index, so no kernel argument is indexed at run time.
#define ONLINE_MAXL 8
#define ONLINE_INS_FIELDS 10
struct OInsArgs {
    i64 f[ONLINE_MAXL][ONLINE_INS_FIELDS];
};

template <int K>
__device__ __forceinline__ void insert_level(const u16* __restrict__ tok, const i64 (&f)[ONLINE_INS_FIELDS], i64 i,
                                             bool count_pairs) {
    if (i >= f[1]) return;
    insert_one<K>(tok, (const int*)f[0], i, (int)f[2], (u64*)f[3], (u64)f[4], (u64*)f[5], (u64)f[6], nullptr, 0,
                  (u64*)f[7], (u32*)f[8], (u64)f[9], count_pairs);
}

__global__ void __launch_bounds__(256) online_insert_levels_k(const u16* __restrict__ tok, int nlv, OInsArgs a,
                                                              bool count_pairs) {
    const int t = blockIdx.y;
    i64 f[ONLINE_INS_FIELDS];
#pragma unroll
    for (int q = 0; q < ONLINE_INS_FIELDS; ++q) f[q] = 0;
#pragma unroll
    for (int l = 0; l < ONLINE_MAXL; ++l)
        if (l == t)
#pragma unroll
            for (int q = 0; q < ONLINE_INS_FIELDS; ++q) f[q] = a.f[l][q];
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    switch ((int)f[2]) {
        case 1: insert_level<1>(tok, f, i, count_pairs); break;
        case 2: insert_level<2>(tok, f, i, count_pairs); break;
        case 3: insert_level<3>(tok, f, i, count_pairs); break;
        case 4: insert_level<4>(tok, f, i, count_pairs); break;
        case 5: insert_level<5>(tok, f, i, count_pairs); break;
        case 6: insert_level<6>(tok, f, i, count_pairs); break;
        case 8: insert_level<8>(tok, f, i, count_pairs); break;
        default: insert_level<0>(tok, f, i, count_pairs); break;
    }
}

// A level's state as the step's merge reads it: desc[t * 5 ...] for tag t = the pair table, its capacity, the
// contexts' records, whether the level keeps top lists (records of OREC_TOP words, else OREC_CNT), its flags.
#define OLEVEL_FIELDS 5
struct OLevel {
    u64* pt;
    u64 pcap;
    u32* rec;
    bool top;
    u32* flags;
    __device__ __forceinline__ u32* at(u64 slot) const { return rec + slot * (top ? OREC_TOP : OREC_CNT); }
};

__device__ __forceinline__ OLevel olevel(const i64* __restrict__ desc, u64 tag) {
    const i64* d = desc + tag * OLEVEL_FIELDS;
    return OLevel{(u64*)d[0], (u64)d[1], (u32*)d[2], d[3] != 0, (u32*)d[4]};
}

// Scores of a step's distinct touched pairs (sorted, tagged keys), i < *n. add_counts: each pair's step occurrences
// agg[i] are added to its count here (found or inserted; a plain update: the keys are distinct), else the inserts
// counted them.
__global__ void online_scores_k(const u64* __restrict__ uk, const u32* __restrict__ agg, const i64* __restrict__ n,
                                i64 m, const i64* __restrict__ desc, int tshift, bool add_counts,
                                u64* __restrict__ score) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= m || i >= *n) return;
    const u64 key = uk[i];
    if (key == EMPTY) {
        score[i] = 0;
        return;
    }
    const OLevel lv = olevel(desc, key >> tshift);
    const u64 pair = key & ((1ull << tshift) - 1);
    u32 c;
    if (add_counts) {
        const i64 s = opair_slot(lv.pt, lv.pcap, pair, lv.flags);
        if (s < 0) {
            score[i] = 0;
            return;
        }
        c = *opair_cnt(lv.pt, s) + agg[i];
        *opair_cnt(lv.pt, s) = c;
    } else {
        c = opair_count(lv.pt, lv.pcap, pair);
    }
    score[i] = ((u64)c << 16) | (0xFFFFu - (u32)(key & 0xFFFF));
}

#define ONLINE_SHORT 12  // the longest context of a step's pairs a lane walks alone within a window

__device__ __forceinline__ void top8_insert(u64 (&t)[8], u64 v) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
        if (v > t[j]) {
            const u64 tmp = t[j];
            t[j] = v;
            v = tmp;
        }
}

// A step's touched pairs uk[0..*n) (distinct, sorted; keys tagged with their level above bit tshift; agg[i] = their
// occurrences in the step, score[i] their ranking scores, count << 16 | 65535 - token), a wave per window of 64: for
// each context starting in the window (a context of one level: the tag is part of key >> 16), its total and distinct
// count grow by the step's occurrences and first-seen pairs (plain stores by the context's first lane: no
// same-address atomics for hot contexts), and (its level's top lists kept) its top-E list is merged with the new
// scores (an old entry of a touched token is superseded by its new score: counts only grow). A short context ending in
// its window is done by its first lane from LDS; a long one, and the one running past the window, by the whole wave.
// Each block is one wave: no barrier makes a wave wait for another's long context.
__global__ void __launch_bounds__(WAVE) online_top_k(const u64* __restrict__ uk, const u64* __restrict__ score,
                                                    const u32* __restrict__ agg, const i64* __restrict__ n_ptr, i64 m,
                                                    const i64* __restrict__ desc, int tshift, int E) {
    __shared__ u64 s_key[WAVE];
    __shared__ u64 s_sc[WAVE];
    __shared__ u32 s_ag[WAVE];
    const i64 n = *n_ptr < m ? *n_ptr : m;
    const int lane = (int)(threadIdx.x & (WAVE - 1));
    const i64 nwin = (n + WAVE - 1) / WAVE;
    auto ctx_of = [](u64 key) { return key >> 16; };
    for (i64 wv = blockIdx.x; wv < nwin; wv += gridDim.x) {
        const i64 i = wv * WAVE + lane;
        u64 key = i < n ? uk[i] : EMPTY;
        const bool valid = key != EMPTY;
        const u64 sc = valid ? score[i] : 0;
        const u32 ag = valid ? agg[i] : 0;
        s_key[lane] = key;
        s_sc[lane] = sc;
        s_ag[lane] = ag;
        u64 prev = shfl_up_u64(key, 1);
        if (lane == 0) prev = (valid && i > 0) ? uk[i - 1] : EMPTY;
        u64 next = shfl_down_u64(key, 1);
        if (lane == WAVE - 1) next = i + 1 < n ? uk[i + 1] : EMPTY;
        const u64 c = ctx_of(key);
        const bool head = valid && (i == 0 || prev == EMPTY || ctx_of(prev) != c);
        const bool tail = valid && (next == EMPTY || ctx_of(next) != c);
        const u64 tails = __ballot(tail);
        __syncthreads();
        int e = -1;  // where this head's context ends, if in the window
        if (head && (tails >> lane)) e = lane + __ffsll((unsigned long long)(tails >> lane)) - 1;
        if (e >= 0 && e - lane + 1 <= ONLINE_SHORT) {  // a short context ending in the window: this lane alone, from LDS
            const OLevel lv = olevel(desc, key >> tshift);
            u32* const r = lv.at(c & ((1ull << (tshift - 16)) - 1));
            u32 add = 0, fresh = 0;
            u64 t[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) t[j] = 0;
            for (int q = lane; q <= e; ++q) {
                add += s_ag[q];
                fresh += (u32)(s_sc[q] >> 16) == s_ag[q];
                if (lv.top) top8_insert(t, s_sc[q]);
            }
            if (lv.top) {
                ORec o;
                orec_load(r, o);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const u64 old = o.sc[j];
                    if (old == 0) continue;
                    const u64 tk = (c << 16) | (0xFFFFu - (u32)(old & 0xFFFF));
                    bool touched = false;
                    for (int q = lane; q <= e; ++q) touched |= s_key[q] == tk;
                    if (!touched) top8_insert(t, old);
                }
                orec_store(r, o.tot + add, o.dist + fresh, t, E);
            } else {
                orec_add(r, add, fresh);
            }
        }
        // the whole wave takes the context running past the window (over the following windows) and the long ones
        // ending in it (one pair per lane: one lane's long walk would hold up the wave)
        const bool open = head && !(tails >> lane);
        u64 waved = __ballot(open || (e >= 0 && e - lane + 1 > ONLINE_SHORT));
        while (waved) {  // wave-uniform
            const int h = __ffsll((unsigned long long)waved) - 1;
            waved &= waved - 1;
            const int eh = __shfl(e, h, WAVE);  // -1: the context runs past the window
            const u64 hc = bcast_u64(c, h);
            const OLevel lv = olevel(desc, hc >> (tshift - 16));
            u32* const hr = lv.at(hc & ((1ull << (tshift - 16)) - 1));
            const i64 gi = wv * WAVE + h;
            const bool in = valid && lane >= h && (eh < 0 || lane <= eh);
            u64 add = in ? ag : 0, fresh = (in && (u32)(sc >> 16) == ag) ? 1 : 0;
            u64 lt[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) lt[r] = 0;
            if (in && lv.top) lt[0] = sc;
            i64 ge = wv * WAVE + eh + 1;  // the group's end (found below for an open context)
            bool cont = eh < 0;
            if (cont) ge = wv * WAVE + WAVE;
            for (i64 nx = wv * WAVE + WAVE; cont; nx += WAVE) {
                const i64 j = nx + lane;
                const u64 k2 = j < n ? uk[j] : EMPTY;
                const bool in2 = k2 != EMPTY && ctx_of(k2) == hc;
                const u64 m2 = __ballot(in2);
                if (in2) {
                    const u64 s2 = score[j];
                    const u32 a2 = agg[j];
                    add += a2;
                    fresh += (u32)(s2 >> 16) == a2;
                    if (lv.top) top8_insert(lt, s2);
                }
                ge = nx + __popcll(m2);
                cont = ((m2 >> (WAVE - 1)) & 1ull) && nx + WAVE < n;
            }
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) {
                add += shfl_down_u64(add, d);
                fresh += shfl_down_u64(fresh, d);
            }
            if (lane == 0 && !lv.top) orec_add(hr, (u32)add, (u32)fresh);
            if (lv.top) {
                ORec o;  // every lane loads the record (one line); lane r checks old entry r
                orec_load(hr, o);
                u64 old = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (j == lane) old = o.sc[j];
                if (lane < E) {  // kept unless its token was touched in the step
                    if (old != 0) {
                        const u64 tk = (hc << 16) | (0xFFFFu - (u32)(old & 0xFFFF));
                        i64 a = gi, b = ge;
                        while (a < b) {
                            const i64 mid = (a + b) >> 1;
                            if (uk[mid] < tk) a = mid + 1;
                            else b = mid;
                        }
                        if (!(a < ge && uk[a] == tk)) top8_insert(lt, old);
                    }
                }
                // merge the lanes' lists: E rounds of a wave-wide maximum; the lane holding it moves on (scores are
                // distinct within a context)
                int headq = 0;
                u64 merged[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    u64 mine = 0;
#pragma unroll
                    for (int q = 0; q < 8; ++q)
                        if (q == headq) mine = lt[q];
                    u64 mx = mine;
#pragma unroll
                    for (int d = WAVE / 2; d > 0; d >>= 1) {
                        const u64 o = shfl_down_u64(mx, d);
                        mx = o > mx ? o : mx;
                    }
                    mx = bcast_u64(mx, 0);
                    merged[r] = mx;
                    if (mx != 0 && mine == mx) ++headq;
                }
                if (lane == 0) orec_store(hr, o.tot + (u32)add, o.dist + (u32)fresh, merged, E);
            }
        }
        __syncthreads();
    }
}

// ---- A step's merge by buckets of contexts (ng_online_merge): the step's events are not sorted ----
// The events (tagged pair keys tag << tshift | slot << 16 | next, as ng_online_top's sort takes them) are scattered by
// the low OM_BITS bits of their context slot into OM_NB buckets, so that all of a context's events land in one bucket
// (slots are hashed: the buckets are about equal). A block per bucket then
//   A. counts the distinct pairs of its events in an LDS hash (a packed word per pair: the pair key without the
//      bucket's bits, shifted above an occurrence count that LDS atomics add to),
//   B. sorts the distinct pairs in LDS (bitonic), which makes each context's pairs consecutive,
//   C. adds each pair's occurrences to its count in the level's pair table (one plain update: every pair of the step
//      is in one bucket and one round),
//   D. merges each context's record (total, distinct count, top-E entries) as online_top_k does, with the step's pairs
//      read from LDS: a context with many pairs in the step is walked by the wave over LDS, not over global memory.
// A bucket with more than OM_DCAP distinct pairs is done in rounds, its events split by a hash of the pair (halving
// until each round fits; nothing global is written before a round fits). A context whose pairs fall in several rounds
// is merged once per round: each merge supersedes the old entries of the pairs it touches, and a pair touched in a
// later round but absent from that round's top 8 scores below all 8 of them, so the list ends as one merge leaves it.
#ifndef OM_FRESH
#define OM_FRESH 1  // a pair whose home slot reads EMPTY is inserted there at once (no walk, no count read)
#endif
#define OM_BITS 11
#define OM_NB (1 << OM_BITS)
#define OM_BLOCK 512
#define OM_H 6144        // LDS hash slots
#define OM_DCAP 4096     // distinct pairs in a round at most (the hash at load <= 2/3; the sort's size)
#define OM_MAXSPLIT 40   // rounds split at most 40 times (2^40 rounds); beyond it level 0's flags[0] bit 2 is set
#define OM_CHUNK 8192    // events per histogram segment (ng_seg_scatter's segments)
#define OM_PER (OM_H / OM_BLOCK)
#define OM_EV 8       // events a thread loads at once
#define OM_PB 1       // pairs a thread looks up at once (2 and 4 measured 3-5% slower)

// Per segment of OM_CHUNK events, its count per bucket (digit-major: hist[d * nseg + s]) and its size.
__global__ void __launch_bounds__(1024) om_hist_k(const u64* __restrict__ ev, i64 m, i64 nseg, u32* __restrict__ hist,
                                                  u32* __restrict__ seg_n) {
    __shared__ u32 h[OM_NB];
    const int t = threadIdx.x;
    for (i64 sg = blockIdx.x; sg < nseg; sg += gridDim.x) {
        for (int d = t; d < OM_NB; d += 1024) h[d] = 0;
        lds_barrier();
        const i64 a = sg * OM_CHUNK, b = a + OM_CHUNK < m ? a + OM_CHUNK : m;
        for (i64 i = a + t; i < b; i += 1024) atomicAdd(&h[(u32)(ev[i] >> 16) & (OM_NB - 1)], 1u);
        lds_barrier();
        for (int d = t; d < OM_NB; d += 1024) hist[(i64)d * nseg + sg] = h[d];
        if (t == 0) seg_n[sg] = (u32)(b - a);
        lds_barrier();
    }
}

// Bucket b = the events evb[dpre[b * nseg], dpre[(b + 1) * nseg]) (the last one ends at m). cb: the count bits of
// the packed words (a pair's occurrences in the step < 2^cb - 1). At most 128 registers a lane (waves_per_eu 4), so
// that two blocks share a CU (its LDS allows two); uncapped, the kernel took 141 and ran 15% slower at one block.
__global__ void __launch_bounds__(OM_BLOCK) __attribute__((amdgpu_waves_per_eu(4))) om_merge_k(const u64* __restrict__ evb, const u32* __restrict__ dpre,
                                                       i64 nseg, i64 m, const i64* __restrict__ desc, int ntag,
                                                       int tshift, int cb, int E) {
    __shared__ u64 hs[OM_H];
    __shared__ u32 cs[OM_DCAP];
    __shared__ u32 s_part[OM_BLOCK / WAVE];
    __shared__ u64 s_stack[OM_MAXSPLIT + 2];  // pending rounds: residue << 8 | log2 of the rounds
    __shared__ int s_sp, s_nd, s_over;
    __shared__ i64 s_desc[ONLINE_MAXL * OLEVEL_FIELDS];  // the levels' descriptors: no global load before a lookup
    const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
    for (int i = t; i < ONLINE_MAXL * OLEVEL_FIELDS; i += OM_BLOCK) s_desc[i] = i < ntag * OLEVEL_FIELDS ? desc[i] : 0;
    const int hb = tshift - 16 - OM_BITS;  // slot bits above the bucket's
    const u64 hbm = (1ull << hb) - 1;
    const u64 cmask = (1ull << cb) - 1;
    const int csh = cb + 16;  // packed word >> csh = the context within the bucket (tag, slot bits above the bucket's)
    for (i64 b = blockIdx.x; b < OM_NB; b += gridDim.x) {
        const i64 e0 = dpre[b * nseg], e1 = b + 1 < OM_NB ? (i64)dpre[(b + 1) * nseg] : m;
        __syncthreads();  // every thread is done with the previous bucket's round stack
        if (t == 0) {
            s_stack[0] = 0;
            s_sp = 1;
        }
        for (;;) {
            __syncthreads();  // the previous round's global stores visible to this round; the round stack settled
            const int sp = s_sp;
            if (sp == 0) break;
            const u64 rtop = s_stack[sp - 1];
            const u64 res = rtop >> 8;
            const int lg = (int)(rtop & 0xFF);
            for (int i = t; i < OM_H; i += OM_BLOCK) hs[i] = EMPTY;
            if (t == 0) {
                s_nd = 0;
                s_over = 0;
            }
            lds_barrier();
            if (t == 0) s_sp = sp - 1;
            // A. the round's distinct pairs and their occurrences: OM_EV events a thread loaded together, then counted
            for (i64 base = e0; base < e1; base += (i64)OM_BLOCK * OM_EV) {
                if (*(volatile int*)&s_over) break;
                u64 ev[OM_EV];
#pragma unroll
                for (int j = 0; j < OM_EV; ++j) {
                    const i64 i = base + (i64)j * OM_BLOCK + t;
                    ev[j] = i < e1 ? evb[i] : EMPTY;
                }
#pragma unroll
                for (int j = 0; j < OM_EV; ++j) {
                    const u64 e = ev[j];
                    if (e == EMPTY) continue;
                    const u64 hx = mix64(e);
                    if (lg && (hx & ((1ull << lg) - 1)) != res) continue;
                    const u64 kp = ((e >> (16 + OM_BITS)) << 16) | (e & 0xFFFF);
                    u32 h = (u32)__umul64hi(hx, (u64)OM_H);
                    // ends: s_over is set at the (OM_DCAP + 1)-th insert, with a third of the slots still free, and a
                    // walk that meets it stops
                    for (;;) {
                        if (*(volatile int*)&s_over) break;
                        u64 cur = hs[h];
                        if (cur == EMPTY) {
                            cur = atomicCAS((unsigned long long*)&hs[h], EMPTY,
                                            (unsigned long long)((kp << cb) | 1ull));
                            if (cur == EMPTY) {
                                if (atomicAdd(&s_nd, 1) >= OM_DCAP) s_over = 1;
                                break;
                            }
                        }
                        if ((cur >> cb) == kp) {
                            atomicAdd((unsigned long long*)&hs[h], 1ull);
                            break;
                        }
                        h = h + 1 == OM_H ? 0 : h + 1;
                    }
                }
            }
            lds_barrier();
            if (s_over) {  // block-uniform: split the round in two by one more hash bit
                if (t == 0) {
                    if (lg >= OM_MAXSPLIT) {  // level 0's flags word (its descriptor's field 4): the host raises
                        static_assert(OLEVEL_FIELDS == 5, "a level descriptor's flags are its field 4");
                        atomicOr((u32*)s_desc[4], 4u);
                    } else {
                        s_stack[sp - 1] = ((res + (1ull << lg)) << 8) | (u64)(lg + 1);
                        s_stack[sp] = (res << 8) | (u64)(lg + 1);
                        s_sp = sp + 1;
                    }
                }
                continue;
            }
            const int D = s_nd;
            // B. the distinct pairs packed to hs[0, D), then sorted (EMPTY pads to a power of two)
            u64 v[OM_PER];
            u32 cnt = 0;
#pragma unroll
            for (int j = 0; j < OM_PER; ++j) {
                v[j] = hs[t * OM_PER + j];
                cnt += v[j] != EMPTY;
            }
            u32 incl = cnt;
#pragma unroll
            for (int d = 1; d < WAVE; d <<= 1) {
                const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
                if (lane >= d) incl += o;
            }
            if (lane == WAVE - 1) s_part[wid] = incl;
            lds_barrier();  // every slot read into registers before any is overwritten
            u32 o = incl - cnt;
            for (int w2 = 0; w2 < wid; ++w2) o += s_part[w2];
#pragma unroll
            for (int j = 0; j < OM_PER; ++j)
                if (v[j] != EMPTY) hs[o++] = v[j];
            u32 P = 1;
            while (P < (u32)D) P <<= 1;
            for (u32 i = (u32)D + t; i < P; i += OM_BLOCK) hs[i] = EMPTY;
            lds_barrier();
            for (u32 k = 2; k <= P; k <<= 1) {
                for (u32 j = k >> 1; j > 0; j >>= 1) {
                    for (u32 q = t; q < P / 2; q += OM_BLOCK) {
                        const u32 i = ((q & ~(j - 1)) << 1) | (q & (j - 1));
                        const u32 l = i | j;
                        const u64 x = hs[i], y = hs[l];
                        if ((x > y) == ((i & k) == 0)) {
                            hs[i] = y;
                            hs[l] = x;
                        }
                    }
                    lds_barrier();
                }
            }
            // C. each pair's count grows by its occurrences: OM_PB pairs a thread, their home slots (key and count)
            // loaded together; a pair not at its home slot walks on (opair_slot)
            for (int i0 = 0; i0 < D; i0 += OM_BLOCK * OM_PB) {
                u64 key[OM_PB], cur[OM_PB];
                i64 at[OM_PB];
                u32 cc[OM_PB], tg[OM_PB];
#pragma unroll
                for (int j = 0; j < OM_PB; ++j) {
                    const int i = i0 + j * OM_BLOCK + t;
                    at[j] = -1;
                    if (i < D) {
                        const u64 kp = hs[i] >> cb;
                        const u64 hi = kp >> 16;
                        tg[j] = (u32)(hi >> hb);
                        key[j] = ((((hi & hbm) << OM_BITS) | (u64)b) << 16) | (kp & 0xFFFF);
                        const OLevel lv = olevel(s_desc, tg[j]);
                        at[j] = (i64)__umul64hi(mix64(key[j]), lv.pcap);
                        const ulonglong2 v = *(const ulonglong2*)(lv.pt + 2 * at[j]);  // key and count: one load
                        cur[j] = v.x;
                        cc[j] = (u32)v.y;
                    }
                }
#pragma unroll
                for (int j = 0; j < OM_PB; ++j) {
                    const int i = i0 + j * OM_BLOCK + t;
                    if (i >= D) continue;
                    const OLevel lv = olevel(s_desc, tg[j]);
                    // an empty home slot is taken at once: a slot whose key was EMPTY holds count 0 (counts are
                    // written only after their key), so neither the slot nor its count is read again
                    u64 prev = cur[j];
                    if (OM_FRESH && cur[j] == EMPTY)
                        prev = atomicCAS((unsigned long long*)(lv.pt + 2 * at[j]), EMPTY, (unsigned long long)key[j]);
                    if (OM_FRESH && cur[j] == EMPTY && prev == EMPTY) {
                        cc[j] = 0;
                    } else if (prev != key[j]) {
                        at[j] = opair_slot(lv.pt, lv.pcap, key[j], lv.flags);
                        cc[j] = at[j] >= 0 ? *opair_cnt(lv.pt, at[j]) : 0;
                    } else if (cur[j] != key[j]) {  // another lane's insert of the same key (not within a merge)
                        cc[j] = *opair_cnt(lv.pt, at[j]);
                    }
                    u32 c = 0;
                    if (at[j] >= 0) {
                        c = cc[j] + (u32)(hs[i] & cmask);
                        *opair_cnt(lv.pt, at[j]) = c;
                    }
                    cs[i] = c;
                }
            }
            lds_barrier();
            // D. per context (its pairs consecutive in hs): windows of 64 pairs, a wave each (online_top_k's scheme)
            const u32 nwin = ((u32)D + WAVE - 1) / WAVE;
            for (u32 wv = wid; wv < nwin; wv += OM_BLOCK / WAVE) {
                const u32 i = wv * WAVE + lane;
                const bool valid = i < (u32)D;
                const u64 w = valid ? hs[i] : 0;
                const u64 cx = w >> csh;
                const u32 c = valid ? cs[i] : 0;
                const u32 ag = (u32)(w & cmask);
                const u64 sc = valid && c ? ((u64)c << 16) | (0xFFFFu - (u32)((w >> cb) & 0xFFFF)) : 0;
                u64 pcx = shfl_up_u64(cx, 1);
                if (lane == 0) pcx = valid && i > 0 ? hs[i - 1] >> csh : 0;
                u64 ncx = shfl_down_u64(cx, 1);
                if (lane == WAVE - 1) ncx = i + 1 < (u32)D ? hs[i + 1] >> csh : 0;
                const bool head = valid && (i == 0 || pcx != cx);
                const bool tail = valid && (i + 1 == (u32)D || ncx != cx);
                const u64 tails = __ballot(tail);
                int e = -1;  // where this head's context ends, if in the window
                if (head && (tails >> lane)) e = lane + __ffsll((unsigned long long)(tails >> lane)) - 1;
                if (e >= 0 && e - lane + 1 <= ONLINE_SHORT) {  // a short context ending in the window: this lane alone
                    const OLevel lv = olevel(s_desc, cx >> hb);
                    const u64 slot = ((cx & hbm) << OM_BITS) | (u64)b;
                    const u32 ge = wv * WAVE + (u32)e;
                    u32 add = 0, fresh = 0;
                    u64 tt[8];
#pragma unroll
                    for (int r = 0; r < 8; ++r) tt[r] = 0;
                    for (u32 q = i; q <= ge; ++q) {
                        const u64 wq = hs[q];
                        const u32 cq = cs[q], aq = (u32)(wq & cmask);
                        add += aq;
                        fresh += cq == aq;
                        if (lv.top && cq) top8_insert(tt, ((u64)cq << 16) | (0xFFFFu - (u32)((wq >> cb) & 0xFFFF)));
                    }
                    u32* const r = lv.at(slot);
                    if (lv.top) {
                        ORec o;
                        orec_load(r, o);
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const u64 old = o.sc[j];
                            if (old == 0) continue;
                            const u64 tk = (cx << 16) | (0xFFFFu - (u32)(old & 0xFFFF));
                            bool touched = false;
                            for (u32 q = i; q <= ge; ++q) touched |= (hs[q] >> cb) == tk;
                            if (!touched) top8_insert(tt, old);
                        }
                        orec_store(r, o.tot + add, o.dist + fresh, tt, E);
                    } else {
                        orec_add(r, add, fresh);
                    }
                }
                // the whole wave takes the context running past the window and the long ones ending in it
                const bool open = head && !(tails >> lane);
                u64 waved = __ballot(open || (e >= 0 && e - lane + 1 > ONLINE_SHORT));
                while (waved) {  // wave-uniform
                    const int h = __ffsll((unsigned long long)waved) - 1;
                    waved &= waved - 1;
                    const int eh = __shfl(e, h, WAVE);  // -1: the context runs past the window
                    const u64 hc = bcast_u64(cx, h);
                    const OLevel lv = olevel(s_desc, hc >> hb);
                    u32* const hr = lv.at(((hc & hbm) << OM_BITS) | (u64)b);
                    const u32 gi = wv * WAVE + (u32)h;
                    const bool in = valid && lane >= h && (eh < 0 || lane <= eh);
                    u64 add = in ? ag : 0, fresh = (in && c == ag) ? 1 : 0;
                    u64 lt[8];
#pragma unroll
                    for (int r = 0; r < 8; ++r) lt[r] = 0;
                    if (in && lv.top) lt[0] = sc;
                    u32 ge = wv * WAVE + (u32)eh + 1;  // the context's end (found below for an open one)
                    bool cont = eh < 0;
                    if (cont) ge = wv * WAVE + WAVE;
                    for (u32 nx = wv * WAVE + WAVE; cont; nx += WAVE) {
                        const u32 j = nx + lane;
                        const bool jv = j < (u32)D;
                        const u64 w2 = jv ? hs[j] : 0;
                        const bool in2 = jv && (w2 >> csh) == hc;
                        const u64 m2 = __ballot(in2);
                        if (in2) {
                            const u32 c2 = cs[j], a2 = (u32)(w2 & cmask);
                            add += a2;
                            fresh += c2 == a2;
                            if (lv.top && c2)
                                top8_insert(lt, ((u64)c2 << 16) | (0xFFFFu - (u32)((w2 >> cb) & 0xFFFF)));
                        }
                        ge = nx + (u32)__popcll(m2);
                        cont = ((m2 >> (WAVE - 1)) & 1ull) && nx + WAVE < (u32)D;
                    }
#pragma unroll
                    for (int d = WAVE / 2; d > 0; d >>= 1) {
                        add += shfl_down_u64(add, d);
                        fresh += shfl_down_u64(fresh, d);
                    }
                    if (lane == 0 && !lv.top) orec_add(hr, (u32)add, (u32)fresh);
                    if (lv.top) {
                        ORec o;  // every lane loads the record (one line); lane r checks old entry r
                        orec_load(hr, o);
                        u64 old = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j)
                            if (j == lane) old = o.sc[j];
                        if (lane < E) {  // kept unless its token was touched
                            if (old != 0) {
                                const u64 tk = (hc << 16) | (0xFFFFu - (u32)(old & 0xFFFF));
                                u32 lo = gi, hi2 = ge;
                                while (lo < hi2) {
                                    const u32 mid = (lo + hi2) >> 1;
                                    if ((hs[mid] >> cb) < tk) lo = mid + 1;
                                    else hi2 = mid;
                                }
                                if (!(lo < ge && (hs[lo] >> cb) == tk)) top8_insert(lt, old);
                            }
                        }
                        int headq = 0;
                        u64 merged[8];
#pragma unroll
                        for (int r = 0; r < 8; ++r) {
                            u64 mine = 0;
#pragma unroll
                            for (int q = 0; q < 8; ++q)
                                if (q == headq) mine = lt[q];
                            u64 mx = mine;
#pragma unroll
                            for (int d = WAVE / 2; d > 0; d >>= 1) {
                                const u64 ot = shfl_down_u64(mx, d);
                                mx = ot > mx ? ot : mx;
                            }
                            mx = bcast_u64(mx, 0);
                            merged[r] = mx;
                            if (mx != 0 && mine == mx) ++headq;
                        }
                        if (lane == 0) orec_store(hr, o.tot + (u32)add, o.dist + (u32)fresh, merged, E);
                    }
                }
            }
        }
    }
}

// Queries at pos[i] (input position g, context tok[g-k+1..g] valid iff avail[g] >= k): per level its context's
// slot (or -1) into qslot[i]; with count outputs (tot != NULL) tot / dist / cnt of the position into row g, column ci
// of [n, nc] arrays (cnt: the count of tok[g+1] if has_next[g]). rec: the level's records, rw words each.
template <int K>
__device__ __forceinline__ void query_one(const u16* __restrict__ tok, const int* __restrict__ avail,
                                          const unsigned char* __restrict__ has_next, const int* __restrict__ pos,
                                          i64 i, int k, const u64* __restrict__ ck, u64 ccap,
                                          const u64* __restrict__ pt, u64 pcap, const u32* __restrict__ rec, int rw,
                                          int* __restrict__ qslot, u32* __restrict__ tot, u16* __restrict__ dist,
                                          u32* __restrict__ cnt, int nc, int ci) {
    const i64 g = pos[i];
    i64 slot = -1;
    if (avail[g] >= (K > 0 ? K : k)) slot = octx_find(ck, ccap, okey<K>(tok + g + 1, k));
    uint2 td = make_uint2(0u, 0u);  // the context's total and distinct count: one load
    if (slot >= 0) td = *(const uint2*)(rec + slot * rw);
    if (td.x == 0) slot = -1;
    if (qslot) qslot[i] = (int)slot;
    if (tot && slot >= 0) {
        const i64 at = g * nc + ci;
        tot[at] = td.x;
        dist[at] = (u16)(td.y < 65535u ? td.y : 65535u);
        cnt[at] = has_next[g] ? opair_count(pt, pcap, ((u64)slot << 16) | tok[g + 1]) : 0u;
    }
}

template <int K>
__global__ void online_query_k(const u16* __restrict__ tok, const int* __restrict__ avail,
                               const unsigned char* __restrict__ has_next, const int* __restrict__ pos, i64 m, int k,
                               const u64* __restrict__ ck, u64 ccap, const u64* __restrict__ pt, u64 pcap,
                               const u32* __restrict__ rec, int rw, int* __restrict__ qslot, u32* __restrict__ tot,
                               u16* __restrict__ dist, u32* __restrict__ cnt, int nc, int ci) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < m) query_one<K>(tok, avail, has_next, pos, i, k, ck, ccap, pt, pcap, rec, rw, qslot, tot, dist, cnt, nc, ci);
}

// Every level's queries of a step in one launch (the same reason and layout as online_insert_levels_k).
#define ONLINE_QRY_FIELDS 13
struct OQryArgs {
    i64 f[ONLINE_MAXL][ONLINE_QRY_FIELDS];
};

template <int K>
__device__ __forceinline__ void query_level(const u16* __restrict__ tok, const int* __restrict__ avail,
                                            const unsigned char* __restrict__ has_next, const int* __restrict__ pos,
                                            i64 i, const i64 (&f)[ONLINE_QRY_FIELDS]) {
    query_one<K>(tok, avail, has_next, pos, i, (int)f[0], (const u64*)f[1], (u64)f[2], (const u64*)f[3], (u64)f[4],
                 (const u32*)f[5], (int)f[6], (int*)f[7], (u32*)f[8], (u16*)f[9], (u32*)f[10], (int)f[11],
                 (int)f[12]);
}

__global__ void __launch_bounds__(256) online_query_levels_k(const u16* __restrict__ tok, const int* __restrict__ avail,
                                                             const unsigned char* __restrict__ has_next,
                                                             const int* __restrict__ pos, i64 m, OQryArgs a) {
    const int t = blockIdx.y;
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= m) return;
    i64 f[ONLINE_QRY_FIELDS];
#pragma unroll
    for (int q = 0; q < ONLINE_QRY_FIELDS; ++q) f[q] = 0;
#pragma unroll
    for (int l = 0; l < ONLINE_MAXL; ++l)
        if (l == t)
#pragma unroll
            for (int q = 0; q < ONLINE_QRY_FIELDS; ++q) f[q] = a.f[l][q];
    switch ((int)f[0]) {
        case 1: query_level<1>(tok, avail, has_next, pos, i, f); break;
        case 2: query_level<2>(tok, avail, has_next, pos, i, f); break;
        case 3: query_level<3>(tok, avail, has_next, pos, i, f); break;
        case 4: query_level<4>(tok, avail, has_next, pos, i, f); break;
        case 5: query_level<5>(tok, avail, has_next, pos, i, f); break;
        case 6: query_level<6>(tok, avail, has_next, pos, i, f); break;
        case 8: query_level<8>(tok, avail, has_next, pos, i, f); break;
        default: query_level<0>(tok, avail, has_next, pos, i, f); break;
    }
}

// Position g's (query i's) hint rows: the deepest described levels (desc[v * 3 ...], deepest first: qslot (int [m]),
// the level's records (OREC_TOP words each), bucket) whose context occurred, up to S of them, into its slots
// g * S + j: cell, E next tokens, weights, and (level not NULL) the level's bucket. Returns the slots filled.
__device__ __forceinline__ int online_row(i64 g, i64 i, int nlv, const i64* __restrict__ desc, int E, int S,
                                          short* __restrict__ cell, u16* __restrict__ next, u16* __restrict__ weights,
                                          signed char* __restrict__ level) {
    int j = 0;
    for (int v = 0; v < nlv && j < S; ++v) {
        const i64* d = desc + v * 3;
        const int slot = ((const int*)d[0])[i];
        if (slot < 0) continue;
        ORec o;  // total and entries: one 64-byte record
        orec_load((const u32*)d[1] + (i64)slot * OREC_TOP, o);
        const u32 total = o.tot;
        const u64* top = o.sc;
        const int b = (int)d[2];
        const u32 top1 = (u32)(top[0] >> 16);
        int cb = 0, pb = 0;
        const u32 CE[6] = {2, 3, 5, 9, 17, 33};
        const double PE[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
#pragma unroll
        for (int e = 0; e < 6; ++e) cb += CE[e] <= total;
        const double share = (double)top1 / (double)total;
#pragma unroll
        for (int e = 0; e < 5; ++e) pb += PE[e] <= share;
        double sum = 0;
        for (int r = 0; r < E; ++r) sum += (double)(u32)(top[r] >> 16);
        const i64 row = g * S + j;
        cell[row] = (short)(((1 + b) * 7 + cb) * 6 + pb);
        if (level) level[row] = (signed char)b;
        for (int r = 0; r < E; ++r) {
            const u64 sc = top[r];
            next[row * E + r] = sc ? (u16)(0xFFFFu - (u32)(sc & 0xFFFF)) : (u16)0;
            weights[row * E + r] = sc ? (u16)rint((double)(u32)(sc >> 16) / sum * 65535.0) : (u16)0;
        }
        ++j;
    }
    return j;
}


// Hint rows of the queries pos[i] (online_row's, S slots each); *hinted += the queries with at least one row.
__global__ void online_rows_k(const int* __restrict__ pos, i64 m, int nlv, const i64* __restrict__ desc, int E, int S,
                              short* __restrict__ cell, u16* __restrict__ next, u16* __restrict__ weights,
                              signed char* __restrict__ level, int* __restrict__ hinted) {
    __shared__ int part[4];
    int c = 0;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < m; i += (i64)gridDim.x * blockDim.x)
        c += online_row(pos[i], i, nlv, desc, E, S, cell, next, weights, level) > 0;
    // one counter atomic per block: same-address atomics serialize
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += __shfl_down(c, d, WAVE);
    if ((threadIdx.x & (WAVE - 1)) == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        const int t = part[0] + part[1] + part[2] + part[3];
        if (t) atomicAdd(hinted, t);
    }
}

}  // namespace

#define OLEVELS(k, ...)                                        \
    switch (k) {                                               \
        case 1: { constexpr int K = 1; __VA_ARGS__; } break;   \
        case 2: { constexpr int K = 2; __VA_ARGS__; } break;   \
        case 3: { constexpr int K = 3; __VA_ARGS__; } break;   \
        case 4: { constexpr int K = 4; __VA_ARGS__; } break;   \
        case 5: { constexpr int K = 5; __VA_ARGS__; } break;   \
        case 6: { constexpr int K = 6; __VA_ARGS__; } break;   \
        case 8: { constexpr int K = 8; __VA_ARGS__; } break;   \
        case 10: { constexpr int K = 10; __VA_ARGS__; } break; \
        case 20: { constexpr int K = 20; __VA_ARGS__; } break; \
        default:                                               \
            if (k < 1 || k > MAXK) return -1;                  \
            { constexpr int K = 0; __VA_ARGS__; }              \
            break;                                             \
    }

// Insert the occurrences ending at pos[0..m) at level k, each counted in the pair table pt (pcap 16-byte slots) and,
// with rec (rw words per context: OREC_TOP or OREC_CNT), in its context's total and distinct count (else
// ng_online_top adds those); ev[i] = their pair keys | tag (EMPTY if a table was full: flags). tag: the level's tag <<
// tshift for ng_online_top (0 for one level), above every pair key of the tables.
extern "C" int ng_online_insert(const u16* tok, const int* pos, i64 m, int k, u64* ck, u64 ccap, u64* pt, u64 pcap,
                                u32* rec, int rw, u64* ev, u32* flags, u64 tag, void* stream) {
    if (m <= 0) return 0;
    if (ccap == 0 || pcap == 0 || ccap > (1ull << 40) || (tag && tag < (ccap << 16))) return -1;
    if (rec && rw != OREC_TOP && rw != OREC_CNT) return -1;
    hipStream_t st = (hipStream_t)stream;
    OLEVELS(k, (online_insert_k<K><<<grid_for(m, 256), 256, 0, st>>>(tok, pos, m, k, ck, ccap, pt, pcap, rec, rw, ev, flags, tag)));
    return (int)hipGetLastError();
}

// The inserts of nlv (1..8) levels in one launch: lv[t * 10 ...] = level t's pos, m, k, ck, ccap, pt, pcap, ev, flags,
// tag (host memory, read before the call returns; the pointers device memory), each as ng_online_insert's
// arguments of the same names (its totals and distinct counts left to ng_online_top). count_pairs 0: only the context
// is found or inserted and the event written; each distinct pair is then counted once by ng_online_top (add_counts 1)
// instead of one global atomic per occurrence. -1 on a bad level.
extern "C" int ng_online_insert_levels(const u16* tok, int nlv, const i64* lv, int count_pairs, void* stream) {
    if (nlv < 1 || nlv > ONLINE_MAXL || !lv) return -1;
    OInsArgs a{};
    i64 mmax = 0;
    for (int t = 0; t < nlv; ++t) {
        const i64* f = lv + (i64)t * ONLINE_INS_FIELDS;
        const i64 m = f[1], k = f[2];
        const u64 ccap = (u64)f[4], pcap = (u64)f[6], tag = (u64)f[9];
        if (m < 0 || k < 1 || k > MAXK || ccap == 0 || pcap == 0 || ccap > (1ull << 40) || (tag && tag < (ccap << 16)))
            return -1;
        if (m > 0 && (!f[0] || !f[3] || !f[5] || !f[7] || !f[8])) return -1;
        for (int q = 0; q < ONLINE_INS_FIELDS; ++q) a.f[t][q] = f[q];
        mmax = m > mmax ? m : mmax;
    }
    if (mmax == 0) return 0;
    online_insert_levels_k<<<dim3((unsigned)grid_for(mmax, 256), (unsigned)nlv), 256, 0, (hipStream_t)stream>>>(
        tok, nlv, a, count_pairs != 0);
    return (int)hipGetLastError();
}

// The queries pos[0..m) of nlv (1..8) levels in one launch: lv[t * 13 ...] = level t's k, ck, ccap, pt, pcap, rec, rw,
// qslot, tot, dist, cnt, nc, ci (host memory; as ng_online_query's arguments of the same names).
extern "C" int ng_online_query_levels(const u16* tok, const int* avail, const unsigned char* has_next, const int* pos,
                                      i64 m, int nlv, const i64* lv, void* stream) {
    if (nlv < 1 || nlv > ONLINE_MAXL || !lv) return -1;
    OQryArgs a{};
    for (int t = 0; t < nlv; ++t) {
        const i64* f = lv + (i64)t * ONLINE_QRY_FIELDS;
        if (f[0] < 1 || f[0] > MAXK || f[2] <= 0 || f[4] <= 0 || !f[1] || !f[3] || !f[5] ||
            (f[6] != OREC_TOP && f[6] != OREC_CNT))
            return -1;
        if (f[8] && (!f[9] || !f[10] || f[11] < 1 || f[12] < 0 || f[12] >= f[11])) return -1;
        for (int q = 0; q < ONLINE_QRY_FIELDS; ++q) a.f[t][q] = f[q];
    }
    if (m <= 0) return 0;
    online_query_levels_k<<<dim3((unsigned)grid_for(m, 256), (unsigned)nlv), 256, 0, (hipStream_t)stream>>>(
        tok, avail, has_next, pos, m, a);
    return (int)hipGetLastError();
}

// A step's distinct touched pairs of every level at once, uk[0..*n) (sorted tagged keys: level t's pair keys | t <<
// tshift; agg: their occurrences in the step), merged into their contexts' totals, distinct counts and, where the
// level keeps them, top-E lists; desc[t * 5 ...] describes level t (OLevel: the pair table, its capacity, the records,
// 1 if they hold top lists (OREC_TOP words) else 0 (OREC_CNT), flags; device memory), ntag levels. score: scratch
// [m]. add_counts: the pairs' counts
// grow here by agg (pairs inserted as needed; a full table sets the level's flags[0] bit 0), after inserts made with
// count_pairs 0; else the inserts counted them.
extern "C" int ng_online_top(const u64* uk, const i64* n, i64 m, const u32* agg, const i64* desc, int ntag, int tshift,
                             u64* score, int E, int add_counts, void* stream) {
    if (E < 1 || E > 8 || ntag < 1 || tshift < 17 || tshift > 63 || (tshift + 64 - __builtin_clzll((u64)ntag)) > 64)
        return -1;
    if (m <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    online_scores_k<<<grid_for(m, 256), 256, 0, st>>>(uk, agg, n, m, desc, tshift, add_counts != 0, score);
    const i64 wins = (m + WAVE - 1) / WAVE;
    online_top_k<<<(unsigned)(wins < 262144 ? wins : 262144), WAVE, 0, st>>>(uk, score, agg, n, m, desc, tshift, E);
    return (int)hipGetLastError();
}

extern "C" int ng_seg_scatter(const u64* src, u64 R, const i64* bases, const u32* ev_count, const u32* dpre, i64 nseg,
                              int shift, int nbits, u64* out, u64 cap, void* stream);

// A step's events ev[0..m) of every level at once (tagged pair keys as ng_online_insert_levels writes them with
// count_pairs 0: level t's pair keys | t << tshift, EMPTY skipped) merged into the levels' pair counts, totals,
// distinct counts and top-E lists, as sort_pairs + reduce_by_key + ng_online_top (add_counts 1) do, without sorting
// the events (om_merge_k). desc, ntag, tshift, E: as ng_online_top's. CUB-style two-phase temp storage (temp NULL:
// *temp_bytes set for m). -1 where the packed words cannot hold a pair's occurrences (m >= 2^cb - 1, cb = 64 - tshift
// - tag bits + 11): the caller then takes the sorted path.
extern "C" int ng_online_merge(void* temp, size_t* temp_bytes, const u64* ev, i64 m, const i64* desc, int ntag,
                               int tshift, int E, void* stream) {
    if (!temp_bytes || E < 1 || E > 8 || ntag < 1 || ntag > ONLINE_MAXL || m < 0 || m >= 0xFFFFFFFFll) return -1;
    const int tagbits = ntag > 1 ? 64 - __builtin_clzll((u64)(ntag - 1)) : 1;
    if (tshift < 16 + OM_BITS || tshift + tagbits > 64) return -1;
    const int cb = 64 - (tshift + tagbits - OM_BITS);
    if (cb < 2 || (u64)m >= (1ull << cb) - 1) return -1;
    const i64 nseg = (m + OM_CHUNK - 1) / OM_CHUNK;
    const i64 nh = (i64)OM_NB * (nseg > 0 ? nseg : 1);
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    const size_t b_ev = al((size_t)m * 8), b_hist = al((size_t)nh * 4), b_seg = al((size_t)(nseg + 1) * 4);
    const size_t need = b_ev + b_hist + b_seg + prim::scan_u32_temp_bytes(nh);
    if (!temp) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need || !ev || !desc) return -1;
    if (m == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    char* p = (char*)temp;
    u64* evb = (u64*)p;
    u32* hist = (u32*)(p + b_ev);
    u32* seg_n = (u32*)(p + b_ev + b_hist);
    void* stemp = p + b_ev + b_hist + b_seg;
    om_hist_k<<<(unsigned)(nseg < 16384 ? nseg : 16384), 1024, 0, st>>>(ev, m, nseg, hist, seg_n);
    int rc = (int)hipGetLastError();
    if (rc) return rc;
    if ((rc = prim::exclusive_scan_u32(hist, hist, nh, nullptr, stemp, st))) return rc;
    if ((rc = ng_seg_scatter(ev, OM_CHUNK, nullptr, seg_n, hist, nseg, 16, OM_BITS, evb, (u64)m, stream))) return rc;
    om_merge_k<<<OM_NB, OM_BLOCK, 0, st>>>(evb, hist, nseg, m, desc, ntag, tshift, cb, E);
    return (int)hipGetLastError();
}

extern "C" int ng_online_query(const u16* tok, const int* avail, const unsigned char* has_next, const int* pos, i64 m,
                               int k, const u64* ck, u64 ccap, const u64* pt, u64 pcap, const u32* rec, int rw,
                               int* qslot, u32* tot, u16* dist, u32* cnt, int nc, int ci, void* stream) {
    if (m <= 0) return 0;
    if (!rec || (rw != OREC_TOP && rw != OREC_CNT)) return -1;
    hipStream_t st = (hipStream_t)stream;
    OLEVELS(k, (online_query_k<K><<<grid_for(m, 256), 256, 0, st>>>(tok, avail, has_next, pos, m, k, ck, ccap, pt, pcap, rec, rw, qslot, tot, dist, cnt, nc, ci)));
    return (int)hipGetLastError();
}

// Hint rows of the queries at pos[0..m), slots deepest first: cell [n, S], next / weights [n, S, E], level [n, S]
// (may be NULL) at the query's position; slots with no row are left as they are (callers fill cell 0, level -1).
extern "C" int ng_online_rows(const int* pos, i64 m, int nlv, const i64* desc, int E, int S, short* cell, u16* next,
                              u16* weights, signed char* level, int* hinted, void* stream) {
    if (E < 1 || E > 8 || S < 1 || S > 255) return -1;
    if (m > 0)
        online_rows_k<<<grid_for(m, 256) < 1024 ? grid_for(m, 256) : 1024, 256, 0, (hipStream_t)stream>>>(
            pos, m, nlv, desc, E, S, cell, next, weights, level, hinted);
    return (int)hipGetLastError();
}
