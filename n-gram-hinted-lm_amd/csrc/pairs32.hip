// The 32-bit partitioned count: a level's (context id, next token) events counted with 4 bytes per event after the
// first pass, and each present context's record made in LDS without sorting its pairs (no counterpart in the
// reference's libraries: there a level's hits go through one atomic hash table and two radix sorts,
// old_records/gpu_val_stats.cu:340-434,529-644; the ranking follows exact_match/src/kgram.rs:357-368).
//
//   1. the emitting scan (ng_scan_emit with wbits = W = cb + 16, cb the context-id bits) writes each hit as
//      h = wmix(pair key, W) (part.h: a bijection of W-bit values) with a histogram of its top d1 bits;
//   2. ng_seg_scatter_narrow groups the events by those d1 bits (d1 = max(8, W - 32)) and keeps their low 32 bits;
//   3. ng_msd_pass sub-groups each of those buckets by the next d2 bits (tiles within a bucket, LDS-staged), giving
//      2^(d1 + d2) partitions = the top pbits = d1 + d2 bits of h, and each partition's start;
//   4. ng_part_count32 counts every partition in an LDS table of u32 keys (the h bits below the partition, unique
//      within it: 14336 slots in buckets of four, one 16-byte read per bucket), answers the partition's lookups and
//      writes each distinct pair, unhashed, as a packed word (pair key << (48 - cb) | count) with a histogram of the
//      words' top context bits;
//   5. ng_seg_scatter groups the words by those context bits (dc = min(11, cb));
//   6. ng_ctx_agg makes every context's record (total, pairs, top entries by count descending then token ascending)
//      from its bucket's words in LDS: counts and totals by LDS atomics, the top entries by a cascade of 64-bit
//      atomic maxima; every id of the bucket gets its pair count (0 for absent contexts).
// Per event: 8 bytes written by the scan, 8 read + 4 written (pass 2), 4 + 4 + 4 (pass 3: histogram, read, write),
// 4 read by the count; per distinct pair 8 written, 8 + 8 moved (pass 5) and 8 read at least once (pass 6, whose
// later rounds over a bucket read it from L2). Nothing here reads a device count on the host: grids are bounded by
// the capacities and blocks stop at the device-side totals; a wrapped total is raised by the host from the flags
// and the exact totals afterwards.
#include "part.h"
#include "prim.h"
#include "scatter.h"
#include "pairs32.h"

namespace {

#define MSD_TILE SS_CHUNK

// Buckets 2t and 2t + 1 (nb <= 2048) of a pass's digit groups are thread t's: bstart[b] = bucket b's first key (the
// first pass's digit offsets dpre[b * nseg], clamped to cap), tfirst[b] = its first tile of MSD_TILE keys;
// bstart[nb] = the total (*total, clamped), tfirst[nb] = the number of tiles.
__global__ void __launch_bounds__(1024) msd_tiles_k(const u32* __restrict__ dpre, i64 nseg, int nb,
                                                    const u64* __restrict__ total, u64 cap, i64* __restrict__ bstart,
                                                    u32* __restrict__ tfirst) {
    __shared__ u32 wt[1024 / WAVE];
    const int t = threadIdx.x, lane = lane_id(), w = t / WAVE;
    const u64 tot = *total < cap ? *total : cap;
    u64 a[2] = {0, 0};
    u32 nt[2] = {0, 0};
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * t + h;
        if (b >= nb) break;
        u64 x = dpre[(i64)b * nseg];
        u64 e = b + 1 < nb ? (u64)dpre[(i64)(b + 1) * nseg] : tot;
        x = x < cap ? x : cap;
        e = e < cap ? e : cap;
        e = e < x ? x : e;
        a[h] = x;
        nt[h] = (u32)((e - x + MSD_TILE - 1) / MSD_TILE);
        if (b == nb - 1) bstart[nb] = (i64)e;
    }
    const u32 mine = nt[0] + nt[1];
    u32 incl = mine;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    if (lane == WAVE - 1) wt[w] = incl;
    __syncthreads();
    u32 before = incl - mine;
    for (int i = 0; i < w; ++i) before += wt[i];
    for (int h = 0; h < 2; ++h) {
        const int b = 2 * t + h;
        if (b >= nb) break;
        bstart[b] = (i64)a[h];
        tfirst[b] = before;
        before += nt[h];
        if (b == nb - 1) tfirst[nb] = before;
    }
}

// Per tile (grid-stride) its digit counts, at hist[(tfirst[b] << nbits) + d * ntiles(b) + (tile - tfirst[b])].
template <typename K>
__global__ void __launch_bounds__(1024) msd_hist_k(const K* __restrict__ keys, const i64* __restrict__ bstart,
                                                   const u32* __restrict__ tfirst, int nb, int shift, int nbits,
                                                   i64 max_tiles, u32* __restrict__ hist) {
    __shared__ u32 h[SS_MAXB];
    const int t = threadIdx.x;
    const u32 B = 1u << nbits, mask = B - 1u;
    const i64 ntl = (i64)tfirst[nb] < max_tiles ? (i64)tfirst[nb] : max_tiles;
    constexpr int IT = MSD_TILE / 1024;
    for (i64 s = blockIdx.x; s < ntl; s += gridDim.x) {
        for (u32 d = t; d < B; d += 1024) h[d] = 0;
        __syncthreads();
        const int b = tile_bucket(tfirst, nb, (u32)s);
        const u64 off = (u64)bstart[b] + (u64)(s - tfirst[b]) * MSD_TILE;
        const u64 end = (u64)bstart[b + 1];
        const u32 n = end - off < (u64)MSD_TILE ? (u32)(end - off) : (u32)MSD_TILE;
        K k[IT];
#pragma unroll
        for (int j = 0; j < IT; ++j) {
            const u32 i = (u32)(j * 1024 + t);
            k[j] = i < n ? keys[off + i] : (K)0;
        }
#pragma unroll
        for (int j = 0; j < IT; ++j)
            if ((u32)(j * 1024 + t) < n) atomicAdd(&h[(u32)(k[j] >> shift) & mask], 1u);
        __syncthreads();
        const u32 nt = tfirst[b + 1] - tfirst[b];
        const u64 at = ((u64)tfirst[b] << nbits) + (u64)(s - tfirst[b]);
        for (u32 d = t; d < B; d += 1024) hist[at + (u64)d * nt] = h[d];
        __syncthreads();
    }
}

// start[p] for the 2^(nb_bits + nbits) partitions p = bucket << nbits | digit, start[P] = the total.
__global__ void msd_starts_k(const i64* __restrict__ bstart, const u32* __restrict__ tfirst, int nb, int nbits,
                             const u32* __restrict__ hscan, i64* __restrict__ start) {
    const i64 P = (i64)nb << nbits;
    const i64 p = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (p > P) return;
    if (p == P) {
        start[P] = bstart[nb];
        return;
    }
    const int b = (int)(p >> nbits);
    const u32 d = (u32)(p & ((1 << nbits) - 1));
    const u32 nt = tfirst[b + 1] - tfirst[b];
    start[p] = nt ? (i64)hscan[((u64)tfirst[b] << nbits) + (u64)d * nt] : bstart[b];
}

// Lookup j of query position i = pos[j] (pos NULL: i = j): kmix(ctx_of[i] << 16 | tgt[i], W, M) << (64 - W) for
// context ids in [lo, hi) (the partition digits then are its top bits, as the events'), else EMPTY (no such key: its
// low 64 - W bits are ones); value i.
__global__ void lookups_w_k(const int* __restrict__ ctx_of, const u16* __restrict__ tgt, const int* __restrict__ pos,
                            i64 n, const u64* __restrict__ n_dev, i64 lo, i64 hi, int W, int M, u64* __restrict__ qk,
                            u32* __restrict__ qv) {
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= n) return;
    if (n_dev && (u64)j >= *n_dev) {  // past a device-side count of pos's entries
        qk[j] = EMPTY;
        qv[j] = 0;
        return;
    }
    const i64 i = pos ? pos[j] : j;
    const i64 c = ctx_of[i];
    qk[j] = (c >= lo && c < hi) ? kmix(((u64)c << 16) | tgt[i], W, M) << (64 - W) : EMPTY;
    qv[j] = (u32)i;
}

// The positions i < n with v[i] > 0, in order: SEL_ITEMS consecutive positions per thread, a block of 256 threads
// per 256 * SEL_ITEMS. sel_count_k counts each block's; sel_write_k writes them from the blocks' exclusive offsets
// (at most cap of them: out holds cap).
#define SEL_ITEMS 16
__global__ void __launch_bounds__(256) sel_count_k(const int* __restrict__ v, i64 n, u32* __restrict__ cnt) {
    __shared__ u32 part[256 / WAVE];
    const i64 a = (blockIdx.x * (i64)256 + threadIdx.x) * SEL_ITEMS;
    u32 c = 0;
#pragma unroll
    for (int j = 0; j < SEL_ITEMS; ++j) c += (a + j < n && v[a + j] > 0) ? 1u : 0u;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += (u32)__shfl_down((int)c, d, WAVE);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) cnt[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

__global__ void __launch_bounds__(256) sel_write_k(const int* __restrict__ v, i64 n, const u32* __restrict__ off,
                                                   int* __restrict__ out, i64 cap) {
    __shared__ u32 wt[256 / WAVE];
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const i64 a = (blockIdx.x * (i64)256 + threadIdx.x) * SEL_ITEMS;
    u32 bits = 0;
#pragma unroll
    for (int j = 0; j < SEL_ITEMS; ++j) bits |= (a + j < n && v[a + j] > 0) ? 1u << j : 0u;
    const u32 c = (u32)__popc(bits);
    u32 incl = c;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    if (lane == WAVE - 1) wt[w] = incl;
    __syncthreads();
    u64 at = (u64)off[blockIdx.x] + incl - c;
    for (int i = 0; i < w; ++i) at += wt[i];
    while (bits) {
        const int j = __ffs(bits) - 1;
        bits &= bits - 1;
        if (at < (u64)cap) out[at] = (int)(a + j);
        ++at;
    }
}


// The runs mode's table: run s (of 2^gbits) of partition p = b << rbits | j (bucket b of the first pass, 2^rbits
// partitions a bucket) at entry ((b << gbits) + s) << rbits | j, so that a group's runs (one per partition of its
// bucket) lie side by side: start | end << 32 (word indexes below 2^32).
__device__ __forceinline__ i64 run_at(i64 p, int s, int gbits, int rbits) {
    return ((((p >> rbits) << gbits) + s) << rbits) | (p & ((1ll << rbits) - 1));
}

// Block b counts the partitions it owns (part_owner: about equal events per block) in turn. Events: u32, a
// partition's key = its low lbits = W - pbits bits (h = p << lbits | key). A round of P32_ITEMS events per thread:
// the lanes holding a wave's first key add once for all of them (a hot pair would serialize the LDS atomics); every
// item's home bucket is read before any is used, an item whose key is there adds to its count, and the others are
// inserted (a compare-and-swap on the bucket's first free slot), each new slot appended to the partition's slot list.
// The output pass walks the list only (not the whole table): its distinct pairs (at most its events) go to
// out_k[start[p0] ...] as packed words, segment b = (seg_base[b], seg_cnt[b]); dhist[d * G + b] the block's words per
// dbits-bit digit at dshift. Lookups: qk (sorted like the events: wmix keys << (64 - W), or EMPTY), qv their query
// positions, qstart their partitions' bounds: qcnt[qv[j]] = the pair's count or 0. A partition reaching `limit`
// distinct pairs (at most P32_LIMIT) sets flags[0] bit 0; its count may be incomplete.
__global__ void __launch_bounds__(P32_BLOCK) count32_k(const u32* __restrict__ ev, const i64* __restrict__ start,
                                                      i64 P, int pbits, int W, int M, const u64* __restrict__ qk,
                                                      const u32* __restrict__ qv, const i64* __restrict__ qstart,
                                                      u64* __restrict__ out_k, int cb, u64* esc_k, u32* esc_c,
                                                      u64 esc_cap, u32* __restrict__ seg_cnt,
                                                      i64* __restrict__ seg_base, u32* __restrict__ qcnt,
                                                      u32* __restrict__ dhist, int dshift, int dbits, u32 limit,
                                                      u32* flags, u64* __restrict__ slab, u64* __restrict__ runs,
                                                      int gbits, int gshift, int rbits, i64 live_np, u64* n_words) {
    __shared__ __align__(16) u32 tk[P32_SLOTS];
    __shared__ u32 tc[P32_SLOTS];
    __shared__ u16 list[P32_SLOTS];
    __shared__ u32 dh[SS_MAXB];
    __shared__ u32 nocc;  // the partition's distinct pairs so far = the list's length
    const int t = threadIdx.x, lane = lane_id();
    const int lbits = W - pbits;
    const u32 lmask = (1u << lbits) - 1u;
    const i64 n_ev = start[P], G = gridDim.x;
    const i64 p0 = part_first(start, P, n_ev, G, blockIdx.x), p1 = part_first(start, P, n_ev, G, blockIdx.x + 1);
    const int nd = runs ? 0 : 1 << dbits;  // with runs: no words' histogram
    if (p0 >= p1) {
        if (t == 0) {
            seg_cnt[blockIdx.x] = 0;
            seg_base[blockIdx.x] = 0;
        }
        for (int d = t; d < nd; d += P32_BLOCK) dhist[(i64)d * G + blockIdx.x] = 0;
        return;
    }
    const i64 out_base = start[p0];
    u32 cur = 0;  // the block's words so far (block-uniform)
    if (t == 0) nocc = 0;
    for (int d = t; d < nd; d += P32_BLOCK) dh[d] = 0;
    for (int j = t; j < P32_SLOTS; j += P32_BLOCK) {
        tk[j] = EMPTY32;
        tc[j] = 0;
    }
    __syncthreads();
    constexpr i64 ROUND = (i64)P32_BLOCK * P32_ITEMS;
    auto load_round = [&](u32 (&dst)[P32_ITEMS], i64 i0, i64 end) {
#pragma unroll
        for (int r = 0; r < P32_ITEMS; ++r) {
            const i64 i = i0 + (i64)r * P32_BLOCK + t;
            dst[r] = i < end ? (ev[i] & lmask) : EMPTY32;
        }
    };
    u32 ahead[P32_ITEMS];
    i64 ahead_of = -1;
    const u64 esc = (1ull << (48 - cb)) - 1;
    const i64 e_end = start[p1];  // the end of the block's events
    for (i64 p = p0; p < p1; ++p) {
        const i64 a = start[p], b = start[p + 1], qa = qstart[p], qb = qstart[p + 1];
        if (a == e_end) {
            // this partition and the block's later ones hold no events (the trailing partitions of a level whose
            // context ids fill only part of their bit range, all of them the last block's): no words, and their
            // lookups' counts stay 0; their runs and slabs, empty, are written at once where they may be read (below
            // live_np)
            const i64 pe = p1 < live_np ? p1 : live_np;
            if (runs) {
                const u64 base = (u64)(out_base + (i64)cur);
                for (i64 x = t; x < (pe - p) << gbits; x += P32_BLOCK) {
                    const i64 q = p + (x >> gbits);
                    runs[run_at(q, (int)(x & ((1 << gbits) - 1)), gbits, rbits)] = base | (base << 32);
                }
            }
            if (slab)
                for (i64 x = t; x < (pe - p) * P32_SLOTS; x += P32_BLOCK) slab[(u64)p * P32_SLOTS + x] = EMPTY32;
            break;
        }
        const bool has_q = qa + t < qb;
        u64 lk = EMPTY;
        u32 lv = 0;
        if (has_q) {
            lk = qk[qa + t];
            lv = qv[qa + t];
        }
        if (ahead_of != p && a < b) load_round(ahead, a, b);
        for (i64 i0 = a; i0 < b; i0 += ROUND) {
            u32 key[P32_ITEMS], add[P32_ITEMS];
#pragma unroll
            for (int r = 0; r < P32_ITEMS; ++r) key[r] = ahead[r];
            if (i0 + ROUND < b) {
                load_round(ahead, i0 + ROUND, b);
                ahead_of = p;
            } else if (p + 1 < p1) {
                load_round(ahead, b, start[p + 2]);
                ahead_of = p + 1;
            }
            // the lanes holding the wave's first key add once (a hot pair would serialize the LDS atomics); the
            // item's add is 0 where another lane adds for it
#pragma unroll
            for (int r = 0; r < P32_ITEMS; ++r) {
                const bool valid = key[r] != EMPTY32;
                const u64 vb = __ballot(valid);
                add[r] = valid ? 1u : 0u;
                if (vb) {
                    const int ld = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)vb) - 1);
                    const u32 k0 = (u32)__builtin_amdgcn_readlane((int)key[r], ld);
                    const bool same = valid && key[r] == k0;
                    const u64 m = __ballot(same);
                    if (same) add[r] = lane == ld ? (u32)__popcll(m) : 0u;
                }
            }
            // in two halves (register pressure): every item's home bucket read before any is used; an item whose
            // key is there adds to its count; the others try their bucket's first free slot by compare-and-swap, all
            // of a half's swaps issued before any result is used (a key already put there by another lane counts as
            // found); the few whose swap lost to another key, or whose bucket was full, walk on one item at a time;
            // the half's new slots join the list with one LDS atomic per wave
            constexpr int HI = P32_ITEMS / 2;
#pragma unroll
            for (int h = 0; h < P32_ITEMS; h += HI) {
                uint4 q[HI];
                u32 bk[HI];
#pragma unroll
                for (int r = 0; r < HI; ++r) {
                    bk[r] = add[h + r] ? p32_bucket(key[h + r]) : 0u;
                    if (add[h + r]) q[r] = *(const uint4*)(tk + 4 * bk[r]);
                }
                bool pend = false;
#pragma unroll
                for (int r = 0; r < HI; ++r) {
                    const int s = add[h + r] ? p32_in(q[r], bk[r], key[h + r]) : -1;
                    if (s >= 0) {
                        atomicAdd(&tc[s], add[h + r]);
                        add[h + r] = 0;
                    }
                    pend |= add[h + r] != 0;
                }
                if (!__ballot(pend)) continue;
                if (__builtin_amdgcn_readfirstlane(nocc) >= limit) {  // overfull: counted again with a bit more
                    if (lane == 0) atomicOr(&flags[0], 1u);
                    continue;
                }
                int slot[HI];
                u32 prev[HI];
#pragma unroll
                for (int r = 0; r < HI; ++r) {
                    slot[r] = -1;
                    prev[r] = 0;
                    if (add[h + r]) {
                        const uint4 qq = q[r];
                        const int e = qq.x == EMPTY32 ? 0 : qq.y == EMPTY32 ? 1 : qq.z == EMPTY32 ? 2 : qq.w == EMPTY32 ? 3 : -1;
                        if (e >= 0) {
                            slot[r] = 4 * (int)bk[r] + e;
                            prev[r] = atomicCAS(&tk[slot[r]], EMPTY32, key[h + r]);
                        }
                    }
                }
                bool fresh[HI];
#pragma unroll
                for (int r = 0; r < HI; ++r) {
                    fresh[r] = false;
                    if (!add[h + r]) continue;
                    if (slot[r] >= 0 && prev[r] == EMPTY32) {
                        fresh[r] = true;
                    } else if (slot[r] < 0 || prev[r] != key[h + r]) {  // lost to another key, or a full bucket
                        const uint4 qq = *(const uint4*)(tk + 4 * bk[r]);
                        bool f = false;
                        slot[r] = p32_insert(tk, key[h + r], bk[r], qq, &f);
                        fresh[r] = f;
                    }
                    atomicAdd(&tc[slot[r]], add[h + r]);
                }
                u64 fb[HI];
                u32 nf = 0;
#pragma unroll
                for (int r = 0; r < HI; ++r) {
                    fb[r] = __ballot(fresh[r]);
                    nf += (u32)__popcll(fb[r]);
                }
                if (nf) {  // wave-uniform
                    u32 at = 0;
                    if (lane == 0) at = atomicAdd(&nocc, nf);
                    at = (u32)__shfl((int)at, 0, WAVE);
#pragma unroll
                    for (int r = 0; r < HI; ++r) {
                        if (fresh[r]) list[at + (u32)__popcll(fb[r] & lanemask_lt())] = (u16)slot[r];
                        at += (u32)__popcll(fb[r]);
                    }
                }
            }
        }
        lds_barrier();
        if (qb > qa) {  // block-uniform
            auto lkey = [&](u64 qq) { return (u32)((qq >> (64 - W)) & lmask); };
            // an EMPTY lookup (no context, or past the lookups' count) writes nothing: qcnt starts at zero
            if (has_q && lk != EMPTY) qcnt[lv] = p32_find(tk, tc, lkey(lk));
            for (i64 j = qa + P32_BLOCK + t; j < qb; j += P32_BLOCK) {
                const u64 qq = qk[j];
                if (qq != EMPTY) qcnt[qv[j]] = p32_find(tk, tc, lkey(qq));
            }
        }
        const u32 nl = nocc;
        // a wave checks the limit once per half-round, so a partition can pass it by up to a round's new keys
        // without a skipped insert: it is declared overfull all the same
        if (t == 0 && nl >= limit) atomicOr(&flags[0], 1u);
        lds_barrier();  // every lookup has probed and nocc is read before the output pass empties the slots
        if (slab) {  // the table as it stands, slot s = count << 32 | key (empty slots: 0 << 32 | EMPTY32)
            u64* sp = slab + (u64)p * P32_SLOTS;
            for (int j = t; j < P32_SLOTS; j += P32_BLOCK) sp[j] = ((u64)tc[j] << 32) | tk[j];
            lds_barrier();  // read before the output pass empties the slots
        }
        if (runs && p < live_np) {
            // the partition's words grouped by the gbits-bit digit (pair key >> gshift) of their context ids (an LDS
            // count, a scan by wave 0, then a slot per word from the group's cursor), group s's run of words at
            // [runs[p * (2^gbits + 1) + s], runs[p * (2^gbits + 1) + s + 1]) of out_k
            const u32 ng = 1u << gbits, gm = ng - 1u;
            if (t < (int)ng) dh[t] = 0;
            lds_barrier();
            for (u32 i = t; i < nl; i += P32_BLOCK) {
                const u64 pk = unkmix(((u64)p << lbits) | tk[list[i]], W, M);
                atomicAdd(&dh[(u32)(pk >> gshift) & gm], 1u);
            }
            lds_barrier();
            if (t < WAVE) {
                const u32 c = t < (int)ng ? dh[t] : 0u;
                u32 incl = c;
#pragma unroll
                for (int d = 1; d < WAVE; d <<= 1) {
                    const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
                    if (lane >= d) incl += o;
                }
                const u64 base = (u64)(out_base + (i64)cur);
                if (t < (int)ng) {
                    runs[run_at(p, t, gbits, rbits)] = (base + incl - c) | ((base + incl) << 32);
                    dh[t] = incl - c;
                }
            }
            lds_barrier();
            for (u32 i = t; i < nl; i += P32_BLOCK) {
                const int j = list[i];
                const u32 key = tk[j], n = tc[j];
                tk[j] = EMPTY32;
                tc[j] = 0;
                const u64 pk = unkmix(((u64)p << lbits) | key, W, M);
                const u64 word = (pk << (48 - cb)) | ((u64)n < esc ? (u64)n : esc);
                const u32 at = atomicAdd(&dh[(u32)(pk >> gshift) & gm], 1u);
                out_k[(u64)out_base + cur + at] = word;
                if ((u64)n >= esc) esc_put(esc_k, esc_c, esc_cap, pk, n, flags);
            }
        } else {
            for (u32 i = t; i < nl; i += P32_BLOCK) {
                const int j = list[i];
                const u32 key = tk[j], n = tc[j];
                tk[j] = EMPTY32;
                tc[j] = 0;
                const u64 pk = unkmix(((u64)p << lbits) | key, W, M);
                const u64 word = (pk << (48 - cb)) | ((u64)n < esc ? (u64)n : esc);
                out_k[(u64)out_base + cur + i] = word;
                if ((u64)n >= esc) esc_put(esc_k, esc_c, esc_cap, pk, n, flags);
                if (nd) atomicAdd(&dh[(u32)(word >> dshift) & (u32)(nd - 1)], 1u);  // none in runs mode
            }
        }
        cur += nl;
        if (t == 0) nocc = 0;
        lds_barrier();  // the slots are empty again (the output stores need not have completed)
    }
    if (t == 0) {
        seg_cnt[blockIdx.x] = cur;
        seg_base[blockIdx.x] = out_base;
        if (n_words && cur) atomicAdd((unsigned long long*)n_words, (unsigned long long)cur);
    }
    for (int d = t; d < nd; d += P32_BLOCK) dhist[(i64)d * G + blockIdx.x] = dh[d];
}

// Per context from packed words grouped by context: partition q (words [start[q], start[q + 1])) holds the
// contexts of ids [q << ibits, (q + 1) << ibits), 2^ibits <= AGG_IDS_FOR(KT). A block takes partitions q, q + grid,
// ... in turn and streams each one's words once, accumulating per id its total, its pairs and its top KT scores
// (count << 16 | 65535 - token) in LDS. The top scores come from a cascade of atomic maxima: a score displaced from
// (or kept out of) slot r goes on to slot r + 1, so slot r ends with the r-th largest; a score not above slot
// KT - 1's current value (which only grows, and below which KT larger scores already exist) is not inserted. Then
// every id of the partition below n_ids gets dist[c] = its pairs and, if present, its record (CtxRecord<KT>,
// first-word index 0); with `deep`, every context of more than deep_min pairs is appended to deep (*deep_n counts
// them). flags[0] bit 2: a total reached 2^32.
#define AGG_BLOCK 1024
#define AGG_IDS 2048
// the ids of a partition at most for top KT: 1024 for KT 8, so that its LDS (72 KB) lets two blocks share a CU
#define AGG_IDS_FOR(KT) ((KT) >= 8 ? AGG_IDS / 2 : AGG_IDS)
#define AGG_RUN_REGS 4  // ctx_agg_runs_k: the runs a lane holds (at most 64 times this per group)

// One round's words into a group's LDS sums (lo: the group's first id, nid its ids; vb: the wave's valid lanes).
template <int KT>
__device__ __forceinline__ void agg_round(u64 word, bool valid, u64 vb, i64 lo, int nid, int cb,
                                          const u64* __restrict__ esc_k, const u32* __restrict__ esc_c, u64 esc_cap,
                                          u32* s_tot, u32* s_dist, u64* s_top, u32* flags) {
    const int lane = lane_id(), sh = 64 - cb, csh = 48 - cb;
    const u64 esc = (1ull << csh) - 1;
    const int lid = (int)((i64)(word >> sh) - lo) & (nid - 1);
    u32 n = 0;
    if (valid) {
        const u64 n64 = word & esc;
        n = n64 < esc ? (u32)n64 : esc_get(esc_k, esc_c, esc_cap, word >> csh);
    }
    // the lanes of the wave's first context add its total and pairs once when many share it (a context with many
    // pairs would serialize the LDS atomics on its two counters)
    const int ld = __builtin_amdgcn_readfirstlane(__ffsll((unsigned long long)vb) - 1);
    const int l0 = __builtin_amdgcn_readlane(lid, ld);
    const bool same = valid && lid == l0;
    const u64 m = __ballot(same);
    bool own = valid;
    if (__popcll(m) > 4) {  // wave-uniform
        u64 sm = same ? n : 0;
#pragma unroll
        for (int d = WAVE / 2; d > 0; d >>= 1) sm += shfl_down_u64(sm, d);
        sm = bcast_u64(sm, 0);
        if (lane == ld) {
            const u32 old = atomicAdd(&s_tot[l0], (u32)sm);
            if ((sm >> 32) || old + (u32)sm < old) atomicOr(&flags[0], 4u);
            atomicAdd(&s_dist[l0], (u32)__popcll(m));
        }
        own = valid && !same;
    }
    if (own) {
        const u32 old = atomicAdd(&s_tot[lid], n);
        if (old + n < old) atomicOr(&flags[0], 4u);
        atomicAdd(&s_dist[lid], 1u);
    }
    if (valid) {
        u64 v = rank_score(word >> csh, n);
        u64* tp = &s_top[lid * KT];
        if (v > __hip_atomic_load(&tp[KT - 1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) {
#pragma unroll
            for (int r = 0; r < KT; ++r) {
                if (!v) break;
                const u64 o = atomicMax((unsigned long long*)&tp[r], (unsigned long long)v);
                v = o < v ? o : v;
            }
        }
    }
}

// A group's ids below n_ids out of LDS: dist, records of the present ones, the deep list; returns this thread's
// present contexts.
template <int KT>
__device__ __forceinline__ u32 agg_flush(i64 lo, int nid, i64 n_ids, const u32* s_tot, const u32* s_dist,
                                         const u64* s_top, u32* __restrict__ rec, u32* __restrict__ dist,
                                         u32 deep_min, i64* __restrict__ deep, u64 deep_cap, u64* deep_n) {
    u32 mine = 0;
    const int nl = n_ids - lo < nid ? (int)(n_ids - lo) : nid;
    for (int l = threadIdx.x; l < nl; l += AGG_BLOCK) {
        const i64 c = lo + l;
        const u32 d = s_dist[l];
        if (dist) dist[c] = d;
        if (d) {
            ++mine;
            u64 top[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) top[r] = s_top[l * KT + r];
            store_record<KT>(rec, (u64)c, s_tot[l], d, top, 0);
            if (deep && d > deep_min) {
                const u64 at = atomicAdd((unsigned long long*)deep_n, 1ull);
                if (at < deep_cap) deep[at] = c;
            }
        }
    }
    return mine;
}

template <int KT>
__device__ __forceinline__ void agg_clear(int nid, u32* s_tot, u32* s_dist, u64* s_top) {
    for (int l = threadIdx.x; l < nid; l += AGG_BLOCK) {
        s_tot[l] = 0;
        s_dist[l] = 0;
    }
    for (int l = threadIdx.x; l < nid * KT; l += AGG_BLOCK) s_top[l] = 0;
}

// *present += the block's present contexts (one atomic per wave).
__device__ __forceinline__ void agg_present(u32 mine, u64* present) {
    u32 sm = mine;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) sm += (u32)__shfl_down((int)sm, d, WAVE);
    if (lane_id() == 0 && sm) atomicAdd((unsigned long long*)present, (unsigned long long)sm);
}

// Two blocks share a compute unit where the LDS allows (KT <= 4: 80 KB each): 8 waves per SIMD, so at most 96
// scalar registers a wave (amdgpu_waves_per_eu), which the kernel's arguments and walk state would otherwise exceed.
template <int KT>
__global__ void __launch_bounds__(AGG_BLOCK) __attribute__((amdgpu_waves_per_eu(8))) ctx_agg_k(const u64* __restrict__ w, const i64* __restrict__ start,
                                                       i64 P, int ibits, int cb, i64 n_ids,
                                                       const u64* __restrict__ esc_k, const u32* __restrict__ esc_c,
                                                       u64 esc_cap, u32* __restrict__ rec, u32* __restrict__ dist,
                                                       u32* flags, u32 deep_min, i64* __restrict__ deep,
                                                       u64 deep_cap, u64* deep_n, u64* present) {
    __shared__ u32 s_tot[AGG_IDS_FOR(KT)], s_dist[AGG_IDS_FOR(KT)];
    __shared__ u64 s_top[AGG_IDS_FOR(KT) * KT];
    const int t = threadIdx.x;
    const int nid = 1 << ibits;
    // a block walks its partitions with the next round's words (this partition's, else the next partition's first)
    // and the next partition's bounds loaded ahead, so their latency hides behind the LDS work
    i64 q = blockIdx.x;
    if (q >= P) return;
    u32 mine = 0;  // this thread's present contexts, summed over the block at the end
    i64 wa = start[q], we = start[q + 1];
    i64 nwa = 0, nwe = 0;
    if (q + gridDim.x < P) {
        nwa = start[q + gridDim.x];
        nwe = start[q + gridDim.x + 1];
    }
    // loads are unconditional (an index past its range reads word 0, which always exists, and is not used), so the
    // compiler waits for each round's words only, not for the prefetch behind them
    u64 ahead = w[wa + t < we ? wa + t : 0];
    for (;;) {
        const i64 lo = q << ibits;
        if (lo >= n_ids) break;  // partitions ascend with q
        const bool more = q + gridDim.x < P;
        agg_clear<KT>(nid, s_tot, s_dist, s_top);
        lds_barrier();
        if (wa >= we) ahead = w[more && nwa + t < nwe ? nwa + t : 0];  // an empty partition: the next one's words
        for (i64 i0 = wa; i0 < we; i0 += AGG_BLOCK) {  // the same rounds for every wave
            const i64 i = i0 + t;
            const bool valid = i < we;
            const u64 word = valid ? ahead : 0;
            const i64 j = i0 + AGG_BLOCK < we ? (i0 + AGG_BLOCK + t < we ? i0 + AGG_BLOCK + t : 0)
                                               : (more && nwa + t < nwe ? nwa + t : 0);
            ahead = w[j];
            const u64 vb = __ballot(valid);
            if (!vb) continue;
            agg_round<KT>(word, valid, vb, lo, nid, cb, esc_k, esc_c, esc_cap, s_tot, s_dist, s_top, flags);
        }
        lds_barrier();
        mine += agg_flush<KT>(lo, nid, n_ids, s_tot, s_dist, s_top, rec, dist, deep_min, deep, deep_cap, deep_n);
        lds_barrier();  // the LDS is read before the next partition clears it
        if (!more) break;
        q += gridDim.x;
        wa = nwa;
        we = nwe;
        if (q + gridDim.x < P) {
            nwa = start[q + gridDim.x];
            nwe = start[q + gridDim.x + 1];
        }
    }
    if (present) agg_present(mine, present);
}

// ctx_agg_k over ng_part_count32's words left in runs (its `runs` mode, events keyed by kmix(pair key, W, W - d1)):
// group g = b << gbits | s (bucket b of the first pass's d1 bits, sub-group s of the gbits context-id bits below
// them) holds the ids [g << ibits, (g + 1) << ibits), and its words are run s of each of the bucket's 2^d2 <= 256
// partitions b << d2 | j, whose bounds are runs[g << d2 | j] (run_at's layout). A block takes groups g, g + grid, ...
// and streams a group's words as one sequence: every wave holds the group's runs in its lanes (lane l: runs l,
// 64 + l, 128 + l and 192 + l, their starts and the exclusive scan of the lengths; no LDS, so that two blocks still
// share a compute unit). A wave's 64 consecutive words span few runs: the run of its first word is the count of runs
// starting at or before it, and the runs starting inside its window are walked with lane reads. The next round's
// words are loaded ahead, as ctx_agg_k's. Outputs as ctx_agg_k's, without the deep list.
template <int KT>
__global__ void __launch_bounds__(AGG_BLOCK) __attribute__((amdgpu_waves_per_eu(8))) ctx_agg_runs_k(const u64* __restrict__ w, const u64* __restrict__ runs,
                                                       i64 NG, int d2, int gbits, int ibits, int cb, i64 n_ids,
                                                       const u64* __restrict__ esc_k, const u32* __restrict__ esc_c,
                                                       u64 esc_cap, u32* __restrict__ rec, u32* __restrict__ dist,
                                                       u32* flags, u64* present) {
    __shared__ u32 s_tot[AGG_IDS_FOR(KT)], s_dist[AGG_IDS_FOR(KT)];
    __shared__ u64 s_top[AGG_IDS_FOR(KT) * KT];
    const int t = threadIdx.x, lane = lane_id();
    const u32 wbase = (u32)(t & ~(WAVE - 1));  // the wave's first thread
    const int nid = 1 << ibits, R = 1 << d2;
    u32 mine = 0;
    for (i64 g = blockIdx.x; g < NG; g += gridDim.x) {
        const i64 lo = g << ibits;
        if (lo >= n_ids) break;  // groups ascend with g
        agg_clear<KT>(nid, s_tot, s_dist, s_top);
        // word indexes are below 2^32 (the count's capacity)
        const u64* rp = runs + (g << d2);  // the group's runs, side by side
        u32 rlo[AGG_RUN_REGS], rpre[AGG_RUN_REGS], tot = 0;
#pragma unroll
        for (int h = 0; h < AGG_RUN_REGS; ++h) {
            const int j = h * WAVE + lane;
            u32 len = 0;
            rlo[h] = 0;
            if (j < R) {
                const u64 r = rp[j];
                rlo[h] = (u32)r;
                len = (u32)(r >> 32) - (u32)r;
            }
            u32 incl = len;
#pragma unroll
            for (int d = 1; d < WAVE; d <<= 1) {
                const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
                if (lane >= d) incl += o;
            }
            rpre[h] = tot + incl - len;  // runs past R: the total, never at or below a word
            tot += (u32)__builtin_amdgcn_readlane((int)incl, WAVE - 1);
        }
        lds_barrier();
        // the index in w of word base + lane (base wave-uniform; meaningful below tot): its run is the last whose
        // scan is at or below it (a run of length 0 shares its start with the next, which the walk then takes)
        auto at = [&](u32 base) -> u32 {
            const u32 i = base + (u32)lane, last = base + (WAVE - 1);
            int j = -1;  // wave-uniform
#pragma unroll
            for (int h = 0; h < AGG_RUN_REGS; ++h) j += __popcll(__ballot(rpre[h] <= base));
            u32 plo = 0, ppre = 0;
            for (; j < R; ++j) {
                u32 pj = 0, lj = 0;
#pragma unroll
                for (int h = 0; h < AGG_RUN_REGS; ++h)
                    if ((j >> 6) == h) {  // wave-uniform
                        pj = (u32)__builtin_amdgcn_readlane((int)rpre[h], j & (WAVE - 1));
                        lj = (u32)__builtin_amdgcn_readlane((int)rlo[h], j & (WAVE - 1));
                    }
                if (pj > last) break;
                if (i >= pj) {
                    plo = lj;
                    ppre = pj;
                }
            }
            return plo + (i - ppre);
        };
        if (tot) {  // wave-uniform
            const u32 a0 = at(wbase);
            u64 ahead = w[(u32)t < tot ? a0 : 0u];
            for (u32 i0 = 0; i0 < tot; i0 += AGG_BLOCK) {  // the same rounds for every wave
                const u32 i = i0 + (u32)t;
                const bool valid = i < tot;
                const u64 word = valid ? ahead : 0;
                const u32 nx = i + AGG_BLOCK;
                const u32 ad = at(i0 + AGG_BLOCK + wbase);
                ahead = w[nx < tot ? ad : 0u];  // unconditional: word 0 always exists
                const u64 vb = __ballot(valid);
                if (!vb) continue;
                agg_round<KT>(word, valid, vb, lo, nid, cb, esc_k, esc_c, esc_cap, s_tot, s_dist, s_top, flags);
            }
        }
        lds_barrier();
        mine += agg_flush<KT>(lo, nid, n_ids, s_tot, s_dist, s_top, rec, dist, 0, nullptr, 0, nullptr);
        lds_barrier();  // the LDS is read before the next group clears it
    }
    if (present) agg_present(mine, present);
}

static inline int grid_cap(i64 n, int cap) { return n < 1 ? 1 : n > cap ? cap : (int)n; }

static inline i64 msd_max_tiles(u64 cap, int nb) { return (i64)((cap + MSD_TILE - 1) / MSD_TILE) + nb; }

static inline size_t al256(size_t x) { return (x + 255) & ~(size_t)255; }

template <typename K, typename KO = K>
static int msd_pass(void* temp, size_t* temp_bytes, const K* keys, const u32* dpre, i64 nseg, int nb_bits,
                    const u64* total, u64 cap, int shift, int nbits, KO* out, i64* start, hipStream_t st) {
    if (temp_bytes == nullptr || nb_bits < 1 || nb_bits > 11 || nbits < 0 || nbits > 11 || shift < 0 ||
        shift + nbits > (int)(8 * sizeof(K)) || nseg <= 0 || cap > 0xFFFFFFFFull)
        return -1;
    if (sizeof(KO) < sizeof(K) && shift > 32) return -1;  // narrowing keeps the low 32 bits: the bits below the digit
    const int nb = 1 << nb_bits;
    const i64 mt = msd_max_tiles(cap, nb);
    const i64 nh = nbits ? mt << nbits : 0;
    const size_t b0 = al256((size_t)(nb + 1) * 8), b1 = al256((size_t)(nb + 1) * 4), b2 = al256((size_t)nh * 4);
    const size_t need = b0 + b1 + b2 + (nbits ? prim::scan_u32_temp_bytes(nh) : 0);
    if (temp == nullptr) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need) return -1;
    char* tp = (char*)temp;
    u32* tfirst = (u32*)(tp + b0);
    if (nbits == 0) {  // the buckets are the partitions
        msd_tiles_k<<<1, 1024, 0, st>>>(dpre, nseg, nb, total, cap, start, tfirst);
        return (int)hipGetLastError();
    }
    i64* bstart = (i64*)tp;
    u32* hist = (u32*)(tp + b0 + b1);
    void* stemp = tp + b0 + b1 + b2;
    msd_tiles_k<<<1, 1024, 0, st>>>(dpre, nseg, nb, total, cap, bstart, tfirst);
    const int g = grid_cap(mt, 4096);
    msd_hist_k<K><<<g, 1024, 0, st>>>(keys, bstart, tfirst, nb, shift, nbits, mt, hist);
    int e = prim::exclusive_scan_u32(hist, hist, nh, nullptr, stemp, st);
    if (e) return e;
    const TileSegs sg{bstart, tfirst, hist, nb, nbits, mt};
    if (nbits <= 8)
        scatter_k<256, K, KO><<<g, SS_BLOCK, 0, st>>>(keys, sg, shift, nbits, out, cap);
    else
        scatter_k<SS_MAXB, K, KO><<<g, SS_BLOCK, 0, st>>>(keys, sg, shift, nbits, out, cap);
    const i64 P = (i64)nb << nbits;
    msd_starts_k<<<grid_for(P + 1, 256), 256, 0, st>>>(bstart, tfirst, nb, nbits, hist, start);
    return (int)hipGetLastError();
}

}  // namespace

// A most-significant-digit-first second pass (see the file's head): keys (at most cap of them, cap < 2^32) grouped
// into the nb = 2^nb_bits buckets of a first pass's digits (bucket b from dpre[b * nseg], the last up to *total, a
// device-side count; 1 <= nb_bits <= 11) sub-grouped within each bucket by the nbits-bit digit (key >> shift) &
// (2^nbits - 1) (0 <= nbits <= 11) into out (cap keys); start (i64[2^(nb_bits + nbits) + 1]) the partitions'
// starts, partition p = bucket << nbits | digit (nbits 0: the buckets' starts, keys and out unused). CUB-style
// two-phase temp storage (temp NULL: *temp_bytes set). No host read of the total. ng_msd_pass: u32 keys (the 32-bit
// count's events); ng_msd_pass64: u64 keys (its packed words, by context).
extern "C" int ng_msd_pass(void* temp, size_t* temp_bytes, const u32* keys, const u32* dpre, i64 nseg, int nb_bits,
                           const u64* total, u64 cap, int shift, int nbits, u32* out, i64* start, void* stream) {
    return msd_pass<u32>(temp, temp_bytes, keys, dpre, nseg, nb_bits, total, cap, shift, nbits, out, start,
                         (hipStream_t)stream);
}

extern "C" int ng_msd_pass64(void* temp, size_t* temp_bytes, const u64* keys, const u32* dpre, i64 nseg,
                             int nb_bits, const u64* total, u64 cap, int shift, int nbits, u64* out, i64* start,
                             void* stream) {
    return msd_pass<u64>(temp, temp_bytes, keys, dpre, nseg, nb_bits, total, cap, shift, nbits, out, start,
                         (hipStream_t)stream);
}

// ng_msd_pass over u64 keys written out as their low 32 bits (shift <= 32): the second pass of the 32-bit count when
// the events are wider than a first pass's digit can narrow (W > 42, the corpus-wide tables' wide context ids).
extern "C" int ng_msd_pass_narrow(void* temp, size_t* temp_bytes, const u64* keys, const u32* dpre, i64 nseg,
                                  int nb_bits, const u64* total, u64 cap, int shift, int nbits, u32* out, i64* start,
                                  void* stream) {
    return msd_pass<u64, u32>(temp, temp_bytes, keys, dpre, nseg, nb_bits, total, cap, shift, nbits, out, start,
                              (hipStream_t)stream);
}

// The lookups of n query positions (pos[j], or j with pos NULL) for the 32-bit count: qk[j] = kmix(ctx_of[i] << 16 |
// tgt[i], W, M) << (64 - W) (part.h; M 0: W) for context ids in [lo, hi) (below 2^(W - 16)), else EMPTY; qv[j] = i.
// n_dev (may be NULL): a device-side count of pos's entries; lookups j >= *n_dev are EMPTY.
extern "C" int ng_part_lookups_w(const int* ctx_of, const u16* tgt, const int* pos, i64 n, const u64* n_dev, i64 lo,
                                 i64 hi, int W, int M, u64* qk, u32* qv, void* stream) {
    if (M == 0) M = W;
    if (W < 17 || W > 63 || M < 17 || M > W || lo < 0 || hi > (1ll << (W - 16)) || (n_dev && !pos)) return -1;
    if (n <= 0) return 0;
    lookups_w_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, tgt, pos, n, n_dev, lo, hi, W, M, qk,
                                                                     qv);
    return (int)hipGetLastError();
}

// The positions i < n with v[i] > 0 in order into out (at most cap of them), *n_dev = how many there are (which may
// exceed cap: the caller checks); CUB-style two-phase temp storage. No host read.
extern "C" int ng_select_positive(void* temp, size_t* temp_bytes, const int* v, i64 n, int* out, i64 cap, u64* n_dev,
                                  void* stream) {
    if (temp_bytes == nullptr || n < 0 || cap < 0 || n_dev == nullptr) return -1;
    const i64 nb = (n + 256 * SEL_ITEMS - 1) / (256 * SEL_ITEMS);
    const size_t b0 = al256((size_t)(nb > 0 ? nb : 1) * 4);
    const size_t need = b0 + prim::scan_u32_temp_bytes(nb);
    if (temp == nullptr) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need) return -1;
    hipStream_t st = (hipStream_t)stream;
    u32* cnt = (u32*)temp;
    if (nb == 0) return prim::fill_u64(n_dev, 0ull, 1, st);
    sel_count_k<<<(unsigned)nb, 256, 0, st>>>(v, n, cnt);
    int e = prim::exclusive_scan_u32(cnt, cnt, nb, n_dev, (char*)temp + b0, st);
    if (e) return e;
    sel_write_k<<<(unsigned)nb, 256, 0, st>>>(v, n, cnt, out, cap);
    return (int)hipGetLastError();
}

// Count the 32-bit events (ng_msd_pass's output; start its partitions' starts, 2^pbits of them, 1 <= W - pbits <=
// 31, W the pair-key bits; events kmix(pair key, W, M), part.h, M 0: W) partition by partition with `grid` blocks of
// about equal events (at most 65536): block b's distinct pairs as packed words pair key << (48 - cb) | min(count,
// esc), esc = 2^(48 - cb) - 1 (larger counts also in the escape table; context ids below 2^(W - 16), W - 16 <= cb <=
// 44), at out_k + seg_base[b], seg_cnt[b] of them (out_k holds as many words as there are events); dhist[d * grid +
// b] block b's words per dbits-bit digit (word >> dshift) & (2^dbits - 1) (1 <= dbits <= 11), for ng_seg_scatter.
// runs (may be NULL; dhist is then unused and may be NULL): each partition's words are written grouped by the
// gbits-bit digit (pair key >> gshift) & (2^gbits - 1) (0 <= gbits <= 6, 16 <= gshift, gshift + gbits <= W), group s
// of partition p = b << rbits | j (2^rbits partitions a first-pass bucket) at out_k[lo, hi), lo | hi << 32 =
// runs[((b << gbits) + s) << rbits | j]. live_np (<= 2^pbits): the partitions whose runs and slabs are written (those
// of the buckets holding context ids: the others hold no events and are never read; 2^pbits without runs).
// n_words (may be NULL):
// += the words written (the distinct pairs; one atomic per block). Lookups (ng_part_lookups_w's, sorted by
// their top pbits; qstart their partitions' bounds; qk and qv may be NULL with qstart all zeros: none) get qcnt[qv[j]]
// = the pair's count or 0. flags[0] bit 0: a partition reached min(limit, 11000) distinct pairs (its count is
// incomplete: count again with a bit more); bit 1: the escape table is full. slab (may be NULL): 2^pbits * 14336
// u64, partition p's table written to slab + p * 14336 (slot = count << 32 | key, pairs32.h's layout), for queries
// of the counts after the build (p32_pair_count).
extern "C" int ng_part_count32(const u32* ev, const i64* start, int pbits, int W, int M, const u64* qk,
                               const u32* qv, const i64* qstart, u64* out_k, int cb, u64* esc_k, u32* esc_c,
                               u64 esc_cap, u32* seg_cnt, i64* seg_base, u32* qcnt, u32* dhist, int dshift, int dbits,
                               u32 limit, u32* flags, int grid, u64* slab, u64* runs, int gbits, int gshift,
                               int rbits, i64 live_np, u64* n_words, void* stream) {
    if (M == 0) M = W;
    if (pbits < 1 || pbits > 30 || W < 17 || W - 16 > cb || cb > 44 || W - pbits > 31 || W - pbits < 1 ||
        M < 17 || M > W || grid <= 0 || grid > 65536 || esc_k == nullptr || esc_c == nullptr || esc_cap == 0 ||
        qstart == nullptr || limit == 0)
        return -1;
    if (live_np < 0 || live_np > (1ll << pbits)) return -1;
    if (runs ? (gbits < 0 || gbits > 6 || gshift < 16 || gshift + gbits > W || rbits < 0 || rbits > pbits)
             : (dbits < 1 || dbits > 11 || dshift < 0 || dshift + dbits > 64 || dhist == nullptr))
        return -1;
    const i64 P = 1ll << pbits;
    limit = limit < P32_LIMIT ? limit : P32_LIMIT;
    count32_k<<<grid, P32_BLOCK, 0, (hipStream_t)stream>>>(ev, start, P, pbits, W, M, qk, qv, qstart, out_k, cb,
                                                           esc_k, esc_c, esc_cap, seg_cnt, seg_base, qcnt, dhist,
                                                           dshift, dbits, limit, flags, slab, runs, gbits, gshift,
                                                           rbits, live_np, n_words);
    return (int)hipGetLastError();
}

// Per context of ids below n_ids from ng_part_count32's words (cb context bits) grouped by context into P
// partitions (start: i64[P + 1]; partition q = the ids [q << ibits, (q + 1) << ibits), ibits <= 11): dist[c] = its
// pairs (0: absent) for every id (dist may be NULL), and for present contexts the record rec[c] of ng_ctx_summary's layout (topk 1, 2,
// 4, 8; first-word index 0); flags[0] bit 2: a total reached 2^32. deep (may be NULL; deep_n then too): the ids of
// the contexts of more than deep_min pairs, appended in no order (at most deep_cap kept; *deep_n counts all, zeroed by
// the caller), for ng_ctx_kth_grouped. present (may be NULL): *present += the present contexts (zeroed by the caller).
// grid: the blocks, each walking partitions q, q + grid, ... with the next one's words loaded ahead (for many light
// partitions: a couple per compute unit), or 0: a block per partition (for heavy ones, which a fixed walk would leave
// unbalanced).
extern "C" int ng_ctx_agg(const u64* w, const i64* start, i64 P, int ibits, int cb, i64 n_ids, const u64* esc_k,
                          const u32* esc_c, u64 esc_cap, int topk, u32* rec, u32* dist, u32* flags, u32 deep_min,
                          i64* deep, u64 deep_cap, u64* deep_n, u64* present, int grid, void* stream) {
    if (cb < 1 || cb > 44 || ibits < 0 || (1 << ibits) > (topk >= 8 ? AGG_IDS_FOR(8) : AGG_IDS) || P <= 0 ||
        esc_cap == 0 || n_ids < 0 ||
        n_ids > (1ll << cb) || (P << ibits) < n_ids || (deep && !deep_n))
        return -1;
    if (n_ids == 0) return 0;
    const int g = grid_cap(P, grid > 0 ? grid : 1 << 30);
    hipStream_t st = (hipStream_t)stream;
#define AGG_LAUNCH(KT)                                                                                         \
    ctx_agg_k<KT><<<g, AGG_BLOCK, 0, st>>>(w, start, P, ibits, cb, n_ids, esc_k, esc_c, esc_cap, rec, dist, flags, \
                                           deep_min, deep, deep_cap, deep_n, present)
    switch (topk) {
        case 1: AGG_LAUNCH(1); break;
        case 2: AGG_LAUNCH(2); break;
        case 4: AGG_LAUNCH(4); break;
        case 8: AGG_LAUNCH(8); break;
        default: return -1;
    }
#undef AGG_LAUNCH
    return (int)hipGetLastError();
}

// ng_ctx_agg over ng_part_count32's words left in runs (its runs mode, with gbits, rbits = d2 and gshift = 16 +
// ibits): group g (of NG = 2^(d1 + gbits), d1 the first pass's digit bits; ids [g << ibits, (g + 1) << ibits), ibits
// <= 11, 10 for topk 8) is run g & (2^gbits - 1) of partitions (g >> gbits) << d2 ... + 2^d2 - 1, their bounds at
// runs[g << d2 ...] (0 <= d2 <= 8, 0 <= gbits <= 6; word indexes below 2^32).
// Outputs and grid as ng_ctx_agg's (no deep list).
extern "C" int ng_ctx_agg_runs(const u64* w, const u64* runs, i64 NG, int d2, int gbits, int ibits, int cb,
                               i64 n_ids, const u64* esc_k, const u32* esc_c, u64 esc_cap, int topk, u32* rec,
                               u32* dist, u32* flags, u64* present, int grid, void* stream) {
    if (cb < 1 || cb > 44 || ibits < 0 || (1 << ibits) > (topk >= 8 ? AGG_IDS_FOR(8) : AGG_IDS) || NG <= 0 ||
        d2 < 0 || (1 << d2) > AGG_RUN_REGS * WAVE || gbits < 0 || gbits > 6 || (NG & ((1ll << gbits) - 1)) || esc_cap == 0 ||
        n_ids < 0 || n_ids > (1ll << cb) || (NG << ibits) < n_ids || runs == nullptr)
        return -1;
    if (n_ids == 0) return 0;
    const int g = grid_cap(NG, grid > 0 ? grid : 1 << 30);
    hipStream_t st = (hipStream_t)stream;
#define AGG_LAUNCH(KT)                                                                                             \
    ctx_agg_runs_k<KT><<<g, AGG_BLOCK, 0, st>>>(w, runs, NG, d2, gbits, ibits, cb, n_ids, esc_k, esc_c, esc_cap, rec, \
                                                dist, flags, present)
    switch (topk) {
        case 1: AGG_LAUNCH(1); break;
        case 2: AGG_LAUNCH(2); break;
        case 4: AGG_LAUNCH(4); break;
        case 8: AGG_LAUNCH(8); break;
        default: return -1;
    }
#undef AGG_LAUNCH
    return (int)hipGetLastError();
}
