// Device code behind the reference's two C ABIs (old_records/gpu_val_stats.cu and
// record_367_gpu_counts/track_1_short/counts/kernels.cu export the same entry points with their own pair-key widths):
// the packed pair table, the level scan's tile kernel, the grouping of emitted keys by sub-table and their counting,
// and the table's extraction by owner. Each flavour's library includes this header once and instantiates it with its
// pair-key width KB (40 or 41 bits).
//
// Packed pair table (the ABI's table format: the host allocates pk u64[cap] EMPTY-filled and wraps u32[(cap + 3) / 4]
// zeroed, and reads nothing else): a slot holds a pair key (context id << 16 | next token) in its low KB bits and the
// pair's count in the 64 - KB bits above; a count passing 2^(64-KB) - 1 carries into the slot's byte of `wraps`
// (four slots per u32), so counts up to 2^(72-KB) - 1 are exact. The table is 2^pbits sub-tables of sub_cap slots
// (sub-table = the top pbits bits of mix64(pair key)); within a sub-table a key's probe sequence starts at an 8-slot
// bucket (one 64-byte line) chosen by the next bits of the hash and runs linearly over the sub-table's slots, eight
// at a time. A slot's key bits never change once written, so a probe may compare stale copies of occupied slots and
// needs a compare-and-swap only to take an empty one.
//
// Counting design (MI355X): a scan's wave merges the hits of equal pair keys first (a ballot per distinct key), so a
// hot pair costs one atomic per wave rather than one per hit; `aggregate` merges a whole chunk of grouped keys in an LDS
// hash table before it touches the global table. Emitted keys go to one buffer through block-level staging in LDS: one
// global atomic per 4096-position tile (a counter hit per wave would serialize: same-address atomics run at about
// 80 M/s on MI355X).
#pragma once
#include "../probe.h"

namespace abi {

#define ABI_TILE 4096        // positions per scan tile (128 bitmap words; 1024 per wave)
#define ABI_PPL 4            // lookups per lane in flight
#define GROUP_TILE 4096      // keys per block pass of the sub-table grouping
#define GROUP_MAX_BITS 12    // sub-table bits the grouping supports (its LDS counters)
#define AGG_CHUNK 2048       // grouped keys merged per LDS pass of aggregate
#define AGG_SLOTS 4096       // the LDS hash table of that pass

template <int KB>
struct Fmt {
    static constexpr u64 KMASK = (1ull << KB) - 1;
    static constexpr int CB = 64 - KB;
    static constexpr u64 CMAX = (1ull << CB) - 1;
};

__device__ __forceinline__ u64 sub_of(u64 h, int pbits) { return pbits ? h >> (64 - pbits) : 0; }

// Add n (1 <= n < 2^23) to slot i's count, carrying a wrap into its byte of `wraps`.
template <int KB>
__device__ __forceinline__ void slot_bump(u64* pk, u32* wraps, u64 i, u32 n) {
    const u64 old = atomicAdd((unsigned long long*)&pk[i], (unsigned long long)n << KB);
    if ((old >> KB) + n > Fmt<KB>::CMAX) atomicAdd(&wraps[i >> 2], 1u << (8 * (i & 3)));
}

// The exact count of an occupied slot i read as v.
template <int KB>
__device__ __forceinline__ u32 slot_total(const u32* __restrict__ wraps, u64 i, u64 v) {
    const u32 wb = (wraps[i >> 2] >> (8 * (i & 3))) & 0xFFu;
    return (u32)(v >> KB) + (wb << Fmt<KB>::CB);
}

// Count pair key `key` n times; false (and flags[0] |= 1) when MAXPROBE slots held no room.
template <int KB>
__device__ __forceinline__ bool packed_add(u64* pk, u32* wraps, u64 sub_cap, int pbits, u64 key, u32 n, u32* flags) {
    const u64 h = mix64(key);
    const u64 base = sub_of(h, pbits) * sub_cap;
    const u64 nb = sub_cap >= 8 ? sub_cap >> 3 : 1;
    u64 s = __umul64hi(pbits ? h << pbits : h, nb) << 3;
    if (s >= sub_cap) s = 0;
    for (int probe = 0; probe < MAXPROBE; probe += 8) {
        u64 v[8], at[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u64 t = s + j;
            if (t >= sub_cap) t -= sub_cap;
            at[j] = base + t;
            v[j] = pk[at[j]];  // eight loads of one line in flight together
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (v[j] != EMPTY) {
                if ((v[j] & Fmt<KB>::KMASK) == key) {
                    slot_bump<KB>(pk, wraps, at[j], n);
                    return true;
                }
                continue;
            }
            const u64 prev = atomicCAS((unsigned long long*)&pk[at[j]], EMPTY, key | ((u64)n << KB));
            if (prev == EMPTY) return true;
            if ((prev & Fmt<KB>::KMASK) == key) {
                slot_bump<KB>(pk, wraps, at[j], n);
                return true;
            }
        }
        s += 8;
        if (s >= sub_cap) s -= sub_cap;
    }
    atomicOr(&flags[0], 1u);
    return false;
}

// The wave's hits merged by pair key: each distinct key's first lane (in lane order) learns how many lanes hold it.
// One ballot per distinct key of the wave.
__device__ __forceinline__ u32 wave_merge(bool hit, u64 key) {
    u64 pending = __ballot(hit);
    u32 mine = 0;
    while (pending) {
        const int l = __ffsll((unsigned long long)pending) - 1;
        const u64 lk = bcast_u64(key, l);
        const u64 same = __ballot(hit && key == lk);
        if (lane_id() == l) mine = (u32)__popcll(same);
        pending &= ~same;
    }
    return mine;
}

// What a scan does with its hits besides the bitmap.
struct TableSink {  // count in the packed table (mode "count")
    static constexpr bool APPEND = false;
    u64* pk;
    u32* wraps;
    u64 sub_cap;
    int pbits;
};
struct AppendSink {  // append the pair keys to emit[*emitted ...] (mode "emit")
    static constexpr bool APPEND = true;
    u64* emit;
    u64* emitted;
};

// One level's scan over positions [0, L), in tiles of ABI_TILE positions (a block-uniform loop: blocks take tiles
// round-robin). GATED: only positions whose bit is set in bm_in are looked up; each wave lists its 32 words' set
// positions in LDS and its lanes take the list ABI_PPL entries at a time, so lanes stay busy whatever the density.
// Ungated: every position, a lane per position. Hits set their bit in the wave's LDS copy of its words, written out
// whole; with a TableSink they are merged per wave and counted (skipped once flags[0] says the table overflowed, the
// bitmap still made), with an AppendSink staged in LDS and written out once per tile.
template <int K, bool SORTED, bool GATED, int KB, class S>
__global__ void __launch_bounds__(256) tile_scan_k(const u16* __restrict__ tok, i64 L, int k,
                                                   const u32* __restrict__ bm_in, u32* __restrict__ bm_out,
                                                   const u64* __restrict__ vt, u64 vcap, const u32* __restrict__ vrep,
                                                   const u16* __restrict__ x, u32* flags, S sink) {
    __shared__ u16 list[GATED ? 4 : 1][GATED ? 1024 : 1];
    __shared__ u32 words[4][32];
    __shared__ u64 stage[S::APPEND ? ABI_TILE : 1];
    __shared__ u32 nstage;
    __shared__ u64 gbase;
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const i64 nwords = (L + 31) >> 5;
    if constexpr (S::APPEND) {
        if (threadIdx.x == 0) nstage = 0;
        __syncthreads();
    }
    for (i64 t0 = (i64)blockIdx.x * ABI_TILE; t0 < L; t0 += (i64)gridDim.x * ABI_TILE) {
        const i64 wbase = (t0 >> 5) + w * 32;  // the wave's first word
        const i64 pbase = wbase << 5;
        u32 total = 0;
        if (lane < 32) words[w][lane] = 0;
        if constexpr (GATED) {
            const i64 wi = wbase + lane;
            const u32 word = (lane < 32 && wi < nwords) ? bm_in[wi] : 0u;
            const u32 c = __popc(word);
            u32 incl = c;
#pragma unroll
            for (int d = 1; d < 32; d <<= 1) {
                const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
                if (lane >= d) incl += o;
            }
            total = (u32)__shfl((int)incl, 31, WAVE);
            u32 at = incl - c;
            for (u32 bits = word; bits; bits &= bits - 1) list[w][at++] = (u16)(lane * 32 + __ffs(bits) - 1);
        } else {
            const i64 left = L - pbase;
            total = left <= 0 ? 0u : left >= 1024 ? 1024u : (u32)left;
        }
        bool full = false;
        if constexpr (!S::APPEND) full = *(volatile u32*)&flags[0] != 0u;
        // the wave's list and words are its own: its LDS accesses stay in order without a barrier
        for (u32 r0 = 0; r0 < total; r0 += WAVE * ABI_PPL) {
            Walk wk[ABI_PPL];
            u32 off[ABI_PPL];
#pragma unroll
            for (int q = 0; q < ABI_PPL; ++q) {
                const u32 r = r0 + q * WAVE + lane;
                wk[q].key = EMPTY;
                off[q] = 0;
                if (r < total) {
                    off[q] = GATED ? (u32)list[w][r] : r;
                    if (pbase + off[q] < L) walk_begin<K>(tok, pbase + off[q], k, vt, vcap, wk[q]);
                }
            }
#pragma unroll
            for (int q = 0; q < ABI_PPL; ++q) {
                if (r0 + q * WAVE >= total) break;  // wave-uniform
                const u64 key = walk_end<K, SORTED>(tok, pbase + off[q], k, vt, vrep, x, flags, wk[q]);
                const bool hit = key != EMPTY;
                if (hit) atomicOr(&words[w][off[q] >> 5], 1u << (off[q] & 31));
                if constexpr (S::APPEND) {
                    const u64 b = __ballot(hit);
                    if (b) {
                        u32 at = 0;
                        if (lane == 0) at = atomicAdd(&nstage, (u32)__popcll(b));
                        at = (u32)__shfl((int)at, 0, WAVE) + (u32)__popcll(b & lanemask_lt());
                        if (hit) stage[at] = key;
                    }
                } else {
                    const u32 n = wave_merge(hit, key);
                    if (n && !full) packed_add<KB>(sink.pk, sink.wraps, sink.sub_cap, sink.pbits, key, n, flags);
                }
            }
        }
        if (lane < 32 && wbase + lane < nwords) bm_out[wbase + lane] = words[w][lane];
        if constexpr (S::APPEND) {
            __syncthreads();
            const u32 n = nstage;
            if (threadIdx.x == 0 && n) gbase = atomicAdd((unsigned long long*)sink.emitted, (unsigned long long)n);
            __syncthreads();
            for (u32 i = threadIdx.x; i < n; i += blockDim.x) sink.emit[gbase + i] = stage[i];
            __syncthreads();
            if (threadIdx.x == 0) nstage = 0;
        }
    }
}

template <int KB, class S>
static int launch_tile_scan(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                            const u32* vrep, const u16* x, u32* flags, int grid, const S& sink, hipStream_t st) {
    if (L <= 0) return 0;
    const i64 tiles = (L + ABI_TILE - 1) / ABI_TILE;
    if (grid <= 0 || grid > tiles) grid = (int)(tiles < (1 << 30) ? tiles : (1 << 30));
    if (bm_in) {
        LEVEL_DISPATCH(k, (tile_scan_k<K, true, true, KB, S><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, sink)));
    } else {
        LEVEL_DISPATCH(k, (tile_scan_k<K, true, false, KB, S><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, sink)));
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Emitted pair keys grouped by sub-table, and counted
// ---------------------------------------------------------------------------------------------------------------

// Keys per sub-table (top pbits of mix64(key)) added to counts[]; EMPTY entries are skipped. Small tables of bins are
// kept per wave (fewer LDS atomic conflicts), larger ones per block.
__global__ void __launch_bounds__(256) group_hist_k(const u64* __restrict__ keys, i64 n, int pbits, u64* counts,
                                                    bool vec) {
    extern __shared__ u32 hist[];
    const int P = 1 << pbits;
    const bool per_wave = pbits <= 8;
    const int copies = per_wave ? 4 : 1;
    for (int b = threadIdx.x; b < P * copies; b += blockDim.x) hist[b] = 0;
    __syncthreads();
    u32* h = per_wave ? hist + (threadIdx.x / WAVE) * P : hist;
    const i64 pairs = n >> 1;
    const ulonglong2* k2 = (const ulonglong2*)keys;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < pairs; i += (i64)gridDim.x * blockDim.x) {
        ulonglong2 v;
        if (vec) v = k2[i];  // 16-byte aligned keys: one load for two
        else v.x = keys[2 * i], v.y = keys[2 * i + 1];
        if (v.x != EMPTY) atomicAdd(&h[sub_of(mix64(v.x), pbits)], 1u);
        if (v.y != EMPTY) atomicAdd(&h[sub_of(mix64(v.y), pbits)], 1u);
    }
    if ((n & 1) && blockIdx.x == 0 && threadIdx.x == 0 && keys[n - 1] != EMPTY)
        atomicAdd(&h[sub_of(mix64(keys[n - 1]), pbits)], 1u);
    __syncthreads();
    for (int b = threadIdx.x; b < P; b += blockDim.x) {
        u32 c = 0;
        for (int q = 0; q < copies; ++q) c += hist[q * P + b];
        if (c) atomicAdd((unsigned long long*)&counts[b], (unsigned long long)c);
    }
}

// Keys grouped by sub-table from cursor[] (each sub-table's next free index, advanced here). Per pass a block takes
// GROUP_TILE keys, ranks them within their sub-table by LDS counters, reserves each sub-table's run with one global
// atomic, sorts the tile by sub-table in LDS and writes it out in runs, so consecutive threads write consecutive
// addresses. EMPTY entries are dropped.
__global__ void __launch_bounds__(256) group_scatter_k(const u64* __restrict__ keys, i64 n, int pbits, u64* cursor,
                                                       u64* __restrict__ out) {
    extern __shared__ u64 lds64[];
    __shared__ u32 rsum[256];
    __shared__ u32 staged;
    const int P = 1 << pbits;
    u64* stage = lds64;                          // GROUP_TILE keys, sorted by sub-table
    u64* gpos = lds64 + GROUP_TILE;              // P: each sub-table's run in `out` for this tile
    u32* cnt = (u32*)(gpos + P);                 // P: keys per sub-table, then their first index in `stage`
    constexpr int PER = GROUP_TILE / 256;
    const int per = (P + 255) / 256;             // bins per thread in the prefix sum
    const int b0 = threadIdx.x * per;
    for (i64 t0 = (i64)blockIdx.x * GROUP_TILE; t0 < n; t0 += (i64)gridDim.x * GROUP_TILE) {
        for (int b = threadIdx.x; b < P; b += blockDim.x) cnt[b] = 0;
        __syncthreads();
        u64 key[PER];
        u32 bin[PER], rank[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const i64 i = t0 + j * 256 + threadIdx.x;
            key[j] = i < n ? keys[i] : EMPTY;
            bin[j] = key[j] != EMPTY ? (u32)sub_of(mix64(key[j]), pbits) : 0xFFFFFFFFu;
            rank[j] = bin[j] != 0xFFFFFFFFu ? atomicAdd(&cnt[bin[j]], 1u) : 0u;
        }
        __syncthreads();
        // each sub-table's run reserved, and cnt turned into its exclusive prefix: a thread's range of bins serially,
        // then the 256 range totals by the first wave
        u32 s = 0;
        for (int b = b0; b < b0 + per && b < P; ++b) {
            const u32 c = cnt[b];
            if (c) gpos[b] = atomicAdd((unsigned long long*)&cursor[b], (unsigned long long)c);
            cnt[b] = s;
            s += c;
        }
        rsum[threadIdx.x] = s;
        __syncthreads();
        if (threadIdx.x < WAVE) {
            u32 acc = 0;
            for (int q = 0; q < 4; ++q) {
                const u32 v = rsum[q * WAVE + threadIdx.x];
                u32 incl = v;
#pragma unroll
                for (int d = 1; d < WAVE; d <<= 1) {
                    const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
                    if ((int)threadIdx.x >= d) incl += o;
                }
                rsum[q * WAVE + threadIdx.x] = acc + incl - v;
                acc += (u32)__shfl((int)incl, WAVE - 1, WAVE);
            }
            if (threadIdx.x == 0) staged = acc;
        }
        __syncthreads();
        for (int b = b0; b < b0 + per && b < P; ++b) cnt[b] += rsum[threadIdx.x];
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (bin[j] != 0xFFFFFFFFu) stage[cnt[bin[j]] + rank[j]] = key[j];
        __syncthreads();
        for (u32 i = threadIdx.x; i < staged; i += blockDim.x) {
            const u64 v = stage[i];
            const u32 b = (u32)sub_of(mix64(v), pbits);
            out[gpos[b] + (i - cnt[b])] = v;
        }
        __syncthreads();
    }
}

// LDS bytes of group_scatter_k for pbits.
static inline size_t group_scatter_lds(int pbits) { return (size_t)GROUP_TILE * 8 + ((size_t)12 << pbits); }

// Grouped keys counted into the packed table: a block merges AGG_CHUNK consecutive keys (mostly of one sub-table) in
// an LDS hash table, then adds each distinct key's total with one packed_add. EMPTY entries are skipped. Once the
// table has overflowed (flags[0]) the rest is skipped: the host reruns the level with a bigger table.
template <int KB>
__global__ void __launch_bounds__(256) aggregate_k(const u64* __restrict__ keys, i64 n, u64* pk, u32* wraps,
                                                   u64 sub_cap, int pbits, u32* flags) {
    __shared__ unsigned long long hk[AGG_SLOTS];
    __shared__ u32 hc[AGG_SLOTS];
    __shared__ u32 stop;
    for (i64 c0 = (i64)blockIdx.x * AGG_CHUNK; c0 < n; c0 += (i64)gridDim.x * AGG_CHUNK) {
        // the whole block leaves together: one thread reads the flag for all (a divergent exit would skip barriers)
        if (threadIdx.x == 0) stop = *(volatile u32*)&flags[0];
        for (int s = threadIdx.x; s < AGG_SLOTS; s += blockDim.x) hk[s] = EMPTY, hc[s] = 0;
        __syncthreads();
        if (stop) return;
        for (int j = threadIdx.x; j < AGG_CHUNK; j += blockDim.x) {
            const i64 i = c0 + j;
            if (i >= n) break;
            const u64 key = keys[i];
            if (key == EMPTY) continue;
            u32 s = (u32)(mix64(key) >> 20) & (AGG_SLOTS - 1);
            for (;;) {  // AGG_SLOTS > AGG_CHUNK: a free slot always exists
                const unsigned long long prev = atomicCAS(&hk[s], (unsigned long long)EMPTY, (unsigned long long)key);
                if (prev == EMPTY || prev == key) {
                    atomicAdd(&hc[s], 1u);
                    break;
                }
                s = (s + 1) & (AGG_SLOTS - 1);
            }
        }
        __syncthreads();
        for (int s = threadIdx.x; s < AGG_SLOTS; s += blockDim.x)
            if (hc[s]) packed_add<KB>(pk, wraps, sub_cap, pbits, hk[s], hc[s], flags);
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------------------------
// The table's entries by owner (owner o holds context ids [bounds[o], bounds[o + 1]))
// ---------------------------------------------------------------------------------------------------------------

__device__ __forceinline__ int owner_in(const i64* b, int W, i64 c) {  // b in LDS, W + 1 entries
    int lo = 0, hi = W - 1;
    while (lo < hi) {
        const int m = (lo + hi + 1) >> 1;
        if (c >= b[m]) lo = m;
        else hi = m - 1;
    }
    return lo;
}

#define OWN_PER 8  // slots per lane in the owner kernels (a 2048-slot tile per block pass)

// Entries per owner added to counts[W]: per tile and owner, the lanes' counts summed by the wave, then one LDS add per
// wave and one global atomic per block and owner.
template <int KB>
__global__ void __launch_bounds__(256) own_count_k(const u64* __restrict__ pk, u64 cap, const i64* __restrict__ bounds,
                                                   int W, u64* counts) {
    __shared__ i64 b[MAXW + 1];
    __shared__ u64 h[MAXW];
    if (threadIdx.x <= W) b[threadIdx.x] = bounds[threadIdx.x];
    if (threadIdx.x < W) h[threadIdx.x] = 0;
    __syncthreads();
    for (u64 t0 = (u64)blockIdx.x * (256 * OWN_PER); t0 < cap; t0 += (u64)gridDim.x * (256 * OWN_PER)) {
        int own[OWN_PER];
#pragma unroll
        for (int j = 0; j < OWN_PER; ++j) {
            const u64 s = t0 + (u64)threadIdx.x * OWN_PER + j;
            const u64 v = s < cap ? pk[s] : EMPTY;
            own[j] = v == EMPTY ? -1 : owner_in(b, W, (i64)((v & Fmt<KB>::KMASK) >> 16));
        }
        for (int o = 0; o < W; ++o) {
            u32 c = 0;
#pragma unroll
            for (int j = 0; j < OWN_PER; ++j) c += own[j] == o;
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) c += (u32)__shfl_down((int)c, d, WAVE);
            if (lane_id() == 0 && c) atomicAdd((unsigned long long*)&h[o], (unsigned long long)c);
        }
    }
    __syncthreads();
    if (threadIdx.x < W && h[threadIdx.x]) atomicAdd((unsigned long long*)&counts[threadIdx.x], h[threadIdx.x]);
}

// Entries as (key, exact count) grouped by owner from cursor[o] (advanced here). Per tile and owner: a lane's entries
// of that owner are ranked by a wave prefix sum, the waves' totals combined in LDS, the block's run reserved with one
// atomic, and each lane writes its entries in slot order into the run.
template <int KB>
__global__ void __launch_bounds__(256) own_scatter_k(const u64* __restrict__ pk, const u32* __restrict__ wraps, u64 cap,
                                                     const i64* __restrict__ bounds, int W, u64* cursor,
                                                     u64* __restrict__ ok, u32* __restrict__ oc) {
    __shared__ i64 b[MAXW + 1];
    __shared__ u32 wsum[4];
    __shared__ u64 run;
    if (threadIdx.x <= W) b[threadIdx.x] = bounds[threadIdx.x];
    __syncthreads();
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    for (u64 t0 = (u64)blockIdx.x * (256 * OWN_PER); t0 < cap; t0 += (u64)gridDim.x * (256 * OWN_PER)) {
        u64 v[OWN_PER];
        int own[OWN_PER];
        const u64 s0 = t0 + (u64)threadIdx.x * OWN_PER;
#pragma unroll
        for (int j = 0; j < OWN_PER; ++j) {
            v[j] = s0 + j < cap ? pk[s0 + j] : EMPTY;
            own[j] = v[j] == EMPTY ? -1 : owner_in(b, W, (i64)((v[j] & Fmt<KB>::KMASK) >> 16));
        }
        for (int o = 0; o < W; ++o) {
            u32 c = 0;
#pragma unroll
            for (int j = 0; j < OWN_PER; ++j) c += own[j] == o;
            u32 incl = c;
#pragma unroll
            for (int d = 1; d < WAVE; d <<= 1) {
                const u32 t = (u32)__shfl_up((int)incl, d, WAVE);
                if (lane >= d) incl += t;
            }
            if (lane == WAVE - 1) wsum[w] = incl;
            __syncthreads();
            const u32 bt = wsum[0] + wsum[1] + wsum[2] + wsum[3];
            if (threadIdx.x == 0 && bt) run = atomicAdd((unsigned long long*)&cursor[o], (unsigned long long)bt);
            __syncthreads();
            if (bt) {
                u64 at = run + incl - c;
                for (int q = 0; q < w; ++q) at += wsum[q];
#pragma unroll
                for (int j = 0; j < OWN_PER; ++j)
                    if (own[j] == o) {
                        ok[at] = v[j] & Fmt<KB>::KMASK;
                        oc[at] = slot_total<KB>(wraps, s0 + j, v[j]);
                        ++at;
                    }
            }
            __syncthreads();
        }
    }
}

template <int KB>
static int launch_own_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, hipStream_t st) {
    if (W < 1 || W > MAXW) return -1;
    if (cap > 0) {
        const u64 tiles = (cap + 256 * OWN_PER - 1) / (256 * OWN_PER);
        own_count_k<KB><<<(int)(tiles < 4096 ? tiles : 4096), 256, 0, st>>>(pk, cap, bounds, W, counts);
    }
    return (int)hipGetLastError();
}

template <int KB>
static int launch_own_scatter(const u64* pk, const u32* wraps, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                              u32* oc, hipStream_t st) {
    if (W < 1 || W > MAXW) return -1;
    if (cap > 0) {
        const u64 tiles = (cap + 256 * OWN_PER - 1) / (256 * OWN_PER);
        own_scatter_k<KB><<<(int)(tiles < 4096 ? tiles : 4096), 256, 0, st>>>(pk, wraps, cap, bounds, W, cursor, ok,
                                                                            oc);
    }
    return (int)hipGetLastError();
}

// The grouping and counting launchers (both flavours).
static inline int max_group_bits() { return GROUP_MAX_BITS; }

static inline int launch_group_hist(const u64* keys, i64 n, int pbits, u64* counts, hipStream_t st) {
    if (pbits < 1 || pbits > GROUP_MAX_BITS) return -1;
    if (n > 0) {
        const size_t lds = (size_t)(pbits <= 8 ? 4 : 1) * 4 << pbits;
        const i64 g = (n / 2 + 255) / 256;
        group_hist_k<<<(int)(g < 1 ? 1 : g > 2048 ? 2048 : g), 256, lds, st>>>(keys, n, pbits, counts,
                                                                              ((uintptr_t)keys & 15) == 0);
    }
    return (int)hipGetLastError();
}

static inline int launch_group_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, hipStream_t st) {
    if (pbits < 1 || pbits > GROUP_MAX_BITS) return -1;
    if (n > 0) {
        const size_t lds = group_scatter_lds(pbits);
        if (lds > 48 * 1024) {
            const hipError_t e = hipFuncSetAttribute((const void*)group_scatter_k,
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return (int)e;
        }
        const i64 tiles = (n + GROUP_TILE - 1) / GROUP_TILE;
        group_scatter_k<<<(int)(tiles > 1024 ? 1024 : tiles), 256, lds, st>>>(keys, n, pbits, cursor, out);
    }
    return (int)hipGetLastError();
}

template <int KB>
static int launch_aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                            hipStream_t st) {
    if (pbits < 0 || pbits > 24 || sub_cap == 0) return -1;
    if (n > 0) {
        const i64 chunks = (n + AGG_CHUNK - 1) / AGG_CHUNK;
        if (grid <= 0 || grid > chunks) grid = (int)(chunks < (1 << 30) ? chunks : (1 << 30));
        aggregate_k<KB><<<grid, 256, 0, st>>>(keys, n, pk, wraps, sub_cap, pbits, flags);
    }
    return (int)hipGetLastError();
}

}  // namespace abi
