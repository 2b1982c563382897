// Partitioned pair counting: the engine's count path without global atomics (no counterpart in the reference's
// libraries; it replaces, inside this build's hosts, the split-table counting of ng_scan_count and ng_table_compact).
//
//   1. ng_scan_emit (engine.hip) appends each hit's mix64(pair key) to its block's region;
//   2. ng_seg_offsets + ng_seg_gather pack the regions into one array of events;
//   3. the events are sorted by their top pbits (sort_pairs, keys only): partition p = events whose mixed key has top
//      bits p, i.e. a hash partition of the pairs; ng_part_bounds finds each partition's range;
//   4. ng_part_count: one block per group of partitions counts each partition's events in an LDS hash table (8192
//      slots; a partition with more distinct pairs sets flags[0] bit 0 and the host repeats 3-4 with one more bit),
//      answers that partition's lookups (the query positions' (context, target) pairs, hashed and sorted the same way
//      by ng_part_lookups + sort_pairs), and appends the distinct pairs (unmixed) with their counts to the block's
//      segment, which ng_seg_gather packs again.
// Every event is read three times and written twice, in coalesced runs, and counted by LDS atomics; on MI355X global
// atomics run at about 27 G/s scattered and 80 M/s on one address, far below these streams.
#include "ngram_common.h"

namespace {

// mix64's inverse: each step undone in reverse order. A right xorshift by s is undone by r <- h ^ (r >> s) (each round
// fixes s more bits from the top: three rounds cover 64 bits for s >= 22); a product by an odd constant by the product
// by its inverse modulo 2^64.
__device__ __forceinline__ u64 unxorshift(u64 h, int s) {
    u64 r = h;
#pragma unroll
    for (int i = 0; i < 3; ++i) r = h ^ (r >> s);
    return r;
}
__device__ __forceinline__ u64 unmix64(u64 h) {
    h = unxorshift(h, 31);
    h *= 0x319642b2d24d8ec3ull;  // 0x94d049bb133111eb^-1 mod 2^64
    h = unxorshift(h, 27);
    h *= 0x96de1b173f119089ull;  // 0xbf58476d1ce4e5b9^-1 mod 2^64
    return unxorshift(h, 30);
}

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
        const u32 c = cnt[s];
        const u64 o = off[s];
        for (u32 i = threadIdx.x; i < c; i += 256) {
            dst_k[o + i] = src_k[base + i];
            if (src_v) dst_v[o + i] = src_v[base + i];
        }
    }
}

// start[p] = the first i with ev[i] >> (64 - pbits) >= p, for p = 0..P (ev sorted by its top pbits; start[P] = n).
__global__ void part_bounds_k(const u64* __restrict__ ev, i64 n, int pbits, i64 P, i64* __restrict__ start) {
    const i64 p = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (p > P) return;
    i64 a = 0, b = n;
    if (p == P) a = n;
    else if (pbits > 0) {
        const int sh = 64 - pbits;
        while (a < b) {
            const i64 m = (a + b) >> 1;
            if ((i64)(ev[m] >> sh) < p) a = m + 1;
            else b = m;
        }
    }  // pbits 0: one partition starting at 0
    start[p] = a;
}

// Lookup i: the mixed pair key of query position i's (context, target) if its context id is in [lo, hi) (else EMPTY,
// which no mixed pair key equals: mix64 is a bijection and its preimage of EMPTY is no pair key), value i.
__global__ void part_lookups_k(const int* __restrict__ ctx_of, const u16* __restrict__ tgt, i64 N, i64 lo, i64 hi,
                               u64* __restrict__ qk, u32* __restrict__ qv) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const i64 c = ctx_of[i];
    qk[i] = (c >= lo && c < hi) ? mix64(((u64)c << 16) | tgt[i]) : EMPTY;
    qv[i] = (u32)i;
}

#define PT_SLOTS 8192
#define PT_MASK (PT_SLOTS - 1)
#define PT_BLOCK 1024
#define PT_ITEMS 4

__device__ __forceinline__ void pt_insert(u64* tk, u32* tc, u64 key, u32 add, u32* flags) {
    u32 s = (u32)key & PT_MASK;
    for (int probe = 0; probe < PT_SLOTS; ++probe) {
        const u64 cur = tk[s];
        if (cur == key) {
            atomicAdd(&tc[s], add);
            return;
        }
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&tk[s], EMPTY, key);
            if (prev == EMPTY || prev == key) {
                atomicAdd(&tc[s], add);
                return;
            }
        }
        s = (s + 1) & PT_MASK;
    }
    atomicOr(&flags[0], 1u);  // more distinct pairs than slots: the host repartitions with one more bit
}

__device__ __forceinline__ u32 pt_find(const u64* tk, const u32* tc, u64 key) {
    u32 s = (u32)key & PT_MASK;
    for (int probe = 0; probe < PT_SLOTS; ++probe) {
        const u64 cur = tk[s];
        if (cur == key) return tc[s];
        if (cur == EMPTY) return 0;
        s = (s + 1) & PT_MASK;
    }
    return 0;
}

// Block b counts partitions [b * ppb, (b + 1) * ppb) in turn. Its distinct pairs (at most its events) go to
// out[start[p0] ...]: segment b = (seg_base[b], seg_cnt[b]). qcnt[qv[j]] = the count of lookup j (0: absent).
__global__ void __launch_bounds__(PT_BLOCK) part_count_k(const u64* __restrict__ ev, const i64* __restrict__ start,
                                                        i64 P, i64 ppb, const u64* __restrict__ qk,
                                                        const u32* __restrict__ qv, const i64* __restrict__ qstart,
                                                        u64* __restrict__ out_k, u32* __restrict__ out_c,
                                                        u32* __restrict__ seg_cnt, i64* __restrict__ seg_base,
                                                        u32* __restrict__ qcnt, u32* flags) {
    __shared__ u64 tk[PT_SLOTS];
    __shared__ u32 tc[PT_SLOTS];
    __shared__ u32 cur;
    const int t = threadIdx.x, lane = lane_id();
    const i64 p0 = blockIdx.x * ppb, p1 = p0 + ppb < P ? p0 + ppb : P;
    if (p0 >= P) {
        if (t == 0) {
            seg_cnt[blockIdx.x] = 0;
            seg_base[blockIdx.x] = 0;
        }
        return;
    }
    const i64 out_base = start[p0];
    if (t == 0) cur = 0;
    for (i64 p = p0; p < p1; ++p) {
        for (int j = t; j < PT_SLOTS; j += PT_BLOCK) {
            tk[j] = EMPTY;
            tc[j] = 0;
        }
        __syncthreads();
        const i64 a = start[p], b = start[p + 1];
        for (i64 i0 = a; i0 < b; i0 += (i64)PT_BLOCK * PT_ITEMS) {  // the same rounds for every wave
            u64 key[PT_ITEMS];
#pragma unroll
            for (int r = 0; r < PT_ITEMS; ++r) {
                const i64 i = i0 + (i64)r * PT_BLOCK + t;
                key[r] = i < b ? ev[i] : EMPTY;
            }
#pragma unroll
            for (int r = 0; r < PT_ITEMS; ++r) {
                const bool valid = key[r] != EMPTY;
                const u64 vb = __ballot(valid);
                if (!vb) continue;
                // the lanes holding the wave's first key add once (a hot pair would serialize the LDS atomics)
                const int ld = __ffsll((unsigned long long)vb) - 1;
                const u64 k0 = bcast_u64(key[r], ld);
                const bool same = valid && key[r] == k0;
                const u64 m = __ballot(same);
                if (same && lane != ld) continue;
                if (valid) pt_insert(tk, tc, key[r], same ? (u32)__popcll(m) : 1u, flags);
            }
        }
        __syncthreads();
        for (i64 j = qstart[p] + t; j < qstart[p + 1]; j += PT_BLOCK) {
            const u64 key = qk[j];
            qcnt[qv[j]] = key == EMPTY ? 0u : pt_find(tk, tc, key);
        }
        for (int j0 = 0; j0 < PT_SLOTS; j0 += PT_BLOCK) {
            const int j = j0 + t;
            const u64 key = tk[j];
            const bool occ = key != EMPTY;
            const u64 bal = __ballot(occ);
            if (!bal) continue;
            u32 off = 0;
            if (lane == 0) off = atomicAdd(&cur, (u32)__popcll(bal));
            off = (u32)__shfl((int)off, 0, WAVE);
            if (occ) {
                const u64 at = (u64)out_base + off + (u64)__popcll(bal & lanemask_lt());
                out_k[at] = unmix64(key);
                out_c[at] = tc[j];
            }
        }
        __syncthreads();
    }
    if (t == 0) {
        seg_cnt[blockIdx.x] = cur;
        seg_base[blockIdx.x] = out_base;
    }
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

// start[p] for p = 0..2^pbits (i64[2^pbits + 1]) of events sorted by their top pbits (0 <= pbits <= 24).
extern "C" int ng_part_bounds(const u64* ev, i64 n, int pbits, i64* start, void* stream) {
    if (pbits < 0 || pbits > 24 || n < 0) return -1;
    const i64 P = 1ll << pbits;
    part_bounds_k<<<grid_for(P + 1, 256), 256, 0, (hipStream_t)stream>>>(ev, n, pbits, P, start);
    return (int)hipGetLastError();
}

// The N query positions' lookups: qk[i] = mix64(ctx_of[i] << 16 | tgt[i]) for context ids in [lo, hi), else EMPTY;
// qv[i] = i.
extern "C" int ng_part_lookups(const int* ctx_of, const u16* tgt, i64 N, i64 lo, i64 hi, u64* qk, u32* qv,
                               void* stream) {
    if (N <= 0) return 0;
    part_lookups_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, tgt, N, lo, hi, qk, qv);
    return (int)hipGetLastError();
}

// Count the sorted events partition by partition (start: ng_part_bounds' of 2^pbits partitions) with `grid` blocks
// of consecutive partitions: block b's distinct pairs (pair key, count) at out_k/out_c + seg_base[b], seg_cnt[b] of
// them (out_k/out_c hold as many items as ev). Lookups (qk sorted like ev, qv their query positions, qstart their
// bounds) get qcnt[qv[j]] = the pair's count or 0. flags[0] bit 0: a partition held more than 8192 distinct pairs
// (its count is incomplete: repartition with one more bit).
extern "C" int ng_part_count(const u64* ev, const i64* start, int pbits, const u64* qk, const u32* qv,
                             const i64* qstart, u64* out_k, u32* out_c, u32* seg_cnt, i64* seg_base, u32* qcnt,
                             u32* flags, int grid, void* stream) {
    if (pbits < 0 || pbits > 24 || grid <= 0) return -1;
    const i64 P = 1ll << pbits;
    const i64 ppb = (P + grid - 1) / grid;
    part_count_k<<<grid, PT_BLOCK, 0, (hipStream_t)stream>>>(ev, start, P, ppb, qk, qv, qstart, out_k, out_c, seg_cnt,
                                                             seg_base, qcnt, flags);
    return (int)hipGetLastError();
}
