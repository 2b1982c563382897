// The 32-bit count's per-partition table (pairs32.hip's count32_k holds it in LDS; with a slab output it is also
// written to device memory, one slab of P32_SLOTS u64 per partition, slot s = count << 32 | key, for the corpus-wide
// tables' queries): u32 keys in buckets of four, filled from the front, buckets probed linearly from the key's home.
#pragma once
#include "part.h"

#ifndef P32_SLOTS
#define P32_SLOTS 14336  // 112 KB of LDS (u32 keys and counts) beside the slot list (28 KB): one block per CU
#endif
#define P32_BUCKETS (P32_SLOTS / 4)
#ifndef P32_BLOCK
#define P32_BLOCK 1024
#endif
#define P32_ITEMS 6  // events per thread and round (8 spills registers)
// P32_LIMIT: the distinct pairs a partition may reach before it is declared overfull. A free slot always remains: the
// limit is checked once per half-round, in which the block inserts at most P32_BLOCK * P32_ITEMS / 2 more keys.
#ifndef P32_LIMIT
#define P32_LIMIT 11000
#endif
static_assert(P32_LIMIT + P32_BLOCK * P32_ITEMS / 2 < P32_SLOTS, "a half-round past the limit must leave a free slot");
#define EMPTY32 0xFFFFFFFFu

__device__ __forceinline__ u32 p32_bucket(u32 key) {
    return (u32)(((u64)(key * 0x9E3779B1u) * P32_BUCKETS) >> 32);
}
__device__ __forceinline__ u32 p32_next(u32 b) { return b + 1 == P32_BUCKETS ? 0 : b + 1; }

// The slot of `key` in bucket q (read from bucket b), or -1.
__device__ __forceinline__ int p32_in(const uint4& q, u32 b, u32 key) {
    const int f = q.x == key ? 0 : q.y == key ? 1 : q.z == key ? 2 : q.w == key ? 3 : -1;
    return f < 0 ? -1 : 4 * (int)b + f;
}

// Insert `key` (below 2^31) into the bucketized table (four keys per 16-byte bucket, filled from the front, buckets
// probed linearly) from bucket b, whose contents q were read; returns its slot, *fresh whether it took a free slot.
// A lost race for a slot re-reads the bucket.
__device__ __forceinline__ int p32_insert(u32* tk, u32 key, u32 b, uint4 q, bool* fresh) {
    *fresh = false;
    while (true) {
        const int s = p32_in(q, b, key);
        if (s >= 0) return s;
        const int e = q.x == EMPTY32 ? 0 : q.y == EMPTY32 ? 1 : q.z == EMPTY32 ? 2 : q.w == EMPTY32 ? 3 : -1;
        if (e >= 0) {
            const u32 prev = atomicCAS(&tk[4 * b + e], EMPTY32, key);
            if (prev == EMPTY32 || prev == key) {
                *fresh = prev == EMPTY32;
                return 4 * (int)b + e;
            }
        } else {
            b = p32_next(b);
        }
        q = *(const uint4*)(tk + 4 * b);
    }
}

__device__ __forceinline__ u32 p32_find(const u32* tk, const u32* tc, u32 key) {
    u32 b = p32_bucket(key);
    while (true) {
        const uint4 q = *(const uint4*)(tk + 4 * b);
        const int s = p32_in(q, b, key);
        if (s >= 0) return tc[s];
        if (q.w == EMPTY32) return 0;
        b = p32_next(b);
    }
}

// A key's count in a partition's slab (the LDS table written out: u64 slots count << 32 | key), 0 if absent.
__device__ __forceinline__ u32 p32_slab_find(const u64* __restrict__ slab, u32 key) {
    u32 b = p32_bucket(key);
    for (u32 i = 0; i < P32_BUCKETS; ++i) {
        const ulonglong2* q = (const ulonglong2*)(slab + 4 * (u64)b);
        const ulonglong2 a = q[0], c = q[1];
        if ((u32)a.x == key) return (u32)(a.x >> 32);
        if ((u32)a.y == key) return (u32)(a.y >> 32);
        if ((u32)c.x == key) return (u32)(c.x >> 32);
        if ((u32)c.y == key) return (u32)(c.y >> 32);
        if ((u32)c.y == EMPTY32) return 0;
        b = p32_next(b);
    }
    return 0;
}

// The count of pair key pk (context id << 16 | token, below 2^W) in a level's slabs (2^pbits partitions of the
// W-bit hash wmix(pk, W), partition = its top pbits bits, key = the bits below).
__device__ __forceinline__ u32 p32_pair_count(const u64* __restrict__ slabs, int pbits, int W, u64 pk) {
    const u64 h = wmix(pk, W);
    const int lbits = W - pbits;
    const u64 p = h >> lbits;
    return p32_slab_find(slabs + p * (u64)P32_SLOTS, (u32)(h & ((1ull << lbits) - 1ull)));
}
