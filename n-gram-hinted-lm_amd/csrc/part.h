// Device code shared by the partitioned count (part.hip) and the corpus-wide count tables (table.hip): mix64's
// inverse, the escape table of packed words' large counts, and the per-context record.
#pragma once
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

// A bijection of W-bit values (17 <= W <= 63): a product by an odd constant, a right xorshift by s = ceil(W / 2) (its
// own inverse, since x >> 2s = 0), again, all modulo 2^W. The 32-bit count hashes pair keys below 2^W with it, so
// that its top bits spread every context's pairs over the partitions and the bits below the partition digits
// identify the pair within its partition.
#define WMIX_C1 0x9E3779B97F4A7C15ull
#define WMIX_C2 0xBF58476D1CE4E5B9ull
#define WMIX_I1 0xF1DE83E19937733Dull  // WMIX_C1^-1 mod 2^64
#define WMIX_I2 0x96DE1B173F119089ull  // WMIX_C2^-1 mod 2^64
__host__ __device__ __forceinline__ u64 wmix(u64 x, int W) {
    const u64 m = (1ull << W) - 1ull;
    const int s = (W + 1) >> 1;
    x = (x * WMIX_C1) & m;
    x ^= x >> s;
    x = (x * WMIX_C2) & m;
    return x ^ (x >> s);
}
__host__ __device__ __forceinline__ u64 unwmix(u64 h, int W) {
    const u64 m = (1ull << W) - 1ull;
    const int s = (W + 1) >> 1;
    h ^= h >> s;
    h = (h * WMIX_I2) & m;
    h ^= h >> s;
    return (h * WMIX_I1) & m;
}

// The 32-bit count's event key of a pair key x below 2^W: its bits from M up kept, the M bits below mixed by
// wmix (17 <= M <= W). M = W spreads every context's pairs over all partitions; M = W - d1 keeps the top d1 bits of
// the context id, so that the first pass's buckets are ranges of context ids and a bucket's partitions hold the
// pairs of its contexts only (spread by the hash below those bits).
__host__ __device__ __forceinline__ u64 kmix(u64 x, int W, int M) {
    const u64 lo = (1ull << M) - 1ull;
    return (x & ~lo & ((1ull << W) - 1ull)) | wmix(x & lo, M);
}
__host__ __device__ __forceinline__ u64 unkmix(u64 h, int W, int M) {
    const u64 lo = (1ull << M) - 1ull;
    return (h & ~lo & ((1ull << W) - 1ull)) | unwmix(h & lo, M);
}

// A wave-uniform lane's 64-bit value (readlane: no LDS traffic).
__device__ __forceinline__ u64 readlane_u64(u64 v, int l) {
    const u32 lo = (u32)__builtin_amdgcn_readlane((int)(u32)v, l);
    const u32 hi = (u32)__builtin_amdgcn_readlane((int)(u32)(v >> 32), l);
    return ((u64)hi << 32) | lo;
}

// The block owning partition p: the one whose share of the events holds the partition's first event (start[p] * G /
// n, the last block for trailing empty partitions), so that blocks get equal events, whatever the skew of the
// partitions' sizes (a partition holding a hot pair has far more events than others). Monotone in p.
__device__ __forceinline__ i64 part_owner(const i64* __restrict__ start, i64 p, i64 n, i64 G) {
    if (n <= 0) return 0;
    const i64 o = (i64)((u64)start[p] * (u64)G / (u64)n);  // start * G < 2^63 for n < 2^47 events, G <= 2^16
    return o < G - 1 ? o : G - 1;
}

// The first partition whose owner is at least b (P if none).
__device__ __forceinline__ i64 part_first(const i64* __restrict__ start, i64 P, i64 n, i64 G, i64 b) {
    i64 lo = 0, hi = P;
    while (lo < hi) {
        const i64 m = (lo + hi) >> 1;
        if (part_owner(start, m, n, G) < b) lo = m + 1;
        else hi = m;
    }
    return lo;
}

// A count too large for a packed word's count field: (pair key, count) into the escape table (linear probing; each
// distinct pair is written once). A full table sets flags[0] bit 1.
__device__ __forceinline__ void esc_put(u64* esc_k, u32* esc_c, u64 cap, u64 key, u32 n, u32* flags) {
    u64 s = __umul64hi(mix64(key), cap);
    for (u64 probe = 0; probe < cap; ++probe) {
        if (atomicCAS((unsigned long long*)&esc_k[s], EMPTY, key) == EMPTY) {
            esc_c[s] = n;
            return;
        }
        s = s + 1 == cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 2u);
}

__device__ __forceinline__ u32 esc_get(const u64* __restrict__ esc_k, const u32* __restrict__ esc_c, u64 cap, u64 key) {
    u64 s = __umul64hi(mix64(key), cap);
    for (u64 probe = 0; probe < cap; ++probe) {
        const u64 cur = esc_k[s];
        if (cur == key) return esc_c[s];
        if (cur == EMPTY) return 0;
        s = s + 1 == cap ? 0 : s + 1;
    }
    return 0;
}

// A context's record, WORDS u32: total, pairs, the first KT tokens two per word, their counts, and where two words are
// left (KT 2 and 8) the index of the context's first packed word (u64, low word first); zeros elsewhere.
template <int KT>
struct CtxRecord {
    static constexpr int TOKW = (KT + 1) / 2;
    static constexpr int USED = 2 + TOKW + KT;
    static constexpr int WORDS = USED <= 4 ? 4 : USED <= 8 ? 8 : 16;
    static constexpr int FIRST = WORDS - USED >= 2 ? USED : -1;
};

// A record's words (CtxRecord<KT>): total, pairs, the top tokens two per word, their counts, and (where room) the
// first word's index.
template <int KT>
__device__ __forceinline__ void record_words(u32 (&v)[CtxRecord<KT>::WORDS], u64 total, u32 pairs,
                                             const u64 (&top)[KT], u64 first) {
    using R = CtxRecord<KT>;
#pragma unroll
    for (int q = 0; q < R::WORDS; ++q) v[q] = 0;
    v[0] = (u32)total;
    v[1] = pairs;
    if constexpr (R::FIRST >= 0) {
        v[R::FIRST] = (u32)first;
        v[R::FIRST + 1] = (u32)(first >> 32);
    }
#pragma unroll
    for (int r = 0; r < KT; ++r) {
        const u32 tk = top[r] ? 0xFFFFu - (u32)(top[r] & 0xFFFF) : 0u;
        v[2 + r / 2] |= tk << (16 * (r & 1));
        v[2 + R::TOKW + r] = (u32)(top[r] >> 16);
    }
}

template <int KT>
__device__ __forceinline__ void store_record(u32* __restrict__ rec, u64 c, u64 total, u32 pairs, const u64 (&top)[KT],
                                             u64 first) {
    using R = CtxRecord<KT>;
    u32 v[R::WORDS];
    record_words<KT>(v, total, pairs, top, first);
    uint4* dst = (uint4*)(rec + c * R::WORDS);
#pragma unroll
    for (int q = 0; q < R::WORDS / 4; ++q) dst[q] = make_uint4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

}  // namespace
