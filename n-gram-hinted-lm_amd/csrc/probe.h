// Query-table lookups of corpus contexts, shared by the level scans of the engine and of the C ABI.
//
// A query table holds the distinct query k-contexts' keys (ngram_common.h ctx_key) in u64 slots; a context's id is
// its slot. Lookups walk forward from the home slot umulhi(key, cap) until the key or an EMPTY slot; there is no
// wrap-around, and every table ends with an EMPTY slot, so a walk never leaves the table. Two layouts share this walk:
//   * the canonical layout of the reference's ValIndex (old_records/gpu_val_stats.py:604-651): keys in ascending
//     order of home slot, each at max(home, previous slot + 1). Since the home slot is monotone in the key, the table
//     is the sorted keys with gaps, and a walk may also stop at the first larger key (`sorted` walks);
//   * the engine's tables filled by compare-and-swap (ng_query_index): same walk, keys in no order.
// Keys of k <= 4 tokens are the tokens themselves (exact); longer keys are hashes, and a found key is checked token by
// token against the context's representative query position (rep[slot]); a mismatch is a false hit, counted in
// flags[1] and treated as a miss.
#pragma once
#include "ngram_common.h"

// k dispatch: levels with a kernel of their own; any other k in [1, MAXK] runs the run-time-k kernel (K = 0); k out
// of range returns -1 from the enclosing function.
#define LEVEL_DISPATCH(k, ...)                                  \
    do {                                                        \
        switch (k) {                                            \
            case 1: { constexpr int K = 1; __VA_ARGS__; } break;   \
            case 2: { constexpr int K = 2; __VA_ARGS__; } break;   \
            case 3: { constexpr int K = 3; __VA_ARGS__; } break;   \
            case 4: { constexpr int K = 4; __VA_ARGS__; } break;   \
            case 5: { constexpr int K = 5; __VA_ARGS__; } break;   \
            case 6: { constexpr int K = 6; __VA_ARGS__; } break;   \
            case 7: { constexpr int K = 7; __VA_ARGS__; } break;   \
            case 8: { constexpr int K = 8; __VA_ARGS__; } break;   \
            case 10: { constexpr int K = 10; __VA_ARGS__; } break; \
            case 12: { constexpr int K = 12; __VA_ARGS__; } break; \
            case 16: { constexpr int K = 16; __VA_ARGS__; } break; \
            case 20: { constexpr int K = 20; __VA_ARGS__; } break; \
            default:                                            \
                if ((k) < 1 || (k) > MAXK) return -1;           \
                { constexpr int K = 0; __VA_ARGS__; }           \
        }                                                       \
    } while (0)

// The context length of a kernel instance (K > 0: compile-time).
template <int K>
__device__ __forceinline__ int ctx_len(int k) {
    if constexpr (K > 0) return K;
    else return k;
}

// The key of the k query tokens before e (e[-k..-1]); the caller has checked that they lie in one segment.
template <int K>
__device__ __forceinline__ u64 qctx_key(const u16* __restrict__ e, int k) {
    if constexpr (K > 0) return ctx_key<K>(e);
    else {
        bool gap = false;
        return key_finish(ctx_hash_rt(e, k, gap));
    }
}

// One lookup in flight: the corpus position's context key (EMPTY: no lookup), its next token, the slot reached and the
// key read there.
struct Walk {
    u64 key;
    u64 slot;
    u64 seen;
    u32 next;
};

// First half of a lookup of corpus position p: key and next token from its k + 1 tokens (ctx_key_at: EMPTY where a
// gap token is among the k, or the next token is one), then the home slot's load. Splitting the lookup lets a lane
// start several before waiting for any.
template <int K>
__device__ __forceinline__ void walk_begin(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                           u64 vcap, Walk& w) {
    w.key = ctx_key_at<K>(tok, p, k, w.next);
    if (w.next == SENT) w.key = EMPTY;
    if (w.key == EMPTY) return;
    w.slot = __umul64hi(w.key, vcap);
    w.seen = vt[w.slot];
}

// Second half: the walk from the home slot on; the pair key (id << 16 | next) of a verified hit, else EMPTY.
template <int K, bool SORTED>
__device__ __forceinline__ u64 walk_end(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                        const u32* __restrict__ vrep, const u16* __restrict__ x, u32* flags, Walk& w) {
    if (w.key == EMPTY) return EMPTY;
    for (;;) {
        if (w.seen == w.key) break;
        if (w.seen == EMPTY || (SORTED && w.seen > w.key)) return EMPTY;
        w.seen = vt[++w.slot];
    }
    const int kk = ctx_len<K>(k);
    if (kk > 4 && !same_tokens_rt(tok + p, x + (i64)vrep[w.slot] + 1, kk)) {
        atomicAdd(&flags[1], 1u);
        return EMPTY;
    }
    return (w.slot << 16) | w.next;
}

// A whole lookup.
template <int K, bool SORTED>
__device__ __forceinline__ u64 walk_lookup(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                           u64 vcap, const u32* __restrict__ vrep, const u16* __restrict__ x,
                                           u32* flags) {
    Walk w;
    walk_begin<K>(tok, p, k, vt, vcap, w);
    return walk_end<K, SORTED>(tok, p, k, vt, vrep, x, flags, w);
}

// A lookup whose key and next token are already known (the dense scan loads the tokens before the gate bit).
__device__ __forceinline__ void walk_seed(const u64* __restrict__ vt, u64 vcap, u64 key, u32 next, Walk& w) {
    w.key = key;
    w.next = next;
    if (key == EMPTY) return;
    w.slot = __umul64hi(key, vcap);
    w.seen = vt[w.slot];
}

// Lookups that load the home slot and the one after it together (the engine's scans). At the query tables' load most
// walks end within those two slots (a miss does whenever either is empty), so most lookups wait for one round trip
// instead of a chain of dependent slot loads (c3: the level-2 and level-3 scans 8-11% faster). The table must hold at least one slot past vcap (an engine query table has TAIL of them:
// the home slot is below vcap, so slot + 1 is always inside it).
struct Walk2 {
    u64 key;
    u64 slot;
    u64 seen;
    u64 seen2;
    u32 next;
};

__device__ __forceinline__ void walk_seed2(const u64* __restrict__ vt, u64 vcap, u64 key, u32 next, Walk2& w) {
    w.key = key;
    w.next = next;
    if (key == EMPTY) return;
    w.slot = __umul64hi(key, vcap);
    w.seen = vt[w.slot];
    w.seen2 = vt[w.slot + 1];
}

template <int K>
__device__ __forceinline__ void walk_begin2(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                            u64 vcap, Walk2& w) {
    u32 next;
    const u64 key = ctx_key_at<K>(tok, p, k, next);
    walk_seed2(vt, vcap, next == SENT ? EMPTY : key, next, w);
}

// The pair key (id << 16 | next) of a verified hit, else EMPTY; the same result as walk_end on the same table.
template <int K>
__device__ __forceinline__ u64 walk_end2(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                         const u32* __restrict__ vrep, const u16* __restrict__ x, u32* flags,
                                         Walk2& w) {
    if (w.key == EMPTY) return EMPTY;
    if (w.seen == w.key) {
    } else if (w.seen == EMPTY) {
        return EMPTY;
    } else if (w.seen2 == w.key) {
        ++w.slot;
    } else if (w.seen2 == EMPTY) {
        return EMPTY;
    } else {
        w.slot += 2;
        for (;;) {
            const u64 seen = vt[w.slot];
            if (seen == w.key) break;
            if (seen == EMPTY) return EMPTY;
            ++w.slot;
        }
    }
    const int kk = ctx_len<K>(k);
    if (kk > 4 && !same_tokens_rt(tok + p, x + (i64)vrep[w.slot] + 1, kk)) {
        atomicAdd(&flags[1], 1u);
        return EMPTY;
    }
    return (w.slot << 16) | w.next;
}

template <int K>
__device__ __forceinline__ u64 walk_lookup2(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                            u64 vcap, const u32* __restrict__ vrep, const u16* __restrict__ x,
                                            u32* flags) {
    Walk2 w;
    walk_begin2<K>(tok, p, k, vt, vcap, w);
    return walk_end2<K>(tok, p, k, vt, vrep, x, flags, w);
}
