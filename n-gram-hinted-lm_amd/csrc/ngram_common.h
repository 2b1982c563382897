// Shared device code of the n-gram hint engine (gfx950, wave64): types, the context key, wave helpers.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

typedef unsigned long long u64;
typedef unsigned int u32;
typedef unsigned short u16;
typedef long long i64;

#define EMPTY 0xFFFFFFFFFFFFFFFFull
#define SENT 0xFFFFu
#define NG_BOS 50256u
#define MAXPROBE 4096
#define MAXW 64
#define MAXK 64
#define WAVE 64

// SplitMix64's finalizer (Steele, Lea & Flood 2014): a bijection of u64.
__host__ __device__ __forceinline__ u64 mix64(u64 h) {
    h ^= h >> 30;
    h *= 0xbf58476d1ce4e5b9ull;
    h ^= h >> 27;
    h *= 0x94d049bb133111ebull;
    return h ^ (h >> 31);
}

// A token's 64-bit code for the polynomial key of contexts longer than four tokens (odd: never a zero term).
__host__ __device__ __forceinline__ u64 tok_code(u32 t) { return mix64((u64)(t + 1) * 0x9E3779B97F4A7C15ull) | 1ull; }

#define POLY_BASE 0xD6E8FEB86659FD93ull

// The key of the K tokens ending just before `e` (e[-K..-1]): for K <= 4 the tokens packed 16 bits each (exact), else
// the polynomial sum_j code(e[-j]) * B^(j-1), j = 1..K; both through mix64. EMPTY is reserved (a key equal to it
// becomes EMPTY - 1). Built backward from e[-1], so that ctx_key_stop can stop at the first SENT.
__host__ __device__ __forceinline__ u64 key_finish(u64 h) {
    const u64 k = mix64(h);
    return k == EMPTY ? EMPTY - 1 : k;
}

template <int K>
__device__ __forceinline__ u64 ctx_key(const u16* e) {
    u64 h = 0, bp = 1;
#pragma unroll
    for (int j = 1; j <= K; ++j) {
        const u32 t = e[-j];
        if (K <= 4) h |= (u64)t << (16 * (j - 1));
        else {
            h += tok_code(t) * bp;
            bp *= POLY_BASE;
        }
    }
    return key_finish(h);
}

__host__ __device__ __forceinline__ u64 ctx_key_rt(const u16* e, int k) {
    u64 h = 0, bp = 1;
    for (int j = 1; j <= k; ++j) {
        const u32 t = e[-j];
        if (k <= 4) h |= (u64)t << (16 * (j - 1));
        else {
            h += tok_code(t) * bp;
            bp *= POLY_BASE;
        }
    }
    return key_finish(h);
}

// ctx_key for corpus positions: stops at the first SENT met going backward and returns EMPTY (such a context holds a
// gap token, so it is no query context). A buffer that starts with a SENT token is therefore never read before its
// start, whatever k.
template <int K>
__device__ __forceinline__ u64 ctx_key_stop(const u16* e, int k) {
    u64 h = 0, bp = 1;
    if constexpr (K > 0) {
#pragma unroll
        for (int j = 1; j <= K; ++j) {
            const u32 t = e[-j];
            if (t == SENT) return EMPTY;
            if (K <= 4) h |= (u64)t << (16 * (j - 1));
            else {
                h += tok_code(t) * bp;
                bp *= POLY_BASE;
            }
        }
    } else {
        for (int j = 1; j <= k; ++j) {
            const u32 t = e[-j];
            if (t == SENT) return EMPTY;
            if (k <= 4) h |= (u64)t << (16 * (j - 1));
            else {
                h += tok_code(t) * bp;
                bp *= POLY_BASE;
            }
        }
    }
    return key_finish(h);
}

// ctx_key's sum (before key_finish) of the k tokens before e for a run-time k, the tokens loaded 8 at a time (each
// group's loads in flight together: no load waits for another's value); gap |= any of them is SENT.
__device__ __forceinline__ u64 ctx_hash_rt(const u16* __restrict__ e, int k, bool& gap) {
    u64 h = 0, bp = 1;
    int j = 1;
    for (; j + 7 <= k; j += 8) {
        u32 t[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) t[q] = e[-(j + q)];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            gap |= t[q] == SENT;
            if (k <= 4) h |= (u64)t[q] << (16 * (j + q - 1));
            else {
                h += tok_code(t[q]) * bp;
                bp *= POLY_BASE;
            }
        }
    }
    for (; j <= k; ++j) {
        const u32 t = e[-j];
        gap |= t == SENT;
        if (k <= 4) h |= (u64)t << (16 * (j - 1));
        else {
            h += tok_code(t) * bp;
            bp *= POLY_BASE;
        }
    }
    return h;
}

// The k tokens before a and before b equal (run-time k; loaded 8 pairs at a time).
__device__ __forceinline__ bool same_tokens_rt(const u16* __restrict__ a, const u16* __restrict__ b, int k) {
    bool same = true;
    int j = 1;
    for (; j + 7 <= k; j += 8) {
        u32 ta[8], tb[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) ta[q] = a[-(j + q)], tb[q] = b[-(j + q)];
#pragma unroll
        for (int q = 0; q < 8; ++q) same &= ta[q] == tb[q];
    }
    for (; j <= k; ++j) same &= a[-j] == b[-j];
    return same;
}

// Position p's next token (nxt = tok[p]) and k-context key (tok[p - k .. p - 1]) as ctx_key_stop's, with all k + 1
// tokens loaded together (no load waits for another token's value): EMPTY where any of the k is SENT. A token before
// the buffer's start (p - j < 0) reads as SENT, which is what ctx_key_stop meets there too (the buffer starts with
// SENT, or the token before it is one); nothing before the buffer is read.
template <int K>
__device__ __forceinline__ u64 ctx_key_at(const u16* __restrict__ tok, i64 p, int k, u32& nxt) {
    if constexpr (K > 0) {
        u32 t[K + 1];
#pragma unroll
        for (int j = 0; j <= K; ++j) t[j] = p - j >= 0 ? (u32)tok[p - j] : SENT;
        nxt = t[0];
        u64 h = 0, bp = 1;
        bool gap = false;
#pragma unroll
        for (int j = 1; j <= K; ++j) {
            gap |= t[j] == SENT;
            if (K <= 4) h |= (u64)t[j] << (16 * (j - 1));
            else {
                h += tok_code(t[j]) * bp;
                bp *= POLY_BASE;
            }
        }
        return gap ? EMPTY : key_finish(h);
    } else {
        nxt = tok[p];
        if (p < k) return EMPTY;
        bool gap = false;
        const u64 h = ctx_hash_rt(tok + p, k, gap);
        return gap ? EMPTY : key_finish(h);
    }
}

// Launch helpers
static inline int grid_for(i64 n, int block) {
    i64 g = (n + block - 1) / block;
    if (g < 1) g = 1;
    if (g > (1 << 30)) g = 1 << 30;
    return (int)g;
}

// A workgroup barrier ordering LDS accesses only: unlike __syncthreads it does not wait for the wave's outstanding
// global stores (a block that scatters results to global memory between LDS phases would otherwise wait for each
// phase's writes to complete).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave helpers (wave64)
__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & (WAVE - 1)); }
__device__ __forceinline__ u64 lanemask_lt() { return (1ull << lane_id()) - 1ull; }

__device__ __forceinline__ u64 bcast_u64(u64 v, int src) {
    u32 lo = (u32)__shfl((int)(u32)v, src, WAVE);
    u32 hi = (u32)__shfl((int)(u32)(v >> 32), src, WAVE);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u64 shfl_up_u64(u64 v, int d) {
    u32 lo = (u32)__shfl_up((int)(u32)v, d, WAVE);
    u32 hi = (u32)__shfl_up((int)(u32)(v >> 32), d, WAVE);
    return ((u64)hi << 32) | lo;
}

__device__ __forceinline__ u64 shfl_down_u64(u64 v, int d) {
    u32 lo = (u32)__shfl_down((int)(u32)v, d, WAVE);
    u32 hi = (u32)__shfl_down((int)(u32)(v >> 32), d, WAVE);
    return ((u64)hi << 32) | lo;
}

// Wave-wide segmented inclusive sum of `v` over runs of equal `seg` (which must be non-decreasing across lanes, or at
// least equal within each run of consecutive lanes). Returns the running sum of the lane's run up to the lane.
__device__ __forceinline__ u64 wave_seg_sum(u64 v, u64 seg) {
    const int lane = lane_id();
    const u64 prev = shfl_up_u64(seg, 1);
    bool head = lane == 0 || prev != seg;
    u64 heads = __ballot(head);
    // distance back to the run's head
    u64 below = heads & ((lane == 63) ? ~0ull : ((1ull << (lane + 1)) - 1ull));
    int start = 63 - __clzll(below);
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        u64 o = shfl_up_u64(v, d);
        if (lane - d >= start) v += o;
    }
    return v;
}

// Is the lane the last of its run of equal `seg` within the wave?
__device__ __forceinline__ bool wave_seg_tail(u64 seg, bool valid_next) {
    const int lane = lane_id();
    const u64 nxt = shfl_down_u64(seg, 1);
    return lane == WAVE - 1 || !valid_next || nxt != seg;
}

// top-k insertion of a score (count << 16 | (65535 - token): larger = ranked higher) into a descending list (static
// indices only: the list stays in registers)
template <int KT>
__device__ __forceinline__ void topk_insert(u64 (&t)[KT], u64 v) {
#pragma unroll
    for (int j = 0; j < KT; ++j)
        if (v > t[j]) {
            const u64 tmp = t[j];
            t[j] = v;
            v = tmp;
        }
}

// The ranking score of pair key (context << 16 | token) with count n: count descending, then token ascending.
__device__ __forceinline__ u64 rank_score(u64 key, u32 n) { return ((u64)n << 16) | (0xFFFFu - (u32)(key & 0xFFFF)); }

// A corpus-wide context table (u64 keys, slot = context id, linear probing with wrap-around from umulhi(key, cap)):
// the slot of `key`, inserted if absent, or -1 after MAXPROBE probes (flags[0] |= 2).
__device__ __forceinline__ i64 ctx_find_insert(u64* ck, u64 ccap, u64 key, u32* flags) {
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

// The slot of `key` in such a table, or -1.
__device__ __forceinline__ i64 ctx_find(const u64* __restrict__ ck, u64 ccap, u64 key) {
    u64 s = __umul64hi(key, ccap);
    for (u64 probe = 0; probe < ccap; ++probe) {
        const u64 cur = ck[s];
        if (cur == key) return (i64)s;
        if (cur == EMPTY) return -1;
        s = s + 1 == ccap ? 0 : s + 1;
    }
    return -1;
}
