// The training scan's device code shared by the library's two flavours (gpu_val_stats: 40-bit pair keys; record:
// 41-bit pair keys): the pair table, the query-table probe, the level scans and the owner partition.
//
// A pair table slot packs a pair key (context id << 16 | next token) in its low KB bits and the pair's count in the
// top 64 - KB bits (EMPTY = all ones, never a key). A count that wraps past 2^(64-KB) - 1 adds one to the slot's byte
// in `wraps` (u32 words, four slots each), so counts up to 2^(72-KB) - 1 are exact. 2^pbits sub-tables of sub_cap
// slots (sub-table = the key hash's top pbits bits; pbits 0: one table), linear probing within; MAXPROBE probes
// without a slot set flags[0] (the caller reruns the level with a bigger table). A scan whose table has overflowed
// still writes the level's whole hit bitmap, so the levels after it stay exact and only that level reruns.
#pragma once
#include "ngram_common.h"

#ifdef TEST_WRAP  // tests only: every count starts 64 below the count field's wrap (reference .cu:144-148)
#define COUNT_OFF(KB) ((1u << (64 - (KB))) - 64u)
#else
#define COUNT_OFF(KB) 0u
#endif

// Levels with a specialised kernel; every other k in [1, MAXK] runs the generic kernel (K = 0: k at run time).
// k outside [1, MAXK] returns -1.
#define LEVEL_SWITCH(k, ...)                                    \
    switch (k) {                                                \
        case 1: { constexpr int K = 1; __VA_ARGS__; } break;    \
        case 2: { constexpr int K = 2; __VA_ARGS__; } break;    \
        case 3: { constexpr int K = 3; __VA_ARGS__; } break;    \
        case 4: { constexpr int K = 4; __VA_ARGS__; } break;    \
        case 5: { constexpr int K = 5; __VA_ARGS__; } break;    \
        case 6: { constexpr int K = 6; __VA_ARGS__; } break;    \
        case 7: { constexpr int K = 7; __VA_ARGS__; } break;    \
        case 8: { constexpr int K = 8; __VA_ARGS__; } break;    \
        case 10: { constexpr int K = 10; __VA_ARGS__; } break;  \
        case 12: { constexpr int K = 12; __VA_ARGS__; } break;  \
        case 16: { constexpr int K = 16; __VA_ARGS__; } break;  \
        case 20: { constexpr int K = 20; __VA_ARGS__; } break;  \
        default:                                                \
            if (k < 1 || k > MAXK) return -1;                   \
            { constexpr int K = 0; __VA_ARGS__; }               \
            break;                                              \
    }

template <int K>
__device__ __forceinline__ u64 key_at(const u16* e, int k) {
    if constexpr (K > 0) return ctx_key<K>(e);
    else {
        bool gap = false;
        return key_finish(ctx_hash_rt(e, k, gap));
    }
}

template <int K>
__device__ __forceinline__ int klen(int k) {
    if constexpr (K > 0) return K;
    else return k;
}

template <int KB>
struct PairFmt {
    static constexpr u64 MASK = (1ull << KB) - 1;
    static constexpr u64 ONE = 1ull << KB;
    static constexpr u64 CMAX = (1ull << (64 - KB)) - 1;
};

template <int KB>
__device__ __forceinline__ void pair_add(u64* pk, u32* wraps, u64 sub_cap, int pbits, u64 key, u32* flags) {
    typedef PairFmt<KB> F;
    const u64 h = mix64(key);
    const u64 base = pbits ? (h >> (64 - pbits)) * sub_cap : 0;
    u64 s = __umul64hi(pbits ? h << pbits : h, sub_cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 i = base + s;
        u64 cur = pk[i];
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&pk[i], EMPTY, key | (F::ONE * (1ull + COUNT_OFF(KB))));
            if (prev == EMPTY) return;
            cur = prev;
        }
        if ((cur & F::MASK) == key) {
            const u64 old = atomicAdd((unsigned long long*)&pk[i], F::ONE);
            if ((old >> KB) == F::CMAX) atomicAdd(&wraps[i >> 2], 1u << (8 * (i & 3)));
            return;
        }
        s = s + 1 == sub_cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
}

template <int KB>
__device__ __forceinline__ u32 slot_count(const u32* wraps, u64 s, u64 v) {
    return (u32)(v >> KB) + (((wraps[s >> 2] >> (8 * (s & 3))) & 0xFFu) << (64 - KB)) - COUNT_OFF(KB);
}

// The query-table walk of position p's valid key (its next token nxt not SENT): (context id << 16 | nxt) or EMPTY;
// for hashed keys the hit is verified against the context's representative query position (a false hash hit is
// counted in flags[1]). The table (canonical linear probing without wrap-around) ends with an empty slot.
template <int K>
__device__ __forceinline__ u64 probe_table(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                           u64 vcap, const u32* __restrict__ vrep, const u16* __restrict__ x,
                                           u32* flags, u64 key, u32 nxt) {
    u64 s = __umul64hi(key, vcap);
    while (true) {
        const u64 v = vt[s];
        if (v == key) {
            const int kk = klen<K>(k);
            if (kk > 4 && !same_tokens_rt(tok + p, x + (i64)vrep[s] + 1, kk)) {
                atomicAdd(&flags[1], 1u);
                return EMPTY;
            }
            return (s << 16) | nxt;
        }
        if (v == EMPTY) return EMPTY;
        ++s;
    }
}

// Position p's k-context looked up in the query table: (context id << 16 | next) or EMPTY (no context, a gap token,
// or not a query context). Its k + 1 tokens are loaded together (ctx_key_at).
template <int K>
__device__ __forceinline__ u64 probe_key(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt, u64 vcap,
                                         const u32* __restrict__ vrep, const u16* __restrict__ x, u32* flags) {
    u32 nxt;
    const u64 key = ctx_key_at<K>(tok, p, k, nxt);
    if (nxt == SENT || key == EMPTY) return EMPTY;
    return probe_table<K>(tok, p, k, vt, vcap, vrep, x, flags, key, nxt);
}

// A probe in two halves, so that several positions' first loads are in flight together: probe_start computes the
// position's context key (EMPTY: none, or its next token is a gap) and loads its home slot; probe_finish walks on from
// there exactly as probe_key does.
template <int K>
__device__ __forceinline__ void probe_start(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                            u64 vcap, u64& key, u64& s, u64& v, u32& nxt) {
    key = ctx_key_at<K>(tok, p, k, nxt);
    if (nxt == SENT) key = EMPTY;
    if (key == EMPTY) return;
    s = __umul64hi(key, vcap);
    v = vt[s];
}

template <int K>
__device__ __forceinline__ u64 probe_finish(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt,
                                            const u32* __restrict__ vrep, const u16* __restrict__ x, u32* flags,
                                            u64 key, u64 s, u64 v, u32 nxt) {
    if (key == EMPTY) return EMPTY;
    while (true) {
        if (v == key) {
            const int kk = klen<K>(k);
            if (kk > 4 && !same_tokens_rt(tok + p, x + (i64)vrep[s] + 1, kk)) {
                atomicAdd(&flags[1], 1u);
                return EMPTY;
            }
            return (s << 16) | nxt;
        }
        if (v == EMPTY) return EMPTY;
        v = vt[++s];
    }
}

// Dense levels: a lane per position, a wave per 64 positions (two 32-bit bitmap words). Hits are counted directly,
// or with EMIT appended to `emit` (one atomic per wave for its slots).
template <int K, bool EMIT, int KB>
__global__ void __launch_bounds__(256) scan_dense_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                    u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                    const u32* __restrict__ vrep, const u16* __restrict__ x, u64* pk,
                                                    u32* pc, u64 sub_cap, int pbits, u32* flags, u64* emit, u64* emitted) {
    const int lane = lane_id();
    const i64 nwords = (L + 31) >> 5;
    const i64 stride = (i64)gridDim.x * blockDim.x;
    for (i64 base = blockIdx.x * (i64)blockDim.x + (threadIdx.x & ~(WAVE - 1)); base < L; base += stride) {
        // once the pair table has overflowed (the level reruns bigger) only the bitmap is still made
        const bool full = !EMIT && *(volatile u32*)&flags[0] != 0u;
        const i64 p = base + lane;
        const i64 w = (base >> 5) + (lane >> 5);
        u32 word = 0xFFFFFFFFu;
        if (bm_in) word = w < nwords ? bm_in[w] : 0u;
        u64 key = EMPTY;
        if (p < L && ((word >> (lane & 31)) & 1u)) key = probe_key<K>(tok, p, k, vt, vcap, vrep, x, flags);
        const bool hit = key != EMPTY;
        const u64 b = __ballot(hit);
        if (lane == 0) bm_out[base >> 5] = (u32)b;
        if (lane == 32 && w < nwords) bm_out[w] = (u32)(b >> 32);
        if (EMIT) {
            if (b) {
                u64 at = 0;
                if (lane == 0) at = atomicAdd((unsigned long long*)emitted, (unsigned long long)__popcll(b));
                at = bcast_u64(at, 0);
                if (hit) emit[at + __popcll(b & lanemask_lt())] = key;
            }
        } else if (hit && !full) {
            pair_add<KB>(pk, pc, sub_cap, pbits, key, flags);
        }
    }
}

// Sparse levels: a lane per bitmap word, its set bits in turn, counted directly.
template <int K, int KB>
__global__ void __launch_bounds__(256) scan_sparse_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                     u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                     const u32* __restrict__ vrep, const u16* __restrict__ x, u64* pk,
                                                     u32* pc, u64 sub_cap, int pbits, u32* flags) {
    const i64 nwords = (L + 31) >> 5;
    for (i64 w = blockIdx.x * (i64)blockDim.x + threadIdx.x; w < nwords; w += (i64)gridDim.x * blockDim.x) {
        const bool full = *(volatile u32*)&flags[0] != 0u;  // overflowed: only the bitmap is still made
        u32 word = bm_in[w], out = 0;
        while (word) {
            const int b = __ffs(word) - 1;
            word &= word - 1;
            const i64 p = (w << 5) + b;
            if (p >= L) continue;
            const u64 key = probe_key<K>(tok, p, k, vt, vcap, vrep, x, flags);
            if (key != EMPTY) {
                out |= 1u << b;
                if (!full) pair_add<KB>(pk, pc, sub_cap, pbits, key, flags);
            }
        }
        bm_out[w] = out;
    }
}

// Medium density: a wave per 64 bitmap words, a lane per word; each round every lane with bits left probes its next
// set bit, and the round's hits are appended together.
template <int K>
__global__ void __launch_bounds__(256) scan_words_emit_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                         u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                         const u32* __restrict__ vrep, const u16* __restrict__ x,
                                                         u32* flags, u64* emit, u64* emitted) {
    const int lane = lane_id();
    const i64 nwords = (L + 31) >> 5;
    const i64 wave = (blockIdx.x * (i64)blockDim.x + threadIdx.x) >> 6;
    const i64 nwaves = ((i64)gridDim.x * blockDim.x) >> 6;
    for (i64 wbase = wave * WAVE; wbase < nwords; wbase += nwaves * WAVE) {
        const i64 w = wbase + lane;
        u32 word = w < nwords ? bm_in[w] : 0u, out = 0;
        while (__ballot(word != 0u)) {
            u64 key = EMPTY;
            int b = 0;
            if (word) {
                b = __ffs(word) - 1;
                word &= word - 1;
                const i64 p = (w << 5) + b;
                if (p < L) key = probe_key<K>(tok, p, k, vt, vcap, vrep, x, flags);
            }
            const bool hit = key != EMPTY;
            if (hit) out |= 1u << b;
            const u64 m = __ballot(hit);
            if (m) {
                u64 at = 0;
                if (lane == 0) at = atomicAdd((unsigned long long*)emitted, (unsigned long long)__popcll(m));
                at = bcast_u64(at, 0);
                if (hit) emit[at + __popcll(m & lanemask_lt())] = key;
            }
        }
        if (w < nwords) bm_out[w] = out;
    }
}

// ---------------------------------------------------------------------------------------------------------------
// Partitioned aggregation: emitted keys grouped by sub-table in LDS, then counted sub-table by sub-table
// ---------------------------------------------------------------------------------------------------------------

namespace {  // internal linkage: this header is compiled into several objects of one library

__global__ void subpart_count_k(const u64* __restrict__ keys, i64 n, int pbits, u64* counts) {
    extern __shared__ u32 h[];
    const int P = 1 << pbits;
    for (int b = threadIdx.x; b < P; b += blockDim.x) h[b] = 0;
    __syncthreads();
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x)
        atomicAdd(&h[mix64(keys[i]) >> (64 - pbits)], 1u);
    __syncthreads();
    for (int b = threadIdx.x; b < P; b += blockDim.x)
        if (h[b]) atomicAdd((unsigned long long*)&counts[b], (unsigned long long)h[b]);
}

#define SP_ITEMS 16
__global__ void subpart_scatter_k(const u64* __restrict__ keys, i64 n, int pbits, u64* cursor, u64* __restrict__ out) {
    extern __shared__ u32 sm[];
    const int P = 1 << pbits;
    u32* cnt = sm;
    u32* base = sm + P;
    const i64 tile_size = (i64)blockDim.x * SP_ITEMS;
    for (i64 tile = blockIdx.x * tile_size; tile < n; tile += (i64)gridDim.x * tile_size) {
        for (int b = threadIdx.x; b < P; b += blockDim.x) cnt[b] = 0;
        __syncthreads();
        u64 key[SP_ITEMS];
        int o[SP_ITEMS];
        u32 local[SP_ITEMS];
#pragma unroll
        for (int j = 0; j < SP_ITEMS; ++j) {
            const i64 i = tile + (i64)j * blockDim.x + threadIdx.x;
            o[j] = -1;
            if (i < n) {
                key[j] = keys[i];
                o[j] = (int)(mix64(key[j]) >> (64 - pbits));
                local[j] = atomicAdd(&cnt[o[j]], 1u);
            }
        }
        __syncthreads();
        for (int b = threadIdx.x; b < P; b += blockDim.x)
            if (cnt[b]) base[b] = (u32)atomicAdd((unsigned long long*)&cursor[b], (unsigned long long)cnt[b]);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < SP_ITEMS; ++j)
            if (o[j] >= 0) out[(u64)base[o[j]] + local[j]] = key[j];
        __syncthreads();
    }
}

template <int KB>
__global__ void aggregate_k(const u64* __restrict__ keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) {
        if (*(volatile u32*)&flags[0]) return;
        pair_add<KB>(pk, wraps, sub_cap, pbits, keys[i], flags);
    }
}

static int ng_max_pbits() {
    int dev = 0, smem = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 1;
    if (hipDeviceGetAttribute(&smem, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) return 1;
    int b = 1;
    while (b < 14 && (8 << (b + 1)) <= smem) ++b;
    return b;
}

static int set_smem(const void* fn, size_t bytes) {
    if (bytes > 64 * 1024) return (int)hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    return 0;
}

static int launch_subpart_count(const u64* keys, i64 n, int pbits, u64* counts, hipStream_t stream) {
    if (pbits < 1 || pbits > 14) return -1;
    const size_t bytes = 4u << pbits;
    int e = set_smem((const void*)subpart_count_k, bytes);
    if (e) return e;
    if (n > 0) subpart_count_k<<<1024, 256, bytes, stream>>>(keys, n, pbits, counts);
    return (int)hipGetLastError();
}

static int launch_subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, hipStream_t stream) {
    if (pbits < 1 || pbits > 14) return -1;
    const size_t bytes = 8u << pbits;
    int e = set_smem((const void*)subpart_scatter_k, bytes);
    if (e) return e;
    if (n > 0) subpart_scatter_k<<<1024, 256, bytes, stream>>>(keys, n, pbits, cursor, out);
    return (int)hipGetLastError();
}

template <int KB>
static int launch_aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                            hipStream_t stream) {
    if (n > 0)
        aggregate_k<KB><<<grid > 0 ? grid : grid_for(n, 256), 256, 0, stream>>>(keys, n, pk, wraps, sub_cap, pbits,
                                                                                           flags);
    return (int)hipGetLastError();
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// Local aggregation by owner (context-id ranges [bounds[o], bounds[o + 1]))
// ---------------------------------------------------------------------------------------------------------------

__device__ __forceinline__ int owner_of(i64 c, const i64* b, int W) {
    int o = 0;
    while (o + 1 < W && c >= b[o + 1]) ++o;
    return o;
}

template <int KB>
__global__ void part_count_k(const u64* __restrict__ pk, u64 cap, const i64* __restrict__ bounds, int W, u64* counts) {
    __shared__ unsigned long long h[MAXW];
    __shared__ i64 b[MAXW + 1];
    if (threadIdx.x < W) h[threadIdx.x] = 0;
    if (threadIdx.x <= W) b[threadIdx.x] = bounds[threadIdx.x];
    __syncthreads();
    for (u64 s = blockIdx.x * (u64)blockDim.x + threadIdx.x; s < cap; s += (u64)gridDim.x * blockDim.x) {
        const u64 key = pk[s];
        if (key != EMPTY) atomicAdd(&h[owner_of((i64)((key & PairFmt<KB>::MASK) >> 16), b, W)], 1ull);
    }
    __syncthreads();
    if (threadIdx.x < W && h[threadIdx.x]) atomicAdd((unsigned long long*)&counts[threadIdx.x], h[threadIdx.x]);
}

#define PS_ITEMS 8
template <int KB>
__global__ void part_scatter_k(const u64* __restrict__ pk, const u32* __restrict__ pc, u64 cap,
                               const i64* __restrict__ bounds, int W, u64* cursor, u64* __restrict__ ok,
                               u32* __restrict__ oc) {
    __shared__ u32 cnt[MAXW];
    __shared__ unsigned long long base[MAXW];
    __shared__ i64 b[MAXW + 1];
    if (threadIdx.x <= W) b[threadIdx.x] = bounds[threadIdx.x];
    const u64 tile_size = (u64)blockDim.x * PS_ITEMS;
    for (u64 tile = blockIdx.x * tile_size; tile < cap; tile += (u64)gridDim.x * tile_size) {
        if (threadIdx.x < W) cnt[threadIdx.x] = 0;
        __syncthreads();
        u64 key[PS_ITEMS];
        int o[PS_ITEMS];
        u32 local[PS_ITEMS];
#pragma unroll
        for (int j = 0; j < PS_ITEMS; ++j) {
            const u64 s = tile + (u64)j * blockDim.x + threadIdx.x;
            key[j] = s < cap ? pk[s] : EMPTY;
            o[j] = -1;
            if (key[j] != EMPTY) {
                o[j] = owner_of((i64)((key[j] & PairFmt<KB>::MASK) >> 16), b, W);
                local[j] = atomicAdd(&cnt[o[j]], 1u);
            }
        }
        __syncthreads();
        if (threadIdx.x < W && cnt[threadIdx.x])
            base[threadIdx.x] = atomicAdd((unsigned long long*)&cursor[threadIdx.x], (unsigned long long)cnt[threadIdx.x]);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PS_ITEMS; ++j) {
            if (o[j] >= 0) {
                const u64 s = tile + (u64)j * blockDim.x + threadIdx.x;
                const u64 d = base[o[j]] + local[j];
                ok[d] = key[j] & PairFmt<KB>::MASK;
                oc[d] = slot_count<KB>(pc, s, key[j]);
            }
        }
        __syncthreads();
    }
}

template <int KB>
static int launch_part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, hipStream_t st) {
    if (W < 1 || W > MAXW) return -1;
    if (cap > 0) part_count_k<KB><<<2048, 256, 0, st>>>(pk, cap, bounds, W, counts);
    return (int)hipGetLastError();
}

template <int KB>
static int launch_part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                               u32* oc, hipStream_t st) {
    if (W < 1 || W > MAXW) return -1;
    if (cap > 0) part_scatter_k<KB><<<4096, 256, 0, st>>>(pk, pc, cap, bounds, W, cursor, ok, oc);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Owner side shared by the flavours
// ---------------------------------------------------------------------------------------------------------------

namespace ng {
// Per query position whose context id is in [lo, hi): tot, dist and cnt (the target's count; with rank_of, only if
// its rank is below cnt_top), and bit `li` of mask (if mask) where the context occurred. Defined in common_abi.hip.
int launch_pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                       const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                       int* out_tot, int* out_dist, int* out_cnt, int* mask, hipStream_t st);
// The rank of each pair within its context (if rank_of) and the top `top` tokens/counts per context (if top_tok).
int launch_rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                        u16* top_tok, u32* top_cnt, int top, hipStream_t st);
}  // namespace ng
