// The gpu_val_stats C ABI on gfx950: the entry points old_records/gpu_val_stats.py's `Lib` binds
// (old_records/gpu_val_stats.cu:96-699), same names, argument meaning, return codes and device-side flags, written
// for CDNA4: wave64 (a wave scans 64 positions = two of the ABI's 32-bit bitmap words), 64-bit ballots, LDS
// histograms sized for 160 KB of LDS, and our own device-wide sort/scan/reduce (prim.hip) behind the CUB-style
// two-phase temp-storage calls.
//
// Semantics (old_records/gpu_val_stats.cu:5-13): the training shards are concatenated with >= 32 SENT (0xFFFF) tokens
// before each shard; a corpus position p is an occurrence of the k tokens before it with next token tok[p]; a position
// whose next token is SENT is skipped and a context holding a SENT matches no query context, so no context crosses a
// shard. Query contexts are hashed (ngram_common.h ctx_key); a hashed key's hit (k > 4) is compared token by token with
// the context's representative query position, so counts are exact.
#include "ngram_common.h"
#include "prim.h"

#define KEYBITS 40
#define KEYMASK ((1ull << KEYBITS) - 1)
#define ONE (1ull << KEYBITS)
#ifdef TEST_WRAP  // tests only: every count starts 64 below the 24-bit wrap (reference .cu:144-148)
#define COUNT_OFF ((1u << (64 - KEYBITS)) - 64u)
#else
#define COUNT_OFF 0u
#endif

// Levels with a specialised kernel (the reference's LEVEL_SWITCH, .cu:61-76); every other k in [1, MAXK] runs the
// generic kernel (K = 0: k at run time). k outside [1, MAXK] returns -1.
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
    else return ctx_key_rt(e, k);
}

template <int K>
__device__ __forceinline__ int klen(int k) {
    if constexpr (K > 0) return K;
    else return k;
}

// ---------------------------------------------------------------------------------------------------------------
// Query side
// ---------------------------------------------------------------------------------------------------------------

template <int K>
__global__ void val_keys_k(const u16* __restrict__ x, const int* __restrict__ avail, i64 n, int k, u64* __restrict__ out) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = avail[i] >= klen<K>(k) ? key_at<K>(x + i + 1, k) : EMPTY;
}

extern "C" int val_keys(const u16* x, const int* avail, i64 n, int k, u64* out, void* stream) {
    if (n <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    LEVEL_SWITCH(k, (val_keys_k<K><<<grid_for(n, 256), 256, 0, st>>>(x, avail, n, k, out)));
    return (int)hipGetLastError();
}

__global__ void val_verify_k(const u16* __restrict__ x, const i64* __restrict__ spos, const i64* __restrict__ gid,
                             const i64* __restrict__ rep, i64 n, int k, u64* bad) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const i64 p = spos[i], r = rep[gid[i]];
    for (int j = 0; j < k; ++j)
        if (x[p - j] != x[r - j]) {
            atomicAdd((unsigned long long*)bad, 1ull);
            return;
        }
}

extern "C" int val_verify(const u16* x, const i64* spos, const i64* gid, const i64* rep, i64 n, int k, u64* bad,
                          void* stream) {
    if (n <= 0) return 0;
    val_verify_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(x, spos, gid, rep, n, k, bad);
    return (int)hipGetLastError();
}

__global__ void val_homes_k(const u64* __restrict__ keys, i64 n, u64 cap, i64* __restrict__ home) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < n) home[i] = (i64)__umul64hi(keys[i], cap);
}

extern "C" int val_homes(const u64* keys, i64 n, u64 cap, i64* home, void* stream) {
    if (n > 0) val_homes_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(keys, n, cap, home);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Training scan
// ---------------------------------------------------------------------------------------------------------------

// Open-addressing (pair key -> count) insert: slot = key (40 bits) | count (24 bits); a count wrapping past 2^24 - 1
// bumps the slot's byte in `wraps`. 2^pbits sub-tables of sub_cap slots (sub-table = the hash's top pbits bits);
// linear probing within; MAXPROBE probes without a slot set flags[0] (the caller reruns the level bigger).
__device__ __forceinline__ void pair_add(u64* pk, u32* wraps, u64 sub_cap, int pbits, u64 key, u32* flags) {
    const u64 h = mix64(key);
    const u64 base = pbits ? (h >> (64 - pbits)) * sub_cap : 0;
    u64 s = __umul64hi(h << pbits, sub_cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 i = base + s;
        u64 cur = pk[i];
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&pk[i], EMPTY, key | (ONE * (1ull + COUNT_OFF)));
            if (prev == EMPTY) return;
            cur = prev;
        }
        if ((cur & KEYMASK) == key) {
            const u64 old = atomicAdd((unsigned long long*)&pk[i], ONE);
            if ((old >> KEYBITS) == (1ull << (64 - KEYBITS)) - 1) atomicAdd(&wraps[i >> 2], 1u << (8 * (i & 3)));
            return;
        }
        s = s + 1 == sub_cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
}

__device__ __forceinline__ u32 slot_count(const u32* wraps, u64 s, u64 v) {
    return (u32)(v >> KEYBITS) + (((wraps[s >> 2] >> (8 * (s & 3))) & 0xFFu) << (64 - KEYBITS)) - COUNT_OFF;
}

// Position p's k-context looked up in the query table and, for hashed keys, verified: (context id << 16 | next) or
// EMPTY. The table (canonical linear probing without wrap-around) ends with an empty slot.
template <int K>
__device__ __forceinline__ u64 probe_key(const u16* __restrict__ tok, i64 p, int k, const u64* __restrict__ vt, u64 vcap,
                                         const u32* __restrict__ vrep, const u16* __restrict__ x, u32* flags) {
    const u32 nxt = tok[p];
    if (nxt == SENT) return EMPTY;
    const u64 key = ctx_key_stop<K>(tok + p, k);
    if (key == EMPTY) return EMPTY;
    u64 s = __umul64hi(key, vcap);
    while (true) {
        const u64 v = vt[s];
        if (v == key) {
            const int kk = klen<K>(k);
            if (kk > 4) {
                const u16* a = tok + p - kk;
                const u16* b = x + (i64)vrep[s] + 1 - kk;
                bool same = true;
                for (int j = 0; j < kk; ++j) same &= a[j] == b[j];
                if (!same) {
                    atomicAdd(&flags[1], 1u);
                    return EMPTY;
                }
            }
            return (s << 16) | nxt;
        }
        if (v == EMPTY) return EMPTY;
        ++s;
    }
}

// Dense levels: a lane per position, a wave per 64 positions (two bitmap words). Hits are counted directly, or with
// EMIT appended to `emit` (one atomic per wave for its slots).
template <int K, bool EMIT>
__global__ void __launch_bounds__(256) scan_dense_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                    u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                    const u32* __restrict__ vrep, const u16* __restrict__ x, u64* pk,
                                                    u32* pc, u64 sub_cap, int pbits, u32* flags, u64* emit, u64* emitted) {
    const int lane = lane_id();
    const i64 nwords = (L + 31) >> 5;
    const i64 stride = (i64)gridDim.x * blockDim.x;
    for (i64 base = blockIdx.x * (i64)blockDim.x + (threadIdx.x & ~(WAVE - 1)); base < L; base += stride) {
        const u32 stop = *(volatile u32*)&flags[0];  // the pair table overflowed: the level reruns
        if (__ballot(stop != 0u)) break;
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
        } else if (hit) {
            pair_add(pk, pc, sub_cap, pbits, key, flags);
        }
    }
}

// Sparse levels: a lane per bitmap word, its set bits in turn, counted directly.
template <int K>
__global__ void __launch_bounds__(256) scan_sparse_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                     u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                     const u32* __restrict__ vrep, const u16* __restrict__ x, u64* pk,
                                                     u32* pc, u64 sub_cap, int pbits, u32* flags) {
    const i64 nwords = (L + 31) >> 5;
    for (i64 w = blockIdx.x * (i64)blockDim.x + threadIdx.x; w < nwords; w += (i64)gridDim.x * blockDim.x) {
        if (*(volatile u32*)&flags[0]) break;
        u32 word = bm_in[w], out = 0;
        while (word) {
            const int b = __ffs(word) - 1;
            word &= word - 1;
            const i64 p = (w << 5) + b;
            if (p >= L) continue;
            const u64 key = probe_key<K>(tok, p, k, vt, vcap, vrep, x, flags);
            if (key != EMPTY) {
                out |= 1u << b;
                pair_add(pk, pc, sub_cap, pbits, key, flags);
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

// mode 0: dense, counted directly; 1: sparse, counted directly; 2: dense, emitted; 3: by words, emitted
extern "C" int scan_level(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                          const u32* vrep, const u16* x, u64* pk, u32* pc, u64 sub_cap, int pbits, u32* flags, int grid,
                          int mode, u64* emit, u64* emitted, void* stream) {
    if (L <= 0) return 0;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    if (mode == 1 && bm_in) {
        LEVEL_SWITCH(k, (scan_sparse_k<K><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags)));
    } else if (mode == 3 && bm_in) {
        LEVEL_SWITCH(k, (scan_words_emit_k<K><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, emit, emitted)));
    } else if (mode == 2) {
        LEVEL_SWITCH(k, (scan_dense_k<K, true><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags, emit, emitted)));
    } else {
        LEVEL_SWITCH(k, (scan_dense_k<K, false><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags, emit, emitted)));
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Partitioned aggregation: emitted keys grouped by sub-table in LDS, then counted sub-table by sub-table
// ---------------------------------------------------------------------------------------------------------------

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

__global__ void aggregate_k(const u64* __restrict__ keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) {
        if (*(volatile u32*)&flags[0]) return;
        pair_add(pk, wraps, sub_cap, pbits, keys[i], flags);
    }
}

extern "C" int max_pbits() {
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

extern "C" int subpart_count(const u64* keys, i64 n, int pbits, u64* counts, void* stream) {
    if (pbits < 1 || pbits > 14) return -1;
    const size_t bytes = 4u << pbits;
    int e = set_smem((const void*)subpart_count_k, bytes);
    if (e) return e;
    if (n > 0) subpart_count_k<<<1024, 256, bytes, (hipStream_t)stream>>>(keys, n, pbits, counts);
    return (int)hipGetLastError();
}

extern "C" int subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, void* stream) {
    if (pbits < 1 || pbits > 14) return -1;
    const size_t bytes = 8u << pbits;
    int e = set_smem((const void*)subpart_scatter_k, bytes);
    if (e) return e;
    if (n > 0) subpart_scatter_k<<<1024, 256, bytes, (hipStream_t)stream>>>(keys, n, pbits, cursor, out);
    return (int)hipGetLastError();
}

extern "C" int aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                         void* stream) {
    if (n > 0)
        aggregate_k<<<grid > 0 ? grid : grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(keys, n, pk, wraps, sub_cap, pbits,
                                                                                           flags);
    return (int)hipGetLastError();
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) v += shfl_down_u64(v, d);
    return v;
}

__global__ void popcount_k(const u32* __restrict__ bm, i64 n, u64* out) {
    u64 c = 0;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) c += __popc(bm[i]);
    c = wave_sum_u64(c);
    if (lane_id() == 0 && c) atomicAdd((unsigned long long*)out, (unsigned long long)c);
}

extern "C" int popcount(const u32* bm, i64 n, u64* out, void* stream) {
    if (n > 0) popcount_k<<<1024, 256, 0, (hipStream_t)stream>>>(bm, n, out);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Local aggregation by owner (context-id ranges [bounds[o], bounds[o + 1]))
// ---------------------------------------------------------------------------------------------------------------

__device__ __forceinline__ int owner_of(i64 c, const i64* b, int W) {
    int o = 0;
    while (o + 1 < W && c >= b[o + 1]) ++o;
    return o;
}

__global__ void part_count_k(const u64* __restrict__ pk, u64 cap, const i64* __restrict__ bounds, int W, u64* counts) {
    __shared__ unsigned long long h[MAXW];
    __shared__ i64 b[MAXW + 1];
    if (threadIdx.x < W) h[threadIdx.x] = 0;
    if (threadIdx.x <= W) b[threadIdx.x] = bounds[threadIdx.x];
    __syncthreads();
    for (u64 s = blockIdx.x * (u64)blockDim.x + threadIdx.x; s < cap; s += (u64)gridDim.x * blockDim.x) {
        const u64 key = pk[s];
        if (key != EMPTY) atomicAdd(&h[owner_of((i64)((key & KEYMASK) >> 16), b, W)], 1ull);
    }
    __syncthreads();
    if (threadIdx.x < W && h[threadIdx.x]) atomicAdd((unsigned long long*)&counts[threadIdx.x], h[threadIdx.x]);
}

extern "C" int part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, void* stream) {
    if (W < 1 || W > MAXW) return -1;
    part_count_k<<<2048, 256, 0, (hipStream_t)stream>>>(pk, cap, bounds, W, counts);
    return (int)hipGetLastError();
}

#define PS_ITEMS 8
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
                o[j] = owner_of((i64)((key[j] & KEYMASK) >> 16), b, W);
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
                ok[d] = key[j] & KEYMASK;
                oc[d] = slot_count(pc, s, key[j]);
            }
        }
        __syncthreads();
    }
}

extern "C" int part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                            u32* oc, void* stream) {
    if (W < 1 || W > MAXW) return -1;
    part_scatter_k<<<4096, 256, 0, (hipStream_t)stream>>>(pk, pc, cap, bounds, W, cursor, ok, oc);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Owner side: sorts and reductions (CUB-style two-phase temp storage), segments, ranks, outputs
// ---------------------------------------------------------------------------------------------------------------

extern "C" int sort_pairs(void* temp, size_t* temp_bytes, const u64* kin, u64* kout, const u32* vin, u32* vout, i64 n,
                          int begin_bit, int end_bit, void* stream) {
    if (!temp_bytes) return -1;
    const size_t need = prim::radix_sort_temp_bytes(n, vin != nullptr);
    if (!temp) {
        *temp_bytes = need;
        return 0;
    }
    return prim::radix_sort_pairs(kin, kout, vin, vout, n, begin_bit, end_bit, temp, *temp_bytes, (hipStream_t)stream);
}

extern "C" int inclusive_max(void* temp, size_t* temp_bytes, const i64* in, i64* out, i64 n, void* stream) {
    if (!temp_bytes) return -1;
    const size_t need = prim::max_i64_temp_bytes(n);
    if (!temp) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need) return -1;
    return prim::inclusive_max_i64(in, out, n, temp, (hipStream_t)stream);
}

extern "C" int reduce_by_key(void* temp, size_t* temp_bytes, const u64* kin, u64* kout, const u32* vin, u32* vout,
                             i64* nruns, i64 n, void* stream) {
    if (!temp_bytes) return -1;
    const size_t need = prim::reduce_by_key_temp_bytes(n);
    if (!temp) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need) return -1;
    return prim::reduce_by_key(kin, kout, vin, vout, nruns, n, temp, (hipStream_t)stream);
}

__global__ void seg_bounds_k(const u64* __restrict__ uk, i64 U, i64* __restrict__ start, i64* __restrict__ end) {
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= U) return;
    const u64 c = uk[j] >> 16;
    if (j == 0 || (uk[j - 1] >> 16) != c) start[c] = j;
    if (j == U - 1 || (uk[j + 1] >> 16) != c) end[c] = j + 1;
}

extern "C" int seg_bounds(const u64* uk, i64 U, i64* start, i64* end, void* stream) {
    if (U > 0) seg_bounds_k<<<grid_for(U, 256), 256, 0, (hipStream_t)stream>>>(uk, U, start, end);
    return (int)hipGetLastError();
}

// A lane per context; contexts with many pairs are summed by the whole wave in turn.
__global__ void ctx_tot_k(const i64* __restrict__ start, const i64* __restrict__ end, const u32* __restrict__ agg,
                          i64 nctx, u64* __restrict__ tot) {
    const int lane = lane_id();
    const i64 wave = (blockIdx.x * (i64)blockDim.x + threadIdx.x) >> 6;
    const i64 nwaves = ((i64)gridDim.x * blockDim.x) >> 6;
    for (i64 c0 = wave * WAVE; c0 < nctx; c0 += nwaves * WAVE) {
        const i64 c = c0 + lane;
        i64 a = 0, b = 0;
        if (c < nctx) {
            a = start[c];
            b = end[c];
        }
        const bool big = b - a > 64;
        u64 s = 0;
        if (!big)
            for (i64 j = a; j < b; ++j) s += agg[j];
        u64 bigs = __ballot(big);
        while (bigs) {
            const int l = __ffsll((unsigned long long)bigs) - 1;
            bigs &= bigs - 1;
            const i64 ba = (i64)bcast_u64((u64)a, l), bb = (i64)bcast_u64((u64)b, l);
            u64 part = 0;
            for (i64 j = ba + lane; j < bb; j += WAVE) part += agg[j];
            part = wave_sum_u64(part);
            part = bcast_u64(part, 0);
            if (lane == l) s = part;
        }
        if (c < nctx) tot[c] = s;
    }
}

extern "C" int ctx_tot(const i64* start, const i64* end, const u32* agg, i64 nctx, u64* tot, void* stream) {
    if (nctx > 0) {
        int g = grid_for(nctx, 256);
        ctx_tot_k<<<g > 16384 ? 16384 : g, 256, 0, (hipStream_t)stream>>>(start, end, agg, nctx, tot);
    }
    return (int)hipGetLastError();
}

// The ranking key: context, then count descending; a stable sort keeps the token order (ascending) of ties.
__global__ void rank_keys_k(const u64* __restrict__ uk, const u32* __restrict__ agg, i64 U, u64* __restrict__ key2,
                            u32* __restrict__ val2) {
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= U) return;
    key2[j] = ((uk[j] >> 16) << 32) | (u64)(0xFFFFFFFFu - agg[j]);
    val2[j] = (u32)j;
}

extern "C" int rank_keys(const u64* uk, const u32* agg, i64 U, u64* key2, u32* val2, void* stream) {
    if (U > 0) rank_keys_k<<<grid_for(U, 256), 256, 0, (hipStream_t)stream>>>(uk, agg, U, key2, val2);
    return (int)hipGetLastError();
}

__global__ void rank_scatter_k(const u32* __restrict__ sv, i64 U, const u64* __restrict__ uk, const u32* __restrict__ agg,
                               const i64* __restrict__ start, u32* __restrict__ rank_of, u16* __restrict__ top_tok,
                               u32* __restrict__ top_cnt, int top) {
    const i64 q = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (q >= U) return;
    const u32 j = sv[q];
    const u64 c = uk[j] >> 16;
    const i64 r = q - start[c];
    rank_of[j] = (u32)r;
    if (top_tok && r < top) {
        top_tok[c * top + r] = (u16)(uk[j] & 0xFFFF);
        top_cnt[c * top + r] = agg[j];
    }
}

extern "C" int rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                            u16* top_tok, u32* top_cnt, int top, void* stream) {
    if (U > 0)
        rank_scatter_k<<<grid_for(U, 256), 256, 0, (hipStream_t)stream>>>(sv, U, uk, agg, start, rank_of, top_tok,
                                                                            top_cnt, top);
    return (int)hipGetLastError();
}

// Per query position whose context id is in [lo, hi): tot, dist and cnt (the target's count if among the context's
// cnt_top most frequent next tokens), and bit `li` of mask where the context occurred.
__global__ void pos_outputs_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi, const u16* __restrict__ tgt,
                              const u64* __restrict__ uk, const u32* __restrict__ agg, const u32* __restrict__ rank_of,
                              const i64* __restrict__ start, const i64* __restrict__ end, const u64* __restrict__ tot,
                              int li, int cnt_top, int* __restrict__ out_tot, int* __restrict__ out_dist,
                              int* __restrict__ out_cnt, int* __restrict__ mask) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    i64 c = ctx_of[i];
    if (c < lo || c >= hi) return;
    c -= lo;
    i64 a = start[c], b = end[c];
    if (b <= a) return;
    out_tot[i] = (int)(u32)tot[c];
    out_dist[i] = (int)(b - a < 65535 ? b - a : 65535);
    const u64 want = ((u64)c << 16) | tgt[i];
    while (a < b) {
        const i64 m = (a + b) >> 1;
        if (uk[m] < want) a = m + 1;
        else b = m;
    }
    if (a < end[c] && uk[a] == want && rank_of[a] < (u32)cnt_top) out_cnt[i] = (int)agg[a];
    mask[i] |= 1 << li;
}

extern "C" int pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                           const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                           int* out_tot, int* out_dist, int* out_cnt, int* mask, void* stream) {
    if (N > 0)
        pos_outputs_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, N, lo, hi, tgt, uk, agg, rank_of, start,
                                                                          end, tot, li, cnt_top, out_tot, out_dist,
                                                                          out_cnt, mask);
    return (int)hipGetLastError();
}

// One hint variant's rows (old_records._val_rows with one slot, .cu:646-694): per position its deepest level of the
// variant whose context occurred (mask), if this rank owns that context: cell, top-8 tokens and weights packed in 9
// int32. desc[v * 8 + ...]: mask bit, length bucket, ctx_of pointer, lo, hi, top tokens, top counts, totals pointer.
__constant__ double PURITY_EDGES[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
__constant__ u64 COUNT_EDGES[6] = {2, 3, 5, 9, 17, 33};

__global__ void variant_rows_k(i64 N, const int* __restrict__ mask, int nv, const i64* __restrict__ desc, int* __restrict__ rows) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int m = mask[i];
    for (int v = nv - 1; v >= 0; --v) {
        const i64* d = desc + v * 8;
        if (!((m >> d[0]) & 1)) continue;
        const int* ctx_of = (const int*)d[2];
        i64 c = ctx_of[i];
        if (c < d[3] || c >= d[4]) return;  // another rank's context
        c -= d[3];
        const u16* tt = (const u16*)d[5] + c * 8;
        const u32* tc = (const u32*)d[6] + c * 8;
        const u64 total = ((const u64*)d[7])[c];
        u32 cnt[8];
        double sum = 0;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            cnt[r] = tc[r];
            sum += (double)cnt[r];
        }
        int count_bin = 0;
#pragma unroll
        for (int e = 0; e < 6; ++e) count_bin += COUNT_EDGES[e] <= total;
        const double share = (double)cnt[0] / (double)(total > 1 ? total : 1);
        int purity_bin = 0;
#pragma unroll
        for (int e = 0; e < 5; ++e) purity_bin += PURITY_EDGES[e] <= share;
        const int cell = ((1 + (int)d[1]) * 7 + count_bin) * 6 + purity_bin;
        const double denom = sum > 1 ? sum : 1;
        int* row = rows + i * 9;
        row[0] = cell;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            row[1 + r] = (int)((u32)tt[2 * r] | ((u32)tt[2 * r + 1] << 16));
            const u32 w0 = (u32)rint((double)cnt[2 * r] / denom * 65535.0);
            const u32 w1 = (u32)rint((double)cnt[2 * r + 1] / denom * 65535.0);
            row[5 + r] = (int)(w0 | (w1 << 16));
        }
        return;
    }
}

extern "C" int variant_rows(i64 N, const int* mask, int nv, const i64* desc, int* rows, void* stream) {
    if (N > 0) variant_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, mask, nv, desc, rows);
    return (int)hipGetLastError();
}
