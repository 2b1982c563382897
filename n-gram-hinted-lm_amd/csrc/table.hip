// Corpus-wide exact count tables on the GPU: the restatement of exact_match/src/count_table.rs's CountTable
// (build_level :491-631, query_counts :291-331, query_rows :338-404) for one MI355X. No counterpart in the reference's
// GPU libraries; ngram_amd/count_table.py drives it behind CountTable's Python surface.
//
// Per level k: every corpus position p whose k tokens before it and its next token lie in one shard (the corpus is
// laid out with SENT gaps, so a context holding a SENT is skipped) inserts its context key (ngram_common.h ctx_key:
// packed tokens through SplitMix64's finalizer for k <= 4, exact; a polynomial hash for k > 4, ~2^-64 per pair to
// merge two contexts, as count_table.rs:11-14) into an open-addressing context table (slot = context id), then counts
// (slot << 16 | next) in a split pair table (engine.hip's layout). Afterwards the engine's owner side: compaction, one
// sort, per-context totals and top entries, plus here the count threshold of the CNT_TOP rule for contexts with more
// than CNT_TOP next tokens (the score of their CNT_TOP-th ranked pair, count_table.rs:146-158 deep_last).
#include "pairs.h"

namespace {

// The context table's slot of `key` (inserted if absent), or -1 after MAXPROBE probes (flags[0] |= 2).
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

__device__ __forceinline__ void pair_split_add(u64* keys, u32* cnts, u64 cap, u64 key, u32* flags) {
    u64 s = __umul64hi(mix64(key), cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 cur = keys[s];
        if (cur == key) {
            atomicAdd(&cnts[s], 1u);
            return;
        }
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&keys[s], EMPTY, key);
            if (prev == EMPTY || prev == key) {
                atomicAdd(&cnts[s], 1u);
                return;
            }
        }
        s = s + 1 == cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
}

template <int K>
__global__ void __launch_bounds__(256) table_build_k(const u16* __restrict__ tok, i64 L, int k, u64* ck, u64 ccap,
                                                     u64* pk, u32* pcnt, u64 pcap, u32* flags) {
    for (i64 p = blockIdx.x * (i64)blockDim.x + threadIdx.x; p < L; p += (i64)gridDim.x * blockDim.x) {
        if (*(volatile u32*)&flags[0]) return;  // a table overflowed: the level reruns bigger
        const u32 nxt = tok[p];
        if (nxt == SENT) continue;
        const u64 key = ctx_key_stop<K>(tok + p, k);
        if (key == EMPTY) continue;
        const i64 s = ctx_find_insert(ck, ccap, key, flags);
        if (s < 0) return;
        pair_split_add(pk, pcnt, pcap, ((u64)s << 16) | nxt, flags);
    }
}

__global__ void table_lookup_k(const u64* __restrict__ keys, i64 n, const u64* __restrict__ ck, u64 ccap,
                               int* __restrict__ slot) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const u64 key = keys[i];
    slot[i] = key == EMPTY ? -1 : (int)ctx_find(ck, ccap, key);
}

__device__ __forceinline__ u64 rank_score_t(u64 key, u32 n) { return ((u64)n << 16) | (0xFFFFu - (u32)(key & 0xFFFF)); }

// One block per listed context c = ids[b] with more than kth pairs: thr[c] = the kth largest pair score
// (count << 16 | (65535 - token)) by a radix select over 48-bit scores, 12 bits per round.
__global__ void __launch_bounds__(256) ctx_kth_k(const u64* __restrict__ uk, const u32* __restrict__ agg,
                                                 const i64* __restrict__ start, const i64* __restrict__ end,
                                                 const i64* __restrict__ ids, i64 m, int kth, u64* __restrict__ thr) {
    __shared__ u32 hist[4096];
    __shared__ u64 s_prefix;
    __shared__ u32 s_need;
    for (i64 b = blockIdx.x; b < m; b += gridDim.x) {
        const i64 c = ids[b];
        const i64 a = start[c], e = end[c];
        u64 prefix = 0;          // the selected score's bits above the current round
        u32 need = (u32)kth;     // its rank among the scores matching prefix (1 = the largest)
        for (int round = 0; round < 4; ++round) {
            const int shift = 36 - 12 * round;
            for (int i = threadIdx.x; i < 4096; i += blockDim.x) hist[i] = 0;
            __syncthreads();
            for (i64 j = a + threadIdx.x; j < e; j += blockDim.x) {
                const u64 sc = rank_score_t(uk[j], agg[j]);
                if (round == 0 || (sc >> (shift + 12)) == (prefix >> (shift + 12)))
                    atomicAdd(&hist[(sc >> shift) & 0xFFF], 1u);
            }
            __syncthreads();
            if (threadIdx.x == 0) {
                u32 acc = 0;
                int d = 4095;
                for (; d > 0; --d) {
                    if (acc + hist[d] >= need) break;
                    acc += hist[d];
                }
                s_prefix = prefix | ((u64)d << shift);
                s_need = need - acc;
            }
            __syncthreads();
            prefix = s_prefix;
            need = s_need;
            __syncthreads();
        }
        if (threadIdx.x == 0) thr[c] = prefix;
    }
}

// Hint rows over a CountTable's levels (count_table.rs query_rows :338-404): per position the deepest described level
// whose context occurred: cell ((1 + bucket) * 7 + count bin) * 6 + purity bin, its first `entries` next tokens, their
// weights round_half_even(count / sum of those counts * 65535), and the bucket (level), else 0 / 0 / 0 / -1.
// desc[v * 5 + ...] (deepest first): slot_of (int32 [N]), tot (u64 per slot), top_tok (u16 [slots, 8]), top_cnt
// (u32 [slots, 8]), bucket.
__constant__ double T_PURITY_EDGES[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
__constant__ u64 T_COUNT_EDGES[6] = {2, 3, 5, 9, 17, 33};

__global__ void pos_rows_k(i64 N, int nlv, const i64* __restrict__ desc, int entries, short* __restrict__ cell,
                           u16* __restrict__ next, u16* __restrict__ weights, signed char* __restrict__ level) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    for (int v = 0; v < nlv; ++v) {
        const i64* d = desc + v * 5;
        const int c = ((const int*)d[0])[i];
        if (c < 0) continue;
        const u64 total = ((const u64*)d[1])[c];
        if (total == 0) continue;
        const u16* tt = (const u16*)d[2] + (i64)c * 8;
        const u32* tc = (const u32*)d[3] + (i64)c * 8;
        const int b = (int)d[4];
        int count_bin = 0;
#pragma unroll
        for (int e = 0; e < 6; ++e) count_bin += T_COUNT_EDGES[e] <= total;
        const double share = (double)tc[0] / (double)total;
        int purity_bin = 0;
#pragma unroll
        for (int e = 0; e < 5; ++e) purity_bin += T_PURITY_EDGES[e] <= share;
        double sum = 0;
        for (int r = 0; r < entries; ++r) sum += (double)tc[r];
        cell[i] = (short)(((1 + b) * 7 + count_bin) * 6 + purity_bin);
        level[i] = (signed char)b;
        for (int r = 0; r < entries; ++r) {
            next[i * entries + r] = tt[r];
            weights[i * entries + r] = tc[r] ? (u16)rint((double)tc[r] / sum * 65535.0) : (u16)0;
        }
        return;
    }
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// C ABI (engine extensions)
// ---------------------------------------------------------------------------------------------------------------

// One level's corpus-wide count: contexts into ck (ccap slots, EMPTY-filled), (slot << 16 | next) counted in the split
// pair table pk/pcnt (pcap slots). flags[0] bit 0: pair table full, bit 1: context table full (rerun bigger).
extern "C" int ng_table_build(const u16* tok, i64 L, int k, u64* ck, u64 ccap, u64* pk, u32* pcnt, u64 pcap,
                              u32* flags, int grid, void* stream) {
    if (L <= 0) return 0;
    if (ccap == 0 || pcap == 0 || ccap > (1ull << 31)) return -1;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    LEVEL_SWITCH(k, (table_build_k<K><<<grid, 256, 0, st>>>(tok, L, k, ck, ccap, pk, pcnt, pcap, flags)));
    return (int)hipGetLastError();
}

// Per key (EMPTY: no context): its slot in the context table, or -1.
extern "C" int ng_table_lookup(const u64* keys, i64 n, const u64* ck, u64 ccap, int* slot, void* stream) {
    if (n > 0) table_lookup_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(keys, n, ck, ccap, slot);
    return (int)hipGetLastError();
}

// For each listed context (ids [m]): thr[c] = its kth largest pair score (callers list contexts with > kth pairs).
extern "C" int ng_ctx_kth(const u64* uk, const u32* agg, const i64* start, const i64* end, const i64* ids, i64 m,
                          int kth, u64* thr, void* stream) {
    if (kth < 1) return -1;
    if (m > 0) {
        const int g = m < 65536 ? (int)m : 65536;
        ctx_kth_k<<<g, 256, 0, (hipStream_t)stream>>>(uk, agg, start, end, ids, m, kth, thr);
    }
    return (int)hipGetLastError();
}

extern "C" int ng_pos_rows(i64 N, int nlv, const i64* desc, int entries, short* cell, u16* next, u16* weights,
                           signed char* level, void* stream) {
    if (entries < 1 || entries > 8 || nlv < 0) return -1;
    if (N > 0) pos_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, nlv, desc, entries, cell, next, weights, level);
    return (int)hipGetLastError();
}
