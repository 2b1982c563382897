// Corpus-wide exact count tables on the GPU: the restatement of exact_match/src/count_table.rs's CountTable
// (build_level :491-631, query_counts :291-331, query_rows :338-404) for one MI355X. No counterpart in the reference's
// GPU libraries; ngram_amd/count_table.py drives it behind CountTable's Python surface.
//
// Per level k: every corpus position p whose k tokens before it and its next token lie in one shard (the corpus is
// laid out with SENT gaps, so a context holding a SENT is skipped) inserts its context key (ngram_common.h ctx_key:
// packed tokens through SplitMix64's finalizer for k <= 4, exact; a polynomial hash for k > 4, ~2^-64 per pair to
// merge two contexts, as count_table.rs:11-14) into an open-addressing context table (slot = context id) and writes
// the event mix64(slot << 16 | next) at its own index (EMPTY where it has none). The events are then counted by the
// partitioned count (part.hip: no global atomics) into packed words (pair key << (48 - cb) | count), sorted by pair
// key, and summarized per context into records (total, pairs, top 8, first word). A query reads its context's record
// and finds its target's count by a binary search of the context's words; the CNT_TOP rule (count_table.rs:146-158
// deep_last) compares its score with thr[c], the CNT_TOP-th largest score of a context with more pairs than that.
#include "probe.h"
#include "part.h"
#include "pairs32.h"

namespace {

template <int K>
__global__ void __launch_bounds__(256) table_emit_k(const u16* __restrict__ tok, i64 L, int k, u64* ck, u64 ccap,
                                                    u64* __restrict__ ev, u32* flags) {
    for (i64 p = blockIdx.x * (i64)blockDim.x + threadIdx.x; p < L; p += (i64)gridDim.x * blockDim.x) {
        if (*(volatile u32*)&flags[0]) return;  // the context table overflowed: the level reruns bigger
        u32 nxt;
        const u64 key = ctx_key_at<K>(tok, p, k, nxt);  // the k + 1 tokens loaded together
        u64 e = EMPTY;
        if (nxt != SENT && key != EMPTY) {
            const i64 s = ctx_find_insert(ck, ccap, key, flags);
            if (s < 0) return;
            e = mix64(((u64)s << 16) | nxt);
        }
        ev[p] = e;
    }
}

// The 32-bit count's emitter for a corpus-wide level: as table_emit_k, but each position with a context appends its
// event e = wmix(slot << 16 | next, W) to its block's region ev[b * region ...] (a block-local cursor in LDS, one LDS
// atomic per wave), with the block's histogram of the events' top dbits bits (dhist[d * gridDim.x + b]) and its event
// count (ev_count[b]): the scan-region layout of the 32-bit count's first pass. flags[0] bit 1: the context table is
// full (the block stops; the level reruns bigger), bit 2: a region overflowed.
template <int K>
__global__ void __launch_bounds__(256) table_emit32_k(const u16* __restrict__ tok, i64 L, int k, u64* ck, u64 ccap,
                                                      int W, int dbits, u64* __restrict__ ev, u64 region,
                                                      u32* __restrict__ ev_count, u32* __restrict__ dhist,
                                                      u32* flags) {
    __shared__ u32 cur;
    __shared__ u32 dh[1024];
    const int nd = 1 << dbits, lane = lane_id();
    if (threadIdx.x == 0) cur = 0;
    for (int d = threadIdx.x; d < nd; d += blockDim.x) dh[d] = 0;
    __syncthreads();
    const i64 stride = (i64)gridDim.x * blockDim.x;
    for (i64 base = blockIdx.x * (i64)blockDim.x + (threadIdx.x & ~(WAVE - 1)); base < L; base += stride) {
        if (__builtin_amdgcn_readfirstlane(*(volatile u32*)&flags[0]) & 2u) break;  // wave-uniform
        const i64 p = base + lane;
        u32 nxt = SENT;
        u64 key = EMPTY;
        if (p < L) key = ctx_key_at<K>(tok, p, k, nxt);
        i64 s = -1;
        if (nxt != SENT && key != EMPTY) s = ctx_find_insert(ck, ccap, key, flags);
        const bool hit = s >= 0;
        const u64 b = __ballot(hit);
        if (!b) continue;
        u32 off = 0;
        if (lane == 0) off = atomicAdd(&cur, (u32)__popcll(b));
        off = (u32)__shfl((int)off, 0, WAVE);
        if (hit) {
            const u64 at = (u64)off + (u64)__popcll(b & lanemask_lt());
            const u64 e = wmix(((u64)s << 16) | nxt, W);
            if (at < region) ev[(u64)blockIdx.x * region + at] = e;
            else atomicOr(&flags[0], 4u);
            atomicAdd(&dh[(u32)(e >> (W - dbits))], 1u);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) ev_count[blockIdx.x] = cur < region ? cur : (u32)region;
    for (int d = threadIdx.x; d < nd; d += blockDim.x) dhist[(i64)d * gridDim.x + blockIdx.x] = dh[d];
}

__global__ void table_lookup_k(const u64* __restrict__ keys, i64 n, const u64* __restrict__ ck, u64 ccap,
                               int* __restrict__ slot) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const u64 key = keys[i];
    slot[i] = key == EMPTY ? -1 : (int)ctx_find(ck, ccap, key);
}

using Rec8 = CtxRecord<8>;

__device__ __forceinline__ u64 rec_first(const u32* __restrict__ r) {
    return (u64)r[Rec8::FIRST] | ((u64)r[Rec8::FIRST + 1] << 32);
}

__device__ __forceinline__ u32 word_count(u64 word, int csh, const u64* __restrict__ esc_k,
                                          const u32* __restrict__ esc_c, u64 esc_cap) {
    const u64 esc = (1ull << csh) - 1;
    const u64 n = word & esc;
    return n < esc ? (u32)n : esc_get(esc_k, esc_c, esc_cap, word >> csh);
}

// One block per listed context c = ids[b] (with more than kth pairs): thr[c] = the kth largest score rank_score(pair
// key, count) among its packed words, by a radix select over the 48-bit scores, 12 bits per round (256 threads: 16
// bins each). Its words: w sorted by pair key, its range from its record (gstart NULL); or w grouped by context into
// partitions of 2^ibits ids (gstart their starts), the words of c's partition whose context is c. m_dev (may be NULL):
// a device-side count of the listed ids (the first min(m, *m_dev) are taken).
__global__ void __launch_bounds__(256) ctx_kth_k(const u64* __restrict__ w, int cb, const u64* __restrict__ esc_k,
                                                 const u32* __restrict__ esc_c, u64 esc_cap, const u32* __restrict__ rec,
                                                 const i64* __restrict__ ids, i64 m, int kth, u64* __restrict__ thr,
                                                 const i64* __restrict__ gstart, int ibits, const u64* m_dev) {
    __shared__ u32 hist[4096];
    __shared__ u32 s_wave[4];
    __shared__ u64 s_prefix;
    __shared__ u32 s_need;
    const int csh = 48 - cb;
    if (m_dev && (i64)*m_dev < m) m = (i64)*m_dev;
    for (i64 b = blockIdx.x; b < m; b += gridDim.x) {
        const i64 c = ids[b];
        i64 a, e;
        if (gstart) {
            a = gstart[c >> ibits];
            e = gstart[(c >> ibits) + 1];
        } else {
            const u32* r = rec + c * Rec8::WORDS;
            a = (i64)rec_first(r);
            e = a + r[1];
        }
        u64 prefix = 0;       // the selected score's bits above the current round
        u32 need = (u32)kth;  // its rank among the scores matching prefix (1 = the largest)
        for (int round = 0; round < 4; ++round) {
            const int shift = 36 - 12 * round;
            for (int i = threadIdx.x; i < 4096; i += blockDim.x) hist[i] = 0;
            __syncthreads();
            for (i64 j = a + threadIdx.x; j < e; j += blockDim.x) {
                const u64 wj = w[j];
                if (gstart && (i64)(wj >> (64 - cb)) != c) continue;
                const u64 sc = rank_score(wj >> csh, word_count(wj, csh, esc_k, esc_c, esc_cap));
                if (round == 0 || (sc >> (shift + 12)) == (prefix >> (shift + 12)))
                    atomicAdd(&hist[(sc >> shift) & 0xFFF], 1u);
            }
            __syncthreads();
            // the digit holding the need-th largest: thread t sums bins [16t, 16t + 16), a suffix scan over the
            // threads finds the one thread whose bins cross `need`, which walks them from the top
            const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
            u32 mine = 0;
#pragma unroll
            for (int q = 0; q < 16; ++q) mine += hist[16 * t + q];
            u32 suf = mine;  // sum over this wave's lanes >= lane
#pragma unroll
            for (int d = 1; d < WAVE; d <<= 1) {
                const u32 o = (u32)__shfl_down((int)suf, d, WAVE);
                if (lane + d < WAVE) suf += o;
            }
            if (lane == 0) s_wave[wid] = suf;
            __syncthreads();
            u32 above = suf - mine;
            for (int v = wid + 1; v < 4; ++v) above += s_wave[v];
            if (above < need && above + mine >= need) {
                u32 acc = above;
                int d = 16 * t + 15;
                for (; d > 16 * t; --d) {
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

// Per query position i whose k-context x[i-k+1..i] lies in its segment (avail[i] >= k) and occurred (context id c):
// tot and dist (at most 65535) from rec[c], the first kout top entries, and cnt = the count of (c, tgt[i]) found by a
// binary search of the context's words, kept only if the context has at most cnt_top pairs or thr is NULL or its
// score reaches thr[c]. Positions without a context are left as they are.
template <int K>
__global__ void __launch_bounds__(256) table_query_k(const u16* __restrict__ x, const int* __restrict__ avail,
                                                     const u16* __restrict__ tgt, i64 n, int k,
                                                     const u64* __restrict__ ck, u64 ccap, const u64* __restrict__ w,
                                                     int cb, const u64* __restrict__ esc_k,
                                                     const u32* __restrict__ esc_c, u64 esc_cap,
                                                     const u32* __restrict__ rec, const u64* __restrict__ thr,
                                                     u32 cnt_top, int kout, int* __restrict__ out_tot,
                                                     int* __restrict__ out_dist, int* __restrict__ out_cnt,
                                                     u16* __restrict__ out_tok, u32* __restrict__ out_tcnt) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n || avail[i] < ctx_len<K>(k)) return;
    const i64 c = ctx_find(ck, ccap, qctx_key<K>(x + i + 1, k));
    if (c < 0) return;
    u32 v[Rec8::WORDS];
    const uint4* src = (const uint4*)(rec + c * Rec8::WORDS);
#pragma unroll
    for (int q = 0; q < Rec8::WORDS / 4; ++q) {
        const uint4 t = src[q];
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
    const u32 pairs = v[1];
    out_tot[i] = (int)v[0];
    out_dist[i] = (int)(pairs < 65535u ? pairs : 65535u);
    const int csh = 48 - cb;
    const u64 want = ((u64)c << 16) | tgt[i];
    const i64 end = (i64)((u64)v[Rec8::FIRST] | ((u64)v[Rec8::FIRST + 1] << 32)) + pairs;
    i64 a = end - pairs, b = end;
    while (a < b) {  // the first word whose pair key is not below want
        const i64 mid = (a + b) >> 1;
        if ((w[mid] >> csh) < want) a = mid + 1;
        else b = mid;
    }
    if (a < end) {
        const u64 wa = w[a];
        if ((wa >> csh) == want) {
            const u32 cnt = word_count(wa, csh, esc_k, esc_c, esc_cap);
            if (pairs <= cnt_top || thr == nullptr || rank_score(want, cnt) >= thr[c]) out_cnt[i] = (int)cnt;
        }
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        if (r < kout) {
            out_tok[i * kout + r] = (u16)(v[2 + r / 2] >> (16 * (r & 1)));
            out_tcnt[i * kout + r] = v[2 + Rec8::TOKW + r];
        }
    }
}

// table_query_k over a level counted by the 32-bit count: cnt = the count of (c, tgt[i]) in the level's slabs (the
// count's per-partition tables, pairs32.h), with the same CNT_TOP rule.
template <int K>
__global__ void __launch_bounds__(256) table_query32_k(const u16* __restrict__ x, const int* __restrict__ avail,
                                                       const u16* __restrict__ tgt, i64 n, int k,
                                                       const u64* __restrict__ ck, u64 ccap,
                                                       const u64* __restrict__ slabs, int pbits, int W,
                                                       const u32* __restrict__ rec, const u64* __restrict__ thr,
                                                       u32 cnt_top, int kout, int* __restrict__ out_tot,
                                                       int* __restrict__ out_dist, int* __restrict__ out_cnt,
                                                       u16* __restrict__ out_tok, u32* __restrict__ out_tcnt) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n || avail[i] < ctx_len<K>(k)) return;
    const i64 c = ctx_find(ck, ccap, qctx_key<K>(x + i + 1, k));
    if (c < 0) return;
    u32 v[Rec8::WORDS];
    const uint4* src = (const uint4*)(rec + c * Rec8::WORDS);
#pragma unroll
    for (int q = 0; q < Rec8::WORDS / 4; ++q) {
        const uint4 t = src[q];
        v[4 * q] = t.x;
        v[4 * q + 1] = t.y;
        v[4 * q + 2] = t.z;
        v[4 * q + 3] = t.w;
    }
    const u32 pairs = v[1];
    out_tot[i] = (int)v[0];
    out_dist[i] = (int)(pairs < 65535u ? pairs : 65535u);
    const u64 want = ((u64)c << 16) | tgt[i];
    const u32 cnt = p32_pair_count(slabs, pbits, W, want);
    if (cnt && (pairs <= cnt_top || thr == nullptr || rank_score(want, cnt) >= thr[c])) out_cnt[i] = (int)cnt;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        if (r < kout) {
            out_tok[i * kout + r] = (u16)(v[2 + r / 2] >> (16 * (r & 1)));
            out_tcnt[i * kout + r] = v[2 + Rec8::TOKW + r];
        }
    }
}

// Hint rows over a CountTable's levels (count_table.rs query_rows :338-404): per position the deepest described level
// whose context occurred: cell ((1 + bucket) * 7 + count bin) * 6 + purity bin, its first `entries` next tokens, their
// weights round_half_even(count / sum of those counts * 65535), and the bucket (level), else 0 / 0 / 0 / -1.
// desc[v * 3 + ...] (deepest first): slot_of (int32 [N]), the level's context records (CtxRecord<8>), bucket.
__constant__ double T_PURITY_EDGES[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
__constant__ u64 T_COUNT_EDGES[6] = {2, 3, 5, 9, 17, 33};

__global__ void pos_rows_k(i64 N, int nlv, const i64* __restrict__ desc, int entries, short* __restrict__ cell,
                           u16* __restrict__ next, u16* __restrict__ weights, signed char* __restrict__ level) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    for (int v = 0; v < nlv; ++v) {
        const i64* d = desc + v * 3;
        const int c = ((const int*)d[0])[i];
        if (c < 0) continue;
        const u32* r = (const u32*)d[1] + (i64)c * Rec8::WORDS;
        const u64 total = r[0];
        if (total == 0) continue;
        const int b = (int)d[2];
        u32 tc[8];
        u16 tt[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            tt[e] = (u16)(r[2 + e / 2] >> (16 * (e & 1)));
            tc[e] = r[2 + Rec8::TOKW + e];
        }
        int count_bin = 0;
#pragma unroll
        for (int e = 0; e < 6; ++e) count_bin += T_COUNT_EDGES[e] <= total;
        const double share = (double)tc[0] / (double)total;
        int purity_bin = 0;
#pragma unroll
        for (int e = 0; e < 5; ++e) purity_bin += T_PURITY_EDGES[e] <= share;
        double sum = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (e < entries) sum += (double)tc[e];
        cell[i] = (short)(((1 + b) * 7 + count_bin) * 6 + purity_bin);
        level[i] = (signed char)b;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (e < entries) {
                next[i * entries + e] = tt[e];
                weights[i * entries + e] = tc[e] ? (u16)rint((double)tc[e] / sum * 65535.0) : (u16)0;
            }
        }
        return;
    }
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// C ABI (engine extensions)
// ---------------------------------------------------------------------------------------------------------------

// One level's contexts into ck (ccap slots, EMPTY-filled) and per position p < L its event ev[p] = mix64(slot << 16 |
// tok[p]), EMPTY where p or its context holds a gap. flags[0] bit 1: the context table is full (rerun bigger; the
// events are then incomplete).
extern "C" int ng_table_emit(const u16* tok, i64 L, int k, u64* ck, u64 ccap, u64* ev, u32* flags, int grid,
                             void* stream) {
    if (L <= 0) return 0;
    if (ccap == 0 || ccap > (1ull << 31)) return -1;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (table_emit_k<K><<<grid, 256, 0, st>>>(tok, L, k, ck, ccap, ev, flags)));
    return (int)hipGetLastError();
}

// One level's contexts into ck (ccap slots, EMPTY-filled, ccap <= 2^(W - 16)) and every position's event (one per
// position p < L whose k tokens before it and p itself hold no gap) in the 32-bit count's scan-region layout: block b
// of `grid` appends e = wmix(slot << 16 | tok[p], W) to ev[b * region ...] (region >= ng_emit_region(L, grid)), its
// count to ev_count[b] and its events per top-dbits digit to dhist[d * grid + b] (1 <= dbits <= 10). flags[0] bit 1:
// the context table is full (rerun bigger; the events are then incomplete), bit 2: a region overflowed.
extern "C" int ng_table_emit32(const u16* tok, i64 L, int k, u64* ck, u64 ccap, int W, int dbits, u64* ev, u64 region,
                               u32* ev_count, u32* dhist, u32* flags, int grid, void* stream) {
    if (ccap == 0 || ccap > (1ull << 31) || W < 17 || W > 48 || ccap > (1ull << (W - 16)) || dbits < 1 || dbits > 10 ||
        region == 0 || grid <= 0 || ev_count == nullptr || dhist == nullptr)
        return -1;
    if (L <= 0) L = 0;
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (table_emit32_k<K><<<grid, 256, 0, st>>>(tok, L, k, ck, ccap, W, dbits, ev, region, ev_count,
                                                                dhist, flags)));
    return (int)hipGetLastError();
}

// Per key (EMPTY: no context): its slot in the context table, or -1.
extern "C" int ng_table_lookup(const u64* keys, i64 n, const u64* ck, u64 ccap, int* slot, void* stream) {
    if (n > 0) table_lookup_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(keys, n, ck, ccap, slot);
    return (int)hipGetLastError();
}

// For each listed context (ids [m], callers list those with more than kth pairs): thr[c] = its kth largest pair score
// over the packed words w (sorted by pair key, cb context bits, escape table esc_k/esc_c) and its record rec[c]
// (ng_ctx_summary's with topk 8).
extern "C" int ng_ctx_kth(const u64* w, int cb, const u64* esc_k, const u32* esc_c, u64 esc_cap, const u32* rec,
                          const i64* ids, i64 m, int kth, u64* thr, void* stream) {
    if (kth < 1 || cb <= 0 || cb > 44 || esc_cap == 0) return -1;
    if (m > 0) {
        const int g = m < 65536 ? (int)m : 65536;
        ctx_kth_k<<<g, 256, 0, (hipStream_t)stream>>>(w, cb, esc_k, esc_c, esc_cap, rec, ids, m, kth, thr, nullptr, 0,
                                                      nullptr);
    }
    return (int)hipGetLastError();
}

// ng_ctx_kth over words grouped by context (ng_ctx_agg's input: partitions of 2^ibits ids, gstart their starts) for
// the first min(m, *m_dev) listed ids (m_dev may be NULL).
extern "C" int ng_ctx_kth_grouped(const u64* w, const i64* gstart, int ibits, int cb, const u64* esc_k,
                                  const u32* esc_c, u64 esc_cap, const i64* ids, i64 m, const u64* m_dev, int kth,
                                  u64* thr, void* stream) {
    if (kth < 1 || cb <= 0 || cb > 44 || esc_cap == 0 || gstart == nullptr || ibits < 0 || ibits > 11) return -1;
    if (m > 0) {
        const int g = m < 65536 ? (int)m : 65536;
        ctx_kth_k<<<g, 256, 0, (hipStream_t)stream>>>(w, cb, esc_k, esc_c, esc_cap, nullptr, ids, m, kth, thr, gstart,
                                                      ibits, m_dev);
    }
    return (int)hipGetLastError();
}

// Per query position i < n (x: the query inputs, avail: tokens since the segment start, tgt: the next tokens): the
// level-k context table ck (ccap slots), its packed words w sorted by pair key (cb context bits, escape table
// esc_k/esc_c), its records rec (ng_ctx_summary's with topk 8) and CNT_TOP thresholds thr (NULL: no rank rule; read
// for contexts with more than cnt_top pairs only) give out_tot, out_dist, out_cnt and the first kout (<= 8) top
// tokens / counts (out_tok / out_tcnt [n, kout]; NULL with kout 0). Positions without a context are not written.
extern "C" int ng_table_query(const u16* x, const int* avail, const u16* tgt, i64 n, int k, const u64* ck, u64 ccap,
                              const u64* w, int cb, const u64* esc_k, const u32* esc_c, u64 esc_cap, const u32* rec,
                              const u64* thr, u32 cnt_top, int kout, int* out_tot, int* out_dist, int* out_cnt,
                              u16* out_tok, u32* out_tcnt, void* stream) {
    if (kout < 0 || kout > 8 || cb <= 0 || cb > 44 || esc_cap == 0 || ccap == 0) return -1;
    if (kout > 0 && (out_tok == nullptr || out_tcnt == nullptr)) return -1;
    if (n <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (table_query_k<K><<<grid_for(n, 256), 256, 0, st>>>(x, avail, tgt, n, k, ck, ccap, w, cb, esc_k,
                                                                         esc_c, esc_cap, rec, thr, cnt_top, kout,
                                                                         out_tot, out_dist, out_cnt, out_tok, out_tcnt)));
    return (int)hipGetLastError();
}

// ng_table_query over a level counted by the 32-bit count: cnt from its slabs (2^pbits partitions of 14336 slots,
// pair keys below 2^W, ng_part_count32's slab output) instead of a search of sorted words.
extern "C" int ng_table_query32(const u16* x, const int* avail, const u16* tgt, i64 n, int k, const u64* ck, u64 ccap,
                                const u64* slabs, int pbits, int W, const u32* rec, const u64* thr, u32 cnt_top,
                                int kout, int* out_tot, int* out_dist, int* out_cnt, u16* out_tok, u32* out_tcnt,
                                void* stream) {
    if (kout < 0 || kout > 8 || ccap == 0 || slabs == nullptr || pbits < 1 || W < 17 || W > 63 || W - pbits < 1 ||
        W - pbits > 31)
        return -1;
    if (kout > 0 && (out_tok == nullptr || out_tcnt == nullptr)) return -1;
    if (n <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (table_query32_k<K><<<grid_for(n, 256), 256, 0, st>>>(x, avail, tgt, n, k, ck, ccap, slabs, pbits,
                                                                           W, rec, thr, cnt_top, kout, out_tot,
                                                                           out_dist, out_cnt, out_tok, out_tcnt)));
    return (int)hipGetLastError();
}

// Hint rows (pos_rows_k): desc[v * 3 + ...] = slot_of (int32 [N]) pointer, records pointer, bucket per described level,
// deepest first.
extern "C" int ng_pos_rows(i64 N, int nlv, const i64* desc, int entries, short* cell, u16* next, u16* weights,
                           signed char* level, void* stream) {
    if (entries < 1 || entries > 8 || nlv < 0) return -1;
    if (N > 0) pos_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, nlv, desc, entries, cell, next, weights, level);
    return (int)hipGetLastError();
}
