// The LDS-staged scatter pass shared by the partitioned counts (part.hip, pairs32.hip): keys in segments are moved
// to their digit's range, a segment at a time in chunks of SS_CHUNK keys. A chunk is ranked by LDS counters (the
// order within a digit is free: every pass after one of these is order-free or stable on its own), staged in LDS by
// digit and written out as per-digit runs, so each digit's run of a chunk leaves as contiguous stores. Keys whose
// place is `cap` or beyond are dropped, so a pass launched before its host has checked the totals (a region overflow,
// a 32-bit wrap) stays inside its output.
//
// Two kinds of segments:
//   * RegionSegs: nseg segments of ev_count[s] keys at src + (bases ? bases[s] : s * R) (an emitting scan's regions,
//     or a count's per-block outputs), digit d of segment s placed from dpre[d * nseg + s] (the exclusive scan of the
//     producer's per-segment digit histograms, digit-major);
//   * TileSegs: the tiles of an array already grouped into NB buckets (bucket b = [bstart[b], bstart[b + 1]), cut
//     into tiles of SS_CHUNK keys, bucket b's first tile tfirst[b]); digit d of tile s of bucket b placed from
//     hscan[(tfirst[b] << nbits) + d * ntiles(b) + (s - tfirst[b])] (the exclusive scan of the tiles' digit counts
//     laid out bucket by bucket, digit-major within a bucket), so every bucket's keys stay in its range, sub-grouped
//     by digit: the second pass of a most-significant-digit-first partition.
#pragma once
#include "ngram_common.h"

#define SS_BLOCK 1024
#define SS_ITEMS 16
#define SS_CHUNK (SS_BLOCK * SS_ITEMS)
#define SS_MAXB 2048  // digits of up to 11 bits

namespace {

// A wave-uniform value kept in scalar registers (a segment's bounds: the same for every lane).
__device__ __forceinline__ u64 ss_uniform(u64 v) {
    const u32 lo = (u32)__builtin_amdgcn_readfirstlane((int)(u32)v);
    const u32 hi = (u32)__builtin_amdgcn_readfirstlane((int)(u32)(v >> 32));
    return ((u64)hi << 32) | lo;
}

struct RegionSegs {
    u64 R;
    const i64* bases;
    const u32* ev_count;
    const u32* dpre;
    i64 nseg;
    __device__ __forceinline__ i64 bound() const { return nseg; }
    // segment s's input offset and key count (and what dbase needs of it); false past the last segment
    __device__ __forceinline__ bool seg(i64 s, u64& off, u32& n, int& aux) const {
        aux = 0;
        if (s >= nseg) return false;
        n = !bases && (u64)ev_count[s] > R ? (u32)R : ev_count[s];  // a region holds at most R
        off = bases ? (u64)bases[s] : (u64)s * R;
        return true;
    }
    __device__ __forceinline__ u32 dbase(i64 s, int, u32 d) const { return dpre[(i64)d * nseg + s]; }
};

// The bucket holding tile s: the last b with tfirst[b] <= s (tfirst ascending, tfirst[0] = 0).
__device__ __forceinline__ int tile_bucket(const u32* __restrict__ tfirst, int nb, u32 s) {
    int lo = 0, hi = nb;  // tfirst[lo] <= s < tfirst[hi] (tfirst[nb] = the number of tiles)
    while (hi - lo > 1) {
        const int m = (lo + hi) >> 1;
        if (tfirst[m] <= s) lo = m;
        else hi = m;
    }
    return lo;
}

struct TileSegs {
    const i64* bstart;  // [nb + 1]
    const u32* tfirst;  // [nb + 1]
    const u32* hscan;
    int nb;
    int nbits;
    i64 max_tiles;  // the scan's size bound: tiles beyond it are not scattered
    __device__ __forceinline__ i64 bound() const {
        const i64 t = tfirst[nb];
        return t < max_tiles ? t : max_tiles;
    }
    __device__ __forceinline__ bool seg(i64 s, u64& off, u32& n, int& b) const {
        if (s >= bound()) return false;
        b = tile_bucket(tfirst, nb, (u32)s);
        off = (u64)bstart[b] + (u64)(s - tfirst[b]) * SS_CHUNK;
        const u64 end = (u64)bstart[b + 1];
        n = end - off < (u64)SS_CHUNK ? (u32)(end - off) : (u32)SS_CHUNK;
        return true;
    }
    __device__ __forceinline__ u32 dbase(i64 s, int b, u32 d) const {
        const u32 nt = tfirst[b + 1] - tfirst[b];
        return hscan[((u64)tfirst[b] << nbits) + (u64)d * nt + (u64)(s - tfirst[b])];
    }
};

// One scatter pass: KIN keys in, KOUT keys out (u32 out of u64 in keeps the low 32 bits: a pass whose digits lie at
// or above bit 32 - (bits below them) narrows the keys), digit (key >> shift) & (2^nbits - 1), nbits <= log2(BMAX).
// LDS: the stage (SS_CHUNK keys of KIN) and BMAX-entry digit arrays; BMAX 256 or SS_MAXB. A block walks its chunks
// (a segment's, then the block's next segment's). The next chunk's keys are loaded into the registers the current
// chunk's keys leave free once staged, so those loads are in flight while the stage is written out (one block per CU
// holds 128 KB of stage for u64 keys: no other block hides its loads); the next segment is looked up while the
// current chunk is ranked. A whole chunk (all but a segment's last, mostly) takes a path without per-key bounds, so
// its LDS reads and stores issue back to back.
template <int BMAX, typename KIN, typename KOUT, class SEGS>
__global__ void __launch_bounds__(SS_BLOCK) scatter_k(const KIN* __restrict__ src, SEGS segs, int shift, int nbits,
                                                      KOUT* __restrict__ out, u64 cap) {
    __shared__ KIN stage[SS_CHUNK];
    __shared__ u32 cnt[BMAX], pre[BMAX], base[BMAX], wt[SS_BLOCK / WAVE];
    const int t = threadIdx.x, lane = lane_id(), wid = t / WAVE;
    const u32 B = 1u << nbits, mask = B - 1u;
    KIN key[SS_ITEMS];
    auto load = [&](u64 at, u32 c0, u32 n) {  // chunk c0 of the segment of n keys at src + at
        if (n - c0 >= (u32)SS_CHUNK) {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) key[j] = src[at + c0 + (u32)(j * SS_BLOCK + t)];
        } else {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) {
                const u32 i = c0 + (u32)(j * SS_BLOCK + t);
                key[j] = i < n ? src[at + i] : (KIN)0;
            }
        }
    };
    i64 sg = blockIdx.x;
    u64 off;
    u32 n;
    int aux;
    if (!segs.seg(sg, off, n, aux)) return;  // segments ascend with sg: none after this one either
    u32 c0 = 0;
    load(off, 0, n);
    for (u32 d = t; d < B; d += SS_BLOCK) base[d] = segs.dbase(sg, aux, d);
    for (;;) {
        for (u32 d = t; d < B; d += SS_BLOCK) cnt[d] = 0;
        // the next chunk: this segment's, or the first of the block's next segment (none: the walk ends after this)
        i64 nsg = sg;
        u64 noff = off;
        u32 nn = n, nc0 = c0 + SS_CHUNK;
        int naux = aux;
        bool more = true;
        if (nc0 >= n) {
            nsg = sg + gridDim.x;
            nc0 = 0;
            more = segs.seg(nsg, noff, nn, naux);
            noff = ss_uniform(noff);
            nn = (u32)__builtin_amdgcn_readfirstlane((int)nn);
            naux = __builtin_amdgcn_readfirstlane(naux);
        }
        const bool whole = n - c0 >= (u32)SS_CHUNK;
        lds_barrier();
        u32 rank[SS_ITEMS];
        if (whole) {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) rank[j] = atomicAdd(&cnt[(u32)(key[j] >> shift) & mask], 1u);
        } else {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) {
                const u32 i = c0 + (u32)(j * SS_BLOCK + t);
                rank[j] = i < n ? atomicAdd(&cnt[(u32)(key[j] >> shift) & mask], 1u) : 0u;
            }
        }
        lds_barrier();
        // exclusive scan of the B digit counts: thread t holds digits 2t and 2t + 1 (B <= 2 * SS_BLOCK)
        const u32 d0 = 2u * (u32)t;
        const u32 a0 = d0 < B ? cnt[d0] : 0u, a1 = d0 + 1 < B ? cnt[d0 + 1] : 0u;
        u32 incl = a0 + a1;
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
            if (lane >= d) incl += o;
        }
        if (lane == WAVE - 1) wt[wid] = incl;
        lds_barrier();
        u32 before = 0;
        for (int w = 0; w < wid; ++w) before += wt[w];
        const u32 ex = before + incl - (a0 + a1);
        if (d0 < B) pre[d0] = ex;
        if (d0 + 1 < B) pre[d0 + 1] = ex + a0;
        lds_barrier();
        if (whole) {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) rank[j] += pre[(u32)(key[j] >> shift) & mask];
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) stage[rank[j]] = key[j];
        } else {
#pragma unroll
            for (int j = 0; j < SS_ITEMS; ++j) {
                const u32 i = c0 + (u32)(j * SS_BLOCK + t);
                if (i < n) stage[pre[(u32)(key[j] >> shift) & mask] + rank[j]] = key[j];
            }
        }
        if (more) load(noff, nc0, nn);
        lds_barrier();
        if (whole) {
#pragma unroll 4
            for (int j = 0; j < SS_ITEMS; ++j) {
                const u32 i = (u32)(j * SS_BLOCK + t);
                const KIN k = stage[i];
                const u32 d = (u32)(k >> shift) & mask;
                const u64 at = (u64)base[d] + i - pre[d];
                if (at < cap) out[at] = (KOUT)k;
            }
        } else {
            for (u32 i = t; i < n - c0; i += SS_BLOCK) {
                const KIN k = stage[i];
                const u32 d = (u32)(k >> shift) & mask;
                const u64 at = (u64)base[d] + i - pre[d];
                if (at < cap) out[at] = (KOUT)k;
            }
        }
        lds_barrier();  // the stage, pre and base are read before they are written again
        if (!more) break;
        if (nsg != sg) {
            for (u32 d = t; d < B; d += SS_BLOCK) base[d] = segs.dbase(nsg, naux, d);
        } else {
            for (u32 d = t; d < B; d += SS_BLOCK) base[d] += cnt[d];
        }
        sg = nsg;
        off = noff;
        n = nn;
        c0 = nc0;
        aux = naux;
    }
}

}  // namespace
