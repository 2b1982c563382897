// The engine's own counting and output kernels (no counterpart in the reference's libraries; they replace, inside this
// build's hosts, the record's one-table scan and its owner side of two radix sorts):
//
//   * a split pair table: pair keys (context id << 16 | next token) in u64 slots, their counts in a parallel u32
//     array. An insert reads the key slot (read-only once written, so repeated hits of a hot pair stay cheap) and adds
//     to the count with a no-return atomic. The packed slot of the C ABI (key and count in one word) needs a read and
//     an atomic on the same hot line, which on MI355X runs about three times slower under Zipf-skewed keys.
//   * owner side without a ranking sort: the table compacted, one radix sort by pair key (contexts grouped, tokens
//     ascending), then per context its total and top-k (count descending, token ascending) by selection in registers,
//     and per query position tot / dist / cnt (binary search) / top-k in one gather.
#include "probe.h"
#include "prim.h"
#include "part.h"

namespace {

__device__ __forceinline__ u64 split_home(u64 key, u64 cap) { return __umul64hi(mix64(key), cap); }

// Count `key` in the split table; MAXPROBE probes without a slot set flags[0].
__device__ __forceinline__ void split_add(u64* keys, u32* cnts, u64 cap, u64 key, u32 add, u32* flags) {
    u64 s = split_home(key, cap);
    for (int probe = 0; probe < MAXPROBE; ++probe) {
        const u64 cur = keys[s];
        if (cur == key) {
            atomicAdd(&cnts[s], add);
            return;
        }
        if (cur == EMPTY) {
            const u64 prev = atomicCAS((unsigned long long*)&keys[s], EMPTY, key);
            if (prev == EMPTY || prev == key) {
                atomicAdd(&cnts[s], add);
                return;
            }
        }
        s = s + 1 == cap ? 0 : s + 1;
    }
    atomicOr(&flags[0], 1u);
}

// What a level scan does with each hit besides setting its bitmap bit (the lookup's pair key: context id << 16 | next):
//   CountSink: count it in the split table (once the table has overflowed, only the bitmap is still made: the level
//              reruns bigger);
//   ExistSink: flag its context (bit id of the u32 words hit, set by atomicOr only while it reads unset);
//   EmitSink:  append mix64(pair key) (what 0) or the corpus position (what 1) to the block's own region
//              ev[b * region, (b + 1) * region), at a block-local cursor in LDS (one LDS atomic per wave and round),
//              and store the block's count in ev_count[b] at the end; with `hit`, also flag the context. No global
//              atomic: a single global cursor would serialize (same-address atomics run at about 80 M/s on MI355X).
//              region >= ceil(L / (grid * 8192)) * 8192 (L: positions or list entries) bounds any block's hits in
//              every mode.
struct CountSink {
    static constexpr int KIND = 0;
    u64* keys;
    u32* cnts;
    u64 cap;
};
struct ExistSink {
    static constexpr int KIND = 1;
    u32* hit;
    u32* ids;  // may be NULL: ids[p] = the context id of each hit position p (other positions left as they are)
};
struct EmitSink {
    static constexpr int KIND = 2;
    u64* ev;
    u64 region;
    u32* ev_count;
    int what;
    u32* hit;
    u32* dhist;   // with what 0 (may be NULL): the block's events per digit, at dhist[digit * dstride + block]
    i64 dstride;
    u64 key_add;  // added to each pair key before it is mixed (a context-id offset: several levels' ids in one space)
    int wbits;    // 0: events mix64(pair key), digit = the top 8 bits; else kmix(pair key, wbits, mbits) (pair keys
                  // below 2^wbits), digit = its top dbits bits (dbits <= EMIT_MAXD)
    int dbits;
    int mbits;    // with wbits: the bits below which the pair key is mixed (part.h's kmix; wbits: all of them)
    __device__ __forceinline__ u64 event(u64 key, i64 p) const {
        return what ? (u64)p : wbits ? kmix(key + key_add, wbits, mbits) : mix64(key + key_add);
    }
    __device__ __forceinline__ u32 digit(u64 e) const { return wbits ? (u32)(e >> (wbits - dbits)) : (u32)(e >> 56); }
    __device__ __forceinline__ int ndigits() const { return wbits ? 1 << dbits : 256; }
};

#define EMIT_MAXD 10  // the widest digit of an emitting scan's histogram

// A scan block's LDS for its sink: the emit cursor and the digit histogram.
struct SinkShared {
    u32 cur;
    u32 dh[1 << EMIT_MAXD];
};

// A context's hit flag (bit c of the words hit), set only while it reads unset: a hot context's flag is then read
// from cache rather than set again by every hit, and the bits (an eighth of a byte array) mostly stay in L2.
__device__ __forceinline__ void set_hit(u32* hit, u64 c) {
    const u32 m = 1u << (c & 31);
    if (!(hit[c >> 5] & m)) atomicOr(&hit[c >> 5], m);
}

// A lane's hit (count and exist sinks; the emit sink uses emit_wave / emit_lane).
template <class S>
__device__ __forceinline__ void sink_hit(const S& s, u64 key, i64 p, bool full, u32* flags) {
    if constexpr (S::KIND == 0) {
        if (!full) split_add(s.keys, s.cnts, s.cap, key, 1u, flags);
    } else if constexpr (S::KIND == 1) {
        set_hit(s.hit, key >> 16);
        if (s.ids) s.ids[p] = (u32)(key >> 16);
    }
}

// The wave's hits (b = ballot of `hit`) appended in lane order: called by every lane of the wave.
__device__ __forceinline__ void emit_wave(const EmitSink& s, SinkShared* ss, u64 b, bool hit, u64 key, i64 p, u32* flags) {
    if (!b) return;
    u32 off = 0;
    if (lane_id() == 0) off = atomicAdd(&ss->cur, (u32)__popcll(b));
    off = (u32)__shfl((int)off, 0, WAVE);
    if (hit) {
        const u64 at = (u64)off + (u64)__popcll(b & lanemask_lt());
        const u64 e = s.event(key, p);
        if (at < s.region) s.ev[(u64)blockIdx.x * s.region + at] = e;
        else atomicOr(&flags[0], 4u);
        if (s.dhist) atomicAdd(&ss->dh[s.digit(e)], 1u);
        if (s.hit) set_hit(s.hit, key >> 16);
    }
}

__device__ __forceinline__ void emit_lane(const EmitSink& s, SinkShared* ss, u64 key, i64 p, u32* flags) {
    const u64 at = atomicAdd(&ss->cur, 1u);
    const u64 e = s.event(key, p);
    if (at < s.region) s.ev[(u64)blockIdx.x * s.region + at] = e;
    else atomicOr(&flags[0], 4u);
    if (s.dhist) atomicAdd(&ss->dh[s.digit(e)], 1u);
    if (s.hit) set_hit(s.hit, key >> 16);
}

template <class S>
__device__ __forceinline__ void sink_begin(const S& s, SinkShared* ss) {
    if constexpr (S::KIND == 2) {
        if (threadIdx.x == 0) ss->cur = 0;
        if (s.dhist)
            for (int d = threadIdx.x; d < s.ndigits(); d += blockDim.x) ss->dh[d] = 0;
        __syncthreads();
    }
}

template <class S>
__device__ __forceinline__ void sink_end(const S& s, SinkShared* ss) {
    if constexpr (S::KIND == 2) {
        __syncthreads();
        if (threadIdx.x == 0) s.ev_count[blockIdx.x] = ss->cur < s.region ? ss->cur : (u32)s.region;
        if (s.dhist)
            for (int d = threadIdx.x; d < s.ndigits(); d += blockDim.x)
                s.dhist[(i64)d * s.dstride + blockIdx.x] = ss->dh[d];
    }
}

template <class S>
__device__ __forceinline__ bool sink_full(u32* flags) {
    if constexpr (S::KIND == 0) return *(volatile u32*)&flags[0] != 0u;
    else return false;
}

// A level's gate word over positions 32w .. 32w + 31 from the previous level's hit words bm: its hits, and with the
// prefix rule also hits one position earlier. A k-context occurs only where both its (k-1)-suffix (the position's own
// bit) and its (k-1)-prefix (the bit of the position before) are query contexts that occurred; the prefix rule holds
// when every query context's prefix is itself a query context (ng_avail_closed: avail[i] <= avail[i - 1] + 1), which
// the caller states with *pre != 0 (a device-side flag: no host sync). Word -1 of a range counts as all set.
__device__ __forceinline__ u32 gate_word(const u32* __restrict__ bm, i64 w, bool pre) {
    const u32 b = bm[w];
    if (!pre) return b;
    const u32 before = w > 0 ? bm[w - 1] >> 31 : 1u;
    return b & ((b << 1) | before);
}

__device__ __forceinline__ bool pre_on(const u32* pre) { return pre && *pre != 0u; }

// Dense levels: a wave takes DENSE_PPL * 64 consecutive positions at a time, a lane every 64th of them. A probe is a
// chain of dependent loads (tokens and gate word, then the home slot), so the lane issues the tokens of all its
// positions, then all their home-slot loads, before it waits for any: DENSE_PPL times the loads in flight of a lane
// per position (measured on MI355X at c3: one position per lane leaves the scans bound by load latency).
#define DENSE_PPL 4
template <int K, class S>
__global__ void __launch_bounds__(256) scan_dense_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                    u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                    const u32* __restrict__ vrep, const u16* __restrict__ x, S sink,
                                                    u32* flags, const u32* pre_flag) {
    __shared__ SinkShared ss;
    sink_begin<S>(sink, &ss);
    const int lane = lane_id();
    const bool pre = pre_on(pre_flag);
    const i64 nwords = (L + 31) >> 5;
    const i64 span = (i64)WAVE * DENSE_PPL;
    const i64 stride = (i64)gridDim.x * (blockDim.x / WAVE) * span;
    for (i64 base = (blockIdx.x * (i64)(blockDim.x / WAVE) + threadIdx.x / WAVE) * span; base < L; base += stride) {
        const bool full = sink_full<S>(flags);
        Walk2 wk[DENSE_PPL];
#pragma unroll
        for (int q = 0; q < DENSE_PPL; ++q) {
            const i64 p = base + q * WAVE + lane;
            const i64 w = ((base + q * WAVE) >> 5) + (lane >> 5);
            u32 word = 0xFFFFFFFFu;
            if (bm_in) word = w < nwords ? gate_word(bm_in, w, pre) : 0u;
            // the tokens are loaded whatever the bitmap says, together with its word: one round trip for both
            u32 nxt = SENT;
            u64 ck = EMPTY;
            if (p < L) ck = ctx_key_at<K>(tok, p, k, nxt);
            wk[q].key = ((word >> (lane & 31)) & 1u) && nxt != SENT ? ck : EMPTY;
            wk[q].next = nxt;
        }
#pragma unroll
        for (int q = 0; q < DENSE_PPL; ++q) walk_seed2(vt, vcap, wk[q].key, wk[q].next, wk[q]);
#pragma unroll
        for (int q = 0; q < DENSE_PPL; ++q) {
            const i64 p0 = base + q * WAVE;
            if (p0 >= L) break;  // wave-uniform
            const i64 p = p0 + lane;
            const u64 key = walk_end2<K>(tok, p, k, vt, vrep, x, flags, wk[q]);
            const bool hit = key != EMPTY;
            const u64 b = __ballot(hit);
            const i64 w = (p0 >> 5) + 1;
            if (lane == 0) bm_out[p0 >> 5] = (u32)b;
            if (lane == 32 && w < nwords) bm_out[w] = (u32)(b >> 32);
            if constexpr (S::KIND == 2) emit_wave(sink, &ss, b, hit, key, p, flags);
            else if (hit) sink_hit(sink, key, p, full, flags);
        }
    }
    sink_end(sink, &ss);
}

// Listed positions: a lane per entry of plist (n corpus positions), no bitmap.
template <int K, class S>
__global__ void __launch_bounds__(256) scan_list_k(const u16* __restrict__ tok, const u64* __restrict__ plist, i64 n,
                                                   int k, const u64* __restrict__ vt, u64 vcap,
                                                   const u32* __restrict__ vrep, const u16* __restrict__ x, S sink,
                                                   u32* flags, const u64* __restrict__ n_dev, u32* __restrict__ bm_out) {
    __shared__ SinkShared ss;
    sink_begin<S>(sink, &ss);
    if (n_dev) n = (n > 0 && (i64)*n_dev > n) ? n : (i64)*n_dev;  // a device-side count (at most n when n > 0)
    const int lane = lane_id();
    const i64 stride = (i64)gridDim.x * blockDim.x;
    for (i64 base = blockIdx.x * (i64)blockDim.x + (threadIdx.x & ~(WAVE - 1)); base < n; base += stride) {
        const bool full = sink_full<S>(flags);
        const i64 j = base + lane;
        i64 p = 0;
        u64 key = EMPTY;
        if (j < n) {
            p = (i64)plist[j];
            key = walk_lookup2<K>(tok, p, k, vt, vcap, vrep, x, flags);
        }
        const bool hit = key != EMPTY;
        if (bm_out && hit) atomicOr(&bm_out[p >> 5], 1u << (p & 31));
        if constexpr (S::KIND == 2) emit_wave(sink, &ss, __ballot(hit), hit, key, p, flags);
        else if (hit) sink_hit(sink, key, p, full, flags);
    }
    sink_end(sink, &ss);
}

// Sparse levels: a lane per bitmap word, its set bits in turn.
template <int K, class S>
__global__ void __launch_bounds__(256) scan_sparse_k(const u16* __restrict__ tok, i64 L, int k, const u32* __restrict__ bm_in,
                                                     u32* __restrict__ bm_out, const u64* __restrict__ vt, u64 vcap,
                                                     const u32* __restrict__ vrep, const u16* __restrict__ x, S sink,
                                                     u32* flags, const u32* pre_flag) {
    __shared__ SinkShared ss;
    sink_begin<S>(sink, &ss);
    const bool pre = pre_on(pre_flag);
    const i64 nwords = (L + 31) >> 5;
    for (i64 w = blockIdx.x * (i64)blockDim.x + threadIdx.x; w < nwords; w += (i64)gridDim.x * blockDim.x) {
        const bool full = sink_full<S>(flags);
        u32 word = gate_word(bm_in, w, pre), out = 0;
        while (word) {
            const int b = __ffs(word) - 1;
            word &= word - 1;
            const i64 p = (w << 5) + b;
            if (p >= L) continue;
            const u64 key = walk_lookup2<K>(tok, p, k, vt, vcap, vrep, x, flags);
            if (key != EMPTY) {
                out |= 1u << b;
                if constexpr (S::KIND == 2) emit_lane(sink, &ss, key, p, flags);
                else sink_hit(sink, key, p, full, flags);
            }
        }
        bm_out[w] = out;
    }
    sink_end(sink, &ss);
}

// Gated levels, any density: a block takes 256 bitmap words (8192 positions) at a time; each wave lists its 64 words'
// set positions in LDS (a wave prefix sum of their popcounts), and its lanes then probe the listed positions 64 at a
// time, so every lane has work whatever the density and no position outside the bitmap is visited. Hits set their
// bit in an LDS copy of the words (written out whole).
#define COMPACT_PPL 4  // listed positions probed per lane at once
template <int K, class S>
__global__ void __launch_bounds__(256) scan_compact_k(const u16* __restrict__ tok, i64 L, int k,
                                                      const u32* __restrict__ bm_in, u32* __restrict__ bm_out,
                                                      const u64* __restrict__ vt, u64 vcap, const u32* __restrict__ vrep,
                                                      const u16* __restrict__ x, S sink, u32* flags,
                                                      const u32* pre_flag) {
    __shared__ u32 list[4][64 * 32];
    __shared__ u32 words[4][64];
    __shared__ SinkShared ss;
    sink_begin<S>(sink, &ss);
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const bool pre = pre_on(pre_flag);
    const i64 nwords = (L + 31) >> 5;
    for (i64 g0 = (i64)blockIdx.x * 256; g0 < nwords; g0 += (i64)gridDim.x * 256) {
        const i64 wi = g0 + w * 64 + lane;
        const u32 word = wi < nwords ? gate_word(bm_in, wi, pre) : 0u;
        const u32 c = __popc(word);
        u32 incl = c;
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
            if (lane >= d) incl += o;
        }
        const u32 total = (u32)__shfl((int)incl, WAVE - 1, WAVE);
        u32 at = incl - c;
        u32 bits = word;
        while (bits) {
            const int b = __ffs(bits) - 1;
            bits &= bits - 1;
            list[w][at++] = (u32)(lane * 32 + b);
        }
        words[w][lane] = 0;
        // the list and the words are the wave's own: no block barrier (the wave's LDS accesses stay in order)
        const bool full = sink_full<S>(flags);
        const i64 pbase = (g0 + w * 64) << 5;
        for (u32 r0 = 0; r0 < total; r0 += WAVE * COMPACT_PPL) {  // every lane runs the same rounds
            // COMPACT_PPL probes per lane started together: their first loads are in flight at once
            Walk2 wk[COMPACT_PPL];
            u32 lp[COMPACT_PPL];
#pragma unroll
            for (int q = 0; q < COMPACT_PPL; ++q) {
                const u32 r = r0 + q * WAVE + lane;
                wk[q].key = EMPTY;
                lp[q] = 0;
                if (r < total) {
                    lp[q] = list[w][r];
                    if (pbase + lp[q] < L) walk_begin2<K>(tok, pbase + lp[q], k, vt, vcap, wk[q]);
                }
            }
#pragma unroll
            for (int q = 0; q < COMPACT_PPL; ++q) {
                if (r0 + q * WAVE >= total) break;  // wave-uniform
                const u64 hk = walk_end2<K>(tok, pbase + lp[q], k, vt, vrep, x, flags, wk[q]);
                const bool hit = hk != EMPTY;
                if (hit) atomicOr(&words[w][lp[q] >> 5], 1u << (lp[q] & 31));
                if constexpr (S::KIND == 2)
                    emit_wave(sink, &ss, __ballot(hit), hit, hk, pbase + lp[q], flags);
                else if (hit) sink_hit(sink, hk, pbase + lp[q], full, flags);
            }
        }
        if (wi < nwords) bm_out[wi] = words[w][lane];
    }
    sink_end(sink, &ss);
}

// A bitmap's set bits listed in two passes over blocks of up to BL_ROUNDS rounds of BL_BLOCK words (fewer rounds for
// a small bitmap, so that it still spreads over about 1024 blocks): each block's count, a scan of those counts, then
// each block lists its bits in order (a round of BL_BLOCK words at a time, their offsets by a block-wide scan), so no
// per-word offsets go through memory.
#define BL_BLOCK 256
#define BL_ROUNDS 32
__device__ __forceinline__ u32 bl_block_excl(u32 c, u32* s_w, u32& total) {
    const int lane = lane_id(), wid = threadIdx.x / WAVE;
    u32 incl = c;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    if (lane == WAVE - 1) s_w[wid] = incl;
    __syncthreads();
    u32 before = 0;
    total = 0;
#pragma unroll
    for (int v = 0; v < BL_BLOCK / WAVE; ++v) {
        before += v < wid ? s_w[v] : 0u;
        total += s_w[v];
    }
    __syncthreads();  // s_w is read before the next round writes it
    return before + incl - c;
}

__global__ void __launch_bounds__(BL_BLOCK) bits_count_k(const u32* __restrict__ bm, i64 nwords, u32* __restrict__ cnt,
                                                         const u32* pre_flag, int rounds) {
    __shared__ u32 s_w[BL_BLOCK / WAVE];
    const bool pre = pre_on(pre_flag);
    const i64 w0 = blockIdx.x * (i64)(BL_BLOCK * rounds);
    u32 c = 0;
#pragma unroll 4
    for (int r = 0; r < rounds; ++r) {
        const i64 w = w0 + r * BL_BLOCK + threadIdx.x;
        if (w < nwords) c += (u32)__popc(gate_word(bm, w, pre));
    }
    u32 total;
    bl_block_excl(c, s_w, total);
    if (threadIdx.x == 0) cnt[blockIdx.x] = total;
}

// T: u64 positions, or int (below 2^31) with the first cap kept.
template <typename T>
__global__ void __launch_bounds__(BL_BLOCK) bits_list_k(const u32* __restrict__ bm, i64 nwords,
                                                        const u32* __restrict__ boff, T* __restrict__ out,
                                                        const u32* pre_flag, u64 cap, int rounds) {
    __shared__ u32 s_w[BL_BLOCK / WAVE];
    const bool pre = pre_on(pre_flag);
    const i64 w0 = blockIdx.x * (i64)(BL_BLOCK * rounds);
    u64 run = boff[blockIdx.x];
    for (int r = 0; r < rounds; ++r) {
        const i64 w = w0 + r * BL_BLOCK + threadIdx.x;
        u32 word = w < nwords ? gate_word(bm, w, pre) : 0u;
        u32 total;
        u64 at = run + bl_block_excl((u32)__popc(word), s_w, total);
        while (word) {
            const int b = __ffs(word) - 1;
            word &= word - 1;
            if (at < cap) out[at] = (T)((w << 5) + b);
            ++at;
        }
        run += total;
    }
}

__global__ void fill_u32_small_k(u32* p, u32 v, i64 n) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

static void fill_u32_n(u32* p, u32 v, i64 n, hipStream_t st) {
    if (n > 0) fill_u32_small_k<<<grid_for(n, 256), 256, 0, st>>>(p, v, n);
}

// One level scan with a sink: sparse 0 a lane per position, 1 a lane per bitmap word, 2 LDS-listed (bm_in required
// for 1 and 2).
template <class S>
static int launch_scan(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                        const u32* vrep, const u16* x, const S& sink, u32* flags, int grid, int sparse, hipStream_t st,
                        const u32* pre = nullptr) {
    if (sparse == 2 && bm_in) {
        LEVEL_DISPATCH(k, (scan_compact_k<K, S><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, sink, flags,
                                                                     pre)));
    } else if (sparse && bm_in) {
        LEVEL_DISPATCH(k, (scan_sparse_k<K, S><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, sink, flags,
                                                                    pre)));
    } else {
        LEVEL_DISPATCH(k, (scan_dense_k<K, S><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, sink, flags,
                                                                   pre)));
    }
    return 0;
}

// Occupied slots appended to (out_k, out_c). Each block owns a contiguous range of slots: it counts the range's
// occupied slots, takes its place with one global atomic (a single counter hit per tile would serialize), then
// writes the range tile by tile at a running base.
#define CP_ITEMS 8
__global__ void __launch_bounds__(256) table_compact_k(const u64* __restrict__ keys, const u32* __restrict__ cnts, u64 cap,
                                                       u64 range, u64* __restrict__ out_k, u32* __restrict__ out_c,
                                                       u64* counter) {
    __shared__ u32 wave_n[4];
    __shared__ u64 block_base;
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const u64 tile = 256ull * CP_ITEMS;
    const u64 lo = blockIdx.x * range, hi = lo + range < cap ? lo + range : cap;
    u32 mine = 0;
    for (u64 s = lo + threadIdx.x; s < hi; s += 256) mine += keys[s] != EMPTY;
    u32 red = mine;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) red += (u32)__shfl_down((int)red, d, WAVE);
    if (lane == 0) wave_n[w] = red;
    __syncthreads();
    if (threadIdx.x == 0) {
        const u32 total = wave_n[0] + wave_n[1] + wave_n[2] + wave_n[3];
        block_base = total ? atomicAdd((unsigned long long*)counter, (unsigned long long)total) : 0;
    }
    __syncthreads();
    u64 run = block_base;
    for (u64 t0 = lo; t0 < hi; t0 += tile) {
        u64 key[CP_ITEMS];
        mine = 0;
#pragma unroll
        for (int j = 0; j < CP_ITEMS; ++j) {
            const u64 s = t0 + (u64)j * 256 + threadIdx.x;
            key[j] = s < hi ? keys[s] : EMPTY;
            mine += key[j] != EMPTY;
        }
        // exclusive scan of `mine` over the block
        u32 incl = mine;
#pragma unroll
        for (int d = 1; d < WAVE; d <<= 1) {
            const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
            if (lane >= d) incl += o;
        }
        __syncthreads();  // the previous tile's wave totals are read
        if (lane == WAVE - 1) wave_n[w] = incl;
        __syncthreads();
        u32 before = 0, total = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (i < w) before += wave_n[i];
            total += wave_n[i];
        }
        u64 at = run + before + incl - mine;
#pragma unroll
        for (int j = 0; j < CP_ITEMS; ++j) {
            if (key[j] != EMPTY) {
                const u64 s = t0 + (u64)j * 256 + threadIdx.x;
                out_k[at] = key[j];
                out_c[at] = cnts[s];
                ++at;
            }
        }
        run += total;
    }
}


// Per context c in [0, nctx): tot[c] = sum of its pair counts, its first KT pairs by (count desc, token asc) into
// top_tok/top_cnt [nctx, KT] (0-padded). Pairs sorted by key (context, token), context c's in [start[c], end[c]).
// A lane per context; contexts with more than 64 pairs are done by the whole wave in turn.
template <int KT>
__global__ void __launch_bounds__(256) ctx_topk_k(const u64* __restrict__ uk, const u32* __restrict__ agg,
                                                  const i64* __restrict__ start, const i64* __restrict__ end, i64 nctx,
                                                  u64* __restrict__ tot, u16* __restrict__ top_tok,
                                                  u32* __restrict__ top_cnt) {
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
        u64 t[KT];
#pragma unroll
        for (int r = 0; r < KT; ++r) t[r] = 0;
        u64 s = 0;
        if (!big)
            for (i64 j = a; j < b; ++j) {
                const u32 n = agg[j];
                s += n;
                topk_insert<KT>(t, rank_score(uk[j], n));
            }
        u64 bigs = __ballot(big);
        while (bigs) {
            const int l = __ffsll((unsigned long long)bigs) - 1;
            bigs &= bigs - 1;
            const i64 ba = (i64)bcast_u64((u64)a, l), bb = (i64)bcast_u64((u64)b, l);
            u64 part = 0;
            u64 lt[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) lt[r] = 0;
            for (i64 j = ba + lane; j < bb; j += WAVE) {
                const u32 n = agg[j];
                part += n;
                topk_insert<KT>(lt, rank_score(uk[j], n));
            }
#pragma unroll
            for (int d = WAVE / 2; d > 0; d >>= 1) part += shfl_down_u64(part, d);
            part = bcast_u64(part, 0);
            // merge the lanes' lists: KT rounds of a wave-wide maximum; the lane holding it moves to its next entry
            // (scores are distinct within a context, so exactly one lane holds a nonzero maximum)
            int head = 0;
            u64 merged[KT];
#pragma unroll
            for (int r = 0; r < KT; ++r) {
                u64 mine = 0;
#pragma unroll
                for (int q = 0; q < KT; ++q)
                    if (q == head) mine = lt[q];
                u64 m = mine;
#pragma unroll
                for (int d = WAVE / 2; d > 0; d >>= 1) {
                    const u64 o = shfl_down_u64(m, d);
                    m = o > m ? o : m;
                }
                m = bcast_u64(m, 0);
                merged[r] = m;
                if (m != 0 && mine == m) ++head;
            }
            if (lane == l) {
                s = part;
#pragma unroll
                for (int r = 0; r < KT; ++r) t[r] = merged[r];
            }
        }
        if (c < nctx) {
            tot[c] = s;
#pragma unroll
            for (int r = 0; r < KT; ++r) {
                top_tok[c * KT + r] = t[r] ? (u16)(0xFFFFu - (u32)(t[r] & 0xFFFF)) : (u16)0;
                top_cnt[c * KT + r] = (u32)(t[r] >> 16);
            }
        }
    }
}

// Per query position i whose context id c is in [lo, hi): tot, dist, cnt (the target's count: qcnt[i] when given,
// else looked up in the split table pkeys/pcnts, else by binary search of (c - lo) << 16 | tgt in the context's
// pairs), the first kout of its context's top entries (top_tok/top_cnt [hi - lo, ktop]) and bit li of mask; other
// positions untouched.
__global__ void __launch_bounds__(256) pos_gather_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi,
                                                    const u16* __restrict__ tgt, const u64* __restrict__ uk,
                                                    const u32* __restrict__ agg, const i64* __restrict__ start,
                                                    const i64* __restrict__ end, const u64* __restrict__ tot,
                                                    const u16* __restrict__ top_tok, const u32* __restrict__ top_cnt,
                                                    const u64* __restrict__ thr, const u64* __restrict__ pkeys,
                                                    const u32* __restrict__ pcnts, u64 pcap,
                                                    const u32* __restrict__ qcnt, int ktop, int kout, int li,
                                                    int* __restrict__ out_tot,
                                                    int* __restrict__ out_dist,
                                                    int* __restrict__ out_cnt, u16* __restrict__ out_tok,
                                                    u32* __restrict__ out_tcnt, int* __restrict__ mask) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    i64 c = ctx_of[i];
    if (c < lo || c >= hi) return;
    c -= lo;
    i64 a = start[c], b = end[c];
    if (b <= a) return;
    const i64 e = b;
    out_tot[i] = (int)(u32)tot[c];
    out_dist[i] = (int)(b - a < 65535 ? b - a : 65535);
    const u64 want = ((u64)c << 16) | tgt[i];
    u32 n = 0;
    if (qcnt) {  // counted beforehand (ng_part_count's lookups)
        n = qcnt[i];
    } else if (pkeys) {  // the split table's count of (context, target)
        u64 s = split_home(want + ((u64)lo << 16), pcap);
        for (u64 probe = 0; probe < pcap; ++probe) {
            const u64 cur = pkeys[s];
            if (cur == want + ((u64)lo << 16)) {
                n = pcnts[s];
                break;
            }
            if (cur == EMPTY) break;
            s = s + 1 == pcap ? 0 : s + 1;
        }
    } else {  // binary search of the context's pairs, sorted by token
        while (a < b) {
            const i64 m = (a + b) >> 1;
            if (uk[m] < want) a = m + 1;
            else b = m;
        }
        if (a < e && uk[a] == want) n = agg[a];
    }
    if (n) {
        // the CNT_TOP rule: with a threshold, only a pair ranked at or above it (its score >= thr) gives its count
        const u64 th = thr ? thr[c] : 0;
        if (th == 0 || rank_score(want, n) >= th) out_cnt[i] = (int)n;
    }
    for (int r = 0; r < kout; ++r) {
        out_tok[i * kout + r] = top_tok[c * ktop + r];
        out_tcnt[i * kout + r] = top_cnt[c * ktop + r];
    }
    if (mask) mask[i] |= 1 << li;
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// C ABI (engine extensions)
// ---------------------------------------------------------------------------------------------------------------

// One level's scan counted in a split table (keys u64[cap] filled with EMPTY, cnts u32[cap] zeroed): the record's
// scan_level with the split table. sparse 0: a lane per position; 1: a lane per bitmap word walking its set bits;
// 2: the set positions listed per wave in LDS and probed 64 at a time (any density, bm_in required).
extern "C" int ng_scan_count(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                             const u32* vrep, const u16* x, u64* keys, u32* cnts, u64 cap, u32* flags, int grid,
                             int sparse, void* stream) {
    if (L <= 0) return 0;
    if (cap == 0) return -1;
    if (grid <= 0) grid = grid_for(L, 256);
    if (launch_scan(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, CountSink{keys, cnts, cap}, flags, grid, sparse,
                (hipStream_t)stream) != 0) return -1;
    return (int)hipGetLastError();
}

// One level's existence scan: bm_out = the corpus positions (gated by bm_in) whose k-context is a query context of the
// table, bit id of the u32 words hit set for each such context id (hit zeroed by the caller). sparse as
// ng_scan_count's.
extern "C" int ng_scan_exist(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                             const u32* vrep, const u16* x, u32* hit, u32* ids, u32* flags, int grid, int sparse,
                             const u32* pre, void* stream) {
    if (L <= 0) return 0;
    if (grid <= 0) grid = grid_for(L, 256);
    if (launch_scan(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, ExistSink{hit, ids}, flags, grid, sparse,
                    (hipStream_t)stream, pre) != 0)
        return -1;
    return (int)hipGetLastError();
}

namespace {
// Level 1's existence scan with each 1-context's token as its id (no table: a 65536-bit set of the query tokens in
// LDS): position p hits where tok[p - 1] is a query token and neither it nor tok[p] is SENT (ctx_key_at<1>'s context
// and next token), which sets bm_out bit p, ids[p] = tok[p - 1] (ids may be NULL: the counting scan reads the token)
// and the token's bit in hit (gathered per block in LDS, then one atomicOr per nonzero word). A wave takes TOK1_PPL * 64 consecutive positions at a time, a lane every 64th.
#define TOK1_PPL 4
__global__ void __launch_bounds__(256) scan_tok1_k(const u16* __restrict__ tok, i64 L, const u32* __restrict__ member,
                                                   u32* __restrict__ bm_out, u32* __restrict__ hit,
                                                   u32* __restrict__ ids) {
    __shared__ u32 mem[2048], agg[2048];
    for (int i = threadIdx.x; i < 2048; i += blockDim.x) {
        mem[i] = member[i];
        agg[i] = 0u;
    }
    __syncthreads();
    const int lane = lane_id();
    const i64 nwords = L >> 5;  // L is a multiple of 32
    const i64 span = (i64)WAVE * TOK1_PPL;
    const i64 stride = (i64)gridDim.x * (blockDim.x / WAVE) * span;
    for (i64 base = (blockIdx.x * (i64)(blockDim.x / WAVE) + threadIdx.x / WAVE) * span; base < L; base += stride) {
        u32 c[TOK1_PPL], n[TOK1_PPL];
#pragma unroll
        for (int q = 0; q < TOK1_PPL; ++q) {  // the tokens of every round loaded before any is used
            const i64 p = base + q * WAVE + lane;
            c[q] = n[q] = SENT;
            if (p < L) {
                n[q] = tok[p];
                if (p >= 1) c[q] = tok[p - 1];
            }
        }
#pragma unroll
        for (int q = 0; q < TOK1_PPL; ++q) {
            const i64 p0 = base + q * WAVE;
            if (p0 >= L) break;  // wave-uniform
            const u32 cq = c[q];
            const bool h = cq != SENT && n[q] != SENT && ((mem[cq >> 5] >> (cq & 31)) & 1u);
            const u64 b = __ballot(h);
            if (lane == 0) bm_out[p0 >> 5] = (u32)b;
            if (lane == 32 && (p0 >> 5) + 1 < nwords) bm_out[(p0 >> 5) + 1] = (u32)(b >> 32);
            if (h) {
                if (ids) ids[p0 + lane] = cq;
                const u32 m = 1u << (cq & 31);
                if (!(agg[cq >> 5] & m)) atomicOr(&agg[cq >> 5], m);
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 2048; i += blockDim.x)
        if (agg[i]) atomicOr(&hit[i], agg[i]);
}
}  // namespace

// Level 1's existence scan (ng_scan_exist's k = 1 with no gate) with the 1-context's token as its context id:
// member: 2048 words, bit t set for each query token t; bm_out (L / 32 words) the hit positions; hit (2048 words,
// zeroed by the caller) bit t set where token t occurred as a context; ids (may be NULL) ids[p] = tok[p - 1] at each
// hit position p (others left as they are). L a multiple of 32.
extern "C" int ng_scan_tok1(const u16* tok, i64 L, const u32* member, u32* bm_out, u32* hit, u32* ids, int grid,
                            void* stream) {
    if (L < 0 || (L & 31) || (L > 0 && (!tok || !member || !bm_out || !hit))) return -1;
    if (L == 0) return 0;
    if (grid <= 0) grid = 2048;
    scan_tok1_k<<<grid, 256, 0, (hipStream_t)stream>>>(tok, L, member, bm_out, hit, ids);
    return (int)hipGetLastError();
}

namespace {
// The counting scan of a level whose existence scan stored each hit position's context id (ids; NULL: level 1 by
// token, whose id at p is tok[p - 1]): per position p set in bm, a context id whose bit is set in `final` emits
// mix64(id << 16 | tok[p]) as ng_scan_emit's events. A wave
// loads 64 bitmap words (2048 positions) at a time, skips them if all are empty, else walks them 8 words (256
// positions) per step, a lane 4 consecutive positions: their ids in one 16-byte load and their tokens in one 8-byte
// load, the 4 final-bit loads together; a step whose words are all empty is skipped.
__global__ void __launch_bounds__(256) scan_ids_k(const u16* __restrict__ tok, i64 L, const u32* __restrict__ bm,
                                                  const u32* __restrict__ ids, const u32* __restrict__ final,
                                                  EmitSink sink, u32* flags) {
    __shared__ SinkShared ss;
    sink_begin(sink, &ss);
    const int lane = lane_id();
    const i64 nwords = (L + 31) >> 5;
    const i64 wave = (blockIdx.x * (i64)blockDim.x + threadIdx.x) / WAVE;
    const i64 nwaves = (i64)gridDim.x * (blockDim.x / WAVE);
    for (i64 g0 = wave * 64; g0 < nwords; g0 += nwaves * 64) {
        const u32 wl = g0 + lane < nwords ? bm[g0 + lane] : 0u;  // 64 words (2048 positions) per load
        if (__ballot(wl != 0u) == 0ull) continue;                   // wave-uniform
        for (int sub = 0; sub < 8; ++sub) {                          // 8 words (256 positions) per step
            const u32 word = (u32)__shfl((int)wl, 8 * sub + (lane >> 3), WAVE);
            const u32 bits = (word >> ((lane & 7) * 4)) & 0xFu;
            if (__ballot(bits != 0u) == 0ull) continue;  // wave-uniform
            const i64 p0 = ((g0 + 8 * sub) << 5) + 4 * (i64)lane;
            u32 id[4] = {0, 0, 0, 0};
            u32 t[4] = {0, 0, 0, 0};
            if (bits) {  // a set bit lies below L, and so does its whole 4-aligned group (L is a multiple of 32)
                const ushort4 tv = *(const ushort4*)(tok + p0);
                t[0] = tv.x, t[1] = tv.y, t[2] = tv.z, t[3] = tv.w;
                if (ids) {
                    const uint4 iv = *(const uint4*)(ids + p0);
                    id[0] = iv.x, id[1] = iv.y, id[2] = iv.z, id[3] = iv.w;
                } else {  // level 1 by token (ng_scan_tok1): a hit's context id is the token before it
                    id[0] = p0 >= 1 ? (u32)tok[p0 - 1] : SENT;
                    id[1] = t[0], id[2] = t[1], id[3] = t[2];
                }
            }
            u32 fw[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) fw[i] = ((bits >> i) & 1u) ? final[id[i] >> 5] : 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool hit = (fw[i] >> (id[i] & 31)) & 1u;
                emit_wave(sink, &ss, __ballot(hit), hit, ((u64)id[i] << 16) | t[i], p0 + i, flags);
            }
        }
    }
    sink_end(sink, &ss);
}

__global__ void mark_bits_k(const int* __restrict__ ids, i64 n, u32* bits) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < n) {
        const int c = ids[i];
        if (c >= 0) atomicOr(&bits[c >> 5], 1u << (c & 31));
    }
}
}  // namespace

// An emitting scan's event mode: mix64 events (wbits 0), or W-bit ones, kmix(pair key, wbits, mbits) (mbits 0 taken
// as wbits), with a dbits-bit histogram digit. mbits is made wbits where it is 0.
static inline bool emit_mode_ok(int wbits, int dbits, int& mbits) {
    if (wbits == 0) return true;
    if (mbits == 0) mbits = wbits;
    return wbits >= 17 && wbits <= 63 && dbits >= 1 && dbits <= EMIT_MAXD && dbits < wbits && mbits >= 17 &&
           mbits <= wbits;
}

// A level's counting scan from the context ids its existence scan stored (ng_scan_exist's ids, valid at the
// positions set in bm): the positions whose context's bit is set in `final` emit their events as ng_scan_emit's
// (regions, ev_count, dhist; region >= ng_emit_region(L, grid)), in its modes: wbits 0: mix64(pair key) with a
// histogram of the top 8 bits; wbits in [17, 63]: kmix(pair key, wbits, mbits) (context ids below 2^(wbits - 16);
// part.h; mbits 0: wbits) with a histogram of the top dbits bits (1 <= dbits <= 10), the 32-bit count's events.
extern "C" int ng_scan_ids_emit(const u16* tok, i64 L, const u32* bm, const u32* ids, const u32* final, u64* ev,
                                u64 region, u32* ev_count, u32* flags, int grid, u32* dhist, i64 dstride, int wbits,
                                int dbits, int mbits, void* stream) {
    if (grid <= 0 || region == 0 || region > 0xFFFFFFFFull || (dhist && dstride < grid)) return -1;
    if (!emit_mode_ok(wbits, dbits, mbits)) return -1;
    if ((L & 31) || ((uintptr_t)tok & 7) || ((uintptr_t)ids & 15)) return -1;  // the kernel's vector loads
    hipStream_t st = (hipStream_t)stream;
    const int nd = wbits ? 1 << dbits : 256;
    if (L <= 0) {
        fill_u32_n(ev_count, 0u, grid, st);
        if (dhist)
            for (int d = 0; d < nd; ++d) fill_u32_n(dhist + (i64)d * dstride, 0u, grid, st);
        return (int)hipGetLastError();
    }
    const EmitSink sk{ev, region, ev_count, 0, nullptr, dhist, dstride, 0, wbits, dbits, mbits};
    scan_ids_k<<<grid, 256, 0, st>>>(tok, L, bm, ids, final, sk, flags);
    return (int)hipGetLastError();
}

// bits (u32 words, zeroed by the caller): bit ids[i] set for each ids[i] >= 0, i < n.
extern "C" int ng_mark_bits(const int* ids, i64 n, u32* bits, void* stream) {
    if (n < 0) return -1;
    if (n > 0) mark_bits_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(ids, n, bits);
    return (int)hipGetLastError();
}

// The emitting scan: block b of the `grid` blocks appends its hits' events to ev[b * region ...] and stores their
// number in ev_count[b]; region must be at least ng_emit_region(L, grid). flags[0] bit 2: a region overflowed (only
// with a smaller region). sparse as ng_scan_count's. Events: wbits 0: mix64(pair key), digit its top 8 bits; wbits
// in [17, 63]: kmix(pair key, wbits, mbits) (part.h; pair keys below 2^wbits; mbits 0: wbits, all bits mixed), digit
// its top dbits bits (1 <= dbits <= 10). dhist
// (may be NULL): block b's events per digit d at dhist[d * dstride + b] (dstride >= grid), for ng_seg_scatter.
// pre (may be NULL): a device flag; while it is set, a position of bm_in is probed only if the position before it is
// set too (the prefix rule: ng_avail_closed).
extern "C" u64 ng_emit_region(i64 L, int grid) {
    if (L <= 0 || grid <= 0) return 0;
    const u64 per = (u64)grid * 8192ull;
    return ((u64)L + per - 1) / per * 8192ull;
}


extern "C" int ng_scan_emit(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                            const u32* vrep, const u16* x, u64* ev, u64 region, u32* ev_count, u32* flags, int grid,
                            int sparse, u32* dhist, i64 dstride, const u32* pre, int wbits, int dbits, int mbits,
                            void* stream) {
    if (grid <= 0 || region == 0 || region > 0xFFFFFFFFull || (dhist && dstride < grid)) return -1;
    if (!emit_mode_ok(wbits, dbits, mbits)) return -1;
    if (L <= 0) {
        fill_u32_n(ev_count, 0u, grid, (hipStream_t)stream);
        if (dhist)
            for (int d = 0; d < (wbits ? 1 << dbits : 256); ++d)
                fill_u32_n(dhist + (i64)d * dstride, 0u, grid, (hipStream_t)stream);
        return (int)hipGetLastError();
    }
    const EmitSink sk{ev, region, ev_count, 0, nullptr, dhist, dstride, 0, wbits, dbits, mbits};
    if (launch_scan(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, sk, flags, grid, sparse, (hipStream_t)stream, pre) != 0)
        return -1;
    return (int)hipGetLastError();
}

// The emitting scan over listed positions: the first *n_dev entries of plist (shard-relative corpus positions, a
// device-side count, so no host sync), hits' events appended as ng_scan_emit's (block b of `grid` to
// ev[b * region ...], their number in ev_count[b], events and digit histograms by wbits / dbits / mbits as
// ng_scan_emit's),
// and each hit's bit set in bm_out (zeroed by the caller; may be NULL). region >= ceil(n_max / (grid * 256)) * 256
// for n_max >= *n_dev.
extern "C" int ng_scan_emit_list(const u16* tok, const u64* plist, const u64* n_dev, int k, const u64* vt, u64 vcap,
                                 const u32* vrep, const u16* x, u32* bm_out, u64* ev, u64 region, u32* ev_count,
                                 u32* flags, int grid, u32* dhist, i64 dstride, int wbits, int dbits, int mbits,
                                 void* stream) {
    if (grid <= 0 || n_dev == nullptr || region == 0 || region > 0xFFFFFFFFull || (dhist && dstride < grid)) return -1;
    if (!emit_mode_ok(wbits, dbits, mbits)) return -1;
    const EmitSink sk{ev, region, ev_count, 0, nullptr, dhist, dstride, 0, wbits, dbits, mbits};
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (scan_list_k<K, EmitSink><<<grid, 256, 0, st>>>(tok, plist, 0, k, vt, vcap, vrep, x, sk, flags, n_dev,
                                                                     bm_out)));
    return (int)hipGetLastError();
}

// The list scan of ng_scan_sink over the first *n_dev entries of plist (n_max >= *n_dev; a device-side count, so no
// host sync): hit bits and events (positions, what 1, or mixed pair keys, what 0) as ng_scan_sink's;
// region >= ceil(n_max / (grid * 256)) * 256.
extern "C" int ng_scan_list_dev(const u16* tok, int k, const u64* plist, const u64* n_dev, i64 n_max, const u64* vt,
                                u64 vcap, const u32* vrep, const u16* x, u32* hit, int what, u64* ev, u64 region,
                                u32* ev_count, u32* flags, int grid, u64 key_add, void* stream) {
    if (grid <= 0 || !n_dev || !ev || (what != 0 && what != 1) || region == 0 || region > 0xFFFFFFFFull ||
        (u64)n_max > (u64)grid * region)
        return -1;
    const EmitSink sk{ev, region, ev_count, what, hit, nullptr, 0, key_add};
    hipStream_t st = (hipStream_t)stream;
    LEVEL_DISPATCH(k, (scan_list_k<K, EmitSink><<<grid, 256, 0, st>>>(tok, plist, n_max, k, vt, vcap, vrep, x, sk, flags,
                                                                     n_dev, nullptr)));
    return (int)hipGetLastError();
}

// A level scan with optional outputs, over a bitmap-gated range (plist NULL: positions [0, L) gated by bm_in as
// ng_scan_count's `sparse` modes, hit bitmap into bm_out) or over listed positions (plist: n corpus positions, bm_*
// unused). hit (may be NULL): bit (context id) of the u32 words hit set per hit. ev (may be NULL): block b of `grid` appends per hit
// mix64(pair key + key_add) (what 0) or its position (what 1) to ev[b * region ...] and stores how many in
// ev_count[b]; region >= ng_emit_region(L, grid) over a bitmap, >= ceil(n / (grid * 256)) * 256 over a list.
extern "C" int ng_scan_sink(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* plist, i64 n,
                            const u64* vt, u64 vcap, const u32* vrep, const u16* x, u32* hit, int what,
                            u64* ev, u64 region, u32* ev_count, u32* flags, int grid, int sparse, u64 key_add,
                            void* stream) {
    if (grid <= 0 || (what != 0 && what != 1)) return -1;
    if (ev && (region == 0 || region > 0xFFFFFFFFull)) return -1;
    hipStream_t st = (hipStream_t)stream;
    if (plist) {
        if (n <= 0) {
            if (ev) fill_u32_n(ev_count, 0u, grid, st);
            return (int)hipGetLastError();
        }
        if (ev) {
            const EmitSink sk{ev, region, ev_count, what, hit, nullptr, 0, key_add};
            LEVEL_DISPATCH(k, (scan_list_k<K, EmitSink><<<grid, 256, 0, st>>>(tok, plist, n, k, vt, vcap, vrep, x, sk, flags,
                                                                             nullptr, nullptr)));
        } else {
            LEVEL_DISPATCH(k, (scan_list_k<K, ExistSink><<<grid, 256, 0, st>>>(tok, plist, n, k, vt, vcap, vrep, x,
                                                                              ExistSink{hit, nullptr}, flags, nullptr, nullptr)));
        }
        return (int)hipGetLastError();
    }
    if (L <= 0) return 0;
    int rc;
    if (ev) rc = launch_scan(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, EmitSink{ev, region, ev_count, what, hit, nullptr, 0, key_add},
                             flags, grid, sparse, st);
    else rc = launch_scan(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, ExistSink{hit, nullptr}, flags, grid, sparse, st);
    if (rc != 0) return -1;
    return (int)hipGetLastError();
}

// The set bits of a bitmap (nwords u32 words) as positions, in order: out[r] = the position of the r-th set bit,
// *total = their number. pre (may be NULL): while the device flag is set, only the bits whose previous bit is set too
// (ng_scan_emit's prefix rule). Two-phase temp storage (temp NULL: *temp_bytes set).
template <typename T>
static int bits_list(void* temp, size_t* temp_bytes, const u32* bm, i64 nwords, T* out, u64 cap, u64* total,
                     const u32* pre, hipStream_t st) {
    if (!temp_bytes || nwords < 0) return -1;
    // words per block: BL_ROUNDS rounds of BL_BLOCK, fewer for a small bitmap (about 1024 blocks at least)
    const i64 per = (nwords + 1023) / 1024;
    const int rounds = per >= BL_BLOCK * BL_ROUNDS ? BL_ROUNDS : per <= BL_BLOCK ? 1 : (int)((per + BL_BLOCK - 1) / BL_BLOCK);
    const i64 nb = (nwords + BL_BLOCK * rounds - 1) / (BL_BLOCK * rounds);
    const size_t b0 = ((size_t)(nb + 64) * 4 + 255) & ~(size_t)255;
    const size_t need = b0 + prim::scan_u32_temp_bytes(nb + 1) + 256;
    if (!temp) {
        *temp_bytes = need;
        return 0;
    }
    if (*temp_bytes < need) return -1;
    if (nwords == 0) return prim::fill_u64(total, 0ull, 1, st);
    u32* off = (u32*)temp;
    void* stemp = (char*)temp + b0;
    bits_count_k<<<(unsigned)nb, BL_BLOCK, 0, st>>>(bm, nwords, off, pre, rounds);
    int e = prim::exclusive_scan_u32(off, off, nb, total, stemp, st);
    if (e) return e;
    bits_list_k<T><<<(unsigned)nb, BL_BLOCK, 0, st>>>(bm, nwords, off, out, pre, cap, rounds);
    return (int)hipGetLastError();
}

extern "C" int ng_bits_list(void* temp, size_t* temp_bytes, const u32* bm, i64 nwords, u64* out, u64* total,
                            const u32* pre, void* stream) {
    return bits_list<u64>(temp, temp_bytes, bm, nwords, out, ~0ull, total, pre, (hipStream_t)stream);
}

// ng_bits_list's positions as int (the bitmap below 2^31 bits), the first cap of them kept (*total counts them all).
extern "C" int ng_bits_list32(void* temp, size_t* temp_bytes, const u32* bm, i64 nwords, int* out, i64 cap,
                              u64* total, const u32* pre, void* stream) {
    if (nwords > (1ll << 26) || cap < 0) return -1;
    return bits_list<int>(temp, temp_bytes, bm, nwords, out, (u64)cap, total, pre, (hipStream_t)stream);
}

namespace {
__global__ void __launch_bounds__(256) gate_popcount_k(const u32* __restrict__ bm, i64 nwords, const u32* pre_flag,
                                                       u64* total) {
    __shared__ u64 part[256 / WAVE];
    const bool pre = pre_on(pre_flag);
    u64 c = 0;
    for (i64 w = blockIdx.x * (i64)blockDim.x + threadIdx.x; w < nwords; w += (i64)gridDim.x * blockDim.x)
        c += (u64)__popc(gate_word(bm, w, pre));
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += __shfl_down(c, d, WAVE);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) {  // one atomic per block
        u64 b = 0;
        for (int w = 0; w < 256 / WAVE; ++w) b += part[w];
        if (b) atomicAdd((unsigned long long*)total, (unsigned long long)b);
    }
}

// Random 8-byte loads from a table of cap u64 (the access pattern of a level scan's probes, with nothing else): n
// loads at slots umulhi(mix64(seed + i), cap), four in flight per lane, their sum stored so none is optimized away.
__global__ void __launch_bounds__(256) gather_probe_k(const u64* __restrict__ table, u64 cap, u64 n, u64 seed,
                                                      u64* out) {
    u64 acc = 0;
    const u64 stride = (u64)gridDim.x * blockDim.x * 4;
    for (u64 i = (blockIdx.x * (u64)blockDim.x + threadIdx.x) * 4; i < n; i += stride) {
        u64 v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = i + q < n ? table[__umul64hi(mix64(seed + i + q), cap)] : 0ull;
#pragma unroll
        for (int q = 0; q < 4; ++q) acc += v[q];
    }
    out[blockIdx.x * (u64)blockDim.x + threadIdx.x] = acc;
}
}  // namespace

// *total = the positions a level scan probes behind the hit words bm (nwords words): their set bits, under the
// prefix rule while the device flag pre is set (ng_scan_emit's gate). For a roofline's probe count.
extern "C" int ng_gate_popcount(const u32* bm, i64 nwords, const u32* pre, u64* total, void* stream) {
    if (nwords < 0 || !total) return -1;
    hipStream_t st = (hipStream_t)stream;
    int e = prim::fill_u64(total, 0ull, 1, st);
    if (e) return e;
    if (nwords) {
        const int g = grid_for(nwords, 256);
        gate_popcount_k<<<g < 512 ? g : 512, 256, 0, st>>>(bm, nwords, pre, total);
    }
    return (int)hipGetLastError();
}

// The random-load rate the level scans are measured against: n loads from table (cap u64, any contents) by grid
// blocks of 256, their per-thread sums to out (grid * 256 u64). Time it on the stream it is launched on.
extern "C" int ng_gather_probe(const u64* table, u64 cap, u64 n, u64 seed, int grid, u64* out, void* stream) {
    if (cap == 0 || grid <= 0 || !out) return -1;
    gather_probe_k<<<grid, 256, 0, (hipStream_t)stream>>>(table, cap, n, seed, out);
    return (int)hipGetLastError();
}

namespace {
__global__ void avail_closed_k(const int* __restrict__ avail, i64 n, u32* flag) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const i64 a = avail[i], before = i ? (i64)avail[i - 1] : 0;
    if (a > 1 && a > (before > 0 ? before : 0) + 1) atomicAnd(flag, 0u);
}
}  // namespace

// *flag = 1 if every query position's valid context has its prefix among the valid contexts of the position before
// (avail[i] <= max(avail[i - 1], 0) + 1 wherever avail[i] > 1, avail[-1] read as 0), else 0: the prefix rule of
// ng_scan_emit and ng_bits_list. Stream-ordered, no host sync.
extern "C" int ng_avail_closed(const int* avail, i64 n, u32* flag, void* stream) {
    if (n < 0 || !flag) return -1;
    hipStream_t st = (hipStream_t)stream;
    fill_u32_n(flag, 1u, 1, st);
    if (n > 0) avail_closed_k<<<grid_for(n, 256), 256, 0, st>>>(avail, n, flag);
    return (int)hipGetLastError();
}

// The split table's occupied slots appended to (out_k, out_c) from *counter (zeroed by the caller; any order).
extern "C" int ng_table_compact(const u64* keys, const u32* cnts, u64 cap, u64* out_k, u32* out_c, u64* counter,
                                void* stream) {
    if (cap == 0) return 0;
    const u64 tile = 256 * CP_ITEMS;
    const u64 tiles = (cap + tile - 1) / tile;
    const u64 g = tiles > 2048 ? 2048 : tiles;
    const u64 range = (tiles + g - 1) / g * tile;
    table_compact_k<<<(unsigned)((cap + range - 1) / range), 256, 0, (hipStream_t)stream>>>(keys, cnts, cap, range,
                                                                                          out_k, out_c, counter);
    return (int)hipGetLastError();
}

// Per context: total and top-k (topk of 1, 2, 4, 8) from pairs sorted by key with seg_bounds' start/end.
extern "C" int ng_ctx_topk(const u64* uk, const u32* agg, const i64* start, const i64* end, i64 nctx, int topk,
                           u64* tot, u16* top_tok, u32* top_cnt, void* stream) {
    if (nctx <= 0) return 0;
    int g = grid_for(nctx, 256);
    g = g > 16384 ? 16384 : g;
    hipStream_t st = (hipStream_t)stream;
    switch (topk) {
        case 1: ctx_topk_k<1><<<g, 256, 0, st>>>(uk, agg, start, end, nctx, tot, top_tok, top_cnt); break;
        case 2: ctx_topk_k<2><<<g, 256, 0, st>>>(uk, agg, start, end, nctx, tot, top_tok, top_cnt); break;
        case 4: ctx_topk_k<4><<<g, 256, 0, st>>>(uk, agg, start, end, nctx, tot, top_tok, top_cnt); break;
        case 8: ctx_topk_k<8><<<g, 256, 0, st>>>(uk, agg, start, end, nctx, tot, top_tok, top_cnt); break;
        default: return -1;
    }
    return (int)hipGetLastError();
}

// Per query position: tot, dist, cnt, the first kout <= ktop top entries (out_tok/out_tcnt [N, kout]; kout 0: none)
// and mask bit li (mask may be NULL). thr (may be NULL): per context the score (count << 16 | 65535 - token) of its
// last pair that still gives cnt (0: every pair does). cnt comes from the split table pkeys/pcnts (pcap slots) when
// given, else by binary search of the context's pairs (uk sorted by key).
extern "C" int ng_pos_gather(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                             const i64* start, const i64* end, const u64* tot, const u16* top_tok, const u32* top_cnt,
                             const u64* thr, const u64* pkeys, const u32* pcnts, u64 pcap, const u32* qcnt, int ktop,
                             int kout, int li, int* out_tot, int* out_dist, int* out_cnt, u16* out_tok, u32* out_tcnt,
                             int* mask, void* stream) {
    if (pkeys && pcap == 0) return -1;
    if (kout < 0 || kout > ktop || (mask && (li < 0 || li > 30))) return -1;
    if (N > 0)
        pos_gather_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, N, lo, hi, tgt, uk, agg, start, end, tot,
                                                                        top_tok, top_cnt, thr, pkeys, pcnts, pcap, qcnt,
                                                                        ktop, kout, li, out_tot, out_dist, out_cnt,
                                                                        out_tok, out_tcnt, mask);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// The count mixture's features (record_367_gpu_counts/track_1_short/counts/mix.py features :22-31)
// ---------------------------------------------------------------------------------------------------------------

namespace {
__global__ void features_k(const int* __restrict__ counts, int L, i64 n, int nb, float* __restrict__ tot,
                           float* __restrict__ dist, float* __restrict__ cnt, i64* __restrict__ bin,
                           i64* __restrict__ sparse) {
    const i64 q = blockIdx.x * (i64)blockDim.x + threadIdx.x;  // q = i * L + j, the outputs' [n, L] order
    if (q >= n * L) return;
    const i64 i = q / L;
    const int j = (int)(q - i * L);
    const u32 t = (u32)counts[(i64)j * n + i];
    const float tf = (float)t;  // the uint32 total rounded to float32, as the reference converts it
    const float df = (float)counts[((i64)L + j) * n + i];
    const float cf = (float)counts[(2 * (i64)L + j) * n + i];
    tot[q] = tf;
    dist[q] = df;
    cnt[q] = cf < tf ? cf : tf;
    // floor(log2) of the float32 total (at least 1), as the float64 log2 rounded to float32
    const float lg = (float)log2((double)(tf > 1.0f ? tf : 1.0f));
    float fl = floorf(lg);
    fl = fl < 0.0f ? 0.0f : (fl > (float)(nb - 1) ? (float)(nb - 1) : fl);
    bin[q] = (i64)fl + (i64)nb * j;
    sparse[q] = (i64)(df == 1.0f) + 2 * (i64)j + (i64)nb * L;
}
}  // namespace

// counts int32 [3, L, n] (tot as uint32 bits, dist, cnt) -> tot, dist, min(cnt, tot) float32 [n, L], the bin index
// clamp(floor(log2(max(tot, 1))), 0, nb - 1) + nb * level and the sparse index (dist == 1) + 2 * level + nb * L, int64.
extern "C" int ng_features(const int* counts, int L, i64 n, int nb, float* tot, float* dist, float* cnt, i64* bin,
                           i64* sparse, void* stream) {
    if (L < 1 || nb < 1) return -1;
    if (n > 0) features_k<<<grid_for(n * L, 256), 256, 0, (hipStream_t)stream>>>(counts, L, n, nb, tot, dist, cnt, bin, sparse);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// The engine's query index: the distinct valid query contexts inserted into an open-addressing table by
// compare-and-swap (no sort). Slot = context id; linear probing without wrap-around from umulhi(key, cap) over a
// table of cap + tail slots whose last slot stays empty, which is the layout probe.h walks. rep[slot] = the
// query position whose compare-and-swap inserted the context. The canonical, sorted layout of gpu_val_stats'
// ValIndex is only needed for ids that agree across ranks; on one GPU any layout is exact. No kernel here adds to a
// single global counter per thread or per wave: same-address atomics serialize (about 80 M/s on MI355X), so counts
// are reduced per block first.
// ---------------------------------------------------------------------------------------------------------------

namespace {
template <int K>
// The longest walk an insert takes before it gives up on the table (counters[1] bit 1). At the load the tables are
// sized for (at most 0.5) a walk of even 100 slots is vanishingly rare; a table sized from a wrong estimate of its
// contexts fills up, and without the bound every insert would walk on to the table's end.
#define QI_MAXWALK 256
__global__ void qindex_insert_k(const u16* __restrict__ x, const int* __restrict__ avail, const int* __restrict__ pos,
                                i64 n, int k, u64* table, u64 cap, u64 slots, u32* rep, int* __restrict__ ctx_of,
                                int compact, u64* counters, const u64* __restrict__ n_dev = nullptr,
                                u32* __restrict__ wave_ins = nullptr) {
    if (n_dev && (i64)*n_dev < n) n = (i64)*n_dev;  // a device-side count (at most the grid's n)
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    bool ins = false;  // this position's context took an empty slot
    if (j < n) {
        const i64 i = pos ? pos[j] : j;
        i64 slot = -1;
        if (avail[i] >= (K > 0 ? K : k)) {
            const u64 key = qctx_key<K>(x + i + 1, k);
            u64 s = __umul64hi(key, cap);
            for (int walked = 0;; ++walked) {
                if (s + 1 >= slots) {  // the last slot must stay empty
                    atomicOr((unsigned int*)&counters[1], 1u);
                    break;
                }
                if (walked == QI_MAXWALK) {  // a table far too small for its contexts: stop here, rebuilt bigger
                    atomicOr((unsigned int*)&counters[1], 2u);
                    break;
                }
                const u64 cur = table[s];
                if (cur == key) {
                    slot = (i64)s;
                    break;
                }
                if (cur == EMPTY) {
                    const u64 prev = atomicCAS((unsigned long long*)&table[s], EMPTY, key);
                    if (prev == EMPTY) {  // this position inserted the context: it is the representative
                        rep[s] = (u32)i;
                        slot = (i64)s;
                        ins = true;
                        break;
                    }
                    if (prev == key) {
                        slot = (i64)s;
                        break;
                    }
                }
                ++s;
            }
        }
        if (compact) ctx_of[j] = (int)slot;
        else if (slot >= 0 || !pos) ctx_of[i] = (int)slot;
    }
    // the wave's inserted contexts (no block barrier: a wave done early leaves at once)
    if (wave_ins) {
        const u64 m = __ballot(ins);
        if (lane_id() == 0) wave_ins[j / WAVE] = (u32)__popcll(m);
    }
}

// Occupied slots of a table added to *out: a block-wide sum, then one atomic per block.
__global__ void __launch_bounds__(256) count_occupied_k(const u64* __restrict__ table, u64 slots, u64* out) {
    __shared__ u32 part[4];
    u32 c = 0;
    for (u64 s = blockIdx.x * (u64)blockDim.x + threadIdx.x; s < slots; s += (u64)gridDim.x * blockDim.x)
        c += table[s] != EMPTY;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += (u32)__shfl_down((int)c, d, WAVE);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        const u32 t = part[0] + part[1] + part[2] + part[3];
        if (t) atomicAdd((unsigned long long*)out, (unsigned long long)t);
    }
}

// Re-insert a sparse table's keys (and representatives) into a table sized for them: new slot of each old slot.
__global__ void qindex_shrink_k(const u64* __restrict__ old_t, const u32* __restrict__ old_rep, u64 old_slots,
                                u64* table, u64 cap, u64 slots, u32* rep, int* __restrict__ remap, u64* counters) {
    const i64 o = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (o >= (i64)old_slots) return;
    const u64 key = old_t[o];
    if (key == EMPTY) {
        remap[o] = -1;
        return;
    }
    u64 s = __umul64hi(key, cap);
    while (true) {
        if (s + 1 >= slots) {
            atomicOr((unsigned int*)&counters[1], 1u);
            remap[o] = -1;
            return;
        }
        if (atomicCAS((unsigned long long*)&table[s], EMPTY, key) == EMPTY) break;  // keys are distinct here
        ++s;
    }
    rep[s] = old_rep[o];
    remap[o] = (int)s;
}

__global__ void qindex_remap_k(int* __restrict__ ctx_of, i64 n, const int* __restrict__ remap) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int c = ctx_of[i];
    if (c >= 0) ctx_of[i] = remap[c];
}

// Hashed contexts (k > 4): each position's k tokens against its slot's representative's; mismatches into *bad.
__global__ void qindex_verify_k(const u16* __restrict__ x, const int* __restrict__ pos, i64 n, int k,
                                const int* __restrict__ ctx_of, int compact, const u32* __restrict__ rep, u64* bad,
                                const u64* __restrict__ n_dev = nullptr) {
    if (n_dev && (i64)*n_dev < n) n = (i64)*n_dev;
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= n) return;
    const i64 i = pos ? pos[j] : j;
    const int s = ctx_of[compact ? j : i];
    if (s < 0) return;
    const i64 r = rep[s];
    if (!same_tokens_rt(x + i + 1, x + r + 1, k)) atomicAdd((unsigned long long*)bad, 1ull);
}
}  // namespace

// Move a query index into a smaller table (cap + tail = slots, EMPTY-filled): ctx_of[0..n) re-pointed; remap
// (old_slots ints) is scratch. counters[1] = 1 if the probes ran into the new table's end.
extern "C" int ng_query_index_shrink(const u64* old_t, const u32* old_rep, u64 old_slots, u64* table, u64 cap,
                                     u64 slots, u32* rep, int* ctx_of, i64 n, int* remap, u64* counters,
                                     void* stream) {
    if (cap == 0 || slots <= cap || slots > (1ull << 31)) return -1;
    hipStream_t st = (hipStream_t)stream;
    if (old_slots > 0)
        qindex_shrink_k<<<grid_for((i64)old_slots, 256), 256, 0, st>>>(old_t, old_rep, old_slots, table, cap, slots, rep,
                                                                      remap, counters);
    if (n > 0) qindex_remap_k<<<grid_for(n, 256), 256, 0, st>>>(ctx_of, n, remap);
    return (int)hipGetLastError();
}

// Insert the valid query contexts of positions pos[0..n) (pos NULL: 0..n; with n_dev, pos[0..min(n, *n_dev)): a
// device-side count) into table (cap + tail slots, EMPTY-filled):
// ctx_of[i] = slot (-1 where invalid; with pos, only listed positions are written; compact: ctx_of[j] for pos[j],
// n entries), rep[slot] = the position that inserted it.
// counters[0] += the table's occupied slots afterwards (its contexts: the inserts, counted per wave into wave_ins, of
// grid_for(n, 256) * 4 u32, and summed; wave_ins NULL: a scan of the table), counters[1] bit 0 if a probe ran into the
// table's end, bit 1 if an insert walked QI_MAXWALK slots (a table too small: build it bigger); with k > 4, counters[2] += positions whose tokens differ from their slot's representative (a 64-bit
// key collision).
extern "C" int ng_query_index(const u16* x, const int* avail, const int* pos, i64 n, const u64* n_dev, int k,
                              u64* table, u64 cap, u64 slots, u32* rep, int* ctx_of, int compact, u64* counters,
                              u32* wave_ins, void* stream) {
    if (n <= 0) return 0;
    if (cap == 0 || slots <= cap || slots > (1ull << 31) || (n_dev && !pos)) return -1;
    hipStream_t st = (hipStream_t)stream;
    const int g = grid_for(n, 256);
    LEVEL_DISPATCH(k, (qindex_insert_k<K><<<g, 256, 0, st>>>(x, avail, pos, n, k, table, cap, slots, rep, ctx_of,
                                                             compact, counters, n_dev, wave_ins)));
    if (k > 4) qindex_verify_k<<<grid_for(n, 256), 256, 0, st>>>(x, pos, n, k, ctx_of, compact, rep, counters + 2, n_dev);
    if (wave_ins) return prim::sum_u32(wave_ins, (i64)g * (256 / WAVE), counters, st);
    const int go = grid_for((i64)slots, 256);
    count_occupied_k<<<go < 1024 ? go : 1024, 256, 0, st>>>(table, slots, counters);
    return (int)hipGetLastError();
}

namespace {
// One step of the longest match's active list: entry i (i < *n_dev) of act whose context (ctx_of[i]) has its hit bit
// set matched level k (length[act[i]] = k); those with avail >= k + 1 go on to act_out. SPLIT: the entries that did
// not match go on instead (the matched ones are done at length k). Each thread takes 4 entries; a block counts its
// kept entries and matches and takes its place in act_out with one atomic each (a counter bumped per entry or per
// wave would serialize).
template <bool SPLIT>
__global__ void __launch_bounds__(256) act_next_k(const int* __restrict__ act, const u64* __restrict__ n_dev,
                                                  const int* __restrict__ ctx_of, const u32* __restrict__ hit,
                                                  const int* __restrict__ avail, int k, int* __restrict__ length,
                                                  int* __restrict__ act_out, u64* n_out, u64* matched) {
    __shared__ u32 wave_keep[4], wave_match[4];
    __shared__ u64 base;
    const i64 n = (i64)*n_dev;
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const i64 b0 = (i64)blockIdx.x * 1024;
    int a[4];
    bool keep[4];
    u32 nk = 0, nm = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const i64 i = b0 + q * 256 + threadIdx.x;
        keep[q] = false;
        a[q] = 0;
        if (i < n) {
            a[q] = act[i];
            const int c = ctx_of[i];
            if (c >= 0 && ((hit[c >> 5] >> (c & 31)) & 1u)) {
                length[a[q]] = k;
                ++nm;
                keep[q] = !SPLIT && avail[a[q]] >= k + 1;
            } else {
                keep[q] = SPLIT;
            }
        }
        nk += keep[q];
    }
    // the block's kept entries, in order of (q, thread): per-wave sums, then per-round prefix via ballots
    u32 tk = nk, tm = nm;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) {
        tk += (u32)__shfl_down((int)tk, d, WAVE);
        tm += (u32)__shfl_down((int)tm, d, WAVE);
    }
    if (lane == 0) wave_keep[w] = tk, wave_match[w] = tm;
    __syncthreads();
    if (threadIdx.x == 0) {
        const u32 bk = wave_keep[0] + wave_keep[1] + wave_keep[2] + wave_keep[3];
        const u32 bm = wave_match[0] + wave_match[1] + wave_match[2] + wave_match[3];
        base = bk ? atomicAdd((unsigned long long*)n_out, (unsigned long long)bk) : 0;
        if (bm) atomicAdd((unsigned long long*)matched, (unsigned long long)bm);
    }
    __syncthreads();
    // positions in act_out: the block's base + the entries kept before this thread's (its wave's earlier lanes and
    // the earlier waves), entries of one thread in a row
    u32 incl = nk;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    u64 at = base + incl - nk;
    for (int v = 0; v < w; ++v) at += wave_keep[v];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (keep[q]) act_out[at++] = a[q];
}
}  // namespace

// The query index of the positions pos[0..*n_dev) (n_max >= *n_dev sizes the grid), compact ctx_of, without a host
// sync: the table (cap + tail = slots) is EMPTY-filled here; counters[1] (a table too small) and
// counters[2] (hashed keys that collided, k > 4) are added to, as ng_query_index's; the contexts are not counted.
extern "C" int ng_query_index_dev(const u16* x, const int* avail, const int* pos, const u64* n_dev, i64 n_max, int k,
                                  u64* table, u64 cap, u64 slots, u32* rep, int* ctx_of, u64* counters,
                                  void* stream) {
    if (cap == 0 || slots <= cap || slots > (1ull << 31) || !n_dev || !pos || n_max < 0) return -1;
    hipStream_t st = (hipStream_t)stream;
    fill_u32_n((u32*)table, 0xFFFFFFFFu, (i64)(2 * slots), st);
    if (n_max == 0) return (int)hipGetLastError();
    LEVEL_DISPATCH(k, (qindex_insert_k<K><<<grid_for(n_max, 256), 256, 0, st>>>(x, avail, pos, n_max, k, table, cap, slots,
                                                                                rep, ctx_of, 1, counters, n_dev)));
    if (k > 4)
        qindex_verify_k<<<grid_for(n_max, 256), 256, 0, st>>>(x, pos, n_max, k, ctx_of, 1, rep, counters + 2, n_dev);
    return (int)hipGetLastError();
}

// The longest match's active list, one level on: see act_next_k. n_out and matched are added to (zero them first);
// act_out holds at least *n_dev entries; n_max >= *n_dev sizes the grid.
extern "C" int ng_act_next(const int* act, const u64* n_dev, i64 n_max, const int* ctx_of, const u32* hit,
                           const int* avail, int k, int* length, int* act_out, u64* n_out, u64* matched,
                           void* stream) {
    if (!n_dev || n_max < 0) return -1;
    if (n_max > 0)
        act_next_k<false><<<(int)((n_max + 1023) / 1024), 256, 0, (hipStream_t)stream>>>(
            act, n_dev, ctx_of, hit, avail, k, length, act_out, n_out, matched);
    return (int)hipGetLastError();
}

// The longest match's active list split at level k (see act_next_k): entries whose context's hit bit is set get
// length k and are done; the others go to act_out. n_out and matched are added to (zero them first).
extern "C" int ng_act_split(const int* act, const u64* n_dev, i64 n_max, const int* ctx_of, const u32* hit, int k,
                            int* length, int* act_out, u64* n_out, u64* matched, void* stream) {
    if (!n_dev || n_max < 0) return -1;
    if (n_max > 0)
        act_next_k<true><<<(int)((n_max + 1023) / 1024), 256, 0, (hipStream_t)stream>>>(
            act, n_dev, ctx_of, hit, nullptr, k, length, act_out, n_out, matched);
    return (int)hipGetLastError();
}
