// Entry points both reference ABIs export with one signature (old_records/gpu_val_stats.cu and
// record_367_gpu_counts/track_1_short/counts/kernels.cu): the query index's keys, verification and home slots, the
// CUB-style sort / scan / reduce calls (this build's own device-wide primitives, prim.hip, behind the two-phase
// temp-storage convention), the owner side's segments, totals and ranking keys, and a bitmap's popcount. The per-position
// outputs and the rank scatter, whose signatures differ between the flavours, are defined here once (namespace abi)
// and wrapped by each flavour.
//
// Design notes (MI355X): query keys are computed from a block's window of tokens staged in LDS (each token read from
// HBM once, not k times); verification and counting kernels reduce their counters per block before one global
// atomic; the per-position search takes three probes per step (a 4-ary search: a third of the dependent round trips of
// a binary search); the rank scatter finds segment heads inside the wave by ballot and reads a context's start only for
// a segment that began before the wave's first entry.
#include "../prim.h"
#include "../probe.h"
#include "owner.h"

namespace {

// Vector loads need aligned pointers: callers may pass views at any element offset.
inline bool aligned16(const void* a, const void* b, unsigned to = 16) {
    return (((uintptr_t)a | (uintptr_t)b) & (to - 1)) == 0;
}

#define KEY_TILE 1024  // query positions per block in val_keys

// Keys of the positions [i0, i0 + KEY_TILE): the tile's tokens and the k - 1 before it staged in LDS once.
template <int K>
__global__ void __launch_bounds__(256) val_keys_k(const u16* __restrict__ x, const int* __restrict__ avail, i64 n, int k,
                                                  u64* __restrict__ out) {
    __shared__ u16 win[KEY_TILE + MAXK];
    const int kk = ctx_len<K>(k);
    const i64 i0 = (i64)blockIdx.x * KEY_TILE;
    const i64 lo = i0 - (kk - 1);  // the window's first token
    const int span = KEY_TILE + kk - 1;
    for (int j = threadIdx.x; j < span; j += blockDim.x) {
        const i64 at = lo + j;
        win[j] = (at >= 0 && at < n) ? x[at] : (u16)SENT;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < KEY_TILE; j += blockDim.x) {
        const i64 i = i0 + j;
        if (i >= n) break;
        // x[i - k + 1 .. i] = win[j .. j + k - 1]: the key of the k tokens before win + j + k
        out[i] = avail[i] >= kk ? qctx_key<K>(win + j + kk, kk) : EMPTY;
    }
}

__device__ __forceinline__ void block_count_add(u32 mine, u64* out) {  // one global atomic per block
    __shared__ u32 part[4];
    u32 c = mine;
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += (u32)__shfl_down((int)c, d, WAVE);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        const u32 t = part[0] + part[1] + part[2] + part[3];
        if (t) atomicAdd((unsigned long long*)out, (unsigned long long)t);
    }
}

// Each valid position's k tokens against its group representative's (tokens compared eight at a time).
__global__ void __launch_bounds__(256) val_verify_k(const u16* __restrict__ x, const i64* __restrict__ spos,
                                                    const i64* __restrict__ gid, const i64* __restrict__ rep, i64 n,
                                                    int k, u64* bad) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    u32 differs = 0;
    if (i < n) {
        const i64 p = spos[i], r = rep[gid[i]];
        differs = p != r && !same_tokens_rt(x + p + 1, x + r + 1, k);
    }
    block_count_add(differs, bad);
}

// Home slots of two keys per lane (VEC: one 16-byte load and store for both).
template <bool VEC>
__global__ void __launch_bounds__(256) val_homes_k(const u64* __restrict__ keys, i64 n, u64 cap, i64* __restrict__ home) {
    const i64 j = (blockIdx.x * (i64)blockDim.x + threadIdx.x) * 2;
    if (VEC && j + 1 < n) {
        const ulonglong2 v = *(const ulonglong2*)(keys + j);
        longlong2 h;
        h.x = (i64)__umul64hi(v.x, cap);
        h.y = (i64)__umul64hi(v.y, cap);
        *(longlong2*)(home + j) = h;
    } else {
        if (j < n) home[j] = (i64)__umul64hi(keys[j], cap);
        if (j + 1 < n) home[j + 1] = (i64)__umul64hi(keys[j + 1], cap);
    }
}

__global__ void __launch_bounds__(256) popcount_k(const u32* __restrict__ bm, i64 n, u64* out) {
    u64 c = 0;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) c += __popc(bm[i]);
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) c += shfl_down_u64(c, d);
    if (lane_id() == 0 && c) atomicAdd((unsigned long long*)out, (unsigned long long)c);
}

// Context c = uk >> 16 of sorted pair keys: start[c] at the first of its pairs, end[c] one past the last. A lane takes
// two keys (VEC: one 16-byte load); neighbours come from the adjacent lanes, only the wave's ends read global memory.
template <bool VEC>
__global__ void __launch_bounds__(256) seg_bounds_k(const u64* __restrict__ uk, i64 U, i64* __restrict__ start,
                                                    i64* __restrict__ end) {
    const i64 j = (blockIdx.x * (i64)blockDim.x + threadIdx.x) * 2;
    const int lane = lane_id();
    u64 a = EMPTY, b = EMPTY;  // this lane's two contexts (EMPTY past the end)
    if (VEC && j + 1 < U) {
        const ulonglong2 v = *(const ulonglong2*)(uk + j);
        a = v.x >> 16;
        b = v.y >> 16;
    } else {
        if (j < U) a = uk[j] >> 16;
        if (j + 1 < U) b = uk[j + 1] >> 16;
    }
    u64 before = shfl_up_u64(b, 1);        // the previous lane's second context
    u64 after = shfl_down_u64(a, 1);       // the next lane's first context
    if (lane == 0) before = j > 0 && j - 1 < U ? uk[j - 1] >> 16 : EMPTY - 1;
    if (lane == WAVE - 1) after = j + 2 < U ? uk[j + 2] >> 16 : EMPTY - 1;
    if (j >= U) return;
    if (a != before) start[a] = j;
    if (j + 1 < U) {
        if (b != a) {
            end[a] = j + 1;
            start[b] = j + 1;
        }
        if (after != b) end[b] = j + 2;
    } else {
        end[a] = j + 1;
    }
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) v += shfl_down_u64(v, d);
    return v;
}

// Context totals: a lane per context; contexts with more than 64 pairs are summed by the whole wave in turn.
__global__ void __launch_bounds__(256) ctx_tot_k(const i64* __restrict__ start, const i64* __restrict__ end,
                                                 const u32* __restrict__ agg, i64 nctx, u64* __restrict__ tot) {
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
            part = bcast_u64(wave_sum_u64(part), 0);
            if (lane == l) s = part;
        }
        if (c < nctx) tot[c] = s;
    }
}

// Ranking keys of two pairs per lane: context << 32 | (2^32 - 1 - count), so that a stable ascending sort of the keys
// orders each context's pairs by count descending, ties keeping the pairs' (token ascending) order; value = index.
template <bool VEC>
__global__ void __launch_bounds__(256) rank_keys_k(const u64* __restrict__ uk, const u32* __restrict__ agg, i64 U,
                                                   u64* __restrict__ key2, u32* __restrict__ val2) {
    const i64 j = (blockIdx.x * (i64)blockDim.x + threadIdx.x) * 2;
    if (VEC && j + 1 < U) {
        const ulonglong2 k = *(const ulonglong2*)(uk + j);
        const uint2 c = *(const uint2*)(agg + j);
        ulonglong2 o;
        o.x = ((k.x >> 16) << 32) | (u64)(~c.x);
        o.y = ((k.y >> 16) << 32) | (u64)(~c.y);
        *(ulonglong2*)(key2 + j) = o;
        *(uint2*)(val2 + j) = make_uint2((u32)j, (u32)j + 1);
    } else {
        for (i64 q = j; q < j + 2 && q < U; ++q) {
            key2[q] = ((uk[q] >> 16) << 32) | (u64)(~agg[q]);
            val2[q] = (u32)q;
        }
    }
}

// The rank of each pair in its context from the permutation sv that orders pairs by (context, count desc, token asc):
// entry q's rank = q - (its context's first entry). Heads inside the wave come from a ballot of context changes; only
// the lanes of a context that began before the wave read start[c].
__global__ void __launch_bounds__(256) rank_scatter_k(const u32* __restrict__ sv, i64 U, const u64* __restrict__ uk,
                                                      const u32* __restrict__ agg, const i64* __restrict__ start,
                                                      u32* __restrict__ rank_of, u16* __restrict__ top_tok,
                                                      u32* __restrict__ top_cnt, int top) {
    const i64 q = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    const int lane = lane_id();
    const bool in = q < U;
    u32 j = 0;
    u64 key = EMPTY;
    if (in) {
        j = sv[q];
        key = uk[j];
    }
    const u64 c = key >> 16;
    const u64 prev = shfl_up_u64(c, 1);
    const bool head = in && (lane == 0 ? false : prev != c);
    const u64 heads = __ballot(head);
    const u64 upto = heads & (lane == WAVE - 1 ? ~0ull : ((2ull << lane) - 1));
    if (!in) return;
    i64 r;
    if (upto) r = lane - (63 - __clzll(upto));
    else r = q - start[c];
    if (rank_of) rank_of[j] = (u32)r;
    if (top_tok && r < top) {
        top_tok[c * top + r] = (u16)(key & 0xFFFF);
        top_cnt[c * top + r] = agg[j];
    }
}

// The first index of [a, b) whose key is >= want (b if none): three probes per step, then a short walk.
__device__ __forceinline__ i64 lower_bound4(const u64* __restrict__ uk, i64 a, i64 b, u64 want) {
    i64 lo = a, hi = b;
    while (hi - lo > 3) {
        const i64 step = (hi - lo) >> 2;
        const i64 m1 = lo + step, m2 = m1 + step, m3 = m2 + step;
        const u64 v1 = uk[m1], v2 = uk[m2], v3 = uk[m3];
        if (v1 >= want) hi = m1;
        else if (v2 >= want) lo = m1 + 1, hi = m2;
        else if (v3 >= want) lo = m2 + 1, hi = m3;
        else lo = m3 + 1;
    }
    while (lo < hi && uk[lo] < want) ++lo;
    return lo;
}

// Per position whose context id is in [lo, hi): tot, dist (at most 65535), cnt (the target's count; with rank_of,
// only if its rank is below cnt_top), and mask bit li when mask is given.
__global__ void __launch_bounds__(256) pos_outputs_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi,
                                                     const u16* __restrict__ tgt, const u64* __restrict__ uk,
                                                     const u32* __restrict__ agg, const u32* __restrict__ rank_of,
                                                     const i64* __restrict__ start, const i64* __restrict__ end,
                                                     const u64* __restrict__ tot, int li, int cnt_top,
                                                     int* __restrict__ out_tot, int* __restrict__ out_dist,
                                                     int* __restrict__ out_cnt, int* __restrict__ mask) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const i64 c0 = ctx_of[i];
    if (c0 < lo || c0 >= hi) return;
    const i64 c = c0 - lo;
    const i64 a = start[c], b = end[c];
    if (b <= a) return;
    out_tot[i] = (int)(u32)tot[c];
    out_dist[i] = (int)(b - a > 65535 ? 65535 : b - a);
    const u64 want = ((u64)c << 16) | tgt[i];
    const i64 at = lower_bound4(uk, a, b, want);
    if (at < b && uk[at] == want && (!rank_of || rank_of[at] < (u32)cnt_top)) out_cnt[i] = (int)agg[at];
    if (mask) mask[i] |= 1 << li;
}

}  // namespace

namespace abi {
int launch_pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                       const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                       int* out_tot, int* out_dist, int* out_cnt, int* mask, hipStream_t st) {
    if (mask && (li < 0 || li > 30)) return -1;
    if (N > 0)
        pos_outputs_k<<<grid_for(N, 256), 256, 0, st>>>(ctx_of, N, lo, hi, tgt, uk, agg, rank_of, start, end, tot, li,
                                                        cnt_top, out_tot, out_dist, out_cnt, mask);
    return (int)hipGetLastError();
}

int launch_rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                        u16* top_tok, u32* top_cnt, int top, hipStream_t st) {
    if (top_tok && top < 1) return -1;
    if (U > 0)
        rank_scatter_k<<<grid_for(U, 256), 256, 0, st>>>(sv, U, uk, agg, start, rank_of, top_tok, top_cnt, top);
    return (int)hipGetLastError();
}
}  // namespace abi

// ---------------------------------------------------------------------------------------------------------------
// C ABI (both flavours)
// ---------------------------------------------------------------------------------------------------------------

// per query position i: the key of x[i-k+1..i] if avail[i] >= k, else EMPTY (gpu_val_stats.cu:89-99)
extern "C" int val_keys(const u16* x, const int* avail, i64 n, int k, u64* out, void* stream) {
    if (n <= 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    const i64 blocks = (n + KEY_TILE - 1) / KEY_TILE;
    LEVEL_DISPATCH(k, (val_keys_k<K><<<(int)blocks, 256, 0, st>>>(x, avail, n, k, out)));
    return (int)hipGetLastError();
}

// each valid position's k tokens vs its group representative's; mismatches counted in *bad (gpu_val_stats.cu:101-119)
extern "C" int val_verify(const u16* x, const i64* spos, const i64* gid, const i64* rep, i64 n, int k, u64* bad,
                          void* stream) {
    if (k < 1 || k > MAXK) return -1;
    if (n > 0) val_verify_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(x, spos, gid, rep, n, k, bad);
    return (int)hipGetLastError();
}

// home slot umulhi(key, cap) of each key (gpu_val_stats.cu:121-132)
extern "C" int val_homes(const u64* keys, i64 n, u64 cap, i64* home, void* stream) {
    if (n > 0) {
        const int g = grid_for((n + 1) / 2, 256);
        if (aligned16(keys, home)) val_homes_k<true><<<g, 256, 0, (hipStream_t)stream>>>(keys, n, cap, home);
        else val_homes_k<false><<<g, 256, 0, (hipStream_t)stream>>>(keys, n, cap, home);
    }
    return (int)hipGetLastError();
}

// set bits of a bitmap of n words added to *out (gpu_val_stats.cu:436-446)
extern "C" int popcount(const u32* bm, i64 n, u64* out, void* stream) {
    if (n > 0) {
        const int g = grid_for(n, 256);
        popcount_k<<<g < 1024 ? g : 1024, 256, 0, (hipStream_t)stream>>>(bm, n, out);
    }
    return (int)hipGetLastError();
}

// CUB-style two-phase calls (gpu_val_stats.cu:529-551): temp == NULL writes *temp_bytes and returns
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

// per context id: [start, end) of its pairs in the sorted keys (gpu_val_stats.cu:553-564)
extern "C" int seg_bounds(const u64* uk, i64 U, i64* start, i64* end, void* stream) {
    if (U > 0) {
        const int g = grid_for((U + 1) / 2, 256);
        if (aligned16(uk, uk)) seg_bounds_k<true><<<g, 256, 0, (hipStream_t)stream>>>(uk, U, start, end);
        else seg_bounds_k<false><<<g, 256, 0, (hipStream_t)stream>>>(uk, U, start, end);
    }
    return (int)hipGetLastError();
}

// per context: total = the sum of its pair counts (gpu_val_stats.cu:566-577)
extern "C" int ctx_tot(const i64* start, const i64* end, const u32* agg, i64 nctx, u64* tot, void* stream) {
    if (nctx > 0) {
        const int g = grid_for(nctx, 256);
        ctx_tot_k<<<g > 16384 ? 16384 : g, 256, 0, (hipStream_t)stream>>>(start, end, agg, nctx, tot);
    }
    return (int)hipGetLastError();
}

// ranking keys: context << 32 | (2^32 - 1 - count), value = pair index (gpu_val_stats.cu:579-590)
extern "C" int rank_keys(const u64* uk, const u32* agg, i64 U, u64* key2, u32* val2, void* stream) {
    if (U > 0) {
        const int g = grid_for((U + 1) / 2, 256);
        if (aligned16(uk, key2) && aligned16(agg, val2, 8))
            rank_keys_k<true><<<g, 256, 0, (hipStream_t)stream>>>(uk, agg, U, key2, val2);
        else rank_keys_k<false><<<g, 256, 0, (hipStream_t)stream>>>(uk, agg, U, key2, val2);
    }
    return (int)hipGetLastError();
}
