// Entry points the library's two flavours share (the gpu_val_stats library, old_records/gpu_val_stats.cu, and the
// record's, record_367_gpu_counts/track_1_short/counts/kernels.cu, export them with the same signatures): the query
// index's keys, verification and home slots, the CUB-style sorts/scans/reductions (our own device-wide primitives,
// prim.hip, behind the two-phase temp-storage convention), and the owner side's segments, totals and ranking keys.
// Also the owner side's per-position outputs and rank scatter, which the flavours wrap with their own signatures.
#include "pairs.h"
#include "prim.h"

// ---------------------------------------------------------------------------------------------------------------
// Query side
// ---------------------------------------------------------------------------------------------------------------

template <int K>
__global__ void val_keys_k(const u16* __restrict__ x, const int* __restrict__ avail, i64 n, int k, u64* __restrict__ out) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = avail[i] >= klen<K>(k) ? key_at<K>(x + i + 1, k) : EMPTY;
}

// per query position i: the key of x[i-k+1..i] if avail[i] >= k, else EMPTY (gpu_val_stats.cu:89-99)
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

// each valid position's k tokens vs its group representative's; mismatches counted in *bad (gpu_val_stats.cu:101-119)
extern "C" int val_verify(const u16* x, const i64* spos, const i64* gid, const i64* rep, i64 n, int k, u64* bad,
                          void* stream) {
    if (n <= 0) return 0;
    if (k < 1 || k > MAXK) return -1;
    val_verify_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(x, spos, gid, rep, n, k, bad);
    return (int)hipGetLastError();
}

__global__ void val_homes_k(const u64* __restrict__ keys, i64 n, u64 cap, i64* __restrict__ home) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < n) home[i] = (i64)__umul64hi(keys[i], cap);
}

// home slot umulhi(key, cap) of each key (gpu_val_stats.cu:121-132)
extern "C" int val_homes(const u64* keys, i64 n, u64 cap, i64* home, void* stream) {
    if (n > 0) val_homes_k<<<grid_for(n, 256), 256, 0, (hipStream_t)stream>>>(keys, n, cap, home);
    return (int)hipGetLastError();
}

__device__ __forceinline__ u64 wave_sum_pc(u64 v) {
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) v += shfl_down_u64(v, d);
    return v;
}

__global__ void popcount_k(const u32* __restrict__ bm, i64 n, u64* out) {
    u64 c = 0;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) c += __popc(bm[i]);
    c = wave_sum_pc(c);
    if (lane_id() == 0 && c) atomicAdd((unsigned long long*)out, (unsigned long long)c);
}

// set bits of a bitmap of n words added to *out (gpu_val_stats.cu:436-446)
extern "C" int popcount(const u32* bm, i64 n, u64* out, void* stream) {
    if (n > 0) popcount_k<<<1024, 256, 0, (hipStream_t)stream>>>(bm, n, out);
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// CUB-style two-phase calls (gpu_val_stats.cu:529-551): temp == NULL writes *temp_bytes and returns
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

// ---------------------------------------------------------------------------------------------------------------
// Owner side: segments, totals, ranking
// ---------------------------------------------------------------------------------------------------------------

__global__ void seg_bounds_k(const u64* __restrict__ uk, i64 U, i64* __restrict__ start, i64* __restrict__ end) {
    const i64 j = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (j >= U) return;
    const u64 c = uk[j] >> 16;
    if (j == 0 || (uk[j - 1] >> 16) != c) start[c] = j;
    if (j == U - 1 || (uk[j + 1] >> 16) != c) end[c] = j + 1;
}

// per context id: [start, end) of its pairs in the sorted keys (gpu_val_stats.cu:553-564)
extern "C" int seg_bounds(const u64* uk, i64 U, i64* start, i64* end, void* stream) {
    if (U > 0) seg_bounds_k<<<grid_for(U, 256), 256, 0, (hipStream_t)stream>>>(uk, U, start, end);
    return (int)hipGetLastError();
}

__device__ __forceinline__ u64 wave_sum_u64(u64 v) {
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) v += shfl_down_u64(v, d);
    return v;
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

// per context: total = the sum of its pair counts (gpu_val_stats.cu:566-577)
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

// ranking keys: context << 32 | (2^32 - 1 - count), value = pair index (gpu_val_stats.cu:579-590)
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
    if (rank_of) rank_of[j] = (u32)r;
    if (top_tok && r < top) {
        top_tok[c * top + r] = (u16)(uk[j] & 0xFFFF);
        top_cnt[c * top + r] = agg[j];
    }
}

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
    if (a < end[c] && uk[a] == want && (!rank_of || rank_of[a] < (u32)cnt_top)) out_cnt[i] = (int)agg[a];
    if (mask) mask[i] |= 1 << li;
}

namespace ng {
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
}  // namespace ng
