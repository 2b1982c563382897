// The gpu_val_stats flavour of the C ABI: the entry points old_records/gpu_val_stats.py's `Lib` binds
// (old_records/gpu_val_stats.cu:96-699), with their names, argument meaning, return codes and device-side flags.
// Pair keys of 40 bits (24-bit context ids, 24-bit counts + the wrap byte, gpu_val_stats.cu:139-143).
//
// Semantics (old_records/gpu_val_stats.cu:5-13): the training shards are concatenated with >= 32 SENT (0xFFFF) tokens
// before each shard; a corpus position p is an occurrence of the k tokens before it with next token tok[p]; a position
// whose next token is SENT is skipped, and a context holding a SENT matches no query context, so no context crosses a
// shard. Query tables are in the canonical (sorted) layout of the reference's ValIndex; hashed keys (k > 4) are
// verified against the context's representative query position, so counts are exact.
//
// The kernels are this build's (abi/packed.h, abi/owner.hip): tile scans with LDS-listed gated positions, wave-merged
// counts into bucketed packed tables, LDS-staged appends, LDS pre-aggregation of grouped keys.
#include "owner.h"
#include "packed.h"

#define KB_GVS 40

// mode 0: count every position (bm_in gates when given); 1: count the positions set in bm_in; 2: emit instead of
// counting; 3: emit the positions set in bm_in. Modes 1 and 3 without bm_in run as 0 and 2. flags[0]: the table
// overflowed (rerun bigger); flags[1] += false hash hits.
extern "C" int scan_level(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                          const u32* vrep, const u16* x, u64* pk, u32* pc, u64 sub_cap, int pbits, u32* flags, int grid,
                          int mode, u64* emit, u64* emitted, void* stream) {
    if (mode < 0 || mode > 3) return -1;
    hipStream_t st = (hipStream_t)stream;
    if (mode >= 2) {
        if (!emit || !emitted) return -1;
        return abi::launch_tile_scan<KB_GVS>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, grid,
                                             abi::AppendSink{emit, emitted}, st);
    }
    if (!pk || !pc || sub_cap == 0 || pbits < 0 || pbits > 24) return -1;
    return abi::launch_tile_scan<KB_GVS>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, grid,
                                         abi::TableSink{pk, pc, sub_cap, pbits}, st);
}

// the most sub-table bits subpart_count / subpart_scatter take (gpu_val_stats.cu:396-403)
extern "C" int max_pbits() { return abi::max_group_bits(); }

// emitted keys per sub-table added to counts[2^pbits] (gpu_val_stats.cu:410-418)
extern "C" int subpart_count(const u64* keys, i64 n, int pbits, u64* counts, void* stream) {
    return abi::launch_group_hist(keys, n, pbits, counts, (hipStream_t)stream);
}

// emitted keys grouped by sub-table from cursor[] (gpu_val_stats.cu:420-428)
extern "C" int subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, void* stream) {
    return abi::launch_group_scatter(keys, n, pbits, cursor, out, (hipStream_t)stream);
}

// grouped keys counted into the pair table (gpu_val_stats.cu:430-434)
extern "C" int aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                         void* stream) {
    return abi::launch_aggregate<KB_GVS>(keys, n, pk, wraps, sub_cap, pbits, flags, grid, (hipStream_t)stream);
}

// pair-table entries per owner (gpu_val_stats.cu:472-476)
extern "C" int part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, void* stream) {
    return abi::launch_own_count<KB_GVS>(pk, cap, bounds, W, counts, (hipStream_t)stream);
}

// pair-table entries as (key, count) grouped by owner (gpu_val_stats.cu:518-523)
extern "C" int part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                            u32* oc, void* stream) {
    return abi::launch_own_scatter<KB_GVS>(pk, pc, cap, bounds, W, cursor, ok, oc, (hipStream_t)stream);
}

// rank of each pair within its context; the top `top` tokens/counts per context (gpu_val_stats.cu:606-612)
extern "C" int rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                            u16* top_tok, u32* top_cnt, int top, void* stream) {
    return abi::launch_rank_scatter(sv, U, uk, agg, start, rank_of, top_tok, top_cnt, top, (hipStream_t)stream);
}

// per query position: tot, dist, cnt (the TOP rule: the target's count if its rank < cnt_top), mask bit li
// (gpu_val_stats.cu:637-644)
extern "C" int pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                           const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                           int* out_tot, int* out_dist, int* out_cnt, int* mask, void* stream) {
    return abi::launch_pos_outputs(ctx_of, N, lo, hi, tgt, uk, agg, rank_of, start, end, tot, li, cnt_top, out_tot,
                                   out_dist, out_cnt, mask, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Hint rows of one variant (old_records._val_rows with one slot, src/retrieval_blog_post/old_records.py:94-124, and
// val_hints.deepest, src/retrieval_blog_post/val_hints.py:277-311). The variant's levels ascend; level v's descriptor
// desc[v * 8 ..] = (mask bit, length bucket, ctx_of, lo, hi, top tokens u16 [hi - lo, 8], top counts u32 [hi - lo, 8],
// totals u64 [hi - lo]). Per position: the deepest level whose mask bit is set; if its context is owned here, the
// row (cell, 8 tokens, 8 weights) packed into 9 int32: cell, 4 x (token | token << 16), 4 x (weight | weight << 16).
//   cell = ((1 + bucket) * 7 + count_bin) * 6 + purity_bin, count_bin = #{e in (2,3,5,9,17,33) : e <= total},
//   purity_bin = #{e in (.3,.5,.7,.85,.95) : e <= top1 / max(total, 1)} (float64),
//   weight = round_half_even(count / max(sum of the 8 counts, 1) * 65535) (float64).
// The count edges are 1 + 2^j, so count_bin is the bit length of total - 1, capped at 6.
// ---------------------------------------------------------------------------------------------------------------

namespace {
#define MAX_VLEVELS 16

__device__ __forceinline__ int count_bin(u64 total) {
    if (total < 2) return 0;
    const int bl = 64 - __clzll((long long)(total - 1));
    return bl < 6 ? bl : 6;
}

__device__ __forceinline__ int purity_bin(double share) {
    constexpr double E[5] = {0.3, 0.5, 0.7, 0.85, 0.95};
    int b = 0;
#pragma unroll
    for (int e = 0; e < 5; ++e) b += share >= E[e];
    return b;
}

__device__ __forceinline__ u32 weight16(u32 c, double denom) { return (u32)rint((double)c / denom * 65535.0); }

__global__ void __launch_bounds__(256) variant_rows_k(i64 N, const int* __restrict__ mask, int nv,
                                                      const i64* __restrict__ desc, int* __restrict__ rows) {
    __shared__ i64 d[MAX_VLEVELS * 8];
    for (int j = threadIdx.x; j < nv * 8; j += blockDim.x) d[j] = desc[j];
    __syncthreads();
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    // the levels present at this position as bits, deepest = the highest
    const int m = mask[i];
    u32 present = 0;
    for (int v = 0; v < nv; ++v) present |= (u32)((m >> d[v * 8]) & 1) << v;
    if (!present) return;
    const i64* dv = d + (31 - __clz((int)present)) * 8;
    const i64 c = ((const int*)dv[2])[i];
    if (c < dv[3] || c >= dv[4]) return;  // another rank's context
    const i64 cl = c - dv[3];
    // the context's 8 tokens (one 16-byte load) and 8 counts (two)
    const uint4 tt = *(const uint4*)((const u16*)dv[5] + cl * 8);
    const uint4 c0 = *(const uint4*)((const u32*)dv[6] + cl * 8);
    const uint4 c1 = *(const uint4*)((const u32*)dv[6] + cl * 8 + 4);
    const u32 cnt[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const u64 total = ((const u64*)dv[7])[cl];
    u64 sum = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) sum += cnt[r];
    const double denom = sum > 1 ? (double)sum : 1.0;
    const double share = (double)cnt[0] / (double)(total > 1 ? total : 1);
    int* row = rows + i * 9;
    row[0] = ((1 + (int)dv[1]) * 7 + count_bin(total)) * 6 + purity_bin(share);
    row[1] = (int)tt.x;
    row[2] = (int)tt.y;
    row[3] = (int)tt.z;
    row[4] = (int)tt.w;
#pragma unroll
    for (int r = 0; r < 4; ++r) row[5 + r] = (int)(weight16(cnt[2 * r], denom) | (weight16(cnt[2 * r + 1], denom) << 16));
}
}  // namespace

// one variant's hint rows: cell, 8 tokens, 8 weights packed in int32[N, 9] (gpu_val_stats.cu:696-699); positions whose
// deepest level's context another rank owns, or without a level, are left as they are
extern "C" int variant_rows(i64 N, const int* mask, int nv, const i64* desc, int* rows, void* stream) {
    if (nv < 0 || nv > MAX_VLEVELS) return -1;
    if (N > 0 && nv > 0) variant_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, mask, nv, desc, rows);
    return (int)hipGetLastError();
}
