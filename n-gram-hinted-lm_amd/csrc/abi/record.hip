// The record flavour of the C ABI (record_367_gpu_counts/track_1_short/counts/kernels.cu:237-437, bound by
// counts/build.py:74-92), built into its own library (libngram_amd_record.so) because its entry points keep the
// record's names with other signatures:
//   * pair keys of 41 bits (25-bit context ids: up to 2^25 - 4096 query contexts per level) and 23-bit counts plus
//     the wrap byte (kernels.cu:132-136);
//   * scan_level takes one table (no sub-tables, no emit) and a `sparse` flag instead of a mode;
//   * rank_scatter has no rank_of, pos_outputs no TOP rule, rank_of, level index or mask (kernels.cu:377-437).
// The shared entry points (val_keys, val_verify, val_homes, sort_pairs, inclusive_max, reduce_by_key, seg_bounds,
// ctx_tot, rank_keys, popcount) come from abi/owner.hip; the kernels are this build's (abi/packed.h). Extensions (no
// counterpart in the record's library): pos_topk, the per-position gather of a context's top next tokens that the
// record's host does with torch indexing (build.py:360-368); and the partitioned counting of the gpu_val_stats
// library (scan_emit, subpart_count, subpart_scatter, aggregate) on this flavour's 41-bit pair keys.
#include "owner.h"
#include "packed.h"

#define KB_REC 41

// one level's scan over L positions: lookup, hit bitmap, count in the one pair table of `cap` slots; with bm_in only
// its set positions are looked up (`sparse` only chooses how the reference walks them: here one tile kernel serves
// both)
extern "C" int scan_level(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                          const u32* vrep, const u16* x, u64* pk, u32* pc, u64 cap, u32* flags, int grid, int sparse,
                          void* stream) {
    (void)sparse;
    if (!pk || !pc || cap == 0) return -1;
    return abi::launch_tile_scan<KB_REC>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, grid,
                                         abi::TableSink{pk, pc, cap, 0}, (hipStream_t)stream);
}

extern "C" int part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, void* stream) {
    return abi::launch_own_count<KB_REC>(pk, cap, bounds, W, counts, (hipStream_t)stream);
}

extern "C" int part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                            u32* oc, void* stream) {
    return abi::launch_own_scatter<KB_REC>(pk, pc, cap, bounds, W, cursor, ok, oc, (hipStream_t)stream);
}

extern "C" int rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u16* top_tok,
                            u32* top_cnt, int top, void* stream) {
    return abi::launch_rank_scatter(sv, U, uk, agg, start, nullptr, top_tok, top_cnt, top, (hipStream_t)stream);
}

extern "C" int pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                           const i64* start, const i64* end, const u64* tot, int* out_tot, int* out_dist, int* out_cnt,
                           void* stream) {
    return abi::launch_pos_outputs(ctx_of, N, lo, hi, tgt, uk, agg, nullptr, start, end, tot, 0, 0, out_tot, out_dist,
                                   out_cnt, nullptr, (hipStream_t)stream);
}

namespace {
// Per query position whose context id is in [lo, hi): the first kout of its context's `top` ranked tokens and counts.
// A wave takes 64 positions; its lanes then copy the rows of the wave's owned positions, one entry per lane, so the
// stores of a row are contiguous.
__global__ void __launch_bounds__(256) pos_topk_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi,
                                                  const u16* __restrict__ top_tok, const u32* __restrict__ top_cnt,
                                                  int top, int kout, u16* __restrict__ out_tok,
                                                  u32* __restrict__ out_cnt) {
    const i64 i0 = (blockIdx.x * (i64)blockDim.x + threadIdx.x) & ~(i64)(WAVE - 1);
    const int lane = lane_id();
    const i64 i = i0 + lane;
    i64 c = -1;
    if (i < N) {
        c = ctx_of[i];
        if (c < lo || c >= hi) c = -1;
    }
    u64 owned = __ballot(c >= 0);
    while (owned) {  // the wave's owned positions in turn, kout entries each spread over the lanes
        const int l = __ffsll((unsigned long long)owned) - 1;
        owned &= owned - 1;
        const i64 cl = (i64)bcast_u64((u64)c, l) - lo;
        for (int r = lane; r < kout; r += WAVE) {
            out_tok[(i0 + l) * kout + r] = top_tok[cl * top + r];
            out_cnt[(i0 + l) * kout + r] = top_cnt[cl * top + r];
        }
    }
}
}  // namespace

extern "C" int pos_topk(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* top_tok, const u32* top_cnt, int top,
                        int kout, u16* out_tok, u32* out_cnt, void* stream) {
    if (kout < 1 || kout > top) return -1;
    if (N > 0)
        pos_topk_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, N, lo, hi, top_tok, top_cnt, top, kout,
                                                                       out_tok, out_cnt);
    return (int)hipGetLastError();
}

// A level's scan that appends every hit's pair key to emit[*emitted ...] instead of counting it; `words` is accepted
// for the reference's signature (the tile kernel lists gated positions whatever the density). Hit bitmap as
// scan_level's.
extern "C" int scan_emit(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                         const u32* vrep, const u16* x, u32* flags, int grid, int words, u64* emit, u64* emitted,
                         void* stream) {
    (void)words;
    if (!emit || !emitted) return -1;
    return abi::launch_tile_scan<KB_REC>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, grid,
                                         abi::AppendSink{emit, emitted}, (hipStream_t)stream);
}

extern "C" int max_pbits() { return abi::max_group_bits(); }

extern "C" int subpart_count(const u64* keys, i64 n, int pbits, u64* counts, void* stream) {
    return abi::launch_group_hist(keys, n, pbits, counts, (hipStream_t)stream);
}

extern "C" int subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, void* stream) {
    return abi::launch_group_scatter(keys, n, pbits, cursor, out, (hipStream_t)stream);
}

extern "C" int aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                         void* stream) {
    return abi::launch_aggregate<KB_REC>(keys, n, pk, wraps, sub_cap, pbits, flags, grid, (hipStream_t)stream);
}
