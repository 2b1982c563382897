// The record flavour of the C ABI (record_367_gpu_counts/track_1_short/counts/kernels.cu:237-437), built into its own
// library (libngram_amd_record.so) because its entry points keep the record's names with other signatures:
//   * pair keys of 41 bits (25-bit context ids: up to 2^25 - 4096 query contexts per level) and 23-bit counts plus
//     the wrap byte (kernels.cu:132-136);
//   * scan_level takes one table (no sub-tables, no emit) and a `sparse` flag instead of a mode;
//   * rank_scatter has no rank_of, pos_outputs no TOP rule, rank_of, level index or mask (kernels.cu:377-437).
// The shared entry points (val_keys, val_verify, val_homes, sort_pairs, inclusive_max, reduce_by_key, seg_bounds,
// ctx_tot, rank_keys) come from common_abi.hip. Extensions (no counterpart in the record's library): pos_topk, the
// per-position gather of a context's top next tokens that the record's host does with torch indexing
// (build.py:360-368); and the partitioned counting of the gpu_val_stats library (scan_emit = its scan_level modes 2/3,
// subpart_count, subpart_scatter, aggregate, popcount; gpu_val_stats.cu:268-446) on this flavour's 41-bit pair keys.
#include "../pairs.h"

#define KB_REC 41

extern "C" int scan_level(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                          const u32* vrep, const u16* x, u64* pk, u32* pc, u64 cap, u32* flags, int grid, int sparse,
                          void* stream) {
    if (L <= 0) return 0;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    if (sparse && bm_in) {
        LEVEL_SWITCH(k, (scan_sparse_k<K, KB_REC><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, cap, 0, flags)));
    } else {
        LEVEL_SWITCH(k, (scan_dense_k<K, false, KB_REC><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, cap, 0, flags, nullptr, nullptr)));
    }
    return (int)hipGetLastError();
}

extern "C" int part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, void* stream) {
    return launch_part_count<KB_REC>(pk, cap, bounds, W, counts, (hipStream_t)stream);
}

extern "C" int part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                            u32* oc, void* stream) {
    return launch_part_scatter<KB_REC>(pk, pc, cap, bounds, W, cursor, ok, oc, (hipStream_t)stream);
}

extern "C" int rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u16* top_tok,
                            u32* top_cnt, int top, void* stream) {
    return ng::launch_rank_scatter(sv, U, uk, agg, start, nullptr, top_tok, top_cnt, top, (hipStream_t)stream);
}

extern "C" int pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                           const i64* start, const i64* end, const u64* tot, int* out_tot, int* out_dist, int* out_cnt,
                           void* stream) {
    return ng::launch_pos_outputs(ctx_of, N, lo, hi, tgt, uk, agg, nullptr, start, end, tot, 0, 0, out_tot, out_dist,
                                  out_cnt, nullptr, (hipStream_t)stream);
}

// Per query position whose context id c is in [lo, hi): the first `kout` of the context's `top` ranked next tokens and
// counts (top_tok/top_cnt [hi - lo, top], from rank_scatter) into out_tok/out_cnt [N, kout]; other positions untouched.
__global__ void pos_topk_k(const int* __restrict__ ctx_of, i64 N, i64 lo, i64 hi, const u16* __restrict__ top_tok,
                           const u32* __restrict__ top_cnt, int top, int kout, u16* __restrict__ out_tok,
                           u32* __restrict__ out_cnt) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const i64 c = ctx_of[i];
    if (c < lo || c >= hi) return;
    const u16* tt = top_tok + (c - lo) * top;
    const u32* tc = top_cnt + (c - lo) * top;
    for (int r = 0; r < kout; ++r) {
        out_tok[i * kout + r] = tt[r];
        out_cnt[i * kout + r] = tc[r];
    }
}

extern "C" int pos_topk(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* top_tok, const u32* top_cnt, int top,
                        int kout, u16* out_tok, u32* out_cnt, void* stream) {
    if (kout < 1 || kout > top) return -1;
    if (N > 0)
        pos_topk_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(ctx_of, N, lo, hi, top_tok, top_cnt, top, kout,
                                                                       out_tok, out_cnt);
    return (int)hipGetLastError();
}

// A level's scan that appends every hit's pair key to emit[*emitted ...] instead of counting it (words: a lane per
// bitmap word, for sparse levels; bm_in required); the hit bitmap as scan_level's.
extern "C" int scan_emit(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                         const u32* vrep, const u16* x, u32* flags, int grid, int words, u64* emit, u64* emitted,
                         void* stream) {
    if (L <= 0) return 0;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    if (words && bm_in) {
        LEVEL_SWITCH(k, (scan_words_emit_k<K><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, emit, emitted)));
    } else {
        LEVEL_SWITCH(k, (scan_dense_k<K, true, KB_REC><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, nullptr, nullptr, 0, 0, flags, emit, emitted)));
    }
    return (int)hipGetLastError();
}

extern "C" int max_pbits() { return ng_max_pbits(); }

extern "C" int subpart_count(const u64* keys, i64 n, int pbits, u64* counts, void* stream) {
    return launch_subpart_count(keys, n, pbits, counts, (hipStream_t)stream);
}

extern "C" int subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, void* stream) {
    return launch_subpart_scatter(keys, n, pbits, cursor, out, (hipStream_t)stream);
}

extern "C" int aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                         void* stream) {
    return launch_aggregate<KB_REC>(keys, n, pk, wraps, sub_cap, pbits, flags, grid, (hipStream_t)stream);
}
