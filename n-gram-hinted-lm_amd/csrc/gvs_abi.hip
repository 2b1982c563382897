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
#include "pairs.h"
#include "prim.h"

#define KB_GVS 40  // pair key bits: 24-bit context ids (gpu_val_stats.cu:139-143)

// mode 0: dense, counted directly; 1: sparse, counted directly; 2: dense, emitted; 3: by words, emitted
extern "C" int scan_level(const u16* tok, i64 L, int k, const u32* bm_in, u32* bm_out, const u64* vt, u64 vcap,
                          const u32* vrep, const u16* x, u64* pk, u32* pc, u64 sub_cap, int pbits, u32* flags, int grid,
                          int mode, u64* emit, u64* emitted, void* stream) {
    if (L <= 0) return 0;
    if (grid <= 0) grid = grid_for(L, 256);
    hipStream_t st = (hipStream_t)stream;
    if (mode == 1 && bm_in) {
        LEVEL_SWITCH(k, (scan_sparse_k<K, KB_GVS><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags)));
    } else if (mode == 3 && bm_in) {
        LEVEL_SWITCH(k, (scan_words_emit_k<K><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, flags, emit, emitted)));
    } else if (mode == 2) {
        LEVEL_SWITCH(k, (scan_dense_k<K, true, KB_GVS><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags, emit, emitted)));
    } else {
        LEVEL_SWITCH(k, (scan_dense_k<K, false, KB_GVS><<<grid, 256, 0, st>>>(tok, L, k, bm_in, bm_out, vt, vcap, vrep, x, pk, pc, sub_cap, pbits, flags, emit, emitted)));
    }
    return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------
// Partitioned aggregation (kernels in pairs.h)
// ---------------------------------------------------------------------------------------------------------------

extern "C" int max_pbits() { return ng_max_pbits(); }

// emitted keys per sub-table (gpu_val_stats.cu:340-418)
extern "C" int subpart_count(const u64* keys, i64 n, int pbits, u64* counts, void* stream) {
    return launch_subpart_count(keys, n, pbits, counts, (hipStream_t)stream);
}

// emitted keys grouped by sub-table (gpu_val_stats.cu:420-428)
extern "C" int subpart_scatter(const u64* keys, i64 n, int pbits, u64* cursor, u64* out, void* stream) {
    return launch_subpart_scatter(keys, n, pbits, cursor, out, (hipStream_t)stream);
}

// grouped keys counted into the pair table (gpu_val_stats.cu:384-393, 430-434)
extern "C" int aggregate(const u64* keys, i64 n, u64* pk, u32* wraps, u64 sub_cap, int pbits, u32* flags, int grid,
                         void* stream) {
    return launch_aggregate<KB_GVS>(keys, n, pk, wraps, sub_cap, pbits, flags, grid, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Local aggregation by owner (context-id ranges [bounds[o], bounds[o + 1]))
// ---------------------------------------------------------------------------------------------------------------

// pair-table entries per owner (gpu_val_stats.cu:449-476)
extern "C" int part_count(const u64* pk, u64 cap, const i64* bounds, int W, u64* counts, void* stream) {
    return launch_part_count<KB_GVS>(pk, cap, bounds, W, counts, (hipStream_t)stream);
}

// pair-table entries as (key, count) grouped by owner (gpu_val_stats.cu:478-523)
extern "C" int part_scatter(const u64* pk, const u32* pc, u64 cap, const i64* bounds, int W, u64* cursor, u64* ok,
                            u32* oc, void* stream) {
    return launch_part_scatter<KB_GVS>(pk, pc, cap, bounds, W, cursor, ok, oc, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// Owner side: ranks and per-position outputs
// ---------------------------------------------------------------------------------------------------------------

// rank of each pair within its context; the top `top` tokens/counts per context (gpu_val_stats.cu:592-612)
extern "C" int rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                            u16* top_tok, u32* top_cnt, int top, void* stream) {
    return ng::launch_rank_scatter(sv, U, uk, agg, start, rank_of, top_tok, top_cnt, top, (hipStream_t)stream);
}

// per query position: tot, dist, cnt (the TOP rule: the target's count if its rank < cnt_top), mask bit li
// (gpu_val_stats.cu:614-644)
extern "C" int pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                           const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                           int* out_tot, int* out_dist, int* out_cnt, int* mask, void* stream) {
    return ng::launch_pos_outputs(ctx_of, N, lo, hi, tgt, uk, agg, rank_of, start, end, tot, li, cnt_top, out_tot,
                                  out_dist, out_cnt, mask, (hipStream_t)stream);
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
