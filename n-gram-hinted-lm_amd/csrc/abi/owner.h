// The per-position outputs and rank scatter shared by the two ABI flavours (defined in owner.hip), which wrap them in
// their own signatures: the gpu_val_stats flavour with rank_of, the TOP rule and the mask bit, the record's without.
#pragma once
#include "../ngram_common.h"

namespace abi {
// Per query position whose context id is in [lo, hi): tot, dist, cnt (with rank_of: only if the target's rank is below
// cnt_top) and, with mask, bit li of mask[i].
int launch_pos_outputs(const int* ctx_of, i64 N, i64 lo, i64 hi, const u16* tgt, const u64* uk, const u32* agg,
                       const u32* rank_of, const i64* start, const i64* end, const u64* tot, int li, int cnt_top,
                       int* out_tot, int* out_dist, int* out_cnt, int* mask, hipStream_t st);
// Each pair's rank in its context (rank_of, may be NULL) and each context's first `top` tokens and counts (top_tok /
// top_cnt [contexts, top], may be NULL).
int launch_rank_scatter(const u32* sv, i64 U, const u64* uk, const u32* agg, const i64* start, u32* rank_of,
                        u16* top_tok, u32* top_cnt, int top, hipStream_t st);
}  // namespace abi
