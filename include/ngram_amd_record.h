/* ngram_amd record flavour: the C ABI of libngram_amd_record.so, the drop-in for the record's kernels library that
 * record_367_gpu_counts/track_1_short/counts/build.py binds (Lib :74-92, replacing counts/kernels.cu: same names,
 * argument meaning and return codes). Conventions as ngram_amd.h: device pointers, 64-bit sizes, the HIP stream
 * (hipStream_t as void*) last, 0 or a hipError_t value, -1 for unsupported arguments; nothing allocates.
 * Pair keys are 41 bits (25-bit context ids, the record's MAX_IDS = 2^25 - 4096) with 23-bit counts + a wrap byte
 * (kernels.cu:132-136). k: 1..64 (the record's LEVEL_SWITCH accepts 2-6, 10, 20 and returns -1 otherwise).
 */
#ifndef NGRAM_AMD_RECORD_H
#define NGRAM_AMD_RECORD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef unsigned long long ng_u64;
typedef long long ng_i64;

/* shared with the gpu_val_stats flavour (same signatures): kernels.cu:80-125 and :331-370 */
int val_keys(const uint16_t* x, const int* avail, ng_i64 n, int k, ng_u64* out, void* stream);
int val_verify(const uint16_t* x, const ng_i64* spos, const ng_i64* gid, const ng_i64* rep, ng_i64 n, int k,
               ng_u64* bad, void* stream);
int val_homes(const ng_u64* keys, ng_i64 n, ng_u64 cap, ng_i64* home, void* stream);
int sort_pairs(void* temp, size_t* temp_bytes, const ng_u64* kin, ng_u64* kout, const uint32_t* vin, uint32_t* vout,
               ng_i64 n, int begin_bit, int end_bit, void* stream);
int inclusive_max(void* temp, size_t* temp_bytes, const ng_i64* in, ng_i64* out, ng_i64 n, void* stream);
int reduce_by_key(void* temp, size_t* temp_bytes, const ng_u64* kin, ng_u64* kout, const uint32_t* vin,
                  uint32_t* vout, ng_i64* nruns, ng_i64 n, void* stream);
int seg_bounds(const ng_u64* uk, ng_i64 U, ng_i64* start, ng_i64* end, void* stream);
int ctx_tot(const ng_i64* start, const ng_i64* end, const uint32_t* agg, ng_i64 nctx, ng_u64* tot, void* stream);
int rank_keys(const ng_u64* uk, const uint32_t* agg, ng_i64 U, ng_u64* key2, uint32_t* val2, void* stream);

/* one level's scan over L positions: probe, hit bitmap, count in the one pair table of `cap` slots; `sparse` walks
 * the set bits of bm_in (kernels.cu:237-247) */
int scan_level(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
               ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, ng_u64* pk, uint32_t* pc, ng_u64 cap,
               uint32_t* flags, int grid, int sparse, void* stream);
/* pair-table entries per owner / as (key, count) grouped by owner (kernels.cu:259-328) */
int part_count(const ng_u64* pk, ng_u64 cap, const ng_i64* bounds, int W, ng_u64* counts, void* stream);
int part_scatter(const ng_u64* pk, const uint32_t* pc, ng_u64 cap, const ng_i64* bounds, int W, ng_u64* cursor,
                 ng_u64* ok, uint32_t* oc, void* stream);
/* the top `top` tokens/counts per context, no rank_of (kernels.cu:391-409) */
int rank_scatter(const uint32_t* sv, ng_i64 U, const ng_u64* uk, const uint32_t* agg, const ng_i64* start,
                 uint16_t* top_tok, uint32_t* top_cnt, int top, void* stream);
/* per query position: tot, dist, cnt (the target's count, no TOP rule) (kernels.cu:411-437) */
int pos_outputs(const int* ctx_of, ng_i64 N, ng_i64 lo, ng_i64 hi, const uint16_t* tgt, const ng_u64* uk,
                const uint32_t* agg, const ng_i64* start, const ng_i64* end, const ng_u64* tot, int* out_tot,
                int* out_dist, int* out_cnt, void* stream);

/* Extension (the record gathers these with torch indexing, build.py:360-368): per query position whose context id is
 * in [lo, hi), the first kout of its context's `top` ranked next tokens and counts into out_tok/out_cnt [N, kout]. */
int pos_topk(const int* ctx_of, ng_i64 N, ng_i64 lo, ng_i64 hi, const uint16_t* top_tok, const uint32_t* top_cnt,
             int top, int kout, uint16_t* out_tok, uint32_t* out_cnt, void* stream);

/* Extensions: the gpu_val_stats library's partitioned counting (gpu_val_stats.cu:268-446) on 41-bit pair keys, for a
 * host that counts dense levels in L2/MALL-sized sub-tables instead of one table (same semantics as there):
 * scan_emit = scan_level modes 2 (words = 0) / 3 (words = 1); popcount adds a bitmap's set bits to *out. */
int scan_emit(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
              ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, uint32_t* flags, int grid, int words,
              ng_u64* emit, ng_u64* emitted, void* stream);
int max_pbits(void);
int subpart_count(const ng_u64* keys, ng_i64 n, int pbits, ng_u64* counts, void* stream);
int subpart_scatter(const ng_u64* keys, ng_i64 n, int pbits, ng_u64* cursor, ng_u64* out, void* stream);
int aggregate(const ng_u64* keys, ng_i64 n, ng_u64* pk, uint32_t* wraps, ng_u64 sub_cap, int pbits, uint32_t* flags,
              int grid, void* stream);
int popcount(const uint32_t* bm, ng_i64 n, ng_u64* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* NGRAM_AMD_RECORD_H */
