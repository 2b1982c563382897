/* ngram_amd: the C ABI of the MI355X (gfx950) n-gram hint engine, libngram_amd.so.
 *
 * Conventions (those of the reference's ctypes binding, old_records/gpu_val_stats.py:133-158): plain pointers to
 * device memory, 64-bit sizes, the HIP stream last (a hipStream_t passed as void*); calls are asynchronous on that
 * stream; the return value is 0 or a hipError_t value, -1 for unsupported arguments. No entry point allocates device
 * memory: buffers are the caller's; the *_temp_bytes / two-phase calls size the caller's scratch.
 * Tokens are uint16 (GPT-2 ids, BOS = 50256); SENT = 0xFFFF marks the gaps between concatenated shards.
 */
#ifndef NGRAM_AMD_H
#define NGRAM_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef unsigned long long ng_u64;
typedef long long ng_i64;

/* ------------------------------------------------------------------------------------------------------------
 * gpu_val_stats flavour: the entry points old_records/gpu_val_stats.py binds (replacing
 * old_records/gpu_val_stats.cu, same names, arguments and return codes). k: 1..64 (the reference's LEVEL_SWITCH
 * accepts 1-8, 10, 12, 16, 20 and returns -1 otherwise; this build also runs the other k up to 64).
 * ------------------------------------------------------------------------------------------------------------ */

/* per query position i: the key of x[i-k+1..i] if avail[i] >= k, else EMPTY (gpu_val_stats.cu:96-99) */
int val_keys(const uint16_t* x, const int* avail, ng_i64 n, int k, ng_u64* out, void* stream);
/* each valid position's k tokens vs its group representative's; mismatches counted in *bad (gpu_val_stats.cu:114-119) */
int val_verify(const uint16_t* x, const ng_i64* spos, const ng_i64* gid, const ng_i64* rep, ng_i64 n, int k,
               ng_u64* bad, void* stream);
/* home slot umulhi(key, cap) of each key (gpu_val_stats.cu:129-132) */
int val_homes(const ng_u64* keys, ng_i64 n, ng_u64 cap, ng_i64* home, void* stream);
/* one level's scan: probe, bitmap of hits, count (mode 0 dense / 1 sparse) or emit (2 dense / 3 by words)
 * (gpu_val_stats.cu:306-338) */
int scan_level(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
               ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, ng_u64* pk, uint32_t* pc, ng_u64 sub_cap,
               int pbits, uint32_t* flags, int grid, int mode, ng_u64* emit, ng_u64* emitted, void* stream);
/* emitted keys per sub-table (gpu_val_stats.cu:410-418) */
int subpart_count(const ng_u64* keys, ng_i64 n, int pbits, ng_u64* counts, void* stream);
/* emitted keys grouped by sub-table (gpu_val_stats.cu:420-428) */
int subpart_scatter(const ng_u64* keys, ng_i64 n, int pbits, ng_u64* cursor, ng_u64* out, void* stream);
/* grouped keys counted into the pair table (gpu_val_stats.cu:430-434) */
int aggregate(const ng_u64* keys, ng_i64 n, ng_u64* pk, uint32_t* wraps, ng_u64 sub_cap, int pbits, uint32_t* flags,
              int grid, void* stream);
/* the most sub-table bits the LDS histograms allow on this device (gpu_val_stats.cu:396-403; no stream) */
int max_pbits(void);
/* set bits of a bitmap added to *out (gpu_val_stats.cu:443-446) */
int popcount(const uint32_t* bm, ng_i64 n, ng_u64* out, void* stream);
/* pair-table entries per owner (gpu_val_stats.cu:472-476) */
int part_count(const ng_u64* pk, ng_u64 cap, const ng_i64* bounds, int W, ng_u64* counts, void* stream);
/* pair-table entries as (key, count) grouped by owner (gpu_val_stats.cu:518-523) */
int part_scatter(const ng_u64* pk, const uint32_t* pc, ng_u64 cap, const ng_i64* bounds, int W, ng_u64* cursor,
                 ng_u64* ok, uint32_t* oc, void* stream);
/* stable radix sort of (u64 key, u32 value) by key bits [begin_bit, end_bit); temp == NULL: *temp_bytes = the
 * scratch needed (CUB-style; gpu_val_stats.cu:530-536) */
int sort_pairs(void* temp, size_t* temp_bytes, const ng_u64* kin, ng_u64* kout, const uint32_t* vin, uint32_t* vout,
               ng_i64 n, int begin_bit, int end_bit, void* stream);
/* inclusive running maximum of int64 (gpu_val_stats.cu:539-543) */
int inclusive_max(void* temp, size_t* temp_bytes, const ng_i64* in, ng_i64* out, ng_i64 n, void* stream);
/* runs of equal keys -> unique keys, summed values, *nruns (gpu_val_stats.cu:545-551); vin NULL (an extension):
 * every value counts 1, vout = the runs' lengths */
int reduce_by_key(void* temp, size_t* temp_bytes, const ng_u64* kin, ng_u64* kout, const uint32_t* vin,
                  uint32_t* vout, ng_i64* nruns, ng_i64 n, void* stream);
/* per context id: [start, end) of its pairs in sorted keys (gpu_val_stats.cu:561-564) */
int seg_bounds(const ng_u64* uk, ng_i64 U, ng_i64* start, ng_i64* end, void* stream);
/* per context: total = sum of its pair counts (gpu_val_stats.cu:574-577) */
int ctx_tot(const ng_i64* start, const ng_i64* end, const uint32_t* agg, ng_i64 nctx, ng_u64* tot, void* stream);
/* ranking keys: context << 32 | (2^32 - 1 - count), value = pair index (gpu_val_stats.cu:587-590) */
int rank_keys(const ng_u64* uk, const uint32_t* agg, ng_i64 U, ng_u64* key2, uint32_t* val2, void* stream);
/* rank of each pair within its context; the top `top` tokens/counts per context (gpu_val_stats.cu:606-612) */
int rank_scatter(const uint32_t* sv, ng_i64 U, const ng_u64* uk, const uint32_t* agg, const ng_i64* start,
                 uint32_t* rank_of, uint16_t* top_tok, uint32_t* top_cnt, int top, void* stream);
/* per query position: tot, dist, cnt (TOP rule), mask bit li (gpu_val_stats.cu:637-644) */
int pos_outputs(const int* ctx_of, ng_i64 N, ng_i64 lo, ng_i64 hi, const uint16_t* tgt, const ng_u64* uk,
                const uint32_t* agg, const uint32_t* rank_of, const ng_i64* start, const ng_i64* end,
                const ng_u64* tot, int li, int cnt_top, int* out_tot, int* out_dist, int* out_cnt, int* mask,
                void* stream);
/* one variant's hint rows: cell, 8 tokens, 8 weights packed in int32[N, 9] (gpu_val_stats.cu:696-699) */
int variant_rows(ng_i64 N, const int* mask, int nv, const ng_i64* desc, int* rows, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * Synthetic streams (no counterpart in the reference, whose data are FineWeb shards): the seeded generator of the
 * benchmark configurations, byte-identical to ngram_amd/data.py's numpy generator. A body token of stream `key` at
 * position p: h = splitmix64_finalizer(key + (p + 1) * 0x9E3779B97F4A7C15), u = (h >> 11) * 2^-53,
 * token = perm[min(#{cdf[j] <= u}, ncdf - 1)].
 * ------------------------------------------------------------------------------------------------------------ */

/* out[i] = the draw of position start + i of stream key, i in [0, n) */
int gen_tokens(uint16_t* out, ng_i64 start, ng_i64 n, ng_u64 key, const double* cdf, int ncdf, const uint16_t* perm,
               void* stream);
/* out[pos[i]] = value (the documents' BOS) */
int gen_set(uint16_t* out, const ng_i64* pos, ng_i64 m, int value, void* stream);
/* per copy (dst, src, length) of copies[m][3]: out[dst + j] = src_tokens[src + j], or the draw of position src + j of
 * stream key when src_tokens is NULL */
int gen_copies(uint16_t* out, const ng_i64* copies, ng_i64 m, const uint16_t* src_tokens, ng_u64 key,
               const double* cdf, int ncdf, const uint16_t* perm, void* stream);

/* ------------------------------------------------------------------------------------------------------------
 * Engine entry points: no counterpart in the reference's libraries. They implement, for this repository's hosts
 * (ngram_amd.counts / count_table / online / longest / exact_match), the query-filtered counting of
 * record_367_gpu_counts/track_1_short/counts/build.py, exact_match/src/count_table.rs, online.rs and kgram.rs with
 * split pair tables (u64 pair keys and u32 counts in two arrays) and selection-based ranking. Same conventions as
 * above. k: 1..64. A query table (vt, vcap, vrep) passed to an engine scan is an ng_query_index table: linear probing
 * without wrap-around from umulhi(key, vcap), and at least one slot past vcap (ng_query_index's callers give 4096),
 * since a lookup loads the home slot and the next one together.
 * ------------------------------------------------------------------------------------------------------------ */

/* one level's scan counted in a split table (keys EMPTY-filled, cnts zeroed); sparse 0: a lane per position, 1: a
 * lane per bitmap word, 2: the set positions listed per wave in LDS (bm_in required for 1 and 2); flags[0] = full */
int ng_scan_count(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
                  ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, ng_u64* keys, uint32_t* cnts, ng_u64 cap,
                  uint32_t* flags, int grid, int sparse, void* stream);
/* the emitting scan: block b of `grid` appends its hits' events to ev[b * region ...] and stores how many in
 * ev_count[b]; region >= ng_emit_region(L, grid) = ceil(L / (grid * 8192)) * 8192; flags[0] bit 2 a region
 * overflowed. sparse as ng_scan_count's. Events: wbits 0: mix64(context id << 16 | next), digit its top 8 bits;
 * wbits in [17, 63]: kmix(pair key, wbits, mbits) (the 32-bit count's W-bit bijection, pair keys below 2^wbits: the
 * bits from mbits up kept, the mbits below mixed; 17 <= mbits <= wbits, 0: wbits), digit its top dbits bits
 * (1 <= dbits <= 10). dhist (may be NULL): block b's events per digit d at dhist[d * dstride + b]
 * (dstride >= grid), for ng_seg_scatter / ng_seg_scatter_narrow. pre (may be NULL): a device flag; while set, a
 * position of bm_in is probed only if the position before it is set as well (the prefix rule, ng_avail_closed) */
ng_u64 ng_emit_region(ng_i64 L, int grid);
int ng_scan_emit(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
                 ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, ng_u64* ev, ng_u64 region, uint32_t* ev_count,
                 uint32_t* flags, int grid, int sparse, uint32_t* dhist, ng_i64 dstride, const uint32_t* pre,
                 int wbits, int dbits, int mbits, void* stream);
/* *flag = 1 if avail[i] <= max(avail[i - 1], 0) + 1 wherever avail[i] > 1 (every valid query context's prefix is the
 * previous position's valid context: the prefix rule may gate the scans), else 0; stream-ordered, no host sync */
int ng_avail_closed(const int* avail, ng_i64 n, uint32_t* flag, void* stream);
/* *total = the positions a level scan probes behind hit words bm: their set bits, under the prefix rule while the
 * device flag pre is set (a roofline's probe count) */
int ng_gate_popcount(const uint32_t* bm, ng_i64 nwords, const uint32_t* pre, ng_u64* total, void* stream);
/* n random 8-byte loads from table (cap u64) at umulhi(mix64(seed + i), cap), grid blocks of 256, per-thread sums to
 * out (grid * 256 u64): the random-load rate a level scan's probes are measured against */
int ng_gather_probe(const ng_u64* table, ng_u64 cap, ng_u64 n, ng_u64 seed, int grid, ng_u64* out, void* stream);
/* the emitting scan over listed positions: the first *n_dev entries of plist (a device-side count: no host sync),
 * events (by wbits / dbits / mbits) and digit histograms as ng_scan_emit's, each hit's bit set in bm_out (zeroed by the
 * caller; may be NULL); region >= ceil(n / (grid * 256)) * 256 */
int ng_scan_emit_list(const uint16_t* tok, const ng_u64* plist, const ng_u64* n_dev, int k, const ng_u64* vt,
                      ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, uint32_t* bm_out, ng_u64* ev, ng_u64 region,
                      uint32_t* ev_count, uint32_t* flags, int grid, uint32_t* dhist, ng_i64 dstride, int wbits,
                      int dbits, int mbits, void* stream);
/* a level scan with optional outputs over a bitmap-gated range (plist NULL: [0, L) gated by bm_in in ng_scan_count's
 * sparse modes, hit bitmap into bm_out) or over listed positions (plist: n corpus positions); hit (may be NULL):
 * bit (context id) of the u32 words hit set per hit; ev (may be NULL): block b of grid appends per hit mix64(pair key + key_add) (what 0) or its
 * position (what 1) to ev[b * region ...], how many into ev_count[b]; region >= ng_emit_region(L, grid) over a
 * bitmap, >= ceil(n / (grid * 256)) * 256 over a list */
int ng_scan_sink(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* plist,
                 ng_i64 n, const ng_u64* vt, ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, uint32_t* hit,
                 int what, ng_u64* ev, ng_u64 region, uint32_t* ev_count, uint32_t* flags, int grid, int sparse,
                 ng_u64 key_add, void* stream);
/* the set bits of a bitmap as positions in order (out), *total of them; pre (may be NULL) as ng_scan_emit's: while
 * the device flag is set, only bits whose previous bit is set too; two-phase temp storage (temp NULL: size) */
int ng_bits_list(void* temp, size_t* temp_bytes, const uint32_t* bm, ng_i64 nwords, ng_u64* out, ng_u64* total,
                 const uint32_t* pre, void* stream);
/* ng_bits_list's positions as int32 (nwords <= 2^26), the first cap kept (*total counts every set bit) */
int ng_bits_list32(void* temp, size_t* temp_bytes, const uint32_t* bm, ng_i64 nwords, int* out, ng_i64 cap,
                   ng_u64* total, const uint32_t* pre, void* stream);
/* existence only: hit bitmap and bit (context id) of the u32 words hit set (hit zeroed by the caller); ids (may be
 * NULL): ids[p] = the context id at each hit position p; sparse as ng_scan_count's; pre (may be NULL): the prefix
 * rule's device flag, as ng_scan_emit's (valid where every query context's prefix is a query context of the level
 * before) */
int ng_scan_exist(const uint16_t* tok, ng_i64 L, int k, const uint32_t* bm_in, uint32_t* bm_out, const ng_u64* vt,
                  ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, uint32_t* hit, uint32_t* ids, uint32_t* flags,
                  int grid, int sparse, const uint32_t* pre, void* stream);
/* level 1 of ng_scan_exist (no gate) with each 1-context's token as its context id, so no table: member (2048
 * words) bit t for each query token t; bm_out (L / 32 words) the hit positions (p: tok[p - 1] a query token, neither
 * it nor tok[p] SENT); hit (2048 words, zeroed by the caller) bit t where token t occurred; ids (may be NULL)
 * ids[p] = tok[p - 1] at each hit position p. L a multiple of 32; grid <= 0: 2048 blocks (each block ORs its hit
 * words into hit once) */
int ng_scan_tok1(const uint16_t* tok, ng_i64 L, const uint32_t* member, uint32_t* bm_out, uint32_t* hit,
                 uint32_t* ids, int grid, void* stream);
/* a level's counting scan from ng_scan_exist's ids (NULL: ng_scan_tok1's level, the id at p being tok[p - 1]): each
 * position set in bm whose context's bit is set in `final` emits its (id << 16 | tok[p]) event as ng_scan_emit's (regions, ev_count, dhist; wbits 0: mix64 with the top 8
 * bits' histogram, wbits 17..63: kmix(key, wbits, mbits) with the top dbits bits', dbits <= 10); L a multiple of 32, tok
 * 8-byte and ids 16-byte aligned */
int ng_scan_ids_emit(const uint16_t* tok, ng_i64 L, const uint32_t* bm, const uint32_t* ids, const uint32_t* final,
                     ng_u64* ev, ng_u64 region, uint32_t* ev_count, uint32_t* flags, int grid, uint32_t* dhist,
                     ng_i64 dstride, int wbits, int dbits, int mbits, void* stream);
/* bit ids[i] of the u32 words bits set for each ids[i] >= 0 (bits zeroed by the caller) */
int ng_mark_bits(const int* ids, ng_i64 n, uint32_t* bits, void* stream);
/* a split table's occupied slots appended to (out_k, out_c) from *counter (zeroed by the caller) */
int ng_table_compact(const ng_u64* keys, const uint32_t* cnts, ng_u64 cap, ng_u64* out_k, uint32_t* out_c,
                     ng_u64* counter, void* stream);
/* per context (pairs sorted by key, seg_bounds' start/end): total and top-k (1, 2, 4, 8) by count desc, token asc */
int ng_ctx_topk(const ng_u64* uk, const uint32_t* agg, const ng_i64* start, const ng_i64* end, ng_i64 nctx, int topk,
                ng_u64* tot, uint16_t* top_tok, uint32_t* top_cnt, void* stream);
/* per query position with context in [lo, hi): tot, dist, cnt (qcnt[i] when given, else from the split table
 * pkeys/pcnts of pcap slots when given, else by binary search of the context's sorted pairs; with thr, only if its
 * score count << 16 | 65535 - token >= thr[c]), the first kout of ktop top entries, mask bit li (mask may be NULL) */
int ng_pos_gather(const int* ctx_of, ng_i64 N, ng_i64 lo, ng_i64 hi, const uint16_t* tgt, const ng_u64* uk,
                  const uint32_t* agg, const ng_i64* start, const ng_i64* end, const ng_u64* tot,
                  const uint16_t* top_tok, const uint32_t* top_cnt, const ng_u64* thr, const ng_u64* pkeys,
                  const uint32_t* pcnts, ng_u64 pcap, const uint32_t* qcnt, int ktop, int kout, int li, int* out_tot,
                  int* out_dist, int* out_cnt, uint16_t* out_tok, uint32_t* out_tcnt, int* mask, void* stream);
/* query index without a sort (replaces gpu_val_stats.py:604-651's sort-based one where ids need not agree across
 * ranks): valid k-contexts of positions pos[0..n) (NULL: 0..n; n_dev (may be NULL, pos required): a device-side count,
 * pos[0..min(n, *n_dev)) only) inserted by compare-and-swap into table (cap + tail
 * slots, EMPTY-filled, linear probing without wrap from umulhi(key, cap)); ctx_of[i] = slot or -1 (compact:
 * ctx_of[j] for pos[j]), rep[slot] = the inserting position; counters[0] += the table's occupied slots
 * afterwards (the inserts counted per wave into wave_ins, ceil(n / 256) * 4 u32 of scratch; NULL: a scan of the
 * table), counters[1] != 0: the table is too small (a probe reached its end or walked 256 slots),
 * counters[2] += key collisions found against the representative (k > 4) */
int ng_query_index(const uint16_t* x, const int* avail, const int* pos, ng_i64 n, const ng_u64* n_dev, int k,
                   ng_u64* table, ng_u64 cap, ng_u64 slots, uint32_t* rep, int* ctx_of, int compact,
                   ng_u64* counters, uint32_t* wave_ins, void* stream);
/* move a query index into a smaller EMPTY-filled table (cap + tail = slots): ctx_of[0..n) re-pointed, remap
 * (old_slots ints) scratch, counters[1] = 1 on reaching the new table's end */
int ng_query_index_shrink(const ng_u64* old_t, const uint32_t* old_rep, ng_u64 old_slots, ng_u64* table, ng_u64 cap,
                          ng_u64 slots, uint32_t* rep, int* ctx_of, ng_i64 n, int* remap, ng_u64* counters,
                          void* stream);
/* the query index of pos[0..*n_dev) (compact ctx_of; n_max >= *n_dev sizes the grid) with no host sync: the table
 * is EMPTY-filled here, counters[1] / counters[2] added to as ng_query_index's, contexts not counted */
int ng_query_index_dev(const uint16_t* x, const int* avail, const int* pos, const ng_u64* n_dev, ng_i64 n_max, int k,
                       ng_u64* table, ng_u64 cap, ng_u64 slots, uint32_t* rep, int* ctx_of, ng_u64* counters,
                       void* stream);
/* the longest match's active list one level on: entries i < *n_dev of act whose context's hit bit is set get
 * length[act[i]] = k and, with avail >= k + 1, go to act_out (*n_out, *matched added to) */
int ng_act_next(const int* act, const ng_u64* n_dev, ng_i64 n_max, const int* ctx_of, const uint32_t* hit,
                const int* avail, int k, int* length, int* act_out, ng_u64* n_out, ng_u64* matched, void* stream);
/* the longest match's active list split at level k: entries i < *n_dev of act whose context's hit bit is set get
 * length[act[i]] = k (*matched added to); the others go to act_out (*n_out added to) */
int ng_act_split(const int* act, const ng_u64* n_dev, ng_i64 n_max, const int* ctx_of, const uint32_t* hit, int k,
                 int* length, int* act_out, ng_u64* n_out, ng_u64* matched, void* stream);
/* ng_scan_sink's list scan over the first *n_dev entries of plist (n_max >= *n_dev), with no host sync; region >=
 * ceil(n_max / (grid * 256)) * 256 */
int ng_scan_list_dev(const uint16_t* tok, int k, const ng_u64* plist, const ng_u64* n_dev, ng_i64 n_max,
                     const ng_u64* vt, ng_u64 vcap, const uint32_t* vrep, const uint16_t* x, uint32_t* hit, int what,
                     ng_u64* ev, ng_u64 region, uint32_t* ev_count, uint32_t* flags, int grid, ng_u64 key_add,
                     void* stream);
/* partitioned counting (no global atomics): offsets[s] = cnt[0] + ... + cnt[s - 1], s = 0..nseg */
int ng_seg_offsets(const uint32_t* cnt, ng_i64 nseg, ng_u64* offsets, void* stream);
/* segment s = cnt[s] items at src + (bases ? bases[s] : s * region) packed to dst + offsets[s]; values may be NULL */
int ng_seg_gather(const ng_u64* src_k, const uint32_t* src_v, ng_u64 region, const ng_i64* bases, const uint32_t* cnt,
                  ng_i64 nseg, const ng_u64* offsets, ng_u64* dst_k, uint32_t* dst_v, void* stream);
/* start[p], p = 0..2^pbits, of events sorted by their top pbits (pbits <= 24): msd 0 in key order; msd 1 grouped by
 * the top 8 bits first (ng_seg_scatter), then stably by the pbits - 8 bits below, partition (lo, hi) = lo << 8 | hi */
int ng_part_bounds(const ng_u64* ev, ng_i64 n, int pbits, int msd, ng_i64* start, void* stream);
/* a sort's first pass from segments: nseg segments of ev_count[s] keys at src + (bases ? bases[s] : s * R) scattered
 * by the nbits-bit digit (key >> shift) & (2^nbits - 1), nbits <= 11, to out at dpre (u32 [2^nbits * nseg], the
 * exclusive scan of the producer's digit histograms, digit-major: ng_scan_emit's with shift 56 and 8 bits,
 * ng_part_count's; fewer than 2^32 keys); the order within a digit is free. out holds cap keys: a key whose place is
 * cap or beyond is dropped, and a region segment (bases NULL) is read up to R keys, so the call may be made before the
 * host has read the totals */
int ng_seg_scatter(const ng_u64* src, ng_u64 R, const ng_i64* bases, const uint32_t* ev_count, const uint32_t* dpre,
                   ng_i64 nseg, int shift, int nbits, ng_u64* out, ng_u64 cap, void* stream);
/* ng_seg_scatter with the keys narrowed to their low 32 bits on the way out (u32 out[cap]); shift <= 32 */
int ng_seg_scatter_narrow(const ng_u64* src, ng_u64 R, const ng_i64* bases, const uint32_t* ev_count,
                          const uint32_t* dpre, ng_i64 nseg, int shift, int nbits, uint32_t* out, ng_u64 cap,
                          void* stream);
/* The 32-bit count (a level's events as 4-byte keys after the first pass; every present context's record made in
 * LDS without sorting its pairs): the second pass, most significant digit first. keys (at most cap of them, cap <
 * 2^32) grouped into nb = 2^nb_bits buckets (1 <= nb_bits <= 11; bucket b from dpre[b * nseg], the last up to *total,
 * a device-side count) sub-grouped within each bucket by the nbits-bit digit (key >> shift) & (2^nbits - 1)
 * (0 <= nbits <= 11) into out (cap keys); start (i64[2^(nb_bits + nbits) + 1]) the partitions' starts, partition
 * p = bucket << nbits | digit (nbits 0: the buckets' starts; keys and out unused). Two-phase temp storage (temp NULL:
 * *temp_bytes set). ng_msd_pass: u32 keys (the count's events); ng_msd_pass64: u64 keys (its packed words) */
int ng_msd_pass(void* temp, size_t* temp_bytes, const uint32_t* keys, const uint32_t* dpre, ng_i64 nseg, int nb_bits,
                const ng_u64* total, ng_u64 cap, int shift, int nbits, uint32_t* out, ng_i64* start, void* stream);
int ng_msd_pass64(void* temp, size_t* temp_bytes, const ng_u64* keys, const uint32_t* dpre, ng_i64 nseg, int nb_bits,
                  const ng_u64* total, ng_u64 cap, int shift, int nbits, ng_u64* out, ng_i64* start, void* stream);
/* ng_msd_pass over u64 keys written out as their low 32 bits (shift <= 32): the second pass of the 32-bit count for
 * pair keys wider than its first pass narrows (W > 42: the corpus-wide tables' context ids) */
int ng_msd_pass_narrow(void* temp, size_t* temp_bytes, const ng_u64* keys, const uint32_t* dpre, ng_i64 nseg,
                       int nb_bits, const ng_u64* total, ng_u64 cap, int shift, int nbits, uint32_t* out, ng_i64* start,
                       void* stream);
/* lookups of n query positions i = pos[j] (pos NULL: j) for the 32-bit count: qk[j] = kmix(ctx_of[i] << 16 | tgt[i],
 * W, M) << (64 - W) (M 0: W) for ids in [lo, hi) (hi <= 2^(W - 16)), else EMPTY; qv[j] = i; n_dev (may be NULL, pos
 * required): a device-side count of pos's entries, lookups j >= *n_dev EMPTY */
int ng_part_lookups_w(const int* ctx_of, const uint16_t* tgt, const int* pos, ng_i64 n, const ng_u64* n_dev, ng_i64 lo,
                      ng_i64 hi, int W, int M, ng_u64* qk, uint32_t* qv, void* stream);
/* the positions i < n with v[i] > 0, in order, into out (at most cap of them); *n_dev = how many (may exceed cap);
 * two-phase temp storage; no host read */
int ng_select_positive(void* temp, size_t* temp_bytes, const int* v, ng_i64 n, int* out, ng_i64 cap, ng_u64* n_dev,
                       void* stream);
/* the 32-bit count of ng_msd_pass's partitions (2^pbits of them, 1 <= W - pbits <= 31, W = context-id bits + 16;
 * events kmix(pair key, W, M), M 0: W) in LDS with `grid` blocks (<= 65536): block b's distinct pairs as packed
 * words pair key << (48 - cb) | min(count, esc), esc = 2^(48 - cb) - 1 (W - 16 <= cb <= 44; larger counts also in
 * the escape table), at out_k + seg_base[b], seg_cnt[b] of them; dhist[d * grid + b] its words per dbits-bit digit
 * (word >> dshift) & (2^dbits - 1), dbits <= 11; runs (may be NULL; dhist then unused): each partition's words
 * grouped by the digit (pair key >> gshift) & (2^gbits - 1) (gbits <= 6), group s of partition p = b << rbits | j
 * at out_k[lo, hi), lo | hi << 32 = runs[((b << gbits) + s) << rbits | j]; live_np (<= 2^pbits): the partitions
 * whose runs and slabs are written (the others hold no events and are never read); n_words (may be NULL): += the words written;
 * qcnt[qv[j]] = the count of lookup j (ng_part_lookups_w's sorted by their top pbits, bounds qstart); flags[0]
 * bit 0: a partition reached min(limit, 11000) distinct pairs (count again with a bit more), bit 1: the escape table
 * is full; slab (may be NULL): 2^pbits * 14336 u64, each partition's LDS table written out (slot = count << 32 |
 * key) for the corpus-wide tables' queries */
int ng_part_count32(const uint32_t* ev, const ng_i64* start, int pbits, int W, int M, const ng_u64* qk,
                    const uint32_t* qv, const ng_i64* qstart, ng_u64* out_k, int cb, ng_u64* esc_k, uint32_t* esc_c,
                    ng_u64 esc_cap, uint32_t* seg_cnt, ng_i64* seg_base, uint32_t* qcnt, uint32_t* dhist, int dshift,
                    int dbits, uint32_t limit, uint32_t* flags, int grid, ng_u64* slab, ng_u64* runs, int gbits,
                    int gshift, int rbits, ng_i64 live_np, ng_u64* n_words, void* stream);
/* per context id c < n_ids from ng_part_count32's words grouped by context into P partitions (start: i64[P + 1],
 * partition q = the ids [q << ibits, (q + 1) << ibits), ibits <= 11; ng_seg_scatter then ng_msd_pass64): dist[c] =
 * its pairs (0: absent) for every id (dist may be NULL), and for present contexts the record rec[c] of ng_ctx_summary's layout (topk 1,
 * 2, 4, 8; first-word index 0); flags[0] bit 2: a total reached 2^32; deep (may be NULL, deep_n then too): the ids
 * of the contexts of more than deep_min pairs, in no order (at most deep_cap kept, *deep_n counts all; zeroed by the
 * caller); present (may be NULL): *present += the present contexts; grid: blocks walking the partitions in turn (0:
 * one block per partition) */
int ng_ctx_agg(const ng_u64* w, const ng_i64* start, ng_i64 P, int ibits, int cb, ng_i64 n_ids, const ng_u64* esc_k,
               const uint32_t* esc_c, ng_u64 esc_cap, int topk, uint32_t* rec, uint32_t* dist, uint32_t* flags,
               uint32_t deep_min, ng_i64* deep, ng_u64 deep_cap, ng_u64* deep_n, ng_u64* present, int grid,
               void* stream);
/* ng_ctx_agg over ng_part_count32's words left in runs (gshift = 16 + ibits): group g < NG = 2^(d1 + gbits) (ids
 * [g << ibits, (g + 1) << ibits)) is run g & (2^gbits - 1) of partitions (g >> gbits) << d2 ... + 2^d2 - 1, bounds
 * at runs[g << d2 ...] as ng_part_count32 lays them out (d2 <= 8,
 * gbits <= 6, word indexes below 2^32); outputs as ng_ctx_agg's without the deep list */
int ng_ctx_agg_runs(const ng_u64* w, const ng_u64* runs, ng_i64 NG, int d2, int gbits, int ibits, int cb,
                    ng_i64 n_ids, const ng_u64* esc_k, const uint32_t* esc_c, ng_u64 esc_cap, int topk, uint32_t* rec,
                    uint32_t* dist, uint32_t* flags, ng_u64* present, int grid, void* stream);
/* n words of value v (the hosts' buffer fills, on the caller's stream) */
int ng_fill_u32(uint32_t* p, ng_i64 n, uint32_t v, void* stream);
int ng_fill_u64(ng_u64* p, ng_i64 n, ng_u64 v, void* stream);
/* exclusive prefix sum of n u32 (out may alias in), *total (may be NULL) the sum; CUB-style two-phase temp storage */
int ng_exclusive_scan_u32(void* temp, size_t* temp_bytes, const uint32_t* in, uint32_t* out, ng_i64 n,
                          ng_u64* total, void* stream);
/* lookups of n query positions i = pos[j] (pos NULL: j): qk[j] = mix64(ctx_of[i] << 16 | tgt[i]) for ids in
 * [lo, hi), else EMPTY; qv[j] = i */
int ng_part_lookups(const int* ctx_of, const uint16_t* tgt, const int* pos, ng_i64 n, ng_i64 lo, ng_i64 hi,
                    ng_u64* qk, uint32_t* qv, void* stream);
/* per partition an LDS hash count of its events; block b's distinct (pair key, count) at out + seg_base[b], seg_cnt[b]
 * of them; qcnt[qv[j]] = the count of lookup j (qk sorted like ev, bounds qstart); dhist (may be NULL, packed words
 * only): block b's words per dbits-bit digit (word >> dshift) & (2^dbits - 1), dbits <= 11, at dhist[d * grid + b];
 * flags[0] bit 0: a partition reached 7000 distinct pairs (repartition with one more bit) */
int ng_part_count(const ng_u64* ev, const ng_i64* start, int pbits, const ng_u64* qk, const uint32_t* qv,
                  const ng_i64* qstart, ng_u64* out_k, uint32_t* out_c, int cb, ng_u64* esc_k, uint32_t* esc_c,
                  ng_u64 esc_cap, uint32_t* seg_cnt, ng_i64* seg_base, uint32_t* qcnt, uint32_t* dhist, int dshift,
                  int dbits, uint32_t* flags, int grid, void* stream);
/* with cb > 0 (ids below 2^cb, cb <= 44) ng_part_count writes packed words pair key << (48 - cb) | min(count, esc),
 * esc = 2^(48 - cb) - 1, larger counts also into the escape table esc_k/esc_c (EMPTY-filled; full: flags[0] bit 1).
 * From such words sorted by context: dist[c] (pairs) and the record rec[c] of each present context (callers zero
 * dist): u32 words total, pairs, the first topk (1, 2, 4, 8) tokens by (count desc, token asc) two per word, their
 * counts (4, 8, 8, 16 words for topk 1, 2, 4, 8; for topk 2 and 8 also the index of the context's first word, u64
 * in the two words after the counts); dist may be NULL; with nstat (u32[257], zeroed) the number of contexts is
 * nstat[1] + ... + nstat[256] and with deep the contexts of more than deep_min pairs are appended to deep (nstat[0]
 * of them); flags[0] bit 2: a total reached 2^32 */
int ng_ctx_summary(const ng_u64* w, ng_i64 U, int cb, const ng_u64* esc_k, const uint32_t* esc_c, ng_u64 esc_cap,
                   int topk, uint32_t* rec, uint32_t* dist, uint32_t deep_min, ng_i64* deep, uint32_t* nstat,
                   uint32_t* flags, void* stream);
/* per query position from ng_ctx_summary's records and pair counts and the counted lookups qcnt (may be NULL: no
 * cnt): tot, dist, cnt (thr: the CNT_TOP threshold scores, may be NULL), the first kout of ktop top entries, mask bit
 * li (mask may be NULL); zeros where the context is absent or never occurred, positions of contexts outside [lo, hi)
 * left alone; hit_bits (may be NULL, lo 0): bit i where position i's context occurred (ceil(N / 64) * 2 u32) */
int ng_pos_summary(const int* ctx_of, ng_i64 N, ng_i64 lo, ng_i64 hi, const uint16_t* tgt, const uint32_t* rec,
                   const uint32_t* dist, const ng_u64* thr, const uint32_t* qcnt, int ktop, int kout, int li,
                   int* out_tot, int* out_dist, int* out_cnt, uint16_t* out_tok, uint32_t* out_tcnt, int* mask,
                   uint32_t* hit_bits, void* stream);
/* corpus-wide level build (count_table.rs build_level :491-631): contexts into ck (slot = id) and per corpus position
 * its event ev[p] = mix64(slot << 16 | next) (EMPTY: none), counted afterwards by the partitioned count; flags[0]
 * bit 1: context table full (rerun bigger) */
int ng_table_emit(const uint16_t* tok, ng_i64 L, int k, ng_u64* ck, ng_u64 ccap, ng_u64* ev, uint32_t* flags,
                  int grid, void* stream);
/* corpus-wide level build for the 32-bit count (count_table.rs build_level :491-631): contexts into ck (slot = id,
 * ccap <= 2^(W - 16)) and each position's event wmix(slot << 16 | next, W) appended to its block's region ev[b *
 * region ...] (region >= ceil(L / (grid * 256)) * 256), ev_count[b] and the top-dbits digit histogram dhist[d * grid
 * + b] (dbits <= 10); flags[0] bit 1: context table full (rerun bigger), bit 2: a region overflowed */
int ng_table_emit32(const uint16_t* tok, ng_i64 L, int k, ng_u64* ck, ng_u64 ccap, int W, int dbits, ng_u64* ev,
                    ng_u64 region, uint32_t* ev_count, uint32_t* dhist, uint32_t* flags, int grid, void* stream);
/* per key (EMPTY: none) its context-table slot or -1 */
int ng_table_lookup(const ng_u64* keys, ng_i64 n, const ng_u64* ck, ng_u64 ccap, int* slot, void* stream);
/* thr[c] = the kth largest pair score of each listed context (ids[m]; count_table.rs:146-158 deep_last) over packed
 * words sorted by pair key and ng_ctx_summary's topk-8 records */
int ng_ctx_kth(const ng_u64* w, int cb, const ng_u64* esc_k, const uint32_t* esc_c, ng_u64 esc_cap,
               const uint32_t* rec, const ng_i64* ids, ng_i64 m, int kth, ng_u64* thr, void* stream);
/* ng_ctx_kth over words grouped by context into partitions of 2^ibits ids (gstart: their starts; ng_ctx_agg's
 * input) for the first min(m, *m_dev) listed ids (m_dev may be NULL) */
int ng_ctx_kth_grouped(const ng_u64* w, const ng_i64* gstart, int ibits, int cb, const ng_u64* esc_k,
                       const uint32_t* esc_c, ng_u64 esc_cap, const ng_i64* ids, ng_i64 m, const ng_u64* m_dev, int kth,
                       ng_u64* thr, void* stream);
/* per query position (count_table.rs query_counts :291-331): tot, dist, cnt (CNT_TOP rule by thr, NULL: none) and
 * the first kout top entries of its level-k context, from the context table, the packed words sorted by pair key and
 * the topk-8 records */
int ng_table_query(const uint16_t* x, const int* avail, const uint16_t* tgt, ng_i64 n, int k, const ng_u64* ck,
                   ng_u64 ccap, const ng_u64* w, int cb, const ng_u64* esc_k, const uint32_t* esc_c, ng_u64 esc_cap,
                   const uint32_t* rec, const ng_u64* thr, uint32_t cnt_top, int kout, int* out_tot, int* out_dist,
                   int* out_cnt, uint16_t* out_tok, uint32_t* out_tcnt, void* stream);
/* ng_table_query over a level counted by the 32-bit count: cnt from its slabs (ng_part_count32's, 2^pbits
 * partitions of the W-bit pair hash) */
int ng_table_query32(const uint16_t* x, const int* avail, const uint16_t* tgt, ng_i64 n, int k, const ng_u64* ck,
                     ng_u64 ccap, const ng_u64* slabs, int pbits, int W, const uint32_t* rec, const ng_u64* thr,
                     uint32_t cnt_top, int kout, int* out_tot, int* out_dist, int* out_cnt, uint16_t* out_tok,
                     uint32_t* out_tcnt, void* stream);
/* hint rows over table levels (count_table.rs query_rows :338-404); desc[v * 3]: slot_of, records, bucket */
int ng_pos_rows(ng_i64 N, int nlv, const ng_i64* desc, int entries, short* cell, uint16_t* next, uint16_t* weights,
                signed char* level, void* stream);
/* online state (online.rs step rule), per level: a context table ck (slot = context id); a pair table pt of pcap
 * 16-byte slots (pt[2s] the key slot << 16 | next, EMPTY when free; the low half of pt[2s + 1] its count); a record
 * per context, rw u32 words: [0] total, [1] distinct next tokens, and with rw = 16 (levels with hint rows) [2, 10) the
 * top entries' counts and [10, 14) their tokens, two per word (count descending, then token ascending; count 0 ends
 * the list); rw = 2 without entries. Insert occurrences ending at pos[i] (rec may be NULL: then the sorted pass adds
 * the totals), their pair keys | tag into ev (tag: the level's index << tshift, above every pair key); merge a step's
 * sorted distinct touched pairs of every level at once (uk[0..*n) tagged keys, agg their occurrences in the step;
 * desc[t * 5]: level t's pair table, its capacity, records, 1 if rw = 16 else 0, flags) into their contexts'
 * records (add_counts: the pairs' counts grow by agg there, after inserts that did not count them); answer queries;
 * build hint rows */
int ng_online_insert(const uint16_t* tok, const int* pos, ng_i64 m, int k, ng_u64* ck, ng_u64 ccap, ng_u64* pt,
                     ng_u64 pcap, uint32_t* rec, int rw, ng_u64* ev, uint32_t* flags, ng_u64 tag, void* stream);
int ng_online_top(const ng_u64* uk, const ng_i64* n, ng_i64 m, const uint32_t* agg, const ng_i64* desc, int ntag,
                  int tshift, ng_u64* score, int E, int add_counts, void* stream);
/* a step's events ev[0..m) (unsorted, as ng_online_insert_levels writes them with count_pairs 0) merged as
 * sort_pairs + reduce_by_key + ng_online_top (add_counts 1) merge them, without the sort: the events scattered by the
 * low 11 bits of their context slot, then a block per bucket counts, sorts and merges its distinct pairs in LDS
 * (rounds split by a pair hash where a bucket holds more than 4096). desc, ntag, tshift, E: ng_online_top's.
 * CUB-style two-phase temp storage (temp NULL: *temp_bytes set). -1 where m >= 2^cb - 1 with cb = 64 - tshift -
 * (tag bits) + 11 (a pair's occurrences must fit the packed words' count bits): the sorted path then applies. No
 * counterpart in the reference (online.rs merges on the CPU). */
int ng_online_merge(void* temp, size_t* temp_bytes, const ng_u64* ev, ng_i64 m, const ng_i64* desc, int ntag,
                    int tshift, int E, void* stream);
int ng_online_query(const uint16_t* tok, const int* avail, const unsigned char* has_next, const int* pos, ng_i64 m,
                    int k, const ng_u64* ck, ng_u64 ccap, const ng_u64* pt, ng_u64 pcap, const uint32_t* rec, int rw,
                    int* qslot, uint32_t* tot, uint16_t* dist, uint32_t* cnt, int nc, int ci, void* stream);
/* the inserts / the queries of up to 8 levels of a step in one launch (a level's lookups are chains of dependent
 * table round trips; one launch pays that latency once for all levels). lv: a host array, 10 int64 per level for
 * inserts (pos, m, k, ck, ccap, pt, pcap, ev, flags, tag) and 13 per level for queries (k, ck, ccap, pt, pcap, rec,
 * rw, qslot, tot, dist, cnt, nc, ci), each as the single-level call's argument of that name (pointers as int64; the
 * inserts leave the records to ng_online_top / ng_online_merge, and with count_pairs 0 the pair counts too). -1 on a
 * bad level. */
int ng_online_insert_levels(const uint16_t* tok, int nlv, const ng_i64* lv, int count_pairs, void* stream);
int ng_online_query_levels(const uint16_t* tok, const int* avail, const unsigned char* has_next, const int* pos,
                           ng_i64 m, int nlv, const ng_i64* lv, void* stream);
/* hint rows of the queries at pos[0..m) in S slots, deepest levels first (desc[v * 3]: the level's qslot from
 * ng_online_query, its records (rw = 16), its bucket index): cell [n, S], next / weights [n, S, E], level [n, S] (int8
 * bucket index; may be NULL); empty slots are left as they are */
int ng_online_rows(const int* pos, ng_i64 m, int nlv, const ng_i64* desc, int E, int S, short* cell, uint16_t* next,
                   uint16_t* weights, signed char* level, int* hinted, void* stream);
/* counts/mix.py features: counts int32 [3, L, n] -> float32 tot, dist, min(cnt, tot) [n, L], int64 bin and sparse
 * indices [n, L] */
int ng_features(const int* counts, int L, ng_i64 n, int nb, float* tot, float* dist, float* cnt, ng_i64* bin,
                ng_i64* sparse, void* stream);
/* The hint directory's reader (old_records/hint_runtime.py Hints._upload :171-199, _upload_counts :201-217): a
 * batch's rows staged back to back (cell int16, tokens uint16, weights uint16) widened to int64 cell, int64 tokens and
 * float32 weights (u16 * float32(1 / 65535)); count rows tot (u32), dist (u16), cnt (u32) [n, L] to float32
 * [n, 3, L]. */
int ng_hint_widen(const short* staged, ng_i64 n_cell, ng_i64 n_tok, ng_i64 n_w, ng_i64* cell, ng_i64* tokens,
                  float* weights, void* stream);
int ng_count_rows(const uint32_t* tot, const uint16_t* dist, const uint32_t* cnt, ng_i64 n, int L, float* out,
                  void* stream);

/* Hint rows from ng_ctx_summary's top-8 records (CtxRecord<8>: 16 u32 words per context id, 16-byte aligned).
 * ng_variant_rows: one gpu_val_stats variant's rows int32 [N, 9] (cell, 4 x two tokens, 4 x two weights) -- the
 * output of old_records/gpu_val_stats.cu variant_rows :646-699 -- from desc int64 [nv, 4] = (mask bit, length bucket,
 * ctx_of int32 [N], records) per level of the variant, ascending; positions without a level are left as they are.
 * ng_record_rows: the record's rows (record_367_gpu_counts/track_1_short/counts/build.py:341-387): cells int32 [N],
 * entries int32 [N, 8] (16-byte aligned) from desc int64 [nr, 3] = (tot row int32 [N], ctx_of int32 [N], records)
 * of the ROW_LEVELS levels, ascending.
 * ng_batch_rows: a training batch's rows (build.py batch_rows :390-403): out int32 [n + 2 * capacity] = the n cells,
 * then `capacity` (position, entry) pairs of the non-zero entries of entries int32 [n, 8] (16-byte aligned) in
 * position order, padded with (i % n, 0); *total = the non-zero entries (only the first capacity are written: the
 * caller raises past it); work: ng_batch_rows_work(n) u32 of workspace. */
int ng_variant_rows(ng_i64 N, const int* mask, int nv, const ng_i64* desc, int* rows, void* stream);
int ng_record_rows(ng_i64 N, int nr, const ng_i64* desc, int* cells, int* entries, void* stream);
ng_i64 ng_batch_rows_work(ng_i64 n);
int ng_batch_rows(const int* cells, const int* entries, ng_i64 n, ng_i64 capacity, int* out, uint32_t* work,
                  ng_u64* total, void* stream);
/* No counterpart in the reference: ng_batch_rows for callers that cannot allocate (code under HIP graph capture, a
 * training step's tight loop, harnesses that forbid hipMalloc). Same outputs; the workspace is the library's own
 * device array of 65537 u32 (256 KB per GPU, held until the process ends), so n <= 67,108,864 positions (larger: -1,
 * nothing launched). Every call on one GPU shares that array: calls that overlap on one GPU race. Nothing is
 * allocated, freed or cleared inside. */
int ng_batch_rows_noalloc(const int* cells, const int* entries, ng_i64 n, ng_i64 capacity, int* out, ng_u64* total,
                          void* stream);

#ifdef __cplusplus
}
#endif
#endif /* NGRAM_AMD_H */
