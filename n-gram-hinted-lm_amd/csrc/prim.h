// Device-wide primitives (own kernels, gfx950 wave64): scans, a stable LSD radix sort of (u64 key, u32 value) pairs,
// reduce-by-key. All take a caller-provided temp buffer (sized by the *_temp_bytes functions) and a stream; none
// allocates. They return a hipError_t value (0 = success) or -1 for bad arguments.
#pragma once
#include "ngram_common.h"

namespace prim {

// exclusive prefix sum of u32 (out may alias in); *total (device, may be null) receives the sum (u64)
size_t scan_u32_temp_bytes(i64 n);
int exclusive_scan_u32(const u32* in, u32* out, i64 n, u64* total, void* temp, hipStream_t st);

// exclusive prefix sum of u64 (out may alias in)
size_t scan_u64_temp_bytes(i64 n);
int exclusive_scan_u64(const u64* in, u64* out, i64 n, u64* total, void* temp, hipStream_t st);

// inclusive running maximum of i64 (out may alias in)
size_t max_i64_temp_bytes(i64 n);
int inclusive_max_i64(const i64* in, i64* out, i64 n, void* temp, hipStream_t st);

// stable LSD radix sort of (key, value) pairs by key bits [begin_bit, end_bit); vin/vout may be null (keys only)
size_t radix_sort_temp_bytes(i64 n, bool with_values);
int radix_sort_pairs(const u64* kin, u64* kout, const u32* vin, u32* vout, i64 n, int begin_bit, int end_bit,
                     void* temp, size_t temp_bytes, hipStream_t st);

// consecutive equal keys -> one run: kout[r] = the key, vout[r] = the sum of its values (u32, wrapping), *nruns
size_t reduce_by_key_temp_bytes(i64 n);
int reduce_by_key(const u64* kin, u64* kout, const u32* vin, u32* vout, i64* nruns, i64 n, void* temp,
                  hipStream_t st);

// *total += the sum of n u32 (a small grid: one atomic per block)
int sum_u32(const u32* in, i64 n, u64* total, hipStream_t st);

// fill helpers
int fill_u64(u64* p, u64 v, i64 n, hipStream_t st);
int fill_u32(u32* p, u32 v, i64 n, hipStream_t st);

}  // namespace prim
