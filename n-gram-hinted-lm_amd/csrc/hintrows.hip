// Hint rows from the engine's per-context records (ng_ctx_summary with top-8: total, pairs, the 8 first next tokens by
// (count desc, token asc) and their counts; CtxRecord<8>, 16 u32 words, one 64-byte line per context):
//   * ng_variant_rows: a gpu_val_stats variant's rows (old_records/gpu_val_stats.cu variant_rows :646-694 defines
//     the output; the rule is val_hints.deepest, src/retrieval_blog_post/val_hints.py:277-311, and old_records.py
//     _val_rows_range :102-124, _weights :70-73);
//   * ng_record_rows: the record's rows (record_367_gpu_counts/track_1_short/counts/build.py:341-387): per ROW_LEVELS
//     level the 8 candidates as token | weight << 16 (weight = the count, scaled to 15 bits as ceil(count * 32767 /
//     top) where the top count exceeds 32767), the deepest level with an occurrence chosen per position, and its cell;
//   * ng_batch_rows: a training batch's rows in the record's layout (build.py:390-403): the n cells, then `capacity`
//     (position, entry) pairs of the non-zero entries in position order, padded with (i % n, 0).
// One pass per position; every record read is one line. The float64 steps (share, weights) are the reference's
// definitions, evaluated in the same order.
#include <mutex>

#include "ngram_common.h"
#include "part.h"

namespace {

using Rec8 = CtxRecord<8>;
#define ROWS_MAX_LEVELS 16

struct Top8 {
    u32 total;
    u32 tok[8];
    u32 cnt[8];
};

__device__ __forceinline__ Top8 read_top8(const u32* __restrict__ rec, i64 c) {
    const uint4* r = (const uint4*)(rec + c * Rec8::WORDS);
    const uint4 a = r[0], t = make_uint4(a.z, a.w, r[1].x, r[1].y), c0 = make_uint4(r[1].z, r[1].w, r[2].x, r[2].y),
                c1 = make_uint4(r[2].z, r[2].w, r[3].x, r[3].y);
    Top8 o;
    o.total = a.x;
    const u32 tw[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) o.tok[2 * q] = tw[q] & 0xFFFFu, o.tok[2 * q + 1] = tw[q] >> 16;
    const u32 cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
    for (int q = 0; q < 8; ++q) o.cnt[q] = cw[q];
    return o;
}

// count bin: #{e in (2, 3, 5, 9, 17, 33) : e <= total}; the edges are 1 + 2^j, so it is the bit length of total - 1,
// capped at 6
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

// desc[v * 4 ..] = (mask bit, length bucket, ctx_of, rec) per level of the variant, levels ascending.
__global__ void __launch_bounds__(256) variant_rows_k(i64 N, const int* __restrict__ mask, int nv,
                                                      const i64* __restrict__ desc, int* __restrict__ rows) {
    __shared__ i64 d[ROWS_MAX_LEVELS * 4];
    for (int j = threadIdx.x; j < nv * 4; j += blockDim.x) d[j] = desc[j];
    __syncthreads();
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    const int m = mask[i];
    int v = -1;
    for (int q = 0; q < nv; ++q)
        if ((m >> d[q * 4]) & 1) v = q;
    if (v < 0) return;
    const i64 c = ((const int*)d[v * 4 + 2])[i];
    const Top8 t = read_top8((const u32*)d[v * 4 + 3], c);
    u64 sum = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) sum += t.cnt[r];
    const double denom = sum > 1 ? (double)sum : 1.0;
    const double share = (double)t.cnt[0] / (double)(t.total > 1 ? t.total : 1u);
    int* row = rows + i * 9;
    row[0] = ((1 + (int)d[v * 4 + 1]) * 7 + count_bin(t.total)) * 6 + purity_bin(share);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        row[1 + r] = (int)(t.tok[2 * r] | (t.tok[2 * r + 1] << 16));
        const u32 w0 = (u32)rint((double)t.cnt[2 * r] / denom * 65535.0);
        const u32 w1 = (u32)rint((double)t.cnt[2 * r + 1] / denom * 65535.0);
        row[5 + r] = (int)(w0 | (w1 << 16));
    }
}

// desc[r * 3 ..] = (tot row int32 [N] (uint32 bits), ctx_of, rec) per ROW_LEVELS level r, ascending.
__global__ void __launch_bounds__(256) record_rows_k(i64 N, int nr, const i64* __restrict__ desc,
                                                     int* __restrict__ cells, int* __restrict__ entries) {
    __shared__ i64 d[ROWS_MAX_LEVELS * 3];
    for (int j = threadIdx.x; j < nr * 3; j += blockDim.x) d[j] = desc[j];
    __syncthreads();
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i >= N) return;
    int depth = -1;
    u32 total = 0;
    for (int r = 0; r < nr; ++r) {
        const u32 t = (u32)((const int*)d[r * 3])[i];
        if (t) depth = r, total = t;
    }
    int ent[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int cell = 0;
    if (depth >= 0) {
        const i64 c = ((const int*)d[depth * 3 + 1])[i];
        const Top8 t = read_top8((const u32*)d[depth * 3 + 2], c);
        const u64 top = t.cnt[0] > 1 ? t.cnt[0] : 1;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const u64 n = t.cnt[r];
            const u64 w = top > 32767 ? (n * 32767 + top - 1) / top : n;
            ent[r] = n ? (int)(t.tok[r] | (u32)(w << 16)) : 0;
        }
        const u32 row_top = t.cnt[0] < 0x7FFFFFFFu ? t.cnt[0] : 0x7FFFFFFFu;
        const double share = (double)row_top / (double)(total > 1 ? total : 1u);
        cell = ((1 + depth) * 7 + count_bin(total)) * 6 + purity_bin(share);
    }
    cells[i] = cell;
    int4* e = (int4*)(entries + i * 8);
    e[0] = make_int4(ent[0], ent[1], ent[2], ent[3]);
    e[1] = make_int4(ent[4], ent[5], ent[6], ent[7]);
}

#define BR_TILE 1024  // positions per block of the batch rows

// Non-zero entries per tile of BR_TILE positions.
__global__ void __launch_bounds__(256) batch_count_k(const int* __restrict__ entries, i64 n, u32* __restrict__ work) {
    __shared__ u32 part[4];
    u32 c = 0;
    for (i64 i = (i64)blockIdx.x * BR_TILE + threadIdx.x; i < (i64)(blockIdx.x + 1) * BR_TILE && i < n; i += 256) {
        const int4* e = (const int4*)(entries + i * 8);
        const int4 a = e[0], b = e[1];
        c += (a.x != 0) + (a.y != 0) + (a.z != 0) + (a.w != 0) + (b.x != 0) + (b.y != 0) + (b.z != 0) + (b.w != 0);
    }
#pragma unroll
    for (int dd = WAVE / 2; dd > 0; dd >>= 1) c += (u32)__shfl_down((int)c, dd, WAVE);
    if (lane_id() == 0) part[threadIdx.x / WAVE] = c;
    __syncthreads();
    if (threadIdx.x == 0) work[blockIdx.x] = part[0] + part[1] + part[2] + part[3];
}

// The tiles' counts to exclusive offsets in place (one block; tiles <= a few thousand), the total into *total.
__global__ void __launch_bounds__(1024) batch_scan_k(u32* __restrict__ work, i64 tiles, u64* total) {
    __shared__ u32 wsum[16];
    __shared__ u32 carry;
    if (threadIdx.x == 0) carry = 0;
    __syncthreads();
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    for (i64 t0 = 0; t0 < tiles; t0 += 1024) {
        const i64 t = t0 + threadIdx.x;
        const u32 v = t < tiles ? work[t] : 0u;
        u32 incl = v;
#pragma unroll
        for (int dd = 1; dd < WAVE; dd <<= 1) {
            const u32 o = (u32)__shfl_up((int)incl, dd, WAVE);
            if (lane >= dd) incl += o;
        }
        if (lane == WAVE - 1) wsum[w] = incl;
        __syncthreads();
        u32 before = carry;
        for (int q = 0; q < w; ++q) before += wsum[q];
        if (t < tiles) work[t] = before + incl - v;
        __syncthreads();
        if (threadIdx.x == 1023) carry = before + incl;
        __syncthreads();
    }
    if (threadIdx.x == 0) *total = carry;
}

// The batch's rows: cells, then the entries at their offsets (those past `capacity` dropped: the host raises), and
// the padding (i % n, 0) after the last entry.
__global__ void __launch_bounds__(256) batch_write_k(const int* __restrict__ cells, const int* __restrict__ entries,
                                                     i64 n, i64 capacity, const u32* __restrict__ work,
                                                     int* __restrict__ out) {
    __shared__ u32 wsum[4];
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    const i64 base_pos = (i64)blockIdx.x * BR_TILE;
    u32 run = work[blockIdx.x];  // entries before this tile
    int* pairs = out + n;  // (position, entry) pairs: 4-byte aligned only (n may be odd)
    for (i64 i = base_pos + threadIdx.x; i - threadIdx.x < base_pos + BR_TILE && i - threadIdx.x < n; i += 256) {
        int ent[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        u32 c = 0;
        if (i < n && i < base_pos + BR_TILE) {
            out[i] = cells[i];
            const int4* e = (const int4*)(entries + i * 8);
            const int4 a = e[0], b = e[1];
            ent[0] = a.x, ent[1] = a.y, ent[2] = a.z, ent[3] = a.w, ent[4] = b.x, ent[5] = b.y, ent[6] = b.z,
            ent[7] = b.w;
#pragma unroll
            for (int r = 0; r < 8; ++r) c += ent[r] != 0;
        }
        u32 incl = c;
#pragma unroll
        for (int dd = 1; dd < WAVE; dd <<= 1) {
            const u32 o = (u32)__shfl_up((int)incl, dd, WAVE);
            if (lane >= dd) incl += o;
        }
        if (lane == WAVE - 1) wsum[w] = incl;
        __syncthreads();
        u64 at = run + incl - c;
        for (int q = 0; q < w; ++q) at += wsum[q];
        const u32 round = wsum[0] + wsum[1] + wsum[2] + wsum[3];
#pragma unroll
        for (int r = 0; r < 8; ++r)
            if (ent[r] != 0) {
                if ((i64)at < capacity) {
                    pairs[2 * at] = (int)i;
                    pairs[2 * at + 1] = ent[r];
                }
                ++at;
            }
        run += round;
        __syncthreads();
    }
}

// Padding: pairs [total, capacity) = (j % n, 0).
__global__ void __launch_bounds__(256) batch_pad_k(i64 n, i64 capacity, const u64* __restrict__ total,
                                                   int* __restrict__ out) {
    const u64 m = *total;
    int* pairs = out + n;
    for (i64 j = (i64)m + blockIdx.x * (i64)blockDim.x + threadIdx.x; j < capacity; j += (i64)gridDim.x * blockDim.x) {
        pairs[2 * j] = (int)(j % n);
        pairs[2 * j + 1] = 0;
    }
}

}  // namespace

// One gpu_val_stats variant's rows int32 [N, 9] (cell, 4 x two tokens, 4 x two weights) from per-level records:
// desc int64 [nv, 4] = (mask bit, length bucket, ctx_of (int32 [N]), records (CtxRecord<8> [ids, 16], 16-byte
// aligned)). Positions without a level are left as they are.
extern "C" int ng_variant_rows(i64 N, const int* mask, int nv, const i64* desc, int* rows, void* stream) {
    if (nv < 0 || nv > ROWS_MAX_LEVELS) return -1;
    if (N > 0 && nv > 0) variant_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, mask, nv, desc, rows);
    return (int)hipGetLastError();
}

// The record's rows: cells int32 [N] and entries int32 [N, 8] (16-byte aligned) from desc int64 [nr, 3] = (tot row
// int32 [N], ctx_of int32 [N], records CtxRecord<8>) of the ROW_LEVELS levels, ascending.
extern "C" int ng_record_rows(i64 N, int nr, const i64* desc, int* cells, int* entries, void* stream) {
    if (nr < 1 || nr > ROWS_MAX_LEVELS || ((uintptr_t)entries & 15)) return -1;
    if (N > 0) record_rows_k<<<grid_for(N, 256), 256, 0, (hipStream_t)stream>>>(N, nr, desc, cells, entries);
    return (int)hipGetLastError();
}

// Workspace u32 entries of ng_batch_rows for n positions.
extern "C" i64 ng_batch_rows_work(i64 n) { return (n + BR_TILE - 1) / BR_TILE + 1; }

static int launch_batch_rows(const int* cells, const int* entries, i64 n, i64 capacity, int* out, u32* work,
                             u64* total, hipStream_t st) {
    const i64 tiles = (n + BR_TILE - 1) / BR_TILE;
    batch_count_k<<<(int)tiles, 256, 0, st>>>(entries, n, work);
    batch_scan_k<<<1, 1024, 0, st>>>(work, tiles, total);
    batch_write_k<<<(int)tiles, 256, 0, st>>>(cells, entries, n, capacity, work, out);
    if (capacity > 0) {
        const int g = grid_for(capacity, 256);
        batch_pad_k<<<g < 1024 ? g : 1024, 256, 0, st>>>(n, capacity, total, out);
    }
    return (int)hipGetLastError();
}

// A batch's rows (int32 [n + 2 * capacity]): cells[0..n), then `capacity` (position, entry) pairs of the non-zero
// entries (entries int32 [n, 8], 16-byte aligned) in position order, padded with (i % n, 0); *total = the non-zero
// entries (those past capacity are not written: the caller raises). work: ng_batch_rows_work(n) u32. The tiles'
// offsets and the running offset are u32, so n is at most (2^32 - 1) / 8 (8 entries per position: no offset wraps).
#define BR_MAX_N (0xFFFFFFFFll / 8)
extern "C" int ng_batch_rows(const int* cells, const int* entries, i64 n, i64 capacity, int* out, u32* work,
                             u64* total, void* stream) {
    if (n <= 0 || n > BR_MAX_N || capacity < 0 || ((uintptr_t)entries & 15)) return -1;
    return launch_batch_rows(cells, entries, n, capacity, out, work, total, (hipStream_t)stream);
}

// ---------------------------------------------------------------------------------------------------------------
// ng_batch_rows without a workspace argument, for callers that cannot allocate (HIP graph capture, a training step's
// tight loop): the per-tile offsets live in `scratch`, a file-scope device array of NOALLOC_TILES + 1 u32 (256 KB),
// which each GPU holds until the process ends. Its address is looked up once per device (hipGetSymbolAddress, on the
// first call with that device current) and passed to the kernels. Every call on one GPU shares the array: calls that
// overlap on one GPU (other streams, other threads) race. Nothing is allocated, freed or cleared by a library call:
// the kernels write every entry they read.
// ---------------------------------------------------------------------------------------------------------------

#define NOALLOC_TILES 65536  // at most 65536 * 1024 positions per call
#define NOALLOC_DEVICES 64

static __device__ __align__(256) u32 scratch[NOALLOC_TILES + 1];

static u32* scratch_on_current_device(int& rc) {
    static std::mutex mu;
    static u32* at[NOALLOC_DEVICES] = {};
    int dev = -1;
    rc = (int)hipGetDevice(&dev);
    if (rc != 0) return nullptr;
    if (dev < 0 || dev >= NOALLOC_DEVICES) {
        rc = -1;
        return nullptr;
    }
    std::lock_guard<std::mutex> hold(mu);
    if (!at[dev]) {
        void* p = nullptr;
        rc = (int)hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != 0) return nullptr;
        at[dev] = (u32*)p;
    }
    return at[dev];
}

// ng_batch_rows' outputs (out, *total) for n <= NOALLOC_TILES * 1024 = 67,108,864 positions (larger n: -1, nothing
// launched), the workspace taken from the library's own device array; -1 for the arguments ng_batch_rows refuses.
extern "C" int ng_batch_rows_noalloc(const int* cells, const int* entries, i64 n, i64 capacity, int* out, u64* total,
                                     void* stream) {
    if (n <= 0 || capacity < 0 || ((uintptr_t)entries & 15)) return -1;
    if ((n + BR_TILE - 1) / BR_TILE > NOALLOC_TILES) return -1;
    int rc = 0;
    u32* work = scratch_on_current_device(rc);
    if (!work) return rc;
    return launch_batch_rows(cells, entries, n, capacity, out, work, total, (hipStream_t)stream);
}
