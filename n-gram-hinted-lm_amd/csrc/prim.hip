// Device-wide primitives: scans, stable LSD radix sort, reduce-by-key (see prim.h). Own kernels for gfx950: 256-thread
// workgroups (four wave64s), 4096-item tiles, LDS block scans and wave ballots for stable ranking.
#include "prim.h"

namespace prim {

static constexpr int BLOCK = 256;
static constexpr int ITEMS = 16;
static constexpr int TILE = BLOCK * ITEMS;
static constexpr int NWAVES = BLOCK / WAVE;

static inline size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }
static inline i64 ntiles_of(i64 n) { return (n + TILE - 1) / TILE; }

template <typename T>
struct Sum {
    __device__ static T id() { return (T)0; }
    __device__ static T op(T a, T b) { return a + b; }
};
struct MaxI64 {
    __device__ static i64 id() { return (i64)0x8000000000000000ll; }
    __device__ static i64 op(i64 a, i64 b) { return a > b ? a : b; }
};

template <typename T>
__device__ __forceinline__ T shfl_up_t(T v, int d) {
    if constexpr (sizeof(T) == 8) return (T)shfl_up_u64((u64)v, d);
    else return (T)__shfl_up((int)v, d, WAVE);
}

// Exclusive scan of one value per thread over the 256-thread block; *block_total receives the reduction.
template <typename T, typename Op>
__device__ __forceinline__ T block_exclusive(T v, T* block_total) {
    __shared__ T wave_tot[NWAVES];
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    T incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        T o = shfl_up_t(incl, d);
        if (lane >= d) incl = Op::op(o, incl);
    }
    if (lane == WAVE - 1) wave_tot[w] = incl;
    __syncthreads();
    T before = Op::id(), total = Op::id();
#pragma unroll
    for (int i = 0; i < NWAVES; ++i) {
        if (i < w) before = Op::op(before, wave_tot[i]);
        total = Op::op(total, wave_tot[i]);
    }
    __syncthreads();
    // exclusive within the wave
    T excl_w = shfl_up_t(incl, 1);
    if (lane == 0) excl_w = Op::id();
    if (block_total) *block_total = total;
    return Op::op(before, excl_w);
}

template <typename T, typename Op>
__global__ void __launch_bounds__(BLOCK) tile_reduce_k(const T* __restrict__ in, i64 n, T* __restrict__ partial) {
    const i64 base = (i64)blockIdx.x * TILE;
    T acc = Op::id();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const i64 i = base + (i64)j * BLOCK + threadIdx.x;
        if (i < n) acc = Op::op(acc, in[i]);
    }
    T total;
    block_exclusive<T, Op>(acc, &total);
    if (threadIdx.x == 0) partial[blockIdx.x] = total;
}

// Scan of one tile with the tile's exclusive prefix (prefix null: identity). The last tile writes the grand total.
template <typename T, typename Op, bool INCLUSIVE>
__global__ void __launch_bounds__(BLOCK) tile_scan_k(const T* in, T* out, i64 n, const T* __restrict__ prefix,
                                                      T* total) {
    __shared__ T s[TILE + TILE / 32];
    const i64 base = (i64)blockIdx.x * TILE;
    auto at = [](int i) { return i + (i >> 5); };  // padded index (fewer bank conflicts)
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int l = j * BLOCK + threadIdx.x;
        const i64 i = base + l;
        s[at(l)] = i < n ? in[i] : Op::id();
    }
    __syncthreads();
    T local[ITEMS];
    T run = Op::id();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        local[j] = s[at(threadIdx.x * ITEMS + j)];
        run = Op::op(run, local[j]);
    }
    T btot;
    T carry = block_exclusive<T, Op>(run, &btot);
    if (prefix) carry = Op::op(prefix[blockIdx.x], carry);
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        if (INCLUSIVE) {
            carry = Op::op(carry, local[j]);
            s[at(threadIdx.x * ITEMS + j)] = carry;
        } else {
            s[at(threadIdx.x * ITEMS + j)] = carry;
            carry = Op::op(carry, local[j]);
        }
    }
    if (total && blockIdx.x == gridDim.x - 1 && threadIdx.x == BLOCK - 1) *total = carry;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < ITEMS; ++j) {
        const int l = j * BLOCK + threadIdx.x;
        const i64 i = base + l;
        if (i < n) out[i] = s[at(l)];
    }
}

template <typename T>
static size_t scan_temp(i64 n) {
    size_t bytes = 0;
    i64 m = ntiles_of(n);
    while (m > 1) {
        bytes += align_up((size_t)m * sizeof(T));
        m = ntiles_of(m);
    }
    return bytes + 256;
}

template <typename T, typename Op, bool INCLUSIVE>
static int scan_impl(const T* in, T* out, i64 n, T* total, char* temp, hipStream_t st) {
    if (n <= 0) return 0;
    const i64 nt = ntiles_of(n);
    if (nt == 1) {
        tile_scan_k<T, Op, INCLUSIVE><<<1, BLOCK, 0, st>>>(in, out, n, nullptr, total);
        return (int)hipGetLastError();
    }
    T* partial = (T*)temp;
    temp += align_up((size_t)nt * sizeof(T));
    tile_reduce_k<T, Op><<<(unsigned)nt, BLOCK, 0, st>>>(in, n, partial);
    int e = scan_impl<T, Op, false>(partial, partial, nt, nullptr, temp, st);
    if (e) return e;
    tile_scan_k<T, Op, INCLUSIVE><<<(unsigned)nt, BLOCK, 0, st>>>(in, out, n, partial, total);
    return (int)hipGetLastError();
}

// The sum of n u32 as u64 (*total zeroed by the caller): one atomic per block (atomics on one address serialize, so
// the grid is kept small: SUM_WIDE_BLOCKS).
#define SUM_WIDE_BLOCKS 256
__global__ void __launch_bounds__(BLOCK) sum_wide_k(const u32* __restrict__ in, i64 n, u64* total) {
    __shared__ u64 part[BLOCK / WAVE];
    u64 s = 0;
    for (i64 i = blockIdx.x * (i64)BLOCK + threadIdx.x; i < n; i += (i64)gridDim.x * BLOCK) s += in[i];
#pragma unroll
    for (int d = WAVE / 2; d > 0; d >>= 1) s += __shfl_down(s, d, WAVE);
    if ((threadIdx.x & (WAVE - 1)) == 0) part[threadIdx.x / WAVE] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        u64 b = 0;
        for (int w = 0; w < BLOCK / WAVE; ++w) b += part[w];
        if (b) atomicAdd((unsigned long long*)total, (unsigned long long)b);
    }
}

int sum_u32(const u32* in, i64 n, u64* total, hipStream_t st) {
    if (n < 0) return -1;
    if (n == 0) return 0;
    const i64 g = (n + BLOCK - 1) / BLOCK;
    sum_wide_k<<<(unsigned)(g < SUM_WIDE_BLOCKS ? g : SUM_WIDE_BLOCKS), BLOCK, 0, st>>>(in, n, total);
    return (int)hipGetLastError();
}

size_t scan_u32_temp_bytes(i64 n) { return scan_temp<u32>(n) + 256; }

// The offsets are u32 (they wrap once the sum reaches 2^32); *total is the exact u64 sum, read before the scan (out
// may alias in), so a caller can refuse sums of 2^32 and more.
int exclusive_scan_u32(const u32* in, u32* out, i64 n, u64* total, void* temp, hipStream_t st) {
    if (n < 0) return -1;
    if (total) {
        const int e = fill_u64(total, 0ull, 1, st);
        if (e) return e;
    }
    if (n == 0) return 0;
    if (total) {
        const i64 g = (n + BLOCK - 1) / BLOCK;
        sum_wide_k<<<(unsigned)(g < SUM_WIDE_BLOCKS ? g : SUM_WIDE_BLOCKS), BLOCK, 0, st>>>(in, n, total);
    }
    return scan_impl<u32, Sum<u32>, false>(in, out, n, nullptr, (char*)temp + 256, st);
}

size_t scan_u64_temp_bytes(i64 n) { return scan_temp<u64>(n); }

int exclusive_scan_u64(const u64* in, u64* out, i64 n, u64* total, void* temp, hipStream_t st) {
    if (n < 0) return -1;
    if (n == 0) {
        if (total) return fill_u64(total, 0ull, 1, st);
        return 0;
    }
    return scan_impl<u64, Sum<u64>, false>(in, out, n, total, (char*)temp, st);
}

size_t max_i64_temp_bytes(i64 n) { return scan_temp<i64>(n); }

int inclusive_max_i64(const i64* in, i64* out, i64 n, void* temp, hipStream_t st) {
    if (n < 0) return -1;
    return scan_impl<i64, MaxI64, true>(in, out, n, nullptr, (char*)temp, st);
}

// ---------------------------------------------------------------------------------------------------------------
// Radix sort
// ---------------------------------------------------------------------------------------------------------------

// Radix passes use their own tiles: 1024 threads x 8 items (8192 items), measured on MI355X at 3.6 TB/s for a
// keys-only scatter pass and 2.7 TB/s with values, against 2.9 and 1.9 for 256 x 16 (longer per-digit runs, fewer
// blocks).
static constexpr int RS_BLOCK = 1024;
static constexpr int RS_ITEMS = 8;
static constexpr int RS_TILE = RS_BLOCK * RS_ITEMS;
static constexpr int RS_NW = RS_BLOCK / WAVE;
static inline i64 rs_ntiles(i64 n) { return (n + RS_TILE - 1) / RS_TILE; }

// Exclusive scan of one value per thread over the 1024-thread block (a wave scan, then the 16 wave totals).
__device__ __forceinline__ u32 rs_block_exclusive(u32 v, u32* wt) {
    const int lane = lane_id(), w = threadIdx.x / WAVE;
    u32 incl = v;
#pragma unroll
    for (int d = 1; d < WAVE; d <<= 1) {
        const u32 o = (u32)__shfl_up((int)incl, d, WAVE);
        if (lane >= d) incl += o;
    }
    if (lane == WAVE - 1) wt[w] = incl;
    __syncthreads();
    u32 before = 0;
#pragma unroll
    for (int i = 0; i < RS_NW; ++i)
        if (i < w) before += wt[i];
    __syncthreads();
    return before + incl - v;
}

// Per tile its digit counts, hist[digit * ntiles + tile] (one LDS histogram per wave, summed at the end).
__global__ void __launch_bounds__(RS_BLOCK) rs_hist_k(const u64* __restrict__ keys, i64 n, int shift, u32 mask,
                                                      u32* __restrict__ hist, i64 ntiles) {
    __shared__ u32 h[RS_NW * 256];
    for (int i = threadIdx.x; i < RS_NW * 256; i += RS_BLOCK) h[i] = 0;
    __syncthreads();
    u32* hw = h + (threadIdx.x / WAVE) * 256;
    const i64 base = (i64)blockIdx.x * RS_TILE;
    u64 k[RS_ITEMS];
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        const i64 i = base + (i64)j * RS_BLOCK + threadIdx.x;
        k[j] = i < n ? keys[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        const i64 i = base + (i64)j * RS_BLOCK + threadIdx.x;
        if (i < n) atomicAdd(&hw[(u32)(k[j] >> shift) & mask], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 256) {
        u32 sum = 0;
#pragma unroll
        for (int w = 0; w < RS_NW; ++w) sum += h[w * 256 + threadIdx.x];
        hist[(i64)threadIdx.x * ntiles + blockIdx.x] = sum;
    }
}

// Stable scatter of one tile: items in tile order (row j, thread t) = index j * 1024 + t; per row, each wave ranks its
// lanes by digit with eight ballots; the per-(row, wave, digit) counts (u16) are scanned in LDS in tile order, giving
// each item its place in the tile sorted by digit. The tile is then staged in LDS in that order (aliasing the counts)
// and written out by consecutive threads, so each digit's run of the tile leaves as contiguous, coalesced stores.
// RAW: hist holds the per-tile counts themselves (not their exclusive scan); the block then finds its own bases (each
// digit's total over all tiles, scanned over the digits, plus its count in the tiles before this one), which saves the
// scan's launches when there are few tiles (RS_RAW_TILES at most: a few thousand counts read per block).
static constexpr i64 RS_RAW_TILES = 256;
template <bool VALUES, bool RAW = false>
__global__ void __launch_bounds__(RS_BLOCK) rs_scatter_k(const u64* __restrict__ kin, const u32* __restrict__ vin,
                                                         u64* __restrict__ kout, u32* __restrict__ vout, i64 n,
                                                         int shift, int nbits, const u32* __restrict__ hist,
                                                         i64 ntiles) {
    constexpr int CNT_BYTES = RS_ITEMS * RS_NW * 256 * 2;
    constexpr int STAGE_BYTES = RS_TILE * (VALUES ? 12 : 8);
    constexpr int SMEM_U64 = (CNT_BYTES > STAGE_BYTES ? CNT_BYTES : STAGE_BYTES) / 8;
    __shared__ u64 smem[SMEM_U64];
    __shared__ u32 gbase[256];
    __shared__ u32 tile_off[256];
    __shared__ u32 wt[RS_NW];
    u16* cnt = (u16*)smem;  // [RS_ITEMS][RS_NW][256]
    u64* stage_k = smem;
    u32* stage_v = (u32*)(smem + RS_TILE);
    const int t = threadIdx.x, w = t / WAVE;
    const u32 mask = (1u << nbits) - 1u;
    if constexpr (RAW) {
        u32 before = 0, total = 0;  // thread t < 256 = digit t
        if (t < 256)
            for (i64 b = 0; b < ntiles; ++b) {
                const u32 c = hist[(i64)t * ntiles + b];
                before += b < (i64)blockIdx.x ? c : 0u;
                total += c;
            }
        const u32 dbase = rs_block_exclusive(t < 256 ? total : 0u, wt);
        if (t < 256) gbase[t] = dbase + before;
    } else {
        if (t < 256) gbase[t] = hist[(i64)t * ntiles + blockIdx.x];
    }
    for (int i = t; i < CNT_BYTES / 4; i += RS_BLOCK) ((u32*)smem)[i] = 0;
    __syncthreads();
    const i64 base = (i64)blockIdx.x * RS_TILE;
    const int tile_n = (int)(n - base < RS_TILE ? n - base : RS_TILE);
    u64 key[RS_ITEMS];
    u32 val[RS_ITEMS];
    u32 dr[RS_ITEMS];  // digit | rank << 16 ; rank 0xFFFF = invalid
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        const i64 i = base + (i64)j * RS_BLOCK + t;
        const bool valid = i < n;
        key[j] = valid ? kin[i] : 0;
        if (VALUES) val[j] = valid ? vin[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        const bool valid = base + (i64)j * RS_BLOCK + t < n;
        const u32 d = (u32)(key[j] >> shift) & mask;
        u64 peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            if (b < nbits) {
                const bool bit = (d >> b) & 1u;
                const u64 bal = __ballot(bit);
                peers &= bit ? bal : ~bal;
            }
        }
        const u32 rank = (u32)__popcll(peers & lanemask_lt());
        if (valid && rank == 0) cnt[(j * RS_NW + w) * 256 + d] = (u16)__popcll(peers);
        dr[j] = valid ? (d | (rank << 16)) : 0xFFFF0000u;
    }
    __syncthreads();
    u32 run = 0;  // thread t < 256 = digit t: its items' exclusive offsets in (row, wave) order, and its tile total
    if (t < 256) {
        for (int j = 0; j < RS_ITEMS; ++j)
#pragma unroll
            for (int ww = 0; ww < RS_NW; ++ww) {
                u16* c = &cnt[(j * RS_NW + ww) * 256 + t];
                const u32 v = *c;
                *c = (u16)run;
                run += v;
            }
    }
    const u32 off = rs_block_exclusive(run, wt);
    if (t < 256) tile_off[t] = off;
    __syncthreads();
    u32 local[RS_ITEMS];
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        const u32 d = dr[j] & 0xFFFFu;
        local[j] = (dr[j] >> 16) == 0xFFFFu ? 0xFFFFFFFFu : tile_off[d] + cnt[(j * RS_NW + w) * 256 + d] + (dr[j] >> 16);
    }
    __syncthreads();  // the counts are read: the staging area may overwrite them
#pragma unroll
    for (int j = 0; j < RS_ITEMS; ++j) {
        if (local[j] == 0xFFFFFFFFu) continue;
        stage_k[local[j]] = key[j];
        if (VALUES) stage_v[local[j]] = val[j];
    }
    __syncthreads();
    for (int i = t; i < tile_n; i += RS_BLOCK) {
        const u64 k = stage_k[i];
        const u32 d = (u32)(k >> shift) & mask;
        const u32 pos = gbase[d] + (u32)i - tile_off[d];
        kout[pos] = k;
        if (VALUES) vout[pos] = stage_v[i];
    }
}

__global__ void copy_pairs_k(const u64* kin, u64* kout, const u32* vin, u32* vout, i64 n) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) {
        kout[i] = kin[i];
        if (vin) vout[i] = vin[i];
    }
}

size_t radix_sort_temp_bytes(i64 n, bool with_values) {
    if (n <= 0) return 256;
    const i64 nt = rs_ntiles(n);
    size_t b = align_up((size_t)n * 8);
    if (with_values) b += align_up((size_t)n * 4);
    b += align_up((size_t)nt * 256 * 4);
    b += scan_u32_temp_bytes(nt * 256);
    return b;
}

int radix_sort_pairs(const u64* kin, u64* kout, const u32* vin, u32* vout, i64 n, int begin_bit, int end_bit,
                     void* temp, size_t temp_bytes, hipStream_t st) {
    if (n < 0 || begin_bit < 0 || end_bit > 64 || begin_bit > end_bit) return -1;
    if (n == 0) return 0;
    if ((n >> 32) != 0) return -1;  // offsets are 32-bit
    const bool values = vin != nullptr && vout != nullptr;
    if (kin == kout) return -1;
    if (temp_bytes < radix_sort_temp_bytes(n, values)) return -1;
    if (begin_bit == end_bit) {
        copy_pairs_k<<<grid_for(n, 256) > 4096 ? 4096 : grid_for(n, 256), 256, 0, st>>>(kin, kout, values ? vin : nullptr,
                                                                                     vout, n);
        return (int)hipGetLastError();
    }
    const i64 nt = rs_ntiles(n);
    char* t = (char*)temp;
    u64* tk = (u64*)t;
    t += align_up((size_t)n * 8);
    u32* tv = nullptr;
    if (values) {
        tv = (u32*)t;
        t += align_up((size_t)n * 4);
    }
    u32* hist = (u32*)t;
    t += align_up((size_t)nt * 256 * 4);
    void* stemp = t;
    const int passes = (end_bit - begin_bit + 7) / 8;
    const u64* sk = kin;
    const u32* sv = vin;
    for (int p = 0; p < passes; ++p) {
        const int shift = begin_bit + 8 * p;
        const int nb = end_bit - shift < 8 ? end_bit - shift : 8;
        const bool to_out = ((passes - 1 - p) % 2) == 0;
        u64* dk = to_out ? kout : tk;
        u32* dv = to_out ? vout : tv;
        rs_hist_k<<<(unsigned)nt, RS_BLOCK, 0, st>>>(sk, n, shift, (1u << nb) - 1u, hist, nt);
        int e = 0;
        if (nt <= RS_RAW_TILES) {  // few tiles: each scatter block scans the counts itself
            if (values)
                rs_scatter_k<true, true><<<(unsigned)nt, RS_BLOCK, 0, st>>>(sk, sv, dk, dv, n, shift, nb, hist, nt);
            else
                rs_scatter_k<false, true><<<(unsigned)nt, RS_BLOCK, 0, st>>>(sk, nullptr, dk, nullptr, n, shift, nb, hist,
                                                                           nt);
        } else {
            e = exclusive_scan_u32(hist, hist, nt * 256, nullptr, stemp, st);
            if (e) return e;
            if (values)
                rs_scatter_k<true><<<(unsigned)nt, RS_BLOCK, 0, st>>>(sk, sv, dk, dv, n, shift, nb, hist, nt);
            else
                rs_scatter_k<false><<<(unsigned)nt, RS_BLOCK, 0, st>>>(sk, nullptr, dk, nullptr, n, shift, nb, hist, nt);
        }
        e = (int)hipGetLastError();
        if (e) return e;
        sk = dk;
        sv = dv;
    }
    return 0;
}

// ---------------------------------------------------------------------------------------------------------------
// Reduce by key
// ---------------------------------------------------------------------------------------------------------------

__global__ void rbk_heads_k(const u64* __restrict__ k, i64 n, u32* __restrict__ heads) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x)
        heads[i] = (i == 0 || k[i] != k[i - 1]) ? 1u : 0u;
}

// heads scanned (exclusive) -> run of item i = excl[i] + head[i] - 1
__global__ void rbk_keys_k(const u64* __restrict__ k, i64 n, const u32* __restrict__ excl, u64* __restrict__ kout) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x)
        if (i == 0 || k[i] != k[i - 1]) kout[excl[i]] = k[i];
}

// Each thread sums 16 consecutive items run by run: runs wholly inside its chunk are stored, runs crossing a chunk
// edge are added atomically (vout zeroed first).
__global__ void rbk_values_k(const u64* __restrict__ k, const u32* __restrict__ v, i64 n, const u32* __restrict__ excl,
                             u32* __restrict__ vout) {
    const i64 chunks = (n + 15) / 16;
    for (i64 c = blockIdx.x * (i64)blockDim.x + threadIdx.x; c < chunks; c += (i64)gridDim.x * blockDim.x) {
        const i64 a = c * 16, b = a + 16 < n ? a + 16 : n;
        i64 i = a;
        while (i < b) {
            const u64 key = k[i];
            const bool starts_here = i == 0 || k[i - 1] != key;
            u32 s = 0;
            i64 j = i;
            while (j < b && k[j] == key) s += v[j++];
            const bool ends_here = j == n || k[j] != key;
            const u32 r = starts_here ? excl[i] : excl[i] - 1u;
            if (starts_here && ends_here) vout[r] = s;
            else atomicAdd(&vout[r], s);
            i = j;
        }
    }
}

// Counting mode (no values: each item counts 1): a run's head records where the run starts, then each run's length is
// the distance to the next run's start. Both passes are coalesced and atomic-free.
__global__ void rbk_starts_k(const u64* __restrict__ k, i64 n, const u32* __restrict__ excl, u64* __restrict__ kout,
                             u32* __restrict__ starts) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x)
        if (i == 0 || k[i] != k[i - 1]) {
            kout[excl[i]] = k[i];
            starts[excl[i]] = (u32)i;
        }
}

__global__ void rbk_lengths_k(const u32* __restrict__ starts, const u64* __restrict__ total, i64 n,
                              u32* __restrict__ vout) {
    const i64 runs = (i64)*total;
    for (i64 r = blockIdx.x * (i64)blockDim.x + threadIdx.x; r < runs; r += (i64)gridDim.x * blockDim.x)
        vout[r] = (r + 1 < runs ? starts[r + 1] : (u32)n) - starts[r];
}

__global__ void rbk_nruns_k(const u64* total, i64* nruns) { *nruns = (i64)*total; }

__global__ void fill_u64_k(u64* p, u64 v, i64 n) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) p[i] = v;
}
__global__ void fill_u32_k(u32* p, u32 v, i64 n) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x) p[i] = v;
}

int fill_u64(u64* p, u64 v, i64 n, hipStream_t st) {
    if (n <= 0) return 0;
    int g = grid_for(n, 256);
    fill_u64_k<<<g > 8192 ? 8192 : g, 256, 0, st>>>(p, v, n);
    return (int)hipGetLastError();
}
int fill_u32(u32* p, u32 v, i64 n, hipStream_t st) {
    if (n <= 0) return 0;
    int g = grid_for(n, 256);
    fill_u32_k<<<g > 8192 ? 8192 : g, 256, 0, st>>>(p, v, n);
    return (int)hipGetLastError();
}

size_t reduce_by_key_temp_bytes(i64 n) {
    if (n <= 0) return 512;
    return 2 * align_up((size_t)n * 4) + 256 + scan_u32_temp_bytes(n);
}

int reduce_by_key(const u64* kin, u64* kout, const u32* vin, u32* vout, i64* nruns, i64 n, void* temp,
                  hipStream_t st) {
    if (n < 0) return -1;
    if (n == 0) return fill_u64((u64*)nruns, 0ull, 1, st);
    if ((n >> 32) != 0) return -1;
    char* t = (char*)temp;
    u32* heads = (u32*)t;
    t += align_up((size_t)n * 4);
    u32* starts = (u32*)t;
    t += align_up((size_t)n * 4);
    u64* total = (u64*)t;
    t += 256;
    int g = grid_for(n, 256);
    if (g > 8192) g = 8192;
    rbk_heads_k<<<g, 256, 0, st>>>(kin, n, heads);
    int e = exclusive_scan_u32(heads, heads, n, total, t, st);
    if (e) return e;
    if (!vin) {  // counting: the runs' lengths
        rbk_starts_k<<<g, 256, 0, st>>>(kin, n, heads, kout, starts);
        rbk_lengths_k<<<g, 256, 0, st>>>(starts, total, n, vout);
        rbk_nruns_k<<<1, 1, 0, st>>>(total, nruns);
        return (int)hipGetLastError();
    }
    rbk_keys_k<<<g, 256, 0, st>>>(kin, n, heads, kout);
    e = fill_u32(vout, 0u, n, st);
    if (e) return e;
    int g2 = grid_for((n + 15) / 16, 256);
    rbk_values_k<<<g2 > 8192 ? 8192 : g2, 256, 0, st>>>(kin, vin, n, heads, vout);
    rbk_nruns_k<<<1, 1, 0, st>>>(total, nruns);
    return (int)hipGetLastError();
}

}  // namespace prim
