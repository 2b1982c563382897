// The seeded synthetic token streams of the benchmark configurations, generated on the GPU (the host's numpy
// generator, ngram_amd/data.py, makes the same bytes; the reference's data are FineWeb shards, so this has no
// counterpart there). A body token of stream `key` at position p is a pure function of (key, p):
//   h = SplitMix64 finalizer(key + (p + 1) * 2^64/phi), u = (h >> 11) * 2^-53 (exact in float64),
//   rank = #{cdf entries <= u} (numpy searchsorted side="right"), clamped to ncdf - 1, token = perm[rank].
// Then BOS at the documents' ends and the copies (dst, src, length) of the stream's plan, computed on the host.
#include "ngram_common.h"

#define GOLDEN 0x9E3779B97F4A7C15ull

__device__ __forceinline__ u16 draw(u64 key, i64 p, const double* __restrict__ cdf, int ncdf, const u16* __restrict__ perm) {
    const u64 h = mix64(key + (u64)(p + 1) * GOLDEN);
    const double u = (double)(h >> 11) * 0x1p-53;
    int lo = 0, hi = ncdf;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (cdf[mid] <= u) lo = mid + 1;
        else hi = mid;
    }
    return perm[lo < ncdf - 1 ? lo : ncdf - 1];
}

__global__ void gen_tokens_k(u16* __restrict__ out, i64 start, i64 n, u64 key, const double* __restrict__ cdf, int ncdf,
                             const u16* __restrict__ perm) {
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < n; i += (i64)gridDim.x * blockDim.x)
        out[i] = draw(key, start + i, cdf, ncdf, perm);
}

// out[i] = the draw of position start + i of stream `key`, i in [0, n)
extern "C" int gen_tokens(u16* out, i64 start, i64 n, u64 key, const double* cdf, int ncdf, const u16* perm,
                          void* stream) {
    if (n <= 0) return 0;
    if (ncdf < 1) return -1;
    int g = grid_for(n, 256);
    gen_tokens_k<<<g > 65536 ? 65536 : g, 256, 0, (hipStream_t)stream>>>(out, start, n, key, cdf, ncdf, perm);
    return (int)hipGetLastError();
}

__global__ void gen_set_k(u16* __restrict__ out, const i64* __restrict__ pos, i64 m, u16 value) {
    const i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x;
    if (i < m) out[pos[i]] = value;
}

// out[pos[i]] = value, i in [0, m)
extern "C" int gen_set(u16* out, const i64* pos, i64 m, int value, void* stream) {
    if (m > 0) gen_set_k<<<grid_for(m, 256), 256, 0, (hipStream_t)stream>>>(out, pos, m, (u16)value);
    return (int)hipGetLastError();
}

// A block per copy (dst, src, length) of copies [m, 3]: out[dst + j] = src_tokens[src + j] if src_tokens, else the
// draw of position src + j of stream `key` (a copy from this stream's pure draws; never a document end).
__global__ void gen_copies_k(u16* __restrict__ out, const i64* __restrict__ copies, i64 m, const u16* __restrict__ src_tokens,
                             u64 key, const double* __restrict__ cdf, int ncdf, const u16* __restrict__ perm) {
    for (i64 c = blockIdx.x; c < m; c += gridDim.x) {
        const i64 dst = copies[3 * c], src = copies[3 * c + 1], len = copies[3 * c + 2];
        for (i64 j = threadIdx.x; j < len; j += blockDim.x)
            out[dst + j] = src_tokens ? src_tokens[src + j] : draw(key, src + j, cdf, ncdf, perm);
    }
}

extern "C" int gen_copies(u16* out, const i64* copies, i64 m, const u16* src_tokens, u64 key, const double* cdf,
                          int ncdf, const u16* perm, void* stream) {
    if (m <= 0) return 0;
    if (!src_tokens && ncdf < 1) return -1;
    gen_copies_k<<<m < 65536 ? (int)m : 65536, 256, 0, (hipStream_t)stream>>>(out, copies, m, src_tokens, key, cdf, ncdf,
                                                                            perm);
    return (int)hipGetLastError();
}
