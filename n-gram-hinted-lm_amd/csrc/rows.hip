// The hint rows' consumer side (the hint directory read by a training process): one staged upload of a batch's rows
// widened on the GPU into the tensors the model reads. The reference stages cell, tokens and weights (int16 bits)
// in one pinned buffer, copies it, and widens with torch ops (old_records/hint_runtime.py:171-199): cell and tokens
// to int64 (tokens & 0xFFFF), weights to float32 = (u16) * (1 / 65535) (torch multiplies by the float32 reciprocal
// for a scalar divisor). Count rows (:201-217): tot (u32), dist (u16), cnt (u32) per (position, level) to float32
// [n, 3, L]; the reference converts them on the host, here the raw words are copied (10 bytes instead of 12 per
// (position, level)) and converted in the same pass that interleaves them.
// Both kernels are HBM streaming passes: 2 B read + 8 B (cell, tokens) or 4 B (weights) written per element; 10 B
// read + 12 B written per (position, level) of counts.
#include "ngram_common.h"

namespace {

constexpr float WEIGHT_SCALE = 1.0f / 65535.0f;  // the float32 reciprocal of WEIGHT_ONE

__global__ void __launch_bounds__(256) hint_widen_k(const short* __restrict__ staged, i64 n_cell, i64 n_tok, i64 n_w,
                                                    i64* __restrict__ cell, i64* __restrict__ tokens,
                                                    float* __restrict__ weights) {
    const i64 total = n_cell + n_tok + n_w;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < total; i += (i64)gridDim.x * blockDim.x) {
        const short v = staged[i];
        if (i < n_cell) cell[i] = (i64)v;  // the cell is a signed int16 (0: no hint)
        else if (i < n_cell + n_tok) tokens[i - n_cell] = (i64)(u16)v;
        else weights[i - n_cell - n_tok] = (float)(u16)v * WEIGHT_SCALE;
    }
}

__global__ void __launch_bounds__(256) count_rows_k(const u32* __restrict__ tot, const u16* __restrict__ dist,
                                                    const u32* __restrict__ cnt, i64 n, int L,
                                                    float* __restrict__ out) {
    const i64 total = n * L;
    for (i64 i = blockIdx.x * (i64)blockDim.x + threadIdx.x; i < total; i += (i64)gridDim.x * blockDim.x) {
        const i64 p = i / L;
        const int l = (int)(i - p * L);
        float* o = out + p * 3 * L + l;
        o[0] = (float)tot[i];  // round to nearest, as numpy's uint32 -> float32 assignment
        o[L] = (float)dist[i];
        o[2 * L] = (float)cnt[i];
    }
}

int grid_of(i64 n) {
    const int g = grid_for(n, 256);
    return g < 4096 ? g : 4096;
}

}  // namespace

// staged = cell (n_cell int16) | tokens (n_tok uint16) | weights (n_w uint16), back to back in one device buffer.
extern "C" int ng_hint_widen(const short* staged, i64 n_cell, i64 n_tok, i64 n_w, i64* cell, i64* tokens,
                             float* weights, void* stream) {
    if (n_cell < 0 || n_tok < 0 || n_w < 0) return -1;
    const i64 total = n_cell + n_tok + n_w;
    if (total > 0)
        hint_widen_k<<<grid_of(total), 256, 0, (hipStream_t)stream>>>(staged, n_cell, n_tok, n_w, cell, tokens,
                                                                        weights);
    return (int)hipGetLastError();
}

// tot, dist, cnt: [n, L] row-major; out: float32 [n, 3, L].
extern "C" int ng_count_rows(const u32* tot, const u16* dist, const u32* cnt, i64 n, int L, float* out, void* stream) {
    if (n < 0 || L < 1) return -1;
    if (n > 0) count_rows_k<<<grid_of(n * L), 256, 0, (hipStream_t)stream>>>(tot, dist, cnt, n, L, out);
    return (int)hipGetLastError();
}
