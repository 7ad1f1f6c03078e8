// The t5-encode stage's own kernels on gfx950: the embedding-row gather and the relative-position
// bias table. Both are pure data movement (HBM-bound); the encoder's GEMMs, RMSNorm, attention and
// gated GELU run on the shared kernels.
#include "common.h"

#include <cmath>

namespace bh {
namespace {

// A row id read as the reference reads it ((int64)id, truncation toward zero), valid when it
// names a row of the table; NaN and out-of-range values are not.
__device__ __forceinline__ bool row_ok(float f, int64_t table_rows, int64_t* id) {
    const double v = static_cast<double>(f);
    if (!(v > -1.0 && v < static_cast<double>(table_rows))) return false;
    *id = static_cast<int64_t>(f);
    return true;
}

// out[r, :] = table[ids[r], :], one 16-byte chunk per thread (E elements); an invalid id writes
// a NaN row.
template <typename T, int E>
__global__ void __launch_bounds__(256) k_gather_vec(const T* __restrict__ table,
                                                    const float* __restrict__ ids,
                                                    T* __restrict__ out, int64_t rows, int64_t cols,
                                                    int64_t table_rows) {
    const int64_t per_row = cols / E, n = rows * per_row;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = i / per_row, c = (i - r * per_row) * E;
        int64_t id = 0;
        uint4 v;
        if (row_ok(ids[r], table_rows, &id)) {
            v = *reinterpret_cast<const uint4*>(table + id * cols + c);
        } else if constexpr (sizeof(T) == 2) {
            v = make_uint4(0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u, 0x7fc07fc0u);
        } else {
            v = make_uint4(0x7fc00000u, 0x7fc00000u, 0x7fc00000u, 0x7fc00000u);
        }
        *reinterpret_cast<uint4*>(out + r * cols + c) = v;
    }
}

template <typename T>
__global__ void __launch_bounds__(256) k_gather(const T* __restrict__ table,
                                                const float* __restrict__ ids, T* __restrict__ out,
                                                int64_t rows, int64_t cols, int64_t table_rows) {
    const int64_t n = rows * cols;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = i / cols, c = i - r * cols;
        int64_t id = 0;
        if (row_ok(ids[r], table_rows, &id)) {
            out[i] = table[id * cols + c];
        } else {
            if constexpr (sizeof(T) == 2) {
                out[i] = static_cast<T>(0x7fc0);
            } else {
                out[i] = __builtin_bit_cast(T, 0x7fc00000u);
            }
        }
    }
}

// bias[h, q, k] = rel[bucket[k - q + S - 1], h]: rel is [buckets, heads] (the checkpoint layout),
// bucket holds the 2S-1 relative positions' buckets. 8 keys per thread, one 16-byte store.
__global__ void __launch_bounds__(256) k_rel_bias(const bf16_t* __restrict__ rel,
                                                  const int* __restrict__ bucket,
                                                  bf16_t* __restrict__ bias, int64_t heads,
                                                  int64_t S) {
    const int64_t per_row = (S + 7) / 8, n = heads * S * per_row;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = i / per_row, k0 = (i - row * per_row) * 8;
        const int64_t h = row / S, q = row - h * S;
        bf16_t* dst = bias + row * S + k0;
        for (int e = 0; e < 8 && k0 + e < S; ++e)
            dst[e] = rel[static_cast<int64_t>(bucket[k0 + e - q + S - 1]) * heads + h];
    }
}

int grid_of(int64_t n) {
    const int64_t g = (n + 255) / 256;
    return static_cast<int>(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

void launch_gather(const void* table, const float* ids, void* out, int64_t rows, int64_t cols,
                   int64_t table_rows, bool f32, hipStream_t s) {
    if (rows == 0 || cols == 0) return;
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * rows * cols * (f32 ? 4 : 2));
    const bool vec = aligned16(table) && aligned16(out) && cols % (f32 ? 4 : 8) == 0;
    if (f32) {
        const auto* t = static_cast<const float*>(table);
        auto* o = static_cast<float*>(out);
        if (vec) k_gather_vec<float, 4><<<grid_of(rows * cols / 4), 256, 0, s>>>(t, ids, o, rows, cols, table_rows);
        else k_gather<float><<<grid_of(rows * cols), 256, 0, s>>>(t, ids, o, rows, cols, table_rows);
    } else {
        const auto* t = static_cast<const bf16_t*>(table);
        auto* o = static_cast<bf16_t*>(out);
        if (vec) k_gather_vec<bf16_t, 8><<<grid_of(rows * cols / 8), 256, 0, s>>>(t, ids, o, rows, cols, table_rows);
        else k_gather<bf16_t><<<grid_of(rows * cols), 256, 0, s>>>(t, ids, o, rows, cols, table_rows);
    }
    launch_check("gather");
}

void launch_rel_bias(const bf16_t* rel, const int* bucket, bf16_t* bias, int64_t heads, int64_t S,
                     hipStream_t s) {
    if (heads * S == 0) return;
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * heads * S * S);
    k_rel_bias<<<grid_of(heads * S * ((S + 7) / 8)), 256, 0, s>>>(rel, bucket, bias, heads, S);
    launch_check("relative bias");
}

}  // namespace bh
