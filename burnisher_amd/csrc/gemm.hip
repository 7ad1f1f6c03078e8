// bf16 GEMM for the dit-step on gfx950: out[M,N] = A[M,K] . B[N,K]^T (+bias, activation,
// fused residual), fp32 accumulation on the MFMA cores.
//
// Tile: 256 (M) x 144 (N) x 64 (K) per 512-thread workgroup, one workgroup per CU. 144 divides
// every DiT output width (1152, 3456, 4608, 28*2304) and 256 divides M = 2*4096, so the
// 8192-row GEMMs launch exactly 256, 768 and 1024 tiles: whole waves on 256 CUs, where the usual
// 256x128 tile would leave the last wave of N=1152 one-eighth full.
//
// Waves 0-3 multiply: wave w owns output rows [64w, 64w+64) and all 144 columns as a 4 x 9 grid
// of 16x16 accumulators (v_mfma_f32_16x16x32_bf16). Waves 4-7 only move the operands: direct
// global->LDS loads (global_load_lds_dwordx4, 1 KiB per wave instruction, no VGPRs) into THREE
// LDS stages of 51 KiB, two k-tiles in flight behind the one being multiplied (see k_gemm_tn).
// A DMA instruction can hold its wave for tens of cycles while the address unit is busy; in a
// wave of its own that costs the matrix cores nothing.
//
// LDS rows are 128 bytes (64 bf16 of K) with the 16-byte chunk c of row r stored at slot
// c ^ ((r >> 1) & 7): the 16 rows one ds_read_b128 fragment touches then cover all 64 banks
// exactly once, with no padding (padding would break the 1 KiB contiguity of a DMA write).
//
// The kernel is persistent (one workgroup per CU walking its tiles) and the k-tile pipeline
// runs on across tile boundaries, so the first k-tiles of a CU's next tile load while its
// consumers store the last one. The consumers store straight from the accumulators: the
// producers load A rows and B rows in a permuted order (a_row, b_col) chosen so that each lane
// ends up holding 8 consecutive output columns of 4 consecutive rows, which it finishes (bias,
// activation, residual, gate) and writes 16 bytes at a time, with no trip through LDS.
//
// Tile order is XCD-aware: workgroup i runs on XCD i%8, so tiles are renumbered so that each XCD
// gets a contiguous band of M-tiles x N-tiles, walked 4 M-tiles at a time, whose A and B panels
// share that XCD's L2.
//
// Summation order inside an MFMA differs from the reference oracle's sequential loop
// (ops_cpu.cpp:60-66); products of bf16 are exact in fp32, so results differ only by fp32
// accumulation rounding before the single bf16 rounding at the store.
#include "common.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

namespace bh {
namespace {

#include "gemm_tile.inc"
using namespace gk;

template <int ACT, int MODE, bool CONV, int MT = kMaxMT, int NT = kNT>
__global__ void __launch_bounds__(kWgThreads, 1)
k_gemm_tn(const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, bf16_t* out, int64_t M,
          int64_t N, int64_t K, Epi e, int tiles_m, int tiles_n, int group_m, ConvGeom cv) {
    __shared__ __attribute__((aligned(1024))) char smem[Geom<MT, NT>::kSmemBytes];
    const int T = tiles_m * tiles_n;
    const int my_tiles = (T - static_cast<int>(blockIdx.x) + static_cast<int>(gridDim.x) - 1) /
                         static_cast<int>(gridDim.x);
    // The wave index through readfirstlane: the compiler then knows it is uniform, so the role
    // branch and the DMA's LDS address are scalar.
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int KT = static_cast<int>(K / BK);
    const int64_t ldk = e.ld_k > 0 ? e.ld_k : K;
    if (MODE == EPI_F32 && gridDim.y > 1) {   // split-K: slice blockIdx.y of K, its own partial
        A += static_cast<int64_t>(blockIdx.y) * K;
        B += static_cast<int64_t>(blockIdx.y) * K;
        out += static_cast<int64_t>(blockIdx.y) * M * e.ld_out * 2;   // float elements
    }
    if (wave >= kConsumers) {
        produce<MT, CONV, NT>(smem, Operands{A, B, M, N, K, cv, ldk, e.bias}, KT, my_tiles, tiles_m,
                              tiles_n, group_m, wave - kConsumers, lane);
    } else {
        consume<MT, ACT, MODE, NT>(smem, e, out, M, N, KT, my_tiles, tiles_m, tiles_n, group_m, wave, lane);
    }
    wait_and_join<63>();   // the parked tile is complete and visible
    int64_t m0, n0;
    tile_origin<MT, NT>(blockIdx.x + (my_tiles - 1) * gridDim.x, tiles_m, tiles_n, group_m, m0, n0);
    store_staged<MT, ACT, MODE, NT>(smem, e, out, M, N, m0, n0, bias_slot<MT, NT>(smem, my_tiles - 1));
}

// ---- small M: one wave per output column, both operands read with 16-byte loads ----
constexpr int kGemvMaxM = 8;

__global__ void __launch_bounds__(256) k_gemv(const bf16_t* __restrict__ A,
                                              const bf16_t* __restrict__ B, bf16_t* out,
                                              int64_t M, int64_t N, int64_t K, Epi e, int mode) {
    const int lane = threadIdx.x & 63;
    const int64_t n = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (n >= N) return;
    float part[kGemvMaxM];
#pragma unroll
    for (int m = 0; m < kGemvMaxM; ++m) part[m] = 0.f;
    const int64_t chunks = K / 8;
    for (int64_t c = lane; c < chunks; c += 64) {
        const uint4 wb = *reinterpret_cast<const uint4*>(B + n * K + c * 8);
        const uint32_t w[4] = {wb.x, wb.y, wb.z, wb.w};
        float wf[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            wf[2 * t] = __uint_as_float(w[t] << 16);
            wf[2 * t + 1] = __uint_as_float(w[t] & 0xffff0000u);
        }
#pragma unroll
        for (int m = 0; m < kGemvMaxM; ++m) {
            if (m < M) {
                const uint4 ab = *reinterpret_cast<const uint4*>(A + m * K + c * 8);
                const uint32_t a[4] = {ab.x, ab.y, ab.z, ab.w};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    part[m] += __uint_as_float(a[t] << 16) * wf[2 * t];
                    part[m] += __uint_as_float(a[t] & 0xffff0000u) * wf[2 * t + 1];
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < kGemvMaxM; ++m) {
        float v = part[m];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        part[m] = v;
    }
    if (lane < M) {
        float a = 0.f;
#pragma unroll
        for (int m = 0; m < kGemvMaxM; ++m)
            if (m == lane) a = part[m];
        const int64_t m = lane;
        float v = e.bias ? __fadd_rn(a, bf2f(e.bias[n])) : a;
        v = finish(e, mode, act_exact(e.act, v), m, n, N);
        out[m * e.ld_out + n] = f2bf(v);
    }
}

// ---- reference order: one thread per output, sequential K, any layout and dtype ----
template <typename T> __device__ __forceinline__ float ldv(const T* p, int64_t i);
template <> __device__ __forceinline__ float ldv<float>(const float* p, int64_t i) { return p[i]; }
template <> __device__ __forceinline__ float ldv<bf16_t>(const bf16_t* p, int64_t i) {
    return bf2f(p[i]);
}
template <typename T> __device__ __forceinline__ void stv(T* p, int64_t i, float v);
template <> __device__ __forceinline__ void stv<float>(float* p, int64_t i, float v) { p[i] = v; }
template <> __device__ __forceinline__ void stv<bf16_t>(bf16_t* p, int64_t i, float v) {
    p[i] = f2bf(v);
}

template <typename T>
__global__ void __launch_bounds__(256) k_gemm_generic(const T* __restrict__ A, const T* __restrict__ B,
                                                      const T* __restrict__ bias, T* __restrict__ out,
                                                      int64_t M, int64_t N, int64_t K, bool bt,
                                                      int act) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t i = idx / N, j = idx % N;
    float acc = 0.f;
    for (int64_t p = 0; p < K; ++p) {
        const float bv = bt ? ldv(B, j * K + p) : ldv(B, p * N + j);
        acc = __fadd_rn(acc, __fmul_rn(ldv(A, i * K + p), bv));
    }
    if (bias) acc = __fadd_rn(acc, ldv(bias, j));
    stv(out, idx, act_exact(act, acc));
}

// Reference order with the fused epilogue (bf16, B as [N,K]): shapes whose K is not a multiple
// of the MFMA kernel's 64, e.g. the patch embedding's K = in_channels * patch^2 = 16.
__global__ void __launch_bounds__(256) k_gemm_fused_small(const bf16_t* __restrict__ A,
                                                          const bf16_t* __restrict__ B,
                                                          bf16_t* out, int64_t M, int64_t N,
                                                          int64_t K, Epi e, int mode) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= M * N) return;
    const int64_t m = idx / N, n = idx % N;
    float acc = 0.f;
    for (int64_t p = 0; p < K; ++p)
        acc = __fadd_rn(acc, __fmul_rn(bf2f(A[m * K + p]), bf2f(B[n * K + p])));
    if (e.bias) acc = __fadd_rn(acc, bf2f(e.bias[n]));
    out[m * e.ld_out + n] = f2bf(finish(e, mode, act_exact(e.act, acc), m, n, N));
}

// Small K (the patch embedding's K = in_channels * patch^2 = 16): each thread owns 8 consecutive
// output columns and walks kSmallKRows consecutive rows with them, the reference's sequential k
// order, 16-byte loads and stores. With K = 8 KC fixed (KC > 0) the thread's 8 x K weights are
// read once into registers: the weight rows of neighbouring threads lie 8 rows apart, so every
// 16-byte weight load touches a different cache line per lane, and reading them per output row
// made the patch embedding (8192 x 1152 x 16) take ~47 us. KC = 0 is any K % 8 == 0 up to 256,
// weights read per row. Needs N % 8 == 0 and 16-byte aligned operands. Four rows a thread, every
// load of the band issued before its first store: the patch embedding 27.1 -> 22.8 us (eight
// rows a thread that way take 272 VGPRs and 29.0 us; two rows re-read the weights too often,
// 30.1 us).
constexpr int kSmallKRows = 4;

__device__ __forceinline__ void smallk_store(const Epi& e, int mode, const float (&acc)[8], int m,
                                             int n0, int N, bf16_t* out) {
    float v[8], t[8];
    if (e.bias) {
        unpack8(*reinterpret_cast<const uint4*>(e.bias + n0), t);
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = __fadd_rn(acc[r], t[r]);
    } else {
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = acc[r];
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) v[r] = act_exact(e.act, v[r]);
    if (mode != EPI_STORE && e.round_mid) {
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = round_bf16(v[r]);
    }
    if (mode == EPI_ROW_ADD) {
        const int pr = static_cast<int>(m % static_cast<int>(e.row_add_period));
        unpack8(*reinterpret_cast<const uint4*>(e.row_add + static_cast<int64_t>(pr) * N + n0), t);
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = __fadd_rn(v[r], t[r]);
    } else if (mode == EPI_RESIDUAL || mode == EPI_GATED) {
        float res[8];
        unpack8(*reinterpret_cast<const uint4*>(e.residual + static_cast<int64_t>(m) * e.ld_out + n0), res);
        if (mode == EPI_GATED) {
            const int gr = static_cast<int>(m / static_cast<int>(e.gate_rows));
            unpack8(*reinterpret_cast<const uint4*>(e.gate + static_cast<int64_t>(gr) * N + n0), t);
#pragma unroll
            for (int r = 0; r < 8; ++r) v[r] = __fadd_rn(__fmul_rn(v[r], t[r]), res[r]);
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) v[r] = __fadd_rn(res[r], v[r]);
        }
    }
    *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m) * e.ld_out + n0) = pack8(v);
}

template <int KC>
__global__ void __launch_bounds__(256) k_gemm_smallk(const bf16_t* __restrict__ A,
                                                     const bf16_t* __restrict__ B, bf16_t* out,
                                                     int M, int N, int K, Epi e, int mode) {
    const int groups = N >> 3;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int band = idx / groups;
    if (band >= (M + kSmallKRows - 1) / kSmallKRows) return;
    const int n0 = (idx - band * groups) * 8;
    const int m0 = band * kSmallKRows, m1 = min(M, m0 + kSmallKRows);
    if constexpr (KC > 0) {
        constexpr int kK = 8 * KC;
        float w[8][kK];
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                float f[8];
                unpack8(*reinterpret_cast<const uint4*>(B + static_cast<int64_t>(n0 + r) * kK + 8 * c), f);
#pragma unroll
                for (int t = 0; t < 8; ++t) w[r][8 * c + t] = f[t];
            }
        if (m1 - m0 == kSmallKRows && (mode == EPI_STORE || mode == EPI_ROW_ADD)) {
            // A whole band of a plain or row-add store (the patch embedding, whose row add is the
            // position table): every A row and every row-add row is loaded before the first store,
            // one memory round trip for the band instead of one per row.
            uint4 ar[kSmallKRows][KC], ra[kSmallKRows];
#pragma unroll
            for (int i = 0; i < kSmallKRows; ++i) {
#pragma unroll
                for (int c = 0; c < KC; ++c)
                    ar[i][c] = *reinterpret_cast<const uint4*>(A + static_cast<int64_t>(m0 + i) * kK + 8 * c);
                if (mode == EPI_ROW_ADD) {
                    const int pr = static_cast<int>((m0 + i) % static_cast<int>(e.row_add_period));
                    ra[i] = *reinterpret_cast<const uint4*>(e.row_add + static_cast<int64_t>(pr) * N + n0);
                }
            }
            float bias[8];
            if (e.bias) {
                unpack8(*reinterpret_cast<const uint4*>(e.bias + n0), bias);
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) bias[r] = -0.0f;   // v + (-0.0) is v exactly
            }
#pragma unroll
            for (int i = 0; i < kSmallKRows; ++i) {
                float a[kK];
#pragma unroll
                for (int c = 0; c < KC; ++c) {
                    float f[8];
                    unpack8(ar[i][c], f);
#pragma unroll
                    for (int t = 0; t < 8; ++t) a[8 * c + t] = f[t];
                }
                float v[8];
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    float acc = 0.f;
#pragma unroll
                    for (int t = 0; t < kK; ++t) acc = __fadd_rn(acc, __fmul_rn(a[t], w[r][t]));
                    v[r] = act_exact(e.act, __fadd_rn(acc, bias[r]));
                }
                if (mode == EPI_ROW_ADD) {
                    float t[8];
                    if (e.round_mid) {
#pragma unroll
                        for (int r = 0; r < 8; ++r) v[r] = round_bf16(v[r]);
                    }
                    unpack8(ra[i], t);
#pragma unroll
                    for (int r = 0; r < 8; ++r) v[r] = __fadd_rn(v[r], t[r]);
                }
                *reinterpret_cast<uint4*>(out + static_cast<int64_t>(m0 + i) * e.ld_out + n0) = pack8(v);
            }
            return;
        }
        for (int m = m0; m < m1; ++m) {
            float a[kK];
#pragma unroll
            for (int c = 0; c < KC; ++c) {
                float f[8];
                unpack8(*reinterpret_cast<const uint4*>(A + static_cast<int64_t>(m) * kK + 8 * c), f);
#pragma unroll
                for (int t = 0; t < 8; ++t) a[8 * c + t] = f[t];
            }
            float acc[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                acc[r] = 0.f;
#pragma unroll
                for (int t = 0; t < kK; ++t) acc[r] = __fadd_rn(acc[r], __fmul_rn(a[t], w[r][t]));
            }
            smallk_store(e, mode, acc, m, n0, N, out);
        }
    } else {
        for (int m = m0; m < m1; ++m) {
            float acc[8];
#pragma unroll
            for (int r = 0; r < 8; ++r) acc[r] = 0.f;
            for (int k0 = 0; k0 < K; k0 += 8) {
                float a[8];
                unpack8(*reinterpret_cast<const uint4*>(A + static_cast<int64_t>(m) * K + k0), a);
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    float w[8];
                    unpack8(*reinterpret_cast<const uint4*>(B + static_cast<int64_t>(n0 + r) * K + k0), w);
#pragma unroll
                    for (int t = 0; t < 8; ++t) acc[r] = __fadd_rn(acc[r], __fmul_rn(a[t], w[t]));
                }
            }
            smallk_store(e, mode, acc, m, n0, N, out);
        }
    }
}

// Compute units of the current device, looked up once per device.
int device_cus() {
    static std::atomic<int> cus[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "gemm: device index out of range");
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev),
                  "hipDeviceGetAttribute");
        require(n > 0, "gemm: device reports no compute units");
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

bool aligned(const void* p, int bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

template <int ACT, int MODE, bool CONV = false, int MT = kMaxMT, int NT = kNT>
void launch_tn(const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n, int64_t k,
               const Epi& e, hipStream_t s, const ConvGeom& cv = ConvGeom{}) {
    constexpr int BM = Geom<MT, NT>::BM;
    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + kBN<NT> - 1) / kBN<NT>);
    const int tiles = tiles_m * tiles_n;
    // One persistent workgroup per CU (the LDS stages allow no second one); with the tile count
    // a multiple of 8, so is the grid, which the XCD banding relies on. An XCD's band is walked
    // 16 / MT M-tiles (1024 rows; 960 at the 192-row tile) at a time whatever the tile height.
    int grid = min(tiles, device_cus() & ~7);
    if (grid < 8) grid = min(tiles, device_cus());
    k_gemm_tn<ACT, MODE, CONV, MT, NT><<<grid, kWgThreads, 0, s>>>(a, b, out, m, n, k, e, tiles_m, tiles_n,
                                                               16 / MT, cv);
}

// The tile shape of a GEMM that runs whole (no split-K): the height (64 MT rows) and width (16 NT
// columns: 144, or 128 for widths that are multiples of 128) with the least
// estimated time, rounds x (rows a k-tile loads), where rounds = ceil(tiles / CUs) and a k-tile of
// a BM x BN tile loads BM + BN rows of 128 bytes. The k-loop runs at the rate its operand stream
// is delivered, not at the MFMA rate (~2,100 cycles per 256 x 144 k-tile against 1,152 of MFMA
// issue), so a smaller tile's k-tile is proportionally shorter. Ties keep the taller and the
// 144-wide tile. Every shape sums each output's k-tiles in the same order with the same MFMAs, so
// results do not depend on it.
struct TileShape {
    int mt, nt;
};
TileShape gemm_tile_shape(int64_t m, int64_t n) {
    const int64_t cus = device_cus();
    TileShape best{kMaxMT, kNT};
    int64_t best_cost = -1;
    for (int nt : {kNT, 8}) {
        if (nt == 8 && n % 128 != 0) continue;
        const int64_t bn = 16 * nt, tiles_n = (n + bn - 1) / bn;
        for (int mt = kMaxMT; mt >= 1; --mt) {
            const int64_t bm = 64 * mt, tiles = ((m + bm - 1) / bm) * tiles_n;
            // Over several rounds the XCD banding (tile_origin) needs a tile count divisible by
            // 8; without it an XCD's tiles scatter over the operand panels. 1152px ff2 on 486
            // 192 x 128 tiles measured 23% slower than on 432 of 192 x 144.
            if (tiles > cus && tiles % 8 != 0 && !(mt == kMaxMT && nt == kNT)) continue;
            const int64_t rounds = (tiles + cus - 1) / cus;
            const int64_t cost = rounds * (bm + bn);
            if (best_cost < 0 || cost < best_cost) {
                best = {mt, nt};
                best_cost = cost;
            }
        }
    }
    return best;
}

// Split-K plans in the tile chooser's units (one operand row loaded per k-tile, ~2.75 ns): a
// launch of S slices on BM x BN tiles costs ceil(tiles * S / CUs) rounds of K / S / 64 k-tiles of
// BM + BN rows each, plus its fp32 partials, S * M * N * 4 bytes written and read again by the
// summing epilogue at ~4.7 TB/s (one unit per 12,800 bytes). Fewer slices on shorter tiles can
// win: at 512px ff2 (2048 x 1152 x 4608) 2 slices of 128-row tiles instead of 4 of 256 rows
// halve the partial traffic (gemm_ff2 1.217 -> 1.149 ms per step, interleaved A/B).
int64_t splitk_cost(int64_t m, int64_t n, int64_t k, TileShape sh, int splits) {
    const int64_t bm = 64 * sh.mt, bn = 16 * sh.nt, cus = device_cus();
    const int64_t tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
    const int64_t rounds = (tiles * splits + cus - 1) / cus;
    const int64_t loop = rounds * (k / BK / splits) * (bm + bn);
    const int64_t partials = splits > 1 ? static_cast<int64_t>(splits) * m * n * 8 / 12800 : 0;
    return loop + partials;
}

// The tile shape of an S-slice launch: the cheapest by splitk_cost (ties keep the taller and the
// 144-wide tile; 128-wide for widths that are multiples of 128, with the XCD banding's tile count
// kept whole over several rounds). The shape does not change any sum; the slice count does, and
// is decided on the full batch.
TileShape splitk_tile_shape(int64_t m, int64_t n, int64_t k, int splits) {
    const int64_t cus = device_cus();
    TileShape best{kMaxMT, kNT};
    int64_t best_cost = -1;
    for (int nt : {kNT, 8}) {
        if (nt == 8 && n % 128 != 0) continue;
        for (int mt = kMaxMT; mt >= 1; --mt) {
            const int64_t bm = 64 * mt, bn = 16 * nt, tiles = ((m + bm - 1) / bm) * ((n + bn - 1) / bn);
            if (tiles * splits > cus && tiles % 8 != 0 && !(mt == kMaxMT && nt == kNT)) continue;
            const int64_t c = splitk_cost(m, n, k, TileShape{mt, nt}, splits);
            if (best_cost < 0 || c < best_cost) {
                best = {mt, nt};
                best_cost = c;
            }
        }
    }
    return best;
}

// Split-K partials: `splits` slices of K in one launch (grid.y = slice), each persistent
// workgroup set over the same output tiles, slice s writing fp32 partial[s][m][n].
template <int MT = kMaxMT, int NT = kNT>
void launch_tn_splitk(const bf16_t* a, const bf16_t* b, float* partial, int64_t m, int64_t n, int64_t k,
                      int splits, hipStream_t s) {
    constexpr int BM = Geom<MT, NT>::BM;
    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + kBN<NT> - 1) / kBN<NT>);
    const int tiles = tiles_m * tiles_n;
    const int grid = max(1, min(tiles, device_cus() / splits));
    Epi e{};
    e.row_add_period = 1;
    e.gate_rows = 1;
    e.ld_out = n;
    e.ld_k = k;
    e.vt_dim = 72;
    k_gemm_tn<0, EPI_F32, false, MT, NT><<<dim3(grid, splits), kWgThreads, 0, s>>>(
        a, b, reinterpret_cast<bf16_t*>(partial), m, n, k / splits, e, tiles_m, tiles_n, 16 / MT, ConvGeom{});
}

// The partials of an S-slice split on the tile shape splitk_tile_shape picks for it.
void launch_splitk_partials(const bf16_t* a, const bf16_t* b, float* partial, int64_t m, int64_t n,
                            int64_t k, int splits, hipStream_t s) {
    const TileShape sh = splitk_tile_shape(m, n, k, splits);
    if (sh.nt == 8) {
        switch (sh.mt) {
            case 1: launch_tn_splitk<1, 8>(a, b, partial, m, n, k, splits, s); break;
            case 2: launch_tn_splitk<2, 8>(a, b, partial, m, n, k, splits, s); break;
            case 3: launch_tn_splitk<3, 8>(a, b, partial, m, n, k, splits, s); break;
            default: launch_tn_splitk<kMaxMT, 8>(a, b, partial, m, n, k, splits, s); break;
        }
        return;
    }
    switch (sh.mt) {
        case 1: launch_tn_splitk<1>(a, b, partial, m, n, k, splits, s); break;
        case 2: launch_tn_splitk<2>(a, b, partial, m, n, k, splits, s); break;
        case 3: launch_tn_splitk<3>(a, b, partial, m, n, k, splits, s); break;
        default: launch_tn_splitk<kMaxMT>(a, b, partial, m, n, k, splits, s); break;
    }
}

// The split-K reductions below take the slice count S as a template argument, so a thread issues
// the loads of all S slices (and of the residual and gate) before the first addition: with a
// run-time count each slice's load waited for the previous slice's sum, S + 1 memory round trips
// per thread, which set the launch's time because every thread of the grid is resident at once.

// out[m, n] = bf16(residual[m, n] + bf16(sum_s partial[s][m][n])), the slices summed in order.
template <int S>
__global__ void __launch_bounds__(256) k_splitk_residual(const float* __restrict__ partial,
                                                         const bf16_t* residual, bf16_t* out, int64_t mn) {
    for (int64_t i = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) * 4; i < mn;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x * 4) {
        f32x4_t p[S];
#pragma unroll
        for (int sp = 0; sp < S; ++sp) p[sp] = *reinterpret_cast<const f32x4_t*>(partial + sp * mn + i);
        const uint2 r = *reinterpret_cast<const uint2*>(residual + i);
        f32x4_t acc = p[0];
#pragma unroll
        for (int sp = 1; sp < S; ++sp)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = __fadd_rn(acc[q], p[sp][q]);
        const float res[4] = {__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                              __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u)};
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float lo = __fadd_rn(res[2 * q], round_bf16(acc[2 * q]));
            const float hi = __fadd_rn(res[2 * q + 1], round_bf16(acc[2 * q + 1]));
            o[q] = f2bf2(lo, hi);
        }
        *reinterpret_cast<uint2*>(out + i) = make_uint2(o[0], o[1]);
    }
}

// The split-K epilogue: out[m, n8..n8+7] from the slices summed in order, then exactly the MFMA
// kernel's epilogue (chunk_store): bias, activation, the mid rounding, residual or gated residual,
// one rounding at the store. out may alias the residual (each element is read before written).
template <int ACT, int MODE, int S>
__global__ void __launch_bounds__(256) k_splitk_epi(const float* __restrict__ partial, int64_t M,
                                                    int64_t N, Epi e, bf16_t* out) {
    const int64_t per_row = N / 8;
    const int64_t groups = M * per_row;
    const int64_t mn = M * N;
    for (int64_t g = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; g < groups;
         g += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t m = g / per_row, n = (g - m * per_row) * 8;
        const float* p = partial + m * N + n;
        f32x4_t a[S], b[S];
#pragma unroll
        for (int sp = 0; sp < S; ++sp) {
            a[sp] = *reinterpret_cast<const f32x4_t*>(p + sp * mn);
            b[sp] = *reinterpret_cast<const f32x4_t*>(p + sp * mn + 4);
        }
        const uint4 braw = e.bias ? *reinterpret_cast<const uint4*>(e.bias + n) : uint4{};
        uint4 rraw{}, graw{};
        if (MODE == EPI_RESIDUAL || MODE == EPI_GATED) rraw = *reinterpret_cast<const uint4*>(e.residual + m * e.ld_out + n);
        if (MODE == EPI_GATED) graw = *reinterpret_cast<const uint4*>(e.gate + (m / e.gate_rows) * N + n);
        f32x4_t lo = a[0], hi = b[0];
#pragma unroll
        for (int sp = 1; sp < S; ++sp)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lo[q] = __fadd_rn(lo[q], a[sp][q]);
                hi[q] = __fadd_rn(hi[q], b[sp][q]);
            }
        float x[8], bias[8], t[8];
        bias_or_neg_zero(e, braw, bias);
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = act_fast<ACT>(__fadd_rn(q < 4 ? lo[q] : hi[q - 4], bias[q]));
        if (MODE != EPI_STORE && e.round_mid)
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = round_bf16(x[q]);
        if (MODE == EPI_RESIDUAL) {
            unpack8(rraw, t);
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(t[q], x[q]);
        }
        if (MODE == EPI_GATED) {
            float gq[8];
            unpack8(graw, gq);
            unpack8(rraw, t);
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(__fmul_rn(x[q], gq[q]), t[q]);
        }
        *reinterpret_cast<uint4*>(out + m * e.ld_out + n) = pack8(x);
    }
}

// Per-device fp32 partials for split-K calls that bring no buffer of their own, grown on demand.
float* splitk_workspace(int64_t floats) {
    static std::mutex mu;
    static void* ptr[64] = {};
    static int64_t cap[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "gemm: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] < floats) {
        if (ptr[dev]) hip_check(hipFree(ptr[dev]), "hipFree");
        ptr[dev] = nullptr;
        cap[dev] = 0;
        hip_check(hipMalloc(&ptr[dev], static_cast<size_t>(floats) * sizeof(float)), "hipMalloc (split-K partials)");
        cap[dev] = floats;
    }
    return static_cast<float*>(ptr[dev]);
}

template <int ACT, int S>
void launch_splitk_epi_s(int mode, const float* partial, int64_t m, int64_t n, const Epi& e, bf16_t* out,
                         hipStream_t s) {
    const int64_t groups = m * (n / 8);
    const int blocks = static_cast<int>(std::min<int64_t>((groups + 255) / 256, 8192));
    switch (mode) {
        case EPI_STORE: k_splitk_epi<ACT, EPI_STORE, S><<<blocks, 256, 0, s>>>(partial, m, n, e, out); break;
        case EPI_RESIDUAL: k_splitk_epi<ACT, EPI_RESIDUAL, S><<<blocks, 256, 0, s>>>(partial, m, n, e, out); break;
        default: k_splitk_epi<ACT, EPI_GATED, S><<<blocks, 256, 0, s>>>(partial, m, n, e, out); break;
    }
}

template <int ACT>
void launch_splitk_epi(int mode, const float* partial, int splits, int64_t m, int64_t n, const Epi& e,
                       bf16_t* out, hipStream_t s) {
    switch (splits) {
        case 2: launch_splitk_epi_s<ACT, 2>(mode, partial, m, n, e, out, s); break;
        case 3: launch_splitk_epi_s<ACT, 3>(mode, partial, m, n, e, out, s); break;
        case 4: launch_splitk_epi_s<ACT, 4>(mode, partial, m, n, e, out, s); break;
        case 5: launch_splitk_epi_s<ACT, 5>(mode, partial, m, n, e, out, s); break;
        case 6: launch_splitk_epi_s<ACT, 6>(mode, partial, m, n, e, out, s); break;
        case 7: launch_splitk_epi_s<ACT, 7>(mode, partial, m, n, e, out, s); break;
        default: launch_splitk_epi_s<ACT, 8>(mode, partial, m, n, e, out, s); break;   // 2..8 slices
    }
}

template <int ACT, int MT, int NT = kNT>
void launch_tn_mode(int mode, const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n,
                    int64_t k, const Epi& e, hipStream_t s) {
    switch (mode) {
        case EPI_STORE: launch_tn<ACT, EPI_STORE, false, MT, NT>(a, b, out, m, n, k, e, s); break;
        case EPI_ROW_ADD: launch_tn<ACT, EPI_ROW_ADD, false, MT, NT>(a, b, out, m, n, k, e, s); break;
        case EPI_RESIDUAL: launch_tn<ACT, EPI_RESIDUAL, false, MT, NT>(a, b, out, m, n, k, e, s); break;
        default: launch_tn<ACT, EPI_GATED, false, MT, NT>(a, b, out, m, n, k, e, s); break;
    }
}

template <int ACT>
void launch_tn_mt(TileShape sh, int mode, const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n,
                  int64_t k, const Epi& e, hipStream_t s) {
    if (sh.nt == 8) {
        switch (sh.mt) {
            case 1: launch_tn_mode<ACT, 1, 8>(mode, a, b, out, m, n, k, e, s); break;
            case 2: launch_tn_mode<ACT, 2, 8>(mode, a, b, out, m, n, k, e, s); break;
            case 3: launch_tn_mode<ACT, 3, 8>(mode, a, b, out, m, n, k, e, s); break;
            default: launch_tn_mode<ACT, kMaxMT, 8>(mode, a, b, out, m, n, k, e, s); break;
        }
        return;
    }
    switch (sh.mt) {
        case 1: launch_tn_mode<ACT, 1>(mode, a, b, out, m, n, k, e, s); break;
        case 2: launch_tn_mode<ACT, 2>(mode, a, b, out, m, n, k, e, s); break;
        case 3: launch_tn_mode<ACT, 3>(mode, a, b, out, m, n, k, e, s); break;
        default: launch_tn_mode<ACT, kMaxMT>(mode, a, b, out, m, n, k, e, s); break;
    }
}

}  // namespace

void launch_gemm_generic(const void* a, const void* b, const void* bias, void* out, int64_t m,
                         int64_t n, int64_t k, bool b_transposed, int act, bool f32,
                         hipStream_t s) {
    const int64_t total = m * n;
    if (total == 0) return;
    const int grid = static_cast<int>((total + 255) / 256);
    if (f32) {
        k_gemm_generic<float><<<grid, 256, 0, s>>>(
            static_cast<const float*>(a), static_cast<const float*>(b),
            static_cast<const float*>(bias), static_cast<float*>(out), m, n, k, b_transposed, act);
    } else {
        k_gemm_generic<bf16_t><<<grid, 256, 0, s>>>(
            static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
            static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(out), m, n, k, b_transposed,
            act);
    }
    launch_check("gemm (reference order)");
}

void launch_gemm_bf16(const bf16_t* a, const bf16_t* b, const bf16_t* bias, bf16_t* out,
                      int64_t m, int64_t n, int64_t k, const GemmEpilogue& ep, hipStream_t s) {
    if (m == 0 || n == 0) return;
    require(!ep.gate || ep.residual, "gemm: a gate needs a residual");
    Epi e{bias, ep.act, ep.round_mid, ep.row_add, ep.row_add_period > 0 ? ep.row_add_period : 1,
          ep.residual, ep.gate, ep.gate_rows > 0 ? ep.gate_rows : 1, ep.ld_out > 0 ? ep.ld_out : n, 0,
          ep.vt, ep.vt_period, ep.vt_col0, ep.vt_seq, ep.vt_ld, ep.vt_heads, ep.vt_dim};
    if (ep.vt) {
        require(!ep.residual && !ep.row_add && !ep.round_mid,
                "gemm: the transposed V store has no residual or row-add epilogue");
        require(ep.vt_period > 0 && ep.vt_period % BN == 0 && ep.vt_col0 % BN == 0 &&
                    ep.vt_col0 < ep.vt_period && ep.vt_seq > 0 && m % ep.vt_seq == 0 &&
                    ep.vt_ld >= ep.vt_seq && ep.vt_heads > 0 && ep.vt_dim > 0 &&
                    ep.vt_dim == 72 && (ep.vt_period - ep.vt_col0) == int64_t{ep.vt_heads} * 72 &&
                    ep.vt_ld % 32 == 0 && ep.vt_seq % 4 == 0 && aligned(ep.vt, 16) &&
                    m < (int64_t{1} << 31) && n < (int64_t{1} << 31),
                "gemm: transposed V store geometry");
    }
    const int mode = ep.residual ? (ep.gate ? EPI_GATED : EPI_RESIDUAL)
                                 : (ep.row_add ? EPI_ROW_ADD : EPI_STORE);
    const double flops = 2.0 * static_cast<double>(m) * n * k;
    const bool k8 = (k % 8 == 0) && aligned(a, 16) && aligned(b, 16);
    require(!ep.vt || (k8 && m > kGemvMaxM && k % BK == 0),
            "gemm: the transposed V store needs the MFMA kernel (K % 64 == 0, M > 8)");
    if (k8 && m <= kGemvMaxM) {
        ProfileScope ps(K_GEMV, s, flops);
        const int grid = static_cast<int>((n + 3) / 4);
        k_gemv<<<grid, 256, 0, s>>>(a, b, out, m, n, k, e, mode);
        launch_check("gemm (small M)");
        return;
    }
    // The MFMA kernel's epilogue works on aligned runs of 8 columns.
    const bool vec = (e.ld_out % 8 == 0) && aligned(out, 16) && (!bias || aligned(bias, 16)) &&
                     (!e.residual || aligned(e.residual, 16)) && (!e.gate || aligned(e.gate, 16)) &&
                     (!e.row_add || aligned(e.row_add, 16)) && (n % 8 == 0);
    if (k8 && k % BK != 0 && vec && k <= 256 && m * (n / 8) < (int64_t{1} << 31) &&
        e.row_add_period < (int64_t{1} << 31) && e.gate_rows < (int64_t{1} << 31)) {
        ProfileScope ps(K_GEMM, s, flops);
        const int64_t threads = (m + kSmallKRows - 1) / kSmallKRows * (n / 8);
        const int blocks = static_cast<int>((threads + 255) / 256);
        const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
        if (k == 8) k_gemm_smallk<1><<<blocks, 256, 0, s>>>(a, b, out, mi, ni, ki, e, mode);
        else if (k == 16) k_gemm_smallk<2><<<blocks, 256, 0, s>>>(a, b, out, mi, ni, ki, e, mode);
        else k_gemm_smallk<0><<<blocks, 256, 0, s>>>(a, b, out, mi, ni, ki, e, mode);
        launch_check("gemm (small K)");
        return;
    }
    if (!k8 || k % BK != 0 || !vec || k == 0) {
        ProfileScope ps(K_GEMM, s, flops);
        const int64_t total = m * n;
        k_gemm_fused_small<<<static_cast<int>((total + 255) / 256), 256, 0, s>>>(a, b, out, m, n,
                                                                                k, e, mode);
        launch_check("gemm (reference order, fused epilogue)");
        return;
    }
    // the MFMA kernel's epilogues index rows, gate rows and row-add rows in 32 bits
    require(m < (int64_t{1} << 31) && n < (int64_t{1} << 31) && e.gate_rows < (int64_t{1} << 31) &&
                e.row_add_period < (int64_t{1} << 31),
            "gemm: M, N, the gate's row count and the row-add period must be below 2^31");
    const int splits = ep.splitk > 0 ? ep.splitk : gemm_splits(m, n, k, ep);
    if (splits > 1) {
        require(k % (BK * splits) == 0 && !ep.vt && mode != EPI_ROW_ADD && splits <= 8,
                "gemm split-K: " + std::to_string(splits) + " slices of K = " + std::to_string(k) +
                    " (whole 64-wide k-tiles, plain, residual or gated store only)");
        const int64_t floats = static_cast<int64_t>(splits) * m * n;
        float* partial = ep.splitk_ws;
        if (partial) {
            require(ep.splitk_ws_floats >= floats && aligned(partial, 16),
                    "gemm split-K: the partial buffer holds " + std::to_string(ep.splitk_ws_floats) +
                        " floats, this call needs " + std::to_string(floats));
        } else {
            partial = splitk_workspace(floats);
        }
        ProfileScope ps(K_GEMM, s, flops, gemm_subclass());
        launch_splitk_partials(a, b, partial, m, n, k, splits, s);
        launch_check("gemm (split-K partials)");
        switch (ep.act) {
            case 1: launch_splitk_epi<1>(mode, partial, splits, m, n, e, out, s); break;
            case 2: launch_splitk_epi<2>(mode, partial, splits, m, n, e, out, s); break;
            default: launch_splitk_epi<0>(mode, partial, splits, m, n, e, out, s); break;
        }
        launch_check("gemm (split-K epilogue)");
        return;
    }
    ProfileScope ps(K_GEMM, s, flops, gemm_subclass());
    // the transposed V store: 256 x 144 tiles
    const TileShape mt = ep.vt ? TileShape{kMaxMT, kNT} : gemm_tile_shape(m, n);
    switch (ep.act) {
        case 1: launch_tn_mt<1>(mt, mode, a, b, out, m, n, k, e, s); break;
        case 2: launch_tn_mt<2>(mt, mode, a, b, out, m, n, k, e, s); break;
        default: launch_tn_mt<0>(mt, mode, a, b, out, m, n, k, e, s); break;
    }
    launch_check("gemm (mfma)");
}

void launch_conv3x3_bf16(const ConvGeom& cv, const bf16_t* wr, const bf16_t* bias, bf16_t* out,
                         int64_t c_out, const GemmEpilogue& ep, hipStream_t s) {
    const int64_t m = static_cast<int64_t>(cv.H) * cv.W, k = 9 * static_cast<int64_t>(cv.c_in);
    if (m == 0 || c_out == 0) return;
    require(cv.in && cv.zero && wr && out, "conv3x3: null operand");
    require(cv.c_in % 64 == 0 && cv.c_in > 0, "conv3x3 (mfma): c_in must be a positive multiple of 64");
    require(c_out % 8 == 0, "conv3x3 (mfma): c_out must be a multiple of 8");
    require(cv.up ? (cv.in_h * 2 == cv.H && cv.in_w * 2 == cv.W) : (cv.in_h == cv.H && cv.in_w == cv.W),
            "conv3x3: input and output sizes disagree");
    require(!ep.vt && !ep.row_add && !ep.gate, "conv3x3: epilogue must be a plain store or a residual add");
    require(aligned(cv.in, 16) && aligned(cv.zero, 16) && aligned(wr, 16) && aligned(out, 16) &&
                (!bias || aligned(bias, 16)) && (!ep.residual || aligned(ep.residual, 16)),
            "conv3x3: operands must be 16-byte aligned");
    require(static_cast<int64_t>(cv.in_h) * cv.in_w * cv.c_in < (int64_t{1} << 31),
            "conv3x3: input too large for 32-bit pixel offsets");
    Epi e{bias, ep.act, ep.round_mid, nullptr, 1, ep.residual, nullptr, 1,
          ep.ld_out > 0 ? ep.ld_out : c_out, 0, nullptr, 0, 0, 0, 0, 0, 72};
    require(ep.act == 0, "conv3x3: no activation epilogue (the decoder's SiLU follows a GroupNorm)");
    ProfileScope ps(K_GEMM, s, 2.0 * static_cast<double>(m) * c_out * k);
    // The decoder's channel counts are powers of two: 128-wide tiles cover them exactly, where
    // 144-wide ones would pad every tile row by 16 columns (11% of the MFMAs).
    const bool narrow = c_out % 128 == 0 && c_out % 144 != 0;
    if (ep.residual) {
        if (narrow) launch_tn<0, EPI_RESIDUAL, true, kMaxMT, 8>(cv.in, wr, out, m, c_out, k, e, s, cv);
        else launch_tn<0, EPI_RESIDUAL, true>(cv.in, wr, out, m, c_out, k, e, s, cv);
    } else {
        if (narrow) launch_tn<0, EPI_STORE, true, kMaxMT, 8>(cv.in, wr, out, m, c_out, k, e, s, cv);
        else launch_tn<0, EPI_STORE, true>(cv.in, wr, out, m, c_out, k, e, s, cv);
    }
    launch_check("conv3x3 (mfma)");
}

int gemm_splitk_choice(int64_t m, int64_t n, int64_t k) {
    if (m <= kGemvMaxM || n % 8 != 0 || k % BK != 0) return 1;
    const int64_t tiles = ((m + Geom<kMaxMT>::BM - 1) / Geom<kMaxMT>::BM) * ((n + BN - 1) / BN);
    const int cus = device_cus();
    int best = 1;
    for (int sp = 2; sp <= 8; ++sp)
        if (tiles * sp <= cus && k % (BK * sp) == 0 && k / sp >= 4 * BK) best = sp;
    return best;
}

// Automatic split-K only for long K (>= 48 k-tiles: the 4608-deep ff2 and the 4096-wide caption
// projection). Slices of a 1152-deep GEMM carry more fp32 partial traffic than they save, and
// leaving them whole keeps the fused QKV projection summing exactly like the separate Q, K and V
// projections of the op-by-op graph.
constexpr int kSplitKMinKTiles = 48;

int gemm_splits(int64_t m, int64_t n, int64_t k, const GemmEpilogue& ep) {
    if (ep.splitk > 0) return ep.splitk;
    if (ep.vt || ep.row_add || m <= kGemvMaxM || k % BK != 0 || n % 8 != 0) return 1;
    if (k / BK < kSplitKMinKTiles) return 1;
    const int64_t tiles = ((m + Geom<kMaxMT>::BM - 1) / Geom<kMaxMT>::BM) * ((n + BN - 1) / BN);
    if (tiles * 2 > device_cus()) return 1;
    // the slice count (2..8, whole k-tiles, at least 4 per slice) whose best tile height gives the
    // cheapest plan; against the whole GEMM at its own best height
    int best = 1;
    int64_t best_cost = -1;
    for (int sp = 1; sp <= 8; ++sp) {
        if (sp > 1 && (k % (BK * sp) != 0 || k / sp < 4 * BK)) continue;
        const int64_t c = splitk_cost(m, n, k, splitk_tile_shape(m, n, k, sp), sp);
        if (best_cost < 0 || c < best_cost) {
            best = sp;
            best_cost = c;
        }
    }
    return best;
}

void launch_gemm_splitk_residual(const bf16_t* a, const bf16_t* b, float* partial, int splits,
                                 const bf16_t* residual, bf16_t* out, int64_t m, int64_t n, int64_t k,
                                 hipStream_t s) {
    if (m == 0 || n == 0) return;
    require(splits >= 2 && splits <= 8 && k % (BK * splits) == 0 && n % 8 == 0 && m > kGemvMaxM,
            "gemm split-K: K must split into whole 64-wide k-tiles, N % 8 == 0");
    require(aligned(a, 16) && aligned(b, 16) && aligned(partial, 16) && aligned(residual, 8) && aligned(out, 8),
            "gemm split-K: operands must be 16-byte aligned");
    {
        ProfileScope ps(K_GEMM, s, 2.0 * static_cast<double>(m) * n * k);
        launch_splitk_partials(a, b, partial, m, n, k, splits, s);
        launch_check("gemm (split-K partials)");
    }
    ProfileScope ps(K_ELEMENTWISE, s, static_cast<double>(m) * n * (4.0 * splits + 4.0));
    const int64_t mn = m * n;
    const int64_t blocks = std::min<int64_t>((mn / 4 + 255) / 256, 8192);
    const int g = static_cast<int>(blocks);
    switch (splits) {
        case 2: k_splitk_residual<2><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        case 3: k_splitk_residual<3><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        case 4: k_splitk_residual<4><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        case 5: k_splitk_residual<5><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        case 6: k_splitk_residual<6><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        case 7: k_splitk_residual<7><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
        default: k_splitk_residual<8><<<g, 256, 0, s>>>(partial, residual, out, mn); break;
    }
    launch_check("gemm (split-K reduce)");
}

}  // namespace bh

