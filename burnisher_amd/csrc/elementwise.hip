// Bandwidth-bound kernels of the dit-step: LayerNorm (and LayerNorm fused with the adaLN
// chunk + modulation), modulate with gated residual, add, chunk, activation, patchify and the
// timestep embedding.
//
// Each one reproduces the reference oracle's arithmetic exactly (src/cpu/ops_cpu.cpp:186-349):
// the same fp64 LayerNorm statistics, the same separate fp32 multiplies and adds (written with
// __fmul_rn/__fadd_rn so the compiler cannot contract them into FMAs, which the host oracle
// never forms), one bf16 rounding per stored element. Only the order of the fp64 row sums
// differs, which in fp64 changes the float statistics essentially never.
//
// Layout: one 64-lane wave per row for the row kernels (a DiT row is 1152 bf16 = 2304 B, read
// with 16-byte loads); grid-stride 8-element vectors for the elementwise kernels.
#include "common.h"

#include <cmath>

namespace bh {
namespace {


constexpr int kWave = 64;

// The wave's index in its workgroup through readfirstlane: the compiler then knows it is uniform
// and keeps a one-row-per-wave kernel's row, batch index and row addresses in scalar registers
// instead of redoing that arithmetic (a 64-bit division among it) in every lane.
__device__ __forceinline__ int wave_index() {
    return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kWave);
}

template <typename T> struct Io;
template <> struct Io<float> {
    static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Io<bf16_t> {
    static __device__ __forceinline__ float ld(const bf16_t* p, int64_t i) { return bf2f(p[i]); }
    static __device__ __forceinline__ void st(bf16_t* p, int64_t i, float v) { p[i] = f2bf(v); }
};

// Sum over the 64 lanes of a wave, in VALU cross-lane operations (no LDS round trips): DPP
// within groups of 4, 8 and 16 lanes, then v_permlane16_swap / v_permlane32_swap across them.
// Lanes can finish with sums in different orders, so lane 0's total is broadcast: every lane
// returns the same value.
template <int CTRL>
__device__ __forceinline__ double dpp_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u), CTRL, 0xf, 0xf, true);
    const uint32_t hi = __builtin_amdgcn_update_dpp(0u, static_cast<uint32_t>(u >> 32), CTRL, 0xf, 0xf, true);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}
template <bool SWAP32>
__device__ __forceinline__ double swap_sum_d(double v) {
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(u), hi = static_cast<uint32_t>(u >> 32);
    const auto l = SWAP32 ? __builtin_amdgcn_permlane32_swap(lo, lo, false, false)
                          : __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto h = SWAP32 ? __builtin_amdgcn_permlane32_swap(hi, hi, false, false)
                          : __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    return __builtin_bit_cast(double, (static_cast<uint64_t>(h[0]) << 32) | l[0]) +
           __builtin_bit_cast(double, (static_cast<uint64_t>(h[1]) << 32) | l[1]);
}
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_d<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v += dpp_d<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v += dpp_d<0x141>(v);   // row_half_mirror: the other quad of the 8
    v += dpp_d<0x140>(v);   // row_mirror: the other 8 of the 16
    v = swap_sum_d<false>(v);
    v = swap_sum_d<true>(v);
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

// 8 bf16 <-> 8 floats through one 16-byte access.
struct V8 {
    float f[8];
};
__device__ __forceinline__ V8 unpack_v8(const uint4 raw) {
    V8 r;
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        r.f[2 * i] = __uint_as_float(w[i] << 16);
        r.f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
    return r;
}
__device__ __forceinline__ V8 load8(const bf16_t* p) {
    return unpack_v8(*reinterpret_cast<const uint4*>(p));
}
__device__ __forceinline__ void store8(bf16_t* p, const V8& v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[i] = f2bf2(v.f[2 * i], v.f[2 * i + 1]);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}

// ---- LayerNorm / RMSNorm, generic (the NormArgs op) -----------------------------------------

// One wave per row. Values are re-read from global memory for each pass (the row is L1/L2
// resident), which keeps the kernel valid for any `cols`.
template <typename T>
__global__ void __launch_bounds__(256) k_norm(const T* __restrict__ x, const T* __restrict__ w,
                                              const T* __restrict__ b, T* __restrict__ out,
                                              int64_t rows, int64_t cols, float eps, bool rms) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_index();
    if (row >= rows) return;
    const T* xr = x + row * cols;
    double mean = 0.0;
    if (!rms) {
        double s = 0.0;
        for (int64_t i = lane; i < cols; i += kWave) s += static_cast<double>(Io<T>::ld(xr, i));
        mean = wave_sum(s) / static_cast<double>(cols);
    }
    double var = 0.0;
    for (int64_t i = lane; i < cols; i += kWave) {
        const double d = static_cast<double>(Io<T>::ld(xr, i)) - mean;
        var += d * d;
    }
    var = wave_sum(var) / static_cast<double>(cols);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    const float fmean = static_cast<float>(mean);
    for (int64_t i = lane; i < cols; i += kWave) {
        float v = __fmul_rn(__fsub_rn(Io<T>::ld(xr, i), fmean), inv);
        if (w) v = __fmul_rn(v, Io<T>::ld(w, i));
        if (b) v = __fadd_rn(v, Io<T>::ld(b, i));
        Io<T>::st(out + row * cols, i, v);
    }
}

// The same op for bf16 rows of cols % 8 == 0 and at most NV * 512 columns: one wave per row,
// the row read ONCE into registers as 16-byte vectors (the generic kernel's three scalar passes
// over global memory made a 600 x 4096 RMSNorm latency-bound at ~45 us). Statistics in fp64
// as the oracle forms them; an RMS row's mean is exactly 0.
template <int NV>
__global__ void __launch_bounds__(256) k_norm_rows(const bf16_t* __restrict__ x,
                                                   const bf16_t* __restrict__ w,
                                                   const bf16_t* __restrict__ b,
                                                   bf16_t* __restrict__ out, int64_t rows,
                                                   int64_t cols, float eps, bool rms) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_index();
    if (row >= rows) return;
    const int nvec = static_cast<int>(cols / 8);
    const bf16_t* xr = x + row * cols;
    V8 v[NV];
    uint4 wraw[NV];   // the weight vectors, loaded with the row so their latency overlaps it
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * kWave;
        v[j] = unpack_v8(vi < nvec ? *reinterpret_cast<const uint4*>(xr + vi * 8) : make_uint4(0, 0, 0, 0));
        wraw[j] = (w && vi < nvec) ? *reinterpret_cast<const uint4*>(w + vi * 8) : make_uint4(0, 0, 0, 0);
    }
    double mean = 0.0;
    if (!rms) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < NV; ++j)
#pragma unroll
            for (int e = 0; e < 8; ++e) s += static_cast<double>(v[j].f[e]);
        mean = wave_sum(s) / static_cast<double>(cols);
    }
    double q = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (lane + j * kWave < nvec) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double d = static_cast<double>(v[j].f[e]) - mean;
                q += d * d;
            }
        }
    }
    const double var = wave_sum(q) / static_cast<double>(cols);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    const float fmean = static_cast<float>(mean);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * kWave;
        if (vi >= nvec) continue;
        V8 o;
        const V8 wv = unpack_v8(wraw[j]);
        const V8 bv = b ? load8(b + vi * 8) : V8{};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float t = __fmul_rn(__fsub_rn(v[j].f[e], fmean), inv);
            if (w) t = __fmul_rn(t, wv.f[e]);
            if (b) t = __fadd_rn(t, bv.f[e]);
            o.f[e] = t;
        }
        store8(out + row * cols + vi * 8, o);
    }
}

// ---- LayerNorm fused with the adaLN chunk and modulation (the hot row kernel) ---------------

// Row statistics exactly as the oracle forms them: fp64 mean, fp64 sum of squared deviations,
// then float inverse standard deviation.
template <int NV>
__device__ __forceinline__ void row_stats(const V8 (&v)[NV], int nvec, int lane, int64_t cols,
                                          float eps, float* fmean, float* inv) {
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (lane + j * kWave < nvec) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s += static_cast<double>(v[j].f[e]);
        }
    }
    const double mean = wave_sum(s) / static_cast<double>(cols);
    double q = 0.0;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        if (lane + j * kWave < nvec) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const double d = static_cast<double>(v[j].f[e]) - mean;
                q += d * d;
            }
        }
    }
    const double var = wave_sum(q) / static_cast<double>(cols);
    *inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    *fmean = static_cast<float>(mean);
}

// shift/scale either precomputed ([batch, C] rows, already rounded) or formed here from the
// modulation vector and the table, rounded as the chunk op stores them.
template <int NV, bool PRE>
__global__ void __launch_bounds__(256) k_norm_modulate(
    const bf16_t* __restrict__ x, const bf16_t* __restrict__ mod, int64_t mod_stride,
    const bf16_t* __restrict__ shift_src, const bf16_t* __restrict__ scale_src,
    const bf16_t* __restrict__ shift_tab, const bf16_t* __restrict__ scale_tab,
    bf16_t* __restrict__ out, int64_t rows, int64_t tokens, int64_t cols, float eps) {
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_index();
    if (row >= rows) return;
    const int nvec = static_cast<int>(cols / 8);
    const bf16_t* xr = x + row * cols;
    // The row stays packed (bf16) in registers and is unpacked where it is used: a small
    // register footprint keeps enough rows in flight to cover the memory latency.
    uint4 xv[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * kWave;
        xv[j] = vi < nvec ? *reinterpret_cast<const uint4*>(xr + vi * 8) : make_uint4(0, 0, 0, 0);
    }
    const int64_t b = static_cast<int>(row) / static_cast<int>(tokens);   // rows < 2^31
    // precomputed shift and scale are loaded before the statistics, so their latency overlaps
    uint4 shr[NV], scr[NV];
    if (PRE) {
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int vi = lane + j * kWave;
            if (vi < nvec) {
                shr[j] = *reinterpret_cast<const uint4*>(shift_src + b * cols + vi * 8);
                scr[j] = *reinterpret_cast<const uint4*>(scale_src + b * cols + vi * 8);
            }
        }
    }
    float fmean, inv;
    {
        V8 v[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) v[j] = unpack_v8(xv[j]);
        row_stats<NV>(v, nvec, lane, cols, eps, &fmean, &inv);
    }
    bf16_t* orow = out + row * cols;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const int vi = lane + j * kWave;
        if (vi >= nvec) continue;
        const V8 xj = unpack_v8(xv[j]);
        V8 sh, sc;
        if (PRE) {
            sh = unpack_v8(shr[j]);
            sc = unpack_v8(scr[j]);
        } else {
            const V8 ms = load8(mod + b * mod_stride + (shift_src - mod) + vi * 8);
            const V8 mc = load8(mod + b * mod_stride + (scale_src - mod) + vi * 8);
            const V8 ts = load8(shift_tab + vi * 8);
            const V8 tc = load8(scale_tab + vi * 8);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                sh.f[e] = round_bf16(__fadd_rn(ms.f[e], ts.f[e]));
                sc.f[e] = round_bf16(__fadd_rn(mc.f[e], tc.f[e]));
            }
        }
        V8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            // normed is stored (rounded) by the norm op before modulate reads it.
            const float nrm = round_bf16(__fmul_rn(__fsub_rn(xj.f[e], fmean), inv));
            o.f[e] = __fadd_rn(__fmul_rn(nrm, __fadd_rn(1.0f, sc.f[e])), sh.f[e]);
        }
        store8(orow + vi * 8, o);
    }
}

// The engine's LayerNorm + modulate, every lane busy: a row of C = 512 NV + 128 NP channels is
// NV 16-byte vectors per lane (lane L holds vectors L, L+64, ...) plus NP 4-byte pairs per lane
// after them (C = 1152: two vectors and one pair, 18 channels per lane, where 16-byte vectors
// alone would leave three quarters of the lanes idle in the third vector). Shift and 1 + scale
// arrive as floats (k_chunk_all), so per channel the output costs only the oracle's own
// operations. One row per wave: all rows are in flight at once (a wave walking two rows with the
// next one prefetched measured slower), which needs at most 64 VGPRs a wave.

template <int NV, int NP>
struct NormRow {
    static constexpr int kE = NV * 8 + NP * 2;   // channels per lane
    uint32_t raw[kE / 2];
    __device__ __forceinline__ void load(const bf16_t* xr, int lane) {
        constexpr int pair0 = NV * 8 * kWave;
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const uint4 r = *reinterpret_cast<const uint4*>(xr + (lane + j * kWave) * 8);
            raw[4 * j] = r.x;
            raw[4 * j + 1] = r.y;
            raw[4 * j + 2] = r.z;
            raw[4 * j + 3] = r.w;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p)
            raw[4 * NV + p] = *reinterpret_cast<const uint32_t*>(xr + pair0 + (p * kWave + lane) * 2);
    }
};

template <int NV, int NP>
__global__ void __launch_bounds__(256) k_norm_mod_dense(
    const bf16_t* __restrict__ x, const float* __restrict__ shift, const float* __restrict__ scale1,
    bf16_t* __restrict__ out, int64_t rows, int64_t tokens, int cols, float eps,
    const uint32_t* __restrict__ warm, int64_t warm_lines) {
    using Row = NormRow<NV, NP>;
    constexpr int kE = Row::kE;
    constexpr int pair0 = NV * 8 * kWave;   // first channel of the pairs
    const int lane = threadIdx.x % kWave;
    // Workgroup i runs on XCD i % 8. With a grid of whole eighths, XCD x takes the x-th eighth of
    // the rows: the rows the GEMM before this norm wrote from that XCD's CUs (its tile order gives
    // XCD x the x-th eighth of the M-tiles) and the rows the GEMM after it reads there, so both
    // meet in that XCD's L2.
    int64_t wg = blockIdx.x;
    if ((gridDim.x & 7) == 0) wg = (wg & 7) * (gridDim.x >> 3) + (wg >> 3);
    const int64_t row = wg * (blockDim.x / kWave) + wave_index();
    if (row >= rows) return;
    Row cur;
    cur.load(x + row * cols, lane);
    const int64_t b = static_cast<int>(row) / static_cast<int>(tokens);   // rows < 2^31
    const float* shb = shift + b * cols;
    const float* scb = scale1 + b * cols;
    // The weights of the GEMM that reads this kernel's output: one 4-byte read per 128-byte line,
    // so that they are in the memory-side cache when that GEMM starts instead of meeting it cold
    // from HBM. Line lane * rows + row: the lines spread evenly over the rows (the first few lanes
    // of every wave); lanes past the range all read its last line. Issued after the row load (the
    // scheduling barrier keeps it there), so no wait for the row waits for it, and consumed only
    // after the stores, so its latency hides under the statistics.
    const uint32_t touched = warm[min(lane * rows + row, warm_lines - 1) * 32];
    __builtin_amdgcn_sched_barrier(0);
    // channel e of this lane, widened from the raw row where it is used (kept as bf16 pairs, the
    // row costs kE / 2 registers: few registers per wave keep every row of a SIMD in flight at once)
    auto val = [&](int e) -> float {
        const uint32_t w = cur.raw[e >> 1];
        return (e & 1) ? __uint_as_float(w & 0xffff0000u) : __uint_as_float(w << 16);
    };
    // The deviations' pass widens the row again: the empty asm makes the raw words opaque, so the
    // compiler cannot keep the mean pass's 2 kE fp64 registers alive for it (63 instead of 85
    // VGPRs at 1152 channels: eight waves per SIMD, every row of a SIMD in flight at once;
    // making the output pass re-widen too saves registers the occupancy no longer needs and
    // costs 18 instructions).
    auto reload = [&]() {
#pragma unroll
        for (int i = 0; i < kE / 2; ++i) asm volatile("" : "+v"(cur.raw[i]));
    };
    // statistics exactly as the oracle forms them: fp64 mean, fp64 sum of squared deviations
    double sum = 0.0;
#pragma unroll
    for (int e = 0; e < kE; ++e) sum += static_cast<double>(val(e));
    const double mean = wave_sum(sum) / static_cast<double>(cols);
    reload();
    double q = 0.0;
#pragma unroll
    for (int e = 0; e < kE; ++e) {
        const double d = static_cast<double>(val(e)) - mean;
        q += d * d;
    }
    const double var = wave_sum(q) / static_cast<double>(cols);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    const float fmean = static_cast<float>(mean);
    // normed is stored (rounded) by the norm op before modulate reads it: both values of a pair
    // rounded by one conversion, then widened back
    auto out2 = [&](int i, float s0, float s1, float c0, float c1) -> uint32_t {
        bf16x2_t nb;
        nb[0] = static_cast<__bf16>(__fmul_rn(__fsub_rn(val(2 * i), fmean), inv));
        nb[1] = static_cast<__bf16>(__fmul_rn(__fsub_rn(val(2 * i + 1), fmean), inv));
        const uint32_t nw = __builtin_bit_cast(uint32_t, nb);
        const float n0 = __uint_as_float(nw << 16), n1 = __uint_as_float(nw & 0xffff0000u);
        bf16x2_t rb;
        rb[0] = static_cast<__bf16>(__fadd_rn(__fmul_rn(n0, c0), s0));
        rb[1] = static_cast<__bf16>(__fadd_rn(__fmul_rn(n1, c1), s1));
        return __builtin_bit_cast(uint32_t, rb);
    };
    // Shift and 1 + scale are read per 16-byte vector of the row, after the statistics (the
    // scheduling barriers keep them there): 16 registers at a time instead of 4 kE.
    bf16_t* orow = out + row * cols;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        __builtin_amdgcn_sched_barrier(0);
        const int c = (lane + j * kWave) * 8;
        const float4 a0 = *reinterpret_cast<const float4*>(shb + c);
        const float4 a1 = *reinterpret_cast<const float4*>(shb + c + 4);
        const float4 m0 = *reinterpret_cast<const float4*>(scb + c);
        const float4 m1 = *reinterpret_cast<const float4*>(scb + c + 4);
        uint4 o;
        o.x = out2(4 * j, a0.x, a0.y, m0.x, m0.y);
        o.y = out2(4 * j + 1, a0.z, a0.w, m0.z, m0.w);
        o.z = out2(4 * j + 2, a1.x, a1.y, m1.x, m1.y);
        o.w = out2(4 * j + 3, a1.z, a1.w, m1.z, m1.w);
        *reinterpret_cast<uint4*>(orow + c) = o;
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
        __builtin_amdgcn_sched_barrier(0);
        const int c = pair0 + (p * kWave + lane) * 2;
        const float2 a = *reinterpret_cast<const float2*>(shb + c);
        const float2 m = *reinterpret_cast<const float2*>(scb + c);
        *reinterpret_cast<uint32_t*>(orow + c) = out2(4 * NV + p, a.x, a.y, m.x, m.y);
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::"v"(touched));
}

// LayerNorm / RMSNorm (NormArgs) in the same lane-dense layout (C = 512 NV + 128 NP channels: NV
// 16-byte vectors and NP 4-byte pairs per lane), for widths the 16-byte-vector kernel would run
// with idle lanes (C = 1152: 18 channels in every lane instead of 24 slots in three quarters of
// them). Optional affine weight and bias in the same layout. The arithmetic is k_norm_rows' own.
template <int NV, int NP>
__global__ void __launch_bounds__(256) k_norm_dense(const bf16_t* __restrict__ x,
                                                    const bf16_t* __restrict__ w,
                                                    const bf16_t* __restrict__ b,
                                                    bf16_t* __restrict__ out, int64_t rows, int cols,
                                                    float eps, bool rms) {
    using Row = NormRow<NV, NP>;
    constexpr int kE = Row::kE;
    constexpr int pair0 = NV * 8 * kWave;
    const int lane = threadIdx.x % kWave;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (blockDim.x / kWave) + wave_index();
    if (row >= rows) return;
    Row cur, wr, br;
    cur.load(x + row * cols, lane);
    if (w) wr.load(w, lane);
    if (b) br.load(b, lane);
    float v[kE];
#pragma unroll
    for (int i = 0; i < kE / 2; ++i) {
        v[2 * i] = __uint_as_float(cur.raw[i] << 16);
        v[2 * i + 1] = __uint_as_float(cur.raw[i] & 0xffff0000u);
    }
    double mean = 0.0;
    if (!rms) {
        double sum = 0.0;
#pragma unroll
        for (int e = 0; e < kE; ++e) sum += static_cast<double>(v[e]);
        mean = wave_sum(sum) / static_cast<double>(cols);
    }
    double q = 0.0;
#pragma unroll
    for (int e = 0; e < kE; ++e) {
        const double d = static_cast<double>(v[e]) - mean;
        q += d * d;
    }
    const double var = wave_sum(q) / static_cast<double>(cols);
    const float inv = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    const float fmean = static_cast<float>(mean);
    uint32_t o[kE / 2];
#pragma unroll
    for (int i = 0; i < kE / 2; ++i) {
        float t[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            t[h] = __fmul_rn(__fsub_rn(v[2 * i + h], fmean), inv);
            if (w) t[h] = __fmul_rn(t[h], __uint_as_float(h ? wr.raw[i] & 0xffff0000u : wr.raw[i] << 16));
            if (b) t[h] = __fadd_rn(t[h], __uint_as_float(h ? br.raw[i] & 0xffff0000u : br.raw[i] << 16));
        }
        bf16x2_t r;
        r[0] = static_cast<__bf16>(t[0]);
        r[1] = static_cast<__bf16>(t[1]);
        o[i] = __builtin_bit_cast(uint32_t, r);
    }
    bf16_t* orow = out + row * cols;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        *reinterpret_cast<uint4*>(orow + (lane + j * kWave) * 8) =
            make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
#pragma unroll
    for (int p = 0; p < NP; ++p)
        *reinterpret_cast<uint32_t*>(orow + pair0 + (p * kWave + lane) * 2) = o[4 * NV + p];
}

// ---- modulate (ModulateArgs) ----------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(256) k_modulate(const T* __restrict__ x, const T* __restrict__ scale,
                                                  const T* __restrict__ shift, T* out, int64_t n,
                                                  int64_t tokens, int64_t channels,
                                                  const T* residual, const T* __restrict__ gate) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = i % channels;
        const int64_t bc = (i / (tokens * channels)) * channels + c;
        float v = Io<T>::ld(x, i);
        v = __fadd_rn(__fmul_rn(v, __fadd_rn(1.0f, Io<T>::ld(scale, bc))), Io<T>::ld(shift, bc));
        if (gate) v = __fmul_rn(v, Io<T>::ld(gate, bc));
        if (residual) v = __fadd_rn(v, Io<T>::ld(residual, i));
        Io<T>::st(out, i, v);
    }
}

// bf16, channels % 8 == 0: 8 elements of one (b, token) row per thread. I is the index type:
// 32-bit whenever the tensor has fewer than 2^31 vectors (the divisions by the row and batch
// lengths are then 32-bit).
template <typename I>
__global__ void __launch_bounds__(256) k_modulate_v8(const bf16_t* __restrict__ x,
                                                     const bf16_t* __restrict__ scale,
                                                     const bf16_t* __restrict__ shift, bf16_t* out,
                                                     I nvec, I tokens, I channels,
                                                     const bf16_t* residual,
                                                     const bf16_t* __restrict__ gate) {
    const I cv = channels / 8, bv = tokens * cv;
    for (I i = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; i < nvec;
         i += static_cast<I>(gridDim.x) * blockDim.x) {
        const I c = (i % cv) * 8;
        const I bc = (i / bv) * channels + c;
        const V8 xv = load8(x + i * 8), sc = load8(scale + bc), sh = load8(shift + bc);
        V8 g, r, o;
        if (gate) g = load8(gate + bc);
        if (residual) r = load8(residual + i * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = __fadd_rn(__fmul_rn(xv.f[e], __fadd_rn(1.0f, sc.f[e])), sh.f[e]);
            if (gate) v = __fmul_rn(v, g.f[e]);
            if (residual) v = __fadd_rn(v, r.f[e]);
            o.f[e] = v;
        }
        store8(out + i * 8, o);
    }
}

// ---- add, chunk, activation -----------------------------------------------------------------

template <typename T>
__global__ void __launch_bounds__(256) k_add(const T* a, const T* __restrict__ b, T* out,
                                             int64_t n, int64_t inner, float scale,
                                             bool broadcast) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t bi = broadcast ? (i % inner) : i;
        Io<T>::st(out, i, __fadd_rn(Io<T>::ld(a, i), __fmul_rn(scale, Io<T>::ld(b, bi))));
    }
}

// bf16, n and inner multiples of 8, every operand 16-byte aligned: 8 elements per thread (a may
// alias out: each thread reads its vector before writing it).
template <typename I>
__global__ void __launch_bounds__(256) k_add_v8(const bf16_t* a, const bf16_t* __restrict__ b,
                                                bf16_t* out, I nvec, I inner_vec, float scale,
                                                bool broadcast) {
    for (I i = blockIdx.x * static_cast<I>(blockDim.x) + threadIdx.x; i < nvec;
         i += static_cast<I>(gridDim.x) * blockDim.x) {
        const I bi = broadcast ? i % inner_vec : i;
        const V8 av = load8(a + static_cast<int64_t>(i) * 8), bv = load8(b + static_cast<int64_t>(bi) * 8);
        V8 o;
#pragma unroll
        for (int e = 0; e < 8; ++e) o.f[e] = __fadd_rn(av.f[e], __fmul_rn(scale, bv.f[e]));
        store8(out + static_cast<int64_t>(i) * 8, o);
    }
}

template <typename T>
__global__ void k_chunk(const T* __restrict__ mod, const T* __restrict__ table, T* __restrict__ out,
                        int64_t batch, int64_t channels, int64_t chunks, int64_t chunk,
                        int64_t trow) {
    const int64_t n = batch * channels;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t b = i / channels, c = i % channels;
        Io<T>::st(out, i, __fadd_rn(Io<T>::ld(mod, b * chunks * channels + chunk * channels + c),
                                    Io<T>::ld(table, trow * channels + c)));
    }
}

// `out_f32` (optional) receives the same chunks as floats for the fused norm kernel, with the
// scale chunks (1 and 4) already in the form the modulation multiplies by, 1 + scale (the same
// fp32 addition the modulation would do per element).
__global__ void k_chunk_all(const bf16_t* __restrict__ mod, const bf16_t* const* __restrict__ tables,
                            bf16_t* __restrict__ out, float* __restrict__ out_f32, int64_t layers,
                            int64_t batch, int64_t channels) {
    const int64_t per_layer = 6 * batch * channels;
    const int64_t n = layers * per_layer;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t l = i / per_layer, r = i % per_layer;
        const int64_t k = r / (batch * channels), b = (r / channels) % batch, c = r % channels;
        const float v = __fadd_rn(bf2f(mod[b * 6 * channels + k * channels + c]),
                                  bf2f(tables[l][k * channels + c]));
        out[i] = f2bf(v);
        if (out_f32) out_f32[i] = (k == 1 || k == 4) ? __fadd_rn(1.0f, round_bf16(v)) : round_bf16(v);
    }
}

__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    const float x3 = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fmul_rn(c, __fadd_rn(x, __fmul_rn(0.044715f, x3)));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}
__device__ __forceinline__ float silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x))); }

template <typename T>
__global__ void __launch_bounds__(256) k_activation(const T* __restrict__ x, T* __restrict__ out,
                                                    int64_t n, int kind,
                                                    const T* __restrict__ gate) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const float v = Io<T>::ld(x, i);
        float r = (kind == 2) ? silu(v) : (kind == 0 ? v : gelu_tanh(v));
        if (kind == 3) r = __fmul_rn(r, Io<T>::ld(gate, i));
        Io<T>::st(out, i, r);
    }
}

// out[r, j] = round(gelu_tanh(in[r, j]) * in[r, F + j]): the two halves of a fused wi_0/wi_1
// projection, each already a stored bf16 as in the reference's two GEMM outputs.
__global__ void __launch_bounds__(256) k_gelu_gated_rows(const bf16_t* __restrict__ in,
                                                         bf16_t* __restrict__ out, int64_t rows,
                                                         int64_t F) {
    if (F % 8 == 0) {   // 16-byte vectors (the launcher checks alignment)
        const int64_t per = F / 8, n = rows * per;
        for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
             i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
            const int64_t r = i / per, j = (i - r * per) * 8;
            const bf16_t* row = in + r * 2 * F;
            const V8 h0 = load8(row + j), h1 = load8(row + F + j);
            V8 o;
#pragma unroll
            for (int e = 0; e < 8; ++e) o.f[e] = __fmul_rn(gelu_tanh(h0.f[e]), h1.f[e]);
            store8(out + r * F + j, o);
        }
        return;
    }
    const int64_t n = rows * F;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = i / F, j = i - r * F;
        const bf16_t* row = in + r * 2 * F;
        out[i] = f2bf(__fmul_rn(gelu_tanh(bf2f(row[j])), bf2f(row[F + j])));
    }
}

// ---- patchify / unpatchify ------------------------------------------------------------------

// One thread per token element. Forward: token layout (c, ky, kx); inverse: (ky, kx, c).
template <typename T>
__global__ void __launch_bounds__(256) k_patch(const T* __restrict__ in, T* __restrict__ out,
                                               int64_t batch, int64_t C, int64_t G, int64_t P,
                                               bool inverse) {
    const int64_t per_token = C * P * P;
    const int64_t n = batch * G * G * per_token;
    const int64_t H = G * P;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t e = i % per_token;
        const int64_t tok = (i / per_token) % (G * G);
        const int64_t b = i / (per_token * G * G);
        int64_t c, ky, kx;
        if (inverse) {
            c = e % C;
            kx = (e / C) % P;
            ky = e / (C * P);
        } else {
            kx = e % P;
            ky = (e / P) % P;
            c = e / (P * P);
        }
        const int64_t ty = tok / G, tx = tok % G;
        const int64_t img = ((b * C + c) * H + ty * P + ky) * H + tx * P + kx;
        if (inverse) out[img] = in[i];
        else out[i] = in[img];
    }
}

// ---- timestep embedding ---------------------------------------------------------------------

// cos first, then sin (weights.cpp:107-121), each computed in fp64 and stored as the reference
// stores it: Tensor::set(static_cast<float>(v)), i.e. rounded to float and then through the
// storage type; the row is repeated `batch` times.
__device__ inline void store_f64(float* p, int64_t i, double v) { p[i] = static_cast<float>(v); }
__device__ inline void store_f64(bf16_t* p, int64_t i, double v) { p[i] = bf16_from_f64(v); }

template <typename T>
__global__ void k_timestep_embedding(double t, int dim, int64_t batch, T* out) {
    const int half = dim / 2;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const double freq = exp(-log(10000.0) * static_cast<double>(i) / half);
        const double a = t * freq;
        const double c = cos(a), s = sin(a);
        for (int64_t b = 0; b < batch; ++b) {
            store_f64(out, b * dim + i, c);
            store_f64(out, b * dim + half + i, s);
        }
    }
}

// ScaleArgs (ops_cpu.cpp:351-353): one multiply per element, one rounding at the store.
template <typename T>
__global__ void __launch_bounds__(256) k_scale(const T* in, T* out, int64_t n, float scale) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        Io<T>::st(out, i, __fmul_rn(Io<T>::ld(in, i), scale));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int grid_for(int64_t n, int block = 256) {
    const int64_t g = (n + block - 1) / block;
    return static_cast<int>(g < 1 ? 1 : (g > 65535 * 8 ? 65535 * 8 : g));
}

}  // namespace

void launch_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                 int64_t cols, float eps, bool rms, bool f32, hipStream_t s) {
    if (rows == 0) return;
    const int grid = static_cast<int>((rows + 3) / 4);
    if (f32) {
        k_norm<float><<<grid, 256, 0, s>>>(static_cast<const float*>(x),
                                           static_cast<const float*>(weight),
                                           static_cast<const float*>(bias),
                                           static_cast<float*>(out), rows, cols, eps, rms);
    } else {
        const bool vec = cols % 8 == 0 && cols <= 8192 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(weight) & 15) == 0 &&
                         (reinterpret_cast<uintptr_t>(bias) & 15) == 0;
        if (vec) {
            const auto* xb = static_cast<const bf16_t*>(x);
            const auto* wb = static_cast<const bf16_t*>(weight);
            const auto* bb = static_cast<const bf16_t*>(bias);
            auto* ob = static_cast<bf16_t*>(out);
            const int nv = static_cast<int>(cols / 512), np = static_cast<int>(cols % 512 / 128);
            if (cols % 128 == 0 && np > 0 && nv <= 3) {   // lanes the vector kernel would leave idle
                const int c = static_cast<int>(cols);
#define BH_NDN(NV, NP) k_norm_dense<NV, NP><<<grid, 256, 0, s>>>(xb, wb, bb, ob, rows, c, eps, rms)
                switch (nv * 4 + np) {
                    case 1: BH_NDN(0, 1); break;
                    case 2: BH_NDN(0, 2); break;
                    case 3: BH_NDN(0, 3); break;
                    case 5: BH_NDN(1, 1); break;
                    case 6: BH_NDN(1, 2); break;
                    case 7: BH_NDN(1, 3); break;
                    case 9: BH_NDN(2, 1); break;
                    case 10: BH_NDN(2, 2); break;
                    case 11: BH_NDN(2, 3); break;
                    case 13: BH_NDN(3, 1); break;
                    case 14: BH_NDN(3, 2); break;
                    default: BH_NDN(3, 3); break;
                }
#undef BH_NDN
                launch_check("norm");
                return;
            }
            if (cols <= 1024) k_norm_rows<2><<<grid, 256, 0, s>>>(xb, wb, bb, ob, rows, cols, eps, rms);
            else if (cols <= 2048) k_norm_rows<4><<<grid, 256, 0, s>>>(xb, wb, bb, ob, rows, cols, eps, rms);
            else if (cols <= 4096) k_norm_rows<8><<<grid, 256, 0, s>>>(xb, wb, bb, ob, rows, cols, eps, rms);
            else k_norm_rows<16><<<grid, 256, 0, s>>>(xb, wb, bb, ob, rows, cols, eps, rms);
            launch_check("norm");
            return;
        }
        k_norm<bf16_t><<<grid, 256, 0, s>>>(static_cast<const bf16_t*>(x),
                                            static_cast<const bf16_t*>(weight),
                                            static_cast<const bf16_t*>(bias),
                                            static_cast<bf16_t*>(out), rows, cols, eps, rms);
    }
    launch_check("norm");
}

namespace {
template <bool PRE>
void dispatch_norm_modulate(const bf16_t* x, const bf16_t* mod, int64_t mod_stride,
                            const bf16_t* shift_src, const bf16_t* scale_src,
                            const bf16_t* shift_tab, const bf16_t* scale_tab, bf16_t* out,
                            int64_t rows, int64_t tokens, int64_t cols, float eps, hipStream_t s) {
    require(cols % 8 == 0 && cols <= 8 * kWave * 8,
            "norm_modulate: channels must be a multiple of 8 and at most 4096");
    require(aligned16(x) && aligned16(out) && aligned16(mod) && aligned16(shift_src) &&
                aligned16(scale_src) && aligned16(shift_tab) && aligned16(scale_tab),
            "norm_modulate: every operand must be 16-byte aligned");
    require(rows < (int64_t{1} << 31), "norm_modulate: 2^31 rows or more");
    const int nv = static_cast<int>((cols / 8 + kWave - 1) / kWave);
    const int grid = static_cast<int>((rows + 3) / 4);
#define BH_NM(NV)                                                                             \
    k_norm_modulate<NV, PRE><<<grid, 256, 0, s>>>(x, mod, mod_stride, shift_src, scale_src,   \
                                                  shift_tab, scale_tab, out, rows, tokens,    \
                                                  cols, eps)
    switch (nv) {
        case 1: BH_NM(1); break;
        case 2: BH_NM(2); break;
        case 3: BH_NM(3); break;
        case 4: BH_NM(4); break;
        case 5: BH_NM(5); break;
        case 6: BH_NM(6); break;
        case 7: BH_NM(7); break;
        default: BH_NM(8); break;
    }
#undef BH_NM
    launch_check("norm_modulate");
}
}  // namespace

void launch_norm_modulate(const bf16_t* x, const bf16_t* mod, int64_t mod_chunks,
                          int64_t shift_chunk, int64_t scale_chunk, const bf16_t* table,
                          int64_t shift_row, int64_t scale_row, bf16_t* out, int64_t batch,
                          int64_t tokens, int64_t channels, float eps, hipStream_t s) {
    if (batch * tokens == 0) return;
    dispatch_norm_modulate<false>(x, mod, mod_chunks * channels, mod + shift_chunk * channels,
                                  mod + scale_chunk * channels, table + shift_row * channels,
                                  table + scale_row * channels, out, batch * tokens, tokens,
                                  channels, eps, s);
}

void launch_norm_modulate_pre(const bf16_t* x, const bf16_t* shift, const bf16_t* scale,
                              bf16_t* out, int64_t batch, int64_t tokens, int64_t channels,
                              float eps, hipStream_t s) {
    if (batch * tokens == 0) return;
    dispatch_norm_modulate<true>(x, nullptr, 0, shift, scale, nullptr, nullptr, out,
                                 batch * tokens, tokens, channels, eps, s);
}

void launch_norm_modulate_f32(const bf16_t* x, const float* shift, const float* scale1,
                              bf16_t* out, int64_t batch, int64_t tokens, int64_t channels,
                              float eps, hipStream_t s, const void* warm, int64_t warm_bytes) {
    const int64_t rows = batch * tokens;
    if (rows == 0) return;
    require(norm_modulate_f32_supported(channels),
            "norm_modulate_f32: channels must be a multiple of 128 and at most 4096");
    require(aligned16(x) && aligned16(out) && aligned16(shift) && aligned16(scale1),
            "norm_modulate_f32: every operand must be 16-byte aligned");
    require(rows < (int64_t{1} << 31), "norm_modulate_f32: 2^31 rows or more");
    const int nv = static_cast<int>(channels / 512), np = static_cast<int>(channels % 512 / 128);
    const int grid = static_cast<int>((rows + 3) / 4);
    const int c = static_cast<int>(channels);
    // the 128-byte lines the warm range touches (its first one starts at or before it, inside the
    // same allocation, whose base is aligned further), at most one per lane of the launch; with
    // no range, every lane reads the first 4 bytes of x (the kernel's read is unconditional)
    const uintptr_t w0 = reinterpret_cast<uintptr_t>(warm) & ~uintptr_t{127};
    const bool warm_ok = warm && warm_bytes > 0;
    const int64_t warm_lines =
        warm_ok ? std::min<int64_t>((reinterpret_cast<uintptr_t>(warm) + warm_bytes - w0 + 127) / 128,
                                    rows * kWave)
                : 1;
    const uint32_t* wl = warm_ok ? reinterpret_cast<const uint32_t*>(w0) : reinterpret_cast<const uint32_t*>(x);
#define BH_ND(NV, NP)                                                                         \
    k_norm_mod_dense<NV, NP><<<grid, 256, 0, s>>>(x, shift, scale1, out, rows, tokens, c, eps, \
                                                  wl, warm_lines)
    switch (nv * 4 + np) {
#define BH_NV(NV) \
        case NV * 4 + 0: BH_ND(NV, 0); break; \
        case NV * 4 + 1: BH_ND(NV, 1); break; \
        case NV * 4 + 2: BH_ND(NV, 2); break; \
        case NV * 4 + 3: BH_ND(NV, 3); break;
        case 1: BH_ND(0, 1); break;
        case 2: BH_ND(0, 2); break;
        case 3: BH_ND(0, 3); break;
        BH_NV(1) BH_NV(2) BH_NV(3) BH_NV(4) BH_NV(5) BH_NV(6) BH_NV(7)
        default: BH_ND(8, 0); break;
#undef BH_NV
    }
#undef BH_ND
    launch_check("norm_modulate_f32");
}

bool norm_modulate_f32_supported(int64_t channels) {
    return channels > 0 && channels % 128 == 0 && channels <= 4096;
}

void launch_modulate(const void* x, const void* scale, const void* shift, void* out,
                     int64_t batch, int64_t tokens, int64_t channels, const void* residual,
                     const void* gate, bool f32, hipStream_t s) {
    const int64_t n = batch * tokens * channels;
    if (n == 0) return;
    if (f32) {
        k_modulate<float><<<grid_for(n), 256, 0, s>>>(
            static_cast<const float*>(x), static_cast<const float*>(scale),
            static_cast<const float*>(shift), static_cast<float*>(out), n, tokens, channels,
            static_cast<const float*>(residual), static_cast<const float*>(gate));
    } else if (channels % 8 == 0 && aligned16(x) && aligned16(scale) && aligned16(shift) &&
               aligned16(out) && aligned16(residual) && aligned16(gate)) {
        // 32-bit indices while every element offset (i * 8 < n) fits in 32 bits
        if (n < (int64_t{1} << 32))
            k_modulate_v8<uint32_t><<<grid_for(n / 8), 256, 0, s>>>(
                static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(scale),
                static_cast<const bf16_t*>(shift), static_cast<bf16_t*>(out),
                static_cast<uint32_t>(n / 8), static_cast<uint32_t>(tokens),
                static_cast<uint32_t>(channels), static_cast<const bf16_t*>(residual),
                static_cast<const bf16_t*>(gate));
        else
            k_modulate_v8<int64_t><<<grid_for(n / 8), 256, 0, s>>>(
                static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(scale),
                static_cast<const bf16_t*>(shift), static_cast<bf16_t*>(out), n / 8, tokens,
                channels, static_cast<const bf16_t*>(residual), static_cast<const bf16_t*>(gate));
    } else {
        k_modulate<bf16_t><<<grid_for(n), 256, 0, s>>>(
            static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(scale),
            static_cast<const bf16_t*>(shift), static_cast<bf16_t*>(out), n, tokens, channels,
            static_cast<const bf16_t*>(residual), static_cast<const bf16_t*>(gate));
    }
    launch_check("modulate");
}

void launch_activation(const void* x, void* out, int64_t numel, int kind, const void* gate,
                       bool f32, hipStream_t s) {
    if (numel == 0) return;
    if (f32) {
        k_activation<float><<<grid_for(numel), 256, 0, s>>>(
            static_cast<const float*>(x), static_cast<float*>(out), numel, kind,
            static_cast<const float*>(gate));
    } else {
        k_activation<bf16_t><<<grid_for(numel), 256, 0, s>>>(
            static_cast<const bf16_t*>(x), static_cast<bf16_t*>(out), numel, kind,
            static_cast<const bf16_t*>(gate));
    }
    launch_check("activation");
}

void launch_gelu_gated_rows(const bf16_t* in, bf16_t* out, int64_t rows, int64_t F, hipStream_t s) {
    if (rows * F == 0) return;
    ProfileScope ps(K_ELEMENTWISE, s, 6.0 * rows * F);
    const bool vec = F % 8 == 0 && (reinterpret_cast<uintptr_t>(in) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    // the kernel takes the vector path whenever F % 8 == 0, which needs 16-byte aligned rows
    require(vec || F % 8 != 0, "gated gelu: 16-byte aligned rows expected");
    k_gelu_gated_rows<<<grid_for(vec ? rows * F / 8 : rows * F), 256, 0, s>>>(in, out, rows, F);
    launch_check("gated gelu");
}

void launch_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner,
                float scale, bool broadcast_b, bool f32, hipStream_t s) {
    const int64_t n = outer * inner;
    if (n == 0) return;
    if (f32) {
        k_add<float><<<grid_for(n), 256, 0, s>>>(static_cast<const float*>(a),
                                                 static_cast<const float*>(b),
                                                 static_cast<float*>(out), n, inner, scale,
                                                 broadcast_b);
    } else if (n % 8 == 0 && inner % 8 == 0 && aligned16(a) && aligned16(b) && aligned16(out)) {
        if (n / 8 < (int64_t{1} << 31))
            k_add_v8<uint32_t><<<grid_for(n / 8), 256, 0, s>>>(
                static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                static_cast<bf16_t*>(out), static_cast<uint32_t>(n / 8),
                static_cast<uint32_t>(inner / 8), scale, broadcast_b);
        else
            k_add_v8<int64_t><<<grid_for(n / 8), 256, 0, s>>>(
                static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                static_cast<bf16_t*>(out), n / 8, inner / 8, scale, broadcast_b);
    } else {
        k_add<bf16_t><<<grid_for(n), 256, 0, s>>>(static_cast<const bf16_t*>(a),
                                                  static_cast<const bf16_t*>(b),
                                                  static_cast<bf16_t*>(out), n, inner, scale,
                                                  broadcast_b);
    }
    launch_check("add");
}

void launch_chunk(const void* mod, const void* table, void* out, int64_t batch, int64_t channels,
                  int64_t chunks, int64_t chunk, int64_t table_chunk, bool f32, hipStream_t s) {
    const int64_t n = batch * channels;
    if (n == 0) return;
    const int64_t trow = table_chunk >= 0 ? table_chunk : chunk;
    if (f32) {
        k_chunk<float><<<grid_for(n), 256, 0, s>>>(static_cast<const float*>(mod),
                                                   static_cast<const float*>(table),
                                                   static_cast<float*>(out), batch, channels,
                                                   chunks, chunk, trow);
    } else {
        k_chunk<bf16_t><<<grid_for(n), 256, 0, s>>>(static_cast<const bf16_t*>(mod),
                                                    static_cast<const bf16_t*>(table),
                                                    static_cast<bf16_t*>(out), batch, channels,
                                                    chunks, chunk, trow);
    }
    launch_check("chunk");
}

void launch_chunk_all(const bf16_t* mod, const bf16_t* const* tables_dev, bf16_t* out,
                      float* out_f32, int64_t layers, int64_t batch, int64_t channels,
                      hipStream_t s) {
    const int64_t n = layers * 6 * batch * channels;
    if (n == 0) return;
    k_chunk_all<<<grid_for(n), 256, 0, s>>>(mod, tables_dev, out, out_f32, layers, batch, channels);
    launch_check("chunk_all");
}

void launch_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
                  int64_t patch, bool inverse, bool f32, hipStream_t s) {
    const int64_t n = batch * grid * grid * channels * patch * patch;
    if (n == 0) return;
    if (f32) {
        k_patch<float><<<grid_for(n), 256, 0, s>>>(static_cast<const float*>(in),
                                                   static_cast<float*>(out), batch, channels,
                                                   grid, patch, inverse);
    } else {
        k_patch<bf16_t><<<grid_for(n), 256, 0, s>>>(static_cast<const bf16_t*>(in),
                                                    static_cast<bf16_t*>(out), batch, channels,
                                                    grid, patch, inverse);
    }
    launch_check("patch");
}

void launch_scale(const void* in, void* out, int64_t n, float scale, bool f32, hipStream_t s) {
    if (n == 0) return;
    const int grid = grid_for(n);
    if (f32) k_scale<float><<<grid, 256, 0, s>>>(static_cast<const float*>(in), static_cast<float*>(out), n, scale);
    else k_scale<bf16_t><<<grid, 256, 0, s>>>(static_cast<const bf16_t*>(in), static_cast<bf16_t*>(out), n, scale);
    launch_check("scale");
}

void launch_timestep_embedding(double t, int dim, int64_t batch, void* out, bool f32, hipStream_t s) {
    require(dim > 0 && dim % 2 == 0, "timestep embedding needs an even dimension");
    if (f32) k_timestep_embedding<float><<<1, 128, 0, s>>>(t, dim, batch, static_cast<float*>(out));
    else k_timestep_embedding<bf16_t><<<1, 128, 0, s>>>(t, dim, batch, static_cast<bf16_t*>(out));
    launch_check("timestep_embedding");
}

}  // namespace bh
