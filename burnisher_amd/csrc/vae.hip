// Kernels of the VAE decoder (the vae-decode stage, reference src/models/vae_decoder.cpp) on
// gfx950. The decoder engine (vae_engine.cpp) keeps activations channels-last, [pixels, channels]
// bf16, so that a 3x3 convolution is an implicit GEMM (gemm.hip, launch_conv3x3_bf16) and the
// mid-block attention reads its tokens in place. This file holds what is not a GEMM:
//   - k_transpose       [R, C] -> [C, R] per batch: NCHW <-> NHWC at the stage's two ends, and
//                       the reference's TransposeArgs op (ops.h:184-191);
//   - GroupNorm         two deterministic fp64 passes (sum, then squared deviations) over
//                       per-chunk partials, then one pass that normalises, applies the affine
//                       and, optionally, SiLU (the reference's norm then activation, each rounded
//                       to bf16 as the reference stores them, ops_cpu.cpp:186-224, 265-274; the
//                       SiLU with the hardware exp2 and reciprocal, within one bf16 ulp);
//   - k_conv_direct     a convolution in the reference's summation order, for the layers too thin
//                       for the MFMA tile (conv_in: 4 input channels; conv_out: 3 outputs);
//   - k_upsample_nchw   the reference's UpsampleArgs op (the engine fuses the upsample into the
//                       next convolution's gather instead);
//   - k_vt512, k_flash512  the mid-block's single-head, head_dim-512 attention.
#include "common.h"

#include <algorithm>
#include <cmath>
#include <mutex>

namespace bh {
namespace {

// ---- [R, C] -> [C, R] per batch --------------------------------------------------------------

__global__ void __launch_bounds__(256) k_transpose(const bf16_t* __restrict__ in, bf16_t* __restrict__ out,
                                                   int64_t R, int64_t C, int64_t keep) {
    __shared__ bf16_t tile[32][33];
    const int64_t b = blockIdx.z;
    in += b * R * C;
    out += b * R * keep;
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 32, c0 = static_cast<int64_t>(blockIdx.x) * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int i = ty; i < 32; i += 8) {
        const int64_t r = r0 + i, c = c0 + tx;
        if (r < R && c < C) tile[i][tx] = in[r * C + c];
    }
    __syncthreads();
#pragma unroll
    for (int i = ty; i < 32; i += 8) {
        const int64_t c = c0 + i, r = r0 + tx;
        if (c < keep && r < R) out[c * R + r] = tile[tx][i];
    }
}

// ---- GroupNorm over [pixels, C] --------------------------------------------------------------
//
// A workgroup owns a chunk of pixels; thread t holds channel octet t % (C/8) of pixels
// t / (C/8), t / (C/8) + 256/(C/8), ... and sums its eight channels in fp64; the workgroup then
// sums each group's channels and rows in a fixed order into part[chunk][group]. Pass 0 sums x,
// pass 1 sums (x - mean[group])^2. Sums of bf16 values in fp64 are exact up to 2^45 times the
// smallest term's ulp, so the group mean does not depend on the order; the squared deviations
// round at the last fp64 bit, far below the float they are converted to.
constexpr int kGnThreads = 256;

__global__ void __launch_bounds__(kGnThreads) k_gn_partial(const bf16_t* __restrict__ x, int64_t S,
                                                         int C, int G, int64_t px_per_chunk,
                                                         const double* __restrict__ mean,
                                                         double* __restrict__ part) {
    __shared__ double red[kGnThreads][9];
    const int oct = C / 8, per_row = kGnThreads / oct;   // C/8 divides 256 (checked by the host)
    const int t = threadIdx.x, o = t % oct, prow = t / oct;
    const int cpg = C / G;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * px_per_chunk;
    const int64_t p1 = min(S, p0 + px_per_chunk);
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    double mu[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) mu[q] = mean ? mean[(o * 8 + q) / cpg] : 0.0;
    for (int64_t p = p0 + prow; p < p1; p += per_row) {
        const uint4 raw = *reinterpret_cast<const uint4*>(x + p * C + o * 8);
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float v = __uint_as_float(q & 1 ? (w4[q >> 1] & 0xffff0000u) : (w4[q >> 1] << 16));
            if (mean) {
                const double d = static_cast<double>(v) - mu[q];
                acc[q] += d * d;
            } else {
                acc[q] += static_cast<double>(v);
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) red[t][q] = acc[q];
    __syncthreads();
    if (t < G) {
        double s = 0.0;
        for (int r = 0; r < per_row; ++r)
            for (int c = t * cpg; c < (t + 1) * cpg; ++c) s += red[r * oct + c / 8][c % 8];
        part[static_cast<int64_t>(blockIdx.x) * G + t] = s;
    }
}

// Pass 0: mean[g] = sum / n. Pass 1: var = sum / n, inv[g] = 1 / sqrt(float(var) + eps), the
// reference's rounding (ops_cpu.cpp:208-210). One workgroup per group: thread t sums chunks t,
// t + 256, ... in order, then a fixed pairwise tree over the 256 threads, so the result is the same
// on every run.
__global__ void __launch_bounds__(256) k_gn_finalize(const double* __restrict__ part, int chunks, int G,
                                                     double n, int pass, float eps,
                                                     double* __restrict__ mean, float* __restrict__ inv) {
    __shared__ double red[256];
    const int g = blockIdx.x, t = threadIdx.x;
    double s = 0.0;
    for (int c = t; c < chunks; c += 256) s += part[static_cast<int64_t>(c) * G + g];
    red[t] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w) red[t] += red[t + w];
        __syncthreads();
    }
    if (t != 0) return;
    if (pass == 0) {
        mean[g] = red[0] / n;
    } else {
        const double var = red[0] / n;
        inv[g] = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(static_cast<float>(var), eps)));
    }
}

// SiLU with the hardware exp2 and reciprocal: a few fp32 ulps from x / (1 + exp(-x)), which moves
// the bf16 value it is rounded to by at most one ulp (the same bound as a device expf).
__device__ __forceinline__ float silu_hw(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// (x - float(mean)) * inv, * weight[c], + bias[c] (separate roundings, the reference's order),
// rounded to bf16; with SILU, SiLU of that bf16 value, rounded again. In place is allowed (each
// element is read before it is written by the same thread). The grid stride is a multiple of 256
// and C/8 divides 256, so a thread always sees the same eight channels: their statistics and
// affine are read once, before the loop.
template <bool W, bool B, bool SILU>
__global__ void __launch_bounds__(256) k_gn_apply(const bf16_t* x, bf16_t* out, int64_t S, int C, int G,
                                                  const double* __restrict__ mean,
                                                  const float* __restrict__ inv,
                                                  const bf16_t* __restrict__ w,
                                                  const bf16_t* __restrict__ b) {
    const int oct = C / 8, cpg = C / G;
    const int64_t n = S * oct;
    const int64_t first = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int c0 = static_cast<int>(first % oct) * 8;
    float mf[8], iv[8], wv[8], bv[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int c = c0 + q, g = c / cpg;
        mf[q] = static_cast<float>(mean[g]);
        iv[q] = inv[g];
        wv[q] = W ? bf2f(w[c]) : 1.0f;
        bv[q] = B ? bf2f(b[c]) : 0.0f;
    }
    const uint4* src = reinterpret_cast<const uint4*>(x);
    uint4* dst = reinterpret_cast<uint4*>(out);
    for (int64_t i = first; i < n; i += stride) {
        const uint4 raw = src[i];
        const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
        uint32_t r4[4];
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
            float v2[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int q = 2 * q2 + h;
                const float xv = __uint_as_float(h ? (w4[q2] & 0xffff0000u) : (w4[q2] << 16));
                float v = __fmul_rn(__fsub_rn(xv, mf[q]), iv[q]);
                if (W) v = __fmul_rn(v, wv[q]);
                if (B) v = __fadd_rn(v, bv[q]);
                if (SILU) v = silu_hw(round_bf16(v));
                v2[h] = v;
            }
            r4[q2] = f2bf2(v2[0], v2[1]);
        }
        dst[i] = make_uint4(r4[0], r4[1], r4[2], r4[3]);
    }
}

// ---- direct convolution, channels-last, the reference's summation order ------------------------
//
// out[p, co] = bias[co] + sum over ci, ky, kx (in that order, taps outside the image skipped) of
// x[p + (ky - pad, kx - pad), ci] * w[co, ci, ky, kx], fp32 with separate multiply and add: the
// same operation sequence as conv2d_cpu (ops_cpu.cpp:276-300), so the result is bit-identical.
// A thread owns one pixel and CPT consecutive output channels; with VEC it reads 8 input channels
// of all 9 taps at once (16-byte loads), keeping the per-channel order.
template <int CPT, bool VEC>
__global__ void __launch_bounds__(256) k_conv_direct(const bf16_t* __restrict__ x, const bf16_t* __restrict__ w,
                                                     const bf16_t* __restrict__ bias, bf16_t* __restrict__ out,
                                                     int H, int W, int ci, int co, int k, int pad) {
    const int groups = (co + CPT - 1) / CPT;
    const int64_t idx = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x;
    if (idx >= static_cast<int64_t>(H) * W * groups) return;
    const int cg = static_cast<int>(idx % groups);
    const int64_t p = idx / groups;
    const int y = static_cast<int>(p / W), xx = static_cast<int>(p - static_cast<int64_t>(y) * W);
    const int co0 = cg * CPT;
    float acc[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) acc[j] = (bias && co0 + j < co) ? bf2f(bias[co0 + j]) : 0.0f;
    const int kk = k * k;
    if constexpr (VEC) {
        for (int icb = 0; icb < ci; icb += 8) {
            float xv[9][8];
            bool ok[9];
#pragma unroll
            for (int t = 0; t < 9; ++t) {
                const int ky = t / 3, kx = t % 3;
                const int iy = y + ky - pad, ix = xx + kx - pad;
                ok[t] = t < kk && iy >= 0 && iy < H && ix >= 0 && ix < W;
                uint4 raw = make_uint4(0, 0, 0, 0);
                if (ok[t]) raw = *reinterpret_cast<const uint4*>(x + (static_cast<int64_t>(iy) * W + ix) * ci + icb);
                const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int q = 0; q < 8; ++q)
                    xv[t][q] = __uint_as_float(q & 1 ? (w4[q >> 1] & 0xffff0000u) : (w4[q >> 1] << 16));
            }
#pragma unroll
            for (int q = 0; q < 8; ++q)
#pragma unroll
                for (int t = 0; t < 9; ++t) {
                    if (!ok[t]) continue;
#pragma unroll
                    for (int j = 0; j < CPT; ++j) {
                        if (co0 + j >= co) continue;
                        const float wv = bf2f(w[((static_cast<int64_t>(co0 + j) * ci + icb + q) * kk) + t]);
                        acc[j] = __fadd_rn(acc[j], __fmul_rn(xv[t][q], wv));
                    }
                }
        }
    } else {
        for (int ic = 0; ic < ci; ++ic)
            for (int ky = 0; ky < k; ++ky) {
                const int iy = y + ky - pad;
                if (iy < 0 || iy >= H) continue;
                for (int kx = 0; kx < k; ++kx) {
                    const int ix = xx + kx - pad;
                    if (ix < 0 || ix >= W) continue;
                    const float xv = bf2f(x[(static_cast<int64_t>(iy) * W + ix) * ci + ic]);
#pragma unroll
                    for (int j = 0; j < CPT; ++j) {
                        if (co0 + j >= co) continue;
                        const float wv = bf2f(w[((static_cast<int64_t>(co0 + j) * ci + ic) * k + ky) * k + kx]);
                        acc[j] = __fadd_rn(acc[j], __fmul_rn(xv, wv));
                    }
                }
            }
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j)
        if (co0 + j < co) out[p * co + co0 + j] = f2bf(acc[j]);
}

// ---- nearest upsample, NCHW (UpsampleArgs, ops_cpu.cpp:384-397) ------------------------------

__global__ void __launch_bounds__(256) k_upsample_nchw(const bf16_t* __restrict__ in, bf16_t* __restrict__ out,
                                                       int64_t planes, int64_t H, int64_t W, int64_t f) {
    const int64_t H2 = H * f, W2 = W * f, n = planes * H2 * W2;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t x = i % W2, y = (i / W2) % H2, pl = i / (H2 * W2);
        out[i] = in[(pl * H + y / f) * W + x / f];
    }
}

// ---- the mid-block attention: one head, head_dim 512 ------------------------------------------
//
// softmax(Q K^T / sqrt(512)) V over S tokens, Q, K, O [S, 512] and V given transposed,
// vt[d][slot(key)] (keys permuted within 32-key chunks so that the eight keys a lane group holds
// after a pair of 16x16 score tiles are one 16-byte fragment, see k_vt512; zero past S up to a
// multiple of 32). A workgroup of four waves owns 64 queries, a wave one
// 16-query tile; keys stream in blocks of 32 through two LDS stages of 64 KiB (the block's K rows
// and V^T rows), filled by direct global->LDS loads issued by all four waves after the block
// barrier. Both products run on v_mfma_f32_16x16x32_bf16 with transposed tiles, as in the
// head_dim-72 kernel: S^T = K Q^T (K from LDS, Q in registers: 16 fragments), O^T += V^T P^T
// (V^T from LDS, P in registers as it comes out of the softmax). O^T is 32 16-row tiles: 128
// accumulator registers per lane.
//
// K rows in LDS are 1 KiB (512 dims); 16-byte chunk c of row r sits at c ^ (r & 15), so the 16
// rows a fragment read touches hit 16 different chunks of one 256-byte span (all 64 banks).
//
// Softmax in fp32 with the running maximum in log2 units; it moves only when a block beats it by
// more than 8 (any fixed reference gives the same normalised result; the bound keeps P below
// 2^8). P is rounded to bf16 for the MFMA and the denominator sums those rounded values. Keys
// past S score -inf.
constexpr int kA5Q = 64;                 // queries per workgroup
constexpr int kA5Kv = 32;                // keys per block
constexpr int kA5D = 512;
constexpr int kA5KBytes = kA5Kv * kA5D * 2;   // 32 KiB
constexpr int kA5VBytes = kA5D * kA5Kv * 2;   // 32 KiB
constexpr int kA5Stage = kA5KBytes + kA5VBytes;

struct A5Args {
    const bf16_t* q;
    const bf16_t* k;
    const bf16_t* vt;
    bf16_t* out;
    int S;
    int64_t vt_ld;
    float c;   // scale * log2(e)
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One global_load_lds_dwordx4: lane L's 16 bytes at `src` land at LDS address lds + 16 L.
__device__ __forceinline__ void a5_dma16(const void* src, const char* lds) {
    const uint32_t l = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(lds)));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(l), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

__device__ __forceinline__ bf16x8_t a5_frag(const char* p) { return *reinterpret_cast<const bf16x8_t*>(p); }

__device__ __forceinline__ float a5_pair(float v, bool swap32, bool is_max) {
    const uint32_t x = __float_as_uint(v);
    const auto r = swap32 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                          : __builtin_amdgcn_permlane16_swap(x, x, false, false);
    const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
    return is_max ? fmaxf(a, b) : a + b;
}

// Block j's 64 KiB: pieces 0..31 are K rows (1 KiB each, swizzled), 32..63 V^T rows 16(p-32)..+15
// (64 bytes each); wave w issues pieces 4i + w.
__device__ __forceinline__ void a5_dma_block(char* st, const A5Args& a, int j, int wave, int lane) {
    const int key0 = j * kA5Kv;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int piece = i * 4 + wave;
        if (piece < 32) {
            const int key = min(key0 + piece, a.S - 1);
            const int c = lane ^ (piece & 15);
            a5_dma16(a.k + static_cast<int64_t>(key) * kA5D + c * 8, st + piece * 1024);
        } else {
            const int d = (piece - 32) * 16 + (lane >> 2);
            a5_dma16(a.vt + static_cast<int64_t>(d) * a.vt_ld + key0 + (lane & 3) * 8,
                     st + kA5KBytes + (piece - 32) * 1024);
        }
    }
}

__global__ void __launch_bounds__(256, 1) k_flash512(A5Args a) {
    __shared__ __attribute__((aligned(1024))) char smem[2 * kA5Stage];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, hi = lane >> 4;
    const int q = blockIdx.x * kA5Q + wave * 16 + lr;
    const int qc = min(q, a.S - 1);
    bf16x8_t qf[16];
#pragma unroll
    for (int ks = 0; ks < 16; ++ks) qf[ks] = a5_frag(reinterpret_cast<const char*>(a.q + static_cast<int64_t>(qc) * kA5D + 32 * ks + 8 * hi));
    f32x4_t o[32];
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) o[dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;
    const int nblk = (a.S + kA5Kv - 1) / kA5Kv;
    a5_dma_block(smem, a, 0, wave, lane);
    for (int j = 0; j < nblk; ++j) {
        // block j has landed (every wave's loads) and nobody still reads the other stage
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        s_waitcnt<0, 0>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (j + 1 < nblk) a5_dma_block(smem + ((j + 1) & 1) * kA5Stage, a, j + 1, wave, lane);
        const char* st = smem + (j & 1) * kA5Stage;
        f32x4_t s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 16; ++ks) {
            const int pc = ((4 * ks + hi) ^ lr) * 16;
            const bf16x8_t k0 = a5_frag(st + lr * 1024 + pc);
            const bf16x8_t k1 = a5_frag(st + (16 + lr) * 1024 + pc);
            s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[ks], s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[ks], s1, 0, 0, 0);
        }
        // scores in log2 units; keys past S never count
        const int kb = j * kA5Kv + 4 * hi;
        float x[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            x[t] = kb + t < a.S ? s0[t] * a.c : -INFINITY;
            x[4 + t] = kb + 16 + t < a.S ? s1[t] * a.c : -INFINITY;
        }
        float mx = x[0];
#pragma unroll
        for (int t = 1; t < 8; ++t) mx = fmaxf(mx, x[t]);
        mx = a5_pair(mx, true, true);
        mx = a5_pair(mx, false, true);
        if (__any(mx > m + 8.0f)) {
            const float mn = fmaxf(m, mx);
            const float alpha = exp2f(m - mn);   // 0 on the first block (m = -inf)
            m = mn;
            l *= alpha;
#pragma unroll
            for (int dt = 0; dt < 32; ++dt)
#pragma unroll
                for (int t = 0; t < 4; ++t) o[dt][t] *= alpha;
        }
        bf16x8_t pf;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const __bf16 pb = static_cast<__bf16>(exp2f(x[t] - m));
            pf[t] = pb;
            l += static_cast<float>(pb);
        }
#pragma unroll
        for (int dt = 0; dt < 32; ++dt) {
            const bf16x8_t vf = a5_frag(st + kA5KBytes + (16 * dt + lr) * 64 + hi * 16);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[dt], 0, 0, 0);
        }
    }
    l = a5_pair(l, true, false);
    l = a5_pair(l, false, false);
    if (q >= a.S) return;
    bf16_t* orow = a.out + static_cast<int64_t>(q) * kA5D + 4 * hi;
    const float rl = __frcp_rn(l);   // one reciprocal per query, a multiply per output
#pragma unroll
    for (int dt = 0; dt < 32; ++dt) {
        const uint32_t lo = f2bf2(o[dt][0] * rl, o[dt][1] * rl);
        const uint32_t hi2 = f2bf2(o[dt][2] * rl, o[dt][3] * rl);
        *reinterpret_cast<uint2*>(orow + 16 * dt) = make_uint2(lo, hi2);
    }
}

// V [S, 512] -> vt[d][slot(key)], zero for S <= key < vt_ld. A 32-key x 32-dim tile per block.
__global__ void __launch_bounds__(256) k_vt512(const bf16_t* __restrict__ v, bf16_t* __restrict__ vt,
                                               int S, int64_t vt_ld) {
    __shared__ bf16_t tile[32][33];
    const int key0 = blockIdx.x * 32, d0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;
#pragma unroll
    for (int i = ty; i < 32; i += 8) {
        const int key = key0 + i;
        tile[i][tx] = key < S ? v[static_cast<int64_t>(key) * kA5D + d0 + tx] : bf16_t{0};
    }
    __syncthreads();
    // storage slot tx of the chunk holds key (tx & 3) | ((tx >> 3) & 3) << 2 | ((tx >> 2) & 1) << 4
    const int kk = (tx & 3) | (((tx >> 3) & 3) << 2) | (((tx >> 2) & 1) << 4);
#pragma unroll
    for (int i = ty; i < 32; i += 8) vt[static_cast<int64_t>(d0 + i) * vt_ld + key0 + tx] = tile[kk][i];
}

int grid_for(int64_t n, int per_block) {
    return static_cast<int>(std::min<int64_t>((n + per_block - 1) / per_block, 65535LL * 16));
}

// [co][ci][3][3] -> [co][3][3][ci]: the implicit GEMM's k index is (ky, kx, ci).
__global__ void k_repack3x3(const bf16_t* __restrict__ w, bf16_t* __restrict__ out, int64_t co,
                            int64_t ci) {
    const int64_t n = co * ci * 9;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = i % ci, t = (i / ci) % 9, o = i / (ci * 9);
        out[i] = w[(o * ci + c) * 9 + t];
    }
}

// Scratch of the op-level entry points (NCHW at the boundary, channels-last inside): per device
// and slot, grown on demand, zero-filled when grown, kept until the process ends. Calls that
// overlap on one device share it.
enum OpSlot { SLOT_IN = 0, SLOT_OUT = 1, SLOT_W = 2, SLOT_ZERO = 3, SLOT_GN = 4, SLOT_COUNT = 5 };

void* op_workspace(int slot, size_t bytes) {
    static std::mutex mu;
    static void* ptr[64][SLOT_COUNT] = {};
    static size_t cap[64][SLOT_COUNT] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "op workspace: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev][slot] < bytes) {
        if (ptr[dev][slot]) hip_check(hipFree(ptr[dev][slot]), "hipFree");
        ptr[dev][slot] = nullptr;
        cap[dev][slot] = 0;
        hip_check(hipMalloc(&ptr[dev][slot], bytes), "hipMalloc (op workspace)");
        hip_check(hipMemset(ptr[dev][slot], 0, bytes), "hipMemset (op workspace)");
        cap[dev][slot] = bytes;
    }
    return ptr[dev][slot];
}

GroupNormScratch op_gn_scratch() {
    GroupNormScratch sc;
    sc.max_chunks = 2048;
    char* base = static_cast<char*>(op_workspace(SLOT_GN, 2048 * 64 * 8 + 64 * 8 + 64 * 4));
    sc.part = reinterpret_cast<double*>(base);
    sc.mean = reinterpret_cast<double*>(base + 2048 * 64 * 8);
    sc.inv = reinterpret_cast<float*>(base + 2048 * 64 * 8 + 64 * 8);
    return sc;
}

}  // namespace

void launch_repack3x3(const bf16_t* w, bf16_t* out, int64_t co, int64_t ci, hipStream_t s) {
    k_repack3x3<<<grid_for(co * ci * 9, 256), 256, 0, s>>>(w, out, co, ci);
    launch_check("repack 3x3 weights");
}

// Conv2dArgs (ops.h:120-126) at the op boundary, NCHW bf16, stride 1: per batch image the input
// goes channels-last, the convolution runs on the kernel its shape allows (3x3 "same" with
// c_in % 64 == 0: the MFMA implicit GEMM; 1x1: the MFMA GEMM; other "same" kernels: the direct
// kernel in the reference's order), and the output comes back to NCHW.
void launch_conv2d_nchw(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* out,
                        int64_t batch, int64_t ci, int64_t h, int64_t wd, int64_t co, int64_t k,
                        int64_t pad, hipStream_t s) {
    const int64_t ho = h + 2 * pad - k + 1, wo = wd + 2 * pad - k + 1;
    require(ho == h && wo == wd && 2 * pad == k - 1,
            "conv2d (hip-gfx950): only stride-1 'same' convolutions (2 * pad == k - 1) have a kernel");
    if (batch == 0 || co == 0 || h == 0 || wd == 0) return;
    const int64_t S = h * wd;
    bf16_t* xin = static_cast<bf16_t*>(op_workspace(SLOT_IN, static_cast<size_t>(S * ci * 2)));
    bf16_t* yout = static_cast<bf16_t*>(op_workspace(SLOT_OUT, static_cast<size_t>(S * co * 2)));
    const bool mfma3 = k == 3 && ci % 64 == 0 && co % 8 == 0 && h < (1 << 15) && wd < (1 << 15);
    bf16_t* wr = nullptr;
    if (mfma3) {
        wr = static_cast<bf16_t*>(op_workspace(SLOT_W, static_cast<size_t>(co * ci * 9 * 2)));
        launch_repack3x3(w, wr, co, ci, s);
    }
    for (int64_t b = 0; b < batch; ++b) {
        launch_transpose_bf16(x + b * ci * S, xin, 1, ci, S, s);
        if (mfma3) {
            ConvGeom g;
            g.in = xin;
            g.zero = static_cast<const bf16_t*>(op_workspace(SLOT_ZERO, 256));
            g.H = g.in_h = static_cast<int>(h);
            g.W = g.in_w = static_cast<int>(wd);
            g.c_in = static_cast<int>(ci);
            launch_conv3x3_bf16(g, wr, bias, yout, co, GemmEpilogue{}, s);
        } else if (k == 1) {
            launch_gemm_bf16(xin, w, bias, yout, S, co, ci, GemmEpilogue{}, s);
        } else {
            launch_conv_direct_nhwc(xin, w, bias, yout, h, wd, ci, co, k, pad, s);
        }
        launch_transpose_bf16(yout, out + b * co * S, 1, S, co, s);
    }
}

// NormArgs with groups > 0 (ops_cpu.cpp:186-224): rows = batch, cols = channels * spatial, NCHW.
void launch_group_norm_nchw(const bf16_t* x, const bf16_t* w, const bf16_t* b, bf16_t* out,
                            int64_t rows, int64_t cols, float eps, int64_t groups, int64_t channels,
                            hipStream_t s) {
    const int64_t C = channels ? channels : cols;
    require(cols % groups == 0, "groupnorm: channels*spatial not divisible by groups");
    require(C % groups == 0, "groupnorm: channels not divisible by groups");
    require(cols % C == 0, "groupnorm: cols is not a whole number of channel planes");
    require(gn_nhwc_supported(C, groups),
            "groupnorm (hip-gfx950): needs channels % 8 == 0 with channels / 8 dividing 256");
    const int64_t S = cols / C;
    if (rows == 0 || S == 0) return;
    bf16_t* xin = static_cast<bf16_t*>(op_workspace(SLOT_IN, static_cast<size_t>(cols * 2)));
    bf16_t* yout = static_cast<bf16_t*>(op_workspace(SLOT_OUT, static_cast<size_t>(cols * 2)));
    GroupNormScratch sc = op_gn_scratch();
    for (int64_t r = 0; r < rows; ++r) {
        launch_transpose_bf16(x + r * cols, xin, 1, C, S, s);
        launch_group_norm_nhwc(xin, yout, S, C, groups, eps, w, b, false, sc, s);
        launch_transpose_bf16(yout, out + r * cols, 1, S, C, s);
    }
}


// ---- launchers (declared in common.h) ---------------------------------------------------------

void launch_transpose_bf16(const bf16_t* in, bf16_t* out, int64_t batch, int64_t R, int64_t C,
                           hipStream_t s) {
    if (batch == 0 || R == 0 || C == 0) return;
    require((R + 31) / 32 <= 65535 && batch <= 65535, "transpose: too many rows for one launch");
    const dim3 grid(static_cast<unsigned>((C + 31) / 32), static_cast<unsigned>((R + 31) / 32),
                    static_cast<unsigned>(batch));
    ProfileScope ps(K_ELEMENTWISE, s, 4.0 * static_cast<double>(batch * R * C));
    k_transpose<<<grid, 256, 0, s>>>(in, out, R, C, C);
    launch_check("transpose");
}

void launch_transpose_keep_bf16(const bf16_t* in, bf16_t* out, int64_t R, int64_t C, int64_t keep,
                                hipStream_t s) {
    if (R == 0 || keep == 0) return;
    require(keep <= C && (R + 31) / 32 <= 65535, "transpose: kept columns or rows out of range");
    const dim3 grid(static_cast<unsigned>((keep + 31) / 32), static_cast<unsigned>((R + 31) / 32), 1);
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * static_cast<double>(R * (C + keep)));
    k_transpose<<<grid, 256, 0, s>>>(in, out, R, C, keep);
    launch_check("transpose");
}

// Rows [S][C] -> [S][Cp] with columns C..Cp-1 zero (Cp >= C): the latent, padded to the implicit
// GEMM's 64-channel k-tile.
__global__ void __launch_bounds__(256) k_pad_rows(const bf16_t* __restrict__ in, bf16_t* __restrict__ out,
                                                  int64_t S, int64_t C, int64_t Cp) {
    const int64_t n = S * Cp;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = i % Cp, p = i / Cp;
        out[i] = c < C ? in[p * C + c] : bf16_t{0};
    }
}

void launch_pad_rows(const bf16_t* in, bf16_t* out, int64_t S, int64_t C, int64_t Cp, hipStream_t s) {
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * static_cast<double>(S * (C + Cp)));
    k_pad_rows<<<grid_for(S * Cp, 256), 256, 0, s>>>(in, out, S, C, Cp);
    launch_check("pad rows");
}

// w [co][ci][3][3] -> out [cop][3][3][cip] zero-padded (cop >= co, cip >= ci).
__global__ void k_repack3x3_pad(const bf16_t* __restrict__ w, bf16_t* __restrict__ out, int64_t co,
                                int64_t ci, int64_t cop, int64_t cip) {
    const int64_t n = cop * cip * 9;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t c = i % cip, t = (i / cip) % 9, o = i / (cip * 9);
        out[i] = (o < co && c < ci) ? w[(o * ci + c) * 9 + t] : bf16_t{0};
    }
}

void launch_repack3x3_pad(const bf16_t* w, bf16_t* out, int64_t co, int64_t ci, int64_t cop,
                          int64_t cip, hipStream_t s) {
    k_repack3x3_pad<<<grid_for(cop * cip * 9, 256), 256, 0, s>>>(w, out, co, ci, cop, cip);
    launch_check("repack 3x3 weights (padded)");
}

bool gn_nhwc_supported(int64_t C, int64_t G) {
    return C % 8 == 0 && C / 8 <= kGnThreads && kGnThreads % (C / 8) == 0 && G > 0 && G <= 64 &&
           C % G == 0;
}

void launch_group_norm_nhwc(const bf16_t* x, bf16_t* out, int64_t S, int64_t C, int64_t G,
                            float eps, const bf16_t* w, const bf16_t* b, bool silu,
                            GroupNormScratch& sc, hipStream_t s) {
    require(gn_nhwc_supported(C, G), "groupnorm (nhwc): unsupported channel / group count");
    const int chunks = static_cast<int>(std::min<int64_t>(sc.max_chunks, std::max<int64_t>(1, (S + 15) / 16)));
    const int64_t per = (S + chunks - 1) / chunks;
    const int ci = static_cast<int>(C), gi = static_cast<int>(G);
    const double n = static_cast<double>(S) * (C / G);
    ProfileScope ps(K_NORM, s, 4.0 * static_cast<double>(S * C));
    k_gn_partial<<<chunks, kGnThreads, 0, s>>>(x, S, ci, gi, per, nullptr, sc.part);
    k_gn_finalize<<<gi, 256, 0, s>>>(sc.part, chunks, gi, n, 0, eps, sc.mean, sc.inv);
    k_gn_partial<<<chunks, kGnThreads, 0, s>>>(x, S, ci, gi, per, sc.mean, sc.part);
    k_gn_finalize<<<gi, 256, 0, s>>>(sc.part, chunks, gi, n, 1, eps, sc.mean, sc.inv);
    const int blocks = grid_for(S * (C / 8), 256);
#define BH_GN_APPLY(W_, B_, S_) \
    k_gn_apply<W_, B_, S_><<<blocks, 256, 0, s>>>(x, out, S, ci, gi, sc.mean, sc.inv, w, b)
    if (w && b) {
        if (silu) BH_GN_APPLY(true, true, true);
        else BH_GN_APPLY(true, true, false);
    } else if (w) {
        if (silu) BH_GN_APPLY(true, false, true);
        else BH_GN_APPLY(true, false, false);
    } else if (b) {
        if (silu) BH_GN_APPLY(false, true, true);
        else BH_GN_APPLY(false, true, false);
    } else {
        if (silu) BH_GN_APPLY(false, false, true);
        else BH_GN_APPLY(false, false, false);
    }
#undef BH_GN_APPLY
    launch_check("groupnorm (nhwc)");
}

void launch_conv_direct_nhwc(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* out,
                             int64_t H, int64_t W, int64_t ci, int64_t co, int64_t k, int64_t pad,
                             hipStream_t s) {
    require(k >= 1 && k <= 3 && 2 * pad == k - 1, "conv (direct): odd kernel up to 3, same padding");
    require(H * W < (int64_t{1} << 31) && co < 65536 && ci < 65536, "conv (direct): too large");
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * static_cast<double>(H * W) * ci * co * k * k);
    const int hh = static_cast<int>(H), ww = static_cast<int>(W), cii = static_cast<int>(ci),
              coo = static_cast<int>(co), kk = static_cast<int>(k), pp = static_cast<int>(pad);
    const bool vec = ci % 8 == 0 && k == 3 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    if (co <= 4) {
        const int64_t n = H * W;
        if (vec) k_conv_direct<4, true><<<grid_for(n, 256), 256, 0, s>>>(x, w, bias, out, hh, ww, cii, coo, kk, pp);
        else k_conv_direct<4, false><<<grid_for(n, 256), 256, 0, s>>>(x, w, bias, out, hh, ww, cii, coo, kk, pp);
    } else {
        const int64_t n = H * W * ((co + 7) / 8);
        if (vec) k_conv_direct<8, true><<<grid_for(n, 256), 256, 0, s>>>(x, w, bias, out, hh, ww, cii, coo, kk, pp);
        else k_conv_direct<8, false><<<grid_for(n, 256), 256, 0, s>>>(x, w, bias, out, hh, ww, cii, coo, kk, pp);
    }
    launch_check("conv (direct)");
}

void launch_upsample_nchw(const bf16_t* in, bf16_t* out, int64_t planes, int64_t H, int64_t W,
                          int64_t f, hipStream_t s) {
    const int64_t n = planes * H * W * f * f;
    if (n == 0) return;
    ProfileScope ps(K_ELEMENTWISE, s, 2.0 * static_cast<double>(n + planes * H * W));
    k_upsample_nchw<<<grid_for(n, 256), 256, 0, s>>>(in, out, planes, H, W, f);
    launch_check("upsample");
}

int64_t vt512_ld(int64_t S) { return (S + 31) / 32 * 32; }

void launch_attention512(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* vt, bf16_t* out,
                         int64_t S, float scale, hipStream_t s) {
    require(S > 0 && S < (int64_t{1} << 30), "attention (head_dim 512): sequence length");
    const int64_t ld = vt512_ld(S);
    {
        ProfileScope ps(K_ELEMENTWISE, s, 4.0 * static_cast<double>(S) * kA5D);
        k_vt512<<<dim3(static_cast<unsigned>(ld / 32), kA5D / 32), 256, 0, s>>>(v, vt, static_cast<int>(S), ld);
        launch_check("attention (head_dim 512): V transpose");
    }
    A5Args a{q, k, vt, out, static_cast<int>(S), ld,
             (scale > 0.0f ? scale : 1.0f / std::sqrt(static_cast<float>(kA5D))) * 1.4426950408889634f};
    ProfileScope ps(K_ATTN_SELF, s, 4.0 * static_cast<double>(S) * S * kA5D);
    k_flash512<<<static_cast<unsigned>((S + kA5Q - 1) / kA5Q), 256, 0, s>>>(a);
    launch_check("attention (head_dim 512)");
}

}  // namespace bh
