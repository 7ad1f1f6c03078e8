// bf16 GEMM for the dit-step on gfx950: out[M,N] = A[M,K] . B[N,K]^T (+bias, activation,
// fused residual), fp32 accumulation on the MFMA cores.
//
// Tile: 256 (M) x 144 (N) x 64 (K) per 256-thread workgroup; wave w owns rows [64w, 64w+64)
// and all 144 columns as a 4 x 9 grid of 16x16 accumulators (v_mfma_f32_16x16x32_bf16).
// 144 divides every DiT output width (1152, 3456, 4608) and 256 divides M = 2*4096, so the
// 8192-row GEMMs launch exactly 256, 768 and 1024 tiles: whole waves on 256 CUs, where the
// usual 256x128 tile would leave the last wave of N=1152 one-eighth full.
//
// The MFMA is issued with the weight tile as its first operand, so the accumulator layout puts
// four consecutive OUTPUT COLUMNS of one row in each lane: the epilogue reads bias, residual and
// gate and writes the result with 8-byte accesses.
//
// Operands are staged through LDS, double-buffered: while the waves multiply tile k out of one
// buffer, the next tile's global loads are in flight in registers and land in the other buffer
// after the multiply. Each LDS row is padded from 128 to 144 bytes so the 16-byte fragment reads
// of 8 consecutive rows hit disjoint banks.
//
// Tile order is XCD-aware: workgroup i runs on XCD i%8, so tiles are renumbered so that each
// XCD gets a contiguous band of 4 M-tiles x all N-tiles, whose A and B panels fit its 4 MB L2.
//
// Summation order inside an MFMA differs from the reference oracle's sequential loop
// (ops_cpu.cpp:60-66); products of bf16 are exact in fp32, so results differ only by fp32
// accumulation rounding before the single bf16 rounding at the store.
#include "common.h"

namespace bh {
namespace {

constexpr int BM = 256, BN = 144, BK = 64;
constexpr int kThreads = 256;
constexpr int kLdsRow = BK + 8;                      // bf16 per LDS row: 144 bytes
constexpr int kAElems = BM * kLdsRow;
constexpr int kBElems = BN * kLdsRow;
constexpr int kStage = kAElems + kBElems;            // 57,600 bytes per stage
constexpr int kAChunks = BM * (BK / 8) / kThreads;   // 8 16-byte chunks per thread
constexpr int kBChunks = (BN * (BK / 8) + kThreads - 1) / kThreads;  // 5 (last partial)
constexpr int kMT = 4, kNT = 9;                      // 16x16 tiles per wave

struct Epi {
    const bf16_t* bias;
    int act;
    bool round_mid;
    const bf16_t* row_add;
    int64_t row_add_period;
    const bf16_t* residual;
    const bf16_t* gate;
    int64_t gate_rows;
    int64_t ld_out;
};

__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    const float x3 = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fmul_rn(c, __fadd_rn(x, __fmul_rn(0.044715f, x3)));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}
__device__ __forceinline__ float silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x))); }

// acc (+ bias already added) -> activation -> optional mid rounding -> row add -> residual.
__device__ __forceinline__ float epi_value(float v, int act, bool round_mid) {
    if (act == 1) v = gelu_tanh(v);
    else if (act == 2) v = silu(v);
    if (round_mid) v = round_bf16(v);
    return v;
}

__device__ __forceinline__ void unpack4(uint2 raw, float (&f)[4]) {
    f[0] = __uint_as_float(raw.x << 16);
    f[1] = __uint_as_float(raw.x & 0xffff0000u);
    f[2] = __uint_as_float(raw.y << 16);
    f[3] = __uint_as_float(raw.y & 0xffff0000u);
}
__device__ __forceinline__ uint2 pack4(const float (&f)[4]) {
    uint2 r;
    r.x = static_cast<uint32_t>(f2bf(f[0])) | (static_cast<uint32_t>(f2bf(f[1])) << 16);
    r.y = static_cast<uint32_t>(f2bf(f[2])) | (static_cast<uint32_t>(f2bf(f[3])) << 16);
    return r;
}

// Four consecutive columns [n, n+4) of row m. `vec` means all four are in range and every
// operand is 8-byte aligned there.
__device__ __forceinline__ void store_quad(const Epi& e, bf16_t* out, int64_t m, int64_t n,
                                           int64_t N, const float (&acc)[4], bool vec) {
    if (vec) {
        float v[4], t[4];
        if (e.bias) {
            unpack4(*reinterpret_cast<const uint2*>(e.bias + n), t);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = __fadd_rn(acc[r], t[r]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = acc[r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) v[r] = epi_value(v[r], e.act, e.round_mid);
        if (e.row_add) {
            unpack4(*reinterpret_cast<const uint2*>(e.row_add + (m % e.row_add_period) * N + n), t);
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = __fadd_rn(v[r], t[r]);
        }
        if (e.residual) {
            float res[4];
            unpack4(*reinterpret_cast<const uint2*>(e.residual + m * e.ld_out + n), res);
            if (e.gate) {
                unpack4(*reinterpret_cast<const uint2*>(e.gate + (m / e.gate_rows) * N + n), t);
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = __fadd_rn(__fmul_rn(v[r], t[r]), res[r]);
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = __fadd_rn(res[r], v[r]);
            }
        }
        *reinterpret_cast<uint2*>(out + m * e.ld_out + n) = pack4(v);
        return;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int64_t c = n + r;
        if (c >= N) break;
        float v = acc[r];
        if (e.bias) v = __fadd_rn(v, bf2f(e.bias[c]));
        v = epi_value(v, e.act, e.round_mid);
        if (e.row_add) v = __fadd_rn(v, bf2f(e.row_add[(m % e.row_add_period) * N + c]));
        if (e.residual) {
            const float res = bf2f(e.residual[m * e.ld_out + c]);
            if (e.gate) v = __fadd_rn(__fmul_rn(v, bf2f(e.gate[(m / e.gate_rows) * N + c])), res);
            else v = __fadd_rn(res, v);
        }
        out[m * e.ld_out + c] = f2bf(v);
    }
}

__global__ void __launch_bounds__(kThreads, 1)
k_gemm_mfma(const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, bf16_t* out, int64_t M,
            int64_t N, int64_t K, Epi e, int tiles_m, int tiles_n, int group_m, bool vec_epi) {
    __shared__ __attribute__((aligned(16))) bf16_t smem[2 * kStage];

    // ---- tile selection: XCD-contiguous bands, grouped by `group_m` M-tiles ----
    const int T = tiles_m * tiles_n;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int group_size = group_m * tiles_n;
    const int g = bid / group_size;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_group = bid - g * group_size;
    const int tm = first_m + in_group % gm;
    const int tn = in_group / gm;
    const int64_t m0 = static_cast<int64_t>(tm) * BM;
    const int64_t n0 = static_cast<int64_t>(tn) * BN;

    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int kc = tid & 7;          // 16-byte chunk within a 64-wide K slab
    const int r0 = tid >> 3;         // first row this thread stages

    uint4 ra[kAChunks], rb[kBChunks];
    const int KT = static_cast<int>((K + BK - 1) / BK);

    auto load_tile = [&](int kt) {
        const int64_t k = static_cast<int64_t>(kt) * BK + kc * 8;
        const bool kin = k < K;
#pragma unroll
        for (int i = 0; i < kAChunks; ++i) {
            const int64_t row = m0 + r0 + 32 * i;
            ra[i] = (kin && row < M) ? *reinterpret_cast<const uint4*>(A + row * K + k)
                                     : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kBChunks; ++i) {
            const int lr = r0 + 32 * i;
            const int64_t row = n0 + lr;
            rb[i] = (lr < BN && kin && row < N) ? *reinterpret_cast<const uint4*>(B + row * K + k)
                                                 : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int stage) {
        bf16_t* As = smem + stage * kStage;
        bf16_t* Bs = As + kAElems;
#pragma unroll
        for (int i = 0; i < kAChunks; ++i) {
            *reinterpret_cast<uint4*>(As + (r0 + 32 * i) * kLdsRow + kc * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kBChunks; ++i) {
            const int lr = r0 + 32 * i;
            if (lr < BN) *reinterpret_cast<uint4*>(Bs + lr * kLdsRow + kc * 8) = rb[i];
        }
    };

    f32x4_t acc[kMT][kNT];
#pragma unroll
    for (int i = 0; i < kMT; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int frag_row = lane & 15;
    const int frag_k = (lane >> 4) * 8;
    for (int kt = 0; kt < KT; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < KT) load_tile(kt + 1);
        const bf16_t* As = smem + cur * kStage;
        const bf16_t* Bs = As + kAElems;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 32) {
            bf16x8_t af[kMT];
#pragma unroll
            for (int i = 0; i < kMT; ++i) {
                af[i] = *reinterpret_cast<const bf16x8_t*>(
                    As + (wave * 64 + i * 16 + frag_row) * kLdsRow + kk + frag_k);
            }
#pragma unroll
            for (int j = 0; j < kNT; ++j) {
                const bf16x8_t bw = *reinterpret_cast<const bf16x8_t*>(
                    Bs + (j * 16 + frag_row) * kLdsRow + kk + frag_k);
#pragma unroll
                for (int i = 0; i < kMT; ++i) {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw, af[i], acc[i][j], 0, 0, 0);
                }
            }
        }
        if (kt + 1 < KT) store_tile(cur ^ 1);
        __syncthreads();
    }

    // ---- epilogue: lane holds C[m][n..n+3] for each (i, j) ----
    const int quad = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < kMT; ++i) {
        const int64_t m = m0 + wave * 64 + i * 16 + frag_row;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int64_t n = n0 + j * 16 + quad;
            if (n >= N) continue;
            const float a4[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
            store_quad(e, out, m, n, N, a4, vec_epi && n + 4 <= N);
        }
    }
}

// ---- small M: one wave per output column, both operands read with 16-byte loads ----
constexpr int kGemvMaxM = 8;

__global__ void __launch_bounds__(256) k_gemv(const bf16_t* __restrict__ A,
                                              const bf16_t* __restrict__ B, bf16_t* out,
                                              int64_t M, int64_t N, int64_t K, Epi e) {
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
        v = epi_value(v, e.act, e.round_mid);
        if (e.row_add) v = __fadd_rn(v, bf2f(e.row_add[(m % e.row_add_period) * N + n]));
        if (e.residual) {
            const float res = bf2f(e.residual[m * e.ld_out + n]);
            if (e.gate) v = __fadd_rn(__fmul_rn(v, bf2f(e.gate[(m / e.gate_rows) * N + n])), res);
            else v = __fadd_rn(res, v);
        }
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
    stv(out, idx, epi_value(acc, act, false));
}

bool aligned(const void* p, int bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
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
    Epi e{bias, ep.act, ep.round_mid, ep.row_add, ep.row_add_period > 0 ? ep.row_add_period : 1,
          ep.residual, ep.gate, ep.gate_rows > 0 ? ep.gate_rows : 1, ep.ld_out > 0 ? ep.ld_out : n};
    const bool fast_k = (k % 8 == 0) && aligned(a, 16) && aligned(b, 16);
    const double flops = 2.0 * static_cast<double>(m) * n * k;
    if (!fast_k) {
        require(!ep.row_add && !ep.residual && !ep.round_mid && e.ld_out == n,
                "gemm: fused epilogues need K % 8 == 0 and 16-byte aligned operands");
        ProfileScope ps(K_GEMM, s, flops);
        launch_gemm_generic(a, b, bias, out, m, n, k, true, ep.act, false, s);
        return;
    }
    if (m <= kGemvMaxM) {
        ProfileScope ps(K_GEMV, s, flops);
        const int grid = static_cast<int>((n + 3) / 4);
        k_gemv<<<grid, 256, 0, s>>>(a, b, out, m, n, k, e);
        launch_check("gemm (small M)");
        return;
    }
    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + BN - 1) / BN);
    const bool vec = (n % 4 == 0) && (e.ld_out % 4 == 0) && aligned(out, 8) &&
                     (!bias || aligned(bias, 8)) && (!e.residual || aligned(e.residual, 8)) &&
                     (!e.gate || aligned(e.gate, 8)) && (!e.row_add || aligned(e.row_add, 8));
    ProfileScope ps(K_GEMM, s, flops, gemm_subclass());
    k_gemm_mfma<<<tiles_m * tiles_n, kThreads, 0, s>>>(a, b, out, m, n, k, e, tiles_m, tiles_n,
                                                       4, vec);
    launch_check("gemm (mfma)");
}

}  // namespace bh
