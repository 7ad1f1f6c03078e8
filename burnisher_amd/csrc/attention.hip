// Flash attention for the dit-step on gfx950: softmax(scale * Q K^T, key mask) V over
// head-last [batch, seq, heads, head_dim] operands, bf16 in and out, fp32 scores and softmax.
//
// Workgroup = 4 waves = 256 query rows of one (batch, head); each wave owns 64 query rows as 4
// tiles of 16. K/V stream through LDS in blocks of 64 keys, double-buffered, with the next
// block's global loads in flight in registers while the current block is multiplied.
//
// Both products run on v_mfma_f32_16x16x32_bf16 and the kernel computes TRANSPOSED tiles:
//   S^T[kv, q] = K[kv, :] . Q[q, :]^T       (A = K fragment from LDS, B = Q fragment in VGPRs)
//   O^T[d, q] += V^T[d, kv] . P^T[kv, q]    (A = V^T fragment from LDS, B = P from VGPRs)
// The accumulator of the first MFMA holds, per lane, four consecutive keys of ONE query; two
// such tiles are exactly one lane's 8-element B operand of the second MFMA, with the keys in a
// fixed order that the V^T fragment reads in the same order. So P never leaves registers.
//
// head_dim 72 is zero-padded to 96 for the score product (three K=32 steps, the padding lanes
// are zeroed in registers) and to 80 for the output (five 16-row tiles of V^T, rows 72-79 zero).
//
// Numerics follow the reference oracle (ops_cpu.cpp:84-131): scores in fp32 times `scale`, plus
// the additive bias [heads, q_len, kv_len] when given (T5's relative positions), a
// masked key scores exactly -1e9 (so an all-masked row is uniform over V, not NaN), exp in fp32,
// division by the denominator at the end. Unlike the oracle, P is rounded to bf16 for the MFMA
// and the row max is a running max (online softmax). A block of 64 keys that are all masked is
// skipped when the row has at least one unmasked key: exp(-1e9 - max) is exactly 0 in fp32, so
// skipping it changes nothing.
#include "common.h"

#include <cmath>
#include <mutex>

namespace bh {
namespace {

constexpr int kThreads = 256;
constexpr int kQRows = 256;   // query rows per workgroup
constexpr int kKvBlk = 64;    // keys per LDS block
constexpr int kQT = 4;        // 16-row query tiles per wave
constexpr int kKT = 4;        // 16-key tiles per block
constexpr int kMaxFlagBlocks = 256;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnArgs {
    const bf16_t* q;
    const bf16_t* k;
    const bf16_t* v;
    bf16_t* out;
    const void* mask;
    const bf16_t* bias;   // [H, Sq, Skv] or null
    int bias_vec;         // rows of bias are read 8 bytes at a time (Skv % 4 == 0, 8-byte base)
    int mask_f32;
    int64_t B, H, Sq, Skv, D;
    int64_t ld_q, ld_kv, ld_o;
    float scale;
    int k_row;   // LDS row stride of K, bf16 elements
    int v_row;   // LDS row stride of V^T, bf16 elements
    int qb;      // query blocks per (b, h)
};

__device__ __forceinline__ float mask_at(const void* m, int f32, int64_t i) {
    return f32 ? static_cast<const float*>(m)[i] : bf2f(static_cast<const bf16_t*>(m)[i]);
}

// KS: K=32 steps of the score product (head_dim padded to 32*KS); DT: 16-row tiles of V^T.
template <int KS, int DT, bool VEC>
__global__ void __launch_bounds__(kThreads, 1) k_flash(AttnArgs a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
    const int stage_elems = kKvBlk * a.k_row + DT * 16 * a.v_row;
    bf16_t* smem = reinterpret_cast<bf16_t*>(smem_raw);
    float* mbuf = reinterpret_cast<float*>(smem + 2 * stage_elems);   // [2][64]
    int* blk_ok = reinterpret_cast<int*>(mbuf + 2 * kKvBlk);          // [kMaxFlagBlocks]

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int g = lane >> 4, c16 = lane & 15;

    // ---- which (b, h, query block): blocks of one (b, h) stay on one XCD ----
    const int T = static_cast<int>(a.B * a.H) * a.qb;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int64_t bh = bid / a.qb;
    const int64_t b = bh / a.H, h = bh % a.H;
    const int64_t q0 = static_cast<int64_t>(bid % a.qb) * kQRows + wave * (kQT * 16);
    const int64_t D = a.D;
    const int D8 = static_cast<int>((D + 7) & ~7LL);
    const int nblk = static_cast<int>((a.Skv + kKvBlk - 1) / kKvBlk);

    // ---- key-block skipping flags (only with a mask) ----
    const bool use_flags = a.mask != nullptr && nblk <= kMaxFlagBlocks;
    if (use_flags) {
        // one key per thread (a serial scan per block was 64 dependent loads per thread); threads
        // that find an unmasked key all store the same 1, so the race is benign
        for (int blk = tid; blk < nblk; blk += kThreads) blk_ok[blk] = 0;
        __syncthreads();
        for (int64_t j = tid; j < a.Skv; j += kThreads)
            if (mask_at(a.mask, a.mask_f32, b * a.Skv + j) != 0.0f) blk_ok[j / kKvBlk] = 1;
    }
    // V^T rows at and beyond head_dim stay zero for the whole kernel (both stages).
    for (int s = 0; s < 2; ++s) {
        bf16_t* vt = smem + s * stage_elems + kKvBlk * a.k_row;
        for (int i = tid; i < (DT * 16 - static_cast<int>(D)) * a.v_row; i += kThreads)
            vt[static_cast<int>(D) * a.v_row + i] = 0;
    }
    __syncthreads();
    bool any_valid = true;
    if (use_flags) {
        int any = 0;
        for (int blk = 0; blk < nblk; ++blk) any |= blk_ok[blk];
        any_valid = any != 0;
    }

    // ---- Q fragments, resident for the whole kernel ----
    bf16x8_t qf[kQT][KS];
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        const int64_t qrow = q0 + u * 16 + c16;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int d0 = ks * 32 + g * 8;
            bf16x8_t f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = static_cast<__bf16>(0.0f);
            if (qrow < a.Sq && d0 < D8) {
                const bf16_t* src = a.q + (b * a.Sq + qrow) * a.ld_q + h * D + d0;
                if (VEC) {
                    f = *reinterpret_cast<const bf16x8_t*>(src);
                } else {
                    bf16_t tmp[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) tmp[e] = (d0 + e < D) ? src[e] : 0;
                    f = *reinterpret_cast<const bf16x8_t*>(tmp);
                }
            }
            qf[u][ks] = f;
        }
    }

    // ---- K/V staging ----
    constexpr int kMaxChunks = (kKvBlk * (KS * 32 / 8) + kThreads - 1) / kThreads;
    const int chunks_per_row = D8 / 8;
    const int nchunks = kKvBlk * chunks_per_row;
    uint4 rk[kMaxChunks], rv[kMaxChunks];
    auto load_kv = [&](int blk) {
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) {
            const int cidx = tid + i * kThreads;
            rk[i] = make_uint4(0, 0, 0, 0);
            rv[i] = make_uint4(0, 0, 0, 0);
            if (cidx < nchunks) {
                const int row = cidx / chunks_per_row, ch = cidx % chunks_per_row;
                const int64_t kv = static_cast<int64_t>(blk) * kKvBlk + row;
                if (kv < a.Skv) {
                    const int64_t off = (b * a.Skv + kv) * a.ld_kv + h * D + ch * 8;
                    if (VEC) {
                        rk[i] = *reinterpret_cast<const uint4*>(a.k + off);
                        rv[i] = *reinterpret_cast<const uint4*>(a.v + off);
                    } else {
                        bf16_t tk[8], tv[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const bool in = ch * 8 + e < D;
                            tk[e] = in ? a.k[off + e] : 0;
                            tv[e] = in ? a.v[off + e] : 0;
                        }
                        rk[i] = *reinterpret_cast<const uint4*>(tk);
                        rv[i] = *reinterpret_cast<const uint4*>(tv);
                    }
                }
            }
        }
    };
    auto store_kv = [&](int blk, int stage) {
        bf16_t* ks_ = smem + stage * stage_elems;
        bf16_t* vt = ks_ + kKvBlk * a.k_row;
#pragma unroll
        for (int i = 0; i < kMaxChunks; ++i) {
            const int cidx = tid + i * kThreads;
            if (cidx < nchunks) {
                const int row = cidx / chunks_per_row, ch = cidx % chunks_per_row;
                *reinterpret_cast<uint4*>(ks_ + row * a.k_row + ch * 8) = rk[i];
                const bf16_t* vv = reinterpret_cast<const bf16_t*>(&rv[i]);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int d = ch * 8 + e;
                    if (d < D) vt[d * a.v_row + row] = vv[e];
                }
            }
        }
        if (a.mask && tid < kKvBlk) {
            const int64_t kv = static_cast<int64_t>(blk) * kKvBlk + tid;
            mbuf[stage * kKvBlk + tid] = kv < a.Skv ? mask_at(a.mask, a.mask_f32, b * a.Skv + kv) : 1.0f;
        }
    };
    auto block_live = [&](int blk) { return !use_flags || !any_valid || blk_ok[blk] != 0; };

    // ---- online softmax state ----
    f32x4_t o[DT][kQT];
#pragma unroll
    for (int e = 0; e < DT; ++e)
#pragma unroll
        for (int u = 0; u < kQT; ++u) o[e][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float row_max[kQT], row_sum[kQT];
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        row_max[u] = -INFINITY;
        row_sum[u] = 0.f;
    }
    const float scale_log2 = a.scale * kLog2e;

    // first live block
    int blk = 0;
    while (blk < nblk && !block_live(blk)) ++blk;
    if (blk < nblk) {
        load_kv(blk);
        store_kv(blk, 0);
    }
    __syncthreads();
    int stage = 0;
    while (blk < nblk) {
        int next = blk + 1;
        while (next < nblk && !block_live(next)) ++next;
        if (next < nblk) load_kv(next);

        const bf16_t* ks_ = smem + stage * stage_elems;
        const bf16_t* vt = ks_ + kKvBlk * a.k_row;
        const int64_t kvb = static_cast<int64_t>(blk) * kKvBlk;

        // S^T tiles: s[t][u] holds keys kvb + 16t + 4g + r for query c16 of tile u.
        f32x4_t s[kKT][kQT];
#pragma unroll
        for (int t = 0; t < kKT; ++t) {
#pragma unroll
            for (int u = 0; u < kQT; ++u) s[t][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int d0 = ks * 32 + g * 8;
                bf16x8_t kf;
                if (d0 < D8) {
                    kf = *reinterpret_cast<const bf16x8_t*>(ks_ + (t * 16 + c16) * a.k_row + d0);
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) kf[e] = static_cast<__bf16>(0.0f);
                }
#pragma unroll
                for (int u = 0; u < kQT; ++u)
                    s[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[u][ks], s[t][u], 0, 0, 0);
            }
        }

        // the bias of this lane's four keys per (t, u): one 8-byte load when rows are 8-byte aligned
        float bvals[kKT][kQT][4];
        if (a.bias) {
#pragma unroll
            for (int u = 0; u < kQT; ++u) {
                const int64_t qi = min(q0 + u * 16 + c16, a.Sq - 1);
                const bf16_t* brow = a.bias + (h * a.Sq + qi) * a.Skv;
#pragma unroll
                for (int t = 0; t < kKT; ++t) {
                    const int64_t kv = kvb + t * 16 + g * 4;
                    if (a.bias_vec && kv + 3 < a.Skv) {
                        const uint2 raw = *reinterpret_cast<const uint2*>(brow + kv);
                        bvals[t][u][0] = __uint_as_float(raw.x << 16);
                        bvals[t][u][1] = __uint_as_float(raw.x & 0xffff0000u);
                        bvals[t][u][2] = __uint_as_float(raw.y << 16);
                        bvals[t][u][3] = __uint_as_float(raw.y & 0xffff0000u);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) bvals[t][u][r] = kv + r < a.Skv ? bf2f(brow[kv + r]) : 0.0f;
                    }
                }
            }
        }
        // scale, mask, running max, exponentials (base 2 with log2(e) folded into the scale)
        float mvals[kKT][4];
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = t * 16 + g * 4 + r;
                mvals[t][r] = a.mask ? mbuf[stage * kKvBlk + j] : 1.0f;
            }
#pragma unroll
        for (int u = 0; u < kQT; ++u) {
            float mx = -INFINITY;
#pragma unroll
            for (int t = 0; t < kKT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t kv = kvb + t * 16 + g * 4 + r;
                    float val = s[t][u][r] * a.scale;
                    if (a.bias) val = __fadd_rn(val, bvals[t][u][r]);
                    if (kv >= a.Skv) val = -INFINITY;
                    else if (mvals[t][r] == 0.0f) val = -1e9f;
                    s[t][u][r] = val;
                    mx = fmaxf(mx, val);
                }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(row_max[u], mx);
            const float alpha = exp2f((row_max[u] - m_new) * kLog2e);
            row_max[u] = m_new;
            row_sum[u] *= alpha;
#pragma unroll
            for (int e = 0; e < DT; ++e)
#pragma unroll
                for (int r = 0; r < 4; ++r) o[e][u][r] *= alpha;
            const float mb = m_new * kLog2e;
#pragma unroll
            for (int t = 0; t < kKT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float p = exp2f(s[t][u][r] * kLog2e - mb);
                    row_sum[u] += p;
                    s[t][u][r] = p;
                }
        }
        (void)scale_log2;

        // O^T += V^T P^T over two 32-key chunks
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            bf16x8_t pf[kQT];
#pragma unroll
            for (int u = 0; u < kQT; ++u) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pf[u][r] = static_cast<__bf16>(s[2 * c][u][r]);
                    pf[u][4 + r] = static_cast<__bf16>(s[2 * c + 1][u][r]);
                }
            }
#pragma unroll
            for (int e = 0; e < DT; ++e) {
                const bf16_t* vrow = vt + (e * 16 + c16) * a.v_row + c * 32 + g * 4;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 16);
                const uint4 packed = make_uint4(lo.x, lo.y, hi.x, hi.y);
                const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(&packed);
#pragma unroll
                for (int u = 0; u < kQT; ++u)
                    o[e][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[u], o[e][u], 0, 0, 0);
            }
        }

        if (next < nblk) store_kv(next, stage ^ 1);
        __syncthreads();
        stage ^= 1;
        blk = next;
    }

    // ---- normalise and store: lane holds out[q][d..d+3], d = 16e + 4g ----
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        float l = row_sum[u];
        l += __shfl_xor(l, 16, 64);
        l += __shfl_xor(l, 32, 64);
        const int64_t qrow = q0 + u * 16 + c16;
        if (qrow >= a.Sq) continue;
        bf16_t* dst = a.out + (b * a.Sq + qrow) * a.ld_o + h * D;
        const float rl = __frcp_rn(l);   // one reciprocal per query, a multiply per output
#pragma unroll
        for (int e = 0; e < DT; ++e) {
            const int d = e * 16 + g * 4;
            if (d >= D) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) v[r] = o[e][u][r] * rl;
            if (VEC) {
                uint2 w;
                w.x = f2bf2(v[0], v[1]);
                w.y = f2bf2(v[2], v[3]);
                *reinterpret_cast<uint2*>(dst + d) = w;
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (d + r < D) dst[d + r] = f2bf(v[r]);
            }
        }
    }
}

// ---- reference order: one thread per (b, h, query) row ----
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

constexpr int kGenericMaxD = 256;

template <typename T>
__global__ void __launch_bounds__(128) k_attention_generic(const T* __restrict__ q, const T* __restrict__ k,
                                                           const T* __restrict__ v, T* __restrict__ out,
                                                           AttnShape sh, const T* __restrict__ bias,
                                                           const void* mask, int mask_f32) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (idx >= sh.batch * sh.heads * sh.q_len) return;
    const int64_t i = idx % sh.q_len, h = (idx / sh.q_len) % sh.heads, b = idx / (sh.q_len * sh.heads);
    const int64_t D = sh.head_dim;
    const T* qr = q + (b * sh.q_len + i) * sh.ld_q + h * D;
    auto score = [&](int64_t j) {
        const T* kr = k + (b * sh.kv_len + j) * sh.ld_kv + h * D;
        float s = 0.f;
        for (int64_t d = 0; d < D; ++d) s = __fadd_rn(s, __fmul_rn(ldv(qr, d), ldv(kr, d)));
        s = __fmul_rn(s, sh.scale);
        if (bias) s = __fadd_rn(s, ldv(bias, (h * sh.q_len + i) * sh.kv_len + j));
        if (mask && mask_at(mask, mask_f32, b * sh.kv_len + j) == 0.0f) s = -1e9f;
        return s;
    };
    float row_max = -INFINITY;
    for (int64_t j = 0; j < sh.kv_len; ++j) row_max = fmaxf(row_max, score(j));
    float acc[kGenericMaxD];
    for (int64_t d = 0; d < D; ++d) acc[d] = 0.f;
    float denom = 0.f;
    for (int64_t j = 0; j < sh.kv_len; ++j) {
        const float w = expf(__fsub_rn(score(j), row_max));
        denom = __fadd_rn(denom, w);
        const T* vr = v + (b * sh.kv_len + j) * sh.ld_kv + h * D;
        for (int64_t d = 0; d < D; ++d) acc[d] = __fadd_rn(acc[d], __fmul_rn(w, ldv(vr, d)));
    }
    T* orow = out + (b * sh.q_len + i) * sh.ld_o + h * D;
    for (int64_t d = 0; d < D; ++d) stv(orow, d, __fdiv_rn(acc[d], denom));
}

}  // namespace

namespace {
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The allocation-free entry point's V^T scratch: one fixed array per device, in the code
// object's device memory (each GPU the library runs on holds its own copy until the process
// ends). Host code never uses this name as an address: its device address, per device, comes
// from hipGetSymbolAddress at set-up (noalloc_scratch below).
__device__ __align__(256) bf16_t scratch[kNoAllocScratchBytes / sizeof(bf16_t)];

// V^T scratch for the head_dim-72 path of the op-level entry point: grown on demand, kept until
// the process ends, one per device. Calls that overlap on one device share it.
bf16_t* vt_workspace(size_t elems) {
    static std::mutex mu;
    static void* ptr[64] = {};
    static size_t cap[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "attention: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] < elems) {
        if (ptr[dev]) hip_check(hipFree(ptr[dev]), "hipFree");
        ptr[dev] = nullptr;
        cap[dev] = 0;
        hip_check(hipMalloc(&ptr[dev], elems * sizeof(bf16_t)), "hipMalloc (V^T workspace)");
        cap[dev] = elems;
    }
    return static_cast<bf16_t*>(ptr[dev]);
}

// Which kernel launch_attention_bf16 runs for these operands, and the V^T elements it needs.
struct AttnPlan {
    enum Kind { FLASH512, FLASH72, FLASH } kind;
    int64_t vt_elems;
};

AttnPlan plan_attention(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* out,
                        const AttnShape& sh, const void* key_mask, const bf16_t* bias) {
    // head_dim 512, one head, self-attention, unmasked (the VAE mid-block): its own kernel.
    if (sh.head_dim == 512 && sh.heads == 1 && sh.q_len == sh.kv_len && !key_mask && !bias &&
        sh.ld_q == 512 && sh.ld_kv == 512 && sh.ld_o == 512 && aligned16(q) && aligned16(k) &&
        aligned16(v) && aligned16(out))
        return {AttnPlan::FLASH512, 512 * vt512_ld(sh.kv_len)};
    // head_dim 72 (the DiT): V transposed once, then the flash kernel built for that width.
    const bool fast72 = !bias && sh.head_dim == 72 && sh.kv_len <= 16384 && sh.ld_q % 8 == 0 &&
                        sh.ld_kv % 8 == 0 && sh.ld_o % 4 == 0 && aligned16(q) && aligned16(k) &&
                        aligned16(v) && (reinterpret_cast<uintptr_t>(out) % 8 == 0);
    if (fast72) return {AttnPlan::FLASH72, sh.batch * sh.heads * 72 * flash72_vt_ld(sh.kv_len)};
    return {AttnPlan::FLASH, 0};
}

}  // namespace

int64_t attention_vt_elems(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* out,
                           const AttnShape& sh, const void* key_mask, const bf16_t* bias) {
    if (sh.batch * sh.heads * sh.q_len == 0) return 0;
    return plan_attention(q, k, v, out, sh, key_mask, bias).vt_elems;
}

int64_t attention_part_floats(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* out,
                              const AttnShape& sh, const void* key_mask, const bf16_t* bias) {
    if (sh.batch * sh.heads * sh.q_len == 0) return 0;
    if (plan_attention(q, k, v, out, sh, key_mask, bias).kind != AttnPlan::FLASH72) return 0;
    return flash72_plan_floats(sh.batch, sh.heads, sh.q_len,
                               flash72_plan(sh.batch, sh.heads, sh.q_len, sh.kv_len, out, sh.ld_o));
}

bf16_t* noalloc_scratch() {
    static std::mutex mu;
    static void* ptr[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "attention: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress (attention scratch)");
        require(p != nullptr, "attention: the scratch array has no device address");
        ptr[dev] = p;
    }
    return static_cast<bf16_t*>(ptr[dev]);
}

void launch_attention_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* out,
                           const AttnShape& sh, const void* key_mask, bool mask_f32,
                           hipStream_t s, const bf16_t* bias, bf16_t* vt_buf, int64_t vt_buf_elems,
                           int splits, float* part, int64_t part_floats, int qb0) {
    if (sh.batch * sh.heads * sh.q_len == 0) return;
    const AttnPlan plan = plan_attention(q, k, v, out, sh, key_mask, bias);
    // V^T goes to the caller's buffer when one is given (it must be large enough), else to the
    // per-device workspace.
    auto vt_for = [&](int64_t elems) {
        if (!vt_buf) return vt_workspace(static_cast<size_t>(elems));
        require(vt_buf_elems >= elems, "attention: the V^T buffer holds " + std::to_string(vt_buf_elems) +
                                           " elements, this call needs " + std::to_string(elems));
        return vt_buf;
    };
    if (plan.kind == AttnPlan::FLASH512) {
        bf16_t* vt = vt_for(plan.vt_elems);
        for (int64_t b = 0; b < sh.batch; ++b) {
            const int64_t off = b * sh.q_len * 512;
            launch_attention512(q + off, k + off, v + off, vt, out + off, sh.q_len, sh.scale, s);
        }
        return;
    }
    if (plan.kind == AttnPlan::FLASH72) {
        const int64_t vt_ld = flash72_vt_ld(sh.kv_len);
        bf16_t* vt = vt_for(plan.vt_elems);
        launch_transpose_v72(v, sh.ld_kv, sh.batch, sh.heads, sh.kv_len, vt, vt_ld, s);
        launch_flash72(q, sh.ld_q, k, sh.ld_kv, vt, vt_ld, out, sh.ld_o, sh.batch, sh.heads,
                       sh.q_len, sh.kv_len, sh.scale, key_mask, mask_f32, s, splits, part,
                       part_floats, qb0);
        return;
    }
    require(sh.kv_len > 0, "attention: kv_len must be positive");
    require(sh.head_dim >= 1 && sh.head_dim <= 128,
            "attention (hip-gfx950): head_dim must be in [1, 128]");
    const bool vec = (sh.head_dim % 8 == 0) && (sh.ld_q % 8 == 0) && (sh.ld_kv % 8 == 0) &&
                     (sh.ld_o % 4 == 0) && aligned16(q) && aligned16(k) && aligned16(v) &&
                     (reinterpret_cast<uintptr_t>(out) % 8 == 0);
    AttnArgs a;
    a.q = q; a.k = k; a.v = v; a.out = out;
    a.mask = key_mask; a.mask_f32 = mask_f32 ? 1 : 0;
    a.bias = bias;
    a.bias_vec = bias && sh.kv_len % 4 == 0 && (reinterpret_cast<uintptr_t>(bias) & 7) == 0;
    a.B = sh.batch; a.H = sh.heads; a.Sq = sh.q_len; a.Skv = sh.kv_len; a.D = sh.head_dim;
    a.ld_q = sh.ld_q; a.ld_kv = sh.ld_kv; a.ld_o = sh.ld_o;
    a.scale = sh.scale;
    const int d8 = static_cast<int>((sh.head_dim + 7) & ~7LL);
    // 16-byte fragment reads of 8 consecutive rows are conflict-free when the row is an odd
    // multiple of 16 bytes; pad a row that is a multiple of 32 bytes by 16 bytes.
    a.k_row = (d8 % 16 == 0) ? d8 + 8 : d8;
    a.v_row = kKvBlk + 8;
    a.qb = static_cast<int>((sh.q_len + kQRows - 1) / kQRows);
    const int ks = static_cast<int>((sh.head_dim + 31) / 32);
    const int dt = static_cast<int>((sh.head_dim + 15) / 16);
    const size_t lds = sizeof(bf16_t) * 2 * (kKvBlk * a.k_row + dt * 16 * a.v_row) +
                       sizeof(float) * 2 * kKvBlk + sizeof(int) * kMaxFlagBlocks;
    const int grid = static_cast<int>(sh.batch * sh.heads) * a.qb;
    const double flops = 4.0 * sh.batch * sh.heads * static_cast<double>(sh.q_len) * sh.kv_len *
                         sh.head_dim;
    ProfileScope ps(sh.q_len == sh.kv_len ? K_ATTN_SELF : K_ATTN_CROSS, s, flops);
    // Above 64 KiB of dynamic LDS (head_dim > 96) the launch must opt in to the larger size.
#define BH_FLASH(KS_, DT_)                                                                 \
    do {                                                                                   \
        if (vec) {                                                                         \
            if (lds > 65536)                                                               \
                hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_flash<KS_, DT_, true>), \
                                              hipFuncAttributeMaxDynamicSharedMemorySize,  \
                                              static_cast<int>(lds)), "hipFuncSetAttribute"); \
            k_flash<KS_, DT_, true><<<grid, kThreads, lds, s>>>(a);                        \
        } else {                                                                           \
            if (lds > 65536)                                                               \
                hip_check(hipFuncSetAttribute(reinterpret_cast<const void*>(&k_flash<KS_, DT_, false>), \
                                              hipFuncAttributeMaxDynamicSharedMemorySize,  \
                                              static_cast<int>(lds)), "hipFuncSetAttribute"); \
            k_flash<KS_, DT_, false><<<grid, kThreads, lds, s>>>(a);                       \
        }                                                                                  \
    } while (0)
    if (ks == 1 && dt == 1) BH_FLASH(1, 1);
    else if (ks == 1) BH_FLASH(1, 2);
    else if (ks == 2 && dt == 3) BH_FLASH(2, 3);
    else if (ks == 2) BH_FLASH(2, 4);
    else if (ks == 3 && dt == 5) BH_FLASH(3, 5);
    else if (ks == 3) BH_FLASH(3, 6);
    else if (dt == 7) BH_FLASH(4, 7);
    else BH_FLASH(4, 8);
#undef BH_FLASH
    launch_check("attention (flash)");
}

void launch_attention_generic(const void* q, const void* k, const void* v, void* out,
                              const AttnShape& sh, const void* bias, const void* key_mask,
                              bool mask_f32, bool f32, hipStream_t s) {
    const int64_t rows = sh.batch * sh.heads * sh.q_len;
    if (rows == 0) return;
    require(sh.head_dim <= kGenericMaxD, "attention (reference order): head_dim above 256");
    const int grid = static_cast<int>((rows + 127) / 128);
    if (f32) {
        k_attention_generic<float><<<grid, 128, 0, s>>>(
            static_cast<const float*>(q), static_cast<const float*>(k),
            static_cast<const float*>(v), static_cast<float*>(out), sh,
            static_cast<const float*>(bias), key_mask, mask_f32 ? 1 : 0);
    } else {
        k_attention_generic<bf16_t><<<grid, 128, 0, s>>>(
            static_cast<const bf16_t*>(q), static_cast<const bf16_t*>(k),
            static_cast<const bf16_t*>(v), static_cast<bf16_t*>(out), sh,
            static_cast<const bf16_t*>(bias), key_mask, mask_f32 ? 1 : 0);
    }
    launch_check("attention (reference order)");
}

}  // namespace bh
