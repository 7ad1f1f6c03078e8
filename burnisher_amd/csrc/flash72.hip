// Flash attention at head_dim 72 (PixArt-Sigma: 16 heads x 72) on gfx950.
//
//   out = softmax(scale * Q K^T, key mask) V over head-last [batch, seq, heads, 72] Q and K, and
//   V supplied TRANSPOSED: vt[((b * heads + h) * 72 + d) * vt_ld + kv], zero past kv_len.
//
// Workgroup: 4 waves, 256 queries of one (batch, head); wave w owns queries 64w..64w+63 as four
// 16-query tiles. Keys stream in blocks of 64 through three LDS stages filled by direct
// global->LDS loads (global_load_lds_dwordx4), two blocks in flight behind the one in use.
//
// Both products run on v_mfma_f32_16x16x32_bf16 with the score matrix TRANSPOSED:
//   S^T[kv, q]  = K[kv, :] . Q[q, :]^T      A = K fragment (LDS), B = Q fragment (registers)
//   O^T[d, q]  += V^T[d, kv] . P^T[kv, q]   A = V^T fragment (LDS), B = P (registers)
// The S^T accumulator gives each lane four consecutive keys of one query; two such tiles are
// exactly that lane's 8-element B operand of the second product, with the keys in an order the
// V^T fragment reads in the same order, so P never leaves registers. head_dim 72 is padded to
// 96 for the score product (the padding lanes of K are zeroed in registers, Q's in its load) and
// to 80 for the output: V^T rows 72..79 sit in LDS with row 72 all ONES, so O^T row 72 is the
// softmax denominator sum_kv P[kv] for free, accumulated from the same bf16 P as the numerator.
//
// Softmax: scores stay fp32; exp2(s * scale * log2e - m) with the running maximum m kept in those
// units. The maximum is only moved (and O rescaled by exp2(m_old - m_new)) when a block's maximum
// exceeds it by more than 8: any fixed m gives the same normalised result, and the threshold
// bounds every P by 2^8, far from fp32 range. That keeps the rescale off the common path.
//
// Numerics against the reference oracle (ops_cpu.cpp:84-131): a masked key scores exactly -1e9
// there, so with any unmasked key in the row its weight exp(-1e9 - max) is exactly 0 -- here it
// is -inf, weight 0, and key blocks that are wholly masked are skipped. A row whose keys are ALL
// masked is uniform over V in the oracle; here all its scores are set equal, which is the same
// uniform average. P is rounded to bf16 for the MFMA (the oracle keeps it fp32) and the
// normalisation divides by the sum of those rounded weights.
#include "common.h"

#include <cmath>

namespace bh {
namespace {

constexpr int D = 72;
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kQPerWave = 64;
constexpr int kQPerWg = kWaves * kQPerWave;   // 256
constexpr int kKV = 64;                       // keys per block
constexpr int kQT = 4;                        // 16-query tiles per wave
constexpr int kKT = 4;                        // 16-key tiles per block
constexpr int kKRow = D * 2;                  // 144 bytes per K row in LDS
constexpr int kKBytes = kKV * kKRow;          // 9216 = 9 DMA blocks
constexpr int kVRows = 80;                    // 72 dims + the ones row + zero rows
constexpr int kVBytes = kVRows * 128;         // 128 bytes = 64 keys per V^T row
constexpr int kSpareBytes = 2 * 1024;
constexpr int kStage = kKBytes + kVBytes + kSpareBytes;   // 21504
constexpr int kDmaPerWave = 5;                // 9 K + 9 V^T + 2 spare blocks over 4 waves
constexpr int kMaxBlocks = 256;               // kv_len <= 16384 (the 2048px token count)
constexpr float kRescaleThreshold = 8.0f;     // log2 units

struct Flash72Args {
    const bf16_t* q;
    const bf16_t* k;
    const bf16_t* vt;
    bf16_t* out;
    const void* mask;
    int64_t ld_q, ld_k, vt_ld, ld_o;
    int B, H, Sq, Skv;
    int mask_f32;
    int qblocks;
    float c;   // scale * log2(e)
};

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// One global_load_lds_dwordx4: lane L's 16 bytes at `src` land at LDS address lds + 16 L (`lds`
// wave-uniform). Inline assembly so that the compiler does not track the LDS writes (its
// tracking is conservative at loop headers); the explicit vmcnt waits cover them.
__device__ __forceinline__ void dma16(const void* src, const char* lds) {
    const uint32_t l = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(lds)));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(l), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Waits until this wave has at most N DMA instructions outstanding and no LDS operation, then
// joins the workgroup; the empty asm statements keep every LDS access on its side.
template <int N>
__device__ __forceinline__ void wait_and_join() {
    asm volatile("" ::: "memory");
    s_waitcnt<N, 0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The key blocks stream into `stage` as K rows (144 bytes each, contiguous) in DMA blocks 0..8
// and V^T rows 0..71 (128 bytes = the block's 64 keys, 16-byte chunk c of row d stored at slot
// c ^ ((d >> 1) & 7)) in blocks 9..17, spread over the waves: instruction i of wave w carries
// block 4i + w. Blocks 18-19 re-load block 0 into the spare area so every wave issues exactly
// kDmaPerWave instructions. Which kind an instruction is depends only on (i, wave), so the
// branch on it is scalar. DmaPlan holds this lane's element offset for each instruction at key
// block 0 (for K items including its row's stride), so a block costs one 64-bit add per
// instruction, plus a clamp of the row for the partial last block of a masked run.
struct DmaPlan {
    int64_t off[kDmaPerWave];
    int krow[kDmaPerWave];       // K items: the row within the block
};

__device__ __forceinline__ bool dma_is_v(int i, int wave) {
    const int item = i * kWaves + wave;
    return item >= 9 && item < 18;
}
__device__ __forceinline__ int dma_dst(int i, int wave) {
    const int item = i * kWaves + wave;
    return item < 9 ? item * 1024 : item < 18 ? kKBytes + (item - 9) * 1024
                                              : kKBytes + kVBytes + (item - 18) * 1024;
}

__device__ __forceinline__ DmaPlan dma_plan(const Flash72Args& a, int b, int h, int wave, int lane) {
    DmaPlan p;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const int item = i * kWaves + wave;            // wave-uniform
        if (dma_is_v(i, wave)) {
            const int vi = item - 9;
            const int d = vi * 8 + (lane >> 3);
            const int c = (lane & 7) ^ ((d >> 1) & 7);
            p.off[i] = ((static_cast<int64_t>(b) * a.H + h) * D + d) * a.vt_ld + c * 8;
            p.krow[i] = 0;
        } else {
            const int ki = item < 9 ? item : 0;        // spares (18, 19) re-load K block 0
            const int lg = ki * 64 + lane;
            const int row = lg / 9, ch = lg - row * 9;
            p.off[i] = (static_cast<int64_t>(b) * a.Skv + row) * a.ld_k + h * D + ch * 8;
            p.krow[i] = row;
        }
    }
    return p;
}

// Key block starting at key kv0 into `stage`. `partial`: the block runs past the last key, whose
// row then stands in for the missing ones (their scores are masked).
__device__ __forceinline__ void dma_block(char* stage, const Flash72Args& a, const DmaPlan& p,
                                          int wave, int kv0, bool partial) {
    const int64_t kstep = static_cast<int64_t>(kv0) * a.ld_k;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const bf16_t* src;
        if (dma_is_v(i, wave)) {
            src = a.vt + p.off[i] + kv0;
        } else if (!partial) {
            src = a.k + p.off[i] + kstep;
        } else {
            const int key = min(kv0 + p.krow[i], a.Skv - 1);
            src = a.k + p.off[i] + (static_cast<int64_t>(key) - p.krow[i]) * a.ld_k;
        }
        dma16(src, stage + dma_dst(i, wave));
    }
}

// Three-input maximum (v_max3_f32). This file is compiled with -fno-honor-nans: with IEEE NaN
// rules the compiler would first quiet every MFMA result with an extra v_max, doubling the cost
// of the row maximum. Scores here are finite, or -inf for masked keys.
__device__ __forceinline__ float max3(float a, float b, float c) {
    return __builtin_fmaxf(a, __builtin_fmaxf(b, c));
}

__device__ __forceinline__ bf16x8_t ld_frag(const char* p) {
    return *reinterpret_cast<const bf16x8_t*>(p);
}

template <bool MASKED>
__global__ void __launch_bounds__(kThreads, 1) k_flash72(Flash72Args a) {
    __shared__ __attribute__((aligned(1024))) char smem[3 * kStage];
    __shared__ unsigned long long blk_bits[kMaxBlocks];
    __shared__ int live[kMaxBlocks];
    __shared__ int nlive_s, all_masked_s;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, g = lane >> 4;

    // ---- which (b, h, query block): the blocks of one (b, h) stay on one XCD ----
    const int T = a.B * a.H * a.qblocks;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int bh = bid / a.qblocks;
    const int b = bh / a.H, h = bh - b * a.H;
    const int q_base = (bid - bh * a.qblocks) * kQPerWg + wave * kQPerWave;
    const int nblk = (a.Skv + kKV - 1) / kKV;

    // ---- Q fragments, resident: tile u, K=32 step ks covers dims 32ks + 8g .. +7 (loaded first,
    // so their latency overlaps the set-up below) ----
    bf16x8_t qf[kQT][3];
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        const int q = q_base + u * 16 + lr;
#pragma unroll
        for (int ks = 0; ks < 3; ++ks) {
            const int d0 = ks * 32 + g * 8;
            bf16x8_t f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = static_cast<__bf16>(0.0f);
            if (q < a.Sq && d0 < D)
                f = ld_frag(reinterpret_cast<const char*>(
                    a.q + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_q + h * D + d0));
            qf[u][ks] = f;
        }
    }

    // ---- key validity per block (bit i = key 64 blk + i is in range and unmasked) ----
    if (MASKED) {
        for (int blk = wave; blk < nblk; blk += kWaves) {
            const int key = blk * kKV + lane;
            bool ok = key < a.Skv;
            if (ok && a.mask) {
                const float mv = a.mask_f32 ? static_cast<const float*>(a.mask)[b * a.Skv + key]
                                            : bf2f(static_cast<const bf16_t*>(a.mask)[b * a.Skv + key]);
                ok = mv != 0.0f;
            }
            const unsigned long long bits = __ballot(ok);
            if (lane == 0) blk_bits[blk] = bits;
        }
    }
    // V^T rows 72..79 of every stage: the ones row and zero padding (never written by the DMA)
    for (int i = threadIdx.x; i < 3 * 8 * 128 / 16; i += kThreads) {
        const int st = i / 64, w = i - st * 64;   // 64 16-byte words per stage
        const uint32_t one = w < 8 ? 0x3f803f80u : 0u;
        *reinterpret_cast<uint4*>(smem + st * kStage + kKBytes + 72 * 128 + w * 16) =
            make_uint4(one, one, one, one);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int n = 0;
        unsigned long long any = MASKED ? 0ull : 1ull;
        if (MASKED)
            for (int blk = 0; blk < nblk; ++blk) any |= blk_bits[blk];
        const bool all_masked = any == 0ull;
        for (int blk = 0; blk < nblk; ++blk)
            if (!MASKED || all_masked || blk_bits[blk] != 0ull) live[n++] = blk;
        nlive_s = n;
        all_masked_s = all_masked ? 1 : 0;
    }
    __syncthreads();
    const int nlive = nlive_s;
    const bool all_masked = MASKED && all_masked_s != 0;

    // fragment byte offsets within a stage
    const int sw = (lr >> 1) & 7;
    int koff[3];
#pragma unroll
    for (int ks = 0; ks < 3; ++ks) koff[ks] = lr * kKRow + (ks * 4 + g) * 16;
    // ks = 2 covers dims 64..95 and only g = 0 (dims 64..71) is real: Q is zero in the other
    // lanes, and the K bytes read there are the next row's (or, past the last row, V^T's) finite
    // values, so their products vanish without zeroing K.
    int voff[2][2];
#pragma unroll
    for (int cc = 0; cc < 2; ++cc) {
        const int q1 = cc * 4 + (g >> 1);
        voff[cc][0] = kKBytes + lr * 128 + ((q1 ^ sw) << 4) + (g & 1) * 8;
        voff[cc][1] = kKBytes + lr * 128 + (((q1 + 2) ^ sw) << 4) + (g & 1) * 8;
    }

    f32x4_t o[5][kQT];
#pragma unroll
    for (int e = 0; e < 5; ++e)
#pragma unroll
        for (int u = 0; u < kQT; ++u) o[e][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float mc[kQT];
#pragma unroll
    for (int u = 0; u < kQT; ++u) mc[u] = -INFINITY;

    // ---- the key-block pipeline ----
    // The Q loads are drained here, where the compiler sees it: otherwise it waits for them
    // (vmcnt(0), which also drains the DMA in flight) at their first use in every iteration.
    s_waitcnt<0, 15>();
    const DmaPlan plan = dma_plan(a, b, h, wave, lane);
    const int last_full = a.Skv / kKV;   // blocks below this one hold 64 real keys
    auto issue = [&](char* stage_ptr, int blk) {
        dma_block(stage_ptr, a, plan, wave, blk * kKV, MASKED && blk >= last_full);
    };
    issue(smem, live[0]);
    issue(smem + kStage, live[min(1, nlive - 1)]);
    int stage = 0;
    for (int jj = 0; jj < nlive; ++jj) {
        wait_and_join<kDmaPerWave>();
        {
            const int s2 = stage == 0 ? 2 : stage - 1;
            issue(smem + s2 * kStage, live[min(jj + 2, nlive - 1)]);
        }
        const char* cur = smem + stage * kStage;
        const int blk = live[jj];

        // S^T tiles: s[t][u][r] = score of key 64 blk + 16t + 4g + r, query tile u column lr
        f32x4_t s[kKT][kQT];
#pragma unroll
        for (int t = 0; t < kKT; ++t) {
            bf16x8_t kf[3];
#pragma unroll
            for (int ks = 0; ks < 3; ++ks) kf[ks] = ld_frag(cur + t * 16 * kKRow + koff[ks]);
#pragma unroll
            for (int u = 0; u < kQT; ++u) {
                f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 3; ++ks)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[u][ks], acc, 0, 0, 0);
                s[t][u] = acc;
            }
        }

        if (MASKED) {
            const unsigned long long bits = blk_bits[blk] >> (4 * g);
            const unsigned long long inrange =
                (blk * kKV + kKV <= a.Skv) ? ~0ull
                                           : (((1ull << (a.Skv - blk * kKV)) - 1ull) >> (4 * g));
#pragma unroll
            for (int t = 0; t < kKT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int bit = 16 * t + r;
                    const bool ok = all_masked ? ((inrange >> bit) & 1ull) : ((bits >> bit) & 1ull);
#pragma unroll
                    for (int u = 0; u < kQT; ++u) {
                        const float v = all_masked ? 0.0f : s[t][u][r];
                        s[t][u][r] = ok ? v : -INFINITY;
                    }
                }
        }

        // block maximum per query (the 64 keys of a query sit in lanes lr, lr+16, lr+32, lr+48)
        float lmc[kQT];
        bool need = false;
#pragma unroll
        for (int u = 0; u < kQT; ++u) {
            float m = max3(s[0][u][0], s[0][u][1], s[0][u][2]);
            m = max3(m, s[0][u][3], s[1][u][0]);
            m = max3(m, s[1][u][1], s[1][u][2]);
            m = max3(m, s[1][u][3], s[2][u][0]);
            m = max3(m, s[2][u][1], s[2][u][2]);
            m = max3(m, s[2][u][3], s[3][u][0]);
            m = max3(m, s[3][u][1], s[3][u][2]);
            m = max3(m, s[3][u][3], s[3][u][3]);
            const float m16 = __shfl_xor(m, 16, 64);
            m = max3(m, m16, m16);
            const float m32 = __shfl_xor(m, 32, 64);
            m = max3(m, m32, m32);
            lmc[u] = m * a.c;
            need |= lmc[u] > mc[u] + kRescaleThreshold;
        }
        if (__any(need)) {
#pragma unroll
            for (int u = 0; u < kQT; ++u) {
                const float mn = fmaxf(mc[u], lmc[u]);
                const float alpha = __builtin_amdgcn_exp2f(mc[u] - mn);
                mc[u] = mn;
#pragma unroll
                for (int e = 0; e < 5; ++e)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[e][u][r] *= alpha;
            }
        }

        // P = exp2(s c - m), to bf16, as the B operand of O^T += V^T P^T (two 32-key chunks)
        bf16x8_t pf[kQT][2];
#pragma unroll
        for (int u = 0; u < kQT; ++u)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    pf[u][cc][r] = static_cast<__bf16>(
                        __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * cc][u][r], a.c, -mc[u])));
                    pf[u][cc][4 + r] = static_cast<__bf16>(
                        __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * cc + 1][u][r], a.c, -mc[u])));
                }

#pragma unroll
        for (int e = 0; e < 5; ++e)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const char* vrow = cur + e * 16 * 128;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow + voff[cc][0]);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + voff[cc][1]);
                const uint4 packed = make_uint4(lo.x, lo.y, hi.x, hi.y);
                const bf16x8_t vf = *reinterpret_cast<const bf16x8_t*>(&packed);
#pragma unroll
                for (int u = 0; u < kQT; ++u)
                    o[e][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[u][cc], o[e][u], 0, 0, 0);
            }
        stage = stage == 2 ? 0 : stage + 1;
    }
    s_waitcnt<0, 15>();   // the trailing copies

    // ---- normalise and store: lane holds out[q][d..d+3], d = 16e + 4g; O^T row 72 is the sum ----
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        const float l = __shfl(o[4][u][0], 32 + lr, 64);
        const int q = q_base + u * 16 + lr;
        if (q >= a.Sq) continue;
        bf16_t* dst = a.out + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_o + h * D;
#pragma unroll
        for (int e = 0; e < 5; ++e) {
            const int d = e * 16 + g * 4;
            if (d >= D) continue;
            uint2 w;
            w.x = static_cast<uint32_t>(f2bf(__fdiv_rn(o[e][u][0], l))) |
                  (static_cast<uint32_t>(f2bf(__fdiv_rn(o[e][u][1], l))) << 16);
            w.y = static_cast<uint32_t>(f2bf(__fdiv_rn(o[e][u][2], l))) |
                  (static_cast<uint32_t>(f2bf(__fdiv_rn(o[e][u][3], l))) << 16);
            *reinterpret_cast<uint2*>(dst + d) = w;
        }
    }
}

// V [batch, kv_len, ld_v] (head h at columns 72h..72h+71) -> V^T rows of vt_ld keys, zero-padded
// past kv_len. One workgroup per (b, h, 64-key block), through LDS.
__global__ void __launch_bounds__(256) k_transpose_v72(const bf16_t* __restrict__ v, int64_t ld_v,
                                                       int B, int H, int Skv, bf16_t* vt,
                                                       int64_t vt_ld) {
    __shared__ bf16_t tile[kKV][D + 2];
    const int nblk = static_cast<int>((vt_ld + kKV - 1) / kKV);
    const int blk = blockIdx.x % nblk;
    const int bh = blockIdx.x / nblk;
    const int b = bh / H, h = bh - b * H;
    const int kv0 = blk * kKV;
    for (int i = threadIdx.x; i < kKV * D; i += 256) {
        const int r = i / D, d = i - r * D;
        const int key = kv0 + r;
        tile[r][d] = key < Skv ? v[(static_cast<int64_t>(b) * Skv + key) * ld_v + h * D + d] : bf16_t(0);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < D * kKV; i += 256) {
        const int d = i / kKV, r = i - d * kKV;
        if (kv0 + r < vt_ld) vt[((static_cast<int64_t>(b) * H + h) * D + d) * vt_ld + kv0 + r] = tile[r][d];
    }
}

}  // namespace

int64_t flash72_vt_ld(int64_t kv_len) { return (kv_len + kKV - 1) / kKV * kKV; }

void launch_transpose_v72(const bf16_t* v, int64_t ld_v, int64_t batch, int64_t heads,
                          int64_t kv_len, bf16_t* vt, int64_t vt_ld, hipStream_t s) {
    const int64_t nblk = (vt_ld + kKV - 1) / kKV;
    k_transpose_v72<<<static_cast<int>(batch * heads * nblk), 256, 0, s>>>(
        v, ld_v, static_cast<int>(batch), static_cast<int>(heads), static_cast<int>(kv_len), vt,
        vt_ld);
    launch_check("transpose V (head_dim 72)");
}

void launch_flash72(const bf16_t* q, int64_t ld_q, const bf16_t* k, int64_t ld_k,
                    const bf16_t* vt, int64_t vt_ld, bf16_t* out, int64_t ld_o, int64_t batch,
                    int64_t heads, int64_t q_len, int64_t kv_len, float scale,
                    const void* key_mask, bool mask_f32, hipStream_t s) {
    if (batch * heads * q_len == 0) return;
    require(kv_len > 0, "attention: kv_len must be positive");
    require(kv_len <= kMaxBlocks * kKV, "attention (head_dim 72): kv_len above 16384");
    require(vt_ld >= flash72_vt_ld(kv_len), "attention (head_dim 72): V^T rows too short");
    Flash72Args a;
    a.q = q;
    a.k = k;
    a.vt = vt;
    a.out = out;
    a.mask = key_mask;
    a.ld_q = ld_q;
    a.ld_k = ld_k;
    a.vt_ld = vt_ld;
    a.ld_o = ld_o;
    a.B = static_cast<int>(batch);
    a.H = static_cast<int>(heads);
    a.Sq = static_cast<int>(q_len);
    a.Skv = static_cast<int>(kv_len);
    a.mask_f32 = mask_f32 ? 1 : 0;
    a.qblocks = static_cast<int>((q_len + kQPerWg - 1) / kQPerWg);
    a.c = scale * 1.4426950408889634f;
    const int grid = a.B * a.H * a.qblocks;
    const double flops = 4.0 * batch * heads * static_cast<double>(q_len) * kv_len * D;
    ProfileScope ps(q_len == kv_len ? K_ATTN_SELF : K_ATTN_CROSS, s, flops);
    if (key_mask || kv_len % kKV != 0) k_flash72<true><<<grid, kThreads, 0, s>>>(a);
    else k_flash72<false><<<grid, kThreads, 0, s>>>(a);
    launch_check("attention (flash, head_dim 72)");
}

}  // namespace bh
