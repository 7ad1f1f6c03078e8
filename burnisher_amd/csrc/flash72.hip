// Flash attention at head_dim 72 (PixArt-Sigma: 16 heads x 72) on gfx950.
//
//   out = softmax(scale * Q K^T, key mask) V over head-last [batch, seq, heads, 72] Q and K, and
//   V supplied TRANSPOSED: vt[((b * heads + h) * 72 + d) * vt_ld + vt_pos(kv)], zero past
//   kv_len (vt_pos, common.h: keys permuted within 32-key chunks, runs of four kept).
//
// Workgroup: 8 waves, 512 queries of one (batch, head); wave w owns queries 64w..64w+63 as four
// 16-query tiles. Keys stream in blocks of 64 through FOUR LDS stages filled by direct
// global->LDS loads (global_load_lds_dwordx4).
//
// Both products run on v_mfma_f32_16x16x32_bf16 with the score matrix TRANSPOSED:
//   S^T[kv, q]  = K[kv, :] . Q[q, :]^T      A = K fragment (LDS), B = Q fragment (registers)
//   O^T[d, q]  += V^T[d, kv] . P^T[kv, q]   A = V^T fragment (LDS), B = P (registers)
// The S^T accumulator gives each lane four consecutive keys of one query per 16-key tile; with
// the two tiles of a 32-key chunk, lane group g holds keys 4g..4g+3 and 16+4g..16+4g+3, which
// is its B operand of the second product as it stands, because V^T keeps exactly those eight
// keys together (vt_pos): the matching V^T fragment is one 16-byte LDS read. head_dim 72 is
// padded to 96 for the score product (Q is zero in the padding, so whatever finite K bytes sit
// there vanish) and to 80 for the output: V^T rows 72..79 sit in LDS with row 72 all ONES, so O^T
// row 72 is the softmax denominator sum_kv P[kv], accumulated from the same bf16 P as the
// numerator.
//
// Schedule: a wave alternates a matrix phase (the output product of block j-1, then the scores of
// block j: 88 MFMAs) and a vector phase (softmax of block j: maximum, exp2, conversion to bf16).
// Waves 0-3 and 4-7 run one phase apart, separated by a workgroup barrier per phase, so on every
// SIMD one wave's exponentials overlap the other wave's MFMAs. Waves 0-3 also issue the DMA, at
// the end of their matrix phases (the shorter ones).
//
// Softmax: scores stay fp32; exp2(s * scale * log2e - m) with the running maximum m kept in those
// units. Q is multiplied by c = scale * log2e once, as it is loaded (one extra bf16 rounding of
// q c), and the score MFMAs of a block start from the accumulator value -m, so the matrix cores
// deliver s c - m and the vector phase spends no operation per score on it. The first block
// sets m (its scores are formed against 0); a later block moves it (and rescales O by
// exp2(m_old - m_new)) only when one of its scores exceeds it by more than 8: any fixed m gives
// the same normalised result, and the threshold bounds every P by 2^8, far from fp32 range. The
// common path then needs no maximum per query at all -- one per lane and a wave vote decide --
// which matters because this kernel's vector phase is as long as its matrix phase.
//
// Numerics against the reference oracle (ops_cpu.cpp:84-131): a masked key scores exactly -1e9
// there, so with any unmasked key in the row its weight exp(-1e9 - max) is exactly 0 -- here it
// is -inf, weight 0, and key blocks that are wholly masked are skipped. A row whose keys are ALL
// masked is uniform over V in the oracle; here all its scores are set equal, which is the same
// uniform average. P is rounded to bf16 for the MFMA (the oracle keeps it fp32) and the
// normalisation multiplies by the reciprocal of the sum of those rounded weights.
#include "common.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>

namespace bh {
namespace {

constexpr int D = 72;
constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kQPerWave = 64;
constexpr int kQPerWg = kWaves * kQPerWave;   // 512
constexpr int kKV = 64;                       // keys per block
constexpr int kQT = 4;                        // 16-query tiles per wave
constexpr int kKT = 4;                        // 16-key tiles per block
constexpr int kKRow = D * 2;                  // 144 bytes per K row in LDS
constexpr int kKBytes = kKV * kKRow;          // 9216 = 9 DMA blocks
constexpr int kVRows = 80;                    // 72 dims + the ones row + zero rows
constexpr int kVBytes = kVRows * 128;         // 128 bytes = 64 keys per V^T row
constexpr int kSpareBytes = 2 * 1024;
constexpr int kStage = kKBytes + kVBytes + kSpareBytes;   // 21504
constexpr int kStages = 4;
constexpr int kResidentBlocks = 7;            // key blocks a resident launch holds (kv_len <= 448)
constexpr int kDmaWaves = 4;                  // waves 0-3 issue the DMA
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
    // Split over keys (low-occupancy shapes): workgroup (b, h, query block, split) takes key
    // blocks [split * nblk / splits, (split + 1) * nblk / splits) and, when `part` is set,
    // writes its unnormalised partial instead of the output:
    // part[((split * B + b) * H + h) * Sq + q][0..79] = O over dims 0..71, the row sum at 72, the
    // running maximum (log2 units) at 73.
    int splits = 1;
    float* part = nullptr;
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
    // sched_barrier: no instruction, MFMAs included, is moved across (the memory clobbers only
    // pin memory operations), so each phase's work stays between its two barriers
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    s_waitcnt<N, 0>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// The key blocks stream into `stage` as K rows (144 bytes each, contiguous) in DMA blocks 0..8
// and V^T rows 0..71 (128 bytes = the block's 64 keys, 16-byte chunk c of row d stored at slot
// c ^ ((d >> 1) & 7)) in blocks 9..17, spread over the four DMA waves: instruction i of DMA wave
// w carries block 4i + w. Blocks 18-19 re-load block 0 into the spare area so every wave issues
// exactly kDmaPerWave instructions. Which kind an instruction is depends only on (i, wave), so
// the branch on it is scalar. DmaPlan holds this lane's element offset for each instruction at
// key 0, relative to the (b, h) base of K or V^T, in 32 bits (the launcher checks that it
// fits); a block then costs one add per instruction.
struct DmaPlan {
    int off[kDmaPerWave];
};

__device__ __forceinline__ bool dma_is_v(int i, int wave) {
    const int item = i * kDmaWaves + wave;
    return item >= 9 && item < 18;
}
__device__ __forceinline__ int dma_dst(int i, int wave) {
    const int item = i * kDmaWaves + wave;
    return item < 9 ? item * 1024 : item < 18 ? kKBytes + (item - 9) * 1024
                                              : kKBytes + kVBytes + (item - 18) * 1024;
}
// K items: this lane's row within the block
__device__ __forceinline__ int dma_krow(int i, int wave, int lane) {
    const int item = i * kDmaWaves + wave;
    return ((item < 9 ? item : 0) * 64 + lane) / 9;
}

__device__ __forceinline__ DmaPlan dma_plan(const Flash72Args& a, int wave, int lane) {
    DmaPlan p;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const int item = i * kDmaWaves + wave;
        if (dma_is_v(i, wave)) {
            const int d = (item - 9) * 8 + (lane >> 3);
            const int c = (lane & 7) ^ ((d >> 1) & 7);
            p.off[i] = d * static_cast<int>(a.vt_ld) + c * 8;
        } else {
            const int lg = (item < 9 ? item : 0) * 64 + lane;   // spares (18, 19) re-load block 0
            const int row = lg / 9, ch = lg - row * 9;
            p.off[i] = row * static_cast<int>(a.ld_k) + ch * 8;
        }
    }
    return p;
}

// Key block starting at key kv0 into `stage`. `partial`: the block runs past the last key, whose
// row then stands in for the missing ones (their scores are masked).
__device__ __forceinline__ void dma_block(char* stage, const Flash72Args& a, const DmaPlan& p,
                                          const bf16_t* kbh, const bf16_t* vbh, int wave, int lane,
                                          int kv0, bool partial) {
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        const bf16_t* src;
        if (dma_is_v(i, wave)) {
            src = vbh + (p.off[i] + kv0);
        } else if (!partial) {
            src = kbh + (p.off[i] + kv0 * static_cast<int>(a.ld_k));
        } else {
            const int row = dma_krow(i, wave, lane);
            const int key = min(kv0 + row, a.Skv - 1);
            src = kbh + (p.off[i] + (key - row) * static_cast<int>(a.ld_k));
        }
        dma16(src, stage + dma_dst(i, wave));
    }
}

// DMA item `item` (0..19) of the key block at kv0 into `stage`, any wave: items 0..8 are K, 9..17
// V^T, 18..19 spares (see dma_block). Used by the resident variant's one-time prologue.
__device__ __forceinline__ void dma_item(char* stage, const Flash72Args& a, const bf16_t* kbh,
                                         const bf16_t* vbh, int item, int lane, int kv0,
                                         bool partial) {
    const bf16_t* src;
    int dst;
    if (item >= 9 && item < 18) {
        const int d = (item - 9) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ ((d >> 1) & 7);
        src = vbh + (d * static_cast<int>(a.vt_ld) + c * 8 + kv0);
        dst = kKBytes + (item - 9) * 1024;
    } else {
        const int lg = (item < 9 ? item : 0) * 64 + lane;
        const int row = lg / 9, ch = lg - row * 9;
        const int key = partial ? min(kv0 + row, a.Skv - 1) : kv0 + row;
        src = kbh + (key * static_cast<int>(a.ld_k) + ch * 8);
        dst = item < 9 ? item * 1024 : kKBytes + kVBytes + (item - 18) * 1024;
    }
    dma16(src, stage + dst);
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

// Per-wave state of the pipeline.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct WaveState {
    bf16x8_t qf[kQT][3];       // Q fragments: tile u, K=32 step ks covers dims 32ks + 8g .. +7
    f32x4_t o[5][kQT];         // O^T accumulators: rows 16e + 4g .. +3 (row 72 = denominator)
    f32x4_t s[kKT][kQT];       // S^T of the current block: key 16t + 4g + r, query 16u + lr
    bf16x8_t pf[kQT][2];       // P of the previous block, as the second product's B operand
    float mc[kQT];             // running maximum (scaled, log2 units), per query of the lane
};

// The matrix phase: O^T += V^T P^T for the block whose P is in w.pf (OUT: 40 MFMAs, V^T from
// `vstage`), then the scores of the next block (SCORES: 48 MFMAs, K from `kstage`) into w.s.
//   output: for each V^T fragment (row block e, 32-key chunk cc), four MFMAs (query tiles u);
//           `vbase[cc]`: this lane's byte offset of its V^T chunk at row block 0 (e adds 16 rows).
//   scores: three K=32 steps over dims 0..95 (Q zero past 71, so whatever finite K bytes sit
//           there vanish), step-outer so that four independent MFMAs separate the dependent
//           ones; all three of an accumulator have one shape, which the matrix core forwards
//           back to back. `kbase`: this lane's byte offset of its K chunk (row lane%16, chunk
//           lane/16) at key tile 0 (key tile t adds 16 rows, step ks 64 bytes).
// Fragments are read ahead of their MFMAs: V^T three fragments ahead, K one key tile ahead, the
// first two K tiles during the last output MFMAs. The sched_group_barrier sequence pins that
// order (left alone, the scheduler sinks each read next to its first use and the wave waits out
// the LDS latency in front of every group).
template <bool OUT, bool SCORES>
__device__ __forceinline__ void matrix_phase(WaveState& w, const char* vstage, const int (&vbase)[2],
                                             const char* kstage, int kbase) {
    constexpr int kVF = 10;        // V^T fragments (e, cc)
    constexpr int kKF = 3 * kKT;   // K fragments in MFMA order: p = 4 ks + t
    bf16x8_t vf[kVF];
    bf16x8_t kf[kKF];
    auto read_v = [&](int i) { vf[i] = ld_frag(vstage + vbase[i & 1] + (i >> 1) * 16 * 128); };
    auto read_k = [&](int p) {
        kf[p] = ld_frag(kstage + kbase + (p % kKT) * 16 * kKRow + (p / kKT) * 64);
    };
    if (OUT) {
        read_v(0);
        read_v(1);
        read_v(2);
#pragma unroll
        for (int i = 0; i < kVF; ++i) {
#pragma unroll
            for (int u = 0; u < kQT; ++u)
                w.o[i >> 1][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[i], w.pf[u][i & 1], w.o[i >> 1][u], 0, 0, 0);
            if (i + 3 < kVF) read_v(i + 3);
            else if (SCORES && i >= kVF - 2) read_k(i - (kVF - 2));
        }
    } else if (SCORES) {
        read_k(0);
        read_k(1);
    }
    if (SCORES) {
        // The first K step accumulates onto -m, so the scores come out as s c - m (Q holds c).
        // Step-outer, so -m is live for the first step only; each K fragment is read two
        // fragments (eight MFMAs) ahead of its use.
        f32x4_t negm[kQT];
#pragma unroll
        for (int u = 0; u < kQT; ++u) negm[u] = f32x4_t{-w.mc[u], -w.mc[u], -w.mc[u], -w.mc[u]};
#pragma unroll
        for (int p = 0; p < kKF; ++p) {
            const int t = p % kKT, ks = p / kKT;
#pragma unroll
            for (int u = 0; u < kQT; ++u)
                w.s[t][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    kf[p], w.qf[u][ks], ks == 0 ? negm[u] : w.s[t][u], 0, 0, 0);
            if (p + 2 < kKF) read_k(p + 2);
        }
    }
    // the issue order
    if (OUT) {
        __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
        for (int i = 0; i < kVF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, kQT, 0);
            if (i + 3 < kVF || (SCORES && i >= kVF - 2)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    } else if (SCORES) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    if (SCORES) {
#pragma unroll
        for (int p = 0; p < kKF; ++p) {
            __builtin_amdgcn_sched_group_barrier(0x008, kQT, 0);
            if (p + 2 < kKF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    }
}

__device__ __forceinline__ float lane_max2(float m, bool swap32) {
    const uint32_t x = __float_as_uint(m);
    const auto r = swap32 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                          : __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Softmax of the block whose scores are in w.s: masking, the block maximum (the 64 keys of a
// query sit in lanes lr, lr+16, lr+32, lr+48), the lazy rescale, P = exp2(s c - m) in bf16,
// regrouped into w.pf.
template <bool MASKED, bool FIRST>
__device__ __forceinline__ void softmax(WaveState& w, const Flash72Args& a, int blk,
                                        unsigned long long bits_all, bool all_masked, int g) {
    constexpr bool first = FIRST;   // a compile-time branch: a run-time one keeps both forms of S live
    if (MASKED) {
        const unsigned long long bits = bits_all >> (4 * g);
        const unsigned long long inrange =
            (blk * kKV + kKV <= a.Skv) ? ~0ull : (((1ull << (a.Skv - blk * kKV)) - 1ull) >> (4 * g));
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int bit = 16 * t + r;
                const bool ok = all_masked ? ((inrange >> bit) & 1ull) : ((bits >> bit) & 1ull);
#pragma unroll
                for (int u = 0; u < kQT; ++u) {
                    const float v = all_masked ? 0.0f : w.s[t][u][r];
                    w.s[t][u][r] = ok ? v : -INFINITY;
                }
            }
    }
    if (first) {
        // the first block sets the maximum: per query, over its 64 keys (lanes lr + 16 g)
#pragma unroll
        for (int u = 0; u < kQT; ++u) {
            float m = max3(w.s[0][u][0], w.s[0][u][1], w.s[0][u][2]);
            m = max3(m, w.s[0][u][3], w.s[1][u][0]);
            m = max3(m, w.s[1][u][1], w.s[1][u][2]);
            m = max3(m, w.s[1][u][3], w.s[2][u][0]);
            m = max3(m, w.s[2][u][1], w.s[2][u][2]);
            m = max3(m, w.s[2][u][3], w.s[3][u][0]);
            m = max3(m, w.s[3][u][1], w.s[3][u][2]);
            m = fmaxf(m, w.s[3][u][3]);
            m = lane_max2(m, true);
            m = lane_max2(m, false);
            w.mc[u] = m;
        }
        // x = s c - m in place (the first block's scores were formed against m = 0); later
        // blocks' scores arrive as s c - m from the matrix cores
#pragma unroll
        for (int t = 0; t < kKT; ++t)
#pragma unroll
            for (int u = 0; u < kQT; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) w.s[t][u][r] -= w.mc[u];
    }
    if (!first) {
        // Later blocks move the maximum only when one of their scores exceeds it by more than
        // the threshold: one maximum over this lane's 64 values and a wave vote decide; the exact
        // per-query maxima (across lanes) are formed only then.
        float mx[kKT];
#pragma unroll
        for (int t = 0; t < kKT; ++t) {
            float m = max3(w.s[t][0][0], w.s[t][0][1], w.s[t][0][2]);
            m = max3(m, w.s[t][0][3], w.s[t][1][0]);
            m = max3(m, w.s[t][1][1], w.s[t][1][2]);
            m = max3(m, w.s[t][1][3], w.s[t][2][0]);
            m = max3(m, w.s[t][2][1], w.s[t][2][2]);
            m = max3(m, w.s[t][2][3], w.s[t][3][0]);
            m = max3(m, w.s[t][3][1], w.s[t][3][2]);
            mx[t] = fmaxf(m, w.s[t][3][3]);
        }
        const float m_all = fmaxf(max3(mx[0], mx[1], mx[2]), mx[3]);
        if (__any(m_all > kRescaleThreshold)) {
#pragma unroll
            for (int u = 0; u < kQT; ++u) {
                float m = max3(w.s[0][u][0], w.s[0][u][1], w.s[0][u][2]);
                m = max3(m, w.s[0][u][3], w.s[1][u][0]);
                m = max3(m, w.s[1][u][1], w.s[1][u][2]);
                m = max3(m, w.s[1][u][3], w.s[2][u][0]);
                m = max3(m, w.s[2][u][1], w.s[2][u][2]);
                m = max3(m, w.s[2][u][3], w.s[3][u][0]);
                m = max3(m, w.s[3][u][1], w.s[3][u][2]);
                m = fmaxf(m, w.s[3][u][3]);
                m = lane_max2(m, true);
                m = lane_max2(m, false);
                const float dm = fmaxf(m, 0.0f);   // the query's new maximum is mc + dm
                const float alpha = __builtin_amdgcn_exp2f(-dm);
                w.mc[u] += dm;
#pragma unroll
                for (int e = 0; e < 5; ++e)
#pragma unroll
                    for (int r = 0; r < 4; ++r) w.o[e][u][r] *= alpha;
#pragma unroll
                for (int t = 0; t < kKT; ++t)
#pragma unroll
                    for (int r = 0; r < 4; ++r) w.s[t][u][r] -= dm;
            }
        }
    }
#pragma unroll
    for (int u = 0; u < kQT; ++u)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            uint32_t x[2], y[2];   // key tiles 2cc and 2cc+1, bf16 pairs of keys (4g, 4g+1), (4g+2, 4g+3)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x2_t px, py;   // v_cvt_pk_bf16_f32: round to nearest even (P is finite)
                px[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[2 * cc][u][2 * h]));
                px[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[2 * cc][u][2 * h + 1]));
                py[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[2 * cc + 1][u][2 * h]));
                py[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[2 * cc + 1][u][2 * h + 1]));
                x[h] = __builtin_bit_cast(uint32_t, px);
                y[h] = __builtin_bit_cast(uint32_t, py);
            }
            // keys 32cc + 4g .. +3 and 32cc + 16 + 4g .. +3: V^T's slots 8g .. 8g+7 of the chunk
            const uint4 packed = make_uint4(x[0], x[1], y[0], y[1]);
            w.pf[u][cc] = *reinterpret_cast<const bf16x8_t*>(&packed);
        }
}

// RESIDENT (kv_len <= 448): every key block is loaded once, up front, into a stage of its own;
// after one barrier each wave runs its blocks through without further synchronisation (the two
// waves of a SIMD drift apart, so one's softmax overlaps the other's MFMAs).
// SPLIT (never with RESIDENT): a key split of a.splits, written as an fp32 partial to a.part.
// WAVES: waves per workgroup, 64 queries each. The streaming pipeline needs its two groups of four;
// the resident variant runs with fewer when a full workgroup would leave CUs idle (short query
// sequences): its waves run independently after the one barrier.
template <bool MASKED, bool RESIDENT, bool SPLIT, int WAVES = kWaves>
__global__ void __launch_bounds__(WAVES * 64, 1) k_flash72(Flash72Args a) {
    static_assert(WAVES == kWaves || (RESIDENT && (WAVES == 4 || WAVES == 2 || WAVES == 1)),
                  "fewer waves only for the resident variant");
    constexpr int kNumStages = RESIDENT ? kResidentBlocks : kStages;
    __shared__ __attribute__((aligned(1024))) char smem[kNumStages * kStage];
    __shared__ unsigned long long blk_bits[kMaxBlocks];
    __shared__ int live[kMaxBlocks];
    __shared__ int nlive_s, all_masked_s, empty_s;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lr = lane & 15, g = lane >> 4;

    // ---- which (b, h, query block, key split): the blocks of one (b, h) stay on one XCD ----
    const int splits = SPLIT ? a.splits : 1;
    const int T = a.B * a.H * a.qblocks * splits;
    int bid = blockIdx.x;
    if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
    const int split = SPLIT ? bid % splits : 0;
    if (SPLIT) bid /= splits;
    const int bh = bid / a.qblocks;
    const int b = bh / a.H, h = bh - b * a.H;
    const int q_base = (bid - bh * a.qblocks) * (WAVES * kQPerWave) + wave * kQPerWave;
    const int nblk = (a.Skv + kKV - 1) / kKV;
    const int kb0 = SPLIT ? split * nblk / splits : 0;
    const int kb1 = SPLIT ? (split + 1) * nblk / splits : nblk;

    WaveState w;
    // Q fragments first, so their latency overlaps the set-up below
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        const int q = q_base + u * 16 + lr;
        const bf16_t* qrow = a.q + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_q + h * D;
#pragma unroll
        for (int ks = 0; ks < 3; ++ks) {
            const int d0 = ks * 32 + g * 8;
            bf16x8_t f;
#pragma unroll
            for (int e = 0; e < 8; ++e) f[e] = static_cast<__bf16>(0.0f);
            if (q < a.Sq && d0 < D) f = ld_frag(reinterpret_cast<const char*>(qrow + d0));
            w.qf[u][ks] = f;
        }
    }

    // ---- key validity per block (bit i = key 64 blk + i is in range and unmasked) ----
    if (MASKED) {
        for (int blk = wave; blk < nblk; blk += WAVES) {
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
    for (int i = threadIdx.x; i < kNumStages * 8 * 128 / 16; i += WAVES * 64) {
        const int st = i / 64, x = i - st * 64;   // 64 16-byte words per stage
        const uint32_t one = x < 8 ? 0x3f803f80u : 0u;
        *reinterpret_cast<uint4*>(smem + st * kStage + kKBytes + 72 * 128 + x * 16) =
            make_uint4(one, one, one, one);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int n = 0;
        unsigned long long any = MASKED ? 0ull : 1ull;
        if (MASKED)
            for (int blk = 0; blk < nblk; ++blk) any |= blk_bits[blk];
        const bool all_masked = any == 0ull;   // over the whole row, whatever this split's range
        for (int blk = kb0; blk < kb1; ++blk)
            if (!MASKED || all_masked || blk_bits[blk] != 0ull) live[n++] = blk;
        // A key split whose blocks are all masked still runs its first block (every score -inf)
        // and then writes an empty partial: the pipeline needs at least one block.
        if (SPLIT) {
            empty_s = n == 0 ? 1 : 0;
            if (n == 0) live[n++] = kb0;
        }
        nlive_s = n;
        all_masked_s = all_masked ? 1 : 0;
    }
    __syncthreads();
    const int n = nlive_s;
    const bool all_masked = MASKED && all_masked_s != 0;

    // fragment byte offsets within a stage
    const int kbase = lr * kKRow + g * 16;   // K step 2, g >= 1: the next row's finite bytes (Q is 0)
    int vbase[2];
    {
        const int sw = (lr >> 1) & 7;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) vbase[cc] = kKBytes + lr * 128 + (((cc * 4 + g) ^ sw) << 4);
    }
#pragma unroll
    for (int e = 0; e < 5; ++e)
#pragma unroll
        for (int u = 0; u < kQT; ++u) w.o[e][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kQT; ++u) w.mc[u] = 0.0f;   // the first block's scores are formed against 0

    // The Q loads are drained here, where the compiler sees it: otherwise it waits for them
    // (vmcnt(0), which also drains the DMA in flight) at their first use in every phase.
    s_waitcnt<0, 15>();
    // Q carries the score scale in log2 units, c = scale log2(e), rounded to bf16 once here, so
    // the matrix cores deliver s c - m and the softmax spends no multiply-add per score.
#pragma unroll
    for (int u = 0; u < kQT; ++u)
#pragma unroll
        for (int ks = 0; ks < 3; ++ks)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w.qf[u][ks][e] = static_cast<__bf16>(static_cast<float>(w.qf[u][ks][e]) * a.c);

    // ---- the phases ----
    // Phase p is bracketed by workgroup barriers. Block j (position j of the live list) sits in
    // stage j % 4. Waves 0-3 multiply in even phases (2j: output of block j-1, scores of block
    // j) and run the softmax of block j in phase 2j+1; waves 4-7 are one phase later (matrix in
    // 2j+1, softmax of block j in 2j+2). Block j's K is read in phases 2j, 2j+1 and its V^T in
    // 2j+2, 2j+3. Waves 0-3 also load: at the end of phase 2j they issue block j+2 into stage
    // (j+2) % 4, which held block j-2, last read in phase 2j-1. The vector phases are the longer
    // ones, so the DMA instructions (which can hold their wave while the address unit is busy)
    // go where the wave would otherwise wait at the barrier. Before each even phase 2j waves 0-3
    // wait until block j has landed (block j+1 may still be in flight), so every block has three
    // phases to arrive. Past the last block the loads repeat it, which keeps every wait count
    // identical.
    auto bits_of = [&](int j) -> unsigned long long { return MASKED ? blk_bits[live[j]] : ~0ull; };
    if (RESIDENT) {
        const bf16_t* kbh = a.k + static_cast<int64_t>(b) * a.Skv * a.ld_k + h * D;
        const bf16_t* vbh = a.vt + (static_cast<int64_t>(b) * a.H + h) * D * a.vt_ld;
        const int last_full = a.Skv / kKV;
        for (int j = 0; j < n; ++j) {
            const int blk = live[j];
            for (int item = wave; item < 20; item += WAVES)
                dma_item(smem + j * kStage, a, kbh, vbh, item, lane, blk * kKV,
                         MASKED && blk >= last_full);
        }
        wait_and_join<0>();
        auto res_stage = [&](int j) -> char* { return smem + j * kStage; };
        matrix_phase<false, true>(w, nullptr, vbase, res_stage(0), kbase);
        softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, g);
        for (int j = 1; j < n; ++j) {
            matrix_phase<true, true>(w, res_stage(j - 1), vbase, res_stage(j), kbase);
            softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, g);
        }
        matrix_phase<true, false>(w, res_stage(n - 1), vbase, nullptr, kbase);
    } else {
    auto stage_of = [&](int j) -> char* { return smem + (j & (kStages - 1)) * kStage; };
    if (wave < kDmaWaves) {
        // waves 0-3: the matrix phase in even phases, then the DMA of block j+2
        const bf16_t* kbh = a.k + static_cast<int64_t>(b) * a.Skv * a.ld_k + h * D;
        const bf16_t* vbh = a.vt + (static_cast<int64_t>(b) * a.H + h) * D * a.vt_ld;
        const int last_full = a.Skv / kKV;   // blocks below this one hold 64 real keys
        const DmaPlan plan = dma_plan(a, wave, lane);
        auto issue = [&](int j) {
            const int blk = live[min(j, n - 1)];
            dma_block(stage_of(j), a, plan, kbh, vbh, wave, lane, blk * kKV, MASKED && blk >= last_full);
        };
        issue(0);
        issue(1);
        wait_and_join<kDmaPerWave>();                            // phase 0: block 0 has landed
        matrix_phase<false, true>(w, nullptr, vbase, stage_of(0), kbase);
        issue(2);
        if (n > 1) {   // block 0's softmax peeled off, so FIRST is known at compile time
            wait_and_join<63>();                                 // phase 1
            softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, g);
            wait_and_join<kDmaPerWave>();                        // phase 2: block 1 has landed
            matrix_phase<true, true>(w, stage_of(0), vbase, stage_of(1), kbase);
            issue(3);
            for (int j = 2; j < n; ++j) {
                wait_and_join<63>();                             // phase 2j-1
                softmax<MASKED, false>(w, a, live[j - 1], bits_of(j - 1), all_masked, g);
                wait_and_join<kDmaPerWave>();                    // phase 2j: block j has landed
                matrix_phase<true, true>(w, stage_of(j - 1), vbase, stage_of(j), kbase);
                issue(j + 2);
            }
            wait_and_join<63>();                                 // phase 2n-1
            softmax<MASKED, false>(w, a, live[n - 1], bits_of(n - 1), all_masked, g);
        } else {
            wait_and_join<63>();                                 // phase 1
            softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, g);
        }
        wait_and_join<63>();                                     // phase 2n
        matrix_phase<true, false>(w, stage_of(n - 1), vbase, nullptr, kbase);
        wait_and_join<63>();                                     // phase 2n+1
        s_waitcnt<0, 15>();   // the trailing copies
    } else {
        wait_and_join<63>();                                     // phase 0
        wait_and_join<63>();                                     // phase 1
        matrix_phase<false, true>(w, nullptr, vbase, stage_of(0), kbase);
        wait_and_join<63>();                                     // phase 2
        softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, g);
        for (int j = 1; j < n; ++j) {
            wait_and_join<63>();                                 // phase 2j+1
            matrix_phase<true, true>(w, stage_of(j - 1), vbase, stage_of(j), kbase);
            wait_and_join<63>();                                 // phase 2j+2
            softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, g);
        }
        wait_and_join<63>();                                     // phase 2n+1
        matrix_phase<true, false>(w, stage_of(n - 1), vbase, nullptr, kbase);
    }
    }

    // ---- a key split's partial: O unnormalised, the row sum and the running maximum ----
    if constexpr (SPLIT) {
        const bool empty = empty_s != 0;
#pragma unroll
        for (int u = 0; u < kQT; ++u) {
            const int q = q_base + u * 16 + lr;
            if (q >= a.Sq) continue;
            float* dst = a.part + ((static_cast<int64_t>(split) * a.B + b) * a.H + h) * a.Sq * 80 +
                         static_cast<int64_t>(q) * 80;
#pragma unroll
            for (int e = 0; e < 5; ++e) {
                const int d = e * 16 + g * 4;
                if (d < D) {
                    *reinterpret_cast<f32x4_t*>(dst + d) = empty ? f32x4_t{0.f, 0.f, 0.f, 0.f} : w.o[e][u];
                } else if (d == D) {   // row 72 is the sum; an empty split contributes nothing
                    *reinterpret_cast<f32x4_t*>(dst + d) =
                        empty ? f32x4_t{0.f, -INFINITY, 0.f, 0.f} : f32x4_t{w.o[e][u][0], w.mc[u], 0.f, 0.f};
                }
            }
        }
        return;
    }

    // ---- normalise and store: lane holds out[q][d..d+3], d = 16e + 4g; O^T row 72 is the sum ----
#pragma unroll
    for (int u = 0; u < kQT; ++u) {
        // One correctly rounded reciprocal per query, then a multiply per output (within one fp32
        // ulp of the quotient before the bf16 rounding): an IEEE division per output was ~10
        // instructions, 72 of them per lane.
        const float rl = __frcp_rn(__shfl(w.o[4][u][0], 32 + lr, 64));
        const int q = q_base + u * 16 + lr;
        if (q >= a.Sq) continue;
        bf16_t* dst = a.out + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_o + h * D;
#pragma unroll
        for (int e = 0; e < 5; ++e) {
            const int d = e * 16 + g * 4;
            if (d >= D) continue;
            uint2 x;
            x.x = static_cast<uint32_t>(f2bf(w.o[e][u][0] * rl)) |
                  (static_cast<uint32_t>(f2bf(w.o[e][u][1] * rl)) << 16);
            x.y = static_cast<uint32_t>(f2bf(w.o[e][u][2] * rl)) |
                  (static_cast<uint32_t>(f2bf(w.o[e][u][3] * rl)) << 16);
            *reinterpret_cast<uint2*>(dst + d) = x;
        }
    }
}

// V [batch, kv_len, ld_v] (head h at columns 72h..72h+71) -> V^T rows of vt_ld keys, zero-padded
// past kv_len, keys in vt_pos order. One workgroup per (b, h, 64-key block), through LDS.
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
        if (kv0 + r < vt_ld) vt[((static_cast<int64_t>(b) * H + h) * D + d) * vt_ld + vt_pos(kv0 + r)] = tile[r][d];
    }
}

// The key splits' partials into the output: per (b, h, q), M = the largest running maximum,
// out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), in split order. One thread per 8 dims.
__global__ void __launch_bounds__(256) k_flash72_combine(const float* __restrict__ part, int splits,
                                                         int B, int H, int Sq, bf16_t* out,
                                                         int64_t ld_o) {
    constexpr int kChunks = D / 8;   // 9
    const int64_t rows = static_cast<int64_t>(B) * H * Sq;
    const int64_t split_stride = rows * 80;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < rows * kChunks;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = i / kChunks;   // ((b * H + h) * Sq + q)
        const int c = static_cast<int>(i - row * kChunks);
        const float* p = part + row * 80;
        float mx = -INFINITY;
        for (int sp = 0; sp < splits; ++sp) mx = fmaxf(mx, p[sp * split_stride + 73]);
        float l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < splits; ++sp) {
            const float* ps = p + sp * split_stride;
            const float wgt = __builtin_amdgcn_exp2f(ps[73] - mx);   // 0 for an empty split
            l = __fmaf_rn(ps[72], wgt, l);
            const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(ps + c * 8);
            const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(ps + c * 8 + 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                o[r] = __fmaf_rn(lo[r], wgt, o[r]);
                o[4 + r] = __fmaf_rn(hi[r], wgt, o[4 + r]);
            }
        }
        const float rl = __frcp_rn(l);
        float v[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = o[r] * rl;
        const int64_t q = row % Sq, bh = row / Sq;
        const int64_t b = bh / H, h = bh - b * H;
        uint32_t wv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            wv[r] = static_cast<uint32_t>(f2bf(v[2 * r])) | (static_cast<uint32_t>(f2bf(v[2 * r + 1])) << 16);
        *reinterpret_cast<uint4*>(out + (b * Sq + q) * ld_o + h * D + c * 8) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
}

// Per-device partials for split calls that bring no buffer of their own, grown on demand.
float* flash72_part_workspace(int64_t floats) {
    static std::mutex mu;
    static void* ptr[64] = {};
    static int64_t cap[64] = {};
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < 64, "attention: device index out of range");
    std::lock_guard<std::mutex> lock(mu);
    if (cap[dev] < floats) {
        if (ptr[dev]) hip_check(hipFree(ptr[dev]), "hipFree");
        ptr[dev] = nullptr;
        cap[dev] = 0;
        hip_check(hipMalloc(&ptr[dev], static_cast<size_t>(floats) * sizeof(float)),
                  "hipMalloc (attention partials)");
        cap[dev] = floats;
    }
    return static_cast<float*>(ptr[dev]);
}

template <bool MASKED>
void launch_resident_m(int waves, int grid, const Flash72Args& a, hipStream_t s) {
    switch (waves) {
        case 1: k_flash72<MASKED, true, false, 1><<<grid, 64, 0, s>>>(a); break;
        case 2: k_flash72<MASKED, true, false, 2><<<grid, 128, 0, s>>>(a); break;
        case 4: k_flash72<MASKED, true, false, 4><<<grid, 256, 0, s>>>(a); break;
        default: k_flash72<MASKED, true, false, kWaves><<<grid, kThreads, 0, s>>>(a); break;
    }
}
void launch_resident(bool masked, int waves, int grid, const Flash72Args& a, hipStream_t s) {
    if (masked) launch_resident_m<true>(waves, grid, a, s);
    else launch_resident_m<false>(waves, grid, a, s);
}

}  // namespace

int64_t flash72_vt_ld(int64_t kv_len) { return (kv_len + kKV - 1) / kKV * kKV; }

int flash72_splits(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len, const void* out,
                   int64_t ld_o) {
    const int64_t nblk = (kv_len + kKV - 1) / kKV;
    if (kv_len <= kResidentBlocks * kKV) return 1;   // the resident kernel does not split
    // the combine stores 8 outputs at a time
    if (ld_o % 8 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0) return 1;
    const int64_t wgs = batch * heads * ((q_len + kQPerWg - 1) / kQPerWg);
    int cus = 0, dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    if (wgs * 2 > cus) return 1;
    int best = 1;
    for (int sp = 2; sp <= 8; ++sp)
        if (wgs * sp <= cus && nblk >= 2 * sp) best = sp;
    return best;
}

int64_t flash72_part_floats(int64_t batch, int64_t heads, int64_t q_len, int splits) {
    return splits > 1 ? static_cast<int64_t>(splits) * batch * heads * q_len * 80 : 0;
}

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
                    const void* key_mask, bool mask_f32, hipStream_t s, int splits,
                    float* part, int64_t part_floats) {
    if (batch * heads * q_len == 0) return;
    require(kv_len > 0, "attention: kv_len must be positive");
    require(kv_len <= kMaxBlocks * kKV, "attention (head_dim 72): kv_len above 16384");
    require(vt_ld >= flash72_vt_ld(kv_len), "attention (head_dim 72): V^T rows too short");
    require(kv_len * ld_k < (int64_t{1} << 31) && D * vt_ld < (int64_t{1} << 31),
            "attention (head_dim 72): one (batch, head) slice of K or V^T spans 2^31 elements");
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
    a.c = scale * 1.4426950408889634f;
    const bool masked = key_mask || kv_len % kKV != 0;
    const bool resident = kv_len <= kResidentBlocks * kKV;
    // Resident launches take fewer waves per workgroup until the grid covers the CUs (one
    // workgroup per CU: the resident stages fill the LDS), so a short query sequence runs one
    // wave per SIMD on more CUs instead of two per SIMD on a few.
    int waves = kWaves;
    if (resident) {
        int cus = 0, dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
                  "hipDeviceGetAttribute");
        auto wgs = [&](int w) { return batch * heads * ((q_len + w * kQPerWave - 1) / (w * kQPerWave)); };
        while (waves > 1 && wgs(waves) < cus) waves /= 2;
    }
    a.qblocks = static_cast<int>((q_len + waves * kQPerWave - 1) / (waves * kQPerWave));
    if (splits <= 0) splits = flash72_splits(batch, heads, q_len, kv_len, out, ld_o);
    const int64_t nblk = (kv_len + kKV - 1) / kKV;
    require(splits >= 1 && splits <= 8 && (splits == 1 || (!resident && nblk >= splits)),
            "attention (head_dim 72): " + std::to_string(splits) + " key splits of " +
                std::to_string(nblk) + " key blocks");
    if (splits > 1) {
        const int64_t floats = flash72_part_floats(batch, heads, q_len, splits);
        if (part) {
            require(part_floats >= floats && reinterpret_cast<uintptr_t>(part) % 16 == 0,
                    "attention (head_dim 72): the partial buffer holds " + std::to_string(part_floats) +
                        " floats, this call needs " + std::to_string(floats));
        } else {
            part = flash72_part_workspace(floats);
        }
        require(ld_o % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0,
                "attention (head_dim 72): a key-split output needs 16-byte rows");
        a.splits = splits;
        a.part = part;
    }
    const int grid = a.B * a.H * a.qblocks * a.splits;
    const double flops = 4.0 * batch * heads * static_cast<double>(q_len) * kv_len * D;
    ProfileScope ps(q_len == kv_len ? K_ATTN_SELF : K_ATTN_CROSS, s, flops);
    if (a.splits > 1 && masked) k_flash72<true, false, true><<<grid, kThreads, 0, s>>>(a);
    else if (a.splits > 1) k_flash72<false, false, true><<<grid, kThreads, 0, s>>>(a);
    else if (resident) launch_resident(masked, waves, grid, a, s);
    else if (masked) k_flash72<true, false, false><<<grid, kThreads, 0, s>>>(a);
    else k_flash72<false, false, false><<<grid, kThreads, 0, s>>>(a);
    launch_check("attention (flash, head_dim 72)");
    if (a.splits > 1) {
        const int64_t threads = batch * heads * q_len * (D / 8);
        k_flash72_combine<<<static_cast<int>(std::min<int64_t>((threads + 255) / 256, 8192)), 256, 0, s>>>(
            a.part, a.splits, a.B, a.H, a.Sq, out, ld_o);
        launch_check("attention (head_dim 72, key-split combine)");
    }
}

}  // namespace bh
