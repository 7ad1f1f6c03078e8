// Flash attention at head_dim 72 (PixArt-Sigma: 16 heads x 72) on gfx950.
//
//   out = softmax(scale * Q K^T, key mask) V over head-last [batch, seq, heads, 72] Q and K, and
//   V supplied TRANSPOSED: vt[((b * heads + h) * 72 + d) * vt_ld + vt_pos(kv)], zero past
//   kv_len (vt_pos, common.h: keys permuted within 32-key chunks, runs of four kept).
//
// Workgroup: 8 waves, 512 queries of one (batch, head); wave w owns queries 64w..64w+63. Keys
// stream in blocks of 64 through FOUR LDS stages filled by direct global->LDS loads
// (global_load_lds_dwordx4).
//
// Both products run on the matrix cores with the score matrix TRANSPOSED:
//   S^T[kv, q]  = K[kv, :] . Q[q, :]^T      v_mfma_f32_32x32x16_bf16: A = K (LDS), B = Q (registers)
//   O^T[d, q]  += V^T[d, kv] . P^T[kv, q]   v_mfma_f32_16x16x32_bf16: A = V^T (LDS), B = P (registers)
// The score product runs in 32x32 tiles (two key tiles x two query tiles per block and wave) over
// K = 80 dims in five steps of 16, so head_dim 72 pads to 80: 20 MFMAs, 640 matrix-core cycles
// per block and wave, where 16x16x32 tiles would pad it to 96 (48 MFMAs, 768 cycles). Its accumulator gives lane l sixteen keys of
// query l % 32: 8j + 4h + (0..3), j < 4, h = l / 32. Converted to bf16 pairs and swapped once
// between the lane rows 16r..16r+15 (v_permlane16_swap, four per tile), those are two B operands
// of the output product, one per 16-query half, each lane row holding eight keys that V^T keeps
// together (vt_pos, common.h): the matching V^T fragment is one 16-byte LDS read. The output
// product pads head_dim to 80: V^T rows 72..79 sit in LDS with row 72 all ONES, so O^T row 72 is
// the softmax denominator sum_kv P[kv], accumulated from the same bf16 P as the numerator. The
// score padding carries the running maximum: Q's dim 72 holds -m (dims 73..79 zero) and the
// upper lanes of the last K step read that ones row instead of K, so the matrix cores deliver
// s c - m; whatever finite K bytes would sit past dim 71 never enter.
//
// Schedule: a wave alternates a matrix phase (the output product of block j-1, then the scores of
// block j: 40 + 20 MFMAs) and a vector phase (softmax of block j: maximum, exp2, conversion to bf16).
// Waves 0-3 and 4-7 run one phase apart, separated by a workgroup barrier per phase, so on every
// SIMD one wave's exponentials overlap the other wave's MFMAs. Waves 0-3 also issue the DMA, at
// the end of their matrix phases (the shorter ones).
//
// Softmax: scores stay fp32; exp2(s * scale * log2e - m) with the running maximum m kept in those
// units. Q is multiplied by c = scale * log2e once, as it is loaded (one extra bf16 rounding of
// q c), and the score product's dim 72 adds -m, so the matrix cores deliver s c - m and the
// vector phase spends no operation per score on it. m is kept a bf16 value, so -m in Q is exact.
// The first block sets m (its scores are formed against 0); a later block moves it (and rescales
// O by exp2(m_old - m_new)) only when one of its scores exceeds it by more than 8: any fixed m
// gives the same normalised result, and the threshold bounds every P by about 2^8. The
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
constexpr int kQT = 4;                        // 16-query tiles per wave (output product)
constexpr int kST = 2;                        // 32-query tiles per wave (score product)
constexpr int kSK = 2;                        // 32-key tiles per block (score product)
constexpr int kSSteps = 5;                    // K = 16 steps of the score product: dims 0..79
constexpr int kKRow = D * 2;                  // 144 bytes per K row in LDS
constexpr int kKBytes = kKV * kKRow;          // 9216 = 9 DMA blocks
constexpr int kVRows = 80;                    // 72 dims + the ones row + zero rows
constexpr int kVBytes = kVRows * 128;         // 128 bytes = 64 keys per V^T row
constexpr int kOnesOff = kKBytes + D * 128;   // V^T row 72 of a stage: 64 bf16 ones
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
// The same with a wave-uniform base address in SGPRs and this lane's 32-bit byte offset from it
// (the saddr form: the per-lane address costs no vector instruction).
__device__ __forceinline__ void dma16s(uint32_t voff, const void* base, const char* lds) {
    const uint32_t l = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(lds)));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(l), "v"(voff), "s"(base)
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
// the branch on it is scalar. DmaPlan holds this lane's byte offset for each instruction from the
// block's first key row of K or V^T, in 32 bits (the launcher checks that one (b, h) slice spans
// fewer than 2^31 elements); a block's DMA then needs only its two scalar base addresses.
struct DmaPlan {
    uint32_t off[kDmaPerWave];
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
            p.off[i] = 2u * static_cast<uint32_t>(d * static_cast<int>(a.vt_ld) + c * 8);
        } else {
            const int lg = (item < 9 ? item : 0) * 64 + lane;   // spares (18, 19) re-load block 0
            const int row = lg / 9, ch = lg - row * 9;
            p.off[i] = 2u * static_cast<uint32_t>(row * static_cast<int>(a.ld_k) + ch * 8);
        }
    }
    return p;
}

// Key block starting at key kv0 (wave-uniform) into `stage`. `partial`: the block runs past the
// last key, whose row then stands in for the missing ones (their scores are masked).
__device__ __forceinline__ void dma_block(char* stage, const Flash72Args& a, const DmaPlan& p,
                                          const bf16_t* kbh, const bf16_t* vbh, int wave, int lane,
                                          int kv0, bool partial) {
    const bf16_t* kb = kbh + static_cast<int64_t>(kv0) * a.ld_k;
    const bf16_t* vb = vbh + kv0;
#pragma unroll
    for (int i = 0; i < kDmaPerWave; ++i) {
        char* dst = stage + dma_dst(i, wave);
        if (dma_is_v(i, wave)) {
            dma16s(p.off[i], vb, dst);
        } else if (!partial) {
            dma16s(p.off[i], kb, dst);
        } else {
            const int row = dma_krow(i, wave, lane);
            const int key = min(kv0 + row, a.Skv - 1);   // from kb: key - kv0 - row <= 0 rows
            dma16(kb + (static_cast<int>(p.off[i] / 2u) + (key - kv0 - row) * static_cast<int>(a.ld_k)), dst);
        }
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

// This file is compiled with -fno-honor-nans: with IEEE NaN rules the compiler would first quiet
// every MFMA result with an extra v_max before each maximum. Scores here are finite, or -inf for
// masked keys.
__device__ __forceinline__ bf16x8_t ld_frag(const char* p) {
    return *reinterpret_cast<const bf16x8_t*>(p);
}

// Per-wave state of the pipeline.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

struct WaveState {
    bf16x8_t qf[kST][kSSteps]; // Q fragments: query 32 qt + l%32, dims 16 s + 8 h .. +7 (h = l/32);
                               // lanes h = 1 of step 4 hold (-m, 0, ..., 0) for dims 72..79
    f32x4_t o[5][kQT];         // O^T accumulators: rows 16e + 4g .. +3 (row 72 = denominator)
    f32x16_t s[kSK][kST];      // S^T of the current block: element r is key 32 kt + 8 (r/4) + 4 h + r%4,
                               // query 32 qt + l%32
    bf16x8_t pf[kQT][2];       // P of the previous block, as the second product's B operand
    float mc[kST];             // running maximum (scaled, log2 units, a bf16 value) of query 32 qt + l%32
};

// The matrix phase: O^T += V^T P^T for the block whose P is in w.pf (OUT: 40 MFMAs 16x16x32,
// V^T from `vstage`), then the scores of the next block (SCORES: 20 MFMAs 32x32x16, K from
// `kstage`) into w.s.
//   output: for each V^T fragment (row block e, 32-key chunk cc), four MFMAs (query tiles u);
//           `vbase[cc]`: this lane's byte offset of its V^T chunk at row block 0 (e adds 16 rows).
//   scores: five K=16 steps over dims 0..79, step-outer so that four independent MFMAs separate
//           the dependent ones. `kb[0]`: this lane's byte offset of its K chunk (row l%32, dims
//           8h..8h+7) at key tile 0 and step 0 (key tile kt adds 32 rows, step s 32 bytes);
//           `kb[1 + kt]`: the offset for step 4 -- dims 64..71 of its row for h = 0, the ones row
//           (kOnesOff) for h = 1, which pairs with -m in Q's dim 72.
// Fragments are read ahead of their MFMAs: V^T three fragments ahead, K two ahead, the first two
// K fragments during the last output MFMAs. The sched_group_barrier sequence pins that order (left
// alone, the scheduler sinks each read next to its first use and the wave waits out the LDS
// latency in front of every group).
constexpr int kVAhead = 3;   // V^T fragments read ahead of their MFMAs
constexpr int kKAhead = 2;   // K fragments read ahead of their MFMAs
template <bool OUT, bool SCORES>
__device__ __forceinline__ void matrix_phase(WaveState& w, const char* vstage, const int (&vbase)[2],
                                             const char* kstage, const int (&kb)[3]) {
    constexpr int kVF = 10;                // V^T fragments (e, cc)
    constexpr int kKF = kSSteps * kSK;     // K fragments in MFMA order: p = 2 s + kt
    bf16x8_t vf[kVF];
    bf16x8_t kf[kKF];
    auto read_v = [&](int i) { vf[i] = ld_frag(vstage + vbase[i & 1] + (i >> 1) * 16 * 128); };
    auto read_k = [&](int p) {
        const int kt = p % kSK, st = p / kSK;
        kf[p] = ld_frag(kstage + (st < kSSteps - 1 ? kb[0] + kt * 32 * kKRow + st * 32 : kb[1 + kt]));
    };
    if (OUT) {
#pragma unroll
        for (int i = 0; i < kVAhead; ++i) read_v(i);
#pragma unroll
        for (int i = 0; i < kVF; ++i) {
#pragma unroll
            for (int u = 0; u < kQT; ++u)
                w.o[i >> 1][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf[i], w.pf[u][i & 1], w.o[i >> 1][u], 0, 0, 0);
            if (i + kVAhead < kVF) read_v(i + kVAhead);
            else if (SCORES && i >= kVF - kKAhead) read_k(i - (kVF - kKAhead));
        }
    } else if (SCORES) {
#pragma unroll
        for (int p = 0; p < kKAhead; ++p) read_k(p);
    }
    if (SCORES) {
        const f32x16_t zero = {};
#pragma unroll
        for (int p = 0; p < kKF; ++p) {
            const int kt = p % kSK, st = p / kSK;
#pragma unroll
            for (int qt = 0; qt < kST; ++qt)
                w.s[kt][qt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    kf[p], w.qf[qt][st], st == 0 ? zero : w.s[kt][qt], 0, 0, 0);
            if (p + kKAhead < kKF) read_k(p + kKAhead);
        }
    }
    // the issue order
    if (OUT) {
        __builtin_amdgcn_sched_group_barrier(0x100, kVAhead, 0);
#pragma unroll
        for (int i = 0; i < kVF; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, kQT, 0);
            if (i + kVAhead < kVF || (SCORES && i >= kVF - kKAhead)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    } else if (SCORES) {
        __builtin_amdgcn_sched_group_barrier(0x100, kKAhead, 0);
    }
    if (SCORES) {
#pragma unroll
        for (int p = 0; p < kKF; ++p) {
            __builtin_amdgcn_sched_group_barrier(0x008, kST, 0);
            if (p + kKAhead < kKF) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
    }
}

__device__ __forceinline__ float lane_max2(float m, bool swap32) {
    const uint32_t x = __float_as_uint(m);
    const auto r = swap32 ? __builtin_amdgcn_permlane32_swap(x, x, false, false)
                          : __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Maxima of the 32 scores this lane holds for each query tile qt (its query's keys 8j + 4h + i of
// both key tiles): four chains of v_max3 (one per tile), each link taking two new values,
// interleaved so that no link waits on the one before it (a dependent VALU operand needs two
// instructions between producer and consumer here). The empty asm makes each link opaque:
// otherwise the compiler, with NaNs ignored, rebalances the chains into trees of two-input maxima
// (~50 instructions per 64 values instead of 34).
__device__ __forceinline__ float max3_link(float m, float a, float b) {
    m = __builtin_fmaxf(__builtin_fmaxf(m, a), b);
    asm("" : "+v"(m));
    return m;
}
__device__ __forceinline__ void tile_max(const WaveState& w, float (&tm)[kST]) {
    float c[kSK][kST];
#pragma unroll
    for (int kt = 0; kt < kSK; ++kt)
#pragma unroll
        for (int qt = 0; qt < kST; ++qt) c[kt][qt] = max3_link(w.s[kt][qt][0], w.s[kt][qt][1], w.s[kt][qt][2]);
#pragma unroll
    for (int i = 3; i < 15; i += 2)
#pragma unroll
        for (int kt = 0; kt < kSK; ++kt)
#pragma unroll
            for (int qt = 0; qt < kST; ++qt) c[kt][qt] = max3_link(c[kt][qt], w.s[kt][qt][i], w.s[kt][qt][i + 1]);
#pragma unroll
    for (int qt = 0; qt < kST; ++qt)
        tm[qt] = __builtin_fmaxf(__builtin_fmaxf(c[0][qt], w.s[0][qt][15]),
                                 __builtin_fmaxf(c[1][qt], w.s[1][qt][15]));
}

// Q's dim 72 := -m (lanes h = 1 of the last K step; their dims 73..79 stay zero).
__device__ __forceinline__ void set_neg_max(WaveState& w, int h) {
#pragma unroll
    for (int qt = 0; qt < kST; ++qt) {
        bf16x8_t f = {};
        f[0] = static_cast<__bf16>(-w.mc[qt]);   // exact: m is a bf16 value
        if (h) w.qf[qt][kSSteps - 1] = f;
    }
}

// The smallest bf16 value not below x (x finite or -inf). Applied to integers it gives integers:
// below 256 every integer is a bf16 value, from 256 up every bf16 value is an integer.
__device__ __forceinline__ float ceil_bf16(float x) {
    const uint32_t t = __float_as_uint(x) & 0xffff0000u;
    return __uint_as_float(__uint_as_float(t) < x ? t + 0x10000u : t);
}

// P in w.pf times a power of two, per query: pf[u] holds query 16 u + l%16 in every lane row, so
// tile u takes the factor of the lane that holds that query in the score layout. Exact (the
// factor is 2^-k) unless a product falls below the normal range.
__device__ __forceinline__ void scale_p(bf16x8_t& f, float s) {
    uint32_t x[4];
    __builtin_memcpy(x, &f, sizeof x);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        bf16x2_t p;
        p[0] = static_cast<__bf16>(__uint_as_float(x[v] << 16) * s);
        p[1] = static_cast<__bf16>(__uint_as_float(x[v] & 0xffff0000u) * s);
        x[v] = __builtin_bit_cast(uint32_t, p);
    }
    __builtin_memcpy(&f, x, sizeof x);
}

// P = exp2(x) of the scores in w.s into w.pf. Element r = 4j + i of tile (kt, qt) is key
// 32 kt + 8j + 4h + i. Pairs pk[2j + v] hold keys (8j + 4h + 2v, +1). X = pk[0..3] (j = 0, 1) and
// Y = pk[4..7] (j = 2, 3); swapping X's odd lane rows with Y's even ones leaves in X queries
// 32 qt + 0..15 and in Y queries 32 qt + 16..31, lane row r holding keys
// 16 (r & 1) + 4 (r >> 1) + {0..3, 8..11}: the eight keys at V^T slots 8r..8r+7 of the chunk
// (vt_pos).
__device__ __forceinline__ void form_p(WaveState& w) {
#pragma unroll
    for (int qt = 0; qt < kST; ++qt)
#pragma unroll
        for (int kt = 0; kt < kSK; ++kt) {
            uint32_t pk[8];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int v = 0; v < 2; ++v) {
                    bf16x2_t p;   // v_cvt_pk_bf16_f32: round to nearest even (P is finite)
                    p[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[kt][qt][4 * j + 2 * v]));
                    p[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(w.s[kt][qt][4 * j + 2 * v + 1]));
                    pk[2 * j + v] = __builtin_bit_cast(uint32_t, p);
                }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const auto r = __builtin_amdgcn_permlane16_swap(pk[v], pk[4 + v], false, false);
                pk[v] = r[0];
                pk[4 + v] = r[1];
            }
            const uint4 x = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            const uint4 y = make_uint4(pk[4], pk[5], pk[6], pk[7]);
            w.pf[2 * qt][kt] = *reinterpret_cast<const bf16x8_t*>(&x);
            w.pf[2 * qt + 1][kt] = *reinterpret_cast<const bf16x8_t*>(&y);
        }
}

// Softmax of the block whose scores are in w.s: masking, the block maximum (the 64 keys of a
// query sit in lanes l and l ^ 32), P = exp2(s c - m) in bf16 regrouped into w.pf, the lazy
// rescale. The running maximum m is an integer-valued bf16 number: -m in Q's dim 72 is exact and
// a rescale moves it by an integer k, so a rescale multiplies P and O by 2^-k exactly, and P is
// formed before the decision (the maximum and the exponentials interleave; the scores die as
// they are used).
template <bool MASKED, bool FIRST>
__device__ __forceinline__ void softmax(WaveState& w, const Flash72Args& a, int blk,
                                        unsigned long long bits_all, bool all_masked, int h) {
    if (MASKED) {
        const unsigned long long bits = bits_all >> (4 * h);
        const unsigned long long inrange =
            (blk * kKV + kKV <= a.Skv) ? ~0ull : (((1ull << (a.Skv - blk * kKV)) - 1ull) >> (4 * h));
#pragma unroll
        for (int kt = 0; kt < kSK; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int bit = 32 * kt + 8 * (r >> 2) + (r & 3);
                const bool ok = all_masked ? ((inrange >> bit) & 1ull) : ((bits >> bit) & 1ull);
#pragma unroll
                for (int qt = 0; qt < kST; ++qt) {
                    const float v = all_masked ? 0.0f : w.s[kt][qt][r];
                    w.s[kt][qt][r] = ok ? v : -INFINITY;
                }
            }
    }
    float tm[kST];
    tile_max(w, tm);
    if constexpr (FIRST) {
        // The first block sets the maximum, per query over its 64 keys (lanes l, l ^ 32), rounded
        // up to an integer-valued bf16 number; its scores were formed against m = 0, so x = s c - m
        // is formed here (later blocks' scores arrive as s c - m from the matrix cores).
#pragma unroll
        for (int qt = 0; qt < kST; ++qt) w.mc[qt] = ceil_bf16(ceilf(lane_max2(tm[qt], true)));
#pragma unroll
        for (int kt = 0; kt < kSK; ++kt)
#pragma unroll
            for (int qt = 0; qt < kST; ++qt)
#pragma unroll
                for (int r = 0; r < 16; ++r) w.s[kt][qt][r] -= w.mc[qt];
        set_neg_max(w, h);
        form_p(w);
    } else {
        // Later blocks move the maximum only when one of their scores exceeds it by more than
        // the threshold: one maximum over this lane's 64 values and a wave vote decide; the exact
        // per-query maxima (across lanes) are formed only then.
        form_p(w);
        if (__any(fmaxf(tm[0], tm[1]) > kRescaleThreshold)) {
            const int lr = __lane_id() & 15;
#pragma unroll
            for (int qt = 0; qt < kST; ++qt) {
                const float m = lane_max2(tm[qt], true);
                // the query's new maximum, an integer-valued bf16 number not below the old one
                const float mnew = ceil_bf16(w.mc[qt] + ceilf(fmaxf(m, 0.0f)));
                const float alpha = __builtin_ldexpf(1.0f, -static_cast<int>(mnew - w.mc[qt]));
                w.mc[qt] = mnew;
                // O^T tile u = 2 qt + t and P tile u hold query 32 qt + 16 t + l%16
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const float au = __shfl(alpha, 16 * t + lr, 64);
#pragma unroll
                    for (int e = 0; e < 5; ++e)
#pragma unroll
                        for (int r = 0; r < 4; ++r) w.o[e][2 * qt + t][r] *= au;
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) scale_p(w.pf[2 * qt + t][cc], au);
                }
            }
            set_neg_max(w, h);
        }
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

    // ---- which (b, h, query block, key split): the blocks of one (b, h) stay on one XCD (the
    // self-attention: a head's K and V are read by all its query blocks) ----
    const int splits = SPLIT ? a.splits : 1;
    const int T = a.B * a.H * a.qblocks * splits;
    int b, h, qblk, split = 0;
    if (RESIDENT && ((a.B * a.qblocks) & 7) == 0) {
        // The caption cross-attention: its keys are few and every workgroup loads all of them, so
        // workgroups are placed by query rows instead: XCD x (workgroup i runs on XCD i % 8) takes
        // the x-th eighth of the batch's query rows, every head. Those are the rows the XCD's own
        // CUs wrote in the Q projection just before (the GEMM gives XCD x the x-th eighth of its
        // M-tiles), and the rows its out-projection reads next: both meet this XCD's L2.
        const int x = blockIdx.x & 7, i = blockIdx.x >> 3;
        const int rb = x * (a.B * a.qblocks / 8) + i / a.H;
        h = i % a.H;
        b = rb / a.qblocks;
        qblk = rb - b * a.qblocks;
    } else {
        int bid = blockIdx.x;
        if ((T & 7) == 0) bid = (bid & 7) * (T >> 3) + (bid >> 3);
        split = SPLIT ? bid % splits : 0;
        if (SPLIT) bid /= splits;
        const int bh = bid / a.qblocks;
        b = bh / a.H;
        h = bh - b * a.H;
        qblk = bid - bh * a.qblocks;
    }
    const int q_base = qblk * (WAVES * kQPerWave) + wave * kQPerWave;
    const int nblk = (a.Skv + kKV - 1) / kKV;
    const int kb0 = SPLIT ? split * nblk / splits : 0;
    const int kb1 = SPLIT ? (split + 1) * nblk / splits : nblk;

    WaveState w;
    // Q fragments first, so their latency overlaps the set-up below
    const int lq = lane & 31, hq = lane >> 5;
#pragma unroll
    for (int qt = 0; qt < kST; ++qt) {
        const int q = q_base + qt * 32 + lq;
        const bf16_t* qrow = a.q + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_q + h * D;
#pragma unroll
        for (int st = 0; st < kSSteps; ++st) {
            const int d0 = st * 16 + hq * 8;
            bf16x8_t f = {};
            if (q < a.Sq && d0 < D) f = ld_frag(reinterpret_cast<const char*>(qrow + d0));
            w.qf[qt][st] = f;
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
    int kb[3];
    kb[0] = lq * kKRow + hq * 16;
    kb[1] = hq ? kOnesOff : lq * kKRow + 128;
    kb[2] = hq ? kOnesOff : (32 + lq) * kKRow + 128;
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
    for (int qt = 0; qt < kST; ++qt) w.mc[qt] = 0.0f;   // the first block's scores are formed against 0

    // The Q loads are drained here, where the compiler sees it: otherwise it waits for them
    // (vmcnt(0), which also drains the DMA in flight) at their first use in every phase.
    s_waitcnt<0, 15>();
    // Q carries the score scale in log2 units, c = scale log2(e), rounded to bf16 once here, so
    // the matrix cores deliver s c - m and the softmax spends no multiply-add per score.
#pragma unroll
    for (int qt = 0; qt < kST; ++qt)
#pragma unroll
        for (int st = 0; st < kSSteps; ++st)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                w.qf[qt][st][e] = static_cast<__bf16>(static_cast<float>(w.qf[qt][st][e]) * a.c);

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
        matrix_phase<false, true>(w, nullptr, vbase, res_stage(0), kb);
        softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, hq);
        for (int j = 1; j < n; ++j) {
            matrix_phase<true, true>(w, res_stage(j - 1), vbase, res_stage(j), kb);
            softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, hq);
        }
        matrix_phase<true, false>(w, res_stage(n - 1), vbase, nullptr, kb);
    } else {
    auto stage_of = [&](int j) -> char* { return smem + (j & (kStages - 1)) * kStage; };
    if (wave < kDmaWaves) {
        // waves 0-3: the matrix phase in even phases, then the DMA of block j+2
        const bf16_t* kbh = a.k + static_cast<int64_t>(b) * a.Skv * a.ld_k + h * D;
        const bf16_t* vbh = a.vt + (static_cast<int64_t>(b) * a.H + h) * D * a.vt_ld;
        const int last_full = a.Skv / kKV;   // blocks below this one hold 64 real keys
        const DmaPlan plan = dma_plan(a, wave, lane);
        auto issue = [&](int j) {
            const int blk = __builtin_amdgcn_readfirstlane(live[min(j, n - 1)]);
            dma_block(stage_of(j), a, plan, kbh, vbh, wave, lane, blk * kKV, MASKED && blk >= last_full);
        };
        issue(0);
        issue(1);
        wait_and_join<kDmaPerWave>();                            // phase 0: block 0 has landed
        matrix_phase<false, true>(w, nullptr, vbase, stage_of(0), kb);
        issue(2);
        if (n > 1) {   // block 0's softmax peeled off, so FIRST is known at compile time
            wait_and_join<63>();                                 // phase 1
            softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, hq);
            wait_and_join<kDmaPerWave>();                        // phase 2: block 1 has landed
            matrix_phase<true, true>(w, stage_of(0), vbase, stage_of(1), kb);
            issue(3);
            for (int j = 2; j < n; ++j) {
                wait_and_join<63>();                             // phase 2j-1
                softmax<MASKED, false>(w, a, live[j - 1], bits_of(j - 1), all_masked, hq);
                wait_and_join<kDmaPerWave>();                    // phase 2j: block j has landed
                matrix_phase<true, true>(w, stage_of(j - 1), vbase, stage_of(j), kb);
                issue(j + 2);
            }
            wait_and_join<63>();                                 // phase 2n-1
            softmax<MASKED, false>(w, a, live[n - 1], bits_of(n - 1), all_masked, hq);
        } else {
            wait_and_join<63>();                                 // phase 1
            softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, hq);
        }
        wait_and_join<63>();                                     // phase 2n
        matrix_phase<true, false>(w, stage_of(n - 1), vbase, nullptr, kb);
        wait_and_join<63>();                                     // phase 2n+1
        s_waitcnt<0, 15>();   // the trailing copies
    } else {
        wait_and_join<63>();                                     // phase 0
        wait_and_join<63>();                                     // phase 1
        matrix_phase<false, true>(w, nullptr, vbase, stage_of(0), kb);
        wait_and_join<63>();                                     // phase 2
        softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, hq);
        for (int j = 1; j < n; ++j) {
            wait_and_join<63>();                                 // phase 2j+1
            matrix_phase<true, true>(w, stage_of(j - 1), vbase, stage_of(j), kb);
            wait_and_join<63>();                                 // phase 2j+2
            softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, hq);
        }
        wait_and_join<63>();                                     // phase 2n+1
        matrix_phase<true, false>(w, stage_of(n - 1), vbase, nullptr, kb);
    }
    }

    // ---- a key split's partial: O unnormalised, the row sum and the running maximum ----
    if constexpr (SPLIT) {
        const bool empty = empty_s != 0;
        float mo[kQT];   // the running maximum of query 16 u + l%16 (held by lane 16 (u & 1) + l%16)
#pragma unroll
        for (int u = 0; u < kQT; ++u) mo[u] = __shfl(w.mc[u >> 1], 16 * (u & 1) + lr, 64);
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
                        empty ? f32x4_t{0.f, -INFINITY, 0.f, 0.f} : f32x4_t{w.o[e][u][0], mo[u], 0.f, 0.f};
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

// The same with 16-byte accesses (V and V^T 16-byte aligned, ld_v % 8 == 0, vt_ld % 64 == 0):
// a thread loads 8 dims of one key, then stores the 8 keys of one dim that sit at V^T slots
// 8q..8q+7 of the block. Those are two runs of four keys (vt_pos keeps runs of four):
// 32 (q / 4) + 16 (q & 1) + 4 ((q >> 1) & 1) + {0..3, 8..11}.
__global__ void __launch_bounds__(256) k_transpose_v72_v16(const bf16_t* __restrict__ v, int64_t ld_v,
                                                           int B, int H, int Skv, bf16_t* vt,
                                                           int64_t vt_ld) {
    constexpr int kRow = D + 8;   // 160-byte LDS rows keep every 16-byte chunk aligned
    __shared__ __attribute__((aligned(16))) bf16_t tile[kKV][kRow];
    const int nblk = static_cast<int>(vt_ld / kKV);
    const int blk = blockIdx.x % nblk;
    const int bh = blockIdx.x / nblk;
    const int b = bh / H, h = bh - b * H;
    const int kv0 = blk * kKV;
    for (int i = threadIdx.x; i < kKV * (D / 8); i += 256) {
        const int r = i / (D / 8), ch = i - r * (D / 8);
        const int key = kv0 + r;
        uint4 x = make_uint4(0u, 0u, 0u, 0u);
        if (key < Skv)
            x = *reinterpret_cast<const uint4*>(v + (static_cast<int64_t>(b) * Skv + key) * ld_v + h * D + ch * 8);
        *reinterpret_cast<uint4*>(&tile[r][ch * 8]) = x;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < D * (kKV / 8); i += 256) {
        const int d = i / (kKV / 8), q = i - d * (kKV / 8);
        const int k0 = 32 * (q >> 2) + 16 * (q & 1) + 4 * ((q >> 1) & 1);
        uint32_t w[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int ka = k0 + (t < 2 ? 2 * t : 8 + 2 * (t - 2));
            w[t] = static_cast<uint32_t>(tile[ka][d]) | (static_cast<uint32_t>(tile[ka + 1][d]) << 16);
        }
        *reinterpret_cast<uint4*>(vt + ((static_cast<int64_t>(b) * H + h) * D + d) * vt_ld + kv0 + 8 * q) =
            make_uint4(w[0], w[1], w[2], w[3]);
    }
}

void launch_transpose_v72(const bf16_t* v, int64_t ld_v, int64_t batch, int64_t heads,
                          int64_t kv_len, bf16_t* vt, int64_t vt_ld, hipStream_t s) {
    const int64_t nblk = (vt_ld + kKV - 1) / kKV;
    const bool v16 = ld_v % 8 == 0 && vt_ld % kKV == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(vt) % 16 == 0;
    if (v16)
        k_transpose_v72_v16<<<static_cast<int>(batch * heads * nblk), 256, 0, s>>>(
            v, ld_v, static_cast<int>(batch), static_cast<int>(heads), static_cast<int>(kv_len), vt,
            vt_ld);
    else
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
