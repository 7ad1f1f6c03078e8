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

#include "flash72_core.inc"
using namespace fk;

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
    const int q_base = (a.qb0 + qblk) * (WAVES * kQPerWave) + wave * kQPerWave;
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
            // unmasked, the live blocks are kb0, kb0 + 1, ...: no LDS read (and no wait for every
            // LDS read in flight) in the middle of the matrix phase
            const int blk = MASKED ? __builtin_amdgcn_readfirstlane(live[min(j, n - 1)]) : kb0 + min(j, n - 1);
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
            const int q0 = a.qb0 * kQPerWg;
            float* dst = a.part + ((static_cast<int64_t>(split) * a.B + b) * a.H + h) * (a.Sq - q0) * 80 +
                         static_cast<int64_t>(q - q0) * 80;
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
            x.x = f2bf2(w.o[e][u][0] * rl, w.o[e][u][1] * rl);
            x.y = f2bf2(w.o[e][u][2] * rl, w.o[e][u][3] * rl);
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
// The partials cover queries q0 .. Sq - 1 of every (b, h). The split count is a template
// argument so that a thread issues every load of its S partials before the first use: with a
// run-time count each split's loads waited for the previous split's (2 S memory round trips per
// thread, which set the launch's time, as every thread of the grid is resident at once).
template <int S>
__global__ void __launch_bounds__(256) k_flash72_combine(const float* __restrict__ part, int B, int H,
                                                         int Sq, int q0, bf16_t* out, int64_t ld_o) {
    constexpr int kChunks = D / 8;   // 9
    const int Sp = Sq - q0;
    const int64_t rows = static_cast<int64_t>(B) * H * Sp;
    const int64_t split_stride = rows * 80;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < rows * kChunks;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t row = i / kChunks;   // ((b * H + h) * Sp + q - q0)
        const int c = static_cast<int>(i - row * kChunks);
        const float* p = part + row * 80;
        float2 lm[S];   // (l, m) of each split: floats 72 and 73 of its row
        f32x4_t lo[S], hi[S];
#pragma unroll
        for (int sp = 0; sp < S; ++sp) {
            const float* ps = p + sp * split_stride;
            lm[sp] = *reinterpret_cast<const float2*>(ps + 72);
            lo[sp] = *reinterpret_cast<const f32x4_t*>(ps + c * 8);
            hi[sp] = *reinterpret_cast<const f32x4_t*>(ps + c * 8 + 4);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int sp = 0; sp < S; ++sp) mx = fmaxf(mx, lm[sp].y);
        float l = 0.f, o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < S; ++sp) {
            const float wgt = __builtin_amdgcn_exp2f(lm[sp].y - mx);   // 0 for an empty split
            l = __fmaf_rn(lm[sp].x, wgt, l);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                o[r] = __fmaf_rn(lo[sp][r], wgt, o[r]);
                o[4 + r] = __fmaf_rn(hi[sp][r], wgt, o[4 + r]);
            }
        }
        const float rl = __frcp_rn(l);
        float v[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) v[r] = o[r] * rl;
        const int64_t q = q0 + row % Sp, bh = row / Sp;
        const int64_t b = bh / H, h = bh - b * H;
        uint32_t wv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
            wv[r] = f2bf2(v[2 * r], v[2 * r + 1]);
        *reinterpret_cast<uint4*>(out + (b * Sq + q) * ld_o + h * D + c * 8) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
    }
}

template <int S>
void launch_combine(const Flash72Args& a, int64_t threads, int q0, bf16_t* out, int64_t ld_o, hipStream_t s) {
    k_flash72_combine<S><<<static_cast<int>(std::min<int64_t>((threads + 255) / 256, 8192)), 256, 0, s>>>(
        a.part, a.B, a.H, a.Sq, q0, out, ld_o);
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
    // As many splits as fit in one round, each of at least four key blocks: with two, a
    // workgroup's fixed work (Q load, pipeline fill, the 164 KB partial) and the combine's traffic
    // outweighed the CUs gained (512px at batch 1: 8 splits of 2 blocks 0.80 ms of self-attention
    // per step, 4 of 4 0.75 ms, 2 of 8 0.84 ms; interleaved A/B).
    int best = 1;
    for (int sp = 2; sp <= 8; ++sp)
        if (wgs * sp <= cus && nblk >= 4 * sp) best = sp;
    return best;
}

int64_t flash72_part_floats(int64_t batch, int64_t heads, int64_t q_len, int splits) {
    return splits > 1 ? static_cast<int64_t>(splits) * batch * heads * q_len * 80 : 0;
}

// A grid of W = batch x heads x query blocks whole workgroups over C CUs runs ceil(W / C) rounds;
// when the last one is at most half full (1152px: 352 workgroups, a last round of 96), the query
// blocks past the whole rounds split their keys instead, as many ways as still fit in one round,
// so that round takes a fraction of a query block's time. The blocks of the whole rounds stay
// unsplit: query blocks qb0 and up of every (b, h) are split, qb0 = whole rounds x C / (b x h).
Flash72Plan flash72_plan(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len,
                         const void* out, int64_t ld_o) {
    const int sp = flash72_splits(batch, heads, q_len, kv_len, out, ld_o);
    if (sp > 1) return {sp, 0};
    if (kv_len <= kResidentBlocks * kKV) return {1, 0};
    if (ld_o % 8 != 0 || reinterpret_cast<uintptr_t>(out) % 16 != 0) return {1, 0};
    int cus = 0, dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    const int64_t bh = batch * heads;
    const int64_t qblocks = (q_len + kQPerWg - 1) / kQPerWg;
    const int64_t wgs = bh * qblocks;
    const int64_t rounds = wgs / cus;
    if (rounds == 0 || wgs % cus == 0 || (wgs % cus) * 2 > cus) return {1, 0};
    const int64_t qb0 = rounds * cus / bh;
    const int64_t tail = bh * (qblocks - qb0);
    const int64_t nblk = (kv_len + kKV - 1) / kKV;
    int best = 1;
    for (int s2 = 2; s2 <= 8; ++s2)
        if (tail * s2 <= cus && nblk >= 2 * s2) best = s2;
    if (best == 1 || qb0 <= 0 || qb0 >= qblocks) return {1, 0};
    return {best, static_cast<int>(qb0)};
}

int64_t flash72_plan_floats(int64_t batch, int64_t heads, int64_t q_len, const Flash72Plan& p) {
    return flash72_part_floats(batch, heads, q_len - static_cast<int64_t>(p.qb0) * kQPerWg, p.splits);
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
                    float* part, int64_t part_floats, int qb0) {
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
    if (splits <= 0) {
        const Flash72Plan p = flash72_plan(batch, heads, q_len, kv_len, out, ld_o);
        splits = p.splits;
        qb0 = p.qb0;
    }
    const int64_t nblk = (kv_len + kKV - 1) / kKV;
    require(splits >= 1 && splits <= 8 && (splits == 1 || (!resident && nblk >= splits)),
            "attention (head_dim 72): " + std::to_string(splits) + " key splits of " +
                std::to_string(nblk) + " key blocks");
    require(qb0 >= 0 && (qb0 == 0 || (splits > 1 && qb0 < a.qblocks)),
            "attention (head_dim 72): key splits from query block " + std::to_string(qb0) + " of " +
                std::to_string(a.qblocks));
    if (splits > 1) {
        const int64_t floats = flash72_plan_floats(batch, heads, q_len, Flash72Plan{splits, qb0});
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
    const double flops = 4.0 * batch * heads * static_cast<double>(q_len) * kv_len * D;
    ProfileScope ps(q_len == kv_len ? K_ATTN_SELF : K_ATTN_CROSS, s, flops);
    if (qb0 > 0) {   // query blocks below qb0 whole, then the rest split over keys
        Flash72Args w = a;
        w.qblocks = qb0;
        w.splits = 1;
        w.part = nullptr;
        const int grid0 = w.B * w.H * w.qblocks;
        if (masked) k_flash72<true, false, false><<<grid0, kThreads, 0, s>>>(w);
        else k_flash72<false, false, false><<<grid0, kThreads, 0, s>>>(w);
        launch_check("attention (flash, head_dim 72)");
        a.qb0 = qb0;
        a.qblocks -= qb0;
    }
    const int grid = a.B * a.H * a.qblocks * a.splits;
    if (a.splits > 1 && masked) k_flash72<true, false, true><<<grid, kThreads, 0, s>>>(a);
    else if (a.splits > 1) k_flash72<false, false, true><<<grid, kThreads, 0, s>>>(a);
    else if (resident) launch_resident(masked, waves, grid, a, s);
    else if (masked) k_flash72<true, false, false><<<grid, kThreads, 0, s>>>(a);
    else k_flash72<false, false, false><<<grid, kThreads, 0, s>>>(a);
    launch_check("attention (flash, head_dim 72)");
    if (a.splits > 1) {
        const int q0 = a.qb0 * kQPerWg;
        const int64_t threads = batch * heads * (q_len - q0) * (D / 8);
        switch (a.splits) {
            case 2: launch_combine<2>(a, threads, q0, out, ld_o, s); break;
            case 3: launch_combine<3>(a, threads, q0, out, ld_o, s); break;
            case 4: launch_combine<4>(a, threads, q0, out, ld_o, s); break;
            case 5: launch_combine<5>(a, threads, q0, out, ld_o, s); break;
            case 6: launch_combine<6>(a, threads, q0, out, ld_o, s); break;
            case 7: launch_combine<7>(a, threads, q0, out, ld_o, s); break;
            default: launch_combine<8>(a, threads, q0, out, ld_o, s); break;
        }
        launch_check("attention (head_dim 72, key-split combine)");
    }
}

}  // namespace bh
