// The cross-attention block's query projection and its attention in one kernel (gfx950).
//
//   ctx[b, q, h, :] = softmax(scale * Q K^T, key mask) V,  Q = bf16(x W_q^T + b_q)
//
// which the reference graph runs as a gemm (`attn2.to_q`) and an attention over the caption keys
// (pixart_dit.cpp:251-262). Each workgroup owns one 256 x 144 tile of the projection -- 256 query
// rows of one batch row, 144 columns = two heads of 72 -- and computes it exactly as the GEMM
// kernel does (gemm_tile.inc: four consumer waves on bf16 MFMAs, four producer waves streaming the
// operands into LDS, the k-tiles summed in the same order), then parks the fp32 tile in LDS. The
// same workgroup then attends with those 256 queries x 2 heads to the caption: the eight waves take
// 64 queries of one head each, read their Q fragments straight from the parked tile (+ bias,
// rounded to bf16 as the GEMM stores Q, times scale * log2(e) rounded to bf16 as the attention
// loads it), and run the head_dim-72 attention's resident schedule (flash72_core.inc) over the
// live caption blocks of both heads, at most three per head in LDS at once. Q never goes to HBM,
// and one launch replaces two: the result is bit-identical with the GEMM followed by the
// attention kernel, which the plans' equality tests check.
//
// The caption keys are few (<= 448, the resident attention's limit): K and V^T of a layer come
// from the engine's hoisted caption projection (K rows of stride ld_k, V^T rows of vt_ld keys).
#include "common.h"

#include <algorithm>
#include <cmath>
#include <string>

namespace bh {
namespace {

#include "gemm_tile.inc"
#include "flash72_core.inc"

using G = gk::Geom<4>;
constexpr int kHeadsPerTile = gk::BN / fk::D;           // 2
constexpr int kChunk = 3;                               // live key blocks per head resident at once
constexpr int kKeyStages = kHeadsPerTile * kChunk;      // 6 x 21 KiB
constexpr int kCtileBytes = G::BM * gk::kCRow<gk::kNT> * 4;      // the parked fp32 tile
constexpr int kBitsOff = kCtileBytes;                   // key-block validity words (after the tile)
constexpr int kLiveOff = kBitsOff + fk::kResidentBlocks * 8;
constexpr int kCountOff = kLiveOff + fk::kResidentBlocks * 4;
static_assert(kHeadsPerTile * fk::D == gk::BN, "a tile is two heads");
static_assert(kKeyStages * fk::kStage <= kBitsOff, "key stages overlap the mask words");
static_assert(kCountOff + 16 <= G::kBiasOff, "mask words overlap the bias slots");

template <bool MASKED>
__global__ void __launch_bounds__(gk::kWgThreads, 1)
k_cross_fused(const bf16_t* __restrict__ X, const bf16_t* __restrict__ Wq, gk::Epi e, int64_t M,
              int tiles_m, int tiles_n, int group_m, fk::Flash72Args a) {
    __shared__ __attribute__((aligned(1024))) char smem[G::kSmemBytes];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t N = static_cast<int64_t>(tiles_n) * gk::BN, K = N;
    int64_t m0, n0;
    gk::tile_origin<4>(blockIdx.x, tiles_m, tiles_n, group_m, m0, n0);
    const int b = static_cast<int>(m0 / a.Sq);           // a tile never straddles two batch rows
    const int q0 = static_cast<int>(m0 - static_cast<int64_t>(b) * a.Sq);
    const int h0 = static_cast<int>(n0 / fk::D);
    const int nblk = (a.Skv + fk::kKV - 1) / fk::kKV;    // <= kResidentBlocks (launcher)

    // The caption mask value of key `64 wave + lane`, loaded now and looked at after the projection
    // (its raw bits are kept opaque until then, so the load's latency hides under the k-loop).
    const int mkey = wave * fk::kKV + lane;
    const bool in_range = !MASKED || (wave < nblk && mkey < a.Skv);
    uint32_t mraw = 0x3f800000u;   // 1.0f: keep
    if (MASKED && in_range && a.mask) {
        if (a.mask_f32) mraw = static_cast<const uint32_t*>(a.mask)[b * a.Skv + mkey];
        else mraw = static_cast<const uint16_t*>(a.mask)[b * a.Skv + mkey];
    }

    // ---- the projection: one GEMM tile, parked in LDS as fp32 ----
    const int KT = static_cast<int>(K / gk::BK);
    if (wave >= gk::kConsumers) {
        gk::produce<4, false>(smem, gk::Operands{X, Wq, M, N, K, ConvGeom{}, K, e.bias}, KT, 1, tiles_m,
                              tiles_n, group_m, wave - gk::kConsumers, lane);
    } else {
        gk::consume<4, 0, gk::EPI_STORE>(smem, e, nullptr, M, N, KT, 1, tiles_m, tiles_n, group_m, wave,
                                         lane);
    }
    gk::wait_and_join<63>();   // the parked tile is complete and visible

    // ---- the key blocks' validity words, and this wave's Q fragments from the parked tile ----
    auto* blk_bits = reinterpret_cast<unsigned long long*>(smem + kBitsOff);
    auto* live = reinterpret_cast<int*>(smem + kLiveOff);
    auto* counts = reinterpret_cast<int*>(smem + kCountOff);
    if (MASKED) {
        asm volatile("" : "+v"(mraw));
        const float mv = (a.mask && !a.mask_f32) ? __uint_as_float(mraw << 16) : __uint_as_float(mraw);
        const unsigned long long bits = __ballot(in_range && mv != 0.0f);
        if (wave < nblk && lane == 0) blk_bits[wave] = bits;
    }
    const int hh = wave >> 2;                             // head h0 + hh
    const int r0 = (wave & 3) * fk::kQPerWave;            // tile rows r0 .. r0 + 63
    const int lq = lane & 31, hq = lane >> 5;
    fk::WaveState w;
    {
        const float* ctile = reinterpret_cast<const float*>(smem);
        const bf16_t* bias_lds = gk::bias_slot<4>(smem, 0);
#pragma unroll
        for (int qt = 0; qt < fk::kST; ++qt) {
            const int row = r0 + qt * 32 + lq;
#pragma unroll
            for (int st = 0; st < fk::kSSteps; ++st) {
                const int d0 = st * 16 + hq * 8;
                bf16x8_t f = {};
                if (d0 < fk::D) {
                    const int col = hh * fk::D + d0;
                    const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(ctile + gk::ctile_at<>(row, col));
                    const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(ctile + gk::ctile_at<>(row, col + 4));
                    float bv[8];
                    if (e.bias) {
                        gk::unpack8(*reinterpret_cast<const uint4*>(bias_lds + col), bv);
                    } else {
#pragma unroll
                        for (int i = 0; i < 8; ++i) bv[i] = -0.0f;
                    }
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        // Q as the GEMM stores it, then scaled as the attention loads it
                        const float q = round_bf16(__fadd_rn(i < 4 ? lo[i] : hi[i - 4], bv[i]));
                        f[i] = static_cast<__bf16>(q * a.c);
                    }
                }
                w.qf[qt][st] = f;
            }
        }
    }
    __syncthreads();   // the tile is read: its LDS now takes the key stages
    if (threadIdx.x == 0) {
        int n = 0;
        unsigned long long any = MASKED ? 0ull : 1ull;
        if (MASKED)
            for (int blk = 0; blk < nblk; ++blk) any |= blk_bits[blk];
        const bool all_masked = any == 0ull;
        for (int blk = 0; blk < nblk; ++blk)
            if (!MASKED || all_masked || blk_bits[blk] != 0ull) live[n++] = blk;
        counts[0] = n;
        counts[1] = all_masked ? 1 : 0;
    }
    // V^T rows 72..79 of every key stage: the ones row and zero padding (never written by the DMA)
    for (int i = threadIdx.x; i < kKeyStages * 8 * 128 / 16; i += gk::kWgThreads) {
        const int st = i / 64, x = i - st * 64;
        const uint32_t one = x < 8 ? 0x3f803f80u : 0u;
        *reinterpret_cast<uint4*>(smem + st * fk::kStage + fk::kKBytes + 72 * 128 + x * 16) =
            make_uint4(one, one, one, one);
    }
    // Q's dim 72 of the first block is formed against a maximum of 0 (the softmax sets it)
#pragma unroll
    for (int e5 = 0; e5 < 5; ++e5)
#pragma unroll
        for (int u = 0; u < fk::kQT; ++u) w.o[e5][u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int qt = 0; qt < fk::kST; ++qt) w.mc[qt] = 0.0f;
    __syncthreads();
    const int n = counts[0];
    const bool all_masked = MASKED && counts[1] != 0;

    // ---- the attention over the live caption blocks of both heads, kChunk per head at a time ----
    int kb[3];
    kb[0] = lq * fk::kKRow + hq * 16;
    kb[1] = hq ? fk::kOnesOff : lq * fk::kKRow + 128;
    kb[2] = hq ? fk::kOnesOff : (32 + lq) * fk::kKRow + 128;
    int vbase[2];
    {
        const int lr = lane & 15, g = lane >> 4, sw = (lr >> 1) & 7;
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) vbase[cc] = fk::kKBytes + lr * 128 + (((cc * 4 + g) ^ sw) << 4);
    }
    const int last_full = a.Skv / fk::kKV;
    auto stage = [&](int head, int j) -> char* { return smem + (head * kChunk + j) * fk::kStage; };
    auto bits_of = [&](int j) -> unsigned long long { return MASKED ? blk_bits[live[j]] : ~0ull; };
    // Key blocks live[c0 .. c1) of both heads into the key stages (all eight waves issue), landed.
    auto load_chunk = [&](int c0, int c1) {
        for (int head = 0; head < kHeadsPerTile; ++head) {
            const int h = h0 + head;
            const bf16_t* kbh = a.k + static_cast<int64_t>(b) * a.Skv * a.ld_k + h * fk::D;
            const bf16_t* vbh = a.vt + (static_cast<int64_t>(b) * a.H + h) * fk::D * a.vt_ld;
            for (int j = c0; j < c1; ++j) {
                const int blk = live[j];
                for (int item = wave; item < 20; item += gk::kWgThreads / 64)
                    fk::dma_item(stage(head, j - c0), a, kbh, vbh, item, lane, blk * fk::kKV,
                                 MASKED && blk >= last_full);
            }
        }
        s_waitcnt<0, 15>();
        __syncthreads();
    };
    // The first chunk holds the first block (which sets the running maximum); a caption with more
    // than kChunk live blocks runs the rest in further chunks, once the first chunk's stages are free.
    {
        const int c1 = min(n, kChunk);
        load_chunk(0, c1);
        fk::matrix_phase<false, true>(w, nullptr, vbase, stage(hh, 0), kb);
        fk::softmax<MASKED, true>(w, a, live[0], bits_of(0), all_masked, hq);
        for (int j = 1; j < c1; ++j) {
            fk::matrix_phase<true, true>(w, stage(hh, j - 1), vbase, stage(hh, j), kb);
            fk::softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, hq);
        }
        fk::matrix_phase<true, false>(w, stage(hh, c1 - 1), vbase, nullptr, kb);
    }
    for (int c0 = kChunk; c0 < n; c0 += kChunk) {
        const int c1 = min(n, c0 + kChunk);
        __syncthreads();   // every wave is done with the previous chunk's stages
        load_chunk(c0, c1);
        fk::matrix_phase<false, true>(w, nullptr, vbase, stage(hh, 0), kb);
        fk::softmax<MASKED, false>(w, a, live[c0], bits_of(c0), all_masked, hq);
        for (int j = c0 + 1; j < c1; ++j) {
            fk::matrix_phase<true, true>(w, stage(hh, j - 1 - c0), vbase, stage(hh, j - c0), kb);
            fk::softmax<MASKED, false>(w, a, live[j], bits_of(j), all_masked, hq);
        }
        fk::matrix_phase<true, false>(w, stage(hh, c1 - 1 - c0), vbase, nullptr, kb);
    }

    // ---- normalise and store: lane holds out[q][d..d+3], d = 16e + 4g; O^T row 72 is the sum ----
    const int lr = lane & 15, g = lane >> 4;
    const int h = h0 + hh;
#pragma unroll
    for (int u = 0; u < fk::kQT; ++u) {
        const float rl = __frcp_rn(__shfl(w.o[4][u][0], 32 + lr, 64));
        const int q = q0 + r0 + u * 16 + lr;
        bf16_t* dst = a.out + (static_cast<int64_t>(b) * a.Sq + q) * a.ld_o + h * fk::D;
#pragma unroll
        for (int e5 = 0; e5 < 5; ++e5) {
            const int d = e5 * 16 + g * 4;
            if (d >= fk::D) continue;
            uint2 x;
            x.x = f2bf2(w.o[e5][u][0] * rl, w.o[e5][u][1] * rl);
            x.y = f2bf2(w.o[e5][u][2] * rl, w.o[e5][u][3] * rl);
            *reinterpret_cast<uint2*>(dst + d) = x;
        }
    }
}

}  // namespace

bool cross_fused_supported(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim,
                           int64_t kv_len) {
    int cus = 0, dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    const int64_t tiles = batch * tokens / G::BM * (heads * head_dim / gk::BN);
    // One tile per workgroup and CU, so a launch of up to one round takes about one tile's time
    // whatever its tile count, while the separate projection and attention shrink with the rows:
    // fused when the tiles fill more than half the chip. 768px (144 tiles on 256 CUs) measured
    // 9.26 -> 8.94 ms per step fused; 512px (64 tiles) keeps the pair (13 + 14.5 us against a
    // ~40 us tile).
    return head_dim == fk::D && heads % kHeadsPerTile == 0 && tokens % G::BM == 0 && kv_len > 0 &&
           kv_len <= fk::kResidentBlocks * fk::kKV && tiles * 2 > cus;
}

void launch_cross_fused(const bf16_t* x, const bf16_t* wq, const bf16_t* bq, int64_t batch,
                        int64_t tokens, int64_t heads, const bf16_t* k, int64_t ld_k, const bf16_t* vt,
                        int64_t vt_ld, int64_t kv_len, const void* key_mask, bool mask_f32,
                        bf16_t* ctx, int64_t ld_o, float scale, hipStream_t s) {
    const int64_t d = heads * fk::D, M = batch * tokens;
    require(tokens % G::BM == 0 && heads % kHeadsPerTile == 0 && kv_len > 0 &&
                kv_len <= fk::kResidentBlocks * fk::kKV,
            "cross attention (fused): tokens % 256 == 0, an even head count, 1..448 caption keys");
    require(vt_ld >= flash72_vt_ld(kv_len) && ld_k % 8 == 0 && ld_o % 4 == 0 && ld_o >= d,
            "cross attention (fused): operand strides");
    require(kv_len * ld_k < (int64_t{1} << 31) && fk::D * vt_ld < (int64_t{1} << 31),
            "cross attention (fused): one (batch, head) slice of K or V^T spans 2^31 elements");
    require(M * d < (int64_t{1} << 31), "cross attention (fused): 2^31 query elements or more");
    gk::Epi e{};
    e.bias = bq;
    e.row_add_period = 1;
    e.gate_rows = 1;
    e.ld_out = d;
    e.vt_dim = 72;
    fk::Flash72Args a;
    a.q = nullptr;
    a.k = k;
    a.vt = vt;
    a.out = ctx;
    a.mask = key_mask;
    a.ld_q = d;
    a.ld_k = ld_k;
    a.vt_ld = vt_ld;
    a.ld_o = ld_o;
    a.B = static_cast<int>(batch);
    a.H = static_cast<int>(heads);
    a.Sq = static_cast<int>(tokens);
    a.Skv = static_cast<int>(kv_len);
    a.mask_f32 = mask_f32 ? 1 : 0;
    a.qblocks = static_cast<int>(tokens / G::BM);
    a.c = scale * 1.4426950408889634f;   // as launch_flash72 forms it
    const int tiles_m = static_cast<int>(M / G::BM), tiles_n = static_cast<int>(d / gk::BN);
    const bool masked = key_mask || kv_len % fk::kKV != 0;
    const int grid = tiles_m * tiles_n;   // one tile per workgroup
    // the projection's FLOP and the attention's, as the two kernels it replaces count them
    ProfileScope ps(K_ATTN_CROSS, s, 2.0 * static_cast<double>(M) * d * d +
                                         4.0 * static_cast<double>(M) * heads * kv_len * fk::D);
    if (masked) k_cross_fused<true><<<grid, gk::kWgThreads, 0, s>>>(x, wq, e, M, tiles_m, tiles_n, 4, a);
    else k_cross_fused<false><<<grid, gk::kWgThreads, 0, s>>>(x, wq, e, M, tiles_m, tiles_n, 4, a);
    launch_check("cross attention (fused projection)");
}

}  // namespace bh
