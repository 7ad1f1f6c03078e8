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

constexpr int BN = 144, BK = 64;
constexpr int kRowBytes = BK * 2;                 // 128
constexpr int kBBytes = BN * kRowBytes;           // 18 KiB
constexpr int kNT = 9;                            // 16x16 column tiles per consumer wave
// The bias row of a tile (BN bf16) is loaded into LDS by the producers with the tile's first
// k-tile, into one of kStages slots (tile index % kStages), so the epilogue reads it from LDS. A
// global load there would be issued after the previous chunk's stores, and waiting for it (vmcnt
// counts loads and stores in issue order) would wait for those stores to be acknowledged.
constexpr int kBiasSlotBytes = 512;
static_assert(BN * 2 <= kBiasSlotBytes, "bias row must fit its slot");

// Tile height: each of the four consumer waves owns MT 16-row blocks, so a tile is BM = 64 MT rows
// (256 for the DiT's 8192-row GEMMs; 128 and 64 for short-M shapes, whose 256-row tiles would fill
// few CUs). Each stage also has one spare 1 KiB row block: waves 2-3 have one B row block fewer
// than waves 0-1 and load a duplicate into it, so every wave issues the same number of DMA
// instructions per k-tile (BM / 32 + 5) and the loop body has no per-wave branch. A shorter tile
// keeps more k-tiles in flight in the LDS it frees: kStages - 1 of them ahead of the consumers.
template <int MT>
struct Geom {
    static_assert(MT == 1 || MT == 2 || MT == 4, "tile height: 64, 128 or 256 rows");
    static constexpr int BM = 64 * MT;
    static constexpr int kABytes = BM * kRowBytes;                    // 32 KiB at MT = 4
    static constexpr int kStageBytes = kABytes + kBBytes + 1024;      // 51 KiB at MT = 4
    static constexpr int kStages = MT == 4 ? 3 : MT == 2 ? 4 : 5;
    static constexpr int kDmaItems = BM / 32 + (BN / 8 + 3) / 4;      // 13 per wave at MT = 4
    // The slot of tile t is written kStages - 1 k-tiles ahead of the consumers and read in tile
    // t's epilogue; the next tile to use it starts KT * kBiasSlots k-tiles later, so kStages
    // slots keep the two apart even at one k-tile per tile.
    static constexpr int kBiasSlots = kStages;
    static constexpr int kBiasOff = kStages * kStageBytes;
    static constexpr int kSmemBytes = kBiasOff + kBiasSlots * kBiasSlotBytes;
    static_assert(kSmemBytes <= 160 * 1024, "LDS");
    static_assert((kStages - 2) * kDmaItems + 1 <= 63, "vmcnt");
};
constexpr int kMaxMT = 4;   // the DiT's tile (256 rows): split-K, the transposed V store, convs

// Epilogue modes. v = act(acc + bias), then:
enum EpiMode {
    EPI_STORE = 0,     // out = v
    EPI_ROW_ADD = 1,   // out = v' + row_add[row % period, n]
    EPI_RESIDUAL = 2,  // out = residual[row, n] + v'
    EPI_GATED = 3,     // out = residual[row, n] + gate[row / gate_rows, n] * v'
    EPI_F32 = 4,       // (float*)out = acc: a split-K partial (no bias, activation or rounding)
};                     // v' = round_mid ? bf16(v) : v

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
    int64_t ld_k;               // row stride of A and B in elements (0: K); split-K reads a slice
    bf16_t* vt;                 // transposed V columns (see GemmEpilogue)
    int64_t vt_period, vt_col0, vt_seq, vt_ld;
    int vt_heads, vt_dim;
};

// ---- activations ------------------------------------------------------------------------------

// Exact forms, the oracle's expressions operation for operation (ops_cpu.cpp:27-36).
__device__ __forceinline__ float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    const float x3 = __fmul_rn(__fmul_rn(x, x), x);
    const float inner = __fmul_rn(c, __fadd_rn(x, __fmul_rn(0.044715f, x3)));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}
__device__ __forceinline__ float silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, expf(-x))); }

// The MFMA epilogue's GELU: 0.5 x (1 + tanh u) = x / (1 + exp(-2u)), u = c (x + 0.044715 x^3),
// with exp(-2u) = exp2(x (k0 + k1 x^2)), k0 = -2 c log2(e), k1 = 0.044715 k0: three VALU
// operations before the hardware exp2 and reciprocal. Its fp32 error (under 1e-6 relative) is far
// below the bf16 ulp it is rounded to, so it moves a stored value by at most one bf16 ulp, the
// same bound the summation order already takes. Large |x| saturate cleanly: exp2 gives 0 (x) or
// +inf (reciprocal 0, so -0).
__device__ __forceinline__ float gelu_tanh_fast(float x) {
    constexpr float k0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
    constexpr float k1 = k0 * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(x * x, k1, k0));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}
__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(-1.4426950408889634f * x);   // exp(-x)
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

template <int ACT>
__device__ __forceinline__ float act_fast(float v) {
    if (ACT == 1) return gelu_tanh_fast(v);
    if (ACT == 2) return silu_fast(v);
    return v;
}
__device__ __forceinline__ float act_exact(int act, float v) {
    if (act == 1) return gelu_tanh(v);
    if (act == 2) return silu(v);
    return v;
}

// One output element after the activation, any mode (the scalar tail and the small kernels).
__device__ __forceinline__ float finish(const Epi& e, int mode, float v, int64_t m, int64_t c,
                                        int64_t N) {
    if (mode != EPI_STORE && e.round_mid) v = round_bf16(v);
    if (mode == EPI_ROW_ADD) v = __fadd_rn(v, bf2f(e.row_add[(m % e.row_add_period) * N + c]));
    if (mode == EPI_RESIDUAL) v = __fadd_rn(bf2f(e.residual[m * e.ld_out + c]), v);
    if (mode == EPI_GATED) {
        v = __fadd_rn(__fmul_rn(v, bf2f(e.gate[(m / e.gate_rows) * N + c])),
                      bf2f(e.residual[m * e.ld_out + c]));
    }
    return v;
}

__device__ __forceinline__ void unpack8(uint4 raw, float (&f)[8]) {
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f[2 * i] = __uint_as_float(w[i] << 16);
        f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        w[i] = static_cast<uint32_t>(f2bf(f[2 * i])) | (static_cast<uint32_t>(f2bf(f[2 * i + 1])) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// ---- the MFMA tile kernel ----------------------------------------------------------------------

// Wait until at most N vector-memory operations of this wave are outstanding and every LDS
// operation has completed.
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
    s_waitcnt<N, 0>();
}

// One global_load_lds_dwordx4: lane L's 16 bytes at `src` land at LDS address lds + 16 L, where
// `lds` is wave-uniform. Issued as inline assembly so that the compiler does not track these LDS
// writes: its own tracking of them is conservative at the loop header (it waits for every
// outstanding load before the first LDS read), which would drain the pipeline each round. The
// explicit waits in wait_and_join() cover them instead. M0 carries the LDS address; nothing else in
// these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* src, const char* lds) {
    const uint32_t l = static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const char*)(lds)));
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(l), "v"(src)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// ---- which global rows the producers load into which LDS rows ----------------------------------
//
// The MFMA is issued with the weight fragment first, so lane (lr = lane % 16, hi = lane / 16) of
// consumer wave w ends a tile with acc[i][j][t] = C[LDS row 64w + 16i + lr][LDS column 16j + 4hi + t].
// The producers fill LDS in an order that makes those registers directly storable:
//  - A: LDS row 64w + 16i + lr holds tile row 64w + 4lr + i, so a lane's four rows are four
//    consecutive tokens (the transposed V store writes them as one 8-byte run of a V^T row);
//  - B: LDS row 16j + 4hi + t holds tile column 32(j/2) + 8hi + 4(j%2) + t for j < 8 and
//    128 + 4hi + t for j = 8. A lane then owns columns 32p + 8hi .. +7 (accumulators j = 2p and
//    2p+1, p < 4) and 128 + 4hi .. +3 (j = 8) of each of its rows: one 16-byte store per row and
//    p, and the four lanes of a row cover 64 contiguous bytes.
template <int MT>
__device__ __forceinline__ int a_row(int r) {
    constexpr int W = 16 * MT;   // LDS rows of one consumer wave
    return (r & ~(W - 1)) | ((r & 15) * MT) | ((r >> 4) & (MT - 1));
}
__device__ __forceinline__ int b_col(int n) {
    const int j = n >> 4, hi = (n >> 2) & 3, t = n & 3;
    return j < 8 ? ((j >> 1) << 5) | (hi << 3) | ((j & 1) << 2) | t : 128 + (hi << 2) + t;
}

// Tile v of the launch -> (tm, tn). Workgroup b runs on XCD b % 8 and, persistent, takes tiles
// b, b + G, b + 2G, ... (G = grid, a multiple of 8 whenever T is), so tiles are renumbered to
// give each XCD a contiguous band of the M x N tile grid, walked `group_m` M-tiles at a time,
// whose A and B panels share that XCD's L2.
template <int MT>
__device__ __forceinline__ void tile_origin(int v, int tiles_m, int tiles_n, int group_m,
                                            int64_t& m0, int64_t& n0) {
    const int T = tiles_m * tiles_n;
    if ((T & 7) == 0) v = (v & 7) * (T >> 3) + (v >> 3);
    const int group_size = group_m * tiles_n;
    const int g = v / group_size;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int in_group = v - g * group_size;
    m0 = static_cast<int64_t>(first_m + in_group % gm) * Geom<MT>::BM;
    n0 = static_cast<int64_t>(in_group / gm) * BN;
}

struct Operands {
    const bf16_t* A;
    const bf16_t* B;
    int64_t M, N, K;
    ConvGeom cv;   // cv.in != null: A is the implicit im2col of a 3x3 convolution (see below)
    int64_t ldk;   // row stride of A and B (K, or the full K of a split-K slice)
    const bf16_t* bias;   // [N] or null: copied to the LDS bias slot of each tile
};

template <int MT>
__device__ __forceinline__ const bf16_t* bias_slot(const char* smem, int tile) {
    return reinterpret_cast<const bf16_t*>(smem + Geom<MT>::kBiasOff + (tile % Geom<MT>::kBiasSlots) * kBiasSlotBytes);
}

// The bias row of the tile at n0 into its LDS slot: 18 lanes of producer wave 0, 16 bytes each.
// Columns past N re-read the last 8 valid ones (never stored; N % 8 == 0 on this kernel's path).
template <int MT>
__device__ __forceinline__ void dma_bias(char* smem, const Operands& o, int64_t n0, int tile, int lane) {
    if (lane < BN / 8) {
        const int64_t n = min(n0 + lane * 8, o.N - 8);
        dma16(o.bias + n, const_cast<char*>(reinterpret_cast<const char*>(bias_slot<MT>(smem, tile))));
    }
}

// This lane's source address (at k = 0) for each of the wave's DMA items of a tile (13 at MT = 4):
// items r < BM/32 are A row blocks 4r + wave, the rest B row blocks 4(r - BM/32) + wave; the one B
// block that does not exist (waves 2-3, last item) repeats the last into the stage's spare block. Each lane
// moves 16 bytes: LDS row rb*8 + lane/8, swizzled chunk lane%8. Rows past M or N re-read the
// last valid row; their results are never stored.
template <int MT>
__device__ __forceinline__ void dma_sources(const bf16_t* (&src)[Geom<MT>::kDmaItems], const Operands& o,
                                            int64_t m0, int64_t n0, int wave, int lane) {
    constexpr int BM = Geom<MT>::BM;
    const int sub = lane >> 3, slot = lane & 7;
#pragma unroll
    for (int r = 0; r < Geom<MT>::kDmaItems; ++r) {
        if (r < BM / 32) {
            const int row_in = (r * 4 + wave) * 8 + sub;
            const int c = slot ^ ((row_in >> 1) & 7);
            const int64_t row = min(m0 + a_row<MT>(row_in), o.M - 1);
            src[r] = o.A + row * o.ldk + c * 8;
        } else {
            const int row_in = min((r - BM / 32) * 4 + wave, BN / 8 - 1) * 8 + sub;
            const int c = slot ^ ((row_in >> 1) & 7);
            const int64_t row = min(n0 + b_col(row_in), o.N - 1);
            src[r] = o.B + row * o.ldk + c * 8;
        }
    }
}

// The whole k-tile at `k0` into one stage: 13 DMA instructions per producer wave at MT = 4.
template <int MT>
__device__ __forceinline__ void dma_tile(char* stage, const bf16_t* const (&src)[Geom<MT>::kDmaItems],
                                         int64_t k0, int wave) {
    constexpr int BM = Geom<MT>::BM;
#pragma unroll
    for (int r = 0; r < Geom<MT>::kDmaItems; ++r) {
        const int rb = r < BM / 32 ? r * 4 + wave : min((r - BM / 32) * 4 + wave, BN / 8);
        dma16(src[r] + k0, stage + (r < BM / 32 ? 0 : Geom<MT>::kABytes) + rb * 1024);
    }
}

// The implicit-convolution k-tile `kt` into one stage. k-tile kt covers tap t = kt / (c_in/64)
// (ky = t / 3, kx = t % 3) and input channels 64 (kt % (c_in/64)) .. +63, so an A row of the tile
// is 128 contiguous bytes of one input pixel: the output pixel's neighbour (y + ky - 1,
// x + kx - 1), halved when the input is upsampled 2x on the fly, or the zero row for a tap in the
// padding. B rows (the weights, repacked [c_out][ky][kx][c_in]) stream as in the plain GEMM.
template <int MT>
__device__ __forceinline__ void dma_tile_conv(char* stage, const bf16_t* const (&src)[Geom<MT>::kDmaItems],
                                              const Operands& o, const int (&py)[Geom<MT>::BM / 32],
                                              const int (&px)[Geom<MT>::BM / 32], int kt, int wave, int lane) {
    constexpr int BM = Geom<MT>::BM;
    const ConvGeom& c = o.cv;
    const int cb_count = c.c_in >> 6;
    const int tap = kt / cb_count, cb = kt - tap * cb_count;
    const int ky = tap / 3, kx = tap - 3 * ky;
    const int slot = lane & 7;
#pragma unroll
    for (int r = 0; r < BM / 32; ++r) {
        const int row_in = (r * 4 + wave) * 8 + (lane >> 3);
        const int ch = (slot ^ ((row_in >> 1) & 7)) * 8;
        int sy = py[r] + ky - 1, sx = px[r] + kx - 1;
        const bool inside = static_cast<unsigned>(sy) < static_cast<unsigned>(c.H) &&
                            static_cast<unsigned>(sx) < static_cast<unsigned>(c.W);
        if (c.up) {
            sy >>= 1;
            sx >>= 1;
        }
        const bf16_t* a = inside ? c.in + (static_cast<int64_t>(sy) * c.in_w + sx) * c.c_in + cb * 64 + ch
                                 : c.zero + ch;
        dma16(a, stage + (r * 4 + wave) * 1024);
    }
    const int64_t k0 = static_cast<int64_t>(kt) * BK;
#pragma unroll
    for (int r = BM / 32; r < Geom<MT>::kDmaItems; ++r) {
        const int rb = min((r - BM / 32) * 4 + wave, BN / 8);
        dma16(src[r] + k0, stage + Geom<MT>::kABytes + rb * 1024);
    }
}

// One k-tile of MFMAs for a consumer wave out of `cur`: MT activation fragments per K=32 half
// (rows 16 MT w + 16i + lane%16) and 9 weight fragments (rows 16j + lane%16), 72 MFMAs at MT = 4
// (the figures below are for that tile). The second
// half's weight fragment j is read into the registers of the first half's, right after the four
// MFMAs that consume it, so only 17 fragments (68 VGPRs) are live: two waves per SIMD fit in the
// register file with the 144 accumulators. `off0`/`off1` are this lane's byte offsets of its
// chunk within a 16-row block for the two halves (row lane%16, chunk 4*half + lane/16, swizzled).
__device__ __forceinline__ bf16x8_t frag(const char* p) { return *reinterpret_cast<const bf16x8_t*>(p); }

template <int MT>
__device__ __forceinline__ void consume_tile(f32x4_t (&acc)[MT][kNT], const char* cur, int wave,
                                             int off0, int off1) {
    const char* a_rows = cur + wave * 16 * MT * kRowBytes;
    const char* b_rows = cur + Geom<MT>::kABytes;
    bf16x8_t a0[MT], a1[MT], b[kNT];
#pragma unroll
    for (int i = 0; i < MT; ++i) a0[i] = frag(a_rows + i * 16 * kRowBytes + off0);
#pragma unroll
    for (int j = 0; j < kNT; ++j) b[j] = frag(b_rows + j * 16 * kRowBytes + off0);
#pragma unroll
    for (int i = 0; i < MT; ++i) a1[i] = frag(a_rows + i * 16 * kRowBytes + off1);
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], a0[i], acc[i][j], 0, 0, 0);
        b[j] = frag(b_rows + j * 16 * kRowBytes + off1);
    }
#pragma unroll
    for (int j = 0; j < kNT; ++j)
#pragma unroll
        for (int i = 0; i < MT; ++i)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(b[j], a1[i], acc[i][j], 0, 0, 0);
    // Keep that order: all 17 first reads up front, each second-half weight read right after its
    // register's last use, then the second half. Left alone, the scheduler sinks every read next
    // to its first use and exposes the LDS latency before each group of four MFMAs.
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * MT + kNT, 0);
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, MT, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, MT * kNT, 0);
}

// Waits until this wave has at most N vector-memory operations outstanding and none of its LDS
// reads, then joins the workgroup. The empty asm statements are compiler-level memory barriers:
// no LDS read or DMA may be moved across the wait and the hardware barrier.
template <int N>
__device__ __forceinline__ void wait_and_join() {
    asm volatile("" ::: "memory");
    wait_vm_lgkm0<N>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The kernel is persistent and warp-specialised: each workgroup walks its tiles, waves 0-3
// (consumers: LDS fragment reads, MFMAs, the epilogue straight from the accumulators, one per
// SIMD) and waves 4-7 (producers: the DMA). A wave issues in order and a DMA instruction holds its
// wave until the address unit accepts it; in a single-role wave that stall delays the wave's
// MFMAs, here it only delays the producer, and the consumer on the same SIMD keeps the matrix
// core busy.
//
// The workgroup's k-tiles are numbered g = 0 .. total-1 across all its tiles (stage g % S, S =
// kStages: 3 for the 256-row tile). Per g, every wave:
//   producers: wait until k-tile g has landed (g+1 .. g+S-2 may still be in flight)
//   consumers: wait until their LDS reads of the previous stage are done
//   barrier
//   producers: DMA k-tile g+S-1 -> stage (g+S-1) % S (it held g-1, which every consumer finished
//              reading before the barrier)
//   consumers: multiply stage g % S; after a tile's last k-tile, its epilogue
// so while the consumers store one tile, the first S-1 k-tiles of the next are already loading.
// The last S-1 steps load a copy of the last k-tile into stages nobody reads again, which keeps
// every step's wait count identical.
constexpr int kConsumers = 4;
constexpr int kWgThreads = 2 * kConsumers * 64;   // 512

template <int MT, bool CONV>
__device__ __forceinline__ void produce(char* smem, const Operands& o, int KT, int my_tiles,
                                        int tiles_m, int tiles_n, int group_m, int wave, int lane) {
    using G = Geom<MT>;
    constexpr int BM = G::BM;
    const int total = my_tiles * KT;
    const bf16_t* src[G::kDmaItems];
    int it = 0, kt = 0;   // the next k-tile to issue
    bool fresh = true;    // k-tile kt is the first of tile it, whose bias row is not loaded yet
    int64_t m0, n0;
    tile_origin<MT>(blockIdx.x, tiles_m, tiles_n, group_m, m0, n0);
    dma_sources<MT>(src, o, m0, n0, wave, lane);
    auto advance = [&]() {
        if (++kt == KT) {
            kt = 0;
            ++it;
            fresh = true;
            tile_origin<MT>(blockIdx.x + it * gridDim.x, tiles_m, tiles_n, group_m, m0, n0);
            dma_sources<MT>(src, o, m0, n0, wave, lane);
        }
    };
    // Implicit convolution: the output pixel of each A item of this lane, per tile.
    constexpr bool conv = CONV;
    int py[BM / 32], px[BM / 32];
    auto conv_rows = [&]() {
#pragma unroll
        for (int r = 0; r < BM / 32; ++r) {
            const int row_in = (r * 4 + wave) * 8 + (lane >> 3);
            const int p = static_cast<int>(min(m0 + a_row<MT>(row_in), o.M - 1));
            py[r] = p / o.cv.W;
            px[r] = p - py[r] * o.cv.W;
        }
    };
    // The bias DMA goes out before its k-tile's items, so the producers' wait for that k-tile (at
    // most one k-tile's items outstanding) also covers it, and the consumers see it from that
    // barrier on.
    // Slot it % S was last read in the epilogue of tile it - S, which every consumer finished
    // before the barrier at which this k-tile is issued (S - 1 k-tiles ahead of the consumers).
    auto issue = [&](char* stage_ptr) {
        if (fresh) {
            if (o.bias && wave == 0) dma_bias<MT>(smem, o, n0, it, lane);
            fresh = false;
        }
        if (conv) dma_tile_conv<MT>(stage_ptr, src, o, py, px, kt, wave, lane);
        else dma_tile<MT>(stage_ptr, src, static_cast<int64_t>(kt) * BK, wave);
    };
    constexpr int S = G::kStages;
    if (conv) conv_rows();
    issue(smem);   // k-tiles 0 .. S-2 into stages 0 .. S-2 (past the last k-tile, copies of it)
#pragma unroll
    for (int q = 1; q < S - 1; ++q) {
        if (q < total) {
            const int it0 = it;
            advance();
            if (conv && it != it0) conv_rows();
        }
        issue(smem + q * G::kStageBytes);
    }
    int stage = 0;   // the stage of k-tile g
    for (int g = 0; g < total; ++g) {
        wait_and_join<(S - 2) * G::kDmaItems>();
        if (g + S - 1 < total) {
            const int it0 = it;
            advance();
            if (conv && it != it0) conv_rows();
        }
        const int sf = stage == 0 ? S - 1 : stage - 1;   // (g + S - 1) % S, k-tile g - 1's stage
        issue(smem + sf * G::kStageBytes);
        stage = stage == S - 1 ? 0 : stage + 1;
    }
    wait_and_join<0>();   // the trailing copies have landed before the LDS holds the output
}

// ---- the epilogue, straight from the accumulators ----------------------------------------------

template <int W> struct RawT;
template <> struct RawT<8> { using type = uint4; };
template <> struct RawT<4> { using type = uint2; };
template <int W> using Raw = typename RawT<W>::type;

template <int W>
__device__ __forceinline__ Raw<W> ld_raw(const bf16_t* p) {
    return *reinterpret_cast<const Raw<W>*>(p);
}
__device__ __forceinline__ void unpack(const uint4& r, float (&f)[8]) { unpack8(r, f); }
__device__ __forceinline__ void unpack(const uint2& r, float (&f)[4]) {
    f[0] = __uint_as_float(r.x << 16);
    f[1] = __uint_as_float(r.x & 0xffff0000u);
    f[2] = __uint_as_float(r.y << 16);
    f[3] = __uint_as_float(r.y & 0xffff0000u);
}
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return static_cast<uint32_t>(f2bf(a)) | (static_cast<uint32_t>(f2bf(b)) << 16);
}
__device__ __forceinline__ void pack(const float (&f)[8], uint4& r) { r = pack8(f); }
__device__ __forceinline__ void pack(const float (&f)[4], uint2& r) {
    r = make_uint2(pack2(f[0], f[1]), pack2(f[2], f[3]));
}

// Chunk p of a lane's row: columns 32p + 8hi .. +7 from accumulators 2p, 2p+1 (p < 4), or
// 128 + 4hi .. +3 from accumulator 8 (p = 4).
template <int P> constexpr int kW = P < 4 ? 8 : 4;
template <int P>
__device__ __forceinline__ int chunk_col(int hi) { return P < 4 ? 32 * P + 8 * hi : 128 + 4 * hi; }
template <int MT, int P>
__device__ __forceinline__ float acc_at(const f32x4_t (&acc)[MT][kNT], int i, int q) {
    if constexpr (P < 4) return q < 4 ? acc[i][2 * P][q] : acc[i][2 * P + 1][q - 4];
    else return acc[i][8][q];
}

// Everything chunk p of a lane's four rows reads besides the accumulators, loaded one chunk ahead
// of its stores (the compiler keeps loads below earlier stores that may alias them; the residual
// IS the output in the engine's in-place updates). Stores start as early as they can: at the end
// of a tile every CU stores at once and the epilogue runs at the memory's write rate, so a later
// first store (all loads first) measured slower.
// The bias values of a chunk, or -0.0 when there is no bias: v + (-0.0) is v exactly for every v
// (signed zeros included), so the epilogue adds unconditionally instead of selecting per value.
template <typename R, int W>
__device__ __forceinline__ void bias_or_neg_zero(const Epi& e, const R& raw, float (&b)[W]) {
    if (e.bias) {
        unpack(raw, b);
    } else {
#pragma unroll
        for (int q = 0; q < W; ++q) b[q] = -0.0f;
    }
}

template <int MODE, int W, int MT>
struct ChunkIn {
    Raw<W> bias, gate;
    Raw<W> row[MT];    // residual or row_add
};

template <int MT, int MODE, int P>
__device__ __forceinline__ void chunk_load(ChunkIn<MODE, kW<P>, MT>& in, const Epi& e, int64_t M,
                                           int64_t N, int64_t mb, int64_t n0, int hi,
                                           bool gate_uniform, const bf16_t* bias_lds) {
    constexpr int W = kW<P>;
    const int64_t n = n0 + chunk_col<P>(hi);
    if (n >= N) return;
    if (e.bias) in.bias = ld_raw<W>(bias_lds + chunk_col<P>(hi));
    if (MODE == EPI_GATED && gate_uniform) in.gate = ld_raw<W>(e.gate + (mb / e.gate_rows) * N + n);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int64_t m = mb + i;
        if (m >= M) continue;
        if (MODE == EPI_RESIDUAL || MODE == EPI_GATED)
            in.row[i] = ld_raw<W>(e.residual + m * e.ld_out + n);
        if (MODE == EPI_ROW_ADD) in.row[i] = ld_raw<W>(e.row_add + (m % e.row_add_period) * N + n);
    }
}

template <int MT, int ACT, int MODE, int P>
__device__ __forceinline__ void chunk_store(const f32x4_t (&acc)[MT][kNT],
                                            const ChunkIn<MODE, kW<P>, MT>& in, const Epi& e,
                                            bf16_t* out, int64_t M, int64_t N, int64_t mb,
                                            int64_t n0, int hi, bool gate_uniform) {
    constexpr int W = kW<P>;
    const int64_t n = n0 + chunk_col<P>(hi);
    if (n >= N) return;
    if constexpr (MODE == EPI_F32) {
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int64_t m = mb + i;
            if (m >= M) continue;
            float* dst = reinterpret_cast<float*>(out) + m * e.ld_out + n;
#pragma unroll
            for (int q = 0; q < W; q += 4)
                *reinterpret_cast<f32x4_t*>(dst + q) = f32x4_t{acc_at<MT, P>(acc, i, q), acc_at<MT, P>(acc, i, q + 1),
                                                              acc_at<MT, P>(acc, i, q + 2), acc_at<MT, P>(acc, i, q + 3)};
        }
        return;
    }
    float b[W], gt[W];
    bias_or_neg_zero(e, in.bias, b);
    if (MODE == EPI_GATED && gate_uniform) unpack(in.gate, gt);
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const int64_t m = mb + i;
        if (m >= M) continue;
        float x[W], t[W];
#pragma unroll
        for (int q = 0; q < W; ++q) x[q] = act_fast<ACT>(__fadd_rn(acc_at<MT, P>(acc, i, q), b[q]));
        if (MODE != EPI_STORE && e.round_mid)
#pragma unroll
            for (int q = 0; q < W; ++q) x[q] = round_bf16(x[q]);
        if (MODE == EPI_ROW_ADD) {
            unpack(in.row[i], t);
#pragma unroll
            for (int q = 0; q < W; ++q) x[q] = __fadd_rn(x[q], t[q]);
        }
        if (MODE == EPI_RESIDUAL) {
            unpack(in.row[i], t);
#pragma unroll
            for (int q = 0; q < W; ++q) x[q] = __fadd_rn(t[q], x[q]);
        }
        if (MODE == EPI_GATED) {
            float gq[W];
            if (gate_uniform) {
#pragma unroll
                for (int q = 0; q < W; ++q) gq[q] = gt[q];
            } else {   // a tile across two gate rows (not in the DiT: gate rows are 4096 tokens)
                unpack(ld_raw<W>(e.gate + (m / e.gate_rows) * N + n), gq);
            }
            unpack(in.row[i], t);
#pragma unroll
            for (int q = 0; q < W; ++q) x[q] = __fadd_rn(__fmul_rn(x[q], gq[q]), t[q]);
        }
        Raw<W> r;
        pack(x, r);
        *reinterpret_cast<Raw<W>*>(out + m * e.ld_out + n) = r;
    }
}

// V columns of the fused QKV projection go to V^T (vt[(blk*B + b)*heads + h)*72 + d][vt_pos(token)]):
// a lane's four rows are four consecutive tokens, so each of its columns is one 8-byte store,
// and the 16 lanes of a column group write 128 contiguous bytes of one V^T row.
template <int MT, int ACT, int P>
__device__ __forceinline__ void vt_chunk(const f32x4_t (&acc)[MT][kNT], const Epi& e, int64_t M,
                                         int64_t N, int64_t mb, int64_t n0, int hi,
                                         const bf16_t* bias_lds) {
    constexpr int W = kW<P>;
    const int col = chunk_col<P>(hi);
    if (n0 + col >= N) return;
    float b[W];
    bias_or_neg_zero(e, e.bias ? ld_raw<W>(bias_lds + col) : Raw<W>{}, b);
    const int64_t batches = M / e.vt_seq;
    const int64_t bt = mb / e.vt_seq, tok = mb - bt * e.vt_seq;
    const bool whole = tok + MT <= e.vt_seq && mb + MT <= M;
    const int vbase = static_cast<int>(n0 % e.vt_period - e.vt_col0) + col;
    const int64_t blk = n0 / e.vt_period;
#pragma unroll
    for (int q = 0; q < W; ++q) {
        const int vc = vbase + q;
        const int h = vc / 72, dd = vc - h * 72;   // the vt store is built for head_dim 72
        float v[MT];
#pragma unroll
        for (int i = 0; i < MT; ++i) v[i] = act_fast<ACT>(__fadd_rn(acc_at<MT, P>(acc, i, q), b[q]));
        if (whole) {
            uint2 r;
            pack(v, r);
            *reinterpret_cast<uint2*>(e.vt + (((blk * batches + bt) * e.vt_heads + h) * 72 + dd) *
                                                 e.vt_ld + vt_pos(tok)) = r;
        } else {
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int64_t m = mb + i;
                if (m >= M) break;
                const int64_t bj = m / e.vt_seq, tj = m - bj * e.vt_seq;
                e.vt[(((blk * batches + bj) * e.vt_heads + h) * 72 + dd) * e.vt_ld + vt_pos(tj)] = f2bf(v[i]);
            }
        }
    }
}

template <int MT, int ACT, int MODE>
__device__ __forceinline__ void epilogue(const f32x4_t (&acc)[MT][kNT], const Epi& e,
                                         bf16_t* out, int64_t M, int64_t N, int64_t m0,
                                         int64_t n0, int wave, int lane, const bf16_t* bl) {
    const int lr = lane & 15, hi = lane >> 4;
    const int64_t mb = m0 + wave * 16 * MT + lr * MT;   // this lane's rows: mb .. mb + MT - 1
    if constexpr (MODE == EPI_STORE && MT == kMaxMT) {   // the transposed V store needs four rows a lane
        if (e.vt && n0 % e.vt_period >= e.vt_col0) {
            vt_chunk<MT, ACT, 0>(acc, e, M, N, mb, n0, hi, bl);
            vt_chunk<MT, ACT, 1>(acc, e, M, N, mb, n0, hi, bl);
            vt_chunk<MT, ACT, 2>(acc, e, M, N, mb, n0, hi, bl);
            vt_chunk<MT, ACT, 3>(acc, e, M, N, mb, n0, hi, bl);
            vt_chunk<MT, ACT, 4>(acc, e, M, N, mb, n0, hi, bl);
            return;
        }
    }
    // gate rows are whole batches of tokens: one gate row per tile unless the tile straddles two
    const int64_t m_last = min(m0 + Geom<MT>::BM, M) - 1;
    const bool gu = MODE == EPI_GATED && m0 / e.gate_rows == m_last / e.gate_rows;
    ChunkIn<MODE, 8, MT> c0, c1, c2, c3;
    ChunkIn<MODE, 4, MT> c4;
    chunk_load<MT, MODE, 0>(c0, e, M, N, mb, n0, hi, gu, bl);
    chunk_load<MT, MODE, 1>(c1, e, M, N, mb, n0, hi, gu, bl);
    chunk_store<MT, ACT, MODE, 0>(acc, c0, e, out, M, N, mb, n0, hi, gu);
    chunk_load<MT, MODE, 2>(c2, e, M, N, mb, n0, hi, gu, bl);
    chunk_store<MT, ACT, MODE, 1>(acc, c1, e, out, M, N, mb, n0, hi, gu);
    chunk_load<MT, MODE, 3>(c3, e, M, N, mb, n0, hi, gu, bl);
    chunk_store<MT, ACT, MODE, 2>(acc, c2, e, out, M, N, mb, n0, hi, gu);
    chunk_load<MT, MODE, 4>(c4, e, M, N, mb, n0, hi, gu, bl);
    chunk_store<MT, ACT, MODE, 3>(acc, c3, e, out, M, N, mb, n0, hi, gu);
    chunk_store<MT, ACT, MODE, 4>(acc, c4, e, out, M, N, mb, n0, hi, gu);
}

// ---- the last tile's epilogue, staged through LDS ------------------------------------------------
//
// After a workgroup's last tile nothing more is loaded, so the whole LDS is free: the consumers
// park the fp32 tile there and all 512 threads finish it with full-row 16-byte stores (18
// consecutive lanes per 288-byte output row). When every CU ends its last tile at the same moment
// (one tile per CU), this epilogue is a burst of HBM traffic, and full rows keep it at the write
// bandwidth. Rows are 148 floats; 4-float groups are XOR-swizzled by row so the consumers'
// writes (16 rows 4 apart per quarter-wave) land on disjoint banks.
constexpr int kCRow = BN + 4;
static_assert(Geom<1>::BM * kCRow * 4 <= Geom<1>::kBiasOff && Geom<2>::BM * kCRow * 4 <= Geom<2>::kBiasOff &&
                  Geom<4>::BM * kCRow * 4 <= Geom<4>::kBiasOff,
              "fp32 output tile must fit in the stages");

__device__ __forceinline__ int ctile_at(int row, int col) {
    return row * kCRow + (col ^ (((row >> 4) & 3) << 2));
}

template <int MT>
__device__ __forceinline__ void park_tile(const f32x4_t (&acc)[MT][kNT], char* smem, int wave,
                                          int lane) {
    float* ctile = reinterpret_cast<float*>(smem);
    const int lr = lane & 15, hi = lane >> 4;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
            const int row = wave * 16 * MT + lr * MT + i, col = b_col(j * 16 + hi * 4);
            *reinterpret_cast<f32x4_t*>(ctile + ctile_at(row, col)) = acc[i][j];
        }
}

template <int MT, int ACT, int MODE>
__device__ __forceinline__ void store_staged(const char* smem, const Epi& e, bf16_t* out,
                                             int64_t M, int64_t N, int64_t m0, int64_t n0,
                                             const bf16_t* bias_lds) {
    constexpr int BM = Geom<MT>::BM;
    const float* ctile = reinterpret_cast<const float*>(smem);
    if (MODE == EPI_STORE && MT == kMaxMT && e.vt && n0 % e.vt_period >= e.vt_col0) {
        // V columns: 8 consecutive tokens of one column per 16-byte store, consecutive threads
        // along the token axis of one V^T row. A thread keeps its 8-row group (512 threads over
        // 32 groups), so its batch and token are worked out once.
        constexpr int kGroups = BM / 8;   // 32
        const int rg = threadIdx.x % kGroups;
        const int64_t m = m0 + rg * 8;
        if (m >= M) return;
        const int64_t batches = M / e.vt_seq;
        const int64_t b = m / e.vt_seq, tok = m - b * e.vt_seq;
        const bool whole = tok + 8 <= e.vt_seq && m + 8 <= M;
        const int vbase = static_cast<int>(n0 % e.vt_period - e.vt_col0);
        const int64_t blk = n0 / e.vt_period;
        for (int col = threadIdx.x / kGroups; col < BN; col += kWgThreads / kGroups) {
            if (n0 + col >= N) break;
            const int vc = vbase + col;
            const int h = vc / 72, dd = vc - h * 72;   // the vt store is built for head_dim 72
            const float bias = e.bias ? bf2f(bias_lds[col]) : -0.0f;
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = act_fast<ACT>(__fadd_rn(ctile[ctile_at(rg * 8 + j, col)], bias));
            const int64_t hrow = ((blk * batches + b) * e.vt_heads + h) * 72 + dd;
            if (whole) {   // two runs of four keys (vt_pos keeps runs of four together)
                const uint4 p8 = pack8(v);
                *reinterpret_cast<uint2*>(e.vt + hrow * e.vt_ld + vt_pos(tok)) = make_uint2(p8.x, p8.y);
                *reinterpret_cast<uint2*>(e.vt + hrow * e.vt_ld + vt_pos(tok + 4)) = make_uint2(p8.z, p8.w);
            } else {
                for (int j = 0; j < 8 && m + j < M; ++j) {
                    const int64_t bj = (m + j) / e.vt_seq, tj = (m + j) - bj * e.vt_seq;
                    e.vt[(((blk * batches + bj) * e.vt_heads + h) * 72 + dd) * e.vt_ld + vt_pos(tj)] =
                        f2bf(v[j]);
                }
            }
        }
        return;
    }
    // A thread keeps one 8-column chunk (18 per row, 28 rows per pass over 504 threads) for the
    // whole tile, so bias and gate are loaded once. Rows go in batches of kBatch: every load of a
    // batch (LDS tile, residual, row_add) is issued before its first store, since the compiler
    // may not move a load above a store that could alias it.
    constexpr int kChunks = BN / 8;
    constexpr int kRowStep = kWgThreads / kChunks;   // 28
    constexpr int kBatch = 5;
    const int ch = threadIdx.x % kChunks;
    const int r0 = threadIdx.x / kChunks;
    const int64_t n = n0 + ch * 8;
    if (r0 >= kRowStep || n >= N) return;
    float bias[8];
    bias_or_neg_zero(e, e.bias ? *reinterpret_cast<const uint4*>(bias_lds + ch * 8) : uint4{}, bias);
    // gate rows are whole batches of tokens: one gate row per tile unless the tile straddles two
    const int64_t m_last = min(m0 + BM, M) - 1;
    const bool gate_uniform = MODE == EPI_GATED && m0 / e.gate_rows == m_last / e.gate_rows;
    float gate_t[8];
    if (gate_uniform) unpack8(*reinterpret_cast<const uint4*>(e.gate + (m0 / e.gate_rows) * N + n), gate_t);
    for (int rb = r0; rb < BM; rb += kBatch * kRowStep) {
        float v[kBatch][8];
        uint4 res[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int r = rb + i * kRowStep;
            const int64_t m = m0 + r;
            if (r < BM && m < M) {
                const f32x4_t lo = *reinterpret_cast<const f32x4_t*>(ctile + ctile_at(r, ch * 8));
                const f32x4_t hi = *reinterpret_cast<const f32x4_t*>(ctile + ctile_at(r, ch * 8 + 4));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v[i][q] = lo[q];
                    v[i][4 + q] = hi[q];
                }
                if (MODE == EPI_RESIDUAL || MODE == EPI_GATED)
                    res[i] = *reinterpret_cast<const uint4*>(e.residual + m * e.ld_out + n);
                if (MODE == EPI_ROW_ADD)
                    res[i] = *reinterpret_cast<const uint4*>(e.row_add + (m % e.row_add_period) * N + n);
            }
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int r = rb + i * kRowStep;
            const int64_t m = m0 + r;
            if (r >= BM || m >= M) continue;
            if constexpr (MODE == EPI_F32) {
                float* dst = reinterpret_cast<float*>(out) + m * e.ld_out + n;
                *reinterpret_cast<f32x4_t*>(dst) = f32x4_t{v[i][0], v[i][1], v[i][2], v[i][3]};
                *reinterpret_cast<f32x4_t*>(dst + 4) = f32x4_t{v[i][4], v[i][5], v[i][6], v[i][7]};
                continue;
            }
            float x[8], t[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = act_fast<ACT>(__fadd_rn(v[i][q], bias[q]));
            if (MODE != EPI_STORE && e.round_mid)
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = round_bf16(x[q]);
            if (MODE == EPI_ROW_ADD) {
                unpack8(res[i], t);
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(x[q], t[q]);
            }
            if (MODE == EPI_RESIDUAL) {
                unpack8(res[i], t);
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(t[q], x[q]);
            }
            if (MODE == EPI_GATED) {
                float gq[8];
                if (gate_uniform)
#pragma unroll
                    for (int q = 0; q < 8; ++q) gq[q] = gate_t[q];
                else   // a tile across two gate rows (not in the DiT: gate rows are 4096 tokens)
                    unpack8(*reinterpret_cast<const uint4*>(e.gate + (m / e.gate_rows) * N + n), gq);
                unpack8(res[i], t);
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(__fmul_rn(x[q], gq[q]), t[q]);
            }
            *reinterpret_cast<uint4*>(out + m * e.ld_out + n) = pack8(x);
        }
    }
}

template <int MT, int ACT, int MODE>
__device__ __forceinline__ void consume(char* smem, const Epi& e, bf16_t* out, int64_t M,
                                        int64_t N, int KT, int my_tiles, int tiles_m, int tiles_n,
                                        int group_m, int wave, int lane) {
    const int lr = lane & 15, sw = (lane >> 1) & 7, hi = lane >> 4;
    const int off0 = lr * kRowBytes + ((hi ^ sw) * 16);
    const int off1 = lr * kRowBytes + (((4 + hi) ^ sw) * 16);
    int stage = 0;
    for (int it = 0; it < my_tiles; ++it) {
        f32x4_t acc[MT][kNT];
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < kNT; ++j) acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        for (int kt = 0; kt < KT; ++kt) {
            wait_and_join<63>();   // only this wave's LDS reads (its stores need not wait)
            consume_tile<MT>(acc, smem + stage * Geom<MT>::kStageBytes, wave, off0, off1);
            stage = stage == Geom<MT>::kStages - 1 ? 0 : stage + 1;
        }
        if (it + 1 < my_tiles) {
            int64_t m0, n0;
            tile_origin<MT>(blockIdx.x + it * gridDim.x, tiles_m, tiles_n, group_m, m0, n0);
            epilogue<MT, ACT, MODE>(acc, e, out, M, N, m0, n0, wave, lane, bias_slot<MT>(smem, it));
        } else {
            wait_and_join<63>();   // the producers' trailing copies have landed
            park_tile<MT>(acc, smem, wave, lane);
        }
    }
}

template <int ACT, int MODE, bool CONV, int MT = kMaxMT>
__global__ void __launch_bounds__(kWgThreads, 1)
k_gemm_tn(const bf16_t* __restrict__ A, const bf16_t* __restrict__ B, bf16_t* out, int64_t M,
          int64_t N, int64_t K, Epi e, int tiles_m, int tiles_n, int group_m, ConvGeom cv) {
    __shared__ __attribute__((aligned(1024))) char smem[Geom<MT>::kSmemBytes];
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
        produce<MT, CONV>(smem, Operands{A, B, M, N, K, cv, ldk, e.bias}, KT, my_tiles, tiles_m,
                          tiles_n, group_m, wave - kConsumers, lane);
    } else {
        consume<MT, ACT, MODE>(smem, e, out, M, N, KT, my_tiles, tiles_m, tiles_n, group_m, wave, lane);
    }
    wait_and_join<63>();   // the parked tile is complete and visible
    int64_t m0, n0;
    tile_origin<MT>(blockIdx.x + (my_tiles - 1) * gridDim.x, tiles_m, tiles_n, group_m, m0, n0);
    store_staged<MT, ACT, MODE>(smem, e, out, M, N, m0, n0, bias_slot<MT>(smem, my_tiles - 1));
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

// Small K (the patch embedding's K = in_channels * patch^2 = 16): one thread per 8 consecutive
// output columns of one row, the reference's sequential k order, 16-byte loads and stores. Needs
// K % 8 == 0, N % 8 == 0 and 16-byte aligned operands.
__global__ void __launch_bounds__(256) k_gemm_smallk(const bf16_t* __restrict__ A,
                                                     const bf16_t* __restrict__ B, bf16_t* out,
                                                     int M, int N, int K, Epi e, int mode) {
    const int groups = N >> 3;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= M * groups) return;
    const int m = idx / groups, n0 = (idx - m * groups) * 8;
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

template <int ACT, int MODE, bool CONV = false, int MT = kMaxMT>
void launch_tn(const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n, int64_t k,
               const Epi& e, hipStream_t s, const ConvGeom& cv = ConvGeom{}) {
    constexpr int BM = Geom<MT>::BM;
    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    // One persistent workgroup per CU (the LDS stages allow no second one); with the tile count
    // a multiple of 8, so is the grid, which the XCD banding relies on. An XCD's band is walked
    // 256 rows of M-tiles at a time whatever the tile height.
    int grid = min(tiles, device_cus() & ~7);
    if (grid < 8) grid = min(tiles, device_cus());
    k_gemm_tn<ACT, MODE, CONV, MT><<<grid, kWgThreads, 0, s>>>(a, b, out, m, n, k, e, tiles_m, tiles_n,
                                                               16 / MT, cv);
}

// The tile height of a GEMM that runs whole (no split-K): the one with the least estimated time,
// rounds x (rows a k-tile loads), where rounds = ceil(tiles / CUs) and a k-tile of a BM-row tile
// loads BM + 144 rows of 128 bytes. The k-loop runs at the rate its operand stream is delivered,
// not at the MFMA rate (~2,100 cycles per 256-row k-tile against 1,152 of MFMA issue), so a
// shorter tile's k-tile is proportionally shorter. Ties keep the taller tile. Every height sums
// each output's k-tiles in the same order with the same MFMAs, so results do not depend on it.
int gemm_tile_mt(int64_t m, int64_t n) {
    const int64_t cus = device_cus();
    const int64_t tiles_n = (n + BN - 1) / BN;
    int best = kMaxMT;
    int64_t best_cost = -1;
    for (int mt = kMaxMT; mt >= 1; mt /= 2) {
        const int64_t bm = 64 * mt;
        const int64_t rounds = (((m + bm - 1) / bm) * tiles_n + cus - 1) / cus;
        const int64_t cost = rounds * (bm + BN);
        if (best_cost < 0 || cost < best_cost) {
            best = mt;
            best_cost = cost;
        }
    }
    return best;
}

// Split-K partials: `splits` slices of K in one launch (grid.y = slice), each persistent
// workgroup set over the same output tiles, slice s writing fp32 partial[s][m][n].
void launch_tn_splitk(const bf16_t* a, const bf16_t* b, float* partial, int64_t m, int64_t n, int64_t k,
                      int splits, hipStream_t s) {
    constexpr int BM = Geom<kMaxMT>::BM;
    const int tiles_m = static_cast<int>((m + BM - 1) / BM);
    const int tiles_n = static_cast<int>((n + BN - 1) / BN);
    const int tiles = tiles_m * tiles_n;
    const int grid = max(1, min(tiles, device_cus() / splits));
    Epi e{};
    e.row_add_period = 1;
    e.gate_rows = 1;
    e.ld_out = n;
    e.ld_k = k;
    e.vt_dim = 72;
    k_gemm_tn<0, EPI_F32, false><<<dim3(grid, splits), kWgThreads, 0, s>>>(
        a, b, reinterpret_cast<bf16_t*>(partial), m, n, k / splits, e, tiles_m, tiles_n, 4, ConvGeom{});
}

// out[m, n] = bf16(residual[m, n] + bf16(sum_s partial[s][m][n])), the slices summed in order.
__global__ void __launch_bounds__(256) k_splitk_residual(const float* __restrict__ partial, int splits,
                                                         const bf16_t* residual, bf16_t* out, int64_t mn) {
    for (int64_t i = (blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x) * 4; i < mn;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x * 4) {
        f32x4_t acc = *reinterpret_cast<const f32x4_t*>(partial + i);
        for (int sp = 1; sp < splits; ++sp) {
            const f32x4_t p = *reinterpret_cast<const f32x4_t*>(partial + sp * mn + i);
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = __fadd_rn(acc[q], p[q]);
        }
        const uint2 r = *reinterpret_cast<const uint2*>(residual + i);
        const float res[4] = {__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                              __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u)};
        uint32_t o[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float lo = __fadd_rn(res[2 * q], round_bf16(acc[2 * q]));
            const float hi = __fadd_rn(res[2 * q + 1], round_bf16(acc[2 * q + 1]));
            o[q] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
        }
        *reinterpret_cast<uint2*>(out + i) = make_uint2(o[0], o[1]);
    }
}

// The split-K epilogue: out[m, n8..n8+7] from the slices summed in order, then exactly the MFMA
// kernel's epilogue (chunk_store): bias, activation, the mid rounding, residual or gated residual,
// one rounding at the store. out may alias the residual (each element is read before written).
template <int ACT, int MODE>
__global__ void __launch_bounds__(256) k_splitk_epi(const float* __restrict__ partial, int splits,
                                                    int64_t M, int64_t N, Epi e, bf16_t* out) {
    const int64_t per_row = N / 8;
    const int64_t groups = M * per_row;
    const int64_t mn = M * N;
    for (int64_t g = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; g < groups;
         g += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t m = g / per_row, n = (g - m * per_row) * 8;
        const float* p = partial + m * N + n;
        f32x4_t lo = *reinterpret_cast<const f32x4_t*>(p), hi = *reinterpret_cast<const f32x4_t*>(p + 4);
        for (int sp = 1; sp < splits; ++sp) {
            const f32x4_t a = *reinterpret_cast<const f32x4_t*>(p + sp * mn);
            const f32x4_t b = *reinterpret_cast<const f32x4_t*>(p + sp * mn + 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                lo[q] = __fadd_rn(lo[q], a[q]);
                hi[q] = __fadd_rn(hi[q], b[q]);
            }
        }
        float x[8], bias[8], t[8];
        bias_or_neg_zero(e, e.bias ? *reinterpret_cast<const uint4*>(e.bias + n) : uint4{}, bias);
#pragma unroll
        for (int q = 0; q < 8; ++q) x[q] = act_fast<ACT>(__fadd_rn(q < 4 ? lo[q] : hi[q - 4], bias[q]));
        if (MODE != EPI_STORE && e.round_mid)
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = round_bf16(x[q]);
        if (MODE == EPI_RESIDUAL) {
            unpack8(*reinterpret_cast<const uint4*>(e.residual + m * e.ld_out + n), t);
#pragma unroll
            for (int q = 0; q < 8; ++q) x[q] = __fadd_rn(t[q], x[q]);
        }
        if (MODE == EPI_GATED) {
            float gq[8];
            unpack8(*reinterpret_cast<const uint4*>(e.gate + (m / e.gate_rows) * N + n), gq);
            unpack8(*reinterpret_cast<const uint4*>(e.residual + m * e.ld_out + n), t);
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

template <int ACT>
void launch_splitk_epi(int mode, const float* partial, int splits, int64_t m, int64_t n, const Epi& e,
                       bf16_t* out, hipStream_t s) {
    const int64_t groups = m * (n / 8);
    const int blocks = static_cast<int>(std::min<int64_t>((groups + 255) / 256, 8192));
    switch (mode) {
        case EPI_STORE: k_splitk_epi<ACT, EPI_STORE><<<blocks, 256, 0, s>>>(partial, splits, m, n, e, out); break;
        case EPI_RESIDUAL: k_splitk_epi<ACT, EPI_RESIDUAL><<<blocks, 256, 0, s>>>(partial, splits, m, n, e, out); break;
        default: k_splitk_epi<ACT, EPI_GATED><<<blocks, 256, 0, s>>>(partial, splits, m, n, e, out); break;
    }
}

template <int ACT, int MT>
void launch_tn_mode(int mode, const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n,
                    int64_t k, const Epi& e, hipStream_t s) {
    switch (mode) {
        case EPI_STORE: launch_tn<ACT, EPI_STORE, false, MT>(a, b, out, m, n, k, e, s); break;
        case EPI_ROW_ADD: launch_tn<ACT, EPI_ROW_ADD, false, MT>(a, b, out, m, n, k, e, s); break;
        case EPI_RESIDUAL: launch_tn<ACT, EPI_RESIDUAL, false, MT>(a, b, out, m, n, k, e, s); break;
        default: launch_tn<ACT, EPI_GATED, false, MT>(a, b, out, m, n, k, e, s); break;
    }
}

template <int ACT>
void launch_tn_mt(int mt, int mode, const bf16_t* a, const bf16_t* b, bf16_t* out, int64_t m, int64_t n,
                  int64_t k, const Epi& e, hipStream_t s) {
    switch (mt) {
        case 1: launch_tn_mode<ACT, 1>(mode, a, b, out, m, n, k, e, s); break;
        case 2: launch_tn_mode<ACT, 2>(mode, a, b, out, m, n, k, e, s); break;
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
                    ep.vt_ld % 32 == 0 && ep.vt_seq % 4 == 0 && aligned(ep.vt, 16),
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
        const int64_t threads = m * (n / 8);
        k_gemm_smallk<<<static_cast<int>((threads + 255) / 256), 256, 0, s>>>(
            a, b, out, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), e, mode);
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
    const int splits = ep.splitk > 0 ? ep.splitk : gemm_splits(m, n, k, ep);
    if (splits > 1) {
        require(k % (BK * splits) == 0 && !ep.vt && mode != EPI_ROW_ADD && splits <= 16,
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
        launch_tn_splitk(a, b, partial, m, n, k, splits, s);
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
    const int mt = ep.vt ? kMaxMT : gemm_tile_mt(m, n);   // the transposed V store: 256-row tiles
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
    if (ep.residual) launch_tn<0, EPI_RESIDUAL, true>(cv.in, wr, out, m, c_out, k, e, s, cv);
    else launch_tn<0, EPI_STORE, true>(cv.in, wr, out, m, c_out, k, e, s, cv);
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
    return gemm_splitk_choice(m, n, k);
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
        launch_tn_splitk(a, b, partial, m, n, k, splits, s);
        launch_check("gemm (split-K partials)");
    }
    ProfileScope ps(K_ELEMENTWISE, s, static_cast<double>(m) * n * (4.0 * splits + 4.0));
    const int64_t mn = m * n;
    const int64_t blocks = std::min<int64_t>((mn / 4 + 255) / 256, 8192);
    k_splitk_residual<<<static_cast<int>(blocks), 256, 0, s>>>(partial, splits, residual, out, mn);
    launch_check("gemm (split-K reduce)");
}

}  // namespace bh

