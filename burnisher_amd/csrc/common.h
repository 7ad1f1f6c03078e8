// Internal declarations shared by the HIP kernels and the C-ABI layer of libburnisher_hip.so.
//
// Numerics contract (the reference oracle, src/cpu/ops_cpu.cpp and src/core/tensor.cpp:85-96):
// every op reads bf16 as float exactly, computes in fp32 and rounds once per stored element with
// round-to-nearest-even. Elementwise kernels here use non-contracting fp32 operations
// (__fadd_rn/__fmul_rn) wherever the oracle does a separate multiply and add, so they reproduce
// the oracle bit for bit; only the GEMM and attention reductions differ in summation order.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "../../include/burnisher_hip.h"

namespace bh {

using bf16_t = uint16_t;

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

// ---- bf16 storage ---------------------------------------------------------------------------

__host__ __device__ inline float bf2f(bf16_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
#else
    uint32_t u = static_cast<uint32_t>(v) << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
#endif
}

// Round-to-nearest-even, NaN kept NaN (dtype.h:64-72 semantics). On the device this is the
// hardware conversion (v_cvt_pk_bf16_f32, the same rounding, a NaN stays a quiet NaN): the
// integer form's NaN test compiles to a divergent branch per value, which made every bf16 store
// epilogue branch-bound.
__host__ __device__ inline bf16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_bit_cast(bf16_t, static_cast<__bf16>(f));
#else
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
#endif
}

// What a store through the tensor dtype does to a float.
__host__ __device__ inline float round_bf16(float f) { return bf2f(f2bf(f)); }

// Two bf16 from one conversion (v_cvt_pk_bf16_f32, the same rounding as f2bf): a pair built from
// two f2bf calls costs a conversion per value plus a mask, a shift and an or.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline uint32_t f2bf2(float lo, float hi) {
    bf16x2_t v;
    v[0] = static_cast<__bf16>(lo);
    v[1] = static_cast<__bf16>(hi);
    return __builtin_bit_cast(uint32_t, v);
}

// bf16 of an fp64 value the way the reference's host code stores one: Tensor::set(static_cast<
// float>(v)) rounds to float, then to bf16 (two roundings; the second one sees a tie when the
// float lands exactly halfway between two bf16 values). The second rounding works on the float's
// bits: with the hardware conversion, the compiler may fuse fptrunc f64->f32->bf16 into one
// f64->bf16 rounding (round-to-odd to f32, then RNE), which breaks exactly those ties.
__host__ __device__ inline bf16_t bf16_from_f64(double v) {
    const float f = static_cast<float>(v);
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<bf16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

// s_waitcnt through the builtin (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt
// 11:8; expcnt is left unconstrained). Unlike inline assembly, the compiler's own wait insertion
// sees this wait: after an opaque one it must assume that scalar loads issued before a loop may
// still be outstanding, and then waits for lgkmcnt(0) before the first use of ANY LDS read in
// the loop instead of only the reads that use needs.
template <int VM, int LGKM>
__device__ __forceinline__ void s_waitcnt() {
    static_assert(VM >= 0 && VM < 64 && LGKM >= 0 && LGKM < 16, "waitcnt range");
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (LGKM << 8) | ((VM >> 4) << 14));
}

// Position of key `kv` in a V^T row as the head_dim-72 attention kernel reads it. Within each
// 32-key chunk, with key bits b4..b0, the key sits at slot b2 b4 b3 b1 b0: the 16 bytes at slot
// 8r are the eight keys lane row r (lanes 16r..16r+15) holds after its 32x32 score tile is
// converted to bf16 and one permlane16 swap pairs up the query halves, so P feeds the output
// product with no further exchange. Runs of four keys stay contiguous.
__host__ __device__ inline int64_t vt_pos(int64_t kv) {
    return (kv & ~int64_t{31}) | (((kv >> 2) & 1) << 4) | (((kv >> 4) & 1) << 3) |
           (((kv >> 3) & 1) << 2) | (kv & 3);
}

// ---- errors ---------------------------------------------------------------------------------

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw Error(std::string("hip: ") + what + ": " + hipGetErrorString(e));
}

// Checked after every launch: an asynchronous launch failure otherwise surfaces as a wrong
// number in a later op.
inline void launch_check(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        throw Error(std::string("hip: ") + what + " launch: " + hipGetErrorString(e));
    }
}

inline void require(bool ok, const std::string& msg) {
    if (!ok) throw Error(msg);
}

// The C boundary: the message of the last failing call on this host thread (capi.cpp).
void set_last_error(const std::string& msg);

// A pointer the GPU cannot dereference is refused at the boundary rather than faulting in a
// kernel (the reference's `require_device`, ops_cuda.cu:79-88): null, memory the HIP runtime
// does not know, and registered or pinned HOST memory are all errors naming the operand.
// Whether this host thread's calls look operands up (bh_set_operand_checks, capi.cpp).
bool operand_checks();
inline void require_device_ptr(const void* p, const char* op, const char* operand) {
    if (!p) throw Error(std::string(op) + ": " + operand + " is null");
    if (!operand_checks()) return;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        throw Error(std::string(op) + ": " + operand +
                    " is not memory the HIP runtime knows; host and device operands cannot be "
                    "mixed in one op");
    }
    if (attr.type != hipMemoryTypeDevice && attr.type != hipMemoryTypeManaged) {
        throw Error(std::string(op) + ": " + operand +
                    " is a HOST pointer. Mixing host and device operands in one op is a fault, "
                    "not a slow path.");
    }
}
inline void optional_device_ptr(const void* p, const char* op, const char* operand) {
    if (p) require_device_ptr(p, op, operand);
}

// Runs `fn`, turning an exception into status 1 plus a message for bh_last_error().
template <typename Fn>
int guarded(Fn&& fn) {
    try {
        fn();
        set_last_error("");
        return 0;
    } catch (const std::exception& e) {
        set_last_error(e.what());
        return 1;
    } catch (...) {
        set_last_error("unknown error");
        return 1;
    }
}

// ---- launch profiler (capi.cpp) -------------------------------------------------------------

enum KernelClass {
    K_GEMM = 0,
    K_GEMV = 1,
    K_ATTN_SELF = 2,
    K_ATTN_CROSS = 3,
    K_NORM = 4,
    K_ELEMENTWISE = 5,
    K_GEMM_FF0 = 6,
    K_GEMM_FF2 = 7,
    K_GEMM_QKV = 8,
    K_COUNT = 9
};

// RAII bracket: records a start event on construction and a stop event on destruction, on
// `stream`, when profiling is enabled; a no-op otherwise. `work` is the algorithmic FLOP (or
// bytes) of the launch. `also` is a second class credited with the same interval (-1: none).
struct ProfileScope {
    ProfileScope(int cls, hipStream_t stream, double work, int also = -1);
    ~ProfileScope();
    int cls_, also_;
    hipStream_t stream_;
    double work_;
    int slot_ = -1;
};

// True while bh_profile_enable has a nonzero mask (launches are then bracketed by events).
bool profiling_enabled();

// Geometry of a dit-step engine, for the denoise loop (dit_engine.cpp).
struct DitGeometry {
    int64_t batch, in_channels, out_channels, latent_hw;
    int mode;
};
DitGeometry dit_geometry(const bh_dit* e);
// The engine's row schedule (BH_DIT_ROWS_*): a captured forward holds the schedule it ran.
int dit_rows(const bh_dit* e);
// bh_dit_forward without the C error boundary (throws Error). With caption_ready, a fused engine
// reuses the caption projection and cross-attention K/V of its previous forward, which must have
// had the same caption; the op-by-op plan always recomputes them.
void dit_forward_step(bh_dit* e, const void* latent, double timestep, const void* caption,
                      const void* caption_mask, int mask_dtype, void* out, hipStream_t s,
                      bool caption_ready);

// Engine hint: which engine GEMM is running, so its launch is also credited to a sub-class.
void set_gemm_subclass(int cls);
int gemm_subclass();

// ---- kernel launchers (one per .hip file) ---------------------------------------------------

struct GemmEpilogue {
    int act = 0;               // 0 none, 1 gelu-tanh, 2 silu
    bool round_mid = false;    // round epilogue(acc+bias) to bf16 before row_add/residual
    const bf16_t* row_add = nullptr;
    int64_t row_add_period = 1;
    const bf16_t* residual = nullptr;
    const bf16_t* gate = nullptr;
    int64_t gate_rows = 1;
    int64_t ld_out = 0;        // 0 means n
    // Transposed store of the V columns of a fused projection, for the head_dim-72 attention:
    // column n with w = n % vt_period >= vt_col0 is head h = (w - vt_col0) / vt_dim, dim
    // dd = (w - vt_col0) % vt_dim of block n / vt_period, and row m is token m % vt_seq of batch
    // m / vt_seq; it goes to vt[((blk * batches + b) * vt_heads + h) * vt_dim + dd][token] with
    // rows of vt_ld tokens, and nowhere else. vt_col0 and vt_period must be multiples of 144.
    bf16_t* vt = nullptr;
    int64_t vt_period = 0, vt_col0 = 0, vt_seq = 0, vt_ld = 0;
    int vt_heads = 0, vt_dim = 72;
    // Split-K (GEMMs with too few output tiles to fill the CUs): 0 lets the shape decide
    // (gemm_splits), 1 never splits, 2 <= n <= 8 sums exactly n K slices. The fp32 partials go to
    // `splitk_ws` (splitk_ws_floats floats, at least splits * m * n) or, when it is null, to a
    // per-device library buffer grown on demand (calls that overlap on one device share it).
    int splitk = 0;
    float* splitk_ws = nullptr;
    int64_t splitk_ws_floats = 0;
};

// A 3x3, stride-1, pad-1 convolution read as a GEMM (batch 1, NHWC): out[H*W, c_out] =
// im2col(in)[H*W, 9*c_in] . W[c_out, 9*c_in]^T with W repacked [c_out][ky][kx][c_in]. With `up`
// the input is in_h x in_w = H/2 x W/2 and upsampled 2x (nearest) on the fly. `zero` points at
// 64 zero bf16, the source of the padding taps.
struct ConvGeom {
    const bf16_t* in = nullptr;
    const bf16_t* zero = nullptr;
    int H = 0, W = 0;
    int in_h = 0, in_w = 0;
    int c_in = 0;
    int up = 0;
};
void launch_conv3x3_bf16(const ConvGeom& cv, const bf16_t* wr, const bf16_t* bias, bf16_t* out,
                         int64_t c_out, const GemmEpilogue& ep, hipStream_t s);

// ---- the VAE decoder's kernels (vae.hip) ----
// [batch][R][C] -> [batch][C][R], bf16.
void launch_transpose_bf16(const bf16_t* in, bf16_t* out, int64_t batch, int64_t R, int64_t C,
                           hipStream_t s);
// Device scratch of a channels-last GroupNorm: per-chunk fp64 partials and the group statistics.
struct GroupNormScratch {
    double* part = nullptr;   // max_chunks * 64
    double* mean = nullptr;   // 64
    float* inv = nullptr;     // 64
    int64_t max_chunks = 0;
};
bool gn_nhwc_supported(int64_t C, int64_t G);
// GroupNorm over x [S, C] (channels-last, batch 1), G groups of C/G channels, then optionally
// SiLU; each rounded to bf16 as the reference stores them. out may alias x.
void launch_group_norm_nhwc(const bf16_t* x, bf16_t* out, int64_t S, int64_t C, int64_t G,
                            float eps, const bf16_t* w, const bf16_t* b, bool silu,
                            GroupNormScratch& sc, hipStream_t s);
// Stride-1 "same" convolution, channels-last, w in the checkpoint layout [co][ci][k][k], in the
// reference's summation order (bit-identical with it).
void launch_conv_direct_nhwc(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* out,
                             int64_t H, int64_t W, int64_t ci, int64_t co, int64_t k, int64_t pad,
                             hipStream_t s);
void launch_upsample_nchw(const bf16_t* in, bf16_t* out, int64_t planes, int64_t H, int64_t W,
                          int64_t f, hipStream_t s);
void launch_repack3x3(const bf16_t* w, bf16_t* out, int64_t co, int64_t ci, hipStream_t s);
// The same, zero-padded to cop output and cip input channels.
void launch_repack3x3_pad(const bf16_t* w, bf16_t* out, int64_t co, int64_t ci, int64_t cop,
                          int64_t cip, hipStream_t s);
// [R][C] -> [keep][R] (the first `keep` columns only), batch 1.
void launch_transpose_keep_bf16(const bf16_t* in, bf16_t* out, int64_t R, int64_t C, int64_t keep,
                                hipStream_t s);
// Rows [S][C] -> [S][Cp], columns C..Cp-1 zero.
void launch_pad_rows(const bf16_t* in, bf16_t* out, int64_t S, int64_t C, int64_t Cp, hipStream_t s);
// The op-level (NCHW) convolution and GroupNorm; they use per-device scratch grown on demand.
void launch_conv2d_nchw(const bf16_t* x, const bf16_t* w, const bf16_t* bias, bf16_t* out,
                        int64_t batch, int64_t ci, int64_t h, int64_t wd, int64_t co, int64_t k,
                        int64_t pad, hipStream_t s);
void launch_group_norm_nchw(const bf16_t* x, const bf16_t* w, const bf16_t* b, bf16_t* out,
                            int64_t rows, int64_t cols, float eps, int64_t groups, int64_t channels,
                            hipStream_t s);
// The T5 encoder's tensors with their checkpoint shapes (t5_engine.cpp).
std::vector<std::pair<std::string, std::vector<int64_t>>> t5_tensor_shapes(const bh_t5_config& c);
// The VAE decoder's tensors with their checkpoint shapes (vae_engine.cpp).
std::vector<std::pair<std::string, std::vector<int64_t>>> vae_tensor_shapes(const bh_vae_config& c);
// Keys per V^T row for the head_dim-512 attention (S rounded up to 32).
int64_t vt512_ld(int64_t S);
// Single-head attention at head_dim 512: q, k, v, out [S, 512]; vt is scratch of 512 x vt512_ld(S).
void launch_attention512(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* vt, bf16_t* out,
                         int64_t S, float scale, hipStream_t s);

// bf16 out[m, n] = A[m, k] . B[n, k]^T (+bias) with `ep`. Picks the MFMA tile kernel, the
// small-M kernel or the reference-order kernel by shape.
void launch_gemm_bf16(const bf16_t* a, const bf16_t* b, const bf16_t* bias, bf16_t* out,
                      int64_t m, int64_t n, int64_t k, const GemmEpilogue& ep, hipStream_t s);
// Split-K for GEMMs with too few output tiles to fill the CUs: the number of K slices (1: none)
// that keeps every slice's workgroups resident at once.
int gemm_splitk_choice(int64_t m, int64_t n, int64_t k);
// The K slices launch_gemm_bf16 uses for this shape and epilogue when ep.splitk is 0 (1: none):
// considered when K holds at least 48 k-tiles, at most half the CUs would hold a 256-row tile, the
// MFMA kernel applies and the epilogue is a plain, residual or gated store (no row add, no
// transposed V); then the slice count (up to 8) whose best tile height gives the least estimated
// time, the fp32 partials' traffic included. The tile shape (height and width) of the split
// launch is chosen per launch and changes no sum.
int gemm_splits(int64_t m, int64_t n, int64_t k, const GemmEpilogue& ep);
// out = bf16(residual + bf16(A . B^T)) through `splits` fp32 partials (partial holds
// splits * m * n floats) summed in slice order; out may alias residual.
void launch_gemm_splitk_residual(const bf16_t* a, const bf16_t* b, float* partial, int splits,
                                 const bf16_t* residual, bf16_t* out, int64_t m, int64_t n, int64_t k,
                                 hipStream_t s);
// Any dtype / layout, reference summation order: one thread per output (tests, fp32, [K,N] B).
void launch_gemm_generic(const void* a, const void* b, const void* bias, void* out, int64_t m,
                         int64_t n, int64_t k, bool b_transposed, int act, bool f32,
                         hipStream_t s);

struct AttnShape {
    int64_t batch, heads, q_len, kv_len, head_dim;
    int64_t ld_q, ld_kv, ld_o;  // row strides in elements
    float scale;                // resolved (never 0)
};
// bias: optional bf16 [heads, q_len, kv_len] added to the scaled scores (head_dim <= 128 only).
// The head_dim-72 and -512 kernels read V transposed: into `vt_buf` (vt_buf_elems elements, at
// least attention_vt_elems of the call, else an error) when given, else into a per-device
// workspace that grows on demand and that calls overlapping on one device share.
// `splits`, `part`, `part_floats`, `qb0`: the head_dim-72 kernel's key splits and their fp32
// partials, as launch_flash72 takes them (other kernels ignore them).
void launch_attention_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v, bf16_t* out,
                           const AttnShape& sh, const void* key_mask, bool mask_f32,
                           hipStream_t s, const bf16_t* bias = nullptr, bf16_t* vt_buf = nullptr,
                           int64_t vt_buf_elems = 0, int splits = 0, float* part = nullptr,
                           int64_t part_floats = 0, int qb0 = 0);
// The V^T elements launch_attention_bf16 needs for these operands (0: the kernel reads V as is).
int64_t attention_vt_elems(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* out,
                           const AttnShape& sh, const void* key_mask, const bf16_t* bias);
// The fp32 key-split partials launch_attention_bf16 needs for these operands with splits = 0
// (0: the call does not split).
int64_t attention_part_floats(const bf16_t* q, const bf16_t* k, const bf16_t* v, const bf16_t* out,
                              const AttnShape& sh, const void* key_mask, const bf16_t* bias);
// The allocation-free attention's scratch: a fixed device array of kNoAllocScratchBytes per device,
// its address looked up (hipGetSymbolAddress) on the first call with that device current. It holds
// V^T and, after it at a 256-byte boundary, the key-split partials.
constexpr int64_t kNoAllocScratchBytes = int64_t{64} << 20;
bf16_t* noalloc_scratch();
// Flash attention at head_dim 72 with V supplied transposed (flash72.hip): vt holds, for each
// (b, h, d), a row of vt_ld >= flash72_vt_ld(kv_len) keys, zero past kv_len.
int64_t flash72_vt_ld(int64_t kv_len);
// `splits`: key splits (0: flash72_plan decides, 1: none), for query blocks qb0 and up (the ones
// below run whole). A split launch writes fp32 partials to `part` (part_floats floats, at least
// flash72_plan_floats) or, when it is null, to a per-device library buffer grown on demand, and a
// last kernel combines them into `out`.
void launch_flash72(const bf16_t* q, int64_t ld_q, const bf16_t* k, int64_t ld_k,
                    const bf16_t* vt, int64_t vt_ld, bf16_t* out, int64_t ld_o, int64_t batch,
                    int64_t heads, int64_t q_len, int64_t kv_len, float scale,
                    const void* key_mask, bool mask_f32, hipStream_t s, int splits = 0,
                    float* part = nullptr, int64_t part_floats = 0, int qb0 = 0);
// Key splits for a head_dim-72 attention whose workgroups (512 queries of one batch row and head
// each) would fill at most half the CUs: as many as still fit at once, at least two key blocks
// each; 1 for the resident (kv_len <= 448) kernel and for an output whose rows are not 16-byte
// aligned.
// The cross-attention block's Q projection and its head_dim-72 attention over a short caption in
// one launch (cross_fused.hip): ctx = attention(bf16(x wq^T + bq), K, V^T, mask), bit-identical
// with launch_gemm_bf16 followed by launch_flash72. x is [batch * tokens, heads * 72]; K rows of
// stride ld_k at [batch, kv_len]; V^T as launch_flash72 reads it. Supported when tokens % 256 == 0,
// the head count is even, kv_len <= 448 and the 256 x 144 tiles fill more than half the CUs.
bool cross_fused_supported(int64_t batch, int64_t tokens, int64_t heads, int64_t head_dim, int64_t kv_len);
void launch_cross_fused(const bf16_t* x, const bf16_t* wq, const bf16_t* bq, int64_t batch,
                        int64_t tokens, int64_t heads, const bf16_t* k, int64_t ld_k, const bf16_t* vt,
                        int64_t vt_ld, int64_t kv_len, const void* key_mask, bool mask_f32,
                        bf16_t* ctx, int64_t ld_o, float scale, hipStream_t s);
int flash72_splits(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len,
                   const void* out = nullptr, int64_t ld_o = 8);
int64_t flash72_part_floats(int64_t batch, int64_t heads, int64_t q_len, int splits);
// The key splits launch_flash72 picks with splits = 0: `splits` ways for the query blocks from
// qb0 on (all of them when qb0 == 0), query blocks below qb0 whole. Besides flash72_splits' case,
// it splits the query blocks of a last, at most half-full round of workgroups (qb0 > 0).
struct Flash72Plan {
    int splits;
    int qb0;
};
Flash72Plan flash72_plan(int64_t batch, int64_t heads, int64_t q_len, int64_t kv_len,
                         const void* out = nullptr, int64_t ld_o = 8);
int64_t flash72_plan_floats(int64_t batch, int64_t heads, int64_t q_len, const Flash72Plan& p);
// V [batch, kv_len, ld_v] (head-last, head_dim 72) -> the V^T rows launch_flash72 reads.
void launch_transpose_v72(const bf16_t* v, int64_t ld_v, int64_t batch, int64_t heads,
                          int64_t kv_len, bf16_t* vt, int64_t vt_ld, hipStream_t s);
// Reference-order attention (one thread per query row), any dtype, additive bias supported.
void launch_attention_generic(const void* q, const void* k, const void* v, void* out,
                              const AttnShape& sh, const void* bias, const void* key_mask,
                              bool mask_f32, bool f32, hipStream_t s);

void launch_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                 int64_t cols, float eps, bool rms, bool f32, hipStream_t s);
void launch_norm_modulate(const bf16_t* x, const bf16_t* mod, int64_t mod_chunks,
                          int64_t shift_chunk, int64_t scale_chunk, const bf16_t* table,
                          int64_t shift_row, int64_t scale_row, bf16_t* out, int64_t batch,
                          int64_t tokens, int64_t channels, float eps, hipStream_t s);
// Same, reading precomputed (already rounded) shift/scale rows of [batch, channels].
void launch_norm_modulate_pre(const bf16_t* x, const bf16_t* shift, const bf16_t* scale,
                              bf16_t* out, int64_t batch, int64_t tokens, int64_t channels,
                              float eps, hipStream_t s);
void launch_modulate(const void* x, const void* scale, const void* shift, void* out,
                     int64_t batch, int64_t tokens, int64_t channels, const void* residual,
                     const void* gate, bool f32, hipStream_t s);
void launch_activation(const void* x, void* out, int64_t numel, int kind, const void* gate,
                       bool f32, hipStream_t s);
// Gated GELU over the rows of a fused [rows, 2F] projection: out[r, j] = gelu_tanh(in[r, j]) *
// in[r, F + j], as ActivationArgs GeluGated computes it on two separate tensors.
void launch_gelu_gated_rows(const bf16_t* in, bf16_t* out, int64_t rows, int64_t F, hipStream_t s);
// ---- the T5 encoder's kernels (t5.hip) ----
// GatherArgs: out[r, :] = table[(int64)ids[r], :]; an id outside [0, table_rows) gives a NaN row.
void launch_gather(const void* table, const float* ids, void* out, int64_t rows, int64_t cols,
                   int64_t table_rows, bool f32, hipStream_t s);
// bias[h, q, k] = rel[bucket[k - q + S - 1] * heads + h] (bf16 [heads, S, S]).
void launch_rel_bias(const bf16_t* rel, const int* bucket, bf16_t* bias, int64_t heads, int64_t S,
                     hipStream_t s);
void launch_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner,
                float scale, bool broadcast_b, bool f32, hipStream_t s);
void launch_chunk(const void* mod, const void* table, void* out, int64_t batch, int64_t channels,
                  int64_t chunks, int64_t chunk, int64_t table_chunk, bool f32, hipStream_t s);
// Every chunk of every layer at once: out[l][c6][b][ch] = mod[b, c6*ch_n + ch] + tables[l][c6, ch]
// where tables is `layers` pointers to [6, channels] tables.
void launch_chunk_all(const bf16_t* mod, const bf16_t* const* tables_dev, bf16_t* out,
                      float* out_f32, int64_t layers, int64_t batch, int64_t channels,
                      hipStream_t s);
// LayerNorm + modulate with float shift and 1 + scale rows ([batch, channels], as k_chunk_all
// writes them); channels a multiple of 128, at most 4096. `warm` (device memory, or null): the
// kernel also reads 4 bytes of each 128-byte line of those `warm_bytes` (at most 8 KiB per row)
// and discards them, so that the weights of the GEMM after the norm come from the memory-side
// cache instead of HBM.
bool norm_modulate_f32_supported(int64_t channels);
void launch_norm_modulate_f32(const bf16_t* x, const float* shift, const float* scale1,
                              bf16_t* out, int64_t batch, int64_t tokens, int64_t channels,
                              float eps, hipStream_t s, const void* warm = nullptr,
                              int64_t warm_bytes = 0);
void launch_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
                  int64_t patch, bool inverse, bool f32, hipStream_t s);
// Cos-first sinusoidal timestep embedding, fp64, rounded to bf16, broadcast to `batch` rows
// (weights.cpp:107-121 and the host broadcast at pixart_dit.cpp:156-160).
void launch_timestep_embedding(double t, int dim, int64_t batch, void* out, bool f32, hipStream_t s);
// ScaleArgs: out[i] = in[i] * scale, one rounding (out may alias in).
void launch_scale(const void* in, void* out, int64_t n, float scale, bool f32, hipStream_t s);

}  // namespace bh
