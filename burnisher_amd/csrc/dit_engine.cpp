// The dit-step engine: PixArt-Sigma's denoiser forward (reference: src/models/pixart_dit.cpp:
// 112-304) on one MI355X.
//
// Two plans over the same kernels:
//
//   BH_DIT_FUSED   the MI355X plan. Per layer it launches 10 kernels instead of the
//                  reference's 22: LayerNorm+chunk+modulate as one row kernel; Q,K,V as one
//                  [M, 3d] GEMM (the attention reads the three column blocks in place through
//                  row strides); the gated residuals and the cross-attention residual inside the
//                  out-projection GEMM epilogues; every layer's caption K/V projection -- which
//                  depends only on the caption -- hoisted into one [Mcap, L*2d] GEMM before the
//                  block loop; every layer's six adaLN chunks formed by one kernel up front. The
//                  result equals the reference op sequence with every intermediate rounded where
//                  the reference stores it (the fused epilogues round the GEMM output first), so
//                  fusion itself changes no bits; only GEMM/attention summation order does.
//
//   BH_DIT_OPWISE  the reference graph op by op through the per-op C entry points, exactly the
//                  calls a reference `register_impl` adapter would receive: the drop-in path.
//
// Everything is allocated at create time (zero-filled, as the reference device allocator hands
// out memory); forward allocates nothing and never synchronises the host. The timestep
// embedding is computed on the device from the scalar timestep, so no upload happens per step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/burnisher_hip.h"
#include "common.h"

namespace bh {
namespace {

struct DevBuf {
    void* p = nullptr;
    size_t bytes = 0;
    DevBuf() = default;
    explicit DevBuf(size_t n) : bytes(n) {
        hip_check(hipMalloc(&p, n ? n : 1), "hipMalloc");
        hip_check(hipMemset(p, 0, n ? n : 1), "hipMemset");
    }
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    DevBuf(DevBuf&& o) noexcept : p(o.p), bytes(o.bytes) { o.p = nullptr; o.bytes = 0; }
    DevBuf& operator=(DevBuf&& o) noexcept {
        if (this != &o) {
            reset();
            p = o.p;
            bytes = o.bytes;
            o.p = nullptr;
            o.bytes = 0;
        }
        return *this;
    }
    ~DevBuf() { reset(); }
    void reset() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
    bf16_t* bf() const { return static_cast<bf16_t*>(p); }
};

// 2-D sin/cos position table [grid*grid, dim] in fp64 (pixart_dit.cpp:32-77): each 1-D
// half is SIN first then COS over frequencies 1/10000^(i/half); the first half of the channels
// is driven by the column (x) coordinate, the second by the row (y); the coordinate along an
// axis is i / (grid / base) / interpolation_scale.
std::vector<double> position_table(int dim, int grid, int base, double interp) {
    std::vector<double> axis(grid);
    for (int i = 0; i < grid; ++i) {
        axis[i] = static_cast<double>(i) / (static_cast<double>(grid) / base) / interp;
    }
    const int half_dim = dim / 2;       // channels per axis
    const int quarter = half_dim / 2;   // sin (or cos) channels per axis
    std::vector<double> omega(quarter);
    for (int i = 0; i < quarter; ++i) {
        omega[i] = 1.0 / std::pow(10000.0, static_cast<double>(i) / quarter);
    }
    std::vector<double> out(static_cast<size_t>(grid) * grid * dim);
    for (int r = 0; r < grid; ++r) {
        for (int c = 0; c < grid; ++c) {
            double* row = &out[(static_cast<size_t>(r) * grid + c) * dim];
            for (int i = 0; i < quarter; ++i) {
                const double ax = axis[c] * omega[i];
                const double ay = axis[r] * omega[i];
                row[i] = std::sin(ax);
                row[quarter + i] = std::cos(ax);
                row[half_dim + i] = std::sin(ay);
                row[half_dim + quarter + i] = std::cos(ay);
            }
        }
    }
    return out;
}

}  // namespace
}  // namespace bh

using namespace bh;

struct bh_dit {
    bh_dit_config cfg{};
    bh_dit_weights w{};
    std::vector<bh_dit_block_weights> blocks;
    int mode = BH_DIT_FUSED;
    int64_t B = 0, latent = 0, cap_len = 0, grid = 0, N = 0, M = 0, Mcap = 0, d = 0, dff = 0;
    int64_t patch_in = 0, patch_out = 0;

    DevBuf pos_table, patches, x, normed, modded, q, k, v, qkv, ctx, proj, q2, kc, vc, ff0;
    DevBuf temb, h_t, emb_t, silu_t, modulation, cap_h, cap, kv_all, chunks, tables_dev;
    DevBuf chunks_f32;   // the chunks as floats, scales as 1 + scale (fused norm kernel)
    DevBuf shift, scale, gate, zero, tokens;
    // The fused plan's packed projections: every layer's [3d, d] Q/K/V weight and [3d] bias, and
    // all layers' caption K/V as one [L * 2d, d] weight and [L * 2d] bias. When the caller's
    // weights already lie that way (each layer's q, k, v back to back; every layer's attn2 k, v
    // back to back in layer order) these point into them; otherwise into copies in w_qkv ...
    std::vector<const bf16_t*> qkv_w, qkv_b;
    const bf16_t* kv_w = nullptr;
    const bf16_t* kv_b = nullptr;
    DevBuf w_qkv, b_qkv, w_kv, b_kv;   // ... made at create (fused plan, scattered weights only)
    DevBuf vt_self, vt_cross;         // V transposed for the attention kernel (fused plan)
    DevBuf vt_op;                     // head_dim 72 without the transposed store: the engine's
    int64_t vt_op_elems = 0;          // own V^T buffer (never the op-level shared workspace)
    int64_t vt_ld_self = 0, vt_ld_cross = 0;
    bool vt72 = false;
    int64_t qkv_ld = 0;               // row stride of qkv: 2d when V goes to V^T, else 3d
    // The cross-attention's Q projection fused into its attention (cross_fused.hip), for launches
    // of at least cross_fused_min_rows batch rows (its 256 x 144 tiles must fill more than half
    // the CUs).
    bool cross_fused = false;
    int64_t cross_fused_min_rows = 0;
    int64_t workspace = 0;
    // Row-group schedule of the fused plan (BH_DIT_ROWS_*): the second row group's stream and the
    // fork/join events, created with the engine when the batch has two or more rows.
    int row_split = BH_DIT_ROWS_JOINED;
    hipStream_t s2 = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    DevBuf splitk;                    // fp32 split-K partials of the fused plan's long-K GEMMs
    int64_t splitk_floats = 0;
    Flash72Plan plan_self{1, 0}, plan_cross{1, 0};   // key splits of the head_dim-72 attentions (full batch)
    DevBuf attn_part;                 // their fp32 partials, a row group's slice at its batch offset

    ~bh_dit() {
        if (fork_ev) (void)hipEventDestroy(fork_ev);
        if (join_ev) (void)hipEventDestroy(join_ev);
        if (s2) (void)hipStreamDestroy(s2);
    }

    DevBuf make(int64_t elems) {
        workspace += elems * 2;
        return DevBuf(static_cast<size_t>(elems) * 2);
    }
    DevBuf make_f32(int64_t elems) {
        workspace += elems * 4;
        return DevBuf(static_cast<size_t>(elems) * 4);
    }
};

DitGeometry bh::dit_geometry(const bh_dit* e) {
    return DitGeometry{e->B, e->cfg.in_channels, e->cfg.out_channels, e->latent, e->mode};
}

int bh::dit_rows(const bh_dit* e) { return e->row_split; }

namespace {

void check_weights(const bh_dit_config& c, const bh_dit_weights& w) {
    const void* top[] = {w.pos_embed_w, w.pos_embed_b, w.t_emb1_w, w.t_emb1_b, w.t_emb2_w,
                         w.t_emb2_b,    w.adaln_w,     w.adaln_b,  w.cap1_w,   w.cap1_b,
                         w.cap2_w,      w.cap2_b,      w.out_table, w.proj_out_w, w.proj_out_b};
    for (const void* p : top) {
        require(p != nullptr, "dit: a model weight pointer is null. A model that ran with a missing "
                              "weight would produce a plausible image from wrong numbers.");
        require_device_ptr(p, "dit_create", "a model weight");
    }
    require(w.blocks != nullptr, "dit: null block weight table");
    for (int l = 0; l < c.num_layers; ++l) {
        const bh_dit_block_weights& b = w.blocks[l];
        const void* ps[] = {b.scale_shift_table, b.attn1_q_w, b.attn1_q_b, b.attn1_k_w, b.attn1_k_b,
                            b.attn1_v_w, b.attn1_v_b, b.attn1_o_w, b.attn1_o_b, b.attn2_q_w,
                            b.attn2_q_b, b.attn2_k_w, b.attn2_k_b, b.attn2_v_w, b.attn2_v_b,
                            b.attn2_o_w, b.attn2_o_b, b.ff0_w, b.ff0_b, b.ff2_w, b.ff2_b};
        for (const void* p : ps) {
            require(p != nullptr, "dit: transformer_blocks." + std::to_string(l) +
                                      " has a null weight pointer");
            require_device_ptr(p, "dit_create", "a transformer block weight");
        }
    }
}

void d2d(void* dst, const void* src, size_t bytes, hipStream_t s) {
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync");
}

void ok(int status) {
    if (status != 0) throw Error(bh_last_error());
}

// The reference graph, op by op through the C entry points (pixart_dit.cpp:132-303).
void forward_opwise(bh_dit& e, const void* latent, double t, const void* caption,
                    const void* mask, int mask_dtype, void* out, hipStream_t s) {
    const auto& c = e.cfg;
    const int64_t B = e.B, N = e.N, M = e.M, d = e.d, P = c.patch_size;
    const int BF = BH_BF16;
    void* st = s;
    ok(bh_patch(latent, e.patches.p, B, c.in_channels, e.grid, P, 0, BF, st));
    ok(bh_gemm(e.patches.p, e.w.pos_embed_w, e.w.pos_embed_b, e.x.p, M, d, e.patch_in, 1,
               BH_EPI_NONE, BF, st));
    ok(bh_add(e.x.p, e.pos_table.p, e.x.p, B, N * d, 1.0f, 1, BF, st));

    {
        ProfileScope ps(K_ELEMENTWISE, s, 0.0);
        launch_timestep_embedding(t, 256, B, e.temb.p, false, s);
    }
    ok(bh_gemm(e.temb.p, e.w.t_emb1_w, e.w.t_emb1_b, e.h_t.p, B, d, 256, 1, BH_EPI_SILU, BF, st));
    ok(bh_gemm(e.h_t.p, e.w.t_emb2_w, e.w.t_emb2_b, e.emb_t.p, B, d, d, 1, BH_EPI_NONE, BF, st));
    ok(bh_activation(e.emb_t.p, e.silu_t.p, B * d, BH_EPI_SILU, nullptr, BF, st));
    ok(bh_gemm(e.silu_t.p, e.w.adaln_w, e.w.adaln_b, e.modulation.p, B, 6 * d, d, 1, BH_EPI_NONE,
               BF, st));

    ok(bh_gemm(caption, e.w.cap1_w, e.w.cap1_b, e.cap_h.p, e.Mcap, d, c.caption_channels, 1,
               BH_EPI_GELU, BF, st));
    ok(bh_gemm(e.cap_h.p, e.w.cap2_w, e.w.cap2_b, e.cap.p, e.Mcap, d, d, 1, BH_EPI_NONE, BF, st));

    const float eps = static_cast<float>(c.eps);
    for (int l = 0; l < c.num_layers; ++l) {
        const bh_dit_block_weights& bw = e.blocks[l];
        const void* table = bw.scale_shift_table;
        ok(bh_norm(e.x.p, nullptr, nullptr, e.normed.p, M, d, eps, 0, 0, 0, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.shift.p, B, d, 6, 0, 0, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.scale.p, B, d, 6, 1, 1, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.gate.p, B, d, 6, 2, 2, BF, st));
        ok(bh_modulate(e.normed.p, e.scale.p, e.shift.p, e.modded.p, B, N, d, nullptr, nullptr, BF,
                       st));
        ok(bh_gemm(e.modded.p, bw.attn1_q_w, bw.attn1_q_b, e.q.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_gemm(e.modded.p, bw.attn1_k_w, bw.attn1_k_b, e.k.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_gemm(e.modded.p, bw.attn1_v_w, bw.attn1_v_b, e.v.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_attention(e.q.p, e.k.p, e.v.p, e.ctx.p, B, c.num_heads, N, N, c.head_dim, 0.0f,
                        nullptr, nullptr, BF, BF, st));
        ok(bh_gemm(e.ctx.p, bw.attn1_o_w, bw.attn1_o_b, e.proj.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_modulate(e.proj.p, e.zero.p, e.zero.p, e.x.p, B, N, d, e.x.p, e.gate.p, BF, st));

        ok(bh_gemm(e.x.p, bw.attn2_q_w, bw.attn2_q_b, e.q.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_gemm(e.cap.p, bw.attn2_k_w, bw.attn2_k_b, e.kc.p, e.Mcap, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_gemm(e.cap.p, bw.attn2_v_w, bw.attn2_v_b, e.vc.p, e.Mcap, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_attention(e.q.p, e.kc.p, e.vc.p, e.ctx.p, B, c.num_heads, N, e.cap_len, c.head_dim,
                        0.0f, nullptr, mask, mask_dtype, BF, st));
        ok(bh_gemm(e.ctx.p, bw.attn2_o_w, bw.attn2_o_b, e.proj.p, M, d, d, 1, BH_EPI_NONE, BF, st));
        ok(bh_add(e.x.p, e.proj.p, e.x.p, M, d, 1.0f, 0, BF, st));

        ok(bh_norm(e.x.p, nullptr, nullptr, e.normed.p, M, d, eps, 0, 0, 0, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.shift.p, B, d, 6, 3, 3, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.scale.p, B, d, 6, 4, 4, BF, st));
        ok(bh_chunk(e.modulation.p, table, e.gate.p, B, d, 6, 5, 5, BF, st));
        ok(bh_modulate(e.normed.p, e.scale.p, e.shift.p, e.modded.p, B, N, d, nullptr, nullptr, BF,
                       st));
        ok(bh_gemm(e.modded.p, bw.ff0_w, bw.ff0_b, e.ff0.p, M, e.dff, d, 1, BH_EPI_GELU, BF, st));
        ok(bh_gemm(e.ff0.p, bw.ff2_w, bw.ff2_b, e.proj.p, M, d, e.dff, 1, BH_EPI_NONE, BF, st));
        ok(bh_modulate(e.proj.p, e.zero.p, e.zero.p, e.x.p, B, N, d, e.x.p, e.gate.p, BF, st));
    }

    ok(bh_chunk(e.emb_t.p, e.w.out_table, e.shift.p, B, d, 1, 0, 0, BF, st));
    ok(bh_chunk(e.emb_t.p, e.w.out_table, e.scale.p, B, d, 1, 0, 1, BF, st));
    ok(bh_norm(e.x.p, nullptr, nullptr, e.normed.p, M, d, eps, 0, 0, 0, BF, st));
    ok(bh_modulate(e.normed.p, e.scale.p, e.shift.p, e.modded.p, B, N, d, nullptr, nullptr, BF, st));
    ok(bh_gemm(e.modded.p, e.w.proj_out_w, e.w.proj_out_b, e.tokens.p, M, e.patch_out, d, 1,
               BH_EPI_NONE, BF, st));
    ok(bh_patch(e.tokens.p, out, B, c.out_channels, e.grid, P, 1, BF, st));
}

struct SubclassScope {
    explicit SubclassScope(int cls) { set_gemm_subclass(cls); }
    ~SubclassScope() { set_gemm_subclass(-1); }
};

// Every engine GEMM decides its K split (gemm_splits) on the full batch, so a row group sums
// exactly the slices the whole batch would, and keeps its fp32 partials in the engine's own buffer
// at its rows, so a captured forward holds no library-owned pointer and row groups never share.
void gemm(bh_dit& e, const bf16_t* a, const void* w, const void* b, bf16_t* out, int64_t m,
          int64_t n, int64_t k, const GemmEpilogue& ep, hipStream_t s, int64_t row0 = 0,
          int64_t rows_full = -1) {
    GemmEpilogue g = ep;
    g.splitk = gemm_splits(rows_full < 0 ? m : rows_full, n, k, ep);
    if (g.splitk > 1) {
        require(e.splitk.p != nullptr && g.splitk * (row0 + m) * n <= e.splitk_floats,
                "dit: the engine's split-K partial buffer is smaller than this GEMM needs");
        g.splitk_ws = static_cast<float*>(e.splitk.p) + g.splitk * row0 * n;
        g.splitk_ws_floats = g.splitk * m * n;
    }
    launch_gemm_bf16(a, static_cast<const bf16_t*>(w), static_cast<const bf16_t*>(b), out, m, n, k,
                     g, s);
}

// The fp32 partials of a key-split attention over batch rows [b0, b0 + nb) of q_len queries:
// the engine's buffer at that row group's offset (null when the attention does not split). The
// splits are fixed at create on the full batch, so row groups and the joined batch agree bit for
// bit and a captured forward holds no library-owned pointer.
float* attn_part(bh_dit& e, const Flash72Plan& plan, int64_t b0, int64_t nb, int64_t q_len) {
    if (plan.splits <= 1) return nullptr;
    const int64_t heads = e.cfg.num_heads;
    require(e.attn_part.p != nullptr &&
                flash72_plan_floats(b0 + nb, heads, q_len, plan) * sizeof(float) <= e.attn_part.bytes,
            "dit: the engine's attention partial buffer is smaller than this call needs");
    return static_cast<float*>(e.attn_part.p) + flash72_plan_floats(b0, heads, q_len, plan);
}

// The MI355X plan.
// `caption_ready`: the caption projection and every layer's cross-attention K/V (which depend
// only on the caption) are already in e.cap / e.kv_all / e.vt_cross from an earlier forward
// with the same caption, so that branch is skipped.
void forward_fused(bh_dit& e, const void* latent, double t, const void* caption, const void* mask,
                   int mask_dtype, void* out, hipStream_t s, bool caption_ready = false) {
    const auto& c = e.cfg;
    const int64_t B = e.B, N = e.N, M = e.M, d = e.d, P = c.patch_size, L = c.num_layers;
    const int64_t H = c.num_heads, Dh = c.head_dim;
    const float eps = static_cast<float>(c.eps);
    const GemmEpilogue plain;

    {
        ProfileScope ps(K_ELEMENTWISE, s, 4.0 * e.B * e.N * e.patch_in);
        launch_patch(latent, e.patches.p, B, c.in_channels, e.grid, P, false, false, s);
    }
    {   // patch embedding, then + position table (AddArgs broadcast over the batch)
        GemmEpilogue ep;
        ep.round_mid = true;
        ep.row_add = e.pos_table.bf();
        ep.row_add_period = N;
        gemm(e, e.patches.bf(), e.w.pos_embed_w, e.w.pos_embed_b, e.x.bf(), M, d, e.patch_in, ep, s);
    }
    {   // adaLN-single: one modulation vector per step
        {
            ProfileScope ps(K_ELEMENTWISE, s, 2.0 * B * 256);
            launch_timestep_embedding(t, 256, B, e.temb.p, false, s);
        }
        GemmEpilogue silu;
        silu.act = 2;
        gemm(e, e.temb.bf(), e.w.t_emb1_w, e.w.t_emb1_b, e.h_t.bf(), B, d, 256, silu, s);
        gemm(e, e.h_t.bf(), e.w.t_emb2_w, e.w.t_emb2_b, e.emb_t.bf(), B, d, d, plain, s);
        {
            ProfileScope ps(K_ELEMENTWISE, s, 4.0 * B * d);
            launch_activation(e.emb_t.p, e.silu_t.p, B * d, 2, nullptr, false, s);
        }
        gemm(e, e.silu_t.bf(), e.w.adaln_w, e.w.adaln_b, e.modulation.bf(), B, 6 * d, d, plain, s);
    }
    if (!caption_ready) {   // caption projection, then every layer's cross-attention K and V
        GemmEpilogue gelu;
        gelu.act = 1;
        gemm(e, static_cast<const bf16_t*>(caption), e.w.cap1_w, e.w.cap1_b, e.cap_h.bf(), e.Mcap, d,
             c.caption_channels, gelu, s);
        gemm(e, e.cap_h.bf(), e.w.cap2_w, e.w.cap2_b, e.cap.bf(), e.Mcap, d, d, plain, s);
        GemmEpilogue kv;   // every layer's K into kv_all; V into V^T at head_dim 72
        if (e.vt72) {
            kv.vt = e.vt_cross.bf();
            kv.vt_period = 2 * d;
            kv.vt_col0 = d;
            kv.vt_seq = e.cap_len;
            kv.vt_ld = e.vt_ld_cross;
            kv.vt_heads = c.num_heads;
            kv.vt_dim = c.head_dim;
        }
        gemm(e, e.cap.bf(), e.kv_w, e.kv_b, e.kv_all.bf(), e.Mcap, L * 2 * d, d, kv, s);
    }
    {
        ProfileScope ps(K_ELEMENTWISE, s, 2.0 * (B * 6 * d + L * 6 * d + L * 6 * B * d));
        launch_chunk_all(e.modulation.bf(), static_cast<const bf16_t* const*>(e.tables_dev.p),
                         e.chunks.bf(), static_cast<float*>(e.chunks_f32.p), L, B, d, s);
    }
    const float scale = 1.0f / std::sqrt(static_cast<float>(Dh));
    const bool mask_f32 = mask_dtype == BH_F32;
    const size_t mask_elem = mask_f32 ? 4 : 2;
    const float* chunks_f32 = static_cast<const float*>(e.chunks_f32.p);

    // Every per-row buffer is batch-major, so rows [b0, b0 + nb) of the batch are one contiguous
    // slice of each: a row group is the same launches on offset pointers with batch nb.
    struct Rows {
        int64_t b0, nb;
        hipStream_t s;
    };
    // The offset of a row group's V^T in e.vt_op (the op-level attention transposes V there when
    // the projections do not write V^T): each group gets its own rows, so the two groups of the
    // split schedule never write the same V^T on their two streams.
    auto vt_op_offset = [&](const Rows& g, int64_t kv_len) {
        return g.b0 * H * 72 * flash72_vt_ld(kv_len);
    };
    // LayerNorm + modulation of x into `modded` with chunk pair (shift c, scale c + 1). The norm
    // also reads the weights of the GEMM after it once (QKV after norm 1, ff0 after norm 2), so
    // that GEMM finds them in the memory-side cache instead of meeting each weight panel cold in
    // HBM. (Warming the other GEMMs' weights too -- the projections around the attentions from
    // norm 1, ff2 from norm 2 -- measured slower.)
    auto norm = [&](int64_t l, int c, const Rows& g) {
        const int64_t o = g.b0 * N * d;
        ProfileScope ps(K_NORM, g.s, 4.0 * g.nb * N * d);
        if (chunks_f32) {
            const float* chf = chunks_f32 + (l * 6 + c) * B * d + g.b0 * d;
            const void* warm = c == 0 ? static_cast<const void*>(e.qkv_w[l]) : e.blocks[l].ff0_w;
            const int64_t warm_bytes = (c == 0 ? 3 * d : e.dff) * d * 2;
            launch_norm_modulate_f32(e.x.bf() + o, chf, chf + B * d, e.modded.bf() + o, g.nb, N, d, eps,
                                     g.s, warm, warm_bytes);
        } else {
            const bf16_t* ch = e.chunks.bf() + (l * 6 + c) * B * d + g.b0 * d;
            launch_norm_modulate_pre(e.x.bf() + o, ch, ch + B * d, e.modded.bf() + o, g.nb, N, d, eps,
                                     g.s);
        }
    };
    // 1a. norm, then Q and K into the [M, qkv_ld] buffer; at head_dim 72, V straight into V^T
    // for the attention kernel and the buffer is [M, 2d] (other widths keep V in a [M, 3d]
    // buffer for the generic attention)
    const int64_t qkv_ld = e.qkv_ld;
    auto qkv = [&](int64_t l, const Rows& g) {
        norm(l, 0, g);
        SubclassScope sc(K_GEMM_QKV);
        GemmEpilogue ep;
        ep.ld_out = qkv_ld;
        if (e.vt72) {
            ep.vt = e.vt_self.bf() + g.b0 * H * Dh * e.vt_ld_self;
            ep.vt_period = 3 * d;
            ep.vt_col0 = 2 * d;
            ep.vt_seq = N;
            ep.vt_ld = e.vt_ld_self;
            ep.vt_heads = static_cast<int>(H);
            ep.vt_dim = static_cast<int>(Dh);
        }
        gemm(e, e.modded.bf() + g.b0 * N * d, e.qkv_w[l], e.qkv_b[l],
             e.qkv.bf() + g.b0 * N * qkv_ld, g.nb * N, 3 * d, d, ep, g.s, g.b0 * N, M);
    };
    // 1b. self-attention into ctx
    auto self_attention = [&](const Rows& g) {
        const bf16_t* q = e.qkv.bf() + g.b0 * N * qkv_ld;
        bf16_t* ctx = e.ctx.bf() + g.b0 * N * d;
        const Flash72Plan& sp = e.plan_self;
        float* part = attn_part(e, sp, g.b0, g.nb, N);
        const int64_t pf = flash72_plan_floats(g.nb, H, N, sp);
        if (e.vt72) {
            launch_flash72(q, qkv_ld, q + d, qkv_ld, e.vt_self.bf() + g.b0 * H * Dh * e.vt_ld_self,
                           e.vt_ld_self, ctx, d, g.nb, H, N, N, scale, nullptr, false, g.s, sp.splits,
                           part, pf, sp.qb0);
        } else {
            const int64_t vo = vt_op_offset(g, N);
            launch_attention_bf16(q, q + d, q + 2 * d, ctx, AttnShape{g.nb, H, N, N, Dh, 3 * d, 3 * d, d, scale},
                                  nullptr, false, g.s, nullptr, e.vt_op.bf() + vo, e.vt_op_elems - vo,
                                  sp.splits, part, pf, sp.qb0);
        }
    };
    // 1c-3. the gated out-projection, the cross-attention block and the feed-forward block
    auto rest = [&](int64_t l, const Rows& g) {
        const bh_dit_block_weights& bw = e.blocks[l];
        const int64_t rows = g.nb * N, o = g.b0 * N * d;
        bf16_t* x = e.x.bf() + o;
        bf16_t* ctx = e.ctx.bf() + o;
        const bf16_t* ch = e.chunks.bf() + l * 6 * B * d + g.b0 * d;   // [6][B][d], this group's rows
        {
            GemmEpilogue ep;
            ep.round_mid = true;
            ep.residual = x;
            ep.gate = ch + 2 * B * d;
            ep.gate_rows = N;
            gemm(e, ctx, bw.attn1_o_w, bw.attn1_o_b, x, rows, d, d, ep, g.s, g.b0 * N, M);
        }
        // 2. cross-attention (no norm before it: pixart_dit.cpp:251-253)
        const bf16_t* kv = e.kv_all.bf() + g.b0 * e.cap_len * L * 2 * d + l * 2 * d;
        const void* m = static_cast<const char*>(mask) + g.b0 * e.cap_len * mask_elem;
        const Flash72Plan& sp = e.plan_cross;
        float* part = attn_part(e, sp, g.b0, g.nb, N);
        const int64_t pf = flash72_plan_floats(g.nb, H, N, sp);
        if (e.cross_fused && g.nb >= e.cross_fused_min_rows) {
            // the Q projection and the attention in one launch, bit-identical with the two below
            launch_cross_fused(x, static_cast<const bf16_t*>(bw.attn2_q_w),
                               static_cast<const bf16_t*>(bw.attn2_q_b), g.nb, N, H, kv, L * 2 * d,
                               e.vt_cross.bf() + (l * B + g.b0) * H * Dh * e.vt_ld_cross, e.vt_ld_cross,
                               e.cap_len, m, mask_f32, ctx, d, scale, g.s);
        } else {
            bf16_t* q2 = e.q2.bf() + o;
            gemm(e, x, bw.attn2_q_w, bw.attn2_q_b, q2, rows, d, d, plain, g.s, g.b0 * N, M);
            if (e.vt72) {
                launch_flash72(q2, d, kv, L * 2 * d,
                               e.vt_cross.bf() + (l * B + g.b0) * H * Dh * e.vt_ld_cross, e.vt_ld_cross,
                               ctx, d, g.nb, H, N, e.cap_len, scale, m, mask_f32, g.s, sp.splits, part,
                               pf, sp.qb0);
            } else {
                const int64_t vo = vt_op_offset(g, e.cap_len);
                launch_attention_bf16(q2, kv, kv + d, ctx,
                                      AttnShape{g.nb, H, N, e.cap_len, Dh, d, L * 2 * d, d, scale}, m,
                                      mask_f32, g.s, nullptr, e.vt_op.bf() + vo, e.vt_op_elems - vo,
                                      sp.splits, part, pf, sp.qb0);
            }
        }
        {
            GemmEpilogue ep;
            ep.round_mid = true;
            ep.residual = x;
            gemm(e, ctx, bw.attn2_o_w, bw.attn2_o_b, x, rows, d, d, ep, g.s, g.b0 * N, M);
        }
        // 3. feed-forward
        norm(l, 3, g);
        bf16_t* ff0 = e.ff0.bf() + g.b0 * N * e.dff;
        {
            SubclassScope sc(K_GEMM_FF0);
            GemmEpilogue gelu;
            gelu.act = 1;
            gemm(e, e.modded.bf() + o, bw.ff0_w, bw.ff0_b, ff0, rows, e.dff, d, gelu, g.s, g.b0 * N, M);
        }
        {
            SubclassScope sc(K_GEMM_FF2);
            GemmEpilogue ep;
            ep.round_mid = true;
            ep.residual = x;
            ep.gate = ch + 5 * B * d;
            ep.gate_rows = N;
            gemm(e, ff0, bw.ff2_w, bw.ff2_b, x, rows, d, e.dff, ep, g.s, g.b0 * N, M);
        }
    };

    auto blocks = [&](const Rows& g) {
        for (int64_t l = 0; l < L; ++l) {
            qkv(l, g);
            self_attention(g);
            rest(l, g);
        }
    };
    if (B < 2 || e.row_split == BH_DIT_ROWS_JOINED) {
        blocks(Rows{0, B, s});
    } else {
        // The second group waits for everything before the block loop (on s); s waits for the
        // second group's last launch before the output head.
        hip_check(hipEventRecord(e.fork_ev, s), "hipEventRecord");
        hip_check(hipStreamWaitEvent(e.s2, e.fork_ev, 0), "hipStreamWaitEvent");
        blocks(Rows{0, (B + 1) / 2, s});
        blocks(Rows{(B + 1) / 2, B / 2, e.s2});
        hip_check(hipEventRecord(e.join_ev, e.s2), "hipEventRecord");
        hip_check(hipStreamWaitEvent(s, e.join_ev, 0), "hipStreamWaitEvent");
    }

    // output head: shift = emb_t + table[0], scale = emb_t + table[1] (pixart_dit.cpp:287-294)
    {
        ProfileScope ps(K_ELEMENTWISE, s, 6.0 * B * d);
        launch_chunk(e.emb_t.p, e.w.out_table, e.shift.p, B, d, 1, 0, 0, false, s);
        launch_chunk(e.emb_t.p, e.w.out_table, e.scale.p, B, d, 1, 0, 1, false, s);
    }
    {
        ProfileScope ps(K_NORM, s, 4.0 * M * d);
        launch_norm_modulate_pre(e.x.bf(), e.shift.bf(), e.scale.bf(), e.modded.bf(), B, N, d, eps, s);
    }
    gemm(e, e.modded.bf(), e.w.proj_out_w, e.w.proj_out_b, e.tokens.bf(), M, e.patch_out, d, plain, s);
    {
        ProfileScope ps(K_ELEMENTWISE, s, 4.0 * M * e.patch_out);
        launch_patch(e.tokens.p, out, B, c.out_channels, e.grid, P, true, false, s);
    }
}

}  // namespace

extern "C" {

int bh_dit_create(const bh_dit_config* cfg, const bh_dit_weights* w, int64_t batch,
                  int64_t latent_hw, int64_t caption_len, int mode, bh_dit** out) {
    return guarded([&] {
        require(cfg && w && out, "dit_create: null argument");
        *out = nullptr;
        const bh_dit_config& c = *cfg;
        require(c.num_layers > 0 && c.num_heads > 0 && c.head_dim > 0 && c.patch_size > 0 &&
                    c.in_channels > 0 && c.out_channels > 0 && c.caption_channels > 0 &&
                    c.sample_size > 0,
                "dit_create: every config field must be positive");
        require(batch > 0 && caption_len > 0, "dit_create: batch and caption_len must be positive");
        require(latent_hw > 0 && latent_hw % c.patch_size == 0,
                "dit_create: latent size " + std::to_string(latent_hw) +
                    " is not divisible by the patch size");
        require(mode == BH_DIT_FUSED || mode == BH_DIT_OPWISE, "dit_create: unknown mode");
        check_weights(c, *w);

        auto e = std::make_unique<bh_dit>();
        e->cfg = c;
        e->w = *w;
        e->blocks.assign(w->blocks, w->blocks + c.num_layers);
        e->w.blocks = nullptr;
        e->mode = mode;
        e->B = batch;
        e->latent = latent_hw;
        e->cap_len = caption_len;
        e->grid = latent_hw / c.patch_size;
        e->N = e->grid * e->grid;
        e->M = batch * e->N;
        e->Mcap = batch * caption_len;
        e->d = static_cast<int64_t>(c.num_heads) * c.head_dim;
        e->dff = static_cast<int64_t>(static_cast<double>(e->d) * c.mlp_ratio);
        e->patch_in = static_cast<int64_t>(c.in_channels) * c.patch_size * c.patch_size;
        e->patch_out = static_cast<int64_t>(c.out_channels) * c.patch_size * c.patch_size;
        const int64_t M = e->M, d = e->d, L = c.num_layers, B = batch;

        // position table: fp64 on the host, stored as bf16 once (pixart_dit.cpp:88-105)
        {
            const int base = c.sample_size / c.patch_size;
            const std::vector<double> pe =
                position_table(static_cast<int>(d), static_cast<int>(e->grid), base, 2.0);
            std::vector<bf16_t> host(pe.size());
            for (size_t i = 0; i < pe.size(); ++i) host[i] = f2bf(static_cast<float>(pe[i]));
            e->pos_table = e->make(static_cast<int64_t>(host.size()));
            hip_check(hipMemcpy(e->pos_table.p, host.data(), host.size() * 2, hipMemcpyHostToDevice),
                      "hipMemcpy");
        }
        e->patches = e->make(M * e->patch_in);
        e->x = e->make(M * d);
        e->modded = e->make(M * d);
        e->ctx = e->make(M * d);
        e->ff0 = e->make(M * e->dff);
        e->temb = e->make(B * 256);
        e->h_t = e->make(B * d);
        e->emb_t = e->make(B * d);
        e->silu_t = e->make(B * d);
        e->modulation = e->make(B * 6 * d);
        e->cap_h = e->make(e->Mcap * d);
        e->cap = e->make(e->Mcap * d);
        e->shift = e->make(B * d);
        e->scale = e->make(B * d);
        e->tokens = e->make(M * e->patch_out);
        if (mode == BH_DIT_OPWISE) {
            e->normed = e->make(M * d);
            e->q = e->make(M * d);
            e->k = e->make(M * d);
            e->v = e->make(M * d);
            e->proj = e->make(M * d);
            e->kc = e->make(e->Mcap * d);
            e->vc = e->make(e->Mcap * d);
            e->gate = e->make(B * d);
            e->zero = e->make(B * d);
        } else {
            // the QKV projection's output rows; V goes to V^T instead at head_dim 72 (below)
            e->vt72 = c.head_dim == 72 && e->N <= 16384 && caption_len <= 16384 && d % 144 == 0;
            e->qkv_ld = e->vt72 ? 2 * d : 3 * d;
            e->qkv = e->make(M * e->qkv_ld);
            e->q2 = e->make(M * d);
            e->kv_all = e->make(e->Mcap * L * 2 * d);
            e->chunks = e->make(L * 6 * B * d);
            if (norm_modulate_f32_supported(d)) e->chunks_f32 = e->make_f32(L * 6 * B * d);
            // the head_dim-72 attention reads V transposed, written by the projections' epilogue
            if (e->vt72) {
                for (int64_t nb = 1; nb <= B && !e->cross_fused; ++nb) {
                    if (cross_fused_supported(nb, e->N, c.num_heads, c.head_dim, caption_len)) {
                        e->cross_fused = true;
                        e->cross_fused_min_rows = nb;
                    }
                }
                e->vt_ld_self = flash72_vt_ld(e->N);
                e->vt_ld_cross = flash72_vt_ld(caption_len);
                e->vt_self = e->make(B * c.num_heads * 72 * e->vt_ld_self);
                e->vt_cross = e->make(L * B * c.num_heads * 72 * e->vt_ld_cross);
            } else if (c.head_dim == 72) {
                // The attention transposes V itself; it does so into this buffer, which the
                // engine owns, so a captured forward never holds a pointer another call frees.
                e->vt_op_elems = B * c.num_heads * 72 * flash72_vt_ld(std::max(e->N, caption_len));
                e->vt_op = e->make(e->vt_op_elems);
            }
            const size_t wb = static_cast<size_t>(d * d) * 2, bb = static_cast<size_t>(d) * 2;
            auto at = [](const void* base, size_t bytes) {
                return static_cast<const void*>(static_cast<const char*>(base) + bytes);
            };
            // packed in place: Q, K, V of one layer back to back (weights and biases) ...
            bool qkv_packed = true;
            for (int64_t l = 0; l < L; ++l) {
                const bh_dit_block_weights& bw = e->blocks[l];
                qkv_packed = qkv_packed && bw.attn1_k_w == at(bw.attn1_q_w, wb) &&
                             bw.attn1_v_w == at(bw.attn1_q_w, 2 * wb) && bw.attn1_k_b == at(bw.attn1_q_b, bb) &&
                             bw.attn1_v_b == at(bw.attn1_q_b, 2 * bb);
            }
            // ... and every layer's caption K, V back to back in layer order
            bool kv_packed = true;
            for (int64_t l = 0; l < L; ++l) {
                const bh_dit_block_weights& bw = e->blocks[l];
                const bh_dit_block_weights& b0 = e->blocks[0];
                kv_packed = kv_packed && bw.attn2_k_w == at(b0.attn2_k_w, 2 * l * wb) &&
                            bw.attn2_v_w == at(b0.attn2_k_w, (2 * l + 1) * wb) &&
                            bw.attn2_k_b == at(b0.attn2_k_b, 2 * l * bb) &&
                            bw.attn2_v_b == at(b0.attn2_k_b, (2 * l + 1) * bb);
            }
            if (!qkv_packed) {
                e->w_qkv = e->make(L * 3 * d * d);
                e->b_qkv = e->make(L * 3 * d);
            }
            if (!kv_packed) {
                e->w_kv = e->make(L * 2 * d * d);
                e->b_kv = e->make(L * 2 * d);
            }
            e->qkv_w.resize(L);
            e->qkv_b.resize(L);
            std::vector<const bf16_t*> tables(L);
            for (int64_t l = 0; l < L; ++l) {
                const bh_dit_block_weights& bw = e->blocks[l];
                if (qkv_packed) {
                    e->qkv_w[l] = static_cast<const bf16_t*>(bw.attn1_q_w);
                    e->qkv_b[l] = static_cast<const bf16_t*>(bw.attn1_q_b);
                } else {
                    char* wq = static_cast<char*>(e->w_qkv.p) + l * 3 * wb;
                    char* bq = static_cast<char*>(e->b_qkv.p) + l * 3 * bb;
                    d2d(wq, bw.attn1_q_w, wb, nullptr);
                    d2d(wq + wb, bw.attn1_k_w, wb, nullptr);
                    d2d(wq + 2 * wb, bw.attn1_v_w, wb, nullptr);
                    d2d(bq, bw.attn1_q_b, bb, nullptr);
                    d2d(bq + bb, bw.attn1_k_b, bb, nullptr);
                    d2d(bq + 2 * bb, bw.attn1_v_b, bb, nullptr);
                    e->qkv_w[l] = reinterpret_cast<const bf16_t*>(wq);
                    e->qkv_b[l] = reinterpret_cast<const bf16_t*>(bq);
                }
                if (!kv_packed) {
                    char* wk = static_cast<char*>(e->w_kv.p) + l * 2 * wb;
                    char* bk = static_cast<char*>(e->b_kv.p) + l * 2 * bb;
                    d2d(wk, bw.attn2_k_w, wb, nullptr);
                    d2d(wk + wb, bw.attn2_v_w, wb, nullptr);
                    d2d(bk, bw.attn2_k_b, bb, nullptr);
                    d2d(bk + bb, bw.attn2_v_b, bb, nullptr);
                }
                tables[l] = static_cast<const bf16_t*>(bw.scale_shift_table);
            }
            e->kv_w = kv_packed ? static_cast<const bf16_t*>(e->blocks[0].attn2_k_w) : e->w_kv.bf();
            e->kv_b = kv_packed ? static_cast<const bf16_t*>(e->blocks[0].attn2_k_b) : e->b_kv.bf();
            e->tables_dev = DevBuf(sizeof(void*) * L);
            e->workspace += static_cast<int64_t>(sizeof(void*) * L);
            hip_check(hipMemcpy(e->tables_dev.p, tables.data(), sizeof(void*) * L,
                                hipMemcpyHostToDevice),
                      "hipMemcpy");
            {   // the largest split-K partial set of any GEMM of the fused plan (full batch)
                GemmEpilogue plain, vt_ep;
                vt_ep.vt = e->vt72 ? e->vt_self.bf() : nullptr;
                const int64_t Mcap = e->Mcap, dff = e->dff;
                const int64_t shapes[][4] = {{Mcap, d, c.caption_channels, 0}, {Mcap, d, d, 0},
                                             {Mcap, L * 2 * d, d, 1}, {M, 3 * d, d, 1}, {M, d, d, 0},
                                             {M, dff, d, 0}, {M, d, dff, 0}, {M, e->patch_out, d, 0}};
                for (const auto& sh : shapes) {
                    const int sp = gemm_splits(sh[0], sh[1], sh[2], sh[3] ? vt_ep : plain);
                    if (sp > 1) e->splitk_floats = std::max(e->splitk_floats, sp * sh[0] * sh[1]);
                }
                if (e->splitk_floats > 0) e->splitk = e->make_f32(e->splitk_floats);
            }
            if (c.head_dim == 72) {   // key splits of the attentions, decided on the full batch
                const int64_t H = c.num_heads;
                e->plan_self = flash72_plan(B, H, e->N, e->N);
                e->plan_cross = flash72_plan(B, H, e->N, caption_len);
                const int64_t floats = std::max(flash72_plan_floats(B, H, e->N, e->plan_self),
                                                flash72_plan_floats(B, H, e->N, e->plan_cross));
                if (floats > 0) e->attn_part = e->make_f32(floats);
            }
            if (batch >= 2) {   // the row-split schedule's second stream (default priority)
                hip_check(hipStreamCreateWithFlags(&e->s2, hipStreamNonBlocking), "hipStreamCreate");
                hip_check(hipEventCreateWithFlags(&e->fork_ev, hipEventDisableTiming), "hipEventCreate");
                hip_check(hipEventCreateWithFlags(&e->join_ev, hipEventDisableTiming), "hipEventCreate");
            }
        }
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        *out = e.release();
    });
}

int bh_dit_forward(bh_dit* e, const void* latent, double timestep, const void* caption,
                   const void* caption_mask, int mask_dtype, void* out, void* stream) {
    return guarded([&] {
        require(e != nullptr, "dit_forward: null engine");
        require_device_ptr(latent, "dit_forward", "latent");
        require_device_ptr(caption, "dit_forward", "caption");
        require_device_ptr(caption_mask, "dit_forward", "caption_mask");
        require_device_ptr(out, "dit_forward", "out");
        dit_forward_step(e, latent, timestep, caption, caption_mask, mask_dtype, out,
                         static_cast<hipStream_t>(stream), false);
    });
}

}  // extern "C"

void bh::dit_forward_step(bh_dit* e, const void* latent, double timestep, const void* caption,
                          const void* caption_mask, int mask_dtype, void* out, hipStream_t s,
                          bool caption_ready) {
    require(e != nullptr, "dit_forward: null engine");
    require(latent && caption && caption_mask && out, "dit_forward: null tensor pointer");
    require(mask_dtype == BH_F32 || mask_dtype == BH_BF16, "dit_forward: mask dtype");
    if (e->mode == BH_DIT_OPWISE) {
        forward_opwise(*e, latent, timestep, caption, caption_mask, mask_dtype, out, s);
    } else {
        forward_fused(*e, latent, timestep, caption, caption_mask, mask_dtype, out, s,
                      caption_ready);
    }
}

extern "C" {

int64_t bh_dit_workspace_bytes(const bh_dit* e) { return e ? e->workspace : 0; }

int bh_dit_position_table(const bh_dit* e, void* out, void* stream) {
    return guarded([&] {
        require(e != nullptr, "dit_position_table: null engine");
        require_device_ptr(out, "dit_position_table", "out");
        d2d(out, e->pos_table.p, e->pos_table.bytes, static_cast<hipStream_t>(stream));
    });
}

int bh_dit_set_rows(bh_dit* e, int rows) {
    return guarded([&] {
        require(e != nullptr, "dit_set_rows: null engine");
        require(rows == BH_DIT_ROWS_JOINED || rows == BH_DIT_ROWS_SPLIT,
                "dit_set_rows: unknown row schedule " + std::to_string(rows));
        require(rows == BH_DIT_ROWS_JOINED || e->mode == BH_DIT_FUSED,
                "dit_set_rows: the op-by-op plan runs the reference graph on the caller's stream only");
        e->row_split = rows;
    });
}

void bh_dit_destroy(bh_dit* e) { delete e; }

}  // extern "C"
