// The VAE decoder engine (the vae-decode stage): VaeDecoder::forward (vae_decoder.cpp:127-180) on
// one MI355X, channels-last.
//
// The reference runs the decoder NCHW and transposes around the mid-block attention. Here the
// activation between ops is [pixels, channels] bf16 (NHWC, batch 1), chosen for gfx950:
//   - a 3x3 convolution is an implicit GEMM on the MFMA tile kernel (gemm.hip): a k-tile is one
//     tap x 64 input channels, i.e. 128 contiguous bytes of one neighbouring pixel;
//   - the upsampler's nearest 2x upsample is folded into that gather (the conv reads pixel
//     (y/2, x/2)), so the 4x-larger upsampled tensor is never written (at 1024px it would be
//     0.5 GB written and read back);
//   - the resnet's "skip + conv2" is the residual epilogue of conv2, and the shortcut 1x1 conv
//     is a plain GEMM;
//   - the mid-block attention reads its tokens in place: the reference's two transposes vanish.
// Only the latent (4 channels) and the image (3 channels) change layout, at the two ends.
//
// Rounding follows the reference's graph: every op's output is stored in bf16, including
// conv2 before its residual add (round_mid) and the GroupNorm output before its SiLU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/burnisher_hip.h"
#include "common.h"

using bh::bf16_t;

struct bh_vae {
    bh_vae_config cfg{};
    int64_t h0 = 0;                                   // latent side
    std::map<std::string, const bf16_t*> w;            // the caller's tensors, by name
    std::map<std::string, bf16_t*> rw;                 // 3x3 weights repacked [co][ky][kx][ci]
    std::vector<void*> allocs;
    bf16_t* buf[4] = {nullptr, nullptr, nullptr, nullptr};
    int64_t buf_elems = 0;
    bf16_t *q = nullptr, *k = nullptr, *v = nullptr, *vt = nullptr, *o = nullptr;
    bf16_t* zero = nullptr;
    bf16_t* conv_out_bias = nullptr;   // decoder.conv_out.bias padded to 8 outputs
    bh::GroupNormScratch gn;
    int64_t bytes = 0;

    ~bh_vae() {
        for (void* p : allocs) (void)hipFree(p);
    }
    void* alloc(int64_t n) {
        void* p = nullptr;
        bh::hip_check(hipMalloc(&p, static_cast<size_t>(std::max<int64_t>(n, 256))), "hipMalloc (vae)");
        allocs.push_back(p);
        bh::hip_check(hipMemset(p, 0, static_cast<size_t>(std::max<int64_t>(n, 256))), "hipMemset (vae)");
        bytes += n;
        return p;
    }
    const bf16_t* at(const std::string& n) const {
        auto it = w.find(n);
        if (it == w.end())
            throw bh::Error("vae: weight '" + n + "' is missing. A decoder run with a missing weight "
                            "would produce a plausible image from wrong numbers");
        return it->second;
    }
};

namespace bh {
namespace {

struct Plan {
    std::vector<int64_t> rev;   // up-block channels, reversed block_out_channels
};

Plan plan_of(const bh_vae_config& c) {
    Plan p;
    for (int i = c.num_blocks - 1; i >= 0; --i) p.rev.push_back(c.block_out_channels[i]);
    return p;
}

bool mfma_conv(int64_t ci, int64_t co) { return ci % 64 == 0 && co % 8 == 0; }

}  // namespace

// Every tensor the decoder reads with its checkpoint shape (the VAE part of declare_pixart_shapes,
// weights.cpp:284-320): convolutions [out, in, k, k], projections [out, in], norms [channels].
std::vector<std::pair<std::string, std::vector<int64_t>>> vae_tensor_shapes(const bh_vae_config& c) {
    std::vector<std::pair<std::string, std::vector<int64_t>>> out;
    const Plan p = plan_of(c);
    auto conv = [&](const std::string& n, int64_t ci, int64_t co, int64_t k) {
        out.push_back({n + ".weight", {co, ci, k, k}});
        out.push_back({n + ".bias", {co}});
    };
    auto norm = [&](const std::string& n, int64_t ch) {
        out.push_back({n + ".weight", {ch}});
        out.push_back({n + ".bias", {ch}});
    };
    auto res = [&](const std::string& n, int64_t ci, int64_t co) {
        norm(n + ".norm1", ci);
        conv(n + ".conv1", ci, co, 3);
        norm(n + ".norm2", co);
        conv(n + ".conv2", co, co, 3);
        if (ci != co) conv(n + ".conv_shortcut", ci, co, 1);
    };
    const int64_t zc = c.latent_channels, r0 = p.rev[0];
    conv("post_quant_conv", zc, zc, 1);
    conv("decoder.conv_in", zc, r0, 3);
    res("decoder.mid_block.resnets.0", r0, r0);
    res("decoder.mid_block.resnets.1", r0, r0);
    norm("decoder.mid_block.attentions.0.group_norm", r0);
    for (const char* part : {".to_q", ".to_k", ".to_v", ".to_out.0"}) {
        const std::string n = std::string("decoder.mid_block.attentions.0") + part;
        out.push_back({n + ".weight", {r0, r0}});
        out.push_back({n + ".bias", {r0}});
    }
    int64_t prev = r0;
    for (size_t i = 0; i < p.rev.size(); ++i) {
        for (int j = 0; j <= c.layers_per_block; ++j)
            res("decoder.up_blocks." + std::to_string(i) + ".resnets." + std::to_string(j),
                j == 0 ? prev : p.rev[i], p.rev[i]);
        prev = p.rev[i];
        if (i + 1 != p.rev.size())
            conv("decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv", p.rev[i], p.rev[i], 3);
    }
    norm("decoder.conv_norm_out", prev);
    conv("decoder.conv_out", prev, 3, 3);
    return out;
}

namespace {

// One decode, everything on stream s.
struct Run {
    bh_vae& e;
    hipStream_t s;
    int free_mask = 0xF;   // which of e.buf are free

    bf16_t* take() {
        for (int i = 0; i < 4; ++i)
            if (free_mask & (1 << i)) {
                free_mask &= ~(1 << i);
                return e.buf[i];
            }
        throw Error("vae: activation buffers exhausted");
    }
    void give(const bf16_t* p) {
        for (int i = 0; i < 4; ++i)
            if (e.buf[i] == p) free_mask |= 1 << i;
    }

    void gn(const bf16_t* x, bf16_t* out, const std::string& n, int64_t ch, int64_t h, bool silu) {
        launch_group_norm_nhwc(x, out, h * h, ch, e.cfg.norm_num_groups, static_cast<float>(e.cfg.eps),
                               e.at(n + ".weight"), e.at(n + ".bias"), silu, e.gn, s);
    }

    // 3x3 "same" conv of x (h_in x h_in, ci) to out (h x h, co); up: h = 2 h_in, nearest.
    void conv3(const bf16_t* x, bf16_t* out, const std::string& n, int64_t ci, int64_t co, int64_t h,
               bool up, const bf16_t* residual) {
        const int64_t hin = up ? h / 2 : h;
        if (mfma_conv(ci, co)) {
            ConvGeom g;
            g.in = x;
            g.zero = e.zero;
            g.H = g.W = static_cast<int>(h);
            g.in_h = g.in_w = static_cast<int>(hin);
            g.c_in = static_cast<int>(ci);
            g.up = up ? 1 : 0;
            GemmEpilogue ep;
            ep.residual = residual;
            ep.round_mid = residual != nullptr;
            launch_conv3x3_bf16(g, e.rw.at(n + ".weight"), e.at(n + ".bias"), out, co, ep, s);
            return;
        }
        require(!up && !residual, "vae: a thin convolution cannot be an upsampler or carry a residual");
        launch_conv_direct_nhwc(x, e.at(n + ".weight"), e.at(n + ".bias"), out, h, h, ci, co, 3, 1, s);
    }

    // out = x . W^T + bias over [h*h, ci] (a 1x1 conv or a linear layer), optionally + residual
    // with the product rounded first.
    void linear(const bf16_t* x, bf16_t* out, const std::string& n, int64_t rows, int64_t ci, int64_t co,
                const bf16_t* residual) {
        GemmEpilogue ep;
        ep.residual = residual;
        ep.round_mid = residual != nullptr;
        launch_gemm_bf16(x, e.at(n + ".weight"), e.at(n + ".bias"), out, rows, co, ci, ep, s);
    }

    // ResnetBlock2D (vae_decoder.cpp:64-80): returns the output buffer; x is released.
    bf16_t* resnet(bf16_t* x, const std::string& n, int64_t ci, int64_t co, int64_t h) {
        bf16_t* t = take();
        gn(x, t, n + ".norm1", ci, h, true);                   // t = silu(norm1(x))
        bf16_t* c1 = take();
        conv3(t, c1, n + ".conv1", ci, co, h, false, nullptr);  // c1 = conv1(t)
        gn(c1, c1, n + ".norm2", co, h, true);                  // c1 = silu(norm2(c1))
        if (ci != co) {
            linear(x, t, n + ".conv_shortcut", h * h, ci, co, nullptr);   // t = shortcut(x)
            give(x);
            bf16_t* out = take();
            conv3(c1, out, n + ".conv2", co, co, h, false, t);  // out = t + conv2(c1)
            give(t);
            give(c1);
            return out;
        }
        conv3(c1, t, n + ".conv2", co, co, h, false, x);        // t = x + conv2(c1)
        give(x);
        give(c1);
        return t;
    }

    // Spatial self-attention of the mid-block (vae_decoder.cpp:85-118), tokens read in place.
    bf16_t* attention(bf16_t* x, const std::string& n, int64_t ch, int64_t h) {
        const int64_t S = h * h;
        bf16_t* normed = take();
        gn(x, normed, n + ".group_norm", ch, h, false);
        linear(normed, e.q, n + ".to_q", S, ch, ch, nullptr);
        linear(normed, e.k, n + ".to_k", S, ch, ch, nullptr);
        linear(normed, e.v, n + ".to_v", S, ch, ch, nullptr);
        give(normed);
        const float scale = 1.0f / std::sqrt(static_cast<float>(ch));
        if (ch == 512) {
            launch_attention512(e.q, e.k, e.v, e.vt, e.o, S, scale, s);
        } else {
            AttnShape sh{1, 1, S, S, ch, ch, ch, ch, scale};
            if (ch <= 128) launch_attention_bf16(e.q, e.k, e.v, e.o, sh, nullptr, false, s);
            else launch_attention_generic(e.q, e.k, e.v, e.o, sh, nullptr, nullptr, false, false, s);
        }
        bf16_t* out = take();
        linear(e.o, out, n + ".to_out.0", S, ch, ch, x);
        give(x);
        return out;
    }

    void decode(const bf16_t* latent, bf16_t* image) {
        const bh_vae_config& c = e.cfg;
        const Plan p = plan_of(c);
        const int64_t zc = c.latent_channels;
        int64_t h = e.h0;
        // latent NCHW -> NHWC, post_quant_conv (1x1), conv_in (3x3, 4 channels: direct)
        bf16_t* a = take();
        launch_transpose_bf16(latent, a, 1, zc, h * h, s);
        bf16_t* b = take();
        linear(a, b, "post_quant_conv", h * h, zc, zc, nullptr);
        // conv_in: the latent's channels zero-padded to one 64-channel k-tile, on the MFMA kernel
        // (the padded weights are zero there, so the sums are those of the thin convolution)
        launch_pad_rows(b, a, h * h, zc, 64, s);
        {
            ConvGeom g;
            g.in = a;
            g.zero = e.zero;
            g.H = g.W = g.in_h = g.in_w = static_cast<int>(h);
            g.c_in = 64;
            launch_conv3x3_bf16(g, e.rw.at("decoder.conv_in.weight"), e.at("decoder.conv_in.bias"), b,
                                p.rev[0], GemmEpilogue{}, s);
        }
        std::swap(a, b);
        give(b);
        bf16_t* x = a;
        x = resnet(x, "decoder.mid_block.resnets.0", p.rev[0], p.rev[0], h);
        x = attention(x, "decoder.mid_block.attentions.0", p.rev[0], h);
        x = resnet(x, "decoder.mid_block.resnets.1", p.rev[0], p.rev[0], h);
        int64_t prev = p.rev[0];
        for (size_t i = 0; i < p.rev.size(); ++i) {
            const int64_t co = p.rev[i];
            for (int j = 0; j <= c.layers_per_block; ++j)
                x = resnet(x, "decoder.up_blocks." + std::to_string(i) + ".resnets." + std::to_string(j),
                           j == 0 ? prev : co, co, h);
            prev = co;
            if (i + 1 != p.rev.size()) {
                // nearest 2x upsample folded into the upsampler conv's gather (vae_decoder.cpp:170-175)
                bf16_t* y = take();
                conv3(x, y, "decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv", co, co, 2 * h,
                      true, nullptr);
                give(x);
                x = y;
                h *= 2;
            }
        }
        gn(x, x, "decoder.conv_norm_out", prev, h, true);
        // conv_out: 3 outputs padded to 8 (zero weights and bias), on the MFMA kernel; the
        // transpose to NCHW keeps the first 3 channels
        bf16_t* y = take();
        {
            ConvGeom g;
            g.in = x;
            g.zero = e.zero;
            g.H = g.W = g.in_h = g.in_w = static_cast<int>(h);
            g.c_in = static_cast<int>(prev);
            launch_conv3x3_bf16(g, e.rw.at("decoder.conv_out.weight"), e.conv_out_bias, y, 8, GemmEpilogue{}, s);
        }
        launch_transpose_keep_bf16(y, image, h * h, 8, 3, s);
        give(x);
        give(y);
    }
};

}  // namespace
}  // namespace bh

extern "C" {

int bh_vae_create(const bh_vae_config* cfg, const bh_vae_weights* w, int64_t latent_hw, bh_vae** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "vae_create: null output handle");
        *out = nullptr;
        bh::require(cfg && w, "vae_create: null config or weights");
        bh::require(cfg->num_blocks >= 1 && cfg->num_blocks <= 8 && cfg->layers_per_block >= 0 &&
                        cfg->latent_channels > 0 && cfg->norm_num_groups > 0,
                    "vae_create: configuration out of range");
        bh::require(latent_hw > 0 && latent_hw <= 4096, "vae_create: latent side out of range");
        bh::require(w->count >= 0 && (w->count == 0 || (w->names && w->tensors)), "vae_create: bad weight table");
        auto e = std::make_unique<bh_vae>();
        e->cfg = *cfg;
        e->h0 = latent_hw;
        for (int i = 0; i < w->count; ++i) {
            bh::require(w->names[i] && w->tensors[i], "vae_create: null weight name or tensor");
            e->w[w->names[i]] = static_cast<const bf16_t*>(w->tensors[i]);
        }
        const bh::Plan p = bh::plan_of(*cfg);
        for (const auto& t : bh::vae_tensor_shapes(*cfg)) (void)e->at(t.first);   // all present
        for (int64_t ch : p.rev) {
            bh::require(ch > 0 && bh::gn_nhwc_supported(ch, cfg->norm_num_groups),
                        "vae_create: every block width must split into the groups in whole 8-channel "
                        "runs (width % 8 == 0, width / 8 dividing 256, groups dividing the width)");
        }
        for (size_t i = 0; i < p.rev.size(); ++i)
            bh::require(p.rev[i] % 64 == 0,
                        "vae_create: this decoder runs every resnet and upsampler convolution on the "
                        "MFMA implicit GEMM, which needs block widths that are multiples of 64");
        // activation buffers: the largest [pixels, channels] of any layer
        int64_t h = latent_hw, most = latent_hw * latent_hw * std::max<int64_t>(p.rev[0], cfg->latent_channels);
        for (size_t i = 0; i < p.rev.size(); ++i) {
            const int64_t prev = i == 0 ? p.rev[0] : p.rev[i - 1];
            most = std::max(most, h * h * std::max(prev, p.rev[i]));
            if (i + 1 != p.rev.size()) {
                h *= 2;
                most = std::max(most, h * h * p.rev[i]);
            }
        }
        most = std::max(most, h * h * 3);
        e->buf_elems = most;
        for (auto& b : e->buf) b = static_cast<bf16_t*>(e->alloc(most * 2));
        const int64_t S = latent_hw * latent_hw, ch = p.rev[0];
        e->q = static_cast<bf16_t*>(e->alloc(S * ch * 2));
        e->k = static_cast<bf16_t*>(e->alloc(S * ch * 2));
        e->v = static_cast<bf16_t*>(e->alloc(S * ch * 2));
        e->o = static_cast<bf16_t*>(e->alloc(S * ch * 2));
        e->vt = static_cast<bf16_t*>(e->alloc(ch * bh::vt512_ld(S) * 2));
        e->zero = static_cast<bf16_t*>(e->alloc(256));
        e->gn.max_chunks = 2048;
        e->gn.part = static_cast<double*>(e->alloc(e->gn.max_chunks * 64 * 8));
        e->gn.mean = static_cast<double*>(e->alloc(64 * 8));
        e->gn.inv = static_cast<float*>(e->alloc(64 * 4));
        // repack every 3x3 weight the MFMA conv reads
        auto repack = [&](const std::string& n, int64_t ci, int64_t co) {
            if (!bh::mfma_conv(ci, co) || e->rw.count(n + ".weight")) return;
            bf16_t* r = static_cast<bf16_t*>(e->alloc(co * ci * 9 * 2));
            bh::launch_repack3x3(e->at(n + ".weight"), r, co, ci, nullptr);
            e->rw[n + ".weight"] = r;
        };
        auto res = [&](const std::string& n, int64_t ci, int64_t co) {
            repack(n + ".conv1", ci, co);
            repack(n + ".conv2", co, co);
        };
        res("decoder.mid_block.resnets.0", p.rev[0], p.rev[0]);
        res("decoder.mid_block.resnets.1", p.rev[0], p.rev[0]);
        int64_t prev = p.rev[0];
        for (size_t i = 0; i < p.rev.size(); ++i) {
            for (int j = 0; j <= cfg->layers_per_block; ++j)
                res("decoder.up_blocks." + std::to_string(i) + ".resnets." + std::to_string(j),
                    j == 0 ? prev : p.rev[i], p.rev[i]);
            prev = p.rev[i];
            if (i + 1 != p.rev.size())
                repack("decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv", p.rev[i], p.rev[i]);
        }
        // conv_in (latent channels -> 64, zero-padded) and conv_out (-> 8 outputs, zero-padded)
        bh::require(cfg->latent_channels <= 64, "vae_create: more than 64 latent channels");
        {
            bf16_t* r = static_cast<bf16_t*>(e->alloc(p.rev[0] * 64 * 9 * 2));
            bh::launch_repack3x3_pad(e->at("decoder.conv_in.weight"), r, p.rev[0], cfg->latent_channels,
                                     p.rev[0], 64, nullptr);
            e->rw["decoder.conv_in.weight"] = r;
            bf16_t* ro = static_cast<bf16_t*>(e->alloc(8 * prev * 9 * 2));
            bh::launch_repack3x3_pad(e->at("decoder.conv_out.weight"), ro, 3, prev, 8, prev, nullptr);
            e->rw["decoder.conv_out.weight"] = ro;
            e->conv_out_bias = static_cast<bf16_t*>(e->alloc(16));   // zero-filled by alloc
            bh::hip_check(hipMemcpy(e->conv_out_bias, e->at("decoder.conv_out.bias"), 3 * 2,
                                    hipMemcpyDeviceToDevice), "hipMemcpy (conv_out bias)");
        }
        bh::hip_check(hipDeviceSynchronize(), "vae_create");
        *out = e.release();
    });
}

int bh_vae_decode(bh_vae* e, const void* latent, void* image, void* stream) {
    return bh::guarded([&] {
        bh::require(e != nullptr, "vae_decode: null engine");
        bh::require_device_ptr(latent, "vae_decode", "latent");
        bh::require_device_ptr(image, "vae_decode", "image");
        bh::Run r{*e, static_cast<hipStream_t>(stream)};
        r.decode(static_cast<const bf16_t*>(latent), static_cast<bf16_t*>(image));
    });
}

int64_t bh_vae_workspace_bytes(const bh_vae* e) { return e ? e->bytes : -1; }

// ---- the VAE's ops at the registry boundary (NCHW) ----------------------------------------

int bh_conv2d(const void* x, const void* weight, const void* bias, void* out, int64_t batch,
              int64_t c_in, int64_t h, int64_t w, int64_t c_out, int64_t k, int64_t pad, int dtype,
              void* stream) {
    return bh::guarded([&] {
        bh::require(batch >= 0 && c_in > 0 && h >= 0 && w >= 0 && c_out >= 0 && k > 0 && pad >= 0,
                    "conv2d: negative or zero size");
        bh::require(2 * pad == k - 1,
                    "conv2d (hip-gfx950): only stride-1 'same' convolutions (2 * pad == k - 1) have a kernel");
        bh::require(dtype == BH_BF16, "conv2d (hip-gfx950): bf16 only (fp32 has no kernel here)");
        if (batch == 0 || c_out == 0 || h == 0 || w == 0) return;
        const char* op = "conv2d (hip-gfx950)";
        bh::require_device_ptr(x, op, "x");
        bh::require_device_ptr(weight, op, "weight");
        bh::optional_device_ptr(bias, op, "bias");
        bh::require_device_ptr(out, op, "out");
        bh::launch_conv2d_nchw(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(weight),
                               static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(out), batch,
                               c_in, h, w, c_out, k, pad, static_cast<hipStream_t>(stream));
    });
}

int bh_upsample(const void* in, void* out, int64_t batch, int64_t channels, int64_t h, int64_t w,
                int64_t factor, int dtype, void* stream) {
    return bh::guarded([&] {
        bh::require(batch >= 0 && channels >= 0 && h >= 0 && w >= 0 && factor >= 1,
                    "upsample: negative size or factor below 1");
        bh::require(dtype == BH_BF16, "upsample (hip-gfx950): bf16 only");
        if (batch * channels * h * w == 0) return;
        bh::require_device_ptr(in, "upsample (hip-gfx950)", "in");
        bh::require_device_ptr(out, "upsample (hip-gfx950)", "out");
        bh::launch_upsample_nchw(static_cast<const bf16_t*>(in), static_cast<bf16_t*>(out),
                                 batch * channels, h, w, factor, static_cast<hipStream_t>(stream));
    });
}

int bh_transpose(const void* in, void* out, int64_t batch, int64_t channels, int64_t spatial,
                 int to_channels_first, int dtype, void* stream) {
    return bh::guarded([&] {
        bh::require(batch >= 0 && channels >= 0 && spatial >= 0, "transpose: negative size");
        bh::require(dtype == BH_BF16, "transpose (hip-gfx950): bf16 only");
        if (batch * channels * spatial == 0) return;
        bh::require_device_ptr(in, "transpose (hip-gfx950)", "in");
        bh::require_device_ptr(out, "transpose (hip-gfx950)", "out");
        if (to_channels_first)
            bh::launch_transpose_bf16(static_cast<const bf16_t*>(in), static_cast<bf16_t*>(out), batch,
                                      spatial, channels, static_cast<hipStream_t>(stream));
        else
            bh::launch_transpose_bf16(static_cast<const bf16_t*>(in), static_cast<bf16_t*>(out), batch,
                                      channels, spatial, static_cast<hipStream_t>(stream));
    });
}

void bh_vae_destroy(bh_vae* e) { delete e; }

}  // extern "C"
