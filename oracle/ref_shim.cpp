// oracle/ref_shim.cpp -- TEST INFRASTRUCTURE ONLY. A C entry layer over the REFERENCE runtime's
// own `stock` implementation, compiled together with the reference sources where they lie
// (/root/reference/src/...; see the `ref` target of oracle/Makefile) into
// oracle/_ref/libref_stock.so. It lets the tests pin the restatement in stock.cpp against the
// real reference at small shapes. Nothing here reimplements an op: every call goes through the
// reference's registry (`OpRegistry<Args>::instance().get("stock")`) or its model code.
#include <cstdint>
#include <cstring>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "burnisher/models.h"
#include "burnisher/ops.h"
#include "burnisher/scheduler.h"

#include "../include/burnisher_hip.h"

using namespace burnisher;

namespace {

thread_local std::string g_err;

DType dt_of(int dtype) { return dtype == BH_F32 ? DType::F32 : DType::BF16; }

Tensor view(const void* p, std::vector<int64_t> shape, int dtype) {
    return Tensor::view(const_cast<void*>(p), std::move(shape), dt_of(dtype));
}

template <typename Fn>
int guard(Fn fn) {
    try {
        static bool registered = false;
        if (!registered) {
            register_all_ops();
            registered = true;
        }
        fn();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

Epilogue epi_of(int e) {
    switch (e) {
        case BH_EPI_GELU: return Epilogue::Gelu;
        case BH_EPI_SILU: return Epilogue::Silu;
        case BH_EPI_GELU_GATED: return Epilogue::GeluGated;
        default: return Epilogue::None;
    }
}

// Serves the weight table the tests hand over, by checkpoint name, as bf16 views.
class TableWeights : public WeightSource {
  public:
    TableWeights(const bh_dit_config& c, const bh_dit_weights& w) {
        const int64_t d = static_cast<int64_t>(c.num_heads) * c.head_dim;
        const int64_t dff = static_cast<int64_t>(static_cast<double>(d) * c.mlp_ratio);
        const int64_t p = c.patch_size, p2 = p * p;
        put("pos_embed.proj.weight", w.pos_embed_w, {d, c.in_channels, p, p});
        put("pos_embed.proj.bias", w.pos_embed_b, {d});
        put("adaln_single.emb.timestep_embedder.linear_1.weight", w.t_emb1_w, {d, 256});
        put("adaln_single.emb.timestep_embedder.linear_1.bias", w.t_emb1_b, {d});
        put("adaln_single.emb.timestep_embedder.linear_2.weight", w.t_emb2_w, {d, d});
        put("adaln_single.emb.timestep_embedder.linear_2.bias", w.t_emb2_b, {d});
        put("adaln_single.linear.weight", w.adaln_w, {6 * d, d});
        put("adaln_single.linear.bias", w.adaln_b, {6 * d});
        put("caption_projection.linear_1.weight", w.cap1_w, {d, c.caption_channels});
        put("caption_projection.linear_1.bias", w.cap1_b, {d});
        put("caption_projection.linear_2.weight", w.cap2_w, {d, d});
        put("caption_projection.linear_2.bias", w.cap2_b, {d});
        put("scale_shift_table", w.out_table, {2, d});
        put("proj_out.weight", w.proj_out_w, {p2 * c.out_channels, d});
        put("proj_out.bias", w.proj_out_b, {p2 * c.out_channels});
        for (int i = 0; i < c.num_layers; ++i) {
            const bh_dit_block_weights& b = w.blocks[i];
            const std::string n = "transformer_blocks." + std::to_string(i) + ".";
            put(n + "scale_shift_table", b.scale_shift_table, {6, d});
            const void* ws[2][4][2] = {
                {{b.attn1_q_w, b.attn1_q_b}, {b.attn1_k_w, b.attn1_k_b},
                 {b.attn1_v_w, b.attn1_v_b}, {b.attn1_o_w, b.attn1_o_b}},
                {{b.attn2_q_w, b.attn2_q_b}, {b.attn2_k_w, b.attn2_k_b},
                 {b.attn2_v_w, b.attn2_v_b}, {b.attn2_o_w, b.attn2_o_b}}};
            const char* an[2] = {"attn1", "attn2"};
            const char* pn[4] = {"to_q", "to_k", "to_v", "to_out.0"};
            for (int a = 0; a < 2; ++a)
                for (int j = 0; j < 4; ++j) {
                    put(n + an[a] + "." + pn[j] + ".weight", ws[a][j][0], {d, d});
                    put(n + an[a] + "." + pn[j] + ".bias", ws[a][j][1], {d});
                }
            put(n + "ff.net.0.proj.weight", b.ff0_w, {dff, d});
            put(n + "ff.net.0.proj.bias", b.ff0_b, {dff});
            put(n + "ff.net.2.weight", b.ff2_w, {d, dff});
            put(n + "ff.net.2.bias", b.ff2_b, {d});
        }
    }
    bool has(const std::string& name) const override { return m_.count(name) != 0; }
    Tensor get(const std::string& name) const override { return m_.at(name); }

  private:
    void put(const std::string& name, const void* p, std::vector<int64_t> shape) {
        m_.emplace(name, view(p, std::move(shape), BH_BF16));
    }
    std::map<std::string, Tensor> m_;
};

// Serves a name-keyed table of bf16 tensors (the VAE's weights) with the shapes the reference
// itself declares for those names.
class NamedWeights : public WeightSource {
  public:
    explicit NamedWeights(const bh_vae_weights& w) : NamedWeights(w.count, w.names, w.tensors) {}
    NamedWeights(int count, const char* const* names, const void* const* tensors) {
        for (int i = 0; i < count; ++i) ptr_[names[i]] = tensors[i];
    }
    bool has(const std::string& name) const override { return ptr_.count(name) != 0; }
    Tensor get(const std::string& name) const override {
        auto it = ptr_.find(name);
        if (it == ptr_.end()) throw std::runtime_error("ref weights: no '" + name + "'");
        return view(it->second, shape_.at(name), BH_BF16);
    }
    void set_shape(const std::string& name, std::vector<int64_t> shape) { shape_[name] = std::move(shape); }

  private:
    std::map<std::string, const void*> ptr_;
    std::map<std::string, std::vector<int64_t>> shape_;
};

}  // namespace

extern "C" {

const char* ref_last_error(void) { return g_err.c_str(); }

int ref_gemm(const void* a, const void* b, const void* bias, void* out, int64_t m, int64_t n,
             int64_t k, int b_transposed, int epilogue, int dtype) {
    return guard([&] {
        Tensor ta = view(a, {m, k}, dtype);
        Tensor tb = view(b, b_transposed ? std::vector<int64_t>{n, k} : std::vector<int64_t>{k, n}, dtype);
        Tensor tbias = bias ? view(bias, {n}, dtype) : Tensor();
        Tensor to = view(out, {m, n}, dtype);
        GemmArgs g{&ta, &tb, bias ? &tbias : nullptr, &to, m, n, k, b_transposed != 0,
                   epi_of(epilogue)};
        GemmRegistry::instance().get("stock")(g);
    });
}

int ref_attention(const void* q, const void* k, const void* v, void* out, int64_t batch,
                  int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                  const void* bias, const void* key_mask, int mask_dtype, int dtype,
                  int materialized) {
    return guard([&] {
        Tensor tq = view(q, {batch, q_len, heads, head_dim}, dtype);
        Tensor tk = view(k, {batch, kv_len, heads, head_dim}, dtype);
        Tensor tv = view(v, {batch, kv_len, heads, head_dim}, dtype);
        Tensor to = view(out, {batch, q_len, heads, head_dim}, dtype);
        Tensor tb = bias ? view(bias, {heads, q_len, kv_len}, dtype) : Tensor();
        Tensor tm = key_mask ? view(key_mask, {batch, kv_len}, mask_dtype) : Tensor();
        AttentionArgs args{&tq, &tk, &tv, &to, batch, heads, q_len, kv_len, head_dim, scale,
                           bias ? &tb : nullptr, key_mask ? &tm : nullptr};
        AttentionRegistry::instance().get(materialized ? "materialized" : "stock")(args);
    });
}

int ref_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
             int64_t cols, float eps, int rms, int dtype) {
    return guard([&] {
        Tensor tx = view(x, {rows, cols}, dtype), to = view(out, {rows, cols}, dtype);
        Tensor tw = weight ? view(weight, {cols}, dtype) : Tensor();
        Tensor tb = bias ? view(bias, {cols}, dtype) : Tensor();
        NormArgs a{&tx, weight ? &tw : nullptr, bias ? &tb : nullptr, &to, rows, cols, eps,
                   rms != 0, 0, 0};
        NormRegistry::instance().get("stock")(a);
    });
}

int ref_modulate(const void* x, const void* scale, const void* shift, void* out, int64_t batch,
                 int64_t tokens, int64_t channels, const void* residual, const void* gate,
                 int dtype) {
    return guard([&] {
        Tensor tx = view(x, {batch, tokens, channels}, dtype);
        Tensor to = view(out, {batch, tokens, channels}, dtype);
        Tensor ts = view(scale, {batch, channels}, dtype), th = view(shift, {batch, channels}, dtype);
        Tensor tr = residual ? view(residual, {batch, tokens, channels}, dtype) : Tensor();
        Tensor tg = gate ? view(gate, {batch, channels}, dtype) : Tensor();
        ModulateArgs a{&tx, &ts, &th, &to, batch, tokens, channels, residual ? &tr : nullptr,
                       gate ? &tg : nullptr};
        ModulateRegistry::instance().get("stock")(a);
    });
}

int ref_activation(const void* x, void* out, int64_t n, int kind, const void* gate, int dtype) {
    return guard([&] {
        Tensor tx = view(x, {n}, dtype), to = view(out, {n}, dtype);
        Tensor tg = gate ? view(gate, {n}, dtype) : Tensor();
        ActivationArgs a{&tx, &to, n, epi_of(kind), gate ? &tg : nullptr};
        ActivationRegistry::instance().get("stock")(a);
    });
}

int ref_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner, float scale,
            int broadcast_b, int dtype) {
    return guard([&] {
        Tensor ta = view(a, {outer, inner}, dtype), to = view(out, {outer, inner}, dtype);
        Tensor tb = view(b, broadcast_b ? std::vector<int64_t>{inner} : std::vector<int64_t>{outer, inner}, dtype);
        AddArgs args{&ta, &tb, &to, outer, inner, scale, broadcast_b != 0};
        AddRegistry::instance().get("stock")(args);
    });
}

int ref_chunk(const void* mod, const void* table, void* out, int64_t batch, int64_t channels,
              int64_t chunks, int64_t chunk, int64_t table_chunk, int table_rows, int dtype) {
    return guard([&] {
        Tensor tm = view(mod, {batch, chunks * channels}, dtype);
        Tensor tt = view(table, {table_rows, channels}, dtype);
        Tensor to = view(out, {batch, channels}, dtype);
        ChunkArgs a{&tm, &tt, &to, batch, channels, chunks, chunk, table_chunk};
        ChunkRegistry::instance().get("stock")(a);
    });
}

int ref_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
              int64_t patch, int inverse, int dtype) {
    return guard([&] {
        const int64_t H = grid * patch, tok = grid * grid, per = channels * patch * patch;
        Tensor img = view(inverse ? out : in, {batch, channels, H, H}, dtype);
        Tensor tks = view(inverse ? in : out, {batch, tok, per}, dtype);
        PatchArgs a{inverse ? &tks : &img, inverse ? &img : &tks, batch, channels, grid, patch,
                    inverse != 0};
        PatchRegistry::instance().get("stock")(a);
    });
}

int ref_position_embedding(double* out, int dim, int grid, int base, double interp) {
    return guard([&] {
        const std::vector<double> pe = dit_position_embedding(dim, grid, base, interp);
        std::memcpy(out, pe.data(), pe.size() * sizeof(double));
    });
}

int ref_timestep_embedding(double t, int dim, float* out) {
    return guard([&] {
        Tensor e = sinusoidal_timestep_embedding(t, dim, DType::F32);
        std::memcpy(out, e.data(), sizeof(float) * dim);
    });
}

int ref_dit_forward(const bh_dit_config* cfg, const bh_dit_weights* w, int64_t batch,
                    int64_t latent_hw, int64_t caption_len, const uint16_t* latent,
                    double timestep, const uint16_t* caption, const void* mask, int mask_dtype,
                    uint16_t* image, int layers) {
    return guard([&] {
        DiTConfig dc;
        dc.num_layers = layers >= 0 ? std::min(layers, cfg->num_layers) : cfg->num_layers;
        dc.num_heads = cfg->num_heads;
        dc.head_dim = cfg->head_dim;
        dc.patch_size = cfg->patch_size;
        dc.in_channels = cfg->in_channels;
        dc.out_channels = cfg->out_channels;
        dc.caption_channels = cfg->caption_channels;
        dc.mlp_ratio = cfg->mlp_ratio;
        dc.eps = cfg->eps;
        dc.sample_size = cfg->sample_size;
        TableWeights weights(*cfg, *w);
        PixArtDiT model(dc, weights, DType::BF16);
        Tensor z = view(latent, {batch, cfg->in_channels, latent_hw, latent_hw}, BH_BF16);
        Tensor cap = view(caption, {batch, caption_len, cfg->caption_channels}, BH_BF16);
        Tensor m = view(mask, {batch, caption_len}, mask_dtype);
        Tensor out = model.forward(z, timestep, cap, m, ImplSelection::from_request("stock"));
        std::memcpy(image, out.data(), out.nbytes());
    });
}


int ref_scale(const void* in, void* out, int64_t numel, float scale, int dtype) {
    return guard([&] {
        Tensor x = view(in, {numel}, dtype);
        Tensor y = view(out, {numel}, dtype);
        ScaleRegistry::instance().get("stock")(ScaleArgs{&x, &y, numel, scale});
    });
}

int ref_repeat(const void* in, void* out, int64_t outer, int64_t inner, int dtype) {
    return guard([&] {
        Tensor x = view(in, {inner}, dtype);
        Tensor y = view(out, {outer * inner}, dtype);
        RepeatRegistry::instance().get("stock")(RepeatArgs{&x, &y, outer, inner});
    });
}

int ref_guidance(const void* pred, void* out, int64_t out_channels, int64_t channels,
                 int64_t spatial, float scale, int dtype) {
    return guard([&] {
        Tensor p = view(pred, {2, out_channels, spatial}, dtype);
        Tensor y = view(out, {channels, spatial}, dtype);
        GuidanceRegistry::instance().get("stock")(
            GuidanceArgs{&p, &y, out_channels, channels, spatial, scale});
    });
}

// The reference's own DPMSolverMultistep behind an opaque handle, on host buffers.
int ref_sched_create(const bh_sched_config* c, void** out) {
    return guard([&] {
        SchedulerConfig sc;
        sc.num_train_timesteps = c->num_train_timesteps;
        sc.beta_start = c->beta_start;
        sc.beta_end = c->beta_end;
        sc.beta_schedule = c->beta_schedule;
        sc.solver_order = c->solver_order;
        sc.algorithm_type = c->algorithm_type;
        sc.solver_type = c->solver_type;
        sc.prediction_type = c->prediction_type;
        sc.timestep_spacing = c->timestep_spacing;
        sc.lower_order_final = c->lower_order_final != 0;
        *out = new DPMSolverMultistep(sc);
    });
}

void ref_sched_destroy(void* h) { delete static_cast<DPMSolverMultistep*>(h); }

int ref_sched_set_timesteps(void* h, int steps) {
    return guard([&] { static_cast<DPMSolverMultistep*>(h)->set_timesteps(steps); });
}

int ref_sched_steps(const void* h) { return static_cast<const DPMSolverMultistep*>(h)->steps(); }

int ref_sched_timestep(const void* h, int i, int64_t* out) {
    return guard([&] { *out = static_cast<const DPMSolverMultistep*>(h)->timestep(i); });
}

int ref_sched_sigma(const void* h, int i, double* out) {
    return guard([&] { *out = static_cast<const DPMSolverMultistep*>(h)->sigma(i); });
}

int ref_sched_coefficients(const void* h, int i, bh_sched_coefficients* out) {
    return guard([&] {
        const auto c = static_cast<const DPMSolverMultistep*>(h)->coefficients(i);
        *out = bh_sched_coefficients{c.order,   c.sigma_s0, c.sigma_t,   c.sigma_vp_s0, c.sigma_vp_t,
                                     c.alpha_t, c.alpha_s0, c.exp_neg_h, c.r0};
    });
}

int ref_sched_step(void* h, const void* eps, int i, void* sample, int64_t n, int dtype) {
    return guard([&] {
        Tensor e = view(eps, {n}, dtype);
        Tensor x = view(sample, {n}, dtype);
        static_cast<DPMSolverMultistep*>(h)->step(e, i, x);
    });
}

int ref_sched_reset(void* h) {
    return guard([&] { static_cast<DPMSolverMultistep*>(h)->reset(); });
}

int ref_conv2d(const void* x, const void* w, const void* bias, void* out, int64_t batch, int64_t c_in,
               int64_t h, int64_t wd, int64_t c_out, int64_t k, int64_t pad, int dtype) {
    return guard([&] {
        const int64_t ho = h + 2 * pad - k + 1, wo = wd + 2 * pad - k + 1;
        Tensor tx = view(x, {batch, c_in, h, wd}, dtype), tw = view(w, {c_out, c_in, k, k}, dtype);
        Tensor tb = bias ? view(bias, {c_out}, dtype) : Tensor();
        Tensor to = view(out, {batch, c_out, ho, wo}, dtype);
        Conv2dArgs a{&tx, &tw, bias ? &tb : nullptr, &to, batch, c_in, h, wd, c_out, k, pad};
        Conv2dRegistry::instance().get("stock")(a);
    });
}

int ref_group_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                   int64_t cols, float eps, int64_t groups, int64_t channels, int dtype) {
    return guard([&] {
        Tensor tx = view(x, {rows, cols}, dtype), to = view(out, {rows, cols}, dtype);
        Tensor tw = weight ? view(weight, {channels}, dtype) : Tensor();
        Tensor tb = bias ? view(bias, {channels}, dtype) : Tensor();
        NormArgs a{&tx, weight ? &tw : nullptr, bias ? &tb : nullptr, &to, rows, cols, eps, false,
                   groups, channels};
        NormRegistry::instance().get("stock")(a);
    });
}

int ref_upsample(const void* in, void* out, int64_t batch, int64_t channels, int64_t h, int64_t w,
                 int64_t factor, int dtype) {
    return guard([&] {
        Tensor ti = view(in, {batch, channels, h, w}, dtype);
        Tensor to = view(out, {batch, channels, h * factor, w * factor}, dtype);
        UpsampleArgs a{&ti, &to, batch, channels, h, w, factor};
        UpsampleRegistry::instance().get("stock")(a);
    });
}

int ref_transpose(const void* in, void* out, int64_t batch, int64_t channels, int64_t spatial,
                  int to_channels_first, int dtype) {
    return guard([&] {
        std::vector<int64_t> cf{batch, channels, spatial}, sf{batch, spatial, channels};
        Tensor ti = view(in, to_channels_first ? sf : cf, dtype);
        Tensor to = view(out, to_channels_first ? cf : sf, dtype);
        TransposeArgs a{&ti, &to, batch, channels, spatial, to_channels_first != 0};
        TransposeRegistry::instance().get("stock")(a);
    });
}

// VaeDecoder::forward (vae_decoder.cpp:127-180) on the reference's own model code; the weight
// shapes come from its own declaration (declare_pixart_shapes, weights.cpp:284-320).
int ref_vae_forward(const bh_vae_config* cfg, const bh_vae_weights* w, const uint16_t* latent,
                    int64_t latent_hw, uint16_t* image) {
    return guard([&] {
        VaeConfig vc;
        vc.block_out_channels.assign(cfg->block_out_channels, cfg->block_out_channels + cfg->num_blocks);
        vc.layers_per_block = cfg->layers_per_block;
        vc.latent_channels = cfg->latent_channels;
        vc.norm_num_groups = cfg->norm_num_groups;
        vc.eps = cfg->eps;
        NamedWeights nw(*w);
        T5Config t5;
        t5.num_layers = 0;
        DiTConfig dit;
        dit.num_layers = 0;
        SyntheticWeights decl(DType::BF16, 0);
        declare_pixart_shapes(decl, t5, dit, vc);
        for (int i = 0; i < w->count; ++i) nw.set_shape(w->names[i], decl.get(w->names[i]).shape());
        VaeDecoder dec(vc, nw, DType::BF16);
        const ImplSelection impls = ImplSelection::from_request("stock", Device::CPU);
        Tensor x = view(latent, {1, vc.latent_channels, latent_hw, latent_hw}, BH_BF16);
        Tensor out = dec.forward(x, impls);
        std::memcpy(image, out.data(), static_cast<size_t>(out.numel()) * 2);
    });
}

int ref_t5_bucket(int rp, int num_buckets, int max_distance) {
    return t5_relative_bucket(rp, num_buckets, max_distance);
}

// T5Encoder::forward (t5_encoder.cpp:132-241) on the reference's own model code; the weight shapes
// come from its own declaration (declare_pixart_shapes, weights.cpp:226-244).
int ref_t5_forward(const bh_t5_config* cfg, const bh_t5_weights* w, const float* ids, int64_t batch,
                   int64_t seq, uint16_t* out) {
    return guard([&] {
        T5Config t5;
        t5.num_layers = cfg->num_layers;
        t5.d_model = cfg->d_model;
        t5.d_ff = cfg->d_ff;
        t5.d_kv = cfg->d_kv;
        t5.num_heads = cfg->num_heads;
        t5.vocab_size = cfg->vocab_size;
        t5.gated = cfg->gated != 0;
        t5.eps = cfg->eps;
        if (cfg->num_buckets != 32) throw std::runtime_error("ref t5: the declaration has 32 buckets");
        NamedWeights nw(w->count, w->names, w->tensors);
        DiTConfig dit;
        dit.num_layers = 0;
        VaeConfig vc;
        SyntheticWeights decl(DType::BF16, 0);
        declare_pixart_shapes(decl, t5, dit, vc);
        for (int i = 0; i < w->count; ++i) nw.set_shape(w->names[i], decl.get(w->names[i]).shape());
        T5Encoder enc(t5, nw, DType::BF16);
        const ImplSelection impls = ImplSelection::from_request("stock", Device::CPU);
        Tensor t = view(ids, {batch, seq}, BH_F32);
        Tensor o = enc.forward(t, impls);
        std::memcpy(out, o.data(), static_cast<size_t>(o.numel()) * 2);
    });
}

}  // extern "C"
