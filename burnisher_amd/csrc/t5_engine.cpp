// The T5 v1.1 encoder engine (the t5-encode stage): T5Encoder::forward (t5_encoder.cpp:132-241)
// on one MI355X.
//
// Activations are [batch * seq, width] bf16 rows, as in the reference. What differs is how the
// work is cut for gfx950:
//   - each layer's q/k/v weights are packed into one [3 * inner, d_model] operand and wi_0/wi_1
//     into one [2 * d_ff, d_model] operand at create, so each projection is ONE launch of the
//     persistent MFMA GEMM: at the pipeline's 600 token rows a 4096-wide projection alone has
//     87 output tiles for 256 CUs, the packed ones 258 and 429;
//   - attention reads q/k/v in place from the packed projection (row stride 3 * inner) on the
//     flash kernel, with the relative-position bias added to the scores there;
//   - the attention and FFN output projections add the residual in their epilogue (the projection
//     is rounded to bf16 first, as the reference's separate add sees it);
//   - the gated GELU reads both halves of the packed FFN projection.
// Every op's output is stored in bf16 where the reference stores a tensor.
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

namespace {

constexpr int kMaxDistance = 128;   // t5_encoder.cpp:60, relative_buckets' fixed max_distance

int relative_bucket(int rp, int num_buckets, int max_distance) {
    // Bidirectional: the upper half of the buckets is for keys after the query. Within a half,
    // distances below half/2 get a bucket each; beyond, buckets are log-spaced up to
    // max_distance and saturate at the half's last bucket (t5_encoder.cpp:34-48).
    const int half = num_buckets / 2;
    const int offset = rp > 0 ? half : 0;
    const int dist = std::abs(rp);
    const int exact = half / 2;
    if (dist < exact) return offset + dist;
    const double scaled = std::log(static_cast<double>(dist) / exact) /
                          std::log(static_cast<double>(max_distance) / exact) * (half - exact);
    return offset + std::min(exact + static_cast<int>(scaled), half - 1);
}

std::string blk(int i, const char* tail) { return "encoder.block." + std::to_string(i) + "." + tail; }

}  // namespace

struct bh_t5 {
    bh_t5_config cfg{};
    int64_t B = 0, S = 0, M = 0, d = 0, H = 0, inner = 0, F = 0;
    std::map<std::string, const bf16_t*> w;   // the caller's tensors, by name
    std::vector<bf16_t*> qkv_w, wi_w;          // packed per layer (engine-owned)
    std::vector<void*> allocs;
    bf16_t *x = nullptr, *normed = nullptr, *qkv = nullptr, *ctx = nullptr, *h01 = nullptr,
           *hact = nullptr, *bias = nullptr, *mask = nullptr;
    float* ids = nullptr;
    int* bucket = nullptr;
    float* partial = nullptr;        // split-K partials of the two output projections
    int split_o = 1, split_wo = 1;
    float* ids_host = nullptr;       // pinned staging of one call's ids
    bf16_t* mask_host = nullptr;     // and its key mask
    hipEvent_t staged = nullptr;
    bool staged_pending = false;
    int64_t bytes = 0;

    ~bh_t5() {
        if (staged) {
            (void)hipEventSynchronize(staged);
            (void)hipEventDestroy(staged);
        }
        for (void* p : allocs) (void)hipFree(p);
        if (ids_host) (void)hipHostFree(ids_host);
        if (mask_host) (void)hipHostFree(mask_host);
    }
    void* alloc(int64_t n) {
        void* p = nullptr;
        const size_t sz = static_cast<size_t>(std::max<int64_t>(n, 256));
        bh::hip_check(hipMalloc(&p, sz), "hipMalloc (t5)");
        allocs.push_back(p);
        bh::hip_check(hipMemset(p, 0, sz), "hipMemset (t5)");
        bytes += n;
        return p;
    }
    bf16_t* alloc_bf(int64_t elems) { return static_cast<bf16_t*>(alloc(elems * 2)); }
    const bf16_t* at(const std::string& n) const {
        auto it = w.find(n);
        if (it == w.end()) throw bh::Error("t5: weight '" + n + "' is missing");
        return it->second;
    }
};

namespace {

void encode(bh_t5* e, const float* ids_in, bf16_t* out, hipStream_t s) {
    const bh_t5_config& c = e->cfg;
    const int64_t M = e->M, d = e->d, inner = e->inner, F = e->F;
    // the reference's host check (t5_encoder.cpp:146-156), before any device work
    for (int64_t i = 0; i < M; ++i) {
        const float f = ids_in[i];
        const double v = static_cast<double>(f);
        if (!(v > -1.0 && v < static_cast<double>(c.vocab_size))) {
            const std::string shown = std::isfinite(f) ? std::to_string(static_cast<int64_t>(f)) : "non-finite";
            throw bh::Error("t5: token id " + shown + " is outside the vocabulary; a tokenizer mismatch "
                            "is a changed oracle");
        }
    }
    if (e->staged_pending) bh::hip_check(hipEventSynchronize(e->staged), "hipEventSynchronize (t5 ids)");
    for (int64_t i = 0; i < M; ++i) {
        e->ids_host[i] = ids_in[i];
        e->mask_host[i] = static_cast<int64_t>(ids_in[i]) == 0 ? bf16_t{0} : bf16_t{0x3f80};   // pad id 0
    }
    bh::hip_check(hipMemcpyAsync(e->ids, e->ids_host, M * sizeof(float), hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync (t5 ids)");
    bh::hip_check(hipMemcpyAsync(e->mask, e->mask_host, M * sizeof(bf16_t), hipMemcpyHostToDevice, s),
                  "hipMemcpyAsync (t5 mask)");
    bh::hip_check(hipEventRecord(e->staged, s), "hipEventRecord (t5 ids)");
    e->staged_pending = true;

    bh::launch_gather(e->at("shared.weight"), e->ids, e->x, M, d, c.vocab_size, false, s);
    bh::launch_rel_bias(e->at("encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"),
                        e->bucket, e->bias, e->H, e->S, s);
    const float eps = static_cast<float>(c.eps);
    bh::GemmEpilogue plain;
    bh::GemmEpilogue residual;
    residual.round_mid = true;
    residual.residual = e->x;
    const bh::AttnShape sh{e->B, e->H, e->S, e->S, c.d_kv, 3 * inner, 3 * inner, inner, 1.0f};
    for (int l = 0; l < c.num_layers; ++l) {
        bh::launch_norm(e->x, e->at(blk(l, "layer.0.layer_norm.weight")), nullptr, e->normed, M, d, eps,
                        true, false, s);
        bh::launch_gemm_bf16(e->normed, e->qkv_w[l], nullptr, e->qkv, M, 3 * inner, d, plain, s);
        bh::launch_attention_bf16(e->qkv, e->qkv + inner, e->qkv + 2 * inner, e->ctx, sh, e->mask, false, s,
                                  e->bias);
        if (e->split_o > 1)
            bh::launch_gemm_splitk_residual(e->ctx, e->at(blk(l, "layer.0.SelfAttention.o.weight")), e->partial,
                                            e->split_o, e->x, e->x, M, d, inner, s);
        else
            bh::launch_gemm_bf16(e->ctx, e->at(blk(l, "layer.0.SelfAttention.o.weight")), nullptr, e->x, M, d,
                                 inner, residual, s);
        bh::launch_norm(e->x, e->at(blk(l, "layer.1.layer_norm.weight")), nullptr, e->normed, M, d, eps,
                        true, false, s);
        if (c.gated) {
            bh::launch_gemm_bf16(e->normed, e->wi_w[l], nullptr, e->h01, M, 2 * F, d, plain, s);
            bh::launch_gelu_gated_rows(e->h01, e->hact, M, F, s);
        } else {
            bh::launch_gemm_bf16(e->normed, e->at(blk(l, "layer.1.DenseReluDense.wi_0.weight")), nullptr,
                                 e->h01, M, F, d, plain, s);
            bh::launch_activation(e->h01, e->hact, M * F, BH_EPI_GELU, nullptr, false, s);
        }
        if (e->split_wo > 1)
            bh::launch_gemm_splitk_residual(e->hact, e->at(blk(l, "layer.1.DenseReluDense.wo.weight")),
                                            e->partial, e->split_wo, e->x, e->x, M, d, F, s);
        else
            bh::launch_gemm_bf16(e->hact, e->at(blk(l, "layer.1.DenseReluDense.wo.weight")), nullptr, e->x, M, d,
                                 F, residual, s);
    }
    bh::launch_norm(e->x, e->at("encoder.final_layer_norm.weight"), nullptr, out, M, d, eps, true, false, s);
}

}  // namespace

namespace bh {

// The T5 part of declare_pixart_shapes (weights.cpp:226-244), in its order.
std::vector<std::pair<std::string, std::vector<int64_t>>> t5_tensor_shapes(const bh_t5_config& c) {
    const int64_t d = c.d_model, inner = static_cast<int64_t>(c.num_heads) * c.d_kv, f = c.d_ff;
    std::vector<std::pair<std::string, std::vector<int64_t>>> t{
        {"shared.weight", {c.vocab_size, d}},
        {"encoder.final_layer_norm.weight", {d}},
        {"encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight", {c.num_buckets, c.num_heads}}};
    for (int i = 0; i < c.num_layers; ++i) {
        t.push_back({blk(i, "layer.0.layer_norm.weight"), {d}});
        t.push_back({blk(i, "layer.1.layer_norm.weight"), {d}});
        for (const char* p : {"layer.0.SelfAttention.q.weight", "layer.0.SelfAttention.k.weight",
                              "layer.0.SelfAttention.v.weight"})
            t.push_back({blk(i, p), {inner, d}});
        t.push_back({blk(i, "layer.0.SelfAttention.o.weight"), {d, inner}});
        t.push_back({blk(i, "layer.1.DenseReluDense.wi_0.weight"), {f, d}});
        if (c.gated) t.push_back({blk(i, "layer.1.DenseReluDense.wi_1.weight"), {f, d}});
        t.push_back({blk(i, "layer.1.DenseReluDense.wo.weight"), {d, f}});
    }
    return t;
}

}  // namespace bh

extern "C" {

int bh_t5_relative_bucket(int relative_position, int num_buckets, int max_distance) {
    if (num_buckets < 4 || max_distance < 1) return -1;
    return relative_bucket(relative_position, num_buckets, max_distance);
}

int bh_t5_create(const bh_t5_config* cfg, const bh_t5_weights* w, int64_t batch, int64_t seq_len,
                 bh_t5** out) {
    return bh::guarded([&] {
        bh::require(out != nullptr, "t5_create: null output handle");
        *out = nullptr;
        bh::require(cfg && w, "t5_create: null config or weights");
        const bh_t5_config& c = *cfg;
        bh::require(c.num_layers >= 0 && c.d_model > 0 && c.d_ff > 0 && c.num_heads > 0 && c.vocab_size > 0 &&
                        c.eps > 0.0,
                    "t5_create: configuration out of range");
        bh::require(c.d_kv >= 1 && c.d_kv <= 128, "t5_create: d_kv must be in [1, 128]");
        bh::require(c.num_buckets >= 4 && c.num_buckets % 2 == 0,
                    "t5_create: num_buckets must be even and at least 4");
        bh::require(batch > 0 && seq_len > 0 && seq_len <= 8192, "t5_create: batch or seq_len out of range");
        bh::require(w->count >= 0 && (w->count == 0 || (w->names && w->tensors)), "t5_create: bad weight table");
        auto e = std::make_unique<bh_t5>();
        e->cfg = c;
        e->B = batch;
        e->S = seq_len;
        e->M = batch * seq_len;
        e->d = c.d_model;
        e->H = c.num_heads;
        e->inner = static_cast<int64_t>(c.num_heads) * c.d_kv;
        e->F = c.d_ff;
        for (int i = 0; i < w->count; ++i) {
            bh::require(w->names[i] && w->tensors[i], "t5_create: null weight name or tensor");
            e->w[w->names[i]] = static_cast<const bf16_t*>(w->tensors[i]);
        }
        for (const auto& t : bh::t5_tensor_shapes(c)) (void)e->at(t.first);   // all present
        const int64_t M = e->M, d = e->d, inner = e->inner, F = e->F;
        e->x = e->alloc_bf(M * d);
        e->normed = e->alloc_bf(M * d);
        e->qkv = e->alloc_bf(M * 3 * inner);
        e->ctx = e->alloc_bf(M * inner);
        e->h01 = e->alloc_bf(M * (c.gated ? 2 * F : F));
        e->hact = e->alloc_bf(M * F);
        e->bias = e->alloc_bf(e->H * e->S * e->S);
        e->mask = e->alloc_bf(M);
        e->ids = static_cast<float*>(e->alloc(M * 4));
        e->bucket = static_cast<int*>(e->alloc((2 * e->S - 1) * 4));
        // the two d_model-wide output projections have the fewest output tiles: split their K
        // when that fills more CUs (fp32 partials summed in a fixed order, then the residual)
        e->split_o = bh::gemm_splitk_choice(M, d, inner);
        e->split_wo = bh::gemm_splitk_choice(M, d, F);
        if (std::max(e->split_o, e->split_wo) > 1)
            e->partial = static_cast<float*>(e->alloc(std::max(e->split_o, e->split_wo) * M * d * 4));
        std::vector<int> bucket(static_cast<size_t>(2 * e->S - 1));
        for (int64_t r = -(e->S - 1); r <= e->S - 1; ++r)
            bucket[r + e->S - 1] = relative_bucket(static_cast<int>(r), c.num_buckets, kMaxDistance);
        bh::hip_check(hipMemcpy(e->bucket, bucket.data(), bucket.size() * 4, hipMemcpyHostToDevice),
                      "hipMemcpy (t5 buckets)");
        bh::hip_check(hipHostMalloc(reinterpret_cast<void**>(&e->ids_host), M * sizeof(float)),
                      "hipHostMalloc (t5 ids)");
        bh::hip_check(hipHostMalloc(reinterpret_cast<void**>(&e->mask_host), M * sizeof(bf16_t)),
                      "hipHostMalloc (t5 mask)");
        bh::hip_check(hipEventCreateWithFlags(&e->staged, hipEventDisableTiming), "hipEventCreate (t5)");
        // packed projections
        const size_t proj = static_cast<size_t>(inner * d) * 2, ff = static_cast<size_t>(F * d) * 2;
        for (int l = 0; l < c.num_layers; ++l) {
            bf16_t* q = e->alloc_bf(3 * inner * d);
            const char* parts[3] = {"layer.0.SelfAttention.q.weight", "layer.0.SelfAttention.k.weight",
                                    "layer.0.SelfAttention.v.weight"};
            for (int p = 0; p < 3; ++p)
                bh::hip_check(hipMemcpy(q + p * inner * d, e->at(blk(l, parts[p])), proj, hipMemcpyDeviceToDevice),
                              "hipMemcpy (t5 qkv pack)");
            e->qkv_w.push_back(q);
            if (c.gated) {
                bf16_t* f = e->alloc_bf(2 * F * d);
                bh::hip_check(hipMemcpy(f, e->at(blk(l, "layer.1.DenseReluDense.wi_0.weight")), ff,
                                        hipMemcpyDeviceToDevice), "hipMemcpy (t5 wi pack)");
                bh::hip_check(hipMemcpy(f + F * d, e->at(blk(l, "layer.1.DenseReluDense.wi_1.weight")), ff,
                                        hipMemcpyDeviceToDevice), "hipMemcpy (t5 wi pack)");
                e->wi_w.push_back(f);
            }
        }
        bh::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize (t5 create)");
        *out = e.release();
    });
}

int bh_t5_encode(bh_t5* e, const float* token_ids, void* out, void* stream) {
    return bh::guarded([&] {
        bh::require(e != nullptr, "t5_encode: null engine");
        bh::require(token_ids != nullptr, "t5_encode: null ids");
        bh::require_device_ptr(out, "t5_encode", "out");
        encode(e, token_ids, static_cast<bf16_t*>(out), static_cast<hipStream_t>(stream));
    });
}

int64_t bh_t5_workspace_bytes(const bh_t5* e) { return e ? e->bytes : -1; }

void bh_t5_destroy(bh_t5* e) { delete e; }

}  // extern "C"
