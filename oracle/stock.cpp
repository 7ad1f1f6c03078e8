// oracle/stock.cpp -- TEST INFRASTRUCTURE ONLY. A CPU restatement of the reference runtime's
// `stock` implementation of the dit-step ops and graph, used as the parity checker for the HIP
// path and as the CPU baseline that bench.py times. Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it; the product (burnisher_amd/) never does.
//
// It follows, function by function (cited at each function):
//   /root/reference/src/cpu/ops_cpu.cpp        the op kernels
//   /root/reference/src/models/pixart_dit.cpp  the graph and the position table
//   /root/reference/src/models/weights.cpp     the timestep embedding
//   /root/reference/include/burnisher/dtype.h  bf16 round-to-nearest-even
//
// The numerics contract is the reference's, restated exactly:
//   * every op reads its inputs as float, computes in fp32 and rounds ONCE per stored element
//     to the storage dtype (tensor.cpp:85-96);
//   * every reduction runs in the reference's fixed sequential order with an fp32 accumulator
//     (GEMM over k, attention over d and over keys), LayerNorm statistics in fp64;
//   * no fused multiply-add: this file is compiled with -ffp-contract=off, as the reference's
//     x86-64 build has no FMA to contract into.
// What differs from the reference is only speed: operands are widened to float once per call,
// loops are blocked and vectorised ACROSS independent outputs (never across a reduction), and
// the work is split over threads by output rows. Every output is therefore computed by the same
// sequence of fp32 operations as in the reference, whatever the thread count.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../include/burnisher_hip.h"

namespace {

// ---- dtype (dtype.h:50-72) ------------------------------------------------------------------

inline float bf16_to_f32(uint16_t v) {
    uint32_t u = static_cast<uint32_t>(v) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// A typed buffer: what Tensor::get/set do for one dtype.
struct View {
    const void* p;
    int dt;  // BH_F32 or BH_BF16
    float get(int64_t i) const {
        return dt == BH_F32 ? static_cast<const float*>(p)[i]
                            : bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
};
struct Out {
    void* p;
    int dt;
    void set(int64_t i, float v) const {
        if (dt == BH_F32) static_cast<float*>(p)[i] = v;
        else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
    }
};
// What storing through the dtype does to a value.
inline float stored(float v, int dt) { return dt == BH_F32 ? v : bf16_to_f32(f32_to_bf16(v)); }

std::vector<float> widen(const void* p, int dt, int64_t n) {
    std::vector<float> out(static_cast<size_t>(n));
    View v{p, dt};
    for (int64_t i = 0; i < n; ++i) out[i] = v.get(i);
    return out;
}

// ---- threads --------------------------------------------------------------------------------

int resolve_threads(int t) {
    if (t > 0) return t;
    const unsigned hc = std::thread::hardware_concurrency();
    return hc ? static_cast<int>(hc) : 1;
}

// Calls fn(i) for i in [0, n), items handed out dynamically. Each item writes only its own
// outputs, so the result does not depend on the schedule.
template <typename Fn>
void parallel_for(int64_t n, int threads, Fn fn) {
    threads = std::max(1, std::min<int>(threads, static_cast<int>(std::min<int64_t>(n, 1 << 20))));
    if (threads <= 1) {
        for (int64_t i = 0; i < n; ++i) fn(i);
        return;
    }
    std::atomic<int64_t> next{0};
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        pool.emplace_back([&] {
            for (int64_t i = next++; i < n; i = next++) fn(i);
        });
    }
    for (auto& th : pool) th.join();
}

// ---- activations (ops_cpu.cpp:27-46) --------------------------------------------------------

inline float gelu_tanh(float x) {
    const float c = 0.7978845608028654f;
    float x3 = x * x * x;
    return 0.5f * x * (1.0f + std::tanh(c * (x + 0.044715f * x3)));
}
inline float silu(float x) { return x / (1.0f + std::exp(-x)); }
inline float apply_epilogue(int e, float v) {
    switch (e) {
        case BH_EPI_GELU: return gelu_tanh(v);
        case BH_EPI_SILU: return silu(v);
        case BH_EPI_GELU_GATED: return gelu_tanh(v);
        default: return v;
    }
}

// ---- gemm (ops_cpu.cpp:48-79) ---------------------------------------------------------------

// out[i,j] = epilogue(sum_p a[i,p]*b(p,j) + bias[j]), p sequential from 0, fp32 accumulator.
// Vectorised across j: bt is B widened and laid out [K][N] so that one k step updates a run of
// independent column accumulators.
void gemm_impl(const void* a, const void* b, const void* bias, void* out, int64_t M, int64_t N,
               int64_t K, bool b_transposed, int epilogue, int dt, int threads) {
    std::vector<float> af = widen(a, dt, M * K);
    std::vector<float> bt(static_cast<size_t>(K * N));
    {
        View bv{b, dt};
        for (int64_t p = 0; p < K; ++p)
            for (int64_t j = 0; j < N; ++j)
                bt[p * N + j] = bv.get(b_transposed ? (j * K + p) : (p * N + j));
    }
    std::vector<float> biasf = bias ? widen(bias, dt, N) : std::vector<float>();
    const Out o{out, dt};
    constexpr int64_t RB = 4, CB = 256;
    const int64_t row_blocks = (M + RB - 1) / RB;
    parallel_for(row_blocks, threads, [&](int64_t rb) {
        const int64_t i0 = rb * RB, i1 = std::min(M, i0 + RB);
        float acc[RB][CB];
        for (int64_t j0 = 0; j0 < N; j0 += CB) {
            const int64_t jn = std::min(CB, N - j0);
            for (int64_t r = 0; r < RB; ++r)
                for (int64_t jj = 0; jj < CB; ++jj) acc[r][jj] = 0.0f;
            for (int64_t p = 0; p < K; ++p) {
                const float* brow = &bt[p * N + j0];
                for (int64_t i = i0; i < i1; ++i) {
                    const float av = af[i * K + p];
                    float* ac = acc[i - i0];
                    for (int64_t jj = 0; jj < jn; ++jj) ac[jj] += av * brow[jj];
                }
            }
            for (int64_t i = i0; i < i1; ++i) {
                for (int64_t jj = 0; jj < jn; ++jj) {
                    float v = acc[i - i0][jj];
                    if (bias) v += biasf[j0 + jj];
                    o.set(i * N + j0 + jj, apply_epilogue(epilogue, v));
                }
            }
        }
    });
}

// ---- attention (ops_cpu.cpp:84-184) ---------------------------------------------------------

struct AttnGeom {
    int64_t B, H, Sq, Skv, D;
    int64_t ld_q, ld_kv, ld_o;
};

// Streaming attention (ops_cpu.cpp:84-131), one query row at a time: scores over d sequential,
// times scale, + bias, masked keys set to -1e9; row max; exp(s - max) and the denominator summed
// over keys in order; the value accumulator over keys in order; divide at the end.
void attention_impl(const void* q, const void* k, const void* v, void* out, const AttnGeom& g,
                    float scale, const void* bias, const void* mask, int mask_dt, int dt,
                    int threads, bool materialized) {
    const float sc = scale > 0.0f ? scale : 1.0f / std::sqrt(static_cast<float>(g.D));
    const View qv{q, dt}, kv{k, dt}, vv{v, dt}, bv{bias, dt}, mv{mask, mask_dt};
    const Out o{out, dt};
    // per (b, h): K transposed to [D][Skv] and V as [Skv][D], widened once
    const int64_t BH = g.B * g.H;
    constexpr int64_t QB = 16;
    const int64_t qblocks = (g.Sq + QB - 1) / QB;
    std::vector<std::vector<float>> kt(BH), vf(BH);
    parallel_for(BH, threads, [&](int64_t bh) {
        const int64_t b = bh / g.H, h = bh % g.H;
        kt[bh].resize(static_cast<size_t>(g.D * g.Skv));
        vf[bh].resize(static_cast<size_t>(g.Skv * g.D));
        for (int64_t j = 0; j < g.Skv; ++j) {
            const int64_t base = (b * g.Skv + j) * g.ld_kv + h * g.D;
            for (int64_t d = 0; d < g.D; ++d) {
                kt[bh][d * g.Skv + j] = kv.get(base + d);
                vf[bh][j * g.D + d] = vv.get(base + d);
            }
        }
    });
    std::vector<float> keep(static_cast<size_t>(mask ? g.B * g.Skv : 0));
    for (size_t i = 0; i < keep.size(); ++i) keep[i] = mv.get(static_cast<int64_t>(i));
    parallel_for(BH * qblocks, threads, [&](int64_t item) {
        const int64_t bh = item / qblocks, qb = item % qblocks;
        const int64_t b = bh / g.H, h = bh % g.H;
        std::vector<float> s(static_cast<size_t>(g.Skv)), acc(static_cast<size_t>(g.D)),
            qrow(static_cast<size_t>(g.D));
        const float* K = kt[bh].data();
        const float* V = vf[bh].data();
        for (int64_t i = qb * QB; i < std::min(g.Sq, (qb + 1) * QB); ++i) {
            const int64_t qbase = (b * g.Sq + i) * g.ld_q + h * g.D;
            for (int64_t d = 0; d < g.D; ++d) qrow[d] = qv.get(qbase + d);
            std::fill(s.begin(), s.end(), 0.0f);
            for (int64_t d = 0; d < g.D; ++d) {
                const float qd = qrow[d];
                const float* krow = K + d * g.Skv;
                for (int64_t j = 0; j < g.Skv; ++j) s[j] += qd * krow[j];
            }
            float row_max = -INFINITY;
            for (int64_t j = 0; j < g.Skv; ++j) {
                float x = s[j] * sc;
                if (bias) x += bv.get((h * g.Sq + i) * g.Skv + j);
                if (mask && keep[b * g.Skv + j] == 0.0f) x = -1e9f;
                s[j] = x;
                row_max = std::max(row_max, x);
            }
            float denom = 0.0f;
            for (int64_t j = 0; j < g.Skv; ++j) {
                s[j] = std::exp(s[j] - row_max);
                denom += s[j];
            }
            if (materialized) {
                // ops_cpu.cpp:163-181: weights normalised first, then one accumulation per d.
                for (int64_t j = 0; j < g.Skv; ++j) s[j] /= denom;
                std::fill(acc.begin(), acc.end(), 0.0f);
                for (int64_t j = 0; j < g.Skv; ++j) {
                    const float w = s[j];
                    const float* vrow = V + j * g.D;
                    for (int64_t d = 0; d < g.D; ++d) acc[d] += w * vrow[d];
                }
                const int64_t obase = (b * g.Sq + i) * g.ld_o + h * g.D;
                for (int64_t d = 0; d < g.D; ++d) o.set(obase + d, acc[d]);
            } else {
                std::fill(acc.begin(), acc.end(), 0.0f);
                for (int64_t j = 0; j < g.Skv; ++j) {
                    const float w = s[j];
                    const float* vrow = V + j * g.D;
                    for (int64_t d = 0; d < g.D; ++d) acc[d] += w * vrow[d];
                }
                const int64_t obase = (b * g.Sq + i) * g.ld_o + h * g.D;
                for (int64_t d = 0; d < g.D; ++d) o.set(obase + d, acc[d] / denom);
            }
        }
    });
}

// ---- norm (ops_cpu.cpp:226-246) -------------------------------------------------------------

void norm_impl(const void* x, const void* w, const void* bias, void* out, int64_t rows,
               int64_t cols, float eps, bool rms, int dt, int threads) {
    const View xv{x, dt}, wv{w, dt}, bv{bias, dt};
    const Out o{out, dt};
    parallel_for(rows, threads, [&](int64_t r) {
        const int64_t base = r * cols;
        double mean = 0.0;
        if (!rms) {
            for (int64_t i = 0; i < cols; ++i) mean += xv.get(base + i);
            mean /= cols;
        }
        double var = 0.0;
        for (int64_t i = 0; i < cols; ++i) {
            double d = xv.get(base + i) - mean;
            var += d * d;
        }
        var /= cols;
        const float inv = 1.0f / std::sqrt(static_cast<float>(var) + eps);
        for (int64_t i = 0; i < cols; ++i) {
            float v = (xv.get(base + i) - static_cast<float>(mean)) * inv;
            if (w) v *= wv.get(i);
            if (bias) v += bv.get(i);
            o.set(base + i, v);
        }
    });
}

// ---- modulate, activation, add, chunk, patch (ops_cpu.cpp:249-349) --------------------------

void modulate_impl(const void* x, const void* scale, const void* shift, void* out, int64_t B,
                   int64_t T, int64_t C, const void* residual, const void* gate, int dt) {
    const View xv{x, dt}, sc{scale, dt}, sh{shift, dt}, rv{residual, dt}, gv{gate, dt};
    const Out o{out, dt};
    for (int64_t b = 0; b < B; ++b)
        for (int64_t t = 0; t < T; ++t) {
            const int64_t base = (b * T + t) * C;
            for (int64_t c = 0; c < C; ++c) {
                float v = xv.get(base + c);
                v = v * (1.0f + sc.get(b * C + c)) + sh.get(b * C + c);
                if (gate) v *= gv.get(b * C + c);
                if (residual) v += rv.get(base + c);
                o.set(base + c, v);
            }
        }
}

void activation_impl(const void* x, void* out, int64_t n, int kind, const void* gate, int dt) {
    const View xv{x, dt}, gv{gate, dt};
    const Out o{out, dt};
    for (int64_t i = 0; i < n; ++i) {
        float v = apply_epilogue(kind, xv.get(i));
        if (kind == BH_EPI_GELU_GATED) v *= gv.get(i);
        o.set(i, v);
    }
}

void add_impl(const void* a, const void* b, void* out, int64_t outer, int64_t inner, float scale,
              bool broadcast, int dt) {
    const View av{a, dt}, bv{b, dt};
    const Out o{out, dt};
    for (int64_t r = 0; r < outer; ++r)
        for (int64_t i = 0; i < inner; ++i) {
            const int64_t at = r * inner + i;
            o.set(at, av.get(at) + scale * bv.get(broadcast ? i : at));
        }
}

void chunk_impl(const void* mod, const void* table, void* out, int64_t B, int64_t C,
                int64_t chunks, int64_t chunk, int64_t table_chunk, int dt) {
    const View mv{mod, dt}, tv{table, dt};
    const Out o{out, dt};
    const int64_t trow = table_chunk >= 0 ? table_chunk : chunk;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < C; ++c)
            o.set(b * C + c, mv.get(b * chunks * C + chunk * C + c) + tv.get(trow * C + c));
}

void patch_impl(const void* in, void* out, int64_t B, int64_t C, int64_t G, int64_t P,
                bool inverse, int dt) {
    const View iv{in, dt};
    const Out o{out, dt};
    const int64_t H = G * P, per_token = C * P * P;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t ty = 0; ty < G; ++ty)
            for (int64_t tx = 0; tx < G; ++tx)
                for (int64_t c = 0; c < C; ++c)
                    for (int64_t ky = 0; ky < P; ++ky)
                        for (int64_t kx = 0; kx < P; ++kx) {
                            const int64_t img = ((b * C + c) * H + ty * P + ky) * H + tx * P + kx;
                            const int64_t tok = (b * G * G + ty * G + tx) * per_token +
                                                (inverse ? ((ky * P + kx) * C + c)
                                                         : ((c * P + ky) * P + kx));
                            if (inverse) o.set(img, iv.get(tok));
                            else o.set(tok, iv.get(img));
                        }
}

// ---- embeddings (pixart_dit.cpp:32-77, weights.cpp:107-121) ---------------------------------

void sincos_1d(int dim, const std::vector<double>& pos, std::vector<double>* out) {
    const int half = dim / 2;
    out->assign(pos.size() * dim, 0.0);
    std::vector<double> omega(half);
    for (int i = 0; i < half; ++i) omega[i] = 1.0 / std::pow(10000.0, static_cast<double>(i) / half);
    for (size_t m = 0; m < pos.size(); ++m)
        for (int i = 0; i < half; ++i) {
            const double a = pos[m] * omega[i];
            (*out)[m * dim + i] = std::sin(a);
            (*out)[m * dim + half + i] = std::cos(a);
        }
}

std::vector<double> position_embedding(int dim, int grid, int base, double interp) {
    std::vector<double> axis(grid);
    for (int i = 0; i < grid; ++i)
        axis[i] = static_cast<double>(i) / (static_cast<double>(grid) / base) / interp;
    std::vector<double> first(static_cast<size_t>(grid) * grid), second(first.size());
    for (int r = 0; r < grid; ++r)
        for (int c = 0; c < grid; ++c) {
            first[r * grid + c] = axis[c];
            second[r * grid + c] = axis[r];
        }
    std::vector<double> a, b;
    sincos_1d(dim / 2, first, &a);
    sincos_1d(dim / 2, second, &b);
    std::vector<double> out(static_cast<size_t>(grid) * grid * dim);
    const int half = dim / 2;
    for (int m = 0; m < grid * grid; ++m) {
        for (int i = 0; i < half; ++i) out[m * dim + i] = a[m * half + i];
        for (int i = 0; i < half; ++i) out[m * dim + half + i] = b[m * half + i];
    }
    return out;
}

void timestep_embedding(double t, int dim, float* out) {
    const int half = dim / 2;
    for (int i = 0; i < half; ++i) {
        const double freq = std::exp(-std::log(10000.0) * static_cast<double>(i) / half);
        const double a = t * freq;
        out[i] = static_cast<float>(std::cos(a));
        out[half + i] = static_cast<float>(std::sin(a));
    }
}

// ---- the DiT graph (pixart_dit.cpp:112-304) -------------------------------------------------

struct Buf {
    std::vector<uint16_t> v;
    explicit Buf(int64_t n = 0) : v(static_cast<size_t>(n), 0) {}
    void* p() { return v.data(); }
};

void dit_forward(const bh_dit_config& c, const bh_dit_weights& w, int64_t B, int64_t Hl,
                 int64_t cap_len, const uint16_t* latent, double t, const uint16_t* caption,
                 const void* mask, int mask_dt, uint16_t* image, int threads, int layers) {
    const int BF = BH_BF16;
    const int64_t P = c.patch_size, grid = Hl / P, N = grid * grid, M = B * N;
    const int64_t d = static_cast<int64_t>(c.num_heads) * c.head_dim;
    const int64_t dff = static_cast<int64_t>(static_cast<double>(d) * c.mlp_ratio);
    const int64_t Mcap = B * cap_len, pin = c.in_channels * P * P, pout = c.out_channels * P * P;
    const float eps = static_cast<float>(c.eps);
    auto gemm = [&](const void* a, const void* wt, const void* bias, void* out, int64_t m,
                    int64_t n, int64_t k, int epi) {
        gemm_impl(a, wt, bias, out, m, n, k, true, epi, BF, threads);
    };

    Buf patches(M * pin), x(M * d);
    patch_impl(latent, patches.p(), B, c.in_channels, grid, P, false, BF);
    gemm(patches.p(), w.pos_embed_w, w.pos_embed_b, x.p(), M, d, pin, BH_EPI_NONE);
    {
        const std::vector<double> pe =
            position_embedding(static_cast<int>(d), static_cast<int>(grid), c.sample_size / c.patch_size, 2.0);
        Buf pos(N * d);
        for (int64_t i = 0; i < N * d; ++i) pos.v[i] = f32_to_bf16(static_cast<float>(pe[i]));
        add_impl(x.p(), pos.p(), x.p(), B, N * d, 1.0f, true, BF);
    }

    Buf emb_t(B * d), modulation(B * 6 * d);
    {
        float proj[256];
        timestep_embedding(t, 256, proj);
        Buf broad(B * 256), h(B * d), s(B * d);
        for (int64_t b = 0; b < B; ++b)
            for (int i = 0; i < 256; ++i) broad.v[b * 256 + i] = f32_to_bf16(proj[i]);
        gemm(broad.p(), w.t_emb1_w, w.t_emb1_b, h.p(), B, d, 256, BH_EPI_SILU);
        gemm(h.p(), w.t_emb2_w, w.t_emb2_b, emb_t.p(), B, d, d, BH_EPI_NONE);
        activation_impl(emb_t.p(), s.p(), B * d, BH_EPI_SILU, nullptr, BF);
        gemm(s.p(), w.adaln_w, w.adaln_b, modulation.p(), B, 6 * d, d, BH_EPI_NONE);
    }
    Buf cap(Mcap * d);
    {
        Buf h(Mcap * d);
        gemm(caption, w.cap1_w, w.cap1_b, h.p(), Mcap, d, c.caption_channels, BH_EPI_GELU);
        gemm(h.p(), w.cap2_w, w.cap2_b, cap.p(), Mcap, d, d, BH_EPI_NONE);
    }

    Buf normed(M * d), modded(M * d), q(M * d), k(M * d), v(M * d), kc(Mcap * d), vc(Mcap * d),
        ctx(M * d), proj(M * d), ff0(M * dff), shift(B * d), scale(B * d), gate(B * d), zero(B * d);
    const AttnGeom self{B, c.num_heads, N, N, c.head_dim, d, d, d};
    const AttnGeom cross{B, c.num_heads, N, cap_len, c.head_dim, d, d, d};
    const int nl = layers >= 0 ? std::min(layers, c.num_layers) : c.num_layers;
    for (int l = 0; l < nl; ++l) {
        const bh_dit_block_weights& bw = w.blocks[l];
        const void* table = bw.scale_shift_table;
        norm_impl(x.p(), nullptr, nullptr, normed.p(), M, d, eps, false, BF, threads);
        chunk_impl(modulation.p(), table, shift.p(), B, d, 6, 0, 0, BF);
        chunk_impl(modulation.p(), table, scale.p(), B, d, 6, 1, 1, BF);
        chunk_impl(modulation.p(), table, gate.p(), B, d, 6, 2, 2, BF);
        modulate_impl(normed.p(), scale.p(), shift.p(), modded.p(), B, N, d, nullptr, nullptr, BF);
        gemm(modded.p(), bw.attn1_q_w, bw.attn1_q_b, q.p(), M, d, d, BH_EPI_NONE);
        gemm(modded.p(), bw.attn1_k_w, bw.attn1_k_b, k.p(), M, d, d, BH_EPI_NONE);
        gemm(modded.p(), bw.attn1_v_w, bw.attn1_v_b, v.p(), M, d, d, BH_EPI_NONE);
        attention_impl(q.p(), k.p(), v.p(), ctx.p(), self, 0.0f, nullptr, nullptr, BF, BF, threads,
                       false);
        gemm(ctx.p(), bw.attn1_o_w, bw.attn1_o_b, proj.p(), M, d, d, BH_EPI_NONE);
        modulate_impl(proj.p(), zero.p(), zero.p(), x.p(), B, N, d, x.p(), gate.p(), BF);

        gemm(x.p(), bw.attn2_q_w, bw.attn2_q_b, q.p(), M, d, d, BH_EPI_NONE);
        gemm(cap.p(), bw.attn2_k_w, bw.attn2_k_b, kc.p(), Mcap, d, d, BH_EPI_NONE);
        gemm(cap.p(), bw.attn2_v_w, bw.attn2_v_b, vc.p(), Mcap, d, d, BH_EPI_NONE);
        attention_impl(q.p(), kc.p(), vc.p(), ctx.p(), cross, 0.0f, nullptr, mask, mask_dt, BF,
                       threads, false);
        gemm(ctx.p(), bw.attn2_o_w, bw.attn2_o_b, proj.p(), M, d, d, BH_EPI_NONE);
        add_impl(x.p(), proj.p(), x.p(), M, d, 1.0f, false, BF);

        norm_impl(x.p(), nullptr, nullptr, normed.p(), M, d, eps, false, BF, threads);
        chunk_impl(modulation.p(), table, shift.p(), B, d, 6, 3, 3, BF);
        chunk_impl(modulation.p(), table, scale.p(), B, d, 6, 4, 4, BF);
        chunk_impl(modulation.p(), table, gate.p(), B, d, 6, 5, 5, BF);
        modulate_impl(normed.p(), scale.p(), shift.p(), modded.p(), B, N, d, nullptr, nullptr, BF);
        gemm(modded.p(), bw.ff0_w, bw.ff0_b, ff0.p(), M, dff, d, BH_EPI_GELU);
        gemm(ff0.p(), bw.ff2_w, bw.ff2_b, proj.p(), M, d, dff, BH_EPI_NONE);
        modulate_impl(proj.p(), zero.p(), zero.p(), x.p(), B, N, d, x.p(), gate.p(), BF);
    }

    chunk_impl(emb_t.p(), w.out_table, shift.p(), B, d, 1, 0, 0, BF);
    chunk_impl(emb_t.p(), w.out_table, scale.p(), B, d, 1, 0, 1, BF);
    norm_impl(x.p(), nullptr, nullptr, normed.p(), M, d, eps, false, BF, threads);
    modulate_impl(normed.p(), scale.p(), shift.p(), modded.p(), B, N, d, nullptr, nullptr, BF);
    Buf tokens(M * pout);
    gemm(modded.p(), w.proj_out_w, w.proj_out_b, tokens.p(), M, pout, d, BH_EPI_NONE);
    patch_impl(tokens.p(), image, B, c.out_channels, grid, P, true, BF);
}

// ---- ScaleArgs (ops_cpu.cpp:351-353): one multiply per element, one rounding -------------------

void scale_impl(const void* in, void* out, int64_t n, float scale, int dt) {
    View x{in, dt};
    Out y{out, dt};
    for (int64_t i = 0; i < n; ++i) y.set(i, x.get(i) * scale);
}

// ---- the denoise loop's two ops (ops_cpu.cpp:355-369) -----------------------------------------

void repeat_impl(const void* in, void* out, int64_t outer, int64_t inner, int dt) {
    View x{in, dt};
    Out y{out, dt};
    for (int64_t r = 0; r < outer; ++r)
        for (int64_t i = 0; i < inner; ++i) y.set(r * inner + i, x.get(i));
}

// u + scale*(c - u) in double, one rounding to float, then the store (ops_cpu.cpp:361-369).
void guidance_impl(const void* pred, void* out, int64_t out_channels, int64_t channels,
                   int64_t spatial, float scale, int dt) {
    View p{pred, dt};
    Out y{out, dt};
    for (int64_t ch = 0; ch < channels; ++ch)
        for (int64_t s = 0; s < spatial; ++s) {
            const double u = p.get(ch * spatial + s);
            const double c = p.get((out_channels + ch) * spatial + s);
            y.set(ch * spatial + s, static_cast<float>(u + scale * (c - u)));
        }
}

// ---- the sampler: DPM-Solver++ 2M, midpoint, epsilon (src/sched/dpm_solver.cpp) -------------

struct Sampler {
    int train_steps = 1000;
    int order_cap = 2;          // solver_order
    bool lower_final = true;    // lower_order_final
    bool spacing_ok = true;     // timestep_spacing == "linspace", checked by set_timesteps
    std::vector<double> karras; // sqrt((1 - acp) / acp) per training timestep
    std::vector<int64_t> ts;    // the inference timesteps
    std::vector<double> sig;    // karras sigma per inference step, then a final 0
    std::vector<std::vector<float>> x0s;  // stored x0 predictions, oldest first
    int warm = 0;               // lower_order_nums_: steps taken, capped at solver_order
};

bool same(const char* a, const char* b) { return a && std::strcmp(a, b) == 0; }

// The constructor (dpm_solver.cpp:19-53): cumulative product of (1 - beta) in double over the
// training schedule, beta linear in t, or linear in sqrt(beta) for "scaled_linear".
void sampler_init(Sampler& s, const bh_sched_config& c) {
    if (!same(c.algorithm_type, "dpmsolver++"))
        throw std::runtime_error("scheduler: only dpmsolver++ is implemented");
    if (!same(c.solver_type, "midpoint"))
        throw std::runtime_error("scheduler: only the midpoint solver type is implemented");
    if (!same(c.prediction_type, "epsilon"))
        throw std::runtime_error("scheduler: only epsilon prediction is implemented");
    if (c.num_train_timesteps < 2) throw std::runtime_error("scheduler: num_train_timesteps < 2");
    if (c.solver_order < 1) throw std::runtime_error("scheduler: solver_order < 1");
    const bool scaled = same(c.beta_schedule, "scaled_linear");
    if (!scaled && !same(c.beta_schedule, "linear"))
        throw std::runtime_error("scheduler: unsupported beta_schedule");
    s.train_steps = c.num_train_timesteps;
    s.order_cap = c.solver_order;
    s.lower_final = c.lower_order_final != 0;
    s.spacing_ok = same(c.timestep_spacing, "linspace");
    s.karras.assign(static_cast<size_t>(s.train_steps), 0.0);
    double acp = 1.0;
    const double lo = scaled ? std::sqrt(c.beta_start) : c.beta_start;
    const double hi = scaled ? std::sqrt(c.beta_end) : c.beta_end;
    for (int t = 0; t < s.train_steps; ++t) {
        const double f = lo + (hi - lo) * (static_cast<double>(t) / (s.train_steps - 1));
        acp *= 1.0 - (scaled ? f * f : f);
        s.karras[static_cast<size_t>(t)] = std::sqrt((1.0 - acp) / acp);
    }
}

// set_timesteps (dpm_solver.cpp:55-75): step j of `steps` sits at round(j * (N-1) / steps) for
// j = steps..1 (linspace over [0, N-1] with steps+1 points, reversed, the 0 dropped).
void sampler_set_timesteps(Sampler& s, int steps) {
    if (steps < 1) throw std::runtime_error("scheduler: at least one step");
    if (!s.spacing_ok) throw std::runtime_error("scheduler: only linspace spacing is implemented");
    s.ts.clear();
    s.sig.clear();
    for (int j = steps; j >= 1; --j) {
        const double at = static_cast<double>(j) * (s.train_steps - 1) / static_cast<double>(steps);
        s.ts.push_back(static_cast<int64_t>(std::llround(at)));
        s.sig.push_back(s.karras[static_cast<size_t>(s.ts.back())]);
    }
    s.sig.push_back(0.0);
    s.x0s.clear();
    s.warm = 0;
}

// Karras sigma -> (alpha, sigma) of the variance-preserving form (dpm_solver.cpp:10-16).
void vp_of(double k, double* alpha, double* sigma) {
    const double r = std::sqrt(k * k + 1.0);
    *alpha = 1.0 / r;
    *sigma = k / r;
}

// coefficients(i) (dpm_solver.cpp:100-123).
bh_sched_coefficients sampler_coefficients(const Sampler& s, int i) {
    if (i < 0 || static_cast<size_t>(i) + 1 >= s.sig.size())
        throw std::runtime_error("scheduler: step index out of range");
    const size_t at = static_cast<size_t>(i);
    bh_sched_coefficients c{};
    c.sigma_s0 = s.sig[at];
    c.sigma_t = s.sig[at + 1];
    vp_of(c.sigma_t, &c.alpha_t, &c.sigma_vp_t);
    vp_of(c.sigma_s0, &c.alpha_s0, &c.sigma_vp_s0);
    c.exp_neg_h = c.sigma_s0 > 0.0 ? c.sigma_t / c.sigma_s0 : 0.0;
    const bool final_step = at + 2 == s.sig.size();
    const bool second = s.warm >= 1 && !(s.lower_final && final_step) && s.order_cap >= 2;
    c.order = second ? 2 : 1;
    if (second) {
        if (at == 0) throw std::runtime_error("scheduler: a second-order step needs step i-1");
        const double h = std::log(c.sigma_s0 / c.sigma_t);
        const double h0 = std::log(s.sig[at - 1] / c.sigma_s0);
        c.r0 = h0 / h;
    }
    return c;
}

// step (dpm_solver.cpp:89-98, 125-162) on a host sample of n elements. x0 is stored through the
// sample's dtype before it is used, as the reference keeps it in a tensor of that dtype.
void sampler_step(Sampler& s, const void* eps, int i, void* sample, int64_t n, int dt) {
    if (i < 0 || static_cast<size_t>(i) >= s.ts.size())
        throw std::runtime_error("scheduler: step index out of range");
    double alpha_s, sigma_s;
    vp_of(s.sig[static_cast<size_t>(i)], &alpha_s, &sigma_s);
    View e{eps, dt}, x{sample, dt};
    std::vector<float> x0(static_cast<size_t>(n));
    for (int64_t k = 0; k < n; ++k)
        x0[k] = stored(static_cast<float>((x.get(k) - sigma_s * e.get(k)) / alpha_s), dt);
    s.x0s.push_back(std::move(x0));
    if (static_cast<int>(s.x0s.size()) > s.order_cap) s.x0s.erase(s.x0s.begin());
    const bh_sched_coefficients c = sampler_coefficients(s, i);
    const std::vector<float>& m0 = s.x0s.back();
    const double ratio = c.sigma_vp_s0 > 0.0 ? c.sigma_vp_t / c.sigma_vp_s0 : 0.0;
    const double coef = c.alpha_t * (c.exp_neg_h - 1.0);
    Out y{sample, dt};
    if (c.order == 1) {
        for (int64_t k = 0; k < n; ++k)
            y.set(k, static_cast<float>(ratio * static_cast<double>(x.get(k)) - coef * m0[k]));
    } else {
        const std::vector<float>& m1 = s.x0s[s.x0s.size() - 2];
        for (int64_t k = 0; k < n; ++k) {
            const double d0 = m0[k];
            const double d1 = (1.0 / c.r0) * (d0 - m1[k]);
            y.set(k, static_cast<float>(ratio * static_cast<double>(x.get(k)) - coef * d0 -
                                        0.5 * coef * d1));
        }
    }
    if (s.warm < s.order_cap) ++s.warm;
}

// ---- the VAE decoder's ops (ops_cpu.cpp:186-224, 276-300, 384-412) -----------------------------

// GroupNorm (ops_cpu.cpp:186-224): rows = batch, cols = channels * spatial (NCHW), the group split
// over channels: per (row, group) an fp64 mean, then an fp64 sum of squared deviations, inv =
// 1/sqrt(float(var) + eps), (x - float(mean)) * inv, then * weight[channel], + bias[channel].
void group_norm_impl(const void* x, const void* w, const void* bias, void* out, int64_t rows,
                     int64_t cols, float eps, int64_t groups, int64_t channels, int dt,
                     int threads) {
    const int64_t per_group = cols / groups;
    if (channels && (channels % groups)) throw std::runtime_error("groupnorm: channels not divisible by groups");
    if (per_group * groups != cols) throw std::runtime_error("groupnorm: channels*spatial not divisible by groups");
    const View xv{x, dt}, wv{w, dt}, bv{bias, dt};
    const Out o{out, dt};
    const int64_t spatial = channels ? cols / channels : 1;
    parallel_for(rows * groups, threads, [&](int64_t rg) {
        const int64_t r = rg / groups, g = rg - r * groups;
        const int64_t base = r * cols + g * per_group;
        double mean = 0.0;
        for (int64_t i = 0; i < per_group; ++i) mean += xv.get(base + i);
        mean /= per_group;
        double var = 0.0;
        for (int64_t i = 0; i < per_group; ++i) {
            double d = xv.get(base + i) - mean;
            var += d * d;
        }
        var /= per_group;
        const float inv = 1.0f / std::sqrt(static_cast<float>(var) + eps);
        for (int64_t i = 0; i < per_group; ++i) {
            float v = (xv.get(base + i) - static_cast<float>(mean)) * inv;
            if (w || bias) {
                const int64_t ch = (g * per_group + i) / spatial;
                if (w) v *= wv.get(ch);
                if (bias) v += bv.get(ch);
            }
            o.set(base + i, v);
        }
    });
}

// conv2d (ops_cpu.cpp:276-300), NCHW, stride 1: acc starts at the bias, then ic, ky, kx in that
// order, taps outside the input skipped, one fp32 product and add each. Vectorised across ox
// (independent outputs); every output sees the same sequence of operations.
void conv2d_impl(const void* x, const void* w, const void* bias, void* out, int64_t B,
                 int64_t ci, int64_t H, int64_t W, int64_t co, int64_t k, int64_t pad, int dt,
                 int threads) {
    const int64_t Ho = H + 2 * pad - k + 1, Wo = W + 2 * pad - k + 1;
    const std::vector<float> xf = widen(x, dt, B * ci * H * W);
    const std::vector<float> wf = widen(w, dt, co * ci * k * k);
    const View bv{bias, dt};
    const Out o{out, dt};
    parallel_for(B * co * Ho, threads, [&](int64_t row) {
        const int64_t oy = row % Ho, oc = (row / Ho) % co, b = row / (Ho * co);
        std::vector<float> acc(static_cast<size_t>(Wo), bias ? bv.get(oc) : 0.0f);
        for (int64_t ic = 0; ic < ci; ++ic)
            for (int64_t ky = 0; ky < k; ++ky) {
                const int64_t iy = oy + ky - pad;
                if (iy < 0 || iy >= H) continue;
                const float* xr = &xf[static_cast<size_t>(((b * ci + ic) * H + iy) * W)];
                for (int64_t kx = 0; kx < k; ++kx) {
                    const float wt = wf[static_cast<size_t>(((oc * ci + ic) * k + ky) * k + kx)];
                    const int64_t lo = std::max<int64_t>(0, pad - kx), hi = std::min<int64_t>(Wo, W + pad - kx);
                    for (int64_t ox = lo; ox < hi; ++ox) acc[ox] += xr[ox + kx - pad] * wt;
                }
            }
        for (int64_t ox = 0; ox < Wo; ++ox) o.set(((b * co + oc) * Ho + oy) * Wo + ox, acc[ox]);
    });
}

// Nearest upsample (ops_cpu.cpp:384-397) and the [C, S] <-> [S, C] transpose (:399-412): copies.
void upsample_impl(const void* in, void* out, int64_t B, int64_t C, int64_t H, int64_t W,
                   int64_t f, int dt) {
    const int64_t es = dt == BH_F32 ? 4 : 2, H2 = H * f, W2 = W * f;
    const char* src = static_cast<const char*>(in);
    char* dst = static_cast<char*>(out);
    for (int64_t bc = 0; bc < B * C; ++bc)
        for (int64_t y = 0; y < H2; ++y)
            for (int64_t x = 0; x < W2; ++x)
                std::memcpy(dst + ((bc * H2 + y) * W2 + x) * es, src + ((bc * H + y / f) * W + x / f) * es, es);
}

void transpose_impl(const void* in, void* out, int64_t B, int64_t C, int64_t S, bool to_cf, int dt) {
    const int64_t es = dt == BH_F32 ? 4 : 2;
    const char* src = static_cast<const char*>(in);
    char* dst = static_cast<char*>(out);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < C; ++c)
            for (int64_t s = 0; s < S; ++s) {
                const int64_t cf = (b * C + c) * S + s, sf = (b * S + s) * C + c;
                if (to_cf) std::memcpy(dst + cf * es, src + sf * es, es);
                else std::memcpy(dst + sf * es, src + cf * es, es);
            }
}

// ---- the VAE decoder graph (vae_decoder.cpp:127-180), NCHW, batch 1 ----------------------------

struct VaeTable {
    std::vector<std::pair<std::string, const void*>> t;
    const void* at(const std::string& n) const {
        for (const auto& kv : t)
            if (kv.first == n) return kv.second;
        throw std::runtime_error("vae weights: '" + n + "' is missing");
    }
};

struct VaeRun {
    const VaeTable& w;
    double eps;
    int64_t groups;
    int threads;
    using Buf = std::vector<uint16_t>;

    Buf conv(const Buf& x, const std::string& n, int64_t ci, int64_t co, int64_t h, int64_t k,
             int64_t pad) const {
        const int64_t ho = h + 2 * pad - k + 1;
        Buf out(static_cast<size_t>(co * ho * ho));
        conv2d_impl(x.data(), w.at(n + ".weight"), w.at(n + ".bias"), out.data(), 1, ci, h, h, co,
                    k, pad, BH_BF16, threads);
        return out;
    }
    Buf gn(const Buf& x, const std::string& n, int64_t ch, int64_t h) const {
        Buf out(x.size());
        group_norm_impl(x.data(), w.at(n + ".weight"), w.at(n + ".bias"), out.data(), 1, ch * h * h,
                        static_cast<float>(eps), groups, ch, BH_BF16, threads);
        return out;
    }
    Buf silu(const Buf& x) const {
        Buf out(x.size());
        activation_impl(x.data(), out.data(), static_cast<int64_t>(x.size()), BH_EPI_SILU, nullptr, BH_BF16);
        return out;
    }
    Buf add(const Buf& a, const Buf& b) const {
        Buf out(a.size());
        add_impl(a.data(), b.data(), out.data(), 1, static_cast<int64_t>(a.size()), 1.0f, false, BH_BF16);
        return out;
    }
    Buf resnet(const Buf& x, const std::string& n, int64_t ci, int64_t co, int64_t h) const {
        Buf t = silu(gn(x, n + ".norm1", ci, h));
        t = conv(t, n + ".conv1", ci, co, h, 3, 1);
        t = silu(gn(t, n + ".norm2", co, h));
        t = conv(t, n + ".conv2", co, co, h, 3, 1);
        const Buf skip = ci != co ? conv(x, n + ".conv_shortcut", ci, co, h, 1, 0) : x;
        return add(skip, t);
    }
    Buf attention(const Buf& x, const std::string& n, int64_t ch, int64_t h) const {
        const int64_t s = h * h;
        const Buf normed = gn(x, n + ".group_norm", ch, h);
        Buf seq(static_cast<size_t>(s * ch));
        transpose_impl(normed.data(), seq.data(), 1, ch, s, false, BH_BF16);
        Buf q(seq.size()), k(seq.size()), v(seq.size()), o(seq.size()), proj(seq.size());
        const std::pair<const char*, Buf*> qkv[3] = {{"to_q", &q}, {"to_k", &k}, {"to_v", &v}};
        for (const auto& pr : qkv)
            gemm_impl(seq.data(), w.at(n + "." + pr.first + ".weight"), w.at(n + "." + pr.first + ".bias"),
                      pr.second->data(), s, ch, ch, true, BH_EPI_NONE, BH_BF16, threads);
        attention_impl(q.data(), k.data(), v.data(), o.data(), AttnGeom{1, 1, s, s, ch, ch, ch, ch}, 0.0f,
                       nullptr, nullptr, BH_F32, BH_BF16, threads, false);
        gemm_impl(o.data(), w.at(n + ".to_out.0.weight"), w.at(n + ".to_out.0.bias"), proj.data(), s,
                  ch, ch, true, BH_EPI_NONE, BH_BF16, threads);
        Buf back(seq.size());
        transpose_impl(proj.data(), back.data(), 1, ch, s, true, BH_BF16);
        return add(x, back);
    }
    Buf upsample(const Buf& x, int64_t ch, int64_t h) const {
        Buf out(x.size() * 4);
        upsample_impl(x.data(), out.data(), 1, ch, h, h, 2, BH_BF16);
        return out;
    }
};

void vae_forward(const bh_vae_config& c, const VaeTable& w, const uint16_t* latent, int64_t h,
                 uint16_t* image, int threads, int stop_after) {
    VaeRun r{w, c.eps, c.norm_num_groups, threads};
    std::vector<int64_t> rev;
    for (int i = c.num_blocks - 1; i >= 0; --i) rev.push_back(c.block_out_channels[i]);
    const int64_t zc = c.latent_channels;
    VaeRun::Buf x(latent, latent + zc * h * h);
    x = r.conv(x, "post_quant_conv", zc, zc, h, 1, 0);
    x = r.conv(x, "decoder.conv_in", zc, rev[0], h, 3, 1);
    x = r.resnet(x, "decoder.mid_block.resnets.0", rev[0], rev[0], h);
    x = r.attention(x, "decoder.mid_block.attentions.0", rev[0], h);
    x = r.resnet(x, "decoder.mid_block.resnets.1", rev[0], rev[0], h);
    int64_t prev = rev[0];
    for (size_t i = 0; i < rev.size(); ++i) {
        if (stop_after >= 0 && static_cast<int>(i) >= stop_after) break;
        const int64_t co = rev[i];
        for (int j = 0; j <= c.layers_per_block; ++j)
            x = r.resnet(x, "decoder.up_blocks." + std::to_string(i) + ".resnets." + std::to_string(j),
                         j == 0 ? prev : co, co, h);
        prev = co;
        if (i + 1 != rev.size()) {
            x = r.upsample(x, co, h);
            h *= 2;
            x = r.conv(x, "decoder.up_blocks." + std::to_string(i) + ".upsamplers.0.conv", co, co, h, 3, 1);
        }
    }
    if (stop_after >= 0) {   // a truncated decoder returns the activation where it stopped
        std::memcpy(image, x.data(), x.size() * 2);
        return;
    }
    x = r.silu(r.gn(x, "decoder.conv_norm_out", prev, h));
    x = r.conv(x, "decoder.conv_out", prev, 3, h, 3, 1);
    std::memcpy(image, x.data(), x.size() * 2);
}

VaeTable vae_table(const bh_vae_weights& w) {
    VaeTable t;
    for (int i = 0; i < w.count; ++i) t.t.emplace_back(w.names[i], w.tensors[i]);
    return t;
}

// ---- the T5 v1.1 encoder (t5_encoder.cpp:132-241), rows [batch * seq, d_model] ------------

// t5_relative_bucket (t5_encoder.cpp:34-48): half the buckets for keys before the query (or at
// it), half for keys after; distances below a quarter of the buckets are exact, the rest are
// log-spaced up to max_distance and saturate at the last bucket of the half.
int t5_bucket(int rp, int num_buckets, int max_distance) {
    const int half = num_buckets / 2;
    const int side = rp > 0 ? half : 0;
    const int n = rp < 0 ? -rp : rp;
    const int exact = half / 2;
    if (n < exact) return side + n;
    const double frac = std::log(static_cast<double>(n) / exact) /
                        std::log(static_cast<double>(max_distance) / exact) * (half - exact);
    const int large = std::min(exact + static_cast<int>(frac), half - 1);
    return side + large;
}

// The encoder (t5_encoder.cpp:132-241): embedding rows of the ids (checked against the
// vocabulary first, :146-156); a [heads, S, S] bias from the bucket of k - q (:63-120); a key
// mask of id != 0 (:180-184); per layer RMSNorm, q/k/v projections, attention with scale 1,
// the bias and the mask, the output projection and a residual add; RMSNorm, the gated-GELU
// FFN and a residual add; a final RMSNorm. Every intermediate is a bf16 tensor, as there.
void t5_forward(const bh_t5_config& c, const VaeTable& w, const float* ids, int64_t B, int64_t S,
                uint16_t* out, int threads) {
    using Buf = std::vector<uint16_t>;
    const int64_t d = c.d_model, H = c.num_heads, inner = H * c.d_kv, M = B * S, F = c.d_ff;
    for (int64_t i = 0; i < M; ++i) {
        const int64_t id = static_cast<int64_t>(ids[i]);
        if (id < 0 || id >= c.vocab_size)
            throw std::runtime_error("t5: token id " + std::to_string(id) + " is outside the vocabulary");
    }
    const auto* table = static_cast<const uint16_t*>(w.at("shared.weight"));
    Buf x(static_cast<size_t>(M * d));
    for (int64_t i = 0; i < M; ++i)
        std::memcpy(&x[i * d], table + static_cast<int64_t>(ids[i]) * d, static_cast<size_t>(d) * 2);
    const auto* rel = static_cast<const uint16_t*>(
        w.at("encoder.block.0.layer.0.SelfAttention.relative_attention_bias.weight"));
    Buf bias(static_cast<size_t>(H * S * S));
    for (int64_t q = 0; q < S; ++q)
        for (int64_t k = 0; k < S; ++k) {
            const int bk = t5_bucket(static_cast<int>(k - q), c.num_buckets, 128);
            for (int64_t h = 0; h < H; ++h) bias[(h * S + q) * S + k] = rel[bk * H + h];
        }
    Buf mask(static_cast<size_t>(M));
    for (int64_t i = 0; i < M; ++i) mask[i] = static_cast<int64_t>(ids[i]) == 0 ? 0 : 0x3f80;
    Buf normed(x.size()), q(static_cast<size_t>(M * inner)), k(q.size()), v(q.size()), ctx(q.size()),
        proj(x.size()), h0(static_cast<size_t>(M * F)), h1(h0.size()), hact(h0.size());
    const float eps = static_cast<float>(c.eps);
    auto blk = [](int i, const char* tail) { return "encoder.block." + std::to_string(i) + "." + tail; };
    auto gemm = [&](const Buf& a, const std::string& wn, Buf& o, int64_t n, int64_t kk) {
        gemm_impl(a.data(), w.at(wn), nullptr, o.data(), M, n, kk, true, BH_EPI_NONE, BH_BF16, threads);
    };
    for (int l = 0; l < c.num_layers; ++l) {
        norm_impl(x.data(), w.at(blk(l, "layer.0.layer_norm.weight")), nullptr, normed.data(), M, d, eps,
                  true, BH_BF16, threads);
        gemm(normed, blk(l, "layer.0.SelfAttention.q.weight"), q, inner, d);
        gemm(normed, blk(l, "layer.0.SelfAttention.k.weight"), k, inner, d);
        gemm(normed, blk(l, "layer.0.SelfAttention.v.weight"), v, inner, d);
        attention_impl(q.data(), k.data(), v.data(), ctx.data(),
                       AttnGeom{B, H, S, S, c.d_kv, inner, inner, inner}, 1.0f, bias.data(), mask.data(),
                       BH_BF16, BH_BF16, threads, false);
        gemm(ctx, blk(l, "layer.0.SelfAttention.o.weight"), proj, d, inner);
        add_impl(x.data(), proj.data(), x.data(), M, d, 1.0f, false, BH_BF16);
        norm_impl(x.data(), w.at(blk(l, "layer.1.layer_norm.weight")), nullptr, normed.data(), M, d, eps,
                  true, BH_BF16, threads);
        gemm(normed, blk(l, "layer.1.DenseReluDense.wi_0.weight"), h0, F, d);
        if (c.gated) {
            gemm(normed, blk(l, "layer.1.DenseReluDense.wi_1.weight"), h1, F, d);
            activation_impl(h0.data(), hact.data(), M * F, BH_EPI_GELU_GATED, h1.data(), BH_BF16);
        } else {
            activation_impl(h0.data(), hact.data(), M * F, BH_EPI_GELU, nullptr, BH_BF16);
        }
        gemm(hact, blk(l, "layer.1.DenseReluDense.wo.weight"), proj, d, F);
        add_impl(x.data(), proj.data(), x.data(), M, d, 1.0f, false, BH_BF16);
    }
    norm_impl(x.data(), w.at("encoder.final_layer_norm.weight"), nullptr, out, M, d, eps, true, BH_BF16,
              threads);
}

VaeTable name_table(int count, const char* const* names, const void* const* tensors) {
    VaeTable t;
    for (int i = 0; i < count; ++i) t.t.emplace_back(names[i], tensors[i]);
    return t;
}

thread_local std::string g_err;

template <typename Fn>
int guard(Fn fn) {
    try {
        fn();
        return 0;
    } catch (const std::exception& e) {
        g_err = e.what();
        return 1;
    }
}

}  // namespace

extern "C" {

const char* stock_last_error(void) { return g_err.c_str(); }

int stock_gemm(const void* a, const void* b, const void* bias, void* out, int64_t m, int64_t n,
               int64_t k, int b_transposed, int epilogue, int dtype, int threads) {
    return guard([&] {
        gemm_impl(a, b, bias, out, m, n, k, b_transposed != 0, epilogue, dtype,
                  resolve_threads(threads));
    });
}

int stock_attention(const void* q, const void* k, const void* v, void* out, int64_t batch,
                    int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                    const void* bias, const void* key_mask, int mask_dtype, int dtype,
                    int materialized, int threads) {
    return guard([&] {
        const int64_t ld = heads * head_dim;
        attention_impl(q, k, v, out, AttnGeom{batch, heads, q_len, kv_len, head_dim, ld, ld, ld},
                       scale, bias, key_mask, mask_dtype, dtype, resolve_threads(threads),
                       materialized != 0);
    });
}

int stock_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
               int64_t cols, float eps, int rms, int dtype, int threads) {
    return guard([&] {
        norm_impl(x, weight, bias, out, rows, cols, eps, rms != 0, dtype, resolve_threads(threads));
    });
}

int stock_modulate(const void* x, const void* scale, const void* shift, void* out, int64_t batch,
                   int64_t tokens, int64_t channels, const void* residual, const void* gate,
                   int dtype) {
    return guard([&] {
        modulate_impl(x, scale, shift, out, batch, tokens, channels, residual, gate, dtype);
    });
}

int stock_activation(const void* x, void* out, int64_t n, int kind, const void* gate, int dtype) {
    return guard([&] { activation_impl(x, out, n, kind, gate, dtype); });
}

int stock_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner, float scale,
              int broadcast_b, int dtype) {
    return guard([&] { add_impl(a, b, out, outer, inner, scale, broadcast_b != 0, dtype); });
}

int stock_chunk(const void* mod, const void* table, void* out, int64_t batch, int64_t channels,
                int64_t chunks, int64_t chunk, int64_t table_chunk, int dtype) {
    return guard([&] { chunk_impl(mod, table, out, batch, channels, chunks, chunk, table_chunk, dtype); });
}

int stock_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
                int64_t patch, int inverse, int dtype) {
    return guard([&] { patch_impl(in, out, batch, channels, grid, patch, inverse != 0, dtype); });
}

int stock_position_embedding(double* out, int dim, int grid, int base, double interp) {
    return guard([&] {
        const std::vector<double> pe = position_embedding(dim, grid, base, interp);
        std::copy(pe.begin(), pe.end(), out);
    });
}

int stock_timestep_embedding(double t, int dim, float* out) {
    return guard([&] {
        if (dim % 2) throw std::runtime_error("timestep embedding needs an even dimension");
        timestep_embedding(t, dim, out);
    });
}

// `layers` < 0 runs every block; otherwise the first `layers` blocks (the reference's
// `dit-step --layers`, burnisher_main.cpp:704-707).
int stock_dit_forward(const bh_dit_config* cfg, const bh_dit_weights* w, int64_t batch,
                      int64_t latent_hw, int64_t caption_len, const uint16_t* latent,
                      double timestep, const uint16_t* caption, const void* mask, int mask_dtype,
                      uint16_t* image, int threads, int layers) {
    return guard([&] {
        if (!cfg || !w) throw std::runtime_error("stock_dit_forward: null argument");
        dit_forward(*cfg, *w, batch, latent_hw, caption_len, latent, timestep, caption, mask,
                    mask_dtype, image, resolve_threads(threads), layers);
    });
}


int stock_scale(const void* in, void* out, int64_t numel, float scale, int dtype) {
    return guard([&] { scale_impl(in, out, numel, scale, dtype); });
}

int stock_repeat(const void* in, void* out, int64_t outer, int64_t inner, int dtype) {
    return guard([&] { repeat_impl(in, out, outer, inner, dtype); });
}

int stock_guidance(const void* pred, void* out, int64_t out_channels, int64_t channels,
                   int64_t spatial, float scale, int dtype) {
    return guard([&] {
        if (channels > out_channels) throw std::runtime_error("guidance: channels > out_channels");
        guidance_impl(pred, out, out_channels, channels, spatial, scale, dtype);
    });
}

// The sampler behind an opaque handle (host buffers only).
int stock_sched_create(const bh_sched_config* cfg, void** out) {
    return guard([&] {
        if (!cfg || !out) throw std::runtime_error("stock_sched_create: null argument");
        auto* s = new Sampler();
        try {
            sampler_init(*s, *cfg);
        } catch (...) {
            delete s;
            throw;
        }
        *out = s;
    });
}

void stock_sched_destroy(void* h) { delete static_cast<Sampler*>(h); }

int stock_sched_set_timesteps(void* h, int steps) {
    return guard([&] { sampler_set_timesteps(*static_cast<Sampler*>(h), steps); });
}

int stock_sched_steps(const void* h) { return static_cast<int>(static_cast<const Sampler*>(h)->ts.size()); }

int stock_sched_timestep(const void* h, int i, int64_t* out) {
    return guard([&] { *out = static_cast<const Sampler*>(h)->ts.at(static_cast<size_t>(i)); });
}

int stock_sched_sigma(const void* h, int i, double* out) {
    return guard([&] { *out = static_cast<const Sampler*>(h)->sig.at(static_cast<size_t>(i)); });
}

int stock_sched_coefficients(const void* h, int i, bh_sched_coefficients* out) {
    return guard([&] { *out = sampler_coefficients(*static_cast<const Sampler*>(h), i); });
}

int stock_sched_step(void* h, const void* eps, int i, void* sample, int64_t n, int dtype) {
    return guard([&] { sampler_step(*static_cast<Sampler*>(h), eps, i, sample, n, dtype); });
}

int stock_sched_reset(void* h) {
    return guard([&] {
        auto* s = static_cast<Sampler*>(h);
        s->x0s.clear();
        s->warm = 0;
    });
}

int stock_conv2d(const void* x, const void* w, const void* bias, void* out, int64_t batch,
                 int64_t c_in, int64_t h, int64_t wd, int64_t c_out, int64_t k, int64_t pad,
                 int dtype, int threads) {
    return guard([&] {
        conv2d_impl(x, w, bias, out, batch, c_in, h, wd, c_out, k, pad, dtype, resolve_threads(threads));
    });
}

int stock_group_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
                     int64_t cols, float eps, int64_t groups, int64_t channels, int dtype,
                     int threads) {
    return guard([&] {
        group_norm_impl(x, weight, bias, out, rows, cols, eps, groups, channels, dtype,
                        resolve_threads(threads));
    });
}

int stock_upsample(const void* in, void* out, int64_t batch, int64_t channels, int64_t h,
                   int64_t w, int64_t factor, int dtype) {
    return guard([&] { upsample_impl(in, out, batch, channels, h, w, factor, dtype); });
}

int stock_transpose(const void* in, void* out, int64_t batch, int64_t channels, int64_t spatial,
                    int to_channels_first, int dtype) {
    return guard([&] { transpose_impl(in, out, batch, channels, spatial, to_channels_first != 0, dtype); });
}

int stock_vae_forward(const bh_vae_config* cfg, const bh_vae_weights* w, const uint16_t* latent,
                      int64_t latent_hw, uint16_t* image, int threads, int stop_after) {
    return guard([&] {
        vae_forward(*cfg, vae_table(*w), latent, latent_hw, image, resolve_threads(threads), stop_after);
    });
}

int stock_t5_bucket(int rp, int num_buckets, int max_distance) {
    return t5_bucket(rp, num_buckets, max_distance);
}

int stock_t5_forward(const bh_t5_config* cfg, const bh_t5_weights* w, const float* ids, int64_t batch,
                     int64_t seq, uint16_t* out, int threads) {
    return guard([&] {
        t5_forward(*cfg, name_table(w->count, w->names, w->tensors), ids, batch, seq, out,
                   resolve_threads(threads));
    });
}

}  // extern "C"
