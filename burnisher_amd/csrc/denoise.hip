// The denoise loop around the dit-step, on the device (pipeline.cpp:104-131).
//
//   * repeat and guidance, the two ops the reference runs between dit-steps
//     (ops_cpu.cpp:355-369, ops_cuda.cu:1033-1073);
//   * DPM-Solver++ 2M (src/sched/dpm_solver.cpp). The reference keeps the whole sampler on the
//     host and copies eps and the latent down and back every step (pipeline.cpp:124-130). Here
//     the schedule, the step order and the fp64 coefficients stay host scalars, computed by the
//     same double operations as the reference, while the sample, the model output and the x0
//     history stay in HBM and one kernel per step applies the update in fp64;
//   * the loop itself, eagerly or as one HIP graph of every step's launches.
//
// Numerics: the reference evaluates the guidance combine and the solver update in double and
// rounds once to float and once more through the storage dtype (Tensor::set, tensor.cpp:85-96).
// The kernels do the same operations in the same order in fp64, and this file is compiled with
// -ffp-contract=off (host and device) so no multiply-add is fused, as in the reference's x86-64
// build. All three ops are therefore bit-exact with the reference.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/burnisher_hip.h"
#include "common.h"

namespace bh {
namespace {

constexpr int kThreads = 256;

int blocks_for(int64_t n) {
    const int64_t b = (n + kThreads - 1) / kThreads;
    return static_cast<int>(b < 1 ? 1 : (b > 8192 ? 8192 : b));
}

__device__ inline float load(float v) { return v; }
__device__ inline float load(bf16_t v) { return bf2f(v); }
template <typename T>
__device__ inline T store(float v);
template <>
__device__ inline float store<float>(float v) { return v; }
template <>
__device__ inline bf16_t store<bf16_t>(float v) { return f2bf(v); }

// ---- repeat: out[r*inner + i] = in[i] -------------------------------------------------------

// A copy in units of U (16, 4 or 2 bytes): the widest unit that divides the row.
template <typename U>
__global__ void k_repeat(const U* __restrict__ in, U* __restrict__ out, int64_t outer,
                         int64_t inner) {
    const int64_t n = outer * inner;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        out[i] = in[i % inner];
    }
}

void launch_repeat(const void* in, void* out, int64_t outer, int64_t inner, size_t elem,
                   hipStream_t s) {
    const int64_t bytes = inner * static_cast<int64_t>(elem);
    const auto aligned = [&](size_t a) {
        return bytes % static_cast<int64_t>(a) == 0 &&
               reinterpret_cast<uintptr_t>(in) % a == 0 && reinterpret_cast<uintptr_t>(out) % a == 0;
    };
    if (aligned(16)) {
        const int64_t w = bytes / 16;
        k_repeat<uint4><<<blocks_for(outer * w), kThreads, 0, s>>>(
            static_cast<const uint4*>(in), static_cast<uint4*>(out), outer, w);
    } else if (aligned(4)) {
        const int64_t w = bytes / 4;
        k_repeat<uint32_t><<<blocks_for(outer * w), kThreads, 0, s>>>(
            static_cast<const uint32_t*>(in), static_cast<uint32_t*>(out), outer, w);
    } else {
        const int64_t w = bytes / 2;
        k_repeat<uint16_t><<<blocks_for(outer * w), kThreads, 0, s>>>(
            static_cast<const uint16_t*>(in), static_cast<uint16_t*>(out), outer, w);
    }
    launch_check("repeat");
}

// ---- guidance: out[c, s] = u + scale*(k - u) in fp64 (ops_cpu.cpp:361-369) ---------------------

// `cond` is the second prediction row; without guidance it is the first row again, so the
// result is u itself.
template <typename T>
__global__ void k_guidance(const T* __restrict__ uncond, const T* __restrict__ cond,
                           T* __restrict__ out, int64_t channels, int64_t spatial, float scale) {
    const int64_t n = channels * spatial;
    const double sc = scale;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const double u = load(uncond[i]);
        const double k = load(cond[i]);
        out[i] = store<T>(static_cast<float>(u + sc * (k - u)));
    }
}

// The prediction rows are [out_channels, spatial] each; the first `channels` of a row are the
// contiguous run [0, channels*spatial).
void launch_guidance(const void* pred, bool two_rows, void* out, int64_t out_channels,
                     int64_t channels, int64_t spatial, float scale, bool f32, hipStream_t s) {
    const int64_t n = channels * spatial;
    const int64_t row = out_channels * spatial;
    if (f32) {
        const float* u = static_cast<const float*>(pred);
        k_guidance<float><<<blocks_for(n), kThreads, 0, s>>>(u, two_rows ? u + row : u,
                                                            static_cast<float*>(out), channels,
                                                            spatial, scale);
    } else {
        const bf16_t* u = static_cast<const bf16_t*>(pred);
        k_guidance<bf16_t><<<blocks_for(n), kThreads, 0, s>>>(u, two_rows ? u + row : u,
                                                              static_cast<bf16_t*>(out), channels,
                                                              spatial, scale);
    }
    launch_check("guidance");
}

// ---- the solver update (dpm_solver.cpp:89-98, 125-162) ---------------------------------------

struct StepScalars {
    double sigma_s, alpha_s;  // variance-preserving sigma and alpha at step i (x0 conversion)
    double ratio;             // sigma_vp_t / sigma_vp_s0, the coefficient on the sample
    double coef;              // alpha_t * (exp(-h) - 1)
    double half_coef;         // 0.5 * coef
    double inv_r0;            // 1 / r0 (second order only)
    int order;
};

// x0 = (x - sigma_s*eps) / alpha_s, stored through the dtype into the history slot `x0_new`,
// then x <- ratio*x - coef*x0                                   (first order)
//      x <- ratio*x - coef*x0 - half_coef*(inv_r0*(x0 - x0_prev)) (second order, midpoint)
template <typename T>
__global__ void k_dpm_step(const T* __restrict__ eps, T* __restrict__ sample,
                           T* __restrict__ x0_new, const T* __restrict__ x0_prev, int64_t n,
                           StepScalars a) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kThreads) {
        const double x = load(sample[i]);
        const T m0 = store<T>(static_cast<float>((x - a.sigma_s * load(eps[i])) / a.alpha_s));
        x0_new[i] = m0;
        const double d0 = load(m0);
        double v;
        if (a.order == 1) {
            v = a.ratio * x - a.coef * d0;
        } else {
            const double d1 = a.inv_r0 * (d0 - load(x0_prev[i]));
            v = a.ratio * x - a.coef * d0 - a.half_coef * d1;
        }
        sample[i] = store<T>(static_cast<float>(v));
    }
}

// ---- device buffers -------------------------------------------------------------------------

struct Mem {
    void* p = nullptr;
    Mem() = default;
    explicit Mem(size_t bytes) {
        hip_check(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
        hip_check(hipMemset(p, 0, bytes ? bytes : 1), "hipMemset");
    }
    Mem(const Mem&) = delete;
    Mem& operator=(const Mem&) = delete;
    Mem& operator=(Mem&& o) noexcept {
        std::swap(p, o.p);
        return *this;
    }
    ~Mem() {
        if (p) (void)hipFree(p);
    }
};

bool same(const char* a, const char* b) { return a && std::strcmp(a, b) == 0; }

size_t elem_size(int dtype) {
    require(dtype == BH_F32 || dtype == BH_BF16, "dtype must be BH_F32 or BH_BF16");
    return dtype == BH_F32 ? 4 : 2;
}

}  // namespace
}  // namespace bh

// ---- the scheduler --------------------------------------------------------------------------

struct bh_sched {
    int train_steps = 1000;
    int order_cap = 2;        // solver_order
    bool lower_final = true;  // lower_order_final
    bool linspace = true;     // timestep_spacing is "linspace" (checked by set_timesteps)
    std::vector<double> karras;  // sqrt((1 - acp) / acp) for every training timestep
    std::vector<int64_t> ts;     // inference timesteps, descending
    std::vector<double> sig;     // their Karras sigmas, then a final 0
    int warm = 0;                // lower_order_nums_: steps taken since reset, capped at order_cap
    int64_t pushes = 0;          // x0 predictions written since reset; slot = pushes % 2
    bh::Mem hist[2];             // the last two x0 predictions
    int64_t hist_numel = -1;
    int hist_dtype = -1;
    uint64_t version = 1;        // bumped when anything a captured loop baked in changes

    // coefficients(i) (dpm_solver.cpp:100-123) from the current history.
    bh_sched_coefficients coefficients(int i) const {
        bh::require(i >= 0 && static_cast<size_t>(i) + 1 < sig.size(),
                    "scheduler: step index " + std::to_string(i) + " out of range");
        const size_t at = static_cast<size_t>(i);
        bh_sched_coefficients c{};
        c.sigma_s0 = sig[at];
        c.sigma_t = sig[at + 1];
        vp(c.sigma_t, &c.alpha_t, &c.sigma_vp_t);
        vp(c.sigma_s0, &c.alpha_s0, &c.sigma_vp_s0);
        // exp(-h) as the ratio of Karras sigmas: finite on the last step, where sigma_t is 0.
        c.exp_neg_h = c.sigma_s0 > 0.0 ? c.sigma_t / c.sigma_s0 : 0.0;
        const bool final_step = at + 2 == sig.size();
        const bool second = warm >= 1 && order_cap >= 2 && !(lower_final && final_step);
        c.order = second ? 2 : 1;
        if (second) {
            bh::require(at >= 1, "scheduler: a second-order step at index 0 has no step i-1");
            const double h = std::log(c.sigma_s0 / c.sigma_t);
            const double h0 = std::log(sig[at - 1] / c.sigma_s0);
            c.r0 = h0 / h;
        }
        return c;
    }

    // Karras sigma -> alpha and sigma of the variance-preserving form (dpm_solver.cpp:10-16).
    static void vp(double k, double* alpha, double* sigma) {
        const double r = std::sqrt(k * k + 1.0);
        *alpha = 1.0 / r;
        *sigma = k / r;
    }

    void reserve(int64_t numel, int dtype) {
        const size_t es = bh::elem_size(dtype);
        if (numel == hist_numel && dtype == hist_dtype) return;
        hist[0] = bh::Mem(static_cast<size_t>(numel) * es);
        hist[1] = bh::Mem(static_cast<size_t>(numel) * es);
        hist_numel = numel;
        hist_dtype = dtype;
        ++version;
    }

    // step (dpm_solver.cpp:125-162): enqueue the update and advance the host state.
    void step(const void* eps, int i, void* sample, int64_t numel, int dtype, hipStream_t s) {
        bh::require(i >= 0 && static_cast<size_t>(i) < ts.size(),
                    "scheduler: step index " + std::to_string(i) + " out of range");
        reserve(numel, dtype);
        const int slot = static_cast<int>(pushes % 2);
        // The reference appends x0 to its history before it asks for the coefficients; the
        // order those coefficients pick depends only on `warm`, which is advanced after.
        const bh_sched_coefficients c = coefficients(i);
        bh::StepScalars a{};
        vp(sig[static_cast<size_t>(i)], &a.alpha_s, &a.sigma_s);
        a.ratio = c.sigma_vp_s0 > 0.0 ? c.sigma_vp_t / c.sigma_vp_s0 : 0.0;
        a.coef = c.alpha_t * (c.exp_neg_h - 1.0);
        a.half_coef = 0.5 * a.coef;
        a.inv_r0 = c.order == 2 ? 1.0 / c.r0 : 0.0;
        a.order = c.order;
        if (numel > 0) {
            const int grid = bh::blocks_for(numel);
            if (dtype == BH_F32) {
                bh::k_dpm_step<float><<<grid, bh::kThreads, 0, s>>>(
                    static_cast<const float*>(eps), static_cast<float*>(sample),
                    static_cast<float*>(hist[slot].p), static_cast<const float*>(hist[slot ^ 1].p),
                    numel, a);
            } else {
                bh::k_dpm_step<bh::bf16_t><<<grid, bh::kThreads, 0, s>>>(
                    static_cast<const bh::bf16_t*>(eps), static_cast<bh::bf16_t*>(sample),
                    static_cast<bh::bf16_t*>(hist[slot].p),
                    static_cast<const bh::bf16_t*>(hist[slot ^ 1].p), numel, a);
            }
            bh::launch_check("dpm step");
        }
        ++pushes;
        if (warm < order_cap) ++warm;
    }

    void reset() {
        warm = 0;
        pushes = 0;
    }
};

// ---- the denoise loop -----------------------------------------------------------------------

struct bh_denoiser {
    bh_dit* dit = nullptr;
    bh_sched* sched = nullptr;
    bool guided = true;
    float scale = 0.0f;
    bh::DitGeometry g{};
    int64_t per = 0, spatial = 0;
    bh::Mem batched, pred, eps;

    // The captured loop and what it was captured for.
    hipStream_t capture_stream = nullptr;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    void* b_latent = nullptr;
    const void* b_caption = nullptr;
    const void* b_mask = nullptr;
    int b_mask_dtype = -1;
    int b_rows = -1;
    uint64_t b_version = 0;
    int end_warm = 0;
    int64_t end_pushes = 0;

    ~bh_denoiser() {
        drop_graph();
        if (capture_stream) (void)hipStreamDestroy(capture_stream);
    }

    void drop_graph() {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (graph) (void)hipGraphDestroy(graph);
        exec = nullptr;
        graph = nullptr;
    }

    // Every step of the schedule (pipeline.cpp:110-131), enqueued on `s`.
    void enqueue(void* latent, const void* caption, const void* mask, int mask_dtype,
                 hipStream_t s) {
        sched->reset();
        const int steps = static_cast<int>(sched->ts.size());
        for (int i = 0; i < steps; ++i) {
            bh::launch_repeat(latent, batched.p, g.batch, per, 2, s);
            // The caption branch depends on nothing that changes between steps: computed at
            // step 0, reused by the rest.
            bh::dit_forward_step(dit, batched.p, static_cast<double>(sched->ts[i]), caption,
                                 mask, mask_dtype, pred.p, s, i > 0);
            bh::launch_guidance(pred.p, guided, eps.p, g.out_channels, g.in_channels, spatial,
                                guided ? scale : 0.0f, false, s);
            sched->step(eps.p, i, latent, per, BH_BF16, s);
        }
    }
};

// ---- C ABI ----------------------------------------------------------------------------------

extern "C" {

int bh_repeat(const void* in, void* out, int64_t outer, int64_t inner, int dtype, void* stream) {
    return bh::guarded([&] {
        const size_t es = bh::elem_size(dtype);
        bh::require(outer >= 0 && inner >= 0, "repeat: negative extent");
        if (outer * inner == 0) return;
        bh::require_device_ptr(in, "repeat (hip-gfx950)", "in");
        bh::require_device_ptr(out, "repeat (hip-gfx950)", "out");
        bh::ProfileScope ps(bh::K_ELEMENTWISE, static_cast<hipStream_t>(stream),
                            static_cast<double>((outer + 1) * inner * static_cast<int64_t>(es)));
        bh::launch_repeat(in, out, outer, inner, es, static_cast<hipStream_t>(stream));
    });
}

int bh_guidance(const void* prediction, void* out, int64_t out_channels, int64_t channels,
                int64_t spatial, float scale, int dtype, void* stream) {
    return bh::guarded([&] {
        const size_t es = bh::elem_size(dtype);
        bh::require(out_channels >= 0 && channels >= 0 && spatial >= 0,
                    "guidance: negative extent");
        bh::require(channels <= out_channels, "guidance: channels exceeds out_channels");
        if (channels * spatial == 0) return;
        bh::require_device_ptr(prediction, "guidance (hip-gfx950)", "prediction");
        bh::require_device_ptr(out, "guidance (hip-gfx950)", "out");
        bh::ProfileScope ps(bh::K_ELEMENTWISE, static_cast<hipStream_t>(stream),
                            3.0 * channels * spatial * static_cast<double>(es));
        bh::launch_guidance(prediction, true, out, out_channels, channels, spatial, scale,
                            dtype == BH_F32, static_cast<hipStream_t>(stream));
    });
}

void bh_sched_config_default(bh_sched_config* c) {
    if (!c) return;
    c->num_train_timesteps = 1000;
    c->beta_start = 0.0001;
    c->beta_end = 0.02;
    c->beta_schedule = "linear";
    c->solver_order = 2;
    c->algorithm_type = "dpmsolver++";
    c->solver_type = "midpoint";
    c->prediction_type = "epsilon";
    c->timestep_spacing = "linspace";
    c->lower_order_final = 1;
}

// The constructor (dpm_solver.cpp:19-53): the cumulative product of (1 - beta) in double over
// the training schedule; beta is linear in t, or its square root is ("scaled_linear").
int bh_sched_create(const bh_sched_config* c, bh_sched** out) {
    return bh::guarded([&] {
        bh::require(c && out, "sched_create: null argument");
        bh::require(bh::same(c->algorithm_type, "dpmsolver++"),
                    "scheduler: only dpmsolver++ is implemented");
        bh::require(bh::same(c->solver_type, "midpoint"),
                    "scheduler: only the midpoint solver type is implemented");
        bh::require(bh::same(c->prediction_type, "epsilon"),
                    "scheduler: only epsilon prediction is implemented");
        const bool scaled = bh::same(c->beta_schedule, "scaled_linear");
        bh::require(scaled || bh::same(c->beta_schedule, "linear"),
                    std::string("scheduler: unsupported beta_schedule '") +
                        (c->beta_schedule ? c->beta_schedule : "(null)") + "'");
        bh::require(c->num_train_timesteps >= 2, "scheduler: num_train_timesteps must be >= 2");
        bh::require(c->solver_order >= 1, "scheduler: solver_order must be >= 1");
        auto s = std::make_unique<bh_sched>();
        s->train_steps = c->num_train_timesteps;
        s->order_cap = c->solver_order;
        s->lower_final = c->lower_order_final != 0;
        s->linspace = bh::same(c->timestep_spacing, "linspace");
        s->karras.resize(static_cast<size_t>(s->train_steps));
        const double lo = scaled ? std::sqrt(c->beta_start) : c->beta_start;
        const double hi = scaled ? std::sqrt(c->beta_end) : c->beta_end;
        double acp = 1.0;
        for (int t = 0; t < s->train_steps; ++t) {
            const double f = lo + (hi - lo) * (static_cast<double>(t) / (s->train_steps - 1));
            acp *= 1.0 - (scaled ? f * f : f);
            s->karras[static_cast<size_t>(t)] = std::sqrt((1.0 - acp) / acp);
        }
        *out = s.release();
    });
}

// set_timesteps (dpm_solver.cpp:55-75): round(j*(N-1)/steps) for j = steps..1.
int bh_sched_set_timesteps(bh_sched* s, int steps) {
    return bh::guarded([&] {
        bh::require(s != nullptr, "sched: null handle");
        bh::require(steps >= 1, "scheduler: at least one step");
        bh::require(s->linspace, "scheduler: only linspace spacing is implemented");
        s->ts.clear();
        s->sig.clear();
        for (int j = steps; j >= 1; --j) {
            const double at = static_cast<double>(j) * (s->train_steps - 1) /
                              static_cast<double>(steps);
            s->ts.push_back(static_cast<int64_t>(std::llround(at)));
            s->sig.push_back(s->karras[static_cast<size_t>(s->ts.back())]);
        }
        s->sig.push_back(0.0);
        s->reset();
        ++s->version;
    });
}

int bh_sched_steps(const bh_sched* s) { return s ? static_cast<int>(s->ts.size()) : 0; }

int64_t bh_sched_timestep(const bh_sched* s, int i) {
    if (!s || i < 0 || static_cast<size_t>(i) >= s->ts.size()) {
        bh::set_last_error("sched: timestep index out of range");
        return -1;
    }
    return s->ts[static_cast<size_t>(i)];
}

double bh_sched_sigma(const bh_sched* s, int i) {
    if (!s || i < 0 || static_cast<size_t>(i) >= s->sig.size()) {
        bh::set_last_error("sched: sigma index out of range");
        return std::nan("");
    }
    return s->sig[static_cast<size_t>(i)];
}

double bh_sched_init_noise_sigma(const bh_sched* s) { return s ? 1.0 : std::nan(""); }

int bh_sched_get_coefficients(const bh_sched* s, int i, bh_sched_coefficients* out) {
    return bh::guarded([&] {
        bh::require(s && out, "sched: null argument");
        *out = s->coefficients(i);
    });
}

int bh_sched_reserve(bh_sched* s, int64_t numel, int dtype) {
    return bh::guarded([&] {
        bh::require(s != nullptr, "sched: null handle");
        bh::require(numel >= 0, "sched: negative size");
        s->reserve(numel, dtype);
    });
}

int bh_sched_step(bh_sched* s, const void* model_output, int i, void* sample, int64_t numel,
                  int dtype, void* stream) {
    return bh::guarded([&] {
        bh::require(s != nullptr, "sched: null handle");
        bh::require(numel >= 0, "sched: negative size");
        bh::elem_size(dtype);
        if (numel > 0) {
            bh::require_device_ptr(model_output, "sched_step", "model_output");
            bh::require_device_ptr(sample, "sched_step", "sample");
        }
        bh::ProfileScope ps(bh::K_ELEMENTWISE, static_cast<hipStream_t>(stream),
                            static_cast<double>(numel) * 5.0 * static_cast<double>(bh::elem_size(dtype)));
        s->step(model_output, i, sample, numel, dtype, static_cast<hipStream_t>(stream));
    });
}

int bh_sched_reset(bh_sched* s) {
    return bh::guarded([&] {
        bh::require(s != nullptr, "sched: null handle");
        s->reset();
    });
}

void bh_sched_destroy(bh_sched* s) { delete s; }

int bh_denoiser_create(bh_dit* e, bh_sched* s, int classifier_free_guidance,
                       float guidance_scale, bh_denoiser** out) {
    return bh::guarded([&] {
        bh::require(e && s && out, "denoiser_create: null argument");
        bh::require(!s->ts.empty(), "denoiser_create: the scheduler has no timesteps set");
        auto d = std::make_unique<bh_denoiser>();
        d->dit = e;
        d->sched = s;
        d->guided = classifier_free_guidance != 0;
        d->scale = guidance_scale;
        d->g = bh::dit_geometry(e);
        bh::require(d->g.batch == (d->guided ? 2 : 1),
                    "denoiser_create: the engine has batch " + std::to_string(d->g.batch) +
                        " but guidance asks for " + std::to_string(d->guided ? 2 : 1) +
                        ". Under classifier-free guidance the negative prompt comes FIRST.");
        bh::require(d->g.out_channels >= d->g.in_channels,
                    "denoiser_create: out_channels < in_channels");
        d->spatial = d->g.latent_hw * d->g.latent_hw;
        d->per = d->g.in_channels * d->spatial;
        d->batched = bh::Mem(static_cast<size_t>(d->g.batch * d->per) * 2);
        d->pred = bh::Mem(static_cast<size_t>(d->g.batch * d->g.out_channels * d->spatial) * 2);
        d->eps = bh::Mem(static_cast<size_t>(d->per) * 2);
        s->reserve(d->per, BH_BF16);
        bh::hip_check(hipStreamCreateWithFlags(&d->capture_stream, hipStreamNonBlocking),
                      "hipStreamCreateWithFlags");
        bh::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        *out = d.release();
    });
}

int bh_denoiser_run(bh_denoiser* d, void* latent, const void* caption, const void* caption_mask,
                    int mask_dtype, int use_graph, void* stream) {
    return bh::guarded([&] {
        bh::require(d != nullptr, "denoiser_run: null handle");
        bh::require_device_ptr(latent, "denoiser_run", "latent");
        bh::require_device_ptr(caption, "denoiser_run", "caption");
        bh::require_device_ptr(caption_mask, "denoiser_run", "caption_mask");
        bh::require(mask_dtype == BH_F32 || mask_dtype == BH_BF16, "denoiser_run: mask dtype");
        bh::require(!d->sched->ts.empty(), "denoiser_run: the scheduler has no timesteps set");
        d->sched->reserve(d->per, BH_BF16);
        hipStream_t s = static_cast<hipStream_t>(stream);
        if (!use_graph) {
            d->enqueue(latent, caption, caption_mask, mask_dtype, s);
            return;
        }
        bh::require(!bh::profiling_enabled(),
                    "denoiser_run: a graph cannot be captured while the launch profiler is on");
        bh::require(d->g.mode == BH_DIT_FUSED,
                    "denoiser_run: graph capture needs an engine in BH_DIT_FUSED mode");
        const bool bound = d->exec && d->b_latent == latent && d->b_caption == caption &&
                           d->b_mask == caption_mask && d->b_mask_dtype == mask_dtype &&
                           d->b_version == d->sched->version && d->b_rows == bh::dit_rows(d->dit);
        if (!bound) {
            d->drop_graph();
            // Work already queued on `s` must not race the capture stream's first replay; the
            // replay itself is ordered on `s`, so only creation needs this wait.
            bh::hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
            bh::hip_check(hipStreamBeginCapture(d->capture_stream, hipStreamCaptureModeRelaxed),
                          "hipStreamBeginCapture");
            try {
                d->enqueue(latent, caption, caption_mask, mask_dtype, d->capture_stream);
            } catch (...) {
                hipGraph_t broken = nullptr;
                (void)hipStreamEndCapture(d->capture_stream, &broken);
                if (broken) (void)hipGraphDestroy(broken);
                throw;
            }
            bh::hip_check(hipStreamEndCapture(d->capture_stream, &d->graph), "hipStreamEndCapture");
            bh::hip_check(hipGraphInstantiate(&d->exec, d->graph, nullptr, nullptr, 0),
                          "hipGraphInstantiate");
            d->b_latent = latent;
            d->b_caption = caption;
            d->b_mask = caption_mask;
            d->b_mask_dtype = mask_dtype;
            d->b_version = d->sched->version;
            d->b_rows = bh::dit_rows(d->dit);
            d->end_warm = d->sched->warm;
            d->end_pushes = d->sched->pushes;
        }
        bh::hip_check(hipGraphLaunch(d->exec, s), "hipGraphLaunch");
        // The host state a run leaves behind, as if the steps had been enqueued one by one.
        d->sched->warm = d->end_warm;
        d->sched->pushes = d->end_pushes;
    });
}

void bh_denoiser_destroy(bh_denoiser* d) { delete d; }

}  // extern "C"
