/*
 * burnisher_hip.h -- the C ABI of libburnisher_hip.so, the MI355X (gfx950) implementation of
 * Burnisher's `dit-step` hot path.
 *
 * Every entry point takes plain device pointers, element counts and a HIP stream (`void*`,
 * NULL = the default stream) and returns 0 on success or a nonzero status with a message
 * readable through bh_last_error(). Nothing here allocates on the hot path except where a
 * function says so. All launches are asynchronous on the given stream; nothing synchronises
 * the host except bh_synchronize().
 *
 * Storage conventions follow the reference runtime:
 *   - element types are `bh_dtype` (storage-only bf16 with round-to-nearest-even, or fp32);
 *     every op reads its inputs as float, computes in fp32 and rounds ONCE per stored element;
 *   - matrices are row-major, weights are the checkpoint's [out_features, in_features];
 *   - attention tensors are HEAD-LAST, [batch, seq, heads, head_dim].
 *
 * The per-op entry points below are one-to-one with the reference's op surface
 * (/root/reference/include/burnisher/ops.h) so a reference `register_impl<Args>` lambda can
 * forward an Args struct field by field.
 */
#ifndef BURNISHER_HIP_H
#define BURNISHER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BH_ABI_VERSION 1

typedef enum bh_dtype { BH_F32 = 0, BH_BF16 = 1 } bh_dtype;

/* Mirrors burnisher::Epilogue (ops.h:17-22). GeluGated is T5-only and is rejected. */
typedef enum bh_epilogue { BH_EPI_NONE = 0, BH_EPI_GELU = 1, BH_EPI_SILU = 2, BH_EPI_GELU_GATED = 3 }
    bh_epilogue;

/* ---- library ------------------------------------------------------------------------------ */

/* ABI version this library was built with (BH_ABI_VERSION). */
int bh_abi_version(void);
/* "gfx950 ..." build string. */
const char* bh_build_info(void);
/* Message of the last failing call on this host thread ("" if none). */
const char* bh_last_error(void);
/* Binds the calling thread to `device` and checks that it is a gfx950 part. Safe to repeat. */
int bh_init(int device);
/* hipStreamSynchronize(stream) with error reporting. */
int bh_synchronize(void* stream);
/* Whether the entry points called from this host thread ask the HIP runtime about every operand
 * pointer (hipPointerGetAttributes) to refuse host memory (on = 1, the default) or only refuse
 * null operands (0). No counterpart in the reference, whose ops read the device from the Tensor
 * (Tensor::device(), tensor.h:39) and refuse a host tensor in `require_device`
 * (ops_cuda.cu:79-88). A caller that knows where its operands live the same way -- the registry
 * adapter, which checks each Tensor's device before every call -- turns the runtime lookups off:
 * they cost several host microseconds per operand and per op. */
int bh_set_operand_checks(int on);

/* ---- per-op entry points (the registry boundary) ------------------------------------------ */

/* GemmArgs (ops.h:29-44): out[M,N] = a[M,K] @ B (+bias[N]) then `epilogue`.
 * B is [N,K] when b_transposed (every DiT call), else [K,N]. One rounding at the store.
 * Replaces the reference `gemm_cuda` (src/cuda/ops_cuda.cu:476-513). */
int bh_gemm(const void* a, const void* b, const void* bias, void* out, int64_t m, int64_t n,
            int64_t k, int b_transposed, int epilogue, int dtype, void* stream);

/* The fused epilogue the dit-step engine uses, exposed so it can be tested on its own.
 * With v = epilogue(acc + bias):
 *   if round_mid, v is rounded to the storage type first (exactly what a separate GEMM stores);
 *   if row_add:  v = v + row_add[(row % row_add_period), n]           (AddArgs broadcast_b)
 *   if residual: v = residual[row, n] + gate[row / gate_rows, n] * v    (ModulateArgs gated
 *                residual with zero scale/shift; gate NULL means 1)
 * `ld_out` is the row stride of out and residual (>= n). b is always [N,K] (b_transposed).
 * bf16 only. out may alias residual. */
typedef struct bh_gemm_fused {
    int epilogue;
    int round_mid;
    const void* row_add;
    int64_t row_add_period;
    const void* residual;
    const void* gate;
    int64_t gate_rows;
    int64_t ld_out;
} bh_gemm_fused;
int bh_gemm_fused_run(const void* a, const void* b, const void* bias, void* out, int64_t m,
                      int64_t n, int64_t k, const bh_gemm_fused* f, void* stream);

/* AttentionArgs (ops.h:62-77): softmax(scale * q k^T (+bias) , key_mask) v, head-last.
 * scale <= 0 means 1/sqrt(head_dim). key_mask is [batch, kv_len] (1 keeps, 0 masks -> score
 * -1e9, so an all-masked row is uniform over v), in `mask_dtype`; bias is [heads,q_len,kv_len].
 * Replaces `attention_cuda` (src/cuda/ops_cuda.cu:883-886). */
int bh_attention(const void* q, const void* k, const void* v, void* out, int64_t batch,
                 int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                 const void* bias, const void* key_mask, int mask_dtype, int dtype, void* stream);

/* bh_attention without any allocation, for callers that cannot allocate: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc. It has no counterpart in the
 * reference. Same arguments, kernels and results as bh_attention; where bh_attention transposes V
 * into a workspace it grows on demand (head_dim 72 and the single-head head_dim-512 kernel) and,
 * at head_dim 72 with few queries, splits the keys with fp32 partials in another, this one uses a
 * fixed array in the library's device memory of 64 MiB per device (V^T of
 * batch x heads x 72 x kv_len rounded up to 64 keys, or 512 x kv_len rounded up to 32, bf16; then
 * splits x batch x heads x q_len x 320 bytes of partials), and a call that needs more is refused
 * with an error. The array's address is looked up by bh_init (or
 * by the first call on a device). Every call on one device shares that array and each call
 * rewrites all of it that it reads, so nothing carries over between calls; calls that overlap on
 * one device (two streams, or two threads) race on it and must be ordered by the caller. */
int bh_attention_noalloc(const void* q, const void* k, const void* v, void* out, int64_t batch,
                         int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                         const void* bias, const void* key_mask, int mask_dtype, int dtype,
                         void* stream);

/* The same op over row-strided operands: element (b,s,h,d) of q lives at
 * q[(b*q_len + s)*ld_q + h*head_dim + d], likewise k/v with ld_kv and out with ld_out.
 * Lets attention read Q,K,V straight out of one fused [M, 3*d] projection. No bias. */
int bh_attention_strided(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_kv,
                         void* out, int64_t ld_out, int64_t batch, int64_t heads, int64_t q_len,
                         int64_t kv_len, int64_t head_dim, float scale, const void* key_mask,
                         int mask_dtype, int dtype, void* stream);

/* NormArgs (ops.h:81-94): LayerNorm (rms=0) or RMSNorm (rms=1) over the last dimension with
 * optional weight/bias; fp64 statistics like the reference oracle. Replaces `k_layernorm`
 * (src/cuda/ops_cuda.cu:227-272). groups > 0 is GroupNorm (ops_cpu.cpp:186-224) over NCHW rows
 * of `channels` x spatial (channels 0: cols), bf16, channels % 8 == 0 with channels/8 dividing
 * 256; it uses per-device scratch grown on demand. Replaces `groupnorm_chunked` (ops_cuda.cu:275-371). */
int bh_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
            int64_t cols, float eps, int rms, int64_t groups, int64_t channels, int dtype,
            void* stream);

/* ModulateArgs (ops.h:101-109): out = x*(1+scale[b,c]) + shift[b,c], then *gate[b,c] and
 * +residual when given. out may alias residual. Replaces `k_modulate` (ops_cuda.cu:194-221). */
int bh_modulate(const void* x, const void* scale, const void* shift, void* out, int64_t batch,
                int64_t tokens, int64_t channels, const void* residual, const void* gate,
                int dtype, void* stream);

/* ActivationArgs (ops.h:111-117): SiLU / GELU-tanh elementwise (GeluGated: * gate). */
int bh_activation(const void* x, void* out, int64_t numel, int kind, const void* gate, int dtype,
                  void* stream);

/* AddArgs (ops.h:135-143): out[r,i] = a[r,i] + scale*b[(broadcast ? 0 : r), i]. out may alias a. */
int bh_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner, float scale,
           int broadcast_b, int dtype, void* stream);

/* ChunkArgs (ops.h:150-159): out[b,c] = modulation[b, chunk*channels + c] + table[trow, c],
 * trow = table_chunk >= 0 ? table_chunk : chunk. */
int bh_chunk(const void* modulation, const void* table, void* out, int64_t batch,
             int64_t channels, int64_t chunks, int64_t chunk, int64_t table_chunk, int dtype,
             void* stream);

/* PatchArgs (ops.h:161-173): forward [B,C,G*P,G*P] -> [B,G*G,C*P*P] in (c,ky,kx) order; inverse
 * [B,G*G,P*P*C] in (ky,kx,c) order -> [B,C,G*P,G*P]. */
int bh_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
             int64_t patch, int inverse, int dtype, void* stream);

/* Conv2dArgs (ops.h:120-126): NCHW bf16, stride 1, "same" padding (2*pad == k-1), weight
 * [c_out, c_in, k, k]. 3x3 with c_in % 64 == 0 runs as an implicit GEMM on the MFMA tile kernel,
 * 1x1 as a GEMM, other kernels in the reference's summation order. Uses per-device scratch grown
 * on demand. Replaces `conv2d_cuda` (src/cuda/ops_cuda.cu:897-1015, cuDNN). */
int bh_conv2d(const void* x, const void* weight, const void* bias, void* out, int64_t batch,
              int64_t c_in, int64_t h, int64_t w, int64_t c_out, int64_t k, int64_t pad, int dtype,
              void* stream);
/* UpsampleArgs (ops.h:178-182): nearest, integer factor, NCHW bf16. Replaces `upsample_cuda`
 * (ops_cuda.cu:1132-1157). */
int bh_upsample(const void* in, void* out, int64_t batch, int64_t channels, int64_t h, int64_t w,
                int64_t factor, int dtype, void* stream);
/* TransposeArgs (ops.h:184-191): [batch, channels, spatial] <-> [batch, spatial, channels],
 * bf16. Replaces `transpose_cuda` (ops_cuda.cu:1159-1170). */
int bh_transpose(const void* in, void* out, int64_t batch, int64_t channels, int64_t spatial,
                 int to_channels_first, int dtype, void* stream);

/* ScaleArgs (ops.h:210-215): out[i] = in[i] * scale, one rounding at the store (out may alias
 * in). Replaces `scale_cuda` (src/cuda/ops_cuda.cu:1018-1031). */
int bh_scale(const void* in, void* out, int64_t numel, float scale, int dtype, void* stream);

/* The timestep embedding of the DiT's adaLN-single (`sinusoidal_timestep_embedding`,
 * src/models/weights.cpp:107-121, broadcast over the batch as pixart_dit.cpp:156-160 does):
 * out[b, i] = cos(t * f_i), out[b, dim/2 + i] = sin(t * f_i) with f_i = exp(-ln(10000) i / (dim/2)),
 * computed in fp64 on the device and rounded once through float to `dtype`; out is [batch, dim].
 * An odd dim is refused, as the reference refuses it. */
int bh_timestep_embedding(double t, int dim, int64_t batch, void* out, int dtype, void* stream);

/* ---- device probe ---------------------------------------------------------------------------- */

/* What the device sustains, measured by this library's own kernels (the reference's `probe`
 * command, src/cuda/device.cu:257-357, which times a stream copy and a vendor GEMM):
 *   mfma_tflops        a register-only bf16 MFMA loop (v_mfma_f32_16x16x32_bf16, eight
 *                      independent accumulators, four waves per SIMD on every CU): the rate no
 *                      MFMA kernel can exceed on this device at the clock it holds;
 *   mfma_shader_mhz    the shader clock during that loop, per wave from the shader clock counter
 *                      over the constant-rate wall clock (median, min and max over waves);
 *   mfma_peak_at_clock_tflops  CUs x 4096 FLOP/clock x that clock;
 *   copy_gbs           a device-to-device copy of copy_bytes (read + write bytes over time);
 *   max_clock_mhz, wall_clock_mhz, cus   what the device reports.
 * copy_src and copy_dst are device buffers of copy_bytes (>= 1 MiB, a multiple of 16). Runs on the
 * default stream and synchronises; allocates two small buffers for the loop's results. */
typedef struct bh_probe_result {
    double mfma_tflops;
    double mfma_shader_mhz, mfma_shader_mhz_min, mfma_shader_mhz_max;
    double mfma_peak_at_clock_tflops;
    double copy_gbs;
    double max_clock_mhz, wall_clock_mhz;
    int cus;
} bh_probe_result;
int bh_probe_device(void* copy_src, void* copy_dst, int64_t copy_bytes, bh_probe_result* out);

/* ---- fused ops (no single reference op; each equals a fixed reference op sequence) -------- */

/* norm -> chunk(shift) -> chunk(scale) -> modulate, as the reference DiT block runs them
 * (pixart_dit.cpp:226-231): with every intermediate rounded where the reference stores it,
 *   shift[b,c] = mod[b, shift_chunk*C + c] + table[shift_row, c]
 *   scale[b,c] = mod[b, scale_chunk*C + c] + table[scale_row, c]
 *   out = LN(x)*(1+scale) + shift.
 * mod is [batch, mod_chunks*C], table is [*, C], x/out are [batch*tokens, C]. bf16 only. */
int bh_norm_modulate(const void* x, const void* mod, int64_t mod_chunks, int64_t shift_chunk,
                     int64_t scale_chunk, const void* table, int64_t shift_row, int64_t scale_row,
                     void* out, int64_t batch, int64_t tokens, int64_t channels, float eps,
                     void* stream);

/* ---- the dit-step engine ------------------------------------------------------------------ */

/* DiTConfig (models.h:105-118). */
typedef struct bh_dit_config {
    int num_layers;       /* 28 */
    int num_heads;        /* 16 */
    int head_dim;         /* 72 */
    int patch_size;       /* 2 */
    int in_channels;      /* 4 */
    int out_channels;     /* 8 */
    int caption_channels; /* 4096 */
    int sample_size;      /* 128: base grid = sample_size / patch_size */
    double mlp_ratio;     /* 4.0 */
    double eps;           /* 1e-6 */
} bh_dit_config;

/* One transformer block's weights, device pointers in bf16, named as in the checkpoint
 * (`transformer_blocks.<i>.<name>`, weights.cpp:267-282). */
typedef struct bh_dit_block_weights {
    const void* scale_shift_table; /* [6, d] */
    const void* attn1_q_w; const void* attn1_q_b;
    const void* attn1_k_w; const void* attn1_k_b;
    const void* attn1_v_w; const void* attn1_v_b;
    const void* attn1_o_w; const void* attn1_o_b; /* to_out.0 */
    const void* attn2_q_w; const void* attn2_q_b;
    const void* attn2_k_w; const void* attn2_k_b;
    const void* attn2_v_w; const void* attn2_v_b;
    const void* attn2_o_w; const void* attn2_o_b;
    const void* ff0_w; const void* ff0_b; /* ff.net.0.proj: [d_ff, d] */
    const void* ff2_w; const void* ff2_b; /* ff.net.2:      [d, d_ff] */
} bh_dit_block_weights;

/* The model's weights (weights.cpp:252-266), device pointers in bf16. */
typedef struct bh_dit_weights {
    const void* pos_embed_w;  /* pos_embed.proj.weight [d, C, p, p] */
    const void* pos_embed_b;
    const void* t_emb1_w;     /* adaln_single.emb.timestep_embedder.linear_1 [d, 256] */
    const void* t_emb1_b;
    const void* t_emb2_w;     /* ...linear_2 [d, d] */
    const void* t_emb2_b;
    const void* adaln_w;      /* adaln_single.linear [6d, d] */
    const void* adaln_b;
    const void* cap1_w;       /* caption_projection.linear_1 [d, caption_channels] */
    const void* cap1_b;
    const void* cap2_w;       /* caption_projection.linear_2 [d, d] */
    const void* cap2_b;
    const void* out_table;    /* scale_shift_table [2, d] */
    const void* proj_out_w;   /* proj_out [p*p*out_channels, d] */
    const void* proj_out_b;
    const bh_dit_block_weights* blocks; /* num_layers entries */
} bh_dit_weights;

/* How bh_dit_forward evaluates the graph. */
typedef enum bh_dit_mode {
    /* The MI355X plan: QKV fused into one GEMM, every layer's caption K/V in one GEMM, LN and
     * modulation fused, gated residuals in GEMM epilogues. */
    BH_DIT_FUSED = 0,
    /* The reference graph (pixart_dit.cpp:112-304) op by op through the per-op entry points:
     * the drop-in path a reference registry would run. */
    BH_DIT_OPWISE = 1
} bh_dit_mode;

typedef struct bh_dit bh_dit;

/* Prepares a forward for a fixed geometry: batch, latent side (H = W) and caption length.
 * Allocates every intermediate once (zero-filled) and any repacked weights; the weight
 * pointers must stay valid for the engine's lifetime. This call allocates; forward does not. */
int bh_dit_create(const bh_dit_config* cfg, const bh_dit_weights* w, int64_t batch,
                  int64_t latent_hw, int64_t caption_len, int mode, bh_dit** out);
/* PixArtDiT::forward (pixart_dit.cpp:112-304): latent [B, in_ch, H, W], caption
 * [B, caption_len, caption_channels], caption_mask [B, caption_len] in mask_dtype, output
 * [B, out_ch, H, W]; all bf16 device pointers except the mask. No host synchronisation. */
int bh_dit_forward(bh_dit* e, const void* latent, double timestep, const void* caption,
                   const void* caption_mask, int mask_dtype, void* out, void* stream);
/* Device bytes the engine holds (intermediates plus repacked weights). */
int64_t bh_dit_workspace_bytes(const bh_dit* e);
/* Copies the engine's 2-D sin/cos position table (`dit_position_embedding` + `position_table`,
 * src/models/pixart_dit.cpp:53-105: fp64 on the host, interpolation scale 2, base
 * sample_size / patch_size, stored bf16), [grid*grid, hidden], into the device buffer `out`. */
int bh_dit_position_table(const bh_dit* e, void* out, void* stream);

/* How the fused plan schedules the batch rows (the CFG pair). No counterpart in the reference,
 * whose graph runs the whole batch through each op in turn; the result is bit-identical under
 * every schedule (rows never mix). */
typedef enum {
    /* The whole batch through each launch, on the caller's stream (the default). */
    BH_DIT_ROWS_JOINED = 0,
    /* The rows in two groups, each on its own stream from the block loop's start to the output
     * head, so one group's launch tails and epilogues can overlap the other group's work. At
     * the current kernels it is slower than JOINED (14.99 against 13.51 ms per 1024px step: each
     * group's GEMMs have half the tiles, and the two streams' persistent kernels contend for the
     * CUs), so it is not the default. The second stream is the engine's own (default
     * priority); it joins the caller's stream by events, so a forward on a capturing stream is
     * captured whole. Each launch then covers half the batch and runs beside the other half's,
     * so per-launch kernel timings no longer describe a kernel alone. */
    BH_DIT_ROWS_SPLIT = 1
} bh_dit_rows;
/* Selects the row schedule of a fused engine (an op-by-op engine refuses any but JOINED). With a
 * batch of one every schedule runs as JOINED. */
int bh_dit_set_rows(bh_dit* e, int rows);
void bh_dit_destroy(bh_dit* e);

/* ---- the denoise loop around the dit-step (pipeline.cpp:104-131) -------------------------- */

/* RepeatArgs (ops.h:217-222): out[r*inner + i] = in[i] for r in [0, outer). A copy, exact in
 * either dtype. Replaces the reference `repeat_cuda` (src/cuda/ops_cuda.cu:1033-1049). */
int bh_repeat(const void* in, void* out, int64_t outer, int64_t inner, int dtype, void* stream);

/* GuidanceArgs (ops.h:224-237): prediction [2, out_channels, spatial] -> out [channels, spatial],
 *   out = u + scale * (c - u),  u = prediction[0, ch, s] (negative prompt), c = prediction[1, ch, s],
 * evaluated in fp64 and rounded once (ops_cpu.cpp:361-369). Only the first `channels` of the
 * `out_channels` are read: the learned-variance half is discarded. Replaces `guidance_cuda`
 * (src/cuda/ops_cuda.cu:1051-1073). */
int bh_guidance(const void* prediction, void* out, int64_t out_channels, int64_t channels,
                int64_t spatial, float scale, int dtype, void* stream);

/* SchedulerConfig (scheduler.h:20-31). Only the pinned configuration is implemented, and the
 * others are refused with the reference's reasons (dpm_solver.cpp:19-53, 55-61):
 * algorithm "dpmsolver++", solver "midpoint", prediction "epsilon", spacing "linspace";
 * beta_schedule "linear" or "scaled_linear". */
typedef struct bh_sched_config {
    int num_train_timesteps;      /* 1000 */
    double beta_start;            /* 1e-4 */
    double beta_end;              /* 0.02 */
    const char* beta_schedule;    /* "linear" */
    int solver_order;             /* 2 (>= 1) */
    const char* algorithm_type;   /* "dpmsolver++" */
    const char* solver_type;      /* "midpoint" */
    const char* prediction_type;  /* "epsilon" */
    const char* timestep_spacing; /* "linspace" */
    int lower_order_final;        /* 1 */
} bh_sched_config;

/* DPMSolverMultistep::StepCoefficients (scheduler.h:52-69): the Karras sigmas (sigma_*), the
 * variance-preserving ones (sigma_vp_*), alpha, exp(-h) = sigma_t / sigma_s0 and r0 = h0 / h
 * (0 for a first-order step). */
typedef struct bh_sched_coefficients {
    int order;
    double sigma_s0, sigma_t;
    double sigma_vp_s0, sigma_vp_t;
    double alpha_t, alpha_s0;
    double exp_neg_h;
    double r0;
} bh_sched_coefficients;

/* DPM-Solver++ 2M (src/sched/dpm_solver.cpp), with its state split the MI355X way: the schedule,
 * the step order and the fp64 coefficients are host scalars computed exactly as the reference
 * does; the sample, the model output and the x0 history stay in device memory and one kernel per
 * step applies the update in fp64 with the reference's rounding (dpm_solver.cpp:89-162). */
typedef struct bh_sched bh_sched;

/* The pinned PixArt-Sigma configuration (scheduler.h:21-30). */
void bh_sched_config_default(bh_sched_config* cfg);
/* DPMSolverMultistep(cfg) (dpm_solver.cpp:19-53). Host memory only. */
int bh_sched_create(const bh_sched_config* cfg, bh_sched** out);
/* set_timesteps (dpm_solver.cpp:55-75): steps >= 1; also resets the step history. */
int bh_sched_set_timesteps(bh_sched* s, int steps);
int bh_sched_steps(const bh_sched* s);
/* timestep(i) and sigma(i) (scheduler.h:39-40); sigma has steps + 1 entries, the last 0.
 * Out of range: -1 and NaN, with bh_last_error set. */
int64_t bh_sched_timestep(const bh_sched* s, int i);
double bh_sched_sigma(const bh_sched* s, int i);
double bh_sched_init_noise_sigma(const bh_sched* s);
/* coefficients(i) (dpm_solver.cpp:100-123), from the current step history. */
int bh_sched_get_coefficients(const bh_sched* s, int i, bh_sched_coefficients* out);
/* Sizes the device x0 history for `numel` elements of `dtype` (two buffers). This call
 * allocates; bh_sched_step allocates only when no reservation of its size and dtype exists. */
int bh_sched_reserve(bh_sched* s, int64_t numel, int dtype);
/* step(model_output, i, sample) (dpm_solver.cpp:89-98, 125-162): `sample` [numel] is updated in place
 * from the epsilon prediction `model_output` [numel], both device pointers of `dtype`. Keeps the
 * last two x0 predictions on the device. Asynchronous on `stream`. */
int bh_sched_step(bh_sched* s, const void* model_output, int i, void* sample, int64_t numel,
                  int dtype, void* stream);
/* reset (dpm_solver.cpp:84-87): forget the history; the next step is first order. */
int bh_sched_reset(bh_sched* s);
void bh_sched_destroy(bh_sched* s);

/* Pipeline::generate's denoise loop (pipeline.cpp:104-131) with every step on the device: per
 * step repeat -> bh_dit_forward at timestep(i) -> guidance -> bh_sched_step, with no host copy
 * and no host synchronisation (the reference copies eps and the latent to the host and back
 * every step, pipeline.cpp:127-130). */
typedef struct bh_denoiser bh_denoiser;

/* `e` must have batch 2 when classifier_free_guidance is set (negative prompt first, as the
 * reference requires, pipeline.cpp:69-75) and batch 1 otherwise; `s` must have timesteps set.
 * Allocates the batched latent, the prediction, eps and the scheduler's history. Both `e` and
 * `s` must outlive the denoiser. */
int bh_denoiser_create(bh_dit* e, bh_sched* s, int classifier_free_guidance,
                       float guidance_scale, bh_denoiser** out);
/* Resets the scheduler and runs every step of its schedule on `latent` [1, in_ch, H, W] (bf16,
 * device, updated in place). With use_graph, the whole loop is captured once into a HIP graph
 * per (latent, caption, caption_mask, mask_dtype) binding and replayed on later calls; the
 * schedule and guidance scale are part of the capture, so bh_sched_set_timesteps on `s`
 * invalidates it. Capture needs the launch profiler off. */
int bh_denoiser_run(bh_denoiser* d, void* latent, const void* caption, const void* caption_mask,
                    int mask_dtype, int use_graph, void* stream);
void bh_denoiser_destroy(bh_denoiser* d);

/* ---- measurement and inputs --------------------------------------------------------------- */

/* Kernel classes timed by the launch profiler. */
typedef enum bh_kernel_class {
    BH_K_GEMM = 0,        /* the MFMA GEMM, every shape */
    BH_K_GEMV = 1,        /* small-M GEMMs (timestep / adaLN projections) */
    BH_K_ATTN_SELF = 2,   /* flash attention, kv_len == q_len */
    BH_K_ATTN_CROSS = 3,  /* flash attention, kv_len != q_len */
    BH_K_NORM = 4,        /* LayerNorm and LayerNorm+modulate */
    BH_K_ELEMENTWISE = 5, /* modulate, add, chunk, activation, patch, embeddings */
    BH_K_GEMM_FF0 = 6,    /* engine: the [M,4608,1152] GELU projection (also counted as GEMM) */
    BH_K_GEMM_FF2 = 7,    /* engine: the [M,1152,4608] projection (also counted as GEMM) */
    BH_K_GEMM_QKV = 8,    /* engine: the fused [M,3456,1152] projection (also counted as GEMM) */
    BH_K_COUNT = 9
} bh_kernel_class;

/* When enabled, every launch is bracketed by HIP events on its own stream and the elapsed
 * time is accumulated per class. Enabling resets the counters. Costs a little per launch;
 * off by default. */
int bh_profile_enable(int class_mask);
/* Bracket only the first of every `every` launches of each enabled class (counted per class from
 * bh_profile_enable; 1, the default, brackets every launch). A sampled profile perturbs the
 * stream it measures less: the launches between samples run with no event around them. It has no
 * counterpart in the reference, whose timer brackets whole iterations. */
int bh_profile_sample(int every);
/* Sums since enable, synchronising on the recorded events: total ms, launches and algorithmic
 * FLOP (or bytes, for the bandwidth classes) per class. */
int bh_profile_read(int kernel_class, double* total_ms, int64_t* launches, double* work);

/* Fills host memory with N(0, std^2) draws, rounded to bf16: Box-Muller over a splitmix64
 * stream seeded from `seed` and the FNV-1a hash of `name` (the reference's per-name keying,
 * weights.cpp:87-88, and noise recipe, pipeline.cpp:41-58). Element i uses stream draws
 * 2*(i/2) and 2*(i/2)+1, so the result does not depend on how the work is split. Host only. */
int bh_fill_normal_bf16(uint16_t* dst, int64_t n, uint64_t seed, const char* name, float std_dev);

/* ---- the VAE decoder (the vae-decode stage, vae_decoder.cpp) ------------------------------ */

/* VaeConfig (models.h:120-130). */
typedef struct bh_vae_config {
    int block_out_channels[8]; /* {128, 256, 512, 512}: decoder up-blocks use them reversed */
    int num_blocks;            /* 4 */
    int layers_per_block;      /* 2: each up-block has layers_per_block + 1 resnets */
    int latent_channels;       /* 4 */
    int norm_num_groups;       /* 32 */
    double eps;                /* 1e-6 */
} bh_vae_config;

/* The decoder's weights by checkpoint name (the VAE part of declare_pixart_shapes,
 * weights.cpp:284-320): `count` names, each with a bf16 tensor in the checkpoint layout
 * (convolutions [out, in, k, k]; linear [out, in]; norms [channels]). */
typedef struct bh_vae_weights {
    int count;
    const char* const* names;
    const void* const* tensors;
} bh_vae_weights;

typedef struct bh_vae bh_vae;

/* Prepares VaeDecoder::forward (vae_decoder.cpp:127-180) for one latent side (batch 1): checks the
 * configuration, repacks the 3x3 convolution weights for the implicit-GEMM kernel and allocates
 * every activation once (4 buffers of the largest layer, the attention's Q/K/V/O). The weight
 * pointers must stay valid for the engine's lifetime. This call allocates; decode does not. */
int bh_vae_create(const bh_vae_config* cfg, const bh_vae_weights* w, int64_t latent_hw, bh_vae** out);
/* latent [1, latent_channels, h, h] -> image [1, 3, h*f, h*f] (f = 2^(num_blocks-1)), bf16 NCHW
 * device pointers, on `stream`. No host synchronisation. The latent is NOT divided by the
 * scaling factor here, as in the reference (the pipeline does that, burnisher_main.cpp:661-663). */
int bh_vae_decode(bh_vae* e, const void* latent, void* image, void* stream);
/* Device bytes the engine holds. */
int64_t bh_vae_workspace_bytes(const bh_vae* e);
void bh_vae_destroy(bh_vae* e);

/* ---- checkpoints: safetensors shards and the DiT's device weights -------------------------- */

/* Element types a safetensors header may name (safetensors.cpp:186-195). */
typedef enum bh_st_dtype { BH_ST_F32 = 0, BH_ST_BF16 = 1, BH_ST_F16 = 2, BH_ST_F8_E4M3 = 3 } bh_st_dtype;

typedef struct bh_checkpoint bh_checkpoint;

/* CheckpointWeights(paths) (weights.cpp:51-54) over SafeTensors::open (safetensors.cpp:207-250):
 * every shard memory-mapped read-only and its header parsed and checked (dtype known, byte range
 * equal to shape x dtype size, inside the file). Host only. */
int bh_checkpoint_open(const char* const* shard_paths, int n_shards, bh_checkpoint** out);
/* CheckpointWeights::component (weights.cpp:26-49): the sorted *.safetensors of <dir>/<component>. */
int bh_checkpoint_open_component(const char* dir, const char* component, bh_checkpoint** out);
void bh_checkpoint_close(bh_checkpoint* ck);
/* Number of tensors over all shards (-1 for a null handle); entries are in shard order, then
 * name order within a shard. */
int64_t bh_checkpoint_count(const bh_checkpoint* ck);
/* Entry `index`: its name (valid while the checkpoint is open), bh_st_dtype and shape. */
int bh_checkpoint_entry(const bh_checkpoint* ck, int64_t index, const char** name, int* dtype,
                        int* rank, int64_t* shape, int max_rank);
/* WeightSource::require (weights.cpp:14-24, 56-65): the entry named `name` in the first shard
 * holding it; a miss is an error naming up to five near misses (safetensors.cpp:256-280). */
int bh_checkpoint_find(const bh_checkpoint* ck, const char* name, int* dtype, int* rank,
                       int64_t* shape, int max_rank);
/* Tensor::convert_into (tensor.cpp:130-160): `numel` elements of `name` into host memory as
 * `dtype` (BH_BF16: fp32 rounded to nearest even; BH_F32). F16 and F8_E4M3 have no per-element
 * conversion in the reference (tensor.cpp:68-82) and are refused. */
int bh_checkpoint_read(const bh_checkpoint* ck, const char* name, int dtype, void* dst,
                       int64_t numel);

typedef struct bh_dit_device_weights bh_dit_device_weights;

/* DeviceWeights over the DiT's tensors (weights.cpp:198-217, names and shapes of
 * declare_pixart_shapes, weights.cpp:246-282): every tensor the configuration needs is checked
 * (present, shape, F32 or BF16) before anything is allocated, then converted to bf16 on the host
 * into page-locked staging and copied into one device arena on `stream`. Returns after the
 * copies have completed. Allocates (the arena, 32 MiB of staging while it runs). */
int bh_dit_weights_load(const bh_checkpoint* ck, const bh_dit_config* cfg, void* stream,
                        bh_dit_device_weights** out);
/* The loaded weights as the struct bh_dit_create takes; valid until bh_dit_weights_free. */
const bh_dit_weights* bh_dit_weights_view(const bh_dit_device_weights* w);
/* Device bytes of the arena (-1 for a null handle). */
int64_t bh_dit_weights_bytes(const bh_dit_device_weights* w);
void bh_dit_weights_free(bh_dit_device_weights* w);

typedef struct bh_vae_device_weights bh_vae_device_weights;

/* DeviceWeights over the VAE decoder's tensors (the `vae/` component; names and shapes of
 * declare_pixart_shapes' VAE part, weights.cpp:284-320): checked (present, shape, F32 or BF16)
 * before anything is allocated, converted to bf16 on the host and copied into one device arena.
 * Allocates. */
int bh_vae_weights_load(const bh_checkpoint* ck, const bh_vae_config* cfg, void* stream,
                        bh_vae_device_weights** out);
/* The loaded weights as the table bh_vae_create takes; valid until bh_vae_weights_free. */
const bh_vae_weights* bh_vae_weights_view(const bh_vae_device_weights* w);
int64_t bh_vae_weights_bytes(const bh_vae_device_weights* w);
void bh_vae_weights_free(bh_vae_device_weights* w);

/* ---- the T5 v1.1 text encoder (the t5-encode stage, t5_encoder.cpp) ------------------------ */

/* T5Config (models.h:94-103), plus the relative-position table's bucket count: the first
 * dimension of relative_attention_bias.weight (weights.cpp:231-232; the reference reads it off
 * that tensor, t5_encoder.cpp:95). The bucket table's max_distance is 128, as there. */
typedef struct bh_t5_config {
    int num_layers;   /* 24 */
    int d_model;      /* 4096 */
    int d_ff;         /* 10240 */
    int d_kv;         /* 64 */
    int num_heads;    /* 64 */
    int vocab_size;   /* 32128 */
    int gated;        /* 1: gelu(wi_0 x) * (wi_1 x); 0: gelu(wi_0 x) */
    int num_buckets;  /* 32 */
    double eps;       /* 1e-6 */
} bh_t5_config;

/* The encoder's weights by checkpoint name (the T5 part of declare_pixart_shapes,
 * weights.cpp:226-244): bf16 tensors, linear weights [out, in], norms [d_model], the shared
 * embedding [vocab_size, d_model], the relative bias [num_buckets, num_heads]. */
typedef struct bh_t5_weights {
    int count;
    const char* const* names;
    const void* const* tensors;
} bh_t5_weights;

typedef struct bh_t5 bh_t5;

/* t5_relative_bucket (t5_encoder.cpp:34-48): the bidirectional bucket of key minus query
 * position. Host only; the encoder builds its table with it. */
int bh_t5_relative_bucket(int relative_position, int num_buckets, int max_distance);

/* GatherArgs (ops.h:198-207): out[r, :] = table[(int64)ids[r], :] for r < rows, ids fp32 on the
 * device (the reference's contract), table [table_rows, cols]. A row whose id lies outside
 * [0, table_rows) is written as NaN instead of being read out of bounds. Replaces `gather_cuda`
 * (src/cuda/ops_cuda.cu:1097-1115). */
int bh_gather(const void* table, const float* ids, void* out, int64_t rows, int64_t cols,
              int64_t table_rows, int dtype, void* stream);

/* Prepares T5Encoder::forward (t5_encoder.cpp:132-241) for [batch, seq_len] token ids: checks
 * the configuration and every weight name, packs each layer's q/k/v weights into one [3*inner,
 * d_model] operand and wi_0/wi_1 into one [2*d_ff, d_model] operand (engine-owned copies, so
 * each projection is one GEMM), and allocates every activation once. The caller's weight
 * pointers must stay valid for the engine's lifetime. Allocates; encode does not. */
int bh_t5_create(const bh_t5_config* cfg, const bh_t5_weights* w, int64_t batch, int64_t seq_len,
                 bh_t5** out);
/* token_ids: HOST fp32 [batch, seq_len] (integers, pad id 0), checked against the vocabulary
 * before any device work as the reference does (t5_encoder.cpp:146-156); out: device bf16
 * [batch, seq_len, d_model]. The key mask (id != 0) and the relative-bias table [heads, seq,
 * seq] are rebuilt from the ids and the weights on every call. On `stream`; it waits only for
 * the previous call's id upload before reusing that staging buffer. */
int bh_t5_encode(bh_t5* e, const float* token_ids, void* out, void* stream);
/* Device bytes the engine holds (activations, packed weights, bias table). */
int64_t bh_t5_workspace_bytes(const bh_t5* e);
void bh_t5_destroy(bh_t5* e);

typedef struct bh_t5_device_weights bh_t5_device_weights;

/* DeviceWeights over the T5 encoder's tensors (the `text_encoder/` component, sharded or not;
 * names and shapes of declare_pixart_shapes' T5 part, weights.cpp:226-244): checked (present,
 * shape, F32 or BF16) before anything is allocated, converted to bf16 on the host and copied into
 * one device arena. Allocates. */
int bh_t5_weights_load(const bh_checkpoint* ck, const bh_t5_config* cfg, void* stream,
                       bh_t5_device_weights** out);
/* The loaded weights as the table bh_t5_create takes; valid until bh_t5_weights_free. */
const bh_t5_weights* bh_t5_weights_view(const bh_t5_device_weights* w);
int64_t bh_t5_weights_bytes(const bh_t5_device_weights* w);
void bh_t5_weights_free(bh_t5_device_weights* w);

#ifdef __cplusplus
}
#endif

#endif /* BURNISHER_HIP_H */
