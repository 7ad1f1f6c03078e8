// The C ABI of libburnisher_hip.so (include/burnisher_hip.h): argument checking, dispatch to
// the kernels, the per-class launch profiler and the seeded input generator.
//
// Errors are C++ exceptions inside the library and become a nonzero status plus a thread-local
// message at this boundary, mirroring the reference runtime's `throw std::runtime_error` naming
// the contract (src/cuda/ops_cuda.cu:79-107): a host pointer, a dtype the kernel does not have,
// a shape it cannot honour -- each is refused with a sentence, never run approximately.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/burnisher_hip.h"
#include "common.h"

namespace bh {
namespace {

thread_local std::string g_error;
thread_local bool g_operand_checks = true;

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

bool is_f32(int dtype) {
    if (dtype == BH_F32) return true;
    if (dtype == BH_BF16) return false;
    throw Error("dtype " + std::to_string(dtype) + " has no kernel in hip-gfx950 (bf16 or fp32)");
}

void require_nonneg(int64_t v, const char* op, const char* what) {
    if (v < 0) throw Error(std::string(op) + ": " + what + " is negative");
}

// ---- launch profiler ------------------------------------------------------------------------

struct Record {
    int cls, also;
    hipEvent_t start, stop;
    double work;
};

struct Profiler {
    std::mutex mu;
    int mask = 0;
    int every = 1;                  // bracket every `every`-th launch of a class
    int64_t seen[K_COUNT] = {};     // launches of each enabled class since enable
    std::vector<hipEvent_t> free_events;
    std::vector<Record> pending;
    double total_ms[K_COUNT] = {};
    int64_t launches[K_COUNT] = {};
    double work[K_COUNT] = {};

    hipEvent_t take() {
        if (!free_events.empty()) {
            hipEvent_t e = free_events.back();
            free_events.pop_back();
            return e;
        }
        hipEvent_t e;
        hip_check(hipEventCreate(&e), "hipEventCreate");
        return e;
    }
    void settle(size_t count) {
        count = std::min(count, pending.size());
        for (size_t i = 0; i < count; ++i) {
            Record& r = pending[i];
            hip_check(hipEventSynchronize(r.stop), "hipEventSynchronize");
            float ms = 0.f;
            hip_check(hipEventElapsedTime(&ms, r.start, r.stop), "hipEventElapsedTime");
            for (int c : {r.cls, r.also}) {
                if (c < 0) continue;
                total_ms[c] += ms;
                launches[c] += 1;
                work[c] += r.work;
            }
            free_events.push_back(r.start);
            free_events.push_back(r.stop);
        }
        pending.erase(pending.begin(), pending.begin() + static_cast<long>(count));
    }
};

Profiler& profiler() {
    static Profiler* p = new Profiler();  // outlives static destructors that might still launch
    return *p;
}

thread_local int g_gemm_subclass = -1;

}  // namespace

bool profiling_enabled() { return profiler().mask != 0; }

ProfileScope::ProfileScope(int cls, hipStream_t stream, double work, int also)
    : cls_(cls), also_(also), stream_(stream), work_(work) {
    Profiler& p = profiler();
    if (p.mask == 0) return;
    const bool want = (p.mask >> cls) & 1 || (also >= 0 && ((p.mask >> also) & 1));
    if (!want) return;
    std::lock_guard<std::mutex> lock(p.mu);
    if (p.seen[cls]++ % p.every != 0) return;
    if (p.pending.size() >= 16384) p.settle(8192);
    Record r{(p.mask >> cls) & 1 ? cls : -1, (also >= 0 && ((p.mask >> also) & 1)) ? also : -1,
             p.take(), p.take(), work};
    hip_check(hipEventRecord(r.start, stream), "hipEventRecord");
    p.pending.push_back(r);
    slot_ = static_cast<int>(p.pending.size()) - 1;
}

ProfileScope::~ProfileScope() {
    if (slot_ < 0) return;
    Profiler& p = profiler();
    std::lock_guard<std::mutex> lock(p.mu);
    if (slot_ < static_cast<int>(p.pending.size())) {
        (void)hipEventRecord(p.pending[slot_].stop, stream_);
    }
}

void set_gemm_subclass(int cls) { g_gemm_subclass = cls; }

void set_last_error(const std::string& msg) { g_error = msg; }
bool operand_checks() { return g_operand_checks; }
int gemm_subclass() { return g_gemm_subclass; }

}  // namespace bh

using namespace bh;

extern "C" {

int bh_abi_version(void) { return BH_ABI_VERSION; }

const char* bh_build_info(void) {
    return "burnisher-hip gfx950: bf16 MFMA GEMM 256x144x64, flash attention 16x16x32, "
           "fp64-statistics LayerNorm";
}

const char* bh_last_error(void) { return g_error.c_str(); }

int bh_set_operand_checks(int on) {
    bh::g_operand_checks = on != 0;
    bh::set_last_error("");
    return 0;
}

int bh_init(int device) {
    return guarded([&] {
        int count = 0;
        hip_check(hipGetDeviceCount(&count), "hipGetDeviceCount");
        require(device >= 0 && device < count,
                "bh_init: device " + std::to_string(device) + " of " + std::to_string(count));
        hip_check(hipSetDevice(device), "hipSetDevice");
        hipDeviceProp_t prop;
        hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
        const std::string arch = prop.gcnArchName;
        require(arch.rfind("gfx950", 0) == 0,
                "bh_init: device " + std::to_string(device) + " is " + arch +
                    "; this library holds gfx950 code only");
        // the allocation-free attention's scratch address on this device, looked up once
        (void)noalloc_scratch();
    });
}

int bh_synchronize(void* stream) {
    return guarded([&] { hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); });
}

int bh_gemm(const void* a, const void* b, const void* bias, void* out, int64_t m, int64_t n,
            int64_t k, int b_transposed, int epilogue, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "gemm (hip-gfx950)";
        require_nonneg(m, op, "m");
        require_nonneg(n, op, "n");
        require_nonneg(k, op, "k");
        if (m * n == 0) return;
        require_device_ptr(a, op, "a");
        require_device_ptr(b, op, "b");
        require_device_ptr(out, op, "out");
        optional_device_ptr(bias, op, "bias");
        require(epilogue >= BH_EPI_NONE && epilogue <= BH_EPI_SILU,
                epilogue == BH_EPI_GELU_GATED
                    ? std::string("gemm (hip-gfx950): GeluGated is the T5 FFN and has no kernel here")
                    : std::string("gemm (hip-gfx950): unknown epilogue"));
        const bool f32 = is_f32(dtype);
        if (f32 || !b_transposed) {
            ProfileScope ps(K_GEMM, as_stream(stream), 2.0 * m * n * k);
            launch_gemm_generic(a, b, bias, out, m, n, k, b_transposed != 0, epilogue, f32,
                                as_stream(stream));
            return;
        }
        GemmEpilogue ep;
        ep.act = epilogue;
        launch_gemm_bf16(static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                         static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(out), m, n, k, ep,
                         as_stream(stream));
    });
}

int bh_gemm_fused_run(const void* a, const void* b, const void* bias, void* out, int64_t m,
                      int64_t n, int64_t k, const bh_gemm_fused* f, void* stream) {
    return guarded([&] {
        const char* op = "gemm_fused (hip-gfx950)";
        require(f != nullptr, "gemm_fused: null epilogue description");
        require_nonneg(m, op, "m");
        require_nonneg(n, op, "n");
        require_nonneg(k, op, "k");
        if (m * n == 0) return;
        require_device_ptr(a, op, "a");
        require_device_ptr(b, op, "b");
        require_device_ptr(out, op, "out");
        optional_device_ptr(bias, op, "bias");
        optional_device_ptr(f->row_add, op, "row_add");
        optional_device_ptr(f->residual, op, "residual");
        optional_device_ptr(f->gate, op, "gate");
        require(f->epilogue >= BH_EPI_NONE && f->epilogue <= BH_EPI_SILU,
                "gemm_fused: unknown epilogue");
        require(!f->gate || f->residual, "gemm_fused: a gate needs a residual");
        require(!f->row_add || f->row_add_period > 0, "gemm_fused: row_add_period must be > 0");
        require(!f->gate || f->gate_rows > 0, "gemm_fused: gate_rows must be > 0");
        require(f->ld_out == 0 || f->ld_out >= n, "gemm_fused: ld_out below n");
        GemmEpilogue ep;
        ep.act = f->epilogue;
        ep.round_mid = f->round_mid != 0;
        ep.row_add = static_cast<const bf16_t*>(f->row_add);
        ep.row_add_period = f->row_add_period;
        ep.residual = static_cast<const bf16_t*>(f->residual);
        ep.gate = static_cast<const bf16_t*>(f->gate);
        ep.gate_rows = f->gate_rows;
        ep.ld_out = f->ld_out;
        launch_gemm_bf16(static_cast<const bf16_t*>(a), static_cast<const bf16_t*>(b),
                         static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(out), m, n, k, ep,
                         as_stream(stream));
    });
}

namespace {
int attention_impl(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_kv,
                   void* out, int64_t ld_o, int64_t batch, int64_t heads, int64_t q_len,
                   int64_t kv_len, int64_t head_dim, float scale, const void* bias,
                   const void* key_mask, int mask_dtype, int dtype, void* stream,
                   bool noalloc = false) {
    return guarded([&] {
        const char* op = noalloc ? "attention_noalloc (hip-gfx950)" : "attention (hip-gfx950)";
        require_nonneg(batch, op, "batch");
        require_nonneg(heads, op, "heads");
        require_nonneg(q_len, op, "q_len");
        require_nonneg(kv_len, op, "kv_len");
        require(head_dim > 0, "attention: head_dim must be positive");
        if (batch * heads * q_len == 0) return;
        require(kv_len > 0, "attention: kv_len must be positive when there are queries");
        require_device_ptr(q, op, "q");
        require_device_ptr(k, op, "k");
        require_device_ptr(v, op, "v");
        require_device_ptr(out, op, "out");
        optional_device_ptr(bias, op, "bias");
        optional_device_ptr(key_mask, op, "key_mask");
        const bool f32 = is_f32(dtype);
        const bool mask_f32 = key_mask ? is_f32(mask_dtype) : false;
        AttnShape sh{batch, heads, q_len, kv_len, head_dim, ld_q, ld_kv, ld_o,
                     // 0 means 1/sqrt(head_dim), computed exactly as the oracle does.
                     scale > 0.0f ? scale : 1.0f / std::sqrt(static_cast<float>(head_dim))};
        const bool flash512 = head_dim == 512 && heads == 1 && q_len == kv_len && !key_mask &&
                              ld_q == 512 && ld_kv == 512 && ld_o == 512;
        if (f32 || (bias && head_dim > 128) || (head_dim > 128 && !flash512)) {
            ProfileScope ps(q_len == kv_len ? K_ATTN_SELF : K_ATTN_CROSS, as_stream(stream),
                            4.0 * batch * heads * static_cast<double>(q_len) * kv_len * head_dim);
            launch_attention_generic(q, k, v, out, sh, bias, key_mask, mask_f32, f32,
                                     as_stream(stream));
            return;
        }
        const auto* qb = static_cast<const bf16_t*>(q);
        const auto* kb = static_cast<const bf16_t*>(k);
        const auto* vb = static_cast<const bf16_t*>(v);
        auto* ob = static_cast<bf16_t*>(out);
        const auto* bb = static_cast<const bf16_t*>(bias);
        if (!noalloc) {
            launch_attention_bf16(qb, kb, vb, ob, sh, key_mask, mask_f32, as_stream(stream), bb);
            return;
        }
        // V^T and the key-split partials (the same splits bh_attention takes, so both give the
        // same bits) into the fixed per-device scratch: nothing is allocated, so the call is
        // refused when they would not fit.
        const int64_t need = attention_vt_elems(qb, kb, vb, ob, sh, key_mask, bb);
        const int64_t part_floats = attention_part_floats(qb, kb, vb, ob, sh, key_mask, bb);
        const int64_t vt_bytes = (need * 2 + 255) / 256 * 256;
        const int64_t total = vt_bytes + part_floats * 4;
        require(total <= kNoAllocScratchBytes,
                "attention_noalloc: V^T and the key-split partials need " + std::to_string(total) +
                    " bytes of scratch, above the fixed maximum of " +
                    std::to_string(kNoAllocScratchBytes) +
                    " bytes (use bh_attention, which grows its workspace)");
        bf16_t* base = total > 0 ? noalloc_scratch() : nullptr;
        float* part = part_floats > 0 ? reinterpret_cast<float*>(reinterpret_cast<char*>(base) + vt_bytes)
                                      : nullptr;
        launch_attention_bf16(qb, kb, vb, ob, sh, key_mask, mask_f32, as_stream(stream), bb,
                              need > 0 ? base : nullptr, vt_bytes / 2, part_floats > 0 ? 0 : 1, part,
                              part_floats);
    });
}
}  // namespace

int bh_attention(const void* q, const void* k, const void* v, void* out, int64_t batch,
                 int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                 const void* bias, const void* key_mask, int mask_dtype, int dtype, void* stream) {
    const int64_t ld = heads * head_dim;
    return attention_impl(q, ld, k, v, ld, out, ld, batch, heads, q_len, kv_len, head_dim, scale,
                          bias, key_mask, mask_dtype, dtype, stream);
}

int bh_attention_noalloc(const void* q, const void* k, const void* v, void* out, int64_t batch,
                         int64_t heads, int64_t q_len, int64_t kv_len, int64_t head_dim, float scale,
                         const void* bias, const void* key_mask, int mask_dtype, int dtype,
                         void* stream) {
    const int64_t ld = heads * head_dim;
    return attention_impl(q, ld, k, v, ld, out, ld, batch, heads, q_len, kv_len, head_dim, scale,
                          bias, key_mask, mask_dtype, dtype, stream, true);
}

int bh_attention_strided(const void* q, int64_t ld_q, const void* k, const void* v, int64_t ld_kv,
                         void* out, int64_t ld_out, int64_t batch, int64_t heads, int64_t q_len,
                         int64_t kv_len, int64_t head_dim, float scale, const void* key_mask,
                         int mask_dtype, int dtype, void* stream) {
    const int64_t row = heads * head_dim;
    if (ld_q < row || ld_kv < row || ld_out < row) {
        g_error = "attention_strided: a row stride is below heads * head_dim";
        return 1;
    }
    return attention_impl(q, ld_q, k, v, ld_kv, out, ld_out, batch, heads, q_len, kv_len,
                          head_dim, scale, nullptr, key_mask, mask_dtype, dtype, stream);
}

int bh_gather(const void* table, const float* ids, void* out, int64_t rows, int64_t cols,
              int64_t table_rows, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "gather (hip-gfx950)";
        require_nonneg(rows, op, "rows");
        require_nonneg(cols, op, "cols");
        require_nonneg(table_rows, op, "table_rows");
        if (rows == 0 || cols == 0) return;
        require_device_ptr(table, op, "table");
        require_device_ptr(ids, op, "ids");
        require_device_ptr(out, op, "out");
        launch_gather(table, ids, out, rows, cols, table_rows, is_f32(dtype), as_stream(stream));
    });
}

int bh_norm(const void* x, const void* weight, const void* bias, void* out, int64_t rows,
            int64_t cols, float eps, int rms, int64_t groups, int64_t channels, int dtype,
            void* stream) {
    return guarded([&] {
        const char* op = "norm (hip-gfx950)";
        require_nonneg(rows, op, "rows");
        require(cols > 0 || rows == 0, "norm: cols must be positive");
        if (groups > 0) {   // GroupNorm (the VAE's), NCHW rows of channels * spatial
            require(!rms, "norm: GroupNorm has no RMS form");
            require(!is_f32(dtype), "norm (hip-gfx950): GroupNorm is bf16 only");
            if (rows == 0) return;
            require_device_ptr(x, op, "x");
            require_device_ptr(out, op, "out");
            optional_device_ptr(weight, op, "weight");
            optional_device_ptr(bias, op, "bias");
            launch_group_norm_nchw(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(weight),
                                   static_cast<const bf16_t*>(bias), static_cast<bf16_t*>(out), rows,
                                   cols, eps, groups, channels, as_stream(stream));
            return;
        }
        if (rows == 0) return;
        require_device_ptr(x, op, "x");
        require_device_ptr(out, op, "out");
        optional_device_ptr(weight, op, "weight");
        optional_device_ptr(bias, op, "bias");
        ProfileScope ps(K_NORM, as_stream(stream), 2.0 * rows * cols * (is_f32(dtype) ? 4 : 2));
        launch_norm(x, weight, bias, out, rows, cols, eps, rms != 0, is_f32(dtype),
                    as_stream(stream));
    });
}

int bh_modulate(const void* x, const void* scale, const void* shift, void* out, int64_t batch,
                int64_t tokens, int64_t channels, const void* residual, const void* gate,
                int dtype, void* stream) {
    return guarded([&] {
        const char* op = "modulate (hip-gfx950)";
        require_nonneg(batch, op, "batch");
        require_nonneg(tokens, op, "tokens");
        require_nonneg(channels, op, "channels");
        if (batch * tokens * channels == 0) return;
        require_device_ptr(x, op, "x");
        require_device_ptr(scale, op, "scale");
        require_device_ptr(shift, op, "shift");
        require_device_ptr(out, op, "out");
        optional_device_ptr(residual, op, "residual");
        optional_device_ptr(gate, op, "gate");
        const double es = is_f32(dtype) ? 4 : 2;
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream),
                        es * batch * tokens * channels * (2 + (residual ? 1 : 0)));
        launch_modulate(x, scale, shift, out, batch, tokens, channels, residual, gate,
                        is_f32(dtype), as_stream(stream));
    });
}

int bh_activation(const void* x, void* out, int64_t numel, int kind, const void* gate, int dtype,
                  void* stream) {
    return guarded([&] {
        const char* op = "activation (hip-gfx950)";
        require_nonneg(numel, op, "numel");
        require(kind >= BH_EPI_NONE && kind <= BH_EPI_GELU_GATED, "activation: unknown kind");
        require(kind != BH_EPI_GELU_GATED || gate, "activation: GeluGated needs a gate");
        if (numel == 0) return;
        require_device_ptr(x, op, "x");
        require_device_ptr(out, op, "out");
        optional_device_ptr(gate, op, "gate");
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream), 2.0 * numel * (is_f32(dtype) ? 4 : 2));
        launch_activation(x, out, numel, kind, gate, is_f32(dtype), as_stream(stream));
    });
}

int bh_add(const void* a, const void* b, void* out, int64_t outer, int64_t inner, float scale,
           int broadcast_b, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "add (hip-gfx950)";
        require_nonneg(outer, op, "outer");
        require_nonneg(inner, op, "inner");
        if (outer * inner == 0) return;
        require_device_ptr(a, op, "a");
        require_device_ptr(b, op, "b");
        require_device_ptr(out, op, "out");
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream), 3.0 * outer * inner * (is_f32(dtype) ? 4 : 2));
        launch_add(a, b, out, outer, inner, scale, broadcast_b != 0, is_f32(dtype),
                   as_stream(stream));
    });
}

int bh_chunk(const void* modulation, const void* table, void* out, int64_t batch,
             int64_t channels, int64_t chunks, int64_t chunk, int64_t table_chunk, int dtype,
             void* stream) {
    return guarded([&] {
        const char* op = "chunk (hip-gfx950)";
        require_nonneg(batch, op, "batch");
        require_nonneg(channels, op, "channels");
        require(chunk >= 0 && chunk < chunks, "chunk: chunk index outside [0, chunks)");
        if (batch * channels == 0) return;
        require_device_ptr(modulation, op, "modulation");
        require_device_ptr(table, op, "table");
        require_device_ptr(out, op, "out");
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream), 3.0 * batch * channels * (is_f32(dtype) ? 4 : 2));
        launch_chunk(modulation, table, out, batch, channels, chunks, chunk, table_chunk,
                     is_f32(dtype), as_stream(stream));
    });
}

int bh_patch(const void* in, void* out, int64_t batch, int64_t channels, int64_t grid,
             int64_t patch, int inverse, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "patch (hip-gfx950)";
        require_nonneg(batch, op, "batch");
        require_nonneg(channels, op, "channels");
        require_nonneg(grid, op, "grid");
        require(patch > 0, "patch: patch size must be positive");
        if (batch * channels * grid == 0) return;
        require_device_ptr(in, op, "in");
        require_device_ptr(out, op, "out");
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream),
                        2.0 * batch * channels * grid * grid * patch * patch * (is_f32(dtype) ? 4 : 2));
        launch_patch(in, out, batch, channels, grid, patch, inverse != 0, is_f32(dtype),
                     as_stream(stream));
    });
}

int bh_scale(const void* in, void* out, int64_t numel, float scale, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "scale (hip-gfx950)";
        require_nonneg(numel, op, "numel");
        if (numel == 0) return;
        require_device_ptr(in, op, "in");
        require_device_ptr(out, op, "out");
        ProfileScope ps(K_ELEMENTWISE, as_stream(stream), 2.0 * numel * (is_f32(dtype) ? 4 : 2));
        launch_scale(in, out, numel, scale, is_f32(dtype), as_stream(stream));
    });
}

int bh_timestep_embedding(double t, int dim, int64_t batch, void* out, int dtype, void* stream) {
    return guarded([&] {
        const char* op = "timestep_embedding (hip-gfx950)";
        require(dim > 0 && dim % 2 == 0, "timestep embedding needs an even dimension");
        require_nonneg(batch, op, "batch");
        if (batch == 0) return;
        require_device_ptr(out, op, "out");
        launch_timestep_embedding(t, dim, batch, out, is_f32(dtype), as_stream(stream));
    });
}

int bh_norm_modulate(const void* x, const void* mod, int64_t mod_chunks, int64_t shift_chunk,
                     int64_t scale_chunk, const void* table, int64_t shift_row, int64_t scale_row,
                     void* out, int64_t batch, int64_t tokens, int64_t channels, float eps,
                     void* stream) {
    return guarded([&] {
        const char* op = "norm_modulate (hip-gfx950)";
        require_nonneg(batch, op, "batch");
        require_nonneg(tokens, op, "tokens");
        require(channels > 0, "norm_modulate: channels must be positive");
        require(shift_chunk >= 0 && shift_chunk < mod_chunks && scale_chunk >= 0 &&
                    scale_chunk < mod_chunks,
                "norm_modulate: chunk index outside [0, mod_chunks)");
        require(shift_row >= 0 && scale_row >= 0, "norm_modulate: negative table row");
        if (batch * tokens == 0) return;
        require_device_ptr(x, op, "x");
        require_device_ptr(mod, op, "mod");
        require_device_ptr(table, op, "table");
        require_device_ptr(out, op, "out");
        ProfileScope ps(K_NORM, as_stream(stream), 4.0 * batch * tokens * channels);
        launch_norm_modulate(static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(mod),
                             mod_chunks, shift_chunk, scale_chunk,
                             static_cast<const bf16_t*>(table), shift_row, scale_row,
                             static_cast<bf16_t*>(out), batch, tokens, channels, eps,
                             as_stream(stream));
    });
}

int bh_profile_enable(int mask) {
    return guarded([&] {
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.settle(p.pending.size());
        p.mask = mask & ((1 << K_COUNT) - 1);
        std::fill(std::begin(p.seen), std::end(p.seen), 0);
        std::fill(std::begin(p.total_ms), std::end(p.total_ms), 0.0);
        std::fill(std::begin(p.launches), std::end(p.launches), 0);
        std::fill(std::begin(p.work), std::end(p.work), 0.0);
    });
}

int bh_profile_sample(int every) {
    return guarded([&] {
        require(every >= 1, "profile_sample: every must be at least 1");
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.every = every;
    });
}

int bh_profile_read(int kernel_class, double* total_ms, int64_t* launches, double* work) {
    return guarded([&] {
        require(kernel_class >= 0 && kernel_class < K_COUNT, "profile_read: unknown class");
        Profiler& p = profiler();
        std::lock_guard<std::mutex> lock(p.mu);
        p.settle(p.pending.size());
        if (total_ms) *total_ms = p.total_ms[kernel_class];
        if (launches) *launches = p.launches[kernel_class];
        if (work) *work = p.work[kernel_class];
    });
}

int bh_fill_normal_bf16(uint16_t* dst, int64_t n, uint64_t seed, const char* name,
                        float std_dev) {
    return guarded([&] {
        require(dst != nullptr || n == 0, "fill_normal: null destination");
        require(n >= 0, "fill_normal: negative count");
        uint64_t h = 0xcbf29ce484222325ull;  // FNV-1a over the name, then mixed with the seed
        for (const char* c = name ? name : ""; *c; ++c) {
            h ^= static_cast<unsigned char>(*c);
            h *= 0x100000001b3ull;
        }
        const uint64_t base = seed ^ h;
        const auto draw = [base](uint64_t index) {  // splitmix64 output number `index` (1-based)
            uint64_t z = base + index * 0x9E3779B97F4A7C15ull;
            z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
            z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
            return static_cast<double>((z ^ (z >> 31)) >> 11) * (1.0 / 9007199254740992.0);
        };
        const int64_t pairs = (n + 1) / 2;
        const auto work = [&](int64_t p0, int64_t p1) {
            for (int64_t p = p0; p < p1; ++p) {
                double u1 = draw(2 * static_cast<uint64_t>(p) + 1);
                const double u2 = draw(2 * static_cast<uint64_t>(p) + 2);
                if (u1 < 1e-300) u1 = 1e-300;
                const double r = std::sqrt(-2.0 * std::log(u1));
                const double t = 2.0 * M_PI * u2;
                dst[2 * p] = f2bf(static_cast<float>(r * std::cos(t) * std_dev));
                if (2 * p + 1 < n) dst[2 * p + 1] = f2bf(static_cast<float>(r * std::sin(t) * std_dev));
            }
        };
        const int64_t threads = std::max<int64_t>(
            1, std::min<int64_t>(std::thread::hardware_concurrency(), pairs / (1 << 16)));
        if (threads <= 1) {
            work(0, pairs);
            return;
        }
        std::vector<std::thread> pool;
        const int64_t per = (pairs + threads - 1) / threads;
        for (int64_t t = 0; t < threads; ++t) {
            const int64_t p0 = t * per, p1 = std::min(pairs, p0 + per);
            if (p0 < p1) pool.emplace_back(work, p0, p1);
        }
        for (auto& th : pool) th.join();
    });
}

}  // extern "C"
