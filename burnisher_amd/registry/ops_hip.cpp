// ops_hip.cpp -- the `hip-gfx950` implementation of every op in Burnisher's registry, as a
// Burnisher maintainer adds it to the reference runtime (as src/hip/ops_hip.cpp, the place of
// src/cuda/ops_cuda.cu:1172-1204 in a ROCm build). Each registration forwards the reference's
// Args struct (include/burnisher/ops.h:17-237) field by field to one entry point of
// libburnisher_hip.so (include/burnisher_hip.h) on the default stream, which is the only stream
// the reference uses (src/cuda/device.cu:72-79), and turns a nonzero status into the
// std::runtime_error the reference's backends throw (ops_cuda.cu:79-107).
//
// Built against the reference's headers, not into libburnisher_hip.so. Registration stores
// function pointers and touches no device (as register_cuda_ops does, tests/test_ops.cpp:
// 318-323); the device is bound on the first op call.
#include <stdexcept>
#include <string>

#include "burnisher/ops.h"
#include "burnisher_hip.h"

namespace burnisher {
namespace {

// The library's dtype for a tensor. Only F32 and BF16 have kernels; the library refuses the rest
// with a message naming the op (F16/FP8/NVFP4 map to a value it rejects).
int dt(const Tensor* t) {
    switch (t->dtype()) {
        case DType::F32: return BH_F32;
        case DType::BF16: return BH_BF16;
        default: return -1;
    }
}
void ok(int status) {
    if (status != 0) throw std::runtime_error(bh_last_error());
}

// An operand's device address, refused with the reference's message when the Tensor lives on
// the host (`require_device`, ops_cuda.cu:79-88). The Tensor says where it lives
// (tensor.h:39), so the library's own per-pointer runtime lookups are switched off in bind().
const void* p(const Tensor* t, const char* op, const char* operand) {
    if (!t) return nullptr;
    if (t->device() != Device::CUDA)
        throw std::runtime_error(std::string("hip-gfx950 ") + op + ": " + operand + " " + t->describe() +
                                 " is a HOST tensor. Mixing host and device operands in one op is a "
                                 "fault, not a slow path.");
    return t->data();
}
void* o(Tensor* t, const char* op) {
    if (!t) throw std::runtime_error(std::string("hip-gfx950 ") + op + ": out is null");
    return const_cast<void*>(p(t, op, "out"));
}

// Binds the calling thread to device 0 (and checks it is a gfx950 part) once per thread, before
// its first op, and switches the library's operand lookups off for this thread (p() checks the
// Tensors instead). Burnisher drives one device from one host thread: the Args carry no stream
// and every backend launches on the default stream (registry.h:34-100, device.cu:72-79).
void bind() {
    thread_local bool bound = false;
    if (!bound) {
        ok(bh_init(0));
        ok(bh_set_operand_checks(0));
        bound = true;
    }
}

void gemm_hip(const GemmArgs& a) {   // replaces gemm_cuda, ops_cuda.cu:476-513
    bind();
    if (a.epilogue == Epilogue::GeluGated)
        throw std::runtime_error("gemm (hip-gfx950): GeluGated is a T5 FFN form that no model graph "
                                 "uses through the gemm op (t5_encoder.cpp:225 gates through the "
                                 "activation op); it has no kernel here");
    ok(bh_gemm(p(a.a, "gemm", "a"), p(a.b, "gemm", "b"), p(a.bias, "gemm", "bias"),
               o(a.out, "gemm"), a.m, a.n, a.k, a.b_transposed ? 1 : 0,
               static_cast<int>(a.epilogue), dt(a.out), nullptr));
}

void attention_hip(const AttentionArgs& a) {   // replaces attention_cuda, ops_cuda.cu:883-886
    bind();
    ok(bh_attention(p(a.q, "attention", "q"), p(a.k, "attention", "k"), p(a.v, "attention", "v"),
                    o(a.out, "attention"), a.batch, a.heads, a.q_len, a.kv_len, a.head_dim, a.scale,
                    p(a.bias, "attention", "bias"), p(a.key_mask, "attention", "key_mask"),
                    a.key_mask ? dt(a.key_mask) : BH_F32, dt(a.out), nullptr));
}

void norm_hip(const NormArgs& a) {   // replaces norm_cuda (LayerNorm, RMSNorm, GroupNorm)
    bind();
    ok(bh_norm(p(a.x, "norm", "x"), p(a.weight, "norm", "weight"), p(a.bias, "norm", "bias"),
               o(a.out, "norm"), a.rows, a.cols, a.eps, a.rms ? 1 : 0, a.groups, a.channels,
               dt(a.out), nullptr));
}

void modulate_hip(const ModulateArgs& a) {   // replaces k_modulate, ops_cuda.cu:194-221
    bind();
    ok(bh_modulate(p(a.x, "modulate", "x"), p(a.scale, "modulate", "scale"),
                   p(a.shift, "modulate", "shift"), o(a.out, "modulate"), a.batch, a.tokens,
                   a.channels, p(a.residual, "modulate", "residual"), p(a.gate, "modulate", "gate"),
                   dt(a.out), nullptr));
}

void activation_hip(const ActivationArgs& a) {   // replaces k_activation, ops_cuda.cu:164-192
    bind();
    ok(bh_activation(p(a.x, "activation", "x"), o(a.out, "activation"), a.numel,
                     static_cast<int>(a.kind), p(a.gate, "activation", "gate"), dt(a.out),
                     nullptr));
}

void conv2d_hip(const Conv2dArgs& a) {   // replaces conv2d_cuda (cuDNN), ops_cuda.cu:897-1015
    bind();
    ok(bh_conv2d(p(a.x, "conv2d", "x"), p(a.weight, "conv2d", "weight"),
                 p(a.bias, "conv2d", "bias"), o(a.out, "conv2d"), a.batch, a.c_in, a.h_in, a.w_in,
                 a.c_out, a.k, a.pad, dt(a.x), nullptr));
}

void add_hip(const AddArgs& a) {   // replaces k_add, ops_cuda.cu:111-132
    bind();
    ok(bh_add(p(a.a, "add", "a"), p(a.b, "add", "b"), o(a.out, "add"), a.outer, a.inner, a.scale,
              a.broadcast_b ? 1 : 0, dt(a.out), nullptr));
}

void chunk_hip(const ChunkArgs& a) {   // replaces k_chunk, ops_cuda.cu:134-156
    bind();
    ok(bh_chunk(p(a.modulation, "chunk", "modulation"), p(a.table, "chunk", "table"),
                o(a.out, "chunk"), a.batch, a.channels, a.chunks, a.chunk, a.table_chunk, dt(a.out),
                nullptr));
}

void patch_hip(const PatchArgs& a) {   // replaces k_patch, ops_cuda.cu:382-415
    bind();
    ok(bh_patch(p(a.in, "patch", "in"), o(a.out, "patch"), a.batch, a.channels, a.grid, a.patch,
                a.inverse ? 1 : 0, dt(a.out), nullptr));
}

void upsample_hip(const UpsampleArgs& a) {   // replaces k_upsample, ops_cuda.cu:1117-1141
    bind();
    ok(bh_upsample(p(a.in, "upsample", "in"), o(a.out, "upsample"), a.batch, a.channels, a.h_in,
                   a.w_in, a.factor, dt(a.in), nullptr));
}

void transpose_hip(const TransposeArgs& a) {   // replaces k_transpose, ops_cuda.cu:1143-1168
    bind();
    ok(bh_transpose(p(a.in, "transpose", "in"), o(a.out, "transpose"), a.batch, a.channels,
                    a.spatial, a.to_channels_first ? 1 : 0, dt(a.in), nullptr));
}

void gather_hip(const GatherArgs& a) {   // replaces k_gather, ops_cuda.cu:1086-1115
    bind();
    if (a.ids->dtype() != DType::F32)
        throw std::runtime_error("gather (hip-gfx950): token ids must be an F32 tensor");
    ok(bh_gather(p(a.table, "gather", "table"),
                 static_cast<const float*>(p(a.ids, "gather", "ids")), o(a.out, "gather"), a.rows,
                 a.cols, a.table->dim(0), dt(a.table), nullptr));
}

void scale_hip(const ScaleArgs& a) {   // replaces scale_cuda, ops_cuda.cu:1018-1031
    bind();
    ok(bh_scale(p(a.in, "scale", "in"), o(a.out, "scale"), a.numel, a.scale, dt(a.in), nullptr));
}

void repeat_hip(const RepeatArgs& a) {   // replaces k_repeat, ops_cuda.cu:1033-1049
    bind();
    ok(bh_repeat(p(a.in, "repeat", "in"), o(a.out, "repeat"), a.outer, a.inner, dt(a.in), nullptr));
}

void guidance_hip(const GuidanceArgs& a) {   // replaces k_guidance, ops_cuda.cu:1051-1073
    bind();
    ok(bh_guidance(p(a.prediction, "guidance", "prediction"), o(a.out, "guidance"), a.out_channels,
                   a.channels, a.spatial, a.scale, dt(a.out), nullptr));
}

}  // namespace

void register_hip_ops() {
    static bool done = false;   // idempotent, as register_builtin_cpu_ops (ops_cpu.cpp:415-417)
    if (done) return;
    done = true;
    const std::string n = "hip-gfx950";
    register_impl<GemmArgs>("gemm", n, gemm_hip,
                            "gfx950 bf16 MFMA GEMM (256x144x64 persistent tiles), fused bias/GELU/SiLU");
    register_impl<AttentionArgs>("attention", n, attention_hip,
                                 "flash attention on bf16 MFMA, head_dim-72 and -512 kernels; fp32 and "
                                 "wide biased heads in reference order");
    register_impl<NormArgs>("norm", n, norm_hip, "LayerNorm/RMSNorm/GroupNorm, fp64 statistics");
    register_impl<ModulateArgs>("modulate", n, modulate_hip, "adaLN modulate and gated residual");
    register_impl<ActivationArgs>("activation", n, activation_hip, "SiLU, GELU-tanh, gated GELU");
    register_impl<Conv2dArgs>("conv2d", n, conv2d_hip, "3x3 as an implicit GEMM on MFMA tiles");
    register_impl<AddArgs>("add", n, add_hip, "residual and broadcast add");
    register_impl<ChunkArgs>("chunk", n, chunk_hip, "adaLN-single chunks");
    register_impl<PatchArgs>("patch", n, patch_hip, "patchify / unpatchify");
    register_impl<UpsampleArgs>("upsample", n, upsample_hip, "nearest integer upsample, NCHW");
    register_impl<TransposeArgs>("transpose", n, transpose_hip, "[C,S] <-> [S,C]");
    register_impl<GatherArgs>("gather", n, gather_hip, "embedding row gather");
    register_impl<ScaleArgs>("scale", n, scale_hip, "one multiply per element");
    register_impl<RepeatArgs>("repeat", n, repeat_hip, "guidance-batch replication");
    register_impl<GuidanceArgs>("guidance", n, guidance_hip, "classifier-free guidance, fp64 combine");
}

}  // namespace burnisher
