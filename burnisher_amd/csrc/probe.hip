// Device probe: what this MI355X actually sustains, measured with kernels of this library (the
// reference's `burnisher probe`, src/cuda/device.cu:257-357, measures a stream copy and a vendor
// GEMM; here the GEMM side is a register-only MFMA loop, which bounds every MFMA kernel, and the
// library's own GEMM is timed by the caller through bh_gemm).
//
//   k_probe_mfma   every SIMD of every CU issues v_mfma_f32_16x16x32_bf16 back to back on eight
//                  independent accumulators held in registers: no LDS, no memory. Each wave also
//                  reads the shader clock counter (s_memtime) and the constant-rate wall clock
//                  (s_memrealtime) at its start and end, so the shader clock the chip holds under
//                  pure MFMA load is measured directly, not inferred.
//   k_probe_copy   a device-to-device copy in 16-byte vectors, grid-stride (HBM read + write).
#include "common.h"

#include <algorithm>
#include <vector>

namespace bh {
namespace {

constexpr int kProbeAcc = 8;          // independent accumulators per wave
constexpr int kProbeThreads = 256;    // one wave per SIMD

__global__ void __launch_bounds__(kProbeThreads)
k_probe_mfma(int iters, float* sink, unsigned long long* stamps) {
    // Operands depend on the thread so nothing folds; small values keep every sum finite.
    const float base = 1e-3f * static_cast<float>((threadIdx.x & 7) + 1);
    bf16x8_t a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = static_cast<__bf16>(base * static_cast<float>(i + 1));
        b[i] = static_cast<__bf16>(base * static_cast<float>(8 - i));
    }
    f32x4_t acc[kProbeAcc];
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const unsigned long long w0 = __builtin_amdgcn_s_memrealtime();
    const unsigned long long c0 = __builtin_amdgcn_s_memtime();
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < kProbeAcc; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[j], 0, 0, 0);
    }
    const unsigned long long c1 = __builtin_amdgcn_s_memtime();
    const unsigned long long w1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < kProbeAcc; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
    const int wave = (blockIdx.x * kProbeThreads + threadIdx.x) >> 6;
    sink[blockIdx.x * kProbeThreads + threadIdx.x] = s;
    if ((threadIdx.x & 63) == 0) {
        stamps[wave * 4 + 0] = w0;
        stamps[wave * 4 + 1] = w1;
        stamps[wave * 4 + 2] = c0;
        stamps[wave * 4 + 3] = c1;
    }
}

__global__ void __launch_bounds__(256) k_probe_copy(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                     int64_t n) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(blockDim.x) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x)
        dst[i] = src[i];
}

struct Events {
    hipEvent_t a = nullptr, b = nullptr;
    Events() {
        hip_check(hipEventCreate(&a), "hipEventCreate");
        hip_check(hipEventCreate(&b), "hipEventCreate");
    }
    ~Events() {
        if (a) (void)hipEventDestroy(a);
        if (b) (void)hipEventDestroy(b);
    }
    float ms() {
        hip_check(hipEventSynchronize(b), "hipEventSynchronize");
        float t = 0.f;
        hip_check(hipEventElapsedTime(&t, a, b), "hipEventElapsedTime");
        return t;
    }
};

}  // namespace
}  // namespace bh

using namespace bh;

extern "C" {

int bh_probe_device(void* copy_src, void* copy_dst, int64_t copy_bytes, bh_probe_result* out) {
    return guarded([&] {
        require(out != nullptr, "probe: null result");
        require(copy_bytes >= (1 << 20) && copy_bytes % 16 == 0,
                "probe: copy_bytes must be a multiple of 16 and at least 1 MiB");
        require_device_ptr(copy_src, "probe", "copy_src");
        require_device_ptr(copy_dst, "probe", "copy_dst");
        *out = bh_probe_result{};
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        int cus = 0, clock_khz = 0, wall_khz = 0;
        hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "attr");
        hip_check(hipDeviceGetAttribute(&clock_khz, hipDeviceAttributeClockRate, dev), "attr");
        hip_check(hipDeviceGetAttribute(&wall_khz, hipDeviceAttributeWallClockRate, dev), "attr");
        require(cus > 0 && wall_khz > 0, "probe: the device reports no compute units or wall clock");
        out->cus = cus;
        out->max_clock_mhz = clock_khz / 1000.0;
        out->wall_clock_mhz = wall_khz / 1000.0;

        // MFMA: four blocks per CU (four waves per SIMD), long enough to reach a steady clock.
        const int blocks = 4 * cus;
        const int waves = blocks * kProbeThreads / 64;
        const int iters = 1 << 16;
        float* sink = nullptr;
        unsigned long long* stamps = nullptr;
        hip_check(hipMalloc(&sink, static_cast<size_t>(blocks) * kProbeThreads * sizeof(float)), "hipMalloc");
        hip_check(hipMalloc(&stamps, static_cast<size_t>(waves) * 4 * sizeof(unsigned long long)), "hipMalloc");
        std::vector<unsigned long long> st(static_cast<size_t>(waves) * 4);
        float mfma_ms = 0.f;
        try {
            k_probe_mfma<<<blocks, kProbeThreads>>>(iters / 16, sink, stamps);   // warm-up
            launch_check("probe mfma");
            Events ev;
            hip_check(hipEventRecord(ev.a, nullptr), "hipEventRecord");
            k_probe_mfma<<<blocks, kProbeThreads>>>(iters, sink, stamps);
            launch_check("probe mfma");
            hip_check(hipEventRecord(ev.b, nullptr), "hipEventRecord");
            mfma_ms = ev.ms();
            hip_check(hipMemcpy(st.data(), stamps, st.size() * sizeof(unsigned long long),
                                hipMemcpyDeviceToHost), "hipMemcpy");
        } catch (...) {
            (void)hipFree(sink);
            (void)hipFree(stamps);
            throw;
        }
        (void)hipFree(sink);
        (void)hipFree(stamps);
        const double flop = static_cast<double>(waves) * iters * kProbeAcc * (2.0 * 16 * 16 * 32);
        out->mfma_tflops = flop / (mfma_ms * 1e-3) / 1e12;
        // Per wave: shader clocks over wall-clock ticks; the median over waves.
        std::vector<double> mhz;
        mhz.reserve(waves);
        for (int w = 0; w < waves; ++w) {
            const double wall = static_cast<double>(st[w * 4 + 1] - st[w * 4 + 0]);
            const double clk = static_cast<double>(st[w * 4 + 3] - st[w * 4 + 2]);
            if (wall > 0) mhz.push_back(clk / wall * out->wall_clock_mhz);
        }
        require(!mhz.empty(), "probe: no wave recorded a clock interval");
        std::sort(mhz.begin(), mhz.end());
        out->mfma_shader_mhz = mhz[mhz.size() / 2];
        out->mfma_shader_mhz_min = mhz.front();
        out->mfma_shader_mhz_max = mhz.back();
        // The MFMA rate the measured clock allows: 4 SIMDs x 1024 FLOP per clock per CU.
        out->mfma_peak_at_clock_tflops = cus * 4096.0 * out->mfma_shader_mhz * 1e6 / 1e12;

        // Copy: one warm-up, then five timed passes.
        const int64_t n = copy_bytes / 16;
        const int grid = std::min<int64_t>((n + 255) / 256, static_cast<int64_t>(cus) * 32);
        auto* s16 = static_cast<const uint4*>(copy_src);
        auto* d16 = static_cast<uint4*>(copy_dst);
        k_probe_copy<<<grid, 256>>>(s16, d16, n);
        launch_check("probe copy");
        Events ev;
        const int reps = 5;
        hip_check(hipEventRecord(ev.a, nullptr), "hipEventRecord");
        for (int r = 0; r < reps; ++r) k_probe_copy<<<grid, 256>>>(s16, d16, n);
        launch_check("probe copy");
        hip_check(hipEventRecord(ev.b, nullptr), "hipEventRecord");
        const float copy_ms = ev.ms() / reps;
        out->copy_gbs = 2.0 * static_cast<double>(copy_bytes) / (copy_ms * 1e-3) / 1e9;
    });
}

}  // extern "C"
