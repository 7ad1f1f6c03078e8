// oracle/registry_main.cpp -- TEST INFRASTRUCTURE ONLY. A driver linked from the REFERENCE
// runtime's own sources (registry, impl_select, tensor, weights, ops_cpu, pixart_dit; compiled
// where they lie under /root/reference by `make -C oracle registry`), this repository's registry
// adapter (burnisher_amd/registry/ops_hip.cpp) and HIP device layer
// (burnisher_amd/registry/device_hip.cpp), and libburnisher_hip.so. It is what a Burnisher
// ROCm build looks like, and it lets the tests check the drop-in from the reference's side:
//
//   registry_main check
//       Registration and selection only (touches no device): every op registers `hip-gfx950`;
//       ImplSelection::from_request("hip-gfx950", Device::CUDA) resolves every op to it, so no
//       op falls back to a host kernel on a device run (tests/test_ops.cpp:310-339); the CPU
//       baseline is unchanged; an unknown name is an error. Prints one JSON line.
//
//   registry_main dit-step LAYERS BATCH LATENT_HW CAPTION_LEN OUT.bin [ITERS]
//       The reference's own PixArtDiT::forward (pixart_dit.cpp:112-304) on Device::CUDA with
//       every op resolved to hip-gfx950, on the seeded workload the Python tests build
//       (burnisher_amd/workload.py: N(0, 0.02) bf16 weights and N(0, 1) latent and caption drawn
//       by bh_fill_normal_bf16 under the checkpoint names, seed 20260911; prefix caption mask).
//       Writes the bf16 output to OUT.bin, then times ITERS forwards the way `burnisher bench`
//       does (burnisher_main.cpp:451-464: device sync, host clock, median) and prints one JSON
//       line with the median, the device peak bytes and the effective implementation per op.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "burnisher/device.h"
#include "burnisher/models.h"
#include "burnisher/ops.h"

#include "../include/burnisher_hip.h"

namespace burnisher {
void register_hip_ops();   // burnisher_amd/registry/ops_hip.cpp
}

using namespace burnisher;

namespace {

constexpr uint64_t kSeed = 20260911;   // burnisher_amd/workload.py SEED

int failures = 0;
std::string report;

void expect(bool ok, const std::string& what) {
    if (!ok) {
        ++failures;
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
    }
}

template <typename Fn>
bool throws(Fn fn) {
    try {
        fn();
    } catch (const std::exception&) {
        return true;
    }
    return false;
}

const char* kOps[] = {"gemm", "attention", "norm", "modulate", "activation", "conv2d", "add",
                      "chunk", "patch", "upsample", "transpose", "gather", "scale", "repeat",
                      "guidance"};

int check() {
    register_all_ops();
    register_hip_ops();
    register_hip_ops();   // idempotent
    // every op carries the name
    const auto listing = list_all_impls();
    for (const char* op : kOps) {
        bool found = false;
        for (const auto& l : listing)
            if (l.op == op)
                for (const auto& i : l.impls) found |= i.name == "hip-gfx950" && !i.doc.empty();
        expect(found, std::string("op '") + op + "' lists hip-gfx950 with a description");
    }
    expect(any_op_has_impl("hip-gfx950"), "any_op_has_impl(hip-gfx950)");
    // a device run: every op resolves to the requested name, none to a host kernel
    const ImplSelection dev = ImplSelection::from_request("hip-gfx950", Device::CUDA);
    for (const auto& kv : dev.as_map()) {
        if (kv.first == "device") {
            expect(kv.second == "cuda", "device field names the GPU device");
            continue;
        }
        expect(kv.second == "hip-gfx950", kv.first + " resolves to hip-gfx950 on the device, got " + kv.second);
        expect(kv.second != "stock", kv.first + " falls back to a host kernel on a device run");
    }
    // per op, through resolve_impl itself (impl_select.cpp:57-67)
    for (const char* op : kOps)
        expect(resolve_impl(op, "hip-gfx950", Device::CUDA) == "hip-gfx950",
               std::string("resolve_impl(") + op + ", hip-gfx950, CUDA)");
    // the host baseline is unchanged (test_ops.cpp:334-339)
    for (const auto& kv : ImplSelection::from_request("materialized", Device::CPU).as_map()) {
        if (kv.first == "device" || kv.first == "attention") continue;
        expect(kv.second == "stock", kv.first + " stays stock on a CPU run");
    }
    for (const auto& kv : ImplSelection::from_request("stock", Device::CPU).as_map())
        if (kv.first != "device") expect(kv.second == "stock", kv.first + " stock on CPU");
    // an unknown name is an error, a duplicate registration is an error
    expect(throws([] { ImplSelection::from_request("hip-gfx951", Device::CUDA); }),
           "an unknown implementation name is refused");
    expect(throws([] { register_impl<GemmArgs>("gemm", "hip-gfx950", [](const GemmArgs&) {}, "dup"); }),
           "a second hip-gfx950 gemm registration is refused");
    // fetching the registered function touches no device
    expect(static_cast<bool>(GemmRegistry::instance().get("hip-gfx950")), "gemm fn is callable");
    std::printf("{\"check\": \"registry\", \"ops\": %zu, \"failures\": %d}\n",
                sizeof(kOps) / sizeof(kOps[0]), failures);
    return failures == 0 ? 0 : 1;
}

// The workload's weights by checkpoint name, drawn exactly as burnisher_amd/workload.py draws
// them (bh_fill_normal_bf16(numel, name, seed, 0.02)), shapes from declare_pixart_shapes.
class SeededWeights : public WeightSource {
  public:
    explicit SeededWeights(const DiTConfig& c) : shapes_(DType::BF16) {
        declare_pixart_shapes(shapes_, T5Config{}, c, VaeConfig{});
    }
    bool has(const std::string& name) const override { return shapes_.declared().count(name) != 0; }
    Tensor get(const std::string& name) const override {
        auto it = shapes_.declared().find(name);
        if (it == shapes_.declared().end()) throw std::runtime_error("no weight named " + name);
        Tensor t(it->second, DType::BF16);
        if (bh_fill_normal_bf16(static_cast<uint16_t*>(t.data()), t.numel(), kSeed, name.c_str(), 0.02f))
            throw std::runtime_error(bh_last_error());
        return t;
    }

  private:
    SyntheticWeights shapes_;
};

Tensor seeded(std::vector<int64_t> shape, const char* name, float std_dev) {
    Tensor t(std::move(shape), DType::BF16);
    if (bh_fill_normal_bf16(static_cast<uint16_t*>(t.data()), t.numel(), kSeed, name, std_dev))
        throw std::runtime_error(bh_last_error());
    return t;
}

int dit_step(int layers, int64_t batch, int64_t latent_hw, int64_t cap_len, const char* out_path,
             int iters) {
    register_all_ops();
    register_hip_ops();
    if (!device::available()) throw std::runtime_error("no HIP device");
    DiTConfig cfg;   // PixArt-Sigma (models.h:105-118)
    cfg.num_layers = layers;
    const ImplSelection impls = ImplSelection::from_request("hip-gfx950", Device::CUDA);
    SeededWeights host(cfg);
    DeviceWeights dw(host, DType::BF16);
    const Tensor latent = seeded({batch, cfg.in_channels, latent_hw, latent_hw}, "latent", 1.0f).to_device();
    const Tensor caption = seeded({batch, cap_len, cfg.caption_channels}, "caption", 1.0f).to_device();
    Tensor mask_host({batch, cap_len}, DType::BF16);
    for (int64_t b = 0; b < batch; ++b) {   // workload.prefix_mask
        const int64_t keep = std::max<int64_t>(1, b % 2 == 0 ? cap_len / 4 : cap_len / 2);
        for (int64_t j = 0; j < cap_len; ++j) mask_host.set(b * cap_len + j, j < keep ? 1.0f : 0.0f);
    }
    const Tensor mask = mask_host.to_device();
    const PixArtDiT dit(cfg, dw, DType::BF16);
    Tensor out = dit.forward(latent, 500.0, caption, mask, impls);
    device::synchronize();
    const Tensor host_out = out.to_host();
    {
        std::ofstream f(out_path, std::ios::binary);
        f.write(static_cast<const char*>(host_out.data()), static_cast<std::streamsize>(host_out.nbytes()));
        if (!f) throw std::runtime_error(std::string("cannot write ") + out_path);
    }
    std::vector<double> ms;
    for (int i = 0; i < iters; ++i) {
        device::synchronize();
        const auto t0 = std::chrono::steady_clock::now();
        Tensor o = dit.forward(latent, 500.0, caption, mask, impls);
        device::synchronize();
        ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
    }
    std::sort(ms.begin(), ms.end());
    const double median = ms.empty() ? 0.0 : (ms.size() % 2 ? ms[ms.size() / 2]
                                                            : 0.5 * (ms[ms.size() / 2 - 1] + ms[ms.size() / 2]));
    std::string eff;
    for (const auto& kv : impls.as_map()) eff += (eff.empty() ? "" : ", ") + ("\"" + kv.first + "\": \"" + kv.second + "\"");
    std::printf("{\"stage\": \"dit-step\", \"layers\": %d, \"batch\": %lld, \"latent\": %lld, \"caption_len\": %lld, "
                "\"iters\": %d, \"median_ms\": %.4f, \"peak_vram_bytes\": %zu, \"weights_bytes\": %zu, "
                "\"effective\": {%s}}\n",
                layers, static_cast<long long>(batch), static_cast<long long>(latent_hw),
                static_cast<long long>(cap_len), iters, median, device::peak_allocated_bytes(),
                dw.resident_bytes(), eff.c_str());
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const std::string cmd = argc > 1 ? argv[1] : "";
        if (cmd == "check") return check();
        if (cmd == "dit-step" && argc >= 7)
            return dit_step(std::atoi(argv[2]), std::atoll(argv[3]), std::atoll(argv[4]), std::atoll(argv[5]),
                            argv[6], argc > 7 ? std::atoi(argv[7]) : 0);
        std::fprintf(stderr, "usage: registry_main check | dit-step LAYERS BATCH LATENT_HW CAPTION_LEN OUT.bin [ITERS]\n");
        return 2;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "!! %s\n", e.what());
        return 1;
    }
}
