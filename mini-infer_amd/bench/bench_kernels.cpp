// bench_kernels -- per-kernel latency with hipEvents, in the reference's
// method (benchmarks/bench_kernels.cpp:34-53: 10 warmup launches, 200 timed
// launches each bracketed by its own event pair, median and p99), through the
// reference-named launch_* entry points.
//
// Part 1 repeats the reference's published shapes (README.md:276-279) so the
// MI355X numbers sit next to its RTX A6000 table; part 2 runs the layer
// kernels at the Qwen2.5-7B shapes of the benchmark configs.  Each row also
// prints algorithmic bytes / median time as GB/s and % of the 8 TB/s peak.
// Inputs are zero-filled: the kernels' timing does not depend on values.
//
// Usage: bench_kernels [iters]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "core/tensor.h"
#include "kernels/gelu_kernel.h"
#include "kernels/model_utils_kernel.h"
#include "kernels/rmsnorm_kernel.h"
#include "kernels/rope_kernel.h"
#include "kernels/softmax_kernel.h"
#include "kernels/swiglu_kernel.h"
#include "layers/rope.h"

using mini_infer::DType;
using mini_infer::Device;
using mini_infer::Tensor;
namespace K = mini_infer::kernels;

namespace {

#define HIP_OK(call)                                                                     \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) {                                                          \
            std::fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, \
                         __LINE__);                                                      \
            std::exit(1);                                                                \
        }                                                                                \
    } while (0)

int g_iters = 200;

template <typename Fn>
void bench(const char* name, double bytes, Fn fn, int warmup = 10) {
    std::vector<float> t(g_iters);
    hipEvent_t s, e;
    HIP_OK(hipEventCreate(&s));
    HIP_OK(hipEventCreate(&e));
    for (int i = 0; i < warmup; ++i) fn();
    HIP_OK(hipDeviceSynchronize());
    for (int i = 0; i < g_iters; ++i) {
        HIP_OK(hipEventRecord(s, 0));
        fn();
        HIP_OK(hipEventRecord(e, 0));
        HIP_OK(hipEventSynchronize(e));
        HIP_OK(hipEventElapsedTime(&t[i], s, e));
    }
    std::sort(t.begin(), t.end());
    const double med = t[g_iters / 2] * 1e-3, p99 = t[(g_iters * 99) / 100] * 1e-3;
    std::printf("  %-44s median=%9.2f us  p99=%9.2f us  %8.1f GB/s  %5.1f%%\n", name, med * 1e6,
                p99 * 1e6, bytes / med / 1e9, 100.0 * bytes / med / 8e12);
    HIP_OK(hipEventDestroy(s));
    HIP_OK(hipEventDestroy(e));
}

Tensor dev16(std::vector<int64_t> shape) {
    Tensor t(std::move(shape), DType::FP16, Device::cuda(0));
    t.fill(0.0f);
    return t;
}

__half* H(Tensor& t) { return static_cast<__half*>(t.data()); }
const __half* C(const Tensor& t) { return static_cast<const __half*>(t.data()); }

}  // namespace

int main(int argc, char** argv) {
    if (argc > 1) g_iters = std::max(10, std::atoi(argv[1]));
    HIP_OK(hipSetDevice(0));

    std::printf("Part 1: the reference's published shapes (RTX A6000 table, README.md:276-279)\n");
    {
        const int N = 4, D = 3584;
        Tensor x = dev16({N, D}), w = dev16({D}), y = dev16({N, D});
        bench("rmsnorm N=4 D=3584", 2.0 * N * D * 2 + D * 2,
              [&] { K::launch_rmsnorm(C(x), C(w), H(y), N, D, 1e-6f, 0, 0); });
    }
    {
        const int B = 4, S = 512, Hh = 28, D = 128;
        Tensor x = dev16({B, S, Hh, D}), y = dev16({B, S, Hh, D});
        Tensor ct = dev16({B * S, D / 2}), st = dev16({B * S, D / 2});
        mini_infer::RoPE rope(D, 1e6f, 0);
        std::vector<int64_t> pos(static_cast<size_t>(B) * S);
        for (size_t i = 0; i < pos.size(); ++i) pos[i] = static_cast<int64_t>(i % S);
        const double bytes = 2.0 * B * S * Hh * D * 2;
        bench("rope B=4 S=512 H=28 D=128 (+precompute)", bytes, [&] {
            K::launch_rope_precompute_batched(rope.inv_freq().data(), pos.data(), H(ct), H(st), B, S,
                                              D / 2, 0);
            K::launch_rope(C(x), C(ct), C(st), H(y), B, S, Hh, D, 0);
        });
        bench("rope B=4 S=512 H=28 D=128 (tables ready)", bytes,
              [&] { K::launch_rope(C(x), C(ct), C(st), H(y), B, S, Hh, D, 0); });
        Tensor p(std::vector<int64_t>{B * S}, DType::INT64, Device::cpu());
        std::copy(pos.begin(), pos.end(), static_cast<int64_t*>(p.data()));
        Tensor pd = p.to(Device::cuda(0));
        Tensor q = dev16({B * S, Hh, D});
        bench("rope B=4 S=512 H=28 D=128 (fused, in place)", bytes + B * S * 8.0, [&] {
            K::launch_rope_qk(H(q), nullptr, static_cast<const int64_t*>(pd.data()),
                              rope.inv_freq().data(), B * S, Hh, 0, D, 0);
        });
    }
    {
        const int N = 57344, D = 512;
        Tensor x = dev16({N, D}), y = dev16({N, D});
        bench("softmax N=57344 D=512", 2.0 * N * D * 2,
              [&] { K::launch_softmax(C(x), H(y), N, D, 0); });
    }
    {
        const int N = 2048, I = 18944;
        Tensor g = dev16({N, I}), u = dev16({N, I}), o = dev16({N, I});
        bench("swiglu N=2048 I=18944", 3.0 * N * I * 2,
              [&] { K::launch_swiglu(C(g), C(u), H(o), N * I, 0); });
    }

    std::printf("\nPart 2: Qwen2.5-7B shapes of the benchmark configs\n");
    {
        const int N = 16, D = 3584;
        Tensor x = dev16({N, D}), w = dev16({D}), y = dev16({N, D});
        bench("rmsnorm [16,3584]", 2.0 * N * D * 2 + D * 2,
              [&] { K::launch_rmsnorm(C(x), C(w), H(y), N, D, 1e-6f, 0, 0); });
    }
    {
        const int N = 8192, D = 3584;
        Tensor x = dev16({N, D}), r = dev16({N, D}), w = dev16({D}), y = dev16({N, D});
        bench("fused add+rmsnorm [8192,3584]", 4.0 * N * D * 2 + D * 2,
              [&] { K::launch_fused_add_rmsnorm(C(x), H(r), C(w), H(y), N, D, 1e-6f, 0, 0); });
        bench("add_inplace then rmsnorm [8192,3584] (ref)", 4.0 * N * D * 2 + D * 2, [&] {
            K::launch_add_inplace(H(r), C(x), static_cast<int64_t>(N) * D, 0);
            K::launch_rmsnorm(C(r), C(w), H(y), N, D, 1e-6f, 0, 0);
        });
    }
    {
        const int T = 4096, Hq = 28, Hkv = 4, D = 128;
        Tensor q = dev16({T, Hq, D}), k = dev16({T, Hkv, D});
        Tensor p(std::vector<int64_t>{T}, DType::INT64, Device::cpu());
        for (int i = 0; i < T; ++i) static_cast<int64_t*>(p.data())[i] = 20000 + i;
        Tensor pd = p.to(Device::cuda(0));
        mini_infer::RoPE rope(D, 1e6f, 0);
        bench("rope q+k in place [4096,28|4,128]", 2.0 * T * (Hq + Hkv) * D * 2 + T * 8.0, [&] {
            K::launch_rope_qk(H(q), H(k), static_cast<const int64_t*>(pd.data()),
                              rope.inv_freq().data(), T, Hq, Hkv, D, 0);
        });
    }
    {
        const int T = 4096, I = 18944, I2 = 14336;
        Tensor g = dev16({T, I}), u = dev16({T, I}), o = dev16({T, I});
        bench("swiglu [4096,18944]", 3.0 * T * I * 2,
              [&] { K::launch_swiglu(C(g), C(u), H(o), T * I, 0); });
        bench("geglu [4096,14336]", 3.0 * T * I2 * 2,
              [&] { K::launch_geglu(C(g), C(u), H(o), static_cast<int64_t>(T) * I2, 0); });
        bench("gelu_tanh then mul_inplace [4096,14336] (ref)", 5.0 * T * I2 * 2, [&] {
            K::launch_gelu_tanh(C(g), H(o), static_cast<int64_t>(T) * I2, 0);
            K::launch_mul_inplace(H(o), C(u), static_cast<int64_t>(T) * I2, 0);
        });
    }
    {
        const int T = 6064, D = 3584;
        const int64_t V = 152064;
        Tensor table = dev16({V, D}), out = dev16({T, D});
        Tensor ids(std::vector<int64_t>{T}, DType::INT64, Device::cpu());
        uint32_t st = 12345u;
        for (int i = 0; i < T; ++i) {
            st ^= st << 13; st ^= st >> 17; st ^= st << 5;
            static_cast<int64_t*>(ids.data())[i] = static_cast<int64_t>(st % V);
        }
        Tensor idd = ids.to(Device::cuda(0));
        bench("embedding gather T=6064 from [152064,3584]", T * 8.0 + 2.0 * T * D * 2, [&] {
            K::launch_embedding_gather(static_cast<const int64_t*>(idd.data()), C(table), H(out), 1,
                                       T, D, 0);
        });
    }
    {
        const int N = 64, V = 152064;
        Tensor x = dev16({N, V}), y = dev16({N, V});
        bench("softmax [64,152064]", 2.0 * N * V * 2, [&] { K::launch_softmax(C(x), H(y), N, V, 0); });
    }
    return 0;
}
