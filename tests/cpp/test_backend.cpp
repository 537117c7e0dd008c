// Drop-in test of the C++ layer: drives KVCache::append -> view ->
// AttentionBackend::run exactly as the reference model forwards do
// (reference src/model/supported/llama/llama3.cu:232-234), for a chunked
// prefill followed by decode steps, with the Adaptive and the Naive backends,
// and checks both against the CPU oracle. Needs a GPU; run by
// tests/test_gpu_cpp_backend.py.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <memory>
#include <vector>

#include <runtherder/attention/factory.h>
#include <runtherder/engine/kv_cache.h>

#include "rth_oracle.h"

using runtherder::attention::AttnConfig;
using runtherder::attention::BackendKind;
using runtherder::attention::make_attention_backend;
using runtherder::engine::KVCache;

namespace {

struct Stats {
    double max_abs = 0.0;
    double mean_abs = 0.0;
};

Stats compare(const std::vector<uint16_t>& a, const std::vector<uint16_t>& b) {
    Stats  s;
    double sum = 0.0;
    for (size_t i = 0; i < a.size(); ++i) {
        const double d = std::fabs(static_cast<double>(rth_ref_bf16_to_f32(a[i])) -
                                   static_cast<double>(rth_ref_bf16_to_f32(b[i])));
        s.max_abs = d > s.max_abs ? d : s.max_abs;
        sum += d;
    }
    s.mean_abs = a.empty() ? 0.0 : sum / static_cast<double>(a.size());
    return s;
}

template <typename T>
T* dev_alloc(size_t n) {
    T* p = nullptr;
    RUNTHERDER_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&p), n * sizeof(T)));
    return p;
}

int run_case(BackendKind kind, const char* name) {
    const int   L = 2, S = 256, Hq = 24, Hkv = 8, D = 128;
    const int   prefill = 37, chunk = 29, steps = 5;
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    const int   total = prefill + chunk + steps;

    KVCache cache(L, S, Hkv, D);
    auto    backend = make_attention_backend(kind, AttnConfig{Hq, Hkv, D, scale});

    // Host copies of everything appended, per layer, to feed the oracle.
    std::vector<std::vector<uint16_t>> kh(L), vh(L), qh(L);
    for (int l = 0; l < L; ++l) {
        kh[l].resize(static_cast<size_t>(total) * Hkv * D);
        vh[l].resize(kh[l].size());
        qh[l].resize(static_cast<size_t>(total) * Hq * D);
        rth_ref_fill_normal_bf16(kh[l].data(), static_cast<int64_t>(kh[l].size()), 100 + l);
        rth_ref_fill_normal_bf16(vh[l].data(), static_cast<int64_t>(vh[l].size()), 200 + l);
        rth_ref_fill_normal_bf16(qh[l].data(), static_cast<int64_t>(qh[l].size()), 300 + l);
    }

    int* pos = dev_alloc<int>(1);
    auto* dk = dev_alloc<uint16_t>(static_cast<size_t>(total) * Hkv * D);
    auto* dv = dev_alloc<uint16_t>(static_cast<size_t>(total) * Hkv * D);
    auto* dq = dev_alloc<uint16_t>(static_cast<size_t>(total) * Hq * D);
    auto* dout = dev_alloc<uint16_t>(static_cast<size_t>(total) * Hq * D);
    hipStream_t stream;
    RUNTHERDER_HIP_CHECK(hipStreamCreate(&stream));

    int fails = 0;
    int start = 0;
    std::vector<int> chunks = {prefill, chunk};
    for (int i = 0; i < steps; ++i) {
        chunks.push_back(1);
    }
    for (int n : chunks) {
        RUNTHERDER_HIP_CHECK(hipMemcpy(pos, &start, sizeof(int), hipMemcpyHostToDevice));
        for (int l = 0; l < L; ++l) {
            const size_t kvo = static_cast<size_t>(start) * Hkv * D;
            const size_t qo  = static_cast<size_t>(start) * Hq * D;
            RUNTHERDER_HIP_CHECK(hipMemcpy(dk, kh[l].data() + kvo, n * Hkv * D * 2, hipMemcpyHostToDevice));
            RUNTHERDER_HIP_CHECK(hipMemcpy(dv, vh[l].data() + kvo, n * Hkv * D * 2, hipMemcpyHostToDevice));
            RUNTHERDER_HIP_CHECK(hipMemcpy(dq, qh[l].data() + qo, n * Hq * D * 2, hipMemcpyHostToDevice));
            cache.append(l, reinterpret_cast<const __hip_bfloat16*>(dk),
                         reinterpret_cast<const __hip_bfloat16*>(dv), n, pos, stream);
            const auto kv = cache.view(l);
            backend->run(reinterpret_cast<__hip_bfloat16*>(dout),
                         reinterpret_cast<const __hip_bfloat16*>(dq), kv, n, pos, stream);
            RUNTHERDER_HIP_CHECK(hipStreamSynchronize(stream));

            // Oracle: quantize the host history, then attend.
            const int keys = start + n;
            std::vector<uint8_t> k8(static_cast<size_t>(keys) * Hkv * D), v8(k8.size());
            std::vector<float>   ks(static_cast<size_t>(keys) * Hkv), vs(ks.size());
            rth_ref_quantize_kv_fp8(k8.data(), ks.data(), kh[l].data(), 0, 1, keys * Hkv, D);
            rth_ref_quantize_kv_fp8(v8.data(), vs.data(), vh[l].data(), 0, 1, keys * Hkv, D);
            std::vector<uint16_t> want(static_cast<size_t>(n) * Hq * D), got(want.size());
            rth_ref_attention_f32(want.data(), qh[l].data() + qo, k8.data(), v8.data(), ks.data(),
                                  vs.data(), n, start, Hq, Hkv, D, scale, 4);
            RUNTHERDER_HIP_CHECK(hipMemcpy(got.data(), dout, got.size() * 2, hipMemcpyDeviceToHost));

            // The cache bytes must equal the oracle's quantization bit for bit.
            std::vector<uint8_t> k8d(static_cast<size_t>(keys) * Hkv * D);
            std::vector<float>   ksd(static_cast<size_t>(keys) * Hkv);
            RUNTHERDER_HIP_CHECK(hipMemcpy(k8d.data(), kv.k, k8d.size(), hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(ksd.data(), kv.k_scale, ksd.size() * 4, hipMemcpyDeviceToHost));
            const bool bytes_ok = std::memcmp(k8d.data(), k8.data(), k8.size()) == 0 &&
                                  std::memcmp(ksd.data(), ks.data(), ks.size() * 4) == 0;
            const Stats st = compare(want, got);
            const bool  ok = bytes_ok && st.max_abs <= 2e-2 && st.mean_abs <= 2e-3;
            std::printf("%s layer=%d start=%d n=%d bytes_ok=%d max_abs=%.3e mean_abs=%.3e %s\n",
                        name, l, start, n, bytes_ok ? 1 : 0, st.max_abs, st.mean_abs,
                        ok ? "OK" : "FAIL");
            std::fflush(stdout);
            fails += ok ? 0 : 1;
        }
        start += n;
    }
    RUNTHERDER_HIP_CHECK(hipStreamDestroy(stream));
    (void)hipFree(pos);
    (void)hipFree(dk);
    (void)hipFree(dv);
    (void)hipFree(dq);
    (void)hipFree(dout);
    return fails;
}

}  // namespace

int main() {
    int fails = 0;
    fails += run_case(BackendKind::Adaptive, "adaptive");
    fails += run_case(BackendKind::Naive, "naive");
    std::printf("%s\n", fails == 0 ? "ALL OK" : "FAILURES");
    return fails == 0 ? 0 : 1;
}
