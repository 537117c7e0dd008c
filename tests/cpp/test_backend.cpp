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

#include <runtherder/attention/adaptive.h>
#include <runtherder/attention/factory.h>
#include <runtherder/engine/kv_cache.h>
#include <runtherder/kernels/flash_decode.h>
#include <runtherder/kernels/rmsnorm.h>
#include <runtherder/kernels/rope.h>

#include "rth_oracle.h"

using runtherder::attention::AttnConfig;
using runtherder::attention::BackendKind;
using runtherder::attention::make_attention_backend;
using runtherder::engine::KVCache;

namespace {

// The scratch size is a constant expression, as in the reference
// (include/runtherder/kernels/flash_decode.cuh:16): callers size static
// buffers with it.
static_assert(runtherder::kernels::flash_split_scratch_floats(24, 128, 256) ==
                  24u * 256u * 2u + 24u * 256u * 128u,
              "flash_split_scratch_floats is constexpr and keeps the reference formula");

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
    const int   L = 2, S = 512, Hq = 24, Hkv = 8, D = 128;
    // Chunks of 300 (the flash prefill), 200 (AdaptiveAttention's flash
    // prefill over key runs), 4 (its split-K decode route for a few tokens),
    // then one-token decode steps.
    const int   prefill = 300, chunk = 200, small = 4, steps = 5;
    const float scale = 1.0f / std::sqrt(static_cast<float>(D));
    const int   total = prefill + chunk + small + steps;

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
    std::vector<int> chunks = {prefill, chunk, small};
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

// KVCache::append_rope against kernels::rope_bf16 followed by
// KVCache::append (the reference's caller order, llama3.cu:228-232), and both
// against the oracle's RoPE then quantize; cache bytes and the rotated q must
// match bit for bit.
int run_rope_case() {
    const int Hq = 32, Hkv = 8, D = 128, n = 257, at = 40, max_seq = at + n;
    std::vector<uint16_t> qh(static_cast<size_t>(n) * Hq * D), kh(static_cast<size_t>(n) * Hkv * D),
        vh(kh.size());
    rth_ref_fill_normal_bf16(qh.data(), static_cast<int64_t>(qh.size()), 900);
    rth_ref_fill_normal_bf16(kh.data(), static_cast<int64_t>(kh.size()), 901);
    rth_ref_fill_normal_bf16(vh.data(), static_cast<int64_t>(vh.size()), 902);
    std::vector<int>   posh(n);
    std::vector<float> inv(D / 2);
    for (int t = 0; t < n; ++t) {
        posh[t] = at + t;
    }
    rth_ref_rope_inv_freq_llama3(inv.data(), D, 5e5f, 32.0f, 1.0f, 4.0f, 8192);

    auto* dq1 = dev_alloc<uint16_t>(qh.size());
    auto* dq2 = dev_alloc<uint16_t>(qh.size());
    auto* dk  = dev_alloc<uint16_t>(kh.size());
    auto* dk2 = dev_alloc<uint16_t>(kh.size());
    auto* dv  = dev_alloc<uint16_t>(vh.size());
    auto* dpos = dev_alloc<int>(n);
    auto* dinv = dev_alloc<float>(inv.size());
    int*  dat  = dev_alloc<int>(1);
    RUNTHERDER_HIP_CHECK(hipMemcpy(dq1, qh.data(), qh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dq2, qh.data(), qh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dk, kh.data(), kh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dk2, kh.data(), kh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dv, vh.data(), vh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dpos, posh.data(), n * sizeof(int), hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dinv, inv.data(), inv.size() * 4, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dat, &at, sizeof(int), hipMemcpyHostToDevice));

    KVCache fused(1, max_seq, Hkv, D), two(1, max_seq, Hkv, D);
    fused.append_rope(0, reinterpret_cast<__hip_bfloat16*>(dq1),
                      reinterpret_cast<const __hip_bfloat16*>(dk),
                      reinterpret_cast<const __hip_bfloat16*>(dv), n, dpos, dinv, dat, Hq,
                      nullptr);
    runtherder::kernels::rope_bf16(reinterpret_cast<__hip_bfloat16*>(dq2),
                                   reinterpret_cast<__hip_bfloat16*>(dk2), dpos, dinv, n, Hq,
                                   Hkv, D, nullptr);
    two.append(0, reinterpret_cast<const __hip_bfloat16*>(dk2),
               reinterpret_cast<const __hip_bfloat16*>(dv), n, dat, nullptr);
    RUNTHERDER_HIP_CHECK(hipDeviceSynchronize());

    const size_t rows = static_cast<size_t>(n) * Hkv;
    const size_t off  = static_cast<size_t>(at) * Hkv;
    auto fetch = [&](const runtherder::attention::KVView& kv, std::vector<uint8_t>& k8,
                     std::vector<uint8_t>& v8, std::vector<float>& ks, std::vector<float>& vs) {
        k8.resize(rows * D);
        v8.resize(rows * D);
        ks.resize(rows);
        vs.resize(rows);
        RUNTHERDER_HIP_CHECK(hipMemcpy(k8.data(), reinterpret_cast<const uint8_t*>(kv.k) + off * D,
                                       rows * D, hipMemcpyDeviceToHost));
        RUNTHERDER_HIP_CHECK(hipMemcpy(v8.data(), reinterpret_cast<const uint8_t*>(kv.v) + off * D,
                                       rows * D, hipMemcpyDeviceToHost));
        RUNTHERDER_HIP_CHECK(hipMemcpy(ks.data(), kv.k_scale + off, rows * 4, hipMemcpyDeviceToHost));
        RUNTHERDER_HIP_CHECK(hipMemcpy(vs.data(), kv.v_scale + off, rows * 4, hipMemcpyDeviceToHost));
    };
    std::vector<uint8_t> k1, v1, k2, v2;
    std::vector<float>   ks1, vs1, ks2, vs2;
    fetch(fused.view(0), k1, v1, ks1, vs1);
    fetch(two.view(0), k2, v2, ks2, vs2);
    std::vector<uint16_t> q1(qh.size()), q2(qh.size());
    RUNTHERDER_HIP_CHECK(hipMemcpy(q1.data(), dq1, qh.size() * 2, hipMemcpyDeviceToHost));
    RUNTHERDER_HIP_CHECK(hipMemcpy(q2.data(), dq2, qh.size() * 2, hipMemcpyDeviceToHost));

    std::vector<uint16_t> qr = qh, kr = kh;
    rth_ref_rope_apply_bf16(qr.data(), posh.data(), inv.data(), n, Hq, D);
    rth_ref_rope_apply_bf16(kr.data(), posh.data(), inv.data(), n, Hkv, D);
    std::vector<uint8_t> wk(rows * D), wv(rows * D);
    std::vector<float>   wks(rows), wvs(rows);
    rth_ref_quantize_kv_fp8(wk.data(), wks.data(), kr.data(), 0, 1, static_cast<int>(rows), D);
    rth_ref_quantize_kv_fp8(wv.data(), wvs.data(), vh.data(), 0, 1, static_cast<int>(rows), D);

    const bool same_two = k1 == k2 && v1 == v2 &&
                          std::memcmp(ks1.data(), ks2.data(), rows * 4) == 0 &&
                          std::memcmp(vs1.data(), vs2.data(), rows * 4) == 0 && q1 == q2;
    const bool same_ref = k1 == wk && v1 == wv &&
                          std::memcmp(ks1.data(), wks.data(), rows * 4) == 0 &&
                          std::memcmp(vs1.data(), wvs.data(), rows * 4) == 0 && q1 == qr;
    std::printf("rope_append n=%d at=%d same_as_two_step=%d same_as_oracle=%d %s\n", n, at,
                same_two ? 1 : 0, same_ref ? 1 : 0, (same_two && same_ref) ? "OK" : "FAIL");
    std::fflush(stdout);
    for (void* p : {static_cast<void*>(dq1), static_cast<void*>(dq2), static_cast<void*>(dk),
                    static_cast<void*>(dk2), static_cast<void*>(dv), static_cast<void*>(dpos),
                    static_cast<void*>(dinv), static_cast<void*>(dat)}) {
        (void)hipFree(p);
    }
    return (same_two && same_ref) ? 0 : 1;
}

// AdaptiveAttention's decode-step methods against the caller sequences they
// replace, on two caches holding the same 40-token prefix, for three steps
// each: run_decode_append vs append -> run; run_decode_rope_append vs
// rope_bf16 -> append -> run (llama3.cu:228-234); run_decode_qk_norm_rope_append
// vs rmsnorm_bf16_forward (q, k per head) -> rope_bf16 -> append -> run
// (qwen3.cu:189-202). Cache bytes must be identical; the outputs agree within
// the attention tolerance (the fused step folds the appended key in after the
// cache's keys, a different summation order).
int run_decode_step_case() {
    const int   Hq = 24, Hkv = 8, D = 128, S = 64, pre = 40, steps = 3;
    const float scale = 1.0f / std::sqrt(static_cast<float>(D)), eps = 1e-6f;
    runtherder::attention::AdaptiveAttention backend(AttnConfig{Hq, Hkv, D, scale});
    std::vector<uint16_t> kh(static_cast<size_t>(pre + steps) * Hkv * D), vh(kh.size()),
        qh(static_cast<size_t>(steps) * Hq * D), gq(D), gk(D);
    rth_ref_fill_normal_bf16(kh.data(), static_cast<int64_t>(kh.size()), 1100);
    rth_ref_fill_normal_bf16(vh.data(), static_cast<int64_t>(vh.size()), 1101);
    rth_ref_fill_normal_bf16(qh.data(), static_cast<int64_t>(qh.size()), 1102);
    rth_ref_fill_normal_bf16(gq.data(), D, 1103);
    rth_ref_fill_normal_bf16(gk.data(), D, 1104);
    std::vector<float> inv(D / 2);
    rth_ref_rope_inv_freq_plain(inv.data(), D, 1e6f);

    auto* dk   = dev_alloc<uint16_t>(kh.size());
    auto* dv   = dev_alloc<uint16_t>(vh.size());
    auto* dq   = dev_alloc<uint16_t>(qh.size());
    auto* dq2  = dev_alloc<uint16_t>(static_cast<size_t>(Hq) * D);
    auto* dk2  = dev_alloc<uint16_t>(static_cast<size_t>(Hkv) * D);
    auto* dgq  = dev_alloc<uint16_t>(D);
    auto* dgk  = dev_alloc<uint16_t>(D);
    auto* dinv = dev_alloc<float>(inv.size());
    auto* o1   = dev_alloc<uint16_t>(static_cast<size_t>(Hq) * D);
    auto* o2   = dev_alloc<uint16_t>(static_cast<size_t>(Hq) * D);
    int*  pos  = dev_alloc<int>(1);
    RUNTHERDER_HIP_CHECK(hipMemcpy(dk, kh.data(), kh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dv, vh.data(), vh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dq, qh.data(), qh.size() * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dgq, gq.data(), D * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dgk, gk.data(), D * 2, hipMemcpyHostToDevice));
    RUNTHERDER_HIP_CHECK(hipMemcpy(dinv, inv.data(), inv.size() * 4, hipMemcpyHostToDevice));
    auto bf = [](uint16_t* p) { return reinterpret_cast<__hip_bfloat16*>(p); };
    auto cbf = [](const uint16_t* p) { return reinterpret_cast<const __hip_bfloat16*>(p); };
    const char* names[3] = {"decode_append", "decode_rope_append", "decode_qk_norm_rope_append"};

    int fails = 0;
    for (int mode = 0; mode < 3; ++mode) {
        KVCache a(1, S, Hkv, D), b(1, S, Hkv, D);
        const int zero = 0;
        RUNTHERDER_HIP_CHECK(hipMemcpy(pos, &zero, sizeof(int), hipMemcpyHostToDevice));
        a.append(0, cbf(dk), cbf(dv), pre, pos, nullptr);
        b.append(0, cbf(dk), cbf(dv), pre, pos, nullptr);
        for (int s = 0; s < steps; ++s) {
            const int p = pre + s;
            RUNTHERDER_HIP_CHECK(hipMemcpy(pos, &p, sizeof(int), hipMemcpyHostToDevice));
            const uint16_t* q  = dq + static_cast<size_t>(s) * Hq * D;
            const uint16_t* kn = dk + static_cast<size_t>(p) * Hkv * D;
            const uint16_t* vn = dv + static_cast<size_t>(p) * Hkv * D;
            if (mode == 0) {
                backend.run_decode_append(bf(o1), cbf(q), a.slabs(0), cbf(kn), cbf(vn), pos,
                                          nullptr);
                b.append(0, cbf(kn), cbf(vn), 1, pos, nullptr);
                backend.run(bf(o2), cbf(q), b.view(0), 1, pos, nullptr);
            } else {
                RUNTHERDER_HIP_CHECK(hipMemcpy(dq2, q, Hq * D * 2, hipMemcpyDeviceToDevice));
                RUNTHERDER_HIP_CHECK(hipMemcpy(dk2, kn, Hkv * D * 2, hipMemcpyDeviceToDevice));
                if (mode == 1) {
                    backend.run_decode_rope_append(bf(o1), cbf(q), a.slabs(0), cbf(kn), cbf(vn),
                                                   pos, dinv, pos, nullptr);
                } else {
                    backend.run_decode_qk_norm_rope_append(bf(o1), cbf(q), a.slabs(0), cbf(kn),
                                                           cbf(vn), cbf(dgq), cbf(dgk), eps, pos,
                                                           dinv, pos, nullptr);
                    runtherder::kernels::rmsnorm_bf16_forward(bf(dq2), cbf(dq2), cbf(dgq), Hq, D,
                                                              eps, nullptr);
                    runtherder::kernels::rmsnorm_bf16_forward(bf(dk2), cbf(dk2), cbf(dgk), Hkv,
                                                              D, eps, nullptr);
                }
                runtherder::kernels::rope_bf16(bf(dq2), bf(dk2), pos, dinv, 1, Hq, Hkv, D,
                                               nullptr);
                b.append(0, cbf(dk2), cbf(vn), 1, pos, nullptr);
                backend.run(bf(o2), cbf(dq2), b.view(0), 1, pos, nullptr);
            }
            RUNTHERDER_HIP_CHECK(hipDeviceSynchronize());
            std::vector<uint16_t> g1(static_cast<size_t>(Hq) * D), g2(g1.size());
            RUNTHERDER_HIP_CHECK(hipMemcpy(g1.data(), o1, g1.size() * 2, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(g2.data(), o2, g2.size() * 2, hipMemcpyDeviceToHost));
            const size_t         n8 = static_cast<size_t>(p + 1) * Hkv * D, ns = n8 / D;
            std::vector<uint8_t> ka(n8), kb(n8), va(n8), vb(n8);
            std::vector<float>   ksa(ns), ksb(ns);
            const auto           av = a.view(0), bv = b.view(0);
            RUNTHERDER_HIP_CHECK(hipMemcpy(ka.data(), av.k, n8, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(kb.data(), bv.k, n8, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(va.data(), av.v, n8, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(vb.data(), bv.v, n8, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(ksa.data(), av.k_scale, ns * 4, hipMemcpyDeviceToHost));
            RUNTHERDER_HIP_CHECK(hipMemcpy(ksb.data(), bv.k_scale, ns * 4, hipMemcpyDeviceToHost));
            const bool  bytes_ok = ka == kb && va == vb &&
                                  std::memcmp(ksa.data(), ksb.data(), ns * 4) == 0;
            const Stats st = compare(g1, g2);
            const bool  ok = bytes_ok && st.max_abs <= 2e-2 && st.mean_abs <= 1e-3;
            std::printf("%s step=%d pos=%d bytes_identical=%d max_abs=%.3e mean_abs=%.3e %s\n",
                        names[mode], s, p, bytes_ok ? 1 : 0, st.max_abs, st.mean_abs,
                        ok ? "OK" : "FAIL");
            std::fflush(stdout);
            fails += ok ? 0 : 1;
        }
    }
    for (void* ptr : {static_cast<void*>(dk), static_cast<void*>(dv), static_cast<void*>(dq),
                      static_cast<void*>(dq2), static_cast<void*>(dk2), static_cast<void*>(dgq),
                      static_cast<void*>(dgk), static_cast<void*>(dinv), static_cast<void*>(o1),
                      static_cast<void*>(o2), static_cast<void*>(pos)}) {
        (void)hipFree(ptr);
    }
    return fails;
}

}  // namespace

int main() {
    int fails = 0;
    fails += run_case(BackendKind::Adaptive, "adaptive");
    fails += run_case(BackendKind::Naive, "naive");
    fails += run_rope_case();
    fails += run_decode_step_case();
    std::printf("%s\n", fails == 0 ? "ALL OK" : "FAILURES");
    return fails == 0 ? 0 : 1;
}
