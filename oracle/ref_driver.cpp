// oracle/ref_driver.cpp - TEST INFRASTRUCTURE ONLY.  Links the reference's own CPU expert kernels (compiled from
// /root/reference/src/kernels/cpu/{iq_avx512,iq_avx2,kq_avx2,cpu_features}.cpp by oracle/Makefile into
// oracle/_ref/libref.so) and exposes them to Python through a C ABI, so the tests can pin the oracle against the
// reference itself and bench.py can time the reference CPU path beside the GPU.
//
//   ref_q8k_quant    -> strata::kernels::cpu::q8k_quant_avx2 (src/kernels/cpu/iq_avx2.cpp:387-454)
//   ref_rows         -> iq512_rows / iq256_rows (IQ3_XXS, IQ3_S against Q8_K; src/kernels/cpu/iq_avx512.cpp:155-186,
//                       iq_avx2.cpp) or kq256_rows (Q4_K against Q8_K, Q8_0 against Q8_0; src/kernels/cpu/kq_avx2.cpp)
//   ref_gu_rows      -> iq512_gu_rows / iq256_gu_rows / kq256_gu_rows (SwiGLU inside, native_expert.cpp:248)
//   ref_moe_decode   -> a stack of decode MoE layers with the reference CPU arithmetic, the structure of
//                       src/lfm2/cpu_experts.cpp:145-235 (quantize, gate/up + SwiGLU, quantize h, down, combine in
//                       pick order), rows shared out over `threads` pinned workers as src/kernels/cpu/pool.cpp does.
#include "strata/kernels/cpu/cpu_features.hpp"
#include "strata/kernels/cpu/iq_avx2.hpp"
#include "strata/kernels/cpu/iq_avx512.hpp"
#include "strata/kernels/cpu/kq_avx2.hpp"

#include <immintrin.h>
#include <pthread.h>
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>
#include <thread>
#include <vector>

namespace C = strata::kernels::cpu;

namespace {
bool is_iq(int t) { return t == 18 || t == 21; }
bool use512() { static const bool v = C::cpu_avx512_ok(); return v; }

void rows(int type, const uint8_t* w, size_t row_bytes, int n, const void* const* act, int nt, float* const* out, int r0, int r1) {
    if (is_iq(type)) {
        if (use512()) C::iq512_rows(type, w, row_bytes, n, act, nt, out, r0, r1);
        else C::iq256_rows(type, w, row_bytes, n, act, nt, out, r0, r1);
    } else {
        C::kq256_rows(type, w, row_bytes, n, act, nt, out, r0, r1);
    }
}
void gu_rows(int type, const uint8_t* blob, size_t gu_row, size_t up_off, int n, const void* const* act, int nt,
             float* const* ff, int r0, int r1) {
    if (is_iq(type)) {
        if (use512()) C::iq512_gu_rows(type, blob, gu_row, up_off, n, act, nt, ff, r0, r1);
        else C::iq256_gu_rows(type, blob, gu_row, up_off, n, act, nt, ff, r0, r1);
    } else {
        C::kq256_gu_rows(type, blob, gu_row, up_off, n, act, nt, ff, r0, r1);
    }
}
size_t row_bytes(int t, int n) {
    switch (t) {
        case 8: return (size_t) (n / 32) * 34;
        case 12: return (size_t) (n / 256) * 144;
        case 18: return (size_t) (n / 256) * 98;
        case 21: return (size_t) (n / 256) * 110;
        default: return 0;
    }
}
// the activation of a weight type: Q8_0 for Q8_0 rows, Q8_K otherwise
size_t act_bytes(int t, int n) { return t == 8 ? (size_t) (n / 32) * 34 : (size_t) (n / 256) * 292; }
uint16_t f2h(float f) {  // round to nearest even, as the F16C instruction
    const __m128i v = _mm_cvtps_ph(_mm_set_ss(f), _MM_FROUND_TO_NEAREST_INT);
    return (uint16_t) _mm_cvtsi128_si32(v);
}
void quant_act(int t, const float* x, int n, void* dst) {
    if (t != 8) { C::q8k_quant_avx2(x, dst, n); return; }
    uint8_t* y = (uint8_t*) dst;   // ggml quantize_row_q8_0_ref
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.f;
        for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[32 * b + j]));
        const float d = amax / 127.f, id = d != 0.f ? 1.0f / d : 0.0f;
        const uint16_t dh = f2h(d);
        std::memcpy(y + 34 * b, &dh, 2);
        for (int j = 0; j < 32; ++j) y[34 * b + 2 + j] = (uint8_t) (int8_t) std::roundf(x[32 * b + j] * id);
    }
}

// A fixed set of pinned workers that run one indexed job list at a time (the calling thread takes part).  Each
// run() publishes its own Batch; a worker counts itself in users_ before it reads the batch pointer, and run()
// takes the pointer down before it waits for users_ to reach 0, so no worker touches a finished batch.
class Pool {
public:
    // worker i (1..n-1) pinned to cpus[i] when cpus is given, else to logical CPU i
    Pool(int n, const int32_t* cpus) : n_(n) {
        for (int i = 1; i < n; ++i) th_.emplace_back([this, i, c = cpus ? cpus[i] : -1] { loop(i, c); });
    }
    ~Pool() {
        quit_.store(true);
        for (auto& t : th_) t.join();
    }
    void run(int jobs, const std::function<void(int)>& fn) {
        Batch b;
        b.fn = &fn;
        b.jobs = jobs;
        b.next.store(0);
        b.left.store(jobs);
        cur_.store(&b);
        gen_.fetch_add(1);
        drain(b);
        while (b.left.load() != 0) {}
        cur_.store(nullptr);
        while (users_.load() != 0) {}
    }

private:
    struct Batch {
        const std::function<void(int)>* fn = nullptr;
        int jobs = 0;
        std::atomic<int> next{0}, left{0};
    };
    static void drain(Batch& b) {
        for (;;) {
            const int j = b.next.fetch_add(1);
            if (j >= b.jobs) break;
            (*b.fn)(j);
            b.left.fetch_sub(1);
        }
    }
    void loop(int i, int cpu) {
        cpu_set_t s;
        CPU_ZERO(&s);
        CPU_SET(cpu >= 0 ? cpu : i % (int) std::thread::hardware_concurrency(), &s);
        pthread_setaffinity_np(pthread_self(), sizeof s, &s);
        uint64_t seen = gen_.load();
        while (!quit_.load()) {
            const uint64_t g = gen_.load();
            if (g == seen) { std::this_thread::yield(); continue; }
            seen = g;
            users_.fetch_add(1);
            Batch* b = cur_.load();
            if (b) drain(*b);
            users_.fetch_sub(1);
        }
    }
    int n_;
    std::vector<std::thread> th_;
    std::atomic<bool> quit_{false};
    std::atomic<uint64_t> gen_{0};
    std::atomic<int> users_{0};
    std::atomic<Batch*> cur_{nullptr};
};
}  // namespace

extern "C" {
__attribute__((visibility("default"))) int ref_isa() { return use512() ? 512 : C::cpu_avx2_ok() ? 256 : 0; }

__attribute__((visibility("default"))) void ref_q8k_quant(const float* x, void* y, int64_t n) { C::q8k_quant_avx2(x, y, n); }

// out[t * n_rows + r] = W[r] . act[t] over rows [0, n_rows); act: nt activations back to back
__attribute__((visibility("default"))) int ref_rows(int type, const uint8_t* w, int n, int n_rows, const void* act, int nt,
                                                    float* out) {
    const size_t rb = row_bytes(type, n), ab = act_bytes(type, n);
    if (rb == 0 || nt < 1 || nt > 8) return -1;
    const void* a[8];
    float* o[8];
    for (int t = 0; t < nt; ++t) { a[t] = (const uint8_t*) act + (size_t) t * ab; o[t] = out + (size_t) t * n_rows; }
    rows(type, w, rb, n, a, nt, o, 0, n_rows);
    return 0;
}

// ff[t * n_ff + r] = silu(gate_r . a[t]) * (up_r . a[t]); blob = [gate rows | up rows]
__attribute__((visibility("default"))) int ref_gu_rows(int type, const uint8_t* blob, int n, int n_ff, const void* act, int nt,
                                                       float* ff) {
    const size_t rb = row_bytes(type, n), ab = act_bytes(type, n);
    if (rb == 0 || nt < 1 || nt > 8) return -1;
    const void* a[8];
    float* o[8];
    for (int t = 0; t < nt; ++t) { a[t] = (const uint8_t*) act + (size_t) t * ab; o[t] = ff + (size_t) t * n_ff; }
    gu_rows(type, blob, rb, (size_t) n_ff * rb, n, a, nt, o, 0, n_ff);
    return 0;
}

// A stack of n_layers decode MoE layers on `threads` workers, `iters` passes; returns the median seconds per layer.
// Layer l: expert blobs at blobs + l * layer_stride (`stride` apart, ids index them), its shared blob (or none) at
// shared + l * layer_stride, routing ids/wts [n_layers][n_tok][k], shared-gate weights sgs [n_layers][n_tok] (already
// sigmoid).  x [n_tok][n_embd] is the first layer's input; each layer adds its output to it (x <- x + moe(x)), so
// the layers run one after another as in a model.  Layout: [gate | up | down], gate/up gu_type, down d_type.
__attribute__((visibility("default"))) double ref_moe_decode(int gu_type, int d_type, int n_embd, int n_ff, int n_tok,
                                                             int k, int n_layers, const int32_t* ids, const float* wts,
                                                             const uint8_t* blobs, uint64_t stride,
                                                             uint64_t layer_stride, const uint8_t* shared,
                                                             const float* sgs, float* x, int threads, int iters,
                                                             const int32_t* cpus) {
    if (n_tok < 1 || n_tok > 8 || k < 1 || n_layers < 1) return -1.0;
    // the calling thread works too: on cpus[0] for the duration of the call (its own mask restored afterwards)
    cpu_set_t saved;
    const bool pin_self = cpus != nullptr && sched_getaffinity(0, sizeof saved, &saved) == 0;
    if (pin_self) {
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(cpus[0], &one);
        sched_setaffinity(0, sizeof one, &one);
    }
    const size_t gu_row = row_bytes(gu_type, n_embd), d_row = row_bytes(d_type, n_ff);
    const size_t up_off = (size_t) n_ff * gu_row, down_off = 2 * up_off;
    const size_t ab = act_bytes(gu_type, n_embd), hb = act_bytes(d_type, n_ff);
    struct Use { const uint8_t* blob; std::vector<int> ents; };
    const int n_ent = n_tok * k + (shared ? n_tok : 0);
    std::vector<std::vector<Use>> uses(n_layers);
    for (int l = 0; l < n_layers; ++l) {
        const int32_t* li = ids + (size_t) l * n_tok * k;
        for (int e = 0; e < n_tok * k; ++e) {
            const uint8_t* b = blobs + l * layer_stride + (uint64_t) li[e] * stride;
            auto it = std::find_if(uses[l].begin(), uses[l].end(), [&](const Use& u) { return u.blob == b; });
            if (it == uses[l].end()) { uses[l].push_back({b, {}}); it = uses[l].end() - 1; }
            it->ents.push_back(e);
        }
        if (shared) {
            uses[l].push_back({shared + l * layer_stride, {}});
            for (int t = 0; t < n_tok; ++t) uses[l].back().ents.push_back(n_tok * k + t);
        }
    }
    std::vector<uint8_t> act((size_t) n_tok * ab), hq((size_t) n_ent * hb);
    std::vector<float> h((size_t) n_ent * n_ff), part((size_t) n_ent * n_embd);
    Pool pool(threads, cpus);
    constexpr int kGuRows = 32, kDownRows = 64;
    const int gu_tasks = (n_ff + kGuRows - 1) / kGuRows, d_tasks = (n_embd + kDownRows - 1) / kDownRows;
    std::vector<double> times;
    for (int it = 0; it < iters; ++it) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int l = 0; l < n_layers; ++l) {
            const std::vector<Use>& U = uses[l];
            const float* lw = wts + (size_t) l * n_tok * k;
            for (int t = 0; t < n_tok; ++t) quant_act(gu_type, x + (size_t) t * n_embd, n_embd, act.data() + (size_t) t * ab);
            pool.run((int) U.size() * gu_tasks, [&](int job) {
                const Use& u = U[job / gu_tasks];
                const int r0 = (job % gu_tasks) * kGuRows, r1 = std::min(n_ff, r0 + kGuRows);
                const void* a[8];
                float* o[8];
                const int nt = (int) u.ents.size();
                for (int i = 0; i < nt; ++i) {
                    const int e = u.ents[i];
                    const int t = e < n_tok * k ? e / k : e - n_tok * k;
                    a[i] = act.data() + (size_t) t * ab;
                    o[i] = h.data() + (size_t) e * n_ff;
                }
                gu_rows(gu_type, u.blob, gu_row, up_off, n_embd, a, nt, o, r0, r1);
            });
            pool.run(n_ent, [&](int e) { quant_act(d_type, h.data() + (size_t) e * n_ff, n_ff, hq.data() + (size_t) e * hb); });
            pool.run((int) U.size() * d_tasks, [&](int job) {
                const Use& u = U[job / d_tasks];
                const int r0 = (job % d_tasks) * kDownRows, r1 = std::min(n_embd, r0 + kDownRows);
                const void* a[8];
                float* o[8];
                const int nt = (int) u.ents.size();
                for (int i = 0; i < nt; ++i) {
                    a[i] = hq.data() + (size_t) u.ents[i] * hb;
                    o[i] = part.data() + (size_t) u.ents[i] * n_embd;
                }
                rows(d_type, u.blob + down_off, d_row, n_ff, a, nt, o, r0, r1);
            });
            const float* sg = shared ? sgs + (size_t) l * n_tok : nullptr;
            for (int t = 0; t < n_tok; ++t)   // the combine in pick order (k_moe_out: first product, then FMA)
                for (int i = 0; i < n_embd; ++i) {
                    float acc = lw[t * k] * part[(size_t) (t * k) * n_embd + i];
                    for (int j = 1; j < k; ++j) acc = std::fmaf(lw[t * k + j], part[(size_t) (t * k + j) * n_embd + i], acc);
                    if (shared) acc += sg[t] * part[(size_t) (n_tok * k + t) * n_embd + i];
                    x[(size_t) t * n_embd + i] += acc;
                }
        }
        times.push_back(std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count() / n_layers);
    }
    if (pin_self) sched_setaffinity(0, sizeof saved, &saved);
    std::sort(times.begin(), times.end());
    return times[times.size() / 2];
}
}
