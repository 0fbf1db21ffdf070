// tsx_pool.cpp - the CPU expert pool of the hybrid split: worker threads that evaluate the routed experts without a
// slot in HBM, in row tasks, while the GPU runs the resident ones.
//
// Reference: strata::kernels::cpu::ExpertPool (include/strata/kernels/cpu/pool.hpp:111-260,
// src/kernels/cpu/pool.cpp:457-817) and the engine's CPU half of a hybrid layer (moe_hybrid_cpu,
// src/qwen35/q36_engine.cu:3090-3209).
//
// The completion protocol is the reference's (pool.hpp:1-15), in code of this library's own:
//   * A batch is published by writing its description, resetting `done`, storing `head` = epoch << 32 |
//     njobs << 16 | 0 and bumping `epoch` (seq_cst, so a worker going to sleep and the host publishing cannot both
//     miss each other: the worker adds itself to `sleepers` and then reads `epoch`, the host bumps `epoch` and then
//     reads `sleepers`).
//   * A claim is a CAS on `head` that succeeds only for the epoch the worker woke for, so a worker that wakes late
//     can never take a job of a later batch, run a job twice, or add to a `done` that was already reset.
//   * The host waits for `done == njobs` and then for every worker to be parked again before it writes the next
//     batch.  Every wait is bounded (`stall`): a pool that sees no progress for that long marks itself failed and
//     returns TSX_ERR_STALLED instead of spinning forever.
//   * A parked worker spins with a pause instruction, yields every 50 us, and sleeps on a condition variable after
//     `spin` (20 ms by default), so an idle engine does not hold every core busy.
// Each shared atomic sits on its own cache line.  The row decomposition changes no result: every output row is one
// tsx_cpu_gu_rows / tsx_cpu_down_rows row, whichever thread computes it.
#include <sched.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstdio>
#include <memory>
#include <mutex>
#include <set>
#include <thread>
#include <utility>
#include <vector>

#include "tsx_common.hpp"
#include "tsx_pool.h"

namespace tsx {
int cpu_gu_rows(const tsx_cpu_fmt& f, const uint8_t* blob, const void* const* act, int nt, float* const* ff, int r0,
                int r1);
int cpu_down_rows(const tsx_cpu_fmt& f, const uint8_t* blob, const void* const* hq, int nt, float* const* out,
                  int r0, int r1);
void cpu_quant(const float* x, int64_t n, void* dst);
}  // namespace tsx

namespace {

using Clock = std::chrono::steady_clock;
double ms_between(Clock::time_point a, Clock::time_point b) {
    return std::chrono::duration<double, std::milli>(b - a).count();
}
inline void cpu_relax() {
#if defined(__x86_64__) || defined(__i386__)
    __builtin_ia32_pause();
#endif
}

// One logical CPU per physical core the process may run on (Linux sysfs topology), in CPU order; empty when the
// topology cannot be read.
std::vector<int> physical_cores() {
    std::vector<int> out;
    cpu_set_t set;
    CPU_ZERO(&set);
    if (sched_getaffinity(0, sizeof set, &set) != 0) return out;
    std::set<std::pair<int, int>> seen;
    for (int c = 0; c < CPU_SETSIZE; ++c) {
        if (!CPU_ISSET(c, &set)) continue;
        int core = -1, pkg = -1;
        char path[128];
        std::snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/core_id", c);
        if (FILE* f = std::fopen(path, "r")) {
            if (std::fscanf(f, "%d", &core) != 1) core = -1;
            std::fclose(f);
        }
        std::snprintf(path, sizeof path, "/sys/devices/system/cpu/cpu%d/topology/physical_package_id", c);
        if (FILE* f = std::fopen(path, "r")) {
            if (std::fscanf(f, "%d", &pkg) != 1) pkg = -1;
            std::fclose(f);
        }
        if (core < 0) return {};
        if (seen.insert({pkg, core}).second) out.push_back(c);
    }
    return out;
}

constexpr uint64_t pack_head(uint32_t epoch, uint32_t n, uint32_t i) {
    return (uint64_t) epoch << 32 | (uint64_t) (n & 0xFFFFu) << 16 | (i & 0xFFFFu);
}

}  // namespace

struct tsx_pool {
    enum Mode { kNone = 0, kGateUp = 1, kDown = 2, kFused = 3 };

    int n_ = 0;
    bool host_works_ = true;
    int tasks_ = 0;
    std::atomic<int64_t> spin_us_{20000};   // set between runs, read by parked workers
    std::atomic<int64_t> stall_ms_{60000};

    alignas(64) std::atomic<uint64_t> head_{0};
    alignas(64) std::atomic<uint32_t> done_{0};
    alignas(64) std::atomic<uint32_t> parked_{0};
    alignas(64) std::atomic<uint32_t> epoch_{0};
    alignas(64) std::atomic<uint32_t> sleepers_{0};
    alignas(64) std::atomic<bool> stop_{false};
    std::atomic<bool> failed_{false};
    std::mutex mu_;
    std::condition_variable cv_;
    std::vector<std::thread> threads_;
    // each worker's state for tsx_pool_diag: parked, sleeping, between batches, or the job it runs
    static constexpr int32_t kParked = -1, kSleeping = -2, kBetween = -3;
    struct alignas(64) WState {  // a line each: a worker's stores never contend with another's
        std::atomic<int32_t> v{kParked};
    };
    std::unique_ptr<WState[]> wstate_;

    // the current batch: written by the host before it publishes, read by the workers after their acquire
    Mode mode_ = kNone;
    const tsx_cpu_fmt* f_ = nullptr;
    const tsx_cpu_job* jobs_ = nullptr;
    int64_t rows_ = 0;
    int ntasks_ = 1, gu_parts_ = 1, down_parts_ = 1, nb_ = 0;
    std::vector<float> ff_;      // [TSX_POOL_MAX_SPLIT][MAXT][n_ff]
    std::vector<uint8_t> hq_;    // [TSX_POOL_MAX_SPLIT][MAXT][h_bytes]
    struct alignas(64) Ready {
        std::atomic<int> gu_left{0};
        std::atomic<bool> ready{false};
    };
    std::unique_ptr<Ready[]> ready_{new Ready[TSX_POOL_MAX_SPLIT]};
    std::vector<uint8_t> acts_;  // the hybrid call's quantized token rows

    // statistics (host thread only)
    double ms_park_ = 0, ms_drain_ = 0, ms_gu_ = 0, ms_q_ = 0, ms_down_ = 0, ms_fused_ = 0;
    int64_t bytes_ = 0;

    float* ff_row(int e, int t) { return ff_.data() + ((size_t) e * TSX_CPU_MAXT + t) * (size_t) f_->n_ff; }
    uint8_t* hq_row(int e, int t) { return hq_.data() + ((size_t) e * TSX_CPU_MAXT + t) * (size_t) f_->h_bytes; }

    // ---- the protocol
    void publish() {
        epoch_.fetch_add(1, std::memory_order_seq_cst);
        if (sleepers_.load(std::memory_order_seq_cst) != 0) {
            std::lock_guard<std::mutex> lk(mu_);
            cv_.notify_all();
        }
    }
    uint32_t begin_batch(int n) {
        done_.store(0, std::memory_order_relaxed);
        const uint32_t e = epoch_.load(std::memory_order_relaxed) + 1;  // only the host bumps the epoch
        head_.store(pack_head(e, (uint32_t) n, 0), std::memory_order_release);
        publish();
        return e;
    }
    int claim(uint32_t epoch) {
        uint64_t h = head_.load(std::memory_order_acquire);
        for (;;) {
            if ((uint32_t) (h >> 32) != epoch) return -1;  // another batch than the one this thread woke for
            const uint32_t n = (uint32_t) (h >> 16) & 0xFFFFu, i = (uint32_t) h & 0xFFFFu;
            if (i >= n) return -1;
            if (head_.compare_exchange_weak(h, h + 1, std::memory_order_acq_rel, std::memory_order_acquire))
                return (int) i;
        }
    }
    void worker(int id) {
        uint32_t seen = 0;
        wstate_[id].v.store(kParked, std::memory_order_relaxed);
        parked_.fetch_add(1, std::memory_order_acq_rel);  // parked from the start: the first run waits for that
        for (;;) {
            const auto parked_at = Clock::now();
            auto yield_at = parked_at + std::chrono::microseconds(50);
            uint32_t spins = 0;
            while (epoch_.load(std::memory_order_acquire) == seen) {
                if (stop_.load(std::memory_order_relaxed)) return;
                cpu_relax();
                if ((++spins & 63u) != 0) continue;
                const auto now = Clock::now();
                if (now - parked_at < std::chrono::microseconds(spin_us_.load(std::memory_order_relaxed))) {
                    if (now >= yield_at) {
                        std::this_thread::yield();
                        yield_at = now + std::chrono::microseconds(50);
                    }
                    continue;
                }
                std::unique_lock<std::mutex> lk(mu_);
                wstate_[id].v.store(kSleeping, std::memory_order_relaxed);
                sleepers_.fetch_add(1, std::memory_order_seq_cst);
                cv_.wait(lk, [&] {
                    return epoch_.load(std::memory_order_seq_cst) != seen || stop_.load(std::memory_order_relaxed);
                });
                sleepers_.fetch_sub(1, std::memory_order_relaxed);
                wstate_[id].v.store(kParked, std::memory_order_relaxed);
            }
            if (stop_.load(std::memory_order_acquire)) return;
            seen = epoch_.load(std::memory_order_acquire);
            parked_.fetch_sub(1, std::memory_order_acq_rel);
            wstate_[id].v.store(kBetween, std::memory_order_relaxed);
            drain(seen, id);
            wstate_[id].v.store(kParked, std::memory_order_relaxed);
            parked_.fetch_add(1, std::memory_order_acq_rel);
        }
    }
    void drain(uint32_t epoch, int id = -1) {
        for (int i; (i = claim(epoch)) >= 0;) {
            if (id >= 0) wstate_[id].v.store(i, std::memory_order_relaxed);
            run_task(i);
            done_.fetch_add(1, std::memory_order_release);
        }
    }
    // a bounded wait: false (and the pool failed) after `stall_` without progress
    template <typename Done, typename Progress>
    bool bounded_wait(Done done, Progress progress, const char* what) {
        uint32_t spins = 0, last = progress();
        auto t0 = Clock::now();
        while (!done()) {
            cpu_relax();
            if ((++spins & 1023u) != 0) continue;
            if (failed_.load(std::memory_order_relaxed)) return false;
            const uint32_t p = progress();
            const auto now = Clock::now();
            if (p != last) {
                last = p;
                t0 = now;
            } else if (now - t0 > std::chrono::milliseconds(stall_ms_.load(std::memory_order_relaxed))) {
                tsx::set_error("tsx_pool: stalled %s (%u of %d jobs done, %u of %d workers parked)", what,
                               done_.load(), ntasks_, parked_.load(), n_);
                failed_.store(true);
                return false;
            }
        }
        return true;
    }
    bool wait_parked(const char* what) {
        return bounded_wait([&] { return parked_.load(std::memory_order_acquire) == (uint32_t) n_; },
                            [&] { return parked_.load(std::memory_order_relaxed); }, what);
    }
    bool run_phase(Mode mode, int n) {
        const auto a = Clock::now();
        if (!wait_parked("before a phase")) return false;
        const auto b = Clock::now();
        mode_ = mode;
        ntasks_ = n;
        const uint32_t e = begin_batch(n);
        if (host_works_) drain(e);
        const bool ok = bounded_wait([&] { return done_.load(std::memory_order_acquire) >= (uint32_t) n; },
                                     [&] { return done_.load(std::memory_order_relaxed); }, "draining a phase") &&
                        wait_parked("after a phase");
        const auto c = Clock::now();
        ms_park_ += ms_between(a, b);
        ms_drain_ += ms_between(b, c);
        return ok;
    }

    // ---- the work
    void rows_task(int i) {  // gate/up or down rows [g0, g1) of the batch's experts, one after another
        const tsx_cpu_fmt& f = *f_;
        const int per = mode_ == kGateUp ? (int) f.n_ff : (int) f.n_embd;
        const int64_t g0 = rows_ * i / ntasks_, g1 = rows_ * (i + 1) / ntasks_;
        for (int64_t r = g0; r < g1;) {
            const int e = (int) (r / per), r0 = (int) (r % per);
            const int r1 = (int) std::min<int64_t>(per, r0 + (g1 - r));
            expert_rows(e, mode_ == kGateUp, r0, r1);
            r += r1 - r0;
        }
    }
    void expert_rows(int e, bool gate_up, int r0, int r1) {
        const tsx_cpu_job& j = jobs_[e];
        if (gate_up) {
            float* ff[TSX_CPU_MAXT];
            for (int t = 0; t < j.nt; ++t) ff[t] = ff_row(e, t);
            tsx::cpu_gu_rows(*f_, j.blob, j.act, j.nt, ff, r0, r1);
        } else {
            const void* hq[TSX_CPU_MAXT];
            for (int t = 0; t < j.nt; ++t) hq[t] = hq_row(e, t);
            tsx::cpu_down_rows(*f_, j.blob, hq, j.nt, j.out, r0, r1);
        }
    }
    void quant_h(int e) {
        for (int t = 0; t < jobs_[e].nt; ++t) tsx::cpu_quant(ff_row(e, t), f_->n_ff, hq_row(e, t));
    }
    void run_task(int i) {
        if (mode_ != kFused) {
            rows_task(i);
            return;
        }
        // gate/up tasks first (index order), then down tasks: a down task waits only for gate/up tasks that are
        // already running
        const int gu_tasks = nb_ * gu_parts_;
        if (i < gu_tasks) {
            const int e = i / gu_parts_, part = i % gu_parts_;
            const int FF = (int) f_->n_ff;
            expert_rows(e, true, FF * part / gu_parts_, FF * (part + 1) / gu_parts_);
            if (ready_[e].gu_left.fetch_sub(1, std::memory_order_acq_rel) == 1) {  // the expert's last rows: h
                quant_h(e);
                ready_[e].ready.store(true, std::memory_order_release);
            }
            return;
        }
        const int d = i - gu_tasks, e = d / down_parts_, part = d % down_parts_;
        if (!ready_[e].ready.load(std::memory_order_acquire) &&
            !bounded_wait([&] { return ready_[e].ready.load(std::memory_order_acquire); },
                          [&] { return done_.load(std::memory_order_relaxed); }, "waiting for an expert's h"))
            return;
        const int N = (int) f_->n_embd;
        expert_rows(e, false, N * part / down_parts_, N * (part + 1) / down_parts_);
    }
    int phase_tasks(int64_t rows) const {
        const int t = tasks_ == 0 ? 3 * (n_ + (host_works_ ? 1 : 0)) : tasks_;
        return (int) std::max<int64_t>(1, std::min<int64_t>(rows, t));
    }

    int stalled() {
        if (*tsx::error_cstr() == 0) tsx::set_error("tsx_pool: a worker stalled waiting for an expert's h");
        return TSX_ERR_STALLED;
    }
    int run(const tsx_cpu_fmt& f, const tsx_cpu_job* jobs, int n) {
        if (failed_.load()) {
            tsx::set_error("tsx_pool: the pool stalled earlier and takes no more work");
            return TSX_ERR_STALLED;
        }
        f_ = &f;
        const size_t ffn = (size_t) TSX_POOL_MAX_SPLIT * TSX_CPU_MAXT * (size_t) f.n_ff;
        const size_t hqn = (size_t) TSX_POOL_MAX_SPLIT * TSX_CPU_MAXT * (size_t) f.h_bytes;
        if (ff_.size() < ffn) ff_.resize(ffn);
        if (hq_.size() < hqn) hq_.resize(hqn);
        const int participants = n_ + (host_works_ ? 1 : 0);
        for (int b0 = 0; b0 < n; b0 += TSX_POOL_MAX_SPLIT) {
            const int nb = std::min(TSX_POOL_MAX_SPLIT, n - b0);
            jobs_ = jobs + b0;
            nb_ = nb;
            if (nb > 1 && participants > 1) {  // dependent gate/up and down tasks per expert
                const auto a = Clock::now();
                // the reference's split of the tasks between the phases by their weight bytes (pool.cpp:782-788)
                const double gu_share =
                    (double) (2 * f.up_off) / (double) (2 * f.up_off + f.d_row * (uint64_t) f.n_embd);
                const int target = 2 * phase_tasks((int64_t) nb * (f.n_ff + f.n_embd));
                gu_parts_ = (int) std::min<int64_t>(f.n_ff, std::max(1L, std::lround(target * gu_share / nb)));
                down_parts_ =
                    (int) std::min<int64_t>(f.n_embd, std::max(1L, std::lround(target * (1.0 - gu_share) / nb)));
                while ((int64_t) nb * (gu_parts_ + down_parts_) > 0xFFFF) {
                    gu_parts_ = std::max(1, gu_parts_ / 2);
                    down_parts_ = std::max(1, down_parts_ / 2);
                }
                for (int e = 0; e < nb; ++e) {
                    ready_[e].gu_left.store(gu_parts_, std::memory_order_relaxed);
                    ready_[e].ready.store(false, std::memory_order_relaxed);
                }
                if (!run_phase(kFused, nb * (gu_parts_ + down_parts_)) || failed_.load()) return stalled();
                ms_fused_ += ms_between(a, Clock::now());
                continue;
            }
            const auto a = Clock::now();
            rows_ = (int64_t) nb * f.n_ff;
            if (!run_phase(kGateUp, phase_tasks(rows_))) return stalled();
            const auto b = Clock::now();
            for (int e = 0; e < nb; ++e) quant_h(e);
            const auto c = Clock::now();
            rows_ = (int64_t) nb * f.n_embd;
            if (!run_phase(kDown, phase_tasks(rows_))) return stalled();
            ms_gu_ += ms_between(a, b);
            ms_q_ += ms_between(b, c);
            ms_down_ += ms_between(c, Clock::now());
        }
        mode_ = kNone;
        bytes_ += (int64_t) n * (int64_t) f.bytes;
        return TSX_OK;
    }

    void shutdown() {
        stop_.store(true, std::memory_order_seq_cst);
        {
            std::lock_guard<std::mutex> lk(mu_);
            cv_.notify_all();
        }
        for (auto& t : threads_) t.join();
        threads_.clear();
    }
};

using namespace tsx;

extern "C" {

TSX_API int tsx_pool_create(int n_workers, int pin, int host_works, int tasks, tsx_pool** out) {
    clear_error();
    TSX_REQUIRE(out != nullptr && tasks >= 0 && tasks <= 4096 && n_workers <= 1024,
                "tsx_pool_create: out, 0 <= tasks <= 4096, n_workers <= 1024");
    *out = nullptr;
    const std::vector<int> cores = physical_cores();
    if (n_workers <= 0) n_workers = std::max(1, (int) cores.size() - 1);
    auto p = std::make_unique<tsx_pool>();
    p->n_ = n_workers;
    p->wstate_.reset(new tsx_pool::WState[(size_t) n_workers]);
    p->host_works_ = host_works != 0;
    p->tasks_ = tasks;
    try {
        for (int i = 0; i < n_workers; ++i) {
            p->threads_.emplace_back([q = p.get(), i] { q->worker(i); });
            // worker i on physical core i + 1 (the first is the host thread's), while there are cores
            if (pin && i + 1 < (int) cores.size()) {
                cpu_set_t set;
                CPU_ZERO(&set);
                CPU_SET(cores[(size_t) i + 1], &set);
                pthread_setaffinity_np(p->threads_.back().native_handle(), sizeof set, &set);
            }
        }
    } catch (const std::exception& e) {
        p->shutdown();
        set_error("tsx_pool_create: %s", e.what());
        return TSX_ERR_ARG;
    }
    *out = p.release();
    return TSX_OK;
}

TSX_API void tsx_pool_destroy(tsx_pool* p) {
    if (!p) return;
    p->shutdown();
    delete p;
}

TSX_API int tsx_pool_workers(const tsx_pool* p) { return p ? p->n_ : 0; }
TSX_API int tsx_pool_host_works(const tsx_pool* p) { return p && p->host_works_ ? 1 : 0; }

TSX_API int tsx_pool_run(tsx_pool* p, const tsx_cpu_fmt* f, const tsx_cpu_job* jobs, int n) {
    clear_error();
    TSX_REQUIRE(p && f && f->gu_act == 9 && f->d_act == 9 && n >= 0 && (n == 0 || jobs),
                "tsx_pool_run: pool, a format from tsx_cpu_fmt_init, n >= 0 jobs");
    for (int i = 0; i < n; ++i) {
        TSX_REQUIRE(jobs[i].blob && jobs[i].nt >= 1 && jobs[i].nt <= TSX_CPU_MAXT, "tsx_pool_run: job %d: blob, 1..8 "
                    "tokens", i);
        for (int t = 0; t < jobs[i].nt; ++t)
            TSX_REQUIRE(jobs[i].act[t] && jobs[i].out[t], "tsx_pool_run: job %d token %d: act and out", i, t);
    }
    if (n == 0) return TSX_OK;
    return p->run(*f, jobs, n);
}

TSX_API int tsx_pool_stats(const tsx_pool* p, double* ms6, int64_t* bytes) {
    clear_error();
    TSX_REQUIRE(p && ms6, "tsx_pool_stats: pool and ms6");
    const double v[6] = {p->ms_park_, p->ms_drain_, p->ms_gu_, p->ms_q_, p->ms_down_, p->ms_fused_};
    for (int i = 0; i < 6; ++i) ms6[i] = v[i];
    if (bytes) *bytes = p->bytes_;
    return TSX_OK;
}

TSX_API int tsx_pool_diag(const tsx_pool* p, char* buf, size_t n) {
    clear_error();
    TSX_REQUIRE(p && buf && n > 0, "tsx_pool_diag: pool and a buffer");
    const uint64_t h = p->head_.load();
    int w = std::snprintf(buf, n, "epoch %u head epoch %u jobs %u next %u done %u parked %u/%d sleepers %u%s; workers:",
                          p->epoch_.load(), (uint32_t) (h >> 32), (uint32_t) (h >> 16) & 0xFFFFu,
                          (uint32_t) h & 0xFFFFu, p->done_.load(), p->parked_.load(), p->n_, p->sleepers_.load(),
                          p->failed_.load() ? " FAILED" : "");
    for (int i = 0; i < p->n_ && w > 0 && (size_t) w < n; ++i) {
        const int32_t st = p->wstate_[i].v.load();
        const char* name = st == tsx_pool::kParked ? "parked" : st == tsx_pool::kSleeping ? "sleeping"
                           : st == tsx_pool::kBetween ? "between" : nullptr;
        w += name ? std::snprintf(buf + w, n - (size_t) w, " %s", name)
                  : std::snprintf(buf + w, n - (size_t) w, " job %d", st);
    }
    return TSX_OK;
}

TSX_API int tsx_pool_set_spin_us(tsx_pool* p, int64_t us) {
    clear_error();
    TSX_REQUIRE(p && us >= 0, "tsx_pool_set_spin_us: pool, us >= 0");
    p->spin_us_.store(us);
    return TSX_OK;
}

TSX_API int tsx_pool_set_stall_ms(tsx_pool* p, int64_t ms) {
    clear_error();
    TSX_REQUIRE(p && ms > 0, "tsx_pool_set_stall_ms: pool, ms > 0");
    p->stall_ms_.store(ms);
    return TSX_OK;
}

TSX_API int tsx_moe_hybrid_cpu(tsx_pool* p, const tsx_cpu_fmt* f, const uint8_t* host_blobs, uint64_t stride,
                               const int32_t* slot_of, int n_expert, int k, int n_tok, const int32_t* ids,
                               const float* x, float* cpu_out, int32_t* miss, int32_t* n_miss) {
    clear_error();
    TSX_REQUIRE(p && f && f->gu_act == 9 && host_blobs && stride >= f->bytes && slot_of && n_expert > 0 && k >= 1 &&
                    n_tok >= 0 && ids && x && cpu_out && miss && n_miss,
                "tsx_moe_hybrid_cpu: pool, format, host blobs (stride >= blob bytes), slot_of, ids, x, outputs");
    const int n_ent = n_tok * k;
    const int64_t N = f->n_embd;
    std::vector<char> quantized((size_t) n_tok, 0);
    std::vector<int> open((size_t) n_expert, -1);  // expert -> its job with room
    std::vector<tsx_cpu_job> jobs;
    if (p->acts_.size() < (size_t) n_tok * f->act_bytes) p->acts_.resize((size_t) n_tok * f->act_bytes);
    int nm = 0;
    for (int e = 0; e < n_ent; ++e) {
        const int xe = ids[e];
        TSX_REQUIRE(xe >= 0 && xe < n_expert, "tsx_moe_hybrid_cpu: entry %d routes to expert %d of %d", e, xe,
                    n_expert);
        if (slot_of[xe] >= 0) {
            miss[e] = -1;
            continue;
        }
        const int row = nm++, t = e / k;
        miss[e] = row;
        uint8_t* act = p->acts_.data() + (size_t) t * f->act_bytes;
        if (!quantized[(size_t) t]) {
            cpu_quant(x + (int64_t) t * N, N, act);
            quantized[(size_t) t] = 1;
        }
        int j = open[(size_t) xe];
        if (j < 0 || jobs[(size_t) j].nt == TSX_CPU_MAXT) {
            tsx_cpu_job nj{};
            nj.blob = host_blobs + (uint64_t) xe * stride;
            jobs.push_back(nj);
            j = open[(size_t) xe] = (int) jobs.size() - 1;
        }
        tsx_cpu_job& jb = jobs[(size_t) j];
        jb.act[jb.nt] = act;
        jb.out[jb.nt] = cpu_out + (int64_t) row * N;
        ++jb.nt;
    }
    *n_miss = nm;
    if (nm == 0) return TSX_OK;
    return p->run(*f, jobs.data(), (int) jobs.size());
}

TSX_API int tsx_moe_hybrid_decode_layer(tsx_pool* p, const tsx_cpu_fmt* f, tsx_hybrid_layer* a, void* stream) {
    clear_error();
    TSX_REQUIRE(p && f && a && a->n_tok >= 1 && a->n_tok <= 8 && a->k >= 1 && a->host_blobs && a->slot_of &&
                    a->d_slot_of && a->slots && a->x && a->logits && a->y && a->ids && a->wts && a->grp_ptr &&
                    a->grp_start && a->n_groups && a->ent_dst && a->ent_tok && a->xq && a->scratch && a->parts &&
                    a->h_ids && a->h_x && a->h_rows && a->h_miss && a->d_rows && a->d_miss &&
                    (!a->shared || (a->sgate && a->sh_gate && a->sh_up && a->sh_hq && a->sh_out)),
                "tsx_moe_hybrid_decode_layer: a null buffer, or n_tok outside 1..8");
    const tsx_expert_layout& L = a->L;
    const int T = a->n_tok, k = a->k, n_ent = T * k, N = (int) L.n_embd, FF = (int) L.n_ff;
    const hipStream_t st = (hipStream_t) stream;
    // one event per calling thread and device (an event records only on a stream of its own device)
    thread_local hipEvent_t events[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        set_error("tsx_moe_hybrid_decode_layer: no current device (or more than 64)");
        return TSX_ERR_ARG;
    }
    hipEvent_t& routed = events[device];
    if (!routed && hipEventCreateWithFlags(&routed, hipEventDisableTiming) != hipSuccess) {
        set_error("tsx_moe_hybrid_decode_layer: hipEventCreate failed");
        return TSX_ERR_ARG;
    }
    int rc;
#define TSX_TRY(call)                    \
    if ((rc = (call)) != TSX_OK) return rc;
#define TSX_HIP(call)                                                                           \
    if (hipError_t e = (call); e != hipSuccess) {                                               \
        set_error("tsx_moe_hybrid_decode_layer: %s: %s", #call, hipGetErrorString(e));          \
        return (int) e;                                                                         \
    }
    // the GPU half: routing and its round trip first, then the resident experts and the shared expert
    TSX_TRY(tsx_moe_router_topk(a->logits, a->ids, a->wts, a->n_expert, k, T, stream));
    TSX_HIP(hipMemcpyAsync(a->h_ids, a->ids, sizeof(int32_t) * (size_t) n_ent, hipMemcpyDeviceToHost, st));
    TSX_HIP(hipMemcpyAsync(a->h_x, a->x, sizeof(float) * (size_t) T * N, hipMemcpyDeviceToHost, st));
    TSX_HIP(hipEventRecord(routed, st));
    TSX_TRY(tsx_moe_group_resident(a->ids, n_ent, k, a->n_expert, a->d_slot_of, a->slots, a->stride, a->grp_ptr,
                                   a->grp_start, a->n_groups, a->ent_dst, a->ent_tok, stream));
    TSX_TRY(tsx_moe_quantize_q8_1(a->x, T, N, a->xq, stream));
    const int64_t cap = std::min(n_ent, a->n_expert);
    TSX_TRY(tsx_moe_expert_grouped(&L, a->grp_ptr, a->grp_start, a->n_groups, a->ent_dst, a->ent_tok, cap, n_ent,
                                   a->xq, a->scratch, a->parts, stream, 0));
    if (a->shared) {
        const uint8_t* sh = (const uint8_t*) a->shared;
        TSX_TRY(tsx_moe_mmvq(L.gu_type, sh, a->xq, a->sh_gate, N, FF, T, stream));
        TSX_TRY(tsx_moe_mmvq(L.gu_type, sh + L.up_off, a->xq, a->sh_up, N, FF, T, stream));
        TSX_TRY(tsx_moe_swiglu_quantize_q8_1(a->sh_gate, a->sh_up, (int64_t) T * FF, a->sh_hq, stream));
        TSX_TRY(tsx_moe_mmvq(L.d_type, sh + L.down_off, a->sh_hq, a->sh_out, FF, N, T, stream));
    }
    // the CPU half while the GPU runs: the misses on the pool, then their rows up and merged before the combine
    TSX_HIP(hipEventSynchronize(routed));
    int32_t nm = 0;
    TSX_TRY(tsx_moe_hybrid_cpu(p, f, a->host_blobs, a->stride, a->slot_of, a->n_expert, k, T, a->h_ids, a->h_x,
                               a->h_rows, a->h_miss, &nm));
    a->n_miss = nm;
    if (nm > 0) {
        TSX_HIP(hipMemcpyAsync(a->d_rows, a->h_rows, sizeof(float) * (size_t) nm * N, hipMemcpyHostToDevice, st));
        TSX_HIP(hipMemcpyAsync(a->d_miss, a->h_miss, sizeof(int32_t) * (size_t) n_ent, hipMemcpyHostToDevice, st));
        TSX_TRY(tsx_moe_merge_rows(a->parts, a->d_rows, a->d_miss, n_ent, N, stream));
    }
    return tsx_moe_combine(a->y, a->parts, nullptr, a->wts, k, a->shared ? a->sh_out : nullptr, a->sgate,
                           a->sg_stride, N, T, stream);
#undef TSX_TRY
#undef TSX_HIP
}

}  // extern "C"
