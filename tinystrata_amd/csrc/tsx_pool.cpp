// tsx_pool.cpp - the CPU expert pool of the hybrid split: worker threads that evaluate the routed experts without a
// slot in HBM while the GPU runs the resident ones.
//
// Reference: strata::kernels::cpu::ExpertPool (include/strata/kernels/cpu/pool.hpp:111-260,
// src/kernels/cpu/pool.cpp:457-817) and the engine's CPU half of a hybrid layer (moe_hybrid_cpu,
// src/qwen35/q36_engine.cu:3090-3209).  What must hold is the reference's contract (pool.hpp:1-15): a worker never
// runs work of a batch other than the one it joined, never runs a piece twice, never counts into a batch the host
// has moved past, and no wait is unbounded.  This file meets it with a design of its own:
//
//   * Two batch slots used in turn.  The host writes a slot's description - its own copy of the format and the job
//     table, fresh counters - and then publishes the batch by storing its sequence number in `current_`.
//   * Joining: a worker adds itself to the slot's `attached` count and only then re-reads `current_`.  If the batch
//     is no longer current it leaves, having touched nothing but `attached`.  The host rewrites a slot only after
//     `attached` has fallen to zero, so a worker that joined a batch sees that batch's description for as long as it
//     stays (both sides use sequentially consistent operations, so either the worker sees the newer batch number or
//     the host sees the worker attached).
//   * Work is claimed per expert and no piece of work ever waits inside: every expert has a cursor over its gate/up
//     row chunks and one over its down row chunks.  The thread that completes an expert's last gate/up chunk
//     quantizes h and opens the expert's down chunks.  A thread that finds nothing open on one expert moves on to
//     the next; it spins only when nothing at all is open (every remaining chunk waits for an h being made).
//   * The host returns once the slot's `finished` count reaches the batch's chunk count (release/acquire: every
//     output row is then visible); it waits for `attached` only when it needs the slot again, two batches later.
//   * Idle workers spin with a pause, yield now and then, and after `spin_us_` sleep on a futex word the host bumps on
//     every publish; a sleeper count spares the system call while nobody sleeps.
//   * Every host wait is bounded by `stall_ms_`: a batch that makes no progress for that long marks the pool failed,
//     the call returns TSX_ERR_STALLED and the pool takes no further work.  The job table lives in the slot, but the
//     pointers in it are the caller's: a worker still busy with a stalled batch may go on reading the weight blobs
//     and activations and writing the output rows, so after a stall every buffer of that batch must stay valid until
//     tsx_pool_destroy has joined the workers.
//
// The row decomposition changes no result: every output row is one tsx_cpu_gu_rows / tsx_cpu_down_rows row, whichever
// thread computes it, and h is quantized from complete rows.
#include <linux/futex.h>
#include <sched.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstdio>
#include <ctime>
#include <memory>
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
int64_t ns_since(Clock::time_point a) {
    return std::chrono::duration_cast<std::chrono::nanoseconds>(Clock::now() - a).count();
}
inline void cpu_relax() {
#if defined(__x86_64__) || defined(__i386__)
    __builtin_ia32_pause();
#endif
}

// Sleep while *word == expected (at most `ms`), and wake every sleeper of *word.
void futex_sleep(std::atomic<uint32_t>* word, uint32_t expected, int ms) {
    static_assert(sizeof(std::atomic<uint32_t>) == sizeof(uint32_t), "a futex word is 32 bits");
    timespec ts{ms / 1000, (long) (ms % 1000) * 1000000L};
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(word), FUTEX_WAIT_PRIVATE, expected, &ts, nullptr, 0);
}
void futex_wake_all(std::atomic<uint32_t>* word) {
    syscall(SYS_futex, reinterpret_cast<uint32_t*>(word), FUTEX_WAKE_PRIVATE, INT_MAX, nullptr, nullptr, 0);
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

// An expert's claim state inside a batch: a cache line each, so threads on different experts never contend.
struct alignas(64) ExpertCursor {
    std::atomic<int32_t> gu_next{0};  // next gate/up chunk to hand out
    std::atomic<int32_t> gu_done{0};  // gate/up chunks completed
    std::atomic<int32_t> dn_next{0};  // next down chunk to hand out
    std::atomic<int32_t> open{0};     // 1 once h is quantized: the down chunks may be taken
};

// One batch: its description (written by the host while no worker is attached) and its counters.
struct Slot {
    alignas(64) std::atomic<int32_t> attached{0};
    alignas(64) std::atomic<int32_t> finished{0};   // chunks completed
    alignas(64) std::atomic<int32_t> unclaimed{0};  // chunks not handed out yet
    alignas(64) uint64_t seq = 0;
    tsx_cpu_fmt f{};
    int nb = 0, gu_chunks = 1, dn_chunks = 1, total = 0;
    tsx_cpu_job jobs[TSX_POOL_MAX_SPLIT];
    ExpertCursor cur[TSX_POOL_MAX_SPLIT];
    std::vector<float> ff;    // [nb][TSX_CPU_MAXT][n_ff]: SwiGLU rows
    std::vector<uint8_t> hq;  // [nb][TSX_CPU_MAXT][h_bytes]: their Q8_1

    float* ff_row(int e, int t) { return ff.data() + ((size_t) e * TSX_CPU_MAXT + t) * (size_t) f.n_ff; }
    uint8_t* hq_row(int e, int t) { return hq.data() + ((size_t) e * TSX_CPU_MAXT + t) * (size_t) f.h_bytes; }
};

// a worker's state for tsx_pool_diag; values >= 0 are the expert it works on
constexpr int32_t kIdle = -1, kSleeping = -2, kWaitingH = -3;

}  // namespace

struct tsx_pool {
    int n_ = 0;
    bool host_works_ = true;
    int tasks_ = 0;
    std::atomic<int64_t> spin_us_{20000};  // set between runs, read by idle workers
    std::atomic<int64_t> stall_ms_{60000};

    alignas(64) std::atomic<uint64_t> current_{0};  // sequence number of the batch on offer (0: none yet)
    alignas(64) std::atomic<uint32_t> bell_{0};     // futex word: bumped on every publish and at shutdown
    alignas(64) std::atomic<int32_t> sleepers_{0};
    alignas(64) std::atomic<bool> stop_{false};
    std::atomic<bool> failed_{false};
    uint64_t seq_ = 0;  // host only: the last batch published
    Slot slot_[2];
    std::vector<std::thread> threads_;
    struct alignas(64) WState {
        std::atomic<int32_t> v{kIdle};
    };
    std::unique_ptr<WState[]> wstate_;
    std::vector<uint8_t> acts_;  // the hybrid call's quantized token rows

    // statistics: [0] waiting for a slot's workers to leave, [1] batches from publish to finished (host);
    // [2] gate/up rows, [3] quantizing h, [4] down rows, [5] spinning with nothing open (all threads, summed)
    std::atomic<int64_t> ns_[6] = {};
    int64_t bytes_ = 0;

    void add_ns(int i, int64_t v) { ns_[i].fetch_add(v, std::memory_order_relaxed); }
    void set_state(int id, int32_t v) {
        if (id >= 0) wstate_[id].v.store(v, std::memory_order_relaxed);
    }

    // ---- the workers
    uint64_t next_batch(uint64_t seen, int id) {  // 0 when stopping
        set_state(id, kIdle);
        const auto t0 = Clock::now();
        for (uint32_t spins = 1;; ++spins) {
            if (stop_.load(std::memory_order_acquire)) return 0;
            const uint64_t c = current_.load(std::memory_order_acquire);
            if (c != seen) return c;
            cpu_relax();
            if (spins % 256) continue;
            if (ns_since(t0) < spin_us_.load(std::memory_order_relaxed) * 1000) {
                if (spins % 4096 == 0) std::this_thread::yield();
                continue;
            }
            set_state(id, kSleeping);
            sleepers_.fetch_add(1, std::memory_order_seq_cst);
            const uint32_t b = bell_.load(std::memory_order_seq_cst);
            if (current_.load(std::memory_order_seq_cst) == seen && !stop_.load(std::memory_order_seq_cst))
                futex_sleep(&bell_, b, 100);
            sleepers_.fetch_sub(1, std::memory_order_relaxed);
            set_state(id, kIdle);
        }
    }
    void worker(int id) {
        uint64_t seen = 0;
        for (;;) {
            const uint64_t s = next_batch(seen, id);
            if (s == 0) return;
            seen = s;
            Slot& S = slot_[s & 1];
            S.attached.fetch_add(1, std::memory_order_seq_cst);
            if (current_.load(std::memory_order_seq_cst) == s) work(S, id);
            S.attached.fetch_sub(1, std::memory_order_release);
        }
    }

    // ---- the work of one batch, for a worker (id >= 0) or the host (id = -1)
    void work(Slot& S, int id) {
        const int nb = S.nb, G = S.gu_chunks, D = S.dn_chunks;
        const int threads = n_ + (host_works_ ? 1 : 0);
        int at = (int) ((int64_t) (id + 1) * nb / std::max(1, threads));  // threads start spread over the experts
        Clock::time_point idle_since{};
        bool idle = false;
        while (S.unclaimed.load(std::memory_order_acquire) > 0) {
            bool did = false;
            for (int i = 0; i < nb && !did; ++i) {
                const int e = (at + i) % nb;
                ExpertCursor& X = S.cur[e];
                if (X.gu_next.load(std::memory_order_relaxed) < G) {
                    const int c = X.gu_next.fetch_add(1, std::memory_order_relaxed);
                    if (c >= G) continue;
                    did = true;
                    at = e;
                    if (idle) add_ns(5, ns_since(idle_since)), idle = false;
                    set_state(id, e);
                    S.unclaimed.fetch_sub(1, std::memory_order_relaxed);
                    gate_up_chunk(S, e, c);
                    if (X.gu_done.fetch_add(1, std::memory_order_acq_rel) + 1 == G) {  // every row of h is in
                        const auto t = Clock::now();
                        for (int tk = 0; tk < S.jobs[e].nt; ++tk) tsx::cpu_quant(S.ff_row(e, tk), S.f.n_ff, S.hq_row(e, tk));
                        add_ns(3, ns_since(t));
                        X.open.store(1, std::memory_order_release);
                    }
                    S.finished.fetch_add(1, std::memory_order_release);
                } else if (X.open.load(std::memory_order_acquire) && X.dn_next.load(std::memory_order_relaxed) < D) {
                    const int c = X.dn_next.fetch_add(1, std::memory_order_relaxed);
                    if (c >= D) continue;
                    did = true;
                    at = e;
                    if (idle) add_ns(5, ns_since(idle_since)), idle = false;
                    set_state(id, e);
                    S.unclaimed.fetch_sub(1, std::memory_order_relaxed);
                    down_chunk(S, e, c);
                    S.finished.fetch_add(1, std::memory_order_release);
                }
            }
            if (did) continue;
            // every chunk left waits for an h that another thread is making
            if (!idle) idle = true, idle_since = Clock::now(), set_state(id, kWaitingH);
            if (failed_.load(std::memory_order_relaxed) || stop_.load(std::memory_order_relaxed)) break;
            cpu_relax();
        }
        if (idle) add_ns(5, ns_since(idle_since));
    }
    void gate_up_chunk(Slot& S, int e, int c) {
        const auto t = Clock::now();
        const tsx_cpu_job& j = S.jobs[e];
        const int FF = (int) S.f.n_ff;
        float* ff[TSX_CPU_MAXT];
        for (int tk = 0; tk < j.nt; ++tk) ff[tk] = S.ff_row(e, tk);
        tsx::cpu_gu_rows(S.f, j.blob, j.act, j.nt, ff, (int) ((int64_t) FF * c / S.gu_chunks),
                         (int) ((int64_t) FF * (c + 1) / S.gu_chunks));
        add_ns(2, ns_since(t));
    }
    void down_chunk(Slot& S, int e, int c) {
        const auto t = Clock::now();
        const tsx_cpu_job& j = S.jobs[e];
        const int N = (int) S.f.n_embd;
        const void* hq[TSX_CPU_MAXT];
        for (int tk = 0; tk < j.nt; ++tk) hq[tk] = S.hq_row(e, tk);
        tsx::cpu_down_rows(S.f, j.blob, hq, j.nt, j.out, (int) ((int64_t) N * c / S.dn_chunks),
                           (int) ((int64_t) N * (c + 1) / S.dn_chunks));
        add_ns(4, ns_since(t));
    }

    // ---- the host
    // Waits for done(); false (and the pool failed) when progress() stays unchanged for the stall limit.
    template <typename Done, typename Progress>
    bool bounded_wait(Done done, Progress progress, const char* what) {
        int64_t last = progress();
        auto t0 = Clock::now();
        for (uint32_t spins = 1; !done(); ++spins) {
            cpu_relax();
            if (spins % 1024) continue;
            const int64_t p = progress();
            if (p != last) {
                last = p;
                t0 = Clock::now();
            } else if (ns_since(t0) > stall_ms_.load(std::memory_order_relaxed) * 1000000) {
                tsx::set_error("tsx_pool: no progress for %lld ms while %s", (long long) stall_ms_.load(), what);
                failed_.store(true);
                return false;
            }
        }
        return true;
    }
    int chunks_per_expert(int nb, int64_t rows) const {
        const int per_phase = tasks_ > 0 ? tasks_ : 3 * (n_ + (host_works_ ? 1 : 0));
        return (int) std::clamp<int64_t>((per_phase + nb - 1) / nb, 1, rows);
    }
    int run_batch(const tsx_cpu_fmt& f, const tsx_cpu_job* jobs, int nb) {
        const uint64_t s = seq_ + 1;
        Slot& S = slot_[s & 1];
        const auto t0 = Clock::now();
        // workers that joined this slot's previous batch (two batches back) must have left before it is rewritten
        if (!bounded_wait([&] { return S.attached.load(std::memory_order_seq_cst) == 0; },
                          [&] { return (int64_t) S.attached.load(std::memory_order_relaxed); },
                          "waiting for workers to leave a finished batch"))
            return TSX_ERR_STALLED;
        const auto t1 = Clock::now();
        S.f = f;
        S.nb = nb;
        std::copy(jobs, jobs + nb, S.jobs);
        S.gu_chunks = chunks_per_expert(nb, f.n_ff);
        S.dn_chunks = chunks_per_expert(nb, f.n_embd);
        S.total = nb * (S.gu_chunks + S.dn_chunks);
        const size_t ffn = (size_t) nb * TSX_CPU_MAXT * (size_t) f.n_ff;
        const size_t hqn = (size_t) nb * TSX_CPU_MAXT * (size_t) f.h_bytes;
        if (S.ff.size() < ffn) S.ff.resize(ffn);
        if (S.hq.size() < hqn) S.hq.resize(hqn);
        for (int e = 0; e < nb; ++e) {
            S.cur[e].gu_next.store(0, std::memory_order_relaxed);
            S.cur[e].gu_done.store(0, std::memory_order_relaxed);
            S.cur[e].dn_next.store(0, std::memory_order_relaxed);
            S.cur[e].open.store(0, std::memory_order_relaxed);
        }
        S.finished.store(0, std::memory_order_relaxed);
        S.unclaimed.store(S.total, std::memory_order_relaxed);
        S.seq = s;
        seq_ = s;
        // publish: the description above happens-before any worker's read of it (its seq_cst load of current_)
        current_.store(s, std::memory_order_seq_cst);
        bell_.fetch_add(1, std::memory_order_seq_cst);
        if (sleepers_.load(std::memory_order_seq_cst) > 0) futex_wake_all(&bell_);
        if (host_works_) work(S, -1);
        const bool ok =
            bounded_wait([&] { return S.finished.load(std::memory_order_acquire) == S.total; },
                         [&] { return (int64_t) S.finished.load(std::memory_order_relaxed); }, "running a batch");
        add_ns(0, std::chrono::duration_cast<std::chrono::nanoseconds>(t1 - t0).count());
        add_ns(1, ns_since(t1));
        return ok ? (int) TSX_OK : (int) TSX_ERR_STALLED;
    }
    int run(const tsx_cpu_fmt& f, const tsx_cpu_job* jobs, int n) {
        if (failed_.load()) {
            tsx::set_error("tsx_pool: the pool stalled earlier and takes no more work");
            return TSX_ERR_STALLED;
        }
        for (int b0 = 0; b0 < n; b0 += TSX_POOL_MAX_SPLIT) {
            const int rc = run_batch(f, jobs + b0, std::min(TSX_POOL_MAX_SPLIT, n - b0));
            if (rc != TSX_OK) return rc;
        }
        bytes_ += (int64_t) n * (int64_t) f.bytes;
        return TSX_OK;
    }

    void shutdown() {
        stop_.store(true, std::memory_order_seq_cst);
        bell_.fetch_add(1, std::memory_order_seq_cst);
        futex_wake_all(&bell_);
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
    for (int i = 0; i < 6; ++i) ms6[i] = (double) p->ns_[i].load() * 1e-6;
    if (bytes) *bytes = p->bytes_;
    return TSX_OK;
}

TSX_API int tsx_pool_diag(const tsx_pool* p, char* buf, size_t n) {
    clear_error();
    TSX_REQUIRE(p && buf && n > 0, "tsx_pool_diag: pool and a buffer");
    const uint64_t c = p->current_.load();
    const Slot& S = p->slot_[c & 1];
    int idle = 0;
    for (int i = 0; i < p->n_; ++i) idle += p->wstate_[i].v.load() == kIdle || p->wstate_[i].v.load() == kSleeping;
    int w = std::snprintf(buf, n,
                          "batch %llu: %d experts, %d/%d chunks finished, %d unclaimed, attached %d|%d; idle %d/%d, "
                          "sleepers %d%s; workers:",
                          (unsigned long long) c, c ? S.nb : 0, c ? S.finished.load() : 0, c ? S.total : 0,
                          c ? S.unclaimed.load() : 0, p->slot_[0].attached.load(), p->slot_[1].attached.load(), idle,
                          p->n_, p->sleepers_.load(), p->failed_.load() ? " FAILED" : "");
    for (int i = 0; i < p->n_ && w > 0 && (size_t) w < n; ++i) {
        const int32_t st = p->wstate_[i].v.load();
        const char* name = st == kIdle ? "idle" : st == kSleeping ? "sleeping" : st == kWaitingH ? "waiting-h" : nullptr;
        w += name ? std::snprintf(buf + w, n - (size_t) w, " %s", name)
                  : std::snprintf(buf + w, n - (size_t) w, " expert %d", st);
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
    if (p->failed_.load()) {  // workers may still read the stalled batch's token rows in acts_
        set_error("tsx_pool: the pool stalled earlier and takes no more work");
        return TSX_ERR_STALLED;
    }
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
    TSX_REQUIRE(f->n_embd == L.n_embd && f->n_ff == L.n_ff && f->gu_type == L.gu_type && f->d_type == L.d_type &&
                    f->up_off == L.up_off && f->down_off == L.down_off && a->stride >= f->bytes,
                "tsx_moe_hybrid_decode_layer: the CPU format does not describe the layer's experts");
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
