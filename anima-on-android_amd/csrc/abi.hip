// C-ABI layer of libanima_hip.so: argument checking, the device context
// (device, stream, grow-only workspace), host<->device marshaling for the
// anima_rt drop-in entry points, and the cross-attention context K/V cache.
// Kernels live in the other translation units.
#include "common.h"

#include "anima_hip.h"

#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <condition_variable>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

namespace anima_hip {

namespace {
thread_local std::string t_last_error;
}

bool fail(const std::string &msg)
{
    t_last_error = msg;
    return false;
}

bool hip_ok(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return true;
    return fail(std::string(what) + ": " + hipGetErrorString(e));
}

namespace {

// Failure injection for tests of the error path: while the environment
// variable ANIMA_HIP_FAIL_ALLOC is set to 1, every growth of a host-entry
// workspace buffer fails as an out-of-memory hipMalloc would.
bool injected_alloc_failure()
{
    const char *e = std::getenv("ANIMA_HIP_FAIL_ALLOC");
    return e && e[0] == '1' && e[1] == '\0';
}

// Grow-only device buffer.
struct DevBuf {
    void *p = nullptr;
    size_t cap = 0;
    bool reserve(size_t bytes, const char *what)
    {
        if (bytes <= cap)
            return true;
        release();
        const size_t want = std::max<size_t>(bytes, 256);
        if (injected_alloc_failure())
            return fail(std::string(what) + ": out of memory (injected by ANIMA_HIP_FAIL_ALLOC)");
        if (!hip_ok(hipMalloc(&p, want), what)) {
            p = nullptr;
            return false;
        }
        cap = want;
        return true;
    }
    void release()
    {
        if (p)
            (void)hipFree(p);
        p = nullptr;
        cap = 0;
    }
};

// Timing hook of the host-pointer entries: events on the runtime stream at
// the first upload, after the last upload, before the first download and
// after the last download of a call.
struct CallTimer {
    hipEvent_t ev[4] = {nullptr, nullptr, nullptr, nullptr};
    bool up = false, down = false;
    float kernel_ms = -1.0f, total_ms = -1.0f;
};

// Host memcpy split over the caller and a few parked worker threads.  One
// thread copies pageable memory into pinned memory at ~30 GB/s on an MI355X
// host, four at ~73 GB/s, above the ~57 GB/s of the host link's DMA.  A
// grouped call (run_groups) feeds both directions' copies through the pool,
// and a fresh output array takes its page faults in the copy-out: six
// threads ran such calls 3-17 % faster than four, eight no faster than six.
class CopyPool {
  public:
    static CopyPool &get()
    {
        // Never destroyed: the workers stay parked until the process ends.
        static CopyPool *pool = new CopyPool();
        return *pool;
    }

    void copy(void *dst, const void *src, size_t n)
    {
        std::lock_guard<std::mutex> one_job(call_mu_);
        // Threads do not survive fork(): a child copies on its own thread.
        if (n < kMinSplit || workers_.empty() || getpid() != pid_) {
            std::memcpy(dst, src, n);
            return;
        }
        const int parts = int(workers_.size()) + 1;
        {
            std::lock_guard<std::mutex> l(mu_);
            dst_ = static_cast<char *>(dst);
            src_ = static_cast<const char *>(src);
            n_ = n;
            parts_ = parts;
            pending_ = parts - 1;
            ++gen_;
        }
        work_cv_.notify_all();
        run_part(0, static_cast<char *>(dst), static_cast<const char *>(src), n, parts);
        std::unique_lock<std::mutex> l(mu_);
        done_cv_.wait(l, [&] { return pending_ == 0; });
    }

  private:
    static constexpr size_t kMinSplit = size_t(1) << 20;

    CopyPool() : pid_(getpid())
    {
        const unsigned hw = std::thread::hardware_concurrency();
        const int n = int(std::min(6u, std::max(1u, hw / 2)));
        for (int i = 1; i < n; ++i)
            workers_.emplace_back([this, i] { worker(i); });
        for (std::thread &t : workers_)
            t.detach();
    }

    // Part i of n of a copy: 64-byte aligned splits.
    static void run_part(int i, char *dst, const char *src, size_t n, int parts)
    {
        const size_t step = (n / parts + 63) & ~size_t(63);
        const size_t lo = std::min(n, step * size_t(i));
        const size_t hi = i == parts - 1 ? n : std::min(n, lo + step);
        if (hi > lo)
            std::memcpy(dst + lo, src + lo, hi - lo);
    }

    void worker(int id)
    {
        uint64_t seen = 0;
        for (;;) {
            std::unique_lock<std::mutex> l(mu_);
            work_cv_.wait(l, [&] { return gen_ != seen; });
            seen = gen_;
            char *dst = dst_;
            const char *src = src_;
            const size_t n = n_;
            const int parts = parts_;
            l.unlock();
            run_part(id, dst, src, n, parts);
            l.lock();
            if (--pending_ == 0)
                done_cv_.notify_one();
        }
    }

    std::mutex call_mu_, mu_;
    std::condition_variable work_cv_, done_cv_;
    std::vector<std::thread> workers_;
    const pid_t pid_;
    char *dst_ = nullptr;
    const char *src_ = nullptr;
    size_t n_ = 0;
    int parts_ = 1, pending_ = 0;
    uint64_t gen_ = 0;
};

// Pinned staging of the host-pointer entries' copies.  The host arrays are
// pageable (numpy), which HIP copies through its own staging at 30 GB/s (H2D)
// and 18 GB/s (D2H) on an MI355X host.  Here each 16 MiB chunk is copied by
// CopyPool into one of kSlots pinned buffers while the previous chunks' DMAs
// run; an event per slot says when the slot may be reused.
struct Staging {
    static constexpr int kSlots = 4;
    static constexpr size_t kChunk = size_t(16) << 20;
    static constexpr size_t kMinStaged = size_t(4) << 20;  // smaller copies go direct
    char *slot[kSlots] = {};
    hipEvent_t done[kSlots] = {};
    bool busy[kSlots] = {};
    int next = 0;
    bool unavailable = false;  // pinned memory could not be had: direct copies

    bool ensure()
    {
        if (slot[0] || unavailable)
            return !unavailable;
        for (int s = 0; s < kSlots; ++s) {
            void *p = nullptr;
            if (hipHostMalloc(&p, kChunk, hipHostMallocDefault) != hipSuccess ||
                hipEventCreateWithFlags(&done[s], hipEventDisableTiming) != hipSuccess) {
                if (p)
                    (void)hipHostFree(p);
                release();
                unavailable = true;
                return false;
            }
            slot[s] = static_cast<char *>(p);
        }
        return true;
    }

    // Waits for the last DMA that used slot s.
    bool drain(int s)
    {
        if (!busy[s])
            return true;
        busy[s] = false;
        return hip_ok(hipEventSynchronize(done[s]), "staging wait");
    }

    bool issue(int s, void *dst, const void *src, size_t n, hipMemcpyKind kind, hipStream_t st)
    {
        if (!hip_ok(hipMemcpyAsync(dst, src, n, kind, st), "staged copy") ||
            !hip_ok(hipEventRecord(done[s], st), "hipEventRecord"))
            return false;
        busy[s] = true;
        return true;
    }

    bool h2d(char *dst, const char *src, size_t n, hipStream_t st)
    {
        for (size_t off = 0; off < n; off += kChunk) {
            const int s = next;
            next = (next + 1) % kSlots;
            const size_t len = std::min(kChunk, n - off);
            if (!drain(s))
                return false;
            CopyPool::get().copy(slot[s], src + off, len);
            if (!issue(s, dst + off, slot[s], len, hipMemcpyHostToDevice, st))
                return false;
        }
        return true;
    }

    // Returns once dst holds the data: chunk i is copied out of its slot
    // while the DMAs of chunks i+1 .. i+kSlots-1 run.
    bool d2h(char *dst, const char *src, size_t n, hipStream_t st)
    {
        const size_t chunks = (n + kChunk - 1) / kChunk;
        const int base = next;
        auto slot_of = [&](size_t i) { return int((base + i) % kSlots); };
        auto len_of = [&](size_t i) { return std::min(kChunk, n - i * kChunk); };
        auto start = [&](size_t i) {
            const int s = slot_of(i);
            return drain(s) &&
                   issue(s, slot[s], src + i * kChunk, len_of(i), hipMemcpyDeviceToHost, st);
        };
        for (size_t i = 0; i < std::min<size_t>(kSlots, chunks); ++i)
            if (!start(i))
                return false;
        for (size_t i = 0; i < chunks; ++i) {
            const int s = slot_of(i);
            if (!drain(s))
                return false;
            CopyPool::get().copy(dst + i * kChunk, slot[s], len_of(i));
            if (i + kSlots < chunks && !start(i + kSlots))
                return false;
        }
        next = slot_of(chunks);
        return true;
    }

    void release()
    {
        for (int s = 0; s < kSlots; ++s) {
            if (busy[s])
                (void)hipEventSynchronize(done[s]);
            if (slot[s])
                (void)hipHostFree(slot[s]);
            if (done[s])
                (void)hipEventDestroy(done[s]);
            slot[s] = nullptr;
            done[s] = nullptr;
            busy[s] = false;
        }
        next = 0;
    }
};

struct Runtime {
    std::recursive_mutex mu;
    bool ready = false;      // device + stream exist
    bool user_init = false;  // anima_rt_init() succeeded (gates rmsnorm / math sdpa)
    int device = 0;
    hipStream_t stream = nullptr;
    DevBuf q, k, v, o, w0, w1, fr, q2, k2, v2, scratch;
    CallTimer timer;
    Staging staging;   // uploads, and the single-stream calls' downloads
    Staging dstaging;  // downloads of a grouped call (run_groups)
    // Compute and download streams and the per-group events of a grouped
    // host-pointer call.
    static constexpr int kMaxGroups = 4;
    hipStream_t cstream = nullptr, dstream = nullptr;
    hipEvent_t up_ev[kMaxGroups] = {}, done_ev[kMaxGroups] = {};
};

Runtime &rt()
{
    static Runtime r;
    return r;
}

bool ensure_ready(Runtime &r)
{
    if (r.ready)
        return true;
    int n = 0;
    if (!hip_ok(hipGetDeviceCount(&n), "hipGetDeviceCount"))
        return false;
    if (n <= 0)
        return fail("no HIP device visible");
    if (!hip_ok(hipGetDevice(&r.device), "hipGetDevice"))
        return false;
    if (!hip_ok(hipStreamCreateWithFlags(&r.stream, hipStreamNonBlocking), "hipStreamCreate"))
        return false;
    for (hipEvent_t &e : r.timer.ev)
        if (!hip_ok(hipEventCreate(&e), "hipEventCreate"))
            return false;
    r.ready = true;
    return true;
}

// The compute and download streams (default priority, like every stream
// here) and the events of a grouped host-pointer call, created at first use.
bool ensure_pipeline(Runtime &r)
{
    for (hipStream_t *s : {&r.cstream, &r.dstream})
        if (!*s && !hip_ok(hipStreamCreateWithFlags(s, hipStreamNonBlocking), "hipStreamCreate"))
            return false;
    for (int g = 0; g < Runtime::kMaxGroups; ++g)
        for (hipEvent_t *e : {&r.up_ev[g], &r.done_ev[g]})
            if (!*e && !hip_ok(hipEventCreateWithFlags(e, hipEventDisableTiming), "hipEventCreate"))
                return false;
    return true;
}

// Drains the runtime streams when a host-pointer call returns early after
// enqueuing work, so that no kernel or copy of a failed call still reads or
// writes the shared workspace or staging when the next call uses them.
struct DrainOnError {
    Runtime &r;
    bool done = false;
    ~DrainOnError()
    {
        if (done || !r.stream)
            return;
        for (hipStream_t s : {r.stream, r.cstream, r.dstream})
            if (s)
                (void)hipStreamSynchronize(s);
    }
};

// Context check for the device-pointer entries: the mutex is held only to
// create the context once, never across the launches themselves.
bool ready_for_device_call()
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    return ensure_ready(r);
}

}  // namespace

bool device_ready() { return ready_for_device_call(); }

namespace {

// Device entry points run on the caller's stream; NULL is HIP's default
// (null) stream, as in other HIP libraries.
hipStream_t pick_stream(void *s) { return static_cast<hipStream_t>(s); }

Strides contiguous(int H, int S, int D)
{
    return Strides{int64_t(H) * S * D, int64_t(S) * D, int64_t(D)};
}

Strides from_array(const int64_t *a, int H, int S, int D)
{
    return a ? Strides{a[0], a[1], a[2]} : contiguous(H, S, D);
}

bool check_dims(int B, int H, int S_q, int S_kv, int D)
{
    if (B < 0 || H < 0 || S_q < 0 || S_kv < 0 || D < 0)
        return fail("negative dimension");
    return true;
}

size_t f32_bytes(int64_t n) { return size_t(n) * sizeof(float); }

// Timing marks on the runtime stream (no-ops on other streams).
void mark(hipStream_t st, int i)
{
    Runtime &r = rt();
    if (st == r.stream && r.timer.ev[i])
        (void)hipEventRecord(r.timer.ev[i], st);
}

bool h2d(void *dst, const void *src, size_t n, hipStream_t st)
{
    if (n == 0)
        return true;
    Runtime &r = rt();
    if (!r.timer.up && st == r.stream) {
        mark(st, 0);
        r.timer.up = true;
    }
    const bool ok = n >= Staging::kMinStaged && r.staging.ensure()
                        ? r.staging.h2d(static_cast<char *>(dst), static_cast<const char *>(src),
                                        n, st)
                        : hip_ok(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, st),
                                 "H2D copy");
    mark(st, 1);
    return ok;
}

bool d2h(void *dst, const void *src, size_t n, hipStream_t st)
{
    if (n == 0)
        return true;
    Runtime &r = rt();
    if (!r.timer.down && st == r.stream) {
        mark(st, 2);
        r.timer.down = true;
    }
    const bool ok = n >= Staging::kMinStaged && r.staging.ensure()
                        ? r.staging.d2h(static_cast<char *>(dst), static_cast<const char *>(src),
                                        n, st)
                        : hip_ok(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, st),
                                 "D2H copy");
    mark(st, 3);
    return ok;
}

bool sync(hipStream_t st) { return hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize"); }

// Start of a timed host-pointer call.
void begin_call(Runtime &r)
{
    r.timer.up = r.timer.down = false;
}

// End of a timed host-pointer call: synchronise, then keep the device time
// between the uploads and the downloads (kernels) and from the first upload
// to the last download (whole call).
bool finish_call(Runtime &r)
{
    if (!sync(r.stream))
        return false;
    CallTimer &t = r.timer;
    float k = 0.0f, w = 0.0f;
    if (t.up && t.down && hipEventElapsedTime(&k, t.ev[1], t.ev[2]) == hipSuccess &&
        hipEventElapsedTime(&w, t.ev[0], t.ev[3]) == hipSuccess) {
        t.kernel_ms = k;
        t.total_ms = w;
    }
    t.up = t.down = false;
    return true;
}

// One host <-> device copy of a grouped host-pointer call.
struct Piece {
    char *dst;
    const char *src;
    size_t n;
};
typedef std::vector<Piece> Pieces[Runtime::kMaxGroups];

// A host-pointer call as G groups (1 <= G <= kMaxGroups): group g's uploads
// on the runtime stream, its kernels (launch(g, stream)) on the compute
// stream once they have landed, its downloads on the download stream once
// the kernels end.  Pieces of kMinStaged bytes or more move in chunks through
// pinned slots, one ring per direction.  The calling thread copies a landed
// download chunk out whenever one is ready and stages the next upload chunk
// otherwise, so the later groups' uploads and the earlier groups' downloads
// use the host link's two directions at the same time.  With G == 1 all of it
// runs on the runtime stream.  Returns once every download has reached host
// memory; the call's timing marks are those of finish_call (end of the last
// upload to the start of the last group's downloads, first upload to last
// download).
bool run_groups(Runtime &r, int G, const Pieces &up, const Pieces &down,
                const std::function<bool(int, hipStream_t)> &launch)
{
    if (G < 1 || G > Runtime::kMaxGroups)
        return fail("internal: group count out of range");
    const hipStream_t st = r.stream;
    if (G > 1 && !ensure_pipeline(r))
        return false;
    const hipStream_t cs = G > 1 ? r.cstream : st, ds = G > 1 ? r.dstream : st;
    Staging &us = r.staging, &dsg = r.dstaging;
    const bool staged = us.ensure() && dsg.ensure();

    struct Chunk {
        int g;
        char *dst;
        const char *src;
        size_t n;
        bool staged;
    };
    std::vector<Chunk> uc, dc;
    for (int g = 0; g < G; ++g) {
        for (int dir = 0; dir < 2; ++dir)
            for (const Piece &p : (dir ? down : up)[g]) {
                std::vector<Chunk> &out = dir ? dc : uc;
                if (p.n == 0)
                    continue;
                if (!staged || p.n < Staging::kMinStaged) {
                    out.push_back({g, p.dst, p.src, p.n, false});
                    continue;
                }
                for (size_t off = 0; off < p.n; off += Staging::kChunk)
                    out.push_back(
                        {g, p.dst + off, p.src + off, std::min(Staging::kChunk, p.n - off), true});
            }
    }

    CallTimer &t = r.timer;
    auto rec = [&](int i, hipStream_t s) {
        return !t.ev[i] || hip_ok(hipEventRecord(t.ev[i], s), "hipEventRecord");
    };
    size_t ui = 0;  // next upload chunk
    int uslot = 0;  // pinned upload slot of the next staged upload chunk
    int launched = 0;
    auto launch_group = [&](int g) {
        if (G > 1 && !(hip_ok(hipEventRecord(r.up_ev[g], st), "hipEventRecord") &&
                       hip_ok(hipStreamWaitEvent(cs, r.up_ev[g], 0), "hipStreamWaitEvent")))
            return false;
        if (!launch(g, cs))
            return false;
        return G == 1 || (hip_ok(hipEventRecord(r.done_ev[g], cs), "hipEventRecord") &&
                          hip_ok(hipStreamWaitEvent(ds, r.done_ev[g], 0), "hipStreamWaitEvent"));
    };
    // Launches every group whose uploads have all been issued (uc is ordered
    // by group).
    auto launch_ready = [&] {
        while (launched < G && (ui == uc.size() || uc[ui].g > launched))
            if (!launch_group(launched++))
                return false;
        return true;
    };
    auto upload_one = [&] {
        const Chunk &c = uc[ui];
        if (ui == 0 && !t.up) {  // the call's first upload
            if (!rec(0, st))
                return false;
            t.up = true;
        }
        if (c.staged) {
            const int s = uslot;
            uslot = (uslot + 1) % Staging::kSlots;
            if (!us.drain(s))
                return false;
            CopyPool::get().copy(us.slot[s], c.src, c.n);
            if (!us.issue(s, c.dst, us.slot[s], c.n, hipMemcpyHostToDevice, st))
                return false;
        } else if (!hip_ok(hipMemcpyAsync(c.dst, c.src, c.n, hipMemcpyHostToDevice, st),
                           "H2D copy")) {
            return false;
        }
        ++ui;
        return ui < uc.size() || rec(1, st);
    };

    // Downloads: chunks [dd, di) are enqueued; the staged ones among them sit
    // in slots dslot[], oldest first.
    size_t di = 0, dd = 0;
    int dnext = 0;  // pinned download slot of the next staged download chunk
    std::vector<int> dslot;
    size_t dslot_head = 0;
    const size_t last_group_first =
        std::find_if(dc.begin(), dc.end(), [&](const Chunk &c) { return c.g == G - 1; }) -
        dc.begin();
    auto enqueue_downloads = [&] {
        while (di < dc.size() && dc[di].g < launched &&
               (!dc[di].staged || dslot.size() - dslot_head < size_t(Staging::kSlots))) {
            const Chunk &c = dc[di];
            if (di == last_group_first) {
                if (!rec(2, ds))
                    return false;
                t.down = true;
            }
            if (c.staged) {
                const int s = dnext;
                dnext = (dnext + 1) % Staging::kSlots;
                if (!dsg.drain(s) ||
                    !dsg.issue(s, dsg.slot[s], c.src, c.n, hipMemcpyDeviceToHost, ds))
                    return false;
                dslot.push_back(s);
            } else if (!hip_ok(hipMemcpyAsync(c.dst, c.src, c.n, hipMemcpyDeviceToHost, ds),
                               "D2H copy")) {
                return false;
            }
            ++di;
            if (di == dc.size() && !rec(3, ds))
                return false;
        }
        return true;
    };
    // Oldest enqueued staged download: landed (or, with wait, once it lands)
    // -> copied out of its slot.  Unstaged chunks before it need no copy-out.
    auto finish_download = [&](bool wait, bool &did) {
        did = false;
        while (dd < di && !dc[dd].staged)
            ++dd;
        if (dd == di)
            return true;
        const int s = dslot[dslot_head];
        if (!wait) {
            const hipError_t q = hipEventQuery(dsg.done[s]);
            if (q == hipErrorNotReady)
                return true;
            if (!hip_ok(q, "staging query"))
                return false;
        }
        if (!dsg.drain(s))
            return false;
        CopyPool::get().copy(dc[dd].dst, dsg.slot[s], dc[dd].n);
        ++dslot_head;
        ++dd;
        did = true;
        return true;
    };

    if (!launch_ready())
        return false;
    while (launched < G || ui < uc.size() || dd < dc.size()) {
        if (!enqueue_downloads())
            return false;
        bool did = false;
        if (!finish_download(false, did))
            return false;
        if (did)
            continue;
        if (ui < uc.size()) {
            if (!upload_one() || !launch_ready())
                return false;
            continue;
        }
        // Every group is launched and every download that fits is enqueued:
        // wait for the oldest staged one (unstaged ones land with the stream).
        if (!launch_ready() || !enqueue_downloads() || !finish_download(true, did))
            return false;
    }
    return sync(ds);
}

// Kernels of the host-pointer SDPA for heads [h0, h0 + nh) of the uploaded
// [BH, S, D] f32 workspace arrays, on stream st: the f32 flash kernel, or the
// bf16 / f32x3 operand passes (Q and K rows, packed V^T) and their kernel.
bool sdpa_heads(Runtime &r, int64_t h0, int nh, int S_q, int S_kv, int D, float scale, bool causal,
                int mode, hipStream_t st)
{
    const bool bf16 = mode == ANIMA_HIP_BF16, x3 = mode == ANIMA_HIP_F32X3;
    const size_t part_bytes = flash_plan(nh, S_q, S_kv, D).bytes;
    FlashProblem p;
    p.q = static_cast<const float *>(r.q.p) + h0 * S_q * D;
    p.k = static_cast<const float *>(r.k.p) + h0 * S_kv * D;
    p.v = static_cast<const float *>(r.v.p) + h0 * S_kv * D;
    p.o = static_cast<float *>(r.o.p) + h0 * S_q * D;
    p.qs = p.os = contiguous(nh, S_q, D);
    p.ks = p.vs = contiguous(nh, S_kv, D);
    p.B = 1;
    p.H = nh;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = causal;
    if (!bf16 && !x3)
        return launch_flash_f32(p, st, r.scratch.p, part_bytes);
    // bf16 copies of Q and K (row kernel without norm/RoPE; rows of [hi | lo]
    // terms in the f32x3 mode) and packed V^T (hi rows, then lo rows).
    const int64_t sp = vt_padded_len(S_kv), w = x3 ? 2 : 1;
    RowProblem c;
    c.x = static_cast<const float *>(p.q);
    c.out = static_cast<uint16_t *>(r.q2.p) + h0 * S_q * D * w;
    c.w = nullptr;
    c.freqs = nullptr;
    c.xs = Strides{0, int64_t(S_q) * D, int64_t(D)};
    c.os = Strides{0, int64_t(S_q) * D * w, int64_t(D) * w};
    c.B = 1;
    c.S = S_q;
    c.H = nh;
    c.D = D;
    c.eps = 0.0f;
    c.norm = false;
    c.out_bf16 = true;
    c.lo_off = x3 ? D : 0;
    RowProblem ck = c;
    ck.x = static_cast<const float *>(p.k);
    ck.out = static_cast<uint16_t *>(r.k2.p) + h0 * S_kv * D * w;
    ck.xs = Strides{0, int64_t(S_kv) * D, int64_t(D)};
    ck.os = Strides{0, int64_t(S_kv) * D * w, int64_t(D) * w};
    ck.S = S_kv;
    const Strides vts{0, w * D * sp, sp};
    const float *vf = static_cast<const float *>(p.v);
    uint16_t *vt = static_cast<uint16_t *>(r.v2.p) + h0 * w * D * sp;
    if (!launch_rows(c, st) || !launch_rows(ck, st) ||
        !(x3 ? launch_vt_pack_terms(vf, p.vs, vt, vts, 1, nh, S_kv, D, st)
             : launch_vt_pack(vf, p.vs, vt, vts, 1, nh, S_kv, D, st)))
        return false;
    p.q = c.out;
    p.k = ck.out;
    p.v = vt;
    p.qs = c.os;
    p.ks = ck.os;
    p.vs = vts;
    return x3 ? launch_flash_x3(p, st, r.scratch.p, part_bytes)
              : launch_flash_bf16(p, st, r.scratch.p, part_bytes);
}

// Head groups of a host-pointer SDPA: the most groups (4 or 2) that still
// fill the GPU each (flash_plan keeps 8-wave workgroups and no key split)
// when the copies are large, else one.  Group g+1 uploads while group g
// computes, and group g's output comes back while later groups upload.
int sdpa_groups(int BH, int S_q, int S_kv, int D)
{
    const int64_t bytes = int64_t(BH) * (2 * int64_t(S_q) + 2 * int64_t(S_kv)) * D * 4;
    if (bytes < (int64_t(64) << 20))
        return 1;
    for (int G = Runtime::kMaxGroups; G > 1; G /= 2) {
        if (BH % G != 0)
            continue;
        const FlashPlan part = flash_plan(BH / G, S_q, S_kv, D);
        if (part.waves == 8 && part.splits == 1)
            return G;
    }
    return 1;
}

// Shared body of the host-pointer SDPA entries ([BH, S, D] f32 host arrays).
bool host_sdpa(const float *Q, const float *K, const float *V, float *out, int BH, int S_q,
               int S_kv, int D, float scale, bool causal, int mode)
{
    const bool bf16 = mode == ANIMA_HIP_BF16, x3 = mode == ANIMA_HIP_F32X3;
    if (!check_dims(1, BH, S_q, S_kv, D))
        return false;
    const int64_t nq = int64_t(BH) * S_q * D, nk = int64_t(BH) * S_kv * D;
    if (nq == 0)
        return true;
    if (!Q || !out || (nk > 0 && (!K || !V)))
        return fail("sdpa: null pointer");
    if ((bf16 || x3) && D != 128)
        return fail(std::string("sdpa: the ") + (bf16 ? "bf16" : "f32x3") + " mode needs D == 128");
    Runtime &r = rt();
    begin_call(r);
    const int G = sdpa_groups(BH, S_q, S_kv, D), nh = BH / G;
    if (!r.q.reserve(f32_bytes(nq), "workspace Q") || !r.o.reserve(f32_bytes(nq), "workspace O") ||
        !r.k.reserve(f32_bytes(nk), "workspace K") || !r.v.reserve(f32_bytes(nk), "workspace V") ||
        !r.scratch.reserve(flash_plan(nh, S_q, S_kv, D).bytes, "workspace split-KV partials"))
        return false;
    if (bf16 || x3) {
        const int64_t w = x3 ? 2 : 1;
        if (!r.q2.reserve(nq * 2 * w, "workspace q bf16") ||
            !r.k2.reserve(nk * 2 * w, "workspace k bf16") ||
            !r.v2.reserve(size_t(BH) * w * D * vt_padded_len(S_kv) * 2, "workspace v^T"))
            return false;
    }
    DrainOnError drain{r};
    const int64_t gq = int64_t(nh) * S_q * D, gk = int64_t(nh) * S_kv * D;  // elements per group
    const auto dev = [](DevBuf &b, int64_t off) { return static_cast<char *>(b.p) + f32_bytes(off); };
    const auto host = [](const float *p, int64_t off) {
        return reinterpret_cast<const char *>(p) + f32_bytes(off);
    };
    Pieces up, down;
    for (int g = 0; g < G; ++g) {
        up[g] = {{dev(r.q, g * gq), host(Q, g * gq), f32_bytes(gq)},
                 {dev(r.k, g * gk), host(K, g * gk), f32_bytes(gk)},
                 {dev(r.v, g * gk), host(V, g * gk), f32_bytes(gk)}};
        down[g] = {{reinterpret_cast<char *>(out) + f32_bytes(g * gq), dev(r.o, g * gq),
                    f32_bytes(gq)}};
    }
    if (!run_groups(r, G, up, down, [&](int g, hipStream_t s) {
            return sdpa_heads(r, int64_t(g) * nh, nh, S_q, S_kv, D, scale, causal, mode, s);
        }))
        return false;
    drain.done = true;
    return finish_call(r);
}

// Host -> device copy of an optional per-head weight or RoPE table.
bool upload_optional(DevBuf &buf, const float *src, size_t n, const char *what, hipStream_t st,
                     const float *&dev)
{
    dev = nullptr;
    if (!src)
        return true;
    if (!buf.reserve(f32_bytes(n), what) || !h2d(buf.p, src, f32_bytes(n), st))
        return false;
    dev = static_cast<const float *>(buf.p);
    return true;
}

bool host_gemm(const float *A, const void *W, bool w_bf16, float *C, int M, int N, int K)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    if (M < 0 || N < 0 || K < 0)
        return fail("gemm: negative dimension");
    if (int64_t(M) * N == 0)
        return true;
    if (!C || (K > 0 && (!A || !W)))
        return fail("gemm: null pointer");
    const hipStream_t st = r.stream;
    begin_call(r);
    const size_t wbytes = size_t(N) * K * (w_bf16 ? 2 : 4);
    if (!r.q.reserve(f32_bytes(int64_t(M) * K), "workspace A") ||
        !r.k.reserve(wbytes, "workspace W") || !r.o.reserve(f32_bytes(int64_t(M) * N), "workspace C"))
        return false;
    if (!h2d(r.q.p, A, f32_bytes(int64_t(M) * K), st) || !h2d(r.k.p, W, wbytes, st))
        return false;
    // bf16 weights: bf16 MFMA with A as exact hi + lo terms; f32 weights: f32 MFMA.
    const size_t sb = w_bf16 ? linear_scratch_bytes(M, K, true) : 0;
    if (!r.scratch.reserve(sb, "workspace linear"))
        return false;
    const bool ok =
        w_bf16 ? launch_linear(static_cast<const float *>(r.q.p), K,
                               static_cast<const uint16_t *>(r.k.p), K,
                               static_cast<float *>(r.o.p), N, M, N, K, true, r.scratch.p, sb, st)
               : launch_gemm(static_cast<const float *>(r.q.p), K, r.k.p, false, K,
                             static_cast<float *>(r.o.p), N, M, N, K, st);
    if (!ok || !d2h(C, r.o.p, f32_bytes(int64_t(M) * N), st))
        return false;
    return finish_call(r);
}

}  // namespace
}  // namespace anima_hip

using namespace anima_hip;

// Device-resident K/V of one text context (see anima_hip_ctx_kv_create).
struct anima_hip_ctx_kv {
    int mode = ANIMA_HIP_F32;
    int Bc = 0, S_kv = 0, H = 0, D = 0;
    int device = 0;
    void *k = nullptr;  // prepared K (layout per mode, see AttnInputs)
    void *v = nullptr;  // prepared V (f32 rows or packed bf16 / term V^T)
};

namespace {

// The attention arithmetic of a public mode value; false with the reason for
// an unknown mode, or a head dim other than 128 in the bf16 / f32x3 modes.
bool attn_mode_of(int mode, int D, const char *who, AttnMode &out)
{
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_BF16 && mode != ANIMA_HIP_F32X3)
        return fail(std::string(who) + ": unknown mode " + std::to_string(mode));
    if (mode != ANIMA_HIP_F32 && D != 128)
        return fail(std::string(who) + ": the bf16 and f32x3 modes need D == 128");
    out = AttnMode(mode);
    return true;
}

// Mode of a size query (unknown modes size as f32; the call itself rejects them).
AttnMode size_mode(int mode)
{
    return mode == ANIMA_HIP_BF16 || mode == ANIMA_HIP_F32X3 ? AttnMode(mode) : kAttnF32;
}

}  // namespace

extern "C" {

bool anima_rt_init(void)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    r.user_init = true;
    return true;
}

void anima_rt_destroy(void)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!r.ready)
        return;
    for (hipStream_t s : {r.stream, r.cstream, r.dstream})
        if (s)
            (void)hipStreamSynchronize(s);
    for (DevBuf *b : {&r.q, &r.k, &r.v, &r.o, &r.w0, &r.w1, &r.fr, &r.q2, &r.k2, &r.v2, &r.scratch})
        b->release();
    r.staging.release();
    r.dstaging.release();
    std::vector<hipEvent_t *> evs = {&r.timer.ev[0], &r.timer.ev[1], &r.timer.ev[2], &r.timer.ev[3]};
    for (int g = 0; g < Runtime::kMaxGroups; ++g) {
        evs.push_back(&r.up_ev[g]);
        evs.push_back(&r.done_ev[g]);
    }
    for (hipEvent_t *e : evs) {
        if (*e)
            (void)hipEventDestroy(*e);
        *e = nullptr;
    }
    for (hipStream_t *s : {&r.cstream, &r.dstream}) {
        if (*s)
            (void)hipStreamDestroy(*s);
        *s = nullptr;
    }
    (void)hipStreamDestroy(r.stream);
    r.stream = nullptr;
    r.ready = false;
    r.user_init = false;
}

bool anima_rt_run_sdpa_flash(const float *Q, const float *K, const float *V, float *out, int BH,
                             int S_q, int S_kv, int D, float scale, bool is_causal)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    return host_sdpa(Q, K, V, out, BH, S_q, S_kv, D, scale, is_causal, ANIMA_HIP_F32);
}

bool anima_rt_run_sdpa(const float *Q, const float *K, const float *V, float *out, int BH,
                       int S_q, int S_kv, int D, float scale, bool is_causal)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!r.user_init)
        return fail("anima_rt_run_sdpa: anima_rt_init() has not been called");
    // The reference multiplies both Q and K by `scale`: softmax(scale^2 QK^T)V.
    return host_sdpa(Q, K, V, out, BH, S_q, S_kv, D, scale * scale, is_causal, ANIMA_HIP_F32);
}

bool anima_rt_run_rmsnorm(const float *x, const float *w, float *out, int m, int d, float eps)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!r.user_init)
        return fail("anima_rt_run_rmsnorm: anima_rt_init() has not been called");
    if (m < 0 || d < 0)
        return fail("rmsnorm: negative dimension");
    const int64_t n = int64_t(m) * d;
    if (n == 0)
        return true;
    if (!x || !out)
        return fail("rmsnorm: null pointer");
    const hipStream_t st = r.stream;
    begin_call(r);
    if (!r.q.reserve(f32_bytes(n), "workspace x") || !r.o.reserve(f32_bytes(n), "workspace y"))
        return false;
    const float *wd = nullptr;
    if (!h2d(r.q.p, x, f32_bytes(n), st) || !upload_optional(r.w0, w, d, "workspace w", st, wd))
        return false;
    RowProblem p;
    p.x = static_cast<const float *>(r.q.p);
    p.out = r.o.p;
    p.w = wd;
    p.freqs = nullptr;
    p.xs = p.os = Strides{0, 0, int64_t(d)};
    p.B = 1;
    p.S = m;
    p.H = 1;
    p.D = d;
    p.eps = eps;
    p.norm = true;
    p.out_bf16 = false;
    if (!launch_rows(p, st) || !d2h(out, r.o.p, f32_bytes(n), st))
        return false;
    return finish_call(r);
}

}  // extern "C"

namespace {

// Host-pointer form of a one-input, one-output operator over n floats: the
// input through the runtime's workspace, `run` on the device, the output
// back; synchronous like the reference.
template <typename Run>
bool host_unary(const char *what, const float *x, float *out, int64_t n, Run run)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!r.user_init)
        return fail(std::string("anima_rt_run_") + what + ": anima_rt_init() has not been called");
    if (n <= 0)
        return true;
    if (!x || !out)
        return fail(std::string(what) + ": null pointer");
    const hipStream_t st = r.stream;
    begin_call(r);
    if (!r.q.reserve(f32_bytes(n), "workspace x") || !r.o.reserve(f32_bytes(n), "workspace y") ||
        !h2d(r.q.p, x, f32_bytes(n), st) ||
        !run(static_cast<const float *>(r.q.p), static_cast<float *>(r.o.p), st) ||
        !d2h(out, r.o.p, f32_bytes(n), st))
        return false;
    return finish_call(r);
}

}  // namespace

extern "C" {

bool anima_rt_run_gelu(const float *x, float *out, int n)
{
    return host_unary("gelu", x, out, n, [&](const float *xd, float *yd, hipStream_t st) {
        return launch_gelu(xd, yd, n, st);
    });
}

bool anima_rt_run_silu(const float *x, float *out, int n)
{
    return host_unary("silu", x, out, n, [&](const float *xd, float *yd, hipStream_t st) {
        return launch_silu(xd, yd, n, st);
    });
}

bool anima_rt_run_layernorm(const float *x, float *out, int m, int d, float eps)
{
    const int64_t n = (m > 0 && d > 0) ? int64_t(m) * d : 0;
    return host_unary("layernorm", x, out, n, [&](const float *xd, float *yd, hipStream_t st) {
        return launch_layernorm_rows(xd, yd, m, d, eps, st);
    });
}

bool anima_rt_run_softmax(const float *x, float *out, int outer, int dim)
{
    const int64_t n = (outer > 0 && dim > 0) ? int64_t(outer) * dim : 0;
    return host_unary("softmax", x, out, n, [&](const float *xd, float *yd, hipStream_t st) {
        return launch_softmax_rows(xd, yd, outer, dim, st);
    });
}

bool anima_rt_run_bias_add(float *C, const float *bias, int M, int N)
{
    if (!bias || M <= 0 || N <= 0)
        return true;
    if (!C)
        return fail("bias_add: null pointer");
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    const int64_t n = int64_t(M) * N;
    const hipStream_t st = r.stream;
    begin_call(r);
    if (!r.o.reserve(f32_bytes(n), "workspace C") || !r.w0.reserve(f32_bytes(N), "workspace bias") ||
        !h2d(r.o.p, C, f32_bytes(n), st) || !h2d(r.w0.p, bias, f32_bytes(N), st) ||
        !launch_bias_add(static_cast<float *>(r.o.p), static_cast<const float *>(r.w0.p), M, N,
                         st) ||
        !d2h(C, r.o.p, f32_bytes(n), st))
        return false;
    return finish_call(r);
}

bool anima_rt_run_rope(const float *t, const float *freqs, float *out, int N, int S, int D)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    if (N < 0 || S < 0 || D < 0)
        return fail("rope: negative dimension");
    const int64_t n = int64_t(N) * S * D, nf = int64_t(S) * D * 2;
    if (n == 0)
        return true;
    if (!t || !freqs || !out)
        return fail("rope: null pointer");
    const hipStream_t st = r.stream;
    begin_call(r);
    if (!r.q.reserve(f32_bytes(n), "workspace t") || !r.o.reserve(f32_bytes(n), "workspace out") ||
        !r.fr.reserve(f32_bytes(nf), "workspace freqs"))
        return false;
    if (!h2d(r.q.p, t, f32_bytes(n), st) || !h2d(r.fr.p, freqs, f32_bytes(nf), st))
        return false;
    RowProblem p;
    p.x = static_cast<const float *>(r.q.p);
    p.out = r.o.p;
    p.w = nullptr;
    p.freqs = static_cast<const float *>(r.fr.p);
    p.xs = p.os = Strides{int64_t(S) * D, 0, int64_t(D)};
    p.B = N;
    p.S = S;
    p.H = 1;
    p.D = D;
    p.eps = 0.0f;
    p.norm = false;
    p.out_bf16 = false;
    if (!launch_rows(p, st) || !d2h(out, r.o.p, f32_bytes(n), st))
        return false;
    return finish_call(r);
}

bool anima_rt_run_gemm_fp32(const float *A, const float *B, float *C, int M, int N, int K)
{
    return host_gemm(A, B, false, C, M, N, K);
}

bool anima_rt_run_gemm_bf16(const float *A, const uint16_t *W, float *C, int M, int N, int K)
{
    return host_gemm(A, W, true, C, M, N, K);
}

bool anima_hip_sdpa(const float *Q, const float *K, const float *V, float *out, int BH, int S_q,
                    int S_kv, int D, float scale, bool is_causal, int mode)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_BF16 && mode != ANIMA_HIP_F32X3)
        return fail("anima_hip_sdpa: unknown mode " + std::to_string(mode));
    return host_sdpa(Q, K, V, out, BH, S_q, S_kv, D, scale, is_causal, mode);
}

const char *anima_hip_last_error(void) { return t_last_error.c_str(); }

int anima_hip_version(void) { return 100; }

bool anima_hip_flash_f32_dev(const float *q, const float *k, const float *v, float *o, int B,
                             int H, int S_q, int S_kv, int D, const int64_t *q_strides,
                             const int64_t *k_strides, const int64_t *v_strides,
                             const int64_t *o_strides, float scale, bool is_causal, void *stream)
{
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !v))))
        return fail("flash_f32_dev: null pointer");
    FlashProblem p;
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.qs = from_array(q_strides, H, S_q, D);
    p.ks = from_array(k_strides, H, S_kv, D);
    p.vs = from_array(v_strides, H, S_kv, D);
    p.os = from_array(o_strides, H, S_q, D);
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_f32(p, pick_stream(stream));
}

bool anima_hip_flash_bf16_dev(const uint16_t *q, const uint16_t *k, const uint16_t *vt, float *o,
                              int B, int H, int S_q, int S_kv, int D, const int64_t *q_strides,
                              const int64_t *k_strides, const int64_t *vt_strides,
                              const int64_t *o_strides, float scale, bool is_causal, void *stream)
{
    // The kernel folds the scale into exp2's argument and takes the row max
    // on raw scores, which needs scale > 0 (NaN and infinities are refused).
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail("flash_bf16_dev: scale must be positive and finite");
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !vt))))
        return fail("flash_bf16_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    FlashProblem p;
    p.q = q;
    p.k = k;
    p.v = vt;
    p.o = o;
    p.qs = from_array(q_strides, H, S_q, D);
    p.ks = from_array(k_strides, H, S_kv, D);
    p.vs = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                      : Strides{int64_t(H) * D * sp, int64_t(D) * sp, sp};
    p.os = from_array(o_strides, H, S_q, D);
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_bf16(p, pick_stream(stream));
}

int64_t anima_hip_vt_padded_len(int S_kv) { return S_kv > 0 ? vt_padded_len(S_kv) : 0; }

bool anima_hip_pack_vt_dev(const float *v, uint16_t *vt, int B, int H, int S_kv, int D,
                           const int64_t *v_strides, const int64_t *vt_strides, void *stream)
{
    if (!ready_for_device_call() || !check_dims(B, H, S_kv, S_kv, D))
        return false;
    if (int64_t(B) * H * S_kv * D > 0 && (!v || !vt))
        return fail("pack_vt_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    const Strides ts = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                                  : Strides{int64_t(H) * D * sp, int64_t(D) * sp, sp};
    if (ts.s != sp)
        return fail("pack_vt_dev: V^T row stride must equal the padded key count");
    return launch_vt_pack(v, from_array(v_strides, H, S_kv, D), vt, ts, B, H, S_kv, D,
                          pick_stream(stream));
}

bool anima_hip_flash_x3_dev(const uint16_t *q, const uint16_t *k, const uint16_t *vt, float *o,
                            int B, int H, int S_q, int S_kv, int D, const int64_t *q_strides,
                            const int64_t *k_strides, const int64_t *vt_strides,
                            const int64_t *o_strides, float scale, bool is_causal, void *stream)
{
    // The kernel folds the scale into exp2's argument and takes the row max
    // on raw scores, which needs scale > 0 (NaN and infinities are refused).
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail("flash_x3_dev: scale must be positive and finite");
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !vt))))
        return fail("flash_x3_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    FlashProblem p;
    p.q = q;
    p.k = k;
    p.v = vt;
    p.o = o;
    // Default strides: rows of 2*D terms, [B, H, S, 2D] contiguous.
    p.qs = q_strides ? Strides{q_strides[0], q_strides[1], q_strides[2]}
                     : Strides{int64_t(H) * S_q * 2 * D, int64_t(S_q) * 2 * D, 2 * int64_t(D)};
    p.ks = k_strides ? Strides{k_strides[0], k_strides[1], k_strides[2]}
                     : Strides{int64_t(H) * S_kv * 2 * D, int64_t(S_kv) * 2 * D, 2 * int64_t(D)};
    p.vs = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                      : Strides{int64_t(H) * 2 * D * sp, 2 * int64_t(D) * sp, sp};
    p.os = from_array(o_strides, H, S_q, D);
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_x3(p, pick_stream(stream));
}

bool anima_hip_flash_f32_rawq_dev(const float *q, const float *q_norm_w, float eps,
                                  const float *k, const float *v, float *o, int B, int H, int S_q,
                                  int S_kv, int D, const int64_t *q_strides,
                                  const int64_t *k_strides, const int64_t *v_strides,
                                  const int64_t *o_strides, float scale, bool is_causal,
                                  void *stream)
{
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail("flash_f32_rawq_dev: scale must be positive and finite");
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !v))))
        return fail("flash_f32_rawq_dev: null pointer");
    FlashProblem p;
    p.q = nullptr;
    p.k = k;
    p.v = v;
    p.o = o;
    p.qs = Strides{0, 0, 0};
    p.ks = from_array(k_strides, H, S_kv, D);
    p.vs = from_array(v_strides, H, S_kv, D);
    p.os = from_array(o_strides, H, S_q, D);
    p.rq.x = q;
    p.rq.s = from_array(q_strides, H, S_q, D);
    p.rq.w = q_norm_w;
    p.rq.eps = eps;
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_f32(p, pick_stream(stream), nullptr, 0);
}

bool anima_hip_flash_x3_rawq_dev(const float *q, const float *q_norm_w, const float *freqs,
                                 float eps, const uint16_t *k, const uint16_t *vt, float *o,
                                 int B, int H, int S_q, int S_kv, int D,
                                 const int64_t *q_strides, const int64_t *k_strides,
                                 const int64_t *vt_strides, const int64_t *o_strides,
                                 float scale, bool is_causal, void *stream)
{
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail("flash_x3_rawq_dev: scale must be positive and finite");
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !vt))))
        return fail("flash_x3_rawq_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    FlashProblem p;
    p.q = nullptr;
    p.k = k;
    p.v = vt;
    p.o = o;
    p.qs = Strides{0, 0, 0};
    p.ks = k_strides ? Strides{k_strides[0], k_strides[1], k_strides[2]}
                     : Strides{int64_t(H) * S_kv * 2 * D, int64_t(S_kv) * 2 * D, 2 * int64_t(D)};
    p.vs = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                      : Strides{int64_t(H) * 2 * D * sp, 2 * int64_t(D) * sp, sp};
    p.os = from_array(o_strides, H, S_q, D);
    p.rq.x = q;
    p.rq.s = from_array(q_strides, H, S_q, D);
    p.rq.w = q_norm_w;
    p.rq.freqs = freqs;
    p.rq.eps = eps;
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_x3(p, pick_stream(stream));
}

bool anima_hip_flash_bf16_rawq_dev(const float *q, const float *q_norm_w, const float *freqs,
                                   float eps, const uint16_t *k, const uint16_t *vt, float *o,
                                   int B, int H, int S_q, int S_kv, int D,
                                   const int64_t *q_strides, const int64_t *k_strides,
                                   const int64_t *vt_strides, const int64_t *o_strides,
                                   float scale, bool is_causal, void *stream)
{
    if (!(scale > 0.0f) || !std::isfinite(scale))
        return fail("flash_bf16_rawq_dev: scale must be positive and finite");
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    if (int64_t(B) * H * S_q * D > 0 && (!q || !o || (S_kv > 0 && (!k || !vt))))
        return fail("flash_bf16_rawq_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    FlashProblem p;
    p.q = nullptr;
    p.k = k;
    p.v = vt;
    p.o = o;
    p.qs = Strides{0, 0, 0};
    p.ks = from_array(k_strides, H, S_kv, D);
    p.vs = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                      : Strides{int64_t(H) * D * sp, int64_t(D) * sp, sp};
    p.os = from_array(o_strides, H, S_q, D);
    p.rq.x = q;
    p.rq.s = from_array(q_strides, H, S_q, D);
    p.rq.w = q_norm_w;
    p.rq.freqs = freqs;
    p.rq.eps = eps;
    p.B = B;
    p.H = H;
    p.S_q = S_q;
    p.S_kv = S_kv;
    p.D = D;
    p.scale = scale;
    p.causal = is_causal;
    return launch_flash_bf16(p, pick_stream(stream));
}

bool anima_hip_pack_vt_terms_dev(const float *v, uint16_t *vt, int B, int H, int S_kv, int D,
                                 const int64_t *v_strides, const int64_t *vt_strides,
                                 void *stream)
{
    if (!ready_for_device_call() || !check_dims(B, H, S_kv, S_kv, D))
        return false;
    if (int64_t(B) * H * S_kv * D > 0 && (!v || !vt))
        return fail("pack_vt_terms_dev: null pointer");
    const int64_t sp = vt_padded_len(S_kv);
    const Strides ts = vt_strides ? Strides{vt_strides[0], vt_strides[1], vt_strides[2]}
                                  : Strides{int64_t(H) * 2 * D * sp, 2 * int64_t(D) * sp, sp};
    if (ts.s != sp)
        return fail("pack_vt_terms_dev: V^T row stride must equal the padded key count");
    return launch_vt_pack_terms(v, from_array(v_strides, H, S_kv, D), vt, ts, B, H, S_kv, D,
                                pick_stream(stream));
}

bool anima_hip_qk_prologue_dev(const float *x, void *out, const float *w, const float *freqs,
                               int B, int S, int H, int D, const int64_t *x_strides,
                               const int64_t *out_strides, float eps, int flags, void *stream)
{
    if (!ready_for_device_call())
        return false;
    if (B < 0 || S < 0 || H < 0 || D < 0)
        return fail("qk_prologue: negative dimension");
    if (int64_t(B) * S * H * D > 0 && (!x || !out))
        return fail("qk_prologue: null pointer");
    RowProblem p;
    p.x = x;
    p.out = out;
    p.w = w;
    p.freqs = freqs;
    // x/out stride arrays describe [B, H, S, D] views, like the attention ones.
    p.xs = from_array(x_strides, H, S, D);
    p.os = from_array(out_strides, H, S, D);
    p.B = B;
    p.S = S;
    p.H = H;
    p.D = D;
    p.eps = eps;
    p.norm = (flags & 1) != 0;
    p.out_bf16 = (flags & 6) != 0;
    p.lo_off = (flags & 4) ? D : 0;  // [hi | lo] term rows
    return launch_rows(p, pick_stream(stream));
}

bool anima_hip_qkv_prologue_dev(const float *q, const float *k, const float *v, int64_t ld,
                                const float *q_norm_w, const float *k_norm_w,
                                const float *freqs, void *qo, void *ko, uint16_t *vt, int B,
                                int S, int H, int D, float eps, int mode, void *stream)
{
    if (!ready_for_device_call() || !check_dims(B, H, S, S, D))
        return false;
    AttnMode am;
    if (!attn_mode_of(mode, D, "qkv_prologue_dev", am))
        return false;
    if (int64_t(B) * S * H == 0)
        return true;
    if (D != 128)
        return fail("qkv_prologue_dev: D must be 128");
    if (ld < 0 || (ld > 0 && ld < int64_t(H) * D))
        return fail("qkv_prologue_dev: token row stride smaller than H*D");
    if (!q || !k || !qo || !ko || (am != kAttnF32 && (!v || !vt)))
        return fail("qkv_prologue_dev: null pointer");
    PrepProblem p;
    p.q = q;
    p.k = k;
    p.v = v;
    p.w[0] = q_norm_w;
    p.w[1] = k_norm_w;
    p.freqs = freqs;
    p.qo = qo;
    p.ko = ko;
    p.vt = vt;
    p.ld = ld > 0 ? ld : int64_t(H) * D;
    p.B = B;
    p.S = S;
    p.H = H;
    p.D = D;
    p.eps = eps;
    p.mode = am;
    return launch_prep_qkv(p, pick_stream(stream));
}

bool anima_hip_qkv_projection_dev(const float *x, int64_t ldx, const uint16_t *w_qkv,
                                  int64_t ldw, int K, const float *q_norm_w,
                                  const float *k_norm_w, const float *freqs, void *qo, void *ko,
                                  void *vo, int B, int S, int H, float eps, int mode,
                                  void *stream)
{
    if (!ready_for_device_call())
        return false;
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_F32X3)
        return fail("qkv_projection_dev: the f32 and f32x3 modes only");
    if (B <= 0 || S <= 0 || H <= 0 || K <= 0)
        return fail("qkv_projection_dev: dimensions must be positive");
    if (!x || !w_qkv || !qo || !ko || !vo)
        return fail("qkv_projection_dev: null pointer");
    QkvPrep p;
    p.qo = qo;
    p.ko = ko;
    p.vo = vo;
    p.w[0] = q_norm_w;
    p.w[1] = k_norm_w;
    p.freqs = freqs;
    p.B = B;
    p.S = S;
    p.H = H;
    p.eps = eps;
    p.mode = mode == ANIMA_HIP_F32 ? kAttnF32 : kAttnF32X3;
    return launch_gemm_f32a_qkv(x, ldx, w_qkv, ldw, K, p, pick_stream(stream));
}

bool anima_hip_gemm_dev(const float *a, int64_t lda, const void *w, int w_bf16, int64_t ldw,
                        float *c, int64_t ldc, int M, int N, int K, void *stream)
{
    if (!ready_for_device_call())
        return false;
    if (int64_t(M) * N > 0 && (!c || (K > 0 && (!a || !w))))
        return fail("gemm_dev: null pointer");
    return launch_gemm(a, lda, w, w_bf16 != 0, ldw, c, ldc, M, N, K, pick_stream(stream));
}

size_t anima_hip_linear_scratch_bytes(int M, int K, int mode)
{
    return linear_scratch_bytes(M, K, mode != ANIMA_HIP_BF16);
}

bool anima_hip_linear_dev(const float *a, int64_t lda, const uint16_t *w, int64_t ldw, float *c,
                          int64_t ldc, int M, int N, int K, int mode, void *scratch,
                          size_t scratch_bytes, void *stream)
{
    if (!ready_for_device_call())
        return false;
    if (mode != ANIMA_HIP_F32 && mode != ANIMA_HIP_BF16 && mode != ANIMA_HIP_F32X3)
        return fail("linear_dev: unknown mode " + std::to_string(mode));
    if (int64_t(M) * N > 0 && (!c || (K > 0 && (!a || !w))))
        return fail("linear_dev: null pointer");
    // The f32x3 mode's projections are the f32 mode's (exact hi + lo terms).
    return launch_linear(a, lda, w, ldw, c, ldc, M, N, K, mode != ANIMA_HIP_BF16, scratch,
                         scratch_bytes, pick_stream(stream));
}

size_t anima_hip_attention_scratch_bytes(int B, int S_q, int Bk, int S_kv, int H, int D,
                                         int mode)
{
    if (B < 0 || S_q < 0 || Bk < 0 || S_kv < 0 || H < 0 || D < 0)
        return 0;
    return attention_scratch_bytes(B, S_q, Bk, S_kv, H, D, size_mode(mode), false);
}

namespace {
// Term-output rules shared by anima_hip_attention_terms_dev and
// anima_hip_cross_attention_terms_dev.
bool check_term_rows(const char *who, const uint16_t *out_terms, int64_t ld_terms,
                     int64_t lo_offset, int H, int D)
{
    const std::string w(who);
    if (D != 128)
        return fail(w + ": the term output needs D == 128");
    const int64_t HD = int64_t(H) * D;
    if (ld_terms < HD || lo_offset < 0 || (lo_offset > 0 && (lo_offset < HD ||
                                                             lo_offset + HD > ld_terms)))
        return fail(w + ": a row of ld_terms elements must hold the hi block [0, H*D) and, "
                        "when lo_offset > 0, the lo block [lo_offset, lo_offset + H*D)");
    if (ld_terms % 8 || lo_offset % 8 || (reinterpret_cast<uintptr_t>(out_terms) & 15u))
        return fail(w + ": out_terms must be 16-byte aligned, ld_terms and lo_offset "
                        "multiples of 8");
    return true;
}

// anima_hip_attention_dev and its term-output form: O goes to out (f32) or,
// when out_t is set, to bf16 term rows (AttnInputs::out_t).
bool attention_dev_call(const char *name, const float *q, const float *k, const float *v,
                        const float *q_norm_w, const float *k_norm_w, const float *freqs,
                        float *out, uint16_t *out_t, int64_t ld_t, int64_t lo_t, void *scratch,
                        size_t scratch_bytes, int B, int S_q, int Bk, int S_kv, int H, int D,
                        float eps, int mode, void *stream)
{
    if (!ready_for_device_call() || !check_dims(B, H, S_q, S_kv, D))
        return false;
    AttnMode am;
    if (!attn_mode_of(mode, D, name, am))
        return false;
    if (int64_t(B) * S_q * H * D == 0)
        return true;
    const std::string who(name);
    if (!q || !(out || out_t) || !scratch || (S_kv > 0 && (!k || !v)))
        return fail(who + ": null pointer");
    if (scratch_bytes < attention_scratch_bytes(B, S_q, Bk, S_kv, H, D, am, false))
        return fail(who + ": scratch smaller than anima_hip_attention_scratch_bytes()");
    AttnInputs in;
    in.q = q;
    in.q_norm_w = q_norm_w;
    in.freqs = freqs;
    in.k = k;
    in.v = v;
    in.k_norm_w = k_norm_w;
    in.out = out;
    in.out_t = out_t;
    in.ld_t = ld_t;
    in.lo_t = lo_t;
    in.B = B;
    in.Bk = Bk;
    in.S_q = S_q;
    in.S_kv = S_kv;
    in.H = H;
    in.D = D;
    in.eps = eps;
    in.mode = am;
    return run_attention(in, scratch, pick_stream(stream));
}
}  // namespace

bool anima_hip_attention_dev(const float *q, const float *k, const float *v,
                             const float *q_norm_w, const float *k_norm_w, const float *freqs,
                             float *out, void *scratch, size_t scratch_bytes, int B, int S_q,
                             int Bk, int S_kv, int H, int D, float eps, int mode, void *stream)
{
    return attention_dev_call("attention_dev", q, k, v, q_norm_w, k_norm_w, freqs, out, nullptr,
                              0, 0, scratch, scratch_bytes, B, S_q, Bk, S_kv, H, D, eps, mode,
                              stream);
}

bool anima_hip_attention_terms_dev(const float *q, const float *k, const float *v,
                                   const float *q_norm_w, const float *k_norm_w,
                                   const float *freqs, uint16_t *out_terms, int64_t ld_terms,
                                   int64_t lo_offset, void *scratch, size_t scratch_bytes, int B,
                                   int S_q, int Bk, int S_kv, int H, int D, float eps, int mode,
                                   void *stream)
{
    if (!check_term_rows("attention_terms_dev", out_terms, ld_terms, lo_offset, H, D))
        return false;
    return attention_dev_call("attention_terms_dev", q, k, v, q_norm_w, k_norm_w, freqs, nullptr,
                              out_terms, ld_terms, lo_offset, scratch, scratch_bytes, B, S_q, Bk,
                              S_kv, H, D, eps, mode, stream);
}

bool anima_hip_attention(const float *q, const float *k, const float *v, const float *q_norm_w,
                         const float *k_norm_w, const float *freqs, float *out, int B, int S_q,
                         int S_kv, int H, int D, float eps, int mode)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r) || !check_dims(B, H, S_q, S_kv, D))
        return false;
    AttnMode am;
    if (!attn_mode_of(mode, D, "anima_hip_attention", am))
        return false;
    if (freqs && S_q != S_kv)
        return fail("anima_hip_attention: RoPE needs S_q == S_kv (self-attention)");
    const int64_t nq = int64_t(B) * S_q * H * D, nk = int64_t(B) * S_kv * H * D;
    if (nq == 0)
        return true;
    if (!q || !out || (nk > 0 && (!k || !v)))
        return fail("anima_hip_attention: null pointer");
    const hipStream_t st = r.stream;
    begin_call(r);
    // Batch groups, like the SDPA's head groups (sdpa_groups), when the
    // copies are large and each group still fills the GPU.
    const int64_t bytes = 2 * f32_bytes(nq) + 2 * f32_bytes(nk);
    int G = 1;
    for (int c = Runtime::kMaxGroups; c > 1 && G == 1 && bytes >= (int64_t(64) << 20); c /= 2) {
        const FlashPlan part = flash_plan(int64_t(B / c) * H, S_q, S_kv, D);
        if (B % c == 0 && part.waves == 8 && part.splits == 1)
            G = c;
    }
    const int Bg = B / G;
    const size_t scratch = attention_scratch_bytes(Bg, S_q, Bg, S_kv, H, D, am, false);
    if (!r.q.reserve(f32_bytes(nq), "workspace q") || !r.k.reserve(f32_bytes(nk), "workspace k") ||
        !r.v.reserve(f32_bytes(nk), "workspace v") || !r.o.reserve(f32_bytes(nq), "workspace o") ||
        !r.scratch.reserve(scratch, "workspace scratch"))
        return false;
    DrainOnError drain{r};
    AttnInputs in;
    if (!upload_optional(r.w0, q_norm_w, D, "workspace q_norm", st, in.q_norm_w) ||
        !upload_optional(r.w1, k_norm_w, D, "workspace k_norm", st, in.k_norm_w) ||
        !upload_optional(r.fr, freqs, size_t(S_q) * D * 2, "workspace freqs", st, in.freqs))
        return false;
    in.B = Bg;
    in.Bk = Bg;
    in.S_q = S_q;
    in.S_kv = S_kv;
    in.H = H;
    in.D = D;
    in.eps = eps;
    in.mode = am;
    const int64_t gq = nq / G, gk = nk / G;  // elements per group
    float *const qd = static_cast<float *>(r.q.p), *const kd = static_cast<float *>(r.k.p);
    float *const vd = static_cast<float *>(r.v.p), *const od = static_cast<float *>(r.o.p);
    const auto bytes_of = [](const float *p) { return reinterpret_cast<const char *>(p); };
    Pieces up, down;
    for (int g = 0; g < G; ++g) {
        up[g] = {{reinterpret_cast<char *>(qd + g * gq), bytes_of(q + g * gq), f32_bytes(gq)},
                 {reinterpret_cast<char *>(kd + g * gk), bytes_of(k + g * gk), f32_bytes(gk)},
                 {reinterpret_cast<char *>(vd + g * gk), bytes_of(v + g * gk), f32_bytes(gk)}};
        down[g] = {{reinterpret_cast<char *>(out + g * gq), bytes_of(od + g * gq), f32_bytes(gq)}};
    }
    if (!run_groups(r, G, up, down, [&](int g, hipStream_t s) {
            in.q = qd + g * gq;
            in.k = kd + g * gk;
            in.v = vd + g * gk;
            in.out = od + g * gq;
            return run_attention(in, r.scratch.p, s);
        }))
        return false;
    drain.done = true;
    return finish_call(r);
}

anima_hip_ctx_kv *anima_hip_ctx_kv_create(const float *ctx, const uint16_t *wk, const uint16_t *wv,
                                          const float *k_norm_w, int Bc, int S_kv, int C, int H,
                                          int D, float eps, int mode)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return nullptr;
    if (Bc <= 0 || S_kv <= 0 || C <= 0 || H <= 0 || D <= 0) {
        fail("ctx_kv_create: all dimensions must be positive");
        return nullptr;
    }
    AttnMode am;
    if (!attn_mode_of(mode, D, "ctx_kv_create", am))
        return nullptr;
    const bool bf16 = am == kAttnBF16;
    if (!ctx || !wk || !wv) {
        fail("ctx_kv_create: null pointer");
        return nullptr;
    }
    const hipStream_t st = r.stream;
    const int M = Bc * S_kv, N = H * D;
    const size_t wbytes = size_t(N) * C * 2;
    DevBuf kf, vf;
    const float *kw = nullptr;
    if (!r.q.reserve(f32_bytes(int64_t(M) * C), "workspace ctx") ||
        !r.k.reserve(wbytes, "workspace Wk") || !r.v.reserve(wbytes, "workspace Wv") ||
        !kf.reserve(f32_bytes(int64_t(M) * N), "ctx K projection") ||
        !vf.reserve(f32_bytes(int64_t(M) * N), "ctx V projection") ||
        !h2d(r.q.p, ctx, f32_bytes(int64_t(M) * C), st) || !h2d(r.k.p, wk, wbytes, st) ||
        !h2d(r.v.p, wv, wbytes, st) ||
        !upload_optional(r.w1, k_norm_w, D, "workspace k_norm", st, kw)) {
        (void)hipStreamSynchronize(st);
        kf.release();
        vf.release();
        return nullptr;
    }
    auto *kv = new anima_hip_ctx_kv;
    kv->mode = mode;
    kv->Bc = Bc;
    kv->S_kv = S_kv;
    kv->H = H;
    kv->D = D;
    kv->device = r.device;
    // K/V projections of the context on bf16 MFMA: the context enters as
    // exact hi + lo bf16 terms in the f32 and f32x3 modes, rounded to bf16 in
    // bf16 mode.
    const size_t sb = linear_scratch_bytes(M, C, !bf16);
    bool ok = r.scratch.reserve(sb, "workspace linear") &&
              launch_linear(static_cast<const float *>(r.q.p), C,
                            static_cast<const uint16_t *>(r.k.p), C, static_cast<float *>(kf.p),
                            N, M, N, C, !bf16, r.scratch.p, sb, st) &&
              launch_linear(static_cast<const float *>(r.q.p), C,
                            static_cast<const uint16_t *>(r.v.p), C, static_cast<float *>(vf.p),
                            N, M, N, C, !bf16, r.scratch.p, sb, st);
    if (ok && am != kAttnF32) {
        ok = hip_ok(hipMalloc(&kv->k, prepared_k_bytes(Bc, S_kv, H, D, am)), "ctx K cache") &&
             hip_ok(hipMalloc(&kv->v, prepared_v_bytes(Bc, S_kv, H, D, am)), "ctx V cache") &&
             prepare_kv(static_cast<const float *>(kf.p), static_cast<const float *>(vf.p), kw,
                        nullptr, kv->k, kv->v, Bc, S_kv, H, D, eps, am, st) &&
             sync(st);
    } else if (ok) {
        // f32: normalise K in place (each row is staged in LDS before it is
        // rewritten); the two projections become the cache.
        ok = prepare_kv(static_cast<const float *>(kf.p), nullptr, kw, nullptr, kf.p, nullptr, Bc,
                        S_kv, H, D, eps, kAttnF32, st) &&
             sync(st);
        if (ok) {
            kv->k = kf.p;
            kv->v = vf.p;
            kf.p = vf.p = nullptr;
        }
    }
    (void)hipStreamSynchronize(st);
    kf.release();
    vf.release();
    if (!ok) {
        if (kv->k)
            (void)hipFree(kv->k);
        if (kv->v)
            (void)hipFree(kv->v);
        delete kv;
        return nullptr;
    }
    return kv;
}

void anima_hip_ctx_kv_destroy(anima_hip_ctx_kv *kv)
{
    if (!kv)
        return;
    // Work that may still read the cache can sit on any stream: drain the device.
    (void)hipDeviceSynchronize();
    if (kv->k)
        (void)hipFree(kv->k);
    if (kv->v)
        (void)hipFree(kv->v);
    delete kv;
}

size_t anima_hip_attention_block_scratch_bytes(const anima_hip_ctx_kv *kv, int B, int S, int Dm,
                                               int H, int D, int mode)
{
    if (B < 0 || S < 0 || Dm < 0 || H < 0 || D < 0)
        return 0;
    if (kv)
        return attention_block_scratch_bytes(B, S, Dm, kv->H, kv->D, kv->Bc, kv->S_kv,
                                             AttnMode(kv->mode), true);
    return attention_block_scratch_bytes(B, S, Dm, H, D, B, S, size_mode(mode), false);
}

bool anima_hip_attention_block_dev(float *x, const float *mod, const uint16_t *wq,
                                   const uint16_t *wk, const uint16_t *wv, const uint16_t *wo,
                                   const float *q_norm_w, const float *k_norm_w,
                                   const float *freqs, const anima_hip_ctx_kv *kv, int B, int S,
                                   int Dm, int H, int D, float eps, int mode, void *scratch,
                                   size_t scratch_bytes, void *stream)
{
    if (!ready_for_device_call())
        return false;
    if (!check_dims(B, H, S, S, D) || Dm < 0)
        return fail("attention_block_dev: negative dimension");
    AttnMode am;
    if (!attn_mode_of(mode, D, "attention_block_dev", am))
        return false;
    BlockProblem p;
    p.x = x;
    p.mod = mod;
    p.wq = wq;
    p.wk = wk;
    p.wv = wv;
    p.wo = wo;
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.freqs = freqs;
    p.B = B;
    p.S = S;
    p.Dm = Dm;
    p.H = H;
    p.D = D;
    p.eps = eps;
    p.mode = am;
    if (kv) {
        int dev = 0;
        if (!hip_ok(hipGetDevice(&dev), "hipGetDevice"))
            return false;
        if (dev != kv->device)
            return fail("attention_block_dev: the context cache lives on another device");
        if (kv->H != H || kv->D != D || kv->mode != mode)
            return fail("attention_block_dev: heads, head dim and mode must match the context cache");
        if (kv->Bc != 1 && kv->Bc != B)
            return fail("attention_block_dev: the context batch must be 1 or B");
        p.k_prep = kv->k;
        p.v_prep = kv->v;
        p.Bk = kv->Bc;
        p.S_kv = kv->S_kv;
    } else if (freqs && !S) {
        return true;
    }
    return run_attention_block(p, scratch, scratch_bytes, pick_stream(stream));
}

size_t anima_hip_cross_attention_scratch_bytes(const anima_hip_ctx_kv *kv, int B, int S_q)
{
    if (!kv || B < 0 || S_q < 0)
        return 0;
    return attention_scratch_bytes(B, S_q, kv->Bc, kv->S_kv, kv->H, kv->D, AttnMode(kv->mode),
                                   true);
}

namespace {
// anima_hip_cross_attention_dev and its term-output form.
bool cross_dev_call(const char *name, const float *q, const float *q_norm_w,
                    const anima_hip_ctx_kv *kv, float *out, uint16_t *out_t, int64_t ld_t,
                    int64_t lo_t, void *scratch, size_t scratch_bytes, int B, int S_q, float eps,
                    void *stream)
{
    if (!ready_for_device_call())
        return false;
    const std::string who(name);
    if (!kv)
        return fail(who + ": null cache handle");
    if (B < 0 || S_q < 0)
        return fail(who + ": negative dimension");
    if (out_t && !check_term_rows(name, out_t, ld_t, lo_t, kv->H, kv->D))
        return false;
    if (int64_t(B) * S_q == 0)
        return true;
    if (!q || !(out || out_t) || !scratch)
        return fail(who + ": null pointer");
    const AttnMode am = AttnMode(kv->mode);
    if (scratch_bytes < attention_scratch_bytes(B, S_q, kv->Bc, kv->S_kv, kv->H, kv->D, am, true))
        return fail(who + ": scratch smaller than anima_hip_cross_attention_scratch_bytes()");
    AttnInputs in;
    in.q = q;
    in.q_norm_w = q_norm_w;
    in.k_prep = kv->k;
    in.v_prep = kv->v;
    in.out = out;
    in.out_t = out_t;
    in.ld_t = ld_t;
    in.lo_t = lo_t;
    in.B = B;
    in.Bk = kv->Bc;
    in.S_q = S_q;
    in.S_kv = kv->S_kv;
    in.H = kv->H;
    in.D = kv->D;
    in.eps = eps;
    in.mode = am;
    return run_attention(in, scratch, pick_stream(stream));
}
}  // namespace

bool anima_hip_cross_attention_dev(const float *q, const float *q_norm_w,
                                   const anima_hip_ctx_kv *kv, float *out, void *scratch,
                                   size_t scratch_bytes, int B, int S_q, float eps, void *stream)
{
    return cross_dev_call("cross_attention_dev", q, q_norm_w, kv, out, nullptr, 0, 0, scratch,
                          scratch_bytes, B, S_q, eps, stream);
}

bool anima_hip_cross_attention_terms_dev(const float *q, const float *q_norm_w,
                                         const anima_hip_ctx_kv *kv, uint16_t *out_terms,
                                         int64_t ld_terms, int64_t lo_offset, void *scratch,
                                         size_t scratch_bytes, int B, int S_q, float eps,
                                         void *stream)
{
    return cross_dev_call("cross_attention_terms_dev", q, q_norm_w, kv, nullptr, out_terms,
                          ld_terms, lo_offset, scratch, scratch_bytes, B, S_q, eps, stream);
}

bool anima_hip_cross_attention(const float *q, const float *q_norm_w, const anima_hip_ctx_kv *kv,
                               float *out, int B, int S_q, float eps)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (!ensure_ready(r))
        return false;
    if (!kv)
        return fail("cross_attention: null cache handle");
    if (B < 0 || S_q < 0)
        return fail("cross_attention: negative dimension");
    const int64_t nq = int64_t(B) * S_q * kv->H * kv->D;
    if (nq == 0)
        return true;
    if (!q || !out)
        return fail("cross_attention: null pointer");
    if (kv->Bc != 1 && kv->Bc != B)
        return fail("cross_attention: context batch must be 1 (broadcast) or equal to the query "
                    "batch");
    const hipStream_t st = r.stream;
    begin_call(r);
    const AttnMode am = AttnMode(kv->mode);
    // Batch groups, like the SDPA's head groups (sdpa_groups), when the
    // copies are large and each group still fills the GPU: group g reads the
    // cache's batch entries of its own queries (or the one shared entry).
    int G = 1;
    for (int c = Runtime::kMaxGroups; c > 1 && G == 1 && 2 * f32_bytes(nq) >= (size_t(64) << 20);
         c /= 2) {
        const FlashPlan part = flash_plan(int64_t(B / c) * kv->H, S_q, kv->S_kv, kv->D);
        if (B % c == 0 && part.waves == 8 && part.splits == 1)
            G = c;
    }
    const int Bg = B / G, Bkg = kv->Bc == 1 ? 1 : Bg;
    const size_t scratch =
        attention_scratch_bytes(Bg, S_q, Bkg, kv->S_kv, kv->H, kv->D, am, true);
    const float *qw = nullptr;
    if (!r.q.reserve(f32_bytes(nq), "workspace q") || !r.o.reserve(f32_bytes(nq), "workspace o") ||
        !r.scratch.reserve(scratch, "workspace scratch"))
        return false;
    DrainOnError drain{r};
    if (!upload_optional(r.w0, q_norm_w, kv->D, "workspace q_norm", st, qw))
        return false;
    const int64_t gq = nq / G;  // elements per group
    float *const qd = static_cast<float *>(r.q.p), *const od = static_cast<float *>(r.o.p);
    Pieces up, down;
    for (int g = 0; g < G; ++g) {
        up[g] = {{reinterpret_cast<char *>(qd + g * gq),
                  reinterpret_cast<const char *>(q + g * gq), f32_bytes(gq)}};
        down[g] = {{reinterpret_cast<char *>(out + g * gq),
                    reinterpret_cast<const char *>(od + g * gq), f32_bytes(gq)}};
    }
    const size_t kb1 = prepared_k_bytes(1, kv->S_kv, kv->H, kv->D, am);
    const size_t vb1 = prepared_v_bytes(1, kv->S_kv, kv->H, kv->D, am);
    if (!run_groups(r, G, up, down, [&](int g, hipStream_t s) {
            const size_t b0 = kv->Bc == 1 ? 0 : size_t(g) * Bg;
            AttnInputs in;
            in.q = qd + g * gq;
            in.q_norm_w = qw;
            in.k_prep = static_cast<const char *>(kv->k) + b0 * kb1;
            in.v_prep = static_cast<const char *>(kv->v) + b0 * vb1;
            in.out = od + g * gq;
            in.B = Bg;
            in.Bk = Bkg;
            in.S_q = S_q;
            in.S_kv = kv->S_kv;
            in.H = kv->H;
            in.D = kv->D;
            in.eps = eps;
            in.mode = am;
            return run_attention(in, r.scratch.p, s);
        }))
        return false;
    drain.done = true;
    return finish_call(r);
}

void *anima_hip_malloc(size_t bytes)
{
    if (!ready_for_device_call())
        return nullptr;
    void *p = nullptr;
    if (!hip_ok(hipMalloc(&p, std::max<size_t>(bytes, 1)), "hipMalloc"))
        return nullptr;
    return p;
}

void anima_hip_free(void *p)
{
    if (p) {
        (void)hipDeviceSynchronize();
        (void)hipFree(p);
    }
}

bool anima_hip_memcpy(void *dst, const void *src, size_t bytes, int kind)
{
    if (!ready_for_device_call())
        return false;
    const hipMemcpyKind k = kind == 1   ? hipMemcpyHostToDevice
                            : kind == 2 ? hipMemcpyDeviceToHost
                            : kind == 3 ? hipMemcpyDeviceToDevice
                                        : hipMemcpyDefault;
    if (kind < 1 || kind > 3)
        return fail("memcpy: kind must be 1, 2 or 3");
    if (bytes == 0)
        return true;
    if (!dst || !src)
        return fail("memcpy: null pointer");
    return hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize") &&
           hip_ok(hipMemcpy(dst, src, bytes, k), "hipMemcpy");
}

bool anima_hip_synchronize(void)
{
    return ready_for_device_call() && hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

bool anima_hip_last_call_ms(float *kernel_ms, float *total_ms)
{
    Runtime &r = rt();
    std::lock_guard<std::recursive_mutex> g(r.mu);
    if (r.timer.total_ms < 0.0f)
        return fail("last_call_ms: no host-pointer call has completed yet");
    if (kernel_ms)
        *kernel_ms = r.timer.kernel_ms;
    if (total_ms)
        *total_ms = r.timer.total_ms;
    return true;
}

}  // extern "C"
