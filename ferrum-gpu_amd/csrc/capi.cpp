// capi.cpp -- the extern "C" boundary declared in include/ferrum_gpu.h.
//
// Every entry point converts C++ exceptions into an FG_ERR_* status plus a
// thread-local message, the C-ABI shape of the reference's Result<_, Error> ->
// PyValueError mapping (crates/ferrum-gpu-py/src/lib.rs:404-406, 497, 577).
#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <string.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "device.hpp"
#include "fft_plan.hpp"
#include "ferrum_gpu.h"
#include "hip_backend.hpp"
#include "host_stage.hpp"
#include "scratch.hpp"

using fg::Buffer;
using fg::Cf32;
using fg::Direction;
using fg::Error;
using fg::FftPlan;
using fg::HipBackend;
using fg::HipDevice;

struct fg_device {
    std::unique_ptr<HipDevice> dev;
    HipBackend::Module fft_module;
    std::mutex mu;  // guards the plan cache and the staging buffer of the host path
    // Host-path plans, key: (dims, log_n or log_cols, log_rows (0 for 1D), batch);
    // the kCachedPlans most recently used are kept (a multi-pass plan holds up
    // to a 128 MiB workspace, so the cache must not grow with every new batch).
    struct CachedPlan {
        std::unique_ptr<FftPlan> plan;
        uint64_t last_use = 0;
    };
    std::map<std::tuple<int, uint32_t, uint32_t, size_t>, CachedPlan> plans;
    uint64_t plan_clock = 0;
    Buffer<Cf32, HipBackend> staging;
    Buffer<Cf32, HipBackend> staging_out;  // out-of-place outputs (plans whose in-place form differs)
    fg::Pointwise pointwise;  // elementwise kernels of fft_module
    std::atomic<int> dependents{0};  // live plans and captured graphs made on this device
    std::unique_ptr<fg::HostStager> stager;  // pinned pieces of the host path (first large call)
    // fg_fft_exec_split_noalloc: calls on this device take turns at the
    // scratch area.  Outside stream capture each call waits for the previous
    // call's last launch (scratch_done, recorded on its stream) before its
    // first, so calls on different streams run one after another on the GPU.
    std::mutex scratch_mu;
    hipEvent_t scratch_done = nullptr;
    ~fg_device() {
        if (scratch_done) {
            (void)hipSetDevice(dev->handle()->ordinal);
            (void)hipEventDestroy(scratch_done);
        }
    }
};

struct fg_module {
    HipBackend::Module mod;
    HipBackend::DeviceHandle dev;
    bool borrowed = false;  // the device's own FFT module: not unloaded by the caller
};

struct fg_kernel {
    HipBackend::KernelHandle fn = nullptr;
    HipBackend::Module keep;  // a kernel keeps its module loaded
};

struct fg_event {
    hipEvent_t ev = nullptr;
    int ordinal = 0;
    // The device's default stream, where a NULL stream records (as NULL means
    // that stream for launches and copies); the handle keeps it alive.
    HipBackend::DeviceHandle dev;
};

struct fg_fft_plan {
    std::unique_ptr<FftPlan> plan;
    fg_device* dev = nullptr;
    std::atomic<int> graphs{0};  // live fg_graph objects that replay this plan
};

struct fg_graph {
    HipBackend::Graph g;
    fg_device* dev = nullptr;
    fg_fft_plan* plan = nullptr;  // fg_fft_graph_create: the plan it replays (else null)
};

namespace {

thread_local std::string g_last_error;

template <class F>
int guarded(F&& f) {
    try {
        f();
        g_last_error.clear();
        return FG_OK;
    } catch (const Error& e) {
        g_last_error = e.what();
        return e.code();
    } catch (const std::bad_alloc&) {
        g_last_error = "host allocation failed";
        return FG_ERR_OUT_OF_MEMORY;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return FG_ERR_INTERNAL;
    } catch (...) {
        g_last_error = "unknown error";
        return FG_ERR_INTERNAL;
    }
}

void need(const void* p, const char* what) {
    if (!p) fg::invalid(std::string(what) + " is null");
}

fg_device* open_device(int ordinal) {
    auto h = HipBackend::open(ordinal);
    std::unique_ptr<fg_device> d(new fg_device);
    d->dev.reset(new HipDevice(h));
    d->fft_module = d->dev->load_or_cache(fg::fft_code_object());
    d->pointwise = fg::Pointwise(d->fft_module);
    // The allocation-free entry point's scratch area: its address on this
    // device, resolved once with the device current (scratch.hip).
    HipBackend::bind(h);
    fg::scratch_init(h->ordinal);
    fg::hip_check(hipEventCreateWithFlags(&d->scratch_done, hipEventDisableTiming), "hipEventCreateWithFlags");
    return d.release();
}

// The one-shot path's device (crates/ferrum-gpu-py/src/lib.rs:254-264 builds a
// transient context per call; this keeps one per process instead).
fg_device* default_device() {
    static std::once_flag once;
    static fg_device* dev = nullptr;
    static std::string err;
    static int code = 0;
    std::call_once(once, [] {
        try {
            dev = open_device(0);
        } catch (const Error& e) {
            err = e.what();
            code = e.code();
        }
    });
    if (!dev) fg::fail(code ? code : FG_ERR_NO_DEVICE, err);
    return dev;
}

constexpr size_t kCachedPlans = 8;

// Caller holds d->mu, which also covers every use of the returned plan, so an
// evicted plan is never in use.
FftPlan& cached_plan(fg_device* d, int dims, uint32_t log_n, uint32_t log_rows, size_t batch) {
    auto key = std::make_tuple(dims, log_n, log_rows, batch);
    const uint64_t now = ++d->plan_clock;
    auto it = d->plans.find(key);
    if (it != d->plans.end()) {
        it->second.last_use = now;
        return *it->second.plan;
    }
    auto p = dims == 1 ? FftPlan::make_1d(*d->dev, d->fft_module, log_n, batch)
                       : FftPlan::make_2d(*d->dev, d->fft_module, log_rows, log_n, batch);
    if (d->plans.size() >= kCachedPlans) {
        auto oldest = d->plans.begin();
        for (auto e = d->plans.begin(); e != d->plans.end(); ++e)
            if (e->second.last_use < oldest->second.last_use) oldest = e;
        d->plans.erase(oldest);
    }
    FftPlan& ref = *p;
    d->plans[key] = fg_device::CachedPlan{std::move(p), now};
    return ref;
}

Direction parse_dir(int direction) {
    if (direction == FG_FORWARD) return Direction::Forward;
    if (direction == FG_INVERSE) return Direction::Inverse;
    fg::invalid("direction must be 1 (forward) or -1 (inverse), got " + std::to_string(direction));
}

// Host arrays from this size up go through HostStager's pinned pieces; below
// it a plain pageable copy costs less than the staging's fixed overheads.
constexpr size_t kStagedBytes = 2u << 20;

// Host path shared by the 1D and 2D entry points: stage through one device
// buffer (grown on demand, kept per device), run in place, copy back.  Plans
// whose in-place execution runs other kernels (the row pairs of 2D plans of
// 2048 / 4096 rows run out of place only) run out of place into a second
// staging buffer, so the host path gives the bits of the device path's
// out-of-place fg_fft_exec.
void run_host(fg_device* d, int dims, uint32_t log_n, uint32_t log_rows, size_t batch, size_t total,
              const float* in, float* out, Direction dir, bool normalize) {
    std::lock_guard<std::mutex> g(d->mu);
    FftPlan& plan = cached_plan(d, dims, log_n, log_rows, batch);
    auto grow = [&](Buffer<Cf32, HipBackend>& b) {
        if (b.len() < total) {
            b.reset();
            b = d->dev->alloc<Cf32>(total);
        }
    };
    grow(d->staging);
    Cf32* src = d->staging.data();
    Cf32* dst = src;
    if (plan.in_place_differs()) {
        grow(d->staging_out);
        dst = d->staging_out.data();
    }
    const auto& h = d->dev->handle();
    const size_t bytes = total * sizeof(Cf32);
    if (bytes >= kStagedBytes) {
        // Through pinned pieces and parallel host copies (host_stage.hpp).
        if (!d->stager) d->stager.reset(new fg::HostStager(h));
        const hipStream_t s = d->dev->default_stream();
        d->stager->to_device(src, in, bytes, s);
        plan.exec(src, dst, dir, normalize, s);
        d->stager->to_host(out, dst, bytes, s);
        return;
    }
    HipBackend::copy_async(h, src, in, bytes, hipMemcpyHostToDevice, nullptr);
    plan.exec(src, dst, dir, normalize, nullptr);
    HipBackend::copy_async(h, out, dst, bytes, hipMemcpyDeviceToHost, nullptr);
    d->dev->sync();
}

// Elements of `batch` images of 2^log_elems points, refusing a product that
// does not fit in size_t (it would size the staging buffer below the plan).
size_t host_2d_elems(uint32_t log_elems, size_t batch) {
    if (batch > (SIZE_MAX >> log_elems) / sizeof(Cf32))
        fg::invalid("batch " + std::to_string(batch) + " too large for images of 2^" + std::to_string(log_elems) +
                    " points");
    return (size_t(1) << log_elems) * batch;
}

}  // namespace

extern "C" {

const char* fg_last_error(void) { return g_last_error.c_str(); }
const char* fg_version(void) { return "0.3.0"; }
int fg_backend_id(void) { return (int)HipBackend::id(); }

int fg_device_count(int* count) {
    return guarded([&] {
        need(count, "count");
        *count = HipBackend::device_count();
    });
}

int fg_device_open(int ordinal, fg_device_t* out) {
    return guarded([&] {
        need(out, "out");
        *out = nullptr;
        *out = open_device(ordinal);
    });
}

int fg_device_close(fg_device_t dev) {
    return guarded([&] {
        if (!dev) return;
        if (dev->dependents.load() > 0)
            fg::invalid("device still has " + std::to_string(dev->dependents.load()) +
                        " plan(s) or graph(s); destroy them first");
        try {
            dev->dev->sync();
        } catch (...) {
        }
        delete dev;
    });
}

int fg_device_sync(fg_device_t dev) {
    return guarded([&] {
        need(dev, "device");
        dev->dev->sync();
    });
}

int fg_device_default_stream(fg_device_t dev, fg_stream_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = (fg_stream_t)dev->dev->default_stream();
    });
}

int fg_device_info(fg_device_t dev, char* arch, size_t arch_cap, int* cu_count, size_t* total_mem_bytes,
                   int* clock_khz) {
    return guarded([&] {
        need(dev, "device");
        const auto& h = dev->dev->handle();
        if (arch && arch_cap) {
            strncpy(arch, h->arch.c_str(), arch_cap - 1);
            arch[arch_cap - 1] = 0;
        }
        if (cu_count) *cu_count = h->cu_count;
        if (total_mem_bytes) *total_mem_bytes = h->total_mem;
        if (clock_khz) *clock_khz = h->clock_khz;
    });
}

int fg_alloc_zeros(fg_device_t dev, size_t bytes, void** dptr) {
    return guarded([&] {
        need(dev, "device");
        need(dptr, "dptr");
        *dptr = HipBackend::alloc_zeros(dev->dev->handle(), bytes);
    });
}

int fg_free(fg_device_t dev, void* dptr) {
    return guarded([&] {
        need(dev, "device");
        HipBackend::free(dev->dev->handle(), dptr);
    });
}

int fg_copy_h2d(fg_device_t dev, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        need(dev, "device");
        if (bytes) {
            need(dst, "dst");
            need(src, "src");
        }
        HipBackend::copy_h2d(dev->dev->handle(), dst, src, bytes);
    });
}

int fg_copy_d2h(fg_device_t dev, void* dst, const void* src, size_t bytes) {
    return guarded([&] {
        need(dev, "device");
        if (bytes) {
            need(dst, "dst");
            need(src, "src");
        }
        HipBackend::copy_d2h(dev->dev->handle(), dst, src, bytes);
    });
}

static int copy_async(fg_device_t dev, void* dst, const void* src, size_t bytes, fg_stream_t stream,
                      hipMemcpyKind kind) {
    return guarded([&] {
        need(dev, "device");
        if (bytes) {
            need(dst, "dst");
            need(src, "src");
        }
        HipBackend::copy_async(dev->dev->handle(), dst, src, bytes, kind, (hipStream_t)stream);
    });
}

int fg_copy_h2d_async(fg_device_t dev, void* dst, const void* src, size_t bytes, fg_stream_t stream) {
    return copy_async(dev, dst, src, bytes, stream, hipMemcpyHostToDevice);
}
int fg_copy_d2h_async(fg_device_t dev, void* dst, const void* src, size_t bytes, fg_stream_t stream) {
    return copy_async(dev, dst, src, bytes, stream, hipMemcpyDeviceToHost);
}
int fg_copy_d2d_async(fg_device_t dev, void* dst, const void* src, size_t bytes, fg_stream_t stream) {
    return copy_async(dev, dst, src, bytes, stream, hipMemcpyDeviceToDevice);
}

int fg_module_load(fg_device_t dev, int backend_id, const void* image, size_t size, fg_module_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = nullptr;
        fg::KernelArtifact a;
        a.backend = (fg::BackendId)backend_id;
        a.name = "user";
        a.image = image;
        a.size = size;
        std::unique_ptr<fg_module> m(new fg_module);
        m->dev = dev->dev->handle();
        m->mod = HipBackend::load_module(m->dev, a);
        *out = m.release();
    });
}

int fg_module_unload(fg_module_t mod) {
    return guarded([&] {
        if (!mod) return;
        delete mod;  // the module itself unloads once no kernel holds it
    });
}

int fg_device_fft_module(fg_device_t dev, fg_module_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        std::unique_ptr<fg_module> m(new fg_module);
        m->dev = dev->dev->handle();
        m->mod = dev->fft_module;
        m->borrowed = true;
        *out = m.release();
    });
}

int fg_kernel_get(fg_module_t mod, const char* name, fg_kernel_t* out) {
    return guarded([&] {
        need(mod, "module");
        need(name, "name");
        need(out, "out");
        *out = nullptr;
        std::unique_ptr<fg_kernel> k(new fg_kernel);
        k->fn = HipBackend::get_kernel(mod->mod, name);
        k->keep = mod->mod;
        *out = k.release();
    });
}

int fg_launch(fg_device_t dev, fg_stream_t stream, fg_kernel_t kernel, const uint32_t grid[3],
              const uint32_t block[3], uint32_t shared_bytes, void** args) {
    return guarded([&] {
        need(dev, "device");
        need(kernel, "kernel");
        need(grid, "grid");
        need(block, "block");
        HipBackend::launch(dev->dev->handle(), (hipStream_t)stream, kernel->fn, fg::Dim3(grid[0], grid[1], grid[2]),
                           fg::Dim3(block[0], block[1], block[2]), shared_bytes, args);
    });
}

int fg_stream_create(fg_device_t dev, fg_stream_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = (fg_stream_t)HipBackend::create_stream(dev->dev->handle());
    });
}

int fg_stream_destroy(fg_device_t dev, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        HipBackend::destroy_stream(dev->dev->handle(), (hipStream_t)stream);
    });
}

int fg_stream_sync(fg_device_t dev, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        HipBackend::sync_stream(dev->dev->handle(), (hipStream_t)stream);
    });
}

int fg_event_create(fg_device_t dev, fg_event_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        HipBackend::bind(dev->dev->handle());
        std::unique_ptr<fg_event> e(new fg_event);
        e->ordinal = dev->dev->handle()->ordinal;
        e->dev = dev->dev->handle();
        fg::hip_check(hipEventCreate(&e->ev), "hipEventCreate");
        *out = e.release();
    });
}

int fg_event_destroy(fg_event_t ev) {
    return guarded([&] {
        if (!ev) return;
        (void)hipSetDevice(ev->ordinal);
        (void)hipEventDestroy(ev->ev);
        delete ev;
    });
}

int fg_event_record(fg_event_t ev, fg_stream_t stream) {
    return guarded([&] {
        need(ev, "event");
        fg::hip_check(hipSetDevice(ev->ordinal), "hipSetDevice");
        const hipStream_t s = stream ? (hipStream_t)stream : HipBackend::default_stream(ev->dev);
        fg::hip_check(hipEventRecord(ev->ev, s), "hipEventRecord");
    });
}

int fg_event_sync(fg_event_t ev) {
    return guarded([&] {
        need(ev, "event");
        fg::hip_check(hipEventSynchronize(ev->ev), "hipEventSynchronize");
    });
}

int fg_event_elapsed_ms(fg_event_t start, fg_event_t end, float* ms) {
    return guarded([&] {
        need(start, "start");
        need(end, "end");
        need(ms, "ms");
        fg::hip_check(hipEventElapsedTime(ms, start->ev, end->ev), "hipEventElapsedTime");
    });
}

int fg_fft_plan_1d(fg_device_t dev, uint32_t log_n, size_t batch, fg_fft_plan_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = nullptr;
        std::unique_ptr<fg_fft_plan> p(new fg_fft_plan);
        p->dev = dev;
        p->plan = FftPlan::make_1d(*dev->dev, dev->fft_module, log_n, batch);
        dev->dependents.fetch_add(1);
        *out = p.release();
    });
}

int fg_fft_plan_2d(fg_device_t dev, uint32_t log_n, size_t batch, fg_fft_plan_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = nullptr;
        std::unique_ptr<fg_fft_plan> p(new fg_fft_plan);
        p->dev = dev;
        p->plan = FftPlan::make_2d(*dev->dev, dev->fft_module, log_n, log_n, batch);
        dev->dependents.fetch_add(1);
        *out = p.release();
    });
}

int fg_fft_plan_destroy(fg_fft_plan_t plan) {
    return guarded([&] {
        if (!plan) return;
        if (plan->graphs.load() > 0)
            fg::invalid("plan still has " + std::to_string(plan->graphs.load()) +
                        " graph(s); destroy them first");
        plan->dev->dependents.fetch_sub(1);
        delete plan;
    });
}

int fg_fft_exec(fg_fft_plan_t plan, const void* d_in, void* d_out, int direction, int normalize,
                fg_stream_t stream) {
    return guarded([&] {
        need(plan, "plan");
        need(d_in, "d_in");
        need(d_out, "d_out");
        plan->plan->exec(d_in, d_out, parse_dir(direction), normalize != 0, (hipStream_t)stream);
    });
}

int fg_fft_exec_split(fg_fft_plan_t plan, const void* d_in_re, const void* d_in_im, void* d_out_re,
                      void* d_out_im, int direction, int normalize, fg_stream_t stream) {
    return guarded([&] {
        need(plan, "plan");
        plan->plan->exec_split(d_in_re, d_in_im, d_out_re, d_out_im, parse_dir(direction), normalize != 0,
                               (hipStream_t)stream);
    });
}

int fg_fft_exec_split_noalloc(fg_fft_plan_t plan, const void* d_in_re, const void* d_in_im, void* d_out_re,
                              void* d_out_im, int direction, int normalize, fg_stream_t stream) {
    return guarded([&] {
        need(plan, "plan");
        const Direction dir = parse_dir(direction);
        std::string why;
        fg_device* d = plan->dev;
        void* scratch = fg::scratch_device_ptr(d->dev->handle()->ordinal, &why);
        const hipStream_t s = stream ? (hipStream_t)stream : d->dev->default_stream();
        // Single-pass plans touch no scratch; a capturing stream cannot wait
        // for an event recorded outside its capture, so captured calls keep
        // the documented race between calls that overlap.
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        HipBackend::bind(d->dev->handle());
        fg::hip_check(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
        const bool serialize = plan->plan->split_staged_exec();
        std::unique_lock<std::mutex> lock(d->scratch_mu, std::defer_lock);
        if (serialize && cap == hipStreamCaptureStatusNone) {
            lock.lock();
            fg::hip_check(hipStreamWaitEvent(s, d->scratch_done, 0), "hipStreamWaitEvent");
        }
        plan->plan->exec_split_into(d_in_re, d_in_im, d_out_re, d_out_im, dir, normalize != 0, s, scratch,
                                    fg::kScratchBytes, why);
        if (lock.owns_lock()) fg::hip_check(hipEventRecord(d->scratch_done, s), "hipEventRecord");
    });
}

int fg_fft_exec_events(fg_fft_plan_t plan, const void* d_in, void* d_out, int direction, int normalize,
                       fg_stream_t stream, fg_event_t* events, int nevents) {
    return guarded([&] {
        need(plan, "plan");
        need(d_in, "d_in");
        need(d_out, "d_out");
        need(events, "events");
        const FftPlan& p = *plan->plan;
        if (nevents != p.launches())
            fg::invalid("fg_fft_exec_events: need " + std::to_string(p.launches()) + " events, got " +
                        std::to_string(nevents));
        std::vector<hipEvent_t> evs((size_t)nevents);
        for (int i = 0; i < nevents; ++i) {
            need(events[i], "event");
            evs[i] = events[i]->ev;
        }
        p.exec(d_in, d_out, parse_dir(direction), normalize != 0, (hipStream_t)stream, evs.data());
    });
}

int fg_fft_graph_create(fg_fft_plan_t plan, const void* d_in, void* d_out, int direction, int normalize,
                        int reps, fg_graph_t* out) {
    return guarded([&] {
        need(plan, "plan");
        need(d_in, "d_in");
        need(d_out, "d_out");
        need(out, "out");
        *out = nullptr;
        const FftPlan& p = *plan->plan;
        const Direction dir = parse_dir(direction);
        if (reps < 1 || (int64_t)reps * p.launches() > 65536)
            fg::invalid("fg_fft_graph_create: reps must be in [1, " + std::to_string(65536 / p.launches()) +
                        "], got " + std::to_string(reps));
        std::unique_ptr<fg_graph> g(new fg_graph);
        g->g = HipBackend::capture(plan->dev->dev->handle(), [&](hipStream_t s) {
            for (int r = 0; r < reps; ++r) p.exec(d_in, d_out, dir, normalize != 0, s);
        });
        g->dev = plan->dev;
        g->plan = plan;
        plan->graphs.fetch_add(1);
        *out = g.release();
    });
}

int fg_graph_capture_begin(fg_device_t dev, fg_stream_t* capture_stream) {
    return guarded([&] {
        need(dev, "device");
        need(capture_stream, "capture_stream");
        *capture_stream = (fg_stream_t)HipBackend::begin_capture(dev->dev->handle());
    });
}

int fg_graph_capture_end(fg_device_t dev, fg_stream_t capture_stream, fg_graph_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = nullptr;
        std::unique_ptr<fg_graph> g(new fg_graph);
        g->g = HipBackend::end_capture(dev->dev->handle(), (hipStream_t)capture_stream);
        g->dev = dev;
        dev->dependents.fetch_add(1);
        *out = g.release();
    });
}

int fg_graph_launch(fg_graph_t graph, fg_stream_t stream) {
    return guarded([&] {
        need(graph, "graph");
        HipBackend::launch_graph(graph->dev->dev->handle(), graph->g, (hipStream_t)stream);
    });
}

int fg_graph_node_count(fg_graph_t graph, size_t* nodes) {
    return guarded([&] {
        need(graph, "graph");
        need(nodes, "nodes");
        *nodes = graph->g->nodes;
    });
}

int fg_graph_destroy(fg_graph_t graph) {
    return guarded([&] {
        if (!graph) return;
        if (graph->plan)
            graph->plan->graphs.fetch_sub(1);  // the plan holds the device
        else
            graph->dev->dependents.fetch_sub(1);
        delete graph;
    });
}

static int plan_kernel(fg_fft_plan_t plan, int index, char* name, size_t cap, bool in_place) {
    return guarded([&] {
        need(plan, "plan");
        need(name, "name");
        auto names = plan->plan->kernel_names(in_place);
        if (index < 0 || (size_t)index >= names.size()) fg::invalid("launch index out of range");
        if (cap) {
            strncpy(name, names[index].c_str(), cap - 1);
            name[cap - 1] = 0;
        }
    });
}

int fg_fft_plan_kernel(fg_fft_plan_t plan, int index, char* name, size_t cap) {
    return plan_kernel(plan, index, name, cap, false);
}

int fg_fft_plan_kernel_in_place(fg_fft_plan_t plan, int index, char* name, size_t cap) {
    return plan_kernel(plan, index, name, cap, true);
}

int fg_fft_set_chunk_bytes(size_t bytes) {
    return guarded([&] { fg::set_chunk_limit_bytes(bytes); });
}

int fg_fft_get_chunk_bytes(size_t* bytes) {
    return guarded([&] {
        need(bytes, "bytes");
        *bytes = fg::chunk_limit_bytes();
    });
}

int fg_fft_plan_chunking(fg_fft_plan_t plan, int* passes, size_t* units_per_chunk, int* chunks, int* cached) {
    return guarded([&] {
        need(plan, "plan");
        const FftPlan& p = *plan->plan;
        if (passes) *passes = p.passes();
        if (units_per_chunk) *units_per_chunk = p.chunk_units();
        if (chunks) *chunks = (int)p.chunks();
        if (cached) *cached = p.cache_resident() ? 1 : 0;
    });
}

int fg_fft_plan_streams(fg_fft_plan_t plan, int* streams) {
    return guarded([&] {
        need(plan, "plan");
        need(streams, "streams");
        *streams = plan->plan->streams();
    });
}

int fg_fft_plan_set_streams(fg_fft_plan_t plan, int streams) {
    return guarded([&] {
        need(plan, "plan");
        plan->plan->set_streams(streams);
    });
}

int fg_fft_plan_describe(fg_fft_plan_t plan, int* launches, char* main_kernel, size_t cap,
                         size_t* workspace_bytes) {
    return guarded([&] {
        need(plan, "plan");
        if (launches) *launches = plan->plan->launches();
        if (main_kernel && cap) {
            strncpy(main_kernel, plan->plan->main_kernel().c_str(), cap - 1);
            main_kernel[cap - 1] = 0;
        }
        if (workspace_bytes) *workspace_bytes = plan->plan->workspace_bytes();
    });
}

int fg_fft_1d_c2c_pow2_host(fg_device_t dev, const float* in, float* out, size_t total_complex, uint32_t log_n,
                            int direction, int normalize) {
    return guarded([&] {
        // Argument checks and messages of crates/ferrum-gpu-py/src/lib.rs:455-477,
        // with the log_n range widened to the two-pass limit.
        if (log_n < fg::kMinLogN1D || log_n > fg::kMaxLogN1D)
            fg::invalid("log_n must be in [" + std::to_string(fg::kMinLogN1D) + ", " +
                        std::to_string(fg::kMaxLogN1D) + "], got " + std::to_string(log_n));
        const size_t n = size_t(1) << log_n;
        if (total_complex == 0 || total_complex % n != 0)
            fg::invalid("arr len " + std::to_string(total_complex) + " must be a positive multiple of N = " +
                        std::to_string(n));
        Direction dir = parse_dir(direction);
        need(in, "in");
        need(out, "out");
        fg_device* d = dev ? dev : default_device();
        run_host(d, 1, log_n, 0, total_complex / n, total_complex, in, out, dir, normalize != 0);
    });
}

int fg_fft_2d_c2c_pow2_host(fg_device_t dev, const float* in, float* out, uint32_t log_n, size_t batch,
                            int direction, int normalize) {
    return guarded([&] {
        // crates/ferrum-gpu-py/src/lib.rs:537-541
        if (log_n < fg::kMinLogN2D || log_n > fg::kMaxLogN2D)
            fg::invalid("2D requires log_n in [" + std::to_string(fg::kMinLogN2D) + ", " +
                        std::to_string(fg::kMaxLogN2D) + "]; got " + std::to_string(log_n));
        if (batch == 0) fg::invalid("batch must be positive");
        const size_t total = host_2d_elems(2 * log_n, batch);
        Direction dir = parse_dir(direction);
        need(in, "in");
        need(out, "out");
        fg_device* d = dev ? dev : default_device();
        run_host(d, 2, log_n, log_n, batch, total, in, out, dir, normalize != 0);
    });
}

int fg_fft_2d_rect_host(fg_device_t dev, const float* in, float* out, uint32_t log_rows, uint32_t log_cols,
                        size_t batch, int direction, int normalize) {
    return guarded([&] {
        for (uint32_t l : {log_rows, log_cols})
            if (l < fg::kMinLogN2D || l > fg::kMaxLogN2D)
                fg::invalid("2D requires log_n in [" + std::to_string(fg::kMinLogN2D) + ", " +
                            std::to_string(fg::kMaxLogN2D) + "]; got " + std::to_string(l));
        if (batch == 0) fg::invalid("batch must be positive");
        const size_t total = host_2d_elems(log_rows + log_cols, batch);
        Direction dir = parse_dir(direction);
        need(in, "in");
        need(out, "out");
        fg_device* d = dev ? dev : default_device();
        run_host(d, 2, log_cols, log_rows, batch, total, in, out, dir, normalize != 0);
    });
}

int fg_fft_plan_2d_rect(fg_device_t dev, uint32_t log_rows, uint32_t log_cols, size_t batch, fg_fft_plan_t* out) {
    return guarded([&] {
        need(dev, "device");
        need(out, "out");
        *out = nullptr;
        std::unique_ptr<fg_fft_plan> p(new fg_fft_plan);
        p->dev = dev;
        p->plan = FftPlan::make_2d(*dev->dev, dev->fft_module, log_rows, log_cols, batch);
        dev->dependents.fetch_add(1);
        *out = p.release();
    });
}

int fg_transpose_c64(fg_device_t dev, const void* d_in, void* d_out, uint32_t rows, uint32_t cols, size_t batch,
                     fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.transpose_c64(dev->dev->handle(), d_in, d_out, rows, cols, batch, (hipStream_t)stream);
    });
}

int fg_cmul_c64(fg_device_t dev, const void* a, const void* b, void* out, size_t n, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.cmul_c64(dev->dev->handle(), a, b, out, n, (hipStream_t)stream);
    });
}

int fg_cmul_split(fg_device_t dev, const void* a_re, const void* a_im, const void* b_re, const void* b_im,
                  void* o_re, void* o_im, size_t n, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.cmul_split(dev->dev->handle(), a_re, a_im, b_re, b_im, o_re, o_im, n, (hipStream_t)stream);
    });
}

int fg_deinterleave_c64(fg_device_t dev, const void* in, void* re, void* im, size_t n, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.deinterleave(dev->dev->handle(), in, re, im, n, (hipStream_t)stream);
    });
}

int fg_interleave_c64(fg_device_t dev, const void* re, const void* im, void* out, size_t n, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.interleave(dev->dev->handle(), re, im, out, n, (hipStream_t)stream);
    });
}

int fg_fill_uniform_c64(fg_device_t dev, void* d_out, size_t n, uint64_t seed, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.fill_c64(dev->dev->handle(), d_out, n, seed, false, (hipStream_t)stream);
    });
}

int fg_fill_normal_c64(fg_device_t dev, void* d_out, size_t n, uint64_t seed, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        dev->pointwise.fill_c64(dev->dev->handle(), d_out, n, seed, true, (hipStream_t)stream);
    });
}

int fg_stream_copy(fg_device_t dev, const void* d_in, void* d_out, size_t bytes, fg_stream_t stream) {
    return guarded([&] {
        need(dev, "device");
        need(d_in, "d_in");
        need(d_out, "d_out");
        dev->pointwise.stream_copy(dev->dev->handle(), d_in, d_out, bytes, (hipStream_t)stream);
    });
}

}  // extern "C"
