// fft_plan.cpp -- plan construction and stream-ordered execution.
#include "fft_plan.hpp"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include <fstream>
#include <iterator>

extern "C" {
// Embedded by embed.S (.incbin of the gfx950 code object).
extern const unsigned char fg_fft_code_object_start[];
extern const unsigned char fg_fft_code_object_end[];
}

namespace fg {

namespace {

// Launch geometry of the single-pass Stockham kernels, mirroring the
// FG_STOCKHAM(LOGN, LOGE, FPB) instantiations in kernels/fft_kernels.hip.
struct StockhamGeom {
    uint32_t log_e;  // log2 of elements per thread
    uint32_t fpb;    // transforms per workgroup
};
constexpr StockhamGeom kStockham[kMaxLogNSingle + 1] = {
    {0, 0}, {0, 0},          // log_n 0, 1: unsupported
    {2, 64}, {3, 64}, {4, 64}, {4, 32}, {4, 16}, {4, 8}, {4, 4}, {4, 2}, {4, 1}, {4, 1}, {4, 1},
};

std::string file_image;  // backing store when FERRUM_GPU_CODE_OBJECT is set

}  // namespace

KernelArtifact fft_code_object() {
    KernelArtifact a;
    a.backend = BackendId::Hip;
    a.name = "ferrum-gpu-fft-kernels";
    a.target = "gfx950";
    if (const char* path = getenv("FERRUM_GPU_CODE_OBJECT")) {
        if (file_image.empty()) {
            std::ifstream f(path, std::ios::binary);
            if (!f) invalid(std::string("FERRUM_GPU_CODE_OBJECT: cannot read ") + path);
            file_image.assign(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
        }
        a.image = file_image.data();
        a.size = file_image.size();
    } else {
        a.image = fg_fft_code_object_start;
        a.size = (size_t)(fg_fft_code_object_end - fg_fft_code_object_start);
    }
    return a;
}

std::vector<Cf32> stockham_twiddles(uint32_t log_n, uint32_t log_e) {
    const uint32_t nfull = log_n / log_e, rem = log_n % log_e;
    const uint32_t nstages = nfull + (rem ? 1 : 0);
    std::vector<Cf32> t;
    for (uint32_t s = 1; s < nstages; ++s) {
        const uint32_t logl = s * log_e;
        const uint32_t logr = (s < nfull) ? log_e : rem;
        const uint64_t L = 1ull << logl, R = 1ull << logr, M = L * R;
        for (uint64_t k = 0; k < L; ++k)
            for (uint64_t p = 0; p < R; ++p) {
                const uint64_t e = (p * k) % M;
                const double ang = 2.0 * M_PI * (double)e / (double)M;
                t.push_back(Cf32{(float)cos(ang), (float)-sin(ang)});
            }
    }
    if (t.empty()) t.push_back(Cf32{1.f, 0.f});  // single-stage sizes read no table
    return t;
}

std::unique_ptr<FftPlan> FftPlan::make_1d(HipDevice& dev, const HipBackend::Module& mod, uint32_t log_n,
                                          size_t batch) {
    if (log_n < kMinLogN1D || log_n > kMaxLogN1D)
        invalid("log_n must be in [" + std::to_string(kMinLogN1D) + ", " + std::to_string(kMaxLogN1D) +
                "], got " + std::to_string(log_n));
    if (batch == 0) invalid("batch must be positive");
    if (log_n > kMaxLogNSingle)
        fail(FG_ERR_INVALID_ARGUMENT, "log_n " + std::to_string(log_n) + " needs the two-pass path, not built");
    std::unique_ptr<FftPlan> p(new FftPlan(dev, Kind::Stockham1D, log_n, batch));
    const StockhamGeom g = kStockham[log_n];
    const uint32_t threads = (1u << log_n) >> g.log_e;
    auto tw = stockham_twiddles(log_n, g.log_e);
    p->tables_.push_back(dev.alloc<Cf32>(tw.size()));
    p->tables_.back().copy_from_host(tw.data(), tw.size());

    Step s;
    const std::string base = "fg_fft_n" + std::to_string(log_n);
    s.fwd = HipBackend::get_kernel(mod, (base + "_fwd").c_str());
    s.inv = HipBackend::get_kernel(mod, (base + "_inv").c_str());
    const uint64_t blocks = (batch + g.fpb - 1) / g.fpb;
    if (blocks > 0x7fffffffull) invalid("batch too large for one launch");
    s.grid = Dim3((uint32_t)blocks);
    s.block = Dim3(threads * g.fpb);
    s.src = Buf::In;
    s.dst = Buf::Out;
    s.tw = p->tables_.back().data();
    s.count = batch;
    s.scales = true;
    s.conj_in = true;
    p->steps_.push_back(s);
    p->main_kernel_ = base + "_fwd";
    return p;
}

std::unique_ptr<FftPlan> FftPlan::make_2d(HipDevice&, const HipBackend::Module&, uint32_t log_n, size_t batch) {
    if (log_n < kMinLogN2D || log_n > kMaxLogN2D)
        invalid("2D requires log_n in [" + std::to_string(kMinLogN2D) + ", " + std::to_string(kMaxLogN2D) +
                "]; got " + std::to_string(log_n));
    if (batch == 0) invalid("batch must be positive");
    fail(FG_ERR_INVALID_ARGUMENT, "2D path not built");
}

void FftPlan::exec(const void* in, void* out, Direction dir, bool normalize, hipStream_t stream) const {
    if (!in || !out) invalid("fft exec: null buffer");
    const bool inverse = dir == Direction::Inverse;
    const float scale = (inverse && normalize) ? 1.0f / (float)elems() : 1.0f;
    for (const Step& s : steps_) {
        auto bind = [&](Buf b) -> void* {
            switch (b) {
                case Buf::In: return const_cast<void*>(in);
                case Buf::Out: return out;
                default: return work_.data();
            }
        };
        void* src = bind(s.src);
        void* dst = bind(s.dst);
        const void* tw = s.tw;
        uint64_t count = s.count;
        float sc = s.scales ? scale : 1.0f;
        HipBackend::KernelHandle k = inverse ? s.inv : s.fwd;
        void* args[] = {&src, &dst, (void*)&tw, &count, &sc};
        HipBackend::launch(dev_->handle(), stream, k, s.grid, s.block, 0, args);
    }
}

}  // namespace fg
