// pointwise_ops.cpp -- see pointwise_ops.hpp.
#include "pointwise_ops.hpp"

#include <algorithm>

#include <initializer_list>
#include <string>

namespace fg {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint64_t kMaxBlocks = 1u << 16;  // 16.8 M threads; the kernels stride over the rest

bool aligned16(std::initializer_list<const void*> ps) {
    for (const void* p : ps)
        if (reinterpret_cast<uintptr_t>(p) & 15u) return false;
    return true;
}

void need_ptrs(const char* op, std::initializer_list<const void*> ps) {
    for (const void* p : ps)
        if (!p) invalid(std::string(op) + ": null buffer");
}

// Input and output ranges of n complex (8n bytes) or n floats (4n bytes) must
// be identical or disjoint where the kernel reads one array and writes another
// with a different stride.
bool overlap(const void* a, uint64_t abytes, const void* b, uint64_t bbytes) {
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bbytes && y < x + abytes;
}

void launch(const HipBackend::DeviceHandle& dev, hipStream_t stream, HipBackend::KernelHandle k, uint64_t n,
            int width, void** args) {
    const uint64_t chunks = (n + width - 1) / width;
    uint64_t blocks = (chunks + kThreads - 1) / kThreads;
    if (blocks > kMaxBlocks) blocks = kMaxBlocks;
    HipBackend::launch(dev, stream, k, Dim3((uint32_t)blocks), Dim3(kThreads), 0, args);
}

}  // namespace

Pointwise::Pointwise(const HipBackend::Module& mod) {
    for (int v = 0; v < 2; ++v) {
        const std::string w = v ? "_vec" : "_elem";
        cmul_c64_[v] = HipBackend::get_kernel(mod, ("fg_cmul_c64" + w).c_str());
        cmul_split_[v] = HipBackend::get_kernel(mod, ("fg_cmul_split" + w).c_str());
        deinterleave_[v] = HipBackend::get_kernel(mod, ("fg_deinterleave_c64" + w).c_str());
        interleave_[v] = HipBackend::get_kernel(mod, ("fg_interleave_c64" + w).c_str());
    }
    fill_ = HipBackend::get_kernel(mod, "fg_fill_c64");
    transpose_ = HipBackend::get_kernel(mod, "fg_transpose_c64");
    transpose128_ = HipBackend::get_kernel(mod, "fg_transpose_c64_t128");
    copy_ = HipBackend::get_kernel(mod, "fg_copy_f4");
}

void Pointwise::cmul_c64(const HipBackend::DeviceHandle& dev, const void* a, const void* b, void* out, uint64_t n,
                         hipStream_t stream) const {
    if (n == 0) return;
    need_ptrs("cmul_c64", {a, b, out});
    // Element i of out depends only on element i of a and b: out may be a or b,
    // but must not overlap either at another offset.
    for (const void* x : {a, b})
        if (x != out && overlap(out, 8 * n, x, 8 * n)) invalid("cmul_c64: out partially overlaps an input");
    const int v = aligned16({a, b, out}) ? 1 : 0;
    void* args[] = {(void*)&a, (void*)&b, &out, &n};
    launch(dev, stream, cmul_c64_[v], n, v ? 2 : 1, args);
}

void Pointwise::cmul_split(const HipBackend::DeviceHandle& dev, const void* a_re, const void* a_im,
                           const void* b_re, const void* b_im, void* o_re, void* o_im, uint64_t n,
                           hipStream_t stream) const {
    if (n == 0) return;
    need_ptrs("cmul_split", {a_re, a_im, b_re, b_im, o_re, o_im});
    const uint64_t nb = 4 * n;
    // Element i of the outputs depends only on element i of the inputs, so
    // o_re may be a_re or b_re and o_im may be a_im or b_im; any other overlap
    // of an output with an input or with the other output is rejected.
    for (const void* x : {a_re, b_re, a_im, b_im}) {
        const bool same_part_re = x == a_re || x == b_re;
        if (!(same_part_re && x == o_re) && overlap(o_re, nb, x, nb))
            invalid("cmul_split: o_re overlaps an input other than a_re / b_re");
        if (!(!same_part_re && x == o_im) && overlap(o_im, nb, x, nb))
            invalid("cmul_split: o_im overlaps an input other than a_im / b_im");
    }
    if (overlap(o_re, nb, o_im, nb)) invalid("cmul_split: o_re and o_im overlap");
    const int v = aligned16({a_re, a_im, b_re, b_im, o_re, o_im}) ? 1 : 0;
    void* args[] = {(void*)&a_re, (void*)&a_im, (void*)&b_re, (void*)&b_im, &o_re, &o_im, &n};
    launch(dev, stream, cmul_split_[v], n, v ? 4 : 1, args);
}

void Pointwise::deinterleave(const HipBackend::DeviceHandle& dev, const void* in, void* re, void* im, uint64_t n,
                             hipStream_t stream) const {
    if (n == 0) return;
    need_ptrs("deinterleave", {in, re, im});
    if (overlap(in, 8 * n, re, 4 * n) || overlap(in, 8 * n, im, 4 * n) || overlap(re, 4 * n, im, 4 * n))
        invalid("deinterleave: buffers overlap");
    const int v = aligned16({in, re, im}) ? 1 : 0;
    void* args[] = {(void*)&in, &re, &im, &n};
    launch(dev, stream, deinterleave_[v], n, v ? 2 : 1, args);
}

void Pointwise::interleave(const HipBackend::DeviceHandle& dev, const void* re, const void* im, void* out,
                           uint64_t n, hipStream_t stream) const {
    if (n == 0) return;
    need_ptrs("interleave", {re, im, out});
    if (overlap(out, 8 * n, re, 4 * n) || overlap(out, 8 * n, im, 4 * n)) invalid("interleave: buffers overlap");
    const int v = aligned16({re, im, out}) ? 1 : 0;
    void* args[] = {(void*)&re, (void*)&im, &out, &n};
    launch(dev, stream, interleave_[v], n, v ? 2 : 1, args);
}

void Pointwise::fill_c64(const HipBackend::DeviceHandle& dev, void* out, uint64_t n, uint64_t seed, bool normal,
                         hipStream_t stream) const {
    if (n == 0) return;
    need_ptrs("fill_c64", {out});
    if (reinterpret_cast<uintptr_t>(out) & 7u) invalid("fill_c64: out must be 8-byte aligned (complex64)");
    uint32_t nrm = normal ? 1u : 0u;
    void* args[] = {&out, &n, &seed, &nrm};
    launch(dev, stream, fill_, n, 1, args);
}

void Pointwise::transpose_c64(const HipBackend::DeviceHandle& dev, const void* in, void* out, uint32_t rows,
                              uint32_t cols, uint64_t batch, hipStream_t stream) const {
    if (!in || !out) invalid("transpose: null buffer");
    if (rows == 0 || cols == 0 || batch == 0) invalid("transpose: rows, cols and batch must be positive");
    const uint64_t nb = 8ull * rows * cols * batch;
    if (overlap(in, nb, out, nb)) invalid("transpose: in and out must not overlap");
    if (rows >= 128 && cols >= 128) {
        // 128 x 128 tiles walked in super-tiles of up to 8 x 8 (fg_transpose_c64_t128)
        const uint32_t tc = (cols + 127) / 128, tr = (rows + 127) / 128;
        const uint32_t sc = std::min<uint32_t>(8, tc), sr = std::min<uint32_t>(8, tr);
        const uint32_t supers_c = (tc + sc - 1) / sc, supers_r = (tr + sr - 1) / sr;
        const uint64_t image_blocks = (uint64_t)supers_c * sc * supers_r * sr;
        if (image_blocks * batch > 0x7fffffffull) invalid("transpose: too many tiles for one launch");
        uint32_t ib = (uint32_t)image_blocks;
        void* args[] = {(void*)&in, &out, &rows, &cols, (void*)&tc, (void*)&tr, (void*)&sc, (void*)&sr,
                        (void*)&supers_c, &ib};
        HipBackend::launch(dev, stream, transpose128_, Dim3((uint32_t)(image_blocks * batch)), Dim3(1024), 0, args);
        return;
    }
    const uint32_t tc = (cols + 63) / 64, tr = (rows + 63) / 64;
    const uint64_t tiles = (uint64_t)tc * tr * batch;
    if (tiles > 0x7fffffffull) invalid("transpose: too many tiles for one launch");
    void* args[] = {(void*)&in, &out, &rows, &cols, (void*)&tc, (void*)&tr};
    HipBackend::launch(dev, stream, transpose_, Dim3((uint32_t)tiles), Dim3(256), 0, args);
}

void Pointwise::stream_copy(const HipBackend::DeviceHandle& dev, const void* in, void* out, uint64_t bytes,
                            hipStream_t stream) const {
    need_ptrs("stream_copy", {in, out});
    if (bytes % 16) invalid("fg_stream_copy: bytes must be a multiple of 16");
    if (!aligned16({in, out})) invalid("fg_stream_copy: d_in and d_out must be 16-byte aligned");
    uint64_t n4 = bytes / 16;
    const uint32_t block = 64;
    uint64_t blocks = (n4 + block - 1) / block;
    if (blocks > 0x7fffffffull) blocks = 0x7fffffffull;  // the kernel strides beyond this
    if (blocks == 0) return;
    void* args[] = {(void*)&in, &out, &n4};
    HipBackend::launch(dev, stream, copy_, Dim3((uint32_t)blocks), Dim3(block), 0, args);
}

}  // namespace fg
