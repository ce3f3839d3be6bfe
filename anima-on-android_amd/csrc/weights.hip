// Model weights from the reference's on-disk format, a safetensors file
// (scripts/phone_pipeline_nd.py:15-43 reads it; vulkan/safetensors_reader.h is
// the reference's C++ reader): u64 little-endian header length, a JSON header
// mapping tensor names to {dtype, shape, data_offsets} (plus an optional
// "__metadata__" object), then the raw tensor bytes.
//
// The file is memory-mapped read-only and the header parsed and validated
// (offsets inside the data region, byte counts matching dtype x shape).
// Tensors are uploaded on first request into device copies that stay
// resident until the handle is closed, so a denoise loop reads its weights
// from HBM only.  Like the reference, names are matched with or without the
// "net." prefix, linear weights stay bf16 bit patterns, and other weights
// can be widened to f32 (bf16 bits << 16, as phone_pipeline_nd.py:37-40 does).
#include "common.h"
#include "safetensors_header.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace anima_hip {
namespace {

using st::dtype_bytes;
using st::kBF16;
using st::kF16;
using st::kF32;

}  // namespace
}  // namespace anima_hip

using namespace anima_hip;

struct anima_hip_weights {
    struct Tensor {
        std::string name;  // as in the file
        int dtype = -1;
        std::vector<int64_t> shape;
        size_t begin = 0, bytes = 0;  // inside the data region
        void *dev[2] = {nullptr, nullptr};  // [as stored, as f32]
    };
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> index;  // file name and prefix-stripped name
    std::vector<std::string> short_names;
    const unsigned char *map = nullptr;
    size_t map_len = 0;
    size_t data_start = 0;
    int device = 0;
    std::mutex mu;

    ~anima_hip_weights()
    {
        for (auto &t : tensors)
            for (void *&p : t.dev)
                if (p)
                    (void)hipFree(p);
        if (map)
            munmap(const_cast<unsigned char *>(map), map_len);
    }
};

namespace {

constexpr const char *kPrefix = "net.";

std::string strip_prefix(const std::string &n)
{
    return n.compare(0, 4, kPrefix) == 0 ? n.substr(4) : n;
}

bool parse_header(anima_hip_weights &w, const char *p, const char *end, size_t data_len)
{
    std::vector<st::Entry> entries;
    std::string err;
    if (!st::parse_header(p, end, data_len, entries, err))
        return fail(err);
    for (st::Entry &e : entries) {
        anima_hip_weights::Tensor t;
        t.name = std::move(e.name);
        t.dtype = e.dtype;
        t.shape = std::move(e.shape);
        t.begin = e.begin;
        t.bytes = e.bytes;
        const size_t idx = w.tensors.size();
        w.index[t.name] = idx;
        w.index.emplace(strip_prefix(t.name), idx);
        w.tensors.push_back(std::move(t));
    }
    for (auto &t : w.tensors)
        w.short_names.push_back(strip_prefix(t.name));
    return true;
}

float half_to_float(uint16_t h)
{
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: normalise
            exp = 127 - 15 + 1;
            while (!(man & 0x400u)) {
                man <<= 1;
                --exp;
            }
            bits = sign | (exp << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

const anima_hip_weights::Tensor *find(const anima_hip_weights *w, const char *name)
{
    if (!w || !name)
        return nullptr;
    auto it = w->index.find(name);
    return it == w->index.end() ? nullptr : &w->tensors[it->second];
}

}  // namespace

extern "C" {

anima_hip_weights *anima_hip_weights_open(const char *path)
{
    if (!path) {
        fail("weights_open: null path");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        fail(std::string("weights_open: cannot open ") + path + ": " + std::strerror(errno));
        return nullptr;
    }
    struct stat stt;
    if (fstat(fd, &stt) != 0 || stt.st_size < 8) {
        close(fd);
        fail(std::string("weights_open: ") + path + " is too short for a safetensors file");
        return nullptr;
    }
    const size_t len = size_t(stt.st_size);
    void *m = mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        fail(std::string("weights_open: mmap failed: ") + std::strerror(errno));
        return nullptr;
    }
    std::unique_ptr<anima_hip_weights> w(new anima_hip_weights);
    w->map = static_cast<const unsigned char *>(m);
    w->map_len = len;
    uint64_t hl = 0;
    for (int i = 7; i >= 0; --i)
        hl = (hl << 8) | w->map[i];
    if (hl > len - 8) {
        fail("weights_open: header length " + std::to_string(hl) + " exceeds the file");
        return nullptr;
    }
    w->data_start = 8 + size_t(hl);
    const char *hp = reinterpret_cast<const char *>(w->map + 8);
    if (!parse_header(*w, hp, hp + hl, len - w->data_start))
        return nullptr;
    (void)hipGetDevice(&w->device);
    return w.release();
}

void anima_hip_weights_close(anima_hip_weights *w)
{
    if (!w)
        return;
    (void)hipDeviceSynchronize();  // copies may still be read by queued work
    delete w;
}

int anima_hip_weights_count(const anima_hip_weights *w)
{
    return w ? int(w->tensors.size()) : 0;
}

const char *anima_hip_weights_name(const anima_hip_weights *w, int i)
{
    if (!w || i < 0 || size_t(i) >= w->short_names.size())
        return nullptr;
    return w->short_names[size_t(i)].c_str();
}

int anima_hip_weights_info(const anima_hip_weights *w, const char *name, int *dtype,
                           int64_t *shape, int max_ndim)
{
    const anima_hip_weights::Tensor *t = find(w, name);
    if (!t) {
        fail(std::string("weights_info: no tensor named ") + (name ? name : "(null)"));
        return -1;
    }
    if (dtype)
        *dtype = t->dtype;
    for (int i = 0; shape && i < max_ndim && size_t(i) < t->shape.size(); ++i)
        shape[i] = t->shape[size_t(i)];
    return int(t->shape.size());
}

const void *anima_hip_weights_device(anima_hip_weights *w, const char *name, int as_f32)
{
    if (!w) {
        fail("weights_device: null handle");
        return nullptr;
    }
    std::lock_guard<std::mutex> g(w->mu);
    auto *t = const_cast<anima_hip_weights::Tensor *>(find(w, name));
    if (!t) {
        fail(std::string("weights_device: no tensor named ") + (name ? name : "(null)"));
        return nullptr;
    }
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice"))
        return nullptr;
    if (dev != w->device) {
        fail("weights_device: the handle was opened on another device");
        return nullptr;
    }
    const int slot = as_f32 ? 1 : 0;
    if (t->dev[slot])
        return t->dev[slot];
    const unsigned char *src = w->map + w->data_start + t->begin;
    const size_t n = t->bytes / size_t(dtype_bytes(t->dtype));
    std::vector<float> widened;
    const void *host = src;
    size_t bytes = t->bytes;
    if (as_f32 && t->dtype != kF32) {
        widened.resize(n);
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            std::memcpy(&h, src + 2 * i, 2);
            if (t->dtype == kBF16) {
                const uint32_t bits = uint32_t(h) << 16;
                std::memcpy(&widened[i], &bits, 4);
            } else {
                widened[i] = half_to_float(h);
            }
        }
        host = widened.data();
        bytes = n * sizeof(float);
    }
    void *d = nullptr;
    if (!hip_ok(hipMalloc(&d, bytes ? bytes : 4), "weights_device: hipMalloc") ||
        !hip_ok(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice), "weights_device: copy")) {
        if (d)
            (void)hipFree(d);
        return nullptr;
    }
    t->dev[slot] = d;
    return d;
}

}  // extern "C"
