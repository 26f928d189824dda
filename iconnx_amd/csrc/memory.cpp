// The memory half of the C ABI: what garboard and IconnxCudaContext / GpuMemoryPool give the
// reference's per-op wrappers (src/cuda/context.rs, src/cuda/memory_pool.rs), on the HIP
// runtime.  Host code only.
//
//   icx_stream_create / _destroy / _synchronize   the context's one stream (context.rs:28-31,
//                                                 sync :226-232); default priority
//   icx_pool_*                                    GpuMemoryPool (memory_pool.rs:47-545)
//   icx_memcpy_h2d_async / _d2h_async             htod / dtoh (context.rs:160-223), both
//                                                 enqueued on the stream
//   icx_host_alloc / _free                        pinned host buffers, so the copies above
//                                                 run asynchronously
//
// The pool keeps the reference's policy — a size class per request, at most eight free
// buffers kept per class, a returned buffer beyond that freed — with two differences: classes
// are bytes (powers of two from 256 B) rather than elements per dtype, and a reused buffer is
// not zero-filled (memory_pool.rs:120 clears every reused slice; every kernel of this library
// writes its whole output).  Buffers are reused in stream order: a caller returns a buffer
// once the last work that reads it is enqueued on the stream that will next use it, which the
// reference's single stream gives by construction.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <new>
#include <unordered_map>
#include <vector>

#include "icx_common.hpp"

struct icx_pool {
    std::map<size_t, std::vector<void*>> free_;  // size class -> free buffers
    std::unordered_map<void*, size_t> live_;     // buffers handed out -> size class
    int64_t hits = 0, misses = 0, held = 0;
    static constexpr size_t kMaxPerClass = 8;  // max_per_bucket, memory_pool.rs:94
};

namespace {
// The largest size class, 2^63 bytes: a request above it has no power-of-two class (the
// doubling would wrap to 0), e.g. (size_t)-1 from a bad size computation.
constexpr size_t kMaxClass = (SIZE_MAX >> 1) + 1;

size_t size_class(size_t bytes) {
    size_t c = 256;
    while (c < bytes) c <<= 1;
    return c;
}
}  // namespace

extern "C" int icx_stream_create(icx_stream_t* out) {
    icx::clear_error();
    if (!out) ICX_FAIL(ICX_ERR_INVALID_ARG, "stream_create: null output");
    hipStream_t s = nullptr;
    ICX_HIP_CHECK(hipStreamCreate(&s));
    *out = reinterpret_cast<icx_stream_t>(s);
    return ICX_OK;
}

extern "C" int icx_stream_destroy(icx_stream_t stream) {
    icx::clear_error();
    if (!stream) return ICX_OK;
    ICX_HIP_CHECK(hipStreamDestroy(reinterpret_cast<hipStream_t>(stream)));
    return ICX_OK;
}

extern "C" int icx_stream_synchronize(icx_stream_t stream) {
    icx::clear_error();
    ICX_HIP_CHECK(hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)));
    return ICX_OK;
}

extern "C" icx_pool* icx_pool_create(void) { return new (std::nothrow) icx_pool(); }

extern "C" void icx_pool_destroy(icx_pool* p) {
    if (!p) return;
    for (auto& kv : p->free_)
        for (void* b : kv.second) (void)hipFree(b);
    for (auto& kv : p->live_) (void)hipFree(kv.first);
    delete p;
}

extern "C" int icx_pool_alloc(icx_pool* p, size_t bytes, void** out) {
    icx::clear_error();
    if (!p || !out) ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_alloc: null pool or output");
    *out = nullptr;
    if (bytes > kMaxClass) ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_alloc: %zu bytes exceeds the largest size class", bytes);
    const size_t c = size_class(bytes);
    auto it = p->free_.find(c);
    if (it != p->free_.end() && !it->second.empty()) {
        void* b = it->second.back();
        it->second.pop_back();
        p->live_[b] = c;
        ++p->hits;
        *out = b;
        return ICX_OK;
    }
    void* b = nullptr;
    ICX_HIP_CHECK(hipMalloc(&b, c));
    ++p->misses;
    p->held += (int64_t)c;
    p->live_[b] = c;
    *out = b;
    return ICX_OK;
}

extern "C" int icx_pool_free(icx_pool* p, void* ptr) {
    icx::clear_error();
    if (!p) ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_free: null pool");
    if (!ptr) return ICX_OK;
    auto it = p->live_.find(ptr);
    if (it == p->live_.end())
        ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_free: %p was not handed out by this pool (or was returned already)",
                 ptr);
    const size_t c = it->second;
    p->live_.erase(it);
    auto& fl = p->free_[c];
    if (fl.size() < icx_pool::kMaxPerClass) {
        fl.push_back(ptr);
        return ICX_OK;
    }
    p->held -= (int64_t)c;  // class full: freed, as the reference drops the slice
    ICX_HIP_CHECK(hipFree(ptr));
    return ICX_OK;
}

extern "C" int icx_pool_stats(icx_pool* p, int64_t* hits, int64_t* misses, int64_t* bytes_held) {
    icx::clear_error();
    if (!p) ICX_FAIL(ICX_ERR_INVALID_ARG, "pool_stats: null pool");
    if (hits) *hits = p->hits;
    if (misses) *misses = p->misses;
    if (bytes_held) *bytes_held = p->held;
    return ICX_OK;
}

extern "C" int icx_host_alloc(size_t bytes, void** out) {
    icx::clear_error();
    if (!out) ICX_FAIL(ICX_ERR_INVALID_ARG, "host_alloc: null output");
    *out = nullptr;
    ICX_HIP_CHECK(hipHostMalloc(out, bytes ? bytes : 1, hipHostMallocDefault));
    return ICX_OK;
}

extern "C" int icx_host_free(void* ptr) {
    icx::clear_error();
    if (ptr) ICX_HIP_CHECK(hipHostFree(ptr));
    return ICX_OK;
}

extern "C" int icx_memcpy_h2d_async(icx_stream_t stream, void* dst, const void* src, size_t bytes) {
    icx::clear_error();
    if (!bytes) return ICX_OK;
    if (!dst || !src) ICX_FAIL(ICX_ERR_INVALID_ARG, "memcpy_h2d_async: null pointer");
    ICX_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, reinterpret_cast<hipStream_t>(stream)));
    return ICX_OK;
}

extern "C" int icx_memcpy_d2h_async(icx_stream_t stream, void* dst, const void* src, size_t bytes) {
    icx::clear_error();
    if (!bytes) return ICX_OK;
    if (!dst || !src) ICX_FAIL(ICX_ERR_INVALID_ARG, "memcpy_d2h_async: null pointer");
    ICX_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, reinterpret_cast<hipStream_t>(stream)));
    return ICX_OK;
}
