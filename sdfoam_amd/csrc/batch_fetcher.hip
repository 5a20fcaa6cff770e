// Host-side batch prefetcher: the training loop's input step
// (src/utils/batch_fetcher.cpp:29-157 and torch_bindings/torch_bindings.cpp:
// 32-63 in the reference).  A worker thread gathers batches of rows of a
// host array (random rows with the reference's per-element seeding, or
// consecutive rows) into pinned staging buffers with a few helper threads,
// uploads each into a slot of a caller-allocated device ring on its own
// stream, and hands slots over in order.  next() makes the caller's stream
// wait for the slot's upload, copies the slot into the caller's buffer on
// that stream, and releases the slot once that copy has run.  The library
// allocates no device memory; the staging buffers are pinned host memory.
#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "trace_kernels.h"

using namespace sdfoam_hip;

namespace {

constexpr int kSlots = 4;

// 32-bit integer hash of the reference's RNG (src/utils/random.h:11-20; the
// "triple32" construction of C. Wellons' hash-prospector) and its seeding
// (src/utils/random.h:27-29).
__host__ __device__ inline uint32_t mix32(uint32_t x) {
    x ^= x >> 17;
    x *= 0xed5ad4bbu;
    x ^= x >> 11;
    x *= 0xac4c1b51u;
    x ^= x >> 15;
    x *= 0x31848babu;
    x ^= x >> 14;
    return x;
}

// Row of element j of batch b (src/utils/batch_fetcher.cpp:63-72): with
// shuffle, the first draw of an RNG seeded with b * batch_size + j, scaled to
// [0, n) as randint(rng, 0, n) does (src/utils/random.h:49-56); otherwise
// the rows in order, wrapping around.
__host__ __device__ inline uint32_t row_of(uint32_t b, size_t batch_size, size_t j, size_t n,
                                           bool shuffle) {
    const size_t k = (size_t)b * batch_size + j;
    if (!shuffle) return (uint32_t)(k % n);
    const uint32_t draw = mix32((uint32_t)k ^ 0x2815db5bu);
    const uint32_t diff = (uint32_t)n;
    const uint32_t x = draw / (0xffffffffu / diff);
    return x < diff - 1u ? x : diff - 1u;
}

// One thread per 32-bit word of the batch: word w of element j is word w of
// row row_of(b, ., j, .) of the device-resident array.
__global__ __launch_bounds__(256) void batch_gather_kernel(const uint32_t *__restrict__ data,
                                                           size_t num_rows, uint32_t row_words,
                                                           uint32_t b, uint64_t batch_size,
                                                           bool shuffle,
                                                           uint32_t *__restrict__ dst) {
    const uint64_t t = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (t >= batch_size * row_words) return;
    const uint64_t j = t / row_words;
    const uint32_t w = (uint32_t)(t - j * row_words);
    const uint32_t row = row_of(b, (size_t)batch_size, (size_t)j, num_rows, shuffle);
    dst[t] = data[(uint64_t)row * row_words + w];
}

struct Slot {
    void *pinned = nullptr;
    hipEvent_t uploaded = nullptr; // recorded on the worker stream after the upload
    bool uploaded_pending = false; // `uploaded` was recorded (worker thread only)
    hipEvent_t consumed = nullptr; // recorded on the caller's stream after its copy
    bool consumed_pending = false; // `consumed` was recorded and not yet waited for
    bool released = true;          // the worker may refill it
};

} // namespace

struct sdf_batch_fetcher {
    const uint8_t *data = nullptr;
    size_t num_rows = 0, stride = 0, batch_size = 0, batch_bytes = 0;
    bool shuffle = false;
    uint8_t *ring = nullptr;
    int device = 0;
    uint32_t threads = 1;
    hipStream_t stream = nullptr;
    Slot slots[kSlots];

    std::mutex mu;
    std::condition_variable cv;
    std::deque<int> ready;
    bool stop = false;
    std::string error; // worker failure, reported by next()
    std::thread worker;

    void gather(int s, uint32_t b) {
        uint8_t *dst = static_cast<uint8_t *>(slots[s].pinned);
        auto part = [&](size_t lo, size_t hi) {
            for (size_t j = lo; j < hi; ++j) {
                const uint32_t r = row_of(b, batch_size, j, num_rows, shuffle);
                std::memcpy(dst + j * stride, data + (size_t)r * stride, stride);
            }
        };
        const uint32_t t = (uint32_t)std::min<size_t>(threads, std::max<size_t>(1, batch_size / 4096));
        if (t <= 1) {
            part(0, batch_size);
            return;
        }
        std::vector<std::thread> pool;
        const size_t chunk = (batch_size + t - 1) / t;
        for (uint32_t i = 1; i < t; ++i) {
            const size_t lo = i * chunk, hi = std::min(batch_size, lo + chunk);
            if (lo < hi) pool.emplace_back(part, lo, hi);
        }
        part(0, std::min(batch_size, chunk));
        for (auto &th : pool) th.join();
    }

    void run() {
        hipError_t e = hipSetDevice(device);
        uint32_t b = 0;
        for (int s = 0; e == hipSuccess; s = (s + 1) % kSlots, ++b) {
            {
                std::unique_lock<std::mutex> lk(mu);
                cv.wait(lk, [&] { return stop || slots[s].released; });
                if (stop) return;
                slots[s].released = false;
            }
            // the previous upload out of this staging buffer has finished
            if (slots[s].uploaded_pending) {
                e = hipEventSynchronize(slots[s].uploaded);
                if (e != hipSuccess) break;
            }
            gather(s, b);
            // the caller's copy out of this ring slot has run
            if (slots[s].consumed_pending) {
                e = hipEventSynchronize(slots[s].consumed);
                if (e != hipSuccess) break;
                slots[s].consumed_pending = false;
            }
            e = hipMemcpyAsync(ring + (size_t)s * batch_bytes, slots[s].pinned, batch_bytes,
                               hipMemcpyHostToDevice, stream);
            if (e != hipSuccess) break;
            e = hipEventRecord(slots[s].uploaded, stream);
            if (e != hipSuccess) break;
            slots[s].uploaded_pending = true;
            {
                std::lock_guard<std::mutex> lk(mu);
                ready.push_back(s);
            }
            cv.notify_all();
        }
        std::lock_guard<std::mutex> lk(mu);
        error = std::string("batch fetcher worker: ") + hipGetErrorString(e);
        cv.notify_all();
    }

    void release_all() {
        for (auto &sl : slots) {
            if (sl.uploaded) (void)hipEventDestroy(sl.uploaded);
            if (sl.consumed) (void)hipEventDestroy(sl.consumed);
            if (sl.pinned) (void)hipHostFree(sl.pinned);
        }
        if (stream) (void)hipStreamDestroy(stream);
    }
};

extern "C" {

size_t sdf_batch_fetcher_ring_bytes(size_t stride, size_t batch_size) {
    return (size_t)kSlots * stride * batch_size;
}

void sdf_batch_rows(uint32_t batch_index, size_t batch_size, size_t num_rows, int shuffle,
                    uint32_t *rows) {
    if (!rows || num_rows == 0) return;
    for (size_t j = 0; j < batch_size; ++j)
        rows[j] = row_of(batch_index, batch_size, j, num_rows, shuffle != 0);
}

int sdf_batch_gather(const void *data, size_t num_rows, size_t stride, uint32_t batch_index,
                     size_t batch_size, int shuffle, void *dst, void *stream) {
    if (batch_size == 0) return SDF_OK;
    if (!data || !dst) return fail(SDF_E_INVALID, "NULL pointer argument");
    if (num_rows == 0 || num_rows > 0xffffffffull)
        return fail(SDF_E_INVALID, "num_rows must be in [1, 2^32)");
    if (stride == 0 || stride % 4 != 0)
        return fail(SDF_E_INVALID, "stride must be a positive multiple of 4 bytes");
    if ((reinterpret_cast<uintptr_t>(data) | reinterpret_cast<uintptr_t>(dst)) & 3u)
        return fail(SDF_E_INVALID, "data and dst must be 4-byte aligned");
    const uint64_t words = (uint64_t)batch_size * (stride / 4);
    if (words > (1ull << 40)) return fail(SDF_E_INVALID, "batch too large");
    hipLaunchKernelGGL(batch_gather_kernel, dim3((unsigned)((words + 255u) / 256u)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const uint32_t *>(data),
                       num_rows, (uint32_t)(stride / 4), batch_index, (uint64_t)batch_size,
                       shuffle != 0, static_cast<uint32_t *>(dst));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, "batch_gather");
    return SDF_OK;
}

int sdf_batch_fetcher_create(const void *data, size_t num_bytes, size_t stride,
                             size_t batch_size, int shuffle, void *device_ring,
                             size_t device_ring_bytes, uint32_t num_threads,
                             sdf_batch_fetcher **out) {
    if (!out) return fail(SDF_E_INVALID, "out must not be NULL");
    *out = nullptr;
    if (!data || stride == 0 || num_bytes < stride)
        return fail(SDF_E_INVALID, "data must hold at least one row of `stride` bytes");
    if (batch_size == 0) return fail(SDF_E_INVALID, "batch_size must be positive");
    const size_t rows = num_bytes / stride;
    if (rows > 0xffffffffull) return fail(SDF_E_INVALID, "Too many elements");
    if (!device_ring || device_ring_bytes < sdf_batch_fetcher_ring_bytes(stride, batch_size))
        return fail(SDF_E_INVALID, "device_ring must hold %zu bytes",
                    sdf_batch_fetcher_ring_bytes(stride, batch_size));
    auto *f = new sdf_batch_fetcher();
    f->data = static_cast<const uint8_t *>(data);
    f->num_rows = rows;
    f->stride = stride;
    f->batch_size = batch_size;
    f->batch_bytes = stride * batch_size;
    f->shuffle = shuffle != 0;
    f->ring = static_cast<uint8_t *>(device_ring);
    f->threads = std::max(1u, std::min(num_threads ? num_threads : 8u, 64u));
    hipError_t e = hipGetDevice(&f->device);
    if (e == hipSuccess) e = hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking);
    for (int s = 0; s < kSlots && e == hipSuccess; ++s) {
        e = hipHostMalloc(&f->slots[s].pinned, f->batch_bytes, hipHostMallocDefault);
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&f->slots[s].uploaded, hipEventDisableTiming);
        if (e == hipSuccess)
            e = hipEventCreateWithFlags(&f->slots[s].consumed, hipEventDisableTiming);
    }
    if (e != hipSuccess) {
        f->release_all();
        delete f;
        return hip_fail(e, "batch fetcher set-up");
    }
    f->worker = std::thread([f] { f->run(); });
    *out = f;
    return SDF_OK;
}

int sdf_batch_fetcher_next(sdf_batch_fetcher *f, void *dst, void *stream) {
    if (!f || !dst) return fail(SDF_E_INVALID, "NULL pointer argument");
    int s;
    {
        std::unique_lock<std::mutex> lk(f->mu);
        f->cv.wait(lk, [&] { return !f->ready.empty() || !f->error.empty(); });
        if (f->ready.empty()) return fail(SDF_E_HIP, "%s", f->error.c_str());
        s = f->ready.front();
        f->ready.pop_front();
    }
    hipStream_t cs = static_cast<hipStream_t>(stream);
    Slot &sl = f->slots[s];
    hipError_t e = hipStreamWaitEvent(cs, sl.uploaded, 0);
    if (e == hipSuccess)
        e = hipMemcpyAsync(dst, f->ring + (size_t)s * f->batch_bytes, f->batch_bytes,
                           hipMemcpyDeviceToDevice, cs);
    if (e == hipSuccess) e = hipEventRecord(sl.consumed, cs);
    {
        std::lock_guard<std::mutex> lk(f->mu);
        sl.consumed_pending = e == hipSuccess;
        sl.released = true;
    }
    f->cv.notify_all();
    if (e != hipSuccess) return hip_fail(e, "batch fetcher next");
    return SDF_OK;
}

int sdf_batch_fetcher_destroy(sdf_batch_fetcher *f) {
    if (!f) return SDF_OK;
    {
        std::lock_guard<std::mutex> lk(f->mu);
        f->stop = true;
    }
    f->cv.notify_all();
    if (f->worker.joinable()) f->worker.join();
    // uploads into the caller's ring must finish before the caller frees it,
    // and the caller's copies out of it before the events go
    hipError_t e = hipStreamSynchronize(f->stream);
    for (auto &sl : f->slots)
        if (sl.consumed_pending) (void)hipEventSynchronize(sl.consumed);
    f->release_all();
    delete f;
    if (e != hipSuccess) return hip_fail(e, "batch fetcher destroy");
    return SDF_OK;
}

} // extern "C"
