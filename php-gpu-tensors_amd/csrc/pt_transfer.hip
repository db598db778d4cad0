// Host <-> device transfers of the C-ABI (pt_memcpy_h2d / pt_memcpy_d2h),
// replacing the cudaMemcpy calls of src/cuda_array/tensor_transfer.c:45-65
// and src/cuda_array/tensor_factory.c:301-326.
//
// The copy engines read and write only pinned host memory.  Handed a
// pageable buffer, hipMemcpy stages it through pinned memory with one host
// thread: 27.5 GB/s host to device and 16.9 GB/s device to host on MI355X,
// against 57 GB/s from pinned memory.  Large pageable transfers therefore go
// through this file's own ring of two pinned chunks: the host copies into
// (or out of) one chunk, split over PT_COPY_THREADS threads, while the DMA
// engine moves the other, so that the host copy (87 GB/s over four threads)
// hides behind the DMA.  Pinned, device and managed pointers and transfers
// below PT_STAGE_MIN_BYTES keep the single hipMemcpyAsync.  Both entry points
// return once the bytes have arrived, as the reference's cudaMemcpy does.
#include "pt_common.h"

#include <algorithm>
#include <condition_variable>
#include <mutex>
#include <string.h>
#include <thread>
#include <unistd.h>
#include <vector>

namespace pt {

#define PT_STAGE_MIN_BYTES ((size_t)4 << 20)
#define PT_STAGE_CHUNK_MAX ((size_t)16 << 20)
#define PT_STAGE_CHUNK_MIN ((size_t)1 << 20)
#define PT_COPY_THREADS 4

// Parallel host memcpy: the caller copies the first part, PT_COPY_THREADS - 1
// resident workers the others.  Workers start on first use and live until
// the process ends (the pool is never destroyed, so no exit-time destructor
// waits on them).  One copy runs at a time (the stager's lock).  A child
// made by fork() has no workers, only their record: it copies on the
// calling thread.
class CopyPool {
public:
    void copy(char *dst, const char *src, size_t n)
    {
        const size_t part = ((n + PT_COPY_THREADS - 1) / PT_COPY_THREADS + 4095) & ~(size_t)4095;
        {
            std::lock_guard<std::mutex> lk(m_);
            if (workers_.empty()) {
                owner_ = getpid();
                for (int w = 1; w < PT_COPY_THREADS; w++) workers_.emplace_back(&CopyPool::work, this, w);
            } else if (owner_ != getpid()) {
                memcpy(dst, src, n);
                return;
            }
            for (int p = 0; p < PT_COPY_THREADS; p++) {
                const size_t off = std::min(n, p * part);
                parts_[p] = Part{dst + off, src + off, std::min(part, n - off)};
            }
            pending_ = PT_COPY_THREADS - 1;
            generation_++;
        }
        cv_work_.notify_all();
        memcpy(parts_[0].dst, parts_[0].src, parts_[0].n);
        std::unique_lock<std::mutex> lk(m_);
        cv_done_.wait(lk, [&] { return pending_ == 0; });
    }

private:
    struct Part {
        char *dst;
        const char *src;
        size_t n;
    };
    void work(int id)
    {
        unsigned long seen = 0;
        std::unique_lock<std::mutex> lk(m_);
        for (;;) {
            cv_work_.wait(lk, [&] { return generation_ != seen; });
            seen = generation_;
            const Part p = parts_[id];
            lk.unlock();
            if (p.n) memcpy(p.dst, p.src, p.n);
            lk.lock();
            if (--pending_ == 0) cv_done_.notify_one();
        }
    }
    std::mutex m_;
    std::condition_variable cv_work_, cv_done_;
    std::vector<std::thread> workers_;
    Part parts_[PT_COPY_THREADS] = {};
    unsigned long generation_ = 0;
    int pending_ = 0;
    pid_t owner_ = 0;  // process whose threads the workers are
};

// The ring of two pinned chunks and the events that mark their DMA done.
struct Stager {
    std::mutex lock;  // one staged transfer at a time
    bool ready = false, failed = false;
    char *chunk[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    CopyPool pool;

    // false when the pinned chunks cannot be had (the plain copy then runs)
    bool setup()
    {
        if (ready || failed) return ready;
        for (int b = 0; b < 2 && !failed; b++) {
            if (hipHostMalloc((void **)&chunk[b], PT_STAGE_CHUNK_MAX, hipHostMallocPortable) != hipSuccess ||
                hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess)
                failed = true;
        }
        if (failed) (void)hipGetLastError();
        ready = !failed;
        return ready;
    }
};

static Stager &stager()
{
    static Stager *s = new Stager();  // lives until the process ends, as its threads do
    return *s;
}

// true for memory the copy engines cannot reach directly: plain malloc'd or
// stack memory, which HIP reports as unregistered (or not at all)
static bool is_pageable(const void *p)
{
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();  // leave no error for the next launch check
        return true;
    }
    return attr.type == hipMemoryTypeUnregistered;
}

static size_t chunk_bytes(size_t bytes)
{
    // at least four chunks, so that the host copy and the DMA overlap
    size_t c = std::min(PT_STAGE_CHUNK_MAX, (bytes / 4 + PT_STAGE_CHUNK_MIN - 1) & ~(PT_STAGE_CHUNK_MIN - 1));
    return std::max(c, PT_STAGE_CHUNK_MIN);
}

// On an error the stream is drained before returning, so that no DMA into or
// out of a chunk is still running when the next transfer reuses it.
static pt_status drain(hipStream_t s, pt_status st)
{
    (void)hipStreamSynchronize(s);
    return st;
}

static pt_status staged_h2d(Stager &st, char *dst, const char *src, size_t bytes, hipStream_t s)
{
    const size_t cb = chunk_bytes(bytes);
    for (size_t off = 0, i = 0; off < bytes; off += cb, i++) {
        const int b = (int)(i & 1);
        const size_t n = std::min(cb, bytes - off);
        if (i >= 2) {  // the DMA out of this chunk two steps ago
            pt_status e = check_hip(hipEventSynchronize(st.done[b]), "host to device copy");
            if (e != PT_OK) return drain(s, e);
        }
        st.pool.copy(st.chunk[b], src + off, n);
        pt_status e = check_hip(hipMemcpyAsync(dst + off, st.chunk[b], n, hipMemcpyHostToDevice, s),
                                "host to device copy");
        if (e == PT_OK) e = check_hip(hipEventRecord(st.done[b], s), "host to device copy");
        if (e != PT_OK) return drain(s, e);
    }
    return check_hip(hipStreamSynchronize(s), "host to device copy");
}

static pt_status staged_d2h(Stager &st, char *dst, const char *src, size_t bytes, hipStream_t s)
{
    const size_t cb = chunk_bytes(bytes);
    const size_t nch = (bytes + cb - 1) / cb;
    auto enqueue = [&](size_t i) {
        const int b = (int)(i & 1);
        const size_t off = i * cb, n = std::min(cb, bytes - off);
        pt_status e = check_hip(hipMemcpyAsync(st.chunk[b], src + off, n, hipMemcpyDeviceToHost, s),
                                "device to host copy");
        if (e == PT_OK) e = check_hip(hipEventRecord(st.done[b], s), "device to host copy");
        return e;
    };
    for (size_t i = 0; i < std::min<size_t>(2, nch); i++) {
        pt_status e = enqueue(i);
        if (e != PT_OK) return drain(s, e);
    }
    for (size_t j = 0; j < nch; j++) {
        const int b = (int)(j & 1);
        const size_t off = j * cb, n = std::min(cb, bytes - off);
        pt_status e = check_hip(hipEventSynchronize(st.done[b]), "device to host copy");
        if (e != PT_OK) return drain(s, e);
        st.pool.copy(dst + off, st.chunk[b], n);
        if (j + 2 < nch && (e = enqueue(j + 2)) != PT_OK) return drain(s, e);
    }
    return PT_OK;
}

}  // namespace pt

using namespace pt;

extern "C" {

pt_status pt_memcpy_h2d(void *dst, const void *src, size_t bytes, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!bytes) return PT_OK;
    hipStream_t s = stream_of(stream);
    if (bytes >= PT_STAGE_MIN_BYTES && is_pageable(src)) {
        Stager &st = stager();
        std::lock_guard<std::mutex> lk(st.lock);
        if (st.setup()) {
            counters().staged_copies++;
            return staged_h2d(st, (char *)dst, (const char *)src, bytes, s);
        }
    }
    PT_TRY(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "host to device copy"));
    return check_hip(hipStreamSynchronize(s), "host to device copy");
}

pt_status pt_memcpy_d2h(void *dst, const void *src, size_t bytes, pt_stream_t stream)
{
    PT_TRY(ensure_init());
    if (!bytes) return PT_OK;
    hipStream_t s = stream_of(stream);
    if (bytes >= PT_STAGE_MIN_BYTES && is_pageable(dst)) {
        Stager &st = stager();
        std::lock_guard<std::mutex> lk(st.lock);
        if (st.setup()) {
            counters().staged_copies++;
            return staged_d2h(st, (char *)dst, (const char *)src, bytes, s);
        }
    }
    PT_TRY(check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "device to host copy"));
    return check_hip(hipStreamSynchronize(s), "device to host copy");
}

}  // extern "C"
