// Host pipeline of the command line: GGUF rows (pread from the input file, or
// copied from host memory) -> pinned staging -> HBM -> quantizer -> pinned ->
// pwrite at the tensor's file offset.
//
// Replaces the reference's CudaPipeline (quant-studio.py:148-213),
// OutputWriter (:103-131) and copy_tensor (:235-241):
//   - a ring of input slots (pinned rows and imatrix, their device copies) and
//     a deeper ring of output slots (pinned host memory the kernel writes
//     directly), so the host read of chunk i+1, the H2D and kernel of chunk i
//     and the file writes of earlier chunks overlap, and a writer a few chunks
//     behind does not hold back the next uploads;
//   - the read (or copy) into pinned memory of a chunk split over a pool of
//     threads (one thread caps the pipeline well below the PCIe rate), and
//     run one chunk ahead of the launches: a queue call starts the pool on
//     its chunk, then queues the previous chunk's upload and kernel while the
//     pool reads, and leaves its own last chunk pending for the next call or
//     qs_pipeline_finish, so reads overlap the launches and the caller's work
//     between tensors;
//   - uploads on a copy stream, kernels on two compute streams taken in turn,
//     ordered by per-slot events; the calling thread never waits on the GPU
//     except for a slot. Consecutive kernels may overlap: the next chunk's
//     waves fill the GPU while the last waves of this one drain (a fixed
//     ~0.36 wave-lifetime per launch, ~10% of a Q4_K + imatrix launch on a
//     9728x2560 tensor);
//   - rows handed to the kernel in their stored type (no f32 upcast pass);
//   - one writer thread that waits on each chunk's kernel event and writes the
//     chunk at its own offset, so the output never depends on the chunking.
#include <hip/hip_runtime.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "quant_studio.h"
#include "qs_host.h"

using qs_host::fail;

namespace {

constexpr size_t kCopyPart = size_t(1) << 20;     // smallest share of a chunk copy per thread

// Fixed pool running the parts of one chunk copy; run() returns when all are done.
class CopyPool {
public:
    explicit CopyPool(int n) {
        for (int i = 0; i < n; i++) threads_.emplace_back([this] { loop(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> l(m_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : threads_) t.join();
    }
    int size() const { return (int)threads_.size(); }

    // Start the tasks on the pool and return; wait() returns once every
    // submitted task has run.
    void submit(std::vector<std::function<void()>>& tasks) {
        std::lock_guard<std::mutex> l(m_);
        for (auto& t : tasks) q_.push_back(std::move(t));
        pending_ += tasks.size();
        cv_.notify_all();
    }
    void wait() {
        std::unique_lock<std::mutex> l(m_);
        done_cv_.wait(l, [this] { return pending_ == 0; });
    }

private:
    void loop() {
        std::unique_lock<std::mutex> l(m_);
        for (;;) {
            cv_.wait(l, [this] { return stop_ || !q_.empty(); });
            if (q_.empty()) return;
            auto t = std::move(q_.front());
            q_.pop_front();
            l.unlock();
            t();
            l.lock();
            if (--pending_ == 0) done_cv_.notify_all();
        }
    }
    std::vector<std::thread> threads_;
    std::deque<std::function<void()>> q_;
    std::mutex m_;
    std::condition_variable cv_, done_cv_;
    size_t pending_ = 0;
    bool stop_ = false;
};

struct WriteJob {
    hipEvent_t ev;            // wait for this before reading buf (nullptr: host data)
    const void* buf;
    size_t n;
    int fd;
    int64_t off;
};

// Single writer thread: jobs complete in submission order; done() counts them.
class Writer {
public:
    explicit Writer(int device) : th_([this, device] { (void)hipSetDevice(device); loop(); }) {}
    ~Writer() {
        {
            std::lock_guard<std::mutex> l(m_);
            stop_ = true;
        }
        cv_.notify_all();
        th_.join();
    }
    uint64_t push(const WriteJob& j) {
        std::lock_guard<std::mutex> l(m_);
        q_.push_back(j);
        cv_.notify_all();
        return ++pushed_;
    }
    void wait(uint64_t seq) {
        std::unique_lock<std::mutex> l(m_);
        done_cv_.wait(l, [&] { return done_ >= seq; });
    }
    void drain() { wait(pushed()); }
    uint64_t pushed() {
        std::lock_guard<std::mutex> l(m_);
        return pushed_;
    }
    // first error seen by the writer ("" if none)
    std::string error() {
        std::lock_guard<std::mutex> l(m_);
        return err_;
    }

private:
    void loop() {
        std::unique_lock<std::mutex> l(m_);
        for (;;) {
            cv_.wait(l, [this] { return stop_ || !q_.empty(); });
            if (q_.empty()) return;
            WriteJob j = q_.front();
            q_.pop_front();
            const bool failed = !err_.empty();
            l.unlock();
            std::string e;
            if (!failed) e = run(j);
            l.lock();
            if (!e.empty() && err_.empty()) err_ = e;
            done_++;
            done_cv_.notify_all();
        }
    }
    static std::string run(const WriteJob& j) {
        if (j.ev) {
            const hipError_t he = hipEventSynchronize(j.ev);
            if (he != hipSuccess) return std::string("device work failed: ") + hipGetErrorString(he);
        }
        const char* p = static_cast<const char*>(j.buf);
        size_t left = j.n;
        int64_t off = j.off;
        while (left) {
            const ssize_t w = pwrite(j.fd, p, std::min(left, size_t(1) << 30), off);
            if (w < 0 && errno == EINTR) continue;
            if (w <= 0) return std::string("write failed: ") + std::strerror(w < 0 ? errno : EIO);
            p += w;
            off += w;
            left -= (size_t)w;
        }
        return "";
    }
    std::deque<WriteJob> q_;
    std::mutex m_;
    std::condition_variable cv_, done_cv_;
    uint64_t pushed_ = 0, done_ = 0;
    std::string err_;
    bool stop_ = false;
    std::thread th_;
};

// Buffer sizes are rounded up (2 MiB for rows and outputs, 64 KiB for an
// imatrix), so chunks whose byte counts differ by a few rows' worth (16 MiB
// of input holds a whole number of rows of each width) and imatrices of
// different widths reuse a slot's buffers: growing a device buffer frees the
// old one, and hipFree waits for all work on the device.
inline size_t alloc_size(size_t want) {
    const size_t g = want > (size_t(64) << 10) ? size_t(2) << 20 : size_t(64) << 10;
    return (std::max<size_t>(want, 1) + g - 1) / g * g;
}

struct PinnedBuf {
    void* p = nullptr;
    size_t n = 0;
    unsigned flags = hipHostMallocDefault;
    bool grow(size_t want) {
        if (n >= want) return true;
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
        want = alloc_size(want);
        if (hipHostMalloc(&p, want, flags) != hipSuccess) return false;
        n = want;
        return true;
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        n = 0;
    }
};

struct DevBuf {
    void* p = nullptr;
    size_t n = 0;
    bool grow(size_t want) {
        if (n >= want) return true;
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
        want = alloc_size(want);
        if (hipMalloc(&p, want) != hipSuccess) return false;
        n = want;
        return true;
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        n = 0;
    }
};

// Input ring: pinned staging of the rows, their device copy and the imatrix.
struct InSlot {
    PinnedBuf in_pin, qw_pin;
    DevBuf x_dev, qw_dev;
    hipEvent_t h2d = nullptr;     // the rows (and imatrix) are on the device
    hipEvent_t kern = nullptr;    // the kernel that read x_dev / qw_dev is done
    bool used = false;            // events recorded at least once
};

// Output ring: pinned host memory (coherent: the device's stores go over the
// bus to host memory, not into its caches) that the kernel writes directly,
// so no download is queued: the chunk's output is a few MB against 16 MiB of
// input, and a download per chunk cost a copy kernel on the device and a
// slow runtime call on the host. Deeper than the input ring, so a writer
// running a few chunks behind the GPU does not stop the calling thread from
// staging the next inputs.
struct OutSlot {
    PinnedBuf out_pin;
    hipEvent_t ready = nullptr;   // the kernel that writes out_pin is done
    bool used = false;
    uint64_t write_seq = 0;       // writer job that reads out_pin
};

int elem_size(int src_type) {
    switch (src_type) {
    case QS_SRC_F32: return 4;
    case QS_SRC_F16:
    case QS_SRC_BF16: return 2;
    default: return 0;
    }
}

// A chunk whose rows are being read into its input slot and whose upload and
// kernel are not queued yet.
struct Chunk {
    bool valid = false;
    size_t slot = 0;          // input slot
    int ggml_type = 0, src_type = 0;
    int64_t n = 0, k = 0, in_row = 0;
    size_t nin = 0, nout = 0, nqw = 0;
    int fd = -1;
    int64_t out_off = 0;
};

}  // namespace

struct qs_pipeline {
    int device = 0;
    hipStream_t h2d = nullptr, compute[2] = {nullptr, nullptr};
    std::vector<InSlot> in_slots;
    std::vector<OutSlot> out_slots;
    size_t next_in = 0, next_out = 0;
    uint64_t launches = 0;    // picks the compute stream of the next kernel
    std::unique_ptr<CopyPool> pool;
    std::unique_ptr<Writer> writer;
    std::string err;          // first failure; every later call reports it
    Chunk pending;            // read in flight on the pool, launch not queued
    std::atomic<int> read_err{0};   // errno of a failed read (0: none)

    int check_writer() {
        if (err.empty()) err = writer->error();
        return err.empty() ? 0 : fail(QS_EIO, "%s", err.c_str());
    }
    int hip_fail(hipError_t e, const char* what) {
        if (err.empty()) err = std::string(what) + ": " + hipGetErrorString(e);
        return fail(QS_EIO, "%s", err.c_str());
    }
};

// Where a tensor's rows come from: host memory (normally the input file's
// mapping) or a file read with pread(), which copies from the page cache
// without mapping the pages into the process (no page faults in the copies,
// no page-table teardown when the mapping goes).
struct RowSource {
    const char* mem = nullptr;
    int fd = -1;
    int64_t off = 0;
};

// One share of a chunk's staging copy; returns 0 or an errno value.
static int copy_rows(const RowSource& src, size_t from, char* to, size_t n) {
    if (!src.mem) {
        while (n) {
            const ssize_t r = pread(src.fd, to, std::min(n, size_t(1) << 30), (off_t)(src.off + (int64_t)from));
            if (r < 0 && errno == EINTR) continue;
            if (r < 0) return errno;
            if (r == 0) return EIO;       // the file ends inside the tensor
            to += r;
            from += (size_t)r;
            n -= (size_t)r;
        }
        return 0;
    }
    std::memcpy(to, src.mem + from, n);
    return 0;
}

static int pipeline_quantize(qs_pipeline* p, int ggml_type, int src_type, const RowSource& rows,
                             int64_t n_rows, int64_t k, const float* imatrix, int64_t rows_per_chunk, int fd,
                             int64_t out_offset);

extern "C" {

int qs_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

int qs_pipeline_create(int device, int n_slots, int n_copy_threads, qs_pipeline** out) {
    qs_host::clear_error();
    if (!out) return fail(QS_EINVAL, "null output handle");
    *out = nullptr;
    if (n_slots < 2 || n_slots > 16) return fail(QS_EINVAL, "n_slots %d outside [2, 16]", n_slots);
    if (n_copy_threads < 1 || n_copy_threads > 64)
        return fail(QS_EINVAL, "n_copy_threads %d outside [1, 64]", n_copy_threads);
    const int ndev = qs_device_count();
    if (device < 0 || device >= ndev)
        return fail(QS_EINVAL, "device %d not present (%d ROCm devices visible)", device, ndev);
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return fail(QS_EIO, "hipSetDevice(%d): %s", device, hipGetErrorString(e));
    auto p = std::make_unique<qs_pipeline>();
    p->device = device;
    if ((e = hipStreamCreateWithFlags(&p->h2d, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&p->compute[0], hipStreamNonBlocking)) != hipSuccess ||
        (e = hipStreamCreateWithFlags(&p->compute[1], hipStreamNonBlocking)) != hipSuccess) {
        qs_pipeline_destroy(p.release());
        return fail(QS_EIO, "stream creation failed: %s", hipGetErrorString(e));
    }
    p->in_slots.resize(n_slots);
    p->out_slots.resize(std::max(8, 2 * n_slots));
    for (auto& s : p->in_slots) {
        if ((e = hipEventCreateWithFlags(&s.h2d, hipEventDisableTiming)) != hipSuccess ||
            (e = hipEventCreateWithFlags(&s.kern, hipEventDisableTiming)) != hipSuccess) {
            qs_pipeline_destroy(p.release());
            return fail(QS_EIO, "event creation failed: %s", hipGetErrorString(e));
        }
    }
    for (auto& s : p->out_slots) {
        s.out_pin.flags = hipHostMallocCoherent;
        if ((e = hipEventCreateWithFlags(&s.ready, hipEventDisableTiming)) != hipSuccess) {
            qs_pipeline_destroy(p.release());
            return fail(QS_EIO, "event creation failed: %s", hipGetErrorString(e));
        }
    }
    p->pool = std::make_unique<CopyPool>(n_copy_threads);
    p->writer = std::make_unique<Writer>(device);
    *out = p.release();
    return 0;
}

int qs_pipeline_quantize(qs_pipeline* p, int ggml_type, int src_type, const void* src, int64_t n_rows,
                         int64_t k, const float* imatrix, int64_t rows_per_chunk, int fd,
                         int64_t out_offset) {
    qs_host::clear_error();
    RowSource rows;
    rows.mem = static_cast<const char*>(src);
    return pipeline_quantize(p, ggml_type, src_type, rows, n_rows, k, imatrix, rows_per_chunk, fd, out_offset);
}

int qs_pipeline_quantize_fd(qs_pipeline* p, int ggml_type, int src_type, int src_fd, int64_t src_offset,
                            int64_t n_rows, int64_t k, const float* imatrix, int64_t rows_per_chunk, int fd,
                            int64_t out_offset) {
    qs_host::clear_error();
    if (src_fd < 0 || src_offset < 0)
        return fail(QS_EINVAL, "bad input fd %d / offset %lld", src_fd, (long long)src_offset);
    RowSource rows;
    rows.fd = src_fd;
    rows.off = src_offset;
    return pipeline_quantize(p, ggml_type, src_type, rows, n_rows, k, imatrix, rows_per_chunk, fd, out_offset);
}

}  // extern "C"

// Touch every page of a newly allocated pinned buffer from the pool's threads
// (and wait). The host mapping of hipHostMalloc memory is filled in on first
// access, a page fault per few pages: the first pread into a 16 MiB input
// slot, or the writer's first pwrite from a 6 MiB output slot, took ~2.5 ms
// longer than later ones on the MI355X machine's host, on the pipeline's
// critical path; touched in parallel the faults cost a fraction of that.
static void touch_pages(qs_pipeline* p, void* buf, size_t n) {
    const size_t parts = std::max<size_t>(1, std::min<size_t>((size_t)p->pool->size(), n / kCopyPart));
    std::vector<std::function<void()>> tasks;
    char* b = static_cast<char*>(buf);
    for (size_t i = 0; i < parts; i++) {
        const size_t lo = n * i / parts, hi = n * (i + 1) / parts;
        tasks.emplace_back([b, lo, hi] { std::memset(b + lo, 0, hi - lo); });
    }
    p->pool->submit(tasks);
    p->pool->wait();
}

// Wait for the pool's reads (the pending chunk's) and report a failed one.
static int wait_reads(qs_pipeline* p) {
    p->pool->wait();
    if (const int re = p->read_err.exchange(0)) {
        p->pending.valid = false;
        if (p->err.empty()) p->err = std::string("reading the input rows failed: ") + std::strerror(re);
        return fail(QS_EIO, "%s", p->err.c_str());
    }
    return 0;
}

// Queue the pending chunk (its rows are in its input slot): upload, kernel on
// the next compute stream writing into an output slot, write job.
static int launch_pending(qs_pipeline* p) {
    if (!p->pending.valid) return 0;
    const Chunk c = p->pending;
    p->pending.valid = false;
    InSlot& si = p->in_slots[c.slot];
    OutSlot& so = p->out_slots[p->next_out];
    p->next_out = (p->next_out + 1) % p->out_slots.size();
    hipError_t e;
    if (so.used) {
        // out_pin is free once its write is done (the writer waited for the
        // kernel that wrote it)
        p->writer->wait(so.write_seq);
        if (int rc = p->check_writer()) return rc;
    }
    const size_t out_had = so.out_pin.n;
    if (!so.out_pin.grow(c.nout)) {
        if (p->err.empty()) p->err = "out of memory staging a chunk";
        return fail(QS_EIO, "out of memory staging the output of a chunk of %lld rows", (long long)c.n);
    }
    if (so.out_pin.n != out_had) touch_pages(p, so.out_pin.p, so.out_pin.n);
    // the upload overwrites x_dev / qw_dev once the kernel that read them is done
    if (si.used && (e = hipStreamWaitEvent(p->h2d, si.kern, 0)) != hipSuccess) return p->hip_fail(e, "wait");
    if ((e = hipMemcpyAsync(si.x_dev.p, si.in_pin.p, c.nin, hipMemcpyHostToDevice, p->h2d)) != hipSuccess)
        return p->hip_fail(e, "H2D");
    if (c.nqw && (e = hipMemcpyAsync(si.qw_dev.p, si.qw_pin.p, c.nqw, hipMemcpyHostToDevice, p->h2d)) != hipSuccess)
        return p->hip_fail(e, "H2D");
    if ((e = hipEventRecord(si.h2d, p->h2d)) != hipSuccess) return p->hip_fail(e, "event");
    si.used = true;
    hipStream_t cs = p->compute[p->launches++ & 1];
    if ((e = hipStreamWaitEvent(cs, si.h2d, 0)) != hipSuccess) return p->hip_fail(e, "wait");
    const int rc = qs_quantize(c.ggml_type, c.src_type, si.x_dev.p, c.n, c.k, c.in_row,
                               c.nqw ? static_cast<const float*>(si.qw_dev.p) : nullptr, so.out_pin.p,
                               (int64_t)c.nout, cs);
    if (rc) {
        if (p->err.empty()) p->err = "quantizer launch failed";
        return rc;
    }
    if ((e = hipEventRecord(si.kern, cs)) != hipSuccess) return p->hip_fail(e, "event");
    if ((e = hipEventRecord(so.ready, cs)) != hipSuccess) return p->hip_fail(e, "event");
    so.used = true;
    so.write_seq = p->writer->push({so.ready, so.out_pin.p, c.nout, c.fd, c.out_off});
    return 0;
}

// Queue what is still pending and wait for the reads.
static int flush_pending(qs_pipeline* p) {
    if (int rc = wait_reads(p)) return rc;
    if (!p->err.empty()) {
        p->pending.valid = false;
        return fail(QS_EIO, "%s", p->err.c_str());
    }
    return launch_pending(p);
}

static int pipeline_quantize(qs_pipeline* p, int ggml_type, int src_type, const RowSource& src,
                             int64_t n_rows, int64_t k, const float* imatrix, int64_t rows_per_chunk, int fd,
                             int64_t out_offset) {
    if (!p) return fail(QS_EINVAL, "null pipeline");
    if (int rc = p->check_writer()) return rc;
    const int esz = elem_size(src_type);
    if (!esz) return fail(QS_EINVAL, "unsupported source type %d (F32=0, F16=1, BF16=30)", src_type);
    if (n_rows < 0 || rows_per_chunk <= 0 || out_offset < 0 || fd < 0)
        return fail(QS_EINVAL, "bad n_rows %lld / rows_per_chunk %lld / offset %lld / fd %d",
                    (long long)n_rows, (long long)rows_per_chunk, (long long)out_offset, fd);
    if (!qs_type_supported(ggml_type)) return fail(QS_ENOTSUP, "ggml type %d has no HIP quantizer", ggml_type);
    const int64_t out_row = qs_row_bytes(ggml_type, k);
    if (out_row < 0) return (int)out_row;
    // the same per-call limit as qs_quantize (2^34 values), checked before any
    // chunk size is formed from n_rows * k
    constexpr int64_t kMaxValues = INT64_C(1) << 34;
    if (k > kMaxValues || n_rows > kMaxValues / k)
        return fail(QS_EINVAL, "%lld x %lld values exceed the 2^34 per tensor", (long long)n_rows,
                    (long long)k);
    if (n_rows == 0) return 0;
    if (!src.mem && src.fd < 0) return fail(QS_EINVAL, "null src");
    if (qs_host::quantizer_requires_imatrix(ggml_type) && !imatrix)
        return fail(QS_EINVAL, "ggml type %d requires an imatrix", ggml_type);
    const bool use_qw = imatrix && qs_type_uses_imatrix(ggml_type) == 1;
    hipError_t e = hipSetDevice(p->device);
    if (e != hipSuccess) return p->hip_fail(e, "hipSetDevice");
    const int64_t in_row = k * esz;

    for (int64_t r0 = 0; r0 < n_rows; r0 += rows_per_chunk) {
        Chunk c;
        c.valid = true;
        c.slot = p->next_in;
        c.ggml_type = ggml_type;
        c.src_type = src_type;
        c.n = std::min(rows_per_chunk, n_rows - r0);
        c.k = k;
        c.in_row = in_row;
        c.nin = (size_t)(c.n * in_row);
        c.nout = (size_t)(c.n * out_row);
        c.nqw = use_qw ? (size_t)k * 4 : 0;
        c.fd = fd;
        c.out_off = out_offset + r0 * out_row;
        InSlot& si = p->in_slots[c.slot];
        p->next_in = (p->next_in + 1) % p->in_slots.size();
        // the pending chunk holds the slot before this one, so this slot's last
        // chunk is queued: wait for its upload (in_pin) and, if the device
        // buffers must grow, for the kernel that read them
        if (si.used) {
            if ((e = hipEventSynchronize(si.h2d)) != hipSuccess) return p->hip_fail(e, "H2D");
            if ((si.x_dev.n < c.nin || si.qw_dev.n < c.nqw) && (e = hipEventSynchronize(si.kern)) != hipSuccess)
                return p->hip_fail(e, "kernel");
        }
        const size_t in_had = si.in_pin.n;
        if (!si.in_pin.grow(c.nin) || !si.qw_pin.grow(c.nqw) || !si.x_dev.grow(c.nin) || !si.qw_dev.grow(c.nqw)) {
            if (p->err.empty()) p->err = "out of memory staging a chunk";
            return fail(QS_EIO, "out of memory staging a chunk of %lld rows x %lld bytes", (long long)c.n,
                        (long long)in_row);
        }
        if (si.in_pin.n != in_had) touch_pages(p, si.in_pin.p, si.in_pin.n);
        if (c.nqw) std::memcpy(si.qw_pin.p, imatrix, c.nqw);
        // the pending chunk's rows are in place once the pool is idle
        if (int rc = wait_reads(p)) return rc;
        // this chunk's rows -> pinned, on the pool, in parts of at least kCopyPart bytes
        const size_t from = (size_t)(r0 * in_row);
        char* to = static_cast<char*>(si.in_pin.p);
        const size_t parts = std::max<size_t>(1, std::min<size_t>((size_t)p->pool->size(), c.nin / kCopyPart));
        std::vector<std::function<void()>> tasks;
        std::atomic<int>* read_err = &p->read_err;
        for (size_t i = 0; i < parts; i++) {
            const size_t a = c.nin * i / parts, b = c.nin * (i + 1) / parts;
            tasks.emplace_back([src, read_err, from, to, a, b] {
                if (const int re = copy_rows(src, from + a, to + a, b - a)) read_err->store(re);
            });
        }
        p->pool->submit(tasks);
        // while the pool reads: the previous chunk's launch
        const int rc = launch_pending(p);
        p->pending = c;
        if (rc) return rc;
    }
    return 0;
}

extern "C" {

int qs_pipeline_write(qs_pipeline* p, const void* src, int64_t nbytes, int fd, int64_t out_offset) {
    qs_host::clear_error();
    if (!p) return fail(QS_EINVAL, "null pipeline");
    if (int rc = p->check_writer()) return rc;
    if (nbytes < 0 || out_offset < 0 || fd < 0 || (nbytes && !src))
        return fail(QS_EINVAL, "bad write of %lld bytes at %lld (fd %d)", (long long)nbytes,
                    (long long)out_offset, fd);
    if (nbytes) p->writer->push({nullptr, src, (size_t)nbytes, fd, out_offset});
    return 0;
}

int qs_pipeline_finish(qs_pipeline* p) {
    qs_host::clear_error();
    if (!p) return fail(QS_EINVAL, "null pipeline");
    hipError_t e = hipSetDevice(p->device);
    // the last chunk's launch (its read may still run), then everything it queued
    const int prc = e == hipSuccess ? flush_pending(p) : p->hip_fail(e, "hipSetDevice");
    p->writer->drain();
    if (e == hipSuccess) e = hipStreamSynchronize(p->h2d);
    for (hipStream_t cs : p->compute)
        if (e == hipSuccess) e = hipStreamSynchronize(cs);
    if (e != hipSuccess) return p->hip_fail(e, "device work failed");
    if (prc) return prc;
    return p->check_writer();
}

void qs_pipeline_destroy(qs_pipeline* p) {
    if (!p) return;
    (void)hipSetDevice(p->device);
    if (p->pool && p->writer) (void)flush_pending(p);
    if (p->writer) p->writer->drain();
    if (p->h2d) (void)hipStreamSynchronize(p->h2d);
    for (hipStream_t cs : p->compute)
        if (cs) (void)hipStreamSynchronize(cs);
    p->writer.reset();
    p->pool.reset();
    for (auto& s : p->in_slots) {
        s.in_pin.release();
        s.qw_pin.release();
        s.x_dev.release();
        s.qw_dev.release();
        if (s.h2d) (void)hipEventDestroy(s.h2d);
        if (s.kern) (void)hipEventDestroy(s.kern);
    }
    for (auto& s : p->out_slots) {
        s.out_pin.release();
        if (s.ready) (void)hipEventDestroy(s.ready);
    }
    if (p->h2d) (void)hipStreamDestroy(p->h2d);
    for (hipStream_t cs : p->compute)
        if (cs) (void)hipStreamDestroy(cs);
    delete p;
}

}  // extern "C"
