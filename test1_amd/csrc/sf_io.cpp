// Storage offload engine: host buffers to and from files on local storage.
//
// The reference moves two kinds of data to NVMe: checkpointed activations
// straight from device memory through GPUDirect Storage (kvikio
// `CuFile.raw_write_async` / `raw_read_async`, sliding_checkpoint.py:133-202)
// and LayerAdam's moments through tensornvme's io_uring `DiskOffloader`
// (optimizer/layer_adam/layer_adam.py:89-103, 197-244).  Neither library
// exists for ROCm, and this platform has no GPU-to-storage DMA, so data
// reaches storage from host memory: activations through pinned bounce slots,
// moments from their host buffers.  This engine is the part both share.
//
// A request (one buffer, one file range) is cut into chunks of `chunk_bytes`
// that a pool of worker threads moves with pread/pwrite, so one large request
// keeps several commands in flight on the device.  Files are opened with
// O_DIRECT where the file system allows it: the page cache is bypassed, the
// host memory the offload is meant to free is not refilled by cached file
// pages, and the transfer rate is the device's.  O_DIRECT needs the buffer,
// the size and the file offset aligned to SF_IO_ALIGN; submit checks this.
// It also needs memory the kernel can pin: buffers from the GPU driver's
// pinned allocator are not, and are moved through a per-worker staging
// buffer (see move_chunk).
//
// Completion is tracked per request (a ticket); callers poll it without
// blocking (sf_io_query) or wait for it (sf_io_wait, which also releases the
// ticket).  The engine keeps byte counts and the time during which at least
// one request was in flight, for the storage rate of a run.

#include <errno.h>
#include <fcntl.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <thread>
#include <unordered_map>
#include <vector>

#include "../../include/slidefsdp.h"

namespace {

uint64_t now_ns() {
    timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return uint64_t(ts.tv_sec) * 1000000000ull + uint64_t(ts.tv_nsec);
}

struct Request {
    std::atomic<size_t> remaining{0};
    std::atomic<int> status{SF_OK};  // first failure wins
    int op = 0;
    size_t bytes = 0;
    uint64_t t_submit = 0;
    uint64_t t_done = 0;
};

struct Chunk {
    std::shared_ptr<Request> req;
    int fd = -1;
    bool direct = false;
    int op = 0;
    char* buf = nullptr;
    size_t bytes = 0;
    uint64_t offset = 0;
};

// One transfer with pread/pwrite; short transfers continue where they
// stopped.  Returns 0 or an errno value; a read that meets the end of the
// file fails with ENODATA (files are sized with sf_io_reserve first).
int transfer(int fd, int op, char* p, size_t left, uint64_t off) {
    while (left > 0) {
        ssize_t r = op == SF_IO_WRITE ? pwrite(fd, p, left, off_t(off)) : pread(fd, p, left, off_t(off));
        if (r < 0) {
            if (errno == EINTR) continue;
            return errno;
        }
        if (r == 0) return op == SF_IO_WRITE ? EIO : ENODATA;
        p += r;
        left -= size_t(r);
        off += uint64_t(r);
    }
    return 0;
}

// Per-worker aligned staging buffer (allocated on first use, freed with
// the thread).
struct Staging {
    char* buf = nullptr;
    size_t size = 0;
    ~Staging() { free(buf); }
    char* get(size_t n) {
        if (size < n) {
            free(buf);
            buf = nullptr;
            size = 0;
            if (posix_memalign(reinterpret_cast<void**>(&buf), SF_IO_ALIGN, n) != 0) return nullptr;
            size = n;
        }
        return buf;
    }
};
thread_local Staging t_staging;

// Moves one chunk.  Direct I/O needs pages the kernel can pin; memory the
// GPU driver maps into the process (hipHostMalloc) is not such memory, and
// the transfer fails with EFAULT before moving a byte.  Such chunks go
// through this worker's staging buffer instead (one extra host copy).
int move_chunk(const Chunk& c, bool direct, std::atomic<uint64_t>& staged) {
    int err = transfer(c.fd, c.op, c.buf, c.bytes, c.offset);
    if (err != EFAULT || !direct) return err;
    char* st = t_staging.get(c.bytes);
    if (!st) return ENOMEM;
    if (c.op == SF_IO_WRITE) {
        memcpy(st, c.buf, c.bytes);
        err = transfer(c.fd, c.op, st, c.bytes, c.offset);
    } else {
        err = transfer(c.fd, c.op, st, c.bytes, c.offset);
        if (err == 0) memcpy(c.buf, st, c.bytes);
    }
    if (err == 0) staged.fetch_add(c.bytes);
    return err;
}

bool is_direct(int fd) {
    int fl = fcntl(fd, F_GETFL);
    return fl >= 0 && (fl & O_DIRECT) != 0;
}

}  // namespace

struct sf_io {
    std::mutex mu;
    std::condition_variable cv_work;
    std::condition_variable cv_done;
    std::deque<Chunk> queue;
    std::unordered_map<uint64_t, std::shared_ptr<Request>> reqs;
    std::vector<std::thread> workers;
    uint64_t next_ticket = 1;
    size_t chunk_bytes = 0;
    bool stop = false;
    // statistics (under mu)
    size_t inflight = 0;
    uint64_t busy_since = 0;
    uint64_t busy_ns = 0;
    uint64_t bytes_read = 0;
    uint64_t bytes_written = 0;
    std::atomic<uint64_t> bytes_staged{0};

    void finish(const std::shared_ptr<Request>& r) {
        std::lock_guard<std::mutex> lk(mu);
        r->t_done = now_ns();
        if (r->op == SF_IO_WRITE)
            bytes_written += r->bytes;
        else
            bytes_read += r->bytes;
        if (--inflight == 0) busy_ns += r->t_done - busy_since;
        cv_done.notify_all();
    }

    void work() {
        for (;;) {
            Chunk c;
            {
                std::unique_lock<std::mutex> lk(mu);
                cv_work.wait(lk, [&] { return stop || !queue.empty(); });
                if (queue.empty()) return;  // stopping and drained
                c = std::move(queue.front());
                queue.pop_front();
            }
            int err = move_chunk(c, c.direct, bytes_staged);
            if (err != 0) {
                int expected = SF_OK;
                c.req->status.compare_exchange_strong(expected, SF_EIO_BASE + err);
            }
            if (c.req->remaining.fetch_sub(1) == 1) finish(c.req);
        }
    }
};

extern "C" {

int sf_io_create(int n_threads, size_t chunk_bytes, sf_io** out) {
    if (!out || n_threads <= 0 || n_threads > 256) return SF_EINVAL;
    if (chunk_bytes == 0) chunk_bytes = size_t(8) << 20;
    chunk_bytes = (chunk_bytes + SF_IO_ALIGN - 1) / SF_IO_ALIGN * SF_IO_ALIGN;
    sf_io* io = new (std::nothrow) sf_io();
    if (!io) return SF_EIO_BASE + ENOMEM;
    io->chunk_bytes = chunk_bytes;
    try {
        for (int i = 0; i < n_threads; ++i) io->workers.emplace_back([io] { io->work(); });
    } catch (...) {
        {
            std::lock_guard<std::mutex> lk(io->mu);
            io->stop = true;
        }
        io->cv_work.notify_all();
        for (auto& t : io->workers) t.join();
        delete io;
        return SF_EIO_BASE + EAGAIN;
    }
    *out = io;
    return SF_OK;
}

int sf_io_destroy(sf_io* io) {
    if (!io) return SF_EINVAL;
    {
        std::lock_guard<std::mutex> lk(io->mu);
        io->stop = true;
    }
    io->cv_work.notify_all();
    for (auto& t : io->workers) t.join();  // workers drain the queue first
    delete io;
    return SF_OK;
}

int sf_io_open(const char* path, int direct, int unlink_now, int* fd_out, int* direct_out) {
    if (!path || !fd_out) return SF_EINVAL;
    const int flags = O_RDWR | O_CREAT | O_CLOEXEC;
    int fd = -1;
    if (direct) fd = open(path, flags | O_DIRECT, 0600);
    // File systems without O_DIRECT (tmpfs, some overlays) refuse it with
    // EINVAL: use buffered I/O there and say so through *direct_out.
    if (fd < 0 && (!direct || errno == EINVAL)) fd = open(path, flags, 0600);
    if (fd < 0) return SF_EIO_BASE + errno;
    if (unlink_now && unlink(path) != 0) {
        int e = errno;
        close(fd);
        return SF_EIO_BASE + e;
    }
    *fd_out = fd;
    if (direct_out) *direct_out = is_direct(fd) ? 1 : 0;
    return SF_OK;
}

int sf_io_reserve(int fd, uint64_t bytes) {
    if (fd < 0) return SF_EINVAL;
    struct stat st;
    if (fstat(fd, &st) != 0) return SF_EIO_BASE + errno;
    if (uint64_t(st.st_size) >= bytes) return SF_OK;
    if (ftruncate(fd, off_t(bytes)) != 0) return SF_EIO_BASE + errno;
    return SF_OK;
}

int sf_io_close(int fd) {
    if (fd < 0) return SF_EINVAL;
    return close(fd) == 0 ? SF_OK : SF_EIO_BASE + errno;
}

int sf_io_submit(sf_io* io, int fd, int op, void* buf, size_t bytes, uint64_t offset, uint64_t* ticket) {
    if (!io || fd < 0 || !ticket || (op != SF_IO_READ && op != SF_IO_WRITE) || (bytes > 0 && !buf))
        return SF_EINVAL;
    const bool direct = is_direct(fd);
    if (direct && ((uintptr_t(buf) | bytes | offset) & uint64_t(SF_IO_ALIGN - 1)) != 0) return SF_EALIGN;
    auto req = std::make_shared<Request>();
    const size_t n_chunks = (bytes + io->chunk_bytes - 1) / io->chunk_bytes;
    req->op = op;
    req->bytes = bytes;
    req->remaining.store(n_chunks);
    std::lock_guard<std::mutex> lk(io->mu);
    if (io->stop) return SF_EINVAL;
    const uint64_t t = io->next_ticket++;
    req->t_submit = now_ns();
    io->reqs.emplace(t, req);
    if (n_chunks == 0) {
        req->t_done = req->t_submit;
    } else {
        if (io->inflight++ == 0) io->busy_since = req->t_submit;
        char* p = static_cast<char*>(buf);
        for (size_t i = 0; i < n_chunks; ++i) {
            Chunk c;
            c.req = req;
            c.fd = fd;
            c.direct = direct;
            c.op = op;
            c.buf = p + i * io->chunk_bytes;
            c.offset = offset + i * io->chunk_bytes;
            c.bytes = std::min(io->chunk_bytes, bytes - i * io->chunk_bytes);
            io->queue.push_back(std::move(c));
        }
        io->cv_work.notify_all();
    }
    *ticket = t;
    return SF_OK;
}

int sf_io_query(sf_io* io, uint64_t ticket, int* done) {
    if (!io || !done) return SF_EINVAL;
    std::lock_guard<std::mutex> lk(io->mu);
    auto it = io->reqs.find(ticket);
    if (it == io->reqs.end()) return SF_ENOREQ;
    *done = it->second->remaining.load() == 0 ? 1 : 0;
    return *done ? it->second->status.load() : SF_OK;
}

int sf_io_wait(sf_io* io, uint64_t ticket, uint64_t* submit_ns, uint64_t* done_ns) {
    if (!io) return SF_EINVAL;
    std::unique_lock<std::mutex> lk(io->mu);
    auto it = io->reqs.find(ticket);
    if (it == io->reqs.end()) return SF_ENOREQ;
    std::shared_ptr<Request> r = it->second;
    io->cv_done.wait(lk, [&] { return r->remaining.load() == 0 && r->t_done != 0; });
    io->reqs.erase(ticket);
    if (submit_ns) *submit_ns = r->t_submit;
    if (done_ns) *done_ns = r->t_done;
    return r->status.load();
}

int sf_io_stats(sf_io* io, uint64_t* bytes_read, uint64_t* bytes_written, uint64_t* busy_ns,
                uint64_t* bytes_staged) {
    if (!io) return SF_EINVAL;
    std::lock_guard<std::mutex> lk(io->mu);
    if (bytes_read) *bytes_read = io->bytes_read;
    if (bytes_written) *bytes_written = io->bytes_written;
    if (bytes_staged) *bytes_staged = io->bytes_staged.load();
    if (busy_ns) *busy_ns = io->busy_ns + (io->inflight > 0 ? now_ns() - io->busy_since : 0);
    return SF_OK;
}

}  // extern "C"
