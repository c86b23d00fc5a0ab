// Row tier reader: batched random reads of fixed-stride rows from a file on NVMe (Linux).
//
// Row i of a tier file occupies bytes [i * stride, i * stride + row_bytes) with stride a multiple of
// 4096 (one sector-aligned slot per row), so every read is one aligned request that O_DIRECT can serve
// without the page cache. fvs_tier_read_rows keeps up to qd requests in flight:
//   * io_uring (raw system calls, no liburing): one submission ring of qd entries, qd sector-aligned
//     bounce slots; every completion's slot is copied to its output row and refilled with the next id;
//   * where io_uring is unavailable (kernel or container policy) or asked for, a pool of qd threads
//     (at most 64) issuing pread() on their share of the ids.
// Host code only: it is built with the host compiler into libfvs_tier.so.
#include "../../include/fvs_tier.h"

#include <errno.h>
#include <fcntl.h>
#include <linux/io_uring.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <thread>
#include <vector>

namespace {

constexpr int kSector = 4096;
constexpr int kMaxQd = 1024;
constexpr int kMaxThreads = 64;

int sys_setup(unsigned entries, io_uring_params *p) { return (int)syscall(__NR_io_uring_setup, entries, p); }
int sys_enter(int fd, unsigned submit, unsigned wait, unsigned flags) {
  return (int)syscall(__NR_io_uring_enter, fd, submit, wait, flags, nullptr, 0);
}

struct Ring {
  int fd = -1;
  void *sq_ptr = nullptr, *cq_ptr = nullptr;
  size_t sq_len = 0, cq_len = 0;
  io_uring_sqe *sqes = nullptr;
  size_t sqes_len = 0;
  unsigned *sq_head, *sq_tail, *sq_mask, *sq_array;
  unsigned *cq_head, *cq_tail, *cq_mask;
  io_uring_cqe *cqes;
  unsigned entries = 0;

  int init(unsigned n) {
    io_uring_params p;
    memset(&p, 0, sizeof(p));
    fd = sys_setup(n, &p);
    if (fd < 0) return -errno;
    entries = p.sq_entries;
    sq_len = p.sq_off.array + p.sq_entries * sizeof(unsigned);
    cq_len = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
    const bool single = (p.features & IORING_FEAT_SINGLE_MMAP) != 0;
    if (single) sq_len = cq_len = std::max(sq_len, cq_len);
    sq_ptr = mmap(nullptr, sq_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_SQ_RING);
    if (sq_ptr == MAP_FAILED) return fail();
    cq_ptr = single ? sq_ptr
                    : mmap(nullptr, cq_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd, IORING_OFF_CQ_RING);
    if (cq_ptr == MAP_FAILED) return fail();
    sqes_len = p.sq_entries * sizeof(io_uring_sqe);
    sqes = (io_uring_sqe *)mmap(nullptr, sqes_len, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd,
                                IORING_OFF_SQES);
    if (sqes == MAP_FAILED) return fail();
    char *sq = (char *)sq_ptr, *cq = (char *)cq_ptr;
    sq_head = (unsigned *)(sq + p.sq_off.head);
    sq_tail = (unsigned *)(sq + p.sq_off.tail);
    sq_mask = (unsigned *)(sq + p.sq_off.ring_mask);
    sq_array = (unsigned *)(sq + p.sq_off.array);
    cq_head = (unsigned *)(cq + p.cq_off.head);
    cq_tail = (unsigned *)(cq + p.cq_off.tail);
    cq_mask = (unsigned *)(cq + p.cq_off.ring_mask);
    cqes = (io_uring_cqe *)(cq + p.cq_off.cqes);
    return 0;
  }
  int fail() {
    const int e = -errno;
    close_all();
    return e;
  }
  void close_all() {
    if (sqes && sqes != MAP_FAILED) munmap(sqes, sqes_len);
    if (cq_ptr && cq_ptr != MAP_FAILED && cq_ptr != sq_ptr) munmap(cq_ptr, cq_len);
    if (sq_ptr && sq_ptr != MAP_FAILED) munmap(sq_ptr, sq_len);
    if (fd >= 0) ::close(fd);
    fd = -1;
    sqes = nullptr;
    sq_ptr = cq_ptr = nullptr;
  }
  // queue one read (the caller keeps at most `entries` in flight)
  void push_read(int file, void *buf, unsigned len, uint64_t off, uint64_t tag) {
    const unsigned tail = *sq_tail;  // only this thread writes the tail
    const unsigned idx = tail & *sq_mask;
    io_uring_sqe *e = &sqes[idx];
    memset(e, 0, sizeof(*e));
    e->opcode = IORING_OP_READ;
    e->fd = file;
    e->addr = (uint64_t)(uintptr_t)buf;
    e->len = len;
    e->off = off;
    e->user_data = tag;
    sq_array[idx] = idx;
    __atomic_store_n(sq_tail, tail + 1, __ATOMIC_RELEASE);
  }
};

struct Tier {
  int file = -1;
  int stride = 0;
  int qd = 0;
  int backend = 0;
  int64_t rows = 0;  // whole rows the file holds
  Ring ring;
  char *slots = nullptr;  // qd sector-aligned bounce slots of `stride` bytes
};

// Returns n, or a negative errno after every request in flight has completed (so no late completion
// can land in a later call). A failing ring is closed; later calls use the thread pool.
int64_t read_uring(Tier *t, const int64_t *ids, int64_t n, char *out, int row_bytes) {
  Ring &r = t->ring;
  const int depth = (int)std::min<int64_t>(std::min<unsigned>((unsigned)t->qd, r.entries), n);
  std::vector<int64_t> slot_item(depth, -1);
  int64_t next = 0, done = 0, err = 0;
  unsigned queued = 0, inflight = 0;
  auto issue = [&](int s) {
    r.push_read(t->file, t->slots + (size_t)s * t->stride, (unsigned)t->stride, (uint64_t)ids[next] * t->stride, s);
    slot_item[s] = next++;
    queued++;
  };
  for (int s = 0; s < depth; s++) issue(s);
  while (queued + inflight > 0) {
    const int got = sys_enter(r.fd, queued, 1, IORING_ENTER_GETEVENTS);
    if (got < 0 && errno == EINTR) continue;
    if (got < 0 || (got == 0 && inflight == 0)) {  // nothing taken and nothing to wait for
      const int64_t e = got < 0 ? -(int64_t)errno : -(int64_t)EAGAIN;
      r.close_all();  // closing the ring cancels and waits for its requests; the slots stay allocated
      t->backend = FVS_TIER_THREADS;
      return e;
    }
    queued -= (unsigned)got;
    inflight += (unsigned)got;
    unsigned head = *r.cq_head;
    const unsigned tail = __atomic_load_n(r.cq_tail, __ATOMIC_ACQUIRE);
    for (; head != tail; head++) {
      const io_uring_cqe &c = r.cqes[head & *r.cq_mask];
      const int s = (int)c.user_data;
      inflight--;
      if (c.res < row_bytes) {
        if (err == 0) err = c.res < 0 ? (int64_t)c.res : -(int64_t)EIO;
      } else {
        memcpy(out + (size_t)slot_item[s] * row_bytes, t->slots + (size_t)s * t->stride, (size_t)row_bytes);
        done++;
      }
      if (err == 0 && next < n) issue(s);
    }
    __atomic_store_n(r.cq_head, head, __ATOMIC_RELEASE);
  }
  return err != 0 ? err : done;
}

int64_t read_threads(Tier *t, const int64_t *ids, int64_t n, char *out, int row_bytes) {
  const int nt = (int)std::min<int64_t>(std::min(t->qd, kMaxThreads), n);
  std::atomic<int64_t> err{0};
  std::atomic<int64_t> cursor{0};
  auto work = [&](int w) {
    char *buf = t->slots + (size_t)w * t->stride;
    for (;;) {
      const int64_t i = cursor.fetch_add(1);
      if (i >= n || err.load() != 0) return;
      int64_t got = 0;
      int e = 0;
      const off_t off = (off_t)ids[i] * t->stride;
      while (got < t->stride) {
        const ssize_t r = pread(t->file, buf + got, (size_t)(t->stride - got), off + got);
        if (r < 0 && errno == EINTR) continue;
        if (r < 0) e = errno;
        if (r <= 0) break;  // an error, or the end of a file whose last row is shorter than the stride
        got += r;
      }
      if (got < row_bytes) {
        int64_t zero = 0;
        err.compare_exchange_strong(zero, e ? -(int64_t)e : -(int64_t)EIO);
        return;
      }
      memcpy(out + (size_t)i * row_bytes, buf, (size_t)row_bytes);
    }
  };
  std::vector<std::thread> pool;
  for (int w = 1; w < nt; w++) pool.emplace_back(work, w);
  work(0);
  for (auto &th : pool) th.join();
  return err.load() != 0 ? err.load() : n;
}

}  // namespace

extern "C" void *fvs_tier_open(const char *path, int32_t stride, int32_t qd, int32_t flags, int32_t *status) {
  auto set = [&](int v) {
    if (status) *status = v;
  };
  if (!path || stride <= 0 || stride % kSector != 0 || qd <= 0 || qd > kMaxQd) {
    set(-EINVAL);
    return nullptr;
  }
  Tier *t = new Tier();
  t->stride = stride;
  t->qd = qd;
  int fd = -1;
  if (!(flags & FVS_TIER_BUFFERED)) fd = open(path, O_RDONLY | O_DIRECT | O_CLOEXEC);
  if (fd < 0) fd = open(path, O_RDONLY | O_CLOEXEC);  // file systems without O_DIRECT (tmpfs)
  if (fd < 0) {
    set(-errno);
    delete t;
    return nullptr;
  }
  t->file = fd;
  struct stat st;
  t->rows = fstat(fd, &st) == 0 ? ((int64_t)st.st_size + stride - 1) / stride : 0;  // the last row may be short
  const int nslots = std::max(qd, kMaxThreads);
  if (posix_memalign((void **)&t->slots, kSector, (size_t)nslots * stride) != 0) {
    set(-ENOMEM);
    ::close(fd);
    delete t;
    return nullptr;
  }
  t->backend = FVS_TIER_THREADS;
  if (!(flags & FVS_TIER_FORCE_THREADS) && t->ring.init((unsigned)qd) == 0) t->backend = FVS_TIER_URING;
  set(0);
  return t;
}

extern "C" int32_t fvs_tier_backend(const void *tier) { return tier ? ((const Tier *)tier)->backend : 0; }

extern "C" int64_t fvs_tier_rows(const void *tier) { return tier ? ((const Tier *)tier)->rows : -1; }

extern "C" int64_t fvs_tier_read_rows(void *tier, const int64_t *ids, int64_t n, void *out, int32_t row_bytes) {
  Tier *t = (Tier *)tier;
  if (!t || n < 0 || row_bytes <= 0 || row_bytes > t->stride) return -EINVAL;
  if (n == 0) return 0;
  if (!ids || !out) return -EINVAL;
  for (int64_t i = 0; i < n; i++)
    if (ids[i] < 0 || ids[i] >= t->rows) return -ERANGE;
  if (t->backend == FVS_TIER_URING) return read_uring(t, ids, n, (char *)out, row_bytes);
  return read_threads(t, ids, n, (char *)out, row_bytes);
}

extern "C" void fvs_tier_close(void *tier) {
  Tier *t = (Tier *)tier;
  if (!t) return;
  t->ring.close_all();
  if (t->file >= 0) ::close(t->file);
  free(t->slots);
  delete t;
}
