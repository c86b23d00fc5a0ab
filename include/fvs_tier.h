/* libfvs_tier: batched reads of fixed-stride rows from a file on NVMe (Linux, host code only).
 *
 * The row tier of the reference's NVMe engine: full-precision vectors kept on an SSD, one row per
 * 4096-byte-aligned slot, and the rows stage 3 needs read with many requests in flight. It replaces
 * the Win32 reader src/native/nvme_reader.c:8-38 (CreateFileW with FILE_FLAG_NO_BUFFERING |
 * FILE_FLAG_OVERLAPPED and an I/O completion port, up to 128 reads in flight) and its ctypes wrapper
 * src/nvme_async.py:13-25 (AsyncTier). Here the reads go through io_uring, or through a pool of pread()
 * threads where io_uring is unavailable; the file is opened with O_DIRECT where the file system
 * supports it.
 *
 * Return codes: 0 / a count on success, a negative errno value on failure.
 */
#ifndef FVS_TIER_H
#define FVS_TIER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FVS_TIER_URING 1          /* fvs_tier_backend: io_uring */
#define FVS_TIER_THREADS 2        /* fvs_tier_backend: pread() thread pool */

#define FVS_TIER_FORCE_THREADS 1  /* fvs_tier_open flag: use the thread pool */
#define FVS_TIER_BUFFERED 2       /* fvs_tier_open flag: do not ask for O_DIRECT */

/* Open a tier file whose row i starts at byte i * stride (stride a positive multiple of 4096); qd
 * (1..1024) is the number of reads kept in flight. Replaces open_tier + make_port + alloc_bufs
 * (src/native/nvme_reader.c:8-12). Returns a handle, or NULL with *status set to a negative errno. */
void *fvs_tier_open(const char *path, int32_t stride, int32_t qd, int32_t flags, int32_t *status);

/* The backend a handle reads with: FVS_TIER_URING or FVS_TIER_THREADS. */
int32_t fvs_tier_backend(const void *tier);

/* Rows the file holds (its size over the stride, rounded up). */
int64_t fvs_tier_rows(const void *tier);

/* Read rows ids[0..n) into out + i * row_bytes (row_bytes <= stride): read_rows of
 * src/native/nvme_reader.c:22-38. Returns n, -ERANGE for an id outside the file (nothing read),
 * -EINVAL for bad arguments, or the negative errno of a failed read (after every read in flight has
 * completed). Not safe to call on one handle from two threads at once. */
int64_t fvs_tier_read_rows(void *tier, const int64_t *ids, int64_t n, void *out, int32_t row_bytes);

/* Close the file and free the handle. */
void fvs_tier_close(void *tier);

#ifdef __cplusplus
}
#endif

#endif
