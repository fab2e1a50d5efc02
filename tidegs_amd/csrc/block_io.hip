// Parallel block reads of the on-disk Gaussian store (host code).
//
// TideGS's LogStorageManager reads each block with f.seek + f.read, then
// copies it through numpy and torch.cat into the pinned staging tensor
// (storage/log_storage_manager.py:208-291, storage/block_reader.py:55-87).
// Here every block is pread() straight into its final place in the caller's
// (pinned) staging buffer by a small pool of threads, so one call fills the
// whole [rows, 59] batch that the GPU unpack consumes.  The caller sorts the
// blocks by (file, offset) so each thread's reads run forward through the
// files.
#include <errno.h>
#include <unistd.h>

#include <atomic>
#include <thread>
#include <vector>

#include "tgs_common.cuh"

namespace {

// Read exactly `nbytes` at `offset` of fd into dst; 0, or errno / -1 (EOF).
int read_full(int fd, char* dst, int64_t offset, int64_t nbytes) {
  constexpr int64_t kChunk = 16ll << 20;  // bounded single pread calls
  while (nbytes > 0) {
    const int64_t want = nbytes < kChunk ? nbytes : kChunk;
    const ssize_t got = pread(fd, dst, (size_t)want, (off_t)offset);
    if (got < 0) {
      if (errno == EINTR) continue;
      return errno ? errno : EIO;
    }
    if (got == 0) return -1;  // end of file before the block ended
    dst += got;
    offset += got;
    nbytes -= got;
  }
  return 0;
}

}  // namespace

extern "C" int tgs_io_read_blocks(uint32_t n, const int32_t* fds, const int64_t* file_offsets,
                                  const int64_t* nbytes, void* dst, const int64_t* dst_offsets,
                                  uint32_t n_threads) {
  const char* name = "tgs_io_read_blocks";
  if (n == 0) return TGS_OK;
  TGS_CHECK_ARG(fds && file_offsets && nbytes && dst && dst_offsets, "%s: null pointer", name);
  for (uint32_t i = 0; i < n; ++i) {
    TGS_CHECK_ARG(fds[i] >= 0 && file_offsets[i] >= 0 && nbytes[i] >= 0 && dst_offsets[i] >= 0,
                  "%s: block %u has a negative descriptor, offset or size", name, i);
  }
  if (n_threads == 0) n_threads = 1;
  if (n_threads > 64) n_threads = 64;
  if (n_threads > n) n_threads = n;
  std::atomic<uint32_t> next{0};
  std::atomic<int> status{0};
  std::atomic<uint32_t> failed_block{0};
  auto worker = [&]() {
    for (;;) {
      const uint32_t i = next.fetch_add(1, std::memory_order_relaxed);
      if (i >= n || status.load(std::memory_order_relaxed) != 0) return;
      const int rc = read_full(fds[i], (char*)dst + dst_offsets[i], file_offsets[i], nbytes[i]);
      if (rc != 0) {
        int expected = 0;
        if (status.compare_exchange_strong(expected, rc)) failed_block.store(i);
        return;
      }
    }
  };
  std::vector<std::thread> pool;
  pool.reserve(n_threads);
  for (uint32_t t = 0; t < n_threads; ++t) pool.emplace_back(worker);
  for (auto& th : pool) th.join();
  const int rc = status.load();
  if (rc == -1) {
    tgs_set_error("%s: block %u ends past the end of its file", name, failed_block.load());
    return TGS_ERR_ARG;
  }
  if (rc != 0) {
    tgs_set_error("%s: pread failed for block %u (errno %d)", name, failed_block.load(), rc);
    return rc;
  }
  return TGS_OK;
}
