/* loader.c -- weights from disk into device buffers.
 *
 * Reference counterpart: the mmap-backed disk tensor (src/tensor/mmap.c:1-30,
 * tinygrad's DISK device), whose bytes reach a GPU through the lazy COPY
 * path, and the weight pack reader of bench/dsv2_decode_bench.c:229-310.
 *
 * MI355X form: the file region is mapped read-only (page-aligned, as
 * mmap.c maps it) and streamed to the device through a ring of two pinned
 * host staging buffers (hipHostMalloc, 32 MiB each): copying one chunk out
 * of the page cache overlaps the DMA of the previous one, and a slot is
 * reused only after the event recorded behind its DMA completes.  No
 * pageable-memory DMA (which would bounce through a driver buffer) and no
 * host copy of the whole tensor. */
#define _GNU_SOURCE
#include "internal.h"

#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define STAGE_SLOTS 2
#define STAGE_BYTES (32ull << 20)

static void *STAGE[STAGE_SLOTS];
static hipEvent_t STAGE_EV[STAGE_SLOTS];
static int STAGE_USED[STAGE_SLOTS];

static int stage_init(void) {
  for (int i = 0; i < STAGE_SLOTS; i++) {
    if (!STAGE[i]) {
      hipError_t e = hipHostMalloc(&STAGE[i], STAGE_BYTES, hipHostMallocDefault);
      if (e != hipSuccess) {
        STAGE[i] = NULL;
        hb_set_error("load_file: hipHostMalloc staging: %s", hipGetErrorString(e));
        return -1;
      }
    }
    if (!STAGE_EV[i] && hipEventCreateWithFlags(&STAGE_EV[i], hipEventDisableTiming) != hipSuccess) {
      STAGE_EV[i] = NULL;
      hb_set_error("load_file: hipEventCreate failed");
      return -1;
    }
  }
  return 0;
}

void hb_loader_reset(void) {
  for (int i = 0; i < STAGE_SLOTS; i++) {
    if (STAGE_EV[i]) hipEventDestroy(STAGE_EV[i]);
    if (STAGE[i]) hipHostFree(STAGE[i]);
    STAGE_EV[i] = NULL;
    STAGE[i] = NULL;
    STAGE_USED[i] = 0;
  }
}

THVM_API int thvm_hip_buf_load_file(uint32_t buf_id, uint64_t dst_off, const char *path,
                                    uint64_t file_off, uint64_t nbytes) {
  if (hb_require_ready("load_file")) return -1;
  if (hb_stream_capturing()) { hb_set_error("load_file: not allowed while a graph capture is open"); return -1; }
  void *dev = hb_buf_ptr(buf_id);
  const u64 cap = hb_buf_size(buf_id);
  if (!dev) { hb_set_error("load_file: buffer %u not live", buf_id); return -1; }
  if (dst_off > cap || nbytes > cap - dst_off) {
    hb_set_error("load_file: [%llu, +%llu) outside buffer %u of %llu bytes",
                 (unsigned long long)dst_off, (unsigned long long)nbytes, buf_id, (unsigned long long)cap);
    return -1;
  }
  if (nbytes == 0) return 0;
  if (!path) { hb_set_error("load_file: null path"); return -1; }
  int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) { hb_set_error("load_file: cannot open %s", path); return -1; }
  struct stat st;
  if (fstat(fd, &st) || (u64)st.st_size < file_off || (u64)st.st_size - file_off < nbytes) {
    close(fd);
    hb_set_error("load_file: %s holds %lld bytes, the region [%llu, +%llu) does not fit", path,
                 (long long)st.st_size, (unsigned long long)file_off, (unsigned long long)nbytes);
    return -1;
  }
  const u64 page = (u64)sysconf(_SC_PAGESIZE);
  const u64 base = file_off - file_off % page, lead = file_off - base, maplen = lead + nbytes;
  void *map = mmap(NULL, maplen, PROT_READ, MAP_PRIVATE, fd, (off_t)base);
  close(fd);
  if (map == MAP_FAILED) { hb_set_error("load_file: mmap of %s failed", path); return -1; }
  madvise(map, maplen, MADV_SEQUENTIAL);
  const char *src = (const char *)map + lead;
  int rc = stage_init();
  u64 done = 0;
  int slot = 0;
  while (!rc && done < nbytes) {
    const u64 n = nbytes - done < STAGE_BYTES ? nbytes - done : STAGE_BYTES;
    if (STAGE_USED[slot] && hipEventSynchronize(STAGE_EV[slot]) != hipSuccess) {
      hb_set_error("load_file: staging event wait failed");
      rc = -1;
      break;
    }
    memcpy(STAGE[slot], src + done, n);
    hipError_t e = hipMemcpyAsync((char *)dev + dst_off + done, STAGE[slot], n,
                                  hipMemcpyHostToDevice, HB_STREAM);
    if (e == hipSuccess) e = hipEventRecord(STAGE_EV[slot], HB_STREAM);
    if (e != hipSuccess) { hb_set_error("load_file: copy: %s", hipGetErrorString(e)); rc = -1; break; }
    STAGE_USED[slot] = 1;
    done += n;
    slot = (slot + 1) % STAGE_SLOTS;
  }
  hipError_t e = hipStreamSynchronize(HB_STREAM);
  if (!rc && e != hipSuccess) { hb_set_error("load_file: %s", hipGetErrorString(e)); rc = -1; }
  munmap(map, maplen);
  return rc;
}
