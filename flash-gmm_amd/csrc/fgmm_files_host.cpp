// Host row sources over local vector files, for the streaming EM driver and for
// loading data sets into device memory (plain C++, no HIP).
//
// The reference tunes on SIFT1M, GloVe and Deep10M (flash_gmm_diag_h100.py:17,
// :299-301; flash_gmm_h100.py:273) but ships no reader.  The binary layouts these
// sets are distributed in:
//   .fvecs  per vector: int32 d, then d float32   (SIFT1M base / GIST1M)
//   .bvecs  per vector: int32 d, then d uint8     (SIFT1B)
//   .fbin   header uint32 n, uint32 d, then n*d float32   (Deep1B / Deep10M)
//   .u8bin  header uint32 n, uint32 d, then n*d uint8
// The file is memory-mapped read-only; a chunk of rows is converted to float32 by
// up to `threads` host threads, each taking a contiguous range of rows.
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "flashgmm.h"

namespace {

// Row n's first value and its stride in bytes between rows.
struct Layout {
  size_t first, stride, width;   // byte offset of row 0's values, row stride, bytes per value
};

bool layout_of(const fgmm_vecs_file* f, Layout* l) {
  switch (f->format) {
    case FGMM_VECS_FVECS: *l = {4, 4 + 4 * (size_t)f->D, 4}; return true;
    case FGMM_VECS_BVECS: *l = {4, 4 + (size_t)f->D, 1}; return true;
    case FGMM_VECS_FBIN: *l = {8, 4 * (size_t)f->D, 4}; return true;
    case FGMM_VECS_U8BIN: *l = {8, (size_t)f->D, 1}; return true;
    default: return false;
  }
}

void convert_rows(const unsigned char* base, const Layout& l, int64_t row0, int64_t n, int64_t D, float* dst) {
  for (int64_t r = 0; r < n; ++r) {
    const unsigned char* src = base + l.first + (size_t)(row0 + r) * l.stride;
    float* out = dst + r * D;
    if (l.width == 4) {
      memcpy(out, src, (size_t)D * 4);
    } else {
      for (int64_t d = 0; d < D; ++d) out[d] = (float)src[d];
    }
  }
}

}  // namespace

extern "C" int fgmm_vecs_open(const char* path, int format, int threads, fgmm_vecs_file* f) {
  if (!path || !f) return FGMM_ERR_INVALID_ARG;
  memset(f, 0, sizeof(*f));
  f->format = format;
  f->threads = threads;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return FGMM_ERR_SOURCE;
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 8) {
    close(fd);
    return FGMM_ERR_SOURCE;
  }
  const size_t bytes = (size_t)st.st_size;
  void* base = mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (base == MAP_FAILED) return FGMM_ERR_SOURCE;
  const unsigned char* b = static_cast<const unsigned char*>(base);
  int64_t N = 0, D = 0;
  if (format == FGMM_VECS_FVECS || format == FGMM_VECS_BVECS) {
    int32_t d0;
    memcpy(&d0, b, 4);
    const size_t w = format == FGMM_VECS_FVECS ? 4 : 1;
    if (d0 < 1 || bytes % (4 + w * (size_t)d0) != 0) {
      munmap(base, bytes);
      return FGMM_ERR_INVALID_ARG;
    }
    D = d0;
    N = (int64_t)(bytes / (4 + w * (size_t)d0));
    // Every vector must declare the same dimension (checked at both ends and a
    // stride through the file).
    const int64_t step = std::max<int64_t>(1, N / 64);
    for (int64_t n = 0; n < N; n += step) {
      int32_t d;
      memcpy(&d, b + (size_t)n * (4 + w * D), 4);
      if (d != d0) {
        munmap(base, bytes);
        return FGMM_ERR_INVALID_ARG;
      }
    }
    int32_t dl;
    memcpy(&dl, b + (size_t)(N - 1) * (4 + w * D), 4);
    if (dl != d0) {
      munmap(base, bytes);
      return FGMM_ERR_INVALID_ARG;
    }
  } else if (format == FGMM_VECS_FBIN || format == FGMM_VECS_U8BIN) {
    uint32_t hn, hd;
    memcpy(&hn, b, 4);
    memcpy(&hd, b + 4, 4);
    const size_t w = format == FGMM_VECS_FBIN ? 4 : 1;
    // The rows must fit in the file.  Tested by division: the product n * d * w of a
    // malformed header can pass 2^64 and wrap around.
    const size_t body = bytes >= 8 ? bytes - 8 : 0;
    if (bytes < 8 || hd < 1 || (size_t)hd > body / w || (size_t)hn > body / (w * (size_t)hd)) {
      munmap(base, bytes);
      return FGMM_ERR_INVALID_ARG;
    }
    N = hn;
    D = hd;
  } else {
    munmap(base, bytes);
    return FGMM_ERR_INVALID_ARG;
  }
  f->base = base;
  f->bytes = bytes;
  f->N = N;
  f->D = D;
  return FGMM_OK;
}

extern "C" int fgmm_vecs_source(void* user, int64_t row0, int64_t nrows, int64_t D, float* dst) {
  const fgmm_vecs_file* f = static_cast<const fgmm_vecs_file*>(user);
  Layout l;
  if (!f || !f->base || !dst || D != f->D || row0 < 0 || nrows < 0 || row0 + nrows > f->N || !layout_of(f, &l))
    return FGMM_ERR_INVALID_ARG;
  const unsigned char* base = static_cast<const unsigned char*>(f->base);
  const int hw = (int)std::max(1u, std::thread::hardware_concurrency());
  int T = f->threads > 0 ? f->threads : hw;
  T = (int)std::min<int64_t>(T, std::max<int64_t>(1, nrows / 1024));
  if (T <= 1) {
    convert_rows(base, l, row0, nrows, D, dst);
    return FGMM_OK;
  }
  std::vector<std::thread> pool;
  pool.reserve(T);
  for (int t = 0; t < T; ++t) {
    const int64_t a = nrows * t / T, e = nrows * (t + 1) / T;
    pool.emplace_back([=] { convert_rows(base, l, row0 + a, e - a, D, dst + a * D); });
  }
  for (auto& th : pool) th.join();
  return FGMM_OK;
}

extern "C" void fgmm_vecs_close(fgmm_vecs_file* f) {
  if (f && f->base) munmap(f->base, f->bytes);
  if (f) f->base = nullptr;
}
