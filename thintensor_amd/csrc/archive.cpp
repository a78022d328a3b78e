// ThinTensor `.thin` v0 archive reader (host code) and page upload into HBM.
//
// Layout (reference thinruntime/archive.py:9-13, 99-208; src/archive.rs:14-41, 583-662):
//   [0, 88)        header: magic "THINv0\0\0", u32 header_len (88), u32 version (0),
//                  u64 manifest_off, manifest_len, page_table_off, page_count, data_off,
//                  32-byte archive hash (reserved, zero in v0); little endian
//   [88, ...)      UTF-8 JSON manifest
//   page table     per page: u16 id_len, id bytes, u64 offset, u64 stored_size,
//                  u64 raw_size, u32 flags, 32-byte BLAKE3 checksum
//   payload        page bytes, back to back from data_off
//
// The file is memory-mapped read-only; page views are pointers into the mapping.
// Validation follows the reference reader's checks and messages, split in the order
// that reader applies them (header, page table, overlaps) so the caller can place the
// manifest checks between them as the reference does.  tt_archive_upload moves a byte
// range of the mapping into device memory through two pinned staging buffers: the host
// copy of chunk i + 1 overlaps the DMA of chunk i.
#include <fcntl.h>
#include <stdarg.h>
#include <hip/hip_runtime_api.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/thintensor_hip.h"

namespace tt {
void set_error(const char* fmt, ...);
}

namespace {

constexpr uint8_t kMagic[8] = {'T', 'H', 'I', 'N', 'v', '0', 0, 0};
constexpr uint32_t kHeaderLen = 88;
constexpr size_t kStageBytes = 32u << 20;

struct Record {
  int64_t id_off;   // offset of the id bytes in the file
  int64_t id_len;
  uint64_t offset, stored_size, raw_size;
  uint32_t flags;
  int64_t checksum_off;
};

uint64_t rd64(const uint8_t* p) {
  uint64_t v;
  memcpy(&v, p, 8);
  return v;
}
uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  memcpy(&v, p, 4);
  return v;
}

// Python-style repr of a short byte string (b'...'), for the magic message.
std::string bytes_repr(const uint8_t* p, size_t n) {
  std::string s = "b'";
  char buf[8];
  for (size_t i = 0; i < n; i++) {
    const uint8_t c = p[i];
    if (c == '\\' || c == '\'') {
      s += '\\';
      s += (char)c;
    } else if (c >= 32 && c < 127) {
      s += (char)c;
    } else {
      snprintf(buf, sizeof(buf), "\\x%02x", c);
      s += buf;
    }
  }
  return s + "'";
}

}  // namespace

struct tt_archive {
  int fd = -1;
  uint8_t* map = nullptr;
  uint64_t size = 0;
  tt_archive_info h{};
  std::vector<Record> pages;
  std::unordered_map<std::string, int64_t> index;
  uint64_t page_table_end = 0;
  // upload staging
  std::mutex mu;
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int stage_device = -1;
};

static int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
static int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  tt::set_error("%s", buf);
  return TT_ERR_INVALID;
}

static void release_stage(tt_archive* a) {
  for (int i = 0; i < 2; i++) {
    if (a->done[i]) {
      (void)hipEventSynchronize(a->done[i]);
      (void)hipEventDestroy(a->done[i]);
      a->done[i] = nullptr;
    }
    if (a->stage[i]) {
      (void)hipHostFree(a->stage[i]);
      a->stage[i] = nullptr;
    }
  }
  a->stage_device = -1;
}

extern "C" int tt_archive_open(const char* path, tt_archive** out) {
  if (!path || !out) return fail("archive: null argument");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail("archive: cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0) {
    ::close(fd);
    return fail("archive: cannot stat %s", path);
  }
  const uint64_t size = (uint64_t)st.st_size;
  if (size < kHeaderLen) {
    ::close(fd);
    return fail("File is too small to contain a ThinTensor header");
  }
  void* m = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  if (m == MAP_FAILED) {
    ::close(fd);
    return fail("archive: cannot map %s", path);
  }
  auto* a = new tt_archive();
  a->fd = fd;
  a->map = static_cast<uint8_t*>(m);
  a->size = size;
  const uint8_t* p = a->map;
  tt_archive_info& h = a->h;
  h.header_len = rd32(p + 8);
  h.version = rd32(p + 12);
  h.manifest_off = rd64(p + 16);
  h.manifest_len = rd64(p + 24);
  h.page_table_off = rd64(p + 32);
  h.page_count = rd64(p + 40);
  h.data_off = rd64(p + 48);
  memcpy(h.archive_hash, p + 56, 32);
  h.file_size = size;
  int rc = TT_OK;
  if (memcmp(p, kMagic, 8) != 0) {
    rc = fail("Invalid magic: %s, expected %s", bytes_repr(p, 8).c_str(), bytes_repr(kMagic, 8).c_str());
  } else if (h.header_len != kHeaderLen) {
    rc = fail("Invalid header length: %u, expected %u", h.header_len, kHeaderLen);
  } else if (h.version != 0) {
    rc = fail("Invalid format version: %u, expected 0", h.version);
  } else if (h.manifest_off != h.header_len) {
    rc = fail("Manifest offset %llu does not follow header length %u", (unsigned long long)h.manifest_off,
              h.header_len);
  } else if (h.manifest_len > size || h.manifest_off + h.manifest_len > size) {
    rc = fail("Manifest range exceeds file size");
  } else if (h.page_table_off != h.manifest_off + h.manifest_len) {
    rc = fail("Page table does not immediately follow the manifest");
  } else if (h.page_table_off > size) {
    rc = fail("Page table offset exceeds file size");
  }
  if (rc != TT_OK) {
    tt_archive_close(a);
    return rc;
  }
  h.manifest = a->map + h.manifest_off;
  *out = a;
  return TT_OK;
}

extern "C" int tt_archive_parse_pages(tt_archive* a) {
  if (!a) return fail("archive: null handle");
  const uint8_t* p = a->map;
  const uint64_t size = a->size;
  uint64_t pos = a->h.page_table_off;
  a->pages.clear();
  a->index.clear();
  for (uint64_t i = 0; i < a->h.page_count; i++) {
    if (pos + 2 > size) return fail("Truncated page table record at page index %llu", (unsigned long long)i);
    const uint16_t id_len = (uint16_t)(p[pos] | (p[pos + 1] << 8));
    pos += 2;
    if (id_len == 0) return fail("Empty page id at page index %llu", (unsigned long long)i);
    if (pos + id_len > size) return fail("Truncated page id at page index %llu", (unsigned long long)i);
    const std::string id(reinterpret_cast<const char*>(p + pos), id_len);
    Record r;
    r.id_off = (int64_t)pos;
    r.id_len = id_len;
    pos += id_len;
    if (a->index.count(id)) return fail("Duplicate page id in page table: %s", id.c_str());
    if (pos + 60 > size) return fail("Truncated page record tail for page %s", id.c_str());
    r.offset = rd64(p + pos);
    r.stored_size = rd64(p + pos + 8);
    r.raw_size = rd64(p + pos + 16);
    r.flags = rd32(p + pos + 24);
    r.checksum_off = (int64_t)(pos + 28);
    pos += 60;
    if (r.offset < a->h.data_off) return fail("Page %s offset starts before data_off", id.c_str());
    // offset + stored_size <= size, written so that no sum can wrap around 2^64
    if (r.offset > size || r.stored_size > size - r.offset)
      return fail("Page %s offset+size exceeds file size", id.c_str());
    if (r.stored_size == 0 && r.raw_size != 0)
      return fail("Page %s has zero stored_size but nonzero raw_size", id.c_str());
    if (r.flags != 0) return fail("Page %s uses unsupported runtime flags 0x%x", id.c_str(), r.flags);
    if (r.stored_size != r.raw_size) return fail("Uncompressed page %s stored/raw sizes differ", id.c_str());
    a->index.emplace(id, (int64_t)a->pages.size());
    a->pages.push_back(r);
  }
  a->page_table_end = pos;
  if (pos != a->h.data_off)
    return fail("Page table ends at %llu, but data_off is %llu", (unsigned long long)pos,
                (unsigned long long)a->h.data_off);
  return TT_OK;
}

extern "C" int tt_archive_check_overlaps(const tt_archive* a) {
  if (!a) return fail("archive: null handle");
  std::vector<int64_t> order(a->pages.size());
  for (size_t i = 0; i < order.size(); i++) order[i] = (int64_t)i;
  std::stable_sort(order.begin(), order.end(),
                   [&](int64_t x, int64_t y) { return a->pages[x].offset < a->pages[y].offset; });
  for (size_t k = 0; k + 1 < order.size(); k++) {
    const Record& r1 = a->pages[order[k]];
    const Record& r2 = a->pages[order[k + 1]];
    if (r1.stored_size > r2.offset - r1.offset) {   // r2.offset >= r1.offset (sorted); no wrap
      const std::string n1(reinterpret_cast<const char*>(a->map + r1.id_off), r1.id_len);
      const std::string n2(reinterpret_cast<const char*>(a->map + r2.id_off), r2.id_len);
      return fail("Overlapping pages detected: %s overlaps with %s", n1.c_str(), n2.c_str());
    }
  }
  return TT_OK;
}

extern "C" int tt_archive_get_info(const tt_archive* a, tt_archive_info* out) {
  if (!a || !out) return fail("archive: null argument");
  *out = a->h;
  return TT_OK;
}

extern "C" int tt_archive_get_record(const tt_archive* a, int64_t i, tt_archive_record* out) {
  if (!a || !out) return fail("archive: null argument");
  if (i < 0 || i >= (int64_t)a->pages.size()) return fail("archive: page index %lld out of range", (long long)i);
  const Record& r = a->pages[i];
  out->id = reinterpret_cast<const char*>(a->map + r.id_off);
  out->id_len = r.id_len;
  out->offset = r.offset;
  out->stored_size = r.stored_size;
  out->raw_size = r.raw_size;
  out->flags = r.flags;
  memcpy(out->checksum, a->map + r.checksum_off, 32);
  return TT_OK;
}

extern "C" int64_t tt_archive_find(const tt_archive* a, const char* id, int64_t id_len) {
  if (!a || !id || id_len <= 0) return -1;
  auto it = a->index.find(std::string(id, (size_t)id_len));
  return it == a->index.end() ? -1 : it->second;
}

extern "C" const uint8_t* tt_archive_data(const tt_archive* a) { return a ? a->map : nullptr; }

extern "C" int tt_archive_upload(tt_archive* a, int64_t offset, int64_t nbytes, void* dst, void* stream) {
  if (!a || !dst) return fail("archive upload: null argument");
  if (offset < 0 || nbytes < 0 || (uint64_t)offset + (uint64_t)nbytes > a->size)
    return fail("archive upload: range [%lld, +%lld) outside the file", (long long)offset, (long long)nbytes);
  if (nbytes == 0) return TT_OK;
  std::lock_guard<std::mutex> lock(a->mu);
  hipStream_t st = static_cast<hipStream_t>(stream);
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail("archive upload: no current device");
  if (a->stage_device != dev) {
    release_stage(a);
    for (int i = 0; i < 2; i++) {
      if (hipHostMalloc(&a->stage[i], kStageBytes, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&a->done[i], hipEventDisableTiming) != hipSuccess) {
        release_stage(a);
        return fail("archive upload: cannot allocate %zu bytes of pinned staging", kStageBytes);
      }
      if (hipEventRecord(a->done[i], st) != hipSuccess) {
        release_stage(a);
        return fail("archive upload: event record failed");
      }
    }
    a->stage_device = dev;
  }
  int64_t done = 0;
  int buf = 0;
  while (done < nbytes) {
    const int64_t n = std::min<int64_t>((int64_t)kStageBytes, nbytes - done);
    // the staging buffer is reused only after its previous copy has left
    if (hipEventSynchronize(a->done[buf]) != hipSuccess) return fail("archive upload: wait failed");
    memcpy(a->stage[buf], a->map + offset + done, (size_t)n);
    if (hipMemcpyAsync(static_cast<uint8_t*>(dst) + done, a->stage[buf], (size_t)n, hipMemcpyHostToDevice, st) !=
            hipSuccess ||
        hipEventRecord(a->done[buf], st) != hipSuccess)
      return fail("archive upload: copy of %lld bytes failed", (long long)n);
    done += n;
    buf ^= 1;
  }
  return TT_OK;
}

extern "C" int tt_archive_close(tt_archive* a) {
  if (!a) return TT_OK;
  release_stage(a);
  if (a->map) munmap(a->map, a->size);
  if (a->fd >= 0) ::close(a->fd);
  delete a;
  return TT_OK;
}
